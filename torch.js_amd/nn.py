"""torch.nn modules for the 'hip' device (src/nn/*.ts): the ones the
autograd hot path uses.  Module bookkeeping mirrors src/nn/module.ts:17-270;
the layer maths is in functional.py.
"""
import math
from collections import OrderedDict

import numpy as np

from . import functional as F
from .tensor import Tensor, from_numpy, ones, randn, zeros


class Parameter(Tensor):
    """A leaf tensor that requires grad (Parameter.create,
    src/nn/parameter.ts:17-33): wraps the data without copying."""

    __slots__ = ()

    def __new__(cls, data, requires_grad=True):
        return data.detach().requires_grad_(requires_grad)

    @staticmethod
    def create(data, requires_grad=True):
        if isinstance(data, Tensor):
            return data.detach().requires_grad_(requires_grad)
        return from_numpy(np.asarray(data, dtype=np.float32), requires_grad=requires_grad)


class Module:
    """nn.Module (src/nn/module.ts:17-270)."""

    def __init__(self):
        object.__setattr__(self, "_parameters", OrderedDict())
        object.__setattr__(self, "_modules", OrderedDict())
        object.__setattr__(self, "training", True)

    def __setattr__(self, name, value):
        params = self.__dict__.get("_parameters")
        mods = self.__dict__.get("_modules")
        if isinstance(value, Module) and mods is not None:
            mods[name] = value
        elif isinstance(value, Tensor) and params is not None and value.requires_grad and \
                value.is_leaf:
            params[name] = value
        object.__setattr__(self, name, value)

    def register_parameter(self, name, param):
        if param is None:
            object.__setattr__(self, name, None)
            return
        self._parameters[name] = param
        object.__setattr__(self, name, param)

    def register_module(self, name, module):
        self._modules[name] = module
        object.__setattr__(self, name, module)

    add_module = register_module

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def named_parameters(self, prefix=""):
        seen = set()
        for name, p in self._parameters.items():
            if p is not None and id(p) not in seen:
                seen.add(id(p))
                yield (prefix + name, p)
        for mname, m in self._modules.items():
            for name, p in m.named_parameters(prefix + mname + "."):
                if id(p) not in seen:
                    seen.add(id(p))
                    yield (name, p)

    def parameters(self):
        return [p for _, p in self.named_parameters()]

    def children(self):
        return list(self._modules.values())

    def modules(self):
        out = [self]
        for m in self._modules.values():
            out.extend(m.modules())
        return out

    def zero_grad(self, set_to_none=True):
        for p in self.parameters():
            p.grad = None

    def train(self, mode=True):
        for m in self.modules():
            object.__setattr__(m, "training", mode)
        return self

    def eval(self):
        return self.train(False)

    def state_dict(self):
        return OrderedDict((n, p.detach()) for n, p in self.named_parameters())

    def load_state_dict(self, state):
        params = dict(self.named_parameters())
        for name, value in state.items():
            if name not in params:
                raise KeyError("unexpected key %s in state_dict" % name)
            tgt = params[name]
            src = value if isinstance(value, Tensor) else from_numpy(np.asarray(value))
            if tuple(src.shape) != tgt.shape:
                raise ValueError("size mismatch for %s: %s vs %s" % (name, list(src.shape),
                                                                   list(tgt.shape)))
            from .tensor import _copy_into
            _copy_into(tgt, src)
        return self


class Linear(Module):
    """nn.Linear (src/nn/linear.ts:15-67); default init randn*sqrt(1/in)
    and zero bias, as torch.js initialises it (linear.ts:27-39)."""

    def __init__(self, in_features, out_features, bias=True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        k = math.sqrt(1.0 / in_features)
        self.register_parameter("weight", Parameter.create(randn(out_features, in_features).mul(k)))
        self.register_parameter("bias", Parameter.create(zeros(out_features)) if bias else None)

    def forward(self, x):
        if x.ndim == 1:
            x = x.unsqueeze(0)
        return F.linear(x, self.weight, self.bias)


class LayerNorm(Module):
    """nn.LayerNorm (src/nn/layernorm.ts:25-119)."""

    def __init__(self, normalized_shape, eps=1e-5, elementwise_affine=True):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.register_parameter("weight", Parameter.create(ones(*self.normalized_shape)))
            self.register_parameter("bias", Parameter.create(zeros(*self.normalized_shape)))
        else:
            self.weight = None
            self.bias = None

    def forward(self, x):
        return F.layer_norm(x, self.normalized_shape, self.weight, self.bias, self.eps)


class Embedding(Module):
    """nn.Embedding (src/nn/embedding.ts:25-101); N(0,1) init."""

    def __init__(self, num_embeddings, embedding_dim):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.register_parameter("weight", Parameter.create(randn(num_embeddings, embedding_dim)))

    def forward(self, ids):
        return F.embedding(ids, self.weight)


class Conv2d(Module):
    """nn.Conv2d (src/nn/conv.ts:470-530); default init randn*sqrt(1/fan_in)
    (conv.ts:504-506)."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True):
        super().__init__()
        kh, kw = (kernel_size, kernel_size) if isinstance(kernel_size, int) else kernel_size
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size = (kh, kw)
        self.stride, self.padding, self.dilation, self.groups = stride, padding, dilation, groups
        fan_in = in_channels // groups * kh * kw
        k = math.sqrt(1.0 / fan_in)
        self.register_parameter(
            "weight", Parameter.create(randn(out_channels, in_channels // groups, kh, kw).mul(k)))
        self.register_parameter("bias", Parameter.create(zeros(out_channels)) if bias else None)

    def forward(self, x):
        return F.conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation,
                        self.groups)


class MultiheadAttention(Module):
    """nn.MultiheadAttention (src/nn/attention.ts:31-271) with the
    reference's parameters: in_proj_weight [3E, E] (rows: the q, k and v
    projections), in_proj_bias [3E], out_proj_weight [E, E] and
    out_proj_bias [E], weights initialised randn * sqrt(1/E) and biases to
    zero (attention.ts:72-95).  `dropout` is stored and not applied, as in
    the reference (attention.ts:224-231).

    On this device the projections are GEMMs with the bias in the epilogue:
    one GEMM over in_proj_weight when query, key and value are one tensor
    (self-attention; q, k and v are then strided views of its output, and
    the backward assembles their gradients into that output's gradient
    with no copy), two when key is value.  Attention runs on the flash
    kernels (head dims up to 128 that are multiples of 4; others on the
    library's GEMM-composed attention) unless attention weights or masks
    are asked for, when the scores are formed by batched GEMMs and
    softmaxed explicitly."""

    def __init__(self, embed_dim, num_heads, dropout=0.0, bias=True, batch_first=False):
        super().__init__()
        if embed_dim <= 0 or num_heads <= 0:
            raise ValueError("embed_dim and num_heads must be greater than 0, got embed_dim=%d "
                             "and num_heads=%d" % (embed_dim, num_heads))
        if embed_dim % num_heads:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.dropout = dropout
        self.batch_first = batch_first
        self.head_dim = embed_dim // num_heads
        k = math.sqrt(1.0 / embed_dim)
        self.register_parameter("in_proj_weight",
                                Parameter.create(randn(3 * embed_dim, embed_dim).mul(k)))
        self.register_parameter("in_proj_bias",
                                Parameter.create(zeros(3 * embed_dim)) if bias else None)
        self.register_parameter("out_proj_weight",
                                Parameter.create(randn(embed_dim, embed_dim).mul(k)))
        self.register_parameter("out_proj_bias",
                                Parameter.create(zeros(embed_dim)) if bias else None)

    def _project(self, x, block, count):
        """x [rows..., E] times `count` row blocks of in_proj_weight starting
        at `block` (+ the same blocks of in_proj_bias), split per block."""
        E = self.embed_dim
        W = self.in_proj_weight
        b = self.in_proj_bias
        if block or count != 3:
            W = W.narrow(0, block * E, count * E)
            b = b.narrow(0, block * E, count * E) if b is not None else None
        y = F.linear(x, W, b)
        return list(y.split(E, dim=-1)) if count > 1 else [y]

    def _mask(self, N, L, S, attn_mask, key_padding_mask):
        """The additive float mask [N or 1, H or 1, L, S] of PyTorch's
        nn.MultiheadAttention (the reference throws on both masks,
        attention.ts:121-126): bool True = not allowed (-inf), float added;
        attn_mask [L, S] or [N * H, L, S], key_padding_mask [N, S]."""
        from .tensor import Tensor as _Tn, tensor as _tensor

        def as_float(m, shape):
            if not isinstance(m, _Tn):
                m = _tensor(np.asarray(m))
            if m.dtype in ("bool", "uint8"):
                m = zeros(*m.shape).masked_fill(m, float("-inf"))
            elif m.dtype != "float32":
                m = m.float()
            return m.reshape(*shape)
        H = self.num_heads
        out = None
        if attn_mask is not None:
            nd = attn_mask.ndim if isinstance(attn_mask, Tensor) else np.ndim(attn_mask)
            if nd == 2:
                out = as_float(attn_mask, (1, 1, L, S))
            elif nd == 3:
                out = as_float(attn_mask, (N, H, L, S))
            else:
                raise RuntimeError("attn_mask must be 2-D [L, S] or 3-D [N * num_heads, L, S]")
        if key_padding_mask is not None:
            kp = as_float(key_padding_mask, (N, 1, 1, S))
            out = kp if out is None else out + kp
        return out

    def forward(self, query, key, value, key_padding_mask=None, need_weights=False,
                attn_mask=None, average_attn_weights=True, is_causal=False):
        """Returns (output, weights).  output is [L, N, E] ([N, L, E] with
        batch_first); weights is None unless need_weights, then the softmax
        weights averaged over heads [N, L, S] (PyTorch's default), or per head
        [N, H, L, S] with average_attn_weights=False (what the reference
        returns, attention.ts:260-266).  is_causal is PyTorch's hint that
        attn_mask is the causal mask: it needs attn_mask, and without a
        key-padding mask or weights the causal kernels run in its place."""
        E, H, hd = self.embed_dim, self.num_heads, self.head_dim
        if query.shape[-1] != E:
            raise RuntimeError("MultiheadAttention: expected embed_dim %d, got %d"
                               % (E, query.shape[-1]))
        if is_causal and attn_mask is None:
            raise RuntimeError("Need attn_mask if specifying the is_causal hint")
        causal = bool(is_causal and key_padding_mask is None and not need_weights)
        if causal:
            attn_mask = None
        if self.batch_first:
            N, L = query.shape[0], query.shape[1]
            S = key.shape[1]
        else:
            L, N = query.shape[0], query.shape[1]
            S = key.shape[0]
        if query is key and key is value:
            q, k, v = self._project(query, 0, 3)
        elif key is value:
            q, = self._project(query, 0, 1)
            k, v = self._project(key, 1, 2)
        else:
            q, = self._project(query, 0, 1)
            k, = self._project(key, 1, 1)
            v, = self._project(value, 2, 1)

        def heads(t, T):  # [N, H, T, hd] view of a projection
            if self.batch_first:
                return t.view(N, T, H, hd).transpose(1, 2)
            return t.view(T, N, H, hd).permute(1, 2, 0, 3)
        q, k, v = heads(q, L), heads(k, S), heads(v, S)
        mask = self._mask(N, L, S, attn_mask, key_padding_mask)
        weights = None
        if need_weights:
            scores = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(hd))
            if mask is not None:
                scores = scores + mask
            p = F.softmax(scores, -1)
            y = p @ v
            weights = p.mean(1) if average_attn_weights else p
        else:
            y = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal)
        # [N, H, L, hd] -> [N, L, E] rows, then the output projection
        y = y.transpose(1, 2).contiguous().view(N, L, E)
        out = F.linear(y, self.out_proj_weight, self.out_proj_bias)
        if not self.batch_first:
            out = out.transpose(0, 1)
        return out, weights


class ReLU(Module):
    def forward(self, x):
        return F.relu(x)


class GELU(Module):
    def forward(self, x):
        return F.gelu(x)


class Sigmoid(Module):
    def forward(self, x):
        return F.sigmoid(x)


class Tanh(Module):
    def forward(self, x):
        return F.tanh(x)


class Identity(Module):
    def forward(self, x):
        return x


class Dropout(Module):
    """Identity in eval mode or with p == 0 (the configs use no dropout)."""

    def __init__(self, p=0.5):
        super().__init__()
        self.p = p

    def forward(self, x):
        if not self.training or self.p == 0:
            return x
        raise NotImplementedError("Dropout with p > 0 in training mode is not on the hip path")


class Flatten(Module):
    def __init__(self, start_dim=1, end_dim=-1):
        super().__init__()
        self.start_dim, self.end_dim = start_dim, end_dim

    def forward(self, x):
        return x.flatten(self.start_dim, self.end_dim)


class Sequential(Module):
    """nn.Sequential (src/nn/sequential.ts:24-30)."""

    def __init__(self, *mods):
        super().__init__()
        for i, m in enumerate(mods):
            self.register_module(str(i), m)

    def forward(self, x):
        for m in self._modules.values():
            x = m(x)
        return x

    def __getitem__(self, i):
        return list(self._modules.values())[i]

    def __len__(self):
        return len(self._modules)


class ModuleList(Module):
    def __init__(self, mods=()):
        super().__init__()
        for i, m in enumerate(mods):
            self.register_module(str(i), m)

    def __iter__(self):
        return iter(self._modules.values())

    def __getitem__(self, i):
        return list(self._modules.values())[i]

    def __len__(self):
        return len(self._modules)

    def append(self, m):
        self.register_module(str(len(self._modules)), m)
        return self


class CrossEntropyLoss(Module):
    """nn.CrossEntropyLoss(weight, reduction, label_smoothing)
    (src/nn/losses.ts:100-124; torch.js's positional order, ignore_index
    keyword-only)."""

    def __init__(self, weight=None, reduction="mean", label_smoothing=0.0, *, ignore_index=-100):
        super().__init__()
        self.weight, self.reduction = weight, reduction
        self.ignore_index, self.label_smoothing = ignore_index, label_smoothing

    def forward(self, input, target):
        return F.cross_entropy(input, target, self.weight, self.reduction, self.label_smoothing,
                               ignore_index=self.ignore_index)


class NLLLoss(Module):
    """nn.NLLLoss(weight, reduction) (src/nn/losses.ts:38-57)."""

    def __init__(self, weight=None, reduction="mean", *, ignore_index=-100):
        super().__init__()
        self.weight, self.reduction, self.ignore_index = weight, reduction, ignore_index

    def forward(self, input, target):
        return F.nll_loss(input, target, self.weight, self.reduction,
                          ignore_index=self.ignore_index)


class MSELoss(Module):
    def __init__(self, reduction="mean"):
        super().__init__()
        self.reduction = reduction

    def forward(self, input, target):
        return F.mse_loss(input, target, self.reduction)


def _fans(t):
    """(fan_in, fan_out) of a weight [out, in, *receptive] (PyTorch's rule;
    torch.js's getFanOut drops the receptive field, init.ts:219-228)."""
    if t.ndim < 2:
        raise ValueError("Fan in and fan out can not be computed for tensor with fewer than "
                         "2 dimensions")
    rf = 1
    for s in t.shape[2:]:
        rf *= s
    return t.shape[1] * rf, t.shape[0] * rf


def calculate_gain(nonlinearity, param=None):
    """nn.init.calculate_gain (init.ts:194-207)."""
    if nonlinearity in ("linear", "conv1d", "conv2d", "conv3d", "conv_transpose1d",
                        "conv_transpose2d", "conv_transpose3d", "sigmoid"):
        return 1.0
    if nonlinearity == "tanh":
        return 5.0 / 3.0
    if nonlinearity == "relu":
        return math.sqrt(2.0)
    if nonlinearity == "leaky_relu":
        slope = 0.01 if param is None else float(param)
        return math.sqrt(2.0 / (1.0 + slope * slope))
    if nonlinearity == "selu":
        return 3.0 / 4.0
    raise ValueError("unsupported nonlinearity %s" % (nonlinearity,))


class init:
    """nn.init (src/nn/init.ts:10-160) over the device generator: every
    random fill draws one seeded rand / randn call (the LCG seed stream of
    manual_seed, creation.ts:921), so initialisation is reproducible
    (torch.js's uniform_ uses unseeded Math.random, init.ts:69-79).  The
    fills run under no_grad and keep the tensor's identity (leaf
    parameters stay leaves)."""

    calculate_gain = staticmethod(calculate_gain)
    calculateGain = staticmethod(calculate_gain)

    @staticmethod
    def _assign(t, src):
        from .tensor import _copy_into, no_grad
        with no_grad():
            _copy_into(t, src)
        return t

    @staticmethod
    def constant_(t, val):
        from .tensor import no_grad
        with no_grad():
            t.fill_(float(val))
        return t

    @staticmethod
    def zeros_(t):
        return init.constant_(t, 0.0)

    @staticmethod
    def ones_(t):
        return init.constant_(t, 1.0)

    @staticmethod
    def eye_(t):
        """Identity into a 2-D tensor (init.ts:44-52; PyTorch also takes
        non-square ones)."""
        from .tensor import Tensor, no_grad
        if t.ndim != 2:
            raise ValueError("eye_ requires a 2-D tensor")
        with no_grad():
            t.zero_()
            n = min(t.shape)
            diag = Tensor(t._storage, (n,), (t._strides[0] + t._strides[1],), t._offset,
                          t._dtype)
            diag.fill_(1.0)
        return t

    @staticmethod
    def normal_(t, mean=0.0, std=1.0):
        """mean + std * randn (init.ts:58-63)."""
        if std < 0:
            raise ValueError("normal_: std must be non-negative")
        from .tensor import no_grad
        with no_grad():
            return init._assign(t, randn(*t.shape).mul(float(std)).add(float(mean)))

    @staticmethod
    def uniform_(t, a=0.0, b=1.0):
        """a + (b - a) * rand (init.ts:69-79), from the seeded device stream."""
        from .tensor import no_grad, rand
        with no_grad():
            return init._assign(t, rand(*t.shape).mul(float(b) - float(a)).add(float(a)))

    @staticmethod
    def xavier_uniform_(t, gain=1.0):
        """U(-a, a), a = gain * sqrt(6 / (fan_in + fan_out)) (init.ts:85-92)."""
        fi, fo = _fans(t)
        a = gain * math.sqrt(2.0 / (fi + fo)) * math.sqrt(3.0)
        return init.uniform_(t, -a, a)

    @staticmethod
    def xavier_normal_(t, gain=1.0):
        """N(0, gain^2 * 2 / (fan_in + fan_out)) (init.ts:98-104)."""
        fi, fo = _fans(t)
        return init.normal_(t, 0.0, gain * math.sqrt(2.0 / (fi + fo)))

    @staticmethod
    def kaiming_uniform_(t, a=0.0, mode="fan_in", nonlinearity="leaky_relu"):
        """U(-b, b), b = gain * sqrt(3 / fan) (init.ts:110-124)."""
        fi, fo = _fans(t)
        fan = fi if mode == "fan_in" else fo
        bound = calculate_gain(nonlinearity, a) / math.sqrt(fan) * math.sqrt(3.0)
        return init.uniform_(t, -bound, bound)

    @staticmethod
    def kaiming_normal_(t, a=0.0, mode="fan_in", nonlinearity="leaky_relu"):
        """N(0, gain^2 / fan) (init.ts:130-144)."""
        fi, fo = _fans(t)
        fan = fi if mode == "fan_in" else fo
        return init.normal_(t, 0.0, calculate_gain(nonlinearity, a) / math.sqrt(fan))
