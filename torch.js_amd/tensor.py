"""Tensor, device storage and the autograd engine of the 'hip' device.

Mirrors torch.js's Tensor (src/tensor/Tensor.ts) for the autograd hot
path: a Tensor owns (a view of) one device allocation made by the
library's caching allocator, ops launch the library's HIP kernels on its
single stream, and `backward()` walks the recorded graph in reverse
topological order (Tensor.backward, Tensor.ts:3686-3740) with the
PyTorch semantics torch.js declares:

  * gradients ACCUMULATE into leaf `.grad` across backward calls until
    zero_grad() (torch.js clears them on every call, Tensor.ts:3714-3719);
  * every op that torch.js records has a correct vector-Jacobian product
    (torch.js's matmul, t(), broadcast, GELU, softmax, LayerNorm,
    Embedding, conv, expand and masked_fill gradients are missing or wrong,
    Tensor.ts:2212-2221, 3395-3404, 3560-3564, 3627-3632, ...);
  * views (reshape, transpose, permute, expand, narrow, indexing) share
    storage and carry strides, so transposed GEMM operands and broadcast
    gradients never materialise a copy; storage is reference counted, so
    destroying one alias never frees another's memory (torch.js frees the
    buffer of every alias, Tensor.ts:241-251).
"""
import ctypes
import functools
import math
import numbers
import os
import struct
import weakref

import numpy as np

from . import _lib as L

# ----------------------------------------------------------------- dtypes

# torch.js stores integer tensors as Int32Array (src/dtype.ts:7-15); int64
# requests map to int32 the same way.
_DT = {
    "float32": (4, np.float32),
    "int32": (4, np.int32),
    "uint8": (1, np.uint8),
    "bool": (1, np.uint8),
}
_ALIAS = {"float": "float32", "float16": "float32", "int64": "int32", "long": "int32",
          "int": "int32", "uint32": "int32", "int8": "int32"}


def _norm_dtype(dt):
    if dt is None:
        return "float32"
    if not isinstance(dt, str):
        dt = np.dtype(dt).name
    dt = _ALIAS.get(dt, dt)
    if dt not in _DT:
        raise TypeError("unsupported dtype %r" % (dt,))
    return dt


# ----------------------------------------------------------------- device state

_state = {"init": False, "ordinal": 0, "seed": None}


def init(ordinal=0):
    """Initialises the 'hip' device (torch.init / initWebGPU,
    src/backend/webgpu/device.ts:27-86).  Idempotent."""
    lib = L.lib()
    L.check(lib.tjh_init(int(ordinal)), "torch.init")
    _state["init"] = True
    _state["ordinal"] = int(ordinal)
    return None


def is_initialized():
    return _state["init"]


def _require_init():
    if not _state["init"]:
        raise RuntimeError("hip backend not initialized. Call torch.init() first.")


def synchronize():
    """Waits for all queued device work (syncDevice, dispatch.ts:115-118)."""
    _require_init()
    L.check(L.lib().tjh_synchronize(), "synchronize")


# ----------------------------------------------------------------- grad mode

_grad = {"enabled": True}
# the implicit seed of the running Tensor.backward() and the id of the root's
# node: the seed is the root VJP's upstream gradient, equal to 1
_unit_seed = {"node": None, "g": None}


def is_grad_enabled():
    return _grad["enabled"]


class set_grad_enabled:
    """Context manager / function (src/grad_mode.ts)."""

    def __init__(self, mode):
        self.prev = _grad["enabled"]
        _grad["enabled"] = bool(mode)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        _grad["enabled"] = self.prev
        return False


class no_grad:
    """Disables graph recording (torch.no_grad).  torch.js's constructor
    never disables it (src/grad_mode.ts:27-29); this one does."""

    def __enter__(self):
        self.prev = _grad["enabled"]
        _grad["enabled"] = False
        return self

    def __exit__(self, *exc):
        _grad["enabled"] = self.prev
        return False

    def __call__(self, fn):
        def wrapper(*a, **k):
            with no_grad():
                return fn(*a, **k)
        wrapper.__name__ = getattr(fn, "__name__", "wrapped")
        return wrapper


class enable_grad(no_grad):
    def __enter__(self):
        self.prev = _grad["enabled"]
        _grad["enabled"] = True
        return self


inference_mode = no_grad

# ----------------------------------------------------------------- storage


class Storage:
    """One device allocation from the library's stream-ordered cache."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes):
        self.ptr = 0
        _require_init()
        p = ctypes.c_void_p()
        L.check(L.lib().tjh_malloc(int(nbytes), ctypes.byref(p)), "malloc")
        self.ptr = p.value or 0
        self.nbytes = int(nbytes)

    def __del__(self):
        lib = L._lib
        if lib is not None and self.ptr:
            try:
                lib.tjh_free(self.ptr)
            except Exception:
                pass
            self.ptr = 0


@functools.lru_cache(maxsize=4096)
def _contig_strides_t(shape):
    st = [1] * len(shape)
    s = 1
    for d in range(len(shape) - 1, -1, -1):
        st[d] = s
        s *= shape[d]
    return tuple(st)


def _contig_strides(shape):
    return _contig_strides_t(shape if type(shape) is tuple else tuple(shape))


def _numel(shape):
    n = 1
    for s in shape:
        n *= s
    return n


def _broadcast_shapes(a, b):
    """broadcastShapes (src/utils/broadcast.ts:11-37)."""
    n = max(len(a), len(b))
    out = []
    for i in range(n):
        da = a[len(a) - n + i] if len(a) - n + i >= 0 else 1
        db = b[len(b) - n + i] if len(b) - n + i >= 0 else 1
        if da != db and da != 1 and db != 1:
            raise ValueError("shapes %s and %s are not broadcastable" % (list(a), list(b)))
        out.append(max(da, db) if da != 0 and db != 0 else 0)
    return tuple(out)


def _wrap_dim(d, ndim):
    if ndim == 0 and d in (0, -1):
        return 0
    if d < -ndim or d >= ndim:
        raise IndexError("dimension %d out of range for %d-d tensor" % (d, ndim))
    return d + ndim if d < 0 else d


# ----------------------------------------------------------------- autograd node


class Node:
    """grad_fn: the vector-Jacobian product of one recorded op
    (GradFn, src/tensor/types.ts:13-17).  `inputs` are the op's tensor
    arguments; `fn(grad)` returns one gradient (or None) per input.

    `acc_slot`: index of an input whose gradient the VJP can add to a
    gradient already pending for that input, in the same kernel: the
    engine then calls `fn(grad, pending=...)` and takes the returned
    gradient as the input's whole gradient (the residual stream of a pre-LN
    block sums the identity path and the LayerNorm path this way).

    `defer_slots`: inputs whose gradients the VJP may leave unfinished
    until the library's tjh_flush_deferred (`fn(grad, defer=True)`); the
    engine allows it when each of them is a leaf receiving its first
    gradient of the pass, and flushes before any of those gradients is
    read (a second contribution, the end of the pass).

    `gfn(grad)`: the same vector-Jacobian product written with recording
    ops, for backward passes that build a graph of their own
    (create_graph=True, second derivatives); None where the op has none."""

    __slots__ = ("name", "inputs", "fn", "acc_slot", "defer_slots", "gfn", "__weakref__")

    def __init__(self, name, inputs, fn, acc_slot=None, defer_slots=(), gfn=None):
        self.name = name
        self.inputs = inputs
        self.fn = fn
        self.acc_slot = acc_slot
        self.defer_slots = defer_slots
        self.gfn = gfn

    def __repr__(self):
        return "<%sBackward>" % self.name

    # torch.js exposes grad_fn._next_tensors (Tensor.ts:3702-3708)
    @property
    def next_tensors(self):
        return [t for t in self.inputs if t is not None]


def _record(out, name, inputs, fn, acc_slot=None, defer_slots=(), gfn=None):
    if _grad["enabled"] and any(t is not None and t.requires_grad for t in inputs):
        out.requires_grad = True
        out.grad_fn = Node(name, [t if (t is not None and t.requires_grad) else None
                                  for t in inputs], fn, acc_slot, defer_slots, gfn)
    return out


# ----------------------------------------------------------------- tensor


class Tensor:
    """A strided view of device memory on the 'hip' device."""

    __slots__ = ("_st", "_lz", "_offset", "_shape", "_strides", "_dtype", "requires_grad",
                 "_grad", "grad_fn", "_retains_grad", "__weakref__")

    def __init__(self, storage, shape, strides=None, offset=0, dtype="float32",
                 requires_grad=False):
        self._st = storage
        self._lz = None  # a deferred elementwise op (_Lz) while _st is None
        self._shape = tuple(map(int, shape))
        self._strides = tuple(strides) if strides is not None else _contig_strides(self._shape)
        self._offset = int(offset)
        self._dtype = dtype
        self.requires_grad = bool(requires_grad)
        self._grad = None
        self.grad_fn = None
        self._retains_grad = False

    # ------------------------------------------------------------ metadata
    @property
    def _storage(self):
        """The device allocation; a deferred elementwise value is computed
        (one fused kernel) the first time anything needs its memory."""
        st = self._st
        if st is None:
            st = _realize(self)
        return st

    @property
    def shape(self):
        return self._shape

    @property
    def dtype(self):
        return self._dtype

    @property
    def device(self):
        return "hip"

    @property
    def ndim(self):
        return len(self._shape)

    def dim(self):
        return len(self._shape)

    def numel(self):
        return _numel(self._shape)

    def size(self, dim=None):
        if dim is None:
            return self._shape
        return self._shape[_wrap_dim(dim, self.ndim)]

    def stride(self, dim=None):
        if dim is None:
            return self._strides
        return self._strides[_wrap_dim(dim, self.ndim)]

    @property
    def itemsize(self):
        return _DT[self._dtype][0]

    @property
    def is_leaf(self):
        return self.grad_fn is None

    @property
    def grad(self):
        return self._grad

    @grad.setter
    def grad(self, g):
        self._grad = g

    def data_ptr(self):
        st = self._st
        if st is None:
            st = _realize(self)
        return st.ptr + self._offset * _DT[self._dtype][0]

    def is_contiguous(self):
        return self._strides == _contig_strides(self._shape) or self.numel() <= 1 or \
            all(st == cs for st, cs, sz in zip(self._strides, _contig_strides(self._shape),
                                               self._shape) if sz != 1)

    def retain_grad(self):
        self._retains_grad = True
        return self

    def requires_grad_(self, value=True):
        self.requires_grad = bool(value)
        return self

    def __repr__(self):
        try:
            arr = self.numpy()
            body = np.array2string(arr, precision=4, threshold=20)
        except Exception as e:  # pragma: no cover
            body = "<unreadable: %s>" % e
        gf = ", grad_fn=%r" % self.grad_fn if self.grad_fn is not None else ""
        return "tensor(%s, device='hip', dtype=%s%s)" % (body, self._dtype, gf)

    def __len__(self):
        if not self._shape:
            raise TypeError("len() of a 0-d tensor")
        return self._shape[0]

    # ------------------------------------------------------------ host copies
    def numpy(self):
        """Blocking device->host copy (readBuffer, buffer.ts:150-206)."""
        t = self if self.is_contiguous() else _k_contiguous(self)
        npdt = _DT[t._dtype][1]
        out = np.empty(t._shape, dtype=npdt)
        if out.size:
            L.check(L.lib().tjh_d2h(out.ctypes.data, t.data_ptr(), out.nbytes), "d2h")
        return out

    def toArray(self):
        """Flat list like torch.js's toArray(), -0 normalised to 0
        (Tensor.ts:253-257)."""
        a = self.numpy().reshape(-1)
        if a.dtype == np.float32:
            a = a + np.float32(0.0)  # -0 -> +0
        return a.tolist()

    def tolist(self):
        return self.numpy().tolist()

    def item(self):
        if self.numel() != 1:
            raise ValueError("item() needs a one-element tensor, got shape %s" % (list(self._shape),))
        return self.numpy().reshape(-1)[0].item()

    def __float__(self):
        return float(self.item())

    # ------------------------------------------------------------ autograd
    def backward(self, gradient=None, retain_graph=False, create_graph=False):
        """Tensor.backward (Tensor.ts:3686-3740).  With create_graph the
        gradients carry graphs of their own (leaf .grad can be
        differentiated again)."""
        if not self.requires_grad:
            raise RuntimeError("element 0 of tensors does not require grad and does not have a grad_fn")
        if gradient is None:
            if self.numel() != 1:
                raise RuntimeError("grad can be implicitly created only for scalar outputs")
            gradient = full(self._shape, 1.0)
            if not create_graph:
                # known on the host to be 1 where it reaches the root's own
                # VJP: a loss may have formed its input's gradient for that
                # seed already (cross_entropy)
                _unit_seed["node"], _unit_seed["g"] = id(self.grad_fn), gradient
        try:
            run_backward([(self, gradient)], retain_graph=retain_graph or create_graph,
                         create_graph=create_graph)
        finally:
            _unit_seed["node"] = _unit_seed["g"] = None

    def detach(self):
        if self._st is None:  # stays deferred, sharing the value
            return _lazy("alias", 0, 0.0, (self,), self._shape)
        return Tensor(self._storage, self._shape, self._strides, self._offset, self._dtype)

    def detach_(self):
        self.grad_fn = None
        self.requires_grad = False
        return self

    def zero_(self):
        _require_writable(self)
        _fill_view(self, 0.0)
        return self

    def fill_(self, value):
        _require_writable(self)
        _fill_view(self, float(value))
        return self

    def copy_(self, src):
        """In-place copy (Tensor.copy_, Tensor.ts:437-446); broadcasts src."""
        _require_writable(self)
        src = _as_tensor(src, like=self)
        if src._dtype != self._dtype:
            src = src.to(self._dtype)
        s = src.expand(self._shape) if src._shape != self._shape else src
        _copy_into(self, s)
        return self

    def to(self, arg=None, dtype=None):
        """Tensor.to(dtype | device) (Tensor.ts:904-936)."""
        target = dtype if dtype is not None else arg
        if target in (None, "hip", "cuda", "webgpu"):
            return self
        if target == "cpu":
            raise RuntimeError("the hip device has no CPU tensors; use .numpy() to read values")
        dt = _norm_dtype(target)
        if dt == self._dtype:
            return self
        return _k_cast(self, dt)

    def bool(self):
        return self.to("bool")

    def float(self):
        return self.to("float32")

    def int(self):
        return self.to("int32")

    def long(self):
        return self.to("int32")

    # ------------------------------------------------------------ operators
    def __add__(self, o):
        return add(self, o)

    def __radd__(self, o):
        return add(self, o)

    def __sub__(self, o):
        return sub(self, o)

    def __rsub__(self, o):
        return rsub(self, o)

    def __mul__(self, o):
        return mul(self, o)

    def __rmul__(self, o):
        return mul(self, o)

    def __truediv__(self, o):
        return div(self, o)

    def __rtruediv__(self, o):
        return rdiv(self, o)

    def __pow__(self, o):
        return pow(self, o)

    def __neg__(self):
        return neg(self)

    def __matmul__(self, o):
        return matmul(self, o)

    def __getitem__(self, idx):
        return _getitem(self, idx)

    def __lt__(self, o):
        return compare(self, o, "lt")

    def __le__(self, o):
        return compare(self, o, "le")

    def __gt__(self, o):
        return compare(self, o, "gt")

    def __ge__(self, o):
        return compare(self, o, "ge")

    # torch.js method names (Tensor.ts:476-2600)
    def add(self, o, alpha=1.0):
        if alpha != 1.0:
            o = mul(o, alpha) if isinstance(o, Tensor) else o * alpha
        return add(self, o)

    def sub(self, o):
        return sub(self, o)

    def mul(self, o):
        return mul(self, o)

    def div(self, o):
        return div(self, o)

    def pow(self, o):
        return pow(self, o)

    def neg(self):
        return neg(self)

    def matmul(self, o):
        return matmul(self, o)

    def mm(self, o):
        if self.ndim != 2 or o.ndim != 2:
            raise RuntimeError("mm expects 2-D tensors")
        return matmul(self, o)

    def bmm(self, o):
        if self.ndim != 3 or o.ndim != 3:
            raise RuntimeError("bmm expects 3-D tensors")
        return matmul(self, o)

    def maximum(self, o):
        return _binary_op("maximum", self, o)

    def minimum(self, o):
        return _binary_op("minimum", self, o)

    def eq(self, o):
        return compare(self, o, "eq")

    def ne(self, o):
        return compare(self, o, "ne")

    def lt(self, o):
        return compare(self, o, "lt")

    def le(self, o):
        return compare(self, o, "le")

    def gt(self, o):
        return compare(self, o, "gt")

    def ge(self, o):
        return compare(self, o, "ge")

    def sum(self, dim=None, keepdim=False):
        return reduce_sum(self, dim, keepdim)

    def mean(self, dim=None, keepdim=False):
        return reduce_mean(self, dim, keepdim)

    def amax(self, dim=None, keepdim=False):
        return reduce_minmax(self, dim, keepdim, "max")

    def amin(self, dim=None, keepdim=False):
        return reduce_minmax(self, dim, keepdim, "min")

    def max(self, dim=None, keepdim=False):
        return reduce_minmax(self, dim, keepdim, "max")

    def min(self, dim=None, keepdim=False):
        return reduce_minmax(self, dim, keepdim, "min")

    def argmax(self, dim=None, keepdim=False):
        return argmax(self, dim, keepdim)

    def triu(self, diagonal=0):
        return triangle(self, diagonal, True)

    def tril(self, diagonal=0):
        return triangle(self, diagonal, False)

    def multinomial(self, num_samples=1, replacement=False):
        return multinomial(self, num_samples, replacement)

    def clamp(self, min=None, max=None):
        return clamp(self, min, max)

    def clamp_min(self, min):
        return clamp(self, min, None)

    def clamp_max(self, max):
        return clamp(self, None, max)

    clip = clamp

    def argmin(self, dim=None, keepdim=False):
        return argmax(self, dim, keepdim, is_min=True)

    def softmax(self, dim=-1):
        from .functional import softmax as _softmax
        return _softmax(self, dim)

    def log_softmax(self, dim=-1):
        from .functional import log_softmax as _log_softmax
        return _log_softmax(self, dim)

    def masked_fill(self, mask, value):
        return masked_fill(self, mask, value)

    def index_select(self, dim, index):
        return index_select(self, dim, index)

    def gather(self, dim, index):
        return gather(self, dim, index)

    def nonzero(self):
        return nonzero(self)

    def clone(self):
        return clone(self)

    def contiguous(self):
        return contiguous(self)

    def reshape(self, *shape):
        return reshape(self, _shape_arg(shape))

    def view(self, *shape):
        return view(self, _shape_arg(shape))

    def flatten(self, start_dim=0, end_dim=-1):
        return flatten(self, start_dim, end_dim)

    def squeeze(self, dim=None):
        return squeeze(self, dim)

    def unsqueeze(self, dim):
        return unsqueeze(self, dim)

    def transpose(self, d0, d1):
        return transpose(self, d0, d1)

    def swapaxes(self, d0, d1):
        return transpose(self, d0, d1)

    def permute(self, *dims):
        return permute(self, _shape_arg(dims))

    def t(self):
        if self.ndim > 2:
            raise RuntimeError("t() expects a tensor with <= 2 dimensions")
        return transpose(self, 0, 1) if self.ndim == 2 else self

    @property
    def T(self):
        return permute(self, tuple(range(self.ndim - 1, -1, -1)))

    def expand(self, *shape):
        return expand(self, _shape_arg(shape))

    def broadcast_to(self, shape):
        return expand(self, tuple(shape))

    def expand_as(self, other):
        return expand(self, other.shape)

    def narrow(self, dim, start, length):
        return narrow(self, dim, start, length)

    def split(self, split_size, dim=0):
        return split(self, split_size, dim)

    def chunk(self, chunks, dim=0):
        return chunk(self, chunks, dim)

    def unbind(self, dim=0):
        return [select(self, dim, i) for i in range(self.shape[_wrap_dim(dim, self.ndim)])]

    def select(self, dim, index):
        return select(self, dim, index)


def _shape_arg(shape):
    if len(shape) == 1 and isinstance(shape[0], (list, tuple)):
        return tuple(shape[0])
    return tuple(shape)


def _add_unary_methods():
    names = ["exp", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "relu", "gelu", "square",
             "reciprocal", "erf", "abs", "sin", "cos", "silu", "softplus", "sign"]
    for n in names:
        def m(self, _n=n):
            return unary(_n, self)
        m.__name__ = n
        setattr(Tensor, n, m)

    def leaky_relu(self, negative_slope=0.01):
        return unary("leaky_relu", self, negative_slope)

    def elu(self, alpha=1.0):
        return unary("elu", self, alpha)

    Tensor.leaky_relu = leaky_relu
    Tensor.elu = elu


# ----------------------------------------------------------------- allocation


def empty(shape, dtype="float32", requires_grad=False):
    shape = tuple(int(s) for s in shape)
    dtype = _norm_dtype(dtype)
    st = Storage(max(1, _numel(shape)) * _DT[dtype][0])
    return Tensor(st, shape, None, 0, dtype, requires_grad)


def _empty_padded(rows, cols):
    """[rows, cols] fp32 whose row stride is rounded up to 4 floats, so every
    row starts 16-byte aligned (GEMM outputs whose N is not a multiple of
    4, e.g. a 50257-wide vocabulary)."""
    ld = (cols + 3) // 4 * 4
    st = Storage(max(1, rows * ld) * 4)
    return Tensor(st, (rows, cols), (ld, 1), 0, "float32")


def _fill_view(t, value):
    _before_write(t)
    lib = L.lib()
    if t.numel() == 0:
        return
    if t.is_contiguous():
        if t._dtype == "float32":
            L.check(lib.tjh_fill_f32(t.data_ptr(), t.numel(), float(value)), "fill")
        elif t._dtype == "int32":
            L.check(lib.tjh_fill_i32(t.data_ptr(), t.numel(), int(value)), "fill")
        else:
            v = (1 if value else 0) if t._dtype == "bool" else int(value) & 0xFF
            L.check(lib.tjh_fill_u8(t.data_ptr(), t.numel(), v), "fill")
        return
    src = full((1,), value, dtype=t._dtype).expand(t._shape)
    _copy_into(t, src)


def _require_writable(t):
    _before_write(t)
    if _grad["enabled"] and t.requires_grad and t.is_leaf:
        raise RuntimeError("a leaf Variable that requires grad is being used in an in-place operation.")


def full(shape, value, dtype="float32", requires_grad=False):
    t = empty(shape, dtype)
    _fill_view(t, value)
    t.requires_grad = requires_grad
    return t


def zeros(*shape, dtype="float32", requires_grad=False):
    return full(_shape_arg(shape), 0.0, dtype, requires_grad)


def ones(*shape, dtype="float32", requires_grad=False):
    return full(_shape_arg(shape), 1.0, dtype, requires_grad)


def zeros_like(t, dtype=None, requires_grad=False):
    return full(t.shape, 0.0, dtype or t.dtype, requires_grad)


def ones_like(t, dtype=None, requires_grad=False):
    return full(t.shape, 1.0, dtype or t.dtype, requires_grad)


def full_like(t, value, dtype=None, requires_grad=False):
    return full(t.shape, value, dtype or t.dtype, requires_grad)


def from_numpy(a, requires_grad=False, dtype=None):
    a = np.asarray(a)
    if dtype is None:
        if a.dtype.kind == "f":
            dtype = "float32"
        elif a.dtype.kind == "b":
            dtype = "bool"
        elif a.dtype.kind in "iu":
            dtype = "int32"
        else:
            raise TypeError("unsupported numpy dtype %s" % a.dtype)
    dtype = _norm_dtype(dtype)
    a = np.asarray(a, dtype=_DT[dtype][1])  # keeps 0-d arrays 0-d
    if not a.flags.c_contiguous:
        a = a.copy(order="C")
    t = empty(a.shape, dtype)
    if a.size:
        L.check(L.lib().tjh_h2d(t.data_ptr(), a.ctypes.data, a.nbytes), "h2d")
    t.requires_grad = requires_grad
    return t


def tensor(data, dtype=None, device="hip", requires_grad=False):
    """torch.tensor (src/ops/creation.ts:60-84).  Python numbers are JS
    numbers there, so lists default to float32; numpy arrays keep their
    kind (integer arrays become int32)."""
    if isinstance(data, Tensor):
        t = clone(data.detach())
        if dtype is not None:
            t = t.to(dtype)
        t.requires_grad = requires_grad
        return t
    if isinstance(data, np.ndarray):
        return from_numpy(data, requires_grad=requires_grad, dtype=dtype)
    a = np.asarray(data, dtype=np.float64)
    return from_numpy(a, requires_grad=requires_grad, dtype=dtype or "float32")


def manual_seed(seed):
    """Sets the global seed of rand/randn (src/ops/creation.ts:906-908)."""
    _state["seed"] = int(seed)


def _next_seed():
    # torch.js seeds each rand/randn call with an LCG step of a global seed
    # (src/ops/creation.ts:921); an unset seed starts from a random value.
    # The step is JavaScript arithmetic: the product and the sum are IEEE
    # doubles (products above 2^53 round before the mask), then ToInt32 and
    # `& 0x7fffffff` keep the low 31 bits of the rounded integer.
    if _state["seed"] is None:
        _state["seed"] = int(np.random.randint(0, 2147483647))
    v = float(_state["seed"]) * 1103515245.0 + 12345.0
    _state["seed"] = int(v) & 0x7FFFFFFF
    return _state["seed"]


def _random(shape, normal, requires_grad):
    t = empty(_shape_arg(shape))
    if t.numel():
        L.check(L.lib().tjh_random(t.data_ptr(), t.numel(), _next_seed(), 1 if normal else 0),
                "random")
    t.requires_grad = requires_grad
    return t


def rand(*shape, requires_grad=False, dtype=None):
    """U[0,1) from random.wgsl:17-29's xorshift generator."""
    return _random(shape, False, requires_grad)


def randn(*shape, requires_grad=False, dtype=None):
    """N(0,1) by Box-Muller from random.wgsl:31-46's generator."""
    return _random(shape, True, requires_grad)


def arange(start, end=None, step=1, dtype=None, requires_grad=False):
    if end is None:
        start, end = 0, start
    isint = all(float(v).is_integer() for v in (start, end, step))
    dtype = _norm_dtype(dtype or ("int32" if isint else "float32"))
    a = np.arange(start, end, step).astype(_DT[dtype][1])
    return from_numpy(a, requires_grad=requires_grad, dtype=dtype)


def _as_tensor(x, like=None):
    if isinstance(x, Tensor):
        return x
    dt = like.dtype if like is not None and like.dtype == "float32" else "float32"
    return full((), float(x), dtype=dt)


# ----------------------------------------------------------------- deferred elementwise ops
# torch.js runs each elementwise op as its own submit (Tensor.ts _unaryOp /
# _binaryOp / _scalarOp, 3409-3656, 3742-3792).  Here an elementwise op on
# a float32 tensor of at least _LAZY["min"] elements returns a tensor whose
# value is deferred: it records the op and its inputs.  A chain of such ops
# is evaluated by one fused kernel (tjh_expr_eval) the first time anything
# needs the memory of a value in it (a GEMM, a readback, a view), and a
# column sum of a deferred value (`sum(0)`, the bias gradient of a
# broadcast add) reads the chain's inputs directly (tjh_expr_colsum), so
# the intermediates of the chain are never written.  The autograd VJPs use
# the same ops, so a backward through such a chain is deferred too and
# recomputes the forward intermediates from their inputs.
#
# Values are those of the op-by-op kernels, bit for bit.  Writes: before
# any in-place write to a storage, every deferred value that reads it is
# evaluated (_before_write), so a deferred value never sees a later write.
# TJH_LAZY=0 turns deferral off.

_LAZY = {"on": os.environ.get("TJH_LAZY", "1") != "0", "min": 1 << 16, "jit": True}
_PENDING = {}  # id -> weakref of each deferred tensor not yet evaluated


def _pend(t):
    key = id(t)
    _PENDING[key] = weakref.ref(t, lambda _r, k=key: _PENDING.pop(k, None))


def _pending_tensors():
    return [p for p in (r() for r in list(_PENDING.values())) if p is not None]
_EXPR_KIND = {"u": "unary", "ub": "unary_bwd", "b": "binary", "t": "ternary", "s": "scalar",
              "sr": "scalar_rev", "axpy": "axpy"}


class _Lz:
    """A deferred op: kind ('u' unary, 'ub' unary backward, 'b' binary,
    't' ternary, 's' / 'sr' scalar, 'axpy', 'alias', or 'thunk': a
    deferred reduction whose `name` is the function that computes it), op
    code, scalar operand, input tensors, and `deps`: ids of the storages
    and deferred tensors its value reads (transitively)."""

    __slots__ = ("kind", "code", "f", "args", "kinds", "deps", "name")

    def __init__(self, kind, code, f, args, kinds, deps, name=None):
        self.kind, self.code, self.f, self.args, self.kinds, self.deps = kind, code, f, args, \
            kinds, deps
        self.name = name  # op name of the single-op kernel


def _is_lazy(t):
    return t._st is None


def _skey(t):
    """Identity of t's storage without evaluating it: a deferred value that
    is not an alias has no storage yet, so it shares none."""
    while t._st is None:
        lz = t._lz
        if lz.kind != "alias":
            return ("deferred", id(t))
        t = lz.args[0]
    return id(t._st)


def _lazy(kind, code, f, args, shape, kinds=None, name=None):
    """A deferred op over `args` with output `shape`; `kinds[i]` is how a
    leaf argument is indexed (None: a deferred argument of the same shape,
    inlined)."""
    if kinds is None:
        kinds = [None] * len(args)
    deps = set()
    for a in args:
        if a is None:
            continue
        if a._st is None:
            deps.add(id(a))
            deps |= a._lz.deps
        else:
            deps.add(id(a._st))
    t = Tensor.__new__(Tensor)
    t._st = None
    t._lz = _Lz(kind, code, float(f), tuple(args), tuple(kinds), deps, name)
    t._shape = tuple(shape)
    t._strides = _contig_strides(t._shape)
    t._offset = 0
    t._dtype = "float32"
    t.requires_grad = False
    t._grad = None
    t.grad_fn = None
    t._retains_grad = False
    _pend(t)
    return t


def _thunk(fn, shape, inputs):
    """A deferred value computed by fn() (an evaluated tensor of `shape`)
    the first time its memory is needed: a reduction of deferred values.
    It is never inlined into a fused program (it is a leaf there)."""
    return _lazy("thunk", 0, 0.0, tuple(inputs), shape, name=fn)


# Forward column sums left deferred (_colsum_deferred): weakrefs of
# (thunk, source, dims, scale); a backward column sum over the same rows
# of values that read the same inputs computes them in its own pass.
_COLSUMS = []


def _leaf_kind(shape, bst):
    """How a leaf with strides `bst` (broadcast to `shape`) is indexed at
    flat output element e: ('contig', 0) e, ('row', P) e % P, ('col', Q)
    e / Q, ('scalar', 0); None for other layouts."""
    dims = [d for d in range(len(shape)) if shape[d] != 1]
    if not dims:
        return ("contig", 0)
    if all(bst[d] == 0 for d in dims):
        return ("scalar", 0)
    cs = _contig_strides(shape)
    if all(bst[d] == cs[d] for d in dims):
        return ("contig", 0)
    # row: leading broadcast dims, then contiguous over the trailing ones
    z = 0
    while z < len(dims) and bst[dims[z]] == 0:
        z += 1
    if 0 < z < len(dims):
        trail = dims[z:]
        inner = _contig_strides([shape[d] for d in trail])
        if all(bst[d] == st for d, st in zip(trail, inner)):
            return ("row", _numel([shape[d] for d in trail]))
    # col: contiguous over the leading dims, broadcast over the trailing ones
    z = 0
    while z < len(dims) and bst[dims[len(dims) - 1 - z]] == 0:
        z += 1
    if 0 < z < len(dims):
        lead = dims[:len(dims) - z]
        outer = _contig_strides([shape[d] for d in lead])
        if all(bst[d] == st for d, st in zip(lead, outer)):
            return ("col", _numel([shape[d] for d in dims[len(dims) - z:]]))
    return None


def _lazy_ok(shape, args):
    """The leaf kinds of `args` when an op with output `shape` may be
    deferred over them, else None."""
    if not _LAZY["on"] or _numel(shape) < _LAZY["min"]:
        return None
    shape = tuple(shape)
    kinds = []
    for a in args:
        if a is None:
            kinds.append(None)
            continue
        if a._dtype != "float32":
            return None
        if a._st is None and a._shape == shape:
            kinds.append(None)
            continue
        k = _kind_of(shape, a._shape, a._strides)
        if k is None:
            return None
        kinds.append(k)
    return kinds


@functools.lru_cache(maxsize=8192)
def _kind_of(shape, tshape, tstrides):
    """_leaf_kind of a (tshape, tstrides) tensor broadcast to `shape`."""
    return _leaf_kind(shape, _bstrides_of(tshape, tstrides, shape))


def _bstrides_of(tshape, tstrides, shape):
    nd = len(shape)
    off = nd - len(tshape)
    st = []
    for d in range(nd):
        if d < off:
            st.append(0)
        else:
            sz = tshape[d - off]
            st.append(0 if (sz == 1 and shape[d] != 1) else tstrides[d - off])
    return st


class _TooBig(Exception):
    pass


def _program(root, root2=None, root3=None):
    """The tjh_expr program of deferred tensor `root` and the tensors it
    keeps alive.  Inputs of another shape, evaluated inputs and views are
    leaves; deferred inputs of the same shape are inlined.  `root2` (same
    shape) becomes the program's second value and `root3` its third,
    sharing loads and common subexpressions with the first."""
    shape = root._shape
    leaves, leaf_ix, code, memo = [], {}, [], {}
    max_ins = L.EXPR_MAX_INS

    def emit(t, kind):
        st = t._st
        while st is None:
            lz = t._lz
            if lz.kind != "alias":
                break
            t = lz.args[0]
            st = t._st
        if st is None and t._shape == shape and t._lz.kind != "thunk":
            v = memo.get(id(t))
            if v is not None:
                return v
            lz = t._lz
            args, kinds = lz.args, lz.kinds
            ops = [None if a is None else emit(a, k) for a, k in zip(args, kinds)]
            ops += [None] * (3 - len(ops))
            code.append((_EXPR_KIND[lz.kind], lz.code, ops[0], ops[1], ops[2], lz.f))
            if len(code) > max_ins:
                raise _TooBig()
            v = memo[id(t)] = len(code) - 1
            return v
        # a leaf: an evaluated tensor, or a deferred one of another shape
        if st is None:
            st = t._storage
        if kind is None:
            kind = _kind_of(shape, t._shape, t._strides)
            if kind is None:
                t = _k_contiguous(t.expand(shape))
                st, kind = t._st, ("contig", 0)
        key = (id(st), t._offset, t._strides, t._shape)
        i = leaf_ix.get(key)
        if i is None:
            if len(leaves) >= L.EXPR_MAX_LEAVES:
                raise _TooBig()
            i = leaf_ix[key] = len(leaves)
            leaves.append((t, kind))
        v = memo.get(("leaf", i))
        if v is None:
            code.append(("load", 0, i, None, None, 0.0))
            v = memo[("leaf", i)] = len(code) - 1
        return v

    result = emit(root, None)
    result2 = emit(root2, None) if root2 is not None else None
    result3 = emit(root3, None) if root3 is not None else None
    sig = (tuple(code), result, result2, result3, tuple(k for _, k in leaves))
    hit = _PROGRAMS.get(sig)
    if hit is None:
        hit = _PROGRAMS[sig] = _pack_code(code, result, result2, result3)
        if len(_PROGRAMS) > 512:
            _PROGRAMS.pop(next(iter(_PROGRAMS)))
    buf = bytearray(hit)
    nl = len(leaves)
    _EXPR_NLEAF.pack_into(buf, 4, nl)
    if nl:
        struct.pack_into("<%dQ" % nl, buf, _EXPR_LEAF_OFF, *[a.data_ptr() for a, _ in leaves])
        struct.pack_into("<%dq" % nl, buf, _EXPR_PER_OFF, *[k[1] for _, k in leaves])
        struct.pack_into("<%di" % nl, buf, _EXPR_KIND_OFF, *[L.LEAF[k[0]] for _, k in leaves])
    return L.Expr.from_buffer(buf), [a for a, _ in leaves]


_PROGRAMS = {}  # (code, results, leaf kinds) -> packed program without its leaves


def _pack_code(code, result, result2=None, result3=None):
    """Packs instructions with registers allocated: a value's register is
    freed after its last use (the results' stay held)."""
    keep = (result, result2, result3)
    last = {}
    for i, ins in enumerate(code):
        for v in (ins[3:5] if ins[0] == "load" else ins[2:5]):  # a load's `a` is a leaf index
            if v is not None:
                last[v] = i
    free = list(range(L.EXPR_MAX_REGS))
    reg = {}
    buf = bytearray(_EXPR_SIZE)
    none = L.EXPR_NONE
    op_ids = L.EXPR_OP
    for i, (op, c, a, b, cc, f) in enumerate(code):
        for v in set(x for x in ((a, b, cc) if op != "load" else (b, cc)) if x is not None):
            if last.get(v) == i and v not in keep:
                free.append(reg[v])
        if not free:
            raise _TooBig()
        free.sort()
        r = free.pop(0)
        reg[i] = r
        if op == "load":
            ra, rb, rc = a, none, none
        else:
            ra = reg[a] if a is not None else none
            rb = reg[b] if b is not None else none
            rc = reg[cc] if cc is not None else none
        _EXPR_INS.pack_into(buf, _EXPR_INS_OFF + _EXPR_INS.size * i, op_ids[op], c, r, ra, rb, rc, f)
        if last.get(i) is None and i not in keep:
            free.append(r)  # never read
    _EXPR_HDR.pack_into(buf, 0, len(code), 0, reg[result],
                        reg[result2] + 1 if result2 is not None else 0,
                        reg[result3] + 1 if result3 is not None else 0, 0)
    return bytes(buf)


_EXPR_SIZE = ctypes.sizeof(L.Expr)
_EXPR_HDR = struct.Struct("<6i")
_EXPR_NLEAF = struct.Struct("<i")
_EXPR_INS = struct.Struct("<6B2xf")
_EXPR_INS_OFF = L.Expr.ins.offset
_EXPR_LEAF_OFF = L.Expr.leaf.offset
_EXPR_PER_OFF = L.Expr.period.offset
_EXPR_KIND_OFF = L.Expr.kind.offset
assert _EXPR_INS.size == ctypes.sizeof(L.ExprIns)


def _program_fit(t):
    """_program(t), evaluating the largest inlined inputs first until the
    program fits the instruction, leaf and register limits."""
    while True:
        try:
            return _program(t)
        except _TooBig:
            cands = [a for a in t._lz.args if a is not None and a._st is None and
                     a._shape == t._shape]
            if not cands:
                raise RuntimeError("elementwise expression too large to fuse")
            max(cands, key=lambda a: len(a._lz.deps))._storage


def _settle(t, st):
    """t's value now lives in `st`: record it and let the deferred values
    that read t know its storage."""
    t._st = st
    t._lz = None
    key = id(t)
    _PENDING.pop(key, None)
    for p in _pending_tensors():
        lz = p._lz
        if lz is not None and key in lz.deps:
            lz.deps.add(id(st))


def _realize(t):
    lz = t._lz
    if lz.kind == "thunk":
        out = lz.name()
        if out._offset or not out.is_contiguous() or out._st is None:
            out = _k_contiguous(out)
        _settle(t, out._st)
        return out._st
    if lz.kind == "alias":
        st = lz.args[0]._storage
        _settle(t, st)
        return st
    if lz.name is not None and all(a is None or a._st is not None for a in lz.args):
        # one op over evaluated inputs: its own single-op kernel
        out = _EAGER[lz.kind](lz, t._shape)
        _settle(t, out._st)
        return out._st
    if not _LAZY["jit"]:
        return _realize_op_by_op(t)
    out = empty(t._shape)
    prog, keep = _program_fit(t)
    rc = L.lib().tjh_expr_eval(ctypes.byref(prog), out.numel(), out.data_ptr())
    if rc and _jit_failed(rc):
        return _realize_op_by_op(t)
    L.check(rc, "expr")
    del keep
    _settle(t, out._st)
    return out._st


def _jit_failed(rc):
    """A fused kernel could not be compiled (hipRTC unavailable): warn once
    and evaluate deferred values op by op with the single-op kernels."""
    msg = (L.lib().tjh_last_error() or b"").decode(errors="replace")
    if "compile failed" not in msg and "hiprtc" not in msg:
        return False
    if _LAZY["jit"]:
        import sys
        print("torchjs_amd: fused elementwise kernels unavailable (%s); running elementwise "
              "ops one kernel each" % msg[:200], file=sys.stderr)
    _LAZY["jit"] = False
    _LAZY["on"] = False
    return True


def _realize_op_by_op(t):
    lz = t._lz
    for a in lz.args:
        if a is not None and a._st is None:
            a._storage
    out = _EAGER[lz.kind](lz, t._shape)
    _settle(t, out._st)
    return out._st


def _before_write(*ts):
    """Evaluates every deferred value that reads the storage of (or is) one
    of `ts`, before that memory is written in place."""
    if not _PENDING:
        return
    keys = set()
    for t in ts:
        # t, and the values it aliases (a detach() or view of a deferred
        # value writes into that value's memory once it is computed)
        while t is not None:
            keys.add(id(t))
            if t._st is not None:
                keys.add(id(t._st))
                break
            lz = t._lz
            t = lz.args[0] if lz is not None and lz.kind == "alias" else None
    for p in _pending_tensors():
        lz = p._lz
        if p._st is None and lz is not None and not keys.isdisjoint(lz.deps):
            p._storage


def _lazy_colsum(x, dims, keep=False):
    """Sum of deferred x over one run of adjacent dims with a fused kernel
    (keepdim layout), or None when the shape does not suit it.  With
    `keep`, x's value is written in the same pass."""
    if not _LAZY["jit"]:
        return None
    shape = list(x._shape)
    dims = sorted(set(dims))
    if not dims or dims != list(range(dims[0], dims[-1] + 1)):
        return None
    beg, end = dims[0], dims[-1] + 1
    outer, r, inner = _numel(shape[:beg]), _numel(shape[beg:end]), _numel(shape[end:])
    if outer > 64 or r < 64 or inner < 2:
        return None
    sib = _sibling_for(x) if keep else None
    third = _pending_colsum_for(x, dims, sib) if 2 * outer <= 64 else None
    prog = None
    if sib is not None or third is not None:
        try:
            prog, keep_alive = _program(x, sib, third[1] if third is not None else None)
        except _TooBig:
            sib = third = None
    if prog is None:
        try:
            prog, keep_alive = _program_fit(x)
        except RuntimeError:
            return None
    kshape = shape[:beg] + [1] * (end - beg) + shape[end:]
    out = empty(kshape)
    vals = empty(x._shape) if keep else None
    vals2 = empty(sib._shape) if sib is not None else None
    out3 = empty(kshape) if third is not None else None
    rc = L.lib().tjh_expr_colsum3(ctypes.byref(prog), outer, r, inner, out.data_ptr(),
                                  vals.data_ptr() if vals is not None else None,
                                  vals2.data_ptr() if vals2 is not None else None,
                                  out3.data_ptr() if out3 is not None else None)
    if rc == L.ERR_UNSUPPORTED or (rc and _jit_failed(rc)):
        return None
    L.check(rc, "expr_colsum")
    del keep_alive
    if vals is not None:
        _settle(x, vals._st)
    if sib is not None:
        _settle(sib, vals2._st)
        _SIBLINGS.remove(sib)
    if third is not None:
        # the pending forward column sum, from the same pass: settled as its
        # own computation would have left it (then scaled for a mean)
        c, _, scale = third
        red = _k_scalar("mul", out3, scale) if scale != 1.0 else out3
        _settle(c, red._st)
    return out


def _pending_colsum_for(x, dims, sib):
    """A deferred column sum (thunk, source value, scale) over the same dims
    of a deferred value of x's shape that reads one of x's inputs and that
    neither x nor sib reads, or None."""
    found = None
    keep = []
    for entry in _COLSUMS:
        c = entry[0]()
        if c is None or c._st is not None:
            continue  # evaluated or gone: dropped from the list
        keep.append(entry)
        if found is not None:
            continue
        z = c._lz.args[0]
        if (z._st is not None or z is x or z._shape != x._shape or entry[1] != tuple(dims) or
                z._lz.kind in ("alias", "thunk")):
            continue
        if z._lz.deps.isdisjoint(x._lz.deps) or id(c) in x._lz.deps or id(x) in z._lz.deps:
            continue
        if sib is not None and (id(c) in sib._lz.deps or sib is z):
            continue
        found = (c, z, entry[2])
    _COLSUMS[:] = keep
    return found


# Deferred leaf gradients of the running backward pass not yet evaluated:
# a column sum that writes another deferred value of the same shape (x's
# gradient with the bias gradient) writes one of these in the same pass
# when they read common inputs (y's gradient of GELU(x + b) * y).
_SIBLINGS = []
# evaluating sibling leaf gradients together; off only to compare in tests
_FUSE_SIB = True


def _sibling_for(x):
    """A pending deferred leaf gradient of x's shape that reads one of x's
    inputs, or None."""
    for s in _SIBLINGS:
        if (s._st is None and s._lz is not None and s._shape == x._shape and
                not s._lz.deps.isdisjoint(x._lz.deps) and id(x) not in s._lz.deps and
                id(s) not in x._lz.deps):
            return s
    return None


def _finish_siblings():
    """Evaluates the sibling gradients no column sum took along."""
    while _SIBLINGS:
        s = _SIBLINGS.pop()
        if s._st is None:
            s._storage


# ----------------------------------------------------------------- HIP graphs

_CAPTURE = {"on": False}  # a Graph is capturing the library stream


def capturing():
    return _CAPTURE["on"]


class Graph:
    """A HIP graph of the work one region enqueues on the library stream
    (in the manner of torch.cuda.CUDAGraph; torch.js has no replay): run
    the region a few times eagerly, capture it once with `graph(g)`, then
    `g.replay()` re-runs all of its kernels with one launch and no host
    work.  Tensors the region created keep their memory across replays
    (replays rewrite it in place), and tensors it read are read again, so
    new inputs go in with copy_.  Readbacks, host copies and
    synchronisation inside the region raise."""

    def __init__(self):
        self._id = None

    def capture_begin(self):
        if self._id is not None:
            raise RuntimeError("this graph has already been captured")
        gid = ctypes.c_int(0)
        L.check(L.lib().tjh_graph_begin(ctypes.byref(gid)), "graph_begin")
        self._id = gid.value
        _CAPTURE["on"] = True

    def capture_end(self):
        # deferred values the region created are computed inside the graph
        try:
            for p in _pending_tensors():
                if p._st is None:
                    p._storage
        finally:
            _CAPTURE["on"] = False
        L.check(L.lib().tjh_graph_end(self._id), "graph_end")

    def replay(self):
        if self._id is None:
            raise RuntimeError("replay of a graph that was never captured")
        L.check(L.lib().tjh_graph_replay(self._id), "graph_replay")

    def reset(self):
        if self._id is not None:
            gid, self._id = self._id, None
            L.check(L.lib().tjh_graph_destroy(gid), "graph_destroy")

    def __del__(self):
        try:
            self.reset()
        except Exception:
            pass


class graph:
    """`with graph(g):` captures the region into Graph g."""

    def __init__(self, g):
        self.g = g

    def __enter__(self):
        self.g.capture_begin()
        return self.g

    def __exit__(self, et, ev, tb):
        if et is None:
            self.g.capture_end()
            return False
        # a failed capture is ended and dropped; the error propagates
        _CAPTURE["on"] = False
        if self.g._id is not None:
            try:
                L.lib().tjh_graph_end(self.g._id)
                L.lib().tjh_graph_destroy(self.g._id)
            finally:
                self.g._id = None
        return False


# ----------------------------------------------------------------- raw kernels
# Non-differentiable helpers: allocate the output and launch.


def _k_contiguous(x):
    out = empty(x._shape, x._dtype)
    _copy_into(out, x)
    return out


def _copy_into(dst, src):
    """dst[...] = src[...] for equal shapes, any strides."""
    if dst.numel() == 0:
        return
    _before_write(dst)
    lib = L.lib()
    shp = L.i64arr(dst._shape)
    nd = len(dst._shape)
    if dst._dtype == "float32":
        L.check(lib.tjh_copy_strided(nd, shp, src.data_ptr(), L.i64arr(src._strides),
                                     dst.data_ptr(), L.i64arr(dst._strides)), "copy")
    elif dst._dtype == "int32":
        L.check(lib.tjh_copy_strided_i32(nd, shp, src.data_ptr(), L.i64arr(src._strides),
                                         dst.data_ptr(), L.i64arr(dst._strides)), "copy")
    else:
        L.check(lib.tjh_copy_strided_u8(nd, shp, src.data_ptr(), L.i64arr(src._strides),
                                        dst.data_ptr(), L.i64arr(dst._strides)), "copy")


def _k_cast(x, dtype):
    """Tensor.to(dtype) on the device (float32 / int32 / uint8 / bool)."""
    x = x.contiguous()
    out = empty(x._shape, dtype)
    if x.numel():
        L.check(L.lib().tjh_cast(L.DTYPE[x._dtype], L.DTYPE[dtype], x.data_ptr(), out.data_ptr(),
                                 x.numel()), "cast")
    return out


def _k_unary(op, x, alpha=0.0):
    k = _lazy_ok(x._shape, (x,))
    if k is not None:
        return _lazy("u", L.UNARY[op], alpha, (x,), x._shape, k, op)
    return _e_unary(op, x, alpha)


def _e_unary(op, x, alpha=0.0):
    x = x.contiguous()
    out = empty(x._shape)
    L.check(L.lib().tjh_unary(L.UNARY[op], x.data_ptr(), out.data_ptr(), x.numel(), float(alpha)),
            op)
    return out


def _k_unary_bwd(op, g, x, y, alpha=0.0):
    k = _lazy_ok(g._shape, (g, x, y))
    if k is not None:
        return _lazy("ub", L.UNARY[op], alpha, (g, x, y), g._shape, k, op)
    return _e_unary_bwd(op, g, x, y, alpha)


def _e_unary_bwd(op, g, x, y, alpha=0.0):
    g = g.contiguous()
    out = empty(g._shape)
    L.check(L.lib().tjh_unary_backward(
        L.UNARY[op], g.data_ptr(), x.contiguous().data_ptr() if x is not None else None,
        y.contiguous().data_ptr() if y is not None else None, out.data_ptr(), g.numel(),
        float(alpha)), op + "_backward")
    return out


def _bstrides(t, shape):
    """Strides of t broadcast to `shape` (0 on broadcast dims)."""
    nd = len(shape)
    off = nd - t.ndim
    st = []
    for d in range(nd):
        if d < off:
            st.append(0)
        else:
            sz = t._shape[d - off]
            st.append(0 if (sz == 1 and shape[d] != 1) else t._strides[d - off])
    return st


def _k_binary(op, a, b):
    shape = _broadcast_shapes(a._shape, b._shape)
    k = _lazy_ok(shape, (a, b))
    if k is not None:
        return _lazy("b", L.BINARY[op], 0.0, (a, b), shape, k, op)
    return _e_binary(op, a, b, shape)


def _e_binary(op, a, b, shape):
    out = empty(shape)
    if out.numel():
        L.check(L.lib().tjh_binary(L.BINARY[op], len(shape), L.i64arr(shape), a.data_ptr(),
                                   L.i64arr(_bstrides(a, shape)), b.data_ptr(),
                                   L.i64arr(_bstrides(b, shape)), out.data_ptr()), op)
    return out


def _k_ternary(op, g, a, b, shape):
    shape = tuple(shape)
    k = _lazy_ok(shape, (g, a, b))
    if k is not None:
        return _lazy("t", L.TERNARY[op], 0.0, (g, a, b), shape, k, op)
    return _e_ternary(op, g, a, b, shape)


def _e_ternary(op, g, a, b, shape):
    out = empty(shape)
    if out.numel():
        L.check(L.lib().tjh_ternary(L.TERNARY[op], len(shape), L.i64arr(shape), g.data_ptr(),
                                    L.i64arr(_bstrides(g, shape)), a.data_ptr(),
                                    L.i64arr(_bstrides(a, shape)), b.data_ptr(),
                                    L.i64arr(_bstrides(b, shape)), out.data_ptr()), op)
    return out


def _k_scalar(op, x, s, reverse=False):
    k = _lazy_ok(x._shape, (x,))
    if k is not None:
        return _lazy("sr" if reverse else "s", L.SCALAR[op], s, (x,), x._shape, k, op)
    return _e_scalar(op, x, s, reverse)


def _e_scalar(op, x, s, reverse=False):
    x = x.contiguous()
    out = empty(x._shape)
    L.check(L.lib().tjh_scalar(L.SCALAR[op], x.data_ptr(), float(s), 1 if reverse else 0,
                               out.data_ptr(), x.numel()), op)
    return out


def _k_axpy(alpha, x, y):
    """alpha*x + y (same shape)."""
    k = _lazy_ok(x._shape, (x, y)) if x._shape == y._shape else None
    if k is not None:
        return _lazy("axpy", 0, alpha, (x, y), x._shape, k, "axpy")
    return _e_axpy(alpha, x, y)


def _e_axpy(alpha, x, y):
    x = x.contiguous()
    y = y.contiguous()
    out = empty(x._shape)
    L.check(L.lib().tjh_axpy(float(alpha), x.data_ptr(), y.data_ptr(), out.data_ptr(), x.numel()),
            "axpy")
    return out


# single-op kernels of deferred ops (by _Lz.kind)
_EAGER = {
    "u": lambda lz, shape: _e_unary(lz.name, lz.args[0], lz.f),
    "ub": lambda lz, shape: _e_unary_bwd(lz.name, *lz.args, alpha=lz.f),
    "b": lambda lz, shape: _e_binary(lz.name, lz.args[0], lz.args[1], shape),
    "t": lambda lz, shape: _e_ternary(lz.name, *lz.args, shape),
    "s": lambda lz, shape: _e_scalar(lz.name, lz.args[0], lz.f, False),
    "sr": lambda lz, shape: _e_scalar(lz.name, lz.args[0], lz.f, True),
    "axpy": lambda lz, shape: _e_axpy(lz.f, lz.args[0], lz.args[1]),
}


def _reduce_runs(shape, dims):
    """Groups sorted reduced dims into maximal runs of adjacent dims."""
    runs = []
    for d in sorted(dims):
        if runs and runs[-1][1] == d:
            runs[-1][1] = d + 1
        else:
            runs.append([d, d + 1])
    return runs


def _k_reduce(op, x, dims, keep=False):
    """Reduces the given dims of x (keepdim=True layout), fp32.  A sum /
    mean of a deferred x reads x's inputs directly (and, with `keep`,
    writes x's value in the same pass)."""
    if op in ("sum", "mean") and _is_lazy(x) and x._lz.kind not in ("alias", "thunk"):
        r = _lazy_colsum(x, dims, keep)
        if r is not None:
            if op == "mean":
                total_r = _numel([x._shape[d] for d in set(dims)])
                r = _k_scalar("mul", r, 1.0 / total_r if total_r else float("nan"))
            return r
    x = x.contiguous()
    shape = list(x._shape)
    dims = sorted(set(dims))
    total_r = 1
    for d in dims:
        total_r *= shape[d]
    cur = x
    # reduce runs from the last to the first so earlier indices stay valid
    for beg, end in reversed(_reduce_runs(shape, dims)):
        cshape = list(cur._shape)
        outer = _numel(cshape[:beg])
        r = _numel(cshape[beg:end])
        inner = _numel(cshape[end:])
        oshape = cshape[:beg] + [1] * (end - beg) + cshape[end:]
        out = empty(oshape)
        kop = op
        if op == "mean":
            kop = "sum"
        L.check(L.lib().tjh_reduce(L.REDUCE[kop], cur.data_ptr(), outer, r, inner,
                                   out.data_ptr()), "reduce")
        cur = out
    if op == "mean":
        cur = _k_scalar("mul", cur, 1.0 / total_r if total_r else float("nan"))
    return cur


def _sum_to(g, shape, keep=False):
    """Sums a broadcast gradient back to `shape` (torch.js only handles 1-D
    against 2-D, Tensor.ts:3560-3591).  `keep`: a deferred g is also
    evaluated by the same pass."""
    shape = tuple(shape)
    if g._shape == shape:
        return g
    nd = g.ndim
    off = nd - len(shape)
    dims = [d for d in range(nd) if d < off or (shape[d - off] == 1 and g._shape[d] != 1)]
    r = _k_reduce("sum", g, dims, keep) if dims else g
    return _view_raw(r.contiguous(), shape)


def _view_raw(t, shape):
    """View of a contiguous tensor with a new shape (no autograd)."""
    if _numel(shape) != t.numel():
        raise RuntimeError("shape %s is invalid for input of size %d" % (list(shape), t.numel()))
    return Tensor(t._storage, shape, None, t._offset, t._dtype)


def _sum_to_g(g, shape):
    """_sum_to with recording ops (a gradient that is itself differentiated)."""
    shape = tuple(shape)
    if g.shape == shape:
        return g
    off = g.ndim - len(shape)
    dims = [d for d in range(g.ndim) if d < off or (shape[d - off] == 1 and g.shape[d] != 1)]
    r = reduce_sum(g, dims, keepdim=True) if dims else g
    return reshape(r, shape)


def _const(t, v):
    return full((), float(v))


def _unary_gvjp(op, g, x, alpha):
    """g * op'(x) with recording ops, so the result can be differentiated
    again (second derivatives through the unary ops)."""
    sc = lambda t, v: _scalar_op("mul", t, v)
    if op == "neg":
        return unary("neg", g)
    if op == "exp":
        return mul(g, unary("exp", x))
    if op == "log":
        return div(g, x)
    if op == "sqrt":
        return mul(g, sc(unary("rsqrt", x), 0.5))
    if op == "rsqrt":
        r = unary("rsqrt", x)
        return mul(g, sc(mul(r, mul(r, r)), -0.5))
    if op == "tanh":
        t = unary("tanh", x)
        return mul(g, _scalar_op("sub", mul(t, t), 1.0, reverse=True))
    if op == "sigmoid":
        sg = unary("sigmoid", x)
        return mul(g, mul(sg, _scalar_op("sub", sg, 1.0, reverse=True)))
    if op == "relu":
        return mul(g, compare_raw(x, _const(x, 0.0), "gt"))
    if op == "square":
        return mul(g, sc(x, 2.0))
    if op == "reciprocal":
        return unary("neg", div(g, mul(x, x)))
    if op == "sin":
        return mul(g, unary("cos", x))
    if op == "cos":
        return unary("neg", mul(g, unary("sin", x)))
    if op == "abs":
        return mul(g, unary("sign", x))
    if op == "sign":
        return sc(g, 0.0)
    if op == "erf":
        return mul(g, sc(unary("exp", unary("neg", mul(x, x))), 2.0 / math.sqrt(math.pi)))
    if op == "gelu":  # Phi(x) + x phi(x)
        phi_cdf = sc(_scalar_op("add", unary("erf", sc(x, 1.0 / math.sqrt(2.0))), 1.0), 0.5)
        pdf = sc(unary("exp", sc(mul(x, x), -0.5)), 1.0 / math.sqrt(2.0 * math.pi))
        return mul(g, add(phi_cdf, mul(x, pdf)))
    if op == "silu":
        sg = unary("sigmoid", x)
        return mul(g, mul(sg, _scalar_op("add", mul(x, _scalar_op("sub", sg, 1.0, reverse=True)),
                                         1.0)))
    if op == "softplus":  # sigmoid(x), and 1 above the threshold of 20
        big = compare_raw(x, _const(x, 20.0), "gt")
        return mul(g, add(mul(unary("sigmoid", x), _scalar_op("sub", big, 1.0, reverse=True)),
                          big))
    if op == "leaky_relu":
        pos = compare_raw(x, _const(x, 0.0), "gt")
        return mul(g, _scalar_op("add", sc(pos, 1.0 - alpha), alpha))
    if op == "elu":
        pos = compare_raw(x, _const(x, 0.0), "gt")
        negw = mul(sc(unary("exp", x), alpha), _scalar_op("sub", pos, 1.0, reverse=True))
        return mul(g, add(negw, pos))
    raise NotImplementedError("create_graph: no differentiable backward for %s" % op)


def _binary_gvjp(op, g, a, b):
    """Both operands' gradients of a (broadcasting) binary op with
    recording ops, summed back to each operand's shape."""
    ra, rb = a.requires_grad, b.requires_grad
    if op == "add":
        ga, gb = g, g
    elif op == "sub":
        ga, gb = g, (unary("neg", g) if rb else None)
    elif op == "mul":
        ga = mul(g, b) if ra else None
        gb = mul(g, a) if rb else None
    elif op == "div":
        ga = div(g, b) if ra else None
        gb = unary("neg", div(mul(g, a), mul(b, b))) if rb else None
    elif op == "pow":
        ga = mul(g, mul(b, _binary_op("pow", a, _scalar_op("sub", b, 1.0)))) if ra else None
        gb = mul(g, mul(_binary_op("pow", a, b), unary("log", a))) if rb else None
    else:  # maximum / minimum: the selected operand, ties split evenly
        sel = compare_raw(a, b, "gt" if op == "maximum" else "lt")
        wa = _k_binary("add", sel, _k_scalar("mul", compare_raw(a, b, "eq"), 0.5))
        ga = mul(g, wa) if ra else None
        gb = mul(g, _scalar_op("sub", wa, 1.0, reverse=True)) if rb else None
    return [_sum_to_g(ga, a.shape) if (ra and ga is not None) else None,
            _sum_to_g(gb, b.shape) if (rb and gb is not None) else None]


def _scalar_gvjp(op, g, x, s, reverse):
    """The gradient of x (op) s, or s (op) x with `reverse`, with recording
    ops."""
    if op == "add":
        return g
    if op == "sub":
        return unary("neg", g) if reverse else g
    if op == "mul":
        return _scalar_op("mul", g, s)
    if op == "div":
        if not reverse:
            return _scalar_op("div", g, s)
        return unary("neg", div(_scalar_op("mul", g, s), mul(x, x)))
    if op == "pow":
        if not reverse:
            return mul(g, _scalar_op("mul", _scalar_op("pow", x, s - 1.0), s))
        return mul(g, _scalar_op("mul", _scalar_op("pow", x, s, reverse=True), math.log(s)))
    if op in ("maximum", "minimum"):
        return mul(g, compare_raw(x, full((), s), "gt" if op == "maximum" else "lt"))
    raise NotImplementedError("create_graph: no differentiable backward for %s_scalar" % op)


# ----------------------------------------------------------------- differentiable ops


def unary(op, x, alpha=0.0):
    """_unaryOp (Tensor.ts:3593-3656) with the backward from unary.wgsl's
    derivatives; GELU uses the exact Phi(x) + x*phi(x) (torch.js uses a tanh
    form with a wrong pdf term, Tensor.ts:3627-3632)."""
    if x.dtype != "float32":
        x = x.float()
    out = _k_unary(op, x, alpha)
    needs_y = op in ("exp", "sqrt", "rsqrt", "tanh", "sigmoid", "reciprocal")
    needs_x = op not in ("neg",) and not needs_y
    saved_x = x if needs_x else None
    saved_y = out.detach() if needs_y else None

    def bwd(g):
        return [_k_unary_bwd(op, g, saved_x, saved_y, alpha)]
    return _record(out, op, [x], bwd, gfn=lambda g: [_unary_gvjp(op, g, x, alpha)])


def neg(x):
    return unary("neg", x)


def _binary_op(op, a, b):
    if not isinstance(b, Tensor):
        return _scalar_op(op, a, b)
    if not isinstance(a, Tensor):
        return _scalar_op(op, b, a, reverse=True)
    if a.dtype != "float32":
        a = a.float()
    if b.dtype != "float32":
        b = b.float()
    out = _k_binary(op, a, b)
    ash, bsh = a.shape, b.shape
    ra, rb = a.requires_grad, b.requires_grad
    if op == "add":
        def bwd(g):
            if ra and rb and _is_lazy(g) and g.shape == ash and ash != bsh:
                # the broadcast operand's column sum evaluates g in the same pass
                return [g, _sum_to(g, bsh, keep=True)]
            if ra and rb and _is_lazy(g) and g.shape == bsh and ash != bsh:
                return [_sum_to(g, ash, keep=True), g]
            return [_sum_to(g, ash) if ra else None, _sum_to(g, bsh) if rb else None]
    elif op == "sub":
        def bwd(g):
            return [_sum_to(g, ash) if ra else None,
                    _sum_to(_k_unary("neg", g), bsh) if rb else None]
    else:
        sa, sb = a.detach(), b.detach()
        if op == "mul":
            def bwd(g):
                return [_sum_to(_k_binary("mul", g, sb), ash) if ra else None,
                        _sum_to(_k_binary("mul", g, sa), bsh) if rb else None]
        elif op == "div":
            def bwd(g):
                return [_sum_to(_k_binary("div", g, sb), ash) if ra else None,
                        _sum_to(_k_ternary("div_b", g, sa, sb, g.shape), bsh) if rb else None]
        elif op == "pow":
            def bwd(g):
                return [_sum_to(_k_ternary("pow_a", g, sa, sb, g.shape), ash) if ra else None,
                        _sum_to(_k_ternary("pow_b", g, sa, sb, g.shape), bsh) if rb else None]
        else:  # maximum / minimum: ties split the gradient evenly
            def bwd(g):
                sel = compare_raw(sa, sb, "gt" if op == "maximum" else "lt")
                eq = compare_raw(sa, sb, "eq")
                wa = _k_binary("add", sel, _k_scalar("mul", eq, 0.5))
                wb = _k_scalar("add", _k_scalar("mul", wa, -1.0), 1.0)
                return [_sum_to(_k_binary("mul", g, wa), ash) if ra else None,
                        _sum_to(_k_binary("mul", g, wb), bsh) if rb else None]
    return _record(out, op, [a, b], bwd, gfn=lambda g: _binary_gvjp(op, g, a, b))


def _scalar_op(op, x, s, reverse=False):
    if isinstance(s, Tensor):
        raise TypeError("scalar op with tensor")
    if x.dtype != "float32":
        x = x.float()
    s = float(s)
    out = _k_scalar(op, x, s, reverse)

    def bwd(g):
        if op == "add":
            return [g]
        if op == "sub":
            return [_k_unary("neg", g) if reverse else g]
        if op == "mul":
            return [_k_scalar("mul", g, s)]
        if op == "div":
            if not reverse:
                return [_k_scalar("div", g, s)]
            # d(s/x) = -s/x^2
            return [_k_ternary("div_b", _k_scalar("mul", g, s), full((), 1.0), x, g.shape)]
        if op == "pow":
            if not reverse:
                gg = g.contiguous()
                o = empty(gg.shape)
                L.check(L.lib().tjh_pow_scalar_backward(gg.data_ptr(), x.contiguous().data_ptr(),
                                                        s, o.data_ptr(), gg.numel()), "pow_bwd")
                return [o]
            # d(s^x) = s^x ln s
            return [_k_scalar("mul", _k_binary("mul", g, out.detach()), math.log(s))]
        if op in ("maximum", "minimum"):
            m = compare_raw(x, full((), s), "gt" if op == "maximum" else "lt")
            return [_k_binary("mul", g, m)]
        raise NotImplementedError(op)
    return _record(out, op + "_scalar", [x], bwd,
                   gfn=lambda g: [_scalar_gvjp(op, g, x, s, reverse)])


def add(a, b):
    return _binary_op("add", a, b)


def sub(a, b):
    return _binary_op("sub", a, b)


def rsub(a, b):
    """b - a for a scalar b."""
    return _scalar_op("sub", a, b, reverse=True)


def mul(a, b):
    return _binary_op("mul", a, b)


def div(a, b):
    return _binary_op("div", a, b)


def rdiv(a, b):
    return _scalar_op("div", a, b, reverse=True)


def pow(a, b):
    """pow with torch.js's integer-exponent rule for scalars (scalar.wgsl:53-66)."""
    if isinstance(a, Tensor) and not isinstance(b, Tensor):
        return _scalar_op("pow", a, b)
    if not isinstance(a, Tensor):
        return _scalar_op("pow", b, a, reverse=True)
    return _binary_op("pow", a, b)


def compare_raw(a, b, op):
    if not isinstance(b, Tensor):
        b = full((), float(b))
    if not isinstance(a, Tensor):
        a = full((), float(a))
    a = a.float() if a.dtype != "float32" else a
    b = b.float() if b.dtype != "float32" else b
    shape = _broadcast_shapes(a.shape, b.shape)
    out = empty(shape)
    if out.numel():
        L.check(L.lib().tjh_compare(L.COMPARE[op], len(shape), L.i64arr(shape), a.data_ptr(),
                                    L.i64arr(_bstrides(a, shape)), b.data_ptr(),
                                    L.i64arr(_bstrides(b, shape)), out.data_ptr()), op)
    return out


def compare(a, b, op):
    """eq/ne/lt/le/gt/ge producing float 0/1 (compare.wgsl); no gradient."""
    return compare_raw(a, b, op)


def triangle(x, diagonal=0, upper=True):
    """triu / tril (triu.wgsl, tril.wgsl) over the last two dims; the
    gradient is the same mask applied to the incoming gradient."""
    if x.ndim < 2:
        raise RuntimeError("triu/tril: expected a tensor with at least 2 dimensions")
    dt = x.dtype
    xf = x if dt == "float32" else x.float()
    xc = xf.contiguous()
    rows, cols = x.shape[-2], x.shape[-1]
    batch = _numel(x.shape[:-2])
    out = empty(x.shape)
    L.check(L.lib().tjh_triangle(xc.data_ptr(), out.data_ptr(), batch, rows, cols, int(diagonal),
                                 1 if upper else 0), "triangle")
    if dt != "float32":
        return out.to(dt)

    def bwd(g):
        gc = g.contiguous()
        o = empty(g.shape)
        L.check(L.lib().tjh_triangle(gc.data_ptr(), o.data_ptr(), batch, rows, cols,
                                     int(diagonal), 1 if upper else 0), "triangle_backward")
        return [o]
    return _record(out, "Triu" if upper else "Tril", [x], bwd,
                   gfn=lambda g: [triangle(g, diagonal, upper)])


def triu(x, diagonal=0):
    return triangle(x, diagonal, True)


def tril(x, diagonal=0):
    return triangle(x, diagonal, False)


def multinomial(x, num_samples=1, replacement=False):
    """Tensor.multinomial (Tensor.ts:271-359) on the device: int32 indices,
    [num_samples] for a 1-D input, [rows, num_samples] for a 2-D one.
    Weights are max(0, x) normalised by their sum (uniform when it is not
    positive); the draws come from the seeded stream (one LCG step of the
    manual_seed state per call, like rand), not Math.random.  A row holding
    NaN or +inf raises RuntimeError (PyTorch's contract; the reference's
    result is undefined there).  The call synchronises with the device."""
    if x.ndim not in (1, 2):
        raise RuntimeError("multinomial: expected a 1-D or 2-D tensor of probabilities")
    cols = x.shape[-1]
    rows = 1 if x.ndim == 1 else x.shape[0]
    if cols == 0:
        raise RuntimeError("multinomial: no categories")
    if not replacement and num_samples > cols:
        raise RuntimeError("Cannot sample %d values from %d categories without replacement"
                           % (num_samples, cols))
    xc = (x if x.dtype == "float32" else x.float()).contiguous()
    out = empty((rows, num_samples) if x.ndim == 2 else (num_samples,), "int32")
    if rows and num_samples:
        L.check(L.lib().tjh_multinomial(xc.data_ptr(), rows, cols, int(num_samples),
                                        1 if replacement else 0, _next_seed(), out.data_ptr()),
                "multinomial")
    return out


def clamp(x, min=None, max=None):
    """clamp / clamp_min / clamp_max (clamp.wgsl): max(x, min) then
    min(., max); the gradient passes where min <= x <= max (PyTorch's
    rule, the bounds included)."""
    if min is None and max is None:
        raise RuntimeError("clamp: at least one of min and max must be given")
    if x.dtype != "float32":
        x = x.float()
    out = x.contiguous().detach()
    if min is not None:
        out = _k_scalar("maximum", out, float(min))
    if max is not None:
        out = _k_scalar("minimum", out, float(max))
    if out is x:
        out = _k_contiguous(x)
    xd = x.detach()

    def mask():
        m = None
        if min is not None:
            m = compare_raw(xd, float(min), "ge")
        if max is not None:
            mx = compare_raw(xd, float(max), "le")
            m = mx if m is None else _k_binary("mul", m, mx)
        return m

    def bwd(g):
        return [_k_binary("mul", g, mask())]
    # the pass-through mask is piecewise constant in x: a constant factor
    return _record(out, "Clamp", [x], bwd, gfn=lambda g: [mul(g, mask())])


# ------------------------------------------------------------ reductions


def _norm_dims(x, dim):
    if dim is None:
        return list(range(x.ndim))
    if isinstance(dim, (list, tuple)):
        return sorted(set(_wrap_dim(d, x.ndim) for d in dim))
    return [_wrap_dim(dim, x.ndim)]


def _squeeze_shape(shape, dims):
    return tuple(s for i, s in enumerate(shape) if i not in dims)


# column sums of deferred values left deferred until a backward pass can
# compute them with the gradients it forms from the same inputs; off only
# to compare with the immediate sums in tests
_DEFER_SUMS = {"on": True}


def _reduced_shape(x, dims, dim, keepdim):
    if keepdim:
        return tuple(1 if i in dims else s for i, s in enumerate(x.shape))
    if dim is None:
        return ()
    return _squeeze_shape(x.shape, dims)


def _deferred_reduce(op, x, dims, oshape):
    """A deferred sum / mean of x over `dims` with output shape `oshape`,
    or None.  A column sum of a deferred elementwise value (one run of
    adjacent dims, the fused column-sum kernel's layout) is registered so
    a backward column sum over the same rows of values reading the same
    inputs computes it in its own pass (_lazy_colsum); a reduction of a
    deferred reduction stays deferred after it."""
    if not (_LAZY["on"] and _LAZY["jit"] and _DEFER_SUMS["on"] and x._st is None and dims):
        return None
    kind = x._lz.kind
    cnt = _numel([x._shape[d] for d in dims])
    scale = 1.0 / cnt if (op == "mean" and cnt) else (float("nan") if op == "mean" else 1.0)
    if kind == "thunk":
        def compute():
            r = _k_reduce(op, x, dims)
            return _view_raw(r.contiguous(), oshape)
        return _thunk(compute, oshape, [x])
    if kind == "alias" or dims != list(range(dims[0], dims[-1] + 1)):
        return None
    shape = x._shape
    outer = _numel(shape[:dims[0]])
    r = _numel(shape[dims[0]:dims[-1] + 1])
    inner = _numel(shape[dims[-1] + 1:])
    if 2 * outer > 64 or r < 64 or inner < 2:
        return None

    def compute():
        red = _k_reduce("sum", x, dims)
        if scale != 1.0:
            red = _k_scalar("mul", red, scale)
        return _view_raw(red.contiguous(), oshape)
    t = _thunk(compute, oshape, [x])
    _COLSUMS.append((weakref.ref(t), tuple(dims), scale))
    return t


def reduce_sum(x, dim=None, keepdim=False):
    """sum (Tensor.ts:2427-2431); backward broadcasts g over the reduced dims
    after restoring them (torch.js expands without unsqueezing, D13)."""
    if x.dtype != "float32":
        x = x.float()
    dims = _norm_dims(x, dim)
    kshape = tuple(1 if i in dims else s for i, s in enumerate(x.shape))
    out = _deferred_reduce("sum", x, dims, _reduced_shape(x, dims, dim, keepdim))
    if out is None:
        r = _k_reduce("sum", x, dims) if dims else x.contiguous()
        out = r if keepdim else _view_raw(r, _squeeze_shape(x.shape, dims))
        if not keepdim and dim is None:
            out = _view_raw(r, ())
    xs = x.shape

    def bwd(g):
        if g._lz is None and g._st is not None and all(st == 0 for st in g._strides):
            # one element broadcast (a mean's gradient): broadcast it on as a
            # view, not materialised (the fused kernels read it as a scalar)
            return [Tensor(g._st, xs, (0,) * len(xs), g._offset, g._dtype)]
        return [_view_raw(g.contiguous(), kshape).expand(xs)]
    return _record(out, "Sum", [x], bwd, gfn=lambda g: [expand(reshape(g, kshape), xs)])


def reduce_mean(x, dim=None, keepdim=False):
    """mean (Tensor.ts:2432-2446)."""
    if x.dtype != "float32":
        x = x.float()
    dims = _norm_dims(x, dim)
    cnt = 1
    for d in dims:
        cnt *= x.shape[d]
    kshape = tuple(1 if i in dims else s for i, s in enumerate(x.shape))
    out = _deferred_reduce("mean", x, dims, _reduced_shape(x, dims, dim, keepdim))
    if out is None:
        r = _k_reduce("mean", x, dims) if dims else x.contiguous()
        out = r if keepdim else _view_raw(r, _squeeze_shape(x.shape, dims))
    xs = x.shape

    def bwd(g):
        gs = _k_scalar("mul", g, 1.0 / cnt) if cnt else g
        return [_view_raw(gs.contiguous(), kshape).expand(xs)]

    def gbwd(g):
        gs = _scalar_op("mul", g, 1.0 / cnt) if cnt else g
        return [expand(reshape(gs, kshape), xs)]
    return _record(out, "Mean", [x], bwd, gfn=gbwd)


def reduce_minmax(x, dim, keepdim, which):
    """amax / amin; ties share the gradient evenly."""
    if x.dtype != "float32":
        x = x.float()
    dims = _norm_dims(x, dim)
    r = _k_reduce(which, x, dims)
    kshape = r.shape
    out = r if keepdim else _view_raw(r, _squeeze_shape(x.shape, dims))
    xs = x.shape

    def share():
        mask = compare_raw(x, r, "eq")
        cnt = _k_reduce("sum", mask, dims)
        return _k_binary("div", mask, cnt)

    def bwd(g):
        return [_k_binary("mul", share(), _view_raw(g.contiguous(), kshape))]
    # the tie shares are piecewise constant in x: a constant factor
    return _record(out, which.capitalize(), [x], bwd,
                   gfn=lambda g: [mul(share(), expand(reshape(g, kshape), xs))])


def argmax(x, dim=None, keepdim=False, is_min=False):
    """argmax / argmin (Tensor.ts:2504-2577): first index of the extreme."""
    if x.dtype != "float32":
        x = x.float()
    x = x.contiguous()
    if dim is None:
        outer, r, inner = 1, x.numel(), 1
        oshape = ()
    else:
        d = _wrap_dim(dim, x.ndim)
        outer, r, inner = _numel(x.shape[:d]), x.shape[d], _numel(x.shape[d + 1:])
        oshape = x.shape[:d] + ((1,) if keepdim else ()) + x.shape[d + 1:]
    out = empty(oshape, "int32")
    L.check(L.lib().tjh_argmax(x.data_ptr(), outer, r, inner, 1 if is_min else 0,
                               out.data_ptr()), "argmax")
    return out


# ------------------------------------------------------------ views


def _view_strides(shape, strides, new_shape):
    """Strides for viewing (shape, strides) as new_shape without a copy, or
    None when impossible.  Walks the old dims from the innermost, splitting
    them into chunks that are contiguous among themselves; every chunk must
    be covered by whole new dims."""
    new_shape = tuple(new_shape)
    if _numel(shape) == 0 or len(shape) == 0:
        return _contig_strides(new_shape)
    new_strides = [0] * len(new_shape)
    view_d = len(new_shape) - 1
    chunk_base = strides[-1]
    tensor_numel = 1
    view_numel = 1
    for td in range(len(shape) - 1, -1, -1):
        tensor_numel *= shape[td]
        if td == 0 or (shape[td - 1] != 1 and strides[td - 1] != tensor_numel * chunk_base):
            while view_d >= 0 and (view_numel < tensor_numel or new_shape[view_d] == 1):
                new_strides[view_d] = view_numel * chunk_base
                view_numel *= new_shape[view_d]
                view_d -= 1
            if view_numel != tensor_numel:
                return None
            if td > 0:
                chunk_base = strides[td - 1]
                tensor_numel = 1
                view_numel = 1
    if view_d != -1:
        return None
    return tuple(new_strides)


def _infer_shape(shape, n):
    """inferShape (src/utils/shape.ts:64-90): one -1 allowed."""
    shape = list(int(s) for s in shape)
    if shape.count(-1) > 1:
        raise RuntimeError("only one dimension can be inferred")
    if -1 in shape:
        known = 1
        for s in shape:
            if s != -1:
                known *= s
        if known == 0 or n % known:
            raise RuntimeError("shape %s is invalid for input of size %d" % (shape, n))
        shape[shape.index(-1)] = n // known
    if _numel(shape) != n:
        raise RuntimeError("shape %s is invalid for input of size %d" % (shape, n))
    return tuple(shape)


def _alias(x, shape, strides, offset):
    return Tensor(x._storage, shape, strides, offset, x._dtype)


def view(x, shape):
    shape = _infer_shape(shape, x.numel())
    st = _view_strides(x.shape, x._strides, shape)
    if st is None:
        raise RuntimeError("view size is not compatible with input tensor's size and stride; use reshape")
    out = _alias(x, shape, st, x._offset)
    xs = x.shape
    return _record(out, "View", [x], lambda g: [reshape_raw(g, xs)],
                   gfn=lambda g: [reshape(g, xs)])


def reshape_raw(g, shape):
    if isinstance(g, _CEGrad):
        return g.reshaped(shape)
    st = _view_strides(g.shape, g._strides, tuple(shape))
    if st is None:
        g = g.contiguous()
        st = _contig_strides(tuple(shape))
    return Tensor(g._storage, tuple(shape), st, g._offset, g._dtype)


def reshape(x, shape):
    """reshape (Tensor.ts:1603-1628): a view when strides allow, else a copy."""
    shape = _infer_shape(shape, x.numel())
    st = _view_strides(x.shape, x._strides, shape)
    if st is None:
        return view(contiguous(x), shape)
    return view(x, shape)


def flatten(x, start_dim=0, end_dim=-1):
    if x.ndim == 0:
        return reshape(x, (1,))
    s = _wrap_dim(start_dim, x.ndim)
    e = _wrap_dim(end_dim, x.ndim)
    shape = x.shape[:s] + (_numel(x.shape[s:e + 1]),) + x.shape[e + 1:]
    return reshape(x, shape)


def squeeze(x, dim=None):
    if dim is None:
        shape = tuple(s for s in x.shape if s != 1)
    else:
        d = _wrap_dim(dim, x.ndim)
        shape = x.shape[:d] + x.shape[d + 1:] if x.shape[d] == 1 else x.shape
    return reshape(x, shape)


def unsqueeze(x, dim):
    d = _wrap_dim(dim, x.ndim + 1)
    shape = x.shape[:d] + (1,) + x.shape[d:]
    st = list(x._strides)
    st.insert(d, (x._strides[d] * x.shape[d]) if d < x.ndim else 1)
    out = _alias(x, shape, tuple(st), x._offset)
    xs = x.shape
    return _record(out, "Unsqueeze", [x], lambda g: [reshape_raw(g, xs)],
                   gfn=lambda g: [reshape(g, xs)])


def permute(x, dims):
    dims = tuple(_wrap_dim(d, x.ndim) for d in dims)
    if sorted(dims) != list(range(x.ndim)):
        raise RuntimeError("permute: dims %s are not a permutation" % (dims,))
    shape = tuple(x.shape[d] for d in dims)
    st = tuple(x._strides[d] for d in dims)
    out = _alias(x, shape, st, x._offset)
    inv = [0] * len(dims)
    for i, d in enumerate(dims):
        inv[d] = i

    def bwd(g):
        return [_alias(g, tuple(g.shape[i] for i in inv), tuple(g._strides[i] for i in inv),
                       g._offset)]
    return _record(out, "Permute", [x], bwd, gfn=lambda g: [permute(g, inv)])


def transpose(x, d0, d1):
    d0 = _wrap_dim(d0, x.ndim)
    d1 = _wrap_dim(d1, x.ndim)
    dims = list(range(x.ndim))
    dims[d0], dims[d1] = dims[d1], dims[d0]
    return permute(x, dims)


def expand(x, shape):
    """expand / broadcast_to (Tensor.ts:1537-1601) as a 0-stride view;
    backward sums over the expanded dims (torch.js has none, D12)."""
    shape = tuple(int(s) for s in shape)
    nd = len(shape)
    off = nd - x.ndim
    if off < 0:
        raise RuntimeError("expand: target has fewer dims than the tensor")
    new_shape = []
    st = []
    for d in range(nd):
        want = shape[d]
        if d < off:
            if want == -1:
                raise RuntimeError("expand: -1 not allowed for new leading dims")
            new_shape.append(want)
            st.append(0)
        else:
            have = x.shape[d - off]
            if want == -1:
                want = have
            if have == want:
                new_shape.append(want)
                st.append(x._strides[d - off])
            elif have == 1:
                new_shape.append(want)
                st.append(0)
            else:
                raise RuntimeError("expand: size %d cannot expand to %d" % (have, want))
    out = _alias(x, tuple(new_shape), tuple(st), x._offset)
    xs = x.shape
    return _record(out, "Expand", [x], lambda g: [_sum_to(g, xs)],
                   gfn=lambda g: [_sum_to_g(g, xs)])


def contiguous(x):
    if x.is_contiguous():
        return x
    out = _k_contiguous(x)
    return _record(out, "Contiguous", [x], lambda g: [g], gfn=lambda g: [g])


def clone(x):
    out = _k_contiguous(x)
    return _record(out, "Clone", [x], lambda g: [g], gfn=lambda g: [g])


def narrow(x, dim, start, length):
    d = _wrap_dim(dim, x.ndim)
    n = x.shape[d]
    if start < 0:
        start += n
    if start < 0 or length < 0 or start + length > n:
        raise IndexError("narrow: range [%d, %d) out of bounds for size %d" % (start, start + length, n))
    shape = x.shape[:d] + (length,) + x.shape[d + 1:]
    out = _alias(x, shape, x._strides, x._offset + start * x._strides[d])
    xs = x.shape

    def gbwd(g):  # g placed at [start, start + length) of zeros along d
        parts = []
        if start:
            parts.append(zeros(*(xs[:d] + (start,) + xs[d + 1:])))
        parts.append(g)
        if start + length < n:
            parts.append(zeros(*(xs[:d] + (n - start - length,) + xs[d + 1:])))
        return [cat(parts, d) if len(parts) > 1 else g]
    return _record(out, "Narrow", [x], lambda g: [_SliceGrad(xs, d, [(start, g)])], gfn=gbwd)


def select(x, dim, index):
    d = _wrap_dim(dim, x.ndim)
    if index < 0:
        index += x.shape[d]
    return squeeze(narrow(x, d, index, 1), d)


def split(x, split_size, dim=0):
    d = _wrap_dim(dim, x.ndim)
    n = x.shape[d]
    if isinstance(split_size, (list, tuple)):
        sizes = list(split_size)
        if sum(sizes) != n:
            raise RuntimeError("split sizes %s do not sum to %d" % (sizes, n))
    else:
        sizes = [min(split_size, n - i) for i in range(0, n, split_size)]
    outs = []
    pos = 0
    for s in sizes:
        outs.append(narrow(x, d, pos, s))
        pos += s
    return outs


def chunk(x, chunks, dim=0):
    d = _wrap_dim(dim, x.ndim)
    n = x.shape[d]
    size = -(-n // chunks)
    return split(x, size, d)


def _getitem(x, idx):
    if not isinstance(idx, tuple):
        idx = (idx,)
    out = x
    d = 0
    for it in idx:
        if it is Ellipsis:
            d = out.ndim - (len(idx) - 1 - idx.index(Ellipsis)) + 0
            continue
        if it is None:
            out = unsqueeze(out, d)
            d += 1
            continue
        if isinstance(it, numbers.Integral):
            out = select(out, d, int(it))
            continue
        if isinstance(it, slice):
            start, stop, step = it.indices(out.shape[d])
            if step != 1:
                raise NotImplementedError("strided slicing")
            out = narrow(out, d, start, max(0, stop - start))
            d += 1
            continue
        if isinstance(it, Tensor):
            # advanced indexing wraps negative indices once (index_select
            # itself rejects them): a gather along d, whose kernel wraps
            out = _take_along(out, d, it)
            d += 1
            continue
        raise TypeError("unsupported index %r" % (it,))
    return out


def cat(tensors, dim=0):
    """cat (Tensor.ts:152-235): one strided copy per input."""
    tensors = list(tensors)
    if not tensors:
        raise RuntimeError("cat of an empty list")
    d = _wrap_dim(dim, tensors[0].ndim)
    dt = tensors[0].dtype
    shape = list(tensors[0].shape)
    shape[d] = sum(t.shape[d] for t in tensors)
    out = empty(shape, dt)
    pos = 0
    sizes = []
    for t in tensors:
        dst = _alias(out, t.shape, out._strides, pos * out._strides[d])
        _copy_into(dst, t)
        sizes.append(t.shape[d])
        pos += t.shape[d]

    def bwd(g):
        res = []
        p = 0
        for s in sizes:
            res.append(_alias(g, g.shape[:d] + (s,) + g.shape[d + 1:], g._strides,
                              g._offset + p * g._strides[d]))
            p += s
        return res

    def gbwd(g):
        res, p = [], 0
        for s in sizes:
            res.append(narrow(g, d, p, s))
            p += s
        return res
    return _record(out, "Cat", tensors, bwd, gfn=gbwd)


def stack(tensors, dim=0):
    tensors = list(tensors)
    d = _wrap_dim(dim, tensors[0].ndim + 1)
    return cat([unsqueeze(t, d) for t in tensors], d)


def masked_fill(x, mask, value):
    """masked_fill (Tensor.ts:804-832) with a broadcastable mask; backward
    zeroes the masked positions (torch.js has none, D12)."""
    if x.dtype != "float32":
        x = x.float()
    m = mask
    if m.dtype != "uint8" and m.dtype != "bool":
        m = _to_mask(m)
    shape = x.shape
    mst = _bstrides(m, shape)
    out = empty(shape)
    if out.numel():
        L.check(L.lib().tjh_masked_fill(len(shape), L.i64arr(shape), x.data_ptr(),
                                        L.i64arr(x._strides), m.data_ptr(), L.i64arr(mst),
                                        float(value), out.data_ptr()), "masked_fill")

    def bwd(g):
        g = g.contiguous()
        o = empty(shape)
        L.check(L.lib().tjh_masked_fill(len(shape), L.i64arr(shape), g.data_ptr(),
                                        L.i64arr(g._strides), m.data_ptr(), L.i64arr(mst), 0.0,
                                        o.data_ptr()), "masked_fill_backward")
        return [o]
    return _record(out, "MaskedFill", [x], bwd, gfn=lambda g: [masked_fill(g, m, 0.0)])


def _to_mask(t):
    """A bool (one byte per element) view of t != 0, on the device."""
    return t if t._dtype == "bool" else _k_cast(t, "bool")


# ------------------------------------------------------------ indexing


def _idx32(index):
    if not isinstance(index, Tensor):
        index = tensor(np.asarray(index, dtype=np.int32), dtype="int32")
    if index.dtype != "int32":
        index = index.to("int32")
    return index.contiguous()


def index_select(x, dim, index):
    """index_select (Tensor.ts:1242-1287) for any rank; backward is an
    ordered index_add (torch.js has none).  Indices must lie in [0, n):
    PyTorch's index_select raises for anything else, negatives included
    (torch.js's index_select.wgsl:32-52 casts them to u32 and reads out of
    bounds), and so does this one."""
    d = _wrap_dim(dim, x.ndim)
    index = _idx32(index)
    if index.ndim != 1:
        raise RuntimeError("index_select: index must be 1-D")
    xc = x.contiguous() if x.dtype == "float32" else x.float().contiguous()
    outer, src, inner = _numel(xc.shape[:d]), xc.shape[d], _numel(xc.shape[d + 1:])
    n = index.numel()
    host = index.numpy()
    if n and (host.max() >= src or host.min() < 0):
        bad = int(host.min()) if host.min() < 0 else int(host.max())
        raise IndexError("index_select: index %d is out of range for dimension of size %d"
                         % (bad, src))
    oshape = xc.shape[:d] + (n,) + xc.shape[d + 1:]
    out = empty(oshape)
    L.check(L.lib().tjh_index_select(xc.data_ptr(), outer, src, inner, index.data_ptr(), n,
                                     out.data_ptr()), "index_select")
    xs = xc.shape

    def bwd(g):
        g = g.contiguous()
        z = zeros(xs)
        L.check(L.lib().tjh_index_add(z.data_ptr(), outer, src, inner, index.data_ptr(), n,
                                      g.data_ptr()), "index_add")
        return [z]
    return _record(out, "IndexSelect", [x], bwd,
                   gfn=lambda g: [_index_add_rec(xs, d, index, g)])


def _index_add_rec(xs, d, index, src):
    """zeros(xs) with src's slices added at `index` along dim d (the ordered
    index_add of index_select's backward) as a recorded op of src, whose
    own gradient is index_select of the incoming one: index_select's
    differentiable backward."""
    src = src.contiguous()
    outer, n_src, inner = _numel(xs[:d]), xs[d], _numel(xs[d + 1:])
    z = zeros(xs)
    L.check(L.lib().tjh_index_add(z.data_ptr(), outer, n_src, inner, index.data_ptr(),
                                  index.numel(), src.data_ptr()), "index_add")
    return _record(z, "IndexAdd", [src], lambda g: [index_select(g, d, index)],
                   gfn=lambda g: [index_select(g, d, index)])


def gather(x, dim, index):
    """gather (Tensor.ts:2651-2705): negative indices wrap; backward is an
    ordered scatter_add."""
    d = _wrap_dim(dim, x.ndim)
    index = _idx32(index)
    if index.ndim != x.ndim:
        raise RuntimeError("gather: index must have the same rank as input")
    for i in range(x.ndim):
        if i != d and index.shape[i] != x.shape[i]:
            raise RuntimeError("gather: index shape %s incompatible with input %s"
                               % (list(index.shape), list(x.shape)))
    xc = x.contiguous() if x.dtype == "float32" else x.float().contiguous()
    outer, src, inner = _numel(xc.shape[:d]), xc.shape[d], _numel(xc.shape[d + 1:])
    ilen = index.shape[d]
    out = empty(index.shape)
    L.check(L.lib().tjh_gather(xc.data_ptr(), outer, src, inner, index.data_ptr(), ilen,
                               out.data_ptr()), "gather")
    xs = xc.shape

    def bwd(g):
        g = g.contiguous()
        z = zeros(xs)
        L.check(L.lib().tjh_scatter_add(z.data_ptr(), outer, src, inner, index.data_ptr(), ilen,
                                        g.data_ptr()), "scatter_add")
        return [z]
    return _record(out, "Gather", [x], bwd, gfn=lambda g: [_scatter_add_rec(xs, d, index, g)])


def _scatter_add_rec(xs, d, index, src):
    """zeros(xs) with src scattered-added at `index` along dim d (gather's
    ordered backward) as a recorded op of src, whose own gradient is the
    gather of the incoming one: gather's differentiable backward."""
    src = src.contiguous()
    outer, n_src, inner = _numel(xs[:d]), xs[d], _numel(xs[d + 1:])
    z = zeros(xs)
    L.check(L.lib().tjh_scatter_add(z.data_ptr(), outer, n_src, inner, index.data_ptr(),
                                    index.shape[d], src.data_ptr()), "scatter_add")
    return _record(z, "ScatterAdd", [src], lambda g: [gather(g, d, index)],
                   gfn=lambda g: [gather(g, d, index)])


def _take_along(x, d, index):
    """x[..., index, ...] along dim d for a 1-D index whose negative entries
    wrap once (advanced indexing): a gather with the index broadcast over
    the other dims, so the wrap happens on the device; the backward is the
    gather's ordered scatter-add."""
    idx = _idx32(index).reshape(-1)
    n = x.shape[d]
    host = idx.numpy()  # range check only (as index_select does)
    if host.size and (host.min() < -n or host.max() >= n):
        raise IndexError("index out of range for dimension of size %d" % n)
    shape = x.shape[:d] + (idx.numel(),) + x.shape[d + 1:]
    st = [0] * len(shape)
    st[d] = 1
    full_idx = _k_contiguous(Tensor(idx._storage, shape, tuple(st), idx._offset, "int32"))
    return gather(x, d, full_idx)


def nonzero(x):
    """nonzero (Tensor.ts:1323-1345): [nnz, ndim] int32, row-major order."""
    xc = x.contiguous() if x.dtype == "float32" else x.float().contiguous()
    nd = max(1, xc.ndim)
    shape = xc.shape if xc.ndim else (1,)
    cnt = ctypes.c_int64(0)
    L.check(L.lib().tjh_nonzero(xc.data_ptr(), nd, L.i64arr(shape), None, 0, ctypes.byref(cnt)),
            "nonzero")
    out = empty((cnt.value, nd), "int32")
    if cnt.value:
        L.check(L.lib().tjh_nonzero(xc.data_ptr(), nd, L.i64arr(shape), out.data_ptr(),
                                    cnt.value, ctypes.byref(cnt)), "nonzero")
    return out


# ------------------------------------------------------------ matmul


def _mat_operand(t):
    """(ptr, ld, trans, batch_stride) of the last two dims of t, or None
    when they are neither row- nor column-major."""
    r, c = t.shape[-2], t.shape[-1]
    s0, s1 = t._strides[-2], t._strides[-1]
    if (s1 == 1 or c == 1) and s0 >= max(1, c):
        return t.data_ptr(), max(s0, 1), False
    if (s0 == 1 or r == 1) and s1 >= max(1, r):
        return t.data_ptr(), max(s1, 1), True
    return None


def _gemm(a, b, out=None, alpha=1.0, beta=0.0, bias=None, bias_mode=0, rowsum_out=None,
          aux=None, act=0):
    """out[M,N] = alpha*a[M,K] @ b[K,N] (+beta*out) (+bias) for 2-D views.
    rowsum_out (a contiguous [M] tensor) receives the row sums of `a` from
    the same launch (bias_mode 3: a Linear layer's bias gradient computed
    with its weight gradient).  act 1 / 2 / 3 with aux ([M,N], row stride
    as out's) fuses an elementwise op into the epilogue: 1 writes the
    pre-activation to aux and GELU of it to out, 2 multiplies by
    GELU'(aux), 3 adds aux (a residual; must not overlap out)."""
    if rowsum_out is not None:
        assert bias is None and bias_mode == 0 and rowsum_out.is_contiguous()
        bias, bias_mode = rowsum_out, 3
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    oa = _mat_operand(a)
    if oa is None:
        a = _k_contiguous(a)
        oa = _mat_operand(a)
    ob = _mat_operand(b)
    if ob is None:
        b = _k_contiguous(b)
        ob = _mat_operand(b)
    if out is None:
        out = _empty_padded(M, N) if N % 4 else empty((M, N))
    ldc = out._strides[0] if out._strides[0] >= N else N
    if act:
        assert aux is not None and aux.shape == (M, N) and aux._strides[1] == 1
        L.check(L.lib().tjh_gemm_act(1 if oa[2] else 0, 1 if ob[2] else 0, M, N, K, float(alpha),
                                     oa[0], oa[1], ob[0], ob[1], float(beta), out.data_ptr(), ldc,
                                     bias.data_ptr() if bias is not None else None, bias_mode,
                                     aux.data_ptr(), aux._strides[0], act), "gemm_act")
        return out
    L.check(L.lib().tjh_gemm(1 if oa[2] else 0, 1 if ob[2] else 0, M, N, K, float(alpha), oa[0],
                             oa[1], 0, ob[0], ob[1], 0, float(beta), out.data_ptr(), ldc, 0, 1,
                             bias.data_ptr() if bias is not None else None, bias_mode), "gemm")
    return out


def _gemm_ce(ce, b, trans):
    """op(D) @ b for the unformed cross-entropy gradient D = ce [rows, cols]:
    trans False gives D [rows, cols] @ b [cols, N], trans True D^T @ b [rows,
    N]; D is formed while the GEMM loads it (tjh_gemm_ce), bit for bit the
    product over the stored gradient."""
    M, K = (ce.cols, ce.rows) if trans else (ce.rows, ce.cols)
    if b.shape[0] != K:
        raise RuntimeError("gemm_ce: %d rows for a K of %d" % (b.shape[0], K))
    N = b.shape[1]
    ob = _mat_operand(b)
    if ob is None or ob[2]:
        b = _k_contiguous(b)
        ob = _mat_operand(b)
    out = _empty_padded(M, N) if N % 4 else empty((M, N))
    ldc = out._strides[0] if out._strides[0] >= N else N
    xp, ld = ce.rows_view()
    rs = ce.row_scale()
    L.check(L.lib().tjh_gemm_ce(1 if trans else 0, M, N, K, xp, ld, ce.lse.data_ptr(),
                                ce.t.data_ptr(), rs.data_ptr(), ob[0], ob[1], out.data_ptr(), ldc),
            "gemm_ce")
    return out


def _bgemm(a, b):
    """Batched a[B,M,K] @ b[B,N,K...] with uniform batch strides (3-D views)."""
    Bn, M, K = a.shape
    _, _, N = b.shape
    oa = _mat_operand(a)
    if oa is None:
        a = _k_contiguous(a)
        oa = _mat_operand(a)
    ob = _mat_operand(b)
    if ob is None:
        b = _k_contiguous(b)
        ob = _mat_operand(b)
    out = empty((Bn, M, N))
    L.check(L.lib().tjh_gemm(1 if oa[2] else 0, 1 if ob[2] else 0, M, N, K, 1.0, oa[0], oa[1],
                             a._strides[0] if Bn > 1 else 0, ob[0], ob[1],
                             b._strides[0] if Bn > 1 else 0, 0.0, out.data_ptr(), N, M * N, Bn,
                             None, 0), "bgemm")
    return out


def _flatten_batch(t, bshape):
    """t expanded to bshape + t.shape[-2:], viewed as [B, r, c] with one
    batch stride; copies when the batch dims cannot share one stride."""
    full_shape = tuple(bshape) + t.shape[-2:]
    e = expand(t, full_shape) if t.shape != full_shape else t
    nb = len(bshape)
    bst = e._strides[:nb]
    # one stride for the flattened batch: all-zero, or mergeable dims
    B = _numel(bshape)
    if B <= 1:
        return Tensor(e._storage, (max(B, 1),) + e.shape[-2:], (0,) + e._strides[-2:], e._offset,
                      e._dtype) if B == 1 else e
    if all(s == 0 for s in bst):
        return Tensor(e._storage, (B,) + e.shape[-2:], (0,) + e._strides[-2:], e._offset, e._dtype)
    ok = all(bst[i] == bst[i + 1] * bshape[i + 1] for i in range(nb - 1))
    if ok:
        return Tensor(e._storage, (B,) + e.shape[-2:], (bst[-1],) + e._strides[-2:], e._offset,
                      e._dtype)
    c = _k_contiguous(e)
    return Tensor(c._storage, (B,) + c.shape[-2:], None, c._offset, c._dtype)


def matmul(a, b):
    """matmul with NumPy batch broadcasting (Tensor.ts:2136-2290); backward
    gives both operands their products (torch.js: the left one only, D1)."""
    if a.dtype != "float32":
        a = a.float()
    if b.dtype != "float32":
        b = b.float()
    if a.ndim == 0 or b.ndim == 0:
        raise RuntimeError("matmul: both arguments need at least 1 dimension")
    if a.ndim == 1 and b.ndim == 1:
        return reduce_sum(mul(a, b))
    if a.ndim == 1:
        return squeeze(matmul(unsqueeze(a, 0), b), -2)
    if b.ndim == 1:
        return squeeze(matmul(a, unsqueeze(b, 1)), -1)
    if a.shape[-1] != b.shape[-2]:
        raise RuntimeError("matmul: shapes %s and %s cannot be multiplied"
                           % (list(a.shape), list(b.shape)))
    if b.ndim == 2 and a.ndim >= 2:
        # [..., M, K] @ [K, N]: flatten leading dims into M
        lead = a.shape[:-1]
        a2 = reshape(a, (_numel(lead), a.shape[-1])) if a.ndim > 2 else a
        out2 = _mm(a2, b)
        return reshape(out2, lead + (b.shape[-1],)) if a.ndim > 2 else out2
    bshape = _broadcast_shapes(a.shape[:-2], b.shape[:-2])
    M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
    a3 = _flatten_batch(a.detach(), bshape)
    b3 = _flatten_batch(b.detach(), bshape)
    out3 = _bgemm(a3, b3)
    out = _view_raw(out3, tuple(bshape) + (M, N))
    ash, bsh = a.shape, b.shape

    def bwd(g):
        g3 = _view_raw(g.contiguous(), (_numel(bshape), M, N))
        ga = gb = None
        if a.requires_grad:
            bt = Tensor(b3._storage, (b3.shape[0], N, K), (b3._strides[0], b3._strides[2],
                                                           b3._strides[1]), b3._offset)
            ga = _sum_to(_view_raw(_bgemm(g3, bt), tuple(bshape) + (M, K)), ash)
        if b.requires_grad:
            at = Tensor(a3._storage, (a3.shape[0], K, M), (a3._strides[0], a3._strides[2],
                                                           a3._strides[1]), a3._offset)
            gb = _sum_to(_view_raw(_bgemm(at, g3), tuple(bshape) + (K, N)), bsh)
        return [ga, gb]

    def gbwd(g):
        return [_sum_to_g(matmul(g, transpose(b, -2, -1)), ash) if a.requires_grad else None,
                _sum_to_g(matmul(transpose(a, -2, -1), g), bsh) if b.requires_grad else None]
    return _record(out, "BMM", [a, b], bwd, gfn=gbwd)


def _mm(a, b):
    out = _gemm(a, b)

    def bwd(g):
        ga = _gemm(g, b.detach().T) if a.requires_grad else None
        gb = _gemm(a.detach().T, g) if b.requires_grad else None
        return [ga, gb]

    def gbwd(g):
        return [matmul(g, transpose(b, 0, 1)) if a.requires_grad else None,
                matmul(transpose(a, 0, 1), g) if b.requires_grad else None]
    return _record(out, "MM", [a, b], bwd, gfn=gbwd)


_add_unary_methods()


# ----------------------------------------------------------------- engine


class _SliceGrad:
    """Gradient of a narrow()/split() output w.r.t. the full input, kept as
    (start, tensor) pieces along `dim` until the input's own node runs.  The
    pieces of one split are then assembled in one go: with no zero fill
    when they tile the input, and with no copy at all when they already sit
    at their places in one buffer (attention's backward writes dq, dk, dv
    into the layout of the fused qkv projection)."""

    __slots__ = ("shape", "dim", "pieces")

    def __init__(self, shape, dim, pieces):
        self.shape = tuple(shape)
        self.dim = dim
        self.pieces = pieces

    def merge(self, other):
        return _SliceGrad(self.shape, self.dim, self.pieces + other.pieces)

    def materialize(self):
        d, n = self.dim, self.shape[self.dim]
        pieces = sorted(self.pieces, key=lambda p: p[0])
        pos, tiles = 0, True
        for start, g in pieces:
            if start != pos:
                tiles = False
                break
            pos += g.shape[d]
        tiles = tiles and pos == n
        if tiles:
            # one buffer already holding every piece at its place?
            g0 = pieces[0][1]
            st = _contig_strides(self.shape)
            base = g0._offset
            if all(g._storage is g0._storage and tuple(g._strides) == st and
                   g._offset == base + start * st[d] and g._dtype == g0._dtype
                   for start, g in pieces):
                return Tensor(g0._storage, self.shape, st, base, g0._dtype)
            out = empty(self.shape, dtype=g0._dtype)
        else:
            out = zeros(self.shape, dtype=pieces[0][1]._dtype)
        covered = [False] * n
        for start, g in pieces:
            ln = g.shape[d]
            dst = _alias(out, g.shape, out._strides, out._offset + start * out._strides[d])
            if any(covered[start:start + ln]):
                _copy_into(dst, _k_binary("add", dst, g))  # overlapping narrows add up
            else:
                _copy_into(dst, g)
            for i in range(start, start + ln):
                covered[i] = True
        return out


class _CEGrad:
    """The cross-entropy gradient of logits x [rows, cols] (row stride ld)
    without weights or smoothing, (softmax(x) - onehot(t)) * s_r, kept
    unformed: the Linear layer that produced the logits forms it while its
    backward GEMMs load their A tiles (tjh_gemm_ce), so the [rows, cols]
    gradient is never written; any other consumer gets it materialized by
    the cross-entropy backward kernel.  `shape` is the logical shape: [rows,
    cols] or a reshape of it that keeps cols last."""

    __slots__ = ("shape", "x", "t", "lse", "g", "rows", "cols", "ignore", "red", "_rs")

    def __init__(self, shape, x, t, lse, g, ignore, red, rs=None):
        self.shape = tuple(shape)
        self.x, self.t, self.lse, self.g = x, t, lse, g
        self.rows, self.cols = x.shape
        self.ignore, self.red = ignore, red
        self._rs = rs

    @property
    def ndim(self):
        return len(self.shape)

    def numel(self):
        return self.rows * self.cols

    def reshaped(self, shape):
        shape = tuple(shape)
        if shape and shape[-1] == self.cols and _numel(shape) == self.numel():
            return _CEGrad(shape, self.x, self.t, self.lse, self.g, self.ignore, self.red,
                           self._rs)
        return reshape_raw(self.materialize(), shape)

    def rows_view(self):
        return self.x.data_ptr(), self.x._strides[0]

    def row_scale(self):
        if self._rs is None:
            rs = empty((self.rows,))
            L.check(L.lib().tjh_cross_entropy_row_scale(
                self.t.data_ptr(), self.g.data_ptr(), self.rows, self.cols, self.ignore,
                self.red, rs.data_ptr()), "cross_entropy_row_scale")
            self._rs = rs
        return self._rs

    def materialize(self):
        rows, cols = self.rows, self.cols
        d = _empty_padded(rows, cols) if cols % 4 else empty((rows, cols))
        xp, ld = self.rows_view()
        L.check(L.lib().tjh_cross_entropy_backward(
            xp, ld, self.t.data_ptr(), None, 0.0, self.lse.data_ptr(), self.g.data_ptr(), rows,
            cols, self.ignore, self.red, d.data_ptr(), d._strides[0], 0), "cross_entropy_backward")
        return d if self.shape == (rows, cols) else reshape_raw(d, self.shape)


# nodes whose VJP takes a _CEGrad as it is (View reshapes it, Linear forms
# it inside its GEMMs); every other node receives it materialized
_CE_NODES = ("View", "Linear")
# forming the cross-entropy gradient inside the LM head's GEMMs instead of
# storing it (TJH_FUSE_CE=1).  Off by default: it saves the [rows, classes]
# gradient's memory and its write and read (0.56 ms per GPT-2 step), but
# the exp per element that every column tile of the two GEMMs repeats runs
# between their MFMAs and their LDS stores and costs them 2.6 ms
_FUSE_CE = os.environ.get("TJH_FUSE_CE", "0") == "1"


def _dense(g):
    if isinstance(g, (_SliceGrad, _CEGrad)):
        return g.materialize()
    return g


def _accumulate(store, key, g):
    prev = store.get(key)
    if prev is None:
        store[key] = g
    elif (isinstance(prev, _SliceGrad) and isinstance(g, _SliceGrad) and
          prev.shape == g.shape and prev.dim == g.dim):
        store[key] = prev.merge(g)
    else:
        store[key] = _k_binary("add", _dense(prev), _dense(g))


def _toposort(roots):
    order = []
    seen = set()
    stack = [(n, False) for n in roots if n is not None]
    while stack:
        node, done = stack.pop()
        if done:
            order.append(node)
            continue
        if id(node) in seen:
            continue
        seen.add(id(node))
        stack.append((node, True))
        for t in node.inputs:
            if t is not None and t.grad_fn is not None and id(t.grad_fn) not in seen:
                stack.append((t.grad_fn, False))
    return order  # post-order: inputs before users


def _graph_vjp(out, g, inputs):
    """Recording VJP of the subgraph between `inputs` and `out`: the
    create_graph sweep run from `out` with gradient g, stopping at the
    inputs (nothing past them is visited).  Returns their gradients (None
    for an input the output does not depend on), which carry graphs back
    to g and to the inputs."""
    stop = {id(t) for t in inputs if t is not None}
    res = [None] * len(inputs)
    if out.grad_fn is None:
        return res
    order, seen = [], set()
    stack = [(out.grad_fn, False)]
    while stack:
        node, done = stack.pop()
        if done:
            order.append(node)
            continue
        if id(node) in seen:
            continue
        seen.add(id(node))
        stack.append((node, True))
        for t in node.inputs:
            if t is not None and id(t) not in stop and t.grad_fn is not None \
                    and id(t.grad_fn) not in seen:
                stack.append((t.grad_fn, False))
    grads = {id(out.grad_fn): g}
    found = {}
    for node in reversed(order):
        gn = grads.pop(id(node), None)
        if gn is None:
            continue
        if node.gfn is None:
            raise NotImplementedError(
                "create_graph: %s has no differentiable backward on the hip device" % node.name)
        for t, gi in zip(node.inputs, node.gfn(gn)):
            if t is None or gi is None:
                continue
            if tuple(gi.shape) != t.shape:
                gi = _sum_to_g(gi, t.shape) if gi.ndim >= t.ndim else reshape(gi, t.shape)
            if id(t) in stop:
                found[id(t)] = gi if id(t) not in found else add(found[id(t)], gi)
            elif t.grad_fn is not None:
                k = id(t.grad_fn)
                grads[k] = gi if k not in grads else add(grads[k], gi)
    return [found.get(id(t)) if t is not None else None for t in inputs]


def _regrad(fn, inputs, g):
    """Recording VJP of a fused op from its definition: fn(*inputs) written
    with recording (differentiable) ops is recomputed in grad mode and its
    subgraph differentiated down to the inputs (_graph_vjp)."""
    prev = _grad["enabled"]
    _grad["enabled"] = True
    try:
        return _graph_vjp(fn(*inputs), g, inputs)
    finally:
        _grad["enabled"] = prev


def _run_backward_graph(pairs, retain_graph, inputs):
    """The sweep of run_backward with create_graph: grad mode stays on and
    every node runs its recording VJP (Node.gfn), so the gradients it
    produces carry graphs back to the leaves and can be differentiated again
    (torch.js runs its backward closures with grad mode on, Tensor.ts:3686,
    so its gradients record the same way).  None of the engine's fusions
    take part: gradients are summed with recording adds."""
    prev = _grad["enabled"]
    _grad["enabled"] = True
    try:
        grads = {}
        roots = []
        wanted = {id(t): t for t in inputs} if inputs is not None else None
        results = {}

        def acc(d, key, g):
            d[key] = g if key not in d else add(d[key], g)

        def to_leaf(t, g):
            if t._grad is None:
                t._grad = g
            else:
                t._grad = add(t._grad, g)

        for t, g in pairs:
            if g.shape != t.shape:
                g = reshape(g, t.shape) if g.numel() == t.numel() else expand(g, t.shape)
            if t.grad_fn is None:
                if wanted is not None:
                    if id(t) in wanted:
                        acc(results, id(t), g)
                elif t.requires_grad:
                    to_leaf(t, g)
                continue
            acc(grads, id(t.grad_fn), g)
            roots.append(t.grad_fn)
        for node in reversed(_toposort(roots)):
            g = grads.pop(id(node), None)
            if g is None:
                continue
            if node.fn is None:
                raise RuntimeError("Trying to backward through the graph a second time; "
                                   "pass retain_graph=True the first time")
            if node.gfn is None:
                raise NotImplementedError(
                    "create_graph: %s has no differentiable backward on the hip device"
                    % node.name)
            in_grads = node.gfn(g)
            for t, gi in zip(node.inputs, in_grads):
                if t is None or gi is None:
                    continue
                if tuple(gi.shape) != t.shape:
                    gi = _sum_to_g(gi, t.shape) if gi.ndim >= t.ndim else reshape(gi, t.shape)
                if wanted is not None and id(t) in wanted:
                    acc(results, id(t), gi)
                if t.grad_fn is not None:
                    acc(grads, id(t.grad_fn), gi)
                    if t._retains_grad and wanted is None:
                        to_leaf(t, gi)
                elif wanted is None and t.requires_grad:
                    to_leaf(t, gi)
            if not retain_graph:
                node.fn = None
                node.gfn = None
                node.inputs = [None] * len(node.inputs)
        if wanted is not None:
            return [results.get(id(t)) for t in inputs]
        return None
    finally:
        _grad["enabled"] = prev


def run_backward(pairs, retain_graph=False, inputs=None, create_graph=False):
    """Reverse-topological VJP sweep (Tensor.backward, Tensor.ts:3686-3740;
    accumulateGrad, Tensor.ts:3670-3677).  With `inputs`, returns their
    gradients instead of accumulating into leaves (autograd.grad).  With
    `create_graph`, the gradients are built from recording ops
    (_run_backward_graph)."""
    if create_graph:
        return _run_backward_graph(pairs, retain_graph, inputs)
    prev = _grad["enabled"]
    _grad["enabled"] = False
    deferred = set()  # ids of leaves whose .grad awaits tjh_flush_deferred
    try:
        grads = {}
        roots = []
        wanted = {id(t): t for t in inputs} if inputs is not None else None
        results = {}
        owned = _Owned()  # gradient memory already handed to a leaf in this pass
        for t, g in pairs:
            if g.shape != t.shape:
                if g.numel() == t.numel():
                    g = reshape_raw(g, t.shape)
                else:
                    g = g.expand(t.shape)
            if t.grad_fn is None:
                if wanted is not None:
                    if id(t) in wanted:
                        _accumulate(results, id(t), g)
                elif t.requires_grad:
                    _leaf_accumulate(t, g, owned, force_copy=True)
                continue
            _accumulate(grads, id(t.grad_fn), g)
            roots.append(t.grad_fn)
        order = _toposort(roots)
        for node in reversed(order):
            g = grads.pop(id(node), None)
            if not (isinstance(g, _CEGrad) and node.name in _CE_NODES):
                g = _dense(g)
            if g is None:
                continue
            if node.fn is None:
                raise RuntimeError("Trying to backward through the graph a second time; "
                                   "pass retain_graph=True the first time")
            if deferred and any(t is not None and id(t) in deferred for t in node.inputs):
                _flush_deferred(deferred)  # this node may read or add to such a .grad
            acc = _pending_for(node, grads, wanted, owned)
            defer = _can_defer(node, wanted)
            kw = {}
            if acc is not None:
                kw["pending"] = acc
            if defer:
                kw["defer"] = True
            in_grads = node.fn(g, **kw)
            del g
            for slot, (t, gi) in enumerate(zip(node.inputs, in_grads)):
                if t is None or gi is None:
                    continue
                if defer and slot in node.defer_slots:
                    # a leaf's first gradient, finished by the next flush
                    t._grad = gi
                    owned.add(gi)
                    deferred.add(id(t))
                    continue
                if acc is not None and slot == node.acc_slot:
                    # gi already holds the pending gradient
                    if t.grad_fn is None:
                        t._grad = gi
                    else:
                        grads[id(t.grad_fn)] = gi
                    continue
                if isinstance(gi, (_SliceGrad, _CEGrad)) and (
                        t.grad_fn is None or t._retains_grad or
                        (wanted is not None and id(t) in wanted)):
                    gi = gi.materialize()
                if isinstance(gi, _CEGrad) and tuple(gi.shape) != t.shape:
                    gi = gi.materialize()
                if tuple(gi.shape) != t.shape:
                    gi = _sum_to(gi, t.shape) if gi.ndim >= t.ndim else reshape_raw(gi, t.shape)
                if wanted is not None and id(t) in wanted:
                    _accumulate(results, id(t), gi)
                if t.grad_fn is not None:
                    _accumulate(grads, id(t.grad_fn), gi)
                    if t._retains_grad and wanted is None:
                        _leaf_accumulate(t, gi, owned)
                elif wanted is None and t.requires_grad:
                    _leaf_accumulate(t, gi, owned)
            if not retain_graph:
                # drop the saved tensors and input references: the graph
                # cannot be replayed (torch.js nulls grad_fn, Tensor.ts:3735-3739)
                node.fn = None
                node.inputs = [None] * len(node.inputs)
        if deferred:
            _flush_deferred(deferred)
        _finish_siblings()
        # a loss that is a deferred reduction is evaluated with the pass
        # (its column sums usually came with the gradients' own kernel)
        for t, _ in pairs:
            if t._st is None and t._lz is not None and t._lz.kind == "thunk":
                t._storage
        if wanted is not None:
            return [_dense(results.get(id(t))) for t in inputs]
        return None
    finally:
        if deferred:
            _flush_deferred(deferred)
        _SIBLINGS.clear()
        _grad["enabled"] = prev


def _can_defer(node, wanted):
    """Whether the VJP may leave the gradients of node.defer_slots for the
    library's next flush: each such input is a distinct leaf that has no
    .grad yet (so the gradient is only stored, never read, until the
    flush)."""
    if not node.defer_slots or not _FUSE_ACC or wanted is not None:
        return False
    seen = set()
    for k in node.defer_slots:
        t = node.inputs[k]
        if t is None:
            continue
        if (t.grad_fn is not None or t._grad is not None or not t.requires_grad or
                id(t) in seen):
            return False
        # the same tensor in another slot (layer_norm(w, (n,), w, b)) gets a
        # second contribution from this node, which a deferred .grad would lose
        if any(j != k and u is t for j, u in enumerate(node.inputs)):
            return False
        seen.add(id(t))
    return bool(seen)


class _Owned:
    """Gradient memory a backward pass has handed to one holder (a leaf's
    .grad, or a gradient folded into a VJP's output).  Memory is recorded
    by storage identity.  A deferred gradient, which has no storage yet, is
    recorded by its own identity and held for the pass (so that identity is
    never reused by another object); once it is computed its storage counts
    as recorded too, so a gradient handed to two leaves is seen as owned
    under either key, before and after it is computed."""

    __slots__ = ("keys", "held", "waiting")

    def __init__(self):
        self.keys = set()
        self.held = []     # every tensor recorded while deferred
        self.waiting = []  # those whose storage is not recorded yet

    def add(self, t):
        k = _skey(t)
        self.keys.add(k)
        if not isinstance(k, int):
            self.held.append(t)
            self.waiting.append(t)

    def has(self, t):
        if self.waiting:
            still = []
            for h in self.waiting:
                k = _skey(h)
                if isinstance(k, int):
                    self.keys.add(k)
                else:
                    still.append(h)
            self.waiting = still
        return _skey(t) in self.keys


def _flush_deferred(deferred):
    L.check(L.lib().tjh_flush_deferred(), "flush_deferred")
    deferred.clear()


def _pending_for(node, grads, wanted, owned):
    """The gradient pending for input `node.acc_slot`, when the VJP may fold
    it in: one dense contiguous float32 tensor of the input's shape, and
    either the pending gradient of a non-leaf that retains no grad, or the
    .grad of a leaf that this backward pass created and that no pending
    gradient shares storage with (the VJP may then add into it in place, as
    the embedding backward of a table tied to the LM head does).  Inputs
    asked for by autograd.grad never take part."""
    k = node.acc_slot
    if k is None or not _FUSE_ACC:
        return None
    t = node.inputs[k]
    if t is None or (wanted is not None):
        return None
    if t.grad_fn is None:
        prev = t._grad
        if prev is None or not owned.has(prev):
            return None
        others = [p for p in grads.values()]
    else:
        if t._retains_grad:
            return None
        prev = grads.get(id(t.grad_fn))
        if prev is None or isinstance(prev, (_SliceGrad, _CEGrad)):
            return None
        # a pending gradient may be the very tensor an add / sub / scalar-add
        # VJP also handed to another input, a leaf's .grad among them: the
        # VJP may add into it in place only if nothing else holds it
        if owned.has(prev):
            return None
        others = [p for key, p in grads.items() if key != id(t.grad_fn)]
    if (prev is None or isinstance(prev, _SliceGrad) or prev.shape != t.shape or
            prev._dtype != "float32" or not prev.is_contiguous()):
        return None
    pk = _skey(prev)
    for p in others:
        if isinstance(p, _CEGrad):
            continue  # holds no gradient storage yet
        pieces = p.pieces if isinstance(p, _SliceGrad) else [(0, p)]
        if any(_skey(q) == pk for _, q in pieces):
            return None
    # the VJP adds into prev in place: deferred values reading it go first
    _before_write(prev)
    return prev


# folding pending gradients into VJPs (acc_slot); off only to compare with
# the plain sum in tests
_FUSE_ACC = True


def _leaf_accumulate(t, g, owned, force_copy=False):
    """Accumulates into t.grad.  A gradient tensor handed to a leaf is never
    shared with another leaf (the same incoming grad can flow to several
    inputs of an add), so later in-place edits of one .grad stay local."""
    lazy = _is_lazy(g) and g._lz.kind != "alias"
    if (lazy and not force_copy and t._grad is None and _FUSE_SIB and _LAZY["jit"] and
            not owned.has(g)):
        # a deferred gradient stays deferred until a column sum over a
        # sibling takes it along, or the pass ends; no other leaf holds it
        owned.add(g)
        t._grad = g
        _SIBLINGS.append(g)
        return
    if lazy and not force_copy and not owned.has(g):
        g._storage  # a deferred gradient evaluates into memory nothing else holds
    elif force_copy or not g.is_contiguous() or owned.has(g):
        g = _k_contiguous(g)
    if t._grad is None:
        owned.add(g)
        t._grad = Tensor(g._storage, g._shape, g._strides, g._offset, g._dtype)
    else:
        t._grad = _k_binary("add", t._grad, g)
