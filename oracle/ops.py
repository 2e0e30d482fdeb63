"""Per-op forward / backward restatements (numpy, float64 unless noted).
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import math

import numpy as np

F64 = np.float64
F32 = np.float32

# ------------------------------------------------------------------ erf / gelu


def erfc_as(a):
    """1 - erf(a), a >= 0, by Abramowitz & Stegun 7.1.26 — the erf of
    torch.js's WGSL (src/backend/webgpu/shaders/unary.wgsl:230-236), with
    the complement P(t) exp(-a^2) kept whole (no 1 - (1 - P) cancellation)."""
    a = np.asarray(a, dtype=F64)
    t = 1.0 / (1.0 + 0.3275911 * a)
    p = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t
         + 0.254829592) * t
    return p * np.exp(-a * a)


def erf_as(x):
    """erf by A&S 7.1.26 (unary.wgsl:230-236): sign(x) * (1 - erfc_as(|x|))."""
    x = np.asarray(x, dtype=F64)
    return np.sign(x) * (1.0 - erfc_as(np.abs(x)))


def phi_cdf(x):
    """Phi(x) = 0.5 (1 + erf_as(x / sqrt 2))."""
    x = np.asarray(x, dtype=F64)
    c = 0.5 * erfc_as(np.abs(x) / math.sqrt(2.0))
    return np.where(x < 0, c, 1.0 - c)


def gelu(x):
    """0.5 x (1 + erf(x / sqrt 2)) (unary.wgsl:246-252) = x Phi(x)."""
    x = np.asarray(x, dtype=F64)
    return x * phi_cdf(x)


def gelu_grad(x):
    """d/dx GELU = Phi(x) + x phi(x) (the contract; torch.js's backward uses
    a tanh form with a wrong pdf term, Tensor.ts:3627-3632)."""
    x = np.asarray(x, dtype=F64)
    return phi_cdf(x) + x * np.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


# ------------------------------------------------------------------ unary


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def unary(op, x, alpha=0.0):
    """_unaryOp forward (Tensor.ts:3593-3610, unary.wgsl)."""
    x = np.asarray(x, dtype=F64)
    with np.errstate(all="ignore"):
        if op == "neg": return -x
        if op == "exp": return np.exp(x)
        if op == "log": return np.log(x)
        if op == "sqrt": return np.sqrt(x)
        if op == "rsqrt": return 1.0 / np.sqrt(x)
        if op == "tanh": return np.tanh(x)
        if op == "sigmoid": return _sigmoid(x)
        if op == "relu": return np.maximum(x, 0.0)
        if op == "gelu": return gelu(x)
        if op == "square": return x * x
        if op == "reciprocal": return 1.0 / x
        if op == "erf": return erf_as(x)
        if op == "abs": return np.abs(x)
        if op == "sin": return np.sin(x)
        if op == "cos": return np.cos(x)
        if op == "silu": return x * _sigmoid(x)
        if op == "leaky_relu": return np.where(x > 0, x, alpha * x)
        if op == "elu": return np.where(x > 0, x, alpha * (np.exp(x) - 1.0))
        if op == "softplus": return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
        if op == "sign": return np.sign(x)
    raise ValueError(op)


def unary_backward(op, g, x, alpha=0.0):
    """VJP of each unary op: g * op'(x)."""
    g = np.asarray(g, dtype=F64)
    x = np.asarray(x, dtype=F64)
    with np.errstate(all="ignore"):
        if op == "neg": return -g
        if op == "exp": return g * np.exp(x)
        if op == "log": return g / x
        if op == "sqrt": return g * 0.5 / np.sqrt(x)
        if op == "rsqrt": return g * -0.5 * x ** -1.5
        if op == "tanh": return g * (1.0 - np.tanh(x) ** 2)
        if op == "sigmoid":
            s = _sigmoid(x)
            return g * s * (1.0 - s)
        if op == "relu": return np.where(x > 0, g, 0.0)
        if op == "gelu": return g * gelu_grad(x)
        if op == "square": return g * 2.0 * x
        if op == "reciprocal": return -g / (x * x)
        if op == "erf": return g * 2.0 / math.sqrt(math.pi) * np.exp(-x * x)
        if op == "abs": return g * np.sign(x)
        if op == "sin": return g * np.cos(x)
        if op == "cos": return -g * np.sin(x)
        if op == "silu":
            s = _sigmoid(x)
            return g * s * (1.0 + x * (1.0 - s))
        if op == "leaky_relu": return np.where(x > 0, g, alpha * g)
        if op == "elu": return np.where(x > 0, g, g * alpha * np.exp(x))
        if op == "softplus": return np.where(x > 20, g, g * _sigmoid(x))
        if op == "sign": return np.zeros_like(g)
    raise ValueError(op)


# ------------------------------------------------------------------ binary


def sum_to(g, shape):
    """Sums a broadcast gradient back to `shape` over every broadcast dim
    (the contract; torch.js reduces only 1-D vs 2-D, Tensor.ts:3560-3591)."""
    g = np.asarray(g, dtype=F64)
    shape = tuple(shape)
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    for d, s in enumerate(shape):
        if s == 1 and g.shape[d] != 1:
            g = g.sum(axis=d, keepdims=True)
    return g.reshape(shape)


def binary(op, a, b):
    """_binaryOp / _broadcastBinaryOp forward (Tensor.ts:3409-3514)."""
    a = np.asarray(a, dtype=F64)
    b = np.asarray(b, dtype=F64)
    with np.errstate(all="ignore"):
        if op == "add": return a + b
        if op == "sub": return a - b
        if op == "mul": return a * b
        if op == "div": return a / b
        if op == "pow": return np.power(a, b)
        if op == "maximum": return np.maximum(a, b)
        if op == "minimum": return np.minimum(a, b)
    raise ValueError(op)


def binary_backward(op, g, a, b):
    """(dL/da, dL/db) reduced to each operand's shape (fixes D3/D4)."""
    g = np.asarray(g, dtype=F64)
    a = np.asarray(a, dtype=F64)
    b = np.asarray(b, dtype=F64)
    with np.errstate(all="ignore"):
        if op == "add": ga, gb = g, g
        elif op == "sub": ga, gb = g, -g
        elif op == "mul": ga, gb = g * b, g * a
        elif op == "div": ga, gb = g / b, -g * a / (b * b)
        elif op == "pow": ga, gb = g * b * np.power(a, b - 1), g * np.power(a, b) * np.log(a)
        elif op in ("maximum", "minimum"):
            # the selected operand takes g; a tie gives each operand g / 2
            # (PyTorch's rule for torch.maximum / torch.minimum)
            wa = np.where(a == b, 0.5, np.where(a > b, 1.0, 0.0) if op == "maximum"
                          else np.where(a < b, 1.0, 0.0))
            ga, gb = g * wa, g * (1.0 - wa)
        else: raise ValueError(op)
    return sum_to(ga, a.shape), sum_to(gb, b.shape)


def pow_scalar(x, e):
    """pow by repeated multiplication for integer exponents 0..10, else pow
    (scalar.wgsl:53-66)."""
    x = np.asarray(x, dtype=F64)
    r = round(e)
    if abs(e - r) < 1e-6 and 0 <= r <= 10:
        out = np.ones_like(x)
        for _ in range(int(r)):
            out = out * x
        return out
    with np.errstate(all="ignore"):
        return np.power(x, e)


# ------------------------------------------------------------------ reductions


def reduce(op, x, dims=None, keepdim=False):
    """sum / mean / max / min / prod over dims (Tensor.ts:2359-2436,
    reduce_dim.wgsl:1-63)."""
    x = np.asarray(x, dtype=F64)
    ax = None if dims is None else tuple(dims)
    f = {"sum": np.sum, "mean": np.mean, "max": np.max, "min": np.min, "prod": np.prod}[op]
    return f(x, axis=ax, keepdims=keepdim)


def reduce_backward(op, g, shape, dims=None, keepdim=False):
    """Gradient of sum / mean over `dims`: g with the reduced dims restored
    as size 1, broadcast to `shape`, divided by the reduced count for mean
    (the contract; torch.js expands without restoring them, D13,
    Tensor.ts:2416-2424)."""
    shape = tuple(shape)
    dims = tuple(range(len(shape))) if dims is None else tuple(d % len(shape) for d in dims)
    g = np.asarray(g, dtype=F64)
    if not keepdim:
        for d in sorted(dims):
            g = np.expand_dims(g, d)
    out = np.broadcast_to(g, shape).astype(F64)
    if op == "mean":
        out = out / int(np.prod([shape[d] for d in dims]))
    elif op != "sum":
        raise ValueError(op)
    return out


def argmax(x, dim=None, is_min=False):
    """First index of the max (min) — Tensor.ts:2568 keeps the first on ties
    (`val > maxVal`)."""
    x = np.asarray(x, dtype=F64)
    f = np.argmin if is_min else np.argmax  # numpy also returns the first
    if dim is None:
        return np.int32(f(x.reshape(-1)))
    return f(x, axis=dim).astype(np.int32)


# ------------------------------------------------------------------ softmax


def log_softmax(x):
    """x - max - log(sum exp(x - max)) over the last dim
    (log_softmax.wgsl:8-36)."""
    x = np.asarray(x, dtype=F64)
    m = x.max(axis=-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))


def softmax(x):
    return np.exp(log_softmax(x))


def softmax_backward(g, y):
    """y * (g - sum(g * y)) over the last dim."""
    g = np.asarray(g, dtype=F64)
    return y * (g - (g * y).sum(axis=-1, keepdims=True))


def log_softmax_backward(g, y):
    """g - softmax * sum(g) (log_softmax_backward.wgsl:17-34)."""
    g = np.asarray(g, dtype=F64)
    return g - np.exp(y) * g.sum(axis=-1, keepdims=True)


# ------------------------------------------------------------------ losses


def _valid(t, cols, ignore_index):
    t = np.asarray(t, dtype=np.int64)
    return (t != ignore_index) & (t >= 0) & (t < cols)


def _denominator(reduction, ok, wt):
    """Divisor of the reduction (apply_reduction, losses.ts:18-32): mean ->
    sum of the valid rows' target weights (their count without weights,
    PyTorch's weighted mean), batchmean -> rows, sum / none -> 1."""
    if reduction == "mean":
        return np.where(ok, wt, 0.0).sum()
    if reduction == "batchmean":
        return float(len(ok))
    return 1.0


def _reduce_rows(rows, reduction, ok, wt):
    if reduction == "none":
        return rows
    return rows.sum() / _denominator(reduction, ok, wt)


def _row_scale(g, reduction, ok, wt):
    g = np.asarray(g, dtype=F64)
    if reduction == "none":
        sc = g.reshape(-1) * np.ones(len(ok))
    else:
        sc = np.full(len(ok), float(g) / _denominator(reduction, ok, wt))
    return np.where(ok, sc, 0.0)


def _class_weights(weight, cols):
    return np.ones(cols) if weight is None else np.asarray(weight, dtype=F64)


def cross_entropy(x, t, reduction="mean", ignore_index=-100, weight=None, label_smoothing=0.0):
    """F.cross_entropy (src/nn/losses.ts:129-168 = nll_loss(log_softmax),
    losses.ts:63-94) under PyTorch's contract: for a valid row with target
    t and smoothing eps, loss = (1-eps) w_t (-logp_t) + (eps/C) sum_c w_c
    (-logp_c); 'mean' divides by the sum of the valid rows' target weights
    (the row count without weights), 'batchmean' by the row count."""
    x = np.asarray(x, dtype=F64)
    t = np.asarray(t, dtype=np.int64)
    C = x.shape[1]
    ok = _valid(t, C, ignore_index)
    w = _class_weights(weight, C)
    ts = np.where(ok, t, 0)
    wt = w[ts]
    lp = log_softmax(x)
    eps = float(label_smoothing)
    rows = (1.0 - eps) * wt * -lp[np.arange(len(t)), ts]
    if eps != 0.0:  # (without smoothing a -inf logit's term is absent, not 0 * inf)
        rows = rows + (eps / C) * (-(lp * w)).sum(axis=1)
    rows = np.where(ok, rows, 0.0)
    return _reduce_rows(rows, reduction, ok, wt)


def cross_entropy_backward(x, t, g=1.0, reduction="mean", ignore_index=-100, weight=None,
                           label_smoothing=0.0):
    """d loss / d x of cross_entropy: row scale s times
    ((1-eps) w_t (p - onehot_t) + (eps/C) (W p - w)), W = sum_c w_c; the
    plain case is (softmax - onehot) * s (nll_loss_backward.wgsl + the
    log_softmax VJP)."""
    x = np.asarray(x, dtype=F64)
    t = np.asarray(t, dtype=np.int64)
    C = x.shape[1]
    ok = _valid(t, C, ignore_index)
    w = _class_weights(weight, C)
    ts = np.where(ok, t, 0)
    wt = w[ts]
    eps = float(label_smoothing)
    p = softmax(x)
    oh = np.zeros_like(p)
    oh[np.arange(len(t)), ts] = 1.0
    d = (1.0 - eps) * wt[:, None] * (p - oh) + (eps / C) * (w.sum() * p - w[None, :])
    return d * _row_scale(g, reduction, ok, wt)[:, None]


def nll_loss(lp, t, reduction="mean", ignore_index=-100, weight=None):
    """F.nll_loss (losses.ts:63-94): -w_t logp[i, t] per valid row."""
    lp = np.asarray(lp, dtype=F64)
    t = np.asarray(t, dtype=np.int64)
    ok = _valid(t, lp.shape[1], ignore_index)
    ts = np.where(ok, t, 0)
    wt = _class_weights(weight, lp.shape[1])[ts]
    rows = np.where(ok, -wt * lp[np.arange(len(t)), ts], 0.0)
    return _reduce_rows(rows, reduction, ok, wt)


def nll_loss_backward(lp_shape, t, g=1.0, reduction="mean", ignore_index=-100, weight=None):
    t = np.asarray(t, dtype=np.int64)
    ok = _valid(t, lp_shape[1], ignore_index)
    ts = np.where(ok, t, 0)
    wt = _class_weights(weight, lp_shape[1])[ts]
    d = np.zeros(lp_shape)
    sc = _row_scale(g, reduction, ok, wt)
    d[np.arange(len(t))[ok], t[ok]] = -(wt * sc)[ok]
    return d


# ------------------------------------------------------------------ layer norm


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    """gamma * (x - mean) / sqrt(biased var + eps) + beta over the last dim
    (layernorm.wgsl:14-42).  Returns (y, mean, rstd)."""
    x = np.asarray(x, dtype=F64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (x - mean) * rstd
    if gamma is not None:
        y = y * gamma
    if beta is not None:
        y = y + beta
    return y, mean[..., 0], rstd[..., 0]


def layer_norm_backward(g, x, gamma=None, eps=1e-5):
    """(dx, dgamma, dbeta): dx = rstd (g*gamma - mean(g*gamma)
    - xhat mean(g*gamma*xhat)); dgamma = sum g*xhat; dbeta = sum g."""
    g = np.asarray(g, dtype=F64)
    x = np.asarray(x, dtype=F64)
    _, mean, rstd = layer_norm(x, eps=eps)
    xh = (x - mean[..., None]) * rstd[..., None]
    gg = g * (gamma if gamma is not None else 1.0)
    dx = rstd[..., None] * (gg - gg.mean(axis=-1, keepdims=True)
                            - xh * (gg * xh).mean(axis=-1, keepdims=True))
    red = tuple(range(x.ndim - 1))
    return dx, (g * xh).sum(axis=red), g.sum(axis=red)


# ------------------------------------------------------------------ embedding / indexing


def embedding(w, ids):
    """out[i] = W[clamp(ids[i], 0, V-1)] (embedding.wgsl:13-27)."""
    w = np.asarray(w, dtype=F64)
    ids = np.clip(np.asarray(ids, dtype=np.int64), 0, w.shape[0] - 1)
    return w[ids]


def embedding_backward(g, ids, num):
    """dW[v] = sum of g rows whose (clamped) id is v, in increasing order."""
    g = np.asarray(g, dtype=F64)
    D = g.shape[-1]
    ids = np.clip(np.asarray(ids, dtype=np.int64).reshape(-1), 0, num - 1)
    g2 = g.reshape(-1, D)
    dw = np.zeros((num, D))
    if ids.size:
        order = np.argsort(ids, kind="stable")
        sid = ids[order]
        starts = np.flatnonzero(np.r_[True, sid[1:] != sid[:-1]])
        dw[sid[starts]] = np.add.reduceat(g2[order], starts, axis=0)
    return dw


def _check_index_range(idx, n):
    """index_select's contract is PyTorch's (the @pytorch tag of
    Tensor.ts:1242): every index in [0, n), else IndexError.  torch.js's
    index_select.wgsl:32-52 casts the i32 index to u32, so a negative one
    reads out of bounds there; no wrap is defined."""
    if idx.size and (idx.min() < 0 or idx.max() >= n):
        raise IndexError("index_select: index out of range for dimension of size %d" % n)


def index_select(x, dim, idx):
    """x.index_select(dim, idx) (Tensor.ts:1242-1287, index_select.wgsl:20-55)."""
    x = np.asarray(x, dtype=F64)
    idx = np.asarray(idx, dtype=np.int64)
    _check_index_range(idx, x.shape[dim])
    return np.take(x, idx, axis=dim)


def index_select_backward(g, shape, dim, idx):
    """index_add of g into zeros: repeated indices sum."""
    idx = np.asarray(idx, dtype=np.int64)
    _check_index_range(idx, shape[dim])
    out = np.zeros(shape)
    gm = np.moveaxis(np.asarray(g, dtype=F64), dim, 0)
    om = np.moveaxis(out, dim, 0)
    np.add.at(om, idx, gm)
    return out


def gather(x, dim, idx):
    """gather with negative-index wrap (Tensor.ts:2686-2687)."""
    x = np.asarray(x, dtype=F64)
    idx = np.asarray(idx, dtype=np.int64)
    idx = np.where(idx < 0, idx + x.shape[dim], idx)
    return np.take_along_axis(x, idx, axis=dim)


def scatter_add(shape, dim, idx, src):
    idx = np.asarray(idx, dtype=np.int64)
    idx = np.where(idx < 0, idx + shape[dim], idx)
    out = np.zeros(shape)
    it = np.indices(idx.shape)
    coords = [it[d] if d != dim else idx for d in range(len(shape))]
    np.add.at(out, tuple(coords), np.asarray(src, dtype=F64))
    return out


def one_hot(x, num_classes=-1):
    """F.one_hot (src/nn/functional.ts:764-796): Math.round (ties toward
    +inf), values outside [0, C) leave the row zero; C = floor(max)+1 when
    not given."""
    x = np.asarray(x, dtype=F64).reshape(-1) if np.ndim(x) else np.asarray([x], dtype=F64)
    if num_classes <= 0:
        num_classes = max(1, int(math.floor(x.max())) + 1)
    r = np.floor(x + 0.5).astype(np.int64)
    out = np.zeros((len(x), num_classes))
    ok = (r >= 0) & (r < num_classes)
    out[np.arange(len(x))[ok], r[ok]] = 1.0
    return out


def nonzero(x):
    """Row-major coordinates of the non-zero elements (Tensor.ts:1323-1345)."""
    return np.argwhere(np.asarray(x) != 0).astype(np.int32)


# ------------------------------------------------------------------ linear / matmul


def linear(x, w, b=None):
    """x W^T + b (src/nn/linear.ts:43-66)."""
    y = np.asarray(x, dtype=F64) @ np.asarray(w, dtype=F64).T
    return y + b if b is not None else y


def linear_backward(g, x, w):
    """(dx, dW, db) = (g W, g^T x, sum_rows g) over flattened leading dims."""
    g = np.asarray(g, dtype=F64)
    x = np.asarray(x, dtype=F64)
    w = np.asarray(w, dtype=F64)
    g2 = g.reshape(-1, g.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    return (g @ w), g2.T @ x2, g2.sum(axis=0)


def matmul_backward(g, a, b):
    """(g B^T, A^T g) with batch broadcasting summed back (fixes D1)."""
    g = np.asarray(g, dtype=F64)
    a = np.asarray(a, dtype=F64)
    b = np.asarray(b, dtype=F64)
    ga = g @ np.swapaxes(b, -1, -2)
    gb = np.swapaxes(a, -1, -2) @ g
    return sum_to(ga, a.shape), sum_to(gb, b.shape)


# ------------------------------------------------------------------ attention


def _scores(q, k, causal, scale, mask):
    D = q.shape[-1]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    s = (q @ np.swapaxes(k, -1, -2)) * sc
    if causal:
        Tq, Tk = s.shape[-2], s.shape[-1]
        s = np.where(np.triu(np.ones((Tq, Tk), dtype=bool), 1), -np.inf, s)
    if mask is not None:
        s = s + np.asarray(mask, dtype=F64)  # additive, broadcast; -inf masks out
    return s, sc


def sdpa(q, k, v, causal=False, scale=None, mask=None):
    """softmax(Q K^T scale [+ causal mask] [+ mask]) V
    (src/nn/functional.ts:866-890 with torch's is_causal: key j > query i
    is masked; `mask` is an additive float mask).  Returns (o, lse)."""
    q = np.asarray(q, dtype=F64)
    k = np.asarray(k, dtype=F64)
    v = np.asarray(v, dtype=F64)
    s, _ = _scores(q, k, causal, scale, mask)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    ssum = e.sum(axis=-1, keepdims=True)
    p = e / ssum
    return p @ v, (m + np.log(ssum))[..., 0]


def sdpa_weights(q, k, causal=False, scale=None, mask=None):
    """The attention weights softmax(Q K^T scale [+ masks]) of sdpa."""
    s, _ = _scores(np.asarray(q, dtype=F64), np.asarray(k, dtype=F64), causal, scale, mask)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return p / p.sum(axis=-1, keepdims=True)


def sdpa_backward(g, q, k, v, causal=False, scale=None, mask=None):
    """(dq, dk, dv) of sdpa."""
    g = np.asarray(g, dtype=F64)
    q = np.asarray(q, dtype=F64)
    k = np.asarray(k, dtype=F64)
    v = np.asarray(v, dtype=F64)
    s, sc = _scores(q, k, causal, scale, mask)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    dv = np.swapaxes(p, -1, -2) @ g
    dp = g @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True)) * sc
    return ds @ k, np.swapaxes(ds, -1, -2) @ q, dv


# ------------------------------------------------------------------ conv2d


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def conv2d(x, w, b=None, stride=1, padding=0, dilation=1, groups=1):
    """NCHW cross-correlation (src/nn/functional.ts:438-660, conv.wgsl:25-60)
    with torch's stride / padding / dilation / groups."""
    x = np.asarray(x, dtype=F64)
    w = np.asarray(w, dtype=F64)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    N, C, H, W = x.shape
    OC, CG, KH, KW = w.shape
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    y = np.zeros((N, OC, OH, OW))
    ocg = OC // groups
    for gi in range(groups):
        xs = xp[:, gi * CG:(gi + 1) * CG]
        ws = w[gi * ocg:(gi + 1) * ocg]
        for i in range(KH):
            for j in range(KW):
                patch = xs[:, :, i * dh: i * dh + sh * (OH - 1) + 1: sh,
                           j * dw: j * dw + sw * (OW - 1) + 1: sw]
                y[:, gi * ocg:(gi + 1) * ocg] += np.einsum("nchw,oc->nohw", patch, ws[:, :, i, j])
    if b is not None:
        y += np.asarray(b, dtype=F64)[None, :, None, None]
    return y


def conv2d_backward(g, x, w, stride=1, padding=0, dilation=1, groups=1):
    """(dx, dw, db) of conv2d."""
    g = np.asarray(g, dtype=F64)
    x = np.asarray(x, dtype=F64)
    w = np.asarray(w, dtype=F64)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw_ = _pair(dilation)
    N, C, H, W = x.shape
    OC, CG, KH, KW = w.shape
    OH, OW = g.shape[2], g.shape[3]
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    dxp = np.zeros_like(xp)
    dwt = np.zeros_like(w)
    ocg = OC // groups
    for gi in range(groups):
        cs = slice(gi * CG, (gi + 1) * CG)
        os_ = slice(gi * ocg, (gi + 1) * ocg)
        for i in range(KH):
            for j in range(KW):
                sl = (slice(None), cs, slice(i * dh, i * dh + sh * (OH - 1) + 1, sh),
                      slice(j * dw_, j * dw_ + sw * (OW - 1) + 1, sw))
                dwt[os_, :, i, j] += np.einsum("nohw,nchw->oc", g[:, os_], xp[sl])
                dxp[sl] += np.einsum("nohw,oc->nchw", g[:, os_], w[os_, :, i, j])
    dx = dxp[:, :, ph:ph + H, pw:pw + W]
    return dx, dwt, g.sum(axis=(0, 2, 3))


# ------------------------------------------------------------------ optimizers


def adam_step(p, g, m, v, step, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
              decoupled=False):
    """One Adam (decoupled=False, src/optim/adam.ts:46-133) or AdamW
    (src/optim/adamw.ts:46-154) step on float32 arrays, rounding like the
    reference: the moments and the denominator are float32 tensor ops there
    (adam.ts:82-96: mul(beta1).add(grad.mul(1-beta1)), pow(2) by repeated
    multiply, div(bc2).sqrt().add(eps)), the parameter update is its JS
    float64 loop (adam.ts:104-120, adamw.ts:114-133) rounded once.
    Returns new (p, m, v) as float32."""
    b1, b2 = betas
    p = np.asarray(p, dtype=F32)
    g = np.asarray(g, dtype=F32)
    m = np.asarray(m, dtype=F32)
    v = np.asarray(v, dtype=F32)
    # float32 arithmetic on float32 arrays rounds every operation to float32
    if not decoupled and weight_decay != 0:
        g = g + p * F32(weight_decay)
    m = m * F32(b1)
    m += g * F32(1.0 - b1)
    g2 = g * g
    g2 *= F32(1.0 - b2)
    v = v * F32(b2)
    v += g2
    bc1 = 1.0 - b1 ** step
    bc2 = 1.0 - b2 ** step
    denom = v / F32(bc2)
    np.sqrt(denom, out=denom)
    denom += F32(eps)
    upd = m.astype(F64)
    upd /= denom
    upd *= lr / bc1
    pd = p.astype(F64)
    if decoupled:
        pd *= 1.0 - lr * weight_decay
    pd -= upd
    return pd.astype(F32), m, v


# ------------------------------------------------------------------ sampling


def multinomial(x, num_samples, replacement, u):
    """Tensor.multinomial (src/tensor/Tensor.ts:271-359) given the draws
    u[row, s] in [0, 1): weights p = max(0, x) (Tensor.ts:316; negative
    weights and -inf weigh 0), uniform when their sum is not positive
    (Tensor.ts:319-322).  With replacement, the first index whose running
    sum of p / sum exceeds u (the last index when none does,
    Tensor.ts:343-353).  Without replacement, each draw picks the first
    untaken index whose running sum of p exceeds u times the untaken mass:
    the distribution of the reference's redraw-until-new loop
    (Tensor.ts:327-341), one draw per sample.  Float64 running sums, in
    index order.

    Two cases the reference leaves undefined get a stated contract:
    - a row holding NaN or +inf raises ValueError (PyTorch raises; in the
      reference Math.max(0, NaN) is NaN, every cumulative probability is
      NaN, and the draws fall to the last index with replacement or loop
      forever without it);
    - without replacement, once every positive-weight category is taken,
      each further draw takes the last untaken index (the reference falls
      back to index 0 and redraws until it finds a new one, which never
      ends when 0 is taken; PyTorch raises)."""
    x = np.asarray(x, dtype=F64)
    one = x.ndim == 1
    x = np.atleast_2d(x)
    u = np.asarray(u, dtype=F64).reshape(x.shape[0], num_samples)
    rows, C = x.shape
    bad = np.isnan(x) | (x == np.inf)
    if bad.any():
        raise ValueError("multinomial: probability row %d contains NaN or inf"
                         % int(np.flatnonzero(bad.any(axis=1))[0]))
    out = np.zeros((rows, num_samples), dtype=np.int32)
    for r in range(rows):
        p = np.where(x[r] > 0, x[r], 0.0)
        total = p.sum()
        if not total > 0:
            p = np.ones(C)
            total = float(C)
        taken = np.zeros(C, dtype=bool)
        for s in range(num_samples):
            if replacement:
                c, idx = 0.0, C - 1
                for i in range(C):
                    c += p[i] / total
                    if u[r, s] < c:
                        idx = i
                        break
            else:
                mass = 0.0
                for i in range(C):
                    if not taken[i]:
                        mass += p[i]
                target = u[r, s] * mass
                c, idx = 0.0, -1
                for i in range(C):
                    if taken[i] or p[i] <= 0:
                        continue
                    c += p[i]
                    if target < c:
                        idx = i
                        break
                if idx < 0:
                    idx = int(np.flatnonzero(~taken)[-1])
                taken[idx] = True
            out[r, s] = idx
    return out[0] if one else out

