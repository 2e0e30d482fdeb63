"""torch.nn.functional for the 'hip' device (src/nn/functional.ts,
src/nn/losses.ts): the hot-path ops as fused kernels with their
backward passes.
"""
import ctypes
import math

import numpy as np

from . import _lib as L
from . import tensor as _T
from .tensor import _e_unary_bwd
from .tensor import (Tensor, _DT, _alias, _contig_strides, _empty_padded, _gemm, _k_binary,
                     _k_contiguous, _k_reduce, _k_scalar, _numel, _record, _view_raw, _wrap_dim,
                     contiguous, empty, full, mul, permute, reduce_mean, reshape, reshape_raw,
                     neg, sub, unary, zeros)


def relu(x, inplace=False):
    return unary("relu", x)


def gelu(x, approximate="none"):
    """Exact GELU with the A&S 7.1.26 erf of unary.wgsl:230-252."""
    if approximate != "none":
        raise NotImplementedError("only the exact (erf) GELU is implemented")
    return unary("gelu", x)


def sigmoid(x):
    return unary("sigmoid", x)


def tanh(x):
    return unary("tanh", x)


def silu(x):
    return unary("silu", x)


def softplus(x):
    return unary("softplus", x)


def leaky_relu(x, negative_slope=0.01):
    return unary("leaky_relu", x, negative_slope)


def elu(x, alpha=1.0):
    return unary("elu", x, alpha)


# ------------------------------------------------------------ softmax


def _rows_view(x):
    """(ptr, ld) when x is a 2-D row-major view with unit column stride."""
    if x.ndim == 2 and (x._strides[1] == 1 or x.shape[1] <= 1) and x._strides[0] >= x.shape[1]:
        return x.data_ptr(), max(x._strides[0], 1)
    return None


def _softmax_impl(x, dim, log):
    if x.dtype != "float32":
        x = x.float()
    nd = x.ndim
    d = _wrap_dim(dim, nd) if nd else 0
    if nd == 0:
        x1 = reshape(x, (1,))
        out = _softmax_impl(x1, 0, log)
        return reshape(out, ())
    if d != nd - 1:
        perm = list(range(nd))
        perm[d], perm[-1] = perm[-1], perm[d]
        y = _softmax_impl(permute(x, perm), -1, log)
        return permute(y, perm)
    xc = contiguous(x.detach())
    cols = x.shape[-1]
    rows = _numel(x.shape[:-1])
    out = empty(x.shape)
    L.check(L.lib().tjh_softmax_forward(xc.data_ptr(), cols, out.data_ptr(), cols, rows, cols,
                                        1 if log else 0), "softmax")
    y = out.detach()

    def bwd(g):
        g = g.contiguous()
        dx = empty(g.shape)
        L.check(L.lib().tjh_softmax_backward(g.data_ptr(), y.data_ptr(), dx.data_ptr(), rows, cols,
                                             1 if log else 0), "softmax_backward")
        return [dx]

    def gbwd(g):  # recording ops, softmax recomputed from x
        p = _softmax_impl(x, -1, False)
        if log:
            return [_T.sub(g, _T.mul(p, _T.reduce_sum(g, -1, keepdim=True)))]
        return [_T.mul(p, _T.sub(g, _T.reduce_sum(_T.mul(g, p), -1, keepdim=True)))]
    return _record(out, "LogSoftmax" if log else "Softmax", [x], bwd, gfn=gbwd)


def softmax(x, dim=-1):
    """F.softmax (src/nn/functional.ts:79-135): max-subtracted; backward
    y*(g - sum(g*y)) (torch.js records none, D6)."""
    return _softmax_impl(x, dim, False)


def log_softmax(x, dim=-1):
    """F.log_softmax (src/nn/functional.ts:137-234, log_softmax.wgsl:8-36);
    backward g - softmax*sum(g) (log_softmax_backward.wgsl:17-34)."""
    return _softmax_impl(x, dim, True)


# ------------------------------------------------------------ losses

_RED = {"none": 0, "mean": 1, "sum": 2, "batchmean": 3}


def _reduction_code(reduction):
    if reduction not in _RED:
        raise ValueError("%s is not a valid value for reduction" % (reduction,))
    return _RED[reduction]


def _class_last_2d(x, target):
    """[N, C] or [N, C, d1, ...] -> ([rows, C] view, flat int32 targets)."""
    if x.ndim == 1:
        x = reshape(x, (1, x.shape[0]))
    if x.ndim > 2:
        perm = [0] + list(range(2, x.ndim)) + [1]
        x = reshape(permute(x, perm), (-1, x.shape[1]))
    t = target
    if not isinstance(t, Tensor):
        from .tensor import tensor as _tensor
        t = _tensor(np.asarray(t, dtype=np.int32), dtype="int32")
    if t.dtype != "int32":
        t = t.to("int32")
    t = contiguous(reshape(t, (-1,)))
    if t.numel() != x.shape[0]:
        raise ValueError("cross_entropy: %d targets for %d rows" % (t.numel(), x.shape[0]))
    return x, t


def _class_weight(weight, cols):
    """Class weights as a contiguous float32 [C] tensor (no gradient flows to
    them, as in PyTorch), or None."""
    if weight is None:
        return None
    if not isinstance(weight, Tensor):
        from .tensor import tensor as _tensor
        weight = _tensor(np.asarray(weight, dtype=np.float32))
    w = weight.detach()
    w = w.float() if w.dtype != "float32" else w
    if w.shape != (cols,):
        raise ValueError("weight should be a 1-D tensor of %d class weights, got shape %s"
                         % (cols, list(w.shape)))
    return w.contiguous()


def _class_coef(t, w, rows, cols, eps, ignore_index, smooth):
    """The constant [rows, cols] coefficients Q with loss_i = -sum_c Q[i, c]
    * logp[i, c] for the losses below: (1 - eps) w_t at the target and
    (eps / C) w_c everywhere when `smooth`, rows whose target is
    ignore_index zero; and the 'mean' divisor, the valid rows' target
    weights summed (computed without recording: no gradient flows to them,
    as in PyTorch)."""
    valid = _T.compare_raw(t.float(), float(ignore_index), "ne")       # [rows]
    oh = one_hot(t, cols)               # a target outside [0, C) gives a zero row
    wt = valid if w is None else _k_binary("mul", valid, _T.index_select(
        w, 0, _k_binary("mul", t.float(), valid).to("int32")))
    q = _k_binary("mul", oh, reshape_raw(_k_scalar("mul", wt, 1.0 - eps), (rows, 1)))
    if smooth and eps:
        wc = full((1, cols), eps / cols) if w is None else \
            reshape_raw(_k_scalar("mul", w, eps / cols), (1, cols))
        q = _k_binary("add", q, _k_binary("mul", wc, reshape_raw(valid, (rows, 1))))
    den = float(_k_reduce("sum", wt, [0]).numpy().reshape(-1)[0])
    return q, den


def _class_loss(logp, q, den, red, rows):
    """-sum_c q * logp per row, reduced as `red` (0 none, 1 mean over den,
    2 sum, 3 sum / rows), with recording ops."""
    per = neg(_T.reduce_sum(mul(logp, q), 1))
    if red == 0:
        return per
    tot = _T.reduce_sum(per)
    if red == 1:
        return mul(tot, 1.0 / den)
    if red == 3:
        return mul(tot, 1.0 / rows)
    return tot


def cross_entropy(input, target, weight=None, reduction="mean", label_smoothing=0.0, *,
                  ignore_index=-100):
    """F.cross_entropy(input, target, weight, reduction, label_smoothing)
    (src/nn/losses.ts:129-168; the positional order is torch.js's) =
    nll_loss(log_softmax) fused: one pass computes logsumexp and the per-row
    loss, the backward writes the logits' gradient in one pass (torch.js's
    nll_loss reinterprets int targets as floats, D9).  Class weights,
    label smoothing and the 'mean' over weights follow PyTorch's contract,
    which torch.js's @pytorch tag declares: loss_i = (1-eps) w_t (-logp_t)
    + (eps/C) sum_c w_c (-logp_c), and 'mean' divides by the sum of the
    valid rows' target weights (torch.js averages over rows).  'batchmean'
    (losses.ts:27-28) divides the sum by the number of rows.
    `ignore_index` (PyTorch's; torch.js has none) is keyword-only."""
    red = _reduction_code(reduction)
    eps = float(label_smoothing)
    if not 0.0 <= eps <= 1.0:
        raise ValueError("label_smoothing must lie in [0, 1], got %r" % (label_smoothing,))
    x, t = _class_last_2d(input, target)
    if x.dtype != "float32":
        x = x.float()
    rv = _rows_view(x)
    xd = x.detach()
    if rv is None:
        xd = _k_contiguous(xd)
        rv = _rows_view(xd)
    rows, cols = x.shape
    w = _class_weight(weight, cols)
    wp = w.data_ptr() if w is not None else None
    lse = empty((rows,))
    loss_rows = empty((rows,))
    out = empty(()) if red else loss_rows
    # The logits' gradient for the unit seed of loss.backward(), formed in
    # the forward's pass over the logits (read once instead of twice) when
    # the loss is a scalar that will be differentiated; another upstream
    # gradient takes the backward kernel below.
    pre, me = [None], [None]
    if (red and w is None and eps == 0.0 and not _T._FUSE_CE and cols > 2048
            and _T._grad["enabled"] and x.requires_grad):
        d = _empty_padded(rows, cols) if cols % 4 else empty((rows, cols))
        L.check(L.lib().tjh_cross_entropy_forward_grad(rv[0], rv[1], t.data_ptr(), rows, cols,
                                                       int(ignore_index), lse.data_ptr(),
                                                       loss_rows.data_ptr(), red,
                                                       out.data_ptr(), d.data_ptr(),
                                                       d._strides[0]),
                "cross_entropy")
        pre[0] = d
    else:
        L.check(L.lib().tjh_cross_entropy_forward(rv[0], rv[1], t.data_ptr(), rows, cols,
                                                  int(ignore_index), wp, eps, lse.data_ptr(),
                                                  loss_rows.data_ptr(), red,
                                                  out.data_ptr() if red else None),
                "cross_entropy")

    def bwd(g):
        d0, pre[0] = pre[0], None  # handed out once (the engine may own it)
        if d0 is not None and g is _T._unit_seed["g"] and me[0] == _T._unit_seed["node"]:
            return [d0]
        g = g.contiguous()
        xp, ld = _rows_view(xd)
        if w is None and eps == 0.0 and _T._FUSE_CE and ld % 4 == 0 and xp % 16 == 0:
            # left unformed: a Linear that produced x forms it in its GEMMs
            return [_T._CEGrad((rows, cols), xd, t, lse, g, int(ignore_index), red)]
        d = _empty_padded(rows, cols) if cols % 4 else empty((rows, cols))
        wb = w.data_ptr() if w is not None else None  # keeps w alive with the graph
        L.check(L.lib().tjh_cross_entropy_backward(xp, ld, t.data_ptr(), wb, eps, lse.data_ptr(),
                                                   g.data_ptr(), rows, cols, int(ignore_index),
                                                   red, d.data_ptr(), d._strides[0], 0),
                "cross_entropy_backward")
        return [d]
    def gbwd(g):  # from log_softmax and the constant coefficients, recorded
        q, den = _class_coef(t, w, rows, cols, eps, ignore_index, True)
        return _T._regrad(lambda xx: _class_loss(log_softmax(xx, 1), q, den, red, rows), [x], g)
    res = _record(out, "CrossEntropy", [x], bwd, gfn=gbwd)
    me[0] = id(res.grad_fn) if res.grad_fn is not None else None
    if pre[0] is not None and res.grad_fn is None:
        pre[0] = None
    if x is not input and input.ndim == 1 and red == 0:
        res = reshape(res, ())
    return res


def nll_loss(input, target, weight=None, reduction="mean", *, ignore_index=-100):
    """F.nll_loss(input, target, weight, reduction) (src/nn/losses.ts:63-94,
    nll_loss(_backward).wgsl): loss_i = -w_t logp[i, t]; 'mean' divides by
    the sum of the valid rows' target weights (PyTorch's contract)."""
    red = _reduction_code(reduction)
    x, t = _class_last_2d(input, target)
    if x.dtype != "float32":
        x = x.float()
    xd = x.detach()
    rv = _rows_view(xd)
    if rv is None:
        xd = _k_contiguous(xd)
        rv = _rows_view(xd)
    rows, cols = x.shape
    w = _class_weight(weight, cols)
    wp = w.data_ptr() if w is not None else None
    loss_rows = empty((rows,))
    out = empty(()) if red else loss_rows
    L.check(L.lib().tjh_nll_loss_forward(rv[0], rv[1], t.data_ptr(), rows, cols, int(ignore_index),
                                         wp, loss_rows.data_ptr(), red,
                                         out.data_ptr() if red else None), "nll_loss")

    def bwd(g):
        g = g.contiguous()
        d = empty((rows, cols))
        wb = w.data_ptr() if w is not None else None  # keeps w alive with the graph
        L.check(L.lib().tjh_nll_loss_backward(t.data_ptr(), wb, g.data_ptr(), rows, cols,
                                              int(ignore_index), red, d.data_ptr()),
                "nll_loss_backward")
        return [d]
    def gbwd(g):
        q, den = _class_coef(t, w, rows, cols, 0.0, ignore_index, False)
        return _T._regrad(lambda xx: _class_loss(xx, q, den, red, rows), [x], g)
    return _record(out, "NLLLoss", [x], bwd, gfn=gbwd)


def mse_loss(input, target, reduction="mean"):
    """F.mse_loss (src/nn/losses.ts): mean((input - target)^2)."""
    d = sub(input, target)
    sq = d.pow(2)
    if reduction == "mean":
        return reduce_mean(sq)
    if reduction == "sum":
        return sq.sum()
    return sq


# ------------------------------------------------------------ normalisation


_LN_DEFER = 2  # TJH_LN_DEFER


def layer_norm(x, normalized_shape, weight=None, bias=None, eps=1e-5):
    """nn.LayerNorm forward (layernorm.wgsl:14-42: biased variance, eps
    inside the sqrt) and backward dx, dgamma, dbeta (torch.js has none, D10)."""
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    normalized_shape = tuple(normalized_shape)
    k = len(normalized_shape)
    if x.shape[x.ndim - k:] != normalized_shape:
        raise RuntimeError("layer_norm: input shape %s does not end with %s"
                           % (list(x.shape), list(normalized_shape)))
    cols = _numel(normalized_shape)
    rows = x.numel() // max(cols, 1)
    xc = contiguous(x.detach()) if x.dtype == "float32" else x.float().detach().contiguous()
    w = weight.detach().contiguous() if weight is not None else None
    b = bias.detach().contiguous() if bias is not None else None
    y = empty(x.shape)
    mean = empty((rows,))
    rstd = empty((rows,))
    L.check(L.lib().tjh_layer_norm_forward(xc.data_ptr(), w.data_ptr() if w is not None else None,
                                           b.data_ptr() if b is not None else None, y.data_ptr(),
                                           mean.data_ptr(), rstd.data_ptr(), rows, cols,
                                           float(eps)), "layer_norm")
    rx = x.requires_grad
    rw = weight is not None and weight.requires_grad
    rb = bias is not None and bias.requires_grad

    def bwd(g, pending=None, defer=False):
        # pending: a gradient already accumulated for x (the residual
        # stream's identity path), added to dx by the same kernel.  defer:
        # the engine will call tjh_flush_deferred before anything reads dw
        # / db, so their finishing pass may wait and run batched
        g = g.contiguous()
        dx = empty(x.shape) if rx else None
        dw = empty(normalized_shape) if rw else None
        db = empty(normalized_shape) if rb else None
        args = (g.data_ptr(), xc.data_ptr(), w.data_ptr() if w is not None else None,
                mean.data_ptr(), rstd.data_ptr())
        outs = (dx.data_ptr() if dx is not None else None,
                dw.data_ptr() if dw is not None else None,
                db.data_ptr() if db is not None else None, rows, cols,
                _LN_DEFER if defer else 0)
        if (pending is not None and dx is not None) or defer:
            L.check(L.lib().tjh_layer_norm_backward_res(
                *args, pending.data_ptr() if pending is not None else None, *outs),
                "layer_norm_backward_res")
        else:
            L.check(L.lib().tjh_layer_norm_backward(*args, *outs), "layer_norm_backward")
        return [dx, dw, db]
    def gbwd(g):  # the forward from recording ops (layernorm.wgsl's arithmetic)
        def ref(xx, ww, bb):
            dims = tuple(range(xx.ndim - k, xx.ndim))
            xm = sub(xx, reduce_mean(xx, dims, keepdim=True))
            var = reduce_mean(mul(xm, xm), dims, keepdim=True)
            yy = mul(xm, (var + float(eps)).pow(-0.5))
            if ww is not None:
                yy = mul(yy, ww)
            return yy if bb is None else _T.add(yy, bb)
        return _T._regrad(ref, [x, weight, bias], g)
    return _record(y, "LayerNorm", [x, weight, bias], bwd, acc_slot=0, defer_slots=(1, 2),
                   gfn=gbwd)


# ------------------------------------------------------------ embedding / linear


def embedding(input, weight):
    """nn.Embedding lookup (embedding.wgsl:13-27, ids clamped); backward is a
    deterministic scatter-add into the table (torch.js: TODO, D11)."""
    ids = input
    if not isinstance(ids, Tensor):
        from .tensor import tensor as _tensor
        ids = _tensor(np.asarray(ids, dtype=np.int32), dtype="int32")
    if ids.dtype != "int32":
        ids = ids.to("int32")
    ids = ids.contiguous()
    V, D = weight.shape
    w = weight.detach().contiguous()
    out = empty(ids.shape + (D,))
    n = ids.numel()
    L.check(L.lib().tjh_embedding_forward(w.data_ptr(), V, D, ids.data_ptr(), n, out.data_ptr()),
            "embedding")

    def bwd(g, pending=None):
        # pending: the table's gradient so far in this backward pass (a table
        # tied to the LM head already holds that layer's weight gradient);
        # the rows are then added into it in place, with no zero fill of a
        # second [V, D] table and no add of the two
        g = g.contiguous()
        dw = pending if pending is not None else empty((V, D))
        L.check(L.lib().tjh_embedding_backward(g.data_ptr(), ids.data_ptr(), n, D, dw.data_ptr(),
                                               V, 1 if pending is not None else 0),
                "embedding_backward")
        return [dw]
    def gbwd(g):  # an index_add of the rows (ids clamped as the lookup clamps)
        ic = _T.tensor(np.clip(ids.numpy().reshape(-1), 0, V - 1).astype(np.int32), dtype="int32")
        return [_T._index_add_rec((V, D), 0, ic, reshape(g, (n, D)))]
    return _record(out, "Embedding", [weight], bwd, acc_slot=0, gfn=gbwd)


def _embedding_pos(input, weight, pos_weight, pos0=0):
    """embedding(input, weight) + embedding(pos0 + arange(T), pos_weight)
    for input [B, T] ids -- a transformer's token plus position embedding
    (two nn.Embedding lookups and an add, src/nn/embedding.ts:25-101) in
    one kernel, the same float add.  The backward gives both tables their
    gradients in one launch: the token rows as embedding() does (added into
    a pending gradient in place, as for a table tied to the LM head) and the
    position rows as the sum over the batch in batch order."""
    ids = input
    if not isinstance(ids, Tensor):
        from .tensor import tensor as _tensor
        ids = _tensor(np.asarray(ids, dtype=np.int32), dtype="int32")
    if ids.dtype != "int32":
        ids = ids.to("int32")
    if ids.ndim != 2:
        raise RuntimeError("_embedding_pos: ids must be [batch, T]")
    ids = ids.contiguous()
    B, T = ids.shape
    V, D = weight.shape
    P, D2 = pos_weight.shape
    if D2 != D:
        raise RuntimeError("_embedding_pos: tables of widths %d and %d" % (D, D2))
    if pos0 < 0 or pos0 + T > P:
        raise RuntimeError("_embedding_pos: positions [%d, %d) past the %d-row table"
                           % (pos0, pos0 + T, P))
    w = weight.detach().contiguous()
    wp = pos_weight.detach().contiguous()
    out = empty((B, T, D))
    L.check(L.lib().tjh_embedding_pos_forward(w.data_ptr(), V, D, ids.data_ptr(), B, T,
                                              wp.data_ptr(), P, pos0, out.data_ptr()),
            "embedding_pos")
    rw, rp = weight.requires_grad, pos_weight.requires_grad

    def bwd(g, pending=None):
        g = g.contiguous()
        dw = (pending if pending is not None else empty((V, D))) if rw else None
        dp = empty((P, D)) if rp else None
        L.check(L.lib().tjh_embedding_pos_backward(
            g.data_ptr(), ids.data_ptr(), B, T, D, dw.data_ptr() if dw is not None else None, V,
            1 if pending is not None else 0, dp.data_ptr() if dp is not None else None, P, pos0,
            0), "embedding_pos_backward")
        return [dw, dp]
    def gbwd(g):  # token rows: an index_add; position rows: the batch sum, placed
        ic = _T.tensor(np.clip(ids.numpy().reshape(-1), 0, V - 1).astype(np.int32), dtype="int32")
        dw = _T._index_add_rec((V, D), 0, ic, reshape(g, (B * T, D))) if rw else None
        dp = None
        if rp:
            parts = [zeros((pos0, D))] if pos0 else []
            parts.append(_T.reduce_sum(reshape(g, (B, T, D)), 0))
            if P - pos0 - T:
                parts.append(zeros((P - pos0 - T, D)))
            dp = _T.cat(parts, 0) if len(parts) > 1 else parts[0]
        return [dw, dp]
    return _record(out, "EmbeddingPos", [weight, pos_weight], bwd, acc_slot=0, gfn=gbwd)


def linear(x, weight, bias=None):
    """y = x W^T + b (src/nn/linear.ts:43-66) as ONE GEMM with the bias in
    the epilogue and W^T read in place; backward dx = g W, and dW = g^T x
    (split-K over tokens) with db = column sums of g from the same GEMM."""
    if x.dtype != "float32":
        x = x.float()
    out_f, in_f = weight.shape
    if x.shape[-1] != in_f:
        raise RuntimeError("linear: input features %d != weight in_features %d"
                           % (x.shape[-1], in_f))
    lead = x.shape[:-1]
    M = _numel(lead)
    x2 = reshape(x.detach(), (M, in_f))
    wd = weight.detach()
    bd = bias.detach().contiguous() if bias is not None else None
    out2 = _gemm(x2, wd.T, bias=bd, bias_mode=1 if bd is not None else 0)
    out = reshape_raw(out2, lead + (out_f,))
    rx, rw = x.requires_grad, weight.requires_grad
    rb = bias is not None and bias.requires_grad

    def bwd(g):
        if isinstance(g, _T._CEGrad):
            if not rb and g.rows == M and g.cols == out_f:
                # the cross-entropy gradient of the logits this layer made,
                # formed inside both GEMMs instead of read from memory
                dx = reshape_raw(_T._gemm_ce(g, wd, False), lead + (in_f,)) if rx else None
                dw = _T._gemm_ce(g, x2, True) if rw else None
                return [dx, dw, None]
            g = g.materialize()
        g2 = reshape_raw(g, (M, out_f))
        dx = reshape_raw(_gemm(g2, wd), lead + (in_f,)) if rx else None
        dw = db = None
        if rw and rb:
            # db = the row sums of g^T, accumulated by the dW GEMM itself
            db = empty((out_f,))
            dw = _gemm(g2.T, x2, rowsum_out=db)
        elif rw:
            dw = _gemm(g2.T, x2)
        elif rb:
            gc = g2 if g2.is_contiguous() else _k_contiguous(g2)
            db = _view_raw(_k_reduce("sum", gc, [0]), (out_f,))
        return [dx, dw, db]

    def gbwd(g):  # recording ops: the gradients can be differentiated again
        g2 = _T.reshape(g, (M, out_f))
        dx = _T.reshape(_T.matmul(g2, weight), lead + (in_f,)) if rx else None
        dw = _T.matmul(_T.transpose(g2, 0, 1), _T.reshape(x, (M, in_f))) if rw else None
        db = _T.reduce_sum(g2, 0) if rb else None
        return [dx, dw, db]
    return _record(out, "Linear", [x, weight, bias], bwd, gfn=gbwd)


def _linear_add(x, weight, bias, residual):
    """residual + linear(x, weight, bias) -- the residual add that follows
    the attention projection of a pre-LN transformer block -- as one GEMM
    whose epilogue adds the residual.  Equal bit for bit to the unfused
    add; the residual's gradient is the incoming gradient itself."""
    if residual is None:
        return linear(x, weight, bias)
    if x.dtype != "float32":
        x = x.float()
    out_f, in_f = weight.shape
    lead = x.shape[:-1]
    if x.shape[-1] != in_f or residual.shape != lead + (out_f,):
        raise RuntimeError("linear_add: shapes %s, %s, %s do not match"
                           % (list(x.shape), list(weight.shape), list(residual.shape)))
    M = _numel(lead)
    x2 = reshape(x.detach(), (M, in_f))
    wd = weight.detach()
    bd = bias.detach().contiguous() if bias is not None else None
    r = residual.detach()
    r2 = reshape(r if r.dtype == "float32" and r.is_contiguous() else r.float().contiguous(),
                 (M, out_f))
    out2 = empty((M, out_f))
    _gemm(x2, wd.T, out=out2, bias=bd, bias_mode=1 if bd is not None else 0, aux=r2, act=3)
    out = reshape_raw(out2, lead + (out_f,))
    rx, rw = x.requires_grad, weight.requires_grad
    rb = bias is not None and bias.requires_grad

    def bwd(g):
        g2 = reshape_raw(g, (M, out_f))
        dx = reshape_raw(_gemm(g2, wd), lead + (in_f,)) if rx else None
        dw = db = None
        if rw and rb:
            db = empty((out_f,))
            dw = _gemm(g2.T, x2, rowsum_out=db)
        elif rw:
            dw = _gemm(g2.T, x2)
        elif rb:
            gc = g2 if g2.is_contiguous() else _k_contiguous(g2)
            db = _view_raw(_k_reduce("sum", gc, [0]), (out_f,))
        return [dx, dw, db, g]
    return _record(out, "LinearAdd", [x, weight, bias, residual], bwd,
                   gfn=lambda g: _T._regrad(lambda xx, ww, bb, rr: _T.add(rr, linear(xx, ww, bb)),
                                            [x, weight, bias, residual], g))


def _mlp_gelu(x, w1, b1, w2, b2, residual=None):
    """linear(gelu(linear(x, w1, b1)), w2, b2) -- the transformer MLP block
    (nn.Linear, nn.GELU, nn.Linear; src/nn/linear.ts:43-66,
    src/nn/activation.ts) -- with GELU fused into the GEMM epilogues: the
    first GEMM writes the pre-activation h and GELU(h), and in the backward
    the second layer's input-gradient GEMM multiplies by GELU'(h) as it
    writes.  With `residual`, returns residual + MLP(x), the add done by
    the second GEMM's epilogue.  Every value equals the unfused sequence's
    bit for bit."""
    if x.dtype != "float32":
        x = x.float()
    hid, d_in = w1.shape
    d_out = w2.shape[0]
    if x.shape[-1] != d_in or w2.shape[1] != hid:
        raise RuntimeError("mlp: shapes %s, %s, %s do not chain" % (x.shape, w1.shape, w2.shape))
    lead = x.shape[:-1]
    M = _numel(lead)
    x2 = reshape(x.detach(), (M, d_in))
    w1d, w2d = w1.detach(), w2.detach()
    b1d = b1.detach().contiguous() if b1 is not None else None
    b2d = b2.detach().contiguous() if b2 is not None else None
    if residual is not None and residual.shape != lead + (d_out,):
        raise RuntimeError("mlp: residual shape %s != output shape %s"
                           % (list(residual.shape), list(lead + (d_out,))))
    h = empty((M, hid))
    a = empty((M, hid))
    _gemm(x2, w1d.T, out=a, bias=b1d, bias_mode=1 if b1d is not None else 0, aux=h, act=1)
    if residual is None:
        y2 = _gemm(a, w2d.T, bias=b2d, bias_mode=1 if b2d is not None else 0)
    else:
        r = residual.detach()
        r2 = reshape(r if r.dtype == "float32" and r.is_contiguous() else r.float().contiguous(),
                     (M, d_out))
        y2 = empty((M, d_out))
        _gemm(a, w2d.T, out=y2, bias=b2d, bias_mode=1 if b2d is not None else 0, aux=r2, act=3)
    out = reshape_raw(y2, lead + (d_out,))
    need = [t is not None and t.requires_grad for t in (x, w1, b1, w2, b2)]

    def bwd(g):
        g2 = reshape_raw(g, (M, d_out))
        if not g2.is_contiguous():
            g2 = _k_contiguous(g2)
        dx = dw1 = db1 = dw2 = db2 = None
        if need[3] or need[4]:
            db2 = empty((d_out,)) if need[4] else None
            if need[3]:
                dw2 = _gemm(g2.T, a, rowsum_out=db2)
            else:
                db2 = _view_raw(_k_reduce("sum", g2, [0]), (d_out,))
        if need[0] or need[1] or need[2]:
            dh = empty((M, hid))
            _gemm(g2, w2d, out=dh, aux=h, act=2)  # (g W2) * GELU'(h)
            if need[0]:
                dx = reshape_raw(_gemm(dh, w1d), lead + (d_in,))
            if need[1]:
                db1 = empty((hid,)) if need[2] else None
                dw1 = _gemm(dh.T, x2, rowsum_out=db1)
            elif need[2]:
                db1 = _view_raw(_k_reduce("sum", dh, [0]), (hid,))
        return [dx, dw1, db1, dw2, db2, g]
    def gbwd(g):  # nn.Linear, GELU, nn.Linear (+ residual) from recording ops
        def ref(xx, a1, c1, a2, c2, rr):
            yy = linear(gelu(linear(xx, a1, c1)), a2, c2)
            return yy if rr is None else _T.add(rr, yy)
        return _T._regrad(ref, [x, w1, b1, w2, b2, residual], g)
    return _record(out, "MLP", [x, w1, b1, w2, b2, residual], bwd, gfn=gbwd)


# ------------------------------------------------------------ convolution


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    """F.conv2d (src/nn/functional.ts:438-660): NCHW cross-correlation with
    stride / padding / dilation / groups; dgrad, wgrad and bias grad
    (torch.js never runs its conv backward, D8)."""
    return _conv2d(input, weight, bias, stride, padding, dilation, groups, False)


def conv2d_relu(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    """F.relu(F.conv2d(...)) as one op: the convolution writes ReLU of its
    output, and the backward takes ReLU's gradient mask from that output
    (y > 0 exactly where the pre-activation is > 0); bit for bit the two
    ops in sequence."""
    return _conv2d(input, weight, bias, stride, padding, dilation, groups, True)


def _conv2d(input, weight, bias, stride, padding, dilation, groups, relu):
    x = input
    if x.dtype != "float32":
        x = x.float()
    if x.ndim != 4 or weight.ndim != 4:
        raise RuntimeError("conv2d expects 4-D input and weight")
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw_ = _pair(dilation)
    n, c, h, w = x.shape
    oc, cg, kh, kw = weight.shape
    if cg * groups != c:
        raise RuntimeError("conv2d: weight expects %d input channels, got %d" % (cg * groups, c))
    oh = (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    ow = (w + 2 * pw - dw_ * (kw - 1) - 1) // sw + 1
    desc = L.Conv2dDesc(n, c, h, w, oc, kh, kw, sh, sw, ph, pw, dh, dw_, groups, oh, ow)
    xc = contiguous(x.detach())
    wc = weight.detach().contiguous()
    bc = bias.detach().contiguous() if bias is not None else None
    y = empty((n, oc, oh, ow))
    L.check(L.lib().tjh_conv2d_forward_act(ctypes.byref(desc), xc.data_ptr(), wc.data_ptr(),
                                           bc.data_ptr() if bc is not None else None,
                                           y.data_ptr(), 1 if relu else 0), "conv2d")
    rx, rw = x.requires_grad, weight.requires_grad
    rb = bias is not None and bias.requires_grad
    yd = y.detach() if relu else None

    def bwd(g):
        if relu:
            g = _e_unary_bwd("relu", g, yd, None)  # ReLU'(pre) = (y > 0)
        g = g.contiguous()
        dx = dwt = db = None
        if rx:
            dx = empty(x.shape)
            L.check(L.lib().tjh_conv2d_backward_input(ctypes.byref(desc), g.data_ptr(),
                                                      wc.data_ptr(), dx.data_ptr()),
                    "conv2d_backward_input")
        if rw:
            # the bias gradient (dy summed over images and pixels) comes out
            # of the weight-gradient product, which stages dy anyway
            dwt = empty(weight.shape)
            db = empty((oc,)) if rb else None
            L.check(L.lib().tjh_conv2d_backward_weight_bias(
                ctypes.byref(desc), g.data_ptr(), xc.data_ptr(), dwt.data_ptr(),
                db.data_ptr() if db is not None else None, 0), "conv2d_backward_weight")
        elif rb:
            db = _view_raw(_k_reduce("sum", g, [0, 2, 3]), (oc,))
        return [dx, dwt, db]
    return _record(y, "Conv2dReLU" if relu else "Conv2d", [x, weight, bias], bwd)


# ------------------------------------------------------------ attention


def _bhtd(t):
    """[B,H,T,D] or [B,T,D] view -> (4-D view, strides of B,H,T)."""
    if t.ndim == 3:
        t = _alias(t, (t.shape[0], 1) + t.shape[1:], (t._strides[0], 0) + t._strides[1:],
                   t._offset)
    if t.ndim != 4:
        raise RuntimeError("scaled_dot_product_attention expects 3-D or 4-D tensors")
    if t._strides[3] != 1 and t.shape[3] > 1:
        t = _k_contiguous(t)
    return t


def scaled_dot_product_attention(query, key, value, attn_mask=None, dropout_p=0.0,
                                 is_causal=False, scale=None):
    """softmax(Q K^T * scale [causal] [mask]) V (src/nn/functional.ts:866-890).
    torch.js ignores is_causal and throws on attn_mask; both follow
    PyTorch's contract here.  Without a mask the flash kernels run (O(T)
    memory); the output is laid out [B, T, H, D] in memory and returned as
    a [B, H, T, D] view, so the usual transpose(1, 2) that follows is free.
    With attn_mask (bool: True takes part in attention; float: added to
    the scores, broadcast over the leading dims) the scores are formed
    explicitly from the library's batched GEMM, masked and softmaxed, so
    autograd runs through those ops."""
    if attn_mask is not None:
        if is_causal:
            raise RuntimeError("scaled_dot_product_attention: pass either attn_mask or "
                               "is_causal, not both")
        return _sdpa_masked(query, key, value, attn_mask, scale)
    if dropout_p:
        raise NotImplementedError("scaled_dot_product_attention: dropout is not on the hip path")
    three = query.ndim == 3
    q = _bhtd(query.detach())
    k = _bhtd(key.detach())
    v = _bhtd(value.detach())
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    ob = empty((B, Tq, H, D))
    o = _alias(ob, (B, H, Tq, D), (Tq * H * D, D, H * D, 1), 0)
    lse = empty((B, H, Tq))
    L.check(L.lib().tjh_sdpa_forward(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     lse.data_ptr(), B, H, Tq, Tk, D, L.i64arr(q._strides[:3]),
                                     L.i64arr(k._strides[:3]), L.i64arr(v._strides[:3]),
                                     L.i64arr(o._strides[:3]), sc, 1 if is_causal else 0), "sdpa")

    def grad_like(t):
        Bx, Hx, Tx, Dx = t.shape
        buf = empty((Bx, Tx, Hx, Dx))
        return _alias(buf, t.shape, (Tx * Hx * Dx, Dx, Hx * Dx, 1), 0)

    def shared_grads():
        """dq, dk, dv laid out exactly like q, k, v inside one new buffer when
        the three are equally strided, disjoint views of one allocation (the
        fused qkv projection split into heads): the gradient of that
        projection's output is then that buffer, assembled with no copy."""
        ts = (q, k, v)
        if not all(t._storage is q._storage and t._strides == q._strides and
                   t.shape == q.shape for t in ts):
            return None
        # innermost dense run of the layout: each view is a set of runs of
        # length `run` at offset + multiples of `period`
        dims = sorted((st, n) for st, n in zip(q._strides, q.shape) if n > 1)
        run, i = 1, 0
        while i < len(dims) and dims[i][0] == run:
            run *= dims[i][1]
            i += 1
        outer = [st for st, _ in dims[i:]]
        if not outer:
            return None
        period = min(outer)
        if run > period or any(st % period for st in outer):
            return None
        res = sorted(t._offset % period for t in ts)
        gaps = [res[1] - res[0], res[2] - res[1], period - (res[2] - res[0])]
        if min(gaps) < run:
            return None  # the views share elements
        ext = [t._offset + sum((n - 1) * st for n, st in zip(t.shape, t._strides)) + 1
               for t in ts]
        lo = min(t._offset for t in ts)
        buf = empty((max(ext) - lo,))
        return [_alias(buf, t.shape, t._strides, t._offset - lo) for t in ts]

    def bwd(g):
        if three:
            g = _alias(g, (g.shape[0], 1) + g.shape[1:], (g._strides[0], 0) + g._strides[1:],
                       g._offset)
        if g._strides[3] != 1:
            g = _k_contiguous(g)
        shared = shared_grads()
        dq, dk, dv = shared if shared else (grad_like(q), grad_like(k), grad_like(v))
        arrs = [L.i64arr(t._strides[:3]) for t in (q, k, v, o, g, dq, dk, dv)]
        ptrs = (L.P_i64 * 8)(*[ctypes.cast(a, L.P_i64) for a in arrs])
        L.check(L.lib().tjh_sdpa_backward(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                          g.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                                          dk.data_ptr(), dv.data_ptr(), B, H, Tq, Tk, D, ptrs, sc,
                                          1 if is_causal else 0), "sdpa_backward")
        if three:
            dq, dk, dv = [_alias(t, (t.shape[0],) + t.shape[2:], (t._strides[0],) + t._strides[2:],
                                 t._offset) for t in (dq, dk, dv)]
        return [dq, dk, dv]
    out = o
    if three:
        out = _alias(ob, (B, Tq, D), (Tq * D, D, 1), 0)
    def gbwd(g):  # softmax(Q K^T * scale [causal]) V with recording ops
        def ref(qq, kk, vv):
            scores = mul(_T.matmul(qq, kk.transpose(-2, -1)), sc)
            if is_causal:
                drop = _T.triu(_T.ones((Tq, Tk)), 1)  # key j > query i
                scores = _T.masked_fill(scores, drop, float("-inf"))
            return _T.matmul(softmax(scores, -1), vv)
        return _T._regrad(ref, [query, key, value], g)
    return _record(out, "SDPA", [query, key, value], bwd, gfn=gbwd)


def _sdpa_masked(query, key, value, attn_mask, scale):
    """SDPA with an explicit mask from differentiable ops: scores = Q K^T *
    scale (batched GEMM), then masked_fill(-inf) where a bool mask is False
    or + a float mask, softmax over keys, times V."""
    from .tensor import compare_raw, masked_fill as _masked_fill, matmul as _matmul
    D = query.shape[-1]
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    kt = key.transpose(-2, -1)
    scores = mul(_matmul(query, kt), sc)
    m = attn_mask
    if not isinstance(m, Tensor):
        from .tensor import tensor as _tensor
        m = _tensor(np.asarray(m))
    if m.dtype in ("bool", "uint8"):
        drop = compare_raw(m.float(), 0.0, "eq")  # 1 where the key is masked out
        scores = _masked_fill(scores, drop, float("-inf"))
    else:
        scores = scores + m.float() if m.dtype != "float32" else scores + m
    return _matmul(softmax(scores, -1), value)


# ------------------------------------------------------------ one_hot


def one_hot(input, num_classes=-1):
    """F.one_hot (src/nn/functional.ts:764-796): values are rounded
    (Math.round), rows whose class is outside [0, C) stay zero, and C
    defaults to floor(max) + 1 (read back from the device, as torch.js
    does).  Float32 output of shape input.shape + (C,)."""
    x = input.contiguous()
    n = x.numel()
    C = int(num_classes)
    if C <= 0:
        mx = float(x.numpy().max()) if n else 0.0
        C = max(1, int(math.floor(mx)) + 1)
    out = empty(x.shape + (C,))
    if n:
        if x.dtype == "int32":
            L.check(L.lib().tjh_one_hot_i32(x.data_ptr(), n, C, out.data_ptr()), "one_hot")
        else:
            xf = x if x.dtype == "float32" else x.float()
            L.check(L.lib().tjh_one_hot(xf.data_ptr(), n, C, out.data_ptr()), "one_hot")
    return out
