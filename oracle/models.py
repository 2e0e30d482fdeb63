"""The benchmark workloads as explicit forward + backward over oracle.ops.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Parameters are dicts of float32 numpy arrays named like the 'hip' modules
(torch.nn layout: Linear weight [out, in]).  Every function returns the
loss (float64) and the gradient of every parameter (float64 arrays).
"""
import math
from dataclasses import dataclass

import numpy as np

from . import ops

F64 = np.float64


# ------------------------------------------------------------------ MLP


def mlp_loss_and_grads(p, x, t):
    """Linear(784,256) -> ReLU -> Linear(256,10) -> cross_entropy."""
    h = ops.linear(x, p["0.weight"], p["0.bias"])
    a = ops.unary("relu", h)
    z = ops.linear(a, p["2.weight"], p["2.bias"])
    loss = ops.cross_entropy(z, t)
    dz = ops.cross_entropy_backward(z, t)
    da, dw2, db2 = ops.linear_backward(dz, a, p["2.weight"])
    dh = ops.unary_backward("relu", da, h)
    _, dw0, db0 = ops.linear_backward(dh, x, p["0.weight"])
    return loss, {"0.weight": dw0, "0.bias": db0, "2.weight": dw2, "2.bias": db2}


# ------------------------------------------------------------------ elementwise chain


def chain_loss_and_grads(x, bias, y):
    """mean(sum_0(gelu(x + bias) * y)) and (dx, dbias, dy)."""
    h = ops.binary("add", x, bias)
    a = ops.gelu(h)
    z = a * np.asarray(y, dtype=F64)
    s = z.sum(axis=0)
    loss = s.mean()
    ds = np.full(s.shape, 1.0 / s.size)
    dz = np.broadcast_to(ds, z.shape)
    da = dz * y
    dy = dz * a
    dh = ops.unary_backward("gelu", da, h)
    return loss, {"x": dh, "bias": ops.sum_to(dh, np.shape(bias)), "y": dy}


# ------------------------------------------------------------------ CNN


def cnn_loss_and_grads(p, x, t):
    """conv(3->32,3x3,p1) -> ReLU -> conv(32->64,3x3,s2,p1) -> ReLU ->
    global avg-pool -> Linear(64,10) -> cross_entropy."""
    c1 = ops.conv2d(x, p["conv1.weight"], p["conv1.bias"], 1, 1)
    r1 = ops.unary("relu", c1)
    c2 = ops.conv2d(r1, p["conv2.weight"], p["conv2.bias"], 2, 1)
    r2 = ops.unary("relu", c2)
    pooled = r2.mean(axis=(2, 3))
    z = ops.linear(pooled, p["fc.weight"], p["fc.bias"])
    loss = ops.cross_entropy(z, t)
    dz = ops.cross_entropy_backward(z, t)
    dpool, dwf, dbf = ops.linear_backward(dz, pooled, p["fc.weight"])
    dr2 = np.broadcast_to(dpool[:, :, None, None] / (r2.shape[2] * r2.shape[3]), r2.shape)
    dc2 = ops.unary_backward("relu", dr2, c2)
    dr1, dw2, db2 = ops.conv2d_backward(dc2, r1, p["conv2.weight"], 2, 1)
    dc1 = ops.unary_backward("relu", dr1, c1)
    _, dw1, db1 = ops.conv2d_backward(dc1, x, p["conv1.weight"], 1, 1)
    return loss, {"conv1.weight": dw1, "conv1.bias": db1, "conv2.weight": dw2,
                  "conv2.bias": db2, "fc.weight": dwf, "fc.bias": dbf}


# ------------------------------------------------------------------ transformer


@dataclass
class Config:
    vocab: int = 50257
    ctx: int = 1024
    d: int = 768
    heads: int = 12
    layers: int = 12


def init_params(cfg, rng, std=0.02):
    """GPT-2 parameters N(0, std) (biases 0, LayerNorm 1/0), float32."""
    d = cfg.d
    p = {"wte.weight": (rng.standard_normal((cfg.vocab, d)) * std).astype(np.float32),
         "wpe.weight": (rng.standard_normal((cfg.ctx, d)) * std).astype(np.float32)}
    for i in range(cfg.layers):
        p.update(block_params(d, rng, std, "h.%d." % i))
    p["ln_f.weight"] = np.ones(d, np.float32)
    p["ln_f.bias"] = np.zeros(d, np.float32)
    return p


def block_params(d, rng, std=0.02, prefix=""):
    def w(o, i):
        return (rng.standard_normal((o, i)) * std).astype(np.float32)
    z = lambda n: np.zeros(n, np.float32)
    return {prefix + "ln_1.weight": np.ones(d, np.float32), prefix + "ln_1.bias": z(d),
            prefix + "attn.c_attn.weight": w(3 * d, d), prefix + "attn.c_attn.bias": z(3 * d),
            prefix + "attn.c_proj.weight": w(d, d), prefix + "attn.c_proj.bias": z(d),
            prefix + "ln_2.weight": np.ones(d, np.float32), prefix + "ln_2.bias": z(d),
            prefix + "mlp.c_fc.weight": w(4 * d, d), prefix + "mlp.c_fc.bias": z(4 * d),
            prefix + "mlp.c_proj.weight": w(d, 4 * d), prefix + "mlp.c_proj.bias": z(d)}


def block_forward(p, pre, x, heads):
    """Pre-LN block: h = x + proj(attn(ln_1 x)); out = h + mlp(ln_2 h).
    Returns (out, cache)."""
    B, T, d = x.shape
    hd = d // heads
    c = {}
    c["x"] = x
    c["ln1"], _, _ = ops.layer_norm(x, p[pre + "ln_1.weight"], p[pre + "ln_1.bias"])
    qkv = ops.linear(c["ln1"], p[pre + "attn.c_attn.weight"], p[pre + "attn.c_attn.bias"])
    q, k, v = np.split(qkv, 3, axis=-1)
    sh = lambda t: t.reshape(B, T, heads, hd).transpose(0, 2, 1, 3)
    c["q"], c["k"], c["v"] = sh(q), sh(k), sh(v)
    o, _ = ops.sdpa(c["q"], c["k"], c["v"], causal=True)
    c["att"] = o.transpose(0, 2, 1, 3).reshape(B, T, d)
    proj = ops.linear(c["att"], p[pre + "attn.c_proj.weight"], p[pre + "attn.c_proj.bias"])
    c["h"] = x + proj
    c["ln2"], _, _ = ops.layer_norm(c["h"], p[pre + "ln_2.weight"], p[pre + "ln_2.bias"])
    c["fc"] = ops.linear(c["ln2"], p[pre + "mlp.c_fc.weight"], p[pre + "mlp.c_fc.bias"])
    c["gelu"] = ops.gelu(c["fc"])
    mo = ops.linear(c["gelu"], p[pre + "mlp.c_proj.weight"], p[pre + "mlp.c_proj.bias"])
    return c["h"] + mo, c


def block_backward(p, pre, dout, c, heads, grads):
    B, T, d = c["x"].shape
    hd = d // heads
    dh = dout.copy()
    dg, dw, db = ops.linear_backward(dout, c["gelu"], p[pre + "mlp.c_proj.weight"])
    grads[pre + "mlp.c_proj.weight"], grads[pre + "mlp.c_proj.bias"] = dw, db
    dfc = ops.unary_backward("gelu", dg, c["fc"])
    dln2, dw, db = ops.linear_backward(dfc, c["ln2"], p[pre + "mlp.c_fc.weight"])
    grads[pre + "mlp.c_fc.weight"], grads[pre + "mlp.c_fc.bias"] = dw, db
    dx2, dgm, dbt = ops.layer_norm_backward(dln2, c["h"], p[pre + "ln_2.weight"])
    grads[pre + "ln_2.weight"], grads[pre + "ln_2.bias"] = dgm, dbt
    dh = dh + dx2
    datt, dw, db = ops.linear_backward(dh, c["att"], p[pre + "attn.c_proj.weight"])
    grads[pre + "attn.c_proj.weight"], grads[pre + "attn.c_proj.bias"] = dw, db
    do = datt.reshape(B, T, heads, hd).transpose(0, 2, 1, 3)
    dq, dk, dv = ops.sdpa_backward(do, c["q"], c["k"], c["v"], causal=True)
    un = lambda t: t.transpose(0, 2, 1, 3).reshape(B, T, d)
    dqkv = np.concatenate([un(dq), un(dk), un(dv)], axis=-1)
    dln1, dw, db = ops.linear_backward(dqkv, c["ln1"], p[pre + "attn.c_attn.weight"])
    grads[pre + "attn.c_attn.weight"], grads[pre + "attn.c_attn.bias"] = dw, db
    dx1, dgm, dbt = ops.layer_norm_backward(dln1, c["x"], p[pre + "ln_1.weight"])
    grads[pre + "ln_1.weight"], grads[pre + "ln_1.bias"] = dgm, dbt
    return dh + dx1


def block_loss_and_grads(p, x, heads):
    """Transformer block with loss = mean(out); grads include 'x'."""
    out, c = block_forward(p, "", np.asarray(x, dtype=F64), heads)
    loss = out.mean()
    grads = {}
    dx = block_backward(p, "", np.full(out.shape, 1.0 / out.size), c, heads, grads)
    grads["x"] = dx
    return loss, grads


def gpt2_loss_and_grads(cfg, p, ids, targets, return_dlogits=False):
    """GPT-2 (tied embeddings) next-token cross_entropy and all grads (and
    the logits' gradient [B*T, vocab] with return_dlogits)."""
    ids = np.asarray(ids)
    B, T = ids.shape
    p = {k: np.asarray(v, dtype=F64) for k, v in p.items()}
    x = ops.embedding(p["wte.weight"], ids) + ops.embedding(p["wpe.weight"], np.arange(T))[None]
    caches = []
    for i in range(cfg.layers):
        x, c = block_forward(p, "h.%d." % i, x, cfg.heads)
        caches.append(c)
    lnf, _, _ = ops.layer_norm(x, p["ln_f.weight"], p["ln_f.bias"])
    logits = ops.linear(lnf, p["wte.weight"]).reshape(B * T, cfg.vocab)
    t = np.asarray(targets).reshape(-1)
    loss = ops.cross_entropy(logits, t)
    dlog = ops.cross_entropy_backward(logits, t).reshape(B, T, cfg.vocab)
    grads = {}
    dlnf, dwte_head, _ = ops.linear_backward(dlog, lnf, p["wte.weight"])
    dx, grads["ln_f.weight"], grads["ln_f.bias"] = ops.layer_norm_backward(dlnf, x,
                                                                          p["ln_f.weight"])
    for i in reversed(range(cfg.layers)):
        dx = block_backward(p, "h.%d." % i, dx, caches[i], cfg.heads, grads)
    grads["wte.weight"] = dwte_head + ops.embedding_backward(dx, ids, cfg.vocab)
    grads["wpe.weight"] = np.zeros_like(p["wpe.weight"], dtype=F64)
    grads["wpe.weight"][:T] = dx.sum(axis=0)
    if return_dlogits:
        return loss, grads, dlog.reshape(B * T, cfg.vocab)
    return loss, grads


def adamw_step(p, grads, lr, wd, step, betas=(0.9, 0.999), eps=1e-8, state=None):
    """AdamW on every parameter (oracle.ops.adam_step, decoupled)."""
    out = {}
    for k, v in p.items():
        m = state[k][0] if state else np.zeros_like(v)
        s = state[k][1] if state else np.zeros_like(v)
        out[k], _, _ = ops.adam_step(v, np.asarray(grads[k], dtype=np.float32), m, s, step, lr,
                                     betas, eps, wd, decoupled=True)
    return out


# ------------------------------------------------------------------ MultiheadAttention


def mha_mask(N, H, L, S, attn_mask=None, key_padding_mask=None):
    """The additive float mask [N, H, L, S] (or None) that nn.MultiheadAttention
    applies, with PyTorch's meanings (the reference throws on both masks,
    src/nn/attention.ts:121-126): a bool mask is True where attention is
    NOT allowed (-inf), a float mask is added; attn_mask is [L, S] or
    [N * H, L, S], key_padding_mask is [N, S]."""
    m = np.zeros((N, H, L, S))
    used = False
    if attn_mask is not None:
        a = np.asarray(attn_mask)
        a = np.where(a, -np.inf, 0.0) if a.dtype == bool else a.astype(F64)
        m = m + (a.reshape(1, 1, L, S) if a.ndim == 2 else a.reshape(N, H, L, S))
        used = True
    if key_padding_mask is not None:
        k = np.asarray(key_padding_mask)
        k = np.where(k, -np.inf, 0.0) if k.dtype == bool else k.astype(F64)
        m = m + k.reshape(N, 1, 1, S)
        used = True
    return m if used else None


def _mha_inputs(query, key, value, batch_first):
    """(N, L, E) views of the three inputs."""
    if batch_first:
        return [np.asarray(t, dtype=F64) for t in (query, key, value)]
    return [np.swapaxes(np.asarray(t, dtype=F64), 0, 1) for t in (query, key, value)]


def mha_forward(p, query, key, value, heads, batch_first=False, mask=None, causal=False):
    """nn.MultiheadAttention.forward (src/nn/attention.ts:112-271): q, k, v
    projected by the three row blocks of in_proj_weight [3E, E] (+ the
    blocks of in_proj_bias), split into heads, softmax(q k^T / sqrt(hd)
    [+ mask]) v, heads merged, out_proj_weight / out_proj_bias; inputs and
    output [L, N, E], or [N, L, E] with batch_first.  Returns (out,
    weights [N, H, L, S], cache for mha_backward)."""
    q_in, k_in, v_in = _mha_inputs(query, key, value, batch_first)
    N, L, E = q_in.shape
    S = k_in.shape[1]
    hd = E // heads
    W = np.asarray(p["in_proj_weight"], dtype=F64)
    b = p.get("in_proj_bias")
    b = np.zeros(3 * E) if b is None else np.asarray(b, dtype=F64)
    proj = [x @ W[i * E:(i + 1) * E].T + b[i * E:(i + 1) * E] for i, x in
            enumerate((q_in, k_in, v_in))]
    qh, kh, vh = [t.reshape(t.shape[0], t.shape[1], heads, hd).transpose(0, 2, 1, 3)
                  for t in proj]
    o, _ = ops.sdpa(qh, kh, vh, causal=causal, mask=mask)
    wts = ops.sdpa_weights(qh, kh, causal=causal, mask=mask)
    y = o.transpose(0, 2, 1, 3).reshape(N, L, E)
    Wo = np.asarray(p["out_proj_weight"], dtype=F64)
    bo = p.get("out_proj_bias")
    out = y @ Wo.T + (0.0 if bo is None else np.asarray(bo, dtype=F64))
    if not batch_first:
        out = np.swapaxes(out, 0, 1)
    cache = dict(q_in=q_in, k_in=k_in, v_in=v_in, qh=qh, kh=kh, vh=vh, y=y, heads=heads,
                 batch_first=batch_first, mask=mask, causal=causal)
    return out, wts, cache


def mha_backward(p, dout, cache):
    """Gradients of mha_forward's output: a dict with in_proj_weight,
    in_proj_bias, out_proj_weight, out_proj_bias and query, key, value (each
    input's own gradient; a caller passing one tensor as several inputs
    adds them)."""
    dout = np.asarray(dout, dtype=F64)
    if not cache["batch_first"]:
        dout = np.swapaxes(dout, 0, 1)
    N, L, E = dout.shape
    heads = cache["heads"]
    hd = E // heads
    Wo = np.asarray(p["out_proj_weight"], dtype=F64)
    W = np.asarray(p["in_proj_weight"], dtype=F64)
    g = {}
    d2 = dout.reshape(-1, E)
    g["out_proj_weight"] = d2.T @ cache["y"].reshape(-1, E)
    g["out_proj_bias"] = d2.sum(axis=0)
    dy = (dout @ Wo).reshape(N, L, heads, hd).transpose(0, 2, 1, 3)
    dqh, dkh, dvh = ops.sdpa_backward(dy, cache["qh"], cache["kh"], cache["vh"],
                                      causal=cache["causal"], mask=cache["mask"])
    dW = np.zeros_like(W)
    db = np.zeros(3 * E)
    for i, (dh, x, name) in enumerate(((dqh, cache["q_in"], "query"), (dkh, cache["k_in"], "key"),
                                       (dvh, cache["v_in"], "value"))):
        dp = dh.transpose(0, 2, 1, 3).reshape(x.shape[0], x.shape[1], E)
        dW[i * E:(i + 1) * E] = dp.reshape(-1, E).T @ x.reshape(-1, E)
        db[i * E:(i + 1) * E] = dp.reshape(-1, E).sum(axis=0)
        dx = dp @ W[i * E:(i + 1) * E]
        g[name] = dx if cache["batch_first"] else np.swapaxes(dx, 0, 1)
    g["in_proj_weight"] = dW
    g["in_proj_bias"] = db
    return g
