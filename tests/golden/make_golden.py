"""Writes tests/golden/*.npz: known-answer vectors for the oracle.

The vectors come from PyTorch 2.x on the CPU in float64 (a library that
implements the same `@pytorch` contracts torch.js declares; it is not the
reference, which is TypeScript/WGSL and cannot run here).  Inputs are
small and seeded; every file holds inputs and expected outputs only.

    python tests/golden/make_golden.py
"""
import collections
import math
import os

import numpy as np
import torch

OUT = os.path.dirname(os.path.abspath(__file__))
torch.set_default_dtype(torch.float64)


def t(a, grad=False):
    return torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=grad)


def save(name, **arrays):
    np.savez_compressed(os.path.join(OUT, name + ".npz"),
                        **{k: np.asarray(v.detach().numpy() if torch.is_tensor(v) else v)
                           for k, v in arrays.items()})


def unary_ops(rng):
    x = rng.uniform(-3, 3, size=64)
    xp = rng.uniform(0.1, 3, size=64)
    g = rng.standard_normal(64)
    d = {"x": x, "xp": xp, "g": g}
    fns = {
        "neg": (torch.neg, x), "exp": (torch.exp, x), "log": (torch.log, xp),
        "sqrt": (torch.sqrt, xp), "rsqrt": (torch.rsqrt, xp), "tanh": (torch.tanh, x),
        "sigmoid": (torch.sigmoid, x), "relu": (torch.relu, x),
        "gelu": (lambda v: torch.nn.functional.gelu(v), x), "square": (torch.square, x),
        "reciprocal": (torch.reciprocal, xp), "erf": (torch.erf, x), "abs": (torch.abs, x),
        "sin": (torch.sin, x), "cos": (torch.cos, x), "silu": (torch.nn.functional.silu, x),
        "softplus": (torch.nn.functional.softplus, x),
    }
    F = torch.nn.functional
    fns.update({
        "leaky_relu_0.01": (lambda v: F.leaky_relu(v, 0.01), x),
        "leaky_relu_0.2": (lambda v: F.leaky_relu(v, 0.2), x),
        "elu_1.0": (lambda v: F.elu(v, 1.0), x), "elu_0.7": (lambda v: F.elu(v, 0.7), x),
        "sign": (torch.sign, np.concatenate([x[:60], [0.0, -0.0, 1e-300, -1e-300]])),
    })
    for name, (fn, inp) in fns.items():
        a = t(inp, True)
        y = fn(a)
        y.backward(t(g))
        d["fwd_" + name] = y
        d["bwd_" + name] = a.grad
    d["x_sign"] = fns["sign"][1]
    save("unary", **d)


def binary_ops(rng):
    a = rng.uniform(0.5, 2.0, size=(3, 4, 5))
    b = rng.uniform(0.5, 2.0, size=(4, 1))
    g = rng.standard_normal((3, 4, 5))
    d = {"a": a, "b": b, "g": g}
    for name, fn in {"add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div,
                     "pow": torch.pow, "maximum": torch.maximum,
                     "minimum": torch.minimum}.items():
        ta, tb = t(a, True), t(b, True)
        y = fn(ta, tb)
        y.backward(t(g))
        d["fwd_" + name], d["ga_" + name], d["gb_" + name] = y, ta.grad, tb.grad
    # maximum / minimum with ties (PyTorch splits a tied gradient evenly)
    rt = np.random.default_rng(20261203)  # own stream: the other files keep theirs
    at = rt.integers(-2, 3, size=(6, 7)).astype(np.float64)
    bt = rt.integers(-2, 3, size=(7,)).astype(np.float64)
    gt = rt.standard_normal((6, 7))
    d["a_tie"], d["b_tie"], d["g_tie"] = at, bt, gt
    for name, fn in {"maximum": torch.maximum, "minimum": torch.minimum}.items():
        ta, tb = t(at, True), t(bt, True)
        y = fn(ta, tb)
        y.backward(t(gt))
        d["tie_fwd_" + name], d["tie_ga_" + name], d["tie_gb_" + name] = y, ta.grad, tb.grad
    save("binary", **d)


def reductions(rng):
    x = rng.standard_normal((4, 5, 6))
    d = {"x": x}
    d["sum_all"] = t(x).sum()
    d["sum_1"] = t(x).sum(1)
    d["mean_02"] = t(x).mean((0, 2))
    d["max_2"] = t(x).amax(2)
    d["argmax_1"] = t(x).argmax(1).to(torch.int32)
    d["min_2"] = t(x).amin(2)
    d["min_0"] = t(x).amin(0)
    d["prod_1"] = t(x).prod(1)
    d["prod_all"] = t(x[:2, :3]).prod()
    d["argmin_1"] = t(x).argmin(1).to(torch.int32)
    d["argmin_all"] = t(x).argmin().to(torch.int32)
    xt = np.random.default_rng(20261204).integers(-2, 3, size=(5, 9)).astype(np.float64)
    # ties: the first index wins
    d["x_tie"] = xt
    d["tie_argmax_1"] = t(xt).argmax(1).to(torch.int32)
    d["tie_argmin_1"] = t(xt).argmin(1).to(torch.int32)
    d["tie_argmin_0"] = t(xt).argmin(0).to(torch.int32)
    ta = t(x, True)
    up = rng.standard_normal(5)
    ta.mean((0, 2)).backward(t(up))
    d["up_mean_02"] = up
    d["g_mean_02"] = ta.grad
    save("reduce", **d)


def softmax_losses(rng):
    x = rng.standard_normal((6, 10)) * 3
    g = rng.standard_normal((6, 10))
    tgt = np.array([3, 0, 9, -100, 5, 1])
    d = {"x": x, "g": g, "t": tgt}
    for name, fn in {"softmax": lambda v: torch.softmax(v, -1),
                     "log_softmax": lambda v: torch.log_softmax(v, -1)}.items():
        a = t(x, True)
        y = fn(a)
        y.backward(t(g))
        d["fwd_" + name], d["bwd_" + name] = y, a.grad
    for red in ("mean", "sum", "none"):
        a = t(x, True)
        loss = torch.nn.functional.cross_entropy(a, torch.tensor(tgt), reduction=red)
        gl = t(rng.standard_normal(6)) if red == "none" else t(1.7)
        loss.backward(gl)
        d["ce_" + red], d["ce_g_" + red], d["ce_dx_" + red] = loss, gl, a.grad
    a = t(x, True)
    lp = torch.log_softmax(a, -1)
    nll = torch.nn.functional.nll_loss(lp, torch.tensor(tgt))
    nll.backward()
    d["nll"], d["nll_dx"] = nll, a.grad
    save("softmax_losses", **d)


def layer_norm(rng):
    x = rng.standard_normal((5, 12)) * 2 + 1
    w = rng.standard_normal(12)
    b = rng.standard_normal(12)
    g = rng.standard_normal((5, 12))
    tx, tw, tb = t(x, True), t(w, True), t(b, True)
    y = torch.nn.functional.layer_norm(tx, (12,), tw, tb, 1e-5)
    y.backward(t(g))
    save("layer_norm", x=x, w=w, b=b, g=g, y=y, dx=tx.grad, dw=tw.grad, db=tb.grad)


def embedding_index(rng):
    w = rng.standard_normal((7, 4))
    ids = np.array([[1, 6, 1], [0, 1, 3]])
    g = rng.standard_normal((2, 3, 4))
    tw = t(w, True)
    y = torch.nn.functional.embedding(torch.tensor(ids), tw)
    y.backward(t(g))
    x = rng.standard_normal((4, 5))
    idx = np.array([4, 0, 4, 2])
    tx = t(x, True)
    ys = tx.index_select(1, torch.tensor(idx))
    gs = rng.standard_normal(ys.shape)
    ys.backward(t(gs))
    gidx = np.array([[0, 4, 4], [1, 1, 0], [3, 2, 2], [4, 0, 1]])
    tx2 = t(x, True)
    yg = torch.gather(tx2, 1, torch.tensor(gidx))
    gg = rng.standard_normal(yg.shape)
    yg.backward(t(gg))
    save("embedding_index", w=w, ids=ids, g=g, y=y, dw=tw.grad, x=x, idx=idx, ys=ys, gs=gs,
         dxs=tx.grad, gidx=gidx, yg=yg, gg=gg, dxg=tx2.grad)


def matmul_linear(rng):
    a = rng.standard_normal((2, 3, 4, 5))
    b = rng.standard_normal((3, 5, 6))
    g = rng.standard_normal((2, 3, 4, 6))
    ta, tb = t(a, True), t(b, True)
    y = ta @ tb
    y.backward(t(g))
    x = rng.standard_normal((2, 3, 5))
    w = rng.standard_normal((4, 5))
    bb = rng.standard_normal(4)
    gl = rng.standard_normal((2, 3, 4))
    tx, tw, tbb = t(x, True), t(w, True), t(bb, True)
    yl = torch.nn.functional.linear(tx, tw, tbb)
    yl.backward(t(gl))
    save("matmul_linear", a=a, b=b, g=g, y=y, ga=ta.grad, gb=tb.grad, x=x, w=w, bias=bb, gl=gl,
         yl=yl, dx=tx.grad, dw=tw.grad, dbias=tbb.grad)


def attention(rng):
    d = {}
    for causal in (False, True):
        q = rng.standard_normal((2, 3, 7, 8))
        k = rng.standard_normal((2, 3, 7, 8))
        v = rng.standard_normal((2, 3, 7, 8))
        g = rng.standard_normal((2, 3, 7, 8))
        tq, tk, tv = t(q, True), t(k, True), t(v, True)
        y = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal)
        y.backward(t(g))
        s = "c" if causal else "n"
        d.update({"q" + s: q, "k" + s: k, "v" + s: v, "g" + s: g, "y" + s: y, "dq" + s: tq.grad,
                  "dk" + s: tk.grad, "dv" + s: tv.grad})
    save("attention", **d)


def conv(rng):
    d = {}
    cases = {"a": dict(stride=1, padding=1, dilation=1, groups=1, cin=3, cout=4),
             "b": dict(stride=2, padding=1, dilation=1, groups=1, cin=4, cout=6),
             "c": dict(stride=1, padding=2, dilation=2, groups=2, cin=4, cout=6)}
    for s, c in cases.items():
        x = rng.standard_normal((2, c["cin"], 7, 6))
        w = rng.standard_normal((c["cout"], c["cin"] // c["groups"], 3, 3))
        b = rng.standard_normal(c["cout"])
        tx, tw, tb = t(x, True), t(w, True), t(b, True)
        y = torch.nn.functional.conv2d(tx, tw, tb, c["stride"], c["padding"], c["dilation"],
                                       c["groups"])
        g = rng.standard_normal(y.shape)
        y.backward(t(g))
        d.update({"x" + s: x, "w" + s: w, "b" + s: b, "g" + s: g, "y" + s: y, "dx" + s: tx.grad,
                  "dw" + s: tw.grad, "db" + s: tb.grad,
                  "cfg" + s: np.array([c["stride"], c["padding"], c["dilation"], c["groups"]])})
    save("conv2d", **d)


def optim(rng):
    d = {}
    for name, cls, wd in (("adam", torch.optim.Adam, 0.01), ("adamw", torch.optim.AdamW, 0.1)):
        p0 = rng.standard_normal(50)
        p = t(p0, True)
        opt = cls([p], lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
        gs = rng.standard_normal((3, 50))
        for i in range(3):
            p.grad = t(gs[i])
            opt.step()
        d.update({name + "_p0": p0, name + "_g": gs, name + "_p3": p})
    save("optim", **d)


def models(rng):
    """Tiny instances of the workloads through torch autograd."""
    d = {}
    # chain
    x = rng.standard_normal((8, 12))
    bias = rng.standard_normal(12)
    y = rng.uniform(-1, 1, (8, 12))
    tx, tb, ty = t(x, True), t(bias, True), t(y, True)
    loss = (torch.nn.functional.gelu(tx + tb) * ty).sum(0).mean()
    loss.backward()
    d.update(chain_x=x, chain_bias=bias, chain_y=y, chain_loss=loss, chain_dx=tx.grad,
             chain_dbias=tb.grad, chain_dy=ty.grad)
    # tiny GPT-2 (2 layers, d=16, 2 heads, vocab 23, ctx 8)
    V, C, D, H, Lr = 23, 8, 16, 2, 2
    P = {"wte.weight": rng.standard_normal((V, D)) * 0.1, "wpe.weight": rng.standard_normal((C, D)) * 0.1,
         "ln_f.weight": 1 + 0.1 * rng.standard_normal(D), "ln_f.bias": 0.1 * rng.standard_normal(D)}
    for i in range(Lr):
        pre = "h.%d." % i
        for nm, shp in (("ln_1.weight", (D,)), ("ln_1.bias", (D,)), ("attn.c_attn.weight", (3 * D, D)),
                        ("attn.c_attn.bias", (3 * D,)), ("attn.c_proj.weight", (D, D)),
                        ("attn.c_proj.bias", (D,)), ("ln_2.weight", (D,)), ("ln_2.bias", (D,)),
                        ("mlp.c_fc.weight", (4 * D, D)), ("mlp.c_fc.bias", (4 * D,)),
                        ("mlp.c_proj.weight", (D, 4 * D)), ("mlp.c_proj.bias", (D,))):
            base = 1.0 if nm.endswith("ln_1.weight") or nm.endswith("ln_2.weight") else 0.0
            P[pre + nm] = base + rng.standard_normal(shp) * 0.2
    T = {k: t(v, True) for k, v in P.items()}
    ids = rng.integers(0, V, size=(2, C + 1))
    F = torch.nn.functional
    inp, tgt = torch.tensor(ids[:, :-1]), torch.tensor(ids[:, 1:])
    h = F.embedding(inp, T["wte.weight"]) + T["wpe.weight"][:C][None]
    for i in range(Lr):
        pre = "h.%d." % i
        a = F.layer_norm(h, (D,), T[pre + "ln_1.weight"], T[pre + "ln_1.bias"])
        qkv = F.linear(a, T[pre + "attn.c_attn.weight"], T[pre + "attn.c_attn.bias"])
        q, k, v = qkv.split(D, 2)
        sh = lambda z: z.view(2, C, H, D // H).transpose(1, 2)
        o = F.scaled_dot_product_attention(sh(q), sh(k), sh(v), is_causal=True)
        o = o.transpose(1, 2).reshape(2, C, D)
        h = h + F.linear(o, T[pre + "attn.c_proj.weight"], T[pre + "attn.c_proj.bias"])
        a = F.layer_norm(h, (D,), T[pre + "ln_2.weight"], T[pre + "ln_2.bias"])
        m = F.linear(F.gelu(F.linear(a, T[pre + "mlp.c_fc.weight"], T[pre + "mlp.c_fc.bias"])),
                     T[pre + "mlp.c_proj.weight"], T[pre + "mlp.c_proj.bias"])
        h = h + m
    h = F.layer_norm(h, (D,), T["ln_f.weight"], T["ln_f.bias"])
    logits = F.linear(h, T["wte.weight"])
    loss = F.cross_entropy(logits.reshape(-1, V), tgt.reshape(-1))
    loss.backward()
    d["gpt_ids"] = ids
    d["gpt_cfg"] = np.array([V, C, D, H, Lr])
    d["gpt_loss"] = loss
    for k, v in P.items():
        d["gpt_p:" + k] = v
        d["gpt_g:" + k] = T[k].grad
    save("models", **d)


def losses_ext(rng):
    """cross_entropy with class weights and / or label smoothing and
    nll_loss with class weights, every reduction, one ignored row."""
    x = rng.standard_normal((7, 9)) * 2
    tgt = np.array([3, 0, 8, -100, 5, 1, 3])
    w = rng.uniform(0.2, 2.0, 9)
    d = {"x": x, "t": tgt, "w": w}
    for tag, kw in (("w", dict(weight=t(w))), ("ls", dict(label_smoothing=0.15)),
                    ("wls", dict(weight=t(w), label_smoothing=0.3))):
        for red in ("mean", "sum", "none"):
            a = t(x, True)
            loss = torch.nn.functional.cross_entropy(a, torch.tensor(tgt), reduction=red, **kw)
            gl = t(rng.standard_normal(7)) if red == "none" else t(0.8)
            loss.backward(gl)
            k = "ce_%s_%s" % (tag, red)
            d[k], d[k + "_g"], d[k + "_dx"] = loss, gl, a.grad
    lp = torch.log_softmax(t(x), -1).detach()
    for red in ("mean", "sum", "none"):
        a = lp.clone().requires_grad_(True)
        loss = torch.nn.functional.nll_loss(a, torch.tensor(tgt), weight=t(w), reduction=red)
        gl = t(rng.standard_normal(7)) if red == "none" else t(1.3)
        loss.backward(gl)
        k = "nll_w_" + red
        d["lp"], d[k], d[k + "_g"], d[k + "_dx"] = lp, loss, gl, a.grad
    save("losses_ext", **d)


def serialization_fixtures():
    """A PyTorch state_dict archive (torch.save) and a torch.js archive laid
    out as src/serialization/common.ts:22-75 writes it, each with the
    values a loader must produce (float32 / int32 / uint8 after the device's
    dtype mapping)."""
    import io
    import json
    import zipfile
    g = torch.Generator().manual_seed(5)
    base = torch.randn(10, generator=g, dtype=torch.float32)
    w = torch.nn.Parameter(torch.randn(3, 4, generator=g, dtype=torch.float32))
    tr = torch.randn(4, 3, generator=g, dtype=torch.float32).t()  # strides (1, 3)
    sd = collections.OrderedDict([
        ("layer.weight", w), ("ids", torch.arange(5, dtype=torch.int64) - 2),
        ("transposed", tr), ("slice", base[3:7]), ("half", torch.tensor([1.5, -2.25, 65504.0]).half()),
        ("bf16", torch.tensor([1.0, -3.140625, 0.0078125]).bfloat16()),
        ("mask", torch.tensor([True, False, True])),
        ("nested", {"list": [torch.ones(2, dtype=torch.float32), 7, "name"], "scale": 0.5})])
    buf = io.BytesIO()
    torch.save(sd, buf)
    with open(os.path.join(OUT, "state_dict.pt"), "wb") as f:
        f.write(buf.getvalue())
    exp = {"layer.weight": w.detach().numpy().astype(np.float32),
           "ids": (np.arange(5) - 2).astype(np.int32),
           "transposed": tr.numpy().astype(np.float32),
           "slice": base[3:7].numpy().astype(np.float32),
           "half": np.array([1.5, -2.25, 65504.0], np.float32),
           "bf16": np.array([1.0, -3.140625, 0.0078125], np.float32),
           "mask": np.array([1, 0, 1], np.uint8),
           "nested.list.0": np.ones(2, np.float32)}
    np.savez_compressed(os.path.join(OUT, "state_dict_expected.npz"), **exp)
    # torch.js layout: model.json with tensor metadata, tensors/<id>.bin
    meta = lambda i, shape, dt, rg=False: {"__tensor__": True, "id": str(i), "shape": shape,
                                          "dtype": dt, "requires_grad": rg, "device": "webgpu"}
    doc = {"model": {"fc.weight": meta(0, [2, 3], "float32", True),
                     "fc.bias": meta(1, [2], "float32", True)},
           "step": 12, "ids": meta(2, [4], "int32"), "h": meta(3, [2], "float16"),
           "flags": meta(4, [3], "bool"), "u": meta(5, [2], "uint32"),
           "hist": [meta(6, [2, 2], "int8"), "tag"]}
    bins = [np.arange(6, dtype="<f4").reshape(2, 3) / 4, np.array([-1.5, 2.0], "<f4"),
            np.array([3, -7, 0, 2 ** 30], "<i4"), np.array([0.5, -1.0], "<f4"),
            np.array([1, 0, 1], "u1"), np.array([7, 2 ** 31 - 1], "<u4"),
            np.array([[-128, 5], [0, 127]], "i1")]
    zb = io.BytesIO()
    with zipfile.ZipFile(zb, "w", zipfile.ZIP_DEFLATED) as z:
        # a fixed entry date, so that a rerun writes the same bytes
        def entry(name):
            return zipfile.ZipInfo(name, date_time=(2026, 12, 2, 3, 23, 0))
        z.writestr(entry("model.json"), json.dumps(doc, indent=2), zipfile.ZIP_DEFLATED)
        for i, a in enumerate(bins):
            z.writestr(entry("tensors/%d.bin" % i), a.tobytes(), zipfile.ZIP_DEFLATED)
    with open(os.path.join(OUT, "torchjs_archive.zip"), "wb") as f:
        f.write(zb.getvalue())


def multihead_attention(rng):
    """nn.MultiheadAttention in float64: self- and cross-attention, both
    layouts, bool / float / key-padding masks, the causal hint, weights
    averaged over heads and per head.  Parameters are stored under the
    reference's names (in_proj_weight, in_proj_bias, out_proj_weight,
    out_proj_bias; src/nn/attention.ts:38-95)."""
    E, H, N, L, S = 16, 4, 2, 5, 7
    d = {"E": E, "H": H}
    cases = [
        # name, batch_first, self, attn_mask kind, key_padding, causal, average
        ("self_sf", False, True, None, False, False, True),
        ("self_bf", True, True, None, False, False, False),
        ("cross_sf", False, False, "bool", True, False, True),
        ("cross_bf", True, False, "float3", True, False, False),
        ("causal_bf", True, True, "causal", False, True, True),
        ("kpm_sf", False, True, None, True, False, True),
    ]
    for name, bf, self_attn, mk, kpm, causal, avg in cases:
        m = torch.nn.MultiheadAttention(E, H, bias=True, batch_first=bf, dtype=torch.float64)
        Wi = rng.standard_normal((3 * E, E)) * 0.3
        bi = rng.standard_normal(3 * E) * 0.1
        Wo = rng.standard_normal((E, E)) * 0.3
        bo = rng.standard_normal(E) * 0.1
        with torch.no_grad():
            m.in_proj_weight.copy_(t(Wi))
            m.in_proj_bias.copy_(t(bi))
            m.out_proj.weight.copy_(t(Wo))
            m.out_proj.bias.copy_(t(bo))
        Lk = L if self_attn else S
        shp_q = (N, L, E) if bf else (L, N, E)
        shp_k = (N, Lk, E) if bf else (Lk, N, E)
        xq = rng.standard_normal(shp_q)
        if self_attn:
            q = t(xq, True)
            k = v = q
        else:
            q = t(xq, True)
            k = t(rng.standard_normal(shp_k), True)
            v = t(rng.standard_normal(shp_k), True)
        am = None
        if mk == "bool":
            am = rng.random((L, Lk)) < 0.3
            am[:, 0] = False  # no query row fully masked
        elif mk == "float3":
            am = rng.standard_normal((N * H, L, Lk))
        elif mk == "causal":
            am = np.triu(np.ones((L, Lk), dtype=bool), 1)
        kp = None
        if kpm:
            kp = np.zeros((N, Lk), dtype=bool)
            kp[0, -2:] = True
            kp[1, 1] = True
        out, w = m(q, k, v, key_padding_mask=None if kp is None else torch.tensor(kp),
                   need_weights=True,
                   attn_mask=None if am is None else (torch.tensor(am) if am.dtype == bool
                                                      else t(am)),
                   average_attn_weights=avg, is_causal=causal)
        g = rng.standard_normal(out.shape)
        out.backward(t(g))
        pre = name + ":"
        d.update({pre + "bf": bf, pre + "self": self_attn, pre + "causal": causal,
                  pre + "avg": avg, pre + "in_proj_weight": Wi, pre + "in_proj_bias": bi,
                  pre + "out_proj_weight": Wo, pre + "out_proj_bias": bo, pre + "query": xq,
                  pre + "g": g, pre + "out": out, pre + "weights": w,
                  pre + "d_in_proj_weight": m.in_proj_weight.grad,
                  pre + "d_in_proj_bias": m.in_proj_bias.grad,
                  pre + "d_out_proj_weight": m.out_proj.weight.grad,
                  pre + "d_out_proj_bias": m.out_proj.bias.grad, pre + "d_query": q.grad})
        if not self_attn:
            d.update({pre + "key": k, pre + "value": v, pre + "d_key": k.grad,
                      pre + "d_value": v.grad})
        if am is not None:
            d[pre + "attn_mask"] = am
        if kp is not None:
            d[pre + "key_padding_mask"] = kp
    save("mha", **d)


def second_order_functions(T, F):
    """f(inputs) -> scalar, written with calls torch and the hip package
    share; the second-derivative golden and its GPU test use the same
    definitions."""
    return {
        "elementwise": lambda x: ((x.tanh() * x.sigmoid()).sum()
                                  + (x.pow(3) / (x * x + 1.0)).mean()
                                  + (x.exp() * x.sin()).sum() + (x * x + 2.0).log().sum()
                                  + (x * x + 1.0).sqrt().sum() + x.cos().pow(2).sum()),
        "linear_gelu": lambda x, w, b: F.gelu(F.linear(x, w, b)).pow(2).sum(),
        "softmax": lambda x, w, t: (F.log_softmax(x @ w, -1) * t).sum()
        + F.softmax(x @ w, -1).pow(2).sum(),
        "broadcast": lambda x, y: ((x + y).exp().sin().sum() + (x * y).maximum(x - y).sum()
                                   + (x / (y * y + 1.0)).sum()),
        "views": lambda x: T.cat([x[0:2] * 2.0, x[2:5].relu() + x[2:5]], 0)
        .transpose(0, 1).reshape(-1).pow(2).sum() + x.permute(1, 0).mean(1).pow(3).sum(),
        "bmm": lambda x, w: (x @ w).tanh().pow(2).sum() + (x.sum(1, keepdim=True) * x).sum(),
        "layer_norm": lambda x, w, b: (F.layer_norm(x, (6,), w, b).pow(3).sum()
                                       + F.layer_norm(x, (6,)).tanh().sum()),
        "cross_entropy": lambda x: (F.cross_entropy(x, T.tensor([1, 0, 4, 2, 4]), label_smoothing=0.1)
                                    + F.cross_entropy(x * 2.0, T.tensor([3, 3, 0, 1, 2]),
                                                      reduction="sum")),
        "nll": lambda x: F.nll_loss(F.log_softmax(x, 1), T.tensor([0, 2, -100, 2])),
        "embedding": lambda w: F.embedding(T.tensor([3, 1, 3, 0]), w).pow(3).sum(),
        "sdpa": lambda q, k, v: F.scaled_dot_product_attention(q, k, v, is_causal=True).pow(2).sum(),
        "clamp_max": lambda x: ((x.clamp(-0.5, 0.8) * x).pow(2).sum() + x.amax(1).pow(2).sum()
                                + (x.triu(1) * x).sum()),
        "index": lambda x: (x.index_select(0, T.tensor([2, 0, 2])).pow(3).sum()
                            + x.gather(1, T.tensor([[0, 1], [2, 2], [1, 0]])).pow(2).sum()),
    }


SECOND_ORDER_SHAPES = {
    "elementwise": [(5, 7)], "linear_gelu": [(6, 5), (4, 5), (4,)],
    "softmax": [(6, 5), (5, 7), (6, 7)], "broadcast": [(4, 6), (6,)], "views": [(5, 3)],
    "bmm": [(2, 3, 4), (2, 4, 5)],
    "layer_norm": [(4, 6), (6,), (6,)], "cross_entropy": [(5, 5)], "nll": [(4, 3)],
    "embedding": [(5, 4)], "sdpa": [(1, 2, 5, 8)] * 3, "clamp_max": [(4, 5)], "index": [(3, 4)],
}
SECOND_ORDER_CONST = {"softmax": [2]}  # inputs that are constants (no gradient)


def second_order(rng):
    """First derivatives built with create_graph=True, then Hessian-vector
    products: grad of sum_i <grad_i, v_i> w.r.t. the inputs."""
    d = {}
    # the math attention backend: PyTorch's CPU flash kernel has no double
    # backward
    from torch.nn.attention import SDPBackend, sdpa_kernel
    ctx = sdpa_kernel(SDPBackend.MATH)
    ctx.__enter__()
    for name, fn in second_order_functions(torch, torch.nn.functional).items():
        const = SECOND_ORDER_CONST.get(name, [])
        xs = [rng.standard_normal(shp) * 0.7 for shp in SECOND_ORDER_SHAPES[name]]
        ts = [t(x, i not in const) for i, x in enumerate(xs)]
        var = [tt for i, tt in enumerate(ts) if i not in const]
        g1 = torch.autograd.grad(fn(*ts), var, create_graph=True)
        vs = [rng.standard_normal(tuple(g.shape)) for g in g1]
        dot = sum((g * t(v)).sum() for g, v in zip(g1, vs))
        h = torch.autograd.grad(dot, var)
        for i, x in enumerate(xs):
            d["%s:x%d" % (name, i)] = x
        for i, (g, v, hv) in enumerate(zip(g1, vs, h)):
            d["%s:g%d" % (name, i)] = g
            d["%s:v%d" % (name, i)] = v
            d["%s:h%d" % (name, i)] = hv
    ctx.__exit__(None, None, None)
    save("second_order", **d)


def main():
    serialization_fixtures()
    losses_ext(np.random.default_rng(20261202))
    rng = np.random.default_rng(20261201)
    unary_ops(rng)
    binary_ops(rng)
    reductions(rng)
    softmax_losses(rng)
    layer_norm(rng)
    embedding_index(rng)
    matmul_linear(rng)
    attention(rng)
    conv(rng)
    optim(rng)
    models(rng)
    multihead_attention(np.random.default_rng(20261205))
    second_order(np.random.default_rng(20261206))
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
