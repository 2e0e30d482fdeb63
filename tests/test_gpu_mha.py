"""nn.MultiheadAttention (src/nn/attention.ts:31-271) on the device against
the oracle (oracle/models.py mha_forward / mha_backward) and against the
torch float64 golden: output, attention weights and the gradient of every
parameter and input, both layouts, self- and cross-attention, bool / float
/ key-padding masks and the causal hint.  Tolerances: rtol 1e-4 / atol
1e-5 (GEMMs and attention reduce in a different order than the float64
oracle), with atol raised to 3x the float32 floor of the same computation
where that floor is larger (PyTorch's CPU float32 module on the same
inputs: the in_proj weight gradient sums products over every token, and
its elements near zero carry that sum's float32 rounding in any float32
implementation), plus a relative-norm bound of 1e-5 per tensor."""
import numpy as np
import pytest

from conftest import golden
from oracle import models as om

pytestmark = pytest.mark.gpu

RED = dict(rtol=1e-4, atol=1e-5)
PARAMS = ("in_proj_weight", "in_proj_bias", "out_proj_weight", "out_proj_bias")


def f32(a):
    return np.asarray(a, dtype=np.float32)


def check(got, want, what="", ref32=None):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    tol = dict(RED)
    if ref32 is not None:
        floor = float(np.nanmax(np.abs(np.asarray(ref32, dtype=np.float64) - want)))
        tol["atol"] = max(tol["atol"], 3.0 * floor)
    np.testing.assert_allclose(got, want, err_msg=what, **tol)
    nrm = np.linalg.norm(want)
    if nrm > 0:
        assert np.linalg.norm(got - want) / nrm <= 1e-5, what


def _cpu32(params, xs, kind, E, H, bf, g, **kw):
    """The same forward + backward through PyTorch's CPU float32 module:
    the float32 floor of each result (a library routine, not the oracle)."""
    import torch as cpu
    m = cpu.nn.MultiheadAttention(E, H, batch_first=bf)
    with cpu.no_grad():
        m.in_proj_weight.copy_(cpu.from_numpy(f32(params["in_proj_weight"])))
        m.in_proj_bias.copy_(cpu.from_numpy(f32(params["in_proj_bias"])))
        m.out_proj.weight.copy_(cpu.from_numpy(f32(params["out_proj_weight"])))
        m.out_proj.bias.copy_(cpu.from_numpy(f32(params["out_proj_bias"])))
    leaves = [cpu.tensor(f32(x), requires_grad=True) for x in xs]
    q = leaves[0]
    k = q if kind == "self" else leaves[1]
    v = k if kind in ("self", "kv") else leaves[2]
    kw = {a: (cpu.from_numpy(np.asarray(b)) if isinstance(b, np.ndarray) else b)
          for a, b in kw.items()}
    out, w = m(q, k, v, **kw)
    out.backward(cpu.from_numpy(f32(g)))
    grads = {"in_proj_weight": m.in_proj_weight.grad, "in_proj_bias": m.in_proj_bias.grad,
             "out_proj_weight": m.out_proj.weight.grad, "out_proj_bias": m.out_proj.bias.grad}
    grads = {n: t.numpy() for n, t in grads.items()}
    grads["inputs"] = [t.grad.numpy() for t in leaves]
    return out.detach().numpy(), (None if w is None else w.detach().numpy()), grads


def _module(torch, E, H, bf, params):
    m = torch.nn.MultiheadAttention(E, H, batch_first=bf)
    m.load_state_dict({k: torch.tensor(f32(v)) for k, v in params.items()})
    return m


def _params(r, E, scale=0.3):
    return {"in_proj_weight": f32(r.standard_normal((3 * E, E)) * scale / np.sqrt(E / 16)),
            "in_proj_bias": f32(r.standard_normal(3 * E) * 0.1),
            "out_proj_weight": f32(r.standard_normal((E, E)) * scale / np.sqrt(E / 16)),
            "out_proj_bias": f32(r.standard_normal(E) * 0.1)}


def _run(torch, m, xs, kind, g, **kw):
    """Forward + backward through the module; returns (out, weights, grads)."""
    leaves = [torch.tensor(x, requires_grad=True) for x in xs]
    q = leaves[0]
    k = q if kind == "self" else leaves[1]
    v = k if kind in ("self", "kv") else leaves[2]
    out, w = m(q, k, v, **kw)
    out.backward(torch.tensor(g))
    grads = {n: getattr(m, n).grad.numpy() for n in PARAMS}
    grads["inputs"] = [t.grad.numpy() for t in leaves]
    return out.numpy(), (None if w is None else w.numpy()), grads


SHAPES = [(256, 4, 2, 128, 128), (128, 4, 3, 96, 96), (256, 4, 2, 64, 160)]
CASES = [(shape, kind) for shape in SHAPES for kind in ("self", "kv", "qkv")
         if kind != "self" or shape[3] == shape[4]]  # self-attention has one length


@pytest.mark.parametrize("shape,kind", CASES)
@pytest.mark.parametrize("bf", [False, True])
@pytest.mark.parametrize("weights", [False, True])
def test_mha_against_oracle(torch, shape, kind, bf, weights):
    """Head dim 64 (flash kernels) and 32; self-attention (one fused
    projection GEMM), key is value (two GEMMs) and three inputs; weights
    averaged over heads when asked for."""
    E, H, N, L, S = shape
    r = np.random.default_rng(E + H + N + L + S + bf * 7 + len(kind) + weights)
    p = _params(r, E)
    shp = lambda T: (N, T, E) if bf else (T, N, E)
    xs = [f32(r.standard_normal(shp(L)))]
    if kind != "self":
        xs.append(f32(r.standard_normal(shp(S))))
    if kind == "qkv":
        xs.append(f32(r.standard_normal(shp(S))))
    m = _module(torch, E, H, bf, p)
    g = f32(r.standard_normal(shp(L)))
    out, w, got = _run(torch, m, xs, kind, g, need_weights=weights)
    q = xs[0]
    k = q if kind == "self" else xs[1]
    v = k if kind in ("self", "kv") else xs[2]
    want, wts, cache = om.mha_forward(p, q, k, v, H, batch_first=bf)
    o32, w32, r32 = _cpu32(p, xs, kind, E, H, bf, g, need_weights=weights)
    check(out, want, "out", o32)
    if weights:
        check(w, wts.mean(axis=1), "weights", w32)
    else:
        assert w is None
    gw = om.mha_backward(p, g, cache)
    for n in PARAMS:
        check(got[n], gw[n], n, r32[n])
    if kind == "self":
        check(got["inputs"][0], gw["query"] + gw["key"] + gw["value"], "d_x", r32["inputs"][0])
    elif kind == "kv":
        check(got["inputs"][0], gw["query"], "d_query", r32["inputs"][0])
        check(got["inputs"][1], gw["key"] + gw["value"], "d_kv", r32["inputs"][1])
    else:
        for i, n in enumerate(("query", "key", "value")):
            check(got["inputs"][i], gw[n], "d_" + n, r32["inputs"][i])


@pytest.mark.parametrize("bf", [False, True])
@pytest.mark.parametrize("masks", ["bool2", "float3", "kpm", "bool2+kpm", "causal"])
def test_mha_masks_against_oracle(torch, bf, masks):
    """PyTorch's mask meanings: a bool attn_mask [L, S] is True where
    attention is not allowed, a float one [N * H, L, S] is added, a
    key_padding_mask [N, S] masks keys per batch item; the causal hint
    with its mask runs the causal kernels (and the mask when weights are
    asked for)."""
    E, H, N, L, S = 256, 4, 2, 96, 96
    r = np.random.default_rng(len(masks) * 13 + bf)
    p = _params(r, E)
    shp = (N, L, E) if bf else (L, N, E)
    x = f32(r.standard_normal(shp))
    g = f32(r.standard_normal(shp))
    am = kp = None
    kw = {}
    if masks.startswith("bool2"):
        am = r.random((L, S)) < 0.3
        am[:, 0] = False
    elif masks == "float3":
        am = f32(r.standard_normal((N * H, L, S)))
    elif masks == "causal":
        am = np.triu(np.ones((L, S), dtype=bool), 1)
        kw["is_causal"] = True
    if "kpm" in masks:
        kp = np.zeros((N, S), dtype=bool)
        kp[0, -5:] = True
        kp[1, 3] = True
    m = _module(torch, E, H, bf, p)
    for weights in (False, True):
        for n in PARAMS:
            getattr(m, n).grad = None
        kwa = dict(kw, need_weights=weights, average_attn_weights=False)
        if am is not None:
            kwa["attn_mask"] = torch.tensor(am)
        if kp is not None:
            kwa["key_padding_mask"] = torch.tensor(kp)
        out, w, got = _run(torch, m, [x], "self", g, **kwa)
        mask = om.mha_mask(N, H, L, S, am, kp)
        want, wts, cache = om.mha_forward(p, x, x, x, H, batch_first=bf, mask=mask)
        kw32 = dict(kw, need_weights=weights, average_attn_weights=False, attn_mask=am,
                    key_padding_mask=kp)
        o32, w32, r32 = _cpu32(p, [x], "self", E, H, bf, g, **kw32)
        check(out, want, "out", o32)
        if weights:
            check(w, wts, "weights", w32)
        gw = om.mha_backward(p, g, cache)
        for n in PARAMS:
            check(got[n], gw[n], n, r32[n])
        check(got["inputs"][0], gw["query"] + gw["key"] + gw["value"], "d_x", r32["inputs"][0])


@pytest.mark.parametrize("case", ["self_sf", "self_bf", "cross_sf", "cross_bf", "causal_bf",
                                  "kpm_sf"])
def test_mha_torch_golden(torch, case):
    """The module against torch.nn.MultiheadAttention in float64 (the golden
    fixture), parameters loaded under the reference's names."""
    z = golden("mha")
    pre = case + ":"
    E, H = int(z["E"]), int(z["H"])
    bf, self_attn = bool(z[pre + "bf"]), bool(z[pre + "self"])
    p = {n: z[pre + n] for n in PARAMS}
    m = _module(torch, E, H, bf, p)
    xs = [f32(z[pre + "query"])]
    if not self_attn:
        xs += [f32(z[pre + "key"]), f32(z[pre + "value"])]
    kw = dict(need_weights=True, average_attn_weights=bool(z[pre + "avg"]),
              is_causal=bool(z[pre + "causal"]))
    if pre + "attn_mask" in z:
        kw["attn_mask"] = torch.tensor(z[pre + "attn_mask"] if z[pre + "attn_mask"].dtype == bool
                                       else f32(z[pre + "attn_mask"]))
    if pre + "key_padding_mask" in z:
        kw["key_padding_mask"] = torch.tensor(z[pre + "key_padding_mask"])
    out, w, got = _run(torch, m, xs, "self" if self_attn else "qkv", f32(z[pre + "g"]), **kw)
    check(out, z[pre + "out"], "out")
    check(w, z[pre + "weights"], "weights")
    for n in PARAMS:
        check(got[n], z[pre + "d_" + n], n)
    names = ("query",) if self_attn else ("query", "key", "value")
    for i, n in enumerate(names):
        check(got["inputs"][i], z[pre + "d_" + n], "d_" + n)


def test_mha_gpt2_shape_causal(torch):
    """Self-attention at GPT-2's shape (E 768, 12 heads of 64, T 1024,
    batch-first, causal hint): the flash kernels, against the oracle."""
    E, H, N, L = 768, 12, 2, 1024
    r = np.random.default_rng(11)
    p = {"in_proj_weight": f32(r.standard_normal((3 * E, E)) * 0.02),
         "in_proj_bias": f32(r.standard_normal(3 * E) * 0.02),
         "out_proj_weight": f32(r.standard_normal((E, E)) * 0.02),
         "out_proj_bias": f32(r.standard_normal(E) * 0.02)}
    x = f32(r.standard_normal((N, L, E)))
    g = f32(r.standard_normal((N, L, E)))
    m = _module(torch, E, H, True, p)
    causal = np.triu(np.ones((L, L), dtype=bool), 1)
    out, w, got = _run(torch, m, [x], "self", g, attn_mask=torch.tensor(causal), is_causal=True)
    assert w is None
    want, _, cache = om.mha_forward(p, x, x, x, H, batch_first=True, causal=True)
    o32, _, r32 = _cpu32(p, [x], "self", E, H, True, g, attn_mask=causal, is_causal=True,
                         need_weights=False)
    check(out, want, "out", o32)
    gw = om.mha_backward(p, g, cache)
    for n in PARAMS:
        check(got[n], gw[n], n, r32[n])
    check(got["inputs"][0], gw["query"] + gw["key"] + gw["value"], "d_x", r32["inputs"][0])


def test_mha_reference_init_and_errors(torch):
    """attention.ts:53-95: parameter shapes and names, randn * sqrt(1/E)
    weights from the seeded stream, zero biases; bias=False has none; the
    reference's constructor errors; is_causal needs attn_mask."""
    torch.manual_seed(5)
    m = torch.nn.MultiheadAttention(64, 8)
    names = [n for n, _ in m.named_parameters()]
    assert names == list(PARAMS)
    assert m.in_proj_weight.shape == (192, 64) and m.out_proj_weight.shape == (64, 64)
    assert not m.in_proj_bias.numpy().any() and not m.out_proj_bias.numpy().any()
    torch.manual_seed(5)
    w0 = (torch.randn(192, 64) * 0.125).numpy()  # sqrt(1 / 64)
    np.testing.assert_array_equal(m.in_proj_weight.numpy(), w0)
    nb = torch.nn.MultiheadAttention(64, 8, bias=False)
    assert [n for n, _ in nb.named_parameters()] == ["in_proj_weight", "out_proj_weight"]
    with pytest.raises(ValueError, match="divisible"):
        torch.nn.MultiheadAttention(10, 3)
    with pytest.raises(ValueError, match="greater than 0"):
        torch.nn.MultiheadAttention(0, 2)
    x = torch.randn(5, 2, 64)
    with pytest.raises(RuntimeError, match="is_causal"):
        m(x, x, x, is_causal=True)
    out, w = m(x, x, x)
    assert out.shape == (5, 2, 64) and w is None
