"""Pins the CPU oracle: golden vectors (PyTorch float64), the literal
known-answer tests of torch.js's own suite, closed forms, published error
bounds and finite differences.  CPU only."""
import math

import numpy as np
import pytest

from conftest import golden
from oracle import models as om
from oracle import ops, rng

RT, AT = 1e-9, 1e-12  # golden vectors vs float64 oracle


def close(a, b, rtol=RT, atol=AT):
    np.testing.assert_allclose(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64),
                               rtol=rtol, atol=atol)


# ------------------------------------------------------------------ golden


def test_unary_golden():
    z = golden("unary")
    for op in ["neg", "exp", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "relu", "square",
               "reciprocal", "abs", "sin", "cos", "silu", "softplus"]:
        x = z["xp"] if op in ("log", "sqrt", "rsqrt", "reciprocal") else z["x"]
        close(ops.unary(op, x), z["fwd_" + op])
        close(ops.unary_backward(op, z["g"], x), z["bwd_" + op])
    # erf / GELU follow the reference's A&S 7.1.26 erf: |error| <= 1.5e-7
    close(ops.unary("erf", z["x"]), z["fwd_erf"], rtol=0, atol=1.5e-7)
    close(ops.gelu(z["x"]), z["fwd_gelu"], rtol=0, atol=3 * 1.5e-7 * 1.5)
    close(ops.unary_backward("gelu", z["g"], z["x"]), z["bwd_gelu"], rtol=0,
          atol=1e-6 * np.abs(z["g"]).max())


@pytest.mark.parametrize("op,alpha", [("leaky_relu", 0.01), ("leaky_relu", 0.2), ("elu", 1.0),
                                      ("elu", 0.7)])
def test_unary_parametric_golden(op, alpha):
    z = golden("unary")
    key = "%s_%s" % (op, alpha)
    close(ops.unary(op, z["x"], alpha), z["fwd_" + key])
    close(ops.unary_backward(op, z["g"], z["x"], alpha), z["bwd_" + key])


def test_sign_golden():
    """sign, including 0, -0 and subnormal-sized inputs; its gradient is 0."""
    z = golden("unary")
    close(ops.unary("sign", z["x_sign"]), z["fwd_sign"], rtol=0, atol=0)
    close(ops.unary_backward("sign", z["g"], z["x_sign"]), z["bwd_sign"], rtol=0, atol=0)


def test_binary_golden():
    z = golden("binary")
    for op in ["add", "sub", "mul", "div", "pow", "maximum", "minimum"]:
        close(ops.binary(op, z["a"], z["b"]), z["fwd_" + op])
        ga, gb = ops.binary_backward(op, z["g"], z["a"], z["b"])
        close(ga, z["ga_" + op])
        close(gb, z["gb_" + op])


@pytest.mark.parametrize("op", ["maximum", "minimum"])
def test_maximum_minimum_ties_golden(op):
    """Integer operands with many ties: a tied gradient is split evenly."""
    z = golden("binary")
    assert (z["a_tie"] == z["b_tie"]).any()
    close(ops.binary(op, z["a_tie"], z["b_tie"]), z["tie_fwd_" + op], rtol=0, atol=0)
    ga, gb = ops.binary_backward(op, z["g_tie"], z["a_tie"], z["b_tie"])
    close(ga, z["tie_ga_" + op])
    close(gb, z["tie_gb_" + op])


def test_reduce_golden():
    z = golden("reduce")
    close(ops.reduce("sum", z["x"]), z["sum_all"])
    close(ops.reduce("sum", z["x"], [1]), z["sum_1"])
    close(ops.reduce("mean", z["x"], [0, 2]), z["mean_02"])
    close(ops.reduce_backward("mean", z["up_mean_02"], z["x"].shape, [0, 2]), z["g_mean_02"])
    close(ops.reduce("max", z["x"], [2]), z["max_2"])
    assert np.array_equal(ops.argmax(z["x"], 1), z["argmax_1"])
    close(ops.reduce("min", z["x"], [2]), z["min_2"], rtol=0, atol=0)
    close(ops.reduce("min", z["x"], [0]), z["min_0"], rtol=0, atol=0)
    close(ops.reduce("prod", z["x"], [1]), z["prod_1"])
    close(ops.reduce("prod", z["x"][:2, :3]), z["prod_all"])
    assert np.array_equal(ops.argmax(z["x"], 1, is_min=True), z["argmin_1"])
    assert ops.argmax(z["x"], None, is_min=True) == z["argmin_all"]
    # ties: the first extreme index (Tensor.ts:2568 keeps the first)
    xt = z["x_tie"]
    assert np.array_equal(ops.argmax(xt, 1), z["tie_argmax_1"])
    assert np.array_equal(ops.argmax(xt, 1, is_min=True), z["tie_argmin_1"])
    assert np.array_equal(ops.argmax(xt, 0, is_min=True), z["tie_argmin_0"])


def test_softmax_losses_golden():
    z = golden("softmax_losses")
    y = ops.softmax(z["x"])
    close(y, z["fwd_softmax"])
    close(ops.softmax_backward(z["g"], y), z["bwd_softmax"])
    ly = ops.log_softmax(z["x"])
    close(ly, z["fwd_log_softmax"])
    close(ops.log_softmax_backward(z["g"], ly), z["bwd_log_softmax"])
    for red in ("mean", "sum", "none"):
        close(ops.cross_entropy(z["x"], z["t"], red), z["ce_" + red])
        close(ops.cross_entropy_backward(z["x"], z["t"], z["ce_g_" + red], red), z["ce_dx_" + red])
    close(ops.nll_loss(ly, z["t"]), z["nll"])
    d = ops.nll_loss_backward(ly.shape, z["t"])
    close(ops.log_softmax_backward(d, ly), z["nll_dx"])


@pytest.mark.parametrize("tag", ["w", "ls", "wls"])
@pytest.mark.parametrize("red", ["mean", "sum", "none"])
def test_weighted_smoothed_losses_golden(tag, red):
    """Class weights (weighted mean) and label smoothing, PyTorch's contract."""
    z = golden("losses_ext")
    kw = {"w": dict(weight=z["w"]), "ls": dict(label_smoothing=0.15),
          "wls": dict(weight=z["w"], label_smoothing=0.3)}[tag]
    k = "ce_%s_%s" % (tag, red)
    close(ops.cross_entropy(z["x"], z["t"], red, **kw), z[k])
    close(ops.cross_entropy_backward(z["x"], z["t"], z[k + "_g"], red, **kw), z[k + "_dx"])
    k = "nll_w_" + red
    close(ops.nll_loss(z["lp"], z["t"], red, weight=z["w"]), z[k])
    close(ops.nll_loss_backward(z["lp"].shape, z["t"], z[k + "_g"], red, weight=z["w"]),
          z[k + "_dx"])


def test_batchmean_is_sum_over_rows():
    """apply_reduction's 'batchmean' (losses.ts:27-28): sum / rows, against
    the pinned 'sum' vectors."""
    z = golden("losses_ext")
    rows = len(z["t"])
    close(ops.cross_entropy(z["x"], z["t"], "batchmean", weight=z["w"]), z["ce_w_sum"] / rows)
    close(ops.cross_entropy_backward(z["x"], z["t"], 0.8 * rows, "batchmean", weight=z["w"]),
          z["ce_w_sum_dx"])


def test_layer_norm_golden():
    z = golden("layer_norm")
    y, _, _ = ops.layer_norm(z["x"], z["w"], z["b"])
    close(y, z["y"])
    dx, dw, db = ops.layer_norm_backward(z["g"], z["x"], z["w"])
    close(dx, z["dx"])
    close(dw, z["dw"])
    close(db, z["db"])


def test_embedding_index_golden():
    z = golden("embedding_index")
    close(ops.embedding(z["w"], z["ids"]), z["y"])
    close(ops.embedding_backward(z["g"], z["ids"], z["w"].shape[0]), z["dw"])
    close(ops.index_select(z["x"], 1, z["idx"]), z["ys"])
    close(ops.index_select_backward(z["gs"], z["x"].shape, 1, z["idx"]), z["dxs"])
    close(ops.gather(z["x"], 1, z["gidx"]), z["yg"])
    close(ops.scatter_add(z["x"].shape, 1, z["gidx"], z["gg"]), z["dxg"])


def test_matmul_linear_golden():
    z = golden("matmul_linear")
    close(z["a"] @ z["b"], z["y"])
    ga, gb = ops.matmul_backward(z["g"], z["a"], z["b"])
    close(ga, z["ga"])
    close(gb, z["gb"])
    close(ops.linear(z["x"], z["w"], z["bias"]), z["yl"])
    dx, dw, db = ops.linear_backward(z["gl"], z["x"], z["w"])
    close(dx, z["dx"])
    close(dw, z["dw"])
    close(db, z["dbias"])


@pytest.mark.parametrize("s,causal", [("n", False), ("c", True)])
def test_attention_golden(s, causal):
    z = golden("attention")
    o, _ = ops.sdpa(z["q" + s], z["k" + s], z["v" + s], causal=causal)
    close(o, z["y" + s])
    dq, dk, dv = ops.sdpa_backward(z["g" + s], z["q" + s], z["k" + s], z["v" + s], causal=causal)
    close(dq, z["dq" + s])
    close(dk, z["dk" + s])
    close(dv, z["dv" + s])


@pytest.mark.parametrize("s", ["a", "b", "c"])
def test_conv2d_golden(s):
    z = golden("conv2d")
    st, pad, dil, grp = (int(v) for v in z["cfg" + s])
    close(ops.conv2d(z["x" + s], z["w" + s], z["b" + s], st, pad, dil, grp), z["y" + s])
    dx, dw, db = ops.conv2d_backward(z["g" + s], z["x" + s], z["w" + s], st, pad, dil, grp)
    close(dx, z["dx" + s])
    close(dw, z["dw" + s])
    close(db, z["db" + s])


@pytest.mark.parametrize("name,decoupled,wd", [("adam", False, 0.01), ("adamw", True, 0.1)])
def test_optim_golden(name, decoupled, wd):
    """The float32-rounded oracle step tracks torch's float64 Adam/AdamW to
    float32 precision over 3 steps."""
    z = golden("optim")
    p = z[name + "_p0"].astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for i in range(3):
        p, m, v = ops.adam_step(p, z[name + "_g"][i], m, v, i + 1, lr=1e-2, weight_decay=wd,
                                decoupled=decoupled)
    close(p, z[name + "_p3"], rtol=1e-5, atol=1e-6)


def test_chain_golden():
    z = golden("models")
    loss, g = om.chain_loss_and_grads(z["chain_x"], z["chain_bias"], z["chain_y"])
    # GELU's A&S erf differs from exact erf by <= 1.5e-7
    close(loss, z["chain_loss"], rtol=0, atol=1e-6)
    close(g["x"], z["chain_dx"], rtol=0, atol=1e-7)
    close(g["bias"], z["chain_dbias"], rtol=0, atol=1e-6)
    close(g["y"], z["chain_dy"], rtol=0, atol=1e-7)


def test_gpt2_golden():
    z = golden("models")
    V, C, D, H, Lr = (int(v) for v in z["gpt_cfg"])
    cfg = om.Config(vocab=V, ctx=C, d=D, heads=H, layers=Lr)
    P = {k[6:]: z[k] for k in z if k.startswith("gpt_p:")}
    ids = z["gpt_ids"]
    loss, grads = om.gpt2_loss_and_grads(cfg, P, ids[:, :-1], ids[:, 1:])
    close(loss, z["gpt_loss"], rtol=0, atol=1e-6)
    for k in P:
        close(grads[k], z["gpt_g:" + k], rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ torch.js literal tests


def test_literal_matmul():
    """tests/browser.test.ts:19-26: [[1,2],[3,4]] @ [[5,6],[7,8]] = [[19,22],[43,50]]."""
    a = np.array([[1., 2.], [3., 4.]])
    b = np.array([[5., 6.], [7., 8.]])
    assert (a @ b).tolist() == [[19., 22.], [43., 50.]]
    ga, gb = ops.matmul_backward(np.ones((2, 2)), a, b)
    assert ga.tolist() == [[11., 15.], [11., 15.]]
    assert gb.tolist() == [[4., 4.], [6., 6.]]


def test_literal_grad_of_mul_and_sum():
    """tests/compatibility/tensor/tensor_backward.test.ts:11-19: d(2x)/dx = 2."""
    ga, _ = ops.binary_backward("mul", np.ones(3), np.array([1., 2., 3.]), np.array(2.))
    assert ga.tolist() == [2., 2., 2.]


def test_literal_exp_grad():
    """tensor_backward.test.ts:396-403: d exp(x)/dx at 1 = e."""
    assert abs(ops.unary_backward("exp", 1.0, 1.0) - math.e) < 1e-12


def test_literal_nll():
    """tests/compatibility/nn/functional.test.ts:144: nll_loss([[-0.1,-2,-3]], [0]) = 0.1;
    and :142 cross_entropy([[2,1,0.1]], [0]) > 0."""
    assert abs(ops.nll_loss(np.array([[-0.1, -2.0, -3.0]]), [0]) - 0.1) < 1e-12
    ce = ops.cross_entropy(np.array([[2.0, 1.0, 0.1]]), [0])
    assert ce > 0 and abs(ce - (math.log(math.exp(2) + math.exp(1) + math.exp(0.1)) - 2)) < 1e-12


def test_literal_one_hot():
    """tests/compatibility/nn/functional.test.ts:130-135: 3 classes and
    auto num_classes = max + 1."""
    assert ops.one_hot(np.array([0, 1, 2]), 3).reshape(-1).tolist() == [1, 0, 0, 0, 1, 0, 0, 0, 1]
    assert ops.one_hot(np.array([0, 2, 4])).shape == (3, 5)
    # Math.round ties go up; out-of-range rows stay zero (functional.ts:786-791)
    assert ops.one_hot(np.array([0.5, 2.4, -1, 7]), 4).tolist() == \
        [[0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 0], [0, 0, 0, 0]]


def test_literal_nonzero():
    """tests/compatibility/tensor/tensor_index.test.ts:305-328."""
    x = np.array([[0, 1, 0], [2, 0, 3]])
    assert ops.nonzero(x).tolist() == [[0, 1], [1, 0], [1, 2]]


def test_literal_argmax_first_on_ties():
    """Tensor.ts:2568 keeps the first maximum (`val > maxVal`)."""
    assert int(ops.argmax(np.array([1., 5., 5., 2.]))) == 1
    assert ops.argmax(np.array([[3., 3.], [1., 4.]]), 1).tolist() == [0, 1]


def test_index_select_rejects_out_of_range():
    """index_select follows PyTorch's contract (Tensor.ts:1242's @pytorch
    tag): indices outside [0, n) raise, negatives included (torch.js's WGSL
    reinterprets them as u32)."""
    x = np.arange(6.0).reshape(2, 3)
    with pytest.raises(IndexError):
        ops.index_select(x, 1, np.array([0, -1]))
    with pytest.raises(IndexError):
        ops.index_select(x, 0, np.array([2]))
    with pytest.raises(IndexError):
        ops.index_select_backward(np.ones((2, 1)), x.shape, 1, np.array([3]))


def test_literal_gather_negative_wrap():
    """Tensor.ts:2686-2687 wraps negative gather indices."""
    x = np.array([[1., 2., 3.]])
    assert ops.gather(x, 1, np.array([[-1, 0]])).tolist() == [[3., 1.]]


def test_literal_mse():
    """tests/compatibility/nn/losses.test.ts:70-73: MSE([1,2,3],[2,4,6]) = 14/3."""
    a = np.array([1., 2., 3.])
    b = np.array([2., 4., 6.])
    assert abs(((a - b) ** 2).mean() - 14 / 3) < 1e-12


def test_pow_scalar_integer_rule():
    """scalar.wgsl:53-66: integer exponents 0..10 by repeated multiply."""
    assert ops.pow_scalar(np.array([3.0]), 2)[0] == 9.0
    assert ops.pow_scalar(np.array([2.0]), 0)[0] == 1.0
    assert abs(ops.pow_scalar(np.array([2.0]), 0.5)[0] - math.sqrt(2)) < 1e-15


# ------------------------------------------------------------------ closed forms / bounds


def test_erf_as_published_bound_and_symmetry():
    x = np.linspace(-6, 6, 20001)
    err = np.abs(ops.erf_as(x) - np.array([math.erf(v) for v in x]))
    assert err.max() <= 1.5e-7  # A&S 7.1.26
    assert np.allclose(ops.erf_as(-x), -ops.erf_as(x), rtol=0, atol=0)


def test_gelu_closed_forms():
    assert ops.gelu(0.0) == 0.0
    assert abs(ops.gelu_grad(0.0) - 0.5) < 1e-7
    assert abs(ops.gelu(10.0) - 10.0) < 1e-12
    assert abs(ops.gelu(-10.0)) < 1e-20
    # gelu' = d/dx gelu by central differences (away from the A&S ripple)
    x = np.linspace(-4, 4, 41)
    h = 1e-5
    fd = (ops.gelu(x + h) - ops.gelu(x - h)) / (2 * h)
    assert np.allclose(ops.gelu_grad(x), fd, atol=2e-6)


def test_softmax_ce_closed_forms():
    c = 7
    x = np.full((3, c), 2.5)
    assert np.allclose(ops.softmax(x), 1.0 / c)
    assert abs(ops.cross_entropy(x, [0, 3, 6]) - math.log(c)) < 1e-12
    x = np.random.default_rng(1).standard_normal((5, c))
    g = ops.cross_entropy_backward(x, [0, 1, 2, 3, 4])
    assert np.allclose(g.sum(axis=1), 0.0, atol=1e-15)
    assert np.allclose(ops.softmax(x).sum(axis=1), 1.0)


def test_minus_inf_logits():
    """A -inf logit is a class with probability 0 (PyTorch's softmax and
    cross_entropy give exactly that, checked here): softmax 0, log-softmax
    -inf, no NaN in the loss or its gradient."""
    import torch as cpu
    x = np.array([[1.0, -np.inf, 2.0, 0.5], [-np.inf, 3.0, -np.inf, -np.inf]])
    t = np.array([2, 1])
    xt = cpu.tensor(x, requires_grad=True)
    lt = cpu.nn.functional.cross_entropy(xt, cpu.tensor(t))
    lt.backward()
    close(ops.softmax(x), cpu.softmax(cpu.tensor(x), -1).numpy())
    assert np.array_equal(np.isneginf(ops.log_softmax(x)), np.isneginf(x))
    close(ops.cross_entropy(x, t), lt.item())
    close(ops.cross_entropy_backward(x, t), xt.grad.numpy())
    assert ops.softmax(x)[1, 1] == 1.0


def test_layer_norm_invariants():
    x = np.random.default_rng(2).standard_normal((4, 33)) * 5 + 3
    y, _, _ = ops.layer_norm(x)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-12)
    assert np.allclose((y ** 2).mean(axis=1), 1, atol=1e-5)


def test_adam_first_step_sign():
    """Adam's first step moves each parameter by ~lr*sign(g) (m_hat/sqrt(v_hat) = +-1)."""
    p = np.zeros(5, np.float32)
    g = np.array([3., -2., 1e-3, -7., 0.5], np.float32)
    p1, _, _ = ops.adam_step(p, g, np.zeros(5, np.float32), np.zeros(5, np.float32), 1, lr=0.1)
    assert np.allclose(p1, -0.1 * np.sign(g), rtol=1e-5)


def test_conv_delta_kernel_is_shift():
    x = np.random.default_rng(3).standard_normal((1, 1, 5, 5))
    w = np.zeros((1, 1, 3, 3))
    w[0, 0, 0, 0] = 1.0  # picks x[i-1, j-1] with padding 1
    y = ops.conv2d(x, w, None, 1, 1)
    assert np.allclose(y[0, 0, 1:, 1:], x[0, 0, :-1, :-1])
    assert np.allclose(y[0, 0, 0, :], 0)


def _fd_check(f, x, g_analytic, eps=1e-6, n=12, seed=0):
    r = np.random.default_rng(seed)
    flat = x.reshape(-1)
    for i in r.choice(flat.size, size=min(n, flat.size), replace=False):
        old = flat[i]
        flat[i] = old + eps
        fp = f()
        flat[i] = old - eps
        fm = f()
        flat[i] = old
        fd = (fp - fm) / (2 * eps)
        assert abs(fd - g_analytic.reshape(-1)[i]) <= 1e-5 * max(1.0, abs(fd)), (i, fd)


def test_finite_differences_block():
    """The transformer-block backward against central differences."""
    r = np.random.default_rng(4)
    d, heads = 8, 2
    p = om.block_params(d, r, std=0.3)
    p = {k: v.astype(np.float64) for k, v in p.items()}
    x = r.standard_normal((2, 5, d))
    loss, g = om.block_loss_and_grads(p, x, heads)
    _fd_check(lambda: om.block_loss_and_grads(p, x, heads)[0], x, g["x"])
    w = p["attn.c_attn.weight"]
    _fd_check(lambda: om.block_loss_and_grads(p, x, heads)[0], w, g["attn.c_attn.weight"])


def test_finite_differences_cnn_mlp():
    r = np.random.default_rng(5)
    p = {"conv1.weight": r.standard_normal((4, 3, 3, 3)) * 0.3, "conv1.bias": r.standard_normal(4) * 0.1,
         "conv2.weight": r.standard_normal((5, 4, 3, 3)) * 0.3, "conv2.bias": r.standard_normal(5) * 0.1,
         "fc.weight": r.standard_normal((3, 5)) * 0.3, "fc.bias": r.standard_normal(3) * 0.1}
    x = r.standard_normal((2, 3, 6, 6))
    t = np.array([0, 2])
    loss, g = om.cnn_loss_and_grads(p, x, t)
    for k in ("conv1.weight", "conv2.weight", "fc.bias"):
        _fd_check(lambda: om.cnn_loss_and_grads(p, x, t)[0], p[k], g[k])
    pm = {"0.weight": r.standard_normal((6, 7)), "0.bias": r.standard_normal(6),
          "2.weight": r.standard_normal((4, 6)), "2.bias": r.standard_normal(4)}
    xm = r.standard_normal((3, 7))
    tm = np.array([1, 3, 0])
    loss, g = om.mlp_loss_and_grads(pm, xm, tm)
    _fd_check(lambda: om.mlp_loss_and_grads(pm, xm, tm)[0], pm["0.weight"], g["0.weight"])


# ------------------------------------------------------------------ rng


def test_lcg_known_answers_js_doubles():
    """creation.ts:921 evaluated as JavaScript does.  The expected states are
    those of the IEEE-double definition: globalSeed*1103515245 is rounded to
    a double (it exceeds 2^53 from the third draw on), 12345 is added in
    double precision, ToInt32 and & 0x7fffffff keep the low 31 bits.  From
    manual_seed(1234) that gives 233191843, 128476320, 85706848,
    2116141344; exact integer arithmetic would give 85706841 third."""
    s, seen = 1234, []
    for _ in range(4):
        s = rng.lcg_next(s)
        seen.append(s)
    assert seen == [233191843, 128476320, 85706848, 2116141344]
    assert (128476320 * 1103515245 + 12345) & 0x7FFFFFFF == 85706841  # the integer result
    assert rng.lcg_next(0) == 12345
    # the generator's seed stream follows the same steps
    g = rng.Generator(1234)
    assert [g._next() for _ in range(4)] == seen


def test_xorshift32_published_known_answer():
    """Marsaglia, "Xorshift RNGs" (J. Stat. Softw. 8(14), 2003): the (13,17,5)
    generator from y = 2463534242 returns 723471715 first; random.wgsl:9-15
    uses the same shifts."""
    assert int(rng.xorshift32(2463534242)) == 723471715
    # shifts, not rotations: the top bits fall off (x=2^31 -> 2^31 ^ 2^14 ^ ...)
    assert int(rng.xorshift32(0)) == 0


def test_rng_integer_streams():
    """Per-element states and the float maps of random.wgsl:17-46."""
    u = rng.rand(1000, 42)
    assert u.min() >= 0 and u.max() < 1 and abs(u.mean() - 0.5) < 0.05
    n = rng.randn(20000, 7)
    assert abs(n.mean()) < 0.05 and abs(n.std() - 1) < 0.05


def _xs_inverse(y):
    """Inverse of xorshift32 (13, 17, 5): each step x ^= x << k (or >> k)
    is undone by repeating it until the shifted-in bits settle."""
    def unshift(y, k, left):
        x = y
        for _ in range(32 // k + 1):
            x = (y ^ ((x << k) & 0xFFFFFFFF)) if left else (y ^ (x >> k))
        return x
    return unshift(unshift(unshift(y, 5, True), 17, False), 13, True)


def _seed_for_states(s2):
    """The call seed whose element 0 has second state s2 (and first state
    s1 = xorshift32^-1(s2)): element 0 starts from seed ^ 1013904223."""
    s1 = _xs_inverse(s2)
    return _xs_inverse(s1) ^ 1013904223, s1


def test_xorshift_inverse():
    for y in (1, 2 ** 30, 2 ** 31, 0xDEADBEEF, 723471715):
        assert int(rng.xorshift32(_xs_inverse(y))) == y
    assert _xs_inverse(723471715) == 2463534242  # Marsaglia's known pair


def test_randn_box_muller_special_states():
    """random.wgsl:31-46 at states whose result the mathematics fixes,
    computed with math.log / math.cos on the float32 inputs:
    - u2 = 1/2 (s2 = 2^31): the angle is float32(2 pi) / 2 = pi + 8.7e-8, cos
      = -1 to double precision, so the output is -sqrt(-2 ln u1);
    - u2 = 1/4 (s2 = 2^30): cos of float32(2 pi) / 4 is -4.37e-8, so the
      output is ~0 (a sine in place of the cosine would give sqrt(-2 ln u1),
      and u1, u2 swapped would give neither);
    - u1 below 1e-7 (s1 < 430): u1 is clamped to float32(1e-7), so the
      radius is sqrt(-2 ln float32(1e-7)) = 5.677, whatever u1 is."""
    for s2, cos_want in ((2 ** 31, -1.0), (2 ** 30, math.cos(float(np.float32(2 * math.pi)) / 4))):
        seed, s1 = _seed_for_states(s2)
        u1 = float(np.float32(s1 / 2 ** 32))
        r = math.sqrt(-2.0 * math.log(u1))
        want = r * cos_want
        assert abs(float(rng.randn(1, seed)[0]) - want) <= 1e-7 * r
        if s2 == 2 ** 30:
            assert abs(want) < 1e-7 and r > 1.0  # a sine would give r
    r_clamp = math.sqrt(-2.0 * math.log(float(np.float32(1e-7))))
    assert abs(r_clamp - 5.6777) < 1e-4
    # among the states with u1 < 1e-7, the one whose u2 puts the angle
    # nearest a multiple of pi: the output is then +-r_clamp
    best = max(range(1, 430), key=lambda s1: abs(math.cos(
        float(np.float32(np.float32(2 * math.pi) * np.float32(int(rng.xorshift32(s1)) / 2 ** 32))))))
    seed = _xs_inverse(best) ^ 1013904223
    u2 = float(np.float32(int(rng.xorshift32(best)) / 2 ** 32))
    theta = float(np.float32(np.float32(2 * math.pi) * np.float32(u2)))
    got = float(rng.randn(1, seed)[0])
    assert abs(abs(math.cos(theta)) - 1.0) < 1e-3
    assert abs(got - r_clamp * math.cos(theta)) <= 1e-6
    # without the clamp the radius would be sqrt(-2 ln(best / 2^32)) > 6.3
    assert math.sqrt(-2.0 * math.log(best / 2 ** 32)) > 6.3


# ------------------------------------------------------------------ sampling


def test_multinomial_inverse_cdf_against_searchsorted():
    """With replacement the oracle is the inverse CDF of the normalised
    weights: numpy's searchsorted on their cumulative sum (a library
    routine) gives the same indices."""
    r = np.random.default_rng(9)
    x = r.random((4, 37))
    x[1, ::3] = -1.0  # negative weights count as 0
    u = r.random((4, 25))
    got = ops.multinomial(x, 25, True, u)
    for i in range(4):
        p = np.where(x[i] > 0, x[i], 0.0)
        want = np.searchsorted(np.cumsum(p / p.sum()), u[i], side="right")
        assert np.array_equal(got[i], np.minimum(want, 36))


def test_multinomial_closed_forms():
    # a one-hot row always draws its index; an all-zero row is uniform:
    # draw u lands in bucket floor(u * C)
    u = np.array([[0.0, 0.3, 0.99999]])
    assert ops.multinomial(np.eye(5)[3], 3, True, u).tolist() == [3, 3, 3]
    assert ops.multinomial(np.zeros(4), 3, True, u).tolist() == [0, 1, 3]
    # without replacement: distinct indices; all C of them is a permutation
    r = np.random.default_rng(4)
    x = r.random((3, 9))
    perm = ops.multinomial(x, 9, False, r.random((3, 9)))
    assert all(sorted(row) == list(range(9)) for row in perm.tolist())
    # zero-weight categories come last without replacement
    x = np.array([0.0, 2.0, 0.0, 1.0])
    got = ops.multinomial(x, 4, False, np.array([0.1, 0.9, 0.5, 0.5]))
    assert sorted(got[:2].tolist()) == [1, 3] and sorted(got[2:].tolist()) == [0, 2]
    # the reference's literal test (tests/gpt2.test.ts:123-131): an index in [0, vocab)
    p = ops.softmax(np.random.default_rng(1).standard_normal(100))
    t = int(ops.multinomial(p, 1, False, np.array([0.42]))[0])
    assert 0 <= t < 100


def test_multinomial_nan_and_inf_contract():
    """NaN or +inf in a row raises (PyTorch's torch.multinomial raises on
    both); -inf and negatives weigh 0 like Math.max(0, x) makes them."""
    u = np.array([[0.5, 0.5]])
    for bad in (np.nan, np.inf):
        with pytest.raises(ValueError, match="row 0"):
            ops.multinomial(np.array([1.0, bad, 1.0]), 2, True, u)
        with pytest.raises(ValueError):
            ops.multinomial(np.array([1.0, bad, 1.0]), 2, False, u)
        import torch
        with pytest.raises(RuntimeError):
            torch.multinomial(torch.tensor([1.0, bad, 1.0]), 2, True)
    # -inf weighs 0: only indices 0 and 2 can be drawn, 2 for u >= 0.5
    got = ops.multinomial(np.array([1.0, -np.inf, 1.0]), 2, True, np.array([0.25, 0.75]))
    assert got.tolist() == [0, 2]


def test_multinomial_distribution():
    """Many draws reproduce the weights (chi-square, 5 dof, p ~ 1e-6 bound)."""
    r = np.random.default_rng(2)
    w = np.array([1.0, 2.0, 3.0, 0.5, 0.5, 3.0])
    draws = ops.multinomial(w, 20000, True, r.random(20000))
    cnt = np.bincount(draws, minlength=6)
    exp = 20000 * w / w.sum()
    assert ((cnt - exp) ** 2 / exp).sum() < 35.0



# ------------------------------------------------------------------ MultiheadAttention


MHA_CASES = ["self_sf", "self_bf", "cross_sf", "cross_bf", "causal_bf", "kpm_sf"]


@pytest.mark.parametrize("case", MHA_CASES)
def test_mha_golden(case):
    """oracle mha_forward / mha_backward against torch.nn.MultiheadAttention
    in float64: output, weights (averaged over heads or per head), and the
    gradient of every parameter and input."""
    z = golden("mha")
    pre = case + ":"
    H = int(z["H"])
    bf, self_attn = bool(z[pre + "bf"]), bool(z[pre + "self"])
    p = {k: z[pre + k] for k in ("in_proj_weight", "in_proj_bias", "out_proj_weight",
                                 "out_proj_bias")}
    q = z[pre + "query"]
    k = q if self_attn else z[pre + "key"]
    v = q if self_attn else z[pre + "value"]
    N = q.shape[0] if bf else q.shape[1]
    L = q.shape[1] if bf else q.shape[0]
    S = k.shape[1] if bf else k.shape[0]
    mask = om.mha_mask(N, H, L, S, z.get(pre + "attn_mask"), z.get(pre + "key_padding_mask"))
    out, w, cache = om.mha_forward(p, q, k, v, H, batch_first=bf, mask=mask)
    close(out, z[pre + "out"])
    close(w.mean(axis=1) if bool(z[pre + "avg"]) else w, z[pre + "weights"])
    g = om.mha_backward(p, z[pre + "g"], cache)
    for name in ("in_proj_weight", "in_proj_bias", "out_proj_weight", "out_proj_bias"):
        close(g[name], z[pre + "d_" + name])
    if self_attn:
        close(g["query"] + g["key"] + g["value"], z[pre + "d_query"])
    else:
        for name in ("query", "key", "value"):
            close(g[name], z[pre + "d_" + name])


def test_mha_causal_flag_equals_causal_mask():
    """The causal flag of the oracle's attention equals an explicit -inf
    upper-triangle mask (the causal golden case uses the mask)."""
    r = np.random.default_rng(3)
    q, k, v = (r.standard_normal((2, 3, 6, 8)) for _ in range(3))
    m = np.where(np.triu(np.ones((6, 6), dtype=bool), 1), -np.inf, 0.0)
    close(ops.sdpa(q, k, v, causal=True)[0], ops.sdpa(q, k, v, mask=m)[0])
    g = r.standard_normal((2, 3, 6, 8))
    for a, b in zip(ops.sdpa_backward(g, q, k, v, causal=True),
                    ops.sdpa_backward(g, q, k, v, mask=m)):
        close(a, b)
