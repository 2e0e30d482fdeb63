"""The operator surface above the kernels on the MI355X: torch.autograd's
grad / vjp / jvp / Function (the literal tests of torch.js's
tests/compatibility/autograd/autograd.test.ts), cat / stack / expand and
their gradients, cross_entropy with class weights and label smoothing,
and nn.init.  Values are checked against the oracle or the reference's
literal expectations."""
import math

import numpy as np
import pytest

from oracle import ops, rng

pytestmark = pytest.mark.gpu

RED = dict(rtol=1e-4, atol=1e-5)
EW = dict(rtol=1e-5, atol=1e-6)


def f32(a):
    return np.asarray(a, dtype=np.float32)


def check(got, want, **tol):
    np.testing.assert_allclose(np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64),
                               **tol)


# ------------------------------------------------------------ torch.autograd
# autograd.test.ts:11-56 (grad), :59-105 (vjp), :107-150 (jvp), :153-228
# (Function); toBeCloseTo(v, 4) is |got - v| < 5e-5.

def close4(got, want):
    assert np.all(np.abs(np.asarray(got, dtype=np.float64) - np.asarray(want)) < 5e-5), (got, want)


def test_autograd_grad_literals(torch):
    x = torch.tensor([2.0, 3.0], requires_grad=True)
    (g,) = torch.autograd.grad(x.pow(2).sum(), x)
    close4(g.toArray(), [4.0, 6.0])                       # :12-20
    x = torch.tensor([2.0, 3.0], requires_grad=True)
    (g,) = torch.autograd.grad(x.pow(2), x, torch.tensor([1.0, 2.0]))
    close4(g.toArray(), [4.0, 12.0])                      # :22-31
    x = torch.tensor([1.0, 2.0], requires_grad=True)
    w = torch.tensor([3.0, 4.0], requires_grad=True)
    gx, gw = torch.autograd.grad(x.mul(w).sum(), [x, w])
    close4(gx.toArray(), [3.0, 4.0])                      # :33-45
    close4(gw.toArray(), [1.0, 2.0])
    # grad leaves .grad untouched
    assert x.grad is None and w.grad is None
    # second order with create_graph (autograd.test.ts:47-55): d2(x^3)/dx2 = 6x = 12
    x = torch.tensor([2.0], requires_grad=True)
    y = x.pow(3)
    (g1,) = torch.autograd.grad(y, x, torch.ones_like(y), True, True)
    close4(g1.toArray(), [12.0])
    assert g1.requires_grad and g1.grad_fn is not None
    (g2,) = torch.autograd.grad(g1, x, torch.ones_like(g1))
    close4(g2.toArray(), [12.0])
    # and a third: d3/dx3 = 6
    x = torch.tensor([2.0], requires_grad=True)
    (g1,) = torch.autograd.grad(x.pow(3), x, create_graph=True)
    (g2,) = torch.autograd.grad(g1, x, create_graph=True)
    (g3,) = torch.autograd.grad(g2, x)
    close4(g3.toArray(), [6.0])
    # backward(create_graph=True): the leaf's .grad carries a graph
    x = torch.tensor([1.5, -0.5], requires_grad=True)
    (x.exp() * x).sum().backward(create_graph=True)
    gx = x.grad
    assert gx.grad_fn is not None
    (h,) = torch.autograd.grad(gx.sum(), x)
    xv = np.array([1.5, -0.5])
    close4(h.toArray(), list(np.exp(xv) * (xv + 2)))       # (x e^x)'' = e^x (x + 2)
    # an op with no differentiable backward says so
    x = torch.tensor(np.ones((1, 1, 4, 4), np.float32), requires_grad=True)
    w = torch.tensor(np.ones((1, 1, 3, 3), np.float32), requires_grad=True)
    with pytest.raises(NotImplementedError, match="Conv2d"):
        torch.autograd.grad(torch.F.conv2d(x, w).pow(2).sum(), x, create_graph=True)


def test_autograd_vjp_literals(torch):
    out, v = torch.autograd.vjp(lambda t: t.pow(2), torch.tensor([1.0, 2.0], requires_grad=True),
                                torch.tensor([1.0, 1.0]))
    close4(out.toArray(), [1.0, 4.0])                     # :60-75
    close4(v.toArray(), [2.0, 4.0])

    def f(t):  # [x0 + x1, x1 + x2]
        return torch.cat([t[0:2].sum(-1, True), t[1:3].sum(-1, True)])
    _, v = torch.autograd.vjp(f, torch.tensor([1.0, 2.0, 3.0], requires_grad=True),
                              torch.tensor([1.0, 1.0]))
    close4(v.toArray(), [1.0, 2.0, 1.0])                  # :77-91
    x = torch.tensor([2.0], requires_grad=True)
    _, v = torch.autograd.vjp(lambda t: t.pow(3), x, torch.tensor([1.0]), True)
    close4(v.toArray(), [12.0])                           # :93-105
    # with create_graph the product differentiates again: d(3x^2)/dx = 12
    (h,) = torch.autograd.grad(v, x)
    close4(h.toArray(), [12.0])


def test_autograd_jvp_literals(torch):
    out, j = torch.autograd.jvp(lambda t: t.pow(2), torch.tensor([1.0, 2.0], requires_grad=True),
                                torch.tensor([3.0, 4.0]))
    close4(out.toArray(), [1.0, 4.0])                     # :108-122
    close4(j.toArray(), [6.0, 16.0])
    _, j = torch.autograd.jvp(lambda t: t.sum(-1, True), torch.tensor([1.0, 2.0, 3.0]),
                              torch.tensor([1.0, 1.0, 1.0]))
    close4(j.toArray(), [3.0])                            # :124-135
    _, j = torch.autograd.jvp(lambda t: t.pow(2).sum(-1, True), torch.tensor([2.0, 3.0]),
                              torch.tensor([1.0, 0.0]))
    close4(j.toArray(), [4.0])                            # :137-149


SECOND_ORDER = ["elementwise", "linear_gelu", "softmax", "broadcast", "views", "bmm",
                "layer_norm", "cross_entropy", "nll", "embedding", "sdpa", "clamp_max", "index"]


@pytest.mark.parametrize("name", SECOND_ORDER)
def test_second_order_golden(torch, name):
    """First derivatives built with create_graph=True and Hessian-vector
    products (the gradient of sum_i <grad_i, v_i>) against PyTorch in
    float64 (tests/golden/second_order.npz), through the unary, binary
    (broadcast), scalar, reduction, view, cat / narrow, matmul, Linear and
    softmax ops.  The functions are the ones the golden was written from."""
    from conftest import golden
    z = golden("second_order")
    fn = _second_order_functions(torch)[name]
    xs = [z["%s:x%d" % (name, i)] for i in range(8) if "%s:x%d" % (name, i) in z]
    const = {"softmax": [2]}.get(name, [])
    ts = [torch.tensor(f32(x), requires_grad=i not in const) for i, x in enumerate(xs)]
    var = [t for i, t in enumerate(ts) if i not in const]
    g1 = torch.autograd.grad(fn(*ts), var, create_graph=True)
    for i, g in enumerate(g1):
        check(g.numpy(), z["%s:g%d" % (name, i)], **RED)
    dot = None
    for i, g in enumerate(g1):
        term = (g * torch.tensor(f32(z["%s:v%d" % (name, i)]))).sum()
        dot = term if dot is None else dot + term
    h = torch.autograd.grad(dot, var)
    for i, hv in enumerate(h):
        check(hv.numpy(), z["%s:h%d" % (name, i)], **RED)


@pytest.mark.parametrize("which", ["mlp", "linear_add", "embedding_pos"])
def test_second_order_fused_ops_equal_composites(torch, which):
    """create_graph through the fused ops the GPT-2 model runs (the GELU
    MLP, the projection with its residual add, the token + position
    embedding): gradients and Hessian-vector products equal those of the
    same function written with the public ops."""
    F = torch.F
    r = np.random.default_rng(7)
    if which == "mlp":
        shapes = [(6, 8), (12, 8), (12,), (8, 12), (8,), (6, 8)]
        fused = lambda x, w1, b1, w2, b2, res: F._mlp_gelu(x, w1, b1, w2, b2, res).pow(2).sum()
        ref = lambda x, w1, b1, w2, b2, res: (
            res + F.linear(F.gelu(F.linear(x, w1, b1)), w2, b2)).pow(2).sum()
    elif which == "linear_add":
        shapes = [(6, 8), (5, 8), (5,), (6, 5)]
        fused = lambda x, w, b, res: F._linear_add(x, w, b, res).pow(3).sum()
        ref = lambda x, w, b, res: (res + F.linear(x, w, b)).pow(3).sum()
    else:
        shapes = [(7, 4), (6, 4)]
        ids = torch.tensor(np.array([[1, 6, 1], [0, 3, 5]], np.int32), dtype="int32")
        fused = lambda w, p: F._embedding_pos(ids, w, p, 2).pow(3).sum()
        ref = lambda w, p: (F.embedding(ids, w) + p[2:5]).pow(3).sum()
    xs = [f32(r.standard_normal(s) * 0.5) for s in shapes]
    vs = [f32(r.standard_normal(s)) for s in shapes]
    res = []
    for fn in (fused, ref):
        ts = [torch.tensor(x, requires_grad=True) for x in xs]
        g1 = torch.autograd.grad(fn(*ts), ts, create_graph=True)
        dot = None
        for g, v in zip(g1, vs):
            term = (g * torch.tensor(v)).sum()
            dot = term if dot is None else dot + term
        h = torch.autograd.grad(dot, ts)
        res.append(([g.numpy() for g in g1], [hh.numpy() for hh in h]))
    for a, b in zip(res[0][0] + res[0][1], res[1][0] + res[1][1]):
        check(a, b, **RED)


def test_second_order_conv2d_refused(torch):
    """The convolution has no differentiable backward: create_graph through
    it raises, naming the op."""
    x = torch.tensor(f32(np.ones((1, 2, 5, 5))), requires_grad=True)
    w = torch.tensor(f32(np.ones((3, 2, 3, 3)) * 0.1), requires_grad=True)
    y = torch.F.conv2d(x, w, None, 1, 1).pow(2).sum()
    with pytest.raises(NotImplementedError, match="Conv2d"):
        torch.autograd.grad(y, [x, w], create_graph=True)


def _second_order_functions(torch):
    """The definitions of tests/golden/make_golden.py second_order_functions,
    over the hip package."""
    T, F = torch, torch.F
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


def test_autograd_function_literals(torch):
    class DoubleFn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            ctx.save_for_backward(x)
            return x.mul(2)

        @staticmethod
        def backward(ctx, g):
            return g.mul(2)

    x = torch.tensor([1.0, 2.0, 3.0], requires_grad=True)
    DoubleFn.apply(x).sum().backward()
    close4(x.grad.toArray(), [2.0, 2.0, 2.0])             # :153-175

    class ReLUFn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            ctx.save_for_backward(x)
            return x.clamp_min(0)

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            return g.mul(x.gt(0))

    x = torch.tensor([-1.0, 0.0, 2.0, 5.0], requires_grad=True)
    y = ReLUFn.apply(x)
    close4(y.toArray(), [0.0, 0.0, 2.0, 5.0])
    y.sum().backward()
    close4(x.grad.toArray(), [0.0, 0.0, 1.0, 1.0])        # :177-200

    class MulAddFn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, y):
            ctx.save_for_backward(x, y)
            return x.mul(y).add(x)

        @staticmethod
        def backward(ctx, g):
            x, y = ctx.saved_tensors
            return [g.mul(y.add(1)), g.mul(x)]

    x = torch.tensor([2.0, 3.0], requires_grad=True)
    y = torch.tensor([4.0, 5.0], requires_grad=True)
    MulAddFn.apply(x, y).sum().backward()
    close4(x.grad.toArray(), [5.0, 6.0])                  # :202-228
    close4(y.grad.toArray(), [2.0, 3.0])


def test_clamp_gradient_includes_bounds(torch):
    x = torch.tensor([-2.0, -1.0, 0.0, 0.5, 1.0, 3.0], requires_grad=True)
    y = x.clamp(-1.0, 1.0)
    assert y.toArray() == [-1.0, -1.0, 0.0, 0.5, 1.0, 1.0]
    y.sum().backward()
    assert x.grad.toArray() == [0.0, 1.0, 1.0, 1.0, 1.0, 0.0]


# ------------------------------------------------------------ cat / stack / expand


@pytest.mark.parametrize("dim", [0, 1, 2, -1])
def test_cat_forward_backward(torch, dim):
    """cat (Tensor.ts:152-235): values and the split gradient, ragged sizes
    along `dim`, one input a transposed view."""
    r = np.random.default_rng(40 + dim)
    shapes = []
    for k in (3, 1, 5):
        s = [4, 6, 7]
        s[dim] = k
        shapes.append(tuple(s))
    arrs = [f32(r.standard_normal(s)) for s in shapes]
    ts = [torch.tensor(a, requires_grad=True) for a in arrs]
    # the middle input enters as a non-contiguous view of its transpose
    tt = torch.tensor(np.ascontiguousarray(np.swapaxes(arrs[1], 0, 2)), requires_grad=True)
    mid = tt.transpose(0, 2)
    out = torch.cat([ts[0], mid, ts[2]], dim)
    want = np.concatenate(arrs, axis=dim)
    assert np.array_equal(out.numpy(), want)
    g = f32(r.standard_normal(want.shape))
    out.backward(torch.tensor(g))
    pieces = np.split(g, np.cumsum([s[dim] for s in shapes])[:-1], axis=dim)
    assert np.array_equal(ts[0].grad.numpy(), pieces[0])
    assert np.array_equal(tt.grad.numpy(), np.swapaxes(pieces[1], 0, 2))
    assert np.array_equal(ts[2].grad.numpy(), pieces[2])


@pytest.mark.parametrize("dim", [0, 1, 2])
def test_stack_forward_backward(torch, dim):
    """stack (src/ops/creation.ts:416-437): a new axis, gradients unstacked."""
    r = np.random.default_rng(50 + dim)
    arrs = [f32(r.standard_normal((5, 3))) for _ in range(4)]
    ts = [torch.tensor(a, requires_grad=True) for a in arrs]
    out = torch.stack(ts, dim)
    want = np.stack(arrs, axis=dim)
    assert np.array_equal(out.numpy(), want)
    g = f32(r.standard_normal(want.shape))
    out.backward(torch.tensor(g))
    for i, t in enumerate(ts):
        assert np.array_equal(t.grad.numpy(), np.take(g, i, axis=dim))


def test_cat_int32_and_empty_piece(torch):
    a = torch.tensor(np.array([[1, 2]], dtype=np.int32))
    b = torch.tensor(np.zeros((0, 2), dtype=np.int32))
    c = torch.tensor(np.array([[3, 4], [5, 6]], dtype=np.int32))
    out = torch.cat([a, b, c], 0)
    assert out.dtype == "int32" and out.numpy().tolist() == [[1, 2], [3, 4], [5, 6]]


@pytest.mark.parametrize("src,target", [((4096,), (64, 4096)), ((1, 7, 1), (3, 7, 5)),
                                        ((6, 1), (2, 6, 9)), ((), (3, 4)), ((5,), (5,))])
def test_expand_backward_sums_broadcast_dims(torch, src, target):
    """expand's gradient is the sum over every expanded dim (torch.js
    records none, D12, Tensor.ts:1541-1601)."""
    r = np.random.default_rng(len(src) * 10 + len(target))
    x = f32(r.standard_normal(src))
    g = f32(r.standard_normal(target))
    t = torch.tensor(x, requires_grad=True)
    e = t.expand(*target)
    assert np.array_equal(e.numpy(), np.broadcast_to(x, target))
    e.backward(torch.tensor(g))
    check(t.grad.numpy(), ops.sum_to(g, src), **RED)
    # -1 keeps a size; expand_as; a materialised copy of the view is still a view's grad
    t2 = torch.tensor(x, requires_grad=True)
    e2 = t2.expand_as(torch.zeros(*target)).contiguous()
    e2.backward(torch.tensor(g))
    check(t2.grad.numpy(), ops.sum_to(g, src), **RED)


# ------------------------------------------------------------ losses


@pytest.mark.parametrize("rows,cols", [(7, 9), (33, 1000), (6, 50257)])
@pytest.mark.parametrize("kind", ["w", "ls", "wls"])
@pytest.mark.parametrize("red", ["mean", "sum", "none", "batchmean"])
def test_cross_entropy_weights_and_smoothing(torch, rows, cols, kind, red):
    """F.cross_entropy(input, target, weight, reduction, label_smoothing)
    (losses.ts:129-168, positional as torch.js orders them) against the
    oracle, with an ignored row."""
    r = np.random.default_rng(rows * 7 + cols + len(kind))
    x = f32(r.standard_normal((rows, cols)) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    t[2] = -100
    w = f32(r.uniform(0.2, 2.0, cols)) if "w" in kind else None
    eps = {"w": 0.0, "ls": 0.1, "wls": 0.25}[kind]
    xt = torch.tensor(x, requires_grad=True)
    loss = torch.F.cross_entropy(xt, torch.tensor(t), torch.tensor(w) if w is not None else None,
                                 red, eps)
    gl = f32(r.standard_normal(rows)) if red == "none" else np.float32(1.1)
    loss.backward(torch.tensor(gl))
    kw = dict(weight=w, label_smoothing=eps)
    check(loss.numpy(), ops.cross_entropy(x, t, red, **kw), **RED)
    check(xt.grad.numpy(), ops.cross_entropy_backward(x, t, gl, red, **kw), **RED)


def test_cross_entropy_module_and_keyword_ignore_index(torch):
    r = np.random.default_rng(3)
    x = f32(r.standard_normal((5, 4)))
    t = np.array([1, 0, 3, 7, 2], dtype=np.int32)
    w = f32([1.0, 2.0, 0.5, 1.5])
    loss = torch.nn.CrossEntropyLoss(torch.tensor(w), "mean", 0.2, ignore_index=7)(
        torch.tensor(x), torch.tensor(t))
    check(loss.item(), ops.cross_entropy(x, t, "mean", 7, weight=w, label_smoothing=0.2), **RED)
    with pytest.raises(ValueError):
        torch.F.cross_entropy(torch.tensor(x), torch.tensor(t), None, "bogus")


@pytest.mark.parametrize("red", ["mean", "sum", "none", "batchmean"])
def test_nll_loss_weighted(torch, red):
    r = np.random.default_rng(17)
    lp = f32(ops.log_softmax(r.standard_normal((9, 6))))
    t = r.integers(0, 6, 9).astype(np.int32)
    t[4] = -100
    w = f32(r.uniform(0.1, 3.0, 6))
    xt = torch.tensor(lp, requires_grad=True)
    loss = torch.F.nll_loss(xt, torch.tensor(t), torch.tensor(w), red)
    gl = f32(r.standard_normal(9)) if red == "none" else np.float32(0.9)
    loss.backward(torch.tensor(gl))
    check(loss.numpy(), ops.nll_loss(lp, t, red, weight=w), **RED)
    check(xt.grad.numpy(), ops.nll_loss_backward(lp.shape, t, gl, red, weight=w), **RED)


# ------------------------------------------------------------ nn.init


def test_nn_init_seeded_and_bounded(torch):
    """nn.init (init.ts:10-144) over the seeded device generator: each fill is
    one rand / randn call of the manual_seed stream (creation.ts:921), so the
    values are the oracle's stream scaled."""
    init = torch.nn.init
    torch.manual_seed(77)
    seeds = []
    s = 77
    for _ in range(4):
        s = rng.lcg_next(s)
        seeds.append(s)
    w = torch.nn.Parameter.create(torch.zeros(64, 48))
    init.normal_(w, 0.5, 0.02)
    check(w.numpy(), 0.5 + 0.02 * rng.randn(64 * 48, seeds[0]).reshape(64, 48), rtol=1e-5,
          atol=1e-6)
    assert w.is_leaf and w.requires_grad
    init.uniform_(w, -0.3, 0.7)
    check(w.numpy(), -0.3 + 1.0 * rng.rand(64 * 48, seeds[1]).reshape(64, 48), **EW)
    init.kaiming_uniform_(w, a=math.sqrt(5))  # PyTorch's Linear default
    bound = math.sqrt(2.0 / (1 + 5)) / math.sqrt(48) * math.sqrt(3)
    u = rng.rand(64 * 48, seeds[2]).reshape(64, 48).astype(np.float64)
    check(w.numpy(), -bound + 2 * bound * u, **EW)
    assert np.abs(w.numpy()).max() <= bound
    conv = torch.zeros(8, 3, 3, 3)
    init.xavier_normal_(conv)  # fan_in 27, fan_out 72 (PyTorch's rule)
    std = math.sqrt(2.0 / (27 + 72))
    check(conv.numpy(), std * rng.randn(8 * 27, seeds[3]).reshape(8, 3, 3, 3), rtol=1e-5,
          atol=1e-6)
    e = torch.zeros(3, 5)
    init.eye_(e)
    assert np.array_equal(e.numpy(), np.eye(3, 5, dtype=np.float32))
    init.constant_(e, 2.5)
    assert (e.numpy() == 2.5).all()
    assert init.calculate_gain("tanh") == 5.0 / 3.0
    assert abs(init.calculate_gain("leaky_relu", 0.2) - math.sqrt(2 / 1.04)) < 1e-15
    with pytest.raises(ValueError):
        init.xavier_uniform_(torch.zeros(5))


# ------------------------------------------------------------ dtypes, masks, triu / tril


def test_casts_on_device(torch):
    """Tensor.to / .bool() between float32, int32, uint8 and bool run on the
    device: bool is `!= 0` (NaN included), float to integer truncates toward
    zero, uint8 keeps the low 8 bits."""
    x = np.array([-2.7, -0.0, 0.0, 0.4, 1.0, 3.9, 255.0, 300.5, np.nan], np.float32)
    t = torch.tensor(x)
    assert t.bool().numpy().tolist() == [1, 0, 0, 1, 1, 1, 1, 1, 1]
    assert t.bool().dtype == "bool"
    assert t[:8].int().numpy().tolist() == [-2, 0, 0, 0, 1, 3, 255, 300]
    assert t[:8].to("uint8").numpy().tolist() == [254, 0, 0, 0, 1, 3, 255, 44]
    i = torch.tensor(np.array([-1, 0, 7, 256], np.int32))
    assert i.bool().numpy().tolist() == [1, 0, 1, 1]
    assert i.to("uint8").numpy().tolist() == [255, 0, 7, 0]
    assert i.float().numpy().tolist() == [-1.0, 0.0, 7.0, 256.0]
    b = torch.tensor(np.array([[1, 0], [0, 1]], np.bool_))
    assert b.dtype == "bool" and b.float().numpy().tolist() == [[1.0, 0.0], [0.0, 1.0]]
    # a strided bool view copied on the device
    assert b.T.contiguous().numpy().tolist() == [[1, 0], [0, 1]]
    u = torch.zeros(5, dtype="uint8")
    u.fill_(300)
    assert u.numpy().tolist() == [44] * 5


@pytest.mark.parametrize("diag", [-2, -1, 0, 1, 3])
def test_triu_tril_forward_backward(torch, diag):
    r = np.random.default_rng(60 + diag)
    x = f32(r.standard_normal((2, 5, 7)))
    g = f32(r.standard_normal((2, 5, 7)))
    for upper, fn in ((True, np.triu), (False, np.tril)):
        t = torch.tensor(x, requires_grad=True)
        y = t.triu(diag) if upper else t.tril(diag)
        assert np.array_equal(y.numpy(), fn(x, diag))
        y.backward(torch.tensor(g))
        assert np.array_equal(t.grad.numpy(), fn(g, diag))


def test_gpt2_inference_ops_literal(torch):
    """tests/gpt2.test.ts:24-100: a causal mask from ones.triu(1).bool(),
    4-D batched Q @ K^T, masked_fill(mask, -1e9), softmax, probs @ V, and
    the transpose / contiguous / reshape of the output, against numpy."""
    r = np.random.default_rng(70)
    B, H, T, hd = 1, 4, 8, 16
    q = f32(r.standard_normal((B, H, T, hd)))
    k = f32(r.standard_normal((B, H, hd, T)))
    v = f32(r.standard_normal((B, H, T, hd)))
    mask = torch.ones(T, T).triu(1).bool()
    assert mask.shape == (T, T) and mask.dtype == "bool"
    att = torch.tensor(q).matmul(torch.tensor(k)).mul(1.0 / np.sqrt(hd))
    assert att.shape == (B, H, T, T)
    probs = att.masked_fill(mask, -1e9).softmax(-1)
    out = probs.matmul(torch.tensor(v))
    s = (q.astype(np.float64) @ k) / np.sqrt(hd)
    s = np.where(np.triu(np.ones((T, T)), 1) > 0, -1e9, s)
    want = ops.softmax(s) @ v
    check(out.numpy(), want, **RED)
    o = out.transpose(1, 2).contiguous().reshape(B, T, H * hd)
    assert o.shape == (B, T, H * hd)
    check(o.numpy(), want.transpose(0, 2, 1, 3).reshape(B, T, H * hd), **RED)


# ------------------------------------------------------------ sampling


@pytest.mark.parametrize("rows,cols,ns,repl", [(1, 10, 1, False), (3, 1000, 7, True),
                                               (2, 50257, 3, True), (4, 37, 37, False),
                                               (5, 300, 20, False), (2, 9, 500, True)])
def test_multinomial_replays_oracle(torch, rows, cols, ns, repl):
    """The device sampler draws u from the seeded stream (element
    r * num_samples + s of rand's generator, seed = the next LCG state):
    replaying those u through the oracle gives the same indices."""
    r = np.random.default_rng(rows * 1000 + cols + ns)
    x = f32(r.random((rows, cols)) ** 3)
    x[0, ::4] = 0.0
    if rows > 2:
        x[1] = -1.0  # no positive weight: uniform
        x[2, 5] = -np.inf  # weighs 0, like a negative weight
    torch.manual_seed(4321)
    got = torch.tensor(x).multinomial(ns, repl).numpy()
    seed = rng.lcg_next(4321)
    u = rng.rand(rows * ns, seed).reshape(rows, ns)
    want = ops.multinomial(x, ns, repl, u)
    assert got.shape == (rows, ns) and got.dtype == np.int32
    assert np.array_equal(got, want)
    if not repl:
        assert all(len(set(row)) == ns for row in got.tolist())


def test_multinomial_literal_and_errors(torch):
    """tests/gpt2.test.ts:123-131: softmax of 100 logits, one draw, an index
    in [0, 100); and the reference's error without replacement."""
    probs = torch.randn(100).softmax(0)
    tok = probs.multinomial(1)
    assert tok.shape == (1,) and 0 <= tok.item() < 100
    with pytest.raises(RuntimeError):
        torch.tensor([0.5, 0.5]).multinomial(3)


@pytest.mark.parametrize("bad", [np.nan, np.inf])
@pytest.mark.parametrize("repl", [True, False])
def test_multinomial_rejects_nan_and_inf_rows(torch, bad, repl):
    """A row holding NaN or +inf raises, as in the oracle (and PyTorch); the
    call reads the per-row status back, so the error names the row.  The
    library stays usable afterwards and a clean row still replays the
    oracle."""
    x = np.full((3, 40), 0.25, dtype=np.float32)
    x[1, 17] = bad
    with pytest.raises(ValueError):
        ops.multinomial(x, 2, repl, np.zeros((3, 2)))
    with pytest.raises(RuntimeError, match="row 1 contains NaN or inf"):
        torch.tensor(x).multinomial(2, repl)
    torch.manual_seed(77)
    got = torch.tensor(x[:1]).multinomial(2, repl).numpy()
    u = rng.rand(2, rng.lcg_next(77)).reshape(1, 2)
    assert np.array_equal(got, ops.multinomial(x[:1], 2, repl, u))


# ------------------------------------------------------------ attention masks, KV cache


@pytest.mark.parametrize("kind", ["bool", "float"])
def test_sdpa_attn_mask(torch, kind):
    """attn_mask (PyTorch's contract; torch.js throws): bool True attends,
    float is added to the scores; gradients through the composite path."""
    r = np.random.default_rng(80)
    B, H, Tq, Tk, D = 2, 3, 5, 7, 16
    q, k, v = (f32(r.standard_normal((B, H, t, D))) for t in (Tq, Tk, Tk))
    if kind == "bool":
        m = r.random((Tq, Tk)) > 0.3
        m[:, 0] = True  # every query keeps one key
        mt = torch.tensor(m)
        add = np.where(m, 0.0, -np.inf)
    else:
        add = f32(r.standard_normal((Tq, Tk)))
        mt = torch.tensor(add)
    g = f32(r.standard_normal((B, H, Tq, D)))
    ts = [torch.tensor(a, requires_grad=True) for a in (q, k, v)]
    out = torch.F.scaled_dot_product_attention(*ts, attn_mask=mt)
    out.backward(torch.tensor(g))
    q64, k64, v64 = (a.astype(np.float64) for a in (q, k, v))
    s = q64 @ k64.transpose(0, 1, 3, 2) / np.sqrt(D) + add
    p = ops.softmax(s)
    check(out.numpy(), p @ v64, **RED)
    g64 = g.astype(np.float64)
    dp = g64 @ v64.transpose(0, 1, 3, 2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True)) / np.sqrt(D)
    check(ts[0].grad.numpy(), ds @ k64, **RED)
    check(ts[1].grad.numpy(), ds.transpose(0, 1, 3, 2) @ q64, **RED)
    check(ts[2].grad.numpy(), p.transpose(0, 1, 3, 2) @ g64, **RED)


def test_gpt2_kv_cache_matches_full_forward(torch):
    """Decoding with the KV cache gives, at every new position, the logits of
    the full forward over the whole sequence; generate() with a fixed seed
    draws the tokens the oracle sampler picks from those logits."""
    from oracle import models as om
    from torchjs_amd import workloads as W
    cfg = om.Config(vocab=211, ctx=64, d=128, heads=4, layers=2)
    r = np.random.default_rng(90)
    p = om.init_params(cfg, r, std=0.2)
    model = W.GPT2(cfg.vocab, cfg.ctx, cfg.d, cfg.heads, cfg.layers)
    W.load_params(model, p)
    prompt = r.integers(0, cfg.vocab, (2, 9)).astype(np.int32)
    torch.manual_seed(77)
    seq = model.generate(torch.tensor(prompt), 12, temperature=0.8).numpy()
    assert seq.shape == (2, 21) and np.array_equal(seq[:, :9], prompt)
    with torch.no_grad():
        full = model(torch.tensor(seq)).numpy()
    # every sampled token replays through the oracle sampler on the full
    # forward's probabilities at the previous position
    s = 77
    for j in range(12):
        s = rng.lcg_next(s)
        u = rng.rand(2, s).reshape(2, 1)
        logits = full[:, 8 + j].astype(np.float64) / 0.8
        want = ops.multinomial(ops.softmax(logits), 1, True, u)
        assert np.array_equal(seq[:, 9 + j], want[:, 0]), j
    # the cached decode's logits equal the full forward's
    with torch.no_grad():
        cache = model.new_cache(2, 21)
        first = model.forward_cached(torch.tensor(seq[:, :9]), cache, 0).numpy()
        check(first, full[:, :9], **RED)
        for j in range(9, 21):
            step = model.forward_cached(torch.tensor(seq[:, j:j + 1]), cache, j).numpy()
            check(step[:, 0], full[:, j], **RED)


# ------------------------------------------------------------ profiler


def test_profiler_record_function(torch):
    """record_function (src/profiler/index.ts:155-210): the context-manager,
    fn and decorator forms record host and device time and the allocator
    delta while a profiler is active; outside one they only run the block
    (and its roctx range)."""
    P = torch.profiler
    assert P.record_function("idle", lambda: 41 + 1) == 42  # no profiler: just runs
    with P.profile() as prof:
        with P.record_function("matmul_block"):
            a = torch.randn(1024, 1024)
            b = a @ a
        s = P.record_function("fn_form", lambda: (b * 2.0).sum())

        @P.record_function("decorated")
        def twice(x):
            return x * 2.0
        twice(a)
        P.mark("checkpoint")
    assert isinstance(s, torch.Tensor)
    ev = {e["name"]: e for e in prof.get_events()}
    assert set(ev) == {"matmul_block", "fn_form", "decorated"}
    for e in ev.values():
        assert e["duration"] > 0 and e["device_duration"] > 0 and e["activity"] == "hip"
    assert ev["matmul_block"]["memory_usage"] >= 2 * 1024 * 1024 * 4
    tab = prof.key_averages().table(sort_by="device_duration")
    assert "matmul_block" in tab and "Device Time" in tab
    out = P.profile(lambda p: P.record_function("inner", lambda: torch.ones(8).sum()))
    assert [e["name"] for e in out.get_events()] == ["inner"]


# ------------------------------------------------------------ weight I/O


def test_save_load_round_trip_on_device(torch, tmp_path):
    """torch.save of a model's state_dict (torch.js's zip layout) and
    torch.load back into a fresh model: every parameter byte for byte; a
    strided view is saved as its values."""
    from torchjs_amd import workloads as W
    torch.manual_seed(5)
    src = W.GPT2(211, 64, 128, 4, 2)
    path = str(tmp_path / "gpt2.zip")
    extra = torch.randn(6, 4).T  # a transposed view
    torch.save({"state": src.state_dict(), "extra": extra, "step": 3}, path)
    obj = torch.load(path)
    assert obj["step"] == 3 and obj["extra"].shape == (4, 6)
    assert np.array_equal(obj["extra"].numpy(), extra.numpy())
    dst = W.GPT2(211, 64, 128, 4, 2)
    dst.load_state_dict(obj["state"])
    for (k, a), (k2, b) in zip(src.named_parameters(), dst.named_parameters()):
        assert k == k2 and a.numpy().tobytes() == b.numpy().tobytes(), k
    assert torch.save(extra)[:2] == b"PK"  # bytes when no file is given


def test_load_pytorch_state_dict_to_device(torch):
    """A torch.save archive (PyTorch's layout: data.pkl + data/N, read with
    the weights-only unpickler, strides and offsets applied) becomes 'hip'
    tensors holding the saved values."""
    import os
    from conftest import GOLDEN
    obj = torch.load(os.path.join(GOLDEN, "state_dict.pt"))
    with np.load(os.path.join(GOLDEN, "state_dict_expected.npz")) as z:
        for k in ("layer.weight", "ids", "transposed", "slice", "half", "bf16", "mask"):
            t = obj[k]
            assert isinstance(t, torch.Tensor), k
            assert np.array_equal(t.numpy(), z[k]), k
        assert np.array_equal(obj["nested"]["list"][0].numpy(), z["nested.list.0"])
    assert obj["layer.weight"].requires_grad and obj["mask"].dtype == "bool"
    same = torch.serialization.load_pytorch_zip(os.path.join(GOLDEN, "state_dict.pt"))
    assert np.array_equal(same["transposed"].numpy(), obj["transposed"].numpy())
