"""Parity of every hot-path kernel with the oracle on identical seeded
inputs (MI355X).  Tolerances: integer / index work bit-exact; fp32
elementwise rtol 1e-5; reductions, GEMM, attention, conv rtol 1e-4 /
atol 1e-5 (reduction order differs from the float64 oracle)."""
import ctypes
import math

import numpy as np
import pytest

from oracle import ops, rng

pytestmark = pytest.mark.gpu

EW = dict(rtol=1e-5, atol=1e-6)
RED = dict(rtol=1e-4, atol=1e-5)


def f32(a):
    return np.asarray(a, dtype=np.float32)


def check(got, want, **tol):
    np.testing.assert_allclose(np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64),
                               **tol)


def check_floor(got, want, ref32, k=3.0):
    """The required rtol 1e-4 / atol 1e-5, with atol raised to k times the
    float32 floor of the same computation when that floor exceeds 1e-5: the
    floor is max |ref32 - want|, ref32 the same product evaluated in
    float32 on the CPU.  Unit-variance operands summed over thousands of
    terms give outputs of size ~sqrt(K), whose elements near zero carry the
    rounding of partial sums of that size in any float32 implementation."""
    want = np.asarray(want, dtype=np.float64)
    floor = float(np.abs(np.asarray(ref32, dtype=np.float64) - want).max())
    check(got, want, rtol=1e-4, atol=max(1e-5, k * floor))


def _tensor_module():
    """The package's tensor module (its engine switches live there);
    `from torchjs_amd import tensor` would return the tensor() factory that
    the package exports under the same name."""
    import sys
    return sys.modules["torchjs_amd.tensor"]


def grad_of(torch, fn, *arrays):
    """Runs fn on leaf tensors, backprops a seeded upstream grad, returns
    (output, upstream, grads)."""
    ts = [torch.tensor(f32(a), requires_grad=True) for a in arrays]
    out = fn(*ts)
    g = np.random.default_rng(99).standard_normal(out.shape).astype(np.float32)
    out.backward(torch.tensor(g))
    return out.numpy(), g, [t.grad.numpy() if t.grad is not None else None for t in ts]


# ------------------------------------------------------------------ runtime


def test_device_is_gfx950(torch):
    info = torch.hip.device_info()
    assert info["arch"].startswith("gfx950"), info
    assert info["warp_size"] == 64


def test_roundtrip_and_allocator(torch):
    a = np.arange(1000, dtype=np.float32) - 500.5
    t = torch.tensor(a)
    assert np.array_equal(t.numpy(), a)
    s0 = torch.hip.memory_stats()
    for _ in range(5):
        u = torch.zeros(1 << 20)
        del u
    s1 = torch.hip.memory_stats()
    assert s1["device_mallocs"] - s0["device_mallocs"] <= 1  # cached blocks are reused
    assert s1["peak_bytes"] >= s1["active_bytes"]
    # torch.webgpu.memory_stats()'s keys (src/webgpu.ts:11-19): total_allocations
    # counts blocks created on a cache miss, like the reference's pool
    assert set(s1) >= {"active_bytes", "pooled_bytes", "peak_bytes", "total_allocations"}
    assert s1["total_allocations"] == s1["device_mallocs"]
    assert s1["allocation_requests"] - s0["allocation_requests"] >= 5
    assert torch.webgpu.memory_stats()["total_allocations"] == s1["total_allocations"]
    summ = torch.webgpu.memory_summary()
    lines = [l for l in summ.splitlines() if l]
    assert lines[0] == "GPU Memory Summary" and lines[1] == "-" * 55
    assert lines[2].startswith("Active Memory:   ") and lines[2].endswith(" MB")
    assert lines[5] == "Total Allocs:    %d" % torch.hip.memory_stats()["total_allocations"]
    ints = torch.tensor(np.array([3, -7, 2 ** 30], dtype=np.int32))
    assert ints.dtype == "int32" and ints.numpy().tolist() == [3, -7, 2 ** 30]
    assert torch.tensor([-0.0, 1.5]).toArray() == [0.0, 1.5]


def test_async_readback_is_stream_ordered(torch):
    """tjh_d2h_start copies in submission order: a fill launched after it
    cannot change what tjh_d2h_finish delivers, even when finish runs on
    another thread while the caller keeps launching."""
    import threading
    from torchjs_amd import _lib as L
    n = 1 << 20
    src = (np.arange(n) % 977).astype(np.float32)
    t = torch.tensor(src)
    tickets = []
    for _ in range(3):
        tk = ctypes.c_uint64(0)
        L.check(L.lib().tjh_d2h_start(t.data_ptr(), n * 4, ctypes.byref(tk)), "d2h_start")
        tickets.append(tk.value)
        t.fill_(7.0)  # lands after the copy just enqueued
    outs = [np.empty(n, np.float32) for _ in tickets]
    errs = []

    def finish(tk, out):
        rc = L.lib().tjh_d2h_finish(tk, out.ctypes.data)
        if rc:
            errs.append(L.lib().tjh_last_error())
    th = [threading.Thread(target=finish, args=(tk, o)) for tk, o in zip(tickets, outs)]
    for x in th:
        x.start()
    for x in th:
        x.join()
    assert not errs, errs
    assert np.array_equal(outs[0], src)
    assert (outs[1] == 7.0).all() and (outs[2] == 7.0).all()
    # a released ticket is unknown afterwards
    assert L.lib().tjh_d2h_finish(tickets[0], outs[0].ctypes.data) != 0


def test_rng_matches_oracle_stream(torch):
    """Six successive rand / randn calls after manual_seed(1234): the seeds
    are creation.ts:921's JS-double LCG states (233191843, 128476320,
    85706848, ...: the third is where exact integer arithmetic would
    diverge), each element the xorshift32 state of random.wgsl."""
    torch.manual_seed(1234)
    sizes = [10007, 4099, 513, 1 << 16, 7, 2049]
    normal = [False, True, False, True, False, True]
    got = [(torch.randn if nm else torch.rand)(n).numpy() for n, nm in zip(sizes, normal)]
    s = 1234
    seeds = []
    for _ in sizes:
        s = rng.lcg_next(s)
        seeds.append(s)
    assert seeds[:4] == [233191843, 128476320, 85706848, 2116141344]
    for g, n, nm, sd in zip(got, sizes, normal, seeds):
        if nm:  # Box-Muller in float32 on the device, float64 in the oracle
            check(g, rng.randn(n, sd), rtol=1e-5, atol=2e-6)
        else:  # integer stream + exact scaling: bit-exact
            assert np.array_equal(g, rng.rand(n, sd))


def test_randn_box_muller_special_states(torch):
    """tjh_random's normal stream at the seeds whose element 0 has the states
    the oracle's closed-form checks use (u2 = 1/2, u2 = 1/4, u1 clamped at
    1e-7, found by inverting xorshift32): the device gives -sqrt(-2 ln u1),
    ~0 and +-5.677 as the mathematics fixes them."""
    from test_oracle import _seed_for_states, _xs_inverse
    from torchjs_amd import _lib as L
    cases = []
    for s2, cos_want in ((2 ** 31, -1.0), (2 ** 30, math.cos(float(np.float32(2 * math.pi)) / 4))):
        seed, s1 = _seed_for_states(s2)
        u1 = float(np.float32(s1 / 2 ** 32))
        cases.append((seed, math.sqrt(-2.0 * math.log(u1)) * cos_want))
    r_clamp = math.sqrt(-2.0 * math.log(float(np.float32(1e-7))))
    for s1 in (1, 7, 429):
        u2 = float(np.float32(int(rng.xorshift32(s1)) / 2 ** 32))
        theta = float(np.float32(np.float32(2 * math.pi) * np.float32(u2)))
        cases.append((_xs_inverse(s1) ^ 1013904223, r_clamp * math.cos(theta)))
    out = torch.empty((1,))
    for seed, want in cases:
        L.check(L.lib().tjh_random(out.data_ptr(), 1, seed, 1), "random")
        got = float(out.numpy()[0])
        assert abs(got - want) <= 2e-6, (seed, got, want)
        assert abs(got - float(rng.randn(1, seed)[0])) <= 2e-6


# ------------------------------------------------------------------ elementwise


UNARY = ["neg", "exp", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "relu", "gelu", "square",
         "reciprocal", "erf", "abs", "sin", "cos", "silu", "softplus"]


@pytest.mark.parametrize("n", [1, 7, 4099, 1 << 20])
@pytest.mark.parametrize("op", UNARY)
def test_unary_fwd_bwd(torch, op, n):
    r = np.random.default_rng(n)
    pos = op in ("log", "sqrt", "rsqrt", "reciprocal")
    x = f32(r.uniform(0.1, 4, n) if pos else r.uniform(-5, 5, n))
    out, g, (gx,) = grad_of(torch, lambda t: getattr(t, op)(), x)
    check(out, ops.unary(op, x), **EW)
    check(gx, ops.unary_backward(op, g, x), **EW)


@pytest.mark.parametrize("n", [7, 4099, 1 << 20])
@pytest.mark.parametrize("op,alpha", [("leaky_relu", 0.01), ("leaky_relu", 0.2), ("elu", 1.0),
                                      ("elu", 0.7), ("sign", 0.0)])
def test_parametric_unary_and_sign(torch, op, alpha, n):
    """leaky_relu / elu at two slopes and sign against the oracle, with
    zeros in the input (x > 0 selects the positive branch; sign(0) = 0 and
    sign's gradient is 0)."""
    r = np.random.default_rng(n + int(alpha * 100))
    x = f32(r.uniform(-5, 5, n))
    x[::5] = 0.0
    if op == "sign":
        fn = lambda t: t.sign()
    else:
        fn = lambda t: getattr(t, op)(alpha)
    out, g, (gx,) = grad_of(torch, fn, x)
    check(out, ops.unary(op, x, alpha), **EW)
    check(gx, ops.unary_backward(op, g, x, alpha), **EW)


@pytest.mark.parametrize("sa,sb", [((64, 33), (64, 33)), ((4096, 1024), (1024,)),
                                   ((7, 5), (7, 1)), ((3, 4, 5), (4, 1))])
@pytest.mark.parametrize("op", ["maximum", "minimum"])
@pytest.mark.parametrize("ties", [False, True])
def test_maximum_minimum_fwd_bwd(torch, op, sa, sb, ties):
    """maximum / minimum forward and both gradients (summed over broadcast
    dims) against the oracle; with integer operands many elements tie and
    the oracle gives each side half of a tied gradient."""
    r = np.random.default_rng(len(sa) * 11 + len(sb) + ties)
    if ties:
        a = f32(r.integers(-2, 3, sa))
        b = f32(r.integers(-2, 3, sb))
    else:
        a = f32(r.uniform(-2.0, 2.0, sa))
        b = f32(r.uniform(-2.0, 2.0, sb))
    out, g, (ga, gb) = grad_of(torch, lambda x, y: getattr(x, op)(y), a, b)
    assert np.array_equal(out, ops.binary(op, a, b).astype(np.float32))
    ra, rb = ops.binary_backward(op, g, a, b)
    tol = RED if (ra.size < g.size or rb.size < g.size) else EW
    check(ga, ra, **tol)
    check(gb, rb, **tol)


def test_unary_on_unaligned_view(torch):
    x = f32(np.random.default_rng(0).uniform(-3, 3, 1001))
    t = torch.tensor(x)[1:]  # offset by one float: not 16-byte aligned
    check(t.gelu().numpy(), ops.gelu(x[1:]), **EW)
    check(t.exp().numpy(), np.exp(x[1:].astype(np.float64)), **EW)


@pytest.mark.parametrize("sa,sb", [((64, 33), (64, 33)), ((4096, 4096), (4096,)),
                                   ((7, 5), (7, 1)), ((3, 4, 5), (4, 1)), ((6,), ()),
                                   ((2, 1, 5), (3, 1)), ((1, 8), (8, 1))])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "pow"])
def test_binary_broadcast_fwd_bwd(torch, op, sa, sb):
    r = np.random.default_rng(len(sa) * 7 + len(sb))
    a = f32(r.uniform(0.5, 2.0, sa))
    b = f32(r.uniform(0.5, 2.0, sb))
    out, g, (ga, gb) = grad_of(torch, lambda x, y: getattr(x, op)(y), a, b)
    check(out, ops.binary(op, a, b), **EW)
    ra, rb = ops.binary_backward(op, g, a, b)
    # the float32 floor of a reduced gradient: its per-element terms formed
    # in float32 (numpy), summed exactly
    with np.errstate(all="ignore"):
        ta32, tb32 = {"add": (g, g), "sub": (g, -g), "mul": (g * b, g * a),
                      "div": (g / b, -g * a / (b * b)),
                      "pow": (g * b * a ** (b - np.float32(1)), g * a ** b * np.log(a))}[op]
    for got_, want_, terms, shp in ((ga, ra, ta32, sa), (gb, rb, tb32, sb)):
        if want_.size < g.size:  # summed over broadcast dims
            check_floor(got_, want_, ops.sum_to(np.broadcast_to(terms, g.shape), shp))
        else:
            check(got_, want_, **EW)


@pytest.mark.parametrize("op,s", [("add", 2.5), ("sub", -1.0), ("mul", 0.3), ("div", 7.0),
                                  ("pow", 2.0), ("pow", 3.0), ("pow", 0.5)])
def test_scalar_ops(torch, op, s):
    x = f32(np.random.default_rng(3).uniform(0.2, 3, 5003))
    out, g, (gx,) = grad_of(torch, lambda t: getattr(t, op)(s), x)
    if op == "pow":
        want = ops.pow_scalar(x, s)
        if s == 2.0:  # repeated multiply: exactly x*x in float32
            assert np.array_equal(out, x * x)
        dwant = g * s * ops.pow_scalar(x, s - 1)
    else:
        want = ops.binary(op, x, s)
        dwant = ops.binary_backward(op, g, x, np.float64(s))[0]
    check(out, want, **EW)
    check(gx, dwant, **EW)


def test_reverse_scalar_and_masked_fill(torch):
    x = f32(np.random.default_rng(4).uniform(0.5, 2, (6, 9)))
    t = torch.tensor(x, requires_grad=True)
    y = (1.0 - t) + (2.0 / t)
    y.sum().backward()
    check(y.numpy(), 1.0 - x.astype(np.float64) + 2.0 / x, **EW)
    check(t.grad.numpy(), -1.0 - 2.0 / x.astype(np.float64) ** 2, **EW)
    mask = np.triu(np.ones((6, 9)), 1)
    m = torch.tensor(mask.astype(np.uint8), dtype="uint8")
    t2 = torch.tensor(x, requires_grad=True)
    z = t2.masked_fill(m, -1e9)
    z.backward(torch.ones(6, 9))
    assert np.array_equal(z.numpy(), np.where(mask > 0, np.float32(-1e9), x))
    assert np.array_equal(t2.grad.numpy(), (1 - mask).astype(np.float32))


# ------------------------------------------------------------------ reductions


@pytest.mark.parametrize("shape,dim", [((16777216,), None), ((4096, 4096), 0), ((4096, 4096), 1),
                                       ((3, 5, 7), (0, 2)), ((8, 1024, 768), (0, 1)),
                                       ((1, 50257), 1), ((37, 3), 1)])
def test_sum_mean(torch, shape, dim):
    x = f32(np.random.default_rng(5).standard_normal(shape))
    t = torch.tensor(x, requires_grad=True)
    s = t.sum(dim)
    m = t.mean(dim)
    dims = None if dim is None else (dim if isinstance(dim, tuple) else (dim,))
    check(s.numpy(), ops.reduce("sum", x, dims), rtol=1e-4, atol=1e-5 * np.sqrt(x.size))
    check(m.numpy(), ops.reduce("mean", x, dims), **RED)
    m.backward(torch.ones(*m.shape))
    cnt = x.size // max(1, m.numel())
    assert np.array_equal(t.grad.numpy(), np.full(shape, np.float32(1.0 / cnt)))


def test_max_min_argmax(torch):
    x = f32(np.random.default_rng(6).integers(-3, 4, (33, 65)))  # many ties
    t = torch.tensor(x)
    check(t.amax(1).numpy(), x.max(1), rtol=0, atol=0)
    check(t.amin(0).numpy(), x.min(0), rtol=0, atol=0)
    assert np.array_equal(t.argmax(1).numpy(), ops.argmax(x, 1))
    assert np.array_equal(t.argmin(0).numpy(), ops.argmax(x, 0, is_min=True))
    assert t.argmax().item() == int(ops.argmax(x))
    big = f32(np.random.default_rng(7).standard_normal((64, 50257)))
    assert np.array_equal(torch.tensor(big).argmax(-1).numpy(), ops.argmax(big, 1))


# ------------------------------------------------------------------ softmax / losses


@pytest.mark.parametrize("shape", [(64, 10), (96, 1024), (5, 50257), (3, 4, 7)])
@pytest.mark.parametrize("log", [False, True])
def test_softmax(torch, shape, log):
    x = f32(np.random.default_rng(8).standard_normal(shape) * 4)
    fn = (lambda t: t.log_softmax(-1)) if log else (lambda t: t.softmax(-1))
    out, g, (gx,) = grad_of(torch, fn, x)
    y = ops.log_softmax(x) if log else ops.softmax(x)
    check(out, y, **RED)
    want = ops.log_softmax_backward(g, y) if log else ops.softmax_backward(g, y)
    check(gx, want, **RED)


@pytest.mark.parametrize("cols", [5, 37, 1000, 5000])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_with_minus_inf_entries(torch, cols, log):
    """Masked scores: -inf at the first, interior and last positions and in
    every lane's first element of some rows (a lane whose running maximum
    is still -inf must add exp(-inf) = 0, not exp(-inf - -inf) = NaN); rows
    with one finite entry give 1 there.  Softmax and log-softmax, forward
    and backward, on row offsets that are not 16-byte aligned."""
    r = np.random.default_rng(cols + log)
    x = f32(r.standard_normal((40, cols)) * 3)
    x[0, 0] = x[1, 1] = x[2, -1] = -np.inf
    x[3, ::2] = -np.inf
    x[4, :-1] = -np.inf  # one finite entry
    x[5, 1:] = -np.inf
    x[6:, :] = np.where(r.random((34, cols)) < 0.4, -np.inf, x[6:])
    x[6:, 0] = 1.0
    fn = (lambda t: t.log_softmax(-1)) if log else (lambda t: t.softmax(-1))
    out, g, (gx,) = grad_of(torch, fn, x)
    y = ops.log_softmax(x) if log else ops.softmax(x)
    assert np.isfinite(out).sum() == np.isfinite(y).sum()
    assert np.array_equal(np.isneginf(out), np.isneginf(y))
    fin = np.isfinite(y)
    check(out[fin], y[fin], **RED)
    if not log:
        assert out[4, -1] == 1.0 and out[5, 0] == 1.0
        want = ops.softmax_backward(g, y)
        check(gx, want, **RED)
    assert not np.isnan(out).any() and not np.isnan(gx).any()


def test_cross_entropy_with_minus_inf_logits(torch):
    """-inf logits of classes other than the target weigh nothing."""
    r = np.random.default_rng(12)
    x = f32(r.standard_normal((16, 37)))
    x[:, 5:9] = -np.inf
    t = r.integers(9, 37, 16).astype(np.int32)
    xt = torch.tensor(x, requires_grad=True)
    loss = torch.F.cross_entropy(xt, torch.tensor(t))
    loss.backward()
    check(loss.item(), ops.cross_entropy(x, t), **RED)
    dx = xt.grad.numpy()
    assert not np.isnan(dx).any() and (dx[:, 5:9] == 0).all()
    check(dx, ops.cross_entropy_backward(x, t), **RED)


def test_softmax_other_dim(torch):
    x = f32(np.random.default_rng(9).standard_normal((4, 6, 5)))
    out, g, (gx,) = grad_of(torch, lambda t: torch.F.softmax(t, 1), x)
    y = np.moveaxis(ops.softmax(np.moveaxis(x, 1, -1)), -1, 1)
    check(out, y, **RED)


@pytest.mark.parametrize("rows,cols", [(64, 10), (37, 50257), (128, 1000), (3, 1)])
@pytest.mark.parametrize("red", ["mean", "sum", "none"])
def test_cross_entropy(torch, rows, cols, red):
    r = np.random.default_rng(rows + cols)
    x = f32(r.standard_normal((rows, cols)) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    t[::5] = -100  # ignore_index rows
    xt = torch.tensor(x, requires_grad=True)
    loss = torch.F.cross_entropy(xt, torch.tensor(t), reduction=red)
    gl = f32(r.standard_normal(rows)) if red == "none" else np.float32(1.3)
    loss.backward(torch.tensor(gl))
    check(loss.numpy(), ops.cross_entropy(x, t, red), **RED)
    check(xt.grad.numpy(), ops.cross_entropy_backward(x, t, gl, red), **RED)


@pytest.mark.parametrize("rows,cols,ld", [(37, 50257, 50260), (19, 4100, 4100), (5, 2049, 2052)])
@pytest.mark.parametrize("red", ["mean", "none"])
def test_cross_entropy_aligned_rows(torch, rows, cols, ld, red):
    # logits whose rows start 16-byte aligned (a column slice of a wider
    # tensor, like the LM head's padded output): the flat backward path
    r = np.random.default_rng(rows * 3 + cols)
    full = f32(r.standard_normal((rows, ld)) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    t[::4] = -100
    t[1] = cols - 1  # target in the last, partial 4-column chunk
    ft = torch.tensor(full, requires_grad=True)
    x = ft[:, :cols]
    loss = torch.F.cross_entropy(x, torch.tensor(t), reduction=red)
    gl = f32(r.standard_normal(rows)) if red == "none" else np.float32(0.7)
    loss.backward(torch.tensor(gl))
    xs = full[:, :cols]
    check(loss.numpy(), ops.cross_entropy(xs, t, red), **RED)
    g = ft.grad.numpy()
    check(g[:, :cols], ops.cross_entropy_backward(xs, t, gl, red), **RED)
    assert not g[:, cols:].any()


@pytest.mark.parametrize("rows,cols,lead", [(37, 50257, 0), (64, 4100, 0), (9, 2049, 0),
                                            (37, 50257, 3), (5, 51201, 0)])
@pytest.mark.parametrize("red", ["mean", "sum", "batchmean"])
def test_cross_entropy_seeded_gradient_in_forward(torch, rows, cols, lead, red):
    """loss.backward() with its implicit unit seed on a cross-entropy of
    more than 2048 classes takes the logits' gradient that the forward
    formed in its pass over the logits: the loss and the gradient equal,
    bit for bit, those of the separate forward and backward passes (an
    explicit seed of 1 and a root that is not the loss take those), and the
    oracle's within 1e-5 relative (RED).  `lead` shifts the rows off 16-byte
    alignment (the library then runs the two passes itself); 51201 classes
    exceed what one block keeps in registers, the same."""
    r = np.random.default_rng(rows * 7 + cols + lead)
    full = f32(r.standard_normal((rows, cols + lead)) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    t[::4] = -100
    t[1] = cols - 1
    t[2] = 0
    runs = []
    for how in ("implicit", "explicit", "not-root"):
        ft = torch.tensor(full, requires_grad=True)
        loss = torch.F.cross_entropy(ft[:, lead:], torch.tensor(t), reduction=red)
        if how == "implicit":
            loss.backward()
        elif how == "explicit":
            loss.backward(torch.tensor(np.float32(1.0)))
        else:
            (loss * 1.0).backward()
        g = ft.grad.numpy()
        assert not g[:, :lead].any()
        runs.append((loss.numpy(), g[:, lead:]))
    for lo, g in runs[1:]:
        assert np.array_equal(lo, runs[0][0]) and np.array_equal(g, runs[0][1])
    xs = full[:, lead:]
    check(runs[0][0], ops.cross_entropy(xs, t, red), **RED)
    check(runs[0][1], ops.cross_entropy_backward(xs, t, np.float32(1.0), red), **RED)


def test_cross_entropy_seeded_gradient_used_once(torch):
    """A second backward through a retained graph gets the gradient from
    the backward kernel (the forward's is handed out once), and an
    unreduced or no-grad loss forms none."""
    r = np.random.default_rng(5)
    x = f32(r.standard_normal((8, 4099)))
    t = r.integers(0, 4099, 8).astype(np.int32)
    xt = torch.tensor(x, requires_grad=True)
    loss = torch.F.cross_entropy(xt, torch.tensor(t))
    loss.backward(retain_graph=True)
    g1 = xt.grad.numpy().copy()
    loss.backward()
    assert np.array_equal(xt.grad.numpy(), 2 * g1)
    with torch.no_grad():
        lo = torch.F.cross_entropy(xt, torch.tensor(t))
    assert lo.grad_fn is None
    check(lo.item(), ops.cross_entropy(x, t), **RED)


def test_nll_loss(torch):
    r = np.random.default_rng(11)
    lp = ops.log_softmax(r.standard_normal((9, 6))).astype(np.float32)
    t = r.integers(0, 6, 9).astype(np.int32)
    xt = torch.tensor(lp, requires_grad=True)
    loss = torch.F.nll_loss(xt, torch.tensor(t))
    loss.backward()
    check(loss.item(), ops.nll_loss(lp, t), **RED)
    check(xt.grad.numpy(), ops.nll_loss_backward(lp.shape, t), **RED)


# ------------------------------------------------------------------ layer norm


@pytest.mark.parametrize("rows,cols", [(8192, 768), (5, 33), (300, 3072), (7, 1024)])
def test_layer_norm(torch, rows, cols):
    r = np.random.default_rng(rows)
    x = f32(r.standard_normal((rows, cols)) * 2 + 0.5)
    w = f32(r.standard_normal(cols))
    b = f32(r.standard_normal(cols))
    out, g, (gx, gw, gb) = grad_of(
        torch, lambda a, ww, bb: torch.F.layer_norm(a, (cols,), ww, bb, 1e-5), x, w, b)
    y, _, _ = ops.layer_norm(x, w, b)
    check(out, y, **RED)
    dx, dw, db = ops.layer_norm_backward(g, x, w)
    check(gx, dx, **RED)
    check(gw, dw, **RED)
    check(gb, db, **RED)


# ------------------------------------------------------------------ embedding / indexing


@pytest.mark.parametrize("V,D,n", [(50257, 768, 8192), (7, 4, 6), (1000, 9, 20000), (3, 64, 1),
                                   (70, 16, 16384), (300000, 8, 16384), (1024, 768, 1024),
                                   (5000, 4, 70000)])
def test_embedding(torch, V, D, n):
    """Lookup and deterministic scatter-add backward.  Index lists up to
    65536 long are summed by workgroups that own row ranges (a row hit more
    often than one LDS list holds is summed in position chunks), longer ones
    after the bitonic sort.  Every row is the float32 sum of its dout rows in
    increasing position order, so the result equals np.add.at's bit for bit
    and untouched rows are exactly zero."""
    r = np.random.default_rng(V + n)
    w = f32(r.standard_normal((V, D)))
    ids = r.integers(0, V, n).astype(np.int32)
    ids[: n // 3] = ids[0] if n else 0  # a long run of one id
    wt = torch.tensor(w, requires_grad=True)
    out = torch.F.embedding(torch.tensor(ids), wt)
    assert np.array_equal(out.numpy(), w[ids])  # a gather: bit-exact
    g = f32(r.standard_normal((n, D)))
    out.backward(torch.tensor(g))
    want = ops.embedding_backward(g, ids, V)
    got = wt.grad.numpy()
    untouched = np.setdiff1d(np.arange(V), ids)
    assert np.all(got[untouched] == 0)  # exactly the referenced rows are written
    ref32 = np.zeros((V, D), np.float32)
    np.add.at(ref32, ids, g)  # float32 sums in position order
    assert np.array_equal(got, ref32)
    check_floor(got, want, ref32)
    # deterministic
    wt.grad = None
    out2 = torch.F.embedding(torch.tensor(ids), wt)
    out2.backward(torch.tensor(g))
    assert np.array_equal(wt.grad.numpy(), got)


@pytest.mark.parametrize("V,P,D,B,T,pos0", [(50257, 1024, 768, 8, 1024, 0), (97, 16, 64, 2, 16, 0),
                                              (211, 64, 128, 3, 40, 7), (30, 9, 6, 4, 5, 2),
                                              (1000, 1200, 768, 80, 1024, 100),
                                              (13, 5, 4, 1, 1, 4)])
def test_embedding_pos_against_oracle(torch, V, P, D, B, T, pos0):
    """F._embedding_pos: wte[ids] + wpe[pos0 + t] and both gradients in one
    launch.  The forward equals the two lookups and the add bit for bit; the
    token table's gradient is np.add.at's (float32, position order) bit for
    bit; each position row is its batch items' rows added in batch order
    (float32, exactly), rows outside [pos0, pos0 + T) zero; both against the
    oracle.  Widths not divisible by 4 take the scalar path, 80 x 1024 ids
    the sorting path for the token table."""
    r = np.random.default_rng(V + P + D + B)
    w = f32(r.standard_normal((V, D)))
    wp = f32(r.standard_normal((P, D)))
    ids = r.integers(0, V, (B, T)).astype(np.int32)
    ids[0, : T // 2] = ids[0, 0]
    wt = torch.tensor(w, requires_grad=True)
    wpt = torch.tensor(wp, requires_grad=True)
    out = torch.F._embedding_pos(torch.tensor(ids), wt, wpt, pos0)
    pos = pos0 + np.arange(T)
    want = w[ids] + wp[pos][None]
    assert np.array_equal(out.numpy(), want)  # the same float add
    g = f32(r.standard_normal((B, T, D)))
    out.backward(torch.tensor(g))
    tok32 = np.zeros((V, D), np.float32)
    np.add.at(tok32, ids.reshape(-1), g.reshape(-1, D))
    assert np.array_equal(wt.grad.numpy(), tok32)
    pos32 = np.zeros((P, D), np.float32)
    for b in range(B):
        pos32[pos] += g[b]
    assert np.array_equal(wpt.grad.numpy(), pos32)
    check_floor(wt.grad.numpy(), ops.embedding_backward(g.reshape(-1, D), ids.reshape(-1), V), tok32)
    check_floor(wpt.grad.numpy(),
                ops.embedding_backward(g.reshape(-1, D), np.tile(pos, B), P), pos32)


def test_embedding_pos_one_table_and_tied(torch):
    """Only the position table wanting a gradient (the token table frozen),
    and a token table tied to a Linear that ran after it: its rows are added
    into that layer's weight gradient in place, as embedding() does."""
    r = np.random.default_rng(3)
    V, P, D, B, T = 211, 64, 128, 3, 64
    w = f32(r.standard_normal((V, D)) * 0.1)
    wp = f32(r.standard_normal((P, D)))
    ids = r.integers(0, V, (B, T)).astype(np.int32)
    g = f32(r.standard_normal((B, T, D)))
    wt = torch.tensor(w)
    wpt = torch.tensor(wp, requires_grad=True)
    torch.F._embedding_pos(torch.tensor(ids), wt, wpt).backward(torch.tensor(g))
    assert wt.grad is None
    assert np.array_equal(wpt.grad.numpy(), g.sum(0, dtype=np.float32) if B == 1 else
                          (g[0] + g[1]) + g[2])
    wt = torch.tensor(w, requires_grad=True)
    x = torch.F._embedding_pos(torch.tensor(ids), wt, torch.tensor(wp))
    logits = torch.F.linear(x, wt)
    gl = f32(r.standard_normal((B, T, V)))
    logits.backward(torch.tensor(gl))
    x64 = w[ids].astype(np.float64) + wp[np.arange(T)][None]
    head = gl.reshape(-1, V).T.astype(np.float64) @ x64.reshape(-1, D)
    dx = gl.reshape(-1, V).astype(np.float64) @ w.astype(np.float64)
    want = head + ops.embedding_backward(dx, ids.reshape(-1), V)
    x32 = (w[ids] + wp[np.arange(T)][None]).reshape(-1, D)
    ref32 = gl.reshape(-1, V).T @ x32
    np.add.at(ref32, ids.reshape(-1), gl.reshape(-1, V) @ w)
    check_floor(wt.grad.numpy(), want, ref32)


@pytest.mark.parametrize("V,D,n", [(50257, 768, 8192), (1024, 768, 1024), (40, 5, 3000),
                                   (600, 8, 70000)])
def test_embedding_backward_accumulates_in_position_order(torch, V, D, n):
    """tjh_embedding_backward with accumulate = 1 (a table tied to the LM
    head): each referenced row becomes prior + dout rows in increasing
    position order, bit for bit; the other rows keep their prior values."""
    from torchjs_amd import _lib as L
    r = np.random.default_rng(n + 5)
    prior = f32(r.standard_normal((V, D)))
    ids = r.integers(-3, V + 3, n).astype(np.int32)  # out-of-range ids clamp
    ids[n // 2: n // 2 + n // 4] = V // 2
    g = f32(r.standard_normal((n, D)))
    dw = torch.tensor(prior)
    gt, it = torch.tensor(g), torch.tensor(ids)
    rc = L.lib().tjh_embedding_backward(gt.data_ptr(), it.data_ptr(), n, D, dw.data_ptr(), V, 1)
    assert rc == 0, L.lib().tjh_last_error()
    want = prior.copy()
    np.add.at(want, np.clip(ids, 0, V - 1), g)
    assert np.array_equal(dw.numpy(), want)


def test_embedding_tied_to_lm_head(torch):
    """A table used by an embedding lookup and as the weight of the output
    projection (GPT-2's tied wte): the embedding backward adds its rows into
    the projection's weight gradient in place; the result matches the sum
    of both gradients (and the unfused path) within tolerance."""
    T = _tensor_module()
    r = np.random.default_rng(31)
    V, D, n = 500, 32, 300
    w = f32(r.standard_normal((V, D)) * 0.1)
    ids = r.integers(0, V, n).astype(np.int32)
    g = f32(r.standard_normal((n, V)))
    got = []
    for fuse in (True, False):
        T._FUSE_ACC = fuse
        try:
            wt = torch.tensor(w, requires_grad=True)
            x = torch.F.embedding(torch.tensor(ids), wt)
            y = torch.F.linear(x * 1.5, wt)
            y.backward(torch.tensor(g))
            got.append(wt.grad.numpy())
        finally:
            T._FUSE_ACC = True
    xd = 1.5 * w[ids].astype(np.float64)
    d_head = g.astype(np.float64).T @ xd
    d_emb = ops.embedding_backward(1.5 * (g.astype(np.float64) @ w.astype(np.float64)), ids, V)
    check(got[0], d_head + d_emb, **RED)
    check(got[0], got[1], **RED)


def test_embedding_clamps_ids(torch):
    w = f32(np.arange(12).reshape(4, 3))
    out = torch.F.embedding(torch.tensor(np.array([-5, 0, 3, 99], dtype=np.int32)),
                            torch.tensor(w))
    assert np.array_equal(out.numpy(), w[[0, 0, 3, 3]])


def test_index_select_gather_nonzero_one_hot(torch):
    r = np.random.default_rng(12)
    x = f32(r.standard_normal((4, 5, 3)))
    idx = np.array([4, 0, 4, 2], dtype=np.int32)
    out, g, (gx,) = grad_of(torch, lambda t: t.index_select(1, torch.tensor(idx)), x)
    assert np.array_equal(out, ops.index_select(x, 1, idx).astype(np.float32))
    check(gx, ops.index_select_backward(g, x.shape, 1, idx), **RED)
    # PyTorch's contract: negative or too large indices raise (no kernel runs)
    for bad in ([0, -1], [5]):
        with pytest.raises(IndexError):
            torch.tensor(x).index_select(1, torch.tensor(np.array(bad, dtype=np.int32)))
    # advanced indexing still wraps negatives once
    assert np.array_equal(torch.tensor(x)[torch.tensor(np.array([-1, 0], dtype=np.int32))].numpy(),
                          x[[-1, 0]])
    gidx = r.integers(-5, 5, (4, 6, 3)).astype(np.int32)
    out, g, (gx,) = grad_of(torch, lambda t: t.gather(1, torch.tensor(gidx)), x)
    assert np.array_equal(out, ops.gather(x, 1, gidx).astype(np.float32))
    check(gx, ops.scatter_add(x.shape, 1, gidx, g), **RED)
    z = f32(r.integers(0, 3, (7, 11)) * (r.random((7, 11)) > 0.6))
    assert np.array_equal(torch.tensor(z).nonzero().numpy(), ops.nonzero(z))
    assert torch.tensor(np.zeros((3, 3), np.float32)).nonzero().shape == (0, 2)
    big = f32(r.random(100000) > 0.999)
    assert np.array_equal(torch.tensor(big).nonzero().numpy(), ops.nonzero(big))
    xf = np.array([0.5, 2.4, -1, 7, 1.5], dtype=np.float32)
    assert np.array_equal(torch.F.one_hot(torch.tensor(xf), 4).numpy(), ops.one_hot(xf, 4))
    xi = np.array([0, 2, 4], dtype=np.int32)
    assert np.array_equal(torch.F.one_hot(torch.tensor(xi)).numpy(), ops.one_hot(xi))


# ------------------------------------------------------------------ GEMM


def _raw_gemm(torch, ta, tb, A, B, M, N, K, alpha=1.0, beta=0.0, C0=None, bias=None, bmode=0):
    from torchjs_amd import _lib as L
    a = torch.tensor(A)
    b = torch.tensor(B)
    c = torch.tensor(C0 if C0 is not None else np.zeros((M, N), np.float32))
    bb = torch.tensor(bias) if bias is not None else None
    lda = A.shape[1]
    ldb = B.shape[1]
    L.check(L.lib().tjh_gemm(ta, tb, M, N, K, alpha, a.data_ptr(), lda, 0, b.data_ptr(), ldb, 0,
                             beta, c.data_ptr(), N, 0, 1, bb.data_ptr() if bb else None, bmode))
    return c.numpy()


@pytest.mark.parametrize("M,N,K", [(67, 45, 23), (128, 128, 16), (256, 384, 768), (1, 1, 1),
                                   (64, 10, 784), (130, 257, 129), (64, 64, 8192),
                                   (768, 768, 8192)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_layouts(torch, M, N, K, ta, tb):
    r = np.random.default_rng(M * 7 + N * 3 + K)
    A = f32(r.standard_normal((K, M) if ta else (M, K)))
    B = f32(r.standard_normal((N, K) if tb else (K, N)))
    want = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    got = _raw_gemm(torch, ta, tb, A, B, M, N, K)
    check_floor(got, want, (A.T if ta else A) @ (B.T if tb else B))


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "256x256",
                                  "256x128w4", "256x192"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(300, 260, 200), (256, 128, 4096)])
def test_gemm_every_tile(torch, monkeypatch, tile, ta, tb, M, N, K):
    # every tile on both kernels: an interior block (K steps of 32), edge
    # strips and a K remainder (first shape), split-K on one tile (second)
    monkeypatch.setenv("TJH_GEMM_TILE", tile)
    r = np.random.default_rng(M + N + K + ta * 2 + tb)
    A = f32(r.standard_normal((K, M) if ta else (M, K)))
    B = f32(r.standard_normal((N, K) if tb else (K, N)))
    bias = f32(r.standard_normal(N))
    C0 = f32(r.standard_normal((M, N)))
    want = 0.5 * ((A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64))
    want += 0.25 * C0 + bias
    got = _raw_gemm(torch, ta, tb, A, B, M, N, K, alpha=0.5, beta=0.25, C0=C0, bias=bias, bmode=1)
    ref32 = np.float32(0.5) * ((A.T if ta else A) @ (B.T if tb else B)) + np.float32(0.25) * C0 + bias
    check_floor(got, want, ref32)


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "256x256",
                                  "256x128w4", "256x192"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_odd_strides_every_tile(torch, monkeypatch, tile, ta, tb):
    """Operands whose rows start at any 4-byte boundary (odd row strides,
    base pointers one float past a 16-byte boundary) load 128 bits per
    access in the unguarded interior kernel: every tile and layout, with an
    interior block, edge strips and a K remainder."""
    from torchjs_amd import _lib as L
    monkeypatch.setenv("TJH_GEMM_TILE", tile)
    M, N, K = 300, 260, 203
    r = np.random.default_rng(M + N + K + 2 * ta + tb)
    ar, ac = (K, M) if ta else (M, K)
    br, bc = (N, K) if tb else (K, N)
    lda, ldb = ac + 3, bc + 1  # odd row strides
    Ab = f32(r.standard_normal(1 + ar * lda))
    Bb = f32(r.standard_normal(1 + br * ldb))
    A = Ab[1:].reshape(ar, lda)[:, :ac]
    B = Bb[1:].reshape(br, ldb)[:, :bc]
    a, b = torch.tensor(Ab), torch.tensor(Bb)
    c = torch.tensor(np.zeros((M, N), np.float32))
    L.check(L.lib().tjh_gemm(ta, tb, M, N, K, 1.0, a.data_ptr() + 4, lda, 0, b.data_ptr() + 4,
                             ldb, 0, 0.0, c.data_ptr(), N, 0, 1, None, 0), "gemm")
    opA, opB = (A.T if ta else A), (B.T if tb else B)
    check_floor(c.numpy(), opA.astype(np.float64) @ opB.astype(np.float64), opA @ opB)


@pytest.mark.parametrize("forced", [None, "256x256"])
def test_gemm_long_k_input_gradient(torch, monkeypatch, forced):
    """A . B with K = 50257 (the LM head's input gradient, dlogits . W), at
    2048 rows the planner takes the 256 x 256 tile over split K slices;
    forced, and by the planner, against float64 on the float32 floor."""
    if forced:
        monkeypatch.setenv("TJH_GEMM_TILE", forced)
    M, N, K = 2048, 768, 50257
    r = np.random.default_rng(50257)
    A = f32(r.standard_normal((M, K)) * 0.02)
    B = f32(r.standard_normal((K, N)) * 0.02)
    want = A.astype(np.float64) @ B.astype(np.float64)
    got = _raw_gemm(torch, 0, 0, A, B, M, N, K)
    check_floor(got, want, A @ B)


def test_gemm_vocab_rows_weight_gradient(torch):
    """A^T . B with vocabulary-sized M (the LM head's weight gradient,
    dlogits^T . x): the planner takes the 256 x 256 tile over two K slices
    here (M = 32768, K = 2048), against float64 on the float32 floor."""
    M, N, K = 32768, 768, 2048
    r = np.random.default_rng(32768)
    A = f32(r.standard_normal((K, M)) * 0.05)
    B = f32(r.standard_normal((K, N)))
    want = A.T.astype(np.float64) @ B.astype(np.float64)
    got = _raw_gemm(torch, 1, 0, A, B, M, N, K)
    check_floor(got, want, A.T @ B)


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "256x128w4",
                                  "256x192"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("M,N,K", [(300, 260, 200), (256, 128, 4096), (768, 192, 8192), (5, 3, 7)])
def test_gemm_row_sums(torch, monkeypatch, tile, ta, M, N, K):
    """bias_mode 3: the GEMM also writes sum_k op(A)[m][k] (a Linear bias
    gradient) -- interior and edge tiles, a K remainder, split-K."""
    from torchjs_amd import _lib as L
    monkeypatch.setenv("TJH_GEMM_TILE", tile)
    r = np.random.default_rng(M * 3 + N + K + ta)
    A = f32(r.standard_normal((K, M) if ta else (M, K)))
    B = f32(r.standard_normal((K, N)))
    a, b = torch.tensor(A), torch.tensor(B)
    c = torch.tensor(np.zeros((M, N), np.float32))
    rs = torch.tensor(np.full(M, 7.0, np.float32))  # written, not accumulated
    L.check(L.lib().tjh_gemm(ta, 0, M, N, K, 1.0, a.data_ptr(), A.shape[1], 0, b.data_ptr(), N,
                             0, 0.0, c.data_ptr(), N, 0, 1, rs.data_ptr(), 3), "gemm")
    opA = (A.T if ta else A).astype(np.float64)
    check_floor(c.numpy(), opA @ B.astype(np.float64), (A.T if ta else A) @ B)
    check_floor(rs.numpy(), opA.sum(1), (A.T if ta else A).sum(1, dtype=np.float32))


def test_gemm_row_sums_unaligned(torch):
    """bias_mode 3 through the guarded path (operand rows not 16-byte aligned)."""
    from torchjs_amd import _lib as L
    r = np.random.default_rng(21)
    M, N, K = 37, 29, 1001
    A = f32(r.standard_normal((K, M + 1)))  # row stride M + 1 = 38: unaligned rows
    B = f32(r.standard_normal((K, N)))
    a, b = torch.tensor(A), torch.tensor(B)
    c = torch.tensor(np.zeros((M, N), np.float32))
    rs = torch.tensor(np.zeros(M, np.float32))
    L.check(L.lib().tjh_gemm(1, 0, M, N, K, 1.0, a.data_ptr(), M + 1, 0, b.data_ptr(), N, 0, 0.0,
                             c.data_ptr(), N, 0, 1, rs.data_ptr(), 3), "gemm")
    opA = A[:, :M].T.astype(np.float64)
    check(c.numpy(), opA @ B.astype(np.float64), **RED)
    check(rs.numpy(), opA.sum(1), **RED)


def test_gemm_epilogue(torch):
    r = np.random.default_rng(13)
    M, N, K = 70, 90, 50
    A, B = f32(r.standard_normal((M, K))), f32(r.standard_normal((K, N)))
    C0 = f32(r.standard_normal((M, N)))
    bn, bm = f32(r.standard_normal(N)), f32(r.standard_normal(M))
    ref = A.astype(np.float64) @ B
    check(_raw_gemm(torch, 0, 0, A, B, M, N, K, 0.5, 2.0, C0), 0.5 * ref + 2 * C0, **RED)
    check(_raw_gemm(torch, 0, 0, A, B, M, N, K, bias=bn, bmode=1), ref + bn, **RED)
    check(_raw_gemm(torch, 0, 0, A, B, M, N, K, bias=bm, bmode=2), ref + bm[:, None], **RED)
    # split-K path with beta and bias
    M, N, K = 64, 96, 6000
    A, B = f32(r.standard_normal((M, K))), f32(r.standard_normal((K, N)))
    C0 = f32(r.standard_normal((M, N)))
    bn = f32(r.standard_normal(N))
    ref = A.astype(np.float64) @ B
    check_floor(_raw_gemm(torch, 0, 0, A, B, M, N, K, 1.0, 1.0, C0, bn, 1), ref + C0 + bn,
                (A @ B + C0) + bn)


def test_matmul_autograd_batched_broadcast(torch):
    r = np.random.default_rng(14)
    a = f32(r.standard_normal((2, 3, 4, 5)))
    b = f32(r.standard_normal((3, 5, 6)))
    out, g, (ga, gb) = grad_of(torch, lambda x, y: x @ y, a, b)
    check(out, a.astype(np.float64) @ b, **RED)
    ra, rb = ops.matmul_backward(g, a, b)
    check(ga, ra, **RED)
    check(gb, rb, **RED)
    # 2-D, vector and transposed-view operands
    m = f32(r.standard_normal((9, 7)))
    v = f32(r.standard_normal(7))
    out, g, (gm, gv) = grad_of(torch, lambda x, y: x @ y, m, v)
    check(out, m.astype(np.float64) @ v, **RED)
    check(gm, np.outer(g, v), **RED)
    check(gv, m.T.astype(np.float64) @ g, **RED)
    out, g, (gm,) = grad_of(torch, lambda x: x.t() @ x, m)
    check(out, m.T.astype(np.float64) @ m, **RED)
    check(gm, m.astype(np.float64) @ (g + g.T), **RED)
    assert torch.tensor([[1., 2.], [3., 4.]]).matmul(torch.tensor([[5., 6.], [7., 8.]])).tolist() \
        == [[19., 22.], [43., 50.]]


@pytest.mark.parametrize("lead,fin,fout", [((64,), 784, 256), ((8, 128), 768, 2304),
                                           ((3, 5), 7, 10), ((4,), 768, 50257)])
def test_linear(torch, lead, fin, fout):
    r = np.random.default_rng(fin + fout)
    x = f32(r.standard_normal(lead + (fin,)))
    w = f32(r.standard_normal((fout, fin)) * 0.05)
    b = f32(r.standard_normal(fout))
    out, g, (gx, gw, gb) = grad_of(torch, lambda a, ww, bb: torch.F.linear(a, ww, bb), x, w, b)
    x2, g2 = x.reshape(-1, fin), g.reshape(-1, fout)
    check_floor(out, ops.linear(x, w, b), x @ w.T + b)
    dx, dw, db = ops.linear_backward(g, x, w)
    check_floor(gx, dx, (g2 @ w).reshape(gx.shape))
    check_floor(gw, dw, g2.T @ x2)
    check_floor(gb, db, g2.sum(0))


# ------------------------------------------------------------------ attention


@pytest.mark.parametrize("B,H,T,D,causal", [(2, 3, 7, 8, False), (2, 3, 7, 8, True),
                                            (1, 12, 130, 64, True), (2, 2, 256, 64, False),
                                            (1, 1, 1, 64, True)])
def test_sdpa(torch, B, H, T, D, causal):
    r = np.random.default_rng(B * T + D)
    q, k, v = (f32(r.standard_normal((B, H, T, D))) for _ in range(3))
    out, g, (dq, dk, dv) = grad_of(
        torch, lambda a, b_, c: torch.F.scaled_dot_product_attention(a, b_, c, is_causal=causal),
        q, k, v)
    o, _ = ops.sdpa(q, k, v, causal)
    check(out, o, rtol=1e-4, atol=1e-5)
    rq, rk, rv = ops.sdpa_backward(g, q, k, v, causal)
    check(dq, rq, **RED)
    check(dk, rk, **RED)
    check(dv, rv, **RED)


def test_sdpa_on_qkv_views(torch):
    """q/k/v as head-split views of one [B,T,3C] projection (GPT-2 layout)."""
    r = np.random.default_rng(15)
    B, T, H, hd = 2, 33, 4, 16
    C = H * hd
    qkv = f32(r.standard_normal((B, T, 3 * C)))

    def fn(t):
        q, k, v = t.split(C, dim=2)
        sh = lambda z: z.view(B, T, H, hd).transpose(1, 2)
        y = torch.F.scaled_dot_product_attention(sh(q), sh(k), sh(v), is_causal=True)
        return y.transpose(1, 2).contiguous().view(B, T, C)
    out, g, (gqkv,) = grad_of(torch, fn, qkv)
    qa, ka, va = np.split(qkv.astype(np.float64), 3, axis=-1)
    sh = lambda z: z.reshape(B, T, H, hd).transpose(0, 2, 1, 3)
    o, _ = ops.sdpa(sh(qa), sh(ka), sh(va), True)
    check(out, o.transpose(0, 2, 1, 3).reshape(B, T, C), rtol=1e-4, atol=1e-5)
    gq, gk, gv = ops.sdpa_backward(sh(g.astype(np.float64)), sh(qa), sh(ka), sh(va), True)
    un = lambda z: z.transpose(0, 2, 1, 3).reshape(B, T, C)
    check(gqkv, np.concatenate([un(gq), un(gk), un(gv)], -1), **RED)


@pytest.mark.parametrize("T,causal", [(77, True), (77, False), (1024, True), (33, True)])
def test_sdpa_flash_gpt2_layout(torch, T, causal):
    """Head dim 64 (the flash kernels) on [B,T,3C] projection views, with
    sequence lengths that are not multiples of the 32-row tiles."""
    r = np.random.default_rng(T)
    B, H, hd = (1, 2, 64) if T >= 1024 else (2, 3, 64)
    C = H * hd
    qkv = f32(r.standard_normal((B, T, 3 * C)))

    def fn(t):
        q, k, v = t.split(C, dim=2)
        sh = lambda z: z.view(B, T, H, hd).transpose(1, 2)
        y = torch.F.scaled_dot_product_attention(sh(q), sh(k), sh(v), is_causal=causal)
        return y.transpose(1, 2).contiguous().view(B, T, C)
    out, g, (gqkv,) = grad_of(torch, fn, qkv)
    qa, ka, va = np.split(qkv.astype(np.float64), 3, axis=-1)
    sh = lambda z: z.reshape(B, T, H, hd).transpose(0, 2, 1, 3)
    o, _ = ops.sdpa(sh(qa), sh(ka), sh(va), causal)
    check(out, o.transpose(0, 2, 1, 3).reshape(B, T, C), rtol=1e-4, atol=1e-5)
    gq, gk, gv = ops.sdpa_backward(sh(g.astype(np.float64)), sh(qa), sh(ka), sh(va), causal)
    un = lambda z: z.transpose(0, 2, 1, 3).reshape(B, T, C)
    check(gqkv, np.concatenate([un(gq), un(gk), un(gv)], -1), **RED)


@pytest.mark.parametrize("Tq,Tk,causal", [(50, 97, True), (130, 64, True), (45, 200, False),
                                          (257, 33, False)])
def test_sdpa_flash_cross_lengths(torch, Tq, Tk, causal):
    """Head dim 64 with different, ragged query and key lengths: the dS
    blocks the key kernel stores cover exactly what the query kernel reads."""
    r = np.random.default_rng(Tq * 1000 + Tk)
    B, H, D = 2, 3, 64
    q = f32(r.standard_normal((B, H, Tq, D)))
    k = f32(r.standard_normal((B, H, Tk, D)))
    v = f32(r.standard_normal((B, H, Tk, D)))
    out, g, (gq, gk, gv) = grad_of(
        torch, lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=causal),
        q, k, v)
    f64 = lambda z: z.astype(np.float64)
    o, _ = ops.sdpa(f64(q), f64(k), f64(v), causal)
    check(out, o, rtol=1e-4, atol=1e-5)
    wq, wk, wv = ops.sdpa_backward(f64(g), f64(q), f64(k), f64(v), causal)
    check(gq, wq, **RED)
    check(gk, wk, **RED)
    check(gv, wv, **RED)


@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_flash_recompute_path(torch, monkeypatch, causal):
    """The query-block kernel that recomputes S and dP (used when the dS
    blocks cannot be allocated) agrees with the stored-dS path."""
    r = np.random.default_rng(5 + causal)
    q, k, v = (f32(r.standard_normal((1, 2, 97, 64))) for _ in range(3))
    fn = lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=causal)
    _, _, stored = grad_of(torch, fn, q, k, v)
    monkeypatch.setenv("TJH_SDPA_RECOMPUTE", "1")
    _, _, recomputed = grad_of(torch, fn, q, k, v)
    for s_, r_ in zip(stored, recomputed):
        check(r_, s_, rtol=1e-4, atol=1e-5)
    assert not np.array_equal(stored[0], recomputed[0])  # two different paths ran


def _sdpa_families(torch, fn):
    """Runs fn with kernel timing on; returns {family: launches}."""
    torch.hip.kernel_timing(True)
    torch.hip.kernel_timing_reset()
    try:
        fn()
        return dict((f, torch.hip.kernel_time(f)[0]) for f in torch.hip.kernel_families())
    finally:
        torch.hip.kernel_timing(False)


@pytest.mark.parametrize("D", [4, 16, 32, 40, 60, 96, 100, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_flash_head_dims(torch, D, causal):
    """Head dims other than 64 on the flash kernels (compiled for 32, 64,
    96 and 128; a smaller D reads its padded columns as zero), ragged and
    cross lengths, against the oracle; the composed path must not run."""
    Tq, Tk = (77, 77) if causal else (45, 130)
    r = np.random.default_rng(D * 10 + causal)
    B, H = 2, 3
    q = f32(r.standard_normal((B, H, Tq, D)))
    k = f32(r.standard_normal((B, H, Tk, D)))
    v = f32(r.standard_normal((B, H, Tk, D)))
    fn = lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=causal)
    res = {}
    fams = _sdpa_families(torch, lambda: res.update(r=grad_of(torch, fn, q, k, v)))
    out, g, (gq, gk, gv) = res["r"]
    # family counts match by prefix: "sdpa_fwd" includes "sdpa_fwd_composite"
    assert fams.get("sdpa_fwd", 0) == 1 and fams.get("sdpa_bwd", 0) >= 1, fams
    assert fams.get("sdpa_fwd_composite", 0) == 0 and fams.get("sdpa_bwd_composite", 0) == 0, fams
    f64 = lambda z: z.astype(np.float64)
    o, _ = ops.sdpa(f64(q), f64(k), f64(v), causal)
    check(out, o, rtol=1e-4, atol=1e-5)
    wq, wk, wv = ops.sdpa_backward(f64(g), f64(q), f64(k), f64(v), causal)
    check(gq, wq, **RED)
    check(gk, wk, **RED)
    check(gv, wv, **RED)


@pytest.mark.parametrize("D", [20, 32, 96, 128])
def test_sdpa_flash_head_dims_recompute_path(torch, monkeypatch, D):
    """The four-product key kernel and the recomputing query kernel at each
    compiled head dim agree with the stored-dS path."""
    r = np.random.default_rng(300 + D)
    q, k, v = (f32(r.standard_normal((1, 2, 97, D))) for _ in range(3))
    fn = lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=True)
    _, _, stored = grad_of(torch, fn, q, k, v)
    monkeypatch.setenv("TJH_SDPA_RECOMPUTE", "1")
    _, _, recomputed = grad_of(torch, fn, q, k, v)
    for s_, r_ in zip(stored, recomputed):
        check(r_, s_, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("D", [96, 128])
def test_sdpa_flash_large_head_dim_full_length(torch, D):
    """T = 1024 causal at head dims 96 and 128 (every query block length of
    the cost-ranked placement), against the oracle."""
    r = np.random.default_rng(400 + D)
    B, H, T = 1, 2, 1024
    q, k, v = (f32(r.standard_normal((B, H, T, D))) for _ in range(3))
    out, g, (gq, gk, gv) = grad_of(
        torch, lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=True),
        q, k, v)
    f64 = lambda z: z.astype(np.float64)
    o, _ = ops.sdpa(f64(q), f64(k), f64(v), True)
    check(out, o, rtol=1e-4, atol=1e-5)
    wq, wk, wv = ops.sdpa_backward(f64(g), f64(q), f64(k), f64(v), True)
    check(gq, wq, **RED)
    check(gk, wk, **RED)
    check(gv, wv, **RED)


@pytest.mark.parametrize("D", [6, 160])
def test_sdpa_composed_path_head_dims(torch, D):
    """Head dims the flash kernels do not take (not a multiple of 4, or
    above 128) run the GEMM-composed path, against the oracle."""
    r = np.random.default_rng(500 + D)
    q, k, v = (f32(r.standard_normal((2, 2, 40, D))) for _ in range(3))
    fn = lambda a, b, c: torch.F.scaled_dot_product_attention(a, b, c, is_causal=True)
    res = {}
    fams = _sdpa_families(torch, lambda: res.update(r=grad_of(torch, fn, q, k, v)))
    out, g, (gq, gk, gv) = res["r"]
    # family counts match by prefix: "sdpa_fwd" includes "sdpa_fwd_composite"
    assert fams.get("sdpa_fwd_composite", 0) >= 1, fams
    assert fams.get("sdpa_fwd", 0) == fams["sdpa_fwd_composite"], fams
    assert fams.get("sdpa_bwd", 0) == fams.get("sdpa_bwd_composite", 0) >= 1, fams
    f64 = lambda z: z.astype(np.float64)
    o, _ = ops.sdpa(f64(q), f64(k), f64(v), True)
    check(out, o, rtol=1e-4, atol=1e-5)
    wq, wk, wv = ops.sdpa_backward(f64(g), f64(q), f64(k), f64(v), True)
    check(gq, wq, **RED)
    check(gk, wk, **RED)
    check(gv, wv, **RED)


def test_split_and_narrow_gradients(torch):
    """Pieces of a split that are unused, overlapping narrows and a reused
    piece: the input gradient is the sum over every use (zero elsewhere)."""
    x = f32(np.random.default_rng(11).normal(size=(3, 10, 6)))
    t = torch.tensor(x, requires_grad=True)
    a, b, c = t.split([3, 5, 2], dim=1)
    n1 = t.narrow(1, 2, 4)  # overlaps a and b
    loss = (a * 2.0).sum() + (b * b).sum() + (n1 * 3.0).sum() + a.sum()  # c unused, a twice
    loss.backward()
    want = np.zeros(x.shape)
    want[:, 0:3] += 3.0
    want[:, 3:8] += 2.0 * x[:, 3:8]
    want[:, 2:6] += 3.0
    check(t.grad.numpy(), want, **EW)
    # a split whose pieces all flow back tiles the input exactly
    t2 = torch.tensor(x, requires_grad=True)
    p, q, r = t2.split(2, dim=2)
    ((p * 1.0) + (q * 2.0) + (r * 3.0)).sum().backward()
    check(t2.grad.numpy(), np.repeat([[[1.0, 1.0, 2.0, 2.0, 3.0, 3.0]]], 3, 0).repeat(10, 1), **EW)


def test_sdpa_self_attention_same_tensor(torch):
    """q = k = v (one tensor used three times): the three gradients must add."""
    r = np.random.default_rng(16)
    B, H, T, D = 2, 3, 40, 64
    x = f32(r.standard_normal((B, H, T, D)))
    out, g, (gx,) = grad_of(torch, lambda t: torch.F.scaled_dot_product_attention(
        t, t, t, is_causal=True), x)
    xd = x.astype(np.float64)
    o, _ = ops.sdpa(xd, xd, xd, True)
    check(out, o, rtol=1e-4, atol=1e-5)
    gq, gk, gv = ops.sdpa_backward(g.astype(np.float64), xd, xd, xd, True)
    check(gx, gq + gk + gv, **RED)


def test_sdpa_attn_mask_errors(torch):
    """attn_mask together with is_causal is refused (PyTorch's contract), and
    a mask that does not broadcast against the scores raises."""
    q = torch.zeros(1, 1, 2, 4)
    with pytest.raises(RuntimeError, match="either attn_mask or is_causal"):
        torch.F.scaled_dot_product_attention(q, q, q, attn_mask=torch.ones(2, 2).bool(),
                                             is_causal=True)
    with pytest.raises(ValueError, match="not broadcastable"):
        torch.F.scaled_dot_product_attention(q, q, q, attn_mask=torch.zeros(3, 5))


# ------------------------------------------------------------------ conv


@pytest.mark.parametrize("N,C,H,W,OC,k,s,p,d,grp", [
    (2, 3, 7, 6, 4, 3, 1, 1, 1, 1), (2, 4, 7, 6, 6, 3, 2, 1, 1, 1), (2, 4, 7, 6, 6, 3, 1, 2, 2, 2),
    (4, 3, 64, 64, 32, 3, 1, 1, 1, 1), (4, 32, 64, 64, 64, 3, 2, 1, 1, 1), (1, 2, 5, 5, 3, 1, 1, 0, 1, 1)])
def test_conv2d(torch, N, C, H, W, OC, k, s, p, d, grp):
    r = np.random.default_rng(N * C + OC)
    x = f32(r.standard_normal((N, C, H, W)))
    w = f32(r.standard_normal((OC, C // grp, k, k)) * 0.2)
    b = f32(r.standard_normal(OC))
    out, g, (gx, gw, gb) = grad_of(
        torch, lambda a, ww, bb: torch.F.conv2d(a, ww, bb, s, p, d, grp), x, w, b)
    y32, (dx32, dw32, db32) = _conv_f32(x, w, b, g, s, p, d, grp)
    check_floor(out, ops.conv2d(x, w, b, s, p, d, grp), y32)
    dx, dw, db = ops.conv2d_backward(g, x, w, s, p, d, grp)
    check_floor(gx, dx, dx32)
    check_floor(gw, dw, dw32)
    check_floor(gb, db, db32)


def _conv_f32(x, w, b, g, s, p, d, grp):
    """The same convolution and its gradients in float32 on the CPU
    (PyTorch's CPU path, a library routine): the float32 floor."""
    import torch as cpu
    tx, tw, tb = (cpu.tensor(a, requires_grad=True) for a in (x, w, b))
    y = cpu.nn.functional.conv2d(tx, tw, tb, s, p, d, grp)
    y.backward(cpu.tensor(g))
    return y.detach().numpy(), (tx.grad.numpy(), tw.grad.numpy(), tb.grad.numpy())


@pytest.mark.parametrize("N,C,H,W,OC,kh,kw,s,p,d,grp", [
    (2, 4, 9, 11, 6, 2, 3, (2, 1), (0, 1), (1, 2), 2),   # rectangular everything, groups
    (3, 5, 8, 8, 7, 3, 1, (3, 2), (2, 0), (2, 1), 1),    # stride 3 skips input rows
    (1, 6, 13, 5, 6, 3, 3, 1, 1, 1, 6),                  # depthwise
    (5, 33, 12, 12, 130, 3, 3, 1, 1, 1, 1),              # M, N and K edges of every tile
    (2, 3, 10, 9, 4, 2, 2, 3, 0, 1, 1),                  # kernel < stride: untouched pixels
    (3, 8, 15, 14, 5, 5, 3, (2, 3), (2, 1), 1, 1)])      # stride classes of unequal size
def test_conv2d_shapes(torch, N, C, H, W, OC, kh, kw, s, p, d, grp):
    r = np.random.default_rng(N * 100 + C + OC)
    x = f32(r.standard_normal((N, C, H, W)))
    w = f32(r.standard_normal((OC, C // grp, kh, kw)) * 0.2)
    b = f32(r.standard_normal(OC))
    out, g, (gx, gw, gb) = grad_of(
        torch, lambda a, ww, bb: torch.F.conv2d(a, ww, bb, s, p, d, grp), x, w, b)
    check(out, ops.conv2d(x, w, b, s, p, d, grp), **RED)
    dx, dw, db = ops.conv2d_backward(g, x, w, s, p, d, grp)
    check(gx, dx, **RED)
    check(gw, dw, **RED)
    check(gb, db, **RED)


@pytest.mark.parametrize("N,H", [(2, 9), (16, 64)])  # one K slice, and a split K
def test_conv2d_weight_grad_accumulates(torch, N, H):
    """tjh_conv2d_backward_weight with accumulate != 0 adds into dW."""
    import ctypes
    from torchjs_amd import _lib as L
    r = np.random.default_rng(N + H)
    C, OC, k = 3, 8, 3
    x = f32(r.standard_normal((N, C, H, H)))
    g = f32(r.standard_normal((N, OC, H, H)))
    w = f32(r.standard_normal((OC, C, k, k)))
    dw0 = f32(r.standard_normal((OC, C, k, k)))
    desc = L.Conv2dDesc(N, C, H, H, OC, k, k, 1, 1, 1, 1, 1, 1, 1, H, H)
    xt, gt, dwt = torch.tensor(x), torch.tensor(g), torch.tensor(dw0)
    L.check(L.lib().tjh_conv2d_backward_weight(ctypes.byref(desc), gt.data_ptr(), xt.data_ptr(),
                                               dwt.data_ptr(), 1), "conv2d_backward_weight")
    _, want, _ = ops.conv2d_backward(g, x, w, 1, 1, 1, 1)
    # dW sums N*H*H products: compared on the float32 floor of that sum
    _, (_, dw32, _) = _conv_f32(x, w, np.zeros(OC, np.float32), g, 1, 1, 1, 1)
    check_floor(dwt.numpy(), dw0 + want, dw0.astype(np.float64) + dw32)


@pytest.mark.parametrize("N,C,H,OC,s,grp,acc", [(2, 3, 9, 8, 1, 1, 0), (16, 3, 64, 32, 1, 1, 1),
                                                 (8, 32, 32, 64, 2, 1, 0), (4, 8, 17, 12, 2, 4, 1)])
def test_conv2d_weight_and_bias_grad_in_one_pass(torch, N, C, H, OC, s, grp, acc):
    """tjh_conv2d_backward_weight_bias: dW bit-identical to
    tjh_conv2d_backward_weight (the same product), db = dy summed over
    images and pixels (the row sums of the product's dy operand, in split
    order), with one K slice and with a split K, groups, and accumulate."""
    import ctypes
    from torchjs_amd import _lib as L
    r = np.random.default_rng(N * 7 + OC + s)
    k = 3
    oh = (H + 2 - k) // s + 1
    x = f32(r.standard_normal((N, C, H, H)))
    g = f32(r.standard_normal((N, OC, oh, oh)))
    dw0 = f32(r.standard_normal((OC, C // grp, k, k)))
    db0 = f32(r.standard_normal(OC))
    desc = L.Conv2dDesc(N, C, H, H, OC, k, k, s, s, 1, 1, 1, 1, grp, oh, oh)
    xt, gt = torch.tensor(x), torch.tensor(g)
    dwa, dwb, dbt = torch.tensor(dw0), torch.tensor(dw0), torch.tensor(db0)
    L.check(L.lib().tjh_conv2d_backward_weight(ctypes.byref(desc), gt.data_ptr(), xt.data_ptr(),
                                               dwa.data_ptr(), acc), "conv2d_backward_weight")
    L.check(L.lib().tjh_conv2d_backward_weight_bias(ctypes.byref(desc), gt.data_ptr(),
                                                    xt.data_ptr(), dwb.data_ptr(),
                                                    dbt.data_ptr(), acc),
            "conv2d_backward_weight_bias")
    assert np.array_equal(dwa.numpy(), dwb.numpy())
    want = g.astype(np.float64).sum(axis=(0, 2, 3)) + (db0 if acc else 0)
    check(dbt.numpy(), want, **RED)
    # deterministic
    dbt2 = torch.tensor(db0)
    L.check(L.lib().tjh_conv2d_backward_weight_bias(ctypes.byref(desc), gt.data_ptr(),
                                                    xt.data_ptr(), dwb.data_ptr(),
                                                    dbt2.data_ptr(), acc),
            "conv2d_backward_weight_bias")
    assert np.array_equal(dbt.numpy(), dbt2.numpy())


@pytest.mark.parametrize("N,C,H,OC,s,p,grp", [(4, 3, 17, 8, 1, 1, 1), (3, 8, 16, 12, 2, 1, 2),
                                               (2, 6, 9, 6, 1, 0, 3)])
def test_conv2d_relu_equals_conv_then_relu(torch, N, C, H, OC, s, p, grp):
    """F.conv2d_relu: the output, and the input, weight and bias gradients,
    equal F.relu(F.conv2d(...)) bit for bit."""
    r = np.random.default_rng(N * 100 + OC + s)
    x0 = f32(r.standard_normal((N, C, H, H)))
    w0 = f32(r.standard_normal((OC, C // grp, 3, 3)) * 0.3)
    b0 = f32(r.standard_normal(OC) * 0.3)
    outs = []
    for fused in (True, False):
        x, w, b = (torch.tensor(a, requires_grad=True) for a in (x0, w0, b0))
        if fused:
            y = torch.F.conv2d_relu(x, w, b, s, p, 1, grp)
        else:
            y = torch.F.relu(torch.F.conv2d(x, w, b, s, p, 1, grp))
        g = f32(np.random.default_rng(5).standard_normal(y.shape))
        y.backward(torch.tensor(g))
        outs.append([y.numpy(), x.grad.numpy(), w.grad.numpy(), b.grad.numpy()])
    for a_, b_ in zip(*outs):
        assert np.array_equal(a_, b_)
    assert (outs[0][0] == 0).any() and (outs[0][0] > 0).any()


# ------------------------------------------------------------------ optimizers


@pytest.mark.parametrize("cls,decoupled,wd", [("Adam", False, 0.0), ("Adam", False, 0.01),
                                              ("AdamW", True, 0.1), ("AdamW", True, 0.01)])
def test_adam_bit_exact(torch, cls, decoupled, wd):
    """The fused kernel reproduces the reference's rounding exactly: fp32
    moments, fp64 update rounded once."""
    r = np.random.default_rng(16)
    shapes = [(257, 31), (4096,), (3,), (768, 768)]
    ps = [f32(r.standard_normal(s)) for s in shapes]
    params = [torch.tensor(p, requires_grad=True) for p in ps]
    opt = getattr(torch.optim, cls)(params, lr=1e-3, weight_decay=wd)
    ms = [np.zeros_like(p) for p in ps]
    vs = [np.zeros_like(p) for p in ps]
    for step in range(1, 4):
        gs = [f32(r.standard_normal(s)) for s in shapes]
        for t, g in zip(params, gs):
            t.grad = torch.tensor(g)
        opt.step()
        for i in range(len(ps)):
            ps[i], ms[i], vs[i] = ops.adam_step(ps[i], gs[i], ms[i], vs[i], step, lr=1e-3,
                                                weight_decay=wd, decoupled=decoupled)
    for t, p, m, v in zip(params, ps, ms, vs):
        st = opt.state[id(t)]
        # fp32 moments: bit-exact
        assert np.array_equal(st["exp_avg"].numpy(), m)
        assert np.array_equal(st["exp_avg_sq"].numpy(), v)
        # fp64 update rounded once: equal but for double-rounding ties
        got = t.numpy()
        assert (got == p).mean() > 0.999
        assert np.max(np.abs(got.astype(np.float64) - p)) <= np.abs(p).max() * 2 ** -23


# ------------------------------------------------------------------ fused MLP


@pytest.mark.parametrize("B,T,d_in,hid,d_out", [(4, 33, 70, 200, 70),     # edges + K remainder
                                               (1, 64, 2048, 128, 2048)])  # split K
@pytest.mark.parametrize("bias", [True, False])
def test_mlp_gelu_fused_equals_unfused(torch, B, T, d_in, hid, d_out, bias):
    """The MLP block with GELU fused into the GEMM epilogues reproduces
    linear -> gelu -> linear bit for bit, forward and backward."""
    r = np.random.default_rng(B * T + d_in + bias)
    x = f32(r.standard_normal((B, T, d_in)))
    w1 = f32(r.standard_normal((hid, d_in)) * 0.05)
    w2 = f32(r.standard_normal((d_out, hid)) * 0.05)
    b1 = f32(r.standard_normal(hid)) if bias else None
    b2 = f32(r.standard_normal(d_out)) if bias else None
    arrays = [a for a in (x, w1, b1, w2, b2) if a is not None]

    def fused(*ts):
        xx, ww1, *rest = ts
        bb1, ww2, bb2 = (rest[0], rest[1], rest[2]) if bias else (None, rest[0], None)
        return torch.F._mlp_gelu(xx, ww1, bb1, ww2, bb2)

    def unfused(*ts):
        xx, ww1, *rest = ts
        bb1, ww2, bb2 = (rest[0], rest[1], rest[2]) if bias else (None, rest[0], None)
        return torch.F.linear(torch.F.gelu(torch.F.linear(xx, ww1, bb1)), ww2, bb2)
    y1, g, grads1 = grad_of(torch, fused, *arrays)
    y2, _, grads2 = grad_of(torch, unfused, *arrays)
    assert np.array_equal(y1, y2)
    for a_, b_ in zip(grads1, grads2):
        assert np.array_equal(a_, b_)
    # and both match the oracle
    h = x.astype(np.float64) @ w1.T.astype(np.float64) + (b1 if bias else 0)
    want = ops.gelu(h) @ w2.T.astype(np.float64) + (b2 if bias else 0)
    check(y1, want, **RED)


@pytest.mark.parametrize("B,T,in_f,out_f,bias", [(2, 33, 64, 80, True), (1, 50, 50, 96, False),
                                                  (1, 64, 4096, 64, True), (2, 64, 768, 768, True)])
def test_linear_add_equals_unfused(torch, B, T, in_f, out_f, bias):
    """residual + linear(x) with the add in the GEMM epilogue (K remainder,
    split-K and edge tiles included) reproduces linear followed by the add
    bit for bit, forward and backward."""
    r = np.random.default_rng(B * T + in_f + out_f)
    x = f32(r.standard_normal((B, T, in_f)))
    w = f32(r.standard_normal((out_f, in_f)) * 0.05)
    b = f32(r.standard_normal(out_f)) if bias else None
    res = f32(r.standard_normal((B, T, out_f)))
    arrays = [a for a in (x, w, b, res) if a is not None]

    def split(ts):
        return (ts[0], ts[1], ts[2], ts[3]) if bias else (ts[0], ts[1], None, ts[2])

    def fused(*ts):
        xx, ww, bb, rr = split(ts)
        return torch.F._linear_add(xx, ww, bb, rr)

    def unfused(*ts):
        xx, ww, bb, rr = split(ts)
        return rr + torch.F.linear(xx, ww, bb)
    y1, _, grads1 = grad_of(torch, fused, *arrays)
    y2, _, grads2 = grad_of(torch, unfused, *arrays)
    assert np.array_equal(y1, y2)
    for a_, b_ in zip(grads1, grads2):
        assert np.array_equal(a_, b_)
    want = res + x.astype(np.float64) @ w.T.astype(np.float64) + (b if bias else 0)
    check(y1, want, **RED)


@pytest.mark.parametrize("rows,cols", [(64, 768), (37, 300), (19, 1001), (8, 2000)])
def test_layer_norm_backward_folds_pending_gradient(torch, rows, cols):
    """x feeding both a LayerNorm and a residual add: the engine hands the
    add's gradient to the LayerNorm backward, which adds it in the same
    kernel (fast row kernel, odd widths and the general path); equal bit
    for bit to the separate add, and to the oracle within tolerance."""
    T = _tensor_module()
    r = np.random.default_rng(rows + cols)
    x0 = f32(r.standard_normal((rows, cols)))
    gm = f32(1 + 0.1 * r.standard_normal(cols))
    bt = f32(0.1 * r.standard_normal(cols))
    res = []
    for fuse in (True, False):
        T._FUSE_ACC = fuse
        try:
            ts = [torch.tensor(a, requires_grad=True) for a in (x0, gm, bt)]
            x = ts[0] * 2.0                      # non-leaf: its gradient is summed by the engine
            y = x + torch.F.layer_norm(x, (cols,), ts[1], ts[2])
            g = np.random.default_rng(5).standard_normal((rows, cols)).astype(np.float32)
            y.backward(torch.tensor(g))
            res.append([t.grad.numpy() for t in ts])
        finally:
            T._FUSE_ACC = True
    for a_, b_ in zip(*res):
        assert np.array_equal(a_, b_)
    dx, dgm, dbt = ops.layer_norm_backward(g, 2.0 * x0.astype(np.float64), gm)
    check(res[0][0], 2.0 * (g + dx), **RED)
    check(res[0][1], dgm, **RED)
    check(res[0][2], dbt, **RED)


def test_block_residual_fusion_equals_unfused(torch):
    """The pre-LN block with both residual adds in GEMM epilogues and the
    add of the residual stream's gradients folded into the LayerNorm
    backward gives the plain op-by-op block's output and gradients bit for
    bit."""
    from torchjs_amd import workloads as W
    T = _tensor_module()
    r = np.random.default_rng(7)
    Bn, Tn, d, H = 2, 40, 64, 4
    blk = W.Block(d, H)
    p0 = {k: f32(r.standard_normal(p.shape) * 0.1) for k, p in blk.named_parameters()}
    x0 = f32(r.standard_normal((Bn, Tn, d)))
    g = f32(r.standard_normal((Bn, Tn, d)))

    def plain(m, x):
        F = torch.F
        a = m.ln_1(x)
        q, k, v = m.attn.c_attn(a).split(d, dim=2)
        q, k, v = (t.view(Bn, Tn, H, d // H).transpose(1, 2) for t in (q, k, v))
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        y = y.transpose(1, 2).contiguous().view(Bn, Tn, d)
        x = x + m.attn.c_proj(y)
        hdn = F.gelu(m.mlp.c_fc(m.ln_2(x)))
        return x + m.mlp.c_proj(hdn)

    outs = []
    for mode in ("fused", "plain", "fused_noacc"):
        W.load_params(blk, p0)
        for prm in blk.parameters():
            prm.grad = None
        T._FUSE_ACC = mode != "fused_noacc"
        try:
            xl = torch.tensor(x0, requires_grad=True)
            xx = xl * 1.0
            y = plain(blk, xx) if mode == "plain" else blk(xx)
            y.backward(torch.tensor(g))
            outs.append([y.numpy(), xl.grad.numpy()] +
                        [prm.grad.numpy() for _, prm in blk.named_parameters()])
        finally:
            T._FUSE_ACC = True
    for other in outs[1:]:
        for a_, b_ in zip(outs[0], other):
            assert np.array_equal(a_, b_)


def test_layer_norm_deferred_weight_grads(torch):
    """LayerNorm weight gradients whose finishing pass the engine defers to
    one batched launch at the end of backward: a LayerNorm applied twice
    (its gamma/beta receive two contributions, forcing an early flush), a
    chain of LayerNorms and leaves with a .grad from an earlier backward;
    bit-identical to the undeferred engine, and to the oracle."""
    T = _tensor_module()
    r = np.random.default_rng(17)
    rows, cols = 96, 768
    x0 = f32(r.standard_normal((rows, cols)))
    gms = [f32(1 + 0.1 * r.standard_normal(cols)) for _ in range(3)]
    bts = [f32(0.1 * r.standard_normal(cols)) for _ in range(3)]
    g = f32(r.standard_normal((rows, cols)))
    runs = []
    for fuse in (True, False):
        T._FUSE_ACC = fuse
        try:
            ps = [torch.tensor(a, requires_grad=True) for a in gms + bts]
            x = torch.tensor(x0, requires_grad=True)
            F = torch.F
            h = F.layer_norm(x * 1.0, (cols,), ps[0], ps[3])
            h = F.layer_norm(h * 2.0, (cols,), ps[1], ps[4])
            h = F.layer_norm(h + x, (cols,), ps[0], ps[3])  # gamma/beta 0 used twice
            y = F.layer_norm(h, (cols,), ps[2], ps[5])
            y.backward(torch.tensor(g))
            first = [p.grad.numpy() for p in ps] + [x.grad.numpy()]
            y2 = F.layer_norm(F.layer_norm(x * 1.0, (cols,), ps[1], ps[4]), (cols,), ps[2], ps[5])
            y2.backward(torch.tensor(g))  # accumulates into existing .grad
            runs.append(first + [p.grad.numpy() for p in ps])
        finally:
            T._FUSE_ACC = True
    for a_, b_ in zip(*runs):
        assert np.array_equal(a_, b_)
    # last LayerNorm's gamma / beta gradients against the oracle
    hd = runs[0]  # first backward's grads
    _, dgm, dbt = ops.layer_norm_backward(g, _ln_chain_input(x0, gms, bts), gms[2])
    check(hd[2], dgm, **RED)
    check(hd[5], dbt, **RED)


def test_layer_norm_batched_finish_wide_rows(torch):
    """Eight LayerNorms of 3072 columns (the widest rows of the
    register-resident kernel): the batched finishing pass for their 16
    weight gradients and the per-LayerNorm passes of the undeferred engine
    agree bit for bit, also when a second backward accumulates into the
    existing .grad; the last LayerNorm's against the oracle."""
    T = _tensor_module()
    r = np.random.default_rng(23)
    rows, cols, n = 40, 3072, 8
    x0 = f32(r.standard_normal((rows, cols)))
    gms = [f32(1 + 0.1 * r.standard_normal(cols)) for _ in range(n)]
    bts = [f32(0.1 * r.standard_normal(cols)) for _ in range(n)]
    g = f32(r.standard_normal((rows, cols)))
    runs = []
    for fuse in (True, False):
        T._FUSE_ACC = fuse
        try:
            ps = [torch.tensor(a, requires_grad=True) for a in gms + bts]
            x = torch.tensor(x0, requires_grad=True)
            F = torch.F
            h = x * 1.0
            for i in range(n):
                h = F.layer_norm(h, (cols,), ps[i], ps[n + i])
            h.backward(torch.tensor(g))
            first = [p.grad.numpy() for p in ps]
            h = x * 1.0
            for i in range(n):
                h = F.layer_norm(h, (cols,), ps[i], ps[n + i])
            h.backward(torch.tensor(g))
            runs.append(first + [p.grad.numpy() for p in ps] + [x.grad.numpy()])
        finally:
            T._FUSE_ACC = True
    for a_, b_ in zip(*runs):
        assert np.array_equal(a_, b_)
    # the last LayerNorm's gamma / beta gradients against the oracle
    h = x0.astype(np.float64)
    for i in range(n - 1):
        h = ops.layer_norm(h, gms[i], bts[i])[0]
    _, dgm, dbt = ops.layer_norm_backward(g, h, gms[n - 1])
    check(runs[0][n - 1], dgm, **RED)
    check(runs[0][2 * n - 1], dbt, **RED)


def test_layer_norm_same_tensor_as_weight_and_bias(torch):
    """gamma and beta given as one tensor: its gradient is the sum of both
    (the engine does not defer a tensor that fills two of a node's slots)."""
    r = np.random.default_rng(23)
    rows, cols = 40, 768
    x0 = f32(r.standard_normal((rows, cols)))
    w0 = f32(1 + 0.1 * r.standard_normal(cols))
    g = f32(r.standard_normal((rows, cols)))
    x = torch.tensor(x0, requires_grad=True)
    w = torch.tensor(w0, requires_grad=True)
    torch.F.layer_norm(x * 1.0, (cols,), w, w).backward(torch.tensor(g))
    _, dgm, dbt = ops.layer_norm_backward(g, x0.astype(np.float64), w0)
    check(w.grad.numpy(), dgm + dbt, **RED)


def test_layer_norm_same_tensor_as_input_and_weight(torch):
    """layer_norm(w, (n,), w, b): the weight gradient is not deferred, since
    w also receives the input gradient from the same node; w.grad is the
    sum of both."""
    r = np.random.default_rng(29)
    n = 768
    w0 = f32(1 + 0.1 * r.standard_normal(n))
    b0 = f32(0.1 * r.standard_normal(n))
    g = f32(r.standard_normal(n))
    w = torch.tensor(w0, requires_grad=True)
    b = torch.tensor(b0, requires_grad=True)
    torch.F.layer_norm(w, (n,), w, b).backward(torch.tensor(g))
    dx, dgm, dbt = ops.layer_norm_backward(g[None], w0[None].astype(np.float64), w0)
    check(w.grad.numpy(), dx[0] + dgm, **RED)
    check(b.grad.numpy(), dbt, **RED)


@pytest.mark.parametrize("emb_first", [True, False])
def test_embedding_fold_never_writes_a_shared_gradient(torch, emb_first):
    """A non-leaf table W = 1.5 * W0 feeds both (W + L) * C and
    embedding(ids, W).  The add's VJP hands one gradient tensor to W and to
    the leaf L; the embedding's in-place row add may not use it, or L.grad
    would pick up the embedding rows."""
    r = np.random.default_rng(31)
    V, D, n = 37, 16, 50
    w0 = f32(r.standard_normal((V, D)))
    l0 = f32(r.standard_normal((V, D)))
    c0 = f32(r.standard_normal((V, D)))
    ids = r.integers(0, V, n).astype(np.int32)
    g1 = f32(r.standard_normal((V, D)))
    g2 = f32(r.standard_normal((n, D)))
    W0 = torch.tensor(w0, requires_grad=True)
    L = torch.tensor(l0, requires_grad=True)
    W = W0 * 1.5
    if emb_first:
        e = torch.F.embedding(torch.tensor(ids), W)
        a = (W + L) * torch.tensor(c0)
    else:
        a = (W + L) * torch.tensor(c0)
        e = torch.F.embedding(torch.tensor(ids), W)
    loss = (a * torch.tensor(g1)).sum() + (e * torch.tensor(g2)).sum()
    loss.backward()
    gw = c0.astype(np.float64) * g1 + ops.embedding_backward(g2, ids, V)
    check(L.grad.numpy(), c0.astype(np.float64) * g1, **RED)
    check(W0.grad.numpy(), 1.5 * gw, **RED)


def _ln_chain_input(x0, gms, bts):
    """The input of the last LayerNorm in test_layer_norm_deferred_weight_grads."""
    x = x0.astype(np.float64)
    h = ops.layer_norm(x, gms[0], bts[0])[0]
    h = ops.layer_norm(2.0 * h, gms[1], bts[1])[0]
    return ops.layer_norm(h + x, gms[0], bts[0])[0]


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "256x128w4",
                                  "256x192"])
@pytest.mark.parametrize("red", ["mean", "sum", "none"])
def test_gemm_ce_equals_stored_gradient(torch, monkeypatch, tile, red):
    """tjh_gemm_ce in both orientations (dx = dlogits W, dW = dlogits^T x)
    on every tile, with edge strips and a K remainder, padded logits rows,
    ignored and out-of-range targets: bit for bit tjh_cross_entropy_backward
    followed by tjh_gemm, and the oracle's products."""
    from torchjs_amd import _lib as L
    monkeypatch.setenv("TJH_GEMM_TILE", tile)
    r = np.random.default_rng(len(tile) * 10 + len(red))
    rows, cols, ld, N = 300, 1030, 1032, 200
    logits = f32(r.standard_normal((rows, ld)) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    t[::7] = -100
    t[3] = cols + 5  # out of range: a zero row, like an ignored one
    t[4] = cols - 1
    W = f32(r.standard_normal((cols, N)))
    X = f32(r.standard_normal((rows, N)))
    gl = f32(r.standard_normal(rows)) if red == "none" else f32([0.7])
    rc = {"none": 0, "mean": 1, "sum": 2}[red]
    xt, tt, wt, xx, gt = (torch.tensor(logits), torch.tensor(t), torch.tensor(W), torch.tensor(X),
                          torch.tensor(gl))
    lse, lrow, out = torch.empty((rows,)), torch.empty((rows,)), torch.empty(())
    L.check(L.lib().tjh_cross_entropy_forward(xt.data_ptr(), ld, tt.data_ptr(), rows, cols, -100,
                                              None, 0.0, lse.data_ptr(), lrow.data_ptr(), rc,
                                              out.data_ptr() if rc else None), "cross_entropy")
    d = torch.tensor(np.zeros((rows, ld), np.float32))
    L.check(L.lib().tjh_cross_entropy_backward(xt.data_ptr(), ld, tt.data_ptr(), None, 0.0,
                                               lse.data_ptr(), gt.data_ptr(), rows, cols, -100, rc,
                                               d.data_ptr(), ld, 0), "cross_entropy_backward")
    rs = torch.empty((rows,))
    L.check(L.lib().tjh_cross_entropy_row_scale(tt.data_ptr(), gt.data_ptr(), rows, cols, -100, rc,
                                                rs.data_ptr()), "cross_entropy_row_scale")

    def stored(ta, M, K, b):
        c = torch.tensor(np.zeros((M, N), np.float32))
        L.check(L.lib().tjh_gemm(ta, 0, M, N, K, 1.0, d.data_ptr(), ld, 0, b.data_ptr(), N, 0, 0.0,
                                 c.data_ptr(), N, 0, 1, None, 0), "gemm")
        return c.numpy()

    def formed(ta, M, K, b):
        c = torch.tensor(np.full((M, N), 7.0, np.float32))  # beta 0: overwritten
        L.check(L.lib().tjh_gemm_ce(ta, M, N, K, xt.data_ptr(), ld, lse.data_ptr(), tt.data_ptr(),
                                    rs.data_ptr(), b.data_ptr(), N, c.data_ptr(), N), "gemm_ce")
        return c.numpy()
    dx = formed(0, rows, cols, wt)
    dw = formed(1, cols, rows, xx)
    assert np.array_equal(dx, stored(0, rows, cols, wt))
    assert np.array_equal(dw, stored(1, cols, rows, xx))
    to = t.copy()
    to[3] = -100
    D = ops.cross_entropy_backward(logits[:, :cols], to, gl if red == "none" else gl[0], red)
    D32 = np.asarray(D, np.float32)
    check_floor(dx, D @ W.astype(np.float64), D32 @ W)
    check_floor(dw, D.T @ X.astype(np.float64), D32.T @ X)


@pytest.mark.parametrize("red", ["mean", "sum", "none"])
def test_lm_head_cross_entropy_formed_in_gemms(torch, monkeypatch, red):
    """A Linear LM head whose weight is also the input embedding (GPT-2's
    tied table) under cross_entropy: with the cross-entropy gradient formed
    inside the head's two GEMMs the input and table gradients equal those
    through the stored gradient bit for bit; autograd.grad and logits read
    by anything but a Linear take the stored gradient."""
    T = _tensor_module()
    r = np.random.default_rng(31 + len(red))
    B, Tn, D, V = 2, 50, 64, 1030
    ids = r.integers(0, V, (B, Tn)).astype(np.int32)
    tg = r.integers(0, V, (B * Tn,)).astype(np.int32)
    tg[::6] = -100
    W0 = f32(r.standard_normal((V, D)) * 0.1)
    h0 = f32(r.standard_normal((B, Tn, D)))
    calls = []
    real = T._gemm_ce
    monkeypatch.setattr(T, "_gemm_ce", lambda *a: calls.append(a[2]) or real(*a))
    F = torch.F

    def loss_of(W, h, head):
        x = F.embedding(torch.tensor(ids), W) + h
        logits = head(x, W)
        loss = F.cross_entropy(logits.view(-1, V), torch.tensor(tg), reduction=red)
        return loss.sum() if red == "none" else loss

    runs = []
    prev = T._FUSE_CE
    for fuse in (True, False):
        T._FUSE_CE = fuse
        try:
            W = torch.tensor(W0, requires_grad=True)
            h = torch.tensor(h0, requires_grad=True)
            loss_of(W, h, F.linear).backward()
            W2 = torch.tensor(W0, requires_grad=True)
            h2 = torch.tensor(h0, requires_grad=True)
            gh = torch.autograd.grad(loss_of(W2, h2, F.linear), [h2])[0]
            W3 = torch.tensor(W0, requires_grad=True)
            h3 = torch.tensor(h0, requires_grad=True)
            loss_of(W3, h3, lambda x, w: F.linear(x, w) * 1.0).backward()
            runs.append([W.grad.numpy(), h.grad.numpy(), gh.numpy(), W3.grad.numpy(),
                         h3.grad.numpy()])
        finally:
            T._FUSE_CE = prev
    assert sorted(calls) == [False, False, True, True]  # dx and dW, two formed backwards
    for a, b in zip(*runs):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "256x128w4",
                                  "256x192"])
def test_gemm_epilogue_activations_every_tile(torch, monkeypatch, tile):
    """The fused epilogues on every tile (interior, edge strips, K
    remainder): act 1 writes the pre-activation and GELU of it, act 2
    multiplies by GELU' of aux, act 3 adds aux; each equals the plain GEMM
    followed by the library's elementwise op, bit for bit."""
    from torchjs_amd import _lib as L
    monkeypatch.setenv("TJH_GEMM_TILE", tile)
    r = np.random.default_rng(5)
    M, N, K = 300, 260, 200
    A = f32(r.standard_normal((M, K)))
    B = f32(r.standard_normal((K, N)))
    bias = f32(r.standard_normal(N))
    aux0 = f32(r.standard_normal((M, N)))
    a, b, bt = torch.tensor(A), torch.tensor(B), torch.tensor(bias)

    def gemm(act, aux):
        c = torch.tensor(np.zeros((M, N), np.float32))
        if act:
            L.check(L.lib().tjh_gemm_act(0, 0, M, N, K, 1.0, a.data_ptr(), K, b.data_ptr(), N, 0.0,
                                         c.data_ptr(), N, bt.data_ptr(), 1, aux.data_ptr(), N, act),
                    "gemm_act")
        else:
            L.check(L.lib().tjh_gemm(0, 0, M, N, K, 1.0, a.data_ptr(), K, 0, b.data_ptr(), N, 0,
                                     0.0, c.data_ptr(), N, 0, 1, bt.data_ptr(), 1), "gemm")
        return c
    plain = gemm(0, None)
    h = torch.tensor(np.zeros((M, N), np.float32))
    y1 = gemm(1, h)
    assert np.array_equal(h.numpy(), plain.numpy())
    assert np.array_equal(y1.numpy(), torch.F.gelu(plain).numpy())
    aux = torch.tensor(aux0)
    y2 = gemm(2, aux)
    dg = torch.tensor(aux0, requires_grad=True)
    torch.F.gelu(dg).backward(plain)
    assert np.array_equal(y2.numpy(), dg.grad.numpy())
    y3 = gemm(3, aux)
    assert np.array_equal(y3.numpy(), (aux + plain).numpy())
