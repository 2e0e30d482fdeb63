"""Deferred elementwise chains on the device: every fused value, column sum
and gradient equals the op-by-op kernels bit for bit (the same ops with
deferral off), chains really run as one kernel, and in-place writes never
leak into a deferred value that read the written memory."""
import sys

import numpy as np
import pytest

from oracle import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T(torch):
    import __graft_entry__ as ge
    return sys.modules[ge.PKG_NAME + ".tensor"]


def _mode(T, on):
    T._LAZY["on"] = on


@pytest.fixture
def both(torch, T):
    """Runs fn with deferral on and off; returns the two results."""
    def run(fn):
        out = []
        for on in (True, False):
            _mode(T, on)
            try:
                out.append(fn())
            finally:
                _mode(T, True)
        return out
    return run


def _np(x):
    return x.numpy() if x is not None else None


def _same(a, b):
    if isinstance(a, (list, tuple)):
        assert len(a) == len(b)
        for u, v in zip(a, b):
            _same(u, v)
        return
    assert a.shape == b.shape and a.dtype == b.dtype
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.max(np.abs(a - b))


def _rand(shape, seed, lo=-2.0, hi=2.0):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def test_chain_fwd_bwd_bitwise_and_fused(torch, T, both):
    """The C2 chain: ((x + bias).gelu() * y).sum(0).mean(), forward and
    backward, fused against op by op; with deferral the whole step is one
    pass over x and y (the forward column sum rides along with x's and y's
    gradients and the bias gradient) and no elementwise kernel writes an
    intermediate."""
    R, C = 512, 2048
    xs, bs, ys = _rand((R, C), 1), _rand((C,), 2), _rand((R, C), 3, -1, 1)

    def step():
        x = torch.tensor(xs, requires_grad=True)
        b = torch.tensor(bs, requires_grad=True)
        y = torch.tensor(ys, requires_grad=True)
        loss = ((x + b).gelu() * y).sum(0).mean()
        loss.backward()
        return [_np(loss), _np(x.grad), _np(b.grad), _np(y.grad)]

    fused, plain = both(step)
    _same(fused, plain)
    # launch accounting with deferral on
    torch.hip.kernel_timing(True)
    torch.hip.kernel_timing_reset()
    try:
        step()
        fams = dict((f, torch.hip.kernel_time(f)[0]) for f in torch.hip.kernel_families())
    finally:
        torch.hip.kernel_timing(False)
    assert fams.get("expr_colsum3", 0) == 1, fams    # sum(0) and the bias gradient, one pass
    assert fams.get("expr_colsum", 0) == 0 and fams.get("expr", 0) == 0, fams
    assert fams.get("unary", 0) == 0 and fams.get("binary", 0) == 0, fams


@pytest.mark.parametrize("extra", [False, True])
def test_chain_sibling_gradients_in_one_pass(torch, T, extra):
    """y's gradient of the C2 chain is written by the column-sum launch that
    writes x's gradient and the bias gradient (one read of x and y for the
    whole backward), bit for bit the separately evaluated gradients; with a
    second contribution to y's gradient (`extra`) as well."""
    R, C = 512, 2048
    xs, bs, ys = _rand((R, C), 21), _rand((C,), 22), _rand((R, C), 23, -1, 1)

    def step():
        x = torch.tensor(xs, requires_grad=True)
        b = torch.tensor(bs, requires_grad=True)
        y = torch.tensor(ys, requires_grad=True)
        loss = ((x + b).gelu() * y).sum(0).mean()
        if extra:
            loss = loss + (y * 3.0).sum()
        loss.backward()
        return [_np(loss), _np(x.grad), _np(b.grad), _np(y.grad)]

    runs, launches = [], []
    prev = T._FUSE_SIB
    for sib in (True, False):
        T._FUSE_SIB = sib
        try:
            runs.append(step())
            torch.hip.kernel_timing(True)
            torch.hip.kernel_timing_reset()
            try:
                step()
                launches.append(dict((f, torch.hip.kernel_time(f)[0])
                                     for f in torch.hip.kernel_families()))
            finally:
                torch.hip.kernel_timing(False)
        finally:
            T._FUSE_SIB = prev
    _same(runs[0], runs[1])
    assert not T._SIBLINGS
    if not extra:
        # one pass for the forward sum(0) and the gradients, and fewer
        # launches in all: y's gradient is not evaluated on its own
        assert launches[0].get("expr_colsum3", 0) == 1, launches[0]
        assert launches[0].get("expr", 0) < launches[1].get("expr", 0), launches
        assert sum(launches[0].values()) < sum(launches[1].values()), launches


@pytest.mark.parametrize("read", ["never", "before", "after", "write_first"])
def test_deferred_forward_column_sum(torch, T, read):
    """sum(0) of a deferred value stays deferred; the backward's column-sum
    pass over the same inputs computes it (expr_colsum3), bit for bit what
    the immediate sum gives, and a loss that is a deferred reduction is
    evaluated by the end of backward().  Read before backward it is computed
    on its own; an in-place write to an input first computes it from the
    old values."""
    R, C = 512, 2048
    xs, bs, ys = _rand((R, C), 31), _rand((C,), 32), _rand((R, C), 33, -1, 1)

    def run(defer):
        T._DEFER_SUMS["on"] = defer
        try:
            x = torch.tensor(xs, requires_grad=True)
            b = torch.tensor(bs, requires_grad=True)
            y = torch.tensor(ys, requires_grad=True)
            col = ((x + b).gelu() * y).sum(0)
            loss = col.mean()
            if defer:
                assert T._is_lazy(col) and T._is_lazy(loss)
            early = loss.numpy().copy() if read == "before" else None
            if read == "write_first":
                with torch.no_grad():
                    y.fill_(0.5)  # the pending sum is computed from the old y first
            else:
                loss.backward()
                assert not T._is_lazy(loss)  # evaluated by the end of the pass
            out = [_np(loss), _np(col)]
            if read != "write_first":
                out += [_np(x.grad), _np(b.grad), _np(y.grad)]
            if early is not None:
                assert np.array_equal(early, out[0])
            return out
        finally:
            T._DEFER_SUMS["on"] = True
    _same(run(True), run(False))
    want = (ops.gelu(xs.astype(np.float64) + bs) * ys).sum(0)
    np.testing.assert_allclose(run(True)[1], want, rtol=1e-5, atol=1e-4)


def test_deferred_gradient_shared_by_two_leaves(torch, T):
    """An add hands one deferred gradient to both of its leaf inputs: each
    leaf's .grad gets memory of its own, so an in-place edit of one leaves
    the other unchanged (with sibling evaluation on and off)."""
    xs, ys = _rand((256, 512), 61), _rand((256, 512), 62)
    prev = T._FUSE_SIB
    try:
        for sib in (True, False):
            T._FUSE_SIB = sib
            a = torch.tensor(xs, requires_grad=True)
            b = torch.tensor(ys, requires_grad=True)
            ((a + b).exp() * 0.5).sum().backward()
            assert not T._SIBLINGS
            want = 0.5 * np.exp(xs.astype(np.float64) + ys)
            np.testing.assert_allclose(a.grad.numpy(), want, rtol=1e-5)
            gb = b.grad.numpy().copy()
            a.grad.zero_()
            assert np.array_equal(b.grad.numpy(), gb), sib
            assert not a.grad.numpy().any()
            # three leaves along a chain of adds, ((q + r) + p): p takes the
            # deferred gradient first, q's copy computes it, r must still get
            # memory of its own (the deferred value's storage is owned by p)
            zs = _rand((256, 512), 63)
            q = torch.tensor(xs, requires_grad=True)
            r = torch.tensor(ys, requires_grad=True)
            p = torch.tensor(zs, requires_grad=True)
            ((q + r) + p).exp().sum().backward()
            assert not T._SIBLINGS
            want = np.exp(xs.astype(np.float64) + ys + zs)
            for leaf in (q, r, p):
                np.testing.assert_allclose(leaf.grad.numpy(), want, rtol=1e-5)
            keep = {id(leaf): leaf.grad.numpy().copy() for leaf in (q, r, p)}
            for victim in (r, p, q):
                victim.grad.zero_()
                for leaf in (q, r, p):
                    if leaf is victim:
                        assert not leaf.grad.numpy().any()
                    else:
                        assert np.array_equal(leaf.grad.numpy(), keep[id(leaf)]), sib
                keep[id(victim)] = victim.grad.numpy().copy()
    finally:
        T._FUSE_SIB = prev


def test_write_through_detached_alias_of_deferred_value(torch, T):
    """y = x.exp() stays deferred, p = y * 2 reads it; writing zeros through
    y.detach() must first compute p from the old y (p = 2 exp(x)), and y
    itself then reads as zeros."""
    xs = _rand((256, 512), 64)  # above the size from which elementwise ops defer
    x = torch.tensor(xs)
    y = x.exp()
    p = y * 2.0
    assert T._is_lazy(y) and T._is_lazy(p)
    y.detach().zero_()
    np.testing.assert_allclose(p.numpy(), 2.0 * np.exp(xs.astype(np.float64)), rtol=1e-6)
    assert not y.numpy().any()


@pytest.mark.parametrize("op", ["neg", "exp", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "relu",
                                "gelu", "square", "reciprocal", "erf", "abs", "sin", "cos",
                                "silu", "leaky_relu", "elu", "softplus", "sign"])
def test_unary_fwd_bwd_bitwise(torch, T, both, op):
    positive = op in ("log", "sqrt", "rsqrt", "reciprocal")
    xs = _rand((300, 257), 10 + len(op), 0.1 if positive else -3.0, 3.0)

    def run():
        x = torch.tensor(xs, requires_grad=True)
        z = T.unary(op, x * 1.25 + 0.125 if not positive else x * 1.25, 0.2)
        w = (z * z + x).sum()
        w.backward()
        return [_np(z), _np(w), _np(x.grad)]

    fused, plain = both(run)
    _same(fused, plain)


def test_binary_scalar_ternary_broadcast_bitwise(torch, T, both):
    a_, row_, col_, s_ = _rand((256, 512), 21, 0.5, 2.0), _rand((512,), 22, 0.5, 2.0), \
        _rand((256, 1), 23, 0.5, 2.0), _rand((), 24, 0.5, 2.0)

    def run():
        a = torch.tensor(a_, requires_grad=True)
        row = torch.tensor(row_, requires_grad=True)
        col = torch.tensor(col_, requires_grad=True)
        s = torch.tensor(s_, requires_grad=True)
        t = (a - row) * col / (s + 1.0)
        t = t.maximum(a * 0.5) - row.minimum(col)
        t = t ** 2 + (a ** row) / 3.0
        t = 2.0 - t + 1.0 / (a + 3.0)
        out = (t * a).sum()
        out.backward()
        return [_np(t), _np(out), _np(a.grad), _np(row.grad), _np(col.grad), _np(s.grad)]

    fused, plain = both(run)
    _same(fused, plain)


@pytest.mark.parametrize("shape,dims", [((512, 1024), (0,)), ((8, 128, 256), (0, 1)),
                                        ((16, 96, 64), (1,)), ((64, 2048), (0,))])
@pytest.mark.parametrize("red", ["sum", "mean"])
def test_column_sums_of_deferred_values(torch, T, both, shape, dims, red):
    xs, ys = _rand(shape, 31), _rand(shape[-1:], 32)

    def run():
        x = torch.tensor(xs)
        y = torch.tensor(ys)
        v = (x * y).exp() - x
        r = getattr(v, red)(dims if len(dims) > 1 else dims[0])
        return [_np(r)]

    fused, plain = both(run)
    _same(fused, plain)


def test_column_sum_keeps_value(torch, T):
    """The broadcast add's backward evaluates the incoming gradient while
    summing its columns: both results equal the unfused ones."""
    R, C = 256, 1024
    xs, bs = _rand((R, C), 41), _rand((C,), 42)

    def run(on):
        _mode(T, on)
        try:
            x = torch.tensor(xs, requires_grad=True)
            b = torch.tensor(bs, requires_grad=True)
            ((x + b).tanh() * 3.0).sum().backward()
            return [_np(x.grad), _np(b.grad)]
        finally:
            _mode(T, True)

    _same(run(True), run(False))


def test_inplace_writes_do_not_reach_deferred_values(torch, T):
    xs = _rand((512, 512), 51)
    x = torch.tensor(xs)
    y = x * 2.0                       # deferred, reads x
    z = (y + 1.0).exp()               # deferred, reads y
    assert T._is_lazy(y) and T._is_lazy(z)
    x.fill_(7.0)                      # evaluates y and z first
    np.testing.assert_array_equal(y.numpy(), xs * np.float32(2.0))
    ref_z = (torch.tensor(xs) * 2.0 + 1.0).exp().numpy()
    _same(z.numpy(), ref_z)
    # copy_ / zero_ into a tensor a deferred value reads, and into the
    # deferred value itself
    a = torch.tensor(xs)
    b = a.sigmoid()
    c = b * 3.0
    a.copy_(torch.tensor(np.zeros_like(xs)))
    b.zero_()
    assert np.all(b.numpy() == 0)
    ref_c = (torch.tensor(xs).sigmoid() * 3.0).numpy()
    _same(c.numpy(), ref_c)


def test_optimizer_step_after_deferred_read(torch, T):
    ps = _rand((256, 512), 61)
    p = torch.tensor(ps, requires_grad=True)
    with torch.no_grad():
        w = p * 3.0                   # deferred, reads the parameter
    (p * p).sum().backward()
    opt = torch.optim.SGD([p], lr=0.5)
    opt.step()
    np.testing.assert_array_equal(w.numpy(), ps * np.float32(3.0))


def test_views_detach_and_alignment(torch, T, both):
    xs = _rand((384, 520), 71)

    def run():
        x = torch.tensor(xs)
        v = x.exp() * 0.5
        d = v.detach()
        outs = [v.reshape(520, 384), v.t().contiguous(), v[3:7, 10:200], d * 2.0]
        # a leaf at an odd element offset takes the 1-wide kernel
        off = torch.tensor(xs.reshape(-1))[1:1 + 384 * 519].reshape(384, 519)
        outs.append(off.tanh() + 1.0)
        return [_np(o) for o in outs] + [np.array(d.data_ptr() == v.data_ptr())]

    fused, plain = both(run)
    _same(fused[:-1], plain[:-1])
    assert fused[-1] and plain[-1]


def test_long_chains_and_many_leaves(torch, T, both):
    xs = [_rand((256, 256), 80 + k) for k in range(12)]

    def run():
        ts = [torch.tensor(a) for a in xs]
        t = ts[0]
        for k in range(70):  # beyond one program's instruction limit
            t = (t * 0.999 + 0.001).tanh() if k % 2 else t - ts[k % 12] * 0.01
        u = ts[0]
        for a in ts[1:]:     # 12 leaves: beyond one program's leaf limit
            u = u + a * 0.5
        return [_np(t), _np(u)]

    fused, plain = both(run)
    _same(fused, plain)


def test_compile_failure_falls_back_to_single_op_kernels(torch, T, capsys):
    """When the fused kernels cannot be compiled, deferred values are
    evaluated op by op with the single-op kernels (same bits) and fusion
    turns itself off."""
    import __graft_entry__ as ge
    L = sys.modules[ge.PKG_NAME + "._lib"]
    real = L.lib()

    class NoCompiler:
        def __getattr__(self, name):
            if name in ("tjh_expr_eval", "tjh_expr_colsum"):
                return lambda *a: 4  # TJH_ERR_HIP
            if name == "tjh_last_error":
                return lambda: b"tjh_expr: compile failed (HIPRTC_ERROR_COMPILATION): test"
            return getattr(real, name)

    xs, ys = _rand((512, 512), 91), _rand((512,), 92)
    _mode(T, True)
    x, y = torch.tensor(xs), torch.tensor(ys)
    want = [((x + y).tanh() * 2.0).numpy(), ((x * y).exp() - x).sum(0).numpy()]
    saved_lib, saved = L.lib, dict(T._LAZY)
    try:
        L.lib = lambda: NoCompiler()
        got = [((x + y).tanh() * 2.0).numpy(), ((x * y).exp() - x).sum(0).numpy()]
        assert T._LAZY["jit"] is False and T._LAZY["on"] is False
        assert "one kernel each" in capsys.readouterr().err
    finally:
        L.lib = saved_lib
        T._LAZY.clear()
        T._LAZY.update(saved)
    _same(got, want)
