"""tjh_layer_norm_backward_noalloc against tjh_layer_norm_backward_res
through the C ABI: bit-identical dx, dgamma and dbeta (same kernels, the
partial rows in the library's static device scratch instead of the caching
allocator), on two calls in a row with the second smaller, with the
allocator's counters unchanged by the calls."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _args(torch, rows, cols, seed, with_res):
    r = np.random.default_rng(seed)
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32))
    x = r.standard_normal((rows, cols)) * 2 + 0.5
    mean = x.mean(axis=1)
    rstd = 1.0 / np.sqrt(x.var(axis=1) + 1e-5)
    ins = dict(dy=t(r.standard_normal((rows, cols))), x=t(x), gamma=t(1 + 0.1 * r.standard_normal(cols)),
               mean=t(mean), rstd=t(rstd),
               res=t(r.standard_normal((rows, cols))) if with_res else None)
    return ins


def _outs(torch, rows, cols, init_gb):
    dx = torch.zeros(rows, cols)
    dg = torch.tensor(np.full(cols, init_gb, np.float32))
    db = torch.tensor(np.full(cols, -init_gb, np.float32))
    return dx, dg, db


def _call(L, fn, ins, outs, rows, cols, acc):
    p = lambda v: v.data_ptr() if v is not None else None
    dx, dg, db = outs
    if fn == "noalloc":
        rc = L.lib().tjh_layer_norm_backward_noalloc(
            p(ins["dy"]), p(ins["x"]), p(ins["gamma"]), p(ins["mean"]), p(ins["rstd"]),
            p(ins["res"]), p(dx), p(dg), p(db), rows, cols, acc)
    else:
        rc = L.lib().tjh_layer_norm_backward_res(
            p(ins["dy"]), p(ins["x"]), p(ins["gamma"]), p(ins["mean"]), p(ins["rstd"]),
            p(ins["res"]), p(dx), p(dg), p(db), rows, cols, acc & 1)
    return rc


@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("acc", [0, 1])
def test_noalloc_equals_allocating_entry(torch, with_res, acc):
    from torchjs_amd import _lib as L
    # the second call is smaller and leaves the first call's partials behind
    # in the scratch: they must not leak into its result
    for rows, cols, seed in ((8192, 768, 1), (37, 256, 2)):
        ins = _args(torch, rows, cols, seed, with_res)
        ref = _outs(torch, rows, cols, 0.25)
        got = _outs(torch, rows, cols, 0.25)
        assert _call(L, "res", ins, ref, rows, cols, acc) == 0, L.lib().tjh_last_error()
        torch.synchronize()
        s0 = torch.hip.memory_stats()
        assert _call(L, "noalloc", ins, got, rows, cols, acc) == 0, L.lib().tjh_last_error()
        torch.synchronize()
        s1 = torch.hip.memory_stats()
        assert s1["allocation_requests"] == s0["allocation_requests"]  # no tjh_malloc
        assert s1["device_mallocs"] == s0["device_mallocs"]  # no hipMalloc
        for a, b in zip(ref, got):
            assert np.array_equal(a.numpy(), b.numpy())


def test_noalloc_larger_rows_and_widths(torch):
    """Every row width class of the kernel (<=768 exact, <=1536, <=3072) and
    a row count past 2 rows per CU (more rows per workgroup)."""
    from torchjs_amd import _lib as L
    for rows, cols, seed in ((20000, 3072, 3), (1000, 1536, 4), (300, 1000, 5), (16, 4, 6)):
        ins = _args(torch, rows, cols, seed, True)
        ref = _outs(torch, rows, cols, 0.0)
        got = _outs(torch, rows, cols, 0.0)
        assert _call(L, "res", ins, ref, rows, cols, 0) == 0
        assert _call(L, "noalloc", ins, got, rows, cols, 0) == 0, L.lib().tjh_last_error()
        for a, b in zip(ref, got):
            assert np.array_equal(a.numpy(), b.numpy())


def test_noalloc_rejects_what_it_cannot_hold(torch):
    from torchjs_amd import _lib as L
    ins = _args(torch, 8, 3074, 7, False)
    outs = _outs(torch, 8, 3074, 0.0)
    rc = _call(L, "noalloc", ins, outs, 8, 3074, 0)
    assert rc == 5 and b"multiple of 4" in L.lib().tjh_last_error()  # TJH_ERR_UNSUPPORTED
    ins = _args(torch, 8, 6, 8, False)
    outs = _outs(torch, 8, 6, 0.0)
    assert _call(L, "noalloc", ins, outs, 8, 6, 0) == 5
    # rows == 0: dgamma / dbeta become zeros without a kernel of their own
    ins = _args(torch, 4, 64, 9, False)
    dx, dg, db = _outs(torch, 4, 64, 3.0)
    assert _call(L, "noalloc", ins, (dx, dg, db), 0, 64, 0) == 0
    assert not dg.numpy().any() and not db.numpy().any()
