"""Fused elementwise expressions on the CPU: the library compiles the
kernel of every op of its program format (hipRTC, no device), and the
host-side program builder (deferred tensors -> tjh_expr) is checked by
interpreting the programs it emits with numpy against direct evaluation of
the same expression graph.  Device results are compared with the
op-by-op kernels in tests/test_gpu_fusion.py."""
import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
import __graft_entry__ as ge  # noqa: E402

LIB = os.path.join(ROOT, "torch.js_amd", "libtorchjs_hip.so")
pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")

ge.load_package()
T = sys.modules[ge.PKG_NAME + ".tensor"]
L = sys.modules[ge.PKG_NAME + "._lib"]


def _prog(ins, leaves, result):
    """ins: (op, code, dst, a, b, c, f); leaves: (ptr, kind, period)."""
    p = L.Expr()
    p.n_ins = len(ins)
    p.n_leaves = len(leaves)
    p.result = result
    for i, (op, code, dst, a, b, c, f) in enumerate(ins):
        q = p.ins[i]
        q.op, q.code, q.dst, q.a, q.b, q.c, q.f = (L.EXPR_OP[op], code, dst, a, b, c, f)
    for k, (ptr, kind, per) in enumerate(leaves):
        p.leaf[k] = ptr
        p.kind[k] = L.LEAF[kind]
        p.period[k] = per
    return p


def _compile(p, n, colsum):
    lib = L.lib()
    rc = lib.tjh_expr_compile(ctypes.byref(p), n, colsum)
    if rc:
        raise AssertionError(lib.tjh_last_error().decode())


N = L.EXPR_NONE
ALIGNED, MISALIGNED = 0x100000, 0x100004


def _all_unary(ptr):
    ins = [("load", 0, 0, 0, N, N, 0.0)]
    for code in range(len(L.UNARY)):
        ins.append(("unary", code, 1 + code % 2, 0, N, N, 0.1))
        ins.append(("unary_bwd", code, 0, 0, 1 + code % 2, 1 + code % 2, 0.1))
    return _prog(ins, [(ptr, "contig", 0)], 0)


def _all_binary(ptr):
    ins = [("load", 0, 0, 0, N, N, 0.0), ("load", 0, 1, 1, N, N, 0.0),
           ("load", 0, 2, 2, N, N, 0.0), ("load", 0, 3, 3, N, N, 0.0), ("const", 0, 4, N, N, N, 2.5)]
    for code in range(len(L.BINARY)):
        ins.append(("binary", code, 5, code % 5, (code + 1) % 5, N, 0.0))
    for code in range(len(L.TERNARY)):
        ins.append(("ternary", code, 6, 5, code % 5, (code + 2) % 5, 0.0))
    for code in range(len(L.SCALAR)):
        ins.append(("scalar", code, 7, 6, N, N, 1.5))
        ins.append(("scalar_rev", code, 8, 7, N, N, 0.5))
    ins.append(("axpy", 0, 9, 8, 6, N, -0.25))
    leaves = [(ptr, "contig", 0), (ptr + 64, "row", 8), (ptr + 128, "col", 8),
              (ptr + 256, "scalar", 0)]
    return _prog(ins, leaves, 9)


@pytest.mark.parametrize("which", ["unary", "binary"])
@pytest.mark.parametrize("ptr", [ALIGNED, MISALIGNED], ids=["w4", "w1"])
@pytest.mark.parametrize("colsum", [0, 1])
def test_every_op_compiles(which, ptr, colsum):
    p = _all_unary(ptr) if which == "unary" else _all_binary(ptr)
    _compile(p, 64 * 64, colsum)


def test_invalid_programs_are_rejected():
    lib = L.lib()
    bad = [
        _prog([("unary", 0, 0, 3, N, N, 0.0)], [], 0),                     # source never written
        _prog([("load", 0, 0, 1, N, N, 0.0)], [(ALIGNED, "contig", 0)], 0),  # leaf out of range
        _prog([("load", 0, 0, 0, N, N, 0.0)], [(ALIGNED, "contig", 0)], 1),  # result unwritten
        _prog([("load", 0, 0, 0, N, N, 0.0), ("binary", 99, 1, 0, 0, N, 0.0)],
              [(ALIGNED, "contig", 0)], 1),                                  # op code
        _prog([("load", 0, 0, 0, N, N, 0.0)], [(ALIGNED, "row", 0)], 0),     # period 0
        _prog([("load", 0, 0, 0, N, N, 0.0)], [(0, "contig", 0)], 0),        # NULL leaf
    ]
    for p in bad:
        assert lib.tjh_expr_compile(ctypes.byref(p), 16, 0) == 1, lib.tjh_last_error()
    p = _prog([], [], 0)
    assert lib.tjh_expr_compile(ctypes.byref(p), 16, 0) == 1
    for r2 in (2, 17, -1):  # second result: unwritten register, out of range
        p = _prog([("load", 0, 0, 0, N, N, 0.0)], [(ALIGNED, "contig", 0)], 0)
        p.result2 = r2
        assert lib.tjh_expr_compile(ctypes.byref(p), 16, 1) == 1, r2


# ------------------------------------------------------------ the host builder


class _FakeStorage:
    """Stands in for a device allocation: the builder only reads pointers."""

    def __init__(self, ptr, n):
        self.ptr, self.nbytes = ptr, 4 * n


_NP_UNARY = {"neg": np.negative, "exp": np.exp, "abs": np.abs, "square": np.square}
_NP_BINARY = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "maximum": np.maximum}
_NP_SCALAR = {"add": np.add, "sub": np.subtract, "mul": np.multiply}


def _interpret(prog, shape, data, second=False):
    """Runs a tjh_expr program over numpy leaves (`data`: ptr -> array);
    returns its value, or its second value (result2)."""
    n = int(np.prod(shape))
    e = np.arange(n)
    leaves = []
    for k in range(prog.n_leaves):
        arr = data[prog.leaf[k]].reshape(-1).astype(np.float64)
        kind, per = prog.kind[k], prog.period[k]
        idx = {0: e, 1: e % max(per, 1), 2: e // max(per, 1), 3: np.zeros_like(e)}[kind]
        leaves.append(arr[idx])
    inv = {v: k for k, v in L.EXPR_OP.items()}
    un = {v: k for k, v in L.UNARY.items()}
    bn = {v: k for k, v in L.BINARY.items()}
    sc = {v: k for k, v in L.SCALAR.items()}
    regs = {}
    for i in range(prog.n_ins):
        q = prog.ins[i]
        op = inv[q.op]
        if op == "load":
            v = leaves[q.a]
        elif op == "unary":
            v = _NP_UNARY[un[q.code]](regs[q.a])
        elif op == "binary":
            v = _NP_BINARY[bn[q.code]](regs[q.a], regs[q.b])
        elif op == "scalar":
            v = _NP_SCALAR[sc[q.code]](regs[q.a], np.float64(q.f))
        elif op == "scalar_rev":
            v = _NP_SCALAR[sc[q.code]](np.float64(q.f), regs[q.a])
        elif op == "axpy":
            v = np.float64(q.f) * regs[q.a] + regs[q.b]
        else:
            raise AssertionError(op)
        regs[q.dst] = v
    return regs[prog.result2 - 1 if second else prog.result].reshape(shape)


def _leaf(shape, ptr, data, rng, strides=None, full=None):
    full = full or shape
    arr = rng.standard_normal(full).astype(np.float32)
    data[ptr] = arr
    return T.Tensor(_FakeStorage(ptr, arr.size), shape, strides, 0, "float32")


@pytest.fixture
def lazy_on():
    saved = dict(T._LAZY)
    T._LAZY.update(on=True, min=1)
    yield
    T._LAZY.clear()
    T._LAZY.update(saved)


def test_builder_matches_graph(lazy_on):
    rng = np.random.default_rng(5)
    data = {}
    S = (6, 8)
    x = _leaf(S, 0x1000, data, rng)
    y = _leaf(S, 0x2000, data, rng)
    b = _leaf((8,), 0x3000, data, rng)            # row leaf
    c = _leaf((6, 1), 0x4000, data, rng)          # column leaf
    s = _leaf((), 0x5000, data, rng)              # scalar leaf
    # (x + b) * y - c, reused twice, then max with |x * s| and an axpy
    t1 = T._k_binary("add", x, b)
    t2 = T._k_binary("mul", t1, y)
    t3 = T._k_binary("sub", t2, c)
    t4 = T._k_binary("mul", x, s)
    t5 = T._k_unary("abs", t4)
    t6 = T._k_binary("maximum", t3, t5)
    t7 = T._k_axpy(0.5, t6, t3)                  # t3 is used twice: computed once
    t8 = T._k_scalar("sub", t7, 2.0, reverse=True)
    for t in (t1, t3, t6, t8):
        assert T._is_lazy(t)
    prog, _ = T._program(t8)
    X, Y, B, C, Sv = (data[p].astype(np.float64) for p in (0x1000, 0x2000, 0x3000, 0x4000, 0x5000))
    T3 = (X + B) * Y - C
    T6 = np.maximum(T3, np.abs(X * Sv))
    ref = 2.0 - (0.5 * T6 + T3)
    np.testing.assert_allclose(_interpret(prog, S, data), ref, rtol=1e-12)
    ops = [prog.ins[i].op for i in range(prog.n_ins)]
    assert ops.count(L.EXPR_OP["load"]) == 5        # one load per leaf
    assert ops.count(L.EXPR_OP["binary"]) == 5       # t3 computed once (7 if recomputed)
    kinds = sorted(prog.kind[k] for k in range(prog.n_leaves))
    assert kinds == sorted([0, 0, L.LEAF["row"], L.LEAF["col"], L.LEAF["scalar"]])
    _compile(prog, 48, 0)


def test_builder_second_value(lazy_on):
    """Two deferred values over common leaves as one program: each leaf
    loaded once, shared subexpressions computed once, the second value's
    register held to the end; both values as the graph computes them, and
    the two-output column-sum kernel compiles."""
    rng = np.random.default_rng(9)
    data = {}
    S = (8, 16)
    x = _leaf(S, 0x1000, data, rng)
    y = _leaf(S, 0x2000, data, rng)
    b = _leaf((16,), 0x3000, data, rng)
    e = T._k_unary("exp", T._k_binary("add", x, b))
    gx = T._k_binary("mul", e, y)                      # x's gradient
    gy = T._k_scalar("mul", e, 2.0)                    # y's gradient
    prog, _ = T._program(gx, gy)
    assert prog.result2 > 0
    X, Y, B = (data[p].astype(np.float64) for p in (0x1000, 0x2000, 0x3000))
    np.testing.assert_allclose(_interpret(prog, S, data), np.exp(X + B) * Y, rtol=1e-12)
    np.testing.assert_allclose(_interpret(prog, S, data, second=True), 2.0 * np.exp(X + B),
                               rtol=1e-12)
    ops = [prog.ins[i].op for i in range(prog.n_ins)]
    assert ops.count(L.EXPR_OP["load"]) == 3
    assert ops.count(L.EXPR_OP["unary"]) == 1           # exp(x + b) once for both
    _compile(prog, 128, 1)


def test_builder_three_values(lazy_on):
    """A backward column sum with its sibling gradient and a pending
    forward column sum of the same inputs as one program: the chain's
    loads and GELU-like subexpression shared by all three values, the
    third value's register held, result3 set; the three-output
    column-sum kernel compiles; a third result register never written is
    rejected."""
    rng = np.random.default_rng(10)
    data = {}
    S = (8, 16)
    x = _leaf(S, 0x1000, data, rng)
    y = _leaf(S, 0x2000, data, rng)
    b = _leaf((16,), 0x3000, data, rng)
    e = T._k_unary("exp", T._k_binary("add", x, b))
    z = T._k_binary("mul", e, y)                       # the forward value
    gx = T._k_binary("mul", T._k_scalar("mul", e, 0.5), y)
    gy = T._k_scalar("mul", e, 0.5)
    prog, _ = T._program(gx, gy, z)
    assert prog.result2 > 0 and prog.result3 > 0
    ops = [prog.ins[i].op for i in range(prog.n_ins)]
    assert ops.count(L.EXPR_OP["load"]) == 3
    assert ops.count(L.EXPR_OP["unary"]) == 1
    X, Y, B = (data[p].astype(np.float64) for p in (0x1000, 0x2000, 0x3000))
    np.testing.assert_allclose(_interpret(prog, S, data), 0.5 * np.exp(X + B) * Y, rtol=1e-12)
    _compile(prog, 128, 1)
    p = _prog([("load", 0, 0, 0, N, N, 0.0)], [(ALIGNED, "contig", 0)], 0)
    p.result3 = 2
    assert L.lib().tjh_expr_compile(ctypes.byref(p), 16, 1) == 1


def test_builder_register_reuse_and_limits(lazy_on):
    rng = np.random.default_rng(6)
    data = {}
    S = (4, 16)
    xs = [_leaf(S, 0x1000 * (k + 1), data, rng) for k in range(6)]
    # a long chain over 6 leaves: registers are freed after their last use
    t = xs[0]
    for k in range(1, 6):
        t = T._k_binary("add" if k % 2 else "mul", t, xs[k])
        t = T._k_unary("neg", t)
    prog, _ = T._program(t)
    ref = data[0x1000].astype(np.float64)
    for k in range(1, 6):
        ref = -(ref + data[0x1000 * (k + 1)] if k % 2 else ref * data[0x1000 * (k + 1)])
    np.testing.assert_allclose(_interpret(prog, S, data), ref, rtol=1e-12)
    used = {prog.ins[i].dst for i in range(prog.n_ins)}
    assert max(used) < 4
    # more than 8 leaves cannot be one program
    more = [_leaf(S, 0x100000 * (k + 1), data, rng) for k in range(9)]
    u = more[0]
    for m in more[1:]:
        u = T._k_binary("add", u, m)
    with pytest.raises(T._TooBig):
        T._program(u)


def test_leaf_kinds():
    S = (2, 3, 4)
    assert T._leaf_kind(S, [12, 4, 1]) == ("contig", 0)
    assert T._leaf_kind(S, [0, 0, 1]) == ("row", 4)
    assert T._leaf_kind(S, [0, 4, 1]) == ("row", 12)
    assert T._leaf_kind(S, [3, 1, 0]) == ("col", 4)
    assert T._leaf_kind(S, [1, 0, 0]) == ("col", 12)
    assert T._leaf_kind(S, [0, 0, 0]) == ("scalar", 0)
    assert T._leaf_kind(S, [1, 2, 6]) is None           # transposed
    assert T._leaf_kind(S, [0, 1, 0]) is None           # middle axis only
    assert T._leaf_kind((1, 5), [0, 1]) == ("contig", 0)


def test_lazy_respects_size_and_dtype():
    saved = dict(T._LAZY)
    try:
        T._LAZY.update(on=True, min=100)
        small = T.Tensor(_FakeStorage(0x1000, 10), (10,), None, 0, "float32")
        assert not T._lazy_ok((10,), (small,))
        big = T.Tensor(_FakeStorage(0x1000, 200), (200,), None, 0, "float32")
        assert T._lazy_ok((200,), (big,))
        ints = T.Tensor(_FakeStorage(0x1000, 200), (200,), None, 0, "int32")
        assert not T._lazy_ok((200,), (ints,))
        tr = T.Tensor(_FakeStorage(0x1000, 200), (10, 20), (1, 10), 0, "float32")
        assert not T._lazy_ok((10, 20), (tr,))
        T._LAZY.update(on=False)
        assert not T._lazy_ok((200,), (big,))
    finally:
        T._LAZY.clear()
        T._LAZY.update(saved)
