"""HIP graphs: a captured step replays to the same results as running it
eagerly (bit for bit), on new inputs fed with copy_, with eager work between
replays; memory the graph owns is never handed to eager allocations; host
readbacks inside a capture raise and leave the device usable."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rand(shape, seed, lo=-2.0, hi=2.0):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def _bits(a, b):
    assert a.shape == b.shape
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.max(np.abs(a - b))


def test_chain_step_replays_bitwise(torch):
    R, C = 512, 2048
    xs, bs, ys = _rand((R, C), 1), _rand((C,), 2), _rand((R, C), 3, -1, 1)
    x = torch.tensor(xs, requires_grad=True)
    b = torch.tensor(bs, requires_grad=True)
    y = torch.tensor(ys, requires_grad=True)

    def step():
        for t in (x, b, y):
            t.grad = None
        loss = ((x + b).gelu() * y).sum(0).mean()
        loss.backward()
        return loss

    def eager(xv, bv, yv):
        xe = torch.tensor(xv, requires_grad=True)
        be = torch.tensor(bv, requires_grad=True)
        ye = torch.tensor(yv, requires_grad=True)
        le = ((xe + be).gelu() * ye).sum(0).mean()
        le.backward()
        return [le.numpy(), xe.grad.numpy(), be.grad.numpy(), ye.grad.numpy()]

    for _ in range(2):
        step()  # warm-up: kernels compiled, allocator primed
    g = torch.hip.Graph()
    with torch.hip.graph(g):
        loss = step()
    ref = eager(xs, bs, ys)
    for k in range(3):
        g.replay()
        _ = (torch.tensor(_rand((64, 64), 9 + k)) * 2.0).numpy()  # eager work between replays
        for got, want in zip([loss.numpy(), x.grad.numpy(), b.grad.numpy(), y.grad.numpy()], ref):
            _bits(got, want)
    # new inputs through copy_
    xs2, ys2 = _rand((R, C), 11), _rand((R, C), 13, -1, 1)
    with torch.no_grad():
        x.copy_(torch.tensor(xs2))
        y.copy_(torch.tensor(ys2))
    g.replay()
    for got, want in zip([loss.numpy(), x.grad.numpy(), b.grad.numpy(), y.grad.numpy()],
                         eager(xs2, bs, ys2)):
        _bits(got, want)
    g.reset()


def test_mlp_sgd_training_replays_bitwise(torch):
    """Linear-ReLU-Linear + cross_entropy + SGD: three replays update the
    parameters exactly as three eager steps do."""
    X = _rand((256, 784), 21)
    Y = np.random.default_rng(22).integers(0, 10, 256).astype(np.int32)

    def build():
        torch.manual_seed(5)
        m = torch.nn.Sequential(torch.nn.Linear(784, 256), torch.nn.ReLU(),
                                torch.nn.Linear(256, 10))
        return m, torch.optim.SGD(m.parameters(), lr=0.05)

    xs, ys = torch.tensor(X), torch.tensor(Y, dtype="int32")

    def step(m, opt):
        opt.zero_grad()
        loss = torch.nn.functional.cross_entropy(m(xs), ys)
        loss.backward()
        opt.step()
        return loss

    m1, o1 = build()
    ref = []
    for _ in range(5):
        ref.append(step(m1, o1).numpy())
    m2, o2 = build()
    step(m2, o2)  # warm-up (eager step 1)
    step(m2, o2)  # eager step 2
    g = torch.hip.Graph()
    with torch.hip.graph(g):
        loss = step(m2, o2)  # captured: runs as step 3 on the first replay
    got = []
    for _ in range(3):
        g.replay()
        got.append(loss.numpy())
    for a, b in zip(got, ref[2:]):
        _bits(a, b)
    for p1, p2 in zip(m1.parameters(), m2.parameters()):
        _bits(p1.numpy(), p2.numpy())
    g.reset()


def test_graph_memory_is_not_shared_with_eager_work(torch):
    xs = _rand((1024, 1024), 31)
    x = torch.tensor(xs)
    g = torch.hip.Graph()
    with torch.hip.graph(g):
        t = x @ x
        u = (t * 1e-3 + 1.0).tanh()
        del t                      # freed inside the capture: stays the graph's
        v = u.sum(0)
    held = [torch.tensor(np.full((1024, 1024), k, np.float32)) for k in range(4)]
    g.replay()
    for k, h in enumerate(held):
        assert np.all(h.numpy() == k)
    xe = torch.tensor(xs)
    ref = ((xe @ xe) * 1e-3 + 1.0).tanh().sum(0).numpy()
    _bits(v.numpy(), ref)
    g.reset()


def test_readback_inside_capture_raises(torch):
    x = torch.tensor(_rand((256, 256), 41))
    g = torch.hip.Graph()
    with pytest.raises(Exception):
        with torch.hip.graph(g):
            y = x * 2.0
            y.numpy()
    # the stream is usable again and no capture is left open
    np.testing.assert_array_equal((x + 1.0).numpy(), x.numpy() + np.float32(1.0))
    g2 = torch.hip.Graph()
    with torch.hip.graph(g2):
        z = x - 1.0
    g2.replay()
    np.testing.assert_array_equal(z.numpy(), x.numpy() - np.float32(1.0))
    g2.reset()
    opt = torch.optim.Adam([torch.zeros(4, requires_grad=True)], lr=0.1)
    g3 = torch.hip.Graph()
    with pytest.raises(RuntimeError):
        with torch.hip.graph(g3):
            opt.step()


@pytest.mark.parametrize("cls", ["Adam", "AdamW"])
def test_capturable_adam_matches_host_steps(torch, cls):
    """Device step counters and bias-correction tables give the host-stepped
    update bit for bit."""
    shapes = [(257, 33), (1024,), (64, 64)]
    params = [[torch.tensor(_rand(s, 50 + i), requires_grad=True) for i, s in enumerate(shapes)]
              for _ in range(2)]
    opts = [getattr(torch.optim, cls)(params[0], lr=3e-3, weight_decay=0.01),
            getattr(torch.optim, cls)(params[1], lr=3e-3, weight_decay=0.01, capturable=True)]
    for step in range(4):
        for ps, opt in zip(params, opts):
            for i, p in enumerate(ps):
                p.grad = torch.tensor(_rand(p.shape, 100 * step + i))
            opt.step()
    for a, b in zip(*params):
        _bits(a.numpy(), b.numpy())


def test_mlp_capturable_adam_replays_bitwise(torch):
    """The C1 step (784-256-ReLU-10, cross_entropy, Adam 1e-3) captured with
    a capturable Adam replays like eager host-stepped Adam steps."""
    X = _rand((64, 784), 61)
    Y = np.random.default_rng(62).integers(0, 10, 64).astype(np.int32)
    xs, ys = torch.tensor(X), torch.tensor(Y, dtype="int32")

    def build(capturable):
        torch.manual_seed(7)
        m = torch.nn.Sequential(torch.nn.Linear(784, 256), torch.nn.ReLU(),
                                torch.nn.Linear(256, 10))
        return m, torch.optim.Adam(m.parameters(), lr=1e-3, capturable=capturable)

    def step(m, opt):
        opt.zero_grad()
        loss = torch.nn.functional.cross_entropy(m(xs), ys)
        loss.backward()
        opt.step()
        return loss

    m1, o1 = build(False)
    ref = [step(m1, o1).numpy() for _ in range(6)]
    m2, o2 = build(True)
    step(m2, o2)
    step(m2, o2)
    g = torch.hip.Graph()
    with torch.hip.graph(g):
        loss = step(m2, o2)
    got = []
    for _ in range(4):
        g.replay()
        got.append(loss.numpy())
    for a, b in zip(got, ref[2:]):
        _bits(a, b)
    for p1, p2 in zip(m1.parameters(), m2.parameters()):
        _bits(p1.numpy(), p2.numpy())
    g.reset()
