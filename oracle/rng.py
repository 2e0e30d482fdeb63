"""torch.js's seeded generators restated exactly.  TEST INFRASTRUCTURE ONLY.

Per rand/randn call the global seed advances by the LCG of
src/ops/creation.ts:921 (seed = (seed*1103515245 + 12345) & 0x7fffffff);
element i then draws xorshift32(seed ^ (i*1664525 + 1013904223)) as in
random.wgsl:9-46.  Uniform = u / 2^32; normal = Box-Muller (cos branch)
over two successive xorshift states with u1 clamped to >= 1e-7, evaluated
in float64 here and rounded to float32 (the device evaluates it in float32,
so normals agree to a few ulp; the integer states agree exactly).
"""
import numpy as np

M32 = np.uint64(0xFFFFFFFF)


def lcg_next(seed):
    return (seed * 1103515245 + 12345) & 0x7FFFFFFF


def xorshift32(x):
    x = np.asarray(x, dtype=np.uint64) & M32
    x = (x ^ (x << np.uint64(13))) & M32
    x = x ^ (x >> np.uint64(17))
    x = (x ^ (x << np.uint64(5))) & M32
    return x


def states(n, seed):
    i = np.arange(n, dtype=np.uint64)
    s = (np.uint64(seed) ^ ((i * np.uint64(1664525) + np.uint64(1013904223)) & M32)) & M32
    s1 = xorshift32(s)
    return s1, xorshift32(s1)


def rand(n, seed):
    s1, _ = states(n, seed)
    return (s1.astype(np.float64) / 4294967296.0).astype(np.float32)


def randn(n, seed):
    s1, s2 = states(n, seed)
    u1 = np.maximum(s1.astype(np.float64) / 4294967296.0, 1e-7)
    u2 = s2.astype(np.float64) / 4294967296.0
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


class Generator:
    """Host-side generator for synthetic inputs and weights: the same LCG
    seed stream and per-element xorshift32 as the device's rand/randn."""

    def __init__(self, seed):
        self.seed = int(seed)

    def _next(self):
        self.seed = lcg_next(self.seed)
        return self.seed

    def rand(self, shape):
        n = int(np.prod(shape))
        return rand(n, self._next()).reshape(shape)

    def randn(self, shape):
        n = int(np.prod(shape))
        return randn(n, self._next()).reshape(shape)

    def uniform(self, shape, lo, hi):
        return (lo + (hi - lo) * self.rand(shape).astype(np.float64)).astype(np.float32)

    def normal(self, shape, std):
        return (self.randn(shape).astype(np.float64) * std).astype(np.float32)

    def integers(self, shape, hi):
        """Uniform ints in [0, hi) from the xorshift states (u * hi)."""
        n = int(np.prod(shape))
        s1, _ = states(n, self._next())
        return ((s1.astype(np.float64) / 4294967296.0) * hi).astype(np.int32).reshape(shape)
