"""The C ABI library loads and exports every symbol include/*.h declares;
host-side logic of the package.  CPU only: no kernel is launched."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names.update(re.findall(r"\b(tjh_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_header_declares_the_boundary():
    names = _declared()
    for must in ("tjh_init", "tjh_malloc", "tjh_free", "tjh_gemm", "tjh_sdpa_backward",
                 "tjh_adam_step", "tjh_layer_norm_backward", "tjh_cross_entropy_backward",
                 "tjh_embedding_backward", "tjh_conv2d_backward_weight"):
        assert must in names


def test_library_exports_every_declared_symbol(pkg):
    from torchjs_amd import _lib
    lib = _lib.load()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    unbound = [n for n in _declared() if n not in _lib.SIGNATURES]
    assert not unbound, unbound


def test_library_is_gfx950_only():
    so = os.path.join(ROOT, "torch.js_amd", "libtorchjs_hip.so")
    data = open(so, "rb").read()
    assert b"gfx950" in data


def test_calls_before_init_fail_cleanly(pkg):
    from torchjs_amd import _lib
    lib = _lib.load()
    if lib.tjh_is_initialized():
        pytest.skip("device already initialised in this process")
    p = ctypes.c_void_p()
    rc = lib.tjh_malloc(16, ctypes.byref(p))
    assert rc == 2  # TJH_ERR_NOT_INITIALIZED
    assert b"Call torch.init() first" in lib.tjh_last_error()
    assert lib.tjh_version().startswith(b"torchjs_hip")
    with pytest.raises(RuntimeError, match="torch.init"):
        pkg.zeros(3)


def test_device_count_without_gpu_is_a_number(pkg):
    from torchjs_amd import _lib
    n = ctypes.c_int(-1)
    assert _lib.load().tjh_device_count(ctypes.byref(n)) == 0
    assert n.value >= 0


# ------------------------------------------------------------------ host logic


def test_view_strides():
    from torchjs_amd.tensor import _view_strides
    assert _view_strides((4, 6), (6, 1), (24,)) == (1,)
    assert _view_strides((4, 6), (6, 1), (2, 2, 6)) == (12, 6, 1)
    # transposed: merging is impossible
    assert _view_strides((6, 4), (1, 6), (24,)) is None
    # padded rows (ld 8 for 5 columns): leading dims merge, the row cannot
    assert _view_strides((2, 3, 5), (24, 8, 1), (6, 5)) == (8, 1)
    assert _view_strides((6, 5), (8, 1), (30,)) is None
    # size-1 dims anywhere
    assert _view_strides((3, 1, 4), (4, 4, 1), (3, 4, 1)) == (4, 1, 1)


def test_broadcast_and_infer():
    from torchjs_amd.tensor import _broadcast_shapes, _infer_shape
    assert _broadcast_shapes((4096, 4096), (4096,)) == (4096, 4096)
    assert _broadcast_shapes((8, 1, 3), (5, 1)) == (8, 5, 3)
    with pytest.raises(ValueError):
        _broadcast_shapes((3,), (4,))
    assert _infer_shape((-1, 768), 8192 * 768) == (8192, 768)
    with pytest.raises(RuntimeError):
        _infer_shape((-1, 7), 10)


def test_reduce_runs():
    from torchjs_amd.tensor import _reduce_runs
    assert _reduce_runs((2, 3, 4, 5), [0, 2, 3]) == [[0, 1], [2, 4]]
    assert _reduce_runs((8, 1024, 768), [0, 1]) == [[0, 2]]


def test_package_has_no_cpu_fallback():
    """The product path never imports the oracle."""
    for f in glob.glob(os.path.join(ROOT, "torch.js_amd", "*.py")):
        src = open(f).read()
        assert "oracle" not in src.replace("the oracle", ""), f
