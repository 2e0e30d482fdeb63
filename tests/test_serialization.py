"""Weight I/O host logic (torch.js_amd/serialization.py), CPU only: the
PyTorch archive fixture written by torch.save and a torch.js archive laid
out as src/serialization/common.ts writes it parse to the expected values;
the unpickler refuses any global outside a state_dict's; save/read round
trips keep every byte."""
import io
import os
import pickle
import zipfile

import numpy as np
import pytest

from conftest import GOLDEN


@pytest.fixture(scope="module")
def S(pkg):
    from torchjs_amd import serialization
    return serialization


def test_pytorch_archive_fixture(S):
    obj = S.read_archive(os.path.join(GOLDEN, "state_dict.pt"))
    with np.load(os.path.join(GOLDEN, "state_dict_expected.npz")) as z:
        exp = {k: z[k] for k in z.files}
    assert list(obj.keys()) == ["layer.weight", "ids", "transposed", "slice", "half", "bf16",
                                "mask", "nested"]
    for k in ("layer.weight", "ids", "transposed", "slice", "half", "bf16", "mask"):
        t = obj[k]
        assert np.array_equal(t.array, exp[k]), k
        assert t.array.flags.c_contiguous
    assert obj["layer.weight"].requires_grad and not obj["ids"].requires_grad  # a Parameter
    assert obj["ids"].dtype == "int32" and obj["mask"].dtype == "bool"
    assert obj["half"].dtype == "float32" and obj["bf16"].dtype == "float32"
    lst = obj["nested"]["list"]
    assert np.array_equal(lst[0].array, exp["nested.list.0"]) and lst[1:] == [7, "name"]
    assert obj["nested"]["scale"] == 0.5


def test_torchjs_archive_fixture(S):
    obj = S.read_archive(os.path.join(GOLDEN, "torchjs_archive.zip"))
    m = obj["model"]
    assert np.array_equal(m["fc.weight"].array, np.arange(6, dtype=np.float32).reshape(2, 3) / 4)
    assert m["fc.weight"].requires_grad and m["fc.bias"].array.tolist() == [-1.5, 2.0]
    assert obj["step"] == 12
    assert obj["ids"].dtype == "int32" and obj["ids"].array.tolist() == [3, -7, 0, 2 ** 30]
    # float16 tensors are Float32Array data in torch.js (src/dtype.ts:9)
    assert obj["h"].dtype == "float32" and obj["h"].array.tolist() == [0.5, -1.0]
    assert obj["flags"].dtype == "bool" and obj["flags"].array.tolist() == [1, 0, 1]
    assert obj["u"].dtype == "int32" and obj["u"].array.tolist() == [7, 2 ** 31 - 1]
    assert obj["hist"][0].array.tolist() == [[-128, 5], [0, 127]] and obj["hist"][1] == "tag"


def _pt_zip(pkl_bytes):
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w") as z:
        z.writestr("archive/data.pkl", pkl_bytes)
    return buf.getvalue()


def test_weights_only_refuses_other_globals(S):
    """A pickle naming any callable outside a state_dict's (here builtins.eval
    and os.system) is refused at find_class, before anything is called."""
    for mod, name in (("builtins", "eval"), ("os", "system"), ("torch", "load")):
        evil = ("c%s\n%s\n(S'1+1'\ntR." % (mod, name)).encode()
        with pytest.raises(pickle.UnpicklingError, match="not allowed"):
            S.read_archive(_pt_zip(evil))
    with pytest.raises(ValueError, match="neither model.json nor data.pkl"):
        buf = io.BytesIO()
        with zipfile.ZipFile(buf, "w") as z:
            z.writestr("other.txt", "x")
        S.read_archive(buf.getvalue())


def test_host_round_trip_keeps_bytes(S):
    r = np.random.default_rng(0)
    obj = {"w": S.HostTensor(r.standard_normal((3, 5)).astype(np.float32), "float32", True),
           "i": S.HostTensor(np.array([-5, 0, 2 ** 31 - 1], np.int32), "int32"),
           "b": S.HostTensor(np.array([1, 0], np.uint8), "bool"),
           "meta": {"epoch": 3, "lr": 1e-3, "names": ["a", "b"]}}

    def arrays_of(o):
        return (o.array, o.dtype, o.requires_grad) if isinstance(o, S.HostTensor) else None
    data = S.dumps_archive(obj, arrays_of)
    with zipfile.ZipFile(io.BytesIO(data)) as z:
        assert sorted(z.namelist()) == ["model.json", "tensors/0.bin", "tensors/1.bin",
                                        "tensors/2.bin"]
    back = S.read_archive(data)
    for k in ("w", "i", "b"):
        assert back[k].dtype == obj[k].dtype
        assert back[k].array.tobytes() == obj[k].array.tobytes()
    assert back["w"].requires_grad and not back["i"].requires_grad
    assert back["meta"] == {"epoch": 3, "lr": 1e-3, "names": ["a", "b"]}


def _crafted_pt(storage_floats, offset, size, stride):
    """A .pt archive whose data.pkl rebuilds one float32 tensor from a
    storage of `storage_floats` elements with the given offset, size and
    stride (written with the real torch._utils._rebuild_tensor_v2 global, so
    the file is what a tampered torch.save output would hold)."""
    import torch

    class _Stor:
        pass
    st = _Stor()

    class _P(pickle.Pickler):
        def persistent_id(self, obj):
            if obj is st:
                return ("storage", torch.FloatStorage, "0", "cpu", storage_floats)
            return None

    class _T:
        def __reduce__(self):
            return (torch._utils._rebuild_tensor_v2, (st, offset, size, stride, False, None))
    buf = io.BytesIO()
    _P(buf, protocol=2).dump({"t": _T()})
    out = io.BytesIO()
    with zipfile.ZipFile(out, "w") as z:
        z.writestr("archive/data.pkl", buf.getvalue())
        z.writestr("archive/data/0", np.arange(storage_floats, dtype="<f4").tobytes())
    return out.getvalue()


def test_pt_loader_bounds_checks_views(S):
    """Views that reach outside their storage are refused: negative strides
    (which would read before the storage's start), negative sizes, offsets
    outside it and views past its end.  Well-formed views still load."""
    ok = S.read_archive(_crafted_pt(12, 2, (2, 3), (4, 1)))["t"]
    assert ok.array.tolist() == [[2, 3, 4], [6, 7, 8]]
    ok = S.read_archive(_crafted_pt(4, 3, (1,), (1,)))["t"]
    assert ok.array.tolist() == [3]
    empty = S.read_archive(_crafted_pt(4, 4, (0,), (1,)))["t"]
    assert empty.array.shape == (0,)
    for off, size, stride in [(0, (3,), (-1,)), (3, (3,), (-1,)), (2, (2, 2), (1, -2)),
                              (-1, (2,), (1,)), (0, (-2,), (1,)), (5, (1,), (1,)),
                              (0, (5,), (1,)), (2, (2, 2), (2, 1)), (4, (1,), (1,))]:
        with pytest.raises(ValueError):
            S.read_archive(_crafted_pt(4, off, size, stride))
    # the advisor's repro, called directly: storage of 4 floats, (3,), (-1,)
    stor = S._Storage(np.arange(4, dtype="<f4").tobytes(), "float32", False)
    with pytest.raises(ValueError):
        S._rebuild_tensor_v2(stor, 0, (3,), (-1,))
