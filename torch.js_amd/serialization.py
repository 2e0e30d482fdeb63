"""torch.save / torch.load for the 'hip' device (src/serialization/common.ts,
src/serialization/pytorch_loader.ts, src/serialization/browser.ts).

Two archive formats, both zip files:

  * torch.js's own (common.ts:22-166): `model.json` holds the saved object
    with every tensor replaced by {"__tensor__": true, "id", "shape",
    "dtype", "requires_grad", "device"}, and `tensors/<id>.bin` holds the
    tensor's elements, little-endian, in its dtype's array type
    (src/dtype.ts:7-15; float16 tensors are kept as Float32Array there, so
    their .bin holds 4-byte floats).
  * PyTorch's (`torch.save`, read by pytorch_loader.ts:32-186): `data.pkl`
    (under one top-level directory) describes the object; each tensor is a
    `_rebuild_tensor_v2(storage, offset, size, stride, ...)` call whose
    storage is the file `data/<key>`.  It is read with a weights-only
    unpickler: only OrderedDict, the tensor / parameter rebuilders and the
    storage types are resolvable; any other global refuses the file, so
    nothing in it is executed.  Unlike the reference's loader, the saved
    strides and storage offset are applied (a transposed or sliced tensor
    comes back as PyTorch saved it).

Host parsing (`read_archive`, numpy arrays) is separate from the upload to
the device (`load`), which creates 'hip' tensors with the library's
allocator.  `load` detects the format as browser.ts:27-46 does: the
PyTorch layout first, then torch.js's.
"""
import collections
import io
import json
import pickle
import zipfile

import numpy as np

MODEL_FILENAME = "model.json"

# torch.js dtype -> (numpy type of its .bin elements, dtype on the hip device)
_TJS_DTYPES = {
    "float32": ("<f4", "float32"),
    "float16": ("<f4", "float32"),  # stored as Float32Array by torch.js (dtype.ts:9)
    "int32": ("<i4", "int32"),
    "uint32": ("<u4", "int32"),
    "int8": ("i1", "int32"),
    "uint8": ("u1", "uint8"),
    "bool": ("u1", "bool"),
}

# PyTorch storage class -> numpy element type (bfloat16 is decoded by hand)
_PT_STORAGES = {
    "FloatStorage": "<f4", "DoubleStorage": "<f8", "HalfStorage": "<f2",
    "BFloat16Storage": "bfloat16", "LongStorage": "<i8", "IntStorage": "<i4",
    "ShortStorage": "<i2", "CharStorage": "i1", "ByteStorage": "u1", "BoolStorage": "?",
}


class HostTensor:
    """A tensor read from an archive, before upload: a contiguous numpy
    array in one of the device's dtypes, and its requires_grad flag."""

    __slots__ = ("array", "dtype", "requires_grad")

    def __init__(self, array, dtype, requires_grad=False):
        self.array = array
        self.dtype = dtype
        self.requires_grad = bool(requires_grad)

    @property
    def shape(self):
        return tuple(self.array.shape)

    def __repr__(self):
        return "HostTensor(shape=%s, dtype=%s)" % (list(self.shape), self.dtype)


def _device_array(a):
    """numpy array -> (contiguous array in a device dtype, that dtype):
    floating types become float32, integers int32 (values must fit),
    uint8 and bool stay."""
    if a.dtype == np.bool_:
        return np.ascontiguousarray(a.astype(np.uint8)), "bool"
    if a.dtype == np.uint8:
        return np.ascontiguousarray(a), "uint8"
    if a.dtype.kind == "f":
        return np.ascontiguousarray(a.astype(np.float32)), "float32"
    if a.dtype.kind in "iu":
        if a.size and (a.min() < -2 ** 31 or a.max() > 2 ** 31 - 1):
            raise OverflowError("integer tensor values do not fit the device's int32")
        return np.ascontiguousarray(a.astype(np.int32)), "int32"
    raise TypeError("unsupported element type %s" % a.dtype)


# ------------------------------------------------------------------ PyTorch format


class _StorageType:
    __slots__ = ("name",)

    def __init__(self, name):
        self.name = name


class _Storage:
    """The elements of one data/<key> file, decoded to numpy."""

    __slots__ = ("values",)

    def __init__(self, raw, kind, big_endian):
        if kind == "bfloat16":
            u = np.frombuffer(raw, dtype=">u2" if big_endian else "<u2").astype(np.uint32)
            self.values = (u << 16).view(np.float32)
        else:
            dt = np.dtype(kind)
            if big_endian and dt.itemsize > 1:
                dt = dt.newbyteorder(">")
            self.values = np.frombuffer(raw, dtype=dt)


def _rebuild_tensor_v2(storage, storage_offset, size, stride, requires_grad=False,
                       backward_hooks=None, metadata=None):
    v = storage.values
    if not isinstance(storage_offset, int) or isinstance(storage_offset, bool):
        raise ValueError("tensor storage offset must be an int")
    if not isinstance(size, (tuple, list)) or not isinstance(stride, (tuple, list)):
        raise ValueError("tensor size and stride must be sequences")
    if len(size) != len(stride):
        raise ValueError("tensor size and stride differ in length")
    for d in tuple(size) + tuple(stride):
        if not isinstance(d, int) or isinstance(d, bool):
            raise ValueError("tensor size and stride entries must be ints")
    size = tuple(size)
    stride = tuple(stride)
    # PyTorch writes no negative sizes or strides; a file that has them is
    # malformed (a negative stride would make the view reach before the
    # start of its storage)
    if any(s < 0 for s in size) or any(st < 0 for st in stride):
        raise ValueError("tensor sizes and strides must be non-negative")
    if storage_offset < 0 or storage_offset > v.size:
        raise ValueError("tensor storage offset outside its storage")
    n = int(np.prod(size)) if size else 1
    if n:
        # with every stride >= 0 the lowest element reached is the offset
        # and the highest is offset + sum((size - 1) * stride)
        last = storage_offset + sum((s - 1) * st for s, st in zip(size, stride))
        if storage_offset >= v.size or last >= v.size:
            raise ValueError("tensor view past the end of its storage")
        view = np.lib.stride_tricks.as_strided(v[storage_offset:], shape=size,
                                               strides=[st * v.itemsize for st in stride])
    else:
        view = np.zeros(size, dtype=v.dtype)
    arr, dt = _device_array(np.array(view))
    return HostTensor(arr, dt, requires_grad)


def _rebuild_parameter(data, requires_grad, backward_hooks, state=None):
    if isinstance(data, HostTensor):
        data.requires_grad = bool(requires_grad)
    return data


class _WeightsOnlyUnpickler(pickle.Unpickler):
    """Resolves only what a saved state_dict needs; every other global is
    refused, so loading never runs code from the file."""

    _ALLOWED = {
        ("collections", "OrderedDict"): collections.OrderedDict,
        ("torch._utils", "_rebuild_tensor_v2"): _rebuild_tensor_v2,
        ("torch._utils", "_rebuild_parameter"): _rebuild_parameter,
        ("torch._utils", "_rebuild_parameter_with_state"): _rebuild_parameter,
    }

    def __init__(self, data, read_storage):
        super().__init__(io.BytesIO(data))
        self._read_storage = read_storage

    def find_class(self, module, name):
        fn = self._ALLOWED.get((module, name))
        if fn is not None:
            return fn
        if module == "torch" and name in _PT_STORAGES:
            return _StorageType(name)
        raise pickle.UnpicklingError("weights-only load: global %s.%s is not allowed"
                                     % (module, name))

    def persistent_load(self, pid):
        if not (isinstance(pid, tuple) and len(pid) >= 3 and pid[0] == "storage" and
                isinstance(pid[1], _StorageType)):
            raise pickle.UnpicklingError("weights-only load: unsupported persistent id %r"
                                         % (pid,))
        return self._read_storage(pid[1].name, str(pid[2]))


def _read_pytorch(z, prefix):
    big = False
    bo = prefix + "byteorder"
    if bo in z.namelist():
        big = z.read(bo).decode().strip() == "big"
    cache = {}

    def read_storage(kind, key):
        if key not in cache:
            cache[key] = _Storage(z.read(prefix + "data/" + key), _PT_STORAGES[kind], big)
        return cache[key]
    return _WeightsOnlyUnpickler(z.read(prefix + "data.pkl"), read_storage).load()


# ------------------------------------------------------------------ torch.js format


def _read_torchjs(z):
    obj = json.loads(z.read(MODEL_FILENAME).decode("utf-8"),
                     object_pairs_hook=collections.OrderedDict)
    names = set(z.namelist())

    def revive(o):
        if isinstance(o, dict):
            if o.get("__tensor__") is True:
                entry = "tensors/%s.bin" % o["id"]
                if entry not in names:
                    raise ValueError("Missing tensor data for id %s" % o["id"])
                if o["dtype"] not in _TJS_DTYPES:
                    raise ValueError("unsupported dtype %r" % o["dtype"])
                elem, dt = _TJS_DTYPES[o["dtype"]]
                shape = tuple(int(s) for s in o["shape"])
                a = np.frombuffer(z.read(entry), dtype=elem)
                if a.size != int(np.prod(shape)):
                    raise ValueError("tensor %s: %d elements for shape %s"
                                     % (o["id"], a.size, list(shape)))
                arr, got = _device_array(a.reshape(shape))
                if dt == "bool":
                    arr, got = (arr != 0).astype(np.uint8), "bool"
                return HostTensor(arr, got, o.get("requires_grad", False))
            return collections.OrderedDict((k, revive(v)) for k, v in o.items())
        if isinstance(o, list):
            return [revive(v) for v in o]
        return o
    return revive(obj)


# ------------------------------------------------------------------ archives


def _open_zip(f):
    if isinstance(f, (bytes, bytearray, memoryview)):
        return zipfile.ZipFile(io.BytesIO(bytes(f)))
    return zipfile.ZipFile(f)


def read_archive(f):
    """Parses a torch.js zip or a PyTorch zip into its object, tensors as
    HostTensor (no device needed).  f: a path, a file object or bytes."""
    with _open_zip(f) as z:
        names = z.namelist()
        pkl = [n for n in names if n == "data.pkl" or n.endswith("/data.pkl")]
        if pkl:
            return _read_pytorch(z, pkl[0][:-len("data.pkl")])
        if MODEL_FILENAME in names:
            return _read_torchjs(z)
    raise ValueError("Invalid archive: neither %s nor data.pkl found." % MODEL_FILENAME)


def _to_device(o):
    from .tensor import from_numpy
    if isinstance(o, HostTensor):
        return from_numpy(o.array, requires_grad=o.requires_grad, dtype=o.dtype)
    if isinstance(o, dict):
        return collections.OrderedDict((k, _to_device(v)) for k, v in o.items())
    if isinstance(o, (list, tuple)):
        return type(o)(_to_device(v) for v in o)
    return o


def load(f):
    """torch.load (browser.ts:27-46): the object of a PyTorch or torch.js
    archive with every tensor on the 'hip' device."""
    return _to_device(read_archive(f))


def load_pytorch_zip(f):
    """loadPyTorchZip (pytorch_loader.ts:32): only PyTorch's layout."""
    with _open_zip(f) as z:
        pkl = [n for n in z.namelist() if n == "data.pkl" or n.endswith("/data.pkl")]
        if not pkl:
            raise ValueError("Not a valid PyTorch zip archive: data.pkl not found")
        return _to_device(_read_pytorch(z, pkl[0][:-len("data.pkl")]))


# ------------------------------------------------------------------ saving


def dumps_archive(obj, arrays_of):
    """serializeToZip (common.ts:32-75) over host data: `arrays_of(t)` gives
    (contiguous numpy array, dtype name, requires_grad) for each tensor-like
    leaf t (None for any other value).  Returns the zip bytes."""
    blobs = []

    def replace(o):
        got = arrays_of(o)
        if got is not None:
            arr, dt, rg = got
            tid = str(len(blobs))
            blobs.append(np.ascontiguousarray(arr))
            return collections.OrderedDict([("__tensor__", True), ("id", tid),
                                            ("shape", [int(s) for s in arr.shape]),
                                            ("dtype", dt), ("requires_grad", bool(rg)),
                                            ("device", "hip")])
        if isinstance(o, dict):
            return collections.OrderedDict((str(k), replace(v)) for k, v in o.items())
        if isinstance(o, (list, tuple)):
            return [replace(v) for v in o]
        if isinstance(o, (np.integer, np.floating)):
            return o.item()
        return o
    doc = json.dumps(replace(obj), indent=2)
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w") as z:
        z.writestr(zipfile.ZipInfo(MODEL_FILENAME), doc.encode("utf-8"),
                   compress_type=zipfile.ZIP_DEFLATED)
        for i, a in enumerate(blobs):
            # little-endian element bytes of the dtype's array type
            z.writestr("tensors/%d.bin" % i, a.astype(a.dtype.newbyteorder("<")).tobytes(),
                       compress_type=zipfile.ZIP_STORED)
    return buf.getvalue()


def save(obj, f=None):
    """torch.save in torch.js's format (serializeToZip, common.ts:32-75;
    browser.ts:3-17 without the download): every 'hip' tensor is read back
    once and written as tensors/<id>.bin.  f: a path or a binary file
    object; with f None the archive bytes are returned."""
    from .tensor import Tensor

    def arrays_of(o):
        if isinstance(o, Tensor):
            return o.numpy(), o.dtype, o.requires_grad
        if isinstance(o, HostTensor):
            return o.array, o.dtype, o.requires_grad
        return None
    data = dumps_archive(obj, arrays_of)
    if f is None:
        return data
    if isinstance(f, (str, bytes)) or hasattr(f, "__fspath__"):
        with open(f, "wb") as fh:
            fh.write(data)
    else:
        f.write(data)
    return None
