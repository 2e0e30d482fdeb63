"""torch.js's autograd hot path on the MI355X 'hip' device.

The host-side mirror of torch.js's operator surface for this path
(src/index.ts, src/core.ts): tensors on the 'hip' device, backward(),
nn modules and Adam/AdamW, all running on libtorchjs_hip.so's HIP kernels
for gfx950.  Usage mirrors torch.js:

    import torchjs_amd as torch          # see __graft_entry__.load_package
    torch.init()                          # await torch.init()
    x = torch.randn(64, 784)
    model = torch.nn.Sequential(torch.nn.Linear(784, 256), torch.nn.ReLU(),
                                torch.nn.Linear(256, 10))
    loss = torch.nn.functional.cross_entropy(model(x), targets)
    loss.backward()
    torch.optim.Adam(model.parameters(), lr=1e-3).step()
"""
import ctypes

from . import _lib
from . import autograd, functional, nn, optim, profiler, serialization
from .serialization import load, save
from .tensor import Graph as _Graph
from .tensor import graph as _graph
from .tensor import (Tensor, arange, cat, chunk, enable_grad, from_numpy, full, full_like,
                     inference_mode, init, is_grad_enabled, is_initialized, manual_seed, matmul,
                     multinomial, no_grad, ones, ones_like, rand, randn, set_grad_enabled, split,
                     stack, synchronize, tensor, tril, triu, zeros, zeros_like, empty)

nn.functional = functional
F = functional

__all__ = [
    "Tensor", "arange", "autograd", "cat", "chunk", "empty", "enable_grad", "from_numpy", "full",
    "full_like", "hip", "inference_mode", "init", "is_grad_enabled", "is_initialized", "load",
    "manual_seed", "matmul", "multinomial", "nn", "no_grad", "ones", "ones_like", "optim",
    "profiler", "rand",
    "randn", "save", "set_grad_enabled", "split", "stack", "synchronize", "tensor", "tril",
    "triu", "webgpu",
    "zeros", "zeros_like",
]


def library_path():
    return _lib.LIB_PATH


class hip:
    """Device memory statistics (torch.webgpu.memory_stats & co.,
    src/webgpu.ts:11-51), launch timing and HIP graphs."""

    Graph = _Graph
    graph = _graph

    @staticmethod
    def memory_stats():
        """torch.webgpu.memory_stats() (src/webgpu.ts:11-19) with its keys:
        active_bytes, pooled_bytes, peak_bytes and total_allocations, the
        number of blocks the allocator created because its cache had none
        to hand out (the reference's totalAllocations grows only when the
        pool creates a buffer, src/backend/webgpu/buffer.ts:50-57).  Two
        keys of this allocator's own: device_mallocs (the same count, under
        the name the library uses) and allocation_requests (every request
        served, cached or not)."""
        s = _lib.MemStats()
        _lib.check(_lib.lib().tjh_memory_stats(ctypes.byref(s)), "memory_stats")
        return {"active_bytes": s.active_bytes, "pooled_bytes": s.pooled_bytes,
                "peak_bytes": s.peak_bytes, "total_allocations": s.device_mallocs,
                "device_mallocs": s.device_mallocs, "allocation_requests": s.allocations}

    @staticmethod
    def memory_summary():
        """torch.webgpu.memory_summary() (src/webgpu.ts:24-37): the same four
        lines, sizes in MB with two decimals."""
        st = hip.memory_stats()

        def mb(b):
            return "%.2f" % (b / 1024 / 1024)
        rule = "-" * 55
        return ("\nGPU Memory Summary\n%s\nActive Memory:   %s MB\nPooled Memory:   %s MB\n"
                "Peak Memory:     %s MB\nTotal Allocs:    %d\n%s\n"
                % (rule, mb(st["active_bytes"]), mb(st["pooled_bytes"]), mb(st["peak_bytes"]),
                   st["total_allocations"], rule))

    @staticmethod
    def empty_cache():
        _lib.check(_lib.lib().tjh_empty_cache(), "empty_cache")

    @staticmethod
    def reset_peak_memory_stats():
        _lib.check(_lib.lib().tjh_reset_peak(), "reset_peak")

    @staticmethod
    def device_info():
        d = _lib.DeviceInfo()
        _lib.check(_lib.lib().tjh_get_device_info(ctypes.byref(d)), "device_info")
        return {"name": d.name.decode(), "arch": d.arch.decode(), "compute_units": d.compute_units,
                "warp_size": d.warp_size, "total_mem": d.total_mem, "lds_per_block": d.lds_per_block,
                "clock_khz": d.clock_khz, "l2_bytes": d.l2_bytes}

    @staticmethod
    def kernel_timing(enable=True, only=None):
        """Brackets launches with HIP events on the library stream; `only`
        restricts the events to one kernel family."""
        _lib.check(_lib.lib().tjh_kprof_filter((only or "").encode()), "kprof_filter")
        _lib.check(_lib.lib().tjh_kprof_enable(1 if enable else 0), "kprof_enable")

    @staticmethod
    def kernel_timing_reset():
        _lib.check(_lib.lib().tjh_kprof_reset(), "kprof_reset")

    @staticmethod
    def kernel_time(family=""):
        n = ctypes.c_int64(0)
        ms = ctypes.c_double(0.0)
        _lib.check(_lib.lib().tjh_kprof_query(family.encode(), ctypes.byref(n), ctypes.byref(ms)),
                   "kprof_query")
        return n.value, ms.value

    @staticmethod
    def kernel_families():
        buf = ctypes.create_string_buffer(65536)
        _lib.check(_lib.lib().tjh_kprof_names(buf, len(buf)), "kprof_names")
        return [s for s in buf.value.decode().split("\n") if s]


# torch.webgpu.* (src/core.ts:24): the memory functions under the name
# torch.js exports them as
webgpu = hip
