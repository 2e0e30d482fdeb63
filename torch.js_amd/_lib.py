"""ctypes binding of libtorchjs_hip.so (the C ABI declared in
include/torchjs_hip.h).

The library is required: importing the package works without it, but the
first call that needs the device raises, naming the missing file.  Nothing
in the package falls back to a CPU implementation.
"""
import ctypes
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtorchjs_hip.so")

c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_u32 = ctypes.c_uint32
c_f32 = ctypes.c_float
c_f64 = ctypes.c_double
c_vp = ctypes.c_void_p
c_sz = ctypes.c_size_t
P_i64 = ctypes.POINTER(c_i64)


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("warp_size", ctypes.c_int32),
        ("total_mem", ctypes.c_int64),
        ("max_alloc", ctypes.c_int64),
        ("lds_per_block", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("l2_bytes", ctypes.c_int32),
        ("ordinal", ctypes.c_int32),
    ]


class MemStats(ctypes.Structure):
    _fields_ = [
        ("active_bytes", ctypes.c_uint64),
        ("pooled_bytes", ctypes.c_uint64),
        ("peak_bytes", ctypes.c_uint64),
        ("allocations", ctypes.c_uint64),
        ("device_mallocs", ctypes.c_uint64),
    ]


class Conv2dDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "n", "c", "h", "w", "oc", "kh", "kw", "stride_h", "stride_w", "pad_h", "pad_w",
        "dil_h", "dil_w", "groups", "oh", "ow")]


# fused elementwise expression programs (tjh_expr, include/torchjs_hip.h)
EXPR_MAX_INS = 48
EXPR_MAX_LEAVES = 8
EXPR_MAX_REGS = 16
EXPR_NONE = 255
EXPR_OP = {"load": 0, "const": 1, "unary": 2, "unary_bwd": 3, "binary": 4, "ternary": 5,
           "scalar": 6, "scalar_rev": 7, "axpy": 8}
LEAF = {"contig": 0, "row": 1, "col": 2, "scalar": 3}


class ExprIns(ctypes.Structure):
    _fields_ = [("op", ctypes.c_uint8), ("code", ctypes.c_uint8), ("dst", ctypes.c_uint8),
                ("a", ctypes.c_uint8), ("b", ctypes.c_uint8), ("c", ctypes.c_uint8),
                ("pad0", ctypes.c_uint8), ("pad1", ctypes.c_uint8), ("f", ctypes.c_float)]


class Expr(ctypes.Structure):
    _fields_ = [("n_ins", ctypes.c_int32), ("n_leaves", ctypes.c_int32),
                ("result", ctypes.c_int32), ("result2", ctypes.c_int32),
                ("result3", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("ins", ExprIns * EXPR_MAX_INS),
                ("leaf", ctypes.c_void_p * EXPR_MAX_LEAVES),
                ("period", ctypes.c_int64 * EXPR_MAX_LEAVES),
                ("kind", ctypes.c_int32 * EXPR_MAX_LEAVES)]


# name -> argtypes (all functions return int status unless listed in _RESTYPE)
SIGNATURES = {
    "tjh_last_error": [],
    "tjh_version": [],
    "tjh_init": [c_int],
    "tjh_is_initialized": [],
    "tjh_device_count": [ctypes.POINTER(c_int)],
    "tjh_get_device_info": [ctypes.POINTER(DeviceInfo)],
    "tjh_synchronize": [],
    "tjh_malloc": [c_sz, ctypes.POINTER(c_vp)],
    "tjh_free": [c_vp],
    "tjh_memory_stats": [ctypes.POINTER(MemStats)],
    "tjh_empty_cache": [],
    "tjh_reset_peak": [],
    "tjh_h2d": [c_vp, c_vp, c_sz],
    "tjh_d2h": [c_vp, c_vp, c_sz],
    "tjh_d2d": [c_vp, c_vp, c_sz],
    "tjh_d2h_start": [c_vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint64)],
    "tjh_d2h_finish": [ctypes.c_uint64, c_vp],
    "tjh_kprof_enable": [c_int],
    "tjh_kprof_filter": [ctypes.c_char_p],
    "tjh_kprof_reset": [],
    "tjh_kprof_query": [ctypes.c_char_p, P_i64, ctypes.POINTER(c_f64)],
    "tjh_kprof_names": [ctypes.c_char_p, c_sz],
    "tjh_timer_start": [ctypes.POINTER(c_int)],
    "tjh_timer_stop": [c_int, ctypes.POINTER(c_f64)],
    "tjh_fill_f32": [c_vp, c_i64, c_f32],
    "tjh_fill_i32": [c_vp, c_i64, ctypes.c_int32],
    "tjh_random": [c_vp, c_i64, c_u32, c_int],
    "tjh_copy_strided": [c_int, P_i64, c_vp, P_i64, c_vp, P_i64],
    "tjh_copy_strided_i32": [c_int, P_i64, c_vp, P_i64, c_vp, P_i64],
    "tjh_cast_f32_i32": [c_vp, c_vp, c_i64],
    "tjh_cast_i32_f32": [c_vp, c_vp, c_i64],
    "tjh_unary": [c_int, c_vp, c_vp, c_i64, c_f32],
    "tjh_unary_backward": [c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_f32],
    "tjh_binary": [c_int, c_int, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp],
    "tjh_ternary": [c_int, c_int, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp],
    "tjh_scalar": [c_int, c_vp, c_f32, c_int, c_vp, c_i64],
    "tjh_pow_scalar_backward": [c_vp, c_vp, c_f32, c_vp, c_i64],
    "tjh_axpy": [c_f32, c_vp, c_vp, c_vp, c_i64],
    "tjh_masked_fill": [c_int, P_i64, c_vp, P_i64, c_vp, P_i64, c_f32, c_vp],
    "tjh_compare": [c_int, c_int, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp],
    "tjh_reduce": [c_int, c_vp, c_i64, c_i64, c_i64, c_vp],
    "tjh_expr_eval": [c_vp, c_i64, c_vp],
    "tjh_graph_begin": [ctypes.POINTER(c_int)],
    "tjh_graph_end": [c_int],
    "tjh_graph_replay": [c_int],
    "tjh_graph_destroy": [c_int],
    "tjh_expr_colsum": [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp],
    "tjh_expr_colsum2": [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "tjh_expr_colsum3": [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp],
    "tjh_expr_compile": [c_vp, c_i64, c_int],
    "tjh_argmax": [c_vp, c_i64, c_i64, c_i64, c_int, c_vp],
    "tjh_softmax_forward": [c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_int],
    "tjh_softmax_backward": [c_vp, c_vp, c_vp, c_i64, c_i64, c_int],
    "tjh_cross_entropy_forward": [c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_int32, c_vp, c_f32,
                                  c_vp, c_vp, c_int, c_vp],
    "tjh_cross_entropy_backward": [c_vp, c_i64, c_vp, c_vp, c_f32, c_vp, c_vp, c_i64, c_i64,
                                   ctypes.c_int32, c_int, c_vp, c_i64, c_int],
    "tjh_cross_entropy_row_scale": [c_vp, c_vp, c_i64, c_i64, ctypes.c_int32, c_int, c_vp],
    "tjh_cross_entropy_forward_grad": [c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_int32, c_vp, c_vp,
                                       c_int, c_vp, c_vp, c_i64],
    "tjh_nll_loss_forward": [c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_int32, c_vp, c_vp, c_int,
                             c_vp],
    "tjh_nll_loss_backward": [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int32, c_int, c_vp],
    "tjh_layer_norm_forward": [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32],
    "tjh_layer_norm_backward": [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                                c_int],
    "tjh_layer_norm_backward_res": [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64,
                                    c_i64, c_int],
    "tjh_flush_deferred": [],
    "tjh_layer_norm_backward_noalloc": [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                        c_i64, c_i64, c_int],
    "tjh_embedding_forward": [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp],
    "tjh_embedding_backward": [c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_int],
    "tjh_embedding_pos_forward": [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                                  c_vp],
    "tjh_embedding_pos_backward": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_int, c_vp,
                                   c_i64, c_i64, c_int],
    "tjh_index_select": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    "tjh_index_add": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    "tjh_gather": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    "tjh_scatter_add": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    "tjh_one_hot": [c_vp, c_i64, c_i64, c_vp],
    "tjh_one_hot_i32": [c_vp, c_i64, c_i64, c_vp],
    "tjh_nonzero": [c_vp, c_int, P_i64, c_vp, c_i64, P_i64],
    "tjh_gemm": [c_int, c_int, c_i64, c_i64, c_i64, c_f32, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                 c_f32, c_vp, c_i64, c_i64, c_i64, c_vp, c_int],
    "tjh_gemm_act": [c_int, c_int, c_i64, c_i64, c_i64, c_f32, c_vp, c_i64, c_vp, c_i64, c_f32,
                     c_vp, c_i64, c_vp, c_int, c_vp, c_i64, c_int],
    "tjh_gemm_ce": [c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp,
                    c_i64],
    "tjh_sdpa_forward": [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, P_i64,
                         P_i64, P_i64, P_i64, c_f32, c_int],
    "tjh_sdpa_backward": [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                          c_i64, c_i64, c_i64, ctypes.POINTER(P_i64), c_f32, c_int],
    "tjh_conv2d_forward": [ctypes.POINTER(Conv2dDesc), c_vp, c_vp, c_vp, c_vp],
    "tjh_conv2d_forward_act": [ctypes.POINTER(Conv2dDesc), c_vp, c_vp, c_vp, c_vp, c_int],
    "tjh_conv2d_backward_input": [ctypes.POINTER(Conv2dDesc), c_vp, c_vp, c_vp],
    "tjh_conv2d_backward_weight": [ctypes.POINTER(Conv2dDesc), c_vp, c_vp, c_vp, c_int],
    "tjh_conv2d_backward_weight_bias": [ctypes.POINTER(Conv2dDesc), c_vp, c_vp, c_vp, c_vp, c_int],
    "tjh_timer_end": [c_int],
    "tjh_timer_read": [c_int, ctypes.POINTER(c_f64)],
    "tjh_range_push": [ctypes.c_char_p],
    "tjh_range_pop": [],
    "tjh_mark": [ctypes.c_char_p],
    "tjh_cast": [c_int, c_int, c_vp, c_vp, c_i64],
    "tjh_fill_u8": [c_vp, c_i64, ctypes.c_uint8],
    "tjh_copy_strided_u8": [c_int, P_i64, c_vp, P_i64, c_vp, P_i64],
    "tjh_triangle": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_int],
    "tjh_multinomial": [c_vp, c_i64, c_i64, c_i64, c_int, c_u32, c_vp],
    "tjh_adam_step": [c_int, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), ctypes.POINTER(c_vp),
                      ctypes.POINTER(c_vp), P_i64, P_i64, c_f64, c_f64, c_f64, c_f64, c_f64,
                      c_int],
    "tjh_adam_step_dev": [c_int, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp),
                          ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), P_i64,
                          ctypes.POINTER(c_vp), c_f64, c_f64, c_f64, c_f64, c_f64, c_int],
}

_RESTYPE = {"tjh_last_error": ctypes.c_char_p, "tjh_version": ctypes.c_char_p}

# op codes (enums of the header)
UNARY = {n: i for i, n in enumerate([
    "neg", "exp", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "relu", "gelu", "square",
    "reciprocal", "erf", "abs", "sin", "cos", "silu", "leaky_relu", "elu", "softplus", "sign"])}
BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3, "pow": 4, "maximum": 5, "minimum": 6}
TERNARY = {"div_b": 0, "pow_a": 1, "pow_b": 2, "mul3": 3}
SCALAR = {"add": 0, "sub": 1, "mul": 2, "div": 3, "pow": 4, "maximum": 5, "minimum": 6}
REDUCE = {"sum": 0, "mean": 1, "max": 2, "min": 3, "prod": 4}
COMPARE = {"eq": 0, "ne": 1, "lt": 2, "le": 3, "gt": 4, "ge": 5}
DTYPE = {"float32": 0, "int32": 1, "uint8": 2, "bool": 3}

_lib = None
_lock = threading.Lock()


class HipError(RuntimeError):
    """Raised when a library call fails; carries the library's message."""


def load(path=None):
    """Loads the shared library (once) and declares every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise HipError(
                "libtorchjs_hip.so not found at %s: build it with "
                "`python torch.js_amd/build.py` (the 'hip' device has no CPU fallback)" % p)
        lib = ctypes.CDLL(p)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, c_int)
        _lib = lib
    return _lib


def lib():
    return _lib if _lib is not None else load()


ERR_UNSUPPORTED = 5  # TJH_ERR_UNSUPPORTED


def check(rc, what=""):
    if rc != 0:
        msg = lib().tjh_last_error()
        msg = msg.decode(errors="replace") if msg else ""
        raise HipError("%s%s" % (what + ": " if what else "", msg or ("status %d" % rc)))


def i64arr(vals):
    vals = list(vals)
    return (c_i64 * max(1, len(vals)))(*vals)
