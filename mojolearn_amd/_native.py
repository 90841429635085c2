"""Loader of libmlgemm.so (the gfx950 kernels behind a C ABI, include/mlgemm.h).

There is no fallback: if the library is missing or cannot load, every call raises.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmlgemm.so")

_lock = threading.Lock()
_lib = None

SINK_T = ctypes.CFUNCTYPE(None, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64)


def _share_hip_runtime():
    """Load PyTorch (when installed) before the library, so that the library's HIP runtime
    dependency binds to the one PyTorch-ROCm already carries.  A process then holds a single
    HIP runtime; with two (the system's and PyTorch's), whichever initialises second finds no
    GPU."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    """The loaded libmlgemm.so, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        _share_hip_runtime()
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"mojolearn_amd: {LIB_PATH} is not built; run `python -c \"import __graft_entry__ as g; g.build()\"` "
                "or `python mojolearn_amd/build.py` (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
        L.linalg_native_v1.argtypes = [i64, i64, i64, i64, i64, i64, i64, i64, i64, SINK_T]
        L.linalg_native_v1.restype = i64
        L.mlg_abi_name.argtypes = []
        L.mlg_abi_name.restype = ctypes.c_char_p
        L.mlg_gemm_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i64, vp]
        L.mlg_gemm_f32.restype = ctypes.c_int
        L.mlg_gemm_bf16w.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i32, i64, vp]
        L.mlg_gemm_bf16w.restype = ctypes.c_int
        L.mlg_gemm_int8w.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, i64, vp]
        L.mlg_gemm_int8w.restype = ctypes.c_int
        L.mlg_gemm_ws.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, i32, i32, i64, vp, i64, vp]
        L.mlg_gemm_ws.restype = ctypes.c_int
        L.mlg_gemm_noalloc.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, i32, i32, i64, vp]
        L.mlg_gemm_noalloc.restype = ctypes.c_int
        L.mlg_gemm_workspace_bytes.argtypes = [i64, i64, i64, i32, i32, i32, i64]
        L.mlg_gemm_workspace_bytes.restype = i64
        L.mlg_gemm_workspace_bytes_for.argtypes = [vp, vp, i64, i64, i64, i32, i32, i32, i64]
        L.mlg_gemm_workspace_bytes_for.restype = i64
        L.mlg_gemm_counter_bytes.argtypes = [i64, i64, i64, i32, i32, i32, i64]
        L.mlg_gemm_counter_bytes.restype = i64
        L.mlg_gemm_route.argtypes = [vp, vp, i64, i64, i64, i32, i32, i32, i64, i32]
        L.mlg_gemm_route.restype = i64
        L.mlg_gemm_leaf_ptr.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp]
        L.mlg_gemm_leaf_ptr.restype = ctypes.c_int
        L.mlg_gemm_leaf_ptr_epi.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, i64, i32, vp, i32, vp]
        L.mlg_gemm_leaf_ptr_epi.restype = ctypes.c_int
        L.mlg_seq_gemm.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, i32, vp]
        L.mlg_seq_gemm.restype = ctypes.c_int
        L.mlg_follow.argtypes = [vp, i64, i64, i64, i32, vp, i32, vp]
        L.mlg_follow.restype = ctypes.c_int
        L.mlg_bf16_widen.argtypes = [vp, vp, i64, vp]
        L.mlg_bf16_widen.restype = ctypes.c_int
        L.mlg_bf16_narrow.argtypes = [vp, vp, i64, vp]
        L.mlg_bf16_narrow.restype = ctypes.c_int
        L.mlg_int8_quantize.argtypes = [vp, vp, vp, i64, i64, vp]
        L.mlg_int8_quantize.restype = ctypes.c_int
        L.mlg_int8_dequantize.argtypes = [vp, vp, vp, i64, i64, vp]
        L.mlg_int8_dequantize.restype = ctypes.c_int
        L.mlg_gemm_int8i32.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, vp]
        L.mlg_gemm_int8i32.restype = ctypes.c_int
        L.mlg_gemm_int8i32_workspace_bytes.argtypes = [vp, vp, i64, i64, i64]
        L.mlg_gemm_int8i32_workspace_bytes.restype = i64
        L.mlg_gemm_int8i32_ws.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, vp, i64, vp]
        L.mlg_gemm_int8i32_ws.restype = ctypes.c_int
        L.mlg_f16_widen.argtypes = [vp, vp, i64, vp]
        L.mlg_f16_widen.restype = ctypes.c_int
        L.mlg_int15_quantize.argtypes = [vp, vp, vp, vp, i64, i64, vp]
        L.mlg_int15_quantize.restype = ctypes.c_int
        L.mlg_int15_dequantize.argtypes = [vp, vp, vp, vp, i64, i64, vp]
        L.mlg_int15_dequantize.restype = ctypes.c_int
        L.mlg_gemm_int15i64.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, vp]
        L.mlg_gemm_int15i64.restype = ctypes.c_int
        L.mlg_gemm_int15i64_workspace_bytes.argtypes = [vp, vp, vp, vp, i64, i64, i64]
        L.mlg_gemm_int15i64_workspace_bytes.restype = i64
        L.mlg_gemm_int15i64_ws.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, vp, i64, vp]
        L.mlg_gemm_int15i64_ws.restype = ctypes.c_int
        L.mlg_stream_read.argtypes = [vp, i64, i64, i32, vp, vp]
        L.mlg_stream_read.restype = ctypes.c_int
        L.mlg_int8w_packed_bytes.argtypes = [i64, i64]
        L.mlg_int8w_packed_bytes.restype = i64
        L.mlg_int8w_pack.argtypes = [vp, vp, i64, i64, vp]
        L.mlg_int8w_pack.restype = ctypes.c_int
        L.mlg_gemv_int8w_packed_workspace_bytes.argtypes = [i64, i64, i64]
        L.mlg_gemv_int8w_packed_workspace_bytes.restype = i64
        L.mlg_gemv_int8w_packed_counter_bytes.argtypes = [i64, i64, i64]
        L.mlg_gemv_int8w_packed_counter_bytes.restype = i64
        L.mlg_gemv_int8w_packed.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, vp, i64, vp]
        L.mlg_gemv_int8w_packed.restype = ctypes.c_int
        L.mlg_last_error.argtypes = []
        L.mlg_last_error.restype = ctypes.c_char_p
        for name in ("mlg_numeric_mode", "mlg_profile_version", "mlg_lowbit_profile_version"):
            getattr(L, name).argtypes = []
            getattr(L, name).restype = i64
        _lib = L
    return _lib


class NativeError(Exception):
    pass


def call(op, addrs, ints):
    """One call of the op table entry `linalg_native_v1` (host pointers).

    Errors come back through the sink exactly once; a message that starts with
    "TypeError: " raises TypeError (prefix removed), anything else RuntimeError.
    """
    L = lib()
    msgs = []

    def _sink(ctx, ptr, n):
        msgs.append(ctypes.string_at(ptr, n).decode("utf-8", "replace"))

    sink = SINK_T(_sink)
    a = (ctypes.c_int64 * max(len(addrs), 1))(*[int(x) for x in addrs])
    p = (ctypes.c_int64 * max(len(ints), 1))(*[int(x) for x in ints])
    result = ctypes.c_int64(0)
    rc = L.linalg_native_v1(op, ctypes.addressof(a), len(addrs), ctypes.addressof(p), len(ints),
                            0, 0, ctypes.addressof(result), 0, sink)
    if rc != 0:
        msg = msgs[0] if msgs else "linalg native ABI: failed without a message"
        if msg.startswith("TypeError: "):
            raise TypeError(msg[len("TypeError: "):])
        raise RuntimeError(msg)
    return result.value


def check(rc):
    """Raise RuntimeError with mlg_last_error() if a device entry failed."""
    if rc != 0:
        raise RuntimeError(lib().mlg_last_error().decode("utf-8", "replace"))


_capsule_keep = None


def capsule():
    """The op table as the reference's providers export it: a PyCapsule named
    "mojolearn.linalg.v1" whose pointer is a one-entry array holding `linalg_native_v1`
    (gemm/linalg_dispatch.mojo:10-11,92-102; providers/python/neural_descriptor_pyapi_door.mojo:76-87).
    The table and the name live for the life of the process, as PyCapsule borrows both."""
    global _capsule_keep
    L = lib()
    if _capsule_keep is None:
        name = ctypes.create_string_buffer(L.mlg_abi_name())
        table = (ctypes.c_void_p * 1)(ctypes.cast(L.linalg_native_v1, ctypes.c_void_p).value)
        new = ctypes.pythonapi.PyCapsule_New
        new.restype = ctypes.py_object
        new.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _capsule_keep = (name, table, new(ctypes.addressof(table), ctypes.addressof(name), None))
    return _capsule_keep[2]
