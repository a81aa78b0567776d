"""ctypes binding of libcvmm_hip.so (declared in include/cvmm_hip.h).

torch is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (same SONAME), i.e. one runtime and one
set of streams per process.  There is no fallback: if the library is missing
every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcvmm_hip.so")

F32, F16, BF16 = 0, 1, 2            # cvmm.py:36-44 dtype ids
FLAG_ATOMIC_REDUCE = 1
FLAG_COUNTERS_ZEROED = 2
FLAG_COUNTS_READY = 16
FLAG_ACCUMULATE = 32
FLAG_ROWS_SCALED = 64
# host-only flag of the extension's backward (never passed to the C ABI):
# the weight gradient on a second stream, concurrent with the grad-input
HOST_OVERLAP_BACKWARD = 1 << 48
CAST_T_INTERLEAVED = 1
CAST_N_INTERLEAVED = 2
TUNE_PANEL_TILES_PER_WG = 1
TUNE_WGRAD_ORDER = 2
TUNE_GEMM_ORDER = 3
TUNE_WGRAD_TILE = 5
TUNE_DENSE_TOPK = 6
TUNE_SORT_CHUNK = 7
TUNE_RING_TILE = 8
TUNE_WGRAD_CHUNK = 9

# kernel classes of the timing hooks (include/cvmm_hip.h CVMM_KC_*)
KC_SORT, KC_OFFSETS, KC_CAST_KEYS, KC_GEMM_FWD, KC_GEMM_BWDX, KC_WGRAD, KC_COMBINE, KC_FILL, KC_ROUTE = (
    1, 2, 4, 8, 16, 32, 64, 128, 512)

_DTYPE_ID = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

_SIGS = {
    "cvmm_last_error": (ctypes.c_char_p, []),
    "cvmm_abi_version": (ctypes.c_int, []),
    "cvmm_timing_enable": (ctypes.c_int, [ctypes.c_uint32]),
    "cvmm_tuning_set": (ctypes.c_int, [_I32, _I64]),
    "cvmm_topk_dense": (ctypes.c_int, [_I64, _I32, _I64, _I64, _I64, _I32]),
    "cvmm_timing_result": (ctypes.c_int, [ctypes.c_uint32, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_int64)]),
    "cvmm_sort_workspace_bytes": (_SZ, [_I64, _I32]),
    "cvmm_sort_routes": (ctypes.c_int, [_P, _I32, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "cvmm_sort_routes_noalloc": (ctypes.c_int, [_P, _I32, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "cvmm_copy_ids": (ctypes.c_int, [_P, _I32, _I64, _P, _P]),
    "cvmm_copy_ids_count": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _P, _SZ, _P]),
    "cvmm_expert_offsets": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
    "cvmm_sort_routes_cast_keys": (ctypes.c_int, [_P, _I32, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _SZ,
                                                  _P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _I32,
                                                  _P]),
    "cvmm_sort_routes_cast_keys_ex": (ctypes.c_int, [_P, _I32, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _SZ,
                                                     _P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _I32,
                                                     _I32, _P]),
    "cvmm_cast_keys": (ctypes.c_int, [_P, _I32, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _I32, _P]),
    "cvmm_route_topk_workspace_bytes": (_SZ, [_I64, _I32, _I64]),
    "cvmm_route_topk": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I64, _I32, _P, _P,
                                       _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "cvmm_route_topk_backward": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I64, _I32, _P, _P, _P, _I64, _P]),
    "cvmm_fwd_workspace_bytes": (_SZ, [_I64, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32]),
    "cvmm_fwd": (ctypes.c_int, [
        _P, _I32, _I64, _I64,                 # x, dtype, rows, ld
        _P, _I32, _I32, _I64, _I64,           # keys, dtype, E, d_in, d_out
        _I64, _I64, _I64,                     # key strides
        _P, _P, _P, _I64,                     # sorted_sel, sel_index, out_index, R
        _P, _P, _P, _I32, _I64,               # offsets, route_pos, rw, rw dtype, reduce_k
        _I32, _P, _I32, _I64, _I64,           # op, out, out dtype, out rows, out ld
        _I32, _P, _SZ, _P]),                  # flags, ws, ws bytes, stream
    "cvmm_fwd_keep_scaled": (ctypes.c_int, [
        _P, _I32, _I64, _I64,                 # x, dtype, rows, ld
        _P, _I32, _I32, _I64, _I64,           # keys, dtype, E, d_in, d_out
        _I64, _I64, _I64,                     # key strides
        _P, _P, _P, _I64,                     # sorted_sel, sel_index, out_index, R
        _P, _P, _P, _I32, _I64,               # offsets, route_pos, rw, rw dtype, reduce_k
        _I32, _P, _I32, _I64, _I64,           # op, out, out dtype, out rows, out ld
        _P, _P,                               # scaled rows, int32 written flag
        _I32, _P, _SZ, _P]),                  # flags, ws, ws bytes, stream
    "cvmm_fwd_gelu": (ctypes.c_int, [
        _P, _I32, _I64, _I64,                 # x, dtype, rows, ld
        _P, _I32, _I32, _I64, _I64,           # keys, dtype, E, d_in, d_out
        _I64, _I64, _I64,                     # key strides
        _P, _P, _P, _I64,                     # sorted_sel, sel_index, out_index, R
        _P, _P,                               # offsets, route_pos
        _I32, _P, _I32, _I64, _I64, _P,       # op, out, out dtype, out rows, out ld, pre_act
        _I32, _P, _SZ, _P]),                  # flags, ws, ws bytes, stream
    "cvmm_gelu_backward": (ctypes.c_int, [_P, _I32, _I64, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P]),
    "cvmm_bwd_x_workspace_bytes": (_SZ, [_I64, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I64, _I32, _I32, _I32,
                                         _I32]),
    "cvmm_bwd_x": (ctypes.c_int, [
        _P, _I32, _I64, _I64,                 # grad, dtype, rows, ld
        _P, _I32, _I32, _I64, _I64,           # keys, dtype, E, d_in, d_out
        _I64, _I64, _I64,                     # key strides
        _P, _P, _P, _I64,                     # sorted_sel, sel_index, out_index, R
        _P, _P, _P, _I32, _I64,               # offsets, route_pos, rw, rw dtype, top_k
        _P, _I32, _I64, _I64, _I32,           # x, x dtype, x rows, x ld, op
        _P, _I32, _I64, _I64,                 # grad_x, dtype, rows, ld
        _P, _I32,                             # grad_rw, dtype
        _I32, _P, _SZ, _P]),
    "cvmm_bwd_w_counter_bytes": (_SZ, [_I64, _I32, _I64, _I64, _I32]),
    "cvmm_bwd_w_workspace_bytes": (_SZ, [_I64, _I32, _I64, _I64, _I32, _I32]),
    "cvmm_bwd_w_workspace_bytes_ex": (_SZ, [_I64, _I32, _I64, _I64, _I32, _I32, _I32]),
    "cvmm_bwd_w": (ctypes.c_int, [
        _P, _I32, _I64, _I64,                 # x
        _P, _I32, _I64, _I64,                 # grad
        _I32, _I64, _I64,                     # E, d_in, d_out
        _P, _P, _P, _I64, _P,                 # sorted_sel, sel_index, out_index, R, offsets
        _P, _I32, _I64, _I32,                 # rw, rw dtype, top_k, op
        _P, _I32, _I64, _I64, _I64,           # grad_keys, dtype, strides
        _I32, _P, _SZ, _P]),
}

EXPORTED = tuple(_SIGS)

_lib = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeLibraryMissing(
                        f"{LIB_PATH} is not built (run `python -m cvmm_codex_amd.build`); "
                        "cvmm_codex_amd has no CPU or PyTorch fallback")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


_host = None


def host():
    """The host glue module (``_host``, C++), loaded after the library; raises
    if either has not been built."""
    global _host
    if _host is None:
        lib()
        try:
            from cvmm_codex_amd import _host as h
        except ImportError as e:
            raise NativeLibraryMissing(
                f"cvmm_codex_amd._host is not built ({e}); run `python -m cvmm_codex_amd.build`") from None
        _host = h
    return _host


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().cvmm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def dtype_id(dt: torch.dtype) -> int:
    try:
        return _DTYPE_ID[dt]
    except KeyError:
        raise TypeError(f"cvmm: unsupported dtype {dt}") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of_tensor(t: torch.Tensor) -> int:
    """Raw handle of the current HIP stream of `t`'s device."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return stream_of(t.device)


def stream_of(device: torch.device) -> int:
    """Raw handle of the current HIP stream of `device` (the kernels launch on it)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream
