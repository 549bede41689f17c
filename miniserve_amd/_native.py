"""ctypes binding of libmsattn.so (the C ABI in include/msattn.h).

The library is loaded from this package directory only. A missing library is
an error, never a reason to fall back to another implementation.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmsattn.so"

F32, F16, BF16, FP8_E4M3 = 0, 1, 2, 3
DTYPE_CODES = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.float8_e4m3fn: FP8_E4M3,
}

OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_HIP = 0, 1, 2, 3, 4

# msattn_route codes: the kernel msattn_paged_attention runs for a call's shape.
ROUTE_PREFILL, ROUTE_PARTITION_FUSED, ROUTE_PARTITION, ROUTE_STREAMK, ROUTE_GENERIC = 1, 2, 3, 4, 5
ROUTE_PREFILL_STREAMK = 6
ROUTE_NAMES = {ROUTE_PREFILL: "prefill", ROUTE_PARTITION_FUSED: "partition-fused",
               ROUTE_PARTITION: "partition", ROUTE_STREAMK: "stream-K",
               ROUTE_GENERIC: "generic", ROUTE_PREFILL_STREAMK: "prefill stream-K"}
NOALLOC_SCRATCH_BYTES = 64 << 20
MAX_HEAD_DIM = 256

c_int, c_i64, c_size, c_vp, c_float = (ctypes.c_int, ctypes.c_int64, ctypes.c_size_t,
                                       ctypes.c_void_p, ctypes.c_float)

# name -> (restype, argtypes); kept in the order of include/msattn.h.
SIGNATURES = {
    "msattn_abi_version": (c_int, []),
    "msattn_status_string": (ctypes.c_char_p, [c_int]),
    "msattn_partition_tokens": (c_int, [c_int] * 6),
    "msattn_workspace_bytes": (c_size, [c_int] * 6),
    "msattn_paged_attention": (c_int, [
        c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_size,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp]),
    "msattn_paged_attention_noalloc": (c_int, [
        c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp]),
    "msattn_paged_attention_route": (c_int, [
        c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_int, c_int, c_int,
        c_int, c_int, c_int, c_size, ctypes.POINTER(c_int)]),
    "msattn_paged_attention_rope": (c_int, [
        c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_size,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_vp]),
    "msattn_prefix_workspace_bytes": (c_size, [c_int] * 7),
    "msattn_paged_attention_prefix": (c_int, [
        c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_size,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp]),
    "msattn_paged_attention_partials": (c_int, [
        c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_size,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp]),
    "msattn_merge_partials": (c_int, [
        c_vp, c_size, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    "msattn_write_kv": (c_int, [
        c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    "msattn_paged_attention_append": (c_int, [
        c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_size,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_float, c_int, c_int, c_vp]),
    "msattn_gather_kv": (c_int, [
        c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    "msattn_probe_stream_read": (c_int, [c_vp, c_size, c_vp, c_vp]),
}

_lib = None
_lock = threading.Lock()


class MsattnError(RuntimeError):
    """A libmsattn call returned a non-zero status."""

    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed: status {status} ({text})")
        self.status = status


def lib() -> ctypes.CDLL:
    """The loaded library, with argtypes/restype set from SIGNATURES."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"libmsattn.so is not built ({LIB_PATH} missing); run "
                        "`python -m miniserve_amd.build` -- there is no non-HIP fallback")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(fn: str, status: int) -> None:
    if status != OK:
        text = lib().msattn_status_string(status).decode()
        if status in (ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE):
            raise ValueError(f"{fn}: {text} (status {status})")
        raise MsattnError(fn, status, text)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype for msattn: {dtype}") from None


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
