"""ctypes binding of the HIP library's C ABI (``include/liteinfer_amd.h``).

The library is loaded on first use, after torch — so the HIP runtime it links
by soname is the one torch already loaded, and a torch stream handle is a
valid ``hipStream_t`` for it. There is no fallback: if the library is missing
the paged path refuses to run and says how to build it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from liteinfer_amd import _build

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libliteinfer_amd.so"

LI_F32, LI_F16, LI_BF16, LI_FP8_E4M3 = 0, 1, 2, 3
LI_OK, LI_EINVAL, LI_EUNSUPPORTED, LI_ELAUNCH, LI_EWORKSPACE = 0, -1, -2, -3, -4
LI_FLAG_FORCE_GENERIC = 1
LI_FLAG_EQUAL_SPLITS = 2
LI_FLAG_PREFILL_ONLY = 4

# Device scratch li_paged_decode_noalloc holds per GPU (include/liteinfer_amd.h).
DECODE_NOALLOC_SCRATCH_BYTES = 32 << 20

DTYPE_CODES = {torch.float32: LI_F32, torch.float16: LI_F16, torch.bfloat16: LI_BF16}

# The pool element type of a quantised cache (OCP e4m3: what gfx950's fp8
# conversions implement).
FP8_POOL_DTYPE = torch.float8_e4m3fn

# Every symbol the header declares, in declaration order.
EXPORTED_SYMBOLS = (
    "li_last_error_string",
    "li_abi_version",
    "li_build_id",
    "li_kv_scatter",
    "li_kv_scatter_fp8",
    "li_rope_kv_write",
    "li_rope_kv_write_fp8",
    "li_choose_num_splits",
    "li_paged_decode_plan",
    "li_paged_decode",
    "li_paged_decode_ex",
    "li_paged_decode_write",
    "li_paged_decode_noalloc",
    "li_paged_prefill_plan",
    "li_prefill_row_groups",
    "li_paged_prefill",
    "li_paged_prefill_ex",
    "li_add_rms_norm",
    "li_silu_mul",
)

_i64, _i32, _p, _f32, _sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "li_add_rms_norm": (_i32, [_p, _p, _p, _p, _i64, _i32, _i64, _i64, _i64, _f32, _i32, _p]),
    "li_silu_mul": (_i32, [_p, _p, _i64, _i32, _i64, _i64, _i32, _p]),
    "li_last_error_string": (ctypes.c_char_p, []),
    "li_abi_version": (_i32, []),
    "li_build_id": (ctypes.c_char_p, []),
    "li_kv_scatter": (
        _i32,
        [_p, _p, _i64p, _i64p, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p],
    ),
    "li_kv_scatter_fp8": (
        _i32,
        [_p, _p, _i64p, _i64p, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _f32, _f32, _p, _p],
    ),
    "li_rope_kv_write": (
        _i32,
        [_p, _i64p, _p, _i64p, _p, _i64p, _p, _p, _i64p, _i64, _i64, _p, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p],
    ),
    "li_rope_kv_write_fp8": (
        _i32,
        [_p, _i64p, _p, _i64p, _p, _i64p, _p, _p, _i64p, _i64, _i64, _p, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _f32, _p, _p],
    ),
    "li_choose_num_splits": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "li_paged_decode_plan": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_sz)],
    ),
    "li_paged_decode": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i64, _i64,
         _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz, _i32, _i32, _p],
    ),
    "li_paged_decode_ex": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i64, _i64,
         _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz, _i32, _i32, _f32, _f32, _i32, _p],
    ),
    "li_paged_decode_write": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
         _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz, _i32, _i32, _f32, _f32, _i32, _p],
    ),
    "li_paged_decode_noalloc": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i64, _i64,
         _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _p],
    ),
    "li_prefill_row_groups": (
        _i32, [ctypes.c_ulonglong, ctypes.c_ulonglong, _i32, _i32, _i32, _i32, _i32, _i32, _i32],
    ),
    "li_paged_prefill_plan": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_sz)]),
    "li_paged_prefill": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i32, _i32, _p, _i64, _i64,
         _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz, _i32, _i32, _p],
    ),
    "li_paged_prefill_ex": (
        _i32,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i32, _i32, _p, _i64, _i64,
         _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz, _i32, _i32, _f32, _f32, _i32, _p],
    ),
}

ABI_VERSION = 7

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    """The HIP library has not been built."""


def library_path() -> Path:
    return LIB_PATH


def is_built() -> bool:
    return LIB_PATH.exists()


def load() -> ctypes.CDLL:
    """The loaded library, with every entry point's signature declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryMissing(
                    f"the liteinfer_amd HIP library is not built ({LIB_PATH} is missing); "
                    "run `python -m liteinfer_amd._build`"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            version = lib.li_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {version}, this package expects {ABI_VERSION}; rebuild it")
            built = lib.li_build_id().decode()
            expected = _build.source_hash()
            if built != expected:
                raise RuntimeError(
                    f"{LIB_PATH} was built from other sources (build id {built}, the sources here hash to "
                    f"{expected}); rebuild it with `python -m liteinfer_amd._build`"
                )
            _lib = lib
    return _lib


def last_error() -> str:
    return load().li_last_error_string().decode(errors="replace")


def check(status: int, what: str) -> None:
    """Raise the error a failed call reports: ValueError for bad arguments, RuntimeError otherwise."""
    if status == LI_OK:
        return
    message = f"{what}: {last_error()}"
    if status in (LI_EINVAL, LI_EUNSUPPORTED, LI_EWORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"the paged kernels take float32, float16 or bfloat16, not {dtype}") from None


def stream_handle(device: torch.device) -> int:
    """The current torch stream of `device`, as the hipStream_t the library takes.

    Read through torch's raw-stream accessor (the handle itself, no Stream
    object built per call); torch.cuda.current_stream where that is absent.
    """
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def i64_array(values) -> ctypes.Array:
    return (ctypes.c_int64 * len(values))(*values)
