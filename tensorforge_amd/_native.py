"""ctypes binding of the gfx950 C-ABI library (``include/tensorforge_amd.h``).

The library is loaded lazily on first use, after ``torch`` so that its
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded; every launch then shares torch's streams.  A missing or unloadable
library raises ``RuntimeError``: there is no fallback path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Any

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "lib" / "libtensorforge_amd.so"

TF_DTYPE_FLOAT32 = 0
TF_DTYPE_FLOAT16 = 1
TF_DTYPE_BFLOAT16 = 2

TF_ATTENTION_GENERIC = 0
TF_ATTENTION_MFMA = 1
TF_ATTENTION_FLAG_FORCE_GENERIC = 1
TF_ATTENTION_FLAG_VALU = 16
TF_ATTENTION_FLAG_BALANCED = 32
TF_ATTENTION_WAVES_PER_CU_SHIFT = 8
TF_ATTENTION_HEADS_PER_WG_SHIFT = 20
TF_ATTENTION_TOKENS_PER_WAVE_SHIFT = 24
TF_NOALLOC_SCRATCH_BYTES = 8 << 20

DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: TF_DTYPE_FLOAT32,
    torch.float16: TF_DTYPE_FLOAT16,
    torch.bfloat16: TF_DTYPE_BFLOAT16,
}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> argument types, in header order.
SIGNATURES: dict[str, tuple[Any, ...]] = {
    "tf_last_error": (),
    "tf_hbm_read_probe": (_p, _i64, _i32, _i32, _i32, _p, _p),
    "tf_hbm_page_gather_probe": (_p, _p, _p, _i32, _i64, _i32, _i32, _i32, _p, _p),
    "tf_abi_version": (),
    "tf_paged_gqa_decode_variant": (_i32, _i32, _i32, _i32, _i32),
    "tf_paged_gqa_decode": (
        _p, _p, _p, _p, _p, _p,  # query, key/value cache, tables, lengths, output
        _p, _p, _p, _p, _i64, _i32,  # partials, counters, capacity, row stride
        _i32, _i32, _i32, _i32,  # batch, query heads, kv heads, head dim
        _i32, _i32, _i32,  # num blocks, block size, table width
        _i32, _i32, _f32, _i32, _i32, _p,  # split size, splits, scale, dtype, flags, stream
    ),
    "tf_paged_gqa_decode_noalloc": (
        _p, _p, _p, _p, _p, _p,  # query, key/value cache, tables, lengths, output
        _i32, _i32, _i32, _i32,  # batch, query heads, kv heads, head dim
        _i32, _i32, _i32,  # num blocks, block size, table width
        _i32, _i32, _f32, _i32, _i32, _p,  # split size, splits, scale, dtype, flags, stream
    ),
    "tf_paged_gqa_decode_rope_append": (
        _p, _i64, _p, _p, _p, _i32,  # qkv, row stride, positions, cos, sin, table rows
        _p, _p, _p, _p, _p,  # key/value cache, append pages, offsets, active mask
        _p, _p, _p,  # tables, lengths, output
        _p, _p, _p, _p, _i64, _i32,  # partials, counters, capacity, row stride
        _i32, _i32, _i32, _i32,  # batch, query heads, kv heads, head dim
        _i32, _i32, _i32,  # num blocks, block size, table width
        _i32, _i32, _f32, _i32, _i32, _p,  # split size, splits, scale, dtype, flags, stream
    ),
    "tf_paged_gqa_decode_partials": (
        _p, _p, _p, _p, _p,
        _p, _p, _p, _i64, _i32,
        _i32, _i32, _i32, _i32,
        _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _p,
    ),
    "tf_paged_gqa_decode_merge": (
        _p, _p, _p, _p, _p, _i64, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p,
    ),
    "tf_paged_kv_write_token": (
        _p, _p, _p, _p, _p, _p, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _p,
    ),
    "tf_paged_kv_write_slots": (
        _p, _p, _p, _p, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _p,
    ),
    "tf_paged_kv_write_range": (
        _p, _p, _p, _p, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p,
    ),
    "tf_rope_kv_append": (
        _p, _i64, _p, _p, _p, _i32,  # qkv, row stride, positions, cos, sin, table rows
        _p, _p, _p, _p, _p, _p, _p,  # query/key out, key/value cache, pages, offsets, active
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p,  # batch .. block size, dtype, stream
    ),
    "tf_rms_norm": (_p, _p, _p, _i64, _i32, _f32, _i32, _p),
    "tf_embedding_rms_norm": (_p, _i64, _p, _p, _p, _i64, _p, _p, _p, _i64, _i32, _f32, _i32,
                              _p),
    "tf_residual_rms_norm": (_p, _p, _p, _p, _p, _i64, _i32, _f32, _i32, _p),
    "tf_residual_rms_norm_partials": (_p, _i32, _p, _p, _p, _p, _i64, _i32, _f32, _i32, _p),
    "tf_swiglu": (_p, _p, _p, _i64, _i32, _p),
    "tf_swiglu_rows": (_p, _i64, _p, _i64, _i64, _i32, _i32, _p),
    "tf_argmax_rows": (_p, _i64, _i32, _i32, _i32, _p, _p),
    "tf_linear_rows": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    "tf_linear_partials": (_p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p),
    "tf_linear_partials_sum": (_p, _i32, _i32, _i32, _p, _i64, _i32, _p),
    "tf_linear_stream": (_p, _i64, _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p),
    "tf_linear_swiglu": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p),
    "tf_linear_kstream": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p),
    "tf_linear_kswiglu": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p),
    "tf_linear_kstream_norm": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _f32, _i32, _p),
    "tf_linear_kswiglu_norm": (_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _f32, _i32, _p),
    "tf_linear_kstream_residual": (_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32,
                                   _i32, _p),
    "tf_prefill_attention": (_p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32,
                             _f32, _i32, _i32, _p),
}

_LIBRARY: ctypes.CDLL | None = None
_LOAD_ERROR: str | None = None


def _load() -> ctypes.CDLL:
    global _LIBRARY, _LOAD_ERROR
    if _LIBRARY is not None:
        return _LIBRARY
    if not LIBRARY_PATH.exists():
        _LOAD_ERROR = (
            f"{LIBRARY_PATH} is missing; build it with `python -m tensorforge_amd.build`"
        )
        raise RuntimeError(_LOAD_ERROR)
    try:
        library = ctypes.CDLL(str(LIBRARY_PATH))
    except OSError as error:
        _LOAD_ERROR = f"cannot load {LIBRARY_PATH}: {error}"
        raise RuntimeError(_LOAD_ERROR) from error
    for name, argtypes in SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = list(argtypes)
        function.restype = ctypes.c_char_p if name == "tf_last_error" else _i32
    _LIBRARY = library
    return library


def library() -> ctypes.CDLL:
    """Return the loaded library, raising ``RuntimeError`` when unavailable."""

    return _load()


def is_available() -> bool:
    """True when the gfx950 library is built and loadable in this process."""

    try:
        _load()
    except RuntimeError:
        return False
    return True


def check(status: int, operation: str) -> None:
    """Map a nonzero ``tf_status`` to ``RuntimeError`` with the library message."""

    if status != 0:
        message = library().tf_last_error().decode(errors="replace")
        raise RuntimeError(f"{operation} failed (status {status}): {message}")


def current_stream(device: torch.device) -> int:
    """HIP stream handle of torch's current stream on ``device``."""

    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    return DTYPE_CODES[dtype]
