"""ctypes binding of ``libopaque_dp.so`` (declared in ``include/opaque_dp.h``).

The library must be built (``python -m opaque_amd.build``); there is no
fallback implementation, so a missing library raises immediately.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libopaque_dp.so"

ODP_OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_HIP = 3
DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F64 = 3
CLIP_FIXED = 0
CLIP_AUTOS = 1

# Problem-table field layouts (must match include/opaque_dp.h).
PF_SRC, PF_LD0, PF_LD1, PF_DTYPES, PF_DIN, PF_R, PF_DST = range(7)
PF_FIELDS = 8
PL_FIELDS = 12
PL_SRC, PL_LDS, PL_R, PL_DST, PL_LDQ, PL_NROWS, PL_SEG_FIRST, PL_NSEG, PL_DTYPE = range(9)
PJ_FIELDS = 12
PJ_P, PJ_LDP, PJ_D, PJ_W, PJ_R, PJ_Q, PJ_LDQ, PJ_NROWS, PJ_SEG_FIRST, PJ_NSEG = range(10)
FT_FIELDS = 24
FT_P, FT_LDP, FT_M, FT_Q, FT_LDQ, FT_R, FT_SEG_FIRST, FT_NSEG, FT_SCALING, FT_NLEAF = range(10)
FT_LEAF0 = 10
FT_WAVE_SLOTS = 4  # partial slots per LoRA leaf and M-tile
FP_W, FP_U = 13, 14
FT_GROUPS = 23
SS_FIELDS = 8
SS_PE, SS_M, SS_RANK, SS_SEG_FIRST, SS_NSEG, SS_OUT, SS_FLAGS, SS_OUT2 = range(8)
NZ_FIELDS = 8
NZ_IN, NZ_OUT, NZ_N, NZ_FLAT_OFFSET, NZ_SIGMA, NZ_DTYPES = range(6)
SQ_FIELDS = 8
SQ_X, SQ_N, SQ_NSEG, SQ_SEG_FIRST, SQ_SLOT, SQ_DTYPE = range(6)
LN_FIELDS = 24
LN_X, LN_LDX, LN_G, LN_LDG, LN_DIN, LN_DOUT, LN_SEG_FIRST, LN_NSEG, LN_SLOT, LN_OUT, LN_FLAGS, LN_NB, LN_NROWS, LN_PE = range(14)
LN_XMASK, LN_GMASK, LN_NFFLAG, LN_SCRATCH, LN_OUT2, LN_XAMAX, LN_GAMAX = 14, 15, 16, 17, 18, 19, 20
NF_FIELDS = 8
NF_P, NF_LDP, NF_D, NF_SEG_FIRST, NF_NSEG, NF_MASK, NF_AMAX = range(7)
FORM_OUTER = 0
FORM_GRAM = 1
FORM_GRAM256 = 2
FORM_OUTER_GUARDED = 3

_c_int = ctypes.c_int
_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_u32 = ctypes.c_uint32
_c_u64 = ctypes.c_uint64
_c_f32 = ctypes.c_float
_c_f64 = ctypes.c_double
_ptr = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "odp_abi_version": (_c_int, []),
    "odp_last_error": (ctypes.c_char_p, []),
    "odp_pack_factors_blocks": (_c_i64, [_c_i64]),
    "odp_pack_factors": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32]),
    "odp_project_blocks": (_c_i64, [_c_int, _c_i64, _c_i32]),
    "odp_project_covered_rows": (_c_i64, [_ptr, _ptr, _c_i32]),
    "odp_project": (_c_int, [_ptr, _c_int, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _c_i32]),
    "odp_seg_factor_tiles": (_c_i64, [_c_int, _c_i64, _c_i32]),
    "odp_seg_factor": (
        _c_int,
        [_ptr, _c_int, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i64, _c_i32],
    ),
    "odp_factor_project_max_len": (_c_i64, []),
    "odp_seg_factor_project": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i64]),
    "odp_seg_factor_stream_groups": (_c_i64, [_c_i64]),
    "odp_seg_factor_stream": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i64, _c_i32]),
    "odp_sqnorm_blocks": (_c_i64, [_c_i64]),
    "odp_sqnorm": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _c_i64]),
    "odp_clip_factors": (
        _c_int,
        [
            _ptr, _ptr, _c_i64, _c_i32, _ptr, _c_i32, _ptr, _c_f64, _c_i32, _c_f64,
            _c_i32, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
        ],
    ),
    "odp_noalloc_max_partials": (_c_i64, []),
    "odp_clip_materialized_noalloc": (
        _c_int,
        [
            _ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _c_i64, _c_i32, _ptr, _c_i32, _ptr, _c_f64, _c_i32, _c_f64,
            _c_i32, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
        ],
    ),
    "odp_scale_sum_blocks": (_c_i64, [_c_i64]),
    "odp_scale_sum": (
        _c_int,
        [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _c_i32, _c_i32, _c_f32],
    ),
    "odp_gaussian_noise_blocks": (_c_i64, [_c_i64, _c_i64]),
    "odp_gaussian_noise": (
        _c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _c_u64, _c_u32, _c_i32, _c_i32, _c_f64, _c_f64]),
    "odp_philox_words": (_c_int, [_ptr, _c_u64, _c_u32, _c_u32, _c_u64, _c_i64, _ptr]),
    "odp_noise_icdf": (_c_int, [_ptr, _c_u32, _c_i64, _ptr]),
    "odp_calibrate_mfma": (_c_int, [_ptr, _c_i32, _c_i32, _ptr]),
    "odp_calibrate_mfma_flops": (_c_i64, [_c_i32, _c_i32]),
    "odp_linear_tiles": (_c_i64, [_c_int, _c_i64, _c_i64, _c_i64]),
    "odp_linear_prescale_blocks": (_c_i64, [_c_i64]),
    "odp_linear_prescale": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i32, _c_i32]),
    "odp_linear_norm_blocks": (_c_i64, [_c_int, _c_i64, _c_i64, _c_i64, _c_i64]),
    "odp_linear_sqnorm": (_c_int, [_ptr, _c_int, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i64]),
    "odp_linear_sum_blocks": (_c_i64, [_c_i64, _c_i64]),
    "odp_nonfinite_blocks": (_c_i64, [_c_i64, _c_i64]),
    "odp_nonfinite_columns": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr]),
    "odp_linear_clipped_sum": (
        _c_int,
        [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i32, _c_i32, _c_f32, _c_i32],
    ),
    "odp_pack_planes_blocks": (_c_i64, [_c_i64]),
    "odp_pack_planes": (_c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr]),
    "odp_linear_moments_blocks": (_c_i64, [_c_i64, _c_i64, _c_i32]),
    "odp_linear_moments": (
        _c_int, [_ptr, _ptr, _ptr, _c_i32, _c_i32, _ptr, _ptr, _ptr, _ptr, _c_i32, _c_i32, _c_f32, _c_i32]),
}

_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load the native library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    # OPAQUE_AMD_LIBRARY names another build of the same library (the
    # sanitizer test loads the instrumented one this way).
    p = Path(path) if path is not None else Path(os.environ.get("OPAQUE_AMD_LIBRARY") or LIB_PATH)
    if not p.exists():
        raise RuntimeError(
            f"opaque_amd native library not found at {p}. Build it with "
            "`python -m opaque_amd.build` (hipcc, gfx950); there is no fallback path."
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load().odp_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    if rc != ODP_OK:
        raise RuntimeError(f"{what} failed with status {rc}: {last_error()}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
