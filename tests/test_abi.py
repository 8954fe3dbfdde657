"""The C-ABI library loads and exports every entry point include/opaque_dp.h declares.

No compute call is made (this runs without a GPU).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from opaque_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "opaque_dp.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(odp_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        from opaque_amd import build

        build.build()
    return N.load()


def test_header_declares_the_bound_functions():
    declared = _declared()
    assert declared, "no declarations parsed"
    assert declared == set(N.exported_symbols())


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_abi_version_and_error_buffer(lib):
    assert lib.odp_abi_version() == 3
    assert isinstance(N.last_error(), str)


def test_field_indices_match_header():
    text = HEADER.read_text()

    def value(name: str) -> int:
        m = re.search(rf"\b{name}\s*=\s*(\d+)", text)
        assert m, name
        return int(m.group(1))

    assert value("ODP_PF_FIELDS") == N.PF_FIELDS
    assert value("ODP_PF_DST") == N.PF_DST
    assert value("ODP_PJ_FIELDS") == N.PJ_FIELDS
    assert value("ODP_FT_FIELDS") == N.FT_FIELDS
    assert value("ODP_FT_LEAF0") == N.FT_LEAF0
    assert value("ODP_FT_WAVE_SLOTS") == N.FT_WAVE_SLOTS
    assert value("ODP_SS_FIELDS") == N.SS_FIELDS
    assert value("ODP_SQ_FIELDS") == N.SQ_FIELDS
    assert value("ODP_NZ_FIELDS") == N.NZ_FIELDS
    assert value("ODP_LN_FIELDS") == N.LN_FIELDS
    assert value("ODP_LN_PE") == N.LN_PE
    assert value("ODP_LN_XMASK") == N.LN_XMASK
    assert value("ODP_LN_GMASK") == N.LN_GMASK
    assert value("ODP_LN_NFFLAG") == N.LN_NFFLAG
    assert value("ODP_LN_SCRATCH") == N.LN_SCRATCH
    assert value("ODP_FORM_GRAM") == N.FORM_GRAM
    assert value("ODP_FORM_GRAM256") == N.FORM_GRAM256
    assert value("ODP_NF_FIELDS") == N.NF_FIELDS
    assert value("ODP_NF_MASK") == N.NF_MASK
    assert value("ODP_CLIP_AUTOS") == N.CLIP_AUTOS
    assert value("ODP_DTYPE_BF16") == N.DTYPE_BF16
    assert value("ODP_FP_W") == N.FP_W and value("ODP_FP_U") == N.FP_U
    assert value("ODP_FT_GROUPS") == N.FT_GROUPS
    assert value("ODP_FT_GROUPS") >= N.FT_LEAF0 + 3 * 4 and value("ODP_FT_GROUPS") < N.FT_FIELDS  # past 4 leaves
    assert value("ODP_LN_OUT2") == N.LN_OUT2
    assert value("ODP_LN_XAMAX") == N.LN_XAMAX and value("ODP_LN_GAMAX") == N.LN_GAMAX
    assert value("ODP_NF_AMAX") == N.NF_AMAX
    assert value("ODP_FORM_OUTER_GUARDED") == N.FORM_OUTER_GUARDED
    assert value("ODP_PL_FIELDS") == N.PL_FIELDS and value("ODP_PL_DTYPE") == N.PL_DTYPE


def test_block_helpers_are_pure_host_code(lib):
    # The *_blocks helpers compute launch sizes on the host (no device needed).
    assert lib.odp_project_blocks(N.DTYPE_F32, 0, 16) == 0
    assert lib.odp_project_blocks(N.DTYPE_F32, 64, 16) == 1
    assert lib.odp_project_blocks(N.DTYPE_F32, 65, 16) == 2
    for r in (16, 48):
        per = (1 << 20) // lib.odp_project_blocks(N.DTYPE_BF16, 1 << 20, r)  # rows per workgroup
        assert per >= 64 and lib.odp_project_blocks(N.DTYPE_BF16, per + 1, r) == 2
    assert lib.odp_sqnorm_blocks(1) >= 1
    assert lib.odp_scale_sum_blocks(4096) >= 1
    assert lib.odp_seg_factor_tiles(N.DTYPE_BF16, 4096, 16) >= 1
    assert lib.odp_nonfinite_blocks(256, 3) == 3
    assert lib.odp_nonfinite_blocks(264, 2) == 4
    assert lib.odp_nonfinite_blocks(0, 2) == 0
    assert lib.odp_pack_factors_blocks(0) == 0
    assert lib.odp_pack_factors_blocks(256) == 1 and lib.odp_pack_factors_blocks(257) == 2
    assert lib.odp_seg_factor_stream_groups(0) == 0
    assert lib.odp_seg_factor_stream_groups(256) == 1
    tiles = lib.odp_seg_factor_tiles(N.DTYPE_BF16, 14336, 16)
    assert 1 < lib.odp_seg_factor_stream_groups(14336) <= tiles


def test_linear_norm_slots_per_form(lib):
    """Partial slots per segment: 256 x 256 output tiles (outer), pairs
    t <= s of 128-row blocks taken two s blocks at a time (Gram), pairs of
    256-row blocks (Gram256: nb (nb + 1) / 2); the norm launches pad the
    segment count to a multiple of 8 (work decoded in XCD order)."""
    assert lib.odp_linear_tiles(N.FORM_OUTER, 4096, 14336, 4096) == 16 * 56
    for L, nb in ((1, 1), (256, 1), (257, 2), (4096, 16), (4100, 17)):
        assert lib.odp_linear_tiles(N.FORM_GRAM256, 4096, 14336, L) == nb * (nb + 1) // 2
    assert lib.odp_linear_tiles(N.FORM_GRAM, 4096, 14336, 4096) == 16 * 17  # 32 blocks
    assert lib.odp_linear_tiles(N.FORM_GRAM256, 4096, 14336, 0) == 0
    assert lib.odp_linear_norm_blocks(N.FORM_GRAM256, 4096, 14336, 4096, 9) == 16 * 136
    assert lib.odp_linear_norm_blocks(N.FORM_GRAM256, 4096, 14336, 4096, 3) == (3 * 136 + 7) // 8 * 8


# ---------------------------------------------------------------------------
# The error contract: invalid arguments return a status code and set the
# thread's error text before any device work (so these run without a GPU).
# ---------------------------------------------------------------------------

_BAD = ctypes.c_void_p(16)  # a non-null address; never dereferenced on these paths


def _err(lib, rc, code, fragment):
    assert rc == code, (rc, N.last_error())
    assert fragment in N.last_error(), N.last_error()


def test_table_checks(lib):
    _err(lib, lib.odp_gaussian_noise(None, None, None, -1, 0, 0, 0, 0, 0, 0.0, 0.0), N.ERR_INVALID_ARGUMENT,
         "negative n_prob")
    _err(lib, lib.odp_gaussian_noise(None, None, None, 0, 0, 0, 0, N.DTYPE_BF16, 0, 0.0, 0.0), N.ERR_UNSUPPORTED,
         "compute_dtype 1")
    _err(lib, lib.odp_gaussian_noise(None, None, None, 0, 0, 0, 0, N.DTYPE_F32, 1, 0.5, 2.0),
         N.ERR_INVALID_ARGUMENT, "low <= 0 <= high")
    _err(lib, lib.odp_noise_icdf(None, 0, (1 << 24) + 1, _BAD), N.ERR_INVALID_ARGUMENT, "n <= 2^24")
    _err(lib, lib.odp_sqnorm(None, None, None, 2, 4, None, None, 1), N.ERR_INVALID_ARGUMENT,
         "null problem table")
    _err(lib, lib.odp_scale_sum(None, None, None, 0, 3, None, None, 1, 1, 1.0), N.ERR_INVALID_ARGUMENT,
         "total_blocks must be 0")
    _err(lib, lib.odp_nonfinite_columns(None, _BAD, _BAD, 1, 1, None, None), N.ERR_INVALID_ARGUMENT,
         "null segment arrays")


def test_kernel_argument_checks(lib):
    _err(lib, lib.odp_project(None, 7, None, None, 0, 0, None, None, 1), N.ERR_UNSUPPORTED, "unsupported dtype")
    _err(lib, lib.odp_project(None, N.DTYPE_BF16, None, None, 0, 0, None, None, 5), N.ERR_UNSUPPORTED, "nkb=5")
    _err(lib, lib.odp_seg_factor(None, N.DTYPE_F32, None, None, 0, 0, None, None, None, None, 1, 0),
         N.ERR_UNSUPPORTED, "nkb=0")
    _err(lib, lib.odp_seg_factor_project(None, _BAD, _BAD, 1, 1, None, None, None, None, 1),
         N.ERR_INVALID_ARGUMENT, "null segment")
    _err(lib, lib.odp_seg_factor_stream(None, _BAD, _BAD, 1, 1, None, None, None, None, 1, 1),
         N.ERR_INVALID_ARGUMENT, "null segment")
    _err(lib, lib.odp_seg_factor_stream(None, _BAD, _BAD, 1, 1, _BAD, _BAD, _BAD, _BAD, 1, 4),
         N.ERR_UNSUPPORTED, "nkb=4")
    _err(lib, lib.odp_pack_planes(None, _BAD, _BAD, 1, 1, None, None), N.ERR_INVALID_ARGUMENT, "null segment")
    _err(lib, lib.odp_linear_sqnorm(None, 9, None, None, 0, 0, None, None, None, None, 1),
         N.ERR_INVALID_ARGUMENT, "unknown form 9")
    _err(lib, lib.odp_scale_sum(None, None, None, 0, 0, None, None, 1, 1, 0.0), N.ERR_INVALID_ARGUMENT,
         "normalize_by must be > 0")
    _err(lib, lib.odp_linear_clipped_sum(None, None, None, 0, 0, None, None, None, None, 1, 1, -1.0, 0),
         N.ERR_INVALID_ARGUMENT, "normalize_by must be > 0")
    _err(lib, lib.odp_philox_words(None, 0, 0, 0, 0, -1, None), N.ERR_INVALID_ARGUMENT, "bad n")
    _err(lib, lib.odp_calibrate_mfma(None, 0, 1, _BAD), N.ERR_INVALID_ARGUMENT, "workgroups (0)")
    _err(lib, lib.odp_calibrate_mfma(None, 1, 1 << 25, _BAD), N.ERR_INVALID_ARGUMENT, "iters")
    _err(lib, lib.odp_calibrate_mfma(None, 1, 1, None), N.ERR_INVALID_ARGUMENT, "null sink")


def test_project_covered_rows(lib):
    import numpy as np

    from opaque_amd.engine import Segments, _SegView

    starts = np.asarray([3, 253, 266, 270, 1024], dtype=np.int32)
    lens = np.asarray([250, 13, 0, 601, 8], dtype=np.int32)
    # [0, 256) + [248, 272) + nothing + [264, 872) + [1024, 1032): 8-row groups, overlaps counted twice.
    want = 256 + 24 + 608 + 8
    got = lib.odp_project_covered_rows(starts.ctypes.data, lens.ctypes.data, len(starts))
    assert got == want
    view = _SegView(Segments(starts.tolist(), lens.tolist(), list(range(5)), 5, 1100), 0)
    assert view.covered == want
    assert lib.odp_project_covered_rows(None, None, 0) == 0
    assert lib.odp_project_covered_rows(None, None, 2) == -1
    assert "null segment arrays" in N.last_error()


def test_calibration_flops(lib):
    # 4 waves x 16 chains x one 16x16x32 MFMA (16384 flops) per round.
    assert lib.odp_calibrate_mfma_flops(1, 1) == 4 * 16 * 16384
    assert lib.odp_calibrate_mfma_flops(512, 1000) == 512 * 1000 * 4 * 16 * 16384


def test_clip_factor_argument_checks(lib):
    def call(n_ex=1, n_groups=1, n_cls=1, mode=N.CLIP_FIXED, gamma=0.0):
        return lib.odp_clip_factors(None, None, 1, n_ex, None, n_groups, None, 1.0, mode, gamma, n_cls,
                                    None, None, None, None, None, None, None)

    _err(lib, call(n_groups=0), N.ERR_UNSUPPORTED, "n_groups=0")
    _err(lib, call(n_cls=9), N.ERR_UNSUPPORTED, "n_cls=9")
    _err(lib, call(mode=3), N.ERR_INVALID_ARGUMENT, "unknown mode 3")
    _err(lib, call(mode=N.CLIP_AUTOS, gamma=0.0), N.ERR_INVALID_ARGUMENT, "gamma must be positive")
    _err(lib, call(n_ex=-1), N.ERR_INVALID_ARGUMENT, "negative n_ex")
    _err(lib, call(), N.ERR_INVALID_ARGUMENT, "null required pointer")
    assert call(n_ex=0) == N.ODP_OK  # an empty batch launches nothing



def test_clip_argument_checks(lib):
    """odp_clip_factors: groups, classes, mode, gamma and required pointers;
    N.check turns a status into an exception carrying the message."""
    args = [None, None, 4, 2, None, 0, None, 1.0, N.CLIP_FIXED, 0.0, 1, None, None, None, None, None, None, None]
    _err(lib, lib.odp_clip_factors(*args), N.ERR_UNSUPPORTED, "n_groups=0")
    args[5], args[10] = 1, 9
    _err(lib, lib.odp_clip_factors(*args), N.ERR_UNSUPPORTED, "n_cls=9")
    args[10], args[8] = 1, 7
    _err(lib, lib.odp_clip_factors(*args), N.ERR_INVALID_ARGUMENT, "unknown mode 7")
    args[8] = N.CLIP_AUTOS
    _err(lib, lib.odp_clip_factors(*args), N.ERR_INVALID_ARGUMENT, "gamma must be positive")
    args[9] = 0.01
    _err(lib, lib.odp_clip_factors(*args), N.ERR_INVALID_ARGUMENT, "null")
    with pytest.raises(RuntimeError, match="odp_noise_icdf failed with status 1"):
        N.check(lib.odp_noise_icdf(None, 0, (1 << 24) + 1, None), "odp_noise_icdf")
