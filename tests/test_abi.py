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
    assert lib.odp_abi_version() == 1
    assert isinstance(N.last_error(), str)


def test_field_indices_match_header():
    text = HEADER.read_text()

    def value(name: str) -> int:
        m = re.search(rf"\b{name}\s*=\s*(\d+)", text)
        assert m, name
        return int(m.group(1))

    assert value("ODP_PJ_FIELDS") == N.PJ_FIELDS
    assert value("ODP_PJ_QLO") == N.PJ_QLO
    assert value("ODP_FT_FIELDS") == N.FT_FIELDS
    assert value("ODP_FT_LEAF0") == N.FT_LEAF0
    assert value("ODP_FT_QLO") == N.FT_QLO
    assert value("ODP_FT_WAVE_SLOTS") == N.FT_WAVE_SLOTS
    assert value("ODP_SS_FIELDS") == N.SS_FIELDS
    assert value("ODP_SQ_FIELDS") == N.SQ_FIELDS
    assert value("ODP_NZ_FIELDS") == N.NZ_FIELDS
    assert value("ODP_CLIP_AUTOS") == N.CLIP_AUTOS
    assert value("ODP_DTYPE_BF16") == N.DTYPE_BF16


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
