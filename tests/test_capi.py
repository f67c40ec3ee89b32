"""The C ABI library loads, exports every entry point include/bmx.h declares, and rejects bad arguments on the host
(no GPU work is launched by these calls)."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "bmx.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bmx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("bmx_exl3_dequant", "bmx_router_topk", "bmx_dispatch", "bmx_moe_forward", "bmx_moe_experts",
                 "bmx_combine", "bmx_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import bmx
    L = bmx.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    # and the ctypes signatures cover them all
    assert set(declared_functions()) <= set(bmx._lib.SIGNATURES)


def test_host_side_checks():
    import bmx
    L = bmx.lib()
    assert L.bmx_abi_version() == 6
    assert [L.bmx_tile_bytes(f) for f in range(4)] == [64, 80, 96, 128] and L.bmx_tile_bytes(9) == -1
    assert L.bmx_exl3_dequant(None, 7, 16, 16, None, None) == bmx._lib.BMX_ERR_ARG
    assert b"format" in L.bmx_last_error()
    assert L.bmx_exl3_dequant(None, 2, 15, 16, None, None) == bmx._lib.BMX_ERR_ARG
    assert L.bmx_router_topk(None, None, 1, 2000, 8, 1, 1, 1, 1, 1.0, 0, None, None, None) == bmx._lib.BMX_ERR_ARG
    assert L.bmx_router_topk(None, None, 1, 64, 8, 3, 1, 1, 1, 1.0, 0, None, None, None) == bmx._lib.BMX_ERR_ARG
    d = bmx._lib.MoeDesc(4096, 1000, 8, 2, 0, 0, 1, 0.0, None, None)
    assert L.bmx_moe_forward(ctypes.byref(d), None, 1, None, None, None, None, 0, 0, None) == bmx._lib.BMX_ERR_ARG
    assert b"multiples of 128" in L.bmx_last_error()
    assert L.bmx_rows_per_group(1, 8, 0) == 1 and L.bmx_rows_per_group(3, 8, 0) == 4 and L.bmx_rows_per_group(60, 8, 0) == 32
    assert L.bmx_rows_per_group(256, 8, 0) == 128 and L.bmx_rows_per_group(64, 8, 0) == 32 and L.bmx_rows_per_group(64, 8, 1) == 8 and L.bmx_rows_per_group(1, 8, 2) == 128
    assert L.bmx_resolve_path(255, 8, 0) == 3 and L.bmx_resolve_path(256, 8, 0) == 2 and L.bmx_resolve_path(1, 8, 2) == 2
    # AUTO below the prefill rows: the mid-size path from 8 tokens, the GEMV path below; explicit paths kept
    assert L.bmx_resolve_path(15, 8, 0) == 3 and L.bmx_resolve_path(8, 8, 0) == 3 and L.bmx_resolve_path(16, 6, 0) == 3
    assert L.bmx_resolve_path(7, 8, 0) == 1 and L.bmx_resolve_path(1, 8, 0) == 1 and L.bmx_resolve_path(85, 6, 0) == 3
    assert L.bmx_resolve_path(16, 6, 1) == 1 and L.bmx_resolve_path(2, 6, 4) == 4 and L.bmx_resolve_path(2, 6, 5) == -1
    assert L.bmx_resolve_path(1, 8, 7) == -1 and L.bmx_rows_per_group(1, 0, 0) == -1


def test_workspace_queries():
    import bmx
    L = bmx.lib()
    d = bmx._lib.MoeDesc(4096, 1536, 288, 8, 0, 0, 1, 0.0, ctypes.c_void_p(1), ctypes.c_void_p(2))
    n1 = L.bmx_moe_workspace(ctypes.byref(d), 1, 0)
    n8 = L.bmx_moe_workspace(ctypes.byref(d), 8, 0)
    assert 0 < n1 < n8
    assert L.bmx_groups_max(1, 8, 288, 1, 1) >= 9


def test_geometry_known_answers():
    """Slot geometry of the reference: tests/test_store.py:50-51 (3 x 4096 B trellis -> off_u 4096, off_d 8192,
    slot 12288), GLM-5.3 (tests/test_engine.py:50-60: slot 9437184, off_u 3145728, off_d 6291456) and DeepSeek-V4.1
    v2 layers (tests/test_engine.py:63-70: 11059200 / 3686400 / 7372800 at K 2.5, off_u 2949120 at K 2)."""
    from bmx.experts import ExpertTable
    assert ExpertTable.geometry(128, 128, [(0, 0, 0)]) == (4096, 8192, 12288)
    assert ExpertTable.geometry(4096, 2048, [(2, 2, 2)]) == (3145728, 6291456, 9437184)
    assert ExpertTable.geometry(5120, 2304, [(1, 1, 1)]) == (3686400, 7372800, 11059200)
    assert ExpertTable.geometry(5120, 2304, [(0, 0, 0)])[0] == 2949120


def test_layer_stages_mask_checks():
    """bmx_moe_layer_stages refuses a mask outside route / prep / gate-up / act / down / combine (before any device
    work, so on the host), and a zero-token call with a valid mask does nothing."""
    import bmx
    B = bmx._lib
    L = bmx.lib()
    d = B.MoeDesc(4096, 1536, 288, 8, 0, 0, 1, 0.0, ctypes.c_void_p(1), ctypes.c_void_p(2))
    r = B.RouterDesc()
    for m in (0, 1 << B.STAGE_DOWN_OUT, 1 << B.STAGE_GATE_UP_STAGED, 1 << 9):
        assert L.bmx_moe_layer_stages(ctypes.byref(d), ctypes.byref(r), None, None, 0, None, None, None, None, 0, 0, m,
                                      None) == B.BMX_ERR_ARG
        assert b"stage mask" in L.bmx_last_error()
    ok = (1 << B.STAGE_ROUTE) | (1 << B.STAGE_GATE_UP)
    assert L.bmx_moe_layer_stages(ctypes.byref(d), ctypes.byref(r), None, None, 0, None, None, None, None, 0, 0, ok,
                                  None) == 0


def test_moe_stage_checks():
    """bmx_moe_stage refuses unknown stages (and BMX_STAGE_ROUTE, which only bmx_moe_layer_stages runs) and the split
    gate / up and down stages without desc->fresh, before any device work; a zero-token call of a known stage does
    nothing."""
    import bmx
    B = bmx._lib
    L = bmx.lib()
    d = B.MoeDesc(4096, 1536, 288, 8, 0, 0, 1, 0.0, ctypes.c_void_p(1), ctypes.c_void_p(2))
    args = (None, 0, None, None, None, None, None, None, 0, 1, None)
    for st in (-1, B.STAGE_ROUTE, B.STAGE_DOWN_STAGED + 1):
        assert L.bmx_moe_stage(ctypes.byref(d), st, *args) == B.BMX_ERR_ARG
        assert b"unknown stage" in L.bmx_last_error()
    for st in (B.STAGE_GATE_UP_RESIDENT, B.STAGE_GATE_UP_STAGED, B.STAGE_DOWN_RESIDENT, B.STAGE_DOWN_STAGED):
        assert L.bmx_moe_stage(ctypes.byref(d), st, *args) == B.BMX_ERR_ARG
        assert b"desc->fresh" in L.bmx_last_error()
    d.fresh = ctypes.c_void_p(3)
    for st in (B.STAGE_GATE_UP, B.STAGE_DOWN, B.STAGE_DOWN_RESIDENT, B.STAGE_DOWN_STAGED, B.STAGE_COMBINE):
        assert L.bmx_moe_stage(ctypes.byref(d), st, *args) == 0


def test_route_slot_step_checks():
    """bmx_route_slot_step refuses, on the host and before any launch: a table that fails the step's checks, a bad
    layer, a router over another expert count than the table's, and the router's own unsupported sizes."""
    import bmx
    B = bmx._lib
    L = bmx.lib()
    dummy = [ctypes.c_void_p(16 * (i + 1)) for i in range(13)]
    t = B.SlotTable(2, 40, 8, 4, 256, 128, 49152, 16384, 32768, *dummy)
    lg, sel, w = ctypes.c_void_p(16), ctypes.c_void_p(32), ctypes.c_void_p(48)
    seq = ctypes.c_int64()

    def call(tab, li=0, E=40, topk=8, n_group=1, topk_group=1):
        return L.bmx_route_slot_step(ctypes.byref(tab), None, li, lg, None, E, topk, n_group, topk_group,
                                     bmx.SCORE_SIGMOID, 1, 1.0, 0, 1, sel, w, ctypes.byref(seq), None)

    bad = B.SlotTable(2, 40, 8, 4, 256, 128, 49152, 16384, 32768, *([None] * 13))
    assert call(bad) == B.BMX_ERR_ARG and b"null table array" in L.bmx_last_error()
    assert call(t, li=2) == B.BMX_ERR_ARG and b"bad layer" in L.bmx_last_error()
    assert call(t, E=48) == B.BMX_ERR_ARG and b"not the table's" in L.bmx_last_error()
    assert call(t, topk=41) == B.BMX_ERR_ARG and b"unsupported sizes" in L.bmx_last_error()
    assert call(t, n_group=3) == B.BMX_ERR_ARG and b"bad groups" in L.bmx_last_error()
