"""ctypes binding of libbmx.so (include/bmx.h). The library is required: nothing here has a fallback."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbmx.so")

BMX_OK, BMX_ERR_ARG, BMX_ERR_HIP, BMX_ERR_WORKSPACE, BMX_ERR_UNSUPPORTED = 0, 1, 2, 3, 4
TF_K2, TF_K25, TF_K3, TF_K4 = 0, 1, 2, 3
TILE_BYTES = {TF_K2: 64, TF_K25: 80, TF_K3: 96, TF_K4: 128}
SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSP = 0, 1, 2
ACT_SILU, ACT_GELU, ACT_RELU2, ACT_SILU_OAI = 0, 1, 2, 3
PATH_AUTO, PATH_DECODE, PATH_PREFILL, PATH_MID, PATH_SPLIT = 0, 1, 2, 3, 4
STAGE_GATE_UP, STAGE_ACT, STAGE_DOWN, STAGE_COMBINE, STAGE_DOWN_OUT, STAGE_PREP = 0, 1, 2, 3, 4, 5
STAGE_GATE_UP_RESIDENT, STAGE_GATE_UP_STAGED = 6, 7
STAGE_ROUTE = 8
STAGE_DOWN_RESIDENT, STAGE_DOWN_STAGED = 9, 10
LANE_VRAM, LANE_ADMIT, LANE_HOME, LANE_CPU = 0, 1, 2, 3
PLAN_MAXP, PLAN_MAXT = 64, 8

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_I64 = ctypes.c_int64


class Expert(ctypes.Structure):
    _fields_ = [("tr", ctypes.c_uint64 * 3), ("suh", ctypes.c_uint64 * 3), ("svh", ctypes.c_uint64 * 3),
                ("fmt", ctypes.c_int32 * 3), ("reserved", ctypes.c_int32)]


class MoeDesc(ctypes.Structure):
    _fields_ = [("H", ctypes.c_int32), ("I", ctypes.c_int32), ("E", ctypes.c_int32), ("topk", ctypes.c_int32),
                ("first", ctypes.c_int64), ("act", ctypes.c_int32), ("gated", ctypes.c_int32),
                ("act_limit", ctypes.c_float), ("experts", _P), ("shared", _P), ("fresh", _P), ("shared_gate", _P)]


class SlotTable(ctypes.Structure):
    _fields_ = [("L", ctypes.c_int32), ("E", ctypes.c_int32), ("S", ctypes.c_int32), ("maxj", ctypes.c_int32),
                ("H", ctypes.c_int32), ("I", ctypes.c_int32),
                ("rec", ctypes.c_int64), ("off_u", ctypes.c_int64), ("off_d", ctypes.c_int64)] + \
               [(n, _P) for n in ("slotof", "owner", "refb", "pin", "ctl", "jobs", "fresh", "stats", "home", "slot_base",
                                  "tables", "pjobs", "pfl")]


class CpuExpert(ctypes.Structure):
    _fields_ = [("tr", _P * 3), ("suh", _P * 3), ("svh", _P * 3), ("fmt", ctypes.c_int32 * 3), ("reserved", ctypes.c_int32)]


class PlanPolicy(ctypes.Structure):
    _fields_ = [("cpu_on", ctypes.c_int32), ("max_cpu", ctypes.c_int32), ("home_single", ctypes.c_int32),
                ("cpu_fast", ctypes.c_int32), ("cpu_measured", ctypes.c_int32)] + \
               [(n, ctypes.c_double) for n in ("gpu_base_us", "gpu_hit_us", "gpu_home_us", "gpu_admit_us", "cpu_base_us",
                                               "cpu_expert_us", "cpu_token_us")]


class RouterDesc(ctypes.Structure):
    _fields_ = [("score_fn", ctypes.c_int32), ("renorm", ctypes.c_int32), ("n_group", ctypes.c_int32),
                ("topk_group", ctypes.c_int32), ("scale", ctypes.c_float), ("reserved", ctypes.c_int32), ("bias", _P),
                ("weight", _P)]


class Routes(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("counts", "offsets", "row_token", "row_slot", "inv", "uexp", "nuniq", "groups",
                                  "ngroups", "row_expert")]


# name -> (restype, argtypes): every symbol include/bmx.h declares
SIGNATURES = {
    "bmx_last_error": (ctypes.c_char_p, []),
    "bmx_abi_version": (_I, []),
    "bmx_tile_bytes": (_I, [_I]),
    "bmx_exl3_dequant": (_I, [_P, _I, _I, _I, _P, _P]),
    "bmx_router_topk": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, _I64, _P, _P, _P]),
    "bmx_router_logits": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "bmx_groups_max": (_I, [_I, _I, _I, _I, _I]),
    "bmx_dispatch_workspace": (_SZ, [_I, _I, _I]),
    "bmx_dispatch": (_I, [_P, _I, _I, _I, _I64, _I, _I, ctypes.POINTER(Routes), _P, _SZ, _P]),
    "bmx_route_dispatch": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, _I64, _I, _I, _P, _P,
                                ctypes.POINTER(Routes), _P]),
    "bmx_moe_workspace": (_SZ, [ctypes.POINTER(MoeDesc), _I, _I]),
    "bmx_moe_forward": (_I, [ctypes.POINTER(MoeDesc), _P, _I, _P, _P, _P, _P, _SZ, _I, _P]),
    "bmx_rows_per_group": (_I, [_I, _I, _I]),
    "bmx_resolve_path": (_I, [_I, _I, _I]),
    "bmx_experts_workspace": (_SZ, [ctypes.POINTER(MoeDesc), _I, _I]),
    "bmx_moe_experts": (_I, [ctypes.POINTER(MoeDesc), _P, _I, ctypes.POINTER(Routes), _P, _P, _P, _SZ, _I, _P]),
    "bmx_moe_stage": (_I, [ctypes.POINTER(MoeDesc), _I, _P, _I, ctypes.POINTER(Routes), _P, _P, _P, _P, _P, _SZ, _I, _P]),
    "bmx_combine": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "bmx_moe_layer_workspace": (_SZ, [ctypes.POINTER(MoeDesc), _I, _I]),
    "bmx_moe_layer": (_I, [ctypes.POINTER(MoeDesc), ctypes.POINTER(RouterDesc), _P, _P, _I, _P, _P, _P, _P, _SZ, _I, _P]),
    "bmx_moe_layer_stages": (_I, [ctypes.POINTER(MoeDesc), ctypes.POINTER(RouterDesc), _P, _P, _I, _P, _P, _P, _P, _SZ, _I, _I,
                                  _P]),
    "bmx_moe_layer_scratch": (_I, [ctypes.POINTER(MoeDesc), ctypes.POINTER(RouterDesc), _P, _P, _I, _P, _P, _P, _I, _P]),
    "bmx_slot_step": (_I, [ctypes.POINTER(SlotTable), _I, _P, _I, _I64, _I, _P]),
    "bmx_slot_copy": (_I, [ctypes.POINTER(SlotTable), _I, _P]),
    "bmx_slot_copy_mats": (_I, [ctypes.POINTER(SlotTable), _I, _I, _P]),
    "bmx_slot_prefetch": (_I, [ctypes.POINTER(SlotTable), _I, _P, _I, _I64, _I, _I, _P]),
    "bmx_slot_prefetch_copy": (_I, [ctypes.POINTER(SlotTable), _I, _I, _I, _P]),
    "bmx_copy_agent_create": (_I, [ctypes.POINTER(SlotTable), _P, _P, ctypes.POINTER(_P)]),
    "bmx_copy_agent_destroy": (_I, [_P]),
    "bmx_copy_agent_status": (_I, [_P, _P]),
    "bmx_copy_agent_control": (_I, [_P, _I, _I64]),
    "bmx_slot_step_agent": (_I, [ctypes.POINTER(SlotTable), _P, _I, _P, _I, _I64, _I, ctypes.POINTER(_I64), _P]),
    "bmx_route_slot_step": (_I, [ctypes.POINTER(SlotTable), _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, ctypes.c_float, _I64,
                                 _I, _P, _P, ctypes.POINTER(_I64), _P]),
    "bmx_slot_prefetch_agent": (_I, [ctypes.POINTER(SlotTable), _P, _I, _P, _I, _I64, _I, ctypes.POINTER(_I64), _P]),
    "bmx_copy_wait": (_I, [_P, _I64, _I, _P]),
    "bmx_copy_wait_layer": (_I, [_P, _I, _I, _P]),
    "bmx_cpu_expert_rows": (_I, [ctypes.POINTER(CpuExpert), _I, _I, _P, _I, _I, _I, _I, _I, _I, ctypes.c_float, _P, _I]),
    "bmx_cpu_expert_rows_fast": (_I, [ctypes.POINTER(CpuExpert), _I, _I, _P, _I, _I, _I, ctypes.c_float, _P, _I]),
    "bmx_decode_splits": (_I, [ctypes.POINTER(MoeDesc), _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "bmx_cpu_dot2": (_I, [_P, _P, _P, _P, _I]),
    "bmx_dot2_f32_f16": (_I, [_P, _P, _P, _P, _I, _P]),
    "bmx_copy_agent_plan": (_I, [_P, ctypes.POINTER(PlanPolicy)]),
    "bmx_copy_agent_cpu_lane": (_I, [_P, ctypes.POINTER(MoeDesc), _P, _I]),
    "bmx_slot_step_planned": (_I, [ctypes.POINTER(SlotTable), _P, _I, _P, _P, _I, _I, _I64, _I, _P, _P, _P, _P,
                                   ctypes.POINTER(_I64), _P]),
    "bmx_cpu_lane_add": (_I, [_P, _I64, _P, _I, _P]),
    "bmx_copy_agent_plan_stats": (_I, [_P, _P]),
    "bmx_slot_stage_async": (_I, [_P, _P, _P, _I, _P]),
    "bmx_slot_stage_rows": (_I, [ctypes.POINTER(SlotTable), _I, _P, _I, ctypes.c_uint64, _I, _P]),
    "bmx_host_device_ptr": (_I, [_P, ctypes.POINTER(ctypes.c_uint64)]),
}

_lib = None


def lib():
    """The loaded libbmx.so. Raises if it is missing: the HIP library is the only implementation."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libbmx.so not built ({LIB_PATH}); run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class BmxError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != BMX_OK:
        msg = lib().bmx_last_error().decode(errors="replace")
        raise BmxError(f"{what}: status {rc}: {msg}")
    return rc
