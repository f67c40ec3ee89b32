"""CPU oracle for the routed-expert MoE layer: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as a reference to
check against. The product (libbmx.so and the bmx package) never imports, links or falls back to it.

Two independent restatements of the reference's EXL3 decode live here:
  * liboracle.so (bmx_oracle.c): the C oracle for decode, rotations, expert, layer, router, dispatch and slot table;
  * a numpy twin of the trellis decode that expands the ring into single bits and reads each 16-bit window bit by bit
    (the closed form of tests/gpu_dsv41_vbmi_tables.py:67-81 of the reference), with the codebook computed by numpy's
    own fp16 rounding.
and ref_lane(): the reference's CPU lane (ft_core.h / ft_n135.h) compiled from the reference tree into _ref/.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libreflane.so")

TF_K2, TF_K25, TF_K3, TF_K4 = 0, 1, 2, 3
TF_KA = {TF_K2: 2, TF_K25: 2, TF_K3: 3, TF_K4: 4}
TF_MASK = {TF_K2: 0, TF_K25: 0xAAAA, TF_K3: 0, TF_K4: 0}
TF_TB = {TF_K2: 64, TF_K25: 80, TF_K3: 96, TF_K4: 128}
SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSP = 0, 1, 2
ACT_SILU, ACT_GELU, ACT_RELU2, ACT_SILU_OAI = 0, 1, 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_lib = None
_ref = None


def build():
    """Compile liboracle.so (and the reference lane when the reference tree is present)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference/src/bigmoe/engine/kernels/nv2"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.bmxo_f32_to_f16.argtypes = [ctypes.c_float]; L.bmxo_f32_to_f16.restype = ctypes.c_uint16
        L.bmxo_f16_to_f32.argtypes = [ctypes.c_uint16]; L.bmxo_f16_to_f32.restype = ctypes.c_float
        L.bmxo_tile_bytes.argtypes = [_I]; L.bmxo_tile_bytes.restype = _I
        L.bmxo_ring_end.argtypes = [_I, _I]; L.bmxo_ring_end.restype = _I
        L.bmxo_tile_states.argtypes = [_P, _I, _P]
        L.bmxo_perm.argtypes = [_P]
        L.bmxo_bytesum.argtypes = [ctypes.c_uint16]; L.bmxo_bytesum.restype = ctypes.c_uint32
        L.bmxo_decode_state.argtypes = [ctypes.c_uint16]; L.bmxo_decode_state.restype = ctypes.c_uint16
        L.bmxo_dequant.argtypes = [_P, _I, _I, _I, _P]
        L.bmxo_had128.argtypes = [_P]
        L.bmxo_prep.argtypes = [_P, _P, _I, _P]
        L.bmxo_expert_forward.argtypes = [_P, _I, _I, _I, _I, ctypes.c_float, _P, _P, _P, _P, _P]
        L.bmxo_moe_forward.argtypes = [_P, _I, ctypes.c_int64, _P, _P, _I, _I, _I, _I, ctypes.c_float, _P, _I, _I, _P, _P,
                                       _P, _I, _P]
        L.bmxo_exp.argtypes = [ctypes.c_float]; L.bmxo_exp.restype = ctypes.c_float
        L.bmxo_sigmoid.argtypes = [ctypes.c_float]; L.bmxo_sigmoid.restype = ctypes.c_float
        L.bmxo_sqrtsp.argtypes = [ctypes.c_float]; L.bmxo_sqrtsp.restype = ctypes.c_float
        L.bmxo_shared_gate.argtypes = [_P, _P, _I]; L.bmxo_shared_gate.restype = ctypes.c_float
        L.bmxo_act.argtypes = [_I, _I, ctypes.c_float, ctypes.c_float, ctypes.c_float]; L.bmxo_act.restype = ctypes.c_float
        L.bmxo_router.argtypes = [_P, _P, _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, ctypes.c_int64, _P, _P]
        L.bmxo_dispatch.argtypes = [_P, _I, _I, _I, ctypes.c_int64, _I, _P, _P, _P, _P, _P, _P]
        L.bmxo_dispatch.restype = _I
        L.bmxo_slot_step.argtypes = [_P, _I, _P, _I, ctypes.c_int64, _I, _I, _P, _P, _P, _P]
        L.bmxo_slot_step.restype = _I
        L.bmxo_slot_step_lanes.argtypes = [_P, _I, _P, _I, ctypes.c_int64, _I, _I, _P, _P, _P, _P, _P]
        L.bmxo_slot_step_lanes.restype = _I
        L.bmxo_slot_prefetch.argtypes = [_P, _I, _P, _I, ctypes.c_int64, _I, _I, _P, _P, _P]
        L.bmxo_slot_prefetch.restype = _I
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- C oracle wrappers -------------------------------------------------------------------------------------------

def f32_to_f16(v):
    v = _c(v, np.float32).ravel()
    return np.array([lib().bmxo_f32_to_f16(float(x)) for x in v], dtype=np.uint16)


def tile_states(tile, fmt):
    tile = _c(tile, np.uint8)
    out = np.zeros(256, np.uint16)
    lib().bmxo_tile_states(_p(tile), fmt, _p(out))
    return out


def perm():
    out = np.zeros(256, np.int32)
    lib().bmxo_perm(_p(out))
    return out


def decode_table():
    """fp16 bits of the codebook weight of every 16-bit state."""
    L = lib()
    return np.array([L.bmxo_decode_state(s) for s in range(65536)], dtype=np.uint16)


def dequant(trellis, fmt, k, n):
    trellis = _c(trellis, np.uint8)
    assert trellis.size == (k // 16) * (n // 16) * TF_TB[fmt]
    out = np.zeros((k, n), np.uint16)
    lib().bmxo_dequant(_p(trellis), fmt, k, n, _p(out))
    return out.view(np.float16)


def prep(x, suh):
    x = _c(x, np.float16).view(np.uint16)
    suh = _c(suh, np.float16).view(np.uint16)
    out = np.zeros(x.size, np.uint16)
    lib().bmxo_prep(_p(x), _p(suh), x.size, _p(out))
    return out.view(np.float16)


class _Expert(ctypes.Structure):
    _fields_ = [("tr", _P * 3), ("suh", _P * 3), ("svh", _P * 3), ("fmt", _I * 3)]


def _expert_struct(ex):
    s = _Expert()
    keep = []
    for m in range(3):
        t = _c(ex["tr"][m], np.uint8); a = _c(ex["suh"][m], np.float16); b = _c(ex["svh"][m], np.float16)
        keep += [t, a, b]
        s.tr[m] = t.ctypes.data; s.suh[m] = a.ctypes.data; s.svh[m] = b.ctypes.data
        s.fmt[m] = int(ex["fmt"][m])
    return s, keep


def expert_forward(ex, H, I, x, act=ACT_SILU, gated=True, limit=0.0):
    """-> (y fp32 [H], gate fp16 [I], up fp16 [I], act fp16 [I])"""
    s, keep = _expert_struct(ex)
    x = _c(x, np.float16).view(np.uint16)
    y = np.zeros(H, np.float32)
    g = np.zeros(I, np.uint16); u = np.zeros(I, np.uint16); a = np.zeros(I, np.uint16)
    lib().bmxo_expert_forward(ctypes.byref(s), H, I, act, int(gated), limit, _p(x), _p(y), _p(g), _p(u), _p(a))
    return y, g.view(np.float16), u.view(np.float16), a.view(np.float16)


def moe_forward(experts, first, shared, H, I, x, sel, w, rows=None, act=ACT_SILU, gated=True, limit=0.0, sh_gate=None):
    """Layer output fp32 [len(rows) or T, H]. experts: list of dicts with tr / suh / svh / fmt (3 each), None for
    experts no selected pick uses. sh_gate: fp16 [H] gate vector of the shared expert (its output scaled by
    sigmoid(x . sh_gate)), or None (weight 1)."""
    E = len(experts)
    arr = (_Expert * E)()
    keep = []
    for i, ex in enumerate(experts):
        if ex is None:        # never touched by the selected picks (the oracle dereferences used experts only)
            continue
        s, k = _expert_struct(ex)
        arr[i] = s
        keep += k
    sh = None
    if shared is not None:
        sh, k = _expert_struct(shared)
        keep += k
    x = _c(x, np.float16).view(np.uint16)
    T, topk = sel.shape
    sel = _c(sel, np.int64); w = _c(w, np.float16).view(np.uint16)
    r = None if rows is None else _c(rows, np.int32)
    nr = T if rows is None else r.size
    out = np.zeros((nr, H), np.float32)
    g = None if sh_gate is None else _c(sh_gate, np.float16).view(np.uint16)
    lib().bmxo_moe_forward(ctypes.cast(arr, _P), E, first, ctypes.byref(sh) if sh is not None else None,
                           _p(g) if g is not None else None, H, I, act,
                           int(gated), limit, _p(x), T, topk, _p(sel), _p(w), _p(r) if r is not None else None, nr,
                           _p(out))
    return out


def router(logits, topk, bias=None, n_group=1, topk_group=1, score_fn=SCORE_SIGMOID, renorm=True, scale=1.0, first=0):
    lg = _c(logits, np.float16).view(np.uint16)
    T, E = lg.shape
    b = None if bias is None else _c(bias, np.float32)
    sel = np.zeros((T, topk), np.int64)
    w = np.zeros((T, topk), np.uint16)
    lib().bmxo_router(_p(lg), _p(b) if b is not None else None, T, E, topk, n_group, topk_group, score_fn, int(renorm),
                      scale, first, _p(sel), _p(w))
    return sel, w.view(np.float16)


def dispatch(sel, E, first=0, shared=False):
    sel = _c(sel, np.int64)
    T, topk = sel.shape
    NE = E + (1 if shared else 0)
    R = T * topk + (T if shared else 0)
    counts = np.zeros(NE, np.int32); offsets = np.zeros(NE + 1, np.int32)
    row_token = np.full(R, -1, np.int32); row_slot = np.full(R, -1, np.int32)
    inv = np.zeros(T * topk, np.int32); uexp = np.zeros(NE, np.int32)
    nu = lib().bmxo_dispatch(_p(sel), T, topk, E, first, int(shared), _p(counts), _p(offsets), _p(row_token),
                             _p(row_slot), _p(inv), _p(uexp))
    n = int(offsets[-1])
    return dict(counts=counts, offsets=offsets, row_token=row_token[:n], row_slot=row_slot[:n], inv=inv.reshape(T, topk),
                uexp=uexp[:nu], nuniq=nu)


class _Slots(ctypes.Structure):
    _fields_ = [("L", _I), ("E", _I), ("S", _I), ("slotof", _P), ("owner", _P), ("refb", _P), ("pin", _P), ("pfl", _P),
                ("hand", ctypes.c_int32), ("epoch", ctypes.c_int32)]


class SlotTable:
    """The oracle's CLOCK expert-slot table (numpy state, C step and prefetch).
    stats: hits, misses, admissions, steps without a victim, evictions, prefetch admissions, prefetched experts used by a
    step, prefetched experts evicted unused."""

    def __init__(self, L, E, S):
        self.L, self.E, self.S = L, E, S
        self.slotof = np.full(L * E, -1, np.int32)
        self.owner = np.full(max(S, 1), -1, np.int32)
        self.refb = np.zeros(max(S, 1), np.int32)
        self.pin = np.zeros(max(S, 1), np.int32)
        self.pfl = np.zeros(max(S, 1), np.int32)
        self.stats = np.zeros(8, np.int64)
        self.fresh = np.zeros(E, np.int32)
        self._s = _Slots(L, E, S, self.slotof.ctypes.data, self.owner.ctypes.data, self.refb.ctypes.data,
                         self.pin.ctypes.data, self.pfl.ctypes.data, 0, 0)

    @property
    def hand(self):
        return self._s.hand

    @property
    def epoch(self):
        return self._s.epoch

    def step(self, li, sel, first=0, admit=True, maxj=1024, elane=None):
        """Returns (jobs [nj, 2] = (expert, slot), evicted owners [nj]); self.fresh is the step's fresh flags.
        elane: int32 [E] lane of each expert (a planned step: only LANE_ADMIT misses are admitted) or None."""
        sel = _c(sel, np.int64).ravel()
        jobs = np.zeros(2 * maxj, np.int32)
        ev = np.zeros(maxj, np.int32)
        if elane is None:
            nj = lib().bmxo_slot_step(ctypes.byref(self._s), li, _p(sel), sel.size, first, int(admit), maxj, _p(jobs),
                                      _p(ev), _p(self.fresh), _p(self.stats))
        else:
            el = _c(elane, np.int32)
            nj = lib().bmxo_slot_step_lanes(ctypes.byref(self._s), li, _p(sel), sel.size, first, int(admit), maxj,
                                            _p(el), _p(jobs), _p(ev), _p(self.fresh), _p(self.stats))
        return jobs[:2 * nj].reshape(nj, 2), ev[:nj]

    def request(self, li, sel, first=0):
        """What a planned step of these picks publishes: (unique local experts ascending, resident flags, pick
        counts)."""
        sel = _c(sel, np.int64).ravel() - first
        sel = sel[(sel >= 0) & (sel < self.E)]
        ex, cnt = np.unique(sel, return_counts=True)
        res = (self.slotof[li * self.E + ex] >= 0).astype(np.int32)
        return ex.astype(np.int32), res, cnt.astype(np.int32)

    def prefetch(self, li, sel, first=0, limit=1 << 30, maxj=1024):
        sel = _c(sel, np.int64).ravel()
        jobs = np.zeros(2 * maxj, np.int32)
        ev = np.zeros(maxj, np.int32)
        nj = lib().bmxo_slot_prefetch(ctypes.byref(self._s), li, _p(sel), sel.size, first, min(limit, 1 << 30), maxj,
                                      _p(jobs), _p(ev), _p(self.stats))
        return jobs[:2 * nj].reshape(nj, 2), ev[:nj]


# ---- residency plan (a planned step's reply) ------------------------------------------------------------------------
LANE_VRAM, LANE_ADMIT, LANE_HOME, LANE_CPU = 0, 1, 2, 3
PLAN_MAXP, PLAN_MAXT = 64, 8
PLAN_DEFAULT = dict(cpu_on=0, max_cpu=0, home_single=0, gpu_base_us=0.0, gpu_hit_us=0.0, gpu_home_us=0.0,
                    gpu_admit_us=0.0, cpu_base_us=0.0, cpu_expert_us=0.0, cpu_token_us=0.0)


def plan_lanes(ex, res, cnt, ntok, npicks, rows, policy=None, cpu_ready=True):
    """The planner's lanes for a request (include/bmx.h bmx_plan_policy; the reference's two-lane rule,
    engine/kernels/nv2/nv2_host.cpp:1017-1030): residents LANE_VRAM; the GPU's estimated time starts at its base plus
    the hits (0 when nothing is resident), the CPU lane's at its base when it is eligible (on, set up, the call's picks
    and rows came with the request) and some expert misses; the misses by picks descending then expert ascending, each
    to the CPU lane when that keeps the later of the two finish times no later than the GPU taking it (and the lane is
    not full), else to the GPU (LANE_HOME for a single-pick expert of a multi-token call under home_single, else
    LANE_ADMIT). rows: the request carried the call's input rows."""
    p = dict(PLAN_DEFAULT, **(policy or {}))
    lanes = np.full(len(ex), LANE_VRAM, np.int32)
    cpu_ok = bool(p["cpu_on"]) and cpu_ready and rows and npicks <= PLAN_MAXP and ntok <= PLAN_MAXT
    nres = int(np.sum(res != 0))
    misses = sorted((u for u in range(len(ex)) if not res[u]), key=lambda u: (-int(cnt[u]), int(ex[u])))
    g = p["gpu_base_us"] + p["gpu_hit_us"] * nres if nres else 0.0
    c, ncpu = (p["cpu_base_us"] if cpu_ok and misses else 0.0), 0
    for u in misses:
        home = bool(p["home_single"]) and ntok > 1 and cnt[u] == 1
        gc = p["gpu_home_us"] if home else p["gpu_admit_us"]
        cc = p["cpu_expert_us"] + p["cpu_token_us"] * (int(cnt[u]) - 1)
        if cpu_ok and ncpu < p["max_cpu"] and max(c + cc, g) <= max(c, g + gc):
            lanes[u] = LANE_CPU
            c += cc
            ncpu += 1
        else:
            lanes[u] = LANE_HOME if home else LANE_ADMIT
            g += gc
    return lanes


def expert_lanes(E, ex, lanes):
    """[E] lane per local expert (LANE_VRAM for the ones not picked)"""
    el = np.full(E, LANE_VRAM, np.int32)
    el[np.asarray(ex, np.int64)] = lanes
    return el


def planned_selection(sel, w, first, elane):
    """(sel_gpu, w_gpu, lanes) of a planned step: CPU-lane picks masked (-1, weight 0); lanes -1 out of range."""
    sel = np.asarray(sel, np.int64).ravel()
    w = np.asarray(w, np.float16).ravel()
    E = len(elane)
    e = sel - first
    inr = (e >= 0) & (e < E)
    ln = np.where(inr, elane[np.clip(e, 0, E - 1)], -1).astype(np.int32)
    cpu = ln == LANE_CPU
    return np.where(cpu, -1, sel), np.where(cpu, np.float16(0), w), ln


def sqrtsp32(x):
    """the fixed-sequence sqrt(softplus(x)) of the router's sqrt-softplus score"""
    return np.float32(lib().bmxo_sqrtsp(float(x)))


def shared_gate(x, g):
    """sigmoid(x . g) of one token in the GPU combine's fixed order (x, g fp16 [H])"""
    x = _c(x, np.float16).view(np.uint16)
    g = _c(g, np.float16).view(np.uint16)
    return np.float32(lib().bmxo_shared_gate(_p(x), _p(g), x.size))


def router_logits(z, weight):
    """The router projection's exact value in float64: z fp16 [T, H] times weight fp16 [E, H] transposed (the GPU's
    fp16 logits are this value's RN16 within the fp32 accumulation's error)."""
    return np.asarray(z, np.float16).astype(np.float64) @ np.asarray(weight, np.float16).astype(np.float64).T


def exp32(x):
    return np.float32(lib().bmxo_exp(float(x)))


def act(a, gated, g, u, limit=0.0):
    """act_gate of one (gate, up) pair (x16_dev.cu:68-112)"""
    return np.float32(lib().bmxo_act(int(a), int(gated), float(g), float(u), float(limit)))


# ---- numpy twin of the decode (independent restatement) ---------------------------------------------------------

def np_ring_end(fmt, i):
    ka, mask = TF_KA[fmt], TF_MASK[fmt]
    s = (i >> 4) * (16 * ka + bin(mask).count("1"))
    for j in range((i & 15) + 1):
        s += ka + ((mask >> j) & 1)
    return s


def np_tile_states(tiles, fmt):
    """tiles uint8 [N, tb] -> states uint16 [N, 256] by expanding the ring to bits (MSB-first in little-endian u32)."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8)
    N, tb = tiles.shape
    words = tiles.view("<u4").astype(np.uint64)
    nbits = tb * 8
    shifts = (31 - (np.arange(nbits) & 31)).astype(np.uint64)
    bits = (words[:, np.arange(nbits) >> 5] >> shifts) & 1          # [N, nbits]
    ends = np.array([np_ring_end(fmt, i) for i in range(256)])
    pos = (ends[:, None] - 16 + np.arange(16)[None, :]) % nbits         # [256, 16]
    sel = bits[:, pos]                                                  # [N, 256, 16]
    weights = (1 << np.arange(15, -1, -1)).astype(np.uint64)
    return (sel * weights).sum(-1).astype(np.uint16)


def np_perm():
    p = np.zeros(256, np.int32)
    for i in range(256):
        g, j = divmod(i, 8)
        r = 2 * (g % 4) + (0, 1, 8, 9)[j % 4]
        c = g // 4 + (8 if j >= 4 else 0)
        p[i] = r * 16 + c
    return p


def np_codebook():
    """fp16 codebook for all states: bytesum of st * 0x83DCD12D, then RN16(fma(1024 + s, KINV, KBIAS)) in float64
    (exact) rounded by numpy's float16 conversion."""
    st = np.arange(65536, dtype=np.uint64)
    x = (st * 0x83DCD12D) & 0xFFFFFFFF
    s = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24)
    kinv = float(np.array(0x1eee, np.uint16).view(np.float16))
    kbias = float(np.array(0xc931, np.uint16).view(np.float16))
    return ((1024.0 + s.astype(np.float64)) * kinv + kbias).astype(np.float16)


def np_dequant(trellis, fmt, k, n, codebook=None):
    cb = np_codebook() if codebook is None else codebook
    tb = TF_TB[fmt]
    tiles = np.ascontiguousarray(trellis, dtype=np.uint8).reshape(-1, tb)
    st = np_tile_states(tiles, fmt).reshape(k // 16, n // 16, 256)
    w = cb[st]                                                        # [tk, tn, 256]
    p = np_perm()
    out = np.zeros((k // 16, n // 16, 256), np.float16)
    out[:, :, p] = w
    return out.reshape(k // 16, n // 16, 16, 16).transpose(0, 2, 1, 3).reshape(k, n)


# ---- reference CPU lane ------------------------------------------------------------------------------------------

def ref_lane():
    """ctypes handle to the reference's CPU lane built from the reference tree (None when it was not built)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        R = ctypes.CDLL(REF_PATH)
        R.ref_dense_weights_k3.argtypes = [_P, _I, _I, _P]
        R.ref_state_scalar_k3.argtypes = [_P, _I]; R.ref_state_scalar_k3.restype = ctypes.c_uint16
        R.ref_w_gpu.argtypes = [ctypes.c_uint16]; R.ref_w_gpu.restype = ctypes.c_float
        R.ref_perm.argtypes = [_I]; R.ref_perm.restype = _I
        R.ref_tf_s.argtypes = [_I, _I]; R.ref_tf_s.restype = _I
        R.ref_prep_block.argtypes = [_P, _P, _P]
        R.ref_prep_block_v.argtypes = [_P, _P, _P]
        R.ref_out_block.argtypes = [_P, _P]
        R.ref_had128.argtypes = [_P]
        R.ref_lane_create.argtypes = [_I, _I, _I, _I, _P, ctypes.c_float]; R.ref_lane_create.restype = _I
        R.ref_lane_set_expert.argtypes = [_I] + [_P] * 9 + [_I] * 3; R.ref_lane_set_expert.restype = _I
        R.ref_lane_forward.argtypes = [_P, _I, _P, _P, _I, _P, _I]; R.ref_lane_forward.restype = _I
        R.ref_vbmi.restype = _I
        R.ref_init()
        _ref = R
    return _ref
