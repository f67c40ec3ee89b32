"""CPU expert lane: one expert's y rows on host cores, bit for bit the GPU decode path's (bmx_cpu_expert_rows), or
fast within the layer tolerance (bmx_cpu_expert_rows_fast).

The reference's CPU lane (engine/kernels/nv2/nv2_host.cpp, docs/x16.md) computes RAM-resident experts on the host with
its own arithmetic. The exact mode replays the MI355X kernels' arithmetic, so a layer can mix GPU and CPU experts and
still produce the all-GPU result bit for bit (the combine sums the y rows in slot order either way); the fast mode keeps
the exact weights and roundings between the GEMVs but sums the products in plain fp32 FMAs, for throughput."""
import ctypes

import numpy as np

from . import _lib as L


def decode_splits(desc, T):
    """(ks_gu, ks_dn, grouped_gu) of the device's decode plan for a call of T tokens."""
    a, b, g = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    L.check(L.lib().bmx_decode_splits(ctypes.byref(desc), int(T), ctypes.byref(a), ctypes.byref(b), ctypes.byref(g)),
            "bmx_decode_splits")
    return a.value, b.value, g.value


def _cpu_expert(host_expert):
    """bmx_cpu_expert of a host expert and the arrays it points into (keep them alive during the call)"""
    keep = [np.ascontiguousarray(t) for t in host_expert["tr"]]
    keep += [np.ascontiguousarray(v, dtype=np.float16) for v in host_expert["suh"]]
    keep += [np.ascontiguousarray(v, dtype=np.float16) for v in host_expert["svh"]]
    ex = L.CpuExpert()
    for m in range(3):
        ex.tr[m] = keep[m].ctypes.data
        ex.suh[m] = keep[3 + m].ctypes.data
        ex.svh[m] = keep[6 + m].ctypes.data
        ex.fmt[m] = int(host_expert["fmt"][m])
    return ex, keep


def expert_rows(host_expert, H, I, x, ks_gu, ks_dn, grouped_gu, act=L.ACT_SILU, gated=True, limit=0.0, threads=8):
    """y rows fp32 [nr, H] of fp16 rows x [nr, H] through one expert, bit for bit the GPU decode path's for the plan
    (ks_gu, ks_dn, grouped_gu). host_expert: ExpertTable.host_expert(e)."""
    x = np.ascontiguousarray(x, dtype=np.float16).reshape(-1, H)
    ex, keep = _cpu_expert(host_expert)
    y = np.zeros((x.shape[0], H), np.float32)
    L.check(L.lib().bmx_cpu_expert_rows(ctypes.byref(ex), H, I, x.ctypes.data, x.shape[0], ks_gu, ks_dn,
                                        int(grouped_gu), int(act), int(gated), float(limit), y.ctypes.data, int(threads)),
            "bmx_cpu_expert_rows")
    del keep
    return y


def expert_rows_fast(host_expert, H, I, x, act=L.ACT_SILU, gated=True, limit=0.0, threads=8):
    """y rows fp32 [nr, H] of fp16 rows x [nr, H] through one expert, fast (within the layer tolerance)."""
    x = np.ascontiguousarray(x, dtype=np.float16).reshape(-1, H)
    ex, keep = _cpu_expert(host_expert)
    y = np.zeros((x.shape[0], H), np.float32)
    L.check(L.lib().bmx_cpu_expert_rows_fast(ctypes.byref(ex), H, I, x.ctypes.data, x.shape[0], int(act), int(gated),
                                             float(limit), y.ctypes.data, int(threads)), "bmx_cpu_expert_rows_fast")
    del keep
    return y


def dot2(a, b, c):
    """The host emulation of v_dot2_f32_f16 over arrays (a, b: uint32 fp16 pairs; c: fp32)."""
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    out = np.empty(c.shape, np.float32)
    L.check(L.lib().bmx_cpu_dot2(a.ctypes.data, b.ctypes.data, c.ctypes.data, out.ctypes.data, c.size), "bmx_cpu_dot2")
    return out
