"""Expert storage for one MoE layer: EXL3 trellis records plus fp16 scales, and the device table (bmx_expert[E])
that the kernels read.

Record geometry follows the reference's VRAM slot: one record per expert holding gate | up @ off_u | down @ off_d, each
matrix 256-byte aligned, uniform over the layer (the largest expert's size; engine/tiers.py:275-303 `Pool` slot
geometry, engine/tiers.py:53-75 store manifests)."""
import ctypes

import torch

from . import _lib as L

ALIGN = 256


def _al(n, a=ALIGN):
    return (n + a - 1) // a * a


def matrix_bytes(k, n, fmt):
    return (k // 16) * (n // 16) * L.TILE_BYTES[fmt]


def device_address(t):
    """Address at which the GPU reads tensor t: its data pointer for device memory, the mapped address
    (hipHostGetDevicePointer) for pinned host memory."""
    if t.is_cuda:
        return t.data_ptr()
    if not t.is_pinned():
        raise ValueError("expert homes in host memory must be pinned (allocated with pin_memory=True)")
    out = ctypes.c_uint64(0)
    L.check(L.lib().bmx_host_device_ptr(ctypes.c_void_p(t.data_ptr()), ctypes.byref(out)), "bmx_host_device_ptr")
    return int(out.value)


class ExpertTable:
    """E routed experts (+ optional shared expert at index E) of one layer.

    arena uint8 [E + shared, rec] (device memory, or pinned host memory the kernels read over PCIe: the home of experts
    an expert-slot table stages into VRAM); suh / svh: lists of three fp16 device tensors [E + shared, k] /
    [E + shared, n]; fmt int [E + shared, 3]. Build with ExpertTable.random(...) or from existing tensors."""

    def __init__(self, H, I, arena, fmt, suh, svh, off_u, off_d, n_routed, has_shared):
        self.H, self.I = H, I
        self.arena, self.fmt, self.suh, self.svh = arena, fmt, suh, svh
        self.off_u, self.off_d, self.rec = off_u, off_d, arena.shape[1]
        self.E, self.has_shared = n_routed, has_shared
        self.device = suh[0].device
        self._table = None
        base = device_address(arena)
        self.addr = [(base + e * self.rec, base + e * self.rec + off_u, base + e * self.rec + off_d)
                     for e in range(n_routed + (1 if has_shared else 0))]   # home trellis addresses

    @staticmethod
    def geometry(H, I, fmts):
        """(off_u, off_d, rec) of a uniform record for the given per-expert formats [(fg, fu, fd), ...]."""
        sg = max(matrix_bytes(H, I, f[0]) for f in fmts)
        su = max(matrix_bytes(H, I, f[1]) for f in fmts)
        sd = max(matrix_bytes(I, H, f[2]) for f in fmts)
        off_u = _al(sg)
        off_d = off_u + _al(su)
        return off_u, off_d, off_d + _al(sd)

    @classmethod
    def random(cls, H, I, E, fmts, shared=False, seed=0, device="cuda", svh_norm=True, home="device"):
        """Random trellis bytes (every bit string is a valid code), suh ~ U(0.5, 1.5), svh ~ U(0.5, 1.5) / sqrt(k) when
        svh_norm (each linear then keeps the norm of its input, so layer outputs are O(1)). fmts: one (fg, fu, fd) for
        every expert (E + shared entries) or a single tuple for all. home = "host": the trellis arena in pinned host
        memory (drawn on the device and copied, the same bytes as a device arena of the same seed)."""
        n = E + (1 if shared else 0)
        if isinstance(fmts, tuple):
            fmts = [fmts] * n
        assert len(fmts) == n
        off_u, off_d, rec = cls.geometry(H, I, fmts)
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        arena = torch.randint(0, 256, (n, rec), dtype=torch.uint8, device=dev, generator=g)
        if home == "host":
            pinned = torch.empty((n, rec), dtype=torch.uint8, pin_memory=True)
            pinned.copy_(arena)
            arena = pinned
        dims = ((H, I), (H, I), (I, H))
        suh, svh = [], []
        for k, nn in dims:
            suh.append((torch.rand((n, k), device=dev, generator=g) + 0.5).half())
            s = torch.rand((n, nn), device=dev, generator=g) + 0.5
            svh.append((s / (k ** 0.5) if svh_norm else s).half())
        fmt = torch.tensor(fmts, dtype=torch.int32)
        return cls(H, I, arena, fmt, suh, svh, off_u, off_d, E, shared)

    def shared_to_device(self):
        """Keep the shared expert's trellis in device memory (a copy; the routed experts stay at their home). Call before
        the table is built."""
        if not self.has_shared or self._table is not None:
            raise ValueError("shared_to_device: no shared expert, or the table is already built")
        self._shared_dev = self.arena[self.E].to(self.device)
        b = self._shared_dev.data_ptr()
        self.addr[self.E] = (b, b + self.off_u, b + self.off_d)

    def mat_bytes(self, e, m):
        k, n = ((self.H, self.I), (self.H, self.I), (self.I, self.H))[m]
        return matrix_bytes(k, n, int(self.fmt[e, m]))

    def expert_bytes(self, e):
        return sum(self.mat_bytes(e, m) for m in range(3))

    def structs(self, tr_addr=None):
        """ctypes array of bmx_expert for every expert (tr from tr_addr[e] when given: slot-table placements)."""
        n = self.E + (1 if self.has_shared else 0)
        arr = (L.Expert * n)()
        for e in range(n):
            tr = tr_addr[e] if tr_addr is not None else self.addr[e]
            for m in range(3):
                arr[e].tr[m] = tr[m]
                arr[e].suh[m] = self.suh[m][e].data_ptr()
                arr[e].svh[m] = self.svh[m][e].data_ptr()
                arr[e].fmt[m] = int(self.fmt[e, m])
        return arr

    def table(self):
        """Device bmx_expert[E (+1)] (built once)."""
        if self._table is None:
            arr = self.structs()
            raw = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
            self._table = raw.to(self.device)
        return self._table

    def desc(self, topk, first=0, act=L.ACT_SILU, gated=True, act_limit=0.0, fresh=None, shared_gate=None):
        """bmx_moe_desc of the layer; shared_gate: fp16 [H] device tensor scaling the shared expert's output by
        sigmoid(x . shared_gate), or None (weight 1)."""
        t = self.table()
        es = ctypes.sizeof(L.Expert)
        shared = t.data_ptr() + self.E * es if self.has_shared else None
        if shared_gate is not None and (shared_gate.dtype != torch.float16 or shared_gate.numel() != self.H or
                                        not shared_gate.is_cuda or not shared_gate.is_contiguous()):
            raise ValueError("shared_gate must be a contiguous fp16 device tensor of H elements")
        return L.MoeDesc(self.H, self.I, self.E, topk, first, act, int(gated), act_limit, t.data_ptr(), shared,
                         fresh.data_ptr() if fresh is not None else None,
                         shared_gate.data_ptr() if shared_gate is not None else None)

    def host_expert(self, e):
        """numpy copies of one expert (trellis per matrix, scales, formats) for the oracle."""
        import numpy as np
        rec = self.arena[e].cpu().numpy()
        offs = (0, self.off_u, self.off_d)
        tr = [np.ascontiguousarray(rec[offs[m]:offs[m] + self.mat_bytes(e, m)]) for m in range(3)]
        suh = [self.suh[m][e].cpu().numpy() for m in range(3)]
        svh = [self.svh[m][e].cpu().numpy() for m in range(3)]
        return {"tr": tr, "suh": suh, "svh": svh, "fmt": [int(self.fmt[e, m]) for m in range(3)]}
