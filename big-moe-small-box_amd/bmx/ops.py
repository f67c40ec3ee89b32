"""Torch-facing wrappers of the C ABI. Tensors are device tensors on the current HIP device; every call is enqueued on
torch's current stream and returns without synchronising."""
import ctypes

import torch

from . import _lib as L
from ._lib import check, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(t, dtype, name):
    if t.dtype != dtype or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous {dtype} device tensor, got {t.dtype} on {t.device}")


def dequant(trellis, fmt, k, n):
    """EXL3 trellis (uint8, tiles [k/16][n/16][32 K]) -> fp16 [k, n] codebook weights."""
    _need(trellis, torch.uint8, "trellis")
    if trellis.numel() != (k // 16) * (n // 16) * L.TILE_BYTES[fmt]:
        raise ValueError("trellis size does not match k, n and the format")
    out = torch.empty((k, n), dtype=torch.float16, device=trellis.device)
    check(lib().bmx_exl3_dequant(_ptr(trellis), fmt, k, n, _ptr(out), _stream()), "bmx_exl3_dequant")
    return out


def router_topk(logits, topk, bias=None, n_group=1, topk_group=1, score=L.SCORE_SIGMOID, renorm=True, scale=1.0,
                first=0):
    """logits fp16 [T, E] -> (sel int64 [T, topk], w fp16 [T, topk])."""
    _need(logits, torch.float16, "logits")
    T, E = logits.shape
    if bias is not None:
        _need(bias, torch.float32, "bias")
    sel = torch.empty((T, topk), dtype=torch.int64, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.float16, device=logits.device)
    check(lib().bmx_router_topk(_ptr(logits), _ptr(bias), T, E, topk, n_group, topk_group, score, int(renorm),
                                float(scale), int(first), _ptr(sel), _ptr(w), _stream()), "bmx_router_topk")
    return sel, w


def router_logits(z, weight):
    """Router projection on the MFMA units: z fp16 [T, H], weight fp16 [E, H] (the gate weight as checkpoints store it)
    -> logits fp16 [T, E] = RN16(z weight^T), fp32 accumulation."""
    _need(z, torch.float16, "z"); _need(weight, torch.float16, "router weight")
    T, H = z.shape
    E = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError(f"router weight {tuple(weight.shape)} does not match H = {H}")
    out = torch.empty((T, E), dtype=torch.float16, device=z.device)
    check(lib().bmx_router_logits(_ptr(z), _ptr(weight), T, H, E, _ptr(out), _stream()), "bmx_router_logits")
    return out


class RoutesBuf:
    """Dispatch outputs (device int32 tensors) and the ctypes struct pointing at them."""

    def __init__(self, T, topk, E, shared, rows_per_group, device):
        NE = E + 1
        R = T * topk + (T if shared else 0)
        G = lib().bmx_groups_max(T, topk, E, int(shared), rows_per_group)
        i32 = dict(dtype=torch.int32, device=device)
        self.counts = torch.zeros(NE, **i32)
        self.offsets = torch.zeros(NE + 1, **i32)
        self.row_token = torch.full((max(R, 1),), -1, **i32)
        self.row_slot = torch.full((max(R, 1),), -1, **i32)
        self.inv = torch.zeros(max(T * topk, 1), **i32)
        self.uexp = torch.zeros(NE, **i32)
        self.nuniq = torch.zeros(1, **i32)
        self.groups = torch.zeros(max(G, 1) * 3, **i32)
        self.ngroups = torch.zeros(1, **i32)
        self.row_expert = torch.full((max(R, 1),), -1, **i32)
        self.T, self.topk, self.E, self.shared, self.R = T, topk, E, bool(shared), R
        self.NE = E + (1 if shared else 0)       # segments written: offsets[0 .. NE]
        self.struct = L.Routes(*[t.data_ptr() for t in (self.counts, self.offsets, self.row_token, self.row_slot,
                                                          self.inv, self.uexp, self.nuniq, self.groups, self.ngroups,
                                                          self.row_expert)])


    def rows(self):
        """Dispatch rows in use (synchronises)."""
        return int(self.offsets[self.NE].item())


def dispatch(sel, E, first=0, shared=False, rows_per_group=8):
    """sel int64 [T, topk] -> RoutesBuf (stable by expert, token, slot)."""
    _need(sel, torch.int64, "sel")
    T, topk = sel.shape
    r = RoutesBuf(T, topk, E, shared, rows_per_group, sel.device)
    nws = lib().bmx_dispatch_workspace(T, topk, E)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=sel.device)
    check(lib().bmx_dispatch(_ptr(sel), T, topk, E, int(first), int(shared), rows_per_group, ctypes.byref(r.struct),
                             _ptr(ws), nws, _stream()), "bmx_dispatch")
    r._ws = ws
    return r


def route_dispatch(logits, topk, bias=None, n_group=1, topk_group=1, score=L.SCORE_SIGMOID, renorm=True, scale=1.0,
                   first=0, shared=False, rows_per_group=1):
    """Router + dispatch in one launch (T * topk <= 256) -> (sel, w, RoutesBuf)."""
    _need(logits, torch.float16, "logits")
    T, E = logits.shape
    if bias is not None:
        _need(bias, torch.float32, "bias")
    sel = torch.empty((T, topk), dtype=torch.int64, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.float16, device=logits.device)
    r = RoutesBuf(T, topk, E, shared, rows_per_group, logits.device)
    check(lib().bmx_route_dispatch(_ptr(logits), _ptr(bias), T, E, topk, n_group, topk_group, score, int(renorm),
                                   float(scale), int(first), int(shared), rows_per_group, _ptr(sel), _ptr(w),
                                   ctypes.byref(r.struct), _stream()), "bmx_route_dispatch")
    return sel, w, r


def moe_forward(desc, x, sel, w, path=L.PATH_AUTO, workspace=None):
    """Layer output fp32 [T, H] for x fp16 [T, H] and routes (sel, w)."""
    _need(x, torch.float16, "x"); _need(sel, torch.int64, "sel"); _need(w, torch.float16, "w")
    T = x.shape[0]
    out = torch.empty((T, desc.H), dtype=torch.float32, device=x.device)
    if T == 0:
        return out
    need = lib().bmx_moe_workspace(ctypes.byref(desc), T, path)
    if need == 0:
        check(1, "bmx_moe_workspace")
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    check(lib().bmx_moe_forward(ctypes.byref(desc), _ptr(x), T, _ptr(sel), _ptr(w), _ptr(out), _ptr(workspace),
                                workspace.numel(), path, _stream()), "bmx_moe_forward")
    return out


def moe_experts(desc, x, routes, path=L.PATH_AUTO, with_act=False):
    """Expert products on given routes -> (y_rows fp32 [R, H], act_rows fp16 [R, I] or None)."""
    T = x.shape[0]
    y = torch.zeros((max(routes.R, 1), desc.H), dtype=torch.float32, device=x.device)
    act = torch.zeros((max(routes.R, 1), desc.I), dtype=torch.float16, device=x.device) if with_act else None
    need = lib().bmx_experts_workspace(ctypes.byref(desc), T, path)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib().bmx_moe_experts(ctypes.byref(desc), _ptr(x), T, ctypes.byref(routes.struct), _ptr(y), _ptr(act),
                                _ptr(ws), need, path, _stream()), "bmx_moe_experts")
    return y, act


def combine(y_rows, routes, w, H):
    """bmx_combine: the weighted slot-ordered sum of the expert rows, the shared expert's row added with weight 1 (a
    layer with a gated shared expert is combined by its own layer call, which applies sigmoid(x . g))."""
    T, topk = routes.T, routes.topk
    out = torch.empty((T, H), dtype=torch.float32, device=y_rows.device)
    check(lib().bmx_combine(_ptr(y_rows), _ptr(routes.inv), _ptr(w), _ptr(routes.offsets), T, topk, H, routes.E,
                            int(routes.shared), _ptr(out), _stream()), "bmx_combine")
    return out


def moe_layer(desc, router, x, logits, path=L.PATH_AUTO, workspace=None):
    """Router + dispatch + experts + combine from logits fp16 [T, E] (None: projected from x with the router descriptor's
    weight) -> (out fp32 [T, H], sel, w)."""
    _need(x, torch.float16, "x")
    if logits is not None:
        _need(logits, torch.float16, "logits")
    T = x.shape[0]
    sel = torch.empty((T, desc.topk), dtype=torch.int64, device=x.device)
    w = torch.empty((T, desc.topk), dtype=torch.float16, device=x.device)
    out = torch.empty((T, desc.H), dtype=torch.float32, device=x.device)
    if T == 0:
        return out, sel, w
    need = lib().bmx_moe_layer_workspace(ctypes.byref(desc), T, path)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    check(lib().bmx_moe_layer(ctypes.byref(desc), ctypes.byref(router), _ptr(x), _ptr(logits), T, _ptr(sel), _ptr(w),
                              _ptr(out), _ptr(workspace), workspace.numel(), path, _stream()), "bmx_moe_layer")
    return out, sel, w


def moe_layer_stages(desc, router, x, logits, sel, w, out, workspace, stages, path=L.PATH_AUTO):
    """The stages in the mask `stages` (1 << STAGE_ROUTE, STAGE_PREP, STAGE_GATE_UP, STAGE_ACT, STAGE_DOWN,
    STAGE_COMBINE) of a moe_layer call into the caller's sel, w, out and workspace (at least
    bmx_moe_layer_workspace bytes); calls over the stages in that order equal one moe_layer call bit for bit."""
    _need(x, torch.float16, "x")
    if logits is not None:
        _need(logits, torch.float16, "logits")
    check(lib().bmx_moe_layer_stages(ctypes.byref(desc), ctypes.byref(router), _ptr(x), _ptr(logits), x.shape[0],
                                     _ptr(sel), _ptr(w), _ptr(out), _ptr(workspace), workspace.numel(), path, stages,
                                     _stream()), "bmx_moe_layer_stages")
