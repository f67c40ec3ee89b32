"""bmx_moe_layer_scratch, the layer call that allocates nothing (its workspace is the library's own device array),
against bmx_moe_layer with a caller workspace, through the C ABI: routes and outputs bit-identical on two calls in a
row, the second on a smaller batch (the array keeps the first call's contents); a call whose workspace exceeds the
array is refused on the host."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def layer_call(layer, x, lg, path, scratch):
    import bmx
    lib = bmx.lib()
    T, k, H = x.shape[0], layer.num_experts_per_tok, layer.hidden_size
    sel = torch.full((T, k), -5, dtype=torch.int64, device=x.device)
    w = torch.zeros((T, k), dtype=torch.float16, device=x.device)
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device=x.device)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    d, r = ctypes.byref(layer.desc), ctypes.byref(layer.router)
    if scratch:
        rc = lib.bmx_moe_layer_scratch(d, r, P(x), P(lg), T, P(sel), P(w), P(out), path, s)
        bmx._lib.check(rc, "bmx_moe_layer_scratch")
    else:
        need = lib.bmx_moe_layer_workspace(d, T, path)
        ws = torch.full((max(need, 1),), 0xA5, dtype=torch.uint8, device=x.device)    # no zero start assumed
        rc = lib.bmx_moe_layer(d, r, P(x), P(lg), T, P(sel), P(w), P(out), P(ws), ws.numel(), path, s)
        bmx._lib.check(rc, "bmx_moe_layer")
    return sel, w, out


def make_layer(cfg, E, cuda):
    import bmx
    from bmx import synth
    c = synth.CONFIGS[cfg]
    tab = synth.table(cfg, seed=21, device=cuda, E=E)
    _, _, bias = synth.inputs(cfg, T=1, seed=22, device=cuda)
    if bias is not None:
        bias = bias[:E].contiguous()
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], bias=bias, n_group=c["n_group"], topk_group=c["topk_group"],
                         renorm=c["renorm"], scale=c["scale"])
    return layer


@pytest.mark.parametrize("cfg,E,T1,T2,path", [("c2", 288, 8, 1, 0), ("c2", 64, 16, 3, 3), ("c5", 64, 16, 2, 3),
                                              ("c1", 64, 4, 1, 1), ("c3", 64, 24, 5, 2), ("c5", 384, 16, 2, 0),
                                              ("c2", 288, 20, 16, 4)])
def test_scratch_layer_matches_workspace_layer(cuda, cfg, E, T1, T2, path):
    from bmx import synth
    layer = make_layer(cfg, E, cuda)
    for call, T in enumerate((T1, T2)):
        x, lg, _ = synth.inputs(cfg, T=T, seed=30 + call, device=cuda)
        lg = lg[:, :E].contiguous()
        say("scratch layer", cfg, "E", E, "call", call, "T", T, "path", path)
        a = layer_call(layer, x, lg, path, scratch=True)
        b = layer_call(layer, x, lg, path, scratch=False)
        torch.cuda.synchronize()
        for u, v, name in zip(a, b, ("sel", "w", "out")):
            assert torch.equal(u, v), (cfg, call, name)
        assert torch.isfinite(a[2]).all()


def test_scratch_layer_refuses_oversized_calls(cuda):
    import bmx
    layer = make_layer("c2", 64, cuda)
    lib = bmx.lib()
    T = 8192
    need = lib.bmx_moe_layer_workspace(ctypes.byref(layer.desc), T, bmx.PATH_PREFILL)
    assert need > (64 << 20)
    dummy = torch.zeros(16, dtype=torch.uint8, device=cuda)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.bmx_moe_layer_scratch(ctypes.byref(layer.desc), ctypes.byref(layer.router), P(dummy), P(dummy), T,
                                   P(dummy), P(dummy), P(dummy), bmx.PATH_PREFILL, s)
    assert rc == bmx._lib.BMX_ERR_WORKSPACE
    assert "scratch array" in lib.bmx_last_error().decode()


@pytest.mark.parametrize("cfg,E", [("c2", 288), ("c1", 64)])
def test_scratch_layer_against_oracle(cuda, oracle, cfg, E):
    """One one-token scratch call (the full C2 / C1 layer) against the oracle directly: 1e-2 max-abs, 1e-3 relative
    RMS, with the picks and weights the call wrote."""
    from bmx import synth
    layer = make_layer(cfg, E, cuda)
    x, lg, _ = synth.inputs(cfg, T=1, seed=40, device=cuda)
    lg = lg[:, :E].contiguous()
    say("scratch layer vs oracle", cfg, "E", E)
    sel, w, out = layer_call(layer, x, lg, 0, scratch=True)
    tab = layer.table
    s, wn = sel.cpu().numpy(), w.cpu().numpy()
    exps = [None] * tab.E
    for e in sorted(set(int(v) for v in s.ravel() if 0 <= v < tab.E)):
        exps[e] = tab.host_expert(e)
    shared = tab.host_expert(tab.E) if tab.has_shared else None
    want = oracle.moe_forward(exps, 0, shared, tab.H, tab.I, x.cpu().numpy(), s, wn, rows=np.arange(1, dtype=np.int32))
    got = out.cpu().numpy()
    err = float(np.abs(got - want).max())
    rel = float(np.sqrt(np.mean((got.astype(np.float64) - want) ** 2)) / np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    say("scratch layer vs oracle", cfg, "max_abs", err, "rel_rms", rel)
    assert err < 1e-2 and rel < 1e-3
