"""GPU edge cases of the layer call through the C ABI: empty batches, every pick dropped, the router's largest sizes,
expert counts that are not multiples of the wave width, and one pick per token — on every expert-products path."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS, REL_RMS = 1e-2, 1e-3
PATHS = [1, 3, 2, 4]       # GEMV, mid-size MFMA, prefill MFMA, split (GEMV or mid-size chosen on the device)


def say(*a):
    print(*a, flush=True)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)) / np.sqrt(np.mean(b.astype(np.float64) ** 2)))


def small_table(E, H, I, shared, seed, cuda):
    import bmx
    return bmx.ExpertTable.random(H, I, E, (2, 2, 2), shared=shared, seed=seed, device=cuda)


@pytest.mark.parametrize("path", PATHS)
def test_empty_batch(cuda, path):
    import bmx
    tab = small_table(8, 256, 128, True, 1, cuda)
    d = tab.desc(2)
    import ctypes
    lib = bmx.lib()
    need = lib.bmx_moe_workspace(ctypes.byref(d), 0, path)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=cuda)
    out = torch.zeros(16, dtype=torch.float32, device=cuda)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.bmx_moe_forward(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), 0, ctypes.c_void_p(ws.data_ptr()),
                             ctypes.c_void_p(ws.data_ptr()), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                             ws.numel(), path, s)
    torch.cuda.synchronize()
    assert rc == 0, bmx.lib().bmx_last_error()
    assert not torch.any(out)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("shared", [False, True])
def test_every_pick_dropped(cuda, oracle, path, shared):
    """Ids outside [first, first + E) drop their pick: the output is the shared expert alone (zero without one)."""
    import bmx
    E, H, I, T = 8, 256, 128, 5
    tab = small_table(E, H, I, shared, 2, cuda)
    x = torch.from_numpy(np.random.default_rng(3).standard_normal((T, H)).astype(np.float16)).to(cuda)
    sel = torch.tensor([[-1, E + 3], [E, 100], [-7, E], [E + 1, -2], [E, E]], dtype=torch.int64, device=cuda) + 4
    w = torch.full((T, 2), 0.5, dtype=torch.float16, device=cuda)
    out = bmx.ops.moe_forward(tab.desc(2, first=4), x, sel, w, path=path).cpu().numpy()
    if not shared:
        assert not np.any(out)
    else:
        want = oracle.moe_forward([None] * E, 4, tab.host_expert(E), H, I, x.cpu().numpy(), sel.cpu().numpy(),
                                  w.cpu().numpy())
        assert float(np.abs(out - want).max()) < MAX_ABS and rel_rms(out, want) < REL_RMS


@pytest.mark.parametrize("E,topk,T", [(1024, 32, 3), (100, 1, 7), (65, 5, 2), (1, 1, 4)])
def test_router_extreme_sizes(cuda, oracle, E, topk, T):
    import bmx
    rng = np.random.default_rng(E + topk)
    lg = (rng.standard_normal((T, E)) * 3).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    for score in (0, 1):
        b = bias if score == 1 else None
        sel, w = bmx.ops.router_topk(torch.from_numpy(lg).to(cuda), topk, torch.from_numpy(b).to(cuda) if b is not None
                                     else None, 1, 1, score, True, 1.5)
        osel, ow = oracle.router(lg, topk, b, 1, 1, score, True, 1.5)
        assert np.array_equal(sel.cpu().numpy(), osel)
        assert np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))


@pytest.mark.parametrize("path", PATHS)
def test_one_pick_per_token_odd_expert_count(cuda, oracle, path):
    """E = 100 experts (not a multiple of 64), top-1 softmax routing, 33 tokens, through the whole layer call."""
    import bmx
    E, H, I, T = 100, 384, 256, 33
    tab = small_table(E, H, I, False, 5, cuda)
    rng = np.random.default_rng(6)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy((rng.standard_normal((T, E)) * 2).astype(np.float16)).to(cuda)
    layer = bmx.MoELayer(tab, 1, score=bmx.SCORE_SOFTMAX, renorm=True, scale=1.0)
    out = layer.forward(x, lg, path=path)
    sel, w = layer.sel, layer.w
    torch.cuda.synchronize()
    used = sorted(set(int(e) for e in sel.cpu().numpy().ravel()))
    exps = [tab.host_expert(e) if e in used else None for e in range(E)]
    want = oracle.moe_forward(exps, 0, None, H, I, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy())
    got = out.cpu().numpy()
    say("top-1 path", path, "max_abs", float(np.abs(got - want).max()), "rel", rel_rms(got, want))
    assert float(np.abs(got - want).max()) < MAX_ABS and rel_rms(got, want) < REL_RMS


@pytest.mark.parametrize("path", PATHS)
def test_run_single_expert(cuda, oracle, path):
    """MoELayer.run_single_expert (the reference's per-expert hook, engine/tiers.py:597-605): expert e's output rows for
    given inputs against the oracle's expert forward, on every path; a layer with a shared expert (left out here)."""
    import bmx
    E, H, I, n = 6, 256, 128, 7
    tab = small_table(E, H, I, True, 31, cuda)
    layer = bmx.MoELayer(tab, 2, first=3)
    x = torch.from_numpy(np.random.default_rng(8).standard_normal((n, H)).astype(np.float16)).to(cuda)
    for e in (0, 4):
        y = torch.full((n, H), float("nan"), dtype=torch.float32, device=cuda)
        got = layer.run_single_expert(y, e, x, path).cpu().numpy()
        want = np.stack([oracle.expert_forward(tab.host_expert(e), H, I, x[i].cpu().numpy())[0] for i in range(n)])
        assert float(np.abs(got - want).max()) < MAX_ABS and rel_rms(got, want) < REL_RMS, (e, path)
        assert torch.equal(layer.run_single_expert_dq(torch.empty_like(y), e, x, path), y)
    with pytest.raises(ValueError):
        layer.run_single_expert(torch.empty((n, H), dtype=torch.float32, device=cuda), E, x)
