"""The split path (BMX_PATH_SPLIT) on the GPU, through the C ABI: one layer call whose experts with at least
BMX_SPLIT_MIN_ROWS rows run on the mid-size MFMA kernels and the rest on the decode GEMVs, chosen on the device from the
dispatch's row counts.

Checks: on routes that mix heavy and light experts (and a heavy shared expert), every expert row of the split path is
bit-identical to the GEMV path's row when its expert is light and to the mid-size path's row when it is heavy; the layer
output is within 1e-2 max-abs / 1e-3 relative RMS of the oracle for thresholds that send every expert to one kernel, to
the other, or split them; the staged gate / up stages of a slot-table call (resident experts, then the admitted ones)
give the same bits as the resident layer."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS, REL_RMS = 1e-2, 1e-3


def say(*a):
    print(*a, flush=True)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)) / np.sqrt(np.mean(b.astype(np.float64) ** 2)))


def mixed_routes(T, topk, E, seed):
    """[T, topk] picks: expert 3 in every token, expert 7 in 10 tokens, expert 11 in 4, expert 20 in 3, the rest spread
    (distinct per token)."""
    rng = np.random.default_rng(seed)
    sel = np.zeros((T, topk), np.int64)
    for t in range(T):
        fixed = [3] + ([7] if t < 10 else []) + ([11] if t % 4 == 0 else []) + ([20] if t in (1, 2, 5) else [])
        rest = [e for e in rng.permutation(E).tolist() if e not in (3, 7, 11, 20)][:topk - len(fixed)]
        sel[t] = rng.permutation(fixed + rest)
    return sel


# (BMX_SPLIT_RATIO, BMX_SPLIT_MIN_ROWS, which experts are heavy): per expert by its rows; every expert (the call's rows
# per expert reach the ratio); none
MODES = [("1000", "4", "rows"), ("0.5", "1000", "all"), ("1000", "1000", "none")]


@pytest.mark.parametrize("ratio,min_rows,heavy", MODES, ids=[m[2] for m in MODES])
@pytest.mark.parametrize("cfg,T,E", [("c5", 16, 64), ("c2", 16, 48), ("c2", 9, 32)])
def test_split_rows_follow_their_kernel(cuda, monkeypatch, cfg, T, E, ratio, min_rows, heavy):
    import bmx
    from bmx import synth
    L = bmx._lib
    c = synth.CONFIGS[cfg]
    tab = synth.table(cfg, seed=61, device=cuda, E=E)
    x, _, _ = synth.inputs(cfg, T=T, seed=62, device=cuda)
    topk = c["topk"]
    sel = torch.from_numpy(mixed_routes(T, topk, E, 63)).to(cuda)
    desc = tab.desc(topk)
    monkeypatch.setenv("BMX_SPLIT_MIN_ROWS", min_rows)
    monkeypatch.setenv("BMX_SPLIT_RATIO", ratio)
    rows = {}
    for name, path in (("split", L.PATH_SPLIT), ("decode", L.PATH_DECODE), ("mid", L.PATH_MID)):
        r = bmx.ops.dispatch(sel, E, 0, tab.has_shared, bmx.lib().bmx_rows_per_group(T, topk, path))
        say("split rows", cfg, T, E, name)
        y, _ = bmx.ops.moe_experts(desc, x, r, path)
        rows[name] = (y.cpu().numpy(), r)
    torch.cuda.synchronize()
    r = rows["split"][1]
    counts, offs = r.counts.cpu().numpy(), r.offsets.cpu().numpy()
    nheavy = nlight = 0
    for e in range(E + (1 if tab.has_shared else 0)):
        r0, r1 = int(offs[e]), int(offs[e + 1])
        if r1 <= r0:
            continue
        is_heavy = heavy == "all" or (heavy == "rows" and counts[e] >= 4)
        ref = rows["mid" if is_heavy else "decode"][0]
        got = rows["split"][0]
        assert np.array_equal(got[r0:r1].view(np.uint32), ref[r0:r1].view(np.uint32)), (cfg, e, int(counts[e]))
        if is_heavy:
            nheavy += 1
        else:
            nlight += 1
    say("split rows", cfg, T, E, heavy, "heavy experts", nheavy, "light experts", nlight)
    if heavy == "rows":
        assert nheavy >= 3 and nlight >= 3
    else:
        assert (nlight if heavy == "all" else nheavy) == 0


@pytest.mark.parametrize("thr,ratio", [("1", "1000"), ("4", "1000"), ("1000", "1000"), ("1000", "0.5"), ("32", "2.5")])
def test_split_layer_against_oracle(cuda, oracle, monkeypatch, thr, ratio):
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c2"]
    T, E = 12, 40
    tab = synth.table("c2", seed=71, device=cuda, E=E)
    x, _, _ = synth.inputs("c2", T=T, seed=72, device=cuda)
    sel = mixed_routes(T, c["topk"], E, 73)
    w = (np.random.default_rng(74).random((T, c["topk"])) * 0.5 + 0.1).astype(np.float16)
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], renorm=c["renorm"], scale=c["scale"])
    monkeypatch.setenv("BMX_SPLIT_MIN_ROWS", thr)
    monkeypatch.setenv("BMX_SPLIT_RATIO", ratio)
    say("split layer vs oracle, threshold", thr, "ratio", ratio)
    out = layer.run_bszN(x, torch.from_numpy(sel).to(cuda), torch.from_numpy(w).to(cuda), bmx.PATH_SPLIT).cpu().numpy()
    rows = [0, 3, 11]
    used = sorted(set(int(e) for e in sel[rows].ravel()))
    exps = [None] * E
    for e in used:
        exps[e] = tab.host_expert(e)
    want = oracle.moe_forward(exps, 0, tab.host_expert(E), tab.H, tab.I, x.cpu().numpy(), sel, w,
                              rows=np.asarray(rows, np.int32))
    got = out[rows]
    err, rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("split layer vs oracle, threshold", thr, "max_abs", err, "rel_rms", rel)
    assert err < MAX_ABS and rel < REL_RMS


@pytest.mark.parametrize("path_name", ["split", "auto"])
def test_split_path_with_slot_table_stages(cuda, monkeypatch, path_name):
    """A slot-table layer call of 16 tokens computes the resident experts' gate / up first and the admitted ones after
    their copies: on the split path on both kernels (the per-expert rule at 4 rows: experts 3 and 7 and the ones that
    happen to reach 4 rows on the mid-size kernel), on AUTO (the mid-size path at 16 tokens) on the MFMA kernels alone;
    outputs bit-identical to the same layer fully resident."""
    import bmx
    from bmx import synth
    from test_gpu_slots import small_layers
    E, H, I, topk, T = 24, 512, 256, 6, 16
    dev_layers = small_layers(2, E, H, I, 80, "device")
    host_layers = small_layers(2, E, H, I, 80, "host")
    slots = bmx.ExpertSlots(host_layers, 10, maxj=4)
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    st = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(2)]
    rf = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(2)]
    monkeypatch.setenv("BMX_SPLIT_MIN_ROWS", "4")
    monkeypatch.setenv("BMX_SPLIT_RATIO", "1000")
    path = bmx.PATH_SPLIT if path_name == "split" else bmx.PATH_AUTO
    if path_name == "auto":
        assert bmx.lib().bmx_resolve_path(T, topk, path) == bmx.PATH_MID
    for step in range(6):
        li = step % 2
        x = torch.from_numpy(np.random.default_rng(90 + step).standard_normal((T, H)).astype(np.float16)).cuda()
        sel = torch.from_numpy(mixed_routes(T, topk, E, 95 + step)).cuda()
        w = torch.from_numpy((np.random.default_rng(99 + step).random((T, topk)) + 0.2).astype(np.float16)).cuda()
        m = st[li]
        sg, wg, _ = m.layer(li, sel, w, x, T)
        out = m.run_bszN(x, sg, wg, path)
        want = rf[li].run_bszN(x, sel, w, path)
        torch.cuda.synchronize()
        say(path_name, "slot-table step", step, "layer", li, "max diff", float((out - want).abs().max()))
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), step
