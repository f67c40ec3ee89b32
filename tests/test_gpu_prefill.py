"""GPU parity of the MFMA (prefill) expert-product path against the oracle, through the C ABI.

Same bars as the decode path: layer outputs within 1e-2 max-abs and 1e-3 relative RMS of the oracle (exact accumulation
at exllamav3's rounding points). The full 8192-token layer is checked on sampled tokens (a token's output depends only
on its own routes) and through exact size-independent properties."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS, REL_RMS = 1e-2, 1e-3
PREFILL, DECODE, MID = 2, 1, 3


def say(*a):
    print(*a, flush=True)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)) / np.sqrt(np.mean(b.astype(np.float64) ** 2)))


def oracle_layer(oracle, tab, x, sel, w, rows):
    used = sorted(set(int(e) for e in sel[rows].ravel() if 0 <= e < tab.E))
    exps = [None] * tab.E
    for e in used:
        exps[e] = tab.host_expert(e)
    shared = tab.host_expert(tab.E) if tab.has_shared else None
    return oracle.moe_forward(exps, 0, shared, tab.H, tab.I, x, sel, w, rows=np.asarray(rows, np.int32))


def make_layer(cfgname, E, seed, cuda, T, H=None, I=None):
    import bmx
    from bmx import synth
    c = synth.CONFIGS[cfgname]
    tab = synth.table(cfgname, seed=seed, device=cuda, E=E, H=H, I=I)
    x, lg, bias = synth.inputs(cfgname, T=T, seed=seed + 1, device=cuda)
    if H is not None:
        x = x[:, :H].contiguous()
    lg = lg[:, :E].contiguous()
    if bias is not None:
        bias = bias[:E].contiguous()
    full = E == c["E"]
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], bias=bias, n_group=c["n_group"] if full else 1,
                         topk_group=c["topk_group"] if full else 1, renorm=c["renorm"], scale=c["scale"])
    return tab, layer, x, lg


PF_LAYERS = [
    # name, config, E, T, H, I, oracle rows
    ("c3 shape E32 T64", "c3", 32, 64, None, None, [0, 1, 17, 40, 63]),
    ("c2 shape E16 T40 shared", "c2", 16, 40, None, None, [0, 13, 39]),
    ("c1 T8 K4", "c1", 64, 8, None, None, None),
    ("c5 T16 K2/K2.5", "c5", 384, 16, None, None, [0, 7, 15]),
    ("odd blocks H384 I256", "c2", 8, 24, 384, 256, [0, 11, 23]),
    # AUTO's path up to 2,048 routed rows: many 32-row groups per expert
    ("c3 shape E64 T300", "c3", 64, 300, None, None, [0, 150, 299]),
    ("c2 shared E48 T200", "c2", 48, 200, None, None, [0, 99, 199]),
]


@pytest.mark.parametrize("name,cfgname,E,T,H,I,rows", PF_LAYERS, ids=[l[0] for l in PF_LAYERS])
def test_prefill_layer_parity(cuda, oracle, name, cfgname, E, T, H, I, rows):
    say("prefill", name, "build")
    tab, layer, x, lg = make_layer(cfgname, E, 11, cuda, T, H, I)
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    say("prefill", name, "run")
    out = layer.run_bszN(x, sel, w, path=PREFILL).cpu().numpy()
    dec = layer.run_bszN(x, sel, w, path=DECODE).cpu().numpy()
    fused = layer.forward(x, lg, path=PREFILL).cpu().numpy()
    assert np.array_equal(fused, out)
    rows = list(range(T)) if rows is None else rows
    say("prefill", name, "oracle rows", rows)
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(), rows)
    got = out[rows]
    err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("prefill", name, "max_abs", err_abs, "rel_rms", err_rel, "|out| rms", float(np.sqrt(np.mean(want ** 2))))
    assert err_abs < MAX_ABS and err_rel < REL_RMS
    # the two paths differ only in fp32 summation order
    assert float(np.abs(out - dec).max()) < MAX_ABS and rel_rms(out, dec.astype(np.float64)) < REL_RMS
    # deterministic
    assert np.array_equal(out, layer.run_bszN(x, sel, w, path=PREFILL).cpu().numpy())


def test_prefill_expert_rows_match_decode(cuda):
    """y rows of every dispatch row (bmx_moe_experts) from the MFMA path against the GEMV path."""
    import bmx
    tab, layer, x, lg = make_layer("c3", 24, 21, cuda, 48)
    sel, w = layer.routing_fn(48, None, x, {"logits": lg})
    d = tab.desc(6)
    say("prefill rows: dispatch")
    rp = bmx.ops.dispatch(sel, tab.E, 0, False, bmx.lib().bmx_rows_per_group(48, 6, PREFILL))
    rd = bmx.ops.dispatch(sel, tab.E, 0, False, bmx.lib().bmx_rows_per_group(48, 6, DECODE))
    yp, ap = bmx.ops.moe_experts(d, x, rp, path=PREFILL, with_act=True)
    yd, ad = bmx.ops.moe_experts(d, x, rd, path=DECODE, with_act=True)
    torch.cuda.synchronize()
    n = rp.rows()
    assert n == 48 * 6
    assert torch.equal(rp.row_token, rd.row_token)
    yp, yd = yp[:n].cpu().numpy(), yd[:n].cpu().numpy()
    ap, ad = ap[:n].cpu().numpy().astype(np.float32), ad[:n].cpu().numpy().astype(np.float32)
    say("prefill rows: y max diff", float(np.abs(yp - yd).max()), "act max diff", float(np.abs(ap - ad).max()))
    assert rel_rms(yp, yd.astype(np.float64)) < REL_RMS
    assert rel_rms(ap, ad.astype(np.float64)) < REL_RMS


def test_prefill_c3_full_size(cuda, oracle):
    """The full c3 layer (384 experts, H 4096, I 2048, K 2 / 3, 8192 tokens, Zipf routing) on the MFMA path: sampled
    tokens against the oracle; doubling every routing weight doubles the output bit for bit; a second call repeats every
    bit; a dropped pick (sentinel id first + E) equals the same pick with weight 0."""
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c3"]
    say("c3 full: build table")
    tab = synth.table("c3", seed=0, device=cuda)
    x, lg, _ = synth.inputs("c3", seed=0, device=cuda)
    T = x.shape[0]
    assert bmx.lib().bmx_resolve_path(T, 6, 0) == PREFILL
    layer = bmx.MoELayer(tab, 6, score=c["score"], n_group=8, topk_group=4, renorm=True, scale=c["scale"])
    say("c3 full: layer")
    out = layer.forward(x, lg)
    sel, w = layer.sel, layer.w
    torch.cuda.synchronize()
    rows = [0, 1, 777, 4096, 8191]
    say("c3 full: oracle rows", rows)
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(), rows)
    got = out.cpu().numpy()[rows]
    err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("c3 full: max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS
    d = tab.desc(6)
    a = bmx.ops.moe_forward(d, x, sel, w)
    assert torch.equal(a, out)
    say("c3 full: properties")
    b = bmx.ops.moe_forward(d, x, sel, (w * 2).contiguous())
    assert torch.equal(b, out * 2)
    s2 = sel.clone()
    s2[::7, 2] = tab.E
    w2 = w.clone()
    w2[::7, 2] = 0
    assert torch.equal(bmx.ops.moe_forward(d, x, s2, w), bmx.ops.moe_forward(d, x, sel, w2))


MID_LAYERS = [
    # name, config, E, T, H, I, oracle rows
    ("c5 T16 K2/K2.5", "c5", 384, 16, None, None, [0, 7, 15]),
    ("c2 T8 shared", "c2", 288, 8, None, None, [0, 5]),
    ("c3 shape E24 T40", "c3", 24, 40, None, None, [0, 17, 39]),
    ("c1 T4 K4", "c1", 64, 4, None, None, None),
    ("odd blocks H384 I256", "c2", 8, 24, 384, 256, [0, 11, 23]),
]


@pytest.mark.parametrize("name,cfgname,E,T,H,I,rows", MID_LAYERS, ids=[l[0] for l in MID_LAYERS])
def test_mid_layer_parity(cuda, oracle, name, cfgname, E, T, H, I, rows):
    """The mid-size MFMA path (groups of 32 rows, k-splits) against the oracle and the GEMV path."""
    import bmx
    say("mid", name, "build")
    tab, layer, x, lg = make_layer(cfgname, E, 13, cuda, T, H, I)
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    say("mid", name, "run")
    out = layer.run_bszN(x, sel, w, path=MID).cpu().numpy()
    dec = layer.run_bszN(x, sel, w, path=DECODE).cpu().numpy()
    fused = layer.forward(x, lg, path=MID).cpu().numpy()
    assert np.array_equal(fused, out)
    assert bmx.lib().bmx_rows_per_group(T, layer.num_experts_per_tok, MID) == 32
    if T >= 8:
        assert bmx.lib().bmx_resolve_path(T, layer.num_experts_per_tok, 0) == MID
    rows = list(range(T)) if rows is None else rows
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(), rows)
    got = out[rows]
    err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("mid", name, "max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS
    assert float(np.abs(out - dec).max()) < MAX_ABS and rel_rms(out, dec.astype(np.float64)) < REL_RMS
    assert np.array_equal(out, layer.run_bszN(x, sel, w, path=MID).cpu().numpy())


def test_mid_experts_rows_and_properties(cuda):
    """Every dispatch row's expert output on the mid path against the GEMV path; weights x 2 -> output x 2 bit for bit."""
    import bmx
    tab, layer, x, lg = make_layer("c5", 384, 23, cuda, 16)
    sel, w = layer.routing_fn(16, None, x, {"logits": lg})
    d = tab.desc(6)
    rm = bmx.ops.dispatch(sel, tab.E, 0, False, bmx.lib().bmx_rows_per_group(16, 6, MID))
    rd = bmx.ops.dispatch(sel, tab.E, 0, False, bmx.lib().bmx_rows_per_group(16, 6, DECODE))
    ym, am = bmx.ops.moe_experts(d, x, rm, path=MID, with_act=True)
    yd, ad = bmx.ops.moe_experts(d, x, rd, path=DECODE, with_act=True)
    torch.cuda.synchronize()
    n = rm.rows()
    assert n == 96 and torch.equal(rm.row_token, rd.row_token)
    assert rel_rms(ym[:n].cpu().numpy(), yd[:n].cpu().numpy().astype(np.float64)) < REL_RMS
    a = bmx.ops.moe_forward(d, x, sel, w, path=MID)
    b = bmx.ops.moe_forward(d, x, sel, (w * 2).contiguous(), path=MID)
    assert torch.equal(b, a * 2)


def forced_picks(T, topk, E, plan, seed):
    """sel [T, topk]: slot k of token t picks plan[k](t); weights random positive"""
    sel = np.array([[plan[k](t) for k in range(topk)] for t in range(T)], np.int64)
    assert all(len(set(r)) == topk for r in sel.tolist())
    w = (np.random.default_rng(seed).random((T, topk)) + 0.25).astype(np.float16)
    return sel, w


PAIR_CASES = [
    # name, H, I, fmts, shared, T, topk, E, slot plans: expert 0 takes 330 rows (groups 128 128 74: a pair and a
    # single), expert 1 260 (128, 128, 4: a pair and a single), expert 2 70; odd block counts (H 384, I 384)
    ("odd blocks, pair + single, shared", 384, 384, (2, 1, 3), True, 330, 2, 6,
     (lambda t: 0, lambda t: 1 if t < 260 else 2)),
    # expert 0: 600 rows (five groups: two pairs and a single), expert 1: 300, the rest spread
    ("two pairs, K4", 1024, 512, (3, 3, 3), False, 600, 3, 9,
     (lambda t: 0, lambda t: 1 if t < 300 else 2 + t % 7, lambda t: 3 + t % 6 if t < 300 else 2 + (t + 3) % 7)),
]


@pytest.mark.parametrize("name,H,I,fmts,shared,T,topk,E,plan", PAIR_CASES, ids=[c[0] for c in PAIR_CASES])
def test_prefill_pairs(cuda, oracle, name, H, I, fmts, shared, T, topk, E, plan):
    """Consecutive 128-row groups of one expert run as one 256-row x 128-column tile (a pair): the same products as
    one tile per group (BMX_PF_PAIRS=0) bit for bit, and rows of both halves of a pair and of the single group after it
    within the oracle's tolerance."""
    import os
    import bmx
    tab = bmx.ExpertTable.random(H, I, E, fmts, shared=shared, seed=31, device=cuda)
    layer = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    g = torch.Generator(device=cuda)
    g.manual_seed(32)
    x = torch.randn((T, H), generator=g, device=cuda).half()
    sel_np, w_np = forced_picks(T, topk, E, plan, 33)
    sel, w = torch.from_numpy(sel_np).to(cuda), torch.from_numpy(w_np).to(cuda)
    say("pairs", name, "run")
    out = layer.run_bszN(x, sel, w, path=PREFILL).clone()
    os.environ["BMX_PF_PAIRS"] = "0"
    try:
        ref = layer.run_bszN(x, sel, w, path=PREFILL).clone()
    finally:
        os.environ.pop("BMX_PF_PAIRS", None)
    torch.cuda.synchronize()
    say("pairs", name, "max |pairs - singles|", float((out - ref).abs().max()))
    assert torch.equal(out, ref) and float(out.abs().max()) > 0
    rows = [0, 127, 128, 200, 255, 256, T - 1]
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel_np, w_np, rows)
    got = out.cpu().numpy()[rows]
    err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("pairs", name, "oracle rows", rows, "max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS


def test_prefill_wide_topk_dropped_picks(cuda, oracle):
    """The prefill path's token-major rotation takes a token's slots 16 at a time: 16 picks plus the shared expert need
    a second pass, and picks with ids outside the layer's experts have no row (their slots are skipped). Every token
    against the oracle."""
    import bmx
    H, I, E, T, topk = 512, 256, 40, 24, 16
    tab = bmx.ExpertTable.random(H, I, E, (0, 3, 2), shared=True, seed=41, device=cuda)
    layer = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.5)
    g = torch.Generator(device=cuda)
    g.manual_seed(42)
    x = torch.randn((T, H), generator=g, device=cuda).half()
    lg = torch.randn((T, E), generator=g, device=cuda).half()
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    sel = sel.clone()
    for t, k in ((0, 3), (5, 0), (5, 15), (11, 7), (23, 15)):
        sel[t, k] = E + 3 if (t + k) % 2 else -2
    say("wide topk: run")
    out = layer.run_bszN(x, sel, w, path=PREFILL).cpu().numpy()
    sel_np, w_np = sel.cpu().numpy(), w.cpu().numpy()
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel_np, w_np, list(range(T)))
    err_abs, err_rel = float(np.abs(out - want).max()), rel_rms(out, want)
    say("wide topk: max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS
    # the dropped picks matter: the oracle without them differs
    kept = sel_np.copy()
    kept[0, 3] = (kept[0, 3] + 1) % E
    assert rel_rms(oracle_layer(oracle, tab, x.cpu().numpy(), kept, w_np, [0]), want[:1]) > 10 * REL_RMS
