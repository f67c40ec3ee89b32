"""GPU parity of the HIP path against the oracle on identical seeded inputs, through the C ABI.

Bars: dequantised fp16 weights, router indices and dispatch order bit-exact; layer outputs within 1e-2 max-abs and
1e-3 relative RMS of the oracle (exact accumulation at exllamav3's rounding points)."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MAX_ABS, REL_RMS = 1e-2, 1e-3


def say(*a):
    print(*a, flush=True)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)) / np.sqrt(np.mean(b.astype(np.float64) ** 2)))


# ---- dequant ----------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_dequant_bitexact(cuda, oracle, fmt):
    import bmx
    rng = np.random.default_rng(100 + fmt)
    k, n = 256, 384
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * bmx.TILE_BYTES[fmt], dtype=np.uint8)
    say("dequant fmt", fmt, k, n)
    got = bmx.ops.dequant(torch.from_numpy(tr).to(cuda), fmt, k, n).cpu().numpy()
    assert np.array_equal(got.view(np.uint16), oracle.dequant(tr, fmt, k, n).view(np.uint16))


def test_dequant_golden_k3(cuda):
    import bmx
    g = np.load(os.path.join(GOLD, "k3_tiles.npz"))
    k, n = int(g["k"]), int(g["n"])
    got = bmx.ops.dequant(torch.from_numpy(g["trellis"]).to(cuda), 2, k, n).cpu().numpy()
    assert np.array_equal(got.view(np.uint16), g["w"].view(np.uint16))


def test_dequant_covers_every_state(cuda, oracle):
    """A 1M-weight K 3 matrix through the GPU decode, bit-exact, whose tiles hold every one of the 65536 states."""
    import bmx
    rng = np.random.default_rng(77)
    k, n = 1024, 1024
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * 96, dtype=np.uint8)
    states = oracle.np_tile_states(tr.reshape(-1, 96), 2)
    assert np.unique(states).size == 65536
    got = bmx.ops.dequant(torch.from_numpy(tr).to(cuda), 2, k, n).cpu().numpy()
    assert np.array_equal(got.view(np.uint16), oracle.dequant(tr, 2, k, n).view(np.uint16))


# ---- router -----------------------------------------------------------------------------------------------------------

ROUTERS = [
    ("c1 softmax", dict(E=64, topk=8, score=0, renorm=True, scale=1.0, n_group=1, topk_group=1, bias=False)),
    ("softmax no renorm", dict(E=64, topk=4, score=0, renorm=False, scale=1.0, n_group=1, topk_group=1, bias=False)),
    ("c2 sigmoid+bias", dict(E=288, topk=8, score=1, renorm=True, scale=2.5, n_group=1, topk_group=1, bias=True)),
    ("c3 groups", dict(E=384, topk=6, score=1, renorm=True, scale=2.5, n_group=8, topk_group=4, bias=True)),
    ("sigmoid raw", dict(E=160, topk=6, score=1, renorm=False, scale=1.0, n_group=1, topk_group=1, bias=False)),
    # group limit: lanes per group 8 / 16 / 1 (one expert per group), and the general path (G = 3 and G = 2)
    ("groups E256 G8", dict(E=256, topk=8, score=1, renorm=True, scale=2.5, n_group=8, topk_group=4, bias=True)),
    ("groups E256 G4", dict(E=256, topk=8, score=1, renorm=True, scale=1.0, n_group=4, topk_group=2, bias=True)),
    ("groups E64 G64", dict(E=64, topk=4, score=1, renorm=True, scale=1.0, n_group=64, topk_group=8, bias=True)),
    ("groups E96 G3", dict(E=96, topk=4, score=1, renorm=True, scale=1.0, n_group=3, topk_group=2, bias=True)),
    ("groups E128 G2", dict(E=128, topk=6, score=0, renorm=True, scale=1.0, n_group=2, topk_group=1, bias=False)),
    ("top2 E64", dict(E=64, topk=2, score=1, renorm=True, scale=1.0, n_group=1, topk_group=1, bias=True)),
]


@pytest.mark.parametrize("name,cfg", ROUTERS, ids=[r[0] for r in ROUTERS])
@pytest.mark.parametrize("T", [1, 8, 513])
def test_router_bitexact(cuda, oracle, name, cfg, T):
    import bmx
    rng = np.random.default_rng(T)
    E = cfg["E"]
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float16)
    lg[0, :4] = lg[0, 4]                                  # ties
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if cfg["bias"] else None
    say("router", name, "T", T)
    sel, w = bmx.ops.router_topk(torch.from_numpy(lg).to(cuda), cfg["topk"],
                                 torch.from_numpy(bias).to(cuda) if bias is not None else None, cfg["n_group"],
                                 cfg["topk_group"], cfg["score"], cfg["renorm"], cfg["scale"], first=11)
    osel, ow = oracle.router(lg, cfg["topk"], bias, cfg["n_group"], cfg["topk_group"], cfg["score"], cfg["renorm"],
                             cfg["scale"], first=11)
    assert np.array_equal(sel.cpu().numpy(), osel)
    gw = w.cpu().numpy()
    if cfg["score"] == 0 and not cfg["renorm"]:
        assert np.allclose(gw.astype(np.float32), ow.astype(np.float32), rtol=2e-3)   # sum over E in parallel order
    else:
        assert np.array_equal(gw.view(np.uint16), ow.view(np.uint16))


@pytest.mark.parametrize("name,cfg", [r for r in ROUTERS if r[0] in ("c2 sigmoid+bias", "c3 groups", "c1 softmax")],
                         ids=["c1", "c2", "c3"])
def test_router_ties(cuda, oracle, name, cfg):
    """Equal values decide by lower index: every logit equal (more candidates than are ranked directly: the bitwise
    search), runs of equal logits at the boundary, and two values only."""
    import bmx
    E = cfg["E"]
    rng = np.random.default_rng(5)
    rows = [np.full(E, 0.5), np.repeat(rng.standard_normal(E // 8), 8)[:E], np.where(np.arange(E) % 3 == 0, 1.0, -1.0),
            np.round(rng.standard_normal(E) * 4) / 4]
    lg = np.stack(rows).astype(np.float16)
    say("router ties", name)
    sel, w = bmx.ops.router_topk(torch.from_numpy(lg).to(cuda), cfg["topk"], None, cfg["n_group"], cfg["topk_group"],
                                 cfg["score"], cfg["renorm"], cfg["scale"])
    osel, ow = oracle.router(lg, cfg["topk"], None, cfg["n_group"], cfg["topk_group"], cfg["score"], cfg["renorm"],
                             cfg["scale"])
    assert np.array_equal(sel.cpu().numpy(), osel)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))


def test_router_zipf_c3(cuda, oracle):
    import bmx
    from bmx import synth
    lg = synth.zipf_logits(2048, 384, 1.1, seed=3)
    sel, w = bmx.ops.router_topk(torch.from_numpy(lg).to(cuda), 6, None, 8, 4, 1, True, 2.5)
    osel, ow = oracle.router(lg, 6, None, 8, 4, 1, True, 2.5)
    assert np.array_equal(sel.cpu().numpy(), osel)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))


# ---- dispatch ---------------------------------------------------------------------------------------------------------

def _check_dispatch(r, d, T, topk, E, shared, rpg):
    n = int(d["offsets"][-1])
    assert np.array_equal(r.counts.cpu().numpy()[:len(d["counts"])], d["counts"])
    assert np.array_equal(r.offsets.cpu().numpy()[:len(d["offsets"])], d["offsets"])
    assert np.array_equal(r.row_token.cpu().numpy()[:n], d["row_token"])
    assert np.array_equal(r.row_slot.cpu().numpy()[:n], d["row_slot"])
    assert np.array_equal(r.inv.cpu().numpy()[:T * topk].reshape(T, topk), d["inv"])
    nu = int(r.nuniq.item())
    assert nu == d["nuniq"] and np.array_equal(r.uexp.cpu().numpy()[:nu], d["uexp"])
    groups = r.groups.cpu().numpy().reshape(-1, 3)[:int(r.ngroups.item())]
    want = []
    for e in d["uexp"]:
        c, o = int(d["counts"][e]), int(d["offsets"][e])
        for q in range(0, c, rpg):
            want.append([e, o + q, min(rpg, c - q)])
    assert groups.tolist() == want
    rexp = r.row_expert.cpu().numpy()[:n]
    assert np.array_equal(rexp, np.searchsorted(d["offsets"], np.arange(n), side="right") - 1)


@pytest.mark.parametrize("T,topk,E,shared,rpg", [(1, 8, 288, True, 1), (8, 8, 288, True, 8), (16, 6, 384, False, 8),
                                                 (600, 6, 384, False, 8), (8192, 6, 384, False, 128),
                                                 (3000, 8, 64, True, 32)])
def test_dispatch_bitexact(cuda, oracle, T, topk, E, shared, rpg):
    import bmx
    from bmx import synth
    lg = synth.zipf_logits(T, E, 1.1, seed=T)
    sel = np.argsort(-lg.astype(np.float32), axis=1, kind="stable")[:, :topk].astype(np.int64)
    if T > 4:
        sel[2, 1] = E          # dropped (sentinel first + E)
        sel[3, 0] = -1         # masked
    say("dispatch", T, topk, E, shared, rpg)
    r = bmx.ops.dispatch(torch.from_numpy(sel).to(cuda), E, 0, shared, rpg)
    torch.cuda.synchronize()
    _check_dispatch(r, oracle.dispatch(sel, E, 0, shared), T, topk, E, shared, rpg)


RD_CASES = [("c2 T1 shared", "c2 sigmoid+bias", 1, True, 1), ("c2 T8 shared", "c2 sigmoid+bias", 8, True, 8),
            ("c1 T1", "c1 softmax", 1, False, 1), ("c3 groups T2", "c3 groups", 2, False, 2),
            ("c3 groups T16", "c3 groups", 16, False, 8), ("c2 T32 shared", "c2 sigmoid+bias", 32, True, 8),
            ("softmax raw T7", "softmax no renorm", 7, True, 4), ("groups T64", "groups E64 G64", 64, True, 8),
            ("top2 T100 workgroup", "top2 E64", 100, True, 8), ("top2 T128 workgroup", "top2 E64", 128, False, 1)]


@pytest.mark.parametrize("name,router,T,shared,rpg", RD_CASES, ids=[c[0] for c in RD_CASES])
def test_route_dispatch_bitexact(cuda, oracle, name, router, T, shared, rpg):
    """The one-launch router + dispatch (the counting sort by one wave up to 64 tokens, by the workgroup beyond, at
    most 256 picks) against the oracle's router and counting sort, bit for bit."""
    import bmx
    cfg = dict(ROUTERS)[router]
    rng = np.random.default_rng(100 + T)
    E, topk = cfg["E"], cfg["topk"]
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float16)
    lg[0, :4] = lg[0, 4]                                  # ties
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if cfg["bias"] else None
    say("route+dispatch", name)
    sel, w, r = bmx.ops.route_dispatch(torch.from_numpy(lg).to(cuda), topk,
                                       torch.from_numpy(bias).to(cuda) if bias is not None else None, cfg["n_group"],
                                       cfg["topk_group"], cfg["score"], cfg["renorm"], cfg["scale"], first=5,
                                       shared=shared, rows_per_group=rpg)
    torch.cuda.synchronize()
    osel, ow = oracle.router(lg, topk, bias, cfg["n_group"], cfg["topk_group"], cfg["score"], cfg["renorm"],
                             cfg["scale"], first=5)
    assert np.array_equal(sel.cpu().numpy(), osel)
    gw = w.cpu().numpy()
    if cfg["score"] == 0 and not cfg["renorm"]:
        assert np.allclose(gw.astype(np.float32), ow.astype(np.float32), rtol=2e-3)
    else:
        assert np.array_equal(gw.view(np.uint16), ow.view(np.uint16))
    _check_dispatch(r, oracle.dispatch(osel, E, 5, shared), T, topk, E, shared, rpg)


# ---- layer ------------------------------------------------------------------------------------------------------------

def oracle_layer(oracle, tab, x, sel, w, rows):
    used = sorted(set(int(e) for e in sel[rows].ravel() if 0 <= e < tab.E))
    exps = [None] * tab.E
    for e in used:
        exps[e] = tab.host_expert(e)
    shared = tab.host_expert(tab.E) if tab.has_shared else None
    return oracle.moe_forward(exps, 0, shared, tab.H, tab.I, x, sel, w, rows=np.asarray(rows, np.int32))


LAYERS = [
    ("c1 T1", "c1", 1, None, dict()),
    ("c2 T1", "c2", 1, None, dict()),
    ("c2 T8", "c2", 8, [0, 5], dict()),
    ("c3 shape T4", "c3", 4, [1, 3], dict()),
    ("c5 shape T16", "c5", 16, [0, 15], dict()),
    ("c2 E32 T3", "c2", 3, None, dict(E=32)),
]


@pytest.mark.parametrize("name,cfgname,T,rows,kw", LAYERS, ids=[l[0] for l in LAYERS])
def test_layer_parity(cuda, oracle, monkeypatch, name, cfgname, T, rows, kw):
    import bmx
    from bmx import synth
    c = synth.CONFIGS[cfgname]
    E = kw.get("E", c["E"])
    say("layer", name, "build table")
    tab = synth.table(cfgname, seed=1, device=cuda, E=E)
    x, lg, bias = synth.inputs(cfgname, T=T, seed=2, device=cuda)
    lg = lg[:, :E].contiguous()
    if bias is not None:
        bias = bias[:E].contiguous()
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], bias=bias, n_group=c["n_group"] if E == c["E"] else 1,
                         topk_group=c["topk_group"] if E == c["E"] else 1, renorm=c["renorm"], scale=c["scale"])
    say("layer", name, "forward")
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    out = layer.run_bszN(x, sel, w).cpu().numpy()
    fused = layer.forward(x, lg).cpu().numpy()          # router + dispatch + experts + combine in one library call
    assert torch.equal(layer.sel, sel) and torch.equal(layer.w, w)
    if T == 1:
        # one token: the gate / up GEMV routes it itself, with as many k-splits as start in one round. With the plan's
        # own split count forced, the one call equals the separate calls bit for bit (the routing and the dispatch inside
        # the GEMV are exact); by default it sums the splits in another order: within the layer tolerance.
        from bmx import cpu_lane
        monkeypatch.setenv("BMX_KS_GU", str(cpu_lane.decode_splits(layer.desc, 1)[0]))
        forced = layer.forward(x, lg).cpu().numpy()
        monkeypatch.delenv("BMX_KS_GU")
        assert np.array_equal(forced, out)
        assert np.abs(fused - out).max() < MAX_ABS and rel_rms(fused, out) < REL_RMS
    else:
        assert np.array_equal(fused, out)
    rows = list(range(T)) if rows is None else rows
    say("layer", name, "oracle rows", rows)
    want = oracle_layer(oracle, tab, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(), rows)
    # both the separate calls and the one-call layer (the path a one-token caller runs) against the oracle directly
    for what, res in (("separate calls", out), ("one call", fused)):
        got = res[rows]
        err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
        say("layer", name, what, "max_abs", err_abs, "rel_rms", err_rel, "|out| rms",
            float(np.sqrt(np.mean(want ** 2))))
        assert err_abs < MAX_ABS and err_rel < REL_RMS, what
    # deterministic: same bits on a second call
    out2 = layer.run_bszN(x, sel, w).cpu().numpy()
    assert np.array_equal(out, out2)


@pytest.mark.parametrize("cus", [16, 40, 80])
def test_one_token_layer_on_fewer_compute_units(cuda, oracle, monkeypatch, cus):
    """The one-token layer call takes its gate / up k-split count from the device's compute units: with the count
    overridden (another device or partition mode) the split count and the summation order change, and the output stays
    within the layer tolerance of the oracle."""
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c2"]
    tab = synth.table("c2", seed=1, device=cuda)
    x, lg, bias = synth.inputs("c2", T=1, seed=2, device=cuda)
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], bias=bias, n_group=c["n_group"], topk_group=c["topk_group"],
                         renorm=c["renorm"], scale=c["scale"])
    monkeypatch.setenv("BMX_CU_COUNT", str(cus))
    say("one-token layer, compute units", cus)
    got = layer.forward(x, lg).cpu().numpy()
    monkeypatch.delenv("BMX_CU_COUNT")
    want = oracle_layer(oracle, tab, x.cpu().numpy(), layer.sel.cpu().numpy(), layer.w.cpu().numpy(), [0])
    err_abs, err_rel = float(np.abs(got - want).max()), rel_rms(got, want)
    say("one-token layer, compute units", cus, "max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS


STAGED = [("c1 T1", "c1", 1, True), ("c2 T1", "c2", 1, False), ("c2 T1 projected", "c2", 1, True),
          ("c2 T8", "c2", 8, False), ("c3 shape T128", "c3", 128, True)]


@pytest.mark.parametrize("name,cfgname,T,project", STAGED, ids=[s[0] for s in STAGED])
@pytest.mark.parametrize("route_in_gemv", ["1", "0"])
def test_layer_stages_equal_one_call(cuda, monkeypatch, name, cfgname, T, project, route_in_gemv):
    """bmx_moe_layer_stages over the stages one call at a time, and in two halves, gives the one-call layer's out, sel
    and w bit for bit: with the one-token gate / up GEMV routing the token itself and without, with the router
    projection in the route stage (no logits given) and without."""
    import bmx
    from bmx import synth
    L = bmx._lib
    monkeypatch.setenv("BMX_ROUTE_IN_GEMV", route_in_gemv)
    c = synth.CONFIGS[cfgname]
    tab = synth.table(cfgname, seed=11, device=cuda, E=min(c["E"], 64))
    E = tab.E
    x, lg, bias = synth.inputs(cfgname, T=T, seed=12, device=cuda)
    lg = lg[:, :E].contiguous()
    bias = bias[:E].contiguous() if bias is not None else None
    rw = (torch.randn(E, tab.H, generator=torch.Generator().manual_seed(13)) * 0.02).half().to(cuda) if project else None
    layer = bmx.MoELayer(tab, c["topk"], score=c["score"], bias=bias, n_group=c["n_group"] if E == c["E"] else 1,
                         topk_group=c["topk_group"] if E == c["E"] else 1, renorm=c["renorm"], scale=c["scale"],
                         router_weight=rw)
    logits = None if project else lg
    say("stages", name, "route_in_gemv", route_in_gemv, "one call")
    out, sel, w = bmx.ops.moe_layer(layer.desc, layer.router, x, logits)
    need = L.lib().bmx_moe_layer_workspace(layer.desc, T, L.PATH_AUTO)
    one = [L.STAGE_ROUTE, L.STAGE_PREP, L.STAGE_GATE_UP, L.STAGE_ACT, L.STAGE_DOWN, L.STAGE_COMBINE]
    for seq in ([1 << st for st in one], [sum(1 << st for st in one[:3]), sum(1 << st for st in one[3:])]):
        ws = torch.full((need,), 0x7f, dtype=torch.uint8, device=cuda)
        o2 = torch.full_like(out, float("nan"))
        s2, w2 = torch.full_like(sel, -7), torch.full_like(w, float("nan"))
        say("stages", name, "masks", [hex(m) for m in seq])
        for m in seq:
            bmx.ops.moe_layer_stages(layer.desc, layer.router, x, logits, s2, w2, o2, ws, m)
        torch.cuda.synchronize()
        assert torch.equal(s2, sel) and torch.equal(w2.view(torch.int16), w.view(torch.int16))
        assert torch.equal(o2.view(torch.int32), out.view(torch.int32))


def test_layer_stages_rejects_bad_mask(cuda):
    import bmx
    from bmx import synth
    tab = synth.table("c1", seed=1, device=cuda, E=16)
    x, lg, _ = synth.inputs("c1", T=1, seed=2, device=cuda)
    layer = bmx.MoELayer(tab, 4)
    o = torch.empty(1, tab.H, device=cuda)
    s, w = torch.empty(1, 4, dtype=torch.int64, device=cuda), torch.empty(1, 4, dtype=torch.float16, device=cuda)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=cuda)
    for m in (0, 1 << bmx._lib.STAGE_DOWN_OUT, 1 << 9):
        with pytest.raises(bmx.BmxError, match="stage mask"):
            bmx.ops.moe_layer_stages(layer.desc, layer.router, x, lg[:, :16].contiguous(), s, w, o, ws, m)


def test_act_rows_match_oracle(cuda, oracle):
    """The fp16 down-input rows (rotated activation) equal the oracle's except where the fp32 vs exact accumulation
    of gate / up lands on the other side of an fp16 rounding boundary; a flipped gate / up value moves all 128 values
    of its rotation block by a fraction of an ulp, so flips come in blocks, bounded by a few fp16 ulps of the row's largest value."""
    import bmx
    from bmx import synth
    tab = synth.table("c2", seed=4, device=cuda, E=16)
    x, lg, bias = synth.inputs("c2", T=2, seed=5, device=cuda)
    sel, w = bmx.ops.router_topk(lg[:, :16].contiguous(), 8, bias[:16].contiguous(), 1, 1, 1, True, 2.5)
    rpg = bmx.lib().bmx_rows_per_group(2, 8, 0)
    routes = bmx.ops.dispatch(sel, 16, 0, True, rpg)
    y, act = bmx.ops.moe_experts(tab.desc(8), x, routes, with_act=True)
    torch.cuda.synchronize()
    rt = routes.row_token.cpu().numpy()
    offs = routes.offsets.cpu().numpy()
    act = act.cpu().numpy()
    xs = x.cpu().numpy()
    nr = int(offs[-1])
    eq, tot = 0, 0
    for r in range(nr):
        e = int(np.searchsorted(offs, r, side="right") - 1)
        ex = tab.host_expert(e)
        yo, g, u, a = oracle.expert_forward(ex, tab.H, tab.I, xs[rt[r]])
        eq += int(np.sum(act[r].view(np.uint16) == a.view(np.uint16)))
        tot += a.size
        assert np.abs(act[r].astype(np.float32) - a.astype(np.float32)).max() <= 2e-3 * max(1.0, float(np.abs(a).max()))
        assert rel_rms(y.cpu().numpy()[r], yo) < REL_RMS
    print("act rows bit-equal", eq / tot, flush=True)
    assert eq / tot > 0.98


def test_combine_matches_standalone(cuda):
    import bmx
    from bmx import synth
    tab = synth.table("c2", seed=6, device=cuda, E=24)
    x, lg, bias = synth.inputs("c2", T=5, seed=7, device=cuda)
    sel, w = bmx.ops.router_topk(lg[:, :24].contiguous(), 8, bias[:24].contiguous(), 1, 1, 1, True, 2.5)
    d = tab.desc(8)
    out = bmx.ops.moe_forward(d, x, sel, w)
    routes = bmx.ops.dispatch(sel, 24, 0, True, bmx.lib().bmx_rows_per_group(5, 8, 0))
    y, _ = bmx.ops.moe_experts(d, x, routes)
    out2 = bmx.ops.combine(y, routes, w, tab.H)
    assert torch.equal(out, out2)


def test_full_size_properties_c2_t8(cuda):
    """Size-independent checks at the full c2 T = 8 size (288 experts, H 4096, I 1536): without the shared expert,
    doubling every routing weight doubles the output bit for bit (scaling by 2 is exact in fp16 and fp32); a pick marked
    dropped (sentinel id first + E) equals the same pick with weight 0; the shared expert adds its own output."""
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c2"]
    tab = synth.table("c2", seed=8, device=cuda)
    x, lg, bias = synth.inputs("c2", T=8, seed=9, device=cuda)
    sel, w = bmx.ops.router_topk(lg, 8, bias, 1, 1, 1, True, c["scale"])
    d = tab.desc(8)
    d.shared = None
    out = bmx.ops.moe_forward(d, x, sel, w)
    out2 = bmx.ops.moe_forward(d, x, sel, (w * 2).contiguous())
    assert torch.equal(out2, out * 2)
    s2 = sel.clone()
    s2[:, 3] = tab.E
    w2 = w.clone()
    w2[:, 3] = 0
    # on the GEMV path and on the mid-size MFMA path (AUTO at 8 tokens) every row is computed on its own (an MFMA output
    # row depends on its own input row only, in a fixed k order): a dropped pick and a weight-0 pick give the same bits.
    # On the split path a row's kernel follows its expert's row count, which the weight-0 pick still adds to, so the other
    # rows of that expert may move to the other kernel: within the layer tolerance there
    assert bmx.lib().bmx_resolve_path(8, 8, bmx.PATH_AUTO) == bmx.PATH_MID
    for path in (bmx.PATH_DECODE, bmx.PATH_AUTO):
        a = bmx.ops.moe_forward(d, x, s2, w, path)
        b = bmx.ops.moe_forward(d, x, sel, w2, path)
        assert torch.equal(a, b) and not torch.equal(a, bmx.ops.moe_forward(d, x, sel, w, path)), path
    a2 = bmx.ops.moe_forward(d, x, s2, w, bmx.PATH_SPLIT)
    b2 = bmx.ops.moe_forward(d, x, sel, w2, bmx.PATH_SPLIT)
    assert float((a2 - b2).abs().max()) < 1e-2 and float((a2 - a).abs().max()) < 1e-2
    full = bmx.ops.moe_forward(tab.desc(8), x, sel, w)
    only_shared = bmx.ops.moe_forward(tab.desc(8), x, sel, torch.zeros_like(w))
    assert torch.allclose(full, out + only_shared, rtol=1e-5, atol=1e-5)


ACTS = [("gelu", 1, True, 0.0), ("relu2", 2, True, 0.0), ("silu_oai", 3, True, 0.0), ("silu_oai limit 7", 3, True, 7.0),
        ("silu limit 0.5", 0, True, 0.5), ("not gated", 0, False, 0.0)]


@pytest.mark.parametrize("name,act,gated,limit", ACTS, ids=[a[0] for a in ACTS])
@pytest.mark.parametrize("path", [1, 2], ids=["decode", "prefill"])
def test_layer_activations(cuda, oracle, name, act, gated, limit, path):
    """Each activation and clamp of the epilogue (x16_dev.cu:68-112) on both expert paths against the oracle."""
    import bmx
    from bmx import synth
    say("act", name, "path", path)
    E, T, H, I = 12, 6, 512, 384
    tab = synth.table("c2", seed=7, device=cuda, E=E, H=H, I=I)
    x, lg, bias = synth.inputs("c2", T=T, seed=8, device=cuda)
    x = x[:, :H].contiguous()
    layer = bmx.MoELayer(tab, 4, score=bmx.SCORE_SIGMOID, bias=bias[:E].contiguous(), renorm=True, scale=2.5, act=act,
                         gated=gated, act_limit=limit)
    sel, w = layer.routing_fn(T, None, x, {"logits": lg[:, :E].contiguous()})
    out = layer.run_bszN(x, sel, w, path=path).cpu().numpy()
    xs, ss, ws = x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()
    exps = [tab.host_expert(e) for e in range(E)]
    want = oracle.moe_forward(exps, 0, tab.host_expert(E), H, I, xs, ss, ws, act=act, gated=gated, limit=limit)
    err_abs, err_rel = float(np.abs(out - want).max()), rel_rms(out, want)
    say("act", name, "max_abs", err_abs, "rel_rms", err_rel)
    assert err_abs < MAX_ABS and err_rel < REL_RMS
    # the activation matters: SiLU without clamp gives a different layer
    if (act, gated, limit) != (0, True, 0.0):
        plain = oracle.moe_forward(exps, 0, tab.host_expert(E), H, I, xs, ss, ws)
        assert rel_rms(plain, want) > 10 * REL_RMS


@pytest.mark.parametrize("fmts,shared", [((2, 1, 3), True), ((0, 0, 0), False), ((3, 2, 1), True)])
def test_one_token_act_in_down(cuda, fmts, shared):
    """One token: the down GEMV computes the activation of its k-range from the gate / up partials itself. The same
    sums as the separate epilogue kernel (BMX_ACT_IN_DOWN=0), so the outputs are bit-identical."""
    import bmx
    E, H, I, topk = 40, 512, 768, 6
    tab = bmx.ExpertTable.random(H, I, E, fmts, shared=shared, seed=11, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(12)
    x = torch.randn((1, H), generator=g, device=cuda).half()
    lg = torch.randn((1, E), generator=g, device=cuda).half()
    layer = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=2.0)
    say("act in down", fmts, shared)
    a = layer.forward(x, lg, path=bmx.PATH_DECODE).cpu().numpy()
    os.environ["BMX_ACT_IN_DOWN"] = "0"
    try:
        b = layer.forward(x, lg, path=bmx.PATH_DECODE).cpu().numpy()
    finally:
        os.environ.pop("BMX_ACT_IN_DOWN", None)
    assert np.array_equal(a, b) and np.abs(a).max() > 0
