"""Pins the oracle's router, dispatch and expert-slot step by independent methods: numpy sorting of the closed forms,
brute force over small cases, libm for exp, and invariants / hand-computed known answers for the CLOCK step."""
import numpy as np
import pytest


def test_exp_fixed_accuracy(oracle):
    xs = np.concatenate([np.linspace(-100, 88, 20001), np.array([0.0, -0.0, 1.0, -1.0, 1e-8, -1e-8])]).astype(np.float32)
    got = np.array([oracle.exp32(v) for v in xs], np.float32)
    want = np.exp(xs.astype(np.float64))
    ok = want > np.finfo(np.float32).tiny
    relerr = np.abs(got[ok] - want[ok]) / want[ok]
    assert relerr.max() < 4 * 2.0 ** -23
    assert oracle.exp32(-200.0) == 0.0 and np.isinf(oracle.exp32(100.0)) and oracle.exp32(0.0) == 1.0


def _choice(oracle, lg, bias, score):
    l = lg.astype(np.float32)
    if score == oracle.SCORE_SOFTMAX:
        return l, np.array([oracle.exp32(v - l.max()) for v in l], np.float32)
    s = np.array([oracle.lib().bmxo_sigmoid(float(v)) for v in l], np.float32)
    return (s + bias if bias is not None else s).astype(np.float32), s


def _topk_order(vals, idx_ok):
    """indices sorted by (value desc, index asc) restricted to idx_ok"""
    cand = [i for i in range(len(vals)) if idx_ok[i]]
    return sorted(cand, key=lambda i: (-float(vals[i]), i))


@pytest.mark.parametrize("score", [0, 1])
def test_router_plain_topk(oracle, score):
    rng = np.random.default_rng(score)
    T, E, k = 16, 64, 8
    lg = rng.standard_normal((T, E)).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if score == 1 else None
    sel, w = oracle.router(lg, k, bias=bias, score_fn=score, renorm=True, scale=2.5, first=3)
    for t in range(T):
        ch, sc = _choice(oracle, lg[t], bias, score)
        want = _topk_order(ch, [True] * E)[:k]
        assert (sel[t] - 3).tolist() == want
        v = sc[want].astype(np.float64)
        assert np.allclose(w[t].astype(np.float64), v / v.sum() * 2.5, rtol=2e-3)
    if score == 0:   # softmax selection is the logits' top-k (monotone)
        for t in range(T):
            assert sorted((sel[t] - 3).tolist()) == sorted(np.argsort(-lg[t].astype(np.float64), kind="stable")[:k].tolist())


def test_router_ties_lower_index(oracle):
    lg = np.zeros((1, 16), np.float16)
    lg[0, [3, 9, 12]] = 1.0
    sel, _ = oracle.router(lg, 5, score_fn=oracle.SCORE_SIGMOID)
    assert sel[0].tolist() == [3, 9, 12, 0, 1]
    sel, w = oracle.router(lg, 4, score_fn=oracle.SCORE_SOFTMAX, renorm=False)
    assert sel[0].tolist() == [3, 9, 12, 0]
    p = np.exp(lg[0].astype(np.float64)); p /= p.sum()
    assert np.allclose(w[0].astype(np.float64), p[[3, 9, 12, 0]], rtol=2e-3)


def test_router_group_limited_vs_brute_force(oracle):
    rng = np.random.default_rng(2)
    T, E, G, TG, k = 24, 64, 8, 3, 6
    lg = rng.standard_normal((T, E)).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.2).astype(np.float32)
    sel, w = oracle.router(lg, k, bias=bias, n_group=G, topk_group=TG, score_fn=oracle.SCORE_SIGMOID, renorm=True)
    gs = E // G
    for t in range(T):
        ch, sc = _choice(oracle, lg[t], bias, oracle.SCORE_SIGMOID)
        gsc = []
        for g in range(G):
            top2 = sorted(ch[g * gs:(g + 1) * gs].tolist(), reverse=True)[:2]
            gsc.append(np.float32(np.float32(top2[0]) + np.float32(top2[1])))
        keep = sorted(range(G), key=lambda g: (-float(gsc[g]), g))[:TG]
        ok = [e // gs in keep for e in range(E)]
        want = _topk_order(ch, ok)[:k]
        assert sel[t].tolist() == want
        assert all((e // gs) in keep for e in sel[t])


def test_router_selection_matters(oracle):
    """Planted mistake check: with the bias omitted the selection changes for this seed."""
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((8, 64)).astype(np.float16)
    bias = (rng.standard_normal(64) * 0.5).astype(np.float32)
    a, _ = oracle.router(lg, 8, bias=bias)
    b, _ = oracle.router(lg, 8, bias=None)
    assert not np.array_equal(a, b)


def test_dispatch_vs_stable_argsort(oracle):
    rng = np.random.default_rng(3)
    T, k, E = 50, 6, 20
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64) + 5
    sel[3, 2] = 5 + E          # sentinel (dropped)
    sel[7, 0] = -1             # masked
    d = oracle.dispatch(sel, E, first=5, shared=True)
    flat = (sel - 5).ravel()
    valid = (flat >= 0) & (flat < E)
    order = np.argsort(np.where(valid, flat, E + 10), kind="stable")[:valid.sum()]
    assert d["row_token"][:valid.sum()].tolist() == (order // k).tolist()
    assert d["row_slot"][:valid.sum()].tolist() == (order % k).tolist()
    assert np.array_equal(d["counts"][:E], np.bincount(flat[valid], minlength=E))
    assert d["counts"][E] == T and d["offsets"][E + 1] == valid.sum() + T
    assert d["inv"][3, 2] == -1 and d["inv"][7, 0] == -1
    inv = d["inv"].ravel()
    assert np.array_equal(np.sort(inv[inv >= 0]), np.arange(valid.sum()))
    assert d["row_token"][valid.sum():].tolist() == list(range(T))
    assert d["uexp"].tolist() == sorted(set(flat[valid].tolist())) + [E]


def test_dispatch_empty_and_all_dropped(oracle):
    sel = np.full((4, 2), -1, np.int64)
    d = oracle.dispatch(sel, 8)
    assert d["nuniq"] == 0 and np.all(d["inv"] == -1) and d["offsets"][-1] == 0


# ---- expert-slot table ----

def _check_maps(st):
    for s in range(st.S):
        o = st.owner[s]
        if o >= 0:
            assert st.slotof[o] == s
    for key in range(st.L * st.E):
        s = st.slotof[key]
        if s >= 0:
            assert st.owner[s] == key


def test_slot_step_known_answer(oracle):
    st = oracle.SlotTable(L=2, E=8, S=3)
    jobs, ev = st.step(0, [1, 4])          # empty table: 1 -> slot 0, 4 -> slot 1
    assert jobs.tolist() == [[1, 0], [4, 1]] and ev.tolist() == [-1, -1]
    assert st.stats.tolist() == [0, 2, 2, 0, 0, 0, 0, 0]
    jobs, ev = st.step(1, [2, 4])          # layer 1: 2 -> slot 2; 4: slots 0, 1 referenced (cleared), 2 pinned
    assert jobs.tolist() == [[2, 2], [4, 0]] and ev.tolist() == [-1, 1]
    # second miss: hand cleared refb of 0 and 1 on the way to slot 2 then wrapped to slot 0 (refb now clear)
    assert st.slotof[1] == -1 and st.owner[0] == 8 + 4
    jobs, ev = st.step(0, [4])             # hit: no jobs
    assert jobs.size == 0 and st.stats[0] == 1
    _check_maps(st)


def test_slot_step_invariants_random(oracle):
    rng = np.random.default_rng(0)
    L, E, S = 4, 32, 20
    st = oracle.SlotTable(L, E, S)
    for it in range(300):
        li = int(rng.integers(L))
        sel = rng.choice(E, 6, replace=False)
        before_pin_epoch = st.epoch + 1
        jobs, ev = st.step(li, sel)
        _check_maps(st)
        # every pick is resident afterwards (6 picks <= S slots, each epoch pins at most 6)
        for e in sel:
            assert st.slotof[li * E + e] >= 0
            assert st.pin[st.slotof[li * E + e]] == before_pin_epoch
        # admitted experts were misses; victims were not picked this step
        for (e, s), old in zip(jobs, ev):
            assert e in sel
            if old >= 0:
                assert not (old // E == li and (old % E) in sel)
    assert st.stats[0] + st.stats[1] == 300 * 6


def test_slot_disabled_slots_never_used(oracle):
    st = oracle.SlotTable(1, 16, 4)
    st.pin[1] = -1
    st.pin[3] = -1
    jobs, _ = st.step(0, [0, 1, 2])
    assert sorted(jobs[:, 1].tolist()) == [0, 2] and st.stats[3] == 1     # third miss: no victim


def test_slot_prefetch_known_answer(oracle):
    """Layer-ahead prefetch: candidates are the distinct in-range guesses that are not resident, in rank order, capped
    at `limit`; they take slots within the current epoch (the last step's slots stay pinned, the epoch does not
    advance) by a gentle sweep that passes referenced slots without clearing their bits and admits with the bit clear;
    a later step's first hit on a prefetched slot counts as used and marks the expert fresh; a prefetched expert evicted
    before any use counts as wasted."""
    st = oracle.SlotTable(L=2, E=8, S=6)
    st.step(1, [3])                                         # epoch 1: L1 e3 -> slot 0
    st.step(0, [1, 4])                                      # epoch 2: L0 e1 -> 1, e4 -> 2; hand 3
    jobs, ev = st.prefetch(1, [3, 6, 6, 9, 2, 5], limit=2)  # 3 resident, 6 dup, 9 out of range: [6, 2]
    assert jobs.tolist() == [[6, 3], [2, 4]] and ev.tolist() == [-1, -1]
    assert st.epoch == 2 and st.hand == 5 and st.pin[3] == st.pin[4] == 2
    assert st.pfl.tolist() == [0, 0, 0, 1, 1, 0] and st.refb.tolist() == [1, 1, 1, 0, 0, 0]
    assert st.stats.tolist() == [0, 3, 3, 0, 0, 2, 0, 0]
    jobs, _ = st.prefetch(1, [5, 7], limit=4)               # 5 -> slot 5; 7: slot 0 referenced, the rest pinned
    assert jobs.tolist() == [[5, 5]] and st.hand == 0 and st.refb[0] == 1 and st.slotof[8 + 3] == 0
    jobs, ev = st.step(1, [2, 6, 0])                        # epoch 3: 2, 6 prefetched hits; 0 misses
    # hand 0: slots 0-2 lose their bits, 3 and 4 are pinned, slot 5 (L1 e5, prefetched, never used, bit clear) taken
    assert jobs.tolist() == [[0, 5]] and ev.tolist() == [8 + 5]
    assert np.flatnonzero(st.fresh).tolist() == [0, 2, 6]
    assert st.stats.tolist() == [2, 4, 4, 0, 1, 3, 2, 1] and st.pfl.tolist() == [0] * 6
    jobs, ev = st.step(0, [5, 6])                           # epoch 4: slot 0 (L1 e3), slot 1 (L0 e1)
    assert jobs.tolist() == [[5, 0], [6, 1]] and ev.tolist() == [8 + 3, 1]
    assert st.stats.tolist() == [2, 6, 6, 0, 3, 3, 2, 1]
    _check_maps(st)


def test_slot_prefetch_properties_random(oracle):
    """Random steps and prefetches: a prefetch never advances the epoch, never moves a slot the last step pinned, never
    changes a reference bit or the hit / miss counts, admits a prefix (in rank order) of the distinct non-resident guesses, and every expert it
    admitted is a hit, marked fresh, at the next step of its layer."""
    rng = np.random.default_rng(1)
    L, E, S = 3, 24, 12
    st = oracle.SlotTable(L, E, S)
    st.pin[5] = -1
    for it in range(400):
        li = int(rng.integers(L))
        st.step(li, rng.choice(E, 4, replace=False))
        lj = int(rng.integers(L))
        guess = rng.integers(-2, E + 2, int(rng.integers(0, 12)))
        limit, maxj = int(rng.integers(1, 8)), int(rng.integers(1, 8))
        epoch, stats0, refb0 = st.epoch, st.stats.copy(), st.refb.copy()
        pinned = {s: int(st.owner[s]) for s in range(S) if st.pin[s] == epoch}
        want, seen = [], set()
        for g in guess:
            if 0 <= g < E and g not in seen:
                seen.add(int(g))
                if st.slotof[lj * E + g] < 0:
                    want.append(int(g))
        want = want[:limit]
        jobs, ev = st.prefetch(lj, guess, limit=limit, maxj=maxj)
        _check_maps(st)
        assert st.epoch == epoch and st.pin[5] == -1 and st.owner[5] == -1
        assert np.array_equal(st.refb, refb0)               # victims had clear bits; nothing else is touched
        assert all(st.owner[s] == o for s, o in pinned.items())
        assert np.array_equal(st.stats[[0, 1, 2, 3, 6]], stats0[[0, 1, 2, 3, 6]])
        got = jobs[:, 0].tolist()
        assert got == want[:len(got)] and len(got) <= maxj
        assert st.stats[5] - stats0[5] == len(got) and st.stats[4] - stats0[4] == int((ev >= 0).sum())
        if got and rng.random() < 0.5:
            st.step(lj, np.array(got))
            assert st.stats[0] - stats0[0] == len(got) and np.flatnonzero(st.fresh).tolist() == sorted(got)
            assert st.stats[6] - stats0[6] == len(got)


# ---- sqrt-softplus score, router projection, shared-expert gate ------------------------------------------------------

def _sqrtsp64(x):
    x = np.asarray(x, np.float64)
    return np.sqrt(np.logaddexp(0.0, x))      # sqrt(log(1 + e^x)) without overflow


def test_sqrtsp_fixed_accuracy(oracle):
    """The fixed-sequence sqrt(softplus(x)) against the float64 closed form: within 2 fp32 ulps over a sweep that covers
    the series' range (|x| small: s near 1/3), the tails (e^-|x| tiny) and the limits; a plausible mistake in the
    restatement (the max(x, 0) term dropped, or log1p replaced by the raw series variable) fails the same bound."""
    xs = np.concatenate([np.linspace(-30, 30, 24001), np.linspace(-80, 104, 2001),
                         np.array([0.0, -0.0, 1e-8, -1e-8, 1e-30, 88.0, -80.0])]).astype(np.float32)
    got = np.array([oracle.sqrtsp32(v) for v in xs], np.float64)
    want = _sqrtsp64(xs)
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 2.0
    # below x = -87 softplus(x) = e^x is subnormal in fp32 and keeps fewer bits: an absolute error of two subnormal
    # spacings (2^-148) in softplus is at most 2^-74 after the square root
    tail = np.linspace(-103, -81, 221).astype(np.float32)
    gt = np.array([oracle.sqrtsp32(v) for v in tail], np.float64)
    wt = _sqrtsp64(tail)
    assert np.all(np.abs(gt - wt) <= 2.0 ** -74 + 4 * np.spacing(wt.astype(np.float32)))
    assert oracle.sqrtsp32(float("inf")) == float("inf") and oracle.sqrtsp32(float("-inf")) == 0.0
    assert np.isnan(oracle.sqrtsp32(float("nan")))
    # planted mistakes, evaluated on the same sweep, must fail the bound
    e = np.exp(-np.abs(xs.astype(np.float64)))
    no_max = np.sqrt(np.log1p(e))
    raw_s = np.sqrt(np.maximum(xs, 0) + 2.0 * e / (2.0 + e))
    for bad in (no_max, raw_s):
        assert np.max(np.abs(bad - want) / ulp) > 100.0


def test_router_sqrtsp_topk(oracle):
    """sqrt-softplus scoring (DeepSeek-V4's router): selection by score + bias, weights = scores renormalised over the
    picks times the scale, or the raw scores without renormalisation; against the float64 closed form."""
    rng = np.random.default_rng(21)
    T, E, k = 32, 256, 6
    lg = (rng.standard_normal((T, E)) * 2.0).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    for renorm in (True, False):
        sel, w = oracle.router(lg, k, bias=bias, score_fn=oracle.SCORE_SQRTSP, renorm=renorm, scale=1.5, first=5)
        for t in range(T):
            sc = _sqrtsp64(lg[t].astype(np.float64))
            ch = sc + bias
            order = sorted(range(E), key=lambda e: (-ch[e], e))
            want = order[:k]
            # a selection boundary closer than fp32 rounding could flip; the draws here have none
            assert ch[order[k - 1]] - ch[order[k]] > 1e-5
            assert (sel[t] - 5).tolist() == want
            v = sc[want]
            ref = v / v.sum() * 1.5 if renorm else v * 1.5
            assert np.allclose(w[t].astype(np.float64), ref, rtol=2e-3, atol=0)
    # grouped selection works on the same scores
    sel, _ = oracle.router(lg, k, bias=bias, n_group=8, topk_group=4, score_fn=oracle.SCORE_SQRTSP)
    gs = E // 8
    for t in range(T):
        ch = _sqrtsp64(lg[t].astype(np.float64)) + bias
        gsc = [np.sort(ch[g * gs:(g + 1) * gs])[-2:].sum() for g in range(8)]
        keep = set(sorted(range(8), key=lambda g: (-gsc[g], g))[:4])
        assert all(int(e) // gs in keep for e in sel[t])


def test_shared_gate_closed_form(oracle):
    """sigmoid(x . g) in the GPU combine's order against float64 (scipy's expit of the exact dot), within 2e-7; the
    order's one-lane-per-16 partial sums matter only at fp32 rounding; planted mistakes (the butterfly's last stage
    dropped, the sigmoid left out) fail."""
    from scipy.special import expit
    rng = np.random.default_rng(5)
    for H in (128, 2048, 4096):
        for _ in range(5):
            x = rng.standard_normal(H).astype(np.float16)
            g = (rng.standard_normal(H) / np.sqrt(H)).astype(np.float16)
            dot = float(x.astype(np.float64) @ g.astype(np.float64))
            got = float(oracle.shared_gate(x, g))
            assert abs(got - expit(dot)) < 2e-7
            # planted: half the partial sums missing (no last butterfly stage), or the raw dot
            parts = [sum(float(x[h]) * float(g[h]) for b in range(H // 128) for h in range(128 * b + 8 * j, 128 * b + 8 * j + 8))
                     for j in range(16)]
            assert abs(expit(sum(parts[:8])) - got) > 1e-6 or abs(sum(parts[8:])) < 1e-3
            assert abs(dot - got) > 1e-3 or abs(expit(dot) - dot) < 1e-3
    z = np.zeros(256, np.float16)
    assert float(oracle.shared_gate(z, z)) == 0.5


def test_moe_forward_shared_gate(oracle):
    """The layer with a gated shared expert: a zero gate vector gives sigmoid(0) = 1/2 exactly, so the output is the
    routed sum plus half the shared expert's output (the ungated layer minus the routed-only layer)."""
    rng = np.random.default_rng(8)
    E, H, I, T, k = 6, 256, 128, 3, 2
    exps = [_rand_expert(rng, H, I) for _ in range(E)]
    sh = _rand_expert(rng, H, I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    sel = np.array([[0, 3], [5, 1], [2, 2]], np.int64)
    w = np.array([[0.6, 0.4], [0.7, 0.3], [0.5, 0.5]], np.float16)
    routed = oracle.moe_forward(exps, 0, None, H, I, x, sel, w)
    full = oracle.moe_forward(exps, 0, sh, H, I, x, sel, w)
    half = oracle.moe_forward(exps, 0, sh, H, I, x, sel, w, sh_gate=np.zeros(H, np.float16))
    assert np.allclose(half, routed + 0.5 * (full - routed), rtol=1e-6, atol=1e-6)
    g = (rng.standard_normal(H) * 0.05).astype(np.float16)
    gated = oracle.moe_forward(exps, 0, sh, H, I, x, sel, w, sh_gate=g)
    for t in range(T):
        gv = float(oracle.shared_gate(x[t], g))
        assert np.allclose(gated[t], routed[t] + gv * (full[t] - routed[t]), rtol=1e-5, atol=1e-6)


def test_router_projection_closed_form(oracle):
    """The oracle's projection (float64 product) against a brute-force sum on a small case."""
    rng = np.random.default_rng(3)
    z = rng.standard_normal((3, 64)).astype(np.float16)
    W = rng.standard_normal((5, 64)).astype(np.float16)
    got = oracle.router_logits(z, W)
    for t in range(3):
        for e in range(5):
            assert got[t, e] == pytest.approx(sum(float(z[t, h]) * float(W[e, h]) for h in range(64)), rel=1e-12, abs=1e-12)


def _rand_expert(rng, H, I, fmt=2):
    tb = {0: 64, 1: 80, 2: 96, 3: 128}[fmt]
    tr = [rng.integers(0, 256, (a // 16) * (b // 16) * tb, dtype=np.uint8) for a, b in ((H, I), (H, I), (I, H))]
    suh = [(rng.random(n) + 0.5).astype(np.float16) for n in (H, H, I)]
    svh = [((rng.random(n) + 0.5) / np.sqrt(kk)).astype(np.float16) for n, kk in ((I, H), (I, H), (H, I))]
    return {"tr": tr, "suh": suh, "svh": svh, "fmt": [fmt] * 3}
