"""CPU expert lane (host only): its expert rows agree with the oracle's expert forward within the layer tolerance,
and its v_dot2_f32_f16 emulation satisfies what the instruction's rule fixes exactly (exact results where the sum is
exactly representable, the plain fp32 sum where no term is truncated). The bit-for-bit checks against the device are
in test_gpu_cpu_lane.py."""
import numpy as np
import pytest


def f16_pairs(lo, hi):
    return (lo.astype(np.float16).view(np.uint16).astype(np.uint32) |
            (hi.astype(np.float16).view(np.uint16).astype(np.uint32) << 16))


TB = {0: 64, 1: 80, 2: 96, 3: 128}


def host_expert(H, I, fmts, seed):
    """A random EXL3 expert in host memory (the ExpertTable.host_expert layout): trellis bytes, suh ~ U(0.5, 1.5),
    svh ~ U(0.5, 1.5) / sqrt(k)."""
    rng = np.random.default_rng(seed)
    dims = ((H, I), (H, I), (I, H))
    return {"tr": [rng.integers(0, 256, (k // 16) * (n // 16) * TB[f], dtype=np.uint8) for (k, n), f in zip(dims, fmts)],
            "suh": [(rng.random(k) + 0.5).astype(np.float16) for k, n in dims],
            "svh": [((rng.random(n) + 0.5) / np.sqrt(k)).astype(np.float16) for k, n in dims],
            "fmt": list(fmts)}


def test_dot2_exact_cases():
    from bmx import cpu_lane
    rng = np.random.default_rng(0)
    n = 20000
    # small integers: every product and sum is exact in fp32, so the result is the exact sum whatever the truncations
    a0, a1, b0, b1 = (rng.integers(-64, 64, n) for _ in range(4))
    c = rng.integers(-4096, 4096, n).astype(np.float32)
    out = cpu_lane.dot2(f16_pairs(a0, a1), f16_pairs(b0, b1), c)
    assert np.array_equal(out, (a0 * b0 + a1 * b1 + c).astype(np.float32))
    # both products zero: c unchanged, including -0 and subnormal c
    z = np.zeros(4, np.uint32)
    cz = np.array([-0.0, 1e-40, -3.5, 7.25e30], np.float32)
    assert np.array_equal(cpu_lane.dot2(z, f16_pairs(np.ones(4), np.ones(4)), cz).view(np.uint32), cz.view(np.uint32))
    # one nonzero product and c = 0: the product itself (exact in fp32)
    a = rng.standard_normal(n).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float16)
    out = cpu_lane.dot2(f16_pairs(a, np.zeros(n)), f16_pairs(b, np.zeros(n)), np.zeros(n, np.float32))
    assert np.array_equal(out, (a.astype(np.float32) * b.astype(np.float32)))
    # a planted difference: the accumulator far above the products truncates them (the plain fp32 formula would not)
    out = cpu_lane.dot2(f16_pairs(np.array([1.0]), np.array([0.0])), f16_pairs(np.array([2.0 ** -14]), np.array([0.0])),
                        np.array([2.0 ** 20], np.float32))
    assert out[0] == np.float32(2.0 ** 20)


@pytest.mark.parametrize("act,gated,limit", [(0, True, 0.0), (1, True, 0.0), (2, True, 0.0), (3, True, 7.0), (0, False, 0.0)])
def test_cpu_lane_rows_match_oracle(oracle, act, gated, limit):
    """Expert rows through the lane vs the oracle's fp64-accumulating expert forward: within the layer tolerance."""
    from bmx import cpu_lane
    H, I = 512, 256
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, H)).astype(np.float16)
    for e, fmts in enumerate([(2, 0, 3), (1, 1, 1), (3, 3, 3)]):
        ex = host_expert(H, I, fmts, seed=10 + e)
        y = cpu_lane.expert_rows(ex, H, I, x, 2, 1, 1, act, gated, limit, threads=2)
        for m in range(3):
            yo = oracle.expert_forward(ex, H, I, x[m], act, gated, limit)[0]
            err = np.sqrt(np.mean((y[m] - yo) ** 2)) / max(1e-30, np.sqrt(np.mean(yo ** 2)))
            assert err < 1e-3 and np.abs(y[m] - yo).max() < 1e-2, (e, m, err)


def test_cpu_lane_rejects_bad_splits():
    import bmx
    from bmx import cpu_lane
    with pytest.raises(bmx.BmxError, match="k-splits"):
        cpu_lane.expert_rows(host_expert(256, 128, (2, 2, 2), 1), 256, 128, np.zeros((1, 256), np.float16), 3, 1, 1)


@pytest.mark.parametrize("fmts,ks", [((2, 0, 3), (2, 1)), ((1, 1, 1), (1, 2)), ((3, 2, 0), (4, 2))])
def test_cpu_lane_vector_equals_scalar(monkeypatch, fmts, ks):
    """The AVX-512 path (8 output columns per step) gives the scalar path's bits (where the host has AVX-512)."""
    from bmx import cpu_lane
    H, I = 512, 256
    ex = host_expert(H, I, fmts, seed=sum(fmts) * 7 + ks[0])
    x = np.random.default_rng(ks[0]).standard_normal((5, H)).astype(np.float16) * np.float16(4.0)
    y_vec = cpu_lane.expert_rows(ex, H, I, x, ks[0], ks[1], 1, 2, True, 0.0, threads=3)
    monkeypatch.setenv("BMX_CPU_LANE_SCALAR", "1")
    y_sca = cpu_lane.expert_rows(ex, H, I, x, ks[0], ks[1], 1, 2, True, 0.0, threads=3)
    assert np.array_equal(y_vec.view(np.uint32), y_sca.view(np.uint32))


# ---- fast mode ----------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmts,nr", [((2, 0, 3), 1), ((1, 1, 1), 3), ((3, 2, 0), 9), ((0, 3, 1), 8)])
def test_fast_lane_vector_equals_scalar(monkeypatch, fmts, nr):
    """The fast mode's AVX-512 decode (byte permute, shift, hash, VNNI byte sum, fp32 FMA, fp16 rounding) against its
    scalar path, which decodes through the exact codebook table: the two sum each column in the same order, so equal
    bits mean every decoded weight equals the exact codebook's (where the host has AVX-512 VBMI and VNNI)."""
    from bmx import cpu_lane
    H, I = 512, 384
    ex = host_expert(H, I, fmts, seed=31 + nr)
    x = np.random.default_rng(nr).standard_normal((nr, H)).astype(np.float16) * np.float16(3.0)
    y_vec = cpu_lane.expert_rows_fast(ex, H, I, x, 0, True, 0.0, threads=3)
    monkeypatch.setenv("BMX_CPU_LANE_SCALAR", "1")
    y_sca = cpu_lane.expert_rows_fast(ex, H, I, x, 0, True, 0.0, threads=3)
    assert np.array_equal(y_vec.view(np.uint32), y_sca.view(np.uint32))
    assert np.abs(y_vec).max() > 0


@pytest.mark.parametrize("act,gated,limit", [(0, True, 0.0), (1, True, 0.0), (2, True, 0.0), (3, True, 7.0), (0, False, 0.0)])
def test_fast_lane_rows_match_oracle(oracle, act, gated, limit):
    """Fast-mode expert rows vs the oracle's fp64-accumulating expert forward: within the layer tolerance."""
    from bmx import cpu_lane
    H, I = 512, 256
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, H)).astype(np.float16)
    for e, fmts in enumerate([(2, 0, 3), (1, 1, 1), (3, 3, 3)]):
        ex = host_expert(H, I, fmts, seed=40 + e)
        y = cpu_lane.expert_rows_fast(ex, H, I, x, act, gated, limit, threads=4)
        for m in range(3):
            yo = oracle.expert_forward(ex, H, I, x[m], act, gated, limit)[0]
            err = np.sqrt(np.mean((y[m] - yo) ** 2)) / max(1e-30, np.sqrt(np.mean(yo ** 2)))
            assert err < 1e-3 and np.abs(y[m] - yo).max() < 1e-2, (e, m, err)


@pytest.mark.parametrize("H,I,fmts", [(2048, 1536, (2, 1, 0)), (4096, 256, (3, 0, 2))])
def test_fast_lane_long_chunks(monkeypatch, oracle, H, I, fmts):
    """Shapes whose chunks hold several tile-rows (K / 512 of them, at most 8: 4 for gate / up and 3 for down at
    (2048, 1536), 8 and 1 at (4096, 256), the last chunk of K 1536 short): the SIMD path equals the scalar one and a
    different worker count gives the same bits, and the rows are within the layer tolerance of the oracle."""
    from bmx import cpu_lane
    ex = host_expert(H, I, fmts, seed=H + I)
    x = np.random.default_rng(H).standard_normal((2, H)).astype(np.float16)
    y = cpu_lane.expert_rows_fast(ex, H, I, x, 0, True, 0.0, threads=1)
    y7 = cpu_lane.expert_rows_fast(ex, H, I, x, 0, True, 0.0, threads=7)
    assert np.array_equal(y.view(np.uint32), y7.view(np.uint32))
    for m in range(2):
        yo = oracle.expert_forward(ex, H, I, x[m], 0, True, 0.0)[0]
        err = np.sqrt(np.mean((y[m] - yo) ** 2)) / max(1e-30, np.sqrt(np.mean(yo ** 2)))
        assert err < 1e-3 and np.abs(y[m] - yo).max() < 1e-2, (m, err)
    monkeypatch.setenv("BMX_CPU_LANE_SCALAR", "1")
    y_sca = cpu_lane.expert_rows_fast(ex, H, I, x, 0, True, 0.0, threads=3)
    assert np.array_equal(y.view(np.uint32), y_sca.view(np.uint32))


def test_fast_lane_close_to_exact_lane():
    """A C2-shaped expert (H 4096, I 1536, K 3): the fast mode's rows within the layer tolerance of the exact lane's,
    and repeated calls (the worker pool kept between them, its size changed) give the same bits."""
    from bmx import cpu_lane
    H, I = 4096, 1536
    ex = host_expert(H, I, (2, 2, 2), seed=77)
    x = np.random.default_rng(78).standard_normal((2, H)).astype(np.float16)
    ye = cpu_lane.expert_rows(ex, H, I, x, 16, 4, 1, threads=8)
    yf = cpu_lane.expert_rows_fast(ex, H, I, x, threads=8)
    err = np.sqrt(np.mean((yf - ye) ** 2)) / np.sqrt(np.mean(ye ** 2))
    assert err < 1e-3 and np.abs(yf - ye).max() < 1e-2, err
    assert np.array_equal(cpu_lane.expert_rows_fast(ex, H, I, x, threads=8).view(np.uint32), yf.view(np.uint32))
    assert np.array_equal(cpu_lane.expert_rows_fast(ex, H, I, x, threads=3).view(np.uint32), yf.view(np.uint32))


def test_fast_lane_rejects_bad_shapes():
    import bmx
    from bmx import cpu_lane
    with pytest.raises(bmx.BmxError, match="multiples of 128"):
        cpu_lane.expert_rows_fast(host_expert(256, 128, (2, 2, 2), 1), 200, 128, np.zeros((1, 200), np.float16))
