"""Pins the oracle's EXL3 decode and rotations: against the reference's own CPU code (golden fixtures written from
oracle/_ref, and the live library when built), against the reference test's ring definition, against an independent
numpy restatement, and against mathematics (Hadamard matrix, exhaustive codebook)."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(40000) * 10.0 ** rng.integers(-9, 6, 40000)).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 6e-8, 2.98e-8, 2.9802322e-8, 5.96e-8, -0.0, 0.0, np.inf, -np.inf,
                     6.1035156e-05, 6.097555e-05], np.float32)
    v = np.concatenate([v, edge])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(v), want)
    h = np.arange(65536, dtype=np.uint16)
    h = h[(h & 0x7c00) != 0x7c00]                       # finite
    back = np.array([oracle.lib().bmxo_f16_to_f32(int(x)) for x in h[::7]], np.float32)
    assert np.array_equal(back, h[::7].view(np.float16).astype(np.float32))


def test_ring_ends_match_reference_tf_s(oracle):
    want = np.load(os.path.join(GOLD, "ring_ends.npy"))
    for f in range(3):
        got = [oracle.lib().bmxo_ring_end(f, i) for i in range(256)]
        assert got == want[f].tolist()
        assert got == [oracle.np_ring_end(f, i) for i in range(256)]
    # K 4 by the same rule: S(i) = 4 (i + 1)
    assert [oracle.lib().bmxo_ring_end(3, i) for i in range(256)] == [4 * (i + 1) for i in range(256)]


@pytest.mark.parametrize("name,fmt", [("k2", 0), ("k25", 1), ("k3", 2), ("k4", 3)])
def test_tile_states_match_ring_definition(oracle, name, fmt):
    g = np.load(os.path.join(GOLD, "ring_tiles.npz"))
    for tile, want in zip(g[name + "_tiles"], g[name + "_states"]):
        assert np.array_equal(oracle.tile_states(tile, fmt), want)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_tile_states_c_vs_numpy_twin(oracle, fmt):
    rng = np.random.default_rng(fmt)
    tiles = rng.integers(0, 256, (64, oracle.TF_TB[fmt]), dtype=np.uint8)
    tiles[0] = 0
    tiles[1] = 255
    a = np.stack([oracle.tile_states(t, fmt) for t in tiles])
    assert np.array_equal(a, oracle.np_tile_states(tiles, fmt))
    assert np.all(a[0] == 0) and np.all(a[1] == 0xFFFF)


def test_codebook_exhaustive(oracle):
    want = np.load(os.path.join(GOLD, "codebook_w_gpu.npy"))
    got = oracle.decode_table()
    assert np.array_equal(got, want)                               # reference w_gpu, all 65536 states
    assert np.array_equal(got, oracle.np_codebook().view(np.uint16))
    w = got.view(np.float16).astype(np.float64)
    assert np.abs(w).max() < 3.5                                   # ft_core.h:242-244 range argument
    assert abs(w.mean()) < 0.01 and 0.9 < w.std() < 1.1


def test_perm_matches_reference(oracle):
    want = np.load(os.path.join(GOLD, "perm.npy"))
    assert np.array_equal(oracle.perm(), want)
    assert np.array_equal(oracle.np_perm(), want)
    assert sorted(want.tolist()) == list(range(256))              # a permutation


def test_dequant_k3_matches_reference_dense_weights(oracle):
    g = np.load(os.path.join(GOLD, "k3_tiles.npz"))
    k, n = int(g["k"]), int(g["n"])
    got = oracle.dequant(g["trellis"], oracle.TF_K3, k, n)
    assert np.array_equal(got.view(np.uint16), g["w"].view(np.uint16))


def test_dequant_live_reference(oracle, ref):
    rng = np.random.default_rng(7)
    k, n = 128, 256
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * 96, dtype=np.uint8)
    W = np.zeros((k, n), np.float32)
    ref.ref_dense_weights_k3(tr.ctypes.data, k, n, W.ctypes.data)
    assert np.array_equal(oracle.dequant(tr, oracle.TF_K3, k, n).astype(np.float32), W)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_dequant_c_vs_numpy_twin(oracle, fmt):
    rng = np.random.default_rng(10 + fmt)
    k, n = 64, 128
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * oracle.TF_TB[fmt], dtype=np.uint8)
    a = oracle.dequant(tr, fmt, k, n).view(np.uint16)
    b = oracle.np_dequant(tr, fmt, k, n).view(np.uint16)
    assert np.array_equal(a, b)


def test_dequant_tile_position(oracle):
    """A single changed tile moves only its own 16 x 16 block (tile (tk, tn) at (tk * n/16 + tn) * tile bytes)."""
    rng = np.random.default_rng(3)
    k, n, fmt = 64, 64, 2
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * 96, dtype=np.uint8)
    a = oracle.dequant(tr, fmt, k, n)
    tr2 = tr.copy()
    tr2[(2 * 4 + 1) * 96:(2 * 4 + 2) * 96] ^= 0x5A
    b = oracle.dequant(tr2, fmt, k, n)
    diff = np.argwhere(a.view(np.uint16) != b.view(np.uint16))
    assert diff.size and diff[:, 0].min() >= 32 and diff[:, 0].max() < 48 and diff[:, 1].min() >= 16 and diff[:, 1].max() < 32


def test_had128_is_sylvester_hadamard(oracle):
    from scipy.linalg import hadamard
    rng = np.random.default_rng(1)
    v = rng.standard_normal(128).astype(np.float32)
    out = v.copy()
    oracle.lib().bmxo_had128(out.ctypes.data)
    assert np.allclose(out, hadamard(128) @ v.astype(np.float64), rtol=1e-5, atol=1e-4)
    e = np.zeros(128, np.float32)
    e[5] = 1.0
    oracle.lib().bmxo_had128(e.ctypes.data)
    assert np.array_equal(e, hadamard(128)[:, 5].astype(np.float32))


def test_prep_matches_reference_prep_block(oracle):
    g = np.load(os.path.join(GOLD, "prep.npz"))
    for x, suh, xt, xv in zip(g["x"], g["suh"], g["xt"], g["xt_v"]):
        got = oracle.prep(x, suh)
        assert np.array_equal(got.view(np.uint16), xt.view(np.uint16))
        assert np.array_equal(got.view(np.uint16), xv.view(np.uint16))


def test_prep_live_reference(oracle, ref):
    rng = np.random.default_rng(11)
    for _ in range(8):
        x = (rng.standard_normal(128) * 3).astype(np.float16)
        suh = rng.uniform(0.5, 1.5, 128).astype(np.float16)
        xt = np.zeros(128, np.float32)
        xf = x.astype(np.float32)
        su = np.ascontiguousarray(suh.view(np.uint16))
        ref.ref_prep_block(xf.ctypes.data, su.ctypes.data, xt.ctypes.data)
        assert np.array_equal(oracle.prep(x, suh).astype(np.float32), xt)
