"""Pins the oracle's DCT restatement (crates/haagenti-core/src/dct.rs) and the
retention rules (crates/haagenti/src/compressive.rs).

Checks: the specification's published test vectors
(docs/HCT-SPECIFICATION-DRAFT.md:239-300,497-512), the f64 closed form,
Parseval, round trips from dct.rs:447-492, and the reference's own compiled
C implementation (ref/c/hct_decoder.h via oracle/_ref).
"""
import numpy as np
import pytest

import oracle_lib as O

SEQ4_DCT = np.array([34.0, -4.460888, 0.000005, -0.317031,
                     -17.843542, 0.0, 0.0, 0.0,
                     0.000008, 0.0, 0.0, 0.0,
                     -1.268111, 0.0, 0.0, 0.0], np.float32).reshape(4, 4)
SEQ4_RECON = np.array([[1.000000, 2.000000, 2.999998, 4.000002],
                       [5.000000, 6.000001, 6.999998, 8.000004],
                       [8.999995, 9.999996, 10.999992, 11.999998],
                       [13.000005, 14.000007, 15.000001, 16.000008]], np.float32)


def _seq4():
    return np.arange(1, 17, dtype=np.float32).reshape(4, 4)


@pytest.mark.parametrize("fn", ["dct_2d", "reference_dct_2d", "dct_2d_f64"])
def test_sequential_4x4_coefficients(fn):
    c = getattr(O, fn)(_seq4())
    assert np.abs(c - SEQ4_DCT).max() < 1e-4


def test_sequential_4x4_retained_indices_and_reconstruction():
    c = O.reference_dct_2d(_seq4())
    bm, idx = O.topk_bitmap(c.ravel(), 8)
    order = sorted(range(16), key=lambda i: (-abs(float(c.ravel()[i])), i))
    assert order[:5] == [0, 4, 1, 12, 3]  # spec B.1 retained_indices (robust part)
    sparse = np.zeros(16, np.float32)
    sparse[idx] = c.ravel()[idx]
    r = O.reference_idct_2d(sparse.reshape(4, 4))
    assert np.abs(r - SEQ4_RECON).max() < 1e-4
    assert np.abs(O.idct_2d(sparse.reshape(4, 4)) - SEQ4_RECON).max() < 1e-4


def test_constant_4x4_dc_only():
    c = O.dct_2d(np.full((4, 4), 42.0, np.float32))
    assert abs(c[0, 0] - 168.0) < 1e-4
    assert np.abs(c.ravel()[1:]).max() < 1e-4


@pytest.mark.parametrize("n", [4, 8, 32, 33, 48, 64, 100, 128, 448, 4096])
def test_1d_vs_f64_closed_form(n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 1, n).astype(np.float32)
    d32, d64 = O.dct_1d(x), O.dct_1d_f64(x.astype(np.float64))
    i32, i64 = O.idct_1d(x), O.idct_1d_f64(x.astype(np.float64))
    scale = np.abs(d64).max()
    assert np.abs(d32 - d64).max() < 2e-5 * scale * max(1.0, np.log2(n) / 6)
    assert np.abs(i32 - i64).max() < 2e-5 * np.abs(i64).max() * max(1.0, np.log2(n) / 6)


def test_f64_parseval_and_inverse():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (64, 64))
    c = O.dct_2d_f64(x)
    assert abs((c ** 2).sum() - (x ** 2).sum()) < 1e-9 * (x ** 2).sum()
    assert np.abs(O.idct_2d_f64(c) - x).max() < 1e-12


def test_f64_closed_form_single_basis():
    # A single coefficient (u, v) reconstructs alpha_u alpha_v cos(.) cos(.)
    n = 64
    c = np.zeros((n, n))
    c[3, 5] = 1.0
    x = O.idct_2d_f64(c)
    i = np.arange(n)
    cu = np.sqrt(2 / n) * np.cos(np.pi * (2 * i + 1) * 3 / (2 * n))
    cv = np.sqrt(2 / n) * np.cos(np.pi * (2 * i + 1) * 5 / (2 * n))
    assert np.abs(x - np.outer(cu, cv)).max() < 1e-14


def test_roundtrips_from_reference_tests():
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    assert np.abs(O.idct_1d(O.dct_1d(x)) - x).max() < 1e-5
    x = np.sin(np.arange(64, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    assert np.abs(O.idct_1d(O.dct_1d(x)) - x).max() < 1e-4
    x = np.sin(np.arange(64, dtype=np.float32) * np.float32(0.1)).reshape(8, 8).astype(np.float32)
    assert np.abs(O.idct_2d(O.dct_2d(x)) - x).max() < 1e-4


def test_direct_small_sizes_match_fft_path_math():
    # n <= 32 uses the direct form; n = 64 the Makhoul path.  Both equal the
    # f64 closed form, hence each other.
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 32).astype(np.float32)
    assert np.abs(O.idct_1d_direct(x) - O.idct_1d_f64(x.astype(np.float64))).max() < 1e-5


@pytest.mark.skipif(not O.ref_available(), reason="reference C decoder not built")
def test_idct_2d_vs_reference_c_decoder():
    rng = np.random.default_rng(4)
    for shape in [(64, 64), (8, 8), (64, 128)]:
        x = rng.normal(0, 0.02, shape).astype(np.float32)
        mine = O.idct_2d(x)
        ref = O.ref_idct_2d(x)
        assert np.abs(mine - ref).max() < 2e-6 * np.abs(ref).max() * 8
        mine = O.dct_2d(x)
        ref = O.ref_dct_2d(x)
        assert np.abs(mine - ref).max() < 2e-6 * np.abs(ref).max() * 8


@pytest.mark.parametrize("shape,threads", [((1, 64), 4), ((37, 53), 3), ((256, 64), 16), ((96, 640), 0),
                                           ((1000, 24), 7)])
def test_idct_2d_threaded_equals_one_thread(shape, threads):
    # the threaded form used for real-size GPU checks splits rows and then
    # columns over threads; every 1-D transform is the one-thread code, so
    # the result must be identical bit for bit (odd, tall, wide and
    # non-power-of-two shapes; more threads than rows)
    rng = np.random.default_rng(shape[0] * 31 + shape[1])
    x = rng.normal(0, 1, shape).astype(np.float32)
    assert np.array_equal(O.idct_2d_mt(x, threads).view(np.uint32), O.idct_2d(x).view(np.uint32))


# ---------------------------------------------------------------- retention
def test_retain_count():
    assert O.retain_count(4096, 0.3) == 1228
    assert O.retain_count(4096, 0.25) == 1024
    assert O.retain_count(4096, 0.01) == 204      # clamped to 0.05
    assert O.retain_count(4096, 2.0) == 4096      # clamped to 1.0
    assert O.retain_count(1, 0.05) == 1           # max(1)
    assert O.retain_count(16, 0.5) == 8


def test_topk_bitmap_brute_force():
    rng = np.random.default_rng(6)
    for n in [1, 7, 16, 63, 200, 4096]:
        c = rng.normal(0, 1, n).astype(np.float32)
        c[rng.integers(0, n, n // 4)] = np.float32(0.5)  # ties
        c[rng.integers(0, n, n // 8)] = -np.float32(0.5)
        for k in sorted({1, max(1, n // 3), n}):
            bm, idx = O.topk_bitmap(c, k)
            expect = sorted(sorted(range(n), key=lambda i: (-abs(float(c[i])), i))[:k])
            assert list(idx) == expect
            eb = np.zeros((n + 7) // 8, np.uint8)
            for i in expect:
                eb[i // 8] |= 1 << (i % 8)
            assert (bm == eb).all()
            assert list(O.bitmap_index_map(bm, n)) == expect
