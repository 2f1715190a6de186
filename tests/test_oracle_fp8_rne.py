"""Pinning of the oracle's nearest-even FP8 encoders (the library's opt-in
rounding for cache writes; the reference contract, cache_ops.cu:13-46, 75-103,
rounds toward zero and is pinned in test_oracle_fp8.py).

The oracle computes the quantum at |x| in double arithmetic and rounds with
rint(); the library encodes with integer bit manipulation.  What pins the
oracle, independently of both:
  * the nearest-even characterisation over all 2^32 float32 patterns, written
    against the decoder only: the chosen code is no farther from x (clamped to
    the largest finite value) than either neighbouring code, and on a tie it
    is even (codes are monotone in value, so local optimality is global);
  * every finite FP8 value encodes back to its own byte;
  * hand-derived known answers at ties, binade and subnormal boundaries and
    saturation."""
import os

import numpy as np
import pytest

import oracle as O


def _f32(vals):
    return np.array(vals, dtype=np.float32)


@pytest.mark.parametrize("e5m2", [False, True], ids=["e4m3", "e5m2"])
def test_rne_exhaustive_characterisation(e5m2):
    bad, first = O.fp8_rne_exhaustive(e5m2, nthreads=max(1, min(16, os.cpu_count() or 1)))
    assert bad == 0, f"{bad} violations, first pattern 0x{first:08x}"


@pytest.mark.parametrize("kind", [O.FP8_E4M3, O.FP8_E5M2], ids=["e4m3", "e5m2"])
def test_rne_round_trips_every_finite_value(kind):
    codes = np.arange(256, dtype=np.uint8)
    vals = O.decode(codes, kind)
    finite = np.isfinite(vals)
    back = O.encode_fp8_rne(vals[finite], kind)
    np.testing.assert_array_equal(back, codes[finite])


def test_rne_known_answers_e4m3():
    x = _f32([1.0, 1.0625, 1.1875, 448.0, 449.0, 464.0, 1e9, np.inf, -np.inf, np.nan,
              2.0 ** -6, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -10, 7.5 * 2.0 ** -9, -2.0 ** -12, -0.0])
    want = [0x38,   # 1.0
            0x38,   # 1 + 1/16: tie between 0x38 and 0x39 -> even
            0x3A,   # 1 + 3/16: tie between 0x39 and 0x3A -> even
            0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE,   # saturation at 448, incl. infinities
            0x7F,   # NaN
            0x08,   # smallest normal
            0x01,   # smallest subnormal
            0x00,   # half the smallest subnormal: tie -> even (zero)
            0x01,   # 0.75 of the smallest subnormal
            0x08,   # 7.5 quanta: tie between 0x07 and 0x08 -> even
            0x80,   # tiny negative rounds to -0
            0x80]
    np.testing.assert_array_equal(O.encode_fp8_rne(x, O.FP8_E4M3), np.array(want, np.uint8))


def test_rne_known_answers_e5m2():
    x = _f32([1.0, 1.125, 1.375, 448.0, 480.0, 57344.0, 61439.0, 61440.0, np.inf, np.nan,
              2.0 ** -14, 2.0 ** -16, 2.0 ** -17, 3 * 2.0 ** -18, -3.5 * 2.0 ** -16])
    want = [0x3C,
            0x3C,   # 1 + 1/8: tie between 0x3C and 0x3D -> even
            0x3E,   # 1 + 3/8: tie between 0x3D and 0x3E -> even
            0x5F,   # 448 = 1.75 * 2^8
            0x60,   # 480: tie between 0x5F and 0x60 -> even
            0x7B, 0x7B, 0x7B, 0x7B,   # saturation at 57344, incl. inf
            0x7F,
            0x04,   # smallest normal
            0x01,   # smallest subnormal
            0x00,   # tie -> even
            0x01,   # 0.75 quanta
            0x84]   # -3.5 quanta: tie between 3 and 4 -> even (4 = smallest normal)
    np.testing.assert_array_equal(O.encode_fp8_rne(x, O.FP8_E5M2), np.array(want, np.uint8))


@pytest.mark.parametrize("kind", [O.FP8_E4M3, O.FP8_E5M2], ids=["e4m3", "e5m2"])
def test_rne_is_unbiased_where_truncation_shrinks(kind):
    # over values spread across the normal range, nearest-even keeps the mean
    # magnitude; round toward zero (the reference contract) shrinks it
    rng = np.random.default_rng(5)
    x = rng.standard_normal(200_000).astype(np.float32) * (64.0 if kind == O.FP8_E4M3 else 4096.0)
    rne = O.decode(O.encode_fp8_rne(x, kind), kind).astype(np.float64)
    rtz = O.decode(O.encode(x, kind), kind).astype(np.float64)
    ax = np.abs(x).astype(np.float64)
    assert abs(np.abs(rne).sum() / ax.sum() - 1) < 5e-3
    assert np.abs(rtz).sum() / ax.sum() < 0.98


def test_cache_write_rounded_matches_encoder():
    rng = np.random.default_rng(9)
    nb, hkv, d, bs, n = 4, 2, 8, 4, 5
    kc = np.zeros((nb, hkv, d, bs), np.uint8)
    vc = np.zeros_like(kc)
    nk = O.encode(rng.standard_normal((n, hkv, d)).astype(np.float32), O.BF16)
    nv = O.encode(rng.standard_normal((n, hkv, d)).astype(np.float32), O.BF16)
    slots = np.array([0, 5, -1, 14, 15], np.int64)
    ks, vs = 0.01, 0.003
    O.cache_write(kc, vc, nk, nv, slots, bs, O.BF16, O.FP8_E4M3, ks, vs, round_nearest=True)
    kx, vx = O.decode(nk, O.BF16) / np.float32(ks), O.decode(nv, O.BF16) / np.float32(vs)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        np.testing.assert_array_equal(kc[s // bs, :, :, s % bs], O.encode_fp8_rne(kx[t], O.FP8_E4M3))
        np.testing.assert_array_equal(vc[s // bs, :, :, s % bs], O.encode_fp8_rne(vx[t], O.FP8_E4M3))
    assert not kc[0, :, :, 2].any()   # untouched slot
