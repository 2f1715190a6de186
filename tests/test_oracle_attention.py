"""Pins the oracle's decode / prefill attention (oracle.c) against an
independent dense numpy float64 formulation, closed-form invariants, and the
committed golden fixtures (tests/golden/)."""
import glob
import os

import numpy as np
import pytest

import oracle as O
from helpers import dense_decode_f64, dense_prefill_f64, random_case

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _decode(q, k, v, bt, sl, scale, kind=O.BF16, precision=1, k_scale=1.0, v_scale=1.0):
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, kind), O.encode(v, kind)
    return O.paged_attention_decode(qb, O.BF16, kb, vb, kind, bt, sl, scale, k_scale, v_scale,
                                    precision=precision)


@pytest.mark.parametrize("hq,hkv,D", [(32, 8, 64), (8, 8, 128), (16, 2, 64), (4, 1, 16)])
def test_decode_matches_dense_numpy(hq, hkv, D):
    rng = np.random.default_rng(hq * 7 + D)
    q, k, v, bt, sl = random_case(rng, 5, hq, hkv, D, (1, 70), neg_blocks=2)
    sl[0] = 0
    qf = O.decode(O.encode(q, O.BF16), O.BF16)
    kf = O.decode(O.encode(k, O.BF16), O.BF16)
    vf = O.decode(O.encode(v, O.BF16), O.BF16)
    scale = 1 / np.sqrt(D)
    ref = dense_decode_f64(qf, kf, vf, bt, sl, scale)
    got64 = _decode(q, k, v, bt, sl, scale, precision=1)
    got32 = _decode(q, k, v, bt, sl, scale, precision=0)
    assert np.max(np.abs(got64 - ref)) < 1e-6
    assert np.max(np.abs(got32 - ref)) < 2e-5
    assert np.all(got64[0] == 0)          # empty context writes zeros


def test_decode_closed_forms():
    rng = np.random.default_rng(21)
    q, k, v, bt, sl = random_case(rng, 4, 8, 2, 32, (20, 60))
    scale = 0.2
    # constant V rows per kv head -> output equals that row
    row = rng.standard_normal((2, 32)).astype(np.float32)
    vc = np.broadcast_to(row[None, :, :, None], v.shape).copy()
    out = _decode(q, k, vc, bt, sl, scale)
    vrow = O.decode(O.encode(row, O.BF16), O.BF16)
    for h in range(2):
        assert np.allclose(out[:, h * 4:(h + 1) * 4], vrow[h], atol=1e-6)
    # context 1 -> output is that token's V
    sl1 = np.ones_like(sl)
    out = _decode(q, k, v, bt, sl1, scale)
    vf = O.decode(O.encode(v, O.BF16), O.BF16)
    for s in range(4):
        for hq in range(8):
            assert np.allclose(out[s, hq], vf[bt[s, 0], hq // 4, :, 0], atol=1e-7)
    # identical q inside a GQA group -> identical outputs
    qs = q.copy()
    qs[:, 1] = qs[:, 0]
    out = _decode(qs, k, v, bt, sl, scale)
    assert np.array_equal(out[:, 0], out[:, 1])


def test_decode_block_permutation_invariance():
    rng = np.random.default_rng(31)
    q, k, v, bt, sl = random_case(rng, 3, 8, 2, 64, (30, 90))
    nb = k.shape[0]
    perm = rng.permutation(nb)
    inv = np.argsort(perm)
    k2, v2 = k[perm], v[perm]
    bt2 = np.where(bt >= 0, inv[np.maximum(bt, 0)], -1).astype(np.int32)
    a = _decode(q, k, v, bt, sl, 0.125)
    b = _decode(q, k2, v2, bt2, sl, 0.125)
    assert np.array_equal(a, b)


def test_decode_aliased_prefix_equals_copies():
    rng = np.random.default_rng(41)
    B, hq, hkv, D, bs = 3, 4, 1, 32, 16
    shared = rng.standard_normal((2, 2, hkv, D, bs)).astype(np.float32)   # 2 prefix blocks
    uniq = rng.standard_normal((2, B, hkv, D, bs)).astype(np.float32)
    # aliased pool: [p0, p1, u0, u1, u2]; copied pool: per sequence its own copies
    ka = np.concatenate([shared[0], uniq[0]])
    va = np.concatenate([shared[1], uniq[1]])
    bta = np.array([[0, 1, 2 + s] for s in range(B)], np.int32)
    kc = np.concatenate([np.concatenate([shared[0], uniq[0][s:s + 1]]) for s in range(B)])
    vc = np.concatenate([np.concatenate([shared[1], uniq[1][s:s + 1]]) for s in range(B)])
    btc = np.array([[3 * s, 3 * s + 1, 3 * s + 2] for s in range(B)], np.int32)
    q = rng.standard_normal((B, hq, D)).astype(np.float32)
    sl = np.array([40, 48, 33], np.int32)
    assert np.array_equal(_decode(q, ka, va, bta, sl, 0.3), _decode(q, kc, vc, btc, sl, 0.3))


def test_decode_fp8_scaled_matches_dense():
    rng = np.random.default_rng(51)
    q, k, v, bt, sl = random_case(rng, 3, 8, 2, 64, (10, 50))
    ks, vs = 0.05, 0.02
    for kind in (O.FP8_E4M3, O.FP8_E5M2):
        kb = O.encode((k / ks).astype(np.float32), kind)
        vb = O.encode((v / vs).astype(np.float32), kind)
        qf = O.decode(O.encode(q, O.BF16), O.BF16)
        ref = dense_decode_f64(qf, O.decode(kb, kind) * np.float32(ks), O.decode(vb, kind) * np.float32(vs),
                               bt, sl, 0.125)
        got = O.paged_attention_decode(O.encode(q, O.BF16), O.BF16, kb, vb, kind, bt, sl, 0.125,
                                       ks, vs, precision=1)
        assert np.max(np.abs(got - ref)) < 1e-6


def test_prefill_matches_dense_numpy_and_reference_without_context():
    rng = np.random.default_rng(61)
    B, hq, hkv, D, bs = 3, 8, 2, 32, 16
    n_new = np.array([5, 17, 1], np.int32)
    cached = np.array([0, 20, 33], np.int32)
    sl = n_new + cached
    nblk = (sl + bs - 1) // bs
    pool = int(nblk.sum()) + 2
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, int(nblk.max())), -1, np.int32)
    p = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[p:p + nblk[s]]
        p += nblk[s]
    qsl = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    T = int(qsl[-1])
    q = rng.standard_normal((T, hq, D)).astype(np.float32)
    k = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    v = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    got = O.paged_attention_prefill(qb, O.BF16, kb, vb, O.BF16, bt, sl, qsl, 0.17, precision=1)
    ref = dense_prefill_f64(O.decode(qb, O.BF16), O.decode(kb, O.BF16), O.decode(vb, O.BF16), bt,
                            sl, qsl, 0.17)
    assert np.max(np.abs(got - ref)) < 1e-6
    # sequence 0 has no cached context: the context-offset causal mask reduces to
    # the reference kernel's chunk-relative mask (paged_attention.cu:285-286);
    # its last token attends the whole chunk, i.e. equals a decode at ctx = n.
    dec = O.paged_attention_decode(qb[qsl[0] + 4:qsl[0] + 5], O.BF16, kb, vb, O.BF16, bt[:1],
                                   np.array([5], np.int32), 0.17, precision=1)
    assert np.array_equal(dec[0], got[4])


def test_golden_fixtures_reproduce():
    files = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))
    assert files, "no golden fixtures committed"
    for f in files:
        z = np.load(f)
        if "kv_kind" not in z:
            continue
        kind = int(z["kv_kind"])
        if "query_start_loc" in z:
            got = O.paged_attention_prefill(z["q"], int(z["q_kind"]), z["k_cache"], z["v_cache"],
                                            kind, z["block_tables"], z["seq_lens"],
                                            z["query_start_loc"], float(z["scale"]),
                                            float(z["k_scale"]), float(z["v_scale"]), precision=1)
        else:
            got = O.paged_attention_decode(z["q"], int(z["q_kind"]), z["k_cache"], z["v_cache"],
                                           kind, z["block_tables"], z["seq_lens"], float(z["scale"]),
                                           float(z["k_scale"]), float(z["v_scale"]), precision=1)
        assert np.max(np.abs(got - z["expected"])) < 1e-6, os.path.basename(f)


def test_golden_fp8_codec_table():
    z = np.load(os.path.join(GOLDEN, "fp8_codec.npz"))
    assert np.array_equal(O.encode(z["x"], O.FP8_E4M3), z["e4m3"])
    assert np.array_equal(O.encode(z["x"], O.FP8_E5M2), z["e5m2"])
