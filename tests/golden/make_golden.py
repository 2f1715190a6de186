"""Writes the small golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Each fixture holds seeded inputs as element bit patterns plus expected outputs
computed by the dense numpy float64 formulation in tests/helpers.py (not by the
C oracle), so the fixtures pin the oracle and the GPU path alike.  The
reference ships no numeric fixtures for this path, so every expected value here
comes from the mathematics of softmax(scale q.K^T) V over the paged layout
[num_blocks, kv_heads, head_dim, block_size] (paged_attention.cu:82-86).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))               # tests/
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root

import oracle as O  # noqa: E402  (codec only: bits <-> float)
from helpers import dense_decode_f64, dense_prefill_f64, random_case  # noqa: E402


def decode_case(name, seed, B, hq, hkv, D, ctx_range, q_kind, kv_kind, k_scale=1.0, v_scale=1.0,
                neg_blocks=0):
    rng = np.random.default_rng(seed)
    q, k, v, bt, sl = random_case(rng, B, hq, hkv, D, ctx_range, neg_blocks=neg_blocks)
    qb = O.encode(q, q_kind)
    kb = O.encode((k / np.float32(k_scale)).astype(np.float32), kv_kind)
    vb = O.encode((v / np.float32(v_scale)).astype(np.float32), kv_kind)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exp = dense_decode_f64(O.decode(qb, q_kind), O.decode(kb, kv_kind) * np.float32(k_scale),
                           O.decode(vb, kv_kind) * np.float32(v_scale), bt, sl, scale)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), q=qb, k_cache=kb, v_cache=vb,
                        block_tables=bt, seq_lens=sl, scale=np.float32(scale),
                        k_scale=np.float32(k_scale), v_scale=np.float32(v_scale),
                        q_kind=np.int32(q_kind), kv_kind=np.int32(kv_kind),
                        expected=exp.astype(np.float32))


def prefill_case(name, seed, n_new, cached, hq, hkv, D, kind):
    rng = np.random.default_rng(seed)
    bs = 16
    n_new = np.array(n_new, np.int32)
    sl = n_new + np.array(cached, np.int32)
    nblk = (sl + bs - 1) // bs
    pool = int(nblk.sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((len(sl), int(nblk.max())), -1, np.int32)
    p = 0
    for s in range(len(sl)):
        bt[s, :nblk[s]] = perm[p:p + nblk[s]]
        p += nblk[s]
    qsl = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    T = int(qsl[-1])
    qb = O.encode(rng.standard_normal((T, hq, D)).astype(np.float32), kind)
    kb = O.encode(rng.standard_normal((pool, hkv, D, bs)).astype(np.float32), kind)
    vb = O.encode(rng.standard_normal((pool, hkv, D, bs)).astype(np.float32), kind)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exp = dense_prefill_f64(O.decode(qb, kind), O.decode(kb, kind), O.decode(vb, kind), bt, sl, qsl,
                            scale)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), q=qb, k_cache=kb, v_cache=vb,
                        block_tables=bt, seq_lens=sl, query_start_loc=qsl, scale=np.float32(scale),
                        k_scale=np.float32(1.0), v_scale=np.float32(1.0), q_kind=np.int32(kind),
                        kv_kind=np.int32(kind), expected=exp.astype(np.float32))


def fp8_table():
    """Encoder fixture: float inputs and the bytes of both FP8 encoders, plus
    the decode of every byte, for the GPU reshape_and_cache / decode paths."""
    rng = np.random.default_rng(77)
    x = np.concatenate([
        np.array([0.0, -0.0, 1.0, -2.0, 448.0, 460.0, 479.9, 480.0, 500.0, 511.9, 512.0, 1e4,
                  57344.0, 6e4, 1e6, 2.0 ** -6, 2.0 ** -7, -(2.0 ** -7), 2.0 ** -14, 2.0 ** -15,
                  1.9375, 1.99, 3.0, 0.1, np.inf, -np.inf], np.float32),
        (rng.standard_normal(4000) * 10.0 ** rng.uniform(-5, 3, 4000)).astype(np.float32),
    ])
    np.savez_compressed(os.path.join(HERE, "fp8_codec.npz"), x=x,
                        e4m3=O.encode(x, O.FP8_E4M3), e5m2=O.encode(x, O.FP8_E5M2),
                        dec_e4m3=O.decode(np.arange(256, dtype=np.uint8), O.FP8_E4M3),
                        dec_e5m2=O.decode(np.arange(256, dtype=np.uint8), O.FP8_E5M2))


def main():
    decode_case("decode_bf16_gqa4_d64", 101, 3, 8, 2, 64, (1, 70), O.BF16, O.BF16, neg_blocks=1)
    decode_case("decode_bf16_gqa4_d128", 102, 2, 8, 2, 128, (17, 300), O.BF16, O.BF16)
    decode_case("decode_f16_mha_d64", 103, 2, 4, 4, 64, (1, 40), O.F16, O.F16)
    decode_case("decode_fp8e4m3_gqa4_d128", 104, 2, 8, 2, 128, (30, 200), O.BF16, O.FP8_E4M3,
                k_scale=4.0 / 448.0, v_scale=4.5 / 448.0)
    decode_case("decode_fp8e5m2_gqa8_d64", 105, 2, 8, 1, 64, (5, 90), O.F16, O.FP8_E5M2)
    prefill_case("prefill_bf16_gqa4_d128", 106, [9, 17], [20, 0], 8, 2, 128, O.BF16)
    prefill_case("prefill_f16_gqa2_d64", 107, [33, 3, 16], [0, 40, 16], 4, 2, 64, O.F16)
    fp8_table()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
