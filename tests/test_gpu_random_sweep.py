"""Seeded random sweep of decode and chunked-prefill parity against the CPU
oracle: shapes, GQA ratios, cache dtypes, context mixes (empty, single-token,
partial blocks, holes in the tables), scales and decode modes drawn per case,
so that combinations the parametrized tests do not enumerate are exercised.
Tolerances as in the other attention tests (bf16/f16 KV 2e-2 + 1e-2|b|, FP8 KV
5e-2 + 5e-2|b|, against the oracle's float64 result)."""
import numpy as np
import pytest
import torch

import oracle as O
import rllm_amd
from gpu_util import f32, log_case, t16, t8, ti
from helpers import TOL_BF16, TOL_FP8, assert_close, random_case
from rllm_amd import ops

pytestmark = pytest.mark.gpu
TORCH = {O.BF16: torch.bfloat16, O.F16: torch.float16}
ABI = {O.F16: rllm_amd.DTYPE_F16, O.BF16: rllm_amd.DTYPE_BF16, O.FP8_E4M3: rllm_amd.DTYPE_FP8_E4M3,
       O.FP8_E5M2: rllm_amd.DTYPE_FP8_E5M2}
FP8 = (O.FP8_E4M3, O.FP8_E5M2)


def _draw(rng):
    D = int(rng.choice([64, 128]))
    G = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    q_kind = int(rng.choice([O.BF16, O.F16]))
    kv_kind = int(rng.choice([q_kind, q_kind, O.FP8_E4M3, O.FP8_E5M2]))
    return D, G, hkv, q_kind, kv_kind


def _encode_kv(k, v, kv_kind, rng):
    if kv_kind in FP8:
        top = 448.0 if kv_kind == O.FP8_E4M3 else 57344.0
        ks = float(np.abs(k).max() / top) * float(rng.uniform(1.0, 4.0))
        vs = float(np.abs(v).max() / top) * float(rng.uniform(1.0, 4.0))
        return (O.encode((k / np.float32(ks)).astype(np.float32), kv_kind),
                O.encode((v / np.float32(vs)).astype(np.float32), kv_kind), ks, vs)
    return O.encode(k, kv_kind), O.encode(v, kv_kind), 1.0, 1.0


def _kv(bits, kind, dev):
    return t8(bits, dev) if kind in FP8 else t16(bits, TORCH[kind], dev)


@pytest.mark.parametrize("case", range(48))
def test_decode_random_sweep(dev, case):
    rng = np.random.default_rng(1000 + case)
    D, G, hkv, q_kind, kv_kind = _draw(rng)
    B = int(rng.integers(1, 41))
    hi = int(rng.choice([40, 700, 3000]))
    q, k, v, bt, sl = random_case(rng, B, hkv * G, hkv, D, (0, hi), neg_blocks=int(rng.integers(0, 3)))
    if B > 2:
        sl[rng.integers(0, B)] = 0                 # an empty sequence
        sl[rng.integers(0, B)] = 1                 # a single token
    qb = O.encode(q, q_kind)
    kb, vb, ks, vs = _encode_kv(k, v, kv_kind, rng)
    scale = float(rng.uniform(0.03, 0.2))
    part = int(rng.choice([0, 0, -1, 512, 1024]))
    log_case(f"decode sweep {case}: D={D} G={G} hkv={hkv} q={q_kind} kv={kv_kind} B={B} "
             f"ctx<={hi} part={part}")
    ref = O.paged_attention_decode(qb, q_kind, kb, vb, kv_kind, bt, sl, scale, ks, vs, precision=1)
    out = ops.paged_decode(t16(qb, TORCH[q_kind], dev), _kv(kb, kv_kind, dev), _kv(vb, kv_kind, dev),
                           ti(bt, torch.int32, dev), ti(sl, torch.int32, dev), scale, kv_dtype=ABI[kv_kind],
                           k_scale=ks, v_scale=vs, partition_size=part)
    torch.cuda.synchronize()
    got = f32(out)
    assert_close(got, ref, TOL_FP8 if kv_kind in FP8 else TOL_BF16, f"decode sweep {case}")
    for s in np.flatnonzero(sl == 0):
        assert np.all(got[s] == 0)


@pytest.mark.parametrize("case", range(32))
def test_prefill_random_sweep(dev, case):
    rng = np.random.default_rng(2000 + case)
    D, G, hkv, q_kind, kv_kind = _draw(rng)
    hkv = min(hkv, 4)
    B = int(rng.integers(1, 6))
    n_new = rng.integers(1, 300, size=B).astype(np.int32)
    cached = rng.integers(0, 800, size=B).astype(np.int32)
    cached[rng.random(B) < 0.3] = 0                # some fresh prompts
    sl = n_new + cached
    bs = 16
    nblk = (sl + bs - 1) // bs
    pool = int(nblk.sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, int(nblk.max())), -1, np.int32)
    p = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[p:p + nblk[s]]
        p += nblk[s]
    qsl = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    T = int(qsl[-1])
    q = rng.standard_normal((T, hkv * G, D)).astype(np.float32)
    k = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    v = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    qb = O.encode(q, q_kind)
    kb, vb, ks, vs = _encode_kv(k, v, kv_kind, rng)
    scale = float(rng.uniform(0.03, 0.2))
    log_case(f"prefill sweep {case}: D={D} G={G} hkv={hkv} q={q_kind} kv={kv_kind} B={B} T={T}")
    ref = O.paged_attention_prefill(qb, q_kind, kb, vb, kv_kind, bt, sl, qsl, scale, ks, vs, precision=1)
    out = ops.paged_prefill(t16(qb, TORCH[q_kind], dev), _kv(kb, kv_kind, dev), _kv(vb, kv_kind, dev),
                            ti(bt, torch.int32, dev), ti(sl, torch.int32, dev), ti(qsl, torch.int32, dev),
                            scale, kv_dtype=ABI[kv_kind], k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert_close(f32(out), ref, TOL_FP8 if kv_kind in FP8 else TOL_BF16, f"prefill sweep {case}")
