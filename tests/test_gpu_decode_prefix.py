"""The cascade decode over a shared prefix (rllm_paged_attention_decode_prefix_ex)
against the oracle's decode on the same tables.

The batch's tables start with the same physical blocks, the prefix sharing
that block_pool.rs:292-302 hands out and AttentionMetadata's
detect_common_prefix_blocks (attention.rs:204-226) finds.  The library attends
the prefix once for the whole batch with matrix cores, attends each
sequence's own blocks separately and merges the two, so these tests compare
it with the oracle's plain decode of the aliased tables (the oracle knows
nothing of the prefix): shapes, cache types, contexts that end inside the
prefix or right at its end, empty contexts, long suffixes split into several
partitions, and config 4a at its own size.

The entry point runs the plain decode where the prefix saves too little; the
tests of the cascade itself force it with RLLM_CASCADE=always, and
test_prefix_auto_choice_follows_the_rule checks the choice."""
import numpy as np
import pytest
import torch

import oracle as O
import rllm_amd
from gpu_util import f32, log_case, t16, t8, ti
from helpers import TOL_BF16, TOL_FP8, assert_close
from rllm_amd import ops, workloads

pytestmark = pytest.mark.gpu
TORCH = {O.BF16: torch.bfloat16, O.F16: torch.float16}


@pytest.fixture(autouse=True)
def _force_cascade(monkeypatch):
    """These small batches would run the plain decode by the entry point's own
    choice; the cascade kernel is what they test."""
    monkeypatch.setenv("RLLM_CASCADE", "always")
ABI = {O.F16: rllm_amd.DTYPE_F16, O.BF16: rllm_amd.DTYPE_BF16, O.FP8_E4M3: rllm_amd.DTYPE_FP8_E4M3,
       O.FP8_E5M2: rllm_amd.DTYPE_FP8_E5M2}


def prefix_case(rng, B, hq, hkv, D, P, suffix_range, bs=16):
    """B sequences whose tables start with the same P physical blocks, then
    blocks of their own; context P * bs + U[suffix_range] tokens."""
    lo, hi = suffix_range
    sl = (P * bs + rng.integers(lo, hi, size=B, endpoint=True)).astype(np.int32)
    nblk = (sl + bs - 1) // bs
    maxb = max(int(nblk.max()), P, 1)
    pool = P + int(np.maximum(nblk - P, 0).sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, maxb), -1, np.int32)
    bt[:, :P] = perm[:P]
    p = P
    for s in range(B):
        n = max(int(nblk[s]) - P, 0)
        bt[s, P:P + n] = perm[p:p + n]
        p += n
    q = rng.standard_normal((B, hq, D)).astype(np.float32)
    k = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    v = rng.standard_normal((pool, hkv, D, bs)).astype(np.float32)
    return q, k, v, bt, sl


def _kv(bits, kind, dev):
    return t8(bits, dev) if kind in (O.FP8_E4M3, O.FP8_E5M2) else t16(bits, TORCH[kind], dev)


def run_prefix(dev, qb, q_kind, kb, vb, kv_kind, bt, sl, scale, P, k_scale=1.0, v_scale=1.0, label=""):
    q = t16(qb, TORCH[q_kind], dev)
    kc, vc = _kv(kb, kv_kind, dev), _kv(vb, kv_kind, dev)
    log_case(f"decode prefix {label} q={q_kind} kv={kv_kind} B={qb.shape[0]} Hq={qb.shape[1]} "
             f"D={qb.shape[2]} Hkv={kb.shape[1]} P={P}")
    out = ops.paged_decode_prefix(q, kc, vc, ti(bt, torch.int32, dev), ti(sl, torch.int32, dev), scale, P,
                                  kv_dtype=ABI[kv_kind], k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    return f32(out)


def oracle_ref(qb, q_kind, kb, vb, kv_kind, bt, sl, scale, k_scale=1.0, v_scale=1.0):
    return O.paged_attention_decode(qb, q_kind, kb, vb, kv_kind, bt, sl, scale, k_scale, v_scale, precision=1)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("kind", [O.BF16, O.F16])
def test_prefix_shapes_vs_oracle(dev, D, G, kind):
    """Nine sequences on a 5-block prefix with 0 to 70 tokens of their own
    (a suffix of 0 tokens ends the context at the prefix's end)."""
    rng = np.random.default_rng(500 + D + 10 * G + kind)
    hkv = 2
    q, k, v, bt, sl = prefix_case(rng, 9, hkv * G, hkv, D, 5, (0, 70))
    sl[0] = 5 * 16
    qb, kb, vb = O.encode(q, kind), O.encode(k, kind), O.encode(v, kind)
    scale = 1 / np.sqrt(D)
    ref = oracle_ref(qb, kind, kb, vb, kind, bt, sl, scale)
    got = run_prefix(dev, qb, kind, kb, vb, kind, bt, sl, scale, 5, label=f"D={D} G={G}")
    assert_close(got, ref, TOL_BF16, f"prefix D={D} G={G} kind={kind}")


@pytest.mark.parametrize("fp8", [O.FP8_E4M3, O.FP8_E5M2])
def test_prefix_fp8_scaled_vs_oracle(dev, fp8):
    """FP8 caches with per-tensor scales (not powers of two)."""
    rng = np.random.default_rng(611 + fp8)
    q, k, v, bt, sl = prefix_case(rng, 12, 32, 8, 128, 9, (1, 300))
    top = 448.0 if fp8 == O.FP8_E4M3 else 57344.0
    ks, vs = float(np.abs(k).max() / top), float(np.abs(v).max() / top)
    kb = O.encode((k / np.float32(ks)).astype(np.float32), fp8)
    vb = O.encode((v / np.float32(vs)).astype(np.float32), fp8)
    qb = O.encode(q, O.BF16)
    scale = 1 / np.sqrt(128)
    ref = oracle_ref(qb, O.BF16, kb, vb, fp8, bt, sl, scale, ks, vs)
    got = run_prefix(dev, qb, O.BF16, kb, vb, fp8, bt, sl, scale, 9, ks, vs, label="fp8")
    assert_close(got, ref, TOL_FP8, f"prefix fp8={fp8}")


def test_prefix_contexts_inside_the_prefix_and_empty(dev):
    """Contexts that end inside the shared prefix attend only their own tokens
    of it (no suffix partition); an empty context gives a zero row, as the
    plain decode does."""
    rng = np.random.default_rng(707)
    P = 6
    q, k, v, bt, sl = prefix_case(rng, 10, 32, 8, 128, P, (0, 100))
    sl[1] = 1
    sl[2] = 37             # inside the prefix's third block
    sl[3] = P * 16 - 1     # one short of the prefix
    sl[4] = 0
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(128)
    ref = oracle_ref(qb, O.BF16, kb, vb, O.BF16, bt, sl, scale)
    assert np.all(ref[4] == 0)
    got = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, P, label="short contexts")
    assert np.all(got[4] == 0), "the empty context's row is not zero"
    assert_close(got, ref, TOL_BF16, "prefix short contexts")


def test_prefix_long_suffixes_in_several_partitions(dev):
    """Suffixes up to 9,000 tokens: the blocks past the prefix are split into
    several partitions per sequence, merged together with the prefix's."""
    rng = np.random.default_rng(808)
    q, k, v, bt, sl = prefix_case(rng, 6, 32, 8, 128, 20, (3000, 9000))
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(128)
    ref = oracle_ref(qb, O.BF16, kb, vb, O.BF16, bt, sl, scale)
    got = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, 20, label="long suffixes")
    assert_close(got, ref, TOL_BF16, "prefix long suffixes")


def test_prefix_config4a_full_vs_oracle_and_plain_decode(dev):
    """Benchmark config 4a at its own size: 128 sequences on one 64-block
    (1024-token) prefix, 16 blocks of their own each.  Against the oracle,
    and within bf16 rounding of the plain decode of the same tables."""
    w = workloads.config(4)
    assert w.num_seqs == 128 and (w.block_tables[:, :64] == w.block_tables[0, :64]).all()
    qb, kb, vb = workloads.host_tensors(w)
    ref = oracle_ref(qb, O.BF16, kb, vb, O.BF16, w.block_tables, w.seq_lens, w.scale)
    got = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, w.block_tables, w.seq_lens, w.scale, 64, label="config 4a")
    rl2 = assert_close(got, ref, TOL_BF16, "config 4a cascade")
    q = t16(qb, torch.bfloat16, dev)
    plain = f32(ops.paged_decode(q, t16(kb, torch.bfloat16, dev), t16(vb, torch.bfloat16, dev),
                                 ti(w.block_tables, torch.int32, dev), ti(w.seq_lens, torch.int32, dev), w.scale))
    assert np.max(np.abs(got - plain)) <= 2 ** -7 * max(1.0, float(np.abs(plain).max()))
    print(f"config 4a cascade: rel_l2 {rl2:.3e}")


@pytest.mark.parametrize("B,hq,hkv,D,P,suffix", [
    (3, 4, 1, 128, 7, (1, 40)),         # three suffix waves: one wave per suffix workgroup
    (251, 6, 3, 64, 8, (0, 40)),        # several waves per workgroup, the last one partly filled
    (24, 8, 2, 128, 8, (2000, 4000)),   # eight suffix partitions per row
    (2100, 32, 8, 64, 4, (0, 16)),      # the prefix workgroups alone fill the GPU (unsplit prefix)
], ids=["one-wave", "partial-tail", "eight-partitions", "prefix-fills-gpu"])
def test_prefix_single_launch_grids_vs_oracle(dev, B, hq, hkv, D, P, suffix):
    """With 16-bit caches the prefix workgroups and the suffix waves share one
    launch, whose suffix workgroups carry 1 to 8 waves (the suffix items over
    the CUs the prefix leaves free).  Grids of each kind, against the oracle."""
    rng = np.random.default_rng(1200 + B + D)
    q, k, v, bt, sl = prefix_case(rng, B, hq, hkv, D, P, suffix)
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(D)
    ref = oracle_ref(qb, O.BF16, kb, vb, O.BF16, bt, sl, scale)
    got = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, P, label=f"grid B={B}")
    assert_close(got, ref, TOL_BF16, f"prefix grid B={B} Hq={hq} Hkv={hkv} D={D}")


def test_prefix_repeated_calls_give_the_same_bits(dev):
    rng = np.random.default_rng(909)
    q, k, v, bt, sl = prefix_case(rng, 33, 32, 8, 128, 12, (1, 600))
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(128)
    runs = [run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, 12, label=f"repeat {i}") for i in range(3)]
    assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[0], runs[2])


def test_prefix_zero_blocks_and_other_shapes_run_the_plain_decode(dev):
    """num_prefix_blocks 0 is the plain decode (same bits); a head_dim outside
    the tuned set runs the shape-general kernel, still against the oracle."""
    rng = np.random.default_rng(1001)
    q, k, v, bt, sl = prefix_case(rng, 7, 16, 4, 128, 4, (1, 200))
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(128)
    got0 = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, 0, label="no prefix")
    plain = f32(ops.paged_decode(t16(qb, torch.bfloat16, dev), t16(kb, torch.bfloat16, dev),
                                 t16(vb, torch.bfloat16, dev), ti(bt, torch.int32, dev), ti(sl, torch.int32, dev),
                                 scale))
    assert np.array_equal(got0, plain)
    q, k, v, bt, sl = prefix_case(rng, 5, 16, 4, 96, 3, (1, 90))
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    ref = oracle_ref(qb, O.BF16, kb, vb, O.BF16, bt, sl, 0.1)
    got = run_prefix(dev, qb, O.BF16, kb, vb, O.BF16, bt, sl, 0.1, 3, label="head_dim 96")
    assert_close(got, ref, TOL_BF16, "prefix head_dim 96")


def test_prefix_invalid_arguments(dev):
    """A prefix wider than the tables is rejected before any launch, and the
    wrapper refuses tables that do not share the prefix."""
    rng = np.random.default_rng(1102)
    q, k, v, bt, sl = prefix_case(rng, 4, 8, 2, 64, 2, (1, 40))
    qt = t16(O.encode(q, O.BF16), torch.bfloat16, dev)
    kc = t16(O.encode(k, O.BF16), torch.bfloat16, dev)
    vc = t16(O.encode(v, O.BF16), torch.bfloat16, dev)
    btt, slt = ti(bt, torch.int32, dev), ti(sl, torch.int32, dev)
    with pytest.raises(rllm_amd.KernelError):
        ops.paged_decode_prefix(qt, kc, vc, btt, slt, 0.125, bt.shape[1] + 1, validate=False)
    bad = bt.copy()
    bad[1, 0] = bt[0, 1]
    with pytest.raises(ValueError):
        ops.paged_decode_prefix(qt, kc, vc, ti(bad, torch.int32, dev), slt, 0.125, 2)


@pytest.mark.parametrize("seed", range(16))
def test_prefix_random_sweep_vs_oracle(dev, seed):
    """Random cascades: head_dim, GQA, kv heads, cache type, batch size,
    prefix length and suffix lengths drawn per case, against the oracle's
    plain decode of the aliased tables."""
    rng = np.random.default_rng(3000 + seed)
    D = int(rng.choice([64, 128]))
    G = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    kind = int(rng.choice([O.BF16, O.F16]))
    kv = kind if rng.random() < 0.7 else int(rng.choice([O.FP8_E4M3, O.FP8_E5M2]))
    if kind == O.F16 and kv != kind:
        kind = O.BF16
    B = int(rng.integers(1, 120))
    P = int(rng.integers(1, 80))
    lo = int(rng.integers(0, 200))
    q, k, v, bt, sl = prefix_case(rng, B, hkv * G, hkv, D, P, (lo, lo + int(rng.integers(1, 800))))
    ks = vs = 1.0
    if kv in (O.FP8_E4M3, O.FP8_E5M2):
        top = 448.0 if kv == O.FP8_E4M3 else 57344.0
        ks, vs = float(np.abs(k).max() / top), float(np.abs(v).max() / top)
        kb = O.encode((k / np.float32(ks)).astype(np.float32), kv)
        vb = O.encode((v / np.float32(vs)).astype(np.float32), kv)
    else:
        kb, vb = O.encode(k, kv), O.encode(v, kv)
    qb = O.encode(q, kind)
    scale = 1 / np.sqrt(D)
    ref = oracle_ref(qb, kind, kb, vb, kv, bt, sl, scale, ks, vs)
    got = run_prefix(dev, qb, kind, kb, vb, kv, bt, sl, scale, P, ks, vs, label=f"sweep {seed}")
    assert_close(got, ref, TOL_BF16 if kv == kind else TOL_FP8, f"prefix sweep {seed}")


@pytest.mark.parametrize("kv", [O.BF16, O.FP8_E4M3])
@pytest.mark.parametrize("B,P,own,cascade", [
    (9, 5, 4, False),      # saves 40 blocks: under the 10,000-tile floor
    (128, 8, 16, False),   # saves 1,016 blocks, under 3/5 of the 2,048 suffix blocks
    (32, 64, 16, True),    # saves 1,984 blocks (15,872 tiles), suffix 512
    (64, 64, 16, True),
], ids=["small", "short-prefix", "cascade-32", "cascade-64"])
def test_prefix_auto_choice_follows_the_rule(dev, monkeypatch, B, P, own, cascade, kv):
    """Without RLLM_CASCADE the entry point runs the cascade only where the
    prefix saves enough: the cascade when (B - 1) * P >= 3/5 * B * own and
    (B - 1) * P * Hkv >= 10,000, else the plain decode.  Its output has the
    forced cascade's bits or the plain decode's, as the rule says, and
    RLLM_CASCADE=never gives the plain decode's."""
    rng = np.random.default_rng(4100 + B + P + kv)
    q, k, v, bt, sl = prefix_case(rng, B, 32, 8, 128, P, (own * 16, own * 16))
    assert bt.shape[1] == P + own
    qb = O.encode(q, O.BF16)
    ks = vs = 1.0
    if kv == O.FP8_E4M3:
        ks, vs = float(np.abs(k).max() / 448.0), float(np.abs(v).max() / 448.0)
        kb = O.encode((k / np.float32(ks)).astype(np.float32), kv)
        vb = O.encode((v / np.float32(vs)).astype(np.float32), kv)
    else:
        kb, vb = O.encode(k, kv), O.encode(v, kv)
    scale = 1 / np.sqrt(128)
    args = (dev, qb, O.BF16, kb, vb, kv, bt, sl, scale, P, ks, vs)
    forced = run_prefix(*args, label=f"forced B={B}")
    monkeypatch.delenv("RLLM_CASCADE")
    auto = run_prefix(*args, label=f"auto B={B}")
    monkeypatch.setenv("RLLM_CASCADE", "never")
    never = run_prefix(*args, label=f"never B={B}")
    plain = f32(ops.paged_decode(t16(qb, torch.bfloat16, dev), _kv(kb, kv, dev), _kv(vb, kv, dev),
                                 ti(bt, torch.int32, dev), ti(sl, torch.int32, dev), scale, kv_dtype=ABI[kv],
                                 k_scale=ks, v_scale=vs))
    assert np.array_equal(never, plain)
    assert np.array_equal(auto, forced if cascade else plain)
    assert np.max(np.abs(forced - plain)) <= 2 ** -7 * max(1.0, float(np.abs(plain).max()))
