"""Pins the oracle's slot arithmetic and reshape_and_cache (oracle.c) with the
reference's own known answers and an independent numpy formulation."""
import numpy as np
import pytest

import oracle as O
from rllm_amd.cache_ops import compute_slot_mappings


# ---- slot mapping: reference known answers ------------------------------

def test_slot_mapping_known_answers_model_runner():
    # model_runner.rs:1068-1084 (test_compute_slot_mappings)
    s = O.slot_mapping([0, 1, 2, 3, 16, 17, 18, 19], [5, 7], 4)
    assert s[:4].tolist() == [20, 21, 22, 23] and s[4] == -1 and s[5] == -1
    # model_runner.rs:1086-1102 (block boundary)
    assert O.slot_mapping([3, 4, 7, 8], [10, 20, 30], 4).tolist() == [43, 80, 83, 120]
    # model_runner.rs:925-967: 32 tokens, blocks 5 and 7, bs 16
    s = O.slot_mapping(list(range(32)), [5, 7], 16)
    assert s.tolist() == [5 * 16 + i for i in range(16)] + [7 * 16 + i for i in range(16)]
    # model_runner.rs:971-1030: decode at position 9, bs 4, table [0,1,2] -> slot 9
    assert O.slot_mapping([9], [0, 1, 2], 4).tolist() == [9]


def test_host_compute_slot_mappings_matches_oracle():
    rng = np.random.default_rng(5)
    for bs in (1, 4, 16, 32):
        bt = rng.permutation(200)[:37]
        pos = rng.integers(0, 40 * bs, size=500)
        assert compute_slot_mappings(pos.tolist(), bt.tolist(), bs) == \
            O.slot_mapping(pos, bt, bs).tolist()
    assert compute_slot_mappings([3, 4, 7, 8], [10, 20, 30], 4) == [43, 80, 83, 120]
    assert compute_slot_mappings([1, 2], [3], 0) == [-1, -1]


# ---- reshape_and_cache -----------------------------------------------------

def _numpy_cache_write(kc, vc, nk, nv, slots, bs, nb):
    """Independent formulation: view the cache as [nb, Hkv, D, bs] and assign
    cache[blk, :, :, off] = new[t] (cache_ops.cu:182-199 semantics)."""
    kc, vc = kc.copy(), vc.copy()
    for t, slot in enumerate(slots):
        if slot < 0:
            continue
        blk, off = divmod(int(slot), bs)
        if blk >= nb:
            continue
        kc[blk, :, :, off] = nk[t]
        vc[blk, :, :, off] = nv[t]
    return kc, vc


@pytest.mark.parametrize("bs,hkv,d", [(16, 8, 128), (16, 2, 64), (4, 3, 5), (32, 1, 8)])
def test_cache_write_16bit_matches_numpy(bs, hkv, d):
    rng = np.random.default_rng(bs * 100 + d)
    nb, n = 12, 20
    kc = rng.integers(0, 65536, size=(nb, hkv, d, bs), dtype=np.uint16)
    vc = rng.integers(0, 65536, size=(nb, hkv, d, bs), dtype=np.uint16)
    nk = rng.integers(0, 65536, size=(n, hkv, d), dtype=np.uint16)
    nv = rng.integers(0, 65536, size=(n, hkv, d), dtype=np.uint16)
    slots = rng.choice(nb * bs, size=n, replace=False).astype(np.int64)
    slots[3] = -1                      # padding token (cache_ops.cu:183)
    slots[7] = nb * bs + 5             # block beyond the pool (cache_ops.cu:188)
    ek, ev = _numpy_cache_write(kc, vc, nk, nv, slots, bs, nb)
    ok, ov = kc.copy(), vc.copy()
    O.cache_write(ok, ov, nk, nv, slots, bs, O.BF16, O.BF16)
    assert np.array_equal(ok, ek) and np.array_equal(ov, ev)
    # canaries: every slot not written keeps its bytes
    written = np.zeros((nb, bs), bool)
    for s in slots:
        if 0 <= s < nb * bs:
            written[s // bs, s % bs] = True
    assert np.array_equal(ok.transpose(0, 3, 1, 2)[~written], kc.transpose(0, 3, 1, 2)[~written])


@pytest.mark.parametrize("kind", [O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("in_kind", [O.F16, O.BF16])
def test_cache_write_fp8_matches_numpy(kind, in_kind):
    rng = np.random.default_rng(11 + kind + 7 * in_kind)
    nb, bs, hkv, d, n = 9, 16, 4, 32, 30
    x = rng.standard_normal((2, n, hkv, d)).astype(np.float32) * 3
    nk = O.encode(x[0], in_kind)
    nv = O.encode(x[1], in_kind)
    kscale, vscale = 0.37, 1.7
    slots = rng.choice(nb * bs, size=n, replace=False).astype(np.int64)
    slots[0] = -1
    kc = rng.integers(0, 256, size=(nb, hkv, d, bs), dtype=np.uint8)
    vc = rng.integers(0, 256, size=(nb, hkv, d, bs), dtype=np.uint8)
    # expected bytes: encode(decode(in) / scale), quotient correctly rounded in fp32
    ekb = O.encode((O.decode(nk, in_kind) / np.float32(kscale)).astype(np.float32), kind)
    evb = O.encode((O.decode(nv, in_kind) / np.float32(vscale)).astype(np.float32), kind)
    ek, ev = _numpy_cache_write(kc, vc, ekb, evb, slots, bs, nb)
    ok, ov = kc.copy(), vc.copy()
    O.cache_write(ok, ov, nk, nv, slots, bs, in_kind, kind, kscale, vscale)
    assert np.array_equal(ok, ek) and np.array_equal(ov, ev)
