"""GPU parity of the batched block copy (copy-on-write) and of the swap to /
from pinned host records (rllm_cache_copy_blocks, rllm_cache_swap_{out,in})
against the CPU oracle: bit-exact."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import log_case
from rllm_amd import KernelError
from rllm_amd import ops

pytestmark = pytest.mark.gpu


def _caches(rng, L, shape, dtype, dev):
    hi = 256 if dtype == np.uint8 else 65536
    host = [rng.integers(0, hi, shape).astype(dtype) for _ in range(2 * L)]
    tdt = torch.uint8 if dtype == np.uint8 else torch.int16
    devc = [torch.from_numpy(h.view(np.int16) if dtype == np.uint16 else h).to(dev) for h in host]
    assert all(d.dtype == tdt for d in devc)
    return host[:L], host[L:], devc[:L], devc[L:]


def _host(t):
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


@pytest.mark.parametrize("shape,dtype", [((64, 8, 128, 16), np.uint16), ((9, 3, 5, 4), np.uint16),
                                         ((40, 8, 128, 16), np.uint8), ((6, 1, 8, 2), np.uint8)])
def test_copy_blocks_bit_exact(dev, shape, dtype):
    rng = np.random.default_rng(shape[0] + shape[2])
    L = 4
    hk, hv, gk, gv = _caches(rng, L, shape, dtype, dev)
    nb = shape[0]
    srcs = rng.permutation(nb)[: nb // 2]
    dsts = rng.permutation(np.setdiff1d(np.arange(nb), srcs))[: len(srcs)]
    pairs = np.stack([srcs[: len(dsts)], dsts], axis=1).astype(np.int64)
    pairs = np.concatenate([pairs, [[0, 0], [nb, 1], [-3, 1], [1, nb + 7]]]).astype(np.int64)
    log_case(f"copy_blocks shape={shape} dtype={dtype.__name__} pairs={len(pairs)}")
    ops.copy_blocks(gk, gv, torch.from_numpy(pairs).to(dev))
    torch.cuda.synchronize()
    O.copy_blocks(hk, hv, pairs, nb, hk[0][0].nbytes)
    for g, h in zip(gk + gv, hk + hv):
        assert np.array_equal(_host(g), h)


@pytest.mark.parametrize("with_slots", [False, True])
def test_swap_out_in_round_trip(dev, with_slots):
    rng = np.random.default_rng(7)
    L, shape = 3, (32, 8, 128, 16)
    hk, hv, gk, gv = _caches(rng, L, shape, np.uint16, dev)
    nb, nbytes = shape[0], hk[0][0].nbytes
    ids = np.array([5, 0, 31, 17, 40, -1, 9], np.int64)
    R = 9
    slots = rng.permutation(R)[: ids.size].astype(np.int64) if with_slots else None
    rec = torch.full((R, L, 2, nbytes), 0xEE, dtype=torch.uint8, pin_memory=True)
    want = np.full((R, L, 2, nbytes), 0xEE, np.uint8)
    gid = torch.from_numpy(ids).to(dev)
    gsl = torch.from_numpy(slots).to(dev) if with_slots else None
    log_case(f"swap_out slots={with_slots}")
    ops.swap_out(gk, gv, gid, rec, slots=gsl)
    torch.cuda.synchronize()
    O.swap_blocks(hk, hv, ids, want, nb, nbytes, out=True, slots=slots)
    assert np.array_equal(rec.numpy(), want)
    # clear the caches on the device, swap the records back in
    for g in gk + gv:
        g.zero_()
    log_case(f"swap_in slots={with_slots}")
    ops.swap_in(gk, gv, gid, rec, slots=gsl)
    torch.cuda.synchronize()
    zk = [np.zeros_like(h) for h in hk]
    zv = [np.zeros_like(h) for h in hv]
    O.swap_blocks(zk, zv, ids, want, nb, nbytes, out=False, slots=slots)
    for g, h in zip(gk + gv, zk + zv):
        assert np.array_equal(_host(g), h)


def test_fork_then_write_leaves_shared_block(dev):
    # copy-on-write flow: block 3 shared by two sequences is forked to block 8
    # (block_pool.rs:292-302), then the forked sequence writes its new token
    # into the fresh block; the shared block keeps the original bytes
    rng = np.random.default_rng(11)
    nb, hkv, D, bs = 12, 2, 64, 16
    kc = torch.from_numpy(rng.standard_normal((nb, hkv, D, bs)).astype(np.float32)).bfloat16().to(dev)
    vc = torch.from_numpy(rng.standard_normal((nb, hkv, D, bs)).astype(np.float32)).bfloat16().to(dev)
    k0, v0 = kc.clone(), vc.clone()
    ops.copy_blocks([kc], [vc], torch.tensor([[3, 8]], dtype=torch.int64, device=dev))
    nk = torch.randn(1, hkv, D, device=dev).bfloat16()
    nv = torch.randn(1, hkv, D, device=dev).bfloat16()
    ops.reshape_and_cache(nk, nv, kc, vc, torch.tensor([8 * bs + 5], dtype=torch.int64, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(kc[3], k0[3]) and torch.equal(vc[3], v0[3])
    expect_k = k0[3].clone()
    expect_k[:, :, 5] = nk[0]
    assert torch.equal(kc[8], expect_k)
    others = [i for i in range(nb) if i != 8]
    assert torch.equal(kc[others], k0[others]) and torch.equal(vc[others], v0[others])


def test_block_moves_reject_bad_arguments(dev):
    c = [torch.zeros((4, 1, 16, 16), dtype=torch.bfloat16, device=dev)]
    kt = ops.layer_table(c, dev)
    from rllm_amd._lib import call
    with pytest.raises(KernelError):   # num_blocks 0
        call("rllm_cache_copy_blocks", kt.data_ptr(), kt.data_ptr(), 1, kt.data_ptr(), 1, 0, 512, 0)
    rec = torch.zeros((1, 1, 2, 512), dtype=torch.uint8, pin_memory=True)
    with pytest.raises(KernelError):   # fewer records than ids without slots
        call("rllm_cache_swap_out", kt.data_ptr(), kt.data_ptr(), 1, kt.data_ptr(), 2, 4, 512, 0, 1,
             rec.data_ptr(), 0)
    pageable = np.zeros((1, 1, 2, 512), np.uint8)
    with pytest.raises(KernelError):   # pageable host memory is refused before any launch
        call("rllm_cache_swap_out", kt.data_ptr(), kt.data_ptr(), 1, kt.data_ptr(), 1, 4, 512, 0, 1,
             pageable.ctypes.data, 0)
    ops.copy_blocks(c, c, torch.zeros((0, 2), dtype=torch.int64, device=dev))   # empty list: no launch
