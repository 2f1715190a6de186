"""rllm_paged_attention_decode_noalloc: the decode entry point that allocates
nothing (its scratch is a fixed device array per GPU).  Checked through the C
ABI against rllm_paged_attention_decode_ex on the same inputs (the same
kernels, so bit-exact) and against the oracle, on two calls in a row, the
second with a smaller batch; the stream mode and a fixed split-K partition;
and a call that would need more scratch than the array holds, which must be
refused before any launch."""
import numpy as np
import pytest
import torch

import oracle as O
import rllm_amd
from gpu_util import f32, log_case, ptr, t16, ti
from helpers import TOL_BF16, assert_close, random_case

pytestmark = pytest.mark.gpu
HQ, HKV, D, BS = 32, 8, 128, 16
SCRATCH_BYTES = 24 << 20


def _case(dev, seed, B, ctx_range):
    rng = np.random.default_rng(seed)
    q, k, v, bt, sl = random_case(rng, B, HQ, HKV, D, ctx_range)
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(D)
    ref = O.paged_attention_decode(qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, precision=1)
    bf = torch.bfloat16
    return dict(q=t16(qb, bf, dev), kc=t16(kb, bf, dev), vc=t16(vb, bf, dev), bt=ti(bt, torch.int32, dev),
                sl=ti(sl, torch.int32, dev), scale=scale, ref=ref, B=B, maxb=bt.shape[1])


def _args(x, out):
    return (ptr(out), ptr(x["q"]), ptr(x["kc"]), ptr(x["vc"]), ptr(x["bt"]), ptr(x["sl"]), x["B"], HQ, HKV, D,
            BS, x["maxb"], x["scale"], rllm_amd.DTYPE_BF16, rllm_amd.DTYPE_BF16, 1.0, 1.0)


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("partition", [0, 512])
def test_noalloc_matches_decode_ex_on_two_calls(dev, partition):
    L = rllm_amd.lib()
    # the second call is smaller: stale partials or counters of the first
    # call in the shared array must not leak into it
    for call, (seed, B, ctx_range) in enumerate([(501, 48, (64, 4000)), (502, 5, (1, 900))]):
        x = _case(dev, seed + partition, B, ctx_range)
        need = L.rllm_paged_attention_decode_workspace_size(B, HQ, HKV, D, BS, x["maxb"], partition)
        assert 0 <= need <= SCRATCH_BYTES
        out_ex = torch.full_like(x["q"], 3.0)
        out_na = torch.full_like(x["q"], 5.0)
        log_case(f"decode_ex call {call} B={B} partition={partition}")
        rc = L.rllm_paged_attention_decode_ex(*_args(x, out_ex), partition, None, 0, _stream())
        assert rc == 0
        log_case(f"decode_noalloc call {call} B={B} partition={partition} scratch need {need}")
        rc = L.rllm_paged_attention_decode_noalloc(*_args(x, out_na), partition, _stream())
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ex), f"call {call}: noalloc output differs from decode_ex"
        assert_close(f32(out_na), x["ref"], TOL_BF16, f"noalloc call {call} partition={partition}")


def test_noalloc_refuses_calls_beyond_its_scratch(dev):
    """Fixed 512-token partitions over 1024 sequences of up to 2048 tokens need
    1024 x 32 x 4 x 130 x 4 bytes of partials, more than the array: the call
    returns hipErrorOutOfMemory and launches nothing (the output keeps its
    sentinel)."""
    L = rllm_amd.lib()
    B, maxb = 1024, 128
    need = L.rllm_paged_attention_decode_workspace_size(B, HQ, HKV, D, BS, maxb, 512)
    assert need > SCRATCH_BYTES
    q = torch.zeros((B, HQ, D), dtype=torch.bfloat16, device=dev)
    kc = torch.zeros((4, HKV, D, BS), dtype=torch.bfloat16, device=dev)
    bt = torch.full((B, maxb), -1, dtype=torch.int32, device=dev)
    sl = torch.zeros((B,), dtype=torch.int32, device=dev)
    out = torch.full_like(q, 9.0)
    x = dict(q=q, kc=kc, vc=kc, bt=bt, sl=sl, B=B, maxb=maxb, scale=0.088)
    log_case("decode_noalloc beyond its scratch (refused before launch)")
    rc = L.rllm_paged_attention_decode_noalloc(*_args(x, out), 512, _stream())
    torch.cuda.synchronize()
    assert rc == 2, rc
    assert bool((out == 9.0).all())
