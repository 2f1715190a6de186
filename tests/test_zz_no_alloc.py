"""rllm_paged_attention_decode_noalloc: the decode entry point that allocates
nothing (its scratch is a fixed device array per GPU).  Checked through the C
ABI against rllm_paged_attention_decode_ex on the same inputs (the same
kernels, so bit-exact) and against the oracle:

* two calls in a row, the second with a smaller batch, in the stream mode and
  with a fixed split-K partition;
* a split-K call followed by two stream-mode calls at config 2's shape: the
  split-K partials must not land on the stream mode's arrival counters, which
  every stream-mode call expects to find at zero;
* a call that would need more scratch than the array holds, which must be
  refused before any launch;
* in a fresh process, a first call under stream capture (refused: the
  counters' one-time clear must not exist only inside a graph), then an eager
  call, then a captured stream-mode call replayed with split-K calls between
  the replays.
"""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle as O
import rllm_amd
from gpu_util import f32, log_case, ptr, t16, ti
from helpers import TOL_BF16, assert_close, random_case
from rllm_amd import workloads

pytestmark = pytest.mark.gpu
HQ, HKV, D, BS = 32, 8, 128, 16
SCRATCH_BYTES = 24 << 20
HIP_ERROR_STREAM_CAPTURE_UNSUPPORTED = 900


def _case(dev, seed, B, ctx_range):
    rng = np.random.default_rng(seed)
    q, k, v, bt, sl = random_case(rng, B, HQ, HKV, D, ctx_range)
    qb, kb, vb = O.encode(q, O.BF16), O.encode(k, O.BF16), O.encode(v, O.BF16)
    scale = 1 / np.sqrt(D)
    ref = O.paged_attention_decode(qb, O.BF16, kb, vb, O.BF16, bt, sl, scale, precision=1)
    bf = torch.bfloat16
    return dict(q=t16(qb, bf, dev), kc=t16(kb, bf, dev), vc=t16(vb, bf, dev), bt=ti(bt, torch.int32, dev),
                sl=ti(sl, torch.int32, dev), scale=scale, ref=ref, B=B, maxb=bt.shape[1])


def _config2_case(dev):
    w = workloads.config(2)
    qb, kb, vb = workloads.host_tensors(w)
    ref = O.paged_attention_decode(qb, O.BF16, kb, vb, O.BF16, w.block_tables, w.seq_lens, w.scale,
                                   precision=0)
    bf = torch.bfloat16
    return dict(q=t16(qb, bf, dev), kc=t16(kb, bf, dev), vc=t16(vb, bf, dev),
                bt=ti(w.block_tables, torch.int32, dev), sl=ti(w.seq_lens, torch.int32, dev),
                scale=w.scale, ref=ref, B=w.num_seqs, maxb=w.block_tables.shape[1])


def _args(x, out):
    return (ptr(out), ptr(x["q"]), ptr(x["kc"]), ptr(x["vc"]), ptr(x["bt"]), ptr(x["sl"]), x["B"], HQ, HKV, D,
            BS, x["maxb"], x["scale"], rllm_amd.DTYPE_BF16, rllm_amd.DTYPE_BF16, 1.0, 1.0)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _noalloc_vs_ex(L, x, partition, label):
    """One decode_ex call and one noalloc call on x; both outputs bit-equal and
    within the bf16 tolerance of the oracle."""
    out_ex = torch.full_like(x["q"], 3.0)
    out_na = torch.full_like(x["q"], 5.0)
    log_case(f"decode_ex {label} B={x['B']} partition={partition}")
    rc = L.rllm_paged_attention_decode_ex(*_args(x, out_ex), partition, None, 0, _stream())
    assert rc == 0
    log_case(f"decode_noalloc {label} B={x['B']} partition={partition}")
    rc = L.rllm_paged_attention_decode_noalloc(*_args(x, out_na), partition, _stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ex), f"{label}: noalloc output differs from decode_ex"
    assert_close(f32(out_na), x["ref"], TOL_BF16, f"noalloc {label} partition={partition}")


@pytest.mark.parametrize("partition", [0, 512])
def test_noalloc_matches_decode_ex_on_two_calls(dev, partition):
    L = rllm_amd.lib()
    # the second call is smaller: stale partials or counters of the first
    # call in the shared array must not leak into it
    for call, (seed, B, ctx_range) in enumerate([(501, 48, (64, 4000)), (502, 5, (1, 900))]):
        x = _case(dev, seed + partition, B, ctx_range)
        need = L.rllm_paged_attention_decode_workspace_size(B, HQ, HKV, D, BS, x["maxb"], partition)
        assert 0 <= need <= SCRATCH_BYTES
        _noalloc_vs_ex(L, x, partition, f"call {call}")


def test_noalloc_split_call_leaves_stream_counters_intact(dev):
    """A split-K call (B=48, mixed contexts, 512-token partitions: ~6.4 MB of
    partials) and then two stream-mode calls at config 2's shape, all through
    the noalloc entry point.  Split-K partials placed over the stream mode's
    arrival counters would start the stream calls with non-zero counters, so
    rows cut between waves would be merged early or never (stale output rows)."""
    L = rllm_amd.lib()
    split = _case(dev, 611, 48, (64, 4000))
    need = L.rllm_paged_attention_decode_workspace_size(48, HQ, HKV, D, BS, split["maxb"], 512)
    assert need > 1 << 20, "the split-K call must write well past the counters' region"
    _noalloc_vs_ex(L, split, 512, "split-K first")
    del split
    c2 = _config2_case(dev)
    _noalloc_vs_ex(L, c2, 0, "config 2 stream after split-K")
    _noalloc_vs_ex(L, c2, 0, "config 2 stream again")


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


def _capture_child():
    """Runs in a fresh process, where no noalloc call has set the device up."""
    dev = torch.device("cuda:0")
    L = rllm_amd.lib()
    x = _case(dev, 701, 24, (200, 3000))
    other = _case(dev, 702, 40, (64, 4000))
    out = torch.zeros_like(x["q"])

    log_case("capture child: first noalloc call under capture (refused)")
    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0):
        rc = L.rllm_paged_attention_decode_noalloc(*_args(x, out), 0, _stream())
    assert rc == HIP_ERROR_STREAM_CAPTURE_UNSUPPORTED, rc

    log_case("capture child: eager noalloc call sets the device up")
    eager = torch.zeros_like(x["q"])
    assert L.rllm_paged_attention_decode_noalloc(*_args(x, eager), 0, _stream()) == 0
    torch.cuda.synchronize()
    assert_close(f32(eager), x["ref"], TOL_BF16, "capture child eager")

    log_case("capture child: captured stream-mode call")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = L.rllm_paged_attention_decode_noalloc(*_args(x, out), 0, _stream())
    assert rc == 0, rc
    torch.cuda.synchronize()
    for r in range(3):
        out.zero_()
        log_case(f"capture child: replay {r}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"
        # an eager split-K call between replays shares the array
        o2 = torch.zeros_like(other["q"])
        log_case(f"capture child: eager split-K call after replay {r}")
        assert L.rllm_paged_attention_decode_noalloc(*_args(other, o2), 512, _stream()) == 0
        torch.cuda.synchronize()
        assert_close(f32(o2), other["ref"], TOL_BF16, f"split-K after replay {r}")
    print("capture child: ok", flush=True)


def test_noalloc_first_call_under_capture_is_refused(dev):
    """In a fresh process (the first noalloc call on a device clears the
    counters, so it must be the first call there)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.path.join(root, "tests")]))
    log_case("noalloc capture child process")
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "--capture-child"], env=env,
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0, f"child exited with {r.returncode}"
    assert "capture child: ok" in r.stdout


if __name__ == "__main__" and "--capture-child" in sys.argv:
    _capture_child()
