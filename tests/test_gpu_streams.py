"""Calls from two host threads on two streams at once.

The library keeps its scratch per (device, stream): the stream decode's arrival
counters and partials, the prefill's KV-split partials, the cascade's partials.
Two threads that call the decode, the chunked prefill, the mixed step and the
cascade on their own streams at the same time must therefore give the bits
that the same calls give one at a time, and the library's host state (scratch
table, occupancy cache) must stand concurrent callers.  The ctypes calls
release the GIL, so the two threads are inside the library together."""
import threading

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import RawStream, ti, t16
from rllm_amd import ops

pytestmark = pytest.mark.gpu


def _case(rng, dev):
    hq, hkv, D, bs = 32, 8, 128, 16
    # decode: 48 sequences of mixed lengths (rows cut between waves, merged
    # through the stream workspace)
    dl = rng.integers(1, 3000, size=48).astype(np.int32)
    dnb = (dl + bs - 1) // bs
    # prefill: one 512-token chunk on 1024 cached tokens (the KV-split path)
    pl = np.array([1536], np.int32)
    pnb = (pl + bs - 1) // bs
    # cascade: 32 sequences on one 16-block prefix, 8 blocks of their own
    cbt_w = 16 + 8
    pool = int(dnb.sum() + pnb.sum()) + 16 + 32 * 8 + 4
    perm = rng.permutation(pool).astype(np.int32)
    dbt = np.full((48, int(dnb.max())), -1, np.int32)
    p = 0
    for s in range(48):
        dbt[s, :dnb[s]] = perm[p:p + dnb[s]]
        p += int(dnb[s])
    pbt = perm[p:p + int(pnb[0])].reshape(1, -1).copy()
    p += int(pnb[0])
    cbt = np.empty((32, cbt_w), np.int32)
    cbt[:, :16] = perm[p:p + 16]
    cbt[:, 16:] = perm[p + 16:p + 16 + 32 * 8].reshape(32, 8)
    csl = (16 * 16 + rng.integers(1, 8 * 16, size=32)).astype(np.int32)
    cq = O.encode(rng.standard_normal((32, hq, D)).astype(np.float32), O.BF16)
    k = O.encode(rng.standard_normal((pool, hkv, D, bs)).astype(np.float32), O.BF16)
    v = O.encode(rng.standard_normal((pool, hkv, D, bs)).astype(np.float32), O.BF16)
    dq = O.encode(rng.standard_normal((48, hq, D)).astype(np.float32), O.BF16)
    pq = O.encode(rng.standard_normal((512, hq, D)).astype(np.float32), O.BF16)
    return dict(
        kc=t16(k, torch.bfloat16, dev), vc=t16(v, torch.bfloat16, dev),
        dq=t16(dq, torch.bfloat16, dev), dbt=ti(dbt, torch.int32, dev), dsl=ti(dl, torch.int32, dev),
        pq=t16(pq, torch.bfloat16, dev), pbt=ti(pbt, torch.int32, dev), psl=ti(pl, torch.int32, dev),
        qsl=ti(np.array([0, 512], np.int32), torch.int32, dev), scale=1 / np.sqrt(D),
        cq=t16(cq, torch.bfloat16, dev), cbt=ti(cbt, torch.int32, dev), csl=ti(csl, torch.int32, dev))


def _decode(c, out, stream=None):
    ops.paged_decode(c["dq"], c["kc"], c["vc"], c["dbt"], c["dsl"], c["scale"], out=out, validate=False,
                     stream=stream)


def _prefill(c, out, stream=None):
    ops.paged_prefill(c["pq"], c["kc"], c["vc"], c["pbt"], c["psl"], c["qsl"], c["scale"], out=out,
                      validate=False, stream=stream)


def _mixed(c, outs, stream=None):
    ops.paged_mixed(c["pq"], c["pbt"], c["psl"], c["qsl"], c["dq"], c["dbt"], c["dsl"], c["kc"], c["vc"],
                    c["scale"], prefill_out=outs[0], decode_out=outs[1], validate=False, stream=stream)


def _cascade(c, out, stream=None):
    ops.paged_decode_prefix(c["cq"], c["kc"], c["vc"], c["cbt"], c["csl"], c["scale"], 16, out=out,
                            validate=False, stream=stream)


def _outputs(c):
    return [torch.zeros_like(c["dq"]), torch.zeros_like(c["pq"]), torch.zeros_like(c["pq"]),
            torch.zeros_like(c["dq"]), torch.zeros_like(c["cq"])]


def _step(c, o, stream=None):
    _decode(c, o[0], stream)
    _prefill(c, o[1], stream)
    _mixed(c, (o[2], o[3]), stream)
    _cascade(c, o[4], stream)


def test_two_threads_on_two_streams_give_the_same_bits(dev, monkeypatch):
    """Decode, split prefill, the one-launch mixed step and the cascade (forced)
    on two streams from two threads, 25 rounds each."""
    monkeypatch.setenv("RLLM_CASCADE", "always")
    rng = np.random.default_rng(5150)
    c = _case(rng, dev)
    ref = _outputs(c)
    _step(c, ref)
    torch.cuda.synchronize()

    n_iter = 25
    outs = [_outputs(c) for _ in range(2)]
    errors = []
    start = threading.Barrier(2)

    def worker(i, stream):
        try:
            start.wait()
            for _ in range(n_iter):
                _step(c, outs[i], stream)
            stream.synchronize()
        except Exception as e:   # reported by the main thread
            errors.append(e)

    with RawStream() as s0, RawStream() as s1:
        torch.cuda.synchronize()
        threads = [threading.Thread(target=worker, args=(i, s)) for i, s in enumerate((s0, s1))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
        torch.cuda.synchronize()
    assert not errors, errors
    names = ["decode", "prefill", "mixed prefill", "mixed decode", "cascade"]
    for i in range(2):
        for j, name in enumerate(names):
            assert torch.equal(outs[i][j], ref[j]), f"{name} bits differ on thread {i}"
