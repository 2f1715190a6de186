"""GPU parity of RMSNorm and SiLU-mul (rllm_rmsnorm_ex, rllm_silu_mul_ex and the
reference symbols rllm_fused_rmsnorm_f16 / rllm_fused_silu_mul_f16) against
the CPU oracle.  Tolerance: the 16-bit results agree exactly or differ by one
unit in the last place (the GPU sums squares in another order than the
oracle's sequential sum, and device expf may differ from libm's by an f32 ulp);
at most 1% of the elements may differ at all."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import bits16, log_case, t16
from rllm_amd import ops
from rllm_amd._lib import call

pytestmark = pytest.mark.gpu
DT = {O.BF16: torch.bfloat16, O.F16: torch.float16}


def _ulp_check(got_bits, want_bits, what):
    g = got_bits.astype(np.int32)
    w = want_bits.astype(np.int32)
    # same-sign neighbours differ by one in the bit pattern
    diff = np.abs(g - w)
    bad = diff > 1
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one ulp"
    frac = float(np.mean(diff != 0))
    assert frac <= 0.01, f"{what}: {frac:.4f} of the elements differ"
    return frac


@pytest.mark.parametrize("kind", [O.BF16, O.F16])
@pytest.mark.parametrize("rows,hidden", [(4096, 4096), (64, 4096), (37, 8), (5, 16384), (3, 1000), (9, 12288)])
def test_rmsnorm_matches_oracle(dev, kind, rows, hidden):
    rng = np.random.default_rng(rows + hidden)
    x = O.encode((rng.standard_normal((rows, hidden)) * 3).astype(np.float32), kind)
    w = O.encode((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32), kind)
    log_case(f"rmsnorm rows={rows} hidden={hidden} kind={kind}")
    y = ops.rmsnorm(t16(x, DT[kind], dev), t16(w, DT[kind], dev), 1e-5)
    torch.cuda.synchronize()
    _ulp_check(bits16(y), O.rmsnorm(x, w, 1e-5, kind), f"rmsnorm {rows}x{hidden}")


@pytest.mark.parametrize("kind", [O.BF16, O.F16])
def test_rmsnorm_bit_exact_when_sums_are_exact(dev, kind):
    # x = k/8 (|k| <= 64): every square and every partial sum is exact in f32,
    # so the summation order cannot matter and the GPU must give the oracle's
    # bytes exactly (this pins the per-element quotient x / sqrt(var))
    rng = np.random.default_rng(17)
    rows, hidden = 512, 4096
    x = O.encode((rng.integers(-64, 65, (rows, hidden)) / 8).astype(np.float32), kind)
    w = O.encode((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32), kind)
    log_case(f"rmsnorm exact sums kind={kind}")
    y = bits16(ops.rmsnorm(t16(x, DT[kind], dev), t16(w, DT[kind], dev), 1e-5))
    want = O.rmsnorm(x, w, 1e-5, kind)
    assert np.array_equal(y, want), f"{int((y != want).sum())} of {y.size} differ"


def test_rmsnorm_reference_symbol_known_answer(dev):
    # fused.rs:512-567 through rllm_fused_rmsnorm_f16_sync
    x = O.encode(np.array([1, 2, 3, 4, 2, 4, 6, 8], np.float32), O.F16)
    x = np.concatenate([x, np.zeros(8, np.uint16)])     # hidden 8 (multiple of 8): rows [x, 0]
    w = O.encode(np.ones(8, np.float32), O.F16)
    gx, gw = t16(x, torch.float16, dev), t16(w, torch.float16, dev)
    out = torch.empty_like(gx)
    call("rllm_fused_rmsnorm_f16_sync", out.data_ptr(), gx.data_ptr(), gw.data_ptr(), 8, 16, 1e-6)
    want = O.rmsnorm(x.reshape(2, 8), w, 1e-6, O.F16).reshape(-1)
    _ulp_check(bits16(out), want, "rllm_fused_rmsnorm_f16_sync")
    y = O.decode(bits16(out), O.F16)[:8]
    ref = np.array([1, 2, 3, 4, 2, 4, 6, 8]) / np.sqrt(np.mean(np.array([1, 2, 3, 4, 2, 4, 6, 8]) ** 2) + 1e-6)
    assert np.all(np.abs(y - ref) < 0.1)


@pytest.mark.parametrize("kind", [O.BF16, O.F16])
@pytest.mark.parametrize("n,offset", [(4096 * 14336, 0), (1000003, 0), (777, 1), (8, 0)])
def test_silu_mul_matches_oracle(dev, kind, n, offset):
    rng = np.random.default_rng(n % 1000 + offset)
    g = O.encode((rng.standard_normal(n + offset) * 4).astype(np.float32), kind)
    u = O.encode(rng.standard_normal(n + offset).astype(np.float32), kind)
    gg, gu = t16(g, DT[kind], dev), t16(u, DT[kind], dev)
    log_case(f"silu_mul n={n} offset={offset} kind={kind}")
    # offset 1: 2-byte aligned views take the scalar path
    out = ops.silu_mul(gg[offset:], gu[offset:])
    torch.cuda.synchronize()
    _ulp_check(bits16(out), O.silu_mul(g[offset:], u[offset:], kind), f"silu_mul n={n}")


def test_silu_mul_reference_symbol_known_answer(dev):
    # fused.rs:476-509 through rllm_fused_silu_mul_f16_sync
    gf = np.array([1.0, 2.0, 0.0, -1.0, 0.5, 3.0, -0.5, 4.0], np.float32)
    uf = np.array([2.0, 0.5, 1.0, 1.0, 3.0, 1.0, 2.0, 0.5], np.float32)
    g, u = O.encode(gf, O.F16), O.encode(uf, O.F16)
    gg, gu = t16(g, torch.float16, dev), t16(u, torch.float16, dev)
    out = torch.empty_like(gg)
    call("rllm_fused_silu_mul_f16_sync", out.data_ptr(), gg.data_ptr(), gu.data_ptr(), 8)
    _ulp_check(bits16(out), O.silu_mul(g, u, O.F16), "rllm_fused_silu_mul_f16_sync")
    got = O.decode(bits16(out), O.F16)
    assert np.all(np.abs(got - gf / (1 + np.exp(-gf)) * uf) < 0.1)


def test_silu_mul_bf16_bit_exact_for_every_gate_value(dev):
    # every bf16 gate pattern (NaN, inf, subnormals, the exp overflow region
    # near -88 included) against 64 up values: the reciprocal quotient and the
    # device expf give the oracle's bytes exactly
    g = np.repeat(np.arange(65536, dtype=np.uint16), 64)
    u = O.encode(np.random.default_rng(0).standard_normal(g.size).astype(np.float32), O.BF16)
    log_case("silu_mul bf16 exhaustive gate")
    out = bits16(ops.silu_mul(t16(g, torch.bfloat16, dev), t16(u, torch.bfloat16, dev)))
    want = O.silu_mul(g, u, O.BF16)
    nan = lambda b: np.isnan(O.decode(b, O.BF16))
    same = (out == want) | (nan(out) & nan(want))
    assert same.all(), f"{int((~same).sum())} mismatches at gate bits {np.unique(g[~same])[:8]}"
