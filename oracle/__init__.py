"""ctypes front end of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, always as the checker or as the timed CPU
baseline.  The product package (``rllm_amd``) never imports it.

The C sources (``oracle.c``) restate the reference algorithms; every function
cites the reference ``file:line`` it follows in ``oracle.h``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F16, BF16, FP8_E4M3, FP8_E5M2 = 0, 1, 2, 3
KIND_BYTES = {F16: 2, BF16: 2, FP8_E4M3: 1, FP8_E5M2: 1}

_lib = None


def build() -> None:
    """Compile liboracle.so with gcc (needs only make + gcc)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    c = ctypes
    P = c.c_void_p
    i64 = c.c_int64
    L.orc_bf16_to_f32.argtypes = [c.c_uint16]
    L.orc_bf16_to_f32.restype = c.c_float
    L.orc_f32_to_bf16.argtypes = [c.c_float]
    L.orc_f32_to_bf16.restype = c.c_uint16
    L.orc_f16_to_f32.argtypes = [c.c_uint16]
    L.orc_f16_to_f32.restype = c.c_float
    L.orc_f32_to_f16.argtypes = [c.c_float]
    L.orc_f32_to_f16.restype = c.c_uint16
    for name in ("orc_fp8_e4m3_encode", "orc_fp8_e4m3_encode_reftext", "orc_fp8_e5m2_encode"):
        getattr(L, name).argtypes = [c.c_float]
        getattr(L, name).restype = c.c_uint8
    for name in ("orc_fp8_e4m3_decode", "orc_fp8_e4m3_decode_reftext", "orc_fp8_e5m2_decode"):
        getattr(L, name).argtypes = [c.c_uint8]
        getattr(L, name).restype = c.c_float
    L.orc_decode_array.argtypes = [P, c.c_int, i64, P]
    L.orc_encode_array.argtypes = [P, c.c_int, i64, P]
    for name in ("orc_fp8_e4m3_exhaustive", "orc_fp8_e5m2_exhaustive"):
        getattr(L, name).argtypes = [c.c_int, c.POINTER(c.c_uint32)]
        getattr(L, name).restype = i64
    for name in ("orc_fp8_e4m3_encode_rne", "orc_fp8_e5m2_encode_rne"):
        getattr(L, name).argtypes = [c.c_float]
        getattr(L, name).restype = c.c_uint8
    L.orc_encode_fp8_rne_array.argtypes = [P, c.c_int, i64, P]
    L.orc_fp8_rne_exhaustive.argtypes = [c.c_int, c.c_int, c.POINTER(c.c_uint32)]
    L.orc_fp8_rne_exhaustive.restype = i64
    L.orc_cache_write_rounded.argtypes = [P, P, P, P, P, i64, i64, i64, i64, i64, c.c_int, c.c_int,
                                          c.c_float, c.c_float, c.c_int]
    L.orc_slot_mapping.argtypes = [P, i64, P, i64, i64, P]
    L.orc_cache_write.argtypes = [P, P, P, P, P, i64, i64, i64, i64, i64, c.c_int, c.c_int,
                                  c.c_float, c.c_float]
    L.orc_rope_interleaved.argtypes = [P, P, P, i64, i64, i64, c.c_float]
    L.orc_rmsnorm.argtypes = [P, P, P, i64, i64, c.c_float, c.c_int]
    L.orc_silu_mul.argtypes = [P, P, P, i64, c.c_int]
    L.orc_copy_blocks.argtypes = [P, P, i64, P, i64, i64, i64]
    L.orc_swap_blocks.argtypes = [P, P, i64, P, i64, P, i64, i64, i64, P, c.c_int]
    L.orc_rope_cache_build.argtypes = [P, P, i64, i64, c.c_float]
    L.orc_rope_cache_write.argtypes = [P, P, P, P, P, P, P, P, P, P, i64, i64, i64, i64, i64,
                                       i64, i64, c.c_int, c.c_int, c.c_float, c.c_float]
    L.orc_rope_cache_write_rounded.argtypes = [P, P, P, P, P, P, P, P, P, P, i64, i64, i64, i64, i64,
                                               i64, i64, c.c_int, c.c_int, c.c_float, c.c_float, c.c_int]
    L.orc_paged_attention_decode.argtypes = [P, P, c.c_int, P, P, c.c_int, P, P, i64, i64, i64,
                                             i64, i64, i64, c.c_float, c.c_float, c.c_float,
                                             c.c_int, c.c_int]
    L.orc_paged_attention_prefill.argtypes = [P, P, c.c_int, P, P, c.c_int, P, P, P, i64, i64,
                                              i64, i64, i64, i64, i64, c.c_float, c.c_float,
                                              c.c_float, c.c_int, c.c_int]
    L.orc_hardware_threads.restype = c.c_int
    _lib = L
    return L


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def hardware_threads() -> int:
    return int(lib().orc_hardware_threads())


# ---- conversions -------------------------------------------------------

def decode(arr: np.ndarray, kind: int) -> np.ndarray:
    """Element bits (uint16 / uint8) -> float32 per the oracle's codec."""
    arr = np.ascontiguousarray(arr)
    out = np.empty(arr.shape, dtype=np.float32)
    lib().orc_decode_array(_p(arr), kind, arr.size, _p(out))
    return out


def encode(x: np.ndarray, kind: int) -> np.ndarray:
    """float32 -> element bits (uint16 for 16-bit kinds, uint8 for fp8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16 if KIND_BYTES[kind] == 2 else np.uint8)
    lib().orc_encode_array(_p(x), kind, x.size, _p(out))
    return out


def encode_fp8_rne(x: np.ndarray, kind: int) -> np.ndarray:
    """float32 -> FP8 bytes rounded to nearest even (the library's opt-in mode)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_encode_fp8_rne_array(_p(x), kind, x.size, _p(out))
    return out


def fp8_rne_exhaustive(e5m2: bool = False, nthreads: int = 8) -> tuple[int, int]:
    """(violations, first violating pattern) of the nearest-even encoder over
    all 2^32 float32 patterns."""
    bad_pat = ctypes.c_uint32(0)
    bad = lib().orc_fp8_rne_exhaustive(1 if e5m2 else 0, nthreads, ctypes.byref(bad_pat))
    return int(bad), int(bad_pat.value)


def fp8_exhaustive(e5m2: bool = False, nthreads: int = 8) -> tuple[int, int]:
    bad_pat = ctypes.c_uint32(0)
    fn = lib().orc_fp8_e5m2_exhaustive if e5m2 else lib().orc_fp8_e4m3_exhaustive
    bad = fn(nthreads, ctypes.byref(bad_pat))
    return int(bad), int(bad_pat.value)


# ---- metadata and cache write ------------------------------------------

def slot_mapping(positions, block_table, block_size: int) -> np.ndarray:
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    bt = np.ascontiguousarray(block_table, dtype=np.uint32)
    out = np.empty(pos.shape, dtype=np.int64)
    lib().orc_slot_mapping(_p(pos), pos.size, _p(bt), bt.size, block_size, _p(out))
    return out


def cache_write(key_cache, value_cache, new_key, new_value, slot_mapping, block_size: int,
                in_kind: int, cache_kind: int, k_scale: float = 1.0, v_scale: float = 1.0,
                round_nearest: bool = False):
    """In place on numpy caches of shape [nb, Hkv, D, bs]; ``round_nearest``
    selects the nearest-even FP8 encoders instead of the reference's
    round-toward-zero."""
    nb, hkv, d, bs = key_cache.shape
    assert bs == block_size
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    lib().orc_cache_write_rounded(_p(key_cache), _p(value_cache), _p(np.ascontiguousarray(new_key)),
                                  _p(np.ascontiguousarray(new_value)), _p(sm), sm.size, hkv, d, bs, nb,
                                  in_kind, cache_kind, k_scale, v_scale, 1 if round_nearest else 0)


def rope_interleaved(x, positions, theta: float):
    """x: f16 bits [T, H, D]; the reference kernel's interleaved rotation."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.empty_like(x)
    lib().orc_rope_interleaved(_p(out), _p(x), _p(pos), x.shape[0], x.shape[1], x.shape[2], theta)
    return out


def rmsnorm(x, weight, eps: float, kind: int):
    """x: 16-bit bits [rows, hidden]; weight [hidden]; returns bits."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(out), _p(x), _p(w), x.shape[0], x.shape[1], eps, kind)
    return out


def silu_mul(gate, up, kind: int):
    g = np.ascontiguousarray(gate, dtype=np.uint16)
    u = np.ascontiguousarray(up, dtype=np.uint16)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(out), _p(g), _p(u), g.size, kind)
    return out


def _ptr_array(arrays):
    for a in arrays:
        assert a.flags["C_CONTIGUOUS"]
    return (ctypes.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])


def copy_blocks(key_caches, value_caches, pairs, num_blocks: int, block_nbytes: int):
    """In place on lists of per-layer numpy caches (any dtype, C-contiguous)."""
    pr = np.ascontiguousarray(pairs, dtype=np.int64).reshape(-1, 2)
    lib().orc_copy_blocks(_ptr_array(key_caches), _ptr_array(value_caches), len(key_caches),
                          _p(pr), pr.shape[0], num_blocks, block_nbytes)


def swap_blocks(key_caches, value_caches, ids, records, num_blocks: int, block_nbytes: int,
                out: bool, slots=None):
    """records: uint8 [num_records, layers, 2, block_nbytes] (modified when out)."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.int64)
    lib().orc_swap_blocks(_ptr_array(key_caches), _ptr_array(value_caches), len(key_caches),
                          _p(ids), ids.size, None if sl is None else _p(sl), records.shape[0],
                          num_blocks, block_nbytes, _p(records), 1 if out else 0)


def rope_cache_build(max_position: int, head_dim: int, theta: float = 10000.0):
    """(cos, sin) float32 [max_position, head_dim // 2] as rope.rs:13-33 builds them."""
    cos = np.empty((max_position, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    lib().orc_rope_cache_build(_p(cos), _p(sin), max_position, head_dim, theta)
    return cos, sin


def rope_cache_write(q, k, v, key_cache, value_cache, slot_mapping, positions, cos, sin,
                     in_kind: int, cache_kind: int, k_scale: float = 1.0, v_scale: float = 1.0,
                     round_nearest: bool = False):
    """Rotate q (returned) and k in the activation dtype, then write the rotated
    key and v into the numpy caches [nb, Hkv, D, bs] in place (FP8 rounded
    toward zero, or to nearest even with ``round_nearest``)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    T, hq, d = q.shape
    nb, hkv, d2, bs = key_cache.shape
    assert d2 == d and k.shape == (T, hkv, d) and v.shape == k.shape
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    cos = np.ascontiguousarray(cos, dtype=np.float32)
    sin = np.ascontiguousarray(sin, dtype=np.float32)
    q_out = np.empty_like(q)
    lib().orc_rope_cache_write_rounded(_p(q_out), _p(q), _p(k), _p(v), _p(key_cache), _p(value_cache),
                                       _p(sm), _p(pos), _p(cos), _p(sin), T, hq, hkv, d, bs, nb,
                                       cos.shape[0], in_kind, cache_kind, k_scale, v_scale,
                                       1 if round_nearest else 0)
    return q_out


# ---- attention -----------------------------------------------------------

def paged_attention_decode(q, q_kind, key_cache, value_cache, cache_kind, block_tables, seq_lens,
                           scale, k_scale=1.0, v_scale=1.0, precision=1, nthreads=None):
    """Returns float32 [B, Hq, D].  precision 0 = fp32, 1 = fp64 arithmetic."""
    q = np.ascontiguousarray(q)
    B, hq, d = q.shape
    nb, hkv, d2, bs = key_cache.shape
    assert d2 == d
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    out = np.zeros((B, hq, d), dtype=np.float32)
    lib().orc_paged_attention_decode(
        _p(out), _p(q), q_kind, _p(np.ascontiguousarray(key_cache)),
        _p(np.ascontiguousarray(value_cache)), cache_kind, _p(bt), _p(sl), B, hq, hkv, d, bs,
        bt.shape[1], scale, k_scale, v_scale, precision,
        nthreads or hardware_threads())
    return out


def paged_attention_prefill(q, q_kind, key_cache, value_cache, cache_kind, block_tables,
                            seq_lens, query_start_loc, scale, k_scale=1.0, v_scale=1.0,
                            precision=1, nthreads=None):
    """Returns float32 [T, Hq, D] with the context-offset causal mask."""
    q = np.ascontiguousarray(q)
    T, hq, d = q.shape
    nb, hkv, d2, bs = key_cache.shape
    assert d2 == d
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    out = np.zeros((T, hq, d), dtype=np.float32)
    lib().orc_paged_attention_prefill(
        _p(out), _p(q), q_kind, _p(np.ascontiguousarray(key_cache)),
        _p(np.ascontiguousarray(value_cache)), cache_kind, _p(bt), _p(sl), _p(qsl), sl.size, T,
        hq, hkv, d, bs, bt.shape[1], scale, k_scale, v_scale, precision,
        nthreads or hardware_threads())
    return out
