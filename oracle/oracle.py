"""numpy front end of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product (orinmllm_amd) never
imports it.  Each function names the reference code it restates; oracle.c holds
the arithmetic and its citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, I, Lg, F = C.c_void_p, C.c_int, C.c_long, C.c_float
        L.oracle_mha_kernel.argtypes = [I, I, I, I, I, I, I, P, P, P, P, P]
        L.oracle_attn_rows.argtypes = [I, I, I, I, F, P, Lg, Lg, P, P, Lg, Lg, P, P, P, Lg, P,
                                       Lg, Lg, I]
        L.oracle_decode_paged.argtypes = [I, I, I, I, F, P, P, P, P, I, I, P, P, I]
        L.oracle_prefill_causal.argtypes = [I, I, I, I, I, F, P, P, P, P, I]
        L.oracle_varlen_bidir.argtypes = [I, I, I, F, P, P, P, P, I, P, I]
        L.oracle_rope_rotate_half.argtypes = [P, I, I, I, I, F]
        L.oracle_rmsnorm_rows.argtypes = [P, Lg, I, F, P]
        L.oracle_vision_cos_sin.argtypes = [I, I, I, I, I, P, P]
        L.oracle_vision_rotary.argtypes = [P, I, I, I, P, P]
        L.oracle_max_threads.restype = I
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def default_scale(d: int) -> float:
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def max_threads() -> int:
    return lib().oracle_max_threads()


# ------------------------------------------------------------------ attention

def mha_kernel(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, query, key_cache,
               value_cache):
    """kernel::mha_kernel (kuiper/source/op/kernels/cpu/mha_kernel.cpp:5-62), fp32.
    Returns (mha_out [head_num*head_size], score [head_num, seq_len])."""
    q, k, v = _f32(query), _f32(key_cache), _f32(value_cache)
    out = np.zeros(head_num * head_size, np.float32)
    score = np.zeros((head_num, seq_len), np.float32)
    lib().oracle_mha_kernel(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                            _p(out), _p(q), _p(score), _p(k), _p(v))
    return out, score


def decode_contig(q, k_cache, v_cache, lens, scale=None, nthreads=1):
    """Batched decode: q [B, Hq, d]; caches [B, S, Hkv, d]; lens [B]. -> [B, Hq, d]."""
    q, k, v, lens = _f32(q), _f32(k_cache), _f32(v_cache), _i32(lens)
    B, Hq, d = q.shape
    _, S, Hkv, _ = k.shape
    out = np.zeros_like(q)
    off = (np.arange(B, dtype=np.int64) * S * Hkv * d).astype(np.int64)
    lib().oracle_attn_rows(B, Hq, Hkv, d, default_scale(d) if scale is None else scale, _p(q),
                           Hq * d, d, _p(k), _p(v), Hkv * d, d, _p(off), _p(lens), None, 0,
                           _p(out), Hq * d, d, nthreads)
    return out


def decode_paged(q, k_pool, v_pool, block_tables, lens, scale=None, nthreads=1):
    """Paged decode: q [B, Hq, d]; pools [nblk, bs, Hkv, d]; block_tables [B, max_blocks]."""
    q, k, v = _f32(q), _f32(k_pool), _f32(v_pool)
    bt, lens = _i32(block_tables), _i32(lens)
    B, Hq, d = q.shape
    _, bs, Hkv, _ = k.shape
    out = np.zeros_like(q)
    lib().oracle_decode_paged(B, Hq, Hkv, d, default_scale(d) if scale is None else scale,
                              _p(q), _p(k), _p(v), _p(bt), bt.shape[1], bs, _p(lens), _p(out),
                              nthreads)
    return out


def prefill_causal(start_pos, q, k_cache, v_cache, Hq, Hkv, d, scale=None, nthreads=1,
                   rows=None):
    """Causal prefill: q [S, Hq*d]; caches [max_seq, Hkv*d] (one layer).  Row i attends
    0..start_pos+i.  `rows` restricts the computation to a subset of query rows
    (returns [len(rows), Hq*d])."""
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    S = q.shape[0]
    idx = np.arange(S) if rows is None else np.asarray(rows)
    qs = _f32(q.reshape(S, Hq * d)[idx])
    lens = _i32(start_pos + idx + 1)
    out = np.zeros_like(qs)
    lib().oracle_attn_rows(len(idx), Hq, Hkv, d, default_scale(d) if scale is None else scale,
                           _p(qs), Hq * d, d, _p(k), _p(v), Hkv * d, d, None, _p(lens), None, 0,
                           _p(out), Hq * d, d, nthreads)
    return out


def varlen_bidir(q, k, v, cu_seqlens, scale=None, nthreads=1, rows=None):
    """Bidirectional varlen: q/k/v [H, N, d] head-major, cu_seqlens [n+1] -> [N, H*d]
    (or [len(rows), H*d] for a subset of query tokens)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    cu = _i32(cu_seqlens)
    H, N, d = q.shape
    sc = default_scale(d) if scale is None else scale
    if rows is None:
        out = np.zeros((N, H * d), np.float32)
        lib().oracle_varlen_bidir(N, H, d, sc, _p(q), _p(k), _p(v), _p(cu), len(cu) - 1, _p(out),
                                  nthreads)
        return out
    idx = np.asarray(rows)
    seg = np.searchsorted(cu, idx, side="right") - 1
    qs = _f32(np.transpose(q[:, idx, :], (1, 0, 2)))  # [R, H, d]
    off = (cu[seg].astype(np.int64) * d).astype(np.int64)
    lens = _i32(cu[seg + 1] - cu[seg])
    out = np.zeros((len(idx), H * d), np.float32)
    lib().oracle_attn_rows(len(idx), H, H, d, sc, _p(qs), H * d, d, _p(k), _p(v), d, N * d,
                           _p(off), _p(lens), None, 0, _p(out), H * d, d, nthreads)
    return out


# ------------------------------------------------------------------ producers

def rope_rotate_half(x, S, H, d, start_pos=0, theta=1e6):
    """Qwen rotate-half RoPE of x [S, H*d] (rope_kernel.cu:86-98, 464-509)."""
    y = _f32(x).copy()
    lib().oracle_rope_rotate_half(_p(y), S, H, d, start_pos, theta)
    return y


def rmsnorm_rows(x, d, eps=1e-6, weight=None):
    """Per-row RMSNorm over the last d values (rmsnorm_kernel.cu:483-545)."""
    y = _f32(x).copy()
    w = None if weight is None else _f32(weight)
    lib().oracle_rmsnorm_rows(_p(y), y.size // d, d, eps, None if w is None else _p(w))
    return y


def vision_cos_sin(grid_t, grid_h, grid_w, merge, d):
    """2-D rotary tables [N, d] of qwen3_vl.cpp:1698-1831."""
    n = grid_t * grid_h * grid_w
    c = np.zeros((n, d), np.float32)
    s = np.zeros((n, d), np.float32)
    lib().oracle_vision_cos_sin(grid_t, grid_h, grid_w, merge, d, _p(c), _p(s))
    return c, s


def vision_rotary(x, cos_t, sin_t):
    """Apply the vision rotary to x [H, N, d] (vision_encoder_kernel.cu:662-744)."""
    y = _f32(x).copy()
    H, N, d = y.shape
    lib().oracle_vision_rotary(_p(y), H, N, d, _p(_f32(cos_t)), _p(_f32(sin_t)))
    return y


# ------------------------------------------------------------------ 16-bit formats

def to_f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16)


def to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) as uint16 bit patterns."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    return bf16_bits_to_f32(to_bf16_bits(x))
