"""Shared helpers for the parity tests (input generation, error metrics)."""
from __future__ import annotations

import numpy as np

from oracle import oracle


def rel_error(a, b) -> float:
    """Max element-wise relative error with denominator max(|a|,|b|) > 1e-8 -- the
    metric of the reference's own kernel check
    (cuda_kernel_optimized/mha_kernel/bench_mha_kernels.cu:467-477, PASS if < 1e-4)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.maximum(np.abs(a), np.abs(b))
    m = den > 1e-8
    if not m.any():
        return 0.0
    return float(np.max(np.abs(a - b)[m] / den[m]))


def assert_fp32_close(got, ref, head_size, tol=1e-4, what=""):
    """fp32 bar (1e-4 relative) against the oracle, stated per head:
      * norm-wise: max|got - ref| / max|ref| over each head's head_size outputs <= tol;
      * element-wise (the reference's metric, bench_mha_kernels.cu:467-477) <= tol on
        the well-conditioned elements, |ref| >= 0.1 * max|ref| of the head.
    Element-wise error on near-zero outputs measures cancellation, not the kernel:
    the sequential-float oracle itself is up to 2e-2 element-wise away from an fp64
    evaluation there."""
    g = np.asarray(got, np.float64).reshape(-1, head_size)
    r = np.asarray(ref, np.float64).reshape(-1, head_size)
    err = np.abs(g - r)
    scale = np.abs(r).max(axis=1, keepdims=True)
    nw = (err.max(axis=1, keepdims=True) / np.maximum(scale, 1e-30)).max()
    well = np.abs(r) >= 0.1 * scale
    ew = (err[well] / np.abs(r[well])).max() if well.any() else 0.0
    assert nw <= tol and ew <= tol, f"{what}: norm-wise {nw:.3g}, element-wise {ew:.3g} > {tol}"


def assert_fp32_elementwise(got, truth, head_size, rtol=1e-4, floor=1e-6, what=""):
    """fp32 bar element by element against an fp64 evaluation of the same inputs:
    |got - truth| <= rtol * |truth| + floor * max|truth of the head| for every output.
    The floor (1e-6 of the head's largest output, ~8 fp32 ulps of it) only matters for
    outputs that cancel to near zero."""
    g = np.asarray(got, np.float64).reshape(-1, head_size)
    t = np.asarray(truth, np.float64).reshape(-1, head_size)
    bound = rtol * np.abs(t) + floor * np.abs(t).max(axis=1, keepdims=True)
    bad = np.abs(g - t) > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outputs outside "
                           f"{rtol} relative + {floor} of the head max")


def fp64_decode(q, k_rows, v_rows, head_num, kv_mul, d):
    """Softmax(q k^T / sqrt(d)) v per head in float64; k_rows / v_rows [n, kv_heads, d]."""
    Q = np.asarray(q, np.float64).reshape(head_num, d)
    Kd = np.asarray(k_rows, np.float64)
    V = np.asarray(v_rows, np.float64)
    out = np.zeros((head_num, d))
    for h in range(head_num):
        s = Kd[:, h // kv_mul] @ Q[h] / np.sqrt(d)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:, h // kv_mul]
    return out.ravel()


def assert_lowp_close(got, ref, atol=2e-3, rtol=1e-2, what=""):
    """fp16/bf16 bar: |got - ref| <= atol + rtol*|ref| against the fp32-accumulated
    oracle on the same (16-bit) inputs."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements outside atol={atol} rtol={rtol}; "
            f"worst at {i}: got {got[i]:.6g} ref {ref[i]:.6g}")


def normal(rng, shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(dtype)


def quantize(x, kind: str) -> np.ndarray:
    """Round fp32 values to the 16-bit type `kind` and return them as fp32."""
    if kind == "fp32":
        return np.asarray(x, np.float32)
    if kind == "fp16":
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
    if kind == "bf16":
        return oracle.round_bf16(x)
    raise ValueError(kind)


def qwen3_qk(rng, S, H, d, start_pos=0, theta=1e6):
    """Qwen3 Q or K rows [S, H*d]: N(0,1) -> per-head RMSNorm (unit weight, eps 1e-6)
    -> rotate-half RoPE (theta 1e6)."""
    x = normal(rng, (S, H * d))
    x = oracle.rmsnorm_rows(x, d, 1e-6)
    return oracle.rope_rotate_half(x, S, H, d, start_pos, theta)
