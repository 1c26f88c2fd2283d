"""Write the golden fixtures used to pin the CPU oracle.

Inputs are regenerated in the tests from the stored numpy seeds (PCG64
`default_rng`); each fixture stores the seed, the shape parameters, a checksum of
the inputs and the expected output computed by PyTorch's CPU
`scaled_dot_product_attention` in float64 (a library routine, independent of the
oracle's code).  Run from the repo root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def sdpa(q, k, v, causal_offset=None, mask=None):
    """q [H, M, d], k/v [H, N, d] float64 -> [H, M, d]."""
    q, k, v = (torch.from_numpy(x).to(torch.float64) for x in (q, k, v))
    if causal_offset is not None:
        M, N = q.shape[1], k.shape[1]
        mask = torch.arange(N)[None, :] <= (torch.arange(M)[:, None] + causal_offset)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask).numpy()


def decode_case(name, seed, Hq, Hkv, d, pos, seq_len):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((seq_len, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((seq_len, Hkv * d)).astype(np.float32)
    rep = Hq // Hkv
    K = np.repeat(k[: pos + 1].reshape(pos + 1, Hkv, d).transpose(1, 0, 2), rep, axis=0)
    V = np.repeat(v[: pos + 1].reshape(pos + 1, Hkv, d).transpose(1, 0, 2), rep, axis=0)
    out = sdpa(q.reshape(Hq, 1, d), K, V)[:, 0, :].reshape(-1)
    np.savez(os.path.join(HERE, f"{name}.npz"), seed=seed, Hq=Hq, Hkv=Hkv, d=d, pos=pos,
             seq_len=seq_len, checksum=float(q.sum() + k.sum() + v.sum()), out=out)


def prefill_case(name, seed, Hq, Hkv, d, start_pos, S):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((S, Hq * d)).astype(np.float32)
    k = rng.standard_normal((start_pos + S, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((start_pos + S, Hkv * d)).astype(np.float32)
    rep = Hq // Hkv
    Q = q.reshape(S, Hq, d).transpose(1, 0, 2)
    K = np.repeat(k.reshape(-1, Hkv, d).transpose(1, 0, 2), rep, axis=0)
    V = np.repeat(v.reshape(-1, Hkv, d).transpose(1, 0, 2), rep, axis=0)
    out = sdpa(Q, K, V, causal_offset=start_pos).transpose(1, 0, 2).reshape(S, Hq * d)
    np.savez(os.path.join(HERE, f"{name}.npz"), seed=seed, Hq=Hq, Hkv=Hkv, d=d,
             start_pos=start_pos, S=S, checksum=float(q.sum() + k.sum() + v.sum()), out=out)


def varlen_case(name, seed, H, d, cu):
    rng = np.random.default_rng(seed)
    N = cu[-1]
    q = rng.standard_normal((H, N, d)).astype(np.float32)
    k = rng.standard_normal((H, N, d)).astype(np.float32)
    v = rng.standard_normal((H, N, d)).astype(np.float32)
    out = np.zeros((N, H * d))
    for a, b in zip(cu[:-1], cu[1:]):
        out[a:b] = sdpa(q[:, a:b], k[:, a:b], v[:, a:b]).transpose(1, 0, 2).reshape(b - a, H * d)
    np.savez(os.path.join(HERE, f"{name}.npz"), seed=seed, H=H, d=d, cu=np.array(cu),
             checksum=float(q.sum() + k.sum() + v.sum()), out=out)


def main():
    # 12 q = 12 kv heads, d 64, query at pos 255 over 256 tokens.
    decode_case("c1_decode", 0xC1, 12, 12, 64, 255, 256)
    decode_case("gqa_decode", 0x61, 8, 2, 32, 100, 128)
    prefill_case("causal_prefill", 0x51, 4, 2, 16, 10, 40)
    varlen_case("varlen_bidir", 0x71, 2, 8, [0, 7, 20, 32])
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
