"""GPU parity of the MFMA prefill when the running row maximum must be raised past the
first tile.

The MFMA kernels keep each row's running maximum m fixed while a tile's weights
2^(c*(s - m)) stay small and raise it (rescaling O and l) only when they would not; random
N(0, 1) inputs almost never take that path after a row's first tile.  Here the scores
are made to climb along the key axis (each key carries a multiple of its position along a
direction the queries share), so later tiles keep raising m, in steps from a fraction of
a tile to far beyond the 2^8 weight bound; a mid-sequence jump and falling scores cover
the other orders.  Results are checked against the oracle at the 16-bit bar."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.util import assert_lowp_close, normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def ramp_keys(rng, n, d, slope, jump_at=None, jump=0.0):
    """Keys N(0, 0.5^2) plus (slope * t [+ jump for t >= jump_at]) * u, u a unit vector."""
    u = normal(rng, (d,))
    u /= np.linalg.norm(u)
    t = np.arange(n, dtype=np.float32)
    along = slope * t
    if jump_at is not None:
        along = along + np.where(t >= jump_at, jump, 0.0)
    return 0.5 * normal(rng, (n, d)) + along[:, None] * u[None, :], u


# slope 0.37: the row maximum climbs ~6 log2 units per 64-key tile (past the 2^8 bound);
# slope 0.05: under one unit per tile; negative: the first tile holds the maximum.
CASES = [("climb", 0.37, None, 0.0), ("creep", 0.05, None, 0.0), ("fall", -0.2, None, 0.0),
         ("jump", 0.0, 700, 60.0)]


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("name,slope,jump_at,jump", CASES)
@pytest.mark.parametrize("shape", ["plain", "key_split"])
def test_prefill_rising_scores(kind, name, slope, jump_at, jump, shape):
    rng = np.random.default_rng(31)
    # plain: 4 query blocks x 64 heads fill the device (ping-pong kernel without a key
    # split); key_split: 8 blocks x 4 heads, so the launch splits each block's keys.
    S, Hq, Hkv, d = (1024, 64, 8, 128) if shape == "plain" else (2048, 4, 1, 128)
    k, u = ramp_keys(rng, S, d, slope, jump_at, jump)
    kc = np.repeat(k[:, None, :], Hkv, axis=1).reshape(S, Hkv * d)
    q = (normal(rng, (S, Hq, d)) + 2.0 * u[None, None, :]).reshape(S, Hq * d)
    vc = normal(rng, (S, Hkv * d))
    q, kc, vc = quantize(q, kind), quantize(kc, kind), quantize(vc, kind)
    out = torch.zeros(S, Hq * d, device="cuda", dtype=TORCH[kind])
    K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d, dev(q, kind), out,
                                 dev(kc, kind), dev(vc, kind))
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1, 63, 64, 65, 255, 256, S - 1],
                                     rng.integers(0, S, 40)]))
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy()[rows], ref, what=f"{name} {shape} {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("name,slope,jump_at,jump", CASES)
def test_varlen_rising_scores(kind, name, slope, jump_at, jump):
    """Bidirectional varlen (the vision path, d 72): every query sees the climbing keys."""
    rng = np.random.default_rng(32)
    H, d = 16, 72
    cu = np.array([0, 1024, 2048, 3072, 4096], np.int32)
    N = int(cu[-1])
    k = np.empty((H, N, d), np.float32)
    q = np.empty((H, N, d), np.float32)
    for s in range(len(cu) - 1):
        n = int(cu[s + 1] - cu[s])
        for h in range(H):
            kk, u = ramp_keys(rng, n, d, slope, jump_at, jump)
            k[h, cu[s]:cu[s + 1]] = kk
            q[h, cu[s]:cu[s + 1]] = normal(rng, (n, d)) + 2.0 * u[None, :]
    v = normal(rng, (H, N, d))
    q, k, v = quantize(q, kind), quantize(k, kind), quantize(v, kind)
    out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), 1024, H, d)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1023, 1024, 4095], rng.integers(0, N, 40)]))
    ref = oracle.varlen_bidir(q, k, v, cu, rows=rows, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy()[rows], ref, what=f"{name} varlen {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("name,slope,jump_at,jump", CASES)
@pytest.mark.parametrize("split", [0, 256, 4096])
def test_decode_rising_scores(kind, name, slope, jump_at, jump, split):
    """Split-KV decode (whole-row mode at split 4096 for 16-bit K/V) over the same climbing,
    creeping, falling and jumping keys; short rows (2, 63, 64, 65 keys) included."""
    rng = np.random.default_rng(33)
    B, Hq, Hkv, d, S = 8, 32, 8, 128, 2048
    lens = np.array([2, 63, 64, 65, 300, 700, 1500, 2048], np.int32)
    kc = np.empty((B, S, Hkv, d), np.float32)
    q = np.empty((B, Hq, d), np.float32)
    for b in range(B):
        for g in range(Hkv):
            kk, u = ramp_keys(rng, S, d, slope, jump_at, jump)
            kc[b, :, g] = kk
            q[b, g * (Hq // Hkv):(g + 1) * (Hq // Hkv)] = normal(rng, (Hq // Hkv, d)) + 2.0 * u
    vc = normal(rng, (B, S, Hkv, d))
    q, kc, vc = quantize(q, kind), quantize(kc, kind), quantize(vc, kind)
    out = torch.zeros(B, Hq, d, device="cuda", dtype=TORCH[kind])
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), out,
                        torch.from_numpy(lens).cuda(), S, Hkv, split_tokens=split)
    torch.cuda.synchronize()
    ref = oracle.decode_contig(q, kc, vc, lens)
    assert_lowp_close(out.float().cpu().numpy(), ref, what=f"{name} decode split {split} {kind}")
