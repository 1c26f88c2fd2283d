"""bf16 values outside fp16's range, through the C ABI.

Decode (every path: dot-product split launches, the kuiper single-sequence entry, the
matrix-core whole-row launches in test_gpu_decode_whole_rows.py) uses bf16 V as stored, so
V scaled far beyond fp16's range (3e30) or into its subnormals (1e-6) keeps the oracle's
relative accuracy.

The prefill and the vision attention run the weighted sum in fp16 (V converted on chip),
and the header states the limits this file pins: |v| <= 65504 is exact (bf16's 8
significant bits fit fp16's 11); a value beyond it makes the outputs that weight it
non-finite (never a silently wrong finite value), those of rows attending to it and
possibly of other rows whose 64-key tile holds it; values below 2^-14 carry an absolute
error of at most 2^-25 each."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_decode import dev, host
from tests.util import assert_lowp_close, normal, quantize

SUBNORMAL_ABS = 2.0 ** -25  # half the spacing of fp16 subnormals


def _decode_case(rng, scale, B=3, Hq=32, Hkv=8, d=128, S=1500):
    lens = np.array([S, 700, 1], np.int32)[:B]
    kc = quantize(normal(rng, (B, S, Hkv, d)), "bf16")
    vc = quantize(normal(rng, (B, S, Hkv, d)) * np.float32(scale), "bf16")
    q = quantize(normal(rng, (B, Hq, d)), "bf16")
    return lens, kc, vc, q


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1e5, 3e30, 1e-6])
@pytest.mark.parametrize("split", [256, 0])
def test_split_decode_bf16_range(scale, split):
    rng = np.random.default_rng(91)
    lens, kc, vc, q = _decode_case(rng, scale)
    B, Hq, d = q.shape
    o = torch.zeros(B, Hq, d, device="cuda", dtype=torch.bfloat16)
    K.batched_decode_cu(dev(q, "bf16"), dev(kc, "bf16"), dev(vc, "bf16"), o,
                        torch.from_numpy(lens).cuda(), int(lens.max()), kc.shape[2],
                        split_tokens=split)
    torch.cuda.synchronize()
    got = host(o)
    assert np.isfinite(got).all()
    ref = oracle.decode_contig(q, kc, vc, lens)
    assert_lowp_close(got / scale, ref / scale, what=f"split decode bf16 V x {scale:g}")


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1e5, 1e-6])
def test_kuiper_flash_decode_bf16_range(scale):
    rng = np.random.default_rng(92)
    Hq, Hkv, d, max_seq, pos = 32, 8, 128, 2048, 1800
    kc = quantize(normal(rng, (max_seq, Hkv * d)), "bf16")
    vc = quantize(normal(rng, (max_seq, Hkv * d)) * np.float32(scale), "bf16")
    q = quantize(normal(rng, (Hq * d,)), "bf16")
    out = torch.empty(Hq * d, device="cuda", dtype=torch.bfloat16)
    K.flash_attention_decode_cu(pos, Hq, Hkv, d, Hq // Hkv, 0, max_seq, Hkv * d,
                                dev(q, "bf16"), out, dev(kc, "bf16"), dev(vc, "bf16"))
    torch.cuda.synchronize()
    got = host(out)
    ref = oracle.decode_contig(q.reshape(1, Hq, d), kc.reshape(1, max_seq, Hkv, d),
                               vc.reshape(1, max_seq, Hkv, d),
                               np.array([pos + 1], np.int32)).ravel()
    assert np.isfinite(got).all()
    assert_lowp_close(got / scale, ref / scale, what=f"kuiper decode bf16 V x {scale:g}")


def _prefill(rng, S, Hq, Hkv, d, vscale, spike=None):
    q = quantize(normal(rng, (S, Hq * d)), "bf16")
    k = quantize(normal(rng, (S, Hkv * d)), "bf16")
    v = normal(rng, (S, Hkv * d)) * np.float32(vscale)
    if spike is not None:
        v[spike] = 1e5
    v = quantize(v, "bf16")
    o = torch.empty(S, Hq * d, device="cuda", dtype=torch.bfloat16)
    K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d, dev(q, "bf16"), o,
                                 dev(k, "bf16"), dev(v, "bf16"))
    torch.cuda.synchronize()
    return q, k, v, host(o)


@pytest.mark.gpu
@pytest.mark.parametrize("S,Hq,Hkv", [(300, 4, 2), (4096, 32, 8)])
def test_prefill_bf16_in_range_is_exact(S, Hq, Hkv):
    """|v| up to ~6e4 (inside fp16's range): the lowp bar on unit-scaled values."""
    rng = np.random.default_rng(93)
    d, scale = 128, 1.1e4
    q, k, v, got = _prefill(rng, S, Hq, Hkv, d, scale)
    assert 25000 < np.abs(v).max() < 65504
    rows = np.unique(np.r_[0, S - 1, rng.integers(0, S, 24)])
    ref = oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(got[rows] / scale, ref / scale, what="bf16 prefill V in range")


@pytest.mark.gpu
def test_prefill_bf16_beyond_fp16_is_non_finite():
    """A V element past 65504 makes every output that weights it non-finite (rows at or
    after its key, in its column, for the query heads of its kv head); rows whose keys end
    before the element's 64-key tile are untouched and keep the lowp bar."""
    rng = np.random.default_rng(94)
    S, Hq, Hkv, d = 300, 4, 2, 128
    key, col = 150, 5  # kv head 0, dimension 5; 64-key tile 2 starts at key 128
    q, k, v, got = _prefill(rng, S, Hq, Hkv, d, 1.0, spike=(key, col))
    for h in range(Hq // Hkv):  # the query heads of kv head 0
        assert not np.isfinite(got[key:, h * d + col]).any(), \
            "outputs weighting the 1e5 element must be non-finite"
    clean = np.arange(128)
    ref = oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, rows=clean)
    assert np.isfinite(got[clean]).all()
    assert_lowp_close(got[clean], ref, what="bf16 prefill rows before the spike's tile")


@pytest.mark.gpu
def test_prefill_bf16_subnormal_error_bound():
    """V ~ 1e-6 (fp16 subnormals): |got - ref| <= 2^-25 + 1e-2 |ref| (conversion error
    of each V element plus the weights' fp16 rounding)."""
    rng = np.random.default_rng(95)
    S, Hq, Hkv, d = 300, 4, 2, 128
    q, k, v, got = _prefill(rng, S, Hq, Hkv, d, 1e-6)
    ref = oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, rows=np.arange(S))
    err = np.abs(got - ref)
    assert (err <= SUBNORMAL_ABS + 1e-2 * np.abs(ref)).all(), float(err.max())


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1.1e4, 1e-6])
def test_vision_bf16_range(scale):
    """The vision attention under the same limits: in-range V exact to the lowp bar on
    unit-scaled values; subnormal V within 2^-25 absolute."""
    rng = np.random.default_rng(96)
    H, N, d = 16, 512, 72
    q = quantize(normal(rng, (H, N, d)), "bf16")
    k = quantize(normal(rng, (H, N, d)), "bf16")
    v = quantize(normal(rng, (H, N, d)) * np.float32(scale), "bf16")
    o = torch.empty(N, H * d, device="cuda", dtype=torch.bfloat16)
    K.vision_attention_pretransposed_cu(dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), o, None,
                                        None, N, H, d, 0.0)
    torch.cuda.synchronize()
    got = host(o)
    ref = oracle.varlen_bidir(q, k, v, np.array([0, N], np.int32), nthreads=8)
    if scale > 1:
        assert np.abs(v).max() < 65504
        assert_lowp_close(got / scale, ref / scale, what="bf16 vision V in range")
    else:
        err = np.abs(got - ref)
        assert (err <= SUBNORMAL_ABS + 1e-2 * np.abs(ref)).all(), float(err.max())
