"""GPU parity of bidirectional (vision) attention, single segment and varlen."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.util import assert_fp32_close, assert_lowp_close, normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def vision_inputs(rng, cu, H, d, kind, grid=None):
    N = int(cu[-1])
    q, k, v = normal(rng, (H, N, d)), normal(rng, (H, N, d)), normal(rng, (H, N, d))
    if grid is not None:  # 2-D rotary per image on a grid x grid patch layout
        c, s = oracle.vision_cos_sin(1, grid, grid, 2, d)
        c = np.concatenate([c] * (len(cu) - 1))
        s = np.concatenate([s] * (len(cu) - 1))
        q, k = oracle.vision_rotary(q, c, s), oracle.vision_rotary(k, c, s)
    return quantize(q, kind), quantize(k, kind), quantize(v, kind)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_c5_vision_varlen(kind):
    """4 images x 1024 patches packed varlen, 16 heads, d 72, 2-D rotary
    on a 32x32 grid."""
    rng = np.random.default_rng(0xC5)
    H, d = 16, 72
    cu = np.array([0, 1024, 2048, 3072, 4096], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind, grid=32)
    out = torch.zeros(4096, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), 1024, H, d)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1023, 1024, 2047, 4095],
                                     rng.integers(0, 4096, 64)]))
    ref = oracle.varlen_bidir(q, k, v, cu, rows=rows, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy()[rows], ref, what=f"C5 {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("d", [64, 72, 80, 128])
def test_varlen_ragged_segments(kind, d):
    rng = np.random.default_rng(d)
    H = 4
    cu = np.array([0, 100, 356, 357, 1000], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    out = torch.zeros(1000, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), 643, H, d)
    torch.cuda.synchronize()
    ref = oracle.varlen_bidir(q, k, v, cu, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy(), ref, what=f"varlen {kind} d {d}")


@pytest.mark.parametrize("kind", ["fp16", "bf16", "fp32"])
def test_pretransposed_single_segment(kind):
    """kernel::vision_attention_pretransposed_cu semantics: one segment of N tokens."""
    rng = np.random.default_rng(5)
    H, N = 16, 300
    d = 64 if kind == "fp32" else 72  # the fp32 path takes d in {64, 128, 256}
    cu = np.array([0, N], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_pretransposed_cu(dev(q, kind), dev(k, kind), dev(v, kind), out, None, None,
                                        N, H, d, 1.0 / np.sqrt(d))
    torch.cuda.synchronize()
    ref = oracle.varlen_bidir(q, k, v, cu, nthreads=8)
    if kind == "fp32":
        assert_fp32_close(out.cpu().numpy(), ref, d, what="fp32 vision")
    else:
        assert_lowp_close(out.float().cpu().numpy(), ref, what=f"single {kind}")


def test_varlen_equals_separate_segments():
    """Packing segments with cu_seqlens gives the same rows as attending each alone."""
    rng = np.random.default_rng(9)
    H, d = 16, 72
    cu = np.array([0, 200, 700, 1024], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, "bf16")
    out = torch.zeros(1024, H * d, device="cuda", dtype=torch.bfloat16)
    K.vision_attention_varlen_cu(dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out,
                                 torch.from_numpy(cu).cuda(), 500, H, d)
    for s in range(3):
        a, b = cu[s], cu[s + 1]
        o = torch.zeros(b - a, H * d, device="cuda", dtype=torch.bfloat16)
        K.vision_attention_pretransposed_cu(dev(q[:, a:b], "bf16"), dev(k[:, a:b], "bf16"),
                                            dev(v[:, a:b], "bf16"), o, None, None, int(b - a), H,
                                            d, 0.0)
        torch.cuda.synchronize()
        assert torch.equal(o, out[a:b]), f"segment {s}"
