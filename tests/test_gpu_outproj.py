"""orin_batched_matmul (the wo output projection on the attention output) against a plain
PyTorch fp32 matmul of the same 16-bit inputs, and chained after the prefill as kuiper's
prefill runs it (kuiper/source/model/qwen_base.cpp:464-474)."""
import numpy as np
import pytest
import torch

from orinmllm_amd import _lib
from orinmllm_amd import kernel as K
from tests.util import assert_lowp_close

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("kind", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("batch,in_dim,out_dim,scale", [(4096, 4096, 4096, 1.0), (7, 96, 200, 0.5),
                                                        (300, 1536, 1536, 1.0)])
def test_batched_matmul_vs_torch_fp32(kind, batch, in_dim, out_dim, scale):
    g = torch.Generator(device="cuda")
    g.manual_seed(batch + in_dim)
    x = torch.randn(batch, in_dim, device="cuda", generator=g).to(TORCH[kind])
    w = (torch.randn(out_dim, in_dim, device="cuda", generator=g) / in_dim ** 0.5).to(TORCH[kind])
    out = torch.full((batch, out_dim), float("nan"), device="cuda", dtype=TORCH[kind])
    K.batched_matmul_kernel_cu(x, w, out, batch, scale)
    ref = scale * (x.float() @ w.float().t())
    torch.cuda.synchronize()
    if kind == "fp32":
        err = (out - ref).abs().max().item()
        assert err <= 1e-4 * max(1.0, ref.abs().max().item()), err
    else:
        assert_lowp_close(out.float().cpu().numpy(), ref.cpu().numpy(), what=f"wo {kind}")


def test_prefill_then_output_projection():
    """The C2-shape prefill output consumed in place by the projection."""
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    S, Hq, Hkv, d = 2048, 12, 2, 128
    q = torch.randn(S, Hq * d, device="cuda", generator=g).half()
    k = torch.randn(S, Hkv * d, device="cuda", generator=g).half()
    v = torch.randn(S, Hkv * d, device="cuda", generator=g).half()
    o = torch.empty_like(q)
    K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d, q, o, k, v)
    w = (torch.randn(Hq * d, Hq * d, device="cuda", generator=g) / (Hq * d) ** 0.5).half()
    y = torch.empty_like(q)
    K.batched_matmul_kernel_cu(o, w, y, S)
    ref = o.float() @ w.float().t()
    torch.cuda.synchronize()
    assert_lowp_close(y.float().cpu().numpy(), ref.cpu().numpy(), what="prefill + wo")


def test_batched_matmul_argument_errors():
    lib = _lib.load()
    x = torch.zeros(4, 8, device="cuda", dtype=torch.float16)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.orin_batched_matmul(x.data_ptr(), x.data_ptr(), x.data_ptr(), 0, 8, 8, 1.0,
                                   _lib.DTYPE_FP16, s) == _lib.ERR_INVALID_ARG
    assert lib.orin_batched_matmul(x.data_ptr(), x.data_ptr(), x.data_ptr(), 4, 8, 8, 1.0, 7,
                                   s) == _lib.ERR_UNSUPPORTED


def test_output_projection_graph_capture():
    """After orin_attn_workspace_reserve_stream (which prepares the device's rocBLAS handle
    and workspace) the projection can be captured: every replay, with new inputs written
    eagerly between replays, equals an eager call."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    B, n = 32, 4096  # the decode step's wo: 32 rows x 4096 -> 4096
    x = torch.randn(B, n, device="cuda", generator=g).half()
    w = (torch.randn(n, n, device="cuda", generator=g) / n ** 0.5).half()
    out = torch.full((B, n), float("nan"), device="cuda", dtype=torch.float16)
    cap = torch.cuda.Stream()
    K.reserve_decode_workspace(32, 128, 4096, stream=cap)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        K.batched_matmul_kernel_cu(x, w, out, B, 1.0, config=K.CudaConfig(cap))
    for i in range(3):
        x.copy_(torch.randn(B, n, device="cuda", generator=g).half())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        K.batched_matmul_kernel_cu(x, w, eager, B, 1.0)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("batch,in_dim,out_dim", [(1, 4096, 4096), (7, 1536, 1536), (16, 512, 16),
                                                  (32, 4096, 4096), (33, 1536, 4096),
                                                  (64, 2048, 1024)])
def test_decode_rows_projection_vs_fp64(kind, batch, in_dim, out_dim):
    """Decode-sized batches (one token per sequence): against a float64 matmul of the same
    16-bit inputs, within the lowp bar."""
    g = torch.Generator(device="cuda")
    g.manual_seed(batch * 7 + in_dim + out_dim)
    x = torch.randn(batch, in_dim, device="cuda", generator=g).to(TORCH[kind])
    w = (torch.randn(out_dim, in_dim, device="cuda", generator=g) / in_dim ** 0.5).to(TORCH[kind])
    out = torch.full((batch, out_dim), float("nan"), device="cuda", dtype=TORCH[kind])
    K.batched_matmul_kernel_cu(x, w, out, batch, 0.75)
    torch.cuda.synchronize()
    ref = 0.75 * (x.double().cpu().numpy() @ w.double().cpu().numpy().T)
    assert_lowp_close(out.float().cpu().numpy(), ref, what=f"decode wo {kind} {batch}x{in_dim}x{out_dim}")


def test_decode_step_then_projection_vs_oracle():
    """The C4 decode step (batch 32, Qwen3 heads, paged fp16 pool) followed by its wo: the
    oracle's decode output multiplied by wo in float64 is the reference."""
    from oracle import oracle
    from tests.test_gpu_decode import make_paged
    from tests.util import normal, quantize
    rng = np.random.default_rng(5)
    B, Hq, Hkv, d, bs = 32, 32, 8, 128, 16
    lens = rng.integers(1, 900, B).astype(np.int32)
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, "fp16")
    q = quantize(normal(rng, (B, Hq, d)), "fp16")
    w = quantize(normal(rng, (Hq * d, Hq * d)) / np.float32(np.sqrt(Hq * d)), "fp16")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", torch.float16)
    attn = torch.empty(B, Hq, d, device="cuda", dtype=torch.float16)
    K.paged_decode_cu(dev(q), dev(kp), dev(vp), attn, torch.from_numpy(bt).cuda(),
                      torch.from_numpy(lens).cuda(), int(lens.max()),
                      layout=K.KV_LAYOUT_TOKEN_MAJOR)
    y = torch.empty(B, Hq * d, device="cuda", dtype=torch.float16)
    K.batched_matmul_kernel_cu(attn.view(B, Hq * d), dev(w), y, B)
    torch.cuda.synchronize()
    ref_attn = oracle.decode_contig(q, kc, vc, lens).reshape(B, Hq * d)
    ref = ref_attn.astype(np.float64) @ w.astype(np.float64).T
    # the decode output is rounded to fp16 before the projection: bound that rounding too
    assert_lowp_close(y.float().cpu().numpy(), ref, atol=4e-3, rtol=2e-2, what="decode + wo")
