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
