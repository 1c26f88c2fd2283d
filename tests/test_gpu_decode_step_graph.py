"""One attention decode step captured whole in a HIP graph, as the reference captures its
decode (kuiper/source/model/qwen_base.cpp:680-756: per layer attention_qkv_with_graph then
attention_mha_with_graph, with the position in device memory):

  layer 0 (Qwen3): orin_qk_norm_rope(pos_ptr) -> RMSNorm + RoPE of q in place, k/v rows
                   stored at *pos; orin_flash_attention_decode_gpu_pos
  layer 1 (Qwen2 / Llama cache append): orin_copy_to_kv_cache of k and v at *pos;
                   orin_flash_attention_decode_gpu_pos

The graph is replayed for consecutive positions with new inputs each time.  Every replay
equals the same calls made eagerly (outputs and caches bit for bit), the produced q/k rows
match the oracle producer, and the attention outputs match the oracle MHA over the cache."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_producers import rope_with_tables
from tests.util import assert_lowp_close, normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_captured_decode_step(kind):
    rng = np.random.default_rng(51)
    Hq, Hkv, d, max_seq, layers, P0 = 32, 8, 128, 2048, 2, 1000
    kv_dim, kv_mul, dt = Hkv * d, Hq // Hkv, TORCH[kind]

    def t(x):
        return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", dt)

    prefix_k = quantize(normal(rng, (layers, P0, kv_dim)), kind)
    prefix_v = quantize(normal(rng, (layers, P0, kv_dim)), kind)

    def caches():
        kc = torch.zeros(layers, max_seq, kv_dim, device="cuda", dtype=dt)
        vc = torch.zeros_like(kc)
        kc[:, :P0] = t(prefix_k)
        vc[:, :P0] = t(prefix_v)
        return kc, vc

    kc_g, vc_g = caches()  # used by the graph
    kc_e, vc_e = caches()  # used by the eager mirror
    s_t = torch.empty(max_seq, d, device="cuda")
    c_t = torch.empty(max_seq, d, device="cuda")
    K.sin_cos_cache_calc_cu(d, max_seq, s_t, c_t, 1e6)
    wq, wk = (t(1.0 + 0.1 * normal(rng, (d,))) for _ in range(2))
    # fixed input buffers, refilled before every replay (the graph's inputs)
    q_in, k_in, v_in = t(np.zeros(Hq * d)), t(np.zeros(kv_dim)), t(np.zeros(kv_dim))
    q1_in, k1_in, v1_in = t(np.zeros(Hq * d)), t(np.zeros(kv_dim)), t(np.zeros(kv_dim))
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")

    def step(kc, vc, q_work, out0, out1, stream):
        cfg = K.CudaConfig(stream)
        q_work.copy_(q_in)
        K.qk_norm_rope_cu(q_work, k_in, v_in, wq, wk, s_t, c_t, kc, vc, 0, max_seq, 0, 1, Hq,
                          Hkv, d, pos_ptr=pos, config=cfg)
        K.flash_attention_decode_fp16_gpu_pos_cu(pos, Hq, Hkv, d, kv_mul, 0, max_seq, kv_dim,
                                                 q_work, out0, kc, vc, config=cfg)
        K.copy_to_kv_cache_kernel(kc, k1_in, pos, kv_dim, 1, max_seq, config=cfg)
        K.copy_to_kv_cache_kernel(vc, v1_in, pos, kv_dim, 1, max_seq, config=cfg)
        K.flash_attention_decode_fp16_gpu_pos_cu(pos, Hq, Hkv, d, kv_mul, 1, max_seq, kv_dim,
                                                 q1_in, out1, kc, vc, config=cfg)

    def bufs():
        return (torch.zeros(Hq * d, device="cuda", dtype=dt),
                torch.zeros(Hq * d, device="cuda", dtype=dt),
                torch.zeros(Hq * d, device="cuda", dtype=dt))

    qw_g, o0_g, o1_g = bufs()
    qw_e, o0_e, o1_e = bufs()
    cap = torch.cuda.Stream()
    K.reserve_decode_workspace(Hq, d, max_seq, stream=cap)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        step(kc_g, vc_g, qw_g, o0_g, o1_g, cap)
    torch.cuda.synchronize()
    # capture queued nothing: the graph's caches still hold only the prefix
    assert not kc_g[:, P0:].any()

    sin_h = s_t.cpu().numpy().astype(np.float64)
    cos_h = c_t.cpu().numpy().astype(np.float64)
    wq_h, wk_h = wq.float().cpu().numpy(), wk.float().cpu().numpy()
    for p in range(P0, P0 + 5):
        x = [quantize(normal(rng, n), kind) for n in (Hq * d, kv_dim, kv_dim, Hq * d, kv_dim,
                                                       kv_dim)]
        for buf, val in zip((q_in, k_in, v_in, q1_in, k1_in, v1_in), x):
            buf.copy_(t(val))
        pos.fill_(p)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        step(kc_e, vc_e, qw_e, o0_e, o1_e, torch.cuda.current_stream())
        torch.cuda.synchronize()
        for a, b, what in [(o0_g, o0_e, "layer-0 output"), (o1_g, o1_e, "layer-1 output"),
                           (qw_g, qw_e, "produced q"), (kc_g, kc_e, "k cache"),
                           (vc_g, vc_e, "v cache")]:
            assert torch.equal(a, b), f"replay at pos {p}: {what} differs from eager"
        # producer rows against the oracle (RMSNorm, then the rotation with the tables)
        qn = oracle.rmsnorm_rows(x[0][None], d, 1e-6, wq_h)
        kn = oracle.rmsnorm_rows(x[1][None], d, 1e-6, wk_h)
        kc_h = kc_g.float().cpu().numpy()
        vc_h = vc_g.float().cpu().numpy()
        q_h = qw_g.float().cpu().numpy()
        assert_lowp_close(q_h, rope_with_tables(qn, sin_h, cos_h, [p], Hq, d)[0],
                          what=f"q at {p}")
        assert_lowp_close(kc_h[0, p], rope_with_tables(kn, sin_h, cos_h, [p], Hkv, d)[0],
                          what=f"k row at {p}")
        np.testing.assert_array_equal(vc_h[0, p], x[2])
        np.testing.assert_array_equal(kc_h[1, p], x[4])
        np.testing.assert_array_equal(vc_h[1, p], x[5])
        # attention outputs against the oracle MHA over the cache rows 0..p
        ref0, _ = oracle.mha_kernel(p, Hq, 0, max_seq, kv_dim, kv_mul, d, q_h, kc_h, vc_h)
        ref1, _ = oracle.mha_kernel(p, Hq, 1, max_seq, kv_dim, kv_mul, d, x[3], kc_h, vc_h)
        assert_lowp_close(o0_g.float().cpu().numpy(), ref0, what=f"layer 0 at {p}")
        assert_lowp_close(o1_g.float().cpu().numpy(), ref1, what=f"layer 1 at {p}")
