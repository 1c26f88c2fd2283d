"""The query producer fused into the prefill's Q load
(orin_flash_attention_prefill_qk_norm_rope) against the two-pass path (orin_qk_norm_rope on
the query, then orin_flash_attention_prefill): bit for bit, on the C3 and C2 shapes (the
latter through the key split), with and without norm weights, with a prefix in the cache and
at head size 64; plus the oracle (RMSNorm, rotation, causal attention) on sampled rows."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import _lib
from orinmllm_amd import kernel as K
from tests.test_gpu_producers import rope_with_tables
from tests.util import assert_lowp_close, normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def run_case(kind, S, Hq, Hkv, d, start, weights, rng, layers=2, layer=1):
    kv_dim, max_seq = Hkv * d, start + S + 16
    q, k, v = normal(rng, (S, Hq * d)), normal(rng, (S, kv_dim)), normal(rng, (S, kv_dim))
    wq = dev(1.0 + 0.1 * normal(rng, (d,)), kind) if weights else None
    wk = dev(1.0 + 0.1 * normal(rng, (d,)), kind) if weights else None
    s_t = torch.empty(max_seq, d, device="cuda")
    c_t = torch.empty(max_seq, d, device="cuda")
    K.sin_cos_cache_calc_cu(d, max_seq, s_t, c_t, 1e6)
    prefix_k = dev(normal(rng, (start, kv_dim)), kind)
    prefix_v = dev(normal(rng, (start, kv_dim)), kind)

    def cache():
        kc = torch.zeros(layers, max_seq, kv_dim, device="cuda", dtype=TORCH[kind])
        vc = torch.zeros_like(kc)
        kc[layer, :start] = prefix_k
        vc[layer, :start] = prefix_v
        return kc, vc

    qd, kd, vd = dev(q, kind), dev(k, kind), dev(v, kind)
    # two passes
    kc1, vc1 = cache()
    q1 = qd.clone()
    K.qk_norm_rope_cu(q1, kd, vd, wq, wk, s_t, c_t, kc1, vc1, layer, max_seq, start, S, Hq, Hkv, d)
    o1 = torch.full_like(qd, float("nan"))
    K.flash_attention_prefill_cu(start, S, Hq, Hkv, d, Hq // Hkv, layer, max_seq, kv_dim, q1, o1,
                                 kc1, vc1)
    # fused
    kc2, vc2 = cache()
    q2 = qd.clone()
    K.qk_norm_rope_cu(None, kd, vd, None, wk, s_t, c_t, kc2, vc2, layer, max_seq, start, S, Hq, Hkv,
                      d)
    o2 = torch.full_like(qd, float("nan"))
    K.flash_attention_prefill_qk_norm_rope_cu(start, S, Hq, Hkv, d, Hq // Hkv, layer, max_seq,
                                              kv_dim, q2, o2, kc2, vc2, wq, s_t, c_t)
    torch.cuda.synchronize()
    assert torch.equal(q2, qd), "the fused prefill must not modify the raw query"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "K/V-only producer differs"
    assert torch.equal(o1, o2), f"fused prefill differs from the two-pass path ({kind} S {S})"
    return dict(q=q, wq=wq, s_t=s_t, c_t=c_t, q1=q1, kc=kc2, vc=vc2, o=o2, max_seq=max_seq)


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_fused_c3_equals_two_pass_and_oracle(kind):
    rng = np.random.default_rng(61)
    S, Hq, Hkv, d = 4096, 32, 8, 128
    r = run_case(kind, S, Hq, Hkv, d, 0, True, rng)
    # oracle: RMSNorm with the weights, rotation with the device tables, causal attention
    wq = r["wq"].float().cpu().numpy()
    qn = oracle.rmsnorm_rows(quantize(r["q"], kind), d, 1e-6, wq)
    sin_h = r["s_t"].cpu().numpy().astype(np.float64)
    cos_h = r["c_t"].cpu().numpy().astype(np.float64)
    q_ref = quantize(rope_with_tables(qn, sin_h, cos_h, np.arange(S), Hq, d), kind)
    assert_lowp_close(r["q1"].float().cpu().numpy(), q_ref, what="two-pass q")
    rows = np.unique(np.concatenate([[0, 1, 255, 256, S - 1], rng.integers(0, S, 27)]))
    kc = r["kc"][1].float().cpu().numpy()
    vc = r["vc"][1].float().cpu().numpy()
    ref = oracle.prefill_causal(0, r["q1"].float().cpu().numpy(), kc, vc, Hq, Hkv, d, rows=rows,
                                nthreads=8)
    assert_lowp_close(r["o"].float().cpu().numpy()[rows], ref, what=f"fused C3 {kind}")


@pytest.mark.parametrize("kind,S,Hq,Hkv,d,start,weights", [
    ("fp16", 2048, 12, 2, 128, 0, True),    # C2 shape: key split + merge
    ("bf16", 700, 8, 2, 128, 300, False),   # prefix in the cache, rope only
    ("fp16", 1000, 16, 4, 64, 37, True),    # head size 64
])
def test_fused_equals_two_pass(kind, S, Hq, Hkv, d, start, weights):
    run_case(kind, S, Hq, Hkv, d, start, weights, np.random.default_rng(S + d + start))


def test_fused_argument_errors():
    lib = _lib.load()
    q = torch.zeros(64, 4 * 96, device="cuda", dtype=torch.float16)
    kc = torch.zeros(1, 64, 96, device="cuda", dtype=torch.float16)
    t = torch.zeros(64, 96, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    # head size 96 has no fused Q load
    st = lib.orin_flash_attention_prefill_qk_norm_rope(0, 64, 4, 1, 96, 4, 0, 64, 96, q.data_ptr(),
                                                       q.data_ptr() + 2, kc.data_ptr(),
                                                       kc.data_ptr(), None, t.data_ptr(),
                                                       t.data_ptr(), 1e-6, _lib.DTYPE_FP16, s)
    assert st == _lib.ERR_UNSUPPORTED
    q = torch.zeros(64, 4 * 128, device="cuda", dtype=torch.float16)
    kc = torch.zeros(1, 64, 128, device="cuda", dtype=torch.float16)
    t = torch.zeros(64, 128, device="cuda")
    # output aliasing the raw query, and missing tables
    st = lib.orin_flash_attention_prefill_qk_norm_rope(0, 64, 4, 1, 128, 4, 0, 64, 128,
                                                       q.data_ptr(), q.data_ptr(), kc.data_ptr(),
                                                       kc.data_ptr(), None, t.data_ptr(),
                                                       t.data_ptr(), 1e-6, _lib.DTYPE_FP16, s)
    assert st == _lib.ERR_INVALID_ARG
    o = torch.zeros_like(q)
    st = lib.orin_flash_attention_prefill_qk_norm_rope(0, 64, 4, 1, 128, 4, 0, 64, 128,
                                                       q.data_ptr(), o.data_ptr(), kc.data_ptr(),
                                                       kc.data_ptr(), None, None, t.data_ptr(),
                                                       1e-6, _lib.DTYPE_FP16, s)
    assert st == _lib.ERR_INVALID_ARG
