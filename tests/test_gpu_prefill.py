"""GPU parity of causal prefill (MFMA fp16/bf16 path and fp32 path) against the oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.util import assert_fp32_close, assert_lowp_close, normal, quantize, qwen3_qk

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def sample_rows(S, n, rng):
    """First, last and a spread of query rows (the causal edges and the middle)."""
    rows = {0, 1, S - 1, S - 2} | set(rng.integers(0, S, n).tolist())
    return np.array(sorted(r for r in rows if 0 <= r < S))


def run_prefill(kind, start_pos, S, Hq, Hkv, d, max_seq, layers, layer, rng, qk_producer=False,
                alias=False):
    kv_dim = Hkv * d
    if qk_producer:
        q = qwen3_qk(rng, S, Hq, d, start_pos)
        k_all = qwen3_qk(rng, start_pos + S, Hkv, d, 0)
    else:
        q = normal(rng, (S, Hq * d))
        k_all = normal(rng, (start_pos + S, kv_dim))
    q = quantize(q, kind)
    kc = np.zeros((layers, max_seq, kv_dim), np.float32)
    vc = np.zeros((layers, max_seq, kv_dim), np.float32)
    kc[layer, : start_pos + S] = quantize(k_all, kind)
    vc[layer, : start_pos + S] = quantize(normal(rng, (start_pos + S, kv_dim)), kind)
    qd = dev(q, kind)
    out = qd if alias else torch.zeros_like(qd)
    K.flash_attention_prefill_cu(start_pos, S, Hq, Hkv, d, Hq // Hkv, layer, max_seq, kv_dim, qd,
                                 out, dev(kc, kind), dev(vc, kind))
    torch.cuda.synchronize()
    return q, kc[layer], vc[layer], out.float().cpu().numpy()


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_c2_qwen25_prefill(kind):
    """S 2048, 12 q / 2 kv heads, d 128."""
    rng = np.random.default_rng(0xC2)
    S, Hq, Hkv, d = 2048, 12, 2, 128
    q, kc, vc, out = run_prefill(kind, 0, S, Hq, Hkv, d, S, 1, 0, rng, qk_producer=True)
    rows = sample_rows(S, 96, rng)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"C2 {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_c3_qwen3_prefill(kind):
    """S 4096, 32 q / 8 kv heads, d 128, Q/K after RMSNorm + RoPE."""
    rng = np.random.default_rng(0xC3)
    S, Hq, Hkv, d = 4096, 32, 8, 128
    q, kc, vc, out = run_prefill(kind, 0, S, Hq, Hkv, d, S, 1, 0, rng, qk_producer=True)
    rows = sample_rows(S, 48, rng)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"C3 {kind}")
    assert np.isfinite(out).all()


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("start_pos,S", [(0, 1), (0, 77), (200, 300), (1000, 129), (5, 64)])
def test_prefill_ragged_and_prefix(kind, start_pos, S):
    """Ragged lengths (not multiples of the 128-row / 64-key tiles) and start_pos > 0
    (prefix-cache reuse: row i attends 0..start_pos+i), in layer 1 of a 2-layer cache."""
    rng = np.random.default_rng(start_pos * 1000 + S)
    Hq, Hkv, d, max_seq = 8, 2, 128, 2048
    q, kc, vc, out = run_prefill(kind, start_pos, S, Hq, Hkv, d, max_seq, 2, 1, rng)
    ref = oracle.prefill_causal(start_pos, q, kc, vc, Hq, Hkv, d, nthreads=8)
    assert_lowp_close(out, ref, what=f"{kind} start {start_pos} S {S}")


@pytest.mark.parametrize("d", [64, 128])
def test_prefill_output_aliases_query(d):
    """output == query is allowed (the Qwen3-VL caller does this)."""
    rng = np.random.default_rng(d)
    S, Hq, Hkv = 333, 16, 4
    q, kc, vc, out = run_prefill("fp16", 0, S, Hq, Hkv, d, 512, 1, 0, rng, alias=True)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, nthreads=8)
    assert_lowp_close(out, ref, what="aliased")


def test_prefill_row_equals_decode():
    """Causal prefill row i agrees with a decode at pos = start_pos + i on the same cache."""
    rng = np.random.default_rng(21)
    S, Hq, Hkv, d, start = 300, 32, 8, 128, 50
    q, kc, vc, out = run_prefill("fp16", start, S, Hq, Hkv, d, 512, 1, 0, rng)
    kd, vd = dev(kc[None], "fp16"), dev(vc[None], "fp16")
    for i in [0, 77, 299]:
        o = torch.zeros(Hq * d, device="cuda", dtype=torch.float16)
        K.flash_attention_decode_cu(start + i, Hq, Hkv, d, Hq // Hkv, 0, 512, Hkv * d,
                                    dev(q[i], "fp16"), o, kd, vd)
        torch.cuda.synchronize()
        assert_lowp_close(out[i], o.float().cpu().numpy(), what=f"row {i}")


@pytest.mark.parametrize("api", ["flash", "batched"])
def test_fp32_prefill(api):
    rng = np.random.default_rng(31)
    start, S, Hq, Hkv, d, max_seq = 10, 200, 16, 4, 128, 256
    kv_dim = Hkv * d
    q = normal(rng, (S, Hq * d))
    kc = normal(rng, (2, max_seq, kv_dim))
    vc = normal(rng, (2, max_seq, kv_dim))
    out = torch.zeros(S, Hq * d, device="cuda")
    args_q, args_k, args_v = dev(q, "fp32"), dev(kc, "fp32"), dev(vc, "fp32")
    if api == "flash":
        K.flash_attention_prefill_cu(start, S, Hq, Hkv, d, Hq // Hkv, 1, max_seq, kv_dim, args_q,
                                     out, args_k, args_v)
    else:
        K.batched_mha_kernel_cu(start, S, Hq, 1, max_seq, Hq * d, kv_dim, Hq // Hkv, d, out,
                                args_q, None, args_k, args_v)
    torch.cuda.synchronize()
    ref = oracle.prefill_causal(start, q, kc[1], vc[1], Hq, Hkv, d, nthreads=8)
    assert_fp32_close(out.cpu().numpy(), ref, d, what=f"fp32 prefill {api}")
