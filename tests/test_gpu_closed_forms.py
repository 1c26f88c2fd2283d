"""Closed forms and invariants of attention checked on the GPU kernels directly (no
oracle): they pin what the mathematics fixes, for both prefill kernels (the 256-query
ping-pong kernel at S = 2048 x 32 heads, the tile kernel at small S), the decode and
the vision path.
  * Q = 0: every weight is equal, so each output row is the mean of its visible V rows.
  * V constant per kv head: every output row equals that constant.
  * one key scored far above the rest: the output is that key's V row.
  * GQA equals MHA on K/V heads repeated kv_mul times, bit for bit.
  * bidirectional attention is invariant under a joint permutation of keys and values."""
import numpy as np
import pytest
import torch

from orinmllm_amd import kernel as K
from tests.util import normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def prefill(kind, q, kc, vc, Hq, Hkv, d, start_pos=0):
    S = q.shape[0]
    max_seq = kc.shape[0]
    o = torch.zeros(S, Hq * d, device="cuda", dtype=TORCH[kind])
    K.flash_attention_prefill_cu(start_pos, S, Hq, Hkv, d, Hq // Hkv, 0, max_seq, Hkv * d,
                                 dev(q, kind), o, dev(kc, kind), dev(vc, kind))
    torch.cuda.synchronize()
    return o.float().cpu().numpy().reshape(S, Hq, d)


def causal_means(v, S, Hq, Hkv, d, start_pos=0):
    """Row i, head h: mean of V rows 0..start_pos+i of kv head h // kv_mul (float64)."""
    vv = v.reshape(-1, Hkv, d).astype(np.float64)
    cs = np.cumsum(vv, axis=0)
    n = np.arange(start_pos + 1, start_pos + S + 1, dtype=np.float64)[:, None, None]
    m = cs[start_pos:start_pos + S] / n
    return np.repeat(m, Hq // Hkv, axis=1)


# S = 2048 x 32 heads fills 256 workgroups of 256 queries (ping-pong kernel); S = 300 x 4
# heads runs on the tile kernel.
SHAPES = [(2048, 32, 8), (300, 4, 2)]


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("S,Hq,Hkv", SHAPES)
def test_prefill_zero_query_gives_running_mean(kind, S, Hq, Hkv):
    rng = np.random.default_rng(S + Hq)
    d = 128
    q = np.zeros((S, Hq * d), np.float32)
    k = normal(rng, (S, Hkv * d))
    v = quantize(normal(rng, (S, Hkv * d)), kind)
    got = prefill(kind, q, k, v, Hq, Hkv, d)
    want = causal_means(v, S, Hq, Hkv, d)
    tol = 4e-3 if kind == "fp16" else 2e-2  # the output is rounded to 16 bits
    assert np.abs(got - want).max() <= tol


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("S,Hq,Hkv", SHAPES)
def test_prefill_constant_values_and_dominant_key(kind, S, Hq, Hkv):
    rng = np.random.default_rng(7 * S + Hq)
    d = 128
    # Constant V per kv head: output = the constant.
    q = normal(rng, (S, Hq * d))
    k = normal(rng, (S, Hkv * d))
    const = quantize(rng.uniform(-2, 2, (Hkv, d)).astype(np.float32), kind)
    v = np.tile(const.reshape(1, -1), (S, 1))
    got = prefill(kind, q, k, v, Hq, Hkv, d)
    want = np.repeat(const[None], Hq // Hkv, axis=1).reshape(1, Hq, d)
    tol = 2e-3 if kind == "fp16" else 1e-2
    assert np.abs(got - want).max() <= tol * 2
    # Dominant key: key 0 of every kv head aligned with every query and scaled so its
    # score exceeds all others by > 30 (weights of the rest < e^-30): O = V[0].
    qd = np.zeros((S, Hq * d), np.float32)
    qd[:, ::d] = 4.0  # q . k_j = 4 * k_j[0] for each head
    kd = quantize(normal(rng, (S, Hkv * d)) * 0.1, kind)
    kd[0, ::d] = 100.0  # key 0: score 400 / sqrt(128) ~ 35 above the rest
    v2 = quantize(normal(rng, (S, Hkv * d)), kind)
    got = prefill(kind, qd, kd, v2, Hq, Hkv, d)
    want = np.repeat(v2[0].reshape(1, Hkv, d), Hq // Hkv, axis=1)
    assert np.abs(got - want).max() <= tol * 2


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_prefill_gqa_equals_mha_with_repeated_kv(kind):
    rng = np.random.default_rng(3)
    S, Hq, Hkv, d = 2048, 32, 8, 128
    q = normal(rng, (S, Hq * d))
    k = normal(rng, (S, Hkv * d))
    v = normal(rng, (S, Hkv * d))
    gqa = prefill(kind, q, k, v, Hq, Hkv, d)
    rep = lambda x: np.repeat(x.reshape(S, Hkv, d), Hq // Hkv, axis=1).reshape(S, Hq * d)
    mha = prefill(kind, q, rep(k), rep(v), Hq, Hq, d)
    assert np.array_equal(gqa, mha)


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_decode_zero_query_gives_mean(kind):
    rng = np.random.default_rng(5)
    Hq, Hkv, d, max_seq, pos = 32, 8, 128, 4096, 3000
    kv_dim = Hkv * d
    kc = normal(rng, (1, max_seq, kv_dim))
    vc = quantize(normal(rng, (1, max_seq, kv_dim)), kind)
    out = torch.zeros(Hq * d, device="cuda", dtype=TORCH[kind])
    K.flash_attention_decode_cu(pos, Hq, Hkv, d, Hq // Hkv, 0, max_seq, kv_dim,
                                torch.zeros(Hq * d, device="cuda", dtype=TORCH[kind]), out,
                                dev(kc, kind), dev(vc, kind))
    torch.cuda.synchronize()
    want = np.repeat(vc[0, : pos + 1].reshape(pos + 1, Hkv, d).astype(np.float64).mean(0),
                     Hq // Hkv, axis=0)
    tol = 2e-3 if kind == "fp16" else 1e-2
    assert np.abs(out.float().cpu().numpy().reshape(Hq, d) - want).max() <= tol


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_vision_joint_permutation_invariance(kind):
    rng = np.random.default_rng(9)
    H, N, d = 16, 1024, 72
    q, k, v = (quantize(normal(rng, (H, N, d)), kind) for _ in range(3))
    perm = rng.permutation(N)

    def run(kk, vv):
        o = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
        K.vision_attention_pretransposed_cu(dev(q, kind), dev(kk, kind), dev(vv, kind), o, None,
                                            None, N, H, d, float(d) ** -0.5)
        torch.cuda.synchronize()
        return o.float().cpu().numpy()

    a = run(k, v)
    b = run(k[:, perm], v[:, perm])
    tol = 2e-3 if kind == "fp16" else 1e-2
    assert np.abs(a - b).max() <= tol
