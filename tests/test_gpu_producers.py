"""GPU parity of the kernels either side of the attention path: KV-cache writes
(kuiper append, paged scatter, contiguous <-> paged), the RoPE sin/cos cache, the fused
Qwen3 Q/K RMSNorm + RoPE producer and the vision QKV split + rotary + transpose.

Byte moves are checked bit-exactly against numpy; the floating-point producers against
the oracle's RMSNorm / rotary restatements within the 16-bit bar."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.util import assert_lowp_close, normal, quantize

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}
KINDS = ["fp32", "fp16", "bf16"]


def dev(x, kind):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def host(t):
    return t.float().cpu().numpy()


# ---------------------------------------------------------------- KV-cache writes

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("kv_dim", [1024, 260])
def test_copy_to_kv_cache(kind, kv_dim):
    """kv_cache[layer][*pos] = src; every other row untouched; the position is read on
    the device (a second launch with a new value in the same tensor)."""
    rng = np.random.default_rng(kv_dim)
    layers, seq = 3, 40
    cache0 = normal(rng, (layers, seq, kv_dim))
    cache = dev(cache0, kind)
    pos = torch.tensor([7], dtype=torch.int32, device="cuda")
    expect = quantize(cache0, kind)
    for p, layer in [(7, 1), (39, 2)]:
        src = normal(rng, (kv_dim,))
        pos.fill_(p)
        K.copy_to_kv_cache_kernel(cache, dev(src, kind), pos, kv_dim, layer, seq)
        expect[layer, p] = quantize(src, kind)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(cache), expect)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("layout", [K.KV_LAYOUT_TOKEN_MAJOR, K.KV_LAYOUT_HEAD_MAJOR])
def test_kv_cache_write_paged(kind, layout):
    rng = np.random.default_rng(3 + layout)
    n, hkv, d, bs, nblk = 300, 8, 128, 16, 40
    ks, vs = normal(rng, (n, hkv, d)), normal(rng, (n, hkv, d))
    slots = rng.permutation(nblk * bs)[:n].astype(np.int32)
    slots[rng.integers(0, n, 20)] = -1  # skipped rows
    shape = (nblk, bs, hkv, d) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (nblk, hkv, bs, d)
    kp0, vp0 = normal(rng, shape), normal(rng, shape)
    kp, vp = dev(kp0, kind), dev(vp0, kind)
    K.kv_cache_write_paged(dev(ks, kind), dev(vs, kind), kp, vp,
                           torch.from_numpy(slots).cuda(), layout=layout)
    torch.cuda.synchronize()
    ek, ev = quantize(kp0, kind), quantize(vp0, kind)
    for r in range(n):
        if slots[r] < 0:
            continue
        b, o = divmod(int(slots[r]), bs)
        if layout == K.KV_LAYOUT_TOKEN_MAJOR:
            ek[b, o], ev[b, o] = quantize(ks[r], kind), quantize(vs[r], kind)
        else:
            ek[b, :, o], ev[b, :, o] = quantize(ks[r], kind), quantize(vs[r], kind)
    np.testing.assert_array_equal(host(kp), ek)
    np.testing.assert_array_equal(host(vp), ev)


@pytest.mark.parametrize("layout", [K.KV_LAYOUT_TOKEN_MAJOR, K.KV_LAYOUT_HEAD_MAJOR])
def test_kv_cache_convert_round_trip_and_decode(layout):
    """contiguous -> paged -> contiguous is the identity on the sequence's tokens, and a
    paged decode over the converted pool equals the contiguous decode bit for bit."""
    rng = np.random.default_rng(11 + layout)
    L, hkv, hq, d, bs = 1000, 8, 32, 128, 16
    nblk = (L + bs - 1) // bs + 5
    kc, vc = normal(rng, (L, hkv, d)), normal(rng, (L, hkv, d))
    kcd, vcd = dev(kc, "fp16"), dev(vc, "fp16")
    shape = (nblk, bs, hkv, d) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (nblk, hkv, bs, d)
    kp = torch.zeros(shape, dtype=torch.float16, device="cuda")
    vp = torch.zeros_like(kp)
    bt = torch.from_numpy(rng.permutation(nblk)[: (L + bs - 1) // bs].astype(np.int32)).cuda()
    K.kv_cache_convert(kcd, kp, bt, L, K.KV_TO_PAGED, layout=layout)
    K.kv_cache_convert(vcd, vp, bt, L, K.KV_TO_PAGED, layout=layout)
    back = torch.zeros_like(kcd)
    K.kv_cache_convert(back, kp, bt, L, K.KV_TO_CONTIGUOUS, layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(back, kcd)

    q = dev(normal(rng, (1, hq, d)), "fp16")
    lens = torch.tensor([L], dtype=torch.int32, device="cuda")
    o_paged = torch.empty_like(q)
    o_contig = torch.empty_like(q)
    K.paged_decode_cu(q, kp, vp, o_paged, bt[None], lens, L, layout=layout)
    K.batched_decode_cu(q, kcd[None], vcd[None], o_contig, lens, L, hkv)
    torch.cuda.synchronize()
    assert torch.equal(o_paged, o_contig)


# ---------------------------------------------------------------- RoPE cache

def test_rope_sin_cos_cache():
    """entry [p][i] = sin/cos(p * theta^(-i/d)) in fp32; the error allowed grows with the
    angle (the fp32 angle itself carries |angle| * 2^-24 of rounding)."""
    d, S, theta = 128, 4096, 1e6
    s = torch.empty(S, d, device="cuda")
    c = torch.empty(S, d, device="cuda")
    K.sin_cos_cache_calc_cu(d, S, s, c, theta)
    torch.cuda.synchronize()
    freq = 1.0 / theta ** (np.arange(d) / d)
    ang = np.arange(S)[:, None] * freq[None]
    tol = 2e-6 + 4e-7 * ang
    assert (np.abs(s.cpu().numpy() - np.sin(ang)) <= tol).all()
    assert (np.abs(c.cpu().numpy() - np.cos(ang)) <= tol).all()
    # position 0 is the identity rotation; entry 0 is the angle p itself
    assert (s.cpu().numpy()[0] == 0).all() and (c.cpu().numpy()[0] == 1).all()


# ---------------------------------------------------------------- Q/K producer

def rope_with_tables(x, sin_t, cos_t, positions, H, d):
    """Rotate pairs (j, j+d/2) of x [S, H*d] with table entries [p][2j] (float64)."""
    y = np.asarray(x, np.float64).reshape(len(positions), H, d).copy()
    j = np.arange(d // 2)
    s = sin_t[positions][:, None, 2 * j]
    c = cos_t[positions][:, None, 2 * j]
    a, b = y[..., : d // 2].copy(), y[..., d // 2:].copy()
    y[..., : d // 2] = c * a - s * b
    y[..., d // 2:] = c * b + s * a
    return y.reshape(len(positions), H * d)


def producer_case(kind, start, S, Hq, Hkv, d, max_seq, layer, rng, unit_weights=False,
                  pos_dev=False):
    q, k, v = normal(rng, (S, Hq * d)), normal(rng, (S, Hkv * d)), normal(rng, (S, Hkv * d))
    wq = np.ones(d, np.float32) if unit_weights else 1.0 + 0.1 * normal(rng, (d,))
    wk = np.ones(d, np.float32) if unit_weights else 1.0 + 0.1 * normal(rng, (d,))
    s_t = torch.empty(max_seq, d, device="cuda")
    c_t = torch.empty(max_seq, d, device="cuda")
    K.sin_cos_cache_calc_cu(d, max_seq, s_t, c_t, 1e6)
    kcache = torch.zeros(2, max_seq, Hkv * d, dtype=TORCH[kind], device="cuda")
    vcache = torch.zeros_like(kcache)
    qd = dev(q, kind)
    pos = torch.tensor([start], dtype=torch.int32, device="cuda") if pos_dev else None
    K.qk_norm_rope_cu(qd, dev(k, kind), dev(v, kind),
                      None if wq is None else dev(wq, kind), None if wk is None else dev(wk, kind),
                      s_t, c_t, kcache, vcache, layer, max_seq, 0 if pos_dev else start, S, Hq,
                      Hkv, d, pos_ptr=pos)
    torch.cuda.synchronize()
    # oracle: RMSNorm (oracle.rmsnorm_rows) on the 16-bit inputs, then the rotation with
    # the device sin/cos tables
    qn = oracle.rmsnorm_rows(quantize(q, kind), d, 1e-6,
                             None if wq is None else quantize(wq, kind))
    kn = oracle.rmsnorm_rows(quantize(k, kind), d, 1e-6,
                             None if wk is None else quantize(wk, kind))
    st, ct = s_t.cpu().numpy().astype(np.float64), c_t.cpu().numpy().astype(np.float64)
    positions = np.arange(start, start + S)
    q_ref = rope_with_tables(qn, st, ct, positions, Hq, d)
    k_ref = rope_with_tables(kn, st, ct, positions, Hkv, d)
    return qd, kcache, vcache, q_ref, k_ref, quantize(v, kind)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("start,S,d", [(0, 64, 128), (100, 37, 128), (5, 9, 256)])
def test_qk_norm_rope(kind, start, S, d):
    rng = np.random.default_rng(start * 7 + S + d)
    Hq, Hkv, max_seq, layer = 8, 2, 256, 1
    qd, kc, vc, q_ref, k_ref, v_ref = producer_case(kind, start, S, Hq, Hkv, d, max_seq, layer,
                                                    rng)
    if kind == "fp32":
        np.testing.assert_allclose(host(qd), q_ref, rtol=2e-5, atol=2e-5)
        np.testing.assert_allclose(host(kc)[layer, start:start + S], k_ref, rtol=2e-5, atol=2e-5)
    else:
        assert_lowp_close(host(qd), q_ref, what=f"q {kind}")
        assert_lowp_close(host(kc)[layer, start:start + S], k_ref, what=f"k {kind}")
    np.testing.assert_array_equal(host(vc)[layer, start:start + S], v_ref)
    # rows outside [start, start+S) and the other layer are untouched
    assert not host(kc)[layer, :start].any() and not host(kc)[layer, start + S:].any()
    assert not host(kc)[0].any() and not host(vc)[0].any()


def test_qk_norm_rope_device_position_and_closed_forms():
    """pos_ptr gives the same bits as start_pos.  At position 0 the rotation is the
    identity: with unit weights every head comes out with unit RMS, and without weights
    (no normalisation, the Qwen2 / Llama producer) query and key pass through unchanged."""
    rng = np.random.default_rng(1)
    a = producer_case("fp16", 33, 12, 4, 2, 128, 64, 0, np.random.default_rng(2), pos_dev=False)
    b = producer_case("fp16", 33, 12, 4, 2, 128, 64, 0, np.random.default_rng(2), pos_dev=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    qd, kc, _, _, _, _ = producer_case("fp32", 0, 1, 4, 2, 128, 16, 0, rng, unit_weights=True)
    rms = np.sqrt((host(qd).reshape(4, 128) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-5)
    rms_k = np.sqrt((host(kc)[0, 0].reshape(2, 128) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms_k, 1.0, rtol=1e-5)
    x = np.random.default_rng(9)
    q, k, v = normal(x, (1, 4 * 128)), normal(x, (1, 2 * 128)), normal(x, (1, 2 * 128))
    s_t = torch.empty(8, 128, device="cuda")
    c_t = torch.empty(8, 128, device="cuda")
    K.sin_cos_cache_calc_cu(128, 8, s_t, c_t, 1e6)
    kc = torch.zeros(1, 8, 256, device="cuda")
    vc = torch.zeros_like(kc)
    qd = dev(q, "fp32")
    K.qk_norm_rope_cu(qd, dev(k, "fp32"), dev(v, "fp32"), None, None, s_t, c_t, kc, vc, 0, 8, 0,
                      1, 4, 2, 128)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(qd), q)
    np.testing.assert_array_equal(host(kc)[0, 0], k[0])


def test_producer_then_prefill_matches_oracle():
    """The producer feeding the prefill kernel: Qwen3-8B head shape, 300 tokens after a
    200-token prefix already in the cache."""
    rng = np.random.default_rng(42)
    start, S, Hq, Hkv, d, max_seq = 200, 300, 32, 8, 128, 512
    qd, kc, vc, q_ref, k_ref, v_ref = producer_case("fp16", start, S, Hq, Hkv, d, max_seq, 1, rng)
    prefix_k = quantize(normal(rng, (start, Hkv * d)), "fp16")
    prefix_v = quantize(normal(rng, (start, Hkv * d)), "fp16")
    kc[1, :start] = torch.from_numpy(prefix_k).cuda().half()
    vc[1, :start] = torch.from_numpy(prefix_v).cuda().half()
    out = torch.empty_like(qd)
    K.flash_attention_prefill_fp16_cu(start, S, Hq, Hkv, d, Hq // Hkv, 1, max_seq, Hkv * d, qd,
                                      out, kc, vc)
    torch.cuda.synchronize()
    kfull = np.zeros((max_seq, Hkv * d), np.float32)
    vfull = np.zeros((max_seq, Hkv * d), np.float32)
    kfull[:start], vfull[:start] = prefix_k, prefix_v
    kfull[start:start + S] = quantize(k_ref, "fp16")
    vfull[start:start + S] = v_ref
    ref = oracle.prefill_causal(start, quantize(q_ref, "fp16"), kfull, vfull, Hq, Hkv, d,
                                nthreads=8)
    assert_lowp_close(host(out), ref, what="producer + prefill")


# ---------------------------------------------------------------- vision producer

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("d,gh,gw", [(72, 32, 32), (72, 26, 22), (80, 26, 22), (76, 26, 22)])
def test_vision_split_rope_transpose(kind, d, gh, gw):
    """qkv [N, 3*H*d] -> q/k/v [H, N, d] with the 2-D rotary of a gh x gw grid on q and k.
    d/2 % 4 == 0 takes the 8-token vectorised kernel (572 tokens leaves a ragged last
    workgroup); d = 76 takes the per-pair kernel."""
    rng = np.random.default_rng(5 + d + gh)
    H = 16
    N = gh * gw
    qkv = normal(rng, (N, 3 * H * d))
    c, s = oracle.vision_cos_sin(1, gh, gw, 2, d)
    out = [torch.empty(H, N, d, dtype=TORCH[kind], device="cuda") for _ in range(3)]
    K.fused_split_rope_transpose_cu(dev(qkv, kind), dev(c, kind), dev(s, kind), *out, N, H, d)
    torch.cuda.synchronize()
    x = quantize(qkv, kind).reshape(N, 3, H, d).transpose(1, 2, 0, 3)  # [3, H, N, d]
    cq, sq = quantize(c, kind), quantize(s, kind)
    q_ref = oracle.vision_rotary(x[0], cq, sq)
    k_ref = oracle.vision_rotary(x[1], cq, sq)
    if kind == "fp32":
        np.testing.assert_allclose(host(out[0]), q_ref, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(host(out[1]), k_ref, rtol=1e-5, atol=1e-5)
    else:
        assert_lowp_close(host(out[0]), q_ref, what=f"vision q {kind}")
        assert_lowp_close(host(out[1]), k_ref, what=f"vision k {kind}")
    np.testing.assert_array_equal(host(out[2]), x[2])
