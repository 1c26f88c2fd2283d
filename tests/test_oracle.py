"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU checker.

The reference holds no attention fixtures or known-answer tests (its softmax test is
commented out, test/test_op/test_cu_softmax.cpp), so the oracle is pinned by:
  * golden outputs of PyTorch's CPU scaled_dot_product_attention in float64
    (tests/golden/, written by tests/golden/make_golden.py);
  * an extended-precision brute force on tiny inputs;
  * closed forms and invariants that a dropped term, a wrong index or a transposed
    operand would break.
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLD, name + ".npz")))


def rel_norm(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b).max() / np.abs(b).max()


# ---------------------------------------------------------------- golden fixtures

def test_golden_c1_decode():
    g = load("c1_decode")
    rng = np.random.default_rng(int(g["seed"]))
    Hq, d, pos, S = int(g["Hq"]), int(g["d"]), int(g["pos"]), int(g["seq_len"])
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((S, Hq * d)).astype(np.float32)
    v = rng.standard_normal((S, Hq * d)).astype(np.float32)
    assert np.isclose(q.sum() + k.sum() + v.sum(), g["checksum"])
    out, score = oracle.mha_kernel(pos, Hq, 0, S, Hq * d, 1, d, q, k[None], v[None])
    assert rel_norm(out, g["out"]) < 2e-6
    # the score scratch holds each head's softmax probabilities (cpu/mha_kernel.cpp:44)
    assert np.allclose(score[:, : pos + 1].sum(axis=1), 1.0, atol=1e-5)


def test_golden_gqa_decode_and_layer_offset():
    g = load("gqa_decode")
    rng = np.random.default_rng(int(g["seed"]))
    Hq, Hkv, d, pos, S = (int(g[x]) for x in ("Hq", "Hkv", "d", "pos", "seq_len"))
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((S, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((S, Hkv * d)).astype(np.float32)
    assert np.isclose(q.sum() + k.sum() + v.sum(), g["checksum"])
    # put the data in layer 2 of a 3-layer cache: the layer offset must select it
    kc = np.zeros((3, S, Hkv * d), np.float32)
    vc = np.zeros((3, S, Hkv * d), np.float32)
    kc[2], vc[2] = k, v
    kc[:2], vc[:2] = 100.0, -100.0
    out, _ = oracle.mha_kernel(pos, Hq, 2, S, Hkv * d, Hq // Hkv, d, q, kc, vc)
    assert rel_norm(out, g["out"]) < 2e-6


def test_golden_causal_prefill():
    g = load("causal_prefill")
    rng = np.random.default_rng(int(g["seed"]))
    Hq, Hkv, d, sp, S = (int(g[x]) for x in ("Hq", "Hkv", "d", "start_pos", "S"))
    q = rng.standard_normal((S, Hq * d)).astype(np.float32)
    k = rng.standard_normal((sp + S, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((sp + S, Hkv * d)).astype(np.float32)
    assert np.isclose(q.sum() + k.sum() + v.sum(), g["checksum"])
    out = oracle.prefill_causal(sp, q, k, v, Hq, Hkv, d)
    assert rel_norm(out, g["out"]) < 2e-6
    rows = np.array([0, 17, S - 1])
    sub = oracle.prefill_causal(sp, q, k, v, Hq, Hkv, d, rows=rows)
    assert np.array_equal(sub, out[rows])


def test_golden_varlen_bidir():
    g = load("varlen_bidir")
    rng = np.random.default_rng(int(g["seed"]))
    H, d, cu = int(g["H"]), int(g["d"]), g["cu"].astype(np.int32)
    N = int(cu[-1])
    q = rng.standard_normal((H, N, d)).astype(np.float32)
    k = rng.standard_normal((H, N, d)).astype(np.float32)
    v = rng.standard_normal((H, N, d)).astype(np.float32)
    assert np.isclose(q.sum() + k.sum() + v.sum(), g["checksum"])
    out = oracle.varlen_bidir(q, k, v, cu)
    assert rel_norm(out, g["out"]) < 2e-6
    rows = np.array([0, 6, 7, 31])
    assert np.array_equal(oracle.varlen_bidir(q, k, v, cu, rows=rows), out[rows])


# ---------------------------------------------------------------- brute force

def brute_decode(q, k, v, Hq, Hkv, d, L):
    """Extended-precision (long double) attention for one query row over L keys."""
    ld = np.longdouble
    out = np.zeros(Hq * d, ld)
    for h in range(Hq):
        g = h // (Hq // Hkv)
        qs = q[h * d:(h + 1) * d].astype(ld)
        s = np.array([np.dot(qs, k[t, g * d:(g + 1) * d].astype(ld)) for t in range(L)])
        s = s / np.sqrt(ld(d))
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * d:(h + 1) * d] = (p[:, None] * v[:L, g * d:(g + 1) * d].astype(ld)).sum(0)
    return out


@pytest.mark.parametrize("Hq,Hkv,d,L", [(1, 1, 4, 1), (2, 1, 8, 5), (4, 2, 8, 16), (3, 3, 2, 9)])
def test_brute_force_tiny(Hq, Hkv, d, L):
    rng = np.random.default_rng(Hq * 100 + d * 10 + L)
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((L, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((L, Hkv * d)).astype(np.float32)
    out, _ = oracle.mha_kernel(L - 1, Hq, 0, L, Hkv * d, Hq // Hkv, d, q, k[None], v[None])
    assert rel_norm(out, brute_decode(q, k, v, Hq, Hkv, d, L).astype(np.float64)) < 1e-6


# ---------------------------------------------------------------- closed forms

def test_single_key_returns_v0_exactly():
    rng = np.random.default_rng(1)
    q = rng.standard_normal(4 * 16).astype(np.float32)
    k = rng.standard_normal((8, 2 * 16)).astype(np.float32)
    v = rng.standard_normal((8, 2 * 16)).astype(np.float32)
    out, _ = oracle.mha_kernel(0, 4, 0, 8, 32, 2, 16, q, k[None], v[None])
    assert np.array_equal(out.reshape(4, 16), np.repeat(v[0].reshape(2, 16), 2, axis=0))


def test_equal_keys_or_zero_query_give_mean_of_values():
    rng = np.random.default_rng(2)
    L, d = 50, 8
    v = rng.standard_normal((L, d)).astype(np.float32)
    k_eq = np.tile(rng.standard_normal(d).astype(np.float32), (L, 1))
    q = rng.standard_normal(d).astype(np.float32)
    out, _ = oracle.mha_kernel(L - 1, 1, 0, L, d, 1, d, q, k_eq[None], v[None])
    assert np.allclose(out, v.mean(0), atol=1e-6)
    k = rng.standard_normal((L, d)).astype(np.float32)
    out0, _ = oracle.mha_kernel(L - 1, 1, 0, L, d, 1, d, np.zeros(d, np.float32), k[None],
                                v[None])
    assert np.allclose(out0, v.mean(0), atol=1e-6)


def test_dominant_key_and_constant_values():
    rng = np.random.default_rng(3)
    L, d = 20, 8
    k = rng.standard_normal((L, d)).astype(np.float32) * 0.1
    q = np.ones(d, np.float32) * 10.0
    k[7] = 10.0  # score gap >> 30 after scaling
    v = rng.standard_normal((L, d)).astype(np.float32)
    out, _ = oracle.mha_kernel(L - 1, 1, 0, L, d, 1, d, q, k[None], v[None])
    assert np.allclose(out, v[7], atol=1e-6)
    vc = np.full((L, d), 0.375, np.float32)
    out, _ = oracle.mha_kernel(L - 1, 1, 0, L, d, 1, d, rng.standard_normal(d).astype(np.float32),
                               rng.standard_normal((L, d)).astype(np.float32)[None], vc[None])
    assert np.allclose(out, 0.375, atol=1e-6)


# ---------------------------------------------------------------- invariants

def test_gqa_equals_mha_with_repeated_kv():
    rng = np.random.default_rng(4)
    Hq, Hkv, d, S = 8, 2, 16, 30
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((S, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((S, Hkv * d)).astype(np.float32)
    rep = lambda x: np.repeat(x.reshape(S, Hkv, d), Hq // Hkv, axis=1).reshape(S, Hq * d)
    a, _ = oracle.mha_kernel(S - 1, Hq, 0, S, Hkv * d, Hq // Hkv, d, q, k[None], v[None])
    b, _ = oracle.mha_kernel(S - 1, Hq, 0, S, Hq * d, 1, d, q, rep(k)[None], rep(v)[None])
    assert np.array_equal(a, b)


def test_prefill_row_equals_decode_bitwise():
    rng = np.random.default_rng(5)
    Hq, Hkv, d, sp, S = 4, 2, 16, 7, 12
    q = rng.standard_normal((S, Hq * d)).astype(np.float32)
    k = rng.standard_normal((sp + S, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((sp + S, Hkv * d)).astype(np.float32)
    out = oracle.prefill_causal(sp, q, k, v, Hq, Hkv, d)
    for i in [0, 5, S - 1]:
        dec, _ = oracle.mha_kernel(sp + i, Hq, 0, sp + S, Hkv * d, Hq // Hkv, d, q[i], k[None],
                                   v[None])
        assert np.array_equal(out[i], dec)


def test_paged_equals_contiguous_bitwise():
    rng = np.random.default_rng(6)
    B, Hq, Hkv, d, bs = 3, 4, 2, 16, 4
    lens = np.array([1, 9, 16], np.int32)
    S = int(lens.max())
    kc = rng.standard_normal((B, S, Hkv, d)).astype(np.float32)
    vc = rng.standard_normal((B, S, Hkv, d)).astype(np.float32)
    nblk = (lens + bs - 1) // bs
    perm = rng.permutation(int(nblk.sum()))
    kp = np.zeros((len(perm), bs, Hkv, d), np.float32)
    vp = np.zeros_like(kp)
    bt = np.zeros((B, int(nblk.max())), np.int32)
    n = 0
    for b in range(B):
        for j in range(nblk[b]):
            blk = perm[n]
            n += 1
            bt[b, j] = blk
            t1 = min((j + 1) * bs, lens[b])
            kp[blk, : t1 - j * bs] = kc[b, j * bs:t1]
            vp[blk, : t1 - j * bs] = vc[b, j * bs:t1]
    q = rng.standard_normal((B, Hq, d)).astype(np.float32)
    assert np.array_equal(oracle.decode_paged(q, kp, vp, bt, lens),
                          oracle.decode_contig(q, kc, vc, lens))


def test_varlen_equals_separate_segments_and_permutation_invariance():
    rng = np.random.default_rng(7)
    H, d = 2, 8
    cu = np.array([0, 5, 12], np.int32)
    q, k, v = (rng.standard_normal((H, 12, d)).astype(np.float32) for _ in range(3))
    out = oracle.varlen_bidir(q, k, v, cu)
    for a, b in [(0, 5), (5, 12)]:
        one = oracle.varlen_bidir(q[:, a:b], k[:, a:b], v[:, a:b], np.array([0, b - a]))
        assert np.array_equal(one, out[a:b])
    # permuting keys and values together inside a segment leaves the output unchanged
    p = np.concatenate([np.arange(5), 5 + rng.permutation(7)])
    outp = oracle.varlen_bidir(q, k[:, p], v[:, p], cu)
    assert np.allclose(outp, out, atol=1e-6)


def test_threads_do_not_change_results():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((64, 4 * 16)).astype(np.float32)
    k = rng.standard_normal((64, 2 * 16)).astype(np.float32)
    v = rng.standard_normal((64, 2 * 16)).astype(np.float32)
    a = oracle.prefill_causal(0, q, k, v, 4, 2, 16, nthreads=1)
    b = oracle.prefill_causal(0, q, k, v, 4, 2, 16, nthreads=4)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- producers

def test_rope_closed_forms():
    rng = np.random.default_rng(9)
    S, H, d = 6, 2, 8
    x = rng.standard_normal((S, H * d)).astype(np.float32)
    y = oracle.rope_rotate_half(x, S, H, d, start_pos=0)
    assert np.allclose(y[0], x[0])  # position 0 is the identity
    # rotation preserves each (j, j+d/2) pair's norm
    xs, ys = x.reshape(S, H, d), y.reshape(S, H, d)
    nx = xs[..., : d // 2] ** 2 + xs[..., d // 2:] ** 2
    ny = ys[..., : d // 2] ** 2 + ys[..., d // 2:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5)
    # pair 0 turns by exactly `pos` radians (freq_0 = 1); pair j by pos * theta^(-2j/d)
    pos, theta = 3, 1e6
    one = np.zeros((1, d), np.float32)
    one[0, 1] = 1.0  # x_1 = 1, x_{1+d/2} = 0
    r = oracle.rope_rotate_half(one, 1, 1, d, start_pos=pos, theta=theta)[0]
    ang = pos * theta ** (-2.0 / d)
    assert np.allclose([r[1], r[1 + d // 2]], [np.cos(ang), np.sin(ang)], atol=1e-6)


def test_rope_scores_depend_on_relative_position():
    rng = np.random.default_rng(10)
    d = 16
    q = rng.standard_normal((1, d)).astype(np.float32)
    k = rng.standard_normal((1, d)).astype(np.float32)
    s = []
    for m, n in [(5, 2), (13, 10), (103, 100)]:
        qm = oracle.rope_rotate_half(q, 1, 1, d, start_pos=m, theta=1e4)
        kn = oracle.rope_rotate_half(k, 1, 1, d, start_pos=n, theta=1e4)
        s.append(float((qm @ kn.T)[0, 0]))
    assert np.allclose(s, s[0], rtol=1e-4)


def test_rmsnorm_unit_rms():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((7, 32)).astype(np.float32) * 3.0
    y = oracle.rmsnorm_rows(x, 32)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)
    w = np.linspace(0.5, 2.0, 32).astype(np.float32)
    assert np.allclose(oracle.rmsnorm_rows(x, 32, weight=w), y * w, rtol=1e-6)


def test_vision_rotary_tables_and_rotation():
    d = 72
    c, s = oracle.vision_cos_sin(1, 4, 4, 2, d)
    assert c.shape == (16, d)
    assert np.allclose(c[0], 1.0) and np.allclose(s[0], 0.0)  # patch (h=0, w=0)
    # token order walks 2x2 merge blocks: token 1 is (h=0, w=1), token 2 is (h=1, w=0)
    q4 = d // 4
    assert np.allclose(c[1, :q4], 1.0) and not np.allclose(c[1, q4:2 * q4], 1.0)
    assert np.allclose(c[2, q4:2 * q4], 1.0) and not np.allclose(c[2, :q4], 1.0)
    # [h, w, h, w] quarters: the second half repeats the first
    assert np.array_equal(c[:, : d // 2], c[:, d // 2:])
    assert np.isclose(c[1, q4], np.cos(1.0))  # w = 1, frequency 0
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 16, d)).astype(np.float32)
    y = oracle.vision_rotary(x, c, s)
    nx = x[..., : d // 2] ** 2 + x[..., d // 2:] ** 2
    ny = y[..., : d // 2] ** 2 + y[..., d // 2:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(10000) * 10 ** rng.uniform(-5, 5, 10000)).astype(np.float32)
    ours = oracle.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours, ref)


def test_vision_rotary_direction_closed_form():
    """Pin the rotation direction (vision_encoder_kernel.cu:715-718): with x1 = 1, x2 = 0
    the pair becomes (c, s); with x1 = 0, x2 = 1 it becomes (-s, c).  A reversed rotation
    (x1*c + x2*s) keeps the pair norms and would pass a norm check, not this one."""
    d, N = 8, 3
    half = d // 2
    ang = np.array([0.3, np.pi / 2, -1.1], np.float64)
    c = np.repeat(np.cos(ang)[:, None], d, 1).astype(np.float32)
    s = np.repeat(np.sin(ang)[:, None], d, 1).astype(np.float32)
    x = np.zeros((2, N, d), np.float32)
    x[0, :, :half] = 1.0  # unit x1
    x[1, :, half:] = 1.0  # unit x2
    y = oracle.vision_rotary(x, c, s)
    for t in range(N):
        assert np.allclose(y[0, t, :half], np.cos(ang[t]), atol=1e-6)
        assert np.allclose(y[0, t, half:], np.sin(ang[t]), atol=1e-6)
        assert np.allclose(y[1, t, :half], -np.sin(ang[t]), atol=1e-6)
        assert np.allclose(y[1, t, half:], np.cos(ang[t]), atol=1e-6)
    # 90 degrees: (1, 0) -> (0, 1)
    assert np.allclose(y[0, 1, :half], 0.0, atol=1e-6) and np.allclose(y[0, 1, half:], 1.0)
    # the two halves use their own table entries (cos[j] / sin[j] for x1',
    # sin[j + d/2] / cos[j + d/2] for x2'): distinct tables per half are honoured
    c2 = np.ones((1, d), np.float32)
    s2 = np.zeros((1, d), np.float32)
    c2[0, half:] = 0.0
    s2[0, half:] = 1.0  # x2' = x1 * 1 + x2 * 0
    xx = np.arange(d, dtype=np.float32).reshape(1, 1, d) + 1.0
    yy = oracle.vision_rotary(xx, c2, s2)[0, 0]
    assert np.allclose(yy[:half], xx[0, 0, :half]) and np.allclose(yy[half:], xx[0, 0, :half])


def test_vision_cos_sin_all_frequencies():
    """Every entry of the [h, w, h, w] tables against an independent float64 evaluation of
    qwen3_vl.cpp:1741-1812: inv_freq[j] = 10000^(-2j/(d/2)), j < d/4, with (h, w) taken
    from the 2x2 merge-block token order.  A wrong exponent (2j/d) or swapped quarters
    fails here at j > 0."""
    d, gh, gw, merge = 72, 6, 4, 2
    q4, half = d // 4, d // 2
    c, s = oracle.vision_cos_sin(1, gh, gw, merge, d)
    pos = []
    for bh in range(gh // merge):
        for bw in range(gw // merge):
            for lh in range(merge):
                for lw in range(merge):
                    pos.append((bh * merge + lh, bw * merge + lw))
    j = np.arange(q4, dtype=np.float64)
    inv = 10000.0 ** (-2.0 * j / half)
    for t, (h, w) in enumerate(pos):
        exp_c = np.concatenate([np.cos(h * inv), np.cos(w * inv)] * 2)
        exp_s = np.concatenate([np.sin(h * inv), np.sin(w * inv)] * 2)
        assert np.allclose(c[t], exp_c, atol=2e-6), t
        assert np.allclose(s[t], exp_s, atol=2e-6), t
    # spot values named in the reference's comments: token (h=0, w=1) is index 1
    t1 = pos.index((0, 1))
    for jj in (1, q4 - 1):
        assert np.isclose(c[t1, q4 + jj], np.cos(10000.0 ** (-2.0 * jj / half)), atol=1e-6)
    t2 = pos.index((1, 0))
    for jj in (1, q4 - 1):
        assert np.isclose(c[t2, jj], np.cos(10000.0 ** (-2.0 * jj / half)), atol=1e-6)
        assert np.isclose(s[t2, half + jj], np.sin(10000.0 ** (-2.0 * jj / half)), atol=1e-6)
