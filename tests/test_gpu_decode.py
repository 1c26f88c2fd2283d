"""GPU parity of the decode path (fp32 MHA, flash decode, batched and paged decode)
against the CPU oracle, through the C ABI."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.util import (assert_fp32_close, assert_fp32_elementwise, assert_lowp_close,
                        fp64_decode, normal, quantize, rel_error)

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def dev(x, kind="fp32"):
    return torch.from_numpy(np.ascontiguousarray(quantize(x, kind))).to("cuda", TORCH[kind])


def host(t):
    return t.float().cpu().numpy()


# ---------------------------------------------------------------- kuiper fp32 MHA

@pytest.mark.parametrize("gpu_pos", [False, True])
def test_c1_fp32_mha_kernel(gpu_pos):
    """12 q = 12 kv heads, d 64, query at pos 255 over a 256-token
    cache; the fp32 bar is the reference's own (rel < 1e-4)."""
    rng = np.random.default_rng(0xC1)
    head_num, head_size, seq_len, pos, layers, layer = 12, 64, 256, 255, 2, 1
    kv_dim = head_num * head_size
    q = normal(rng, head_num * head_size)
    kc = normal(rng, (layers, seq_len, kv_dim))
    vc = normal(rng, (layers, seq_len, kv_dim))
    ref, _ = oracle.mha_kernel(pos, head_num, layer, seq_len, kv_dim, 1, head_size, q, kc, vc)
    out = torch.zeros(head_num * head_size, device="cuda")
    score = torch.zeros(head_num, seq_len, device="cuda")
    if gpu_pos:
        p = torch.tensor([pos], dtype=torch.int32, device="cuda")
        K.mha_kernel_cu_gpu_pos(p, head_num, layer, seq_len, kv_dim, 1, head_size, out, dev(q),
                                score, dev(kc), dev(vc))
    else:
        K.mha_kernel_cu(pos, head_num, layer, seq_len, kv_dim, 1, head_size, out, dev(q), score,
                        dev(kc), dev(vc))
    torch.cuda.synchronize()
    assert_fp32_close(host(out), ref, head_size, what="C1")
    # Element by element against float64: 1e-4 relative (floor 1e-6 of the head max).
    truth = fp64_decode(q, kc[layer, : pos + 1].reshape(pos + 1, head_num, head_size),
                        vc[layer, : pos + 1].reshape(pos + 1, head_num, head_size), head_num, 1,
                        head_size)
    assert_fp32_elementwise(host(out), truth, head_size, what="C1 vs fp64")
    # The reference's own element-wise metric (bench_mha_kernels.cu:467-477), reported:
    # it is dominated by near-zero outputs, see assert_fp32_close.
    print(f"C1 element-wise rel error (reference metric): {rel_error(host(out), ref):.3g}")


@pytest.mark.parametrize("pos", [0, 1, 63, 100, 500, 2000, 4095])
def test_fp32_mha_qwen3_shape(pos):
    """Qwen3-8B shape (32 q / 8 kv heads, d 128) at the positions of the reference's
    benchmark (bench_mha_kernels.cu:780-801), GQA, several splits."""
    rng = np.random.default_rng(1000 + pos)
    head_num, kv_heads, d, seq_len = 32, 8, 128, 4096
    kv_dim, kv_mul = kv_heads * d, head_num // kv_heads
    q = rng.uniform(-1, 1, head_num * d).astype(np.float32)
    kc = rng.uniform(-1, 1, (1, seq_len, kv_dim)).astype(np.float32)
    vc = rng.uniform(-1, 1, (1, seq_len, kv_dim)).astype(np.float32)
    ref, _ = oracle.mha_kernel(pos, head_num, 0, seq_len, kv_dim, kv_mul, d, q, kc, vc)
    out = torch.zeros(head_num * d, device="cuda")
    score = torch.zeros(head_num, seq_len, device="cuda")
    K.get_mha_kernel(K.DeviceType.kDeviceCUDA)(pos, head_num, 0, seq_len, kv_dim, kv_mul, d, out,
                                               dev(q), score, dev(kc), dev(vc))
    torch.cuda.synchronize()
    assert_fp32_close(host(out), ref, d, what=f"pos {pos}")
    # The GPU result is no farther from an fp64 evaluation than the fp32 oracle is.
    Q = q.reshape(head_num, d).astype(np.float64)
    Kd = kc[0, : pos + 1].reshape(pos + 1, kv_heads, d).astype(np.float64)
    V = vc[0, : pos + 1].reshape(pos + 1, kv_heads, d).astype(np.float64)
    truth = np.zeros((head_num, d))
    for h in range(head_num):
        s = Kd[:, h // kv_mul] @ Q[h] / np.sqrt(d)
        p = np.exp(s - s.max())
        truth[h] = (p / p.sum()) @ V[:, h // kv_mul]
    truth = truth.ravel()
    assert np.abs(host(out) - truth).max() <= 2 * np.abs(ref - truth).max() + 1e-7
    assert_fp32_elementwise(host(out), truth, d, what=f"pos {pos} vs fp64")


# ---------------------------------------------------------------- flash decode

@pytest.mark.parametrize("kind", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("pos", [0, 290, 1000, 4095])
@pytest.mark.parametrize("gpu_pos", [False, True])
def test_flash_decode(kind, pos, gpu_pos):
    rng = np.random.default_rng(7 + pos)
    head_num, kv_heads, d, max_seq, layers, layer = 32, 8, 128, 4096, 2, 1
    kv_dim, kv_mul = kv_heads * d, head_num // kv_heads
    q = quantize(normal(rng, head_num * d), kind)
    kc = quantize(normal(rng, (layers, max_seq, kv_dim)), kind)
    vc = quantize(normal(rng, (layers, max_seq, kv_dim)), kind)
    ref, _ = oracle.mha_kernel(pos, head_num, layer, max_seq, kv_dim, kv_mul, d, q, kc, vc)
    out = torch.zeros(head_num * d, device="cuda", dtype=TORCH[kind])
    args = (head_num, kv_heads, d, kv_mul, layer, max_seq, kv_dim, dev(q, kind), out,
            dev(kc, kind), dev(vc, kind))
    if gpu_pos:
        p = torch.tensor([pos], dtype=torch.int32, device="cuda")
        K.flash_attention_decode_fp16_gpu_pos_cu(p, *args)
    else:
        K.flash_attention_decode_cu(pos, *args)
    torch.cuda.synchronize()
    if kind == "fp32":
        assert_fp32_close(host(out), ref, d, what=f"fp32 decode pos {pos}")
    else:
        assert_lowp_close(host(out), ref, what=f"{kind} decode pos {pos}")


def test_decode_single_key_is_v0_exactly():
    """kv_len = 1: the softmax weight is exactly 1, so O = V_0 bit for bit."""
    rng = np.random.default_rng(3)
    for kind in ["fp32", "fp16", "bf16"]:
        q = normal(rng, 32 * 128)
        kc = normal(rng, (1, 64, 1024))
        vc = normal(rng, (1, 64, 1024))
        out = torch.zeros(32 * 128, device="cuda", dtype=TORCH[kind])
        vdev = dev(vc, kind)
        K.flash_attention_decode_cu(0, 32, 8, 128, 4, 0, 64, 1024, dev(q, kind), out,
                                    dev(kc, kind), vdev)
        torch.cuda.synchronize()
        want = vdev[0, 0].view(8, 128).repeat_interleave(4, dim=0).reshape(-1)
        assert torch.equal(out, want), kind


# ---------------------------------------------------------------- batched / paged decode

def make_paged(rng, lens, Hkv, d, bs, kind):
    """Contiguous caches [B, S, Hkv, d] and the same tokens scattered over a pool of
    sum(ceil(L/bs)) blocks in a random permutation."""
    B = len(lens)
    S = int(max(lens))
    maxb = (S + bs - 1) // bs
    kc = quantize(normal(rng, (B, S, Hkv, d)), kind)
    vc = quantize(normal(rng, (B, S, Hkv, d)), kind)
    nblk = [(L + bs - 1) // bs for L in lens]
    total = sum(nblk)
    perm = rng.permutation(total).astype(np.int32)
    kp = np.zeros((total, bs, Hkv, d), np.float32)
    vp = np.zeros((total, bs, Hkv, d), np.float32)
    bt = np.zeros((B, maxb), np.int32)
    n = 0
    for b, L in enumerate(lens):
        for j in range(nblk[b]):
            blk = perm[n]
            n += 1
            bt[b, j] = blk
            t0, t1 = j * bs, min((j + 1) * bs, L)
            kp[blk, : t1 - t0] = kc[b, t0:t1]
            vp[blk, : t1 - t0] = vc[b, t0:t1]
    return kc, vc, kp, vp, bt


@pytest.mark.parametrize("layout", [K.KV_LAYOUT_TOKEN_MAJOR, K.KV_LAYOUT_HEAD_MAJOR])
@pytest.mark.parametrize("kind", ["fp16", "bf16", "fp32"])
def test_paged_equals_contiguous_bit_exact(kind, layout):
    rng = np.random.default_rng(11)
    B, Hq, Hkv, d, bs = 6, 32, 8, 128, 16
    lens = np.array([1, 17, 300, 512, 1000, 2049], np.int32)
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    lens_d = torch.from_numpy(lens).cuda()
    maxlen = int(lens.max())
    # 4096: one split per row (16-bit K/V then run the whole-row 16-wave workgroups)
    for split in [0, 64, 256, 4096]:
        oc = torch.zeros(B, Hq, d, device="cuda", dtype=TORCH[kind])
        op = torch.zeros_like(oc)
        K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), oc, lens_d, maxlen, Hkv,
                            split_tokens=split)
        kpl, vpl = (kp, vp) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (
            kp.transpose(0, 2, 1, 3), vp.transpose(0, 2, 1, 3))
        K.paged_decode_cu(dev(q, kind), dev(kpl, kind), dev(vpl, kind), op,
                          torch.from_numpy(bt).cuda(), lens_d, maxlen, split_tokens=split,
                          layout=layout)
        torch.cuda.synchronize()
        assert torch.equal(oc, op), f"split {split}"
        ref = oracle.decode_contig(q, kc, vc, lens)
        if kind == "fp32":
            assert_fp32_close(host(oc), ref, d, what=f"split {split}")
        else:
            assert_lowp_close(host(oc), ref, what=f"split {split}")


def test_split_count_invariance():
    """Split-KV partial merging: any split size gives the same result within fp32 rounding."""
    rng = np.random.default_rng(12)
    B, Hq, Hkv, d = 3, 16, 2, 128
    lens = np.array([700, 1500, 3000], np.int32)
    kc = normal(rng, (B, 3000, Hkv, d))
    vc = normal(rng, (B, 3000, Hkv, d))
    q = normal(rng, (B, Hq, d))
    lens_d = torch.from_numpy(lens).cuda()
    outs = []
    for split in [64, 128, 640, 4096]:
        o = torch.zeros(B, Hq, d, device="cuda")
        K.batched_decode_cu(dev(q), dev(kc), dev(vc), o, lens_d, 3000, Hkv, split_tokens=split)
        outs.append(host(o))
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert_fp32_close(o, outs[0], d, what="split invariance")


def test_split_merge_repeatable_across_streams():
    """Split partials and their merge: repeated launches, on one stream and on two
    streams running at once (separate outputs, shared inputs), give the first launch's
    output bit for bit."""
    rng = np.random.default_rng(14)
    B, Hq, Hkv, d = 5, 32, 8, 128
    lens = np.array([1, 100, 700, 2000, 4000], np.int32)
    kc = quantize(normal(rng, (B, 4000, Hkv, d)), "fp16")
    vc = quantize(normal(rng, (B, 4000, Hkv, d)), "fp16")
    q = quantize(normal(rng, (B, Hq, d)), "fp16")
    qd, kd, vd = dev(q, "fp16"), dev(kc, "fp16"), dev(vc, "fp16")
    lens_d = torch.from_numpy(lens).cuda()

    def call(o):
        K.batched_decode_cu(qd, kd, vd, o, lens_d, 4000, Hkv, split_tokens=256)

    first = torch.zeros(B, Hq, d, device="cuda", dtype=torch.float16)
    call(first)
    torch.cuda.synchronize()
    ref = oracle.decode_contig(q, kc, vc, lens)
    assert_lowp_close(host(first), ref, what="split merge")
    outs = [torch.zeros_like(first) for _ in range(7)]
    for o in outs[:3]:
        call(o)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for i in range(2):
        for j, st in enumerate(streams):
            with torch.cuda.stream(st):
                call(outs[3 + 2 * i + j])
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, first), f"launch {i} differs"


def test_zero_length_rows_give_zeros():
    rng = np.random.default_rng(13)
    B, Hq, Hkv, d = 3, 8, 8, 64
    lens = np.array([0, 5, 0], np.int32)
    kc = normal(rng, (B, 8, Hkv, d))
    vc = normal(rng, (B, 8, Hkv, d))
    q = normal(rng, (B, Hq, d))
    o = torch.full((B, Hq, d), 7.0, device="cuda", dtype=torch.float16)
    K.batched_decode_cu(dev(q, "fp16"), dev(kc, "fp16"), dev(vc, "fp16"), o,
                        torch.from_numpy(lens).cuda(), 8, Hkv)
    torch.cuda.synchronize()
    assert torch.all(o[0] == 0) and torch.all(o[2] == 0)
    ref = oracle.decode_contig(quantize(q, "fp16"), quantize(kc, "fp16"), quantize(vc, "fp16"),
                               lens)
    assert_lowp_close(host(o)[1], ref[1])


@pytest.mark.parametrize("layout", [K.KV_LAYOUT_TOKEN_MAJOR, K.KV_LAYOUT_HEAD_MAJOR])
@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_c4_paged_decode_full_size(kind, layout):
    """BASELINE config 4 at full size: batch 32, 32 q / 8 kv heads, d 128, KV lengths
    U[512, 4096], block 16, block tables a random permutation of the pool."""
    rng = np.random.default_rng(0xC4)
    B, Hq, Hkv, d, bs = 32, 32, 8, 128, 16
    lens = rng.integers(512, 4097, B).astype(np.int32)
    _, _, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    o = torch.zeros(B, Hq, d, device="cuda", dtype=TORCH[kind])
    kpl, vpl = (kp, vp) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (
        kp.transpose(0, 2, 1, 3), vp.transpose(0, 2, 1, 3))
    K.paged_decode_cu(dev(q, kind), dev(kpl, kind), dev(vpl, kind), o,
                      torch.from_numpy(bt).cuda(), torch.from_numpy(lens).cuda(),
                      int(lens.max()), layout=layout)
    torch.cuda.synchronize()
    ref = oracle.decode_paged(q, kp, vp, bt, lens, nthreads=8)
    assert_lowp_close(host(o), ref, what="C4 paged decode")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_gpu_pos_decode_graph_replay(kind):
    """orin_flash_attention_decode_gpu_pos captured once in a HIP graph and replayed with
    the position (and query) changed on the device between replays: every replay equals
    the eager call bit for bit and the oracle within the 16-bit bar."""
    rng = np.random.default_rng(21)
    head_num, kv_heads, d, max_seq, layers, layer = 32, 8, 128, 4096, 2, 1
    kv_dim, kv_mul = kv_heads * d, head_num // kv_heads
    kc = quantize(normal(rng, (layers, max_seq, kv_dim)), kind)
    vc = quantize(normal(rng, (layers, max_seq, kv_dim)), kind)
    kd, vd = dev(kc, kind), dev(vc, kind)
    qd = torch.zeros(head_num * d, device="cuda", dtype=TORCH[kind])
    p = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.zeros(head_num * d, device="cuda", dtype=TORCH[kind])
    cap = torch.cuda.Stream()
    K.reserve_decode_workspace(head_num, d, max_seq, stream=cap)  # the capture stream's buffer

    def call(o):
        K.flash_attention_decode_fp16_gpu_pos_cu(p, head_num, kv_heads, d, kv_mul, layer,
                                                 max_seq, kv_dim, qd, o, kd, vd)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(out)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        call(out)
    for pos in [4095, 5, 1000, 0, 2047]:
        q = quantize(normal(rng, head_num * d), kind)
        qd.copy_(dev(q, kind))
        p.fill_(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = torch.zeros_like(out)
        call(eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay at pos {pos} differs from eager"
        ref, _ = oracle.mha_kernel(pos, head_num, layer, max_seq, kv_dim, kv_mul, d, q, kc, vc)
        assert_lowp_close(host(out), ref, what=f"{kind} graph replay pos {pos}")


@pytest.mark.parametrize("kind", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("Hq,Hkv,d", [(12, 12, 64), (12, 2, 128), (12, 4, 64), (16, 8, 256),
                                      (28, 4, 128), (40, 5, 128), (64, 8, 128)])
def test_decode_head_shapes(kind, Hq, Hkv, d):
    """GQA ratios 1, 2, 3, 6, 7, 8 (query heads per workgroup G = the largest divisor of
    kv_mul up to 8) and head sizes 64 / 128 / 256, ragged lengths, several splits."""
    rng = np.random.default_rng(Hq * 1000 + Hkv * 10 + d)
    B = 4
    lens = np.array([1, 130, 700, 1500], np.int32)
    S = int(lens.max())
    kc = quantize(normal(rng, (B, S, Hkv, d)), kind)
    vc = quantize(normal(rng, (B, S, Hkv, d)), kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    o = torch.zeros(B, Hq, d, device="cuda", dtype=TORCH[kind])
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), o,
                        torch.from_numpy(lens).cuda(), S, Hkv, split_tokens=256)
    torch.cuda.synchronize()
    ref = oracle.decode_contig(q, kc, vc, lens)
    if kind == "fp32":
        assert_fp32_close(host(o), ref, d, what=f"decode {Hq}/{Hkv} d {d}")
    else:
        assert_lowp_close(host(o), ref, what=f"decode {Hq}/{Hkv} d {d} {kind}")
