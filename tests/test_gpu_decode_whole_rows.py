"""Whole-row decode launches that fill the device (at least one (row, kv head) per CU, one
split per row): the matrix-core decode kernel (decode_mfma.hip), or the dot-product kernel
beyond 16 query heads per kv head.  Every case goes through the C ABI, is checked against
the oracle and, bit for bit, between the paged pool (both layouts, several block sizes) and
the contiguous cache.  Lengths include empty rows, one key, and lengths on and around the
32-token tile edges; the GQA ratios cover one to 32 query heads per kv head; bf16 values far
outside fp16's range must stay exact."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_decode import TORCH, dev, host, make_paged
from tests.util import assert_lowp_close, normal, quantize

N_CU = 256  # MI355X; the launches below have at least this many (row, kv head) units

EDGE_LENS = [0, 1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257]


def _batch(Hkv):
    return -(-N_CU // Hkv)


def _lens(rng, B, hi):
    lens = rng.integers(1, hi, B).astype(np.int32)
    lens[: len(EDGE_LENS)] = EDGE_LENS[:B]
    return lens


def _run(rng, kind, Hq, Hkv, d, bs, layout, lens, q, kc, vc, kp, vp, bt):
    B = len(lens)
    lens_d = torch.from_numpy(lens).cuda()
    maxlen = int(lens.max())
    whole = (maxlen + 63) // 64 * 64
    kpl, vpl = (kp, vp) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (
        kp.transpose(0, 2, 1, 3), vp.transpose(0, 2, 1, 3))
    op = torch.full((B, Hq, d), 7.0, device="cuda", dtype=TORCH[kind])
    oc = torch.full_like(op, -3.0)
    K.paged_decode_cu(dev(q, kind), dev(kpl, kind), dev(vpl, kind), op,
                      torch.from_numpy(bt).cuda(), lens_d, maxlen, split_tokens=whole,
                      layout=layout)
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), oc, lens_d, maxlen, Hkv,
                        split_tokens=whole)
    torch.cuda.synchronize()
    assert torch.equal(op, oc), "whole-row decode: paged != contiguous"
    return host(op)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("Hq,Hkv,d,bs,layout", [
    (32, 8, 128, 16, 1),   # Qwen3-8B heads, the bench's pool
    (32, 8, 128, 8, 0),    # 8-token blocks: four blocks per 32-token tile
    (12, 2, 128, 32, 1),   # Qwen2.5-1.5B heads (6 per kv head)
    (64, 4, 128, 64, 0),   # 16 query heads per kv head
    (16, 16, 64, 16, 1),   # MHA, head size 64
    (24, 8, 64, 8, 1),     # 3 per kv head, head size 64
    (64, 2, 128, 16, 1),   # 32 per kv head: beyond the matrix-core kernel, dot-product kernel
])
def test_whole_row_decode(kind, Hq, Hkv, d, bs, layout):
    rng = np.random.default_rng(Hq * 1000 + Hkv * 10 + d + bs)
    B = _batch(Hkv)
    lens = _lens(rng, B, 700)
    kc, vc, kp, vp, bt = make_paged(rng, np.maximum(lens, 1), Hkv, d, bs, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    got = _run(rng, kind, Hq, Hkv, d, bs, layout, lens, q, kc, vc, kp, vp, bt)
    empty = lens == 0
    assert np.all(got[empty] == 0.0), "empty rows must give zeros"
    live = ~empty
    one = lens == 1
    assert np.array_equal(got[one], np.broadcast_to(
        vc[one, 0][:, np.repeat(np.arange(Hkv), Hq // Hkv)], got[one].shape)), \
        "a single key must return its V row exactly"
    ref = oracle.decode_contig(q[live], kc[live], vc[live], lens[live])
    assert_lowp_close(got[live], ref, what=f"whole-row {kind} {Hq}/{Hkv} d {d} bs {bs}")


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1e5, 3e30, 1e-6])
def test_whole_row_decode_bf16_range(scale):
    """bf16 V outside fp16's range (|v| up to 3e30 overflows fp16; 1e-6 is an fp16
    subnormal): the weights are split into bf16 hi + lo and V is never converted, so the
    result keeps the oracle's relative accuracy at every scale."""
    rng = np.random.default_rng(77)
    Hq, Hkv, d, bs = 32, 8, 128, 16
    B = _batch(Hkv)
    lens = _lens(rng, B, 600)
    lens[lens == 0] = 5
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, "bf16")
    vc = quantize(vc * np.float32(scale), "bf16")
    vp = quantize(vp * np.float32(scale), "bf16")
    q = quantize(normal(rng, (B, Hq, d)), "bf16")
    got = _run(rng, "bf16", Hq, Hkv, d, bs, 1, lens, q, kc, vc, kp, vp, bt)
    assert np.isfinite(got).all()
    ref = oracle.decode_contig(q, kc, vc, lens)
    # the lowp bar on values rescaled to unit size
    assert_lowp_close(got / scale, ref / scale, what=f"bf16 V x {scale:g}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", [0, 1])
def test_long_whole_rows_repeatable(kind, layout):
    """Rows of up to 3000 tokens (lengths on and around 32-token tile edges); five launches,
    with launches of a batch twice as large in between, give the same bits, equal between
    paged and contiguous caches and within the lowp bar of the oracle."""
    rng = np.random.default_rng(500 + layout)
    Hq, Hkv, d, bs = 32, 8, 128, 16
    B = _batch(Hkv)
    lens = rng.integers(1, 3001, B).astype(np.int32)
    lens[:10] = [3000, 1536, 1537, 1538, 1600, 1601, 2047, 2048, 2049, 1]
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    first = _run(rng, kind, Hq, Hkv, d, bs, layout, lens, q, kc, vc, kp, vp, bt)
    ref = oracle.decode_contig(q, kc, vc, lens, nthreads=8)
    assert_lowp_close(first, ref, what=f"long whole rows {kind} layout {layout}")
    B2 = 2 * B
    lens2 = rng.integers(1, 2500, B2).astype(np.int32)
    kc2, vc2, kp2, vp2, bt2 = make_paged(rng, lens2, Hkv, d, bs, kind)
    q2 = quantize(normal(rng, (B2, Hq, d)), kind)
    for rep in range(4):
        got2 = _run(rng, kind, Hq, Hkv, d, bs, layout, lens2, q2, kc2, vc2, kp2, vp2, bt2)
        again = _run(rng, kind, Hq, Hkv, d, bs, layout, lens, q, kc, vc, kp, vp, bt)
        assert np.array_equal(again, first), f"repeat {rep}: whole-row decode not reproducible"
    ref2 = oracle.decode_contig(q2, kc2, vc2, lens2, nthreads=8)
    assert_lowp_close(got2, ref2, what=f"long whole rows, batch {B2}")


@pytest.mark.gpu
@pytest.mark.parametrize("layout", [0, 1])
def test_whole_rows_row_past_bound_is_nan(layout):
    """A device length above max_context_len makes that row NaN (every head); the other
    rows of the launch keep the oracle's accuracy."""
    rng = np.random.default_rng(610 + layout)
    Hq, Hkv, d, bs = 32, 8, 128, 16
    B = _batch(Hkv)
    lens = rng.integers(1, 900, B).astype(np.int32)
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, bs, "fp16")
    q = quantize(normal(rng, (B, Hq, d)), "fp16")
    bound = int(np.sort(lens)[-3])
    bad = lens > bound
    kpl, vpl = (kp, vp) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (
        kp.transpose(0, 2, 1, 3), vp.transpose(0, 2, 1, 3))
    o = torch.zeros(B, Hq, d, device="cuda", dtype=torch.float16)
    K.paged_decode_cu(dev(q, "fp16"), dev(kpl, "fp16"), dev(vpl, "fp16"), o,
                      torch.from_numpy(bt).cuda(), torch.from_numpy(lens).cuda(), bound,
                      split_tokens=(bound + 63) // 64 * 64, layout=layout)
    torch.cuda.synchronize()
    got = host(o)
    assert np.isnan(got[bad]).all()
    ok = ~bad
    ref = oracle.decode_contig(q[ok], kc[ok], vc[ok], lens[ok], nthreads=8)
    assert_lowp_close(got[ok], ref, what="rows within the bound")


@pytest.mark.gpu
def test_whole_rows_graph_replay():
    """The automatic split's whole-row launch captured in a graph: replays with new
    lengths and queries written in place give the bits of the eager launch."""
    rng = np.random.default_rng(620)
    Hq, Hkv, d, bs = 32, 8, 128, 16
    B = _batch(Hkv)
    cap_len = 1024
    lens = rng.integers(1, cap_len + 1, B).astype(np.int32)
    kc, vc, kp, vp, bt = make_paged(rng, np.full(B, cap_len, np.int32), Hkv, d, bs, "fp16")
    dkp = dev(kp.transpose(0, 2, 1, 3), "fp16")
    dvp = dev(vp.transpose(0, 2, 1, 3), "fp16")
    dbt = torch.from_numpy(bt).cuda()
    dlens = torch.from_numpy(lens).cuda()
    q = quantize(normal(rng, (B, Hq, d)), "fp16")
    dq = dev(q, "fp16")
    s = torch.cuda.Stream()
    out = torch.empty(B, Hq, d, device="cuda", dtype=torch.float16)
    with torch.cuda.stream(s):
        K.paged_decode_cu(dq, dkp, dvp, out, dbt, dlens, cap_len, layout=1)  # warm-up
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        K.paged_decode_cu(dq, dkp, dvp, out, dbt, dlens, cap_len, layout=1)
    for rep in range(3):
        lens2 = rng.integers(1, cap_len + 1, B).astype(np.int32)
        q2 = quantize(normal(rng, (B, Hq, d)), "fp16")
        dlens.copy_(torch.from_numpy(lens2))
        dq.copy_(dev(q2, "fp16"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = host(out)
        eager = torch.empty_like(out)
        K.paged_decode_cu(dq, dkp, dvp, eager, dbt, dlens, cap_len, layout=1)
        torch.cuda.synchronize()
        assert np.array_equal(got, host(eager)), f"replay {rep} differs from the eager launch"
        ref = oracle.decode_contig(q2, kc, vc, lens2, nthreads=8)
        assert_lowp_close(got, ref, what=f"replay {rep}")
