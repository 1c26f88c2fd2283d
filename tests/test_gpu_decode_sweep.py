"""Seeded sweep of paged decode launches through the C ABI: batch size, ragged lengths
(empty rows included), block size, pool layout, element type, GQA ratio, head size and
split size all vary.  Each launch must match the oracle and, bit for bit, the contiguous
decode of the same tokens."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_decode import TORCH, dev, host, make_paged
from tests.util import assert_fp32_close, assert_lowp_close, normal, quantize

HEADS = [(8, 8, 128), (32, 8, 128), (12, 2, 128), (16, 4, 64), (28, 4, 128), (8, 1, 256)]


def _cases(n=14, seed=0xDEC0):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv, d = HEADS[int(rng.integers(0, len(HEADS)))]
        kind = ["fp16", "bf16", "fp32"][i % 3]
        B = int(rng.integers(1, 24))
        bs = int(rng.choice([8, 16, 32, 64]))
        layout = int(rng.choice([K.KV_LAYOUT_TOKEN_MAJOR, K.KV_LAYOUT_HEAD_MAJOR]))
        split = int(rng.choice([0, 0, 64, 192, 320, 1024]))
        out.append((i, kind, B, Hq, Hkv, d, bs, layout, split))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("i,kind,B,Hq,Hkv,d,bs,layout,split", _cases())
def test_paged_decode_sweep(i, kind, B, Hq, Hkv, d, bs, layout, split):
    rng = np.random.default_rng(2000 + i)
    lens = rng.integers(1, 2600, B).astype(np.int32)
    if B > 2:
        lens[rng.integers(0, B)] = 0  # an empty row gives zeros
    kc, vc, kp, vp, bt = make_paged(rng, np.maximum(lens, 1), Hkv, d, bs, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    lens_d = torch.from_numpy(lens).cuda()
    maxlen = int(lens.max())
    kpl, vpl = (kp, vp) if layout == K.KV_LAYOUT_TOKEN_MAJOR else (
        kp.transpose(0, 2, 1, 3), vp.transpose(0, 2, 1, 3))
    op = torch.full((B, Hq, d), 7.0, device="cuda", dtype=TORCH[kind])
    oc = torch.zeros_like(op)
    K.paged_decode_cu(dev(q, kind), dev(kpl, kind), dev(vpl, kind), op,
                      torch.from_numpy(bt).cuda(), lens_d, maxlen, split_tokens=split,
                      layout=layout)
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), oc, lens_d, maxlen, Hkv,
                        split_tokens=split)
    torch.cuda.synchronize()
    assert torch.equal(op, oc), f"sweep case {i}: paged != contiguous"
    got = host(op)
    empty = lens == 0
    assert np.all(got[empty] == 0.0), f"sweep case {i}: empty rows"
    live = ~empty
    ref = oracle.decode_contig(q[live], kc[live], vc[live], lens[live])
    if kind == "fp32":
        assert_fp32_close(got[live], ref, d, what=f"sweep case {i}")
    else:
        assert_lowp_close(got[live], ref, what=f"sweep case {i}")
    # The same batch with one split per row: 16-bit K/V run the whole-row (16-wave)
    # workgroups where the shape allows; still bit-equal between paged and contiguous.
    whole = (maxlen + 63) // 64 * 64
    op1 = torch.full((B, Hq, d), 7.0, device="cuda", dtype=TORCH[kind])
    oc1 = torch.zeros_like(op1)
    K.paged_decode_cu(dev(q, kind), dev(kpl, kind), dev(vpl, kind), op1,
                      torch.from_numpy(bt).cuda(), lens_d, maxlen, split_tokens=whole,
                      layout=layout)
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), oc1, lens_d, maxlen, Hkv,
                        split_tokens=whole)
    torch.cuda.synchronize()
    assert torch.equal(op1, oc1), f"sweep case {i}: whole-row paged != contiguous"
    got1 = host(op1)
    assert np.all(got1[empty] == 0.0), f"sweep case {i}: whole-row empty rows"
    if kind == "fp32":
        assert_fp32_close(got1[live], ref, d, what=f"sweep case {i} whole-row")
    else:
        assert_lowp_close(got1[live], ref, what=f"sweep case {i} whole-row")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("B,Hq,Hkv,d", [(1, 32, 8, 128), (2, 12, 2, 128), (3, 16, 4, 64)])
@pytest.mark.parametrize("split", [64, 256])
def test_small_launch_split_decode(kind, B, Hq, Hkv, d, split):
    """Launches with no more workgroups than CUs (here at most 3 rows x 8 kv heads x 32
    splits) run 16-wave workgroups per split where the shape allows, then the merge; the
    result must match the oracle and be bit-equal between paged and contiguous caches."""
    rng = np.random.default_rng(4100 + B * 10 + d + split)
    lens = np.array([2048, 300, 1][:B], np.int32)
    kc, vc, kp, vp, bt = make_paged(rng, lens, Hkv, d, 16, kind)
    q = quantize(normal(rng, (B, Hq, d)), kind)
    lens_d = torch.from_numpy(lens).cuda()
    maxlen = int(lens.max())
    op = torch.full((B, Hq, d), 7.0, device="cuda", dtype=TORCH[kind])
    oc = torch.zeros_like(op)
    K.paged_decode_cu(dev(q, kind), dev(kp, kind), dev(vp, kind), op, torch.from_numpy(bt).cuda(),
                      lens_d, maxlen, split_tokens=split, layout=K.KV_LAYOUT_TOKEN_MAJOR)
    K.batched_decode_cu(dev(q, kind), dev(kc, kind), dev(vc, kind), oc, lens_d, maxlen, Hkv,
                        split_tokens=split)
    torch.cuda.synchronize()
    assert torch.equal(op, oc), "small launch: paged != contiguous"
    ref = oracle.decode_contig(q, kc, vc, lens)
    if kind == "fp32":
        assert_fp32_close(host(op), ref, d, what=f"small launch {kind} B{B} split {split}")
    else:
        assert_lowp_close(host(op), ref, what=f"small launch {kind} B{B} split {split}")
