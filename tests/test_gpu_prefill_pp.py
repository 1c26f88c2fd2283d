"""GPU parity of the 8-wave ping-pong MFMA kernel (head size 128, grids of at least 256
256-query workgroups, which it is picked for) against the oracle: ragged causal lengths,
start_pos > 0, output aliasing query, and bidirectional varlen segments."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_prefill import run_prefill, sample_rows
from tests.test_gpu_vision import TORCH, dev, vision_inputs
from tests.util import assert_lowp_close, quantize

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("start_pos,S", [(0, 2000), (300, 1900), (0, 2049)])
def test_pp_causal_ragged_prefix(kind, start_pos, S):
    """32 q / 8 kv heads, S not a multiple of the 256-row workgroup or 64-key tile; the
    last workgroup's rows past S are never stored."""
    rng = np.random.default_rng(start_pos + S)
    Hq, Hkv, d = 32, 8, 128
    q, kc, vc, out = run_prefill(kind, start_pos, S, Hq, Hkv, d, start_pos + S + 64, 2, 1, rng)
    rows = sample_rows(S, 40, rng)
    ref = oracle.prefill_causal(start_pos, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"pp {kind} start {start_pos} S {S}")


def test_pp_output_aliases_query():
    rng = np.random.default_rng(7)
    S, Hq, Hkv, d = 2048, 32, 4, 128
    q, kc, vc, out = run_prefill("fp16", 0, S, Hq, Hkv, d, S, 1, 0, rng, alias=True)
    rows = sample_rows(S, 40, rng)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what="pp aliased")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("d", [128, 96, 80, 72, 64])
def test_pp_varlen_bidirectional(kind, d):
    """4 segments (one ragged) x 16 heads: 256 workgroups of 256 queries.  Head sizes
    below 128 pad the QK contraction to a multiple of 16 and O^T to a multiple of 32."""
    rng = np.random.default_rng(11 + d)
    H = 16
    cu = np.array([0, 1024, 2048, 2900, 3924], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    N = int(cu[-1])
    out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), 1024, H, d)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1023, 1024, 2047, 2048, 2899, 2900, N - 1],
                                     rng.integers(0, N, 48)]))
    ref = oracle.varlen_bidir(q, k, v, cu, rows=rows, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy()[rows], ref, what=f"pp varlen {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("d", [64, 96])
def test_pp_causal_small_head(kind, d):
    """Causal GQA prefill with head sizes below 128 on the ping-pong kernel (S 2048 x 32
    heads = 256 workgroups)."""
    rng = np.random.default_rng(d)
    S, Hq, Hkv = 2048, 32, 8
    q, kc, vc, out = run_prefill(kind, 0, S, Hq, Hkv, d, S, 1, 0, rng)
    rows = sample_rows(S, 40, rng)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"pp causal d {d} {kind}")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("start_pos,S,Hq,Hkv,d", [(0, 2048, 12, 2, 128), (100, 2049, 12, 2, 128),
                                                  (0, 1024, 32, 8, 128), (0, 300, 12, 2, 128),
                                                  (37, 600, 4, 1, 128), (0, 1500, 12, 12, 128),
                                                  (5, 1800, 8, 2, 64), (0, 2048, 6, 3, 96),
                                                  (6000, 520, 8, 2, 128), (3000, 257, 4, 1, 64)])
def test_pp_causal_key_split(kind, start_pos, S, Hq, Hkv, d):
    """Causal launches with fewer 256-query blocks than CUs cut each block's key tiles into
    near-equal chunks (partials merged by a second launch): BASELINE config 2 (S 2048, 12 q /
    2 kv heads), ragged / prefixed / tiny variants, and long prefixes (6000 and 3000 cached
    tokens before a few hundred queries: up to 8 chunks per block, a one-row last block)."""
    rng = np.random.default_rng(start_pos + S + Hq)
    q, kc, vc, out = run_prefill(kind, start_pos, S, Hq, Hkv, d, start_pos + S, 1, 0, rng)
    rows = sample_rows(S, 60, rng)
    ref = oracle.prefill_causal(start_pos, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"key split {kind} start {start_pos} S {S}")


def test_pp_key_split_aliased_output():
    """Output aliasing query under the key split: every chunk reads Q before the merge
    launch writes O."""
    rng = np.random.default_rng(77)
    S, Hq, Hkv, d = 2048, 12, 2, 128
    q, kc, vc, out = run_prefill("fp16", 0, S, Hq, Hkv, d, S, 1, 0, rng, alias=True)
    rows = sample_rows(S, 60, rng)
    ref = oracle.prefill_causal(0, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what="key split aliased")


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_pp_launches_are_bit_reproducible(kind):
    """The same launch on the same inputs gives the same bits, causal (with and without the
    key split) and varlen: the kernels hold no atomics or order-dependent reductions."""
    rng = np.random.default_rng(23)
    H, d = 16, 128
    cu = np.array([0, 1024, 2048, 2900, 3924], np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    N = int(cu[-1])
    args = [dev(q, kind), dev(k, kind), dev(v, kind)]
    dcu = torch.from_numpy(cu).cuda()
    outs = []
    for _ in range(3):
        out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
        K.vision_attention_varlen_cu(*args, out, dcu, 1024, H, d)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    for S, Hq, Hkv in [(4096, 32, 8), (2048, 12, 2)]:  # one plain launch, one key split
        res = [run_prefill(kind, 0, S, Hq, Hkv, d, S, 1, 0, np.random.default_rng(5))[3]
               for _ in range(2)]
        assert np.array_equal(res[0], res[1]), f"causal S {S}"


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_key_split_close_to_unsplit(kind):
    """The key split's partials (O / l in fp16 for fp16 inputs, fp32 for bf16) add at most
    about one rounding of the output type: C2 (12 heads, split) against the same heads
    launched three times over (36 heads, 288 blocks: no split)."""
    rng = np.random.default_rng(31)
    S, Hq, Hkv, d = 2048, 12, 2, 128
    q = quantize(rng.standard_normal((S, Hq * d)).astype(np.float32), kind)
    k = quantize(rng.standard_normal((S, Hkv * d)).astype(np.float32), kind)
    v = quantize(rng.standard_normal((S, Hkv * d)).astype(np.float32), kind)
    dt = TORCH[kind]

    def run(qh, kh, vh, hq, hkv):
        qd = torch.from_numpy(qh).to(dt).cuda()
        out = torch.zeros_like(qd)
        K.flash_attention_prefill_cu(0, S, hq, hkv, d, hq // hkv, 0, S, hkv * d, qd, out,
                                     torch.from_numpy(kh).to(dt).cuda(),
                                     torch.from_numpy(vh).to(dt).cuda())
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    split = run(q, k, v, Hq, Hkv)
    whole = run(np.tile(q, (1, 3)), np.tile(k, (1, 3)), np.tile(v, (1, 3)), 3 * Hq, 3 * Hkv)
    ulp = 2.0 ** -10 if kind == "fp16" else 2.0 ** -7  # one unit in the last place, relative
    for c in range(3):
        part = whole[:, c * Hq * d:(c + 1) * Hq * d]
        err = np.abs(split - part)
        # Chunks sum their keys in another order than the whole row: the difference is a
        # few roundings of the output type, relative to outputs of order one.
        assert (err <= 2 * ulp * np.abs(part) + 0.5 * ulp).all(), f"{kind} copy {c}: {err.max():.3g}"


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
def test_pp_few_key_tiles(kind):
    """Segments of 64-320 keys (1 to 5 key tiles per workgroup, on and off the tile edges)
    x 16 heads: the ring's first stages are also its last, so the stage issue, the waits
    and (bf16) the register-staged V conversion run their tail cases from the start."""
    rng = np.random.default_rng(77)
    H, d = 16, 128
    seg = [64, 65, 128, 129, 192, 256, 257, 320]
    cu = np.concatenate([[0], np.cumsum(seg)]).astype(np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    N = int(cu[-1])
    out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), max(seg), H, d)
    torch.cuda.synchronize()
    ref = oracle.varlen_bidir(q, k, v, cu, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy(), ref, what=f"pp few tiles {kind}")
