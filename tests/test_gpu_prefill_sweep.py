"""Seeded sweep of causal prefill shapes through the C ABI against the oracle: head size,
element type, GQA ratio, prefix length, chunk length, cache capacity and layer all vary,
so the launch routing (ping-pong kernel with or without key split, tile kernel) and the
edge tiles meet shapes no hand-picked case names."""
import numpy as np
import pytest

from oracle import oracle
from tests.test_gpu_prefill import run_prefill, sample_rows
from tests.util import assert_lowp_close


def _cases(n=16, seed=0x5EE9):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([64, 72, 80, 96, 128]))
        kind = "fp16" if i % 2 == 0 else "bf16"
        hkv = int(rng.choice([1, 2, 4, 8]))
        kv_mul = int(rng.choice([1, 2, 4, 6]))
        S = int(rng.integers(1, 2500))
        start = int(rng.integers(0, 600)) if i % 3 else 0
        pad = int(rng.integers(0, 100))
        out.append((i, kind, d, hkv * kv_mul, hkv, S, start, start + S + pad))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("i,kind,d,Hq,Hkv,S,start,max_seq", _cases())
def test_prefill_shape_sweep(i, kind, d, Hq, Hkv, S, start, max_seq):
    rng = np.random.default_rng(1000 + i)
    q, kc, vc, out = run_prefill(kind, start, S, Hq, Hkv, d, max_seq, 2, 1, rng)
    rows = sample_rows(S, 24, rng)
    ref = oracle.prefill_causal(start, q, kc, vc, Hq, Hkv, d, rows=rows, nthreads=8)
    assert_lowp_close(out[rows], ref, what=f"sweep case {i}")
