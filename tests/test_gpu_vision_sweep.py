"""Seeded sweep of bidirectional varlen attention launches through the C ABI against the
oracle: segment count and lengths (1 token up to 1500), head count and head size vary."""
import numpy as np
import pytest
import torch

from oracle import oracle
from orinmllm_amd import kernel as K
from tests.test_gpu_vision import TORCH, dev, vision_inputs
from tests.util import assert_lowp_close


def _cases(n=10, seed=0x715):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        n_seg = int(rng.integers(1, 7))
        seg = rng.integers(1, 1500, n_seg)
        cu = tuple(int(x) for x in np.concatenate([[0], np.cumsum(seg)]))
        out.append((i, "bf16" if i % 2 else "fp16", int(rng.choice([4, 12, 16])),
                    int(rng.choice([64, 72, 80, 96, 128])), cu))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("i,kind,H,d,cu", _cases())
def test_varlen_bidir_sweep(i, kind, H, d, cu):
    rng = np.random.default_rng(3000 + i)
    cu = np.array(cu, np.int32)
    q, k, v = vision_inputs(rng, cu, H, d, kind)
    N = int(cu[-1])
    out = torch.zeros(N, H * d, device="cuda", dtype=TORCH[kind])
    K.vision_attention_varlen_cu(dev(q, kind), dev(k, kind), dev(v, kind), out,
                                 torch.from_numpy(cu).cuda(), int(np.diff(cu).max()), H, d)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.integers(0, N, 32)]))
    ref = oracle.varlen_bidir(q, k, v, cu, rows=rows, nthreads=8)
    assert_lowp_close(out.float().cpu().numpy()[rows], ref, what=f"sweep case {i}")
