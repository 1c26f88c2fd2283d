"""orin_flash_attention_decode_gpu_pos_noalloc through the C ABI: its partials live in the
library's fixed device array, and its output equals orin_flash_attention_decode_gpu_pos
bit for bit on two calls in a row (the second smaller), both eagerly and under graph
capture; a launch whose partials do not fit is refused before anything is queued."""
import ctypes as C

import numpy as np
import pytest
import torch

from orinmllm_amd import _lib
from tests.util import normal, quantize

pytestmark = pytest.mark.gpu


def _case(rng, Hq, Hkv, d, max_seq, layers, dtype):
    kv_dim = Hkv * d
    tdt = torch.float16 if dtype == _lib.DTYPE_FP16 else torch.bfloat16
    kind = "fp16" if dtype == _lib.DTYPE_FP16 else "bf16"

    def t(shape):
        return torch.from_numpy(quantize(normal(rng, shape), kind)).to("cuda", tdt)

    return dict(Hq=Hq, Hkv=Hkv, d=d, max_seq=max_seq, kv_dim=kv_dim, dtype=dtype,
                kc=t((layers, max_seq, kv_dim)), vc=t((layers, max_seq, kv_dim)),
                q=t((Hq * d,)), pos=torch.zeros(1, dtype=torch.int32, device="cuda"),
                layer=layers - 1, tdt=tdt)


def _call(fn, c, out, stream):
    return fn(c["pos"].data_ptr(), c["Hq"], c["Hkv"], c["d"], c["Hq"] // c["Hkv"], c["layer"],
              c["max_seq"], c["kv_dim"], c["q"].data_ptr(), out.data_ptr(), c["kc"].data_ptr(),
              c["vc"].data_ptr(), c["dtype"], C.c_void_p(stream))


def test_noalloc_decode_matches_gpu_pos():
    lib = _lib.load()
    rng = np.random.default_rng(41)
    stream = torch.cuda.current_stream().cuda_stream
    big = _case(rng, 32, 8, 128, 16384, 2, _lib.DTYPE_FP16)
    small = _case(rng, 16, 2, 64, 3000, 1, _lib.DTYPE_BF16)
    for c, positions in [(big, [16383, 9000]), (small, [2999, 700])]:
        for p in positions:
            c["pos"].fill_(p)
            ref = torch.full((c["Hq"] * c["d"],), float("nan"), device="cuda", dtype=c["tdt"])
            got = torch.full_like(ref, float("nan"))
            torch.cuda.synchronize()
            assert _call(lib.orin_flash_attention_decode_gpu_pos, c, ref, stream) == 0
            assert _call(lib.orin_flash_attention_decode_gpu_pos_noalloc, c, got, stream) == 0
            torch.cuda.synchronize()
            assert not torch.isnan(got.float()).any()
            assert torch.equal(got, ref), f"noalloc differs at Hq {c['Hq']} pos {p}"


def test_noalloc_decode_in_graph_and_size_limit():
    lib = _lib.load()
    rng = np.random.default_rng(42)
    c = _case(rng, 32, 8, 128, 8192, 1, _lib.DTYPE_FP16)
    cap = torch.cuda.Stream()
    out = torch.zeros(c["Hq"] * c["d"], device="cuda", dtype=c["tdt"])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = []
    with torch.cuda.graph(g, stream=cap):  # no reserve needed
        st.append(_call(lib.orin_flash_attention_decode_gpu_pos_noalloc, c, out, cap.cuda_stream))
    assert st == [0]
    for p in [8191, 10, 4096]:
        c["pos"].fill_(p)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = torch.zeros_like(out)
        assert _call(lib.orin_flash_attention_decode_gpu_pos, c, ref,
                     torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"graph replay at pos {p}"
    # partials beyond the fixed array: refused, output untouched
    assert lib.orin_flash_attention_decode_noalloc_max_bytes() == 4 << 20
    marker = torch.full_like(out, 7.0)
    torch.cuda.synchronize()
    status = lib.orin_flash_attention_decode_gpu_pos_noalloc(
        c["pos"].data_ptr(), 32, 8, 128, 4, 0, 200000, 1024, c["q"].data_ptr(),
        marker.data_ptr(), c["kc"].data_ptr(), c["vc"].data_ptr(), c["dtype"],
        C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert status == _lib.ERR_WORKSPACE
    assert torch.equal(marker, torch.full_like(out, 7.0))
