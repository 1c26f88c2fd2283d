"""Library-owned workspaces through the C ABI: reentrancy across streams, capture safety
(a captured decode survives later growth of the library's buffers), the refusal to allocate
while a stream is capturing, and NaN outputs for device lengths past the launch bound."""
import ctypes as C
import warnings

import numpy as np
import pytest
import torch

from orinmllm_amd import _lib
from orinmllm_amd import kernel as K
from tests.util import normal, quantize

pytestmark = pytest.mark.gpu


def dev(x, dtype=torch.float16):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dtype)


class Decode:
    """One kuiper flash decode (Qwen3 shape, fp16) whose launch splits its keys."""

    def __init__(self, rng, max_seq=4096, layers=1):
        self.Hq, self.Hkv, self.d, self.max_seq = 32, 8, 128, max_seq
        kv_dim = self.Hkv * self.d
        self.kc = dev(quantize(normal(rng, (layers, max_seq, kv_dim)), "fp16"))
        self.vc = dev(quantize(normal(rng, (layers, max_seq, kv_dim)), "fp16"))
        self.q = dev(quantize(normal(rng, self.Hq * self.d), "fp16"))
        self.pos = torch.zeros(1, dtype=torch.int32, device="cuda")

    def host_pos(self, pos, out, stream):
        K.flash_attention_decode_cu(pos, self.Hq, self.Hkv, self.d, self.Hq // self.Hkv, 0,
                                    self.max_seq, self.Hkv * self.d, self.q, out, self.kc,
                                    self.vc, config=K.CudaConfig(stream))

    def gpu_pos(self, out, stream):
        K.flash_attention_decode_fp16_gpu_pos_cu(self.pos, self.Hq, self.Hkv, self.d,
                                                 self.Hq // self.Hkv, 0, self.max_seq,
                                                 self.Hkv * self.d, self.q, out, self.kc,
                                                 self.vc, config=K.CudaConfig(stream))

    def new_out(self):
        return torch.full((self.Hq * self.d,), float("nan"), device="cuda", dtype=torch.float16)


class SplitPrefill:
    """C2-shape causal prefill (S 2048, 12 q / 2 kv heads): few enough query blocks that
    the launch splits keys into the library's prefill workspace."""

    def __init__(self, rng, S=2048):
        self.S, self.Hq, self.Hkv, self.d = S, 12, 2, 128
        kv_dim = self.Hkv * self.d
        self.q = dev(quantize(normal(rng, (S, self.Hq * self.d)), "fp16"))
        self.kc = dev(quantize(normal(rng, (S, kv_dim)), "fp16"))
        self.vc = dev(quantize(normal(rng, (S, kv_dim)), "fp16"))
        assert K.prefill_workspace_size(0, S, self.Hq, self.Hkv, self.d, _lib.DTYPE_FP16) > 0

    def run(self, out, stream):
        K.flash_attention_prefill_cu(0, self.S, self.Hq, self.Hkv, self.d, self.Hq // self.Hkv,
                                     0, self.S, self.Hkv * self.d, self.q, out, self.kc,
                                     self.vc, config=K.CudaConfig(stream))

    def new_out(self):
        return torch.full_like(self.q, float("nan"))


def test_decode_and_split_prefill_on_two_streams():
    """Flash decodes on one stream and key-split prefills on another, queued without any
    synchronisation between them: every output equals the single-stream result bit for
    bit (one shared library buffer would mix the two calls' partials)."""
    rng = np.random.default_rng(31)
    dec, pre = Decode(rng), SplitPrefill(rng)
    main = torch.cuda.current_stream()
    positions = [4095, 3000, 2047, 4000, 1500, 3999]
    ref_d = []
    for p in positions:
        o = dec.new_out()
        dec.host_pos(p, o, main)
        ref_d.append(o)
    ref_p = pre.new_out()
    pre.run(ref_p, main)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    # outputs are filled (NaN) on the current stream and synchronised before use
    outs_d = [(i, dec.new_out()) for _ in range(3) for i in range(len(positions))]
    outs_p = [pre.new_out() for _ in range(3 * len(positions[::2]))]
    torch.cuda.synchronize()
    jp = 0
    for j, (i, o) in enumerate(outs_d):
        dec.host_pos(positions[i], o, sa)
        if i % 2 == 0:
            pre.run(outs_p[jp], sb)
            jp += 1
    torch.cuda.synchronize()
    for i, o in outs_d:
        assert torch.equal(o, ref_d[i]), f"decode at pos {positions[i]} differs across streams"
    for op in outs_p:
        assert torch.equal(op, ref_p), "key-split prefill differs across streams"


def test_captured_decode_survives_workspace_growth():
    """Capture a gpu-pos decode, then grow the same stream's library buffers (a key-split
    prefill and a decode over a 16x longer cache), then replay: the graph still reads and
    writes live memory and matches the eager decode bit for bit."""
    rng = np.random.default_rng(32)
    dec = Decode(rng)
    big = Decode(rng, max_seq=65536)
    pre = SplitPrefill(rng)
    cap = torch.cuda.Stream()
    K.reserve_decode_workspace(dec.Hq, dec.d, dec.max_seq, stream=cap)
    out = dec.new_out()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        dec.gpu_pos(out, cap)
    # eager work on the capture stream that needs more workspace than was reserved
    with torch.cuda.stream(cap):
        op = pre.new_out()
        pre.run(op, cap)
        ob = big.new_out()
        big.pos.fill_(60000)
        big.gpu_pos(ob, cap)
    torch.cuda.synchronize()
    assert not torch.isnan(op.float()).any() and not torch.isnan(ob.float()).any()
    for pos in [4095, 17, 2500]:
        dec.pos.fill_(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = dec.new_out()
        dec.host_pos(pos, eager, torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay at pos {pos} after workspace growth"


def test_capture_without_reserve_is_refused():
    """A capturing stream whose library buffer is missing gets ORIN_ERR_WORKSPACE and
    nothing is queued; after a reserve the same capture succeeds."""
    rng = np.random.default_rng(33)
    dec = Decode(rng, max_seq=8192)
    lib = _lib.load()
    cap = torch.cuda.Stream()
    out = dec.new_out()
    g = torch.cuda.CUDAGraph()
    status = []
    # the refused call queues nothing, so the first graph is empty by design
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty")
        with torch.cuda.graph(g, stream=cap):
            status.append(lib.orin_flash_attention_decode_gpu_pos(
                dec.pos.data_ptr(), dec.Hq, dec.Hkv, dec.d, dec.Hq // dec.Hkv, 0, dec.max_seq,
                dec.Hkv * dec.d, dec.q.data_ptr(), out.data_ptr(), dec.kc.data_ptr(),
                dec.vc.data_ptr(), _lib.DTYPE_FP16, C.c_void_p(cap.cuda_stream)))
    assert status == [_lib.ERR_WORKSPACE]
    K.reserve_decode_workspace(dec.Hq, dec.d, dec.max_seq, stream=cap)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=cap):
        dec.gpu_pos(out, cap)
    dec.pos.fill_(8000)
    torch.cuda.synchronize()
    g2.replay()
    torch.cuda.synchronize()
    eager = dec.new_out()
    dec.host_pos(8000, eager, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert torch.equal(out, eager)


def test_device_length_past_launch_bound_is_nan():
    """Paged decode with one context length above max_context_len: that row is NaN (not
    attention over a truncated prefix); the other rows equal a launch sized for all."""
    rng = np.random.default_rng(34)
    B, Hq, Hkv, d, bs = 3, 8, 2, 128, 16
    lens = np.array([100, 300, 200], np.int32)
    nblk = 32
    kp = dev(quantize(normal(rng, (B * nblk, bs, Hkv, d)), "fp16"))
    vp = dev(quantize(normal(rng, (B * nblk, bs, Hkv, d)), "fp16"))
    bt = torch.from_numpy(np.arange(B * nblk, dtype=np.int32).reshape(B, nblk)).cuda()
    q = dev(quantize(normal(rng, (B, Hq, d)), "fp16"))
    cl = torch.from_numpy(lens).cuda()
    o_ok = torch.zeros(B, Hq, d, device="cuda", dtype=torch.float16)
    K.paged_decode_cu(q, kp, vp, o_ok, bt, cl, 512, split_tokens=128)
    o_cut = torch.zeros_like(o_ok)
    K.paged_decode_cu(q, kp, vp, o_cut, bt, cl, 256, split_tokens=128)
    torch.cuda.synchronize()
    assert torch.isnan(o_cut[1].float()).all()
    assert torch.equal(o_cut[0], o_ok[0]) and torch.equal(o_cut[2], o_ok[2])
    # kuiper gpu-pos decode with *pos_ptr >= max_seq_len
    dec = Decode(rng, max_seq=1024)
    dec.pos.fill_(1024)
    out = dec.new_out().zero_()
    dec.gpu_pos(out, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_release_stream():
    """orin_attn_workspace_release_stream frees one stream's buffers (a later call on that
    stream allocates again and gives the same bits) and is refused, freeing nothing, while
    that stream is being captured; orin_attn_workspace_release is refused likewise."""
    rng = np.random.default_rng(34)
    dec = Decode(rng)
    lib = _lib.load()
    s = torch.cuda.Stream()
    first, again = dec.new_out(), dec.new_out()
    dec.host_pos(3000, first, s)
    torch.cuda.synchronize()
    assert lib.orin_attn_workspace_release_stream(C.c_void_p(s.cuda_stream)) == _lib.OK
    dec.host_pos(3000, again, s)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    K.reserve_decode_workspace(dec.Hq, dec.d, dec.max_seq, stream=s)
    out = dec.new_out()
    g = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(g, stream=s):
        dec.gpu_pos(out, s)
        status.append(lib.orin_attn_workspace_release_stream(C.c_void_p(s.cuda_stream)))
        status.append(lib.orin_attn_workspace_release())
    assert status == [_lib.ERR_WORKSPACE, _lib.ERR_WORKSPACE]
    dec.pos.fill_(3000)
    torch.cuda.synchronize()
    g.replay()  # the buffers survived the refused releases
    torch.cuda.synchronize()
    assert torch.equal(out, first)
    del g
    torch.cuda.synchronize()
    # the Python mirror of both entry points, outside capture
    K.release_workspace(s)
    K.release_workspace(all_streams=True)
    dec.host_pos(3000, again, s)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    assert lib.orin_attn_workspace_release_stream(C.c_void_p(s.cuda_stream)) == _lib.OK


def test_host_threads_on_their_own_streams():
    """Four host threads, each on its own stream, run growing flash decodes and key-split
    prefills concurrently (the library call releases the GIL): every output equals the
    same launch run alone, so the per-stream buffers, the first-use kernel attributes and
    the buffer growth are safe under concurrent callers."""
    import threading
    rng = np.random.default_rng(35)
    decs = [Decode(rng, max_seq=8192) for _ in range(4)]
    pre = SplitPrefill(rng)
    positions = [300, 2000, 5000, 8000]
    ref_dec = {}
    for i, d in enumerate(decs):
        for p in positions:
            o = d.new_out()
            d.host_pos(p, o, torch.cuda.current_stream())
            ref_dec[(i, p)] = o
    ref_pre = pre.new_out()
    pre.run(ref_pre, torch.cuda.current_stream())
    torch.cuda.synchronize()
    K.release_workspace(all_streams=True)  # the threads grow their buffers from nothing
    errors, results = [], {}

    def work(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for rep in range(3):
                    for p in positions:
                        o = decs[i].new_out()
                        decs[i].host_pos(p, o, s)
                        results[(i, p, rep)] = o
                    op = pre.new_out()
                    pre.run(op, s)
                    results[(i, "pre", rep)] = op
            s.synchronize()
            K.release_workspace(s)
        except Exception as e:  # surfaced by the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(4):
        for rep in range(3):
            for p in positions:
                assert torch.equal(results[(i, p, rep)], ref_dec[(i, p)]), (i, p, rep)
            assert torch.equal(results[(i, "pre", rep)], ref_pre), (i, rep)
