"""Benchmark of the attention hot path on one MI355X.

One step = one Qwen3-8B-shape causal GQA prefill (S 4096, 32 q / 8 kv
heads, d 128, fp16, Q/K after per-head RMSNorm + RoPE) followed by one batch-32 paged
decode (config 4: 32 q / 8 kv heads, d 128, KV lengths U[512, 4096], block 16, fp16).

`value` is the prefill throughput in TFLOP/s (algorithmic FLOPs 4*d*Hq*S(S+1)/2 per
call); the decode KV-read bandwidth (4096 * sum(L) bytes per call) is reported under
`decode`.  Inputs are synthetic and resident in HBM before timing starts.  The decode
reads one of several KV pools in rotation so that the 256 MB last-level cache does not
serve it.  Each kernel's time is the median of at least 50 launches, each bracketed by
its own pair of HIP events on the stream the kernels run on, after at least 10 warmups
(the mean is reported beside it); `ms_per_step` is the wall time of the K timed steps.

The CPU baseline runs the oracle (oracle/oracle.c, a restatement of the reference's CPU
MHA) on a bounded sample of the same workload on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, TFLOP/s


def _bytes(t):
    """HBM bytes per launch (read + written) from the calibrated rocprof counters."""
    return None if not t else t["read_bytes"] + t["write_bytes"]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-producers", action="store_true",
                    help="skip the timing of the KV-write / Q-K producer kernels")
    ap.add_argument("--pools", type=int, default=4, help="KV pools rotated by the decode")
    ap.add_argument("--reps", type=int, default=100,
                    help="per-launch timings behind the reported medians (at least 50 used)")
    ap.add_argument("--kernel-warmup", type=int, default=10,
                    help="untimed launches before the per-launch timings (at least 10 used)")
    ap.add_argument("--no-decode-4096", action="store_true",
                    help="skip the decode with every KV length 4096")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the C1 / C2 / C3-bf16 / C5 timings")
    ap.add_argument("--no-pipeline", action="store_true",
                    help="skip the C3 producer + prefill + wo pipeline timings")
    ap.add_argument("--only-other-configs", action="store_true",
                    help="time only the C1 / C2 / C3-bf16 / C5 configs and print them as one "
                         "JSON object (for profiling those kernels; not the bench line)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="also run one 512 MiB device copy (the reference traffic for the "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def rmsnorm_rope(x, H, d, theta=1e6):
    """Per-head RMSNorm (unit weight, eps 1e-6) then rotate-half RoPE, on the GPU (input
    synthesis only)."""
    import torch
    S = x.shape[0]
    x = x.view(S, H, d).float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    half = d // 2
    freq = 1.0 / theta ** (torch.arange(0, half, device=x.device, dtype=torch.float32) * 2 / d)
    ang = torch.arange(S, device=x.device, dtype=torch.float32)[:, None] * freq[None]
    c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    x0, x1 = x[..., :half], x[..., half:]
    return torch.cat([c * x0 - s * x1, c * x1 + s * x0], -1).reshape(S, H * d)


def make_prefill(dtype, gen):
    import torch
    S, Hq, Hkv, d = 4096, 32, 8, 128
    dev = "cuda"
    q = rmsnorm_rope(torch.randn(S, Hq * d, device=dev, generator=gen), Hq, d).to(dtype)
    k = rmsnorm_rope(torch.randn(S, Hkv * d, device=dev, generator=gen), Hkv, d).to(dtype)
    v = torch.randn(S, Hkv * d, device=dev, generator=gen).to(dtype)
    o = torch.empty_like(q)
    flops = 4.0 * d * Hq * S * (S + 1) / 2
    return dict(S=S, Hq=Hq, Hkv=Hkv, d=d, q=q, k=k, v=v, o=o, flops=flops)


def make_decode(dtype, gen, pools, layout=1, uniform_len=None):
    """C4 inputs: KV lengths U[512, 4096] (seeded), or all equal to uniform_len."""
    import numpy as np
    import torch
    B, Hq, Hkv, d, bs = 32, 32, 8, 128, 16
    rng = np.random.default_rng(0xC4)
    lens = rng.integers(512, 4097, B).astype(np.int32)
    if uniform_len is not None:
        lens = np.full(B, uniform_len, np.int32)
    nblk = (lens + bs - 1) // bs
    total = int(nblk.sum())
    maxb = int(nblk.max())
    bt = np.zeros((B, maxb), np.int32)
    perm = rng.permutation(total).astype(np.int32)
    off = 0
    for b in range(B):
        bt[b, : nblk[b]] = perm[off: off + nblk[b]]
        off += nblk[b]
    shape = (total, bs, Hkv, d) if layout == 0 else (total, Hkv, bs, d)
    kp = [torch.randn(*shape, device="cuda", generator=gen).to(dtype) for _ in range(pools)]
    vp = [torch.randn(*shape, device="cuda", generator=gen).to(dtype) for _ in range(pools)]
    q = torch.randn(B, Hq, d, device="cuda", generator=gen).to(dtype)
    o = torch.empty_like(q)
    kv_bytes = 2 * int(lens.sum()) * Hkv * d * 2  # K and V, read once per kv head
    return dict(B=B, Hq=Hq, Hkv=Hkv, d=d, bs=bs, lens=lens, layout=layout, lens_d=torch.from_numpy(lens).cuda(),
                bt=torch.from_numpy(bt).cuda(), kp=kp, vp=vp, q=q, o=o, kv_bytes=kv_bytes,
                maxlen=int(lens.max()))


def time_decode_uniform(K, dtype, gen, pools, reps=50):
    """The batch-32 paged decode with every KV length 4096 (the length the decode target
    is stated at), timed like the C4 decode: automatic split size (from max_context_len
    alone), the split orin_attn_decode_split_tokens_for_total picks from the batch's total
    length (a serving loop knows it on the host), and 1024-token splits passed explicitly."""
    import torch
    dc = make_decode(dtype, gen, pools, uniform_len=4096)
    stream = torch.cuda.current_stream()
    out = {"kv_bytes_per_call": dc["kv_bytes"]}
    hint = K.decode_split_tokens_for_total(dc["B"], dc["Hq"], dc["Hkv"], dc["maxlen"],
                                           int(dc["lens"].sum()))
    for name, st in [("auto_split", 0), ("split_for_total", hint), ("split_1024", 1024)]:
        nb = K.decode_workspace_size(dc["B"], dc["Hq"], dc["Hkv"], dc["d"], dc["maxlen"], st)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")

        def run(i):
            p = i % pools
            K.paged_decode_cu(dc["q"], dc["kp"][p], dc["vp"][p], dc["o"], dc["bt"],
                              dc["lens_d"], dc["maxlen"], split_tokens=st, workspace=ws,
                              layout=dc["layout"])

        ms = per_launch(run, reps, 10, stream, indexed=True)["median_ms"]
        gbs = dc["kv_bytes"] / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "split_tokens": st}
    del dc
    torch.cuda.empty_cache()
    return out


def time_other_configs(K, gen, reps=50):
    """The other BASELINE configs on their own (parity-test shapes; not part of `value`):
    C1 fp32 single-sequence decode, C2 fp16 causal prefill (S 2048, 12 q / 2 kv heads),
    C3 in bf16, and C5 bf16 varlen vision attention (4 x 1024 patches, 16 heads, d 72).
    Median time over `reps` calls, each bracketed by HIP events on the current stream."""
    import torch
    stream = torch.cuda.current_stream()

    def timeit(fn):
        return per_launch(fn, reps, 10, stream)["median_ms"]

    out = {}
    # C1: 12 = 12 heads, d 64, query at position 255 of a 256-row fp32 cache.
    H, d1, seq = 12, 64, 256
    q1 = torch.randn(H * d1, device="cuda", generator=gen)
    k1 = torch.randn(1, seq, H * d1, device="cuda", generator=gen)
    v1 = torch.randn_like(k1)
    o1 = torch.empty_like(q1)
    sc = torch.empty(H, seq, device="cuda")
    ms = timeit(lambda: K.mha_kernel_cu(255, H, 0, seq, H * d1, 1, d1, o1, q1, sc, k1, v1))
    kvb = 2 * seq * H * d1 * 4
    out["c1_decode_fp32"] = {"us": round(ms * 1e3, 2), "GB/s": round(kvb / (ms * 1e-3) / 1e9, 1)}
    # C2: causal prefill S 2048, 12 q / 2 kv heads, d 128, fp16.
    S, Hq, Hkv, d = 2048, 12, 2, 128
    q2 = rmsnorm_rope(torch.randn(S, Hq * d, device="cuda", generator=gen), Hq, d).half()
    k2 = rmsnorm_rope(torch.randn(S, Hkv * d, device="cuda", generator=gen), Hkv, d).half()
    v2 = torch.randn(S, Hkv * d, device="cuda", generator=gen).half()
    o2 = torch.empty_like(q2)
    ms = timeit(lambda: K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d,
                                                     q2, o2, k2, v2))
    fl = 4.0 * d * Hq * S * (S + 1) / 2
    tf = fl / (ms * 1e-3) / 1e12
    out["c2_prefill_fp16"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                              "frac_mfma": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    # C3 in bf16.
    pf = make_prefill(torch.bfloat16, gen)
    ms = timeit(lambda: K.flash_attention_prefill_cu(0, pf["S"], pf["Hq"], pf["Hkv"], pf["d"],
                                                     pf["Hq"] // pf["Hkv"], 0, pf["S"],
                                                     pf["Hkv"] * pf["d"], pf["q"], pf["o"],
                                                     pf["k"], pf["v"]))
    tf = pf["flops"] / (ms * 1e-3) / 1e12
    out["c3_prefill_bf16"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                              "frac_mfma": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    # C5: bf16 vision, 4 images x 1024 patches, 16 heads, d 72, bidirectional.
    Hv, dv, N = 16, 72, 4096
    qv, kv, vv = (torch.randn(Hv, N, dv, device="cuda", generator=gen).bfloat16()
                  for _ in range(3))
    ov = torch.empty(N, Hv * dv, device="cuda", dtype=torch.bfloat16)
    cu = torch.tensor([0, 1024, 2048, 3072, 4096], dtype=torch.int32, device="cuda")
    ms = timeit(lambda: K.vision_attention_varlen_cu(qv, kv, vv, ov, cu, 1024, Hv, dv))
    fl = 4.0 * 4 * 1024 * 1024 * dv * Hv
    tf = fl / (ms * 1e-3) / 1e12
    out["c5_vision_bf16"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                             "frac_mfma": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    return out


def make_producers(dtype, gen):
    """Inputs of the kernels either side of the path, at the bench shapes: the Qwen3 Q/K
    producer for the C3 prefill (4096 tokens, 32 q / 8 kv heads), a paged KV write of
    the same 4096 tokens (head-major pool, block 16), and the vision QKV split + rotary
    for C5 (4 x 1024 patches, 16 heads, d 72)."""
    import torch
    S, Hq, Hkv, d = 4096, 32, 8, 128
    dev = "cuda"
    p = {}
    p["q"] = torch.randn(S, Hq * d, device=dev, generator=gen).to(dtype)
    p["k"] = torch.randn(S, Hkv * d, device=dev, generator=gen).to(dtype)
    p["v"] = torch.randn(S, Hkv * d, device=dev, generator=gen).to(dtype)
    p["wq"] = torch.ones(d, device=dev, dtype=dtype)
    p["wk"] = torch.ones(d, device=dev, dtype=dtype)
    p["sin"] = torch.empty(S, d, device=dev)
    p["cos"] = torch.empty(S, d, device=dev)
    p["kc"] = torch.empty(1, S, Hkv * d, device=dev, dtype=dtype)
    p["vc"] = torch.empty_like(p["kc"])
    e = torch.tensor([], dtype=dtype).element_size()
    # q read + written, k and v read, k and v cache rows written, sin/cos tables read
    p["norm_rope_bytes"] = (2 * S * Hq * d + 4 * S * Hkv * d) * e + 2 * S * d * 4
    bs = 16
    nblk = S // bs
    p["kpool"] = torch.empty(nblk, Hkv, bs, d, device=dev, dtype=dtype)
    p["vpool"] = torch.empty_like(p["kpool"])
    perm = torch.randperm(nblk, device=dev, generator=gen).to(torch.int32)
    t = torch.arange(S, device=dev, dtype=torch.int32)
    p["slots"] = (perm[t // bs] * bs + t % bs).to(torch.int32)
    p["scatter_bytes"] = 4 * S * Hkv * d * e  # K and V rows read and written
    N, H, dv = 4096, 16, 72
    p["qkv"] = torch.randn(N, 3 * H * dv, device=dev, generator=gen).to(dtype)
    p["vcos"] = torch.randn(N, dv, device=dev, generator=gen).to(dtype)
    p["vsin"] = torch.randn(N, dv, device=dev, generator=gen).to(dtype)
    p["vout"] = [torch.empty(H, N, dv, device=dev, dtype=dtype) for _ in range(3)]
    p["vision_bytes"] = (2 * N * 3 * H * dv + 2 * N * dv) * e
    p["shape"] = (S, Hq, Hkv, d, N, H, dv)
    return p


def time_producers(K, p, reps=50):
    """Median time (per-launch HIP events on the stream the kernels run on) and HBM GB/s."""
    import torch
    from orinmllm_amd import _lib
    S, Hq, Hkv, d, N, H, dv = p["shape"]
    K.sin_cos_cache_calc_cu(d, S, p["sin"], p["cos"], 1e6)
    K.kv_cache_write_paged(p["k"].view(S, Hkv, d), p["v"].view(S, Hkv, d), p["kpool"], p["vpool"],
                           p["slots"], layout=K.KV_LAYOUT_HEAD_MAJOR)  # argument checks
    kvw = _lib.load().orin_kv_cache_write_paged
    kvw_args = (p["k"].data_ptr(), p["v"].data_ptr(), Hkv * d, p["kpool"].data_ptr(),
                p["vpool"].data_ptr(), p["slots"].data_ptr(), S, Hkv, d, p["kpool"].shape[2],
                K.KV_LAYOUT_HEAD_MAJOR, K._dtype(p["k"], p["v"], p["kpool"], p["vpool"]),
                torch.cuda.current_stream().cuda_stream)
    calls = {
        "qk_norm_rope_c3": (lambda: K.qk_norm_rope_cu(
            p["q"], p["k"], p["v"], p["wq"], p["wk"], p["sin"], p["cos"], p["kc"], p["vc"], 0, S,
            0, S, Hq, Hkv, d), p["norm_rope_bytes"]),
        # The C-ABI entry point called directly with its arguments prepared once, as the C++
        # host layer calls it: the 5-6 us kernel is shorter than the Python wrapper's checks.
        "kv_write_paged_4096": (lambda: _lib.check("orin_kv_cache_write_paged", kvw(*kvw_args)),
                                p["scatter_bytes"]),
        "vision_split_rope_c5": (lambda: K.fused_split_rope_transpose_cu(
            p["qkv"], p["vcos"], p["vsin"], *p["vout"], N, H, dv), p["vision_bytes"]),
    }
    stream = torch.cuda.current_stream()
    out = {}
    for name, (fn, nbytes) in calls.items():
        ms = per_launch(fn, reps, 10, stream)["median_ms"]
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "GB/s": round(gbs, 1),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def per_launch(fn, reps, warmup, stream, indexed=False):
    """Median and mean of `reps` launches of fn, each bracketed by its own pair of HIP
    events on `stream`, after `warmup` untimed launches.  A short device-side spin is
    queued first so the host runs ahead of the device and the event pairs do not include
    host launch time."""
    import statistics

    import torch
    call = (lambda i: fn(i)) if indexed else (lambda i: fn())
    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    try:
        torch.cuda._sleep(20_000_000)
    except Exception:
        pass
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        call(warmup + i)
        b.record(stream)
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) for a, b in ev]
    return {"median_ms": round(statistics.median(ts), 5), "mean_ms": round(sum(ts) / len(ts), 5),
            "min_ms": round(min(ts), 5), "max_ms": round(max(ts), 5)}


def time_fused_pipeline(K, dtype, gen, reps=50):
    """The C3 prefill from raw Q/K/V (Qwen3 producer + attention), two ways: the producer on
    Q, K and V followed by the prefill, and the producer on K and V only followed by the
    prefill with the Q producer fused into its Q load.  Median per-launch times of each
    kernel (HIP events on the current stream) and of the pair."""
    import torch
    S, Hq, Hkv, d = 4096, 32, 8, 128
    dev = "cuda"
    q = torch.randn(S, Hq * d, device=dev, generator=gen).to(dtype)
    k = torch.randn(S, Hkv * d, device=dev, generator=gen).to(dtype)
    v = torch.randn(S, Hkv * d, device=dev, generator=gen).to(dtype)
    wq = (1 + 0.1 * torch.randn(d, device=dev, generator=gen)).to(dtype)
    wk = (1 + 0.1 * torch.randn(d, device=dev, generator=gen)).to(dtype)
    sn = torch.empty(S, d, device=dev)
    cs = torch.empty(S, d, device=dev)
    K.sin_cos_cache_calc_cu(d, S, sn, cs, 1e6)
    kc = torch.empty(1, S, Hkv * d, device=dev, dtype=dtype)
    vc = torch.empty_like(kc)
    qw = q.clone()  # the producer normalises and rotates it in place
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    prod_qkv = lambda: K.qk_norm_rope_cu(qw, k, v, wq, wk, sn, cs, kc, vc, 0, S, 0, S, Hq, Hkv, d)
    prod_kv = lambda: K.qk_norm_rope_cu(None, k, v, None, wk, sn, cs, kc, vc, 0, S, 0, S, Hq, Hkv, d)
    attn = lambda: K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d, qw, o,
                                                kc, vc)
    fused = lambda: K.flash_attention_prefill_qk_norm_rope_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S,
                                                              Hkv * d, q, o, kc, vc, wq, sn, cs)
    wo = (torch.randn(Hq * d, Hq * d, device=dev, generator=gen) / (Hq * d) ** 0.5).to(dtype)
    y = torch.empty_like(q)
    proj = lambda: K.batched_matmul_kernel_cu(o, wo, y, S)
    t = {name: per_launch(fn, reps, 10, stream)["median_ms"] * 1e3
         for name, fn in [("producer_qkv", prod_qkv), ("prefill", attn), ("producer_kv", prod_kv),
                          ("prefill_fused_q", fused), ("wo_projection", proj)]}
    wo_tflops = 2.0 * S * (Hq * d) ** 2 / (t["wo_projection"] * 1e-6) / 1e12
    return {"two_pass_us": round(t["producer_qkv"] + t["prefill"], 2),
            "fused_us": round(t["producer_kv"] + t["prefill_fused_q"], 2),
            "kernels_us": {n: round(x, 2) for n, x in t.items()},
            "wo_projection_TFLOP/s": round(wo_tflops, 1)}


def time_decode_pipeline(K, dtype, gen, dc, ws, pools, reps=50):
    """The C4 decode step followed by its wo projection (kuiper/source/model/qwen_base.cpp:
    464-474): attention output [32, 4096] x wo [4096, 4096]^T.  Median per-launch times of
    the decode, of the projection, and of the two back to back in one event pair; the
    projection is bound by reading wo (32 MB), the attention output round trip between the
    two launches is 2 x 256 KB."""
    import torch
    B, n = dc["B"], dc["Hq"] * dc["d"]
    wo = (torch.randn(n, n, device="cuda", generator=gen) / n ** 0.5).to(dtype)
    y = torch.empty(B, n, device="cuda", dtype=dtype)
    stream = torch.cuda.current_stream()

    def dec(i):
        p = i % pools
        K.paged_decode_cu(dc["q"], dc["kp"][p], dc["vp"][p], dc["o"], dc["bt"], dc["lens_d"],
                          dc["maxlen"], workspace=ws, layout=dc["layout"])

    def proj():
        K.batched_matmul_kernel_cu(dc["o"].view(B, n), wo, y, B)

    def both(i):
        dec(i)
        proj()

    t_dec = per_launch(dec, reps, 10, stream, indexed=True)["median_ms"] * 1e3
    t_proj = per_launch(proj, reps, 10, stream)["median_ms"] * 1e3
    t_both = per_launch(both, reps, 10, stream, indexed=True)["median_ms"] * 1e3
    return {"decode_us": round(t_dec, 2), "wo_us": round(t_proj, 2), "decode_then_wo_us": round(t_both, 2),
            "wo_GB/s": round(2 * n * n / (t_proj * 1e-6) / 1e9, 1),
            "attn_out_roundtrip_bytes": 2 * B * n * 2}


def cpu_baseline(pf, dc, min_seconds=8.0):
    """Time the oracle (all host cores, OpenMP over query rows) on the full C3 prefill and
    the full C4 decode, repeating each until it has run about min_seconds."""
    import numpy as np
    from oracle import oracle

    threads = oracle.max_threads()
    S, Hq, Hkv, d = pf["S"], pf["Hq"], pf["Hkv"], pf["d"]
    q = pf["q"].float().cpu().numpy()
    k = pf["k"].float().cpu().numpy()
    v = pf["v"].float().cpu().numpy()
    oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, rows=np.arange(4), nthreads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while reps < 20 and (reps == 0 or time.perf_counter() - t0 < min_seconds):
        oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, nthreads=threads)
        reps += 1
    t_total = time.perf_counter() - t0
    t_pf = t_total / reps
    flops = pf["flops"]

    nseq = dc["B"]
    kp = dc["kp"][0].float().cpu().numpy()
    vp = dc["vp"][0].float().cpu().numpy()
    if dc["layout"] == 1:  # the oracle takes token-major pools
        kp = np.ascontiguousarray(kp.transpose(0, 2, 1, 3))
        vp = np.ascontiguousarray(vp.transpose(0, 2, 1, 3))
    qd = dc["q"][:nseq].float().cpu().numpy()
    bt = dc["bt"][:nseq].cpu().numpy()
    lens = dc["lens"][:nseq]
    dreps, t0 = 0, time.perf_counter()
    while dreps < 200 and (dreps == 0 or time.perf_counter() - t0 < min_seconds / 4):
        oracle.decode_paged(qd, kp, vp, bt, lens, nthreads=threads)
        dreps += 1
    t_dc = (time.perf_counter() - t0) / dreps
    kv_bytes = 2 * int(lens.sum()) * Hkv * d * 2

    # One core, as the reference's CPU path runs: every 8th query row of the C3 prefill
    # and the first 4 C4 sequences.
    rows = np.arange(0, S, 8)
    t0 = time.perf_counter()
    oracle.prefill_causal(0, q, k, v, Hq, Hkv, d, rows=rows, nthreads=1)
    t1_pf = time.perf_counter() - t0
    flops1 = float(np.sum(4.0 * d * Hq * (rows + 1)))
    t0 = time.perf_counter()
    oracle.decode_paged(qd[:4], kp, vp, bt[:4], lens[:4], nthreads=1)
    t1_dc = time.perf_counter() - t0
    bytes1 = 2 * int(lens[:4].sum()) * Hkv * d * 2
    return {
        "value": flops / t_pf / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"the full C3 causal prefill ({S} rows x {Hq} heads), fp32 oracle on "
                  f"fp16-valued inputs, OpenMP over rows, {reps} runs in {t_total:.1f} s",
        "decode": {"value": kv_bytes / t_dc / 1e9, "unit": "GB/s",
                   "sample": f"the full C4 paged decode ({nseq} sequences), {dreps} runs, "
                             f"{t_dc * 1e3:.1f} ms each"},
        "single_thread": {
            "prefill_TFLOP/s": flops1 / t1_pf / 1e12, "decode_GB/s": bytes1 / t1_dc / 1e9,
            "cores": 1,
            "sample": f"{len(rows)} query rows (every 8th) of C3 in {t1_pf:.1f} s; 4 of the C4 "
                      f"sequences in {t1_dc * 1e3:.0f} ms"},
    }


def main():
    args = parse()
    args.reps = max(args.reps, 50)
    args.kernel_warmup = max(args.kernel_warmup, 10)
    traffic = {}
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(every box has one MI355X; the multi-GPU path is a design, not a build)",
              file=sys.stderr)
        return 2
    import torch
    from orinmllm_amd import kernel as K

    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC3)
    if args.only_other_configs:
        print(json.dumps({"other_configs": time_other_configs(K, gen, reps=args.reps)}))
        return 0
    pf = make_prefill(dtype, gen)
    dc = make_decode(dtype, gen, args.pools)
    ws_bytes = K.decode_workspace_size(dc["B"], dc["Hq"], dc["Hkv"], dc["d"], dc["maxlen"])
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def prefill():
        K.flash_attention_prefill_cu(0, pf["S"], pf["Hq"], pf["Hkv"], pf["d"], pf["Hq"] // pf["Hkv"],
                                     0, pf["S"], pf["Hkv"] * pf["d"], pf["q"], pf["o"], pf["k"],
                                     pf["v"])

    def decode(i):
        p = i % args.pools
        K.paged_decode_cu(dc["q"], dc["kp"][p], dc["vp"][p], dc["o"], dc["bt"], dc["lens_d"],
                          dc["maxlen"], workspace=ws, layout=dc["layout"])

    for i in range(args.warmup):
        prefill()
        decode(i)
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        e = ev[i]
        e[0].record(stream)
        prefill()
        e[1].record(stream)
        e[2].record(stream)
        decode(args.warmup + i)
        e[3].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    step_pf_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    step_dc_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / args.steps
    # Per-kernel figures: median of >= 50 per-launch event pairs after >= 10 warmups.
    reps = max(args.reps, args.steps)
    pf_t = per_launch(prefill, reps, args.kernel_warmup, stream)
    dc_t = per_launch(lambda i: decode(i), reps, args.kernel_warmup, stream, indexed=True)
    pf_ms, dc_ms = pf_t["median_ms"], dc_t["median_ms"]
    pf_tflops = pf["flops"] / (pf_ms * 1e-3) / 1e12
    dc_gbs = dc["kv_bytes"] / (dc_ms * 1e-3) / 1e9

    out = {
        "metric": "attn prefill TFLOP/s + decode KV GB/s (Qwen3-8B GQA fp16), 1 MI355X",
        "value": round(pf_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.dtype == "fp16" else "bf16",
        "data": "synthetic (seeded N(0,1); Q/K RMSNorm+RoPE)",
        "config": {
            "workload": "C3 causal GQA prefill S=4096 Hq=32 Hkv=8 d=128 + C4 paged decode "
                        "B=32 Hq=32 Hkv=8 d=128 L~U[512,4096] block 16",
            "prefill_ms": round(pf_ms, 4),
            "decode_ms": round(dc_ms, 4),
            "timing": {
                "value_is": "median over per-launch HIP event pairs",
                "reps": reps, "warmup": args.kernel_warmup,
                "prefill": pf_t, "decode": dc_t,
                "timed_steps_mean_ms": {"prefill": round(step_pf_ms, 4),
                                        "decode": round(step_dc_ms, 4)},
            },
            "kv_pools_rotated": args.pools,
            "traffic_source": traffic.get("source"),
        },
        "roofline": {
            "bound": "mfma", "achieved": round(pf_tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(pf_tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": _bytes(traffic.get("fwd_causal_c3")),
        },
        "decode": {
            "metric": "paged decode KV-read GB/s", "value": round(dc_gbs, 1), "unit": "GB/s",
            "kv_bytes_per_call": dc["kv_bytes"],
            "roofline": {"bound": "hbm", "achieved": round(dc_gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(dc_gbs / HBM_PEAK_GBS, 4),
                         "traffic": _bytes(traffic.get("decode_paged_c4"))},
        },
    }
    if not args.no_decode_4096:
        out["decode_kv4096"] = time_decode_uniform(K, dtype, gen, args.pools)
    if not args.no_other_configs:
        out["other_configs"] = time_other_configs(K, gen)
    if not args.no_producers and not args.no_pipeline:
        out["c3_pipeline"] = time_fused_pipeline(K, dtype, gen)
    if not args.no_pipeline:
        out["decode_pipeline"] = time_decode_pipeline(K, dtype, gen, dc, ws, args.pools)
    if not args.no_producers:
        out["producers"] = time_producers(K, make_producers(dtype, gen))
        for name, rec in out["producers"].items():
            rec["traffic"] = _bytes(traffic.get(name))
    if args.calibration_copy:
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(pf, dc)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
