"""The C3 fp16 prefill on four kinds of input (seeded N(0,1) as in bench.py, V = 0, Q = K = 0,
all zero), 10 x 200 launches each after 200 untimed ones, with rocm-smi sampling the clock:
the same instruction stream whose time moves with the data it multiplies shows how far the
launch is held by the board's power limit rather than by its schedule.

Usage (on the GPU box): python orinmllm_amd/microbench/prefill_power.py
"""
import sys, os, json, time, subprocess, threading, statistics
import torch
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
import bench
from orinmllm_amd import kernel as K
gen = torch.Generator(device="cuda"); gen.manual_seed(11)
s = torch.cuda.current_stream()
pf = bench.make_prefill(torch.float16, gen)
S, Hq, Hkv, d = pf["S"], pf["Hq"], pf["Hkv"], pf["d"]
def run(q, k, v):
    K.flash_attention_prefill_cu(0, S, Hq, Hkv, d, Hq // Hkv, 0, S, Hkv * d, q, pf["o"], k, v)
samples = []
def sampler(stop):
    while not stop.is_set():
        try:
            out = subprocess.run(["rocm-smi", "--showpower", "--showclocks", "--json"], capture_output=True, text=True, timeout=5).stdout
            samples.append(out)
        except Exception as e:
            samples.append(str(e))
        time.sleep(0.2)
cases = {"random": (pf["q"], pf["k"], pf["v"]), "v_zero": (pf["q"], pf["k"], torch.zeros_like(pf["v"])),
         "all_zero": (torch.zeros_like(pf["q"]), torch.zeros_like(pf["k"]), torch.zeros_like(pf["v"])),
         "qk_zero": (torch.zeros_like(pf["q"]), torch.zeros_like(pf["k"]), pf["v"])}
for name, (q, k, v) in list(cases.items()) + [("random_again", cases["random"])]:
    for _ in range(200): run(q, k, v)
    torch.cuda.synchronize()
    samples.clear(); stop = threading.Event(); th = threading.Thread(target=sampler, args=(stop,)); th.start()
    r = [bench.per_launch(lambda: run(q, k, v), 200, 10, s)["median_ms"] * 1e3 for _ in range(10)]
    stop.set(); th.join()
    pw, clk = [], []
    for o in samples:
        try:
            j = json.loads(o)
            for card, vals in j.items():
                for kk, vv in vals.items():
                    if "Power" in kk and "(W)" in kk: pw.append(float(vv))
                    if kk.startswith("sclk"): clk.append(vv)
        except Exception:
            pass
    print(json.dumps({"case": name, "us_med": round(statistics.median(r), 1), "us_all": [round(x, 1) for x in r], "power_W": pw[:8], "sclk": clk[:6], "n_samples": len(samples)}), flush=True)
