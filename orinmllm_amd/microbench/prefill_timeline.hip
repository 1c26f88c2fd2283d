// Per-workgroup timeline of the ping-pong prefill (fwd_pp_kernel) on C2, C3 and the C5
// vision shape (bidirectional, d 64 / 72 / 128), fp16.
//
// fwd_pp.hip is compiled into this program with ORIN_PP_TIMELINE, which makes wave 0 of
// every workgroup stamp the 100 MHz wall clock at entry, when its first K/V stage has
// landed and at main-loop entry, and every wave at the end of its tiles (the stores of O
// follow).  Inputs are seeded N(0,1) fp16; each shape runs 20 untimed launches, then one
// recorded launch.  Printed per distinct tile count: workgroups, mean duration, the three
// prologue stamps, and a least-squares fit duration = a * tiles + b (b = the fixed cost a
// workgroup pays whatever its work: argument fetch, Q load, the first stages' latency, the
// pipeline's fill and drain steps).  Then, for steps 12-15 of waves 0 and 4 (one of each
// ping-pong group, on one SIMD), the shader clocks of the wave's own phase work and of the
// whole step up to its barrier, split by the phase the wave ran (MFMA or softmax).
//
// Build and run: python orinmllm_amd/microbench/run.py prefill_timeline
#include "fwd_pp.hip"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <vector>

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

static void fill_normal(std::vector<orin::f16>& x, unsigned long long seed) {
  unsigned long long s = seed * 0x9E3779B97F4A7C15ull + 1;
  auto next = [&]() {  // xorshift64*, uniform in (0, 1)
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return ((s * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0) + 1e-300;
  };
  for (size_t i = 0; i < x.size(); i += 2) {  // Box-Muller
    const double r = sqrt(-2.0 * log(next())), t = 6.283185307179586 * next();
    x[i] = (orin::f16)(r * cos(t));
    if (i + 1 < x.size()) x[i + 1] = (orin::f16)(r * sin(t));
  }
}

// causal: one sequence of S tokens; otherwise n_seg bidirectional segments of S tokens each
// (the vision layout, cu_seqlens = 0, S, 2S, ...).
static void run_shape(const char* name, int S, int Hq, int Hkv, int d, int n_cu, int n_seg = 0) {
  const bool causal = n_seg == 0;
  const int n_tok = causal ? S : S * n_seg;
  const size_t nq = (size_t)n_tok * Hq * d, nkv = (size_t)n_tok * Hkv * d;
  std::vector<orin::f16> hq(nq), hk(nkv), hv(nkv);
  fill_normal(hq, 1);
  fill_normal(hk, 2);
  fill_normal(hv, 3);
  void *q, *k, *v, *o, *ws = nullptr;
  int* cu = nullptr;
  CHECK(hipMalloc(&q, nq * 2));
  CHECK(hipMalloc(&k, nkv * 2));
  CHECK(hipMalloc(&v, nkv * 2));
  CHECK(hipMalloc(&o, nq * 2));
  CHECK(hipMemcpy(q, hq.data(), nq * 2, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(k, hk.data(), nkv * 2, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(v, hv.data(), nkv * 2, hipMemcpyHostToDevice));

  orin::FwdArgs a = {};
  a.q = q;
  a.q_tok_stride = (long)Hq * d;
  a.q_head_stride = d;
  a.k = k;
  a.v = v;
  a.kv_tok_stride = (long)Hkv * d;
  a.kv_head_stride = d;
  a.o = o;
  a.o_tok_stride = (long)Hq * d;
  a.o_head_stride = d;
  a.n_q = n_tok;
  if (!causal) {
    std::vector<int> hcu(n_seg + 1);
    for (int i = 0; i <= n_seg; ++i) hcu[i] = i * S;
    CHECK(hipMalloc(&cu, (n_seg + 1) * sizeof(int)));
    CHECK(hipMemcpy(cu, hcu.data(), (n_seg + 1) * sizeof(int), hipMemcpyHostToDevice));
    a.cu_seqlens = cu;
    a.n_seg = n_seg;
    a.max_seqlen = S;
  }
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.kv_mul = Hq / Hkv;
  a.head_size = d;
  a.scale_log2 = (float)(1.0 / sqrt((double)d)) * orin::kLog2e;
  size_t ws_bytes = 0;
  const int chunk = causal ? orin::fwd_pp_key_split(a, orin::kF16, n_cu, &ws_bytes) : 0;
  if (chunk > 0) {
    CHECK(hipMalloc(&ws, ws_bytes));
    a.key_chunk_tiles = chunk;
    a.ws = (float*)ws;
  }
  for (int i = 0; i < 20; ++i) CHECK(orin::launch_fwd_pp(a, orin::kF16, causal, 0));
  CHECK(hipDeviceSynchronize());
  std::vector<unsigned long long> zero(8192 * 24, 0), t(8192 * 16);
  CHECK(hipMemcpyToSymbol(HIP_SYMBOL(orin_pp_timeline), zero.data(), t.size() * 8));
  CHECK(hipMemcpyToSymbol(HIP_SYMBOL(orin_pp_steps), zero.data(), zero.size() * 8));
  CHECK(orin::launch_fwd_pp(a, orin::kF16, causal, 0));
  CHECK(hipDeviceSynchronize());
  CHECK(hipMemcpyFromSymbol(t.data(), HIP_SYMBOL(orin_pp_timeline), t.size() * 8));

  unsigned long long t0 = ~0ull, t_end = 0;
  int n = 0;
  for (; n < 8192 && t[n * 16] != 0; ++n) t0 = t[n * 16] < t0 ? t[n * 16] : t0;
  struct Acc {
    int n = 0;
    double dur = 0, first = 0, loop = 0, ghz = 0;
  };
  std::map<int, Acc> by_tiles;
  double sx = 0, sy = 0, sxx = 0, sxy = 0;
  for (int b = 0; b < n; ++b) {
    const unsigned long long* g = &t[b * 16];
    unsigned long long end = 0;
    for (int w = 0; w < 8; ++w) end = g[3 + w] > end ? g[3 + w] : end;
    t_end = end > t_end ? end : t_end;
    const double dur = (end - g[0]) / 100.0, tiles = (double)g[11];
    Acc& acc = by_tiles[(int)g[11]];
    acc.n++;
    acc.dur += dur;
    acc.first += (g[1] - g[0]) / 100.0;
    acc.loop += (g[2] - g[0]) / 100.0;
    acc.ghz += g[12] / ((g[3] - g[0]) * 10.0);  // clocks / ns
    sx += tiles;
    sy += dur;
    sxx += tiles * tiles;
    sxy += tiles * dur;
  }
  const double slope = (n * sxy - sx * sy) / (n * sxx - sx * sx), icpt = (sy - slope * sx) / n;
  printf("%s: %s %d x %d tokens, %d/%d heads, d %d, key split %s (chunk bound %d tiles): %d workgroups, span %.2f us\n",
         name, causal ? "causal" : "bidirectional", causal ? 1 : n_seg, S, Hq, Hkv, d,
         chunk > 0 ? "on" : "off", chunk, n, (t_end - t0) / 100.0);
  printf("| tiles | workgroups | duration us | first stage landed us | loop entry us | shader GHz |\n");
  printf("|---|---|---|---|---|---|\n");
  for (auto& kv : by_tiles) {
    const Acc& c = kv.second;
    printf("| %d | %d | %.2f | %.2f | %.2f | %.2f |\n", kv.first, c.n, c.dur / c.n, c.first / c.n,
           c.loop / c.n, c.ghz / c.n);
  }
  if (by_tiles.size() > 1) printf("fit: duration = %.3f us/tile + %.3f us\n", slope, icpt);
  // Steady-state steps: per group, the mean of (phase work, step) over the workgroups that
  // reached them; group 0 runs its MFMA phase in even steps, group 1 in odd ones.
  std::vector<unsigned long long> st(8192 * 24);
  CHECK(hipMemcpyFromSymbol(st.data(), HIP_SYMBOL(orin_pp_steps), st.size() * 8));
  double work[2][2] = {{0, 0}, {0, 0}}, step[2][2] = {{0, 0}, {0, 0}};
  int cnt[2][2] = {{0, 0}, {0, 0}};
  for (int b = 0; b < n; ++b)
    for (int g = 0; g < 2; ++g)
      for (int q = 0; q < 4; ++q) {
        const unsigned long long* e = &st[((b * 2 + g) * 4 + q) * 3];
        if (!e[0] || !e[1] || !e[2]) continue;
        const int mf = ((kStepStamp0 + q) & 1) == g ? 1 : 0;  // group g's MFMA phase?
        work[g][mf] += (double)(e[1] - e[0]);
        step[g][mf] += (double)(e[2] - e[0]);
        cnt[g][mf]++;
      }
  for (int g = 0; g < 2; ++g)
    for (int mf = 1; mf >= 0; --mf)
      if (cnt[g][mf])
        printf("group %d %s step: work %.0f clocks, step %.0f clocks (%d samples)\n", g,
               mf ? "MFMA   " : "softmax", work[g][mf] / cnt[g][mf], step[g][mf] / cnt[g][mf], cnt[g][mf]);
  printf("\n");
  CHECK(hipFree(q));
  CHECK(hipFree(k));
  CHECK(hipFree(v));
  CHECK(hipFree(o));
  if (ws) CHECK(hipFree(ws));
  if (cu) CHECK(hipFree(cu));
}

int main() {
  int dev = 0, n_cu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
  run_shape("C2", 2048, 12, 2, 128, n_cu);
  run_shape("C3", 4096, 32, 8, 128, n_cu);
  run_shape("C5 (fp16)", 1024, 16, 16, 72, n_cu, 4);
  run_shape("C5 shape at d 64", 1024, 16, 16, 64, n_cu, 4);
  run_shape("C5 shape at d 128", 1024, 16, 16, 128, n_cu, 4);
  return 0;
}
