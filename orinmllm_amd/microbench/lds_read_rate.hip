// LDS read throughput per CU on gfx950 (bytes per clock at the measured clock) for
// ds_read_b128 and ds_read_b64_tr_b16 with 2-8 reads in flight per wave and 4 or 8 waves
// per CU: the rate a single wave and a full CU can pull from LDS, which bounds the prefill's
// MFMA phase (one 16-byte fragment per MFMA).
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ unsigned long long g_clk[2];
template <int INFLIGHT, int TR>
__global__ void k(unsigned* out, int iters) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int t = threadIdx.x, lane = t & 63, w = t >> 6;
  u32x4* s = (u32x4*)smem;
  for (int i = t; i < 8192; i += blockDim.x) s[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
  __syncthreads();
  if (blockIdx.x == 0 && t == 0) { g_clk[0] = __builtin_amdgcn_s_memtime(); g_clk[1] = __builtin_amdgcn_s_memrealtime(); }
  unsigned addr = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)smem + (TR ? lane * 8 : lane * 16) + (w & 7) * 1024;
  u32x4 acc = {};
  for (int it = 0; it < iters; ++it) {
    u32x4 v[8];
    if (TR == 0) {
#define RD(j) if (j < INFLIGHT) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v[j]) : "v"(addr), "i"(j * 8192));
      RD(0) RD(1) RD(2) RD(3) RD(4) RD(5) RD(6) RD(7)
    } else {
      u32x2 x[8];
#define RT(j) if (j < INFLIGHT) __asm__ volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(x[j]) : "v"(addr), "i"(j * 8192));
      RT(0) RT(1) RT(2) RT(3) RT(4) RT(5) RT(6) RT(7)
      for (int j = 0; j < INFLIGHT; ++j) v[j] = u32x4{x[j][0], x[j][1], 0u, 0u};
    }
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < INFLIGHT; ++j) acc += v[j];
  }
  out[blockIdx.x * blockDim.x + t] = acc[0] + acc[1] + acc[2] + acc[3];
  if (blockIdx.x == 0 && t == 0) { g_clk[0] = __builtin_amdgcn_s_memtime() - g_clk[0]; g_clk[1] = __builtin_amdgcn_s_memrealtime() - g_clk[1]; }
}
template <int INFLIGHT, int TR>
void run(int W, unsigned* out) {
  const int iters = 4096;
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  hipLaunchKernelGGL((k<INFLIGHT, TR>), dim3(256), dim3(64 * W), 130000, 0, out, iters);
  hipEventRecord(e0);
  hipLaunchKernelGGL((k<INFLIGHT, TR>), dim3(256), dim3(64 * W), 130000, 0, out, iters);
  hipEventRecord(e1); hipEventSynchronize(e1);
  float ms; hipEventElapsedTime(&ms, e0, e1);
  unsigned long long c[2]; hipMemcpyFromSymbol(c, HIP_SYMBOL(g_clk), 16);
  double ghz = c[0] / (c[1] * 10.0);
  double bytes = 256.0 * 64 * W * (TR ? 8 : 16) * INFLIGHT * iters;
  printf("%s waves/CU %2d inflight %d: %.1f B/clk/CU  (clk %.2f GHz, %.3f ms)\n", TR ? "tr_b64" : "b128  ", W, INFLIGHT,
         bytes / (ms * 1e-3) / (ghz * 1e9) / 256, ghz, ms);
}
int main() {
  unsigned* out; hipMalloc(&out, 256 * 1024 * 4);
  for (int W : {4, 8}) { run<2, 0>(W, out); run<4, 0>(W, out); run<8, 0>(W, out); }
  for (int W : {4, 8}) { run<4, 1>(W, out); run<8, 1>(W, out); }
  return 0;
}
