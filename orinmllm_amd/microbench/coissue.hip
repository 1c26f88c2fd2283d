// Same-wave MFMA / VALU co-execution on gfx950: cycles per loop iteration of
// {1 v_mfma_f32_32x32x16_f16 ; N independent VALU ops (fma, exp or cvt_pk)} with 1 or 2
// waves per SIMD.  Backs the ping-pong prefill's premise that a VALU wave runs beside an
// MFMA wave on one SIMD without slowing the MFMAs.
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
template <int NV, int KIND, bool MF>
__global__ void k(float* out, long long* clk, int iters) {
  f32x16 acc = {};
  f16x8 a, b;
  for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(threadIdx.x * 0.001f + i); b[i] = (_Float16)(i * 0.5f); }
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = threadIdx.x * 1e-3f + i;
  long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    if (MF) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float& y = x[j & 7];
      if (KIND == 0) __asm__ volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(y) : "v"(1.0001f), "v"(1e-7f));
      else if (KIND == 1) __asm__ volatile("v_exp_f32 %0, %0" : "+v"(y));
      else __asm__ volatile("v_cvt_pk_f16_f32 %0, %0, %0" : "+v"(y));
    }
  }
  long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0; for (int i = 0; i < 8; ++i) s += x[i];
  for (int i = 0; i < 16; ++i) s += acc[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) clk[blockIdx.x] = t1 - t0;
}
template <int NV, int KIND, bool MF>
void run(const char* name, int waves_per_simd, float* out, long long* clk) {
  const int iters = 4096;
  hipLaunchKernelGGL((k<NV, KIND, MF>), dim3(256), dim3(256 * waves_per_simd), 0, 0, out, clk, iters);
  hipDeviceSynchronize();
  long long h[256]; hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
  double a = 0; for (int i = 0; i < 256; ++i) a += h[i]; a /= 256;
  printf("%-22s waves/SIMD %d: %.1f cycles/iter\n", name, waves_per_simd, a / iters);
}
int main() {
  float* out; long long* clk; hipMalloc(&out, 256 * 1024 * 4); hipMalloc(&clk, 256 * 8);
  for (int w : {1, 2}) {
    run<0, 0, true>("mfma only", w, out, clk);
    run<8, 0, false>("8 fma only", w, out, clk);
    run<8, 0, true>("mfma + 8 fma", w, out, clk);
    run<4, 1, false>("4 exp only", w, out, clk);
    run<8, 1, false>("8 exp only", w, out, clk);
    run<2, 1, true>("mfma + 2 exp", w, out, clk);
    run<4, 1, true>("mfma + 4 exp", w, out, clk);
    run<8, 2, false>("8 cvt only", w, out, clk);
    run<4, 2, true>("mfma + 4 cvt", w, out, clk);
  }
  return 0;
}
