// Issue cost of global -> LDS transfers (global_load_lds_dwordx4, M0 = LDS base) against
// plain 16-byte global loads, 8 waves per CU: clocks per step spent issuing and in total.
// The prefill stages its K/V tiles this way.
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void dma16(const void* gptr, unsigned lds_addr) {
  __asm__ volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(lds_addr) : "memory", "m0");
}
template <int MODE>  // 0 dma, 1 plain load
__global__ __launch_bounds__(512) void k(const char* src, long long* clk, unsigned* out, int steps) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
  const char* p = src + (size_t)blockIdx.x * (1 << 20) + wave * 2048 + lane * 16;
  long long issue = 0, total0 = clock64();
  u32x4 acc = {0, 0, 0, 0};
  for (int s = 0; s < steps; ++s) {
    long long t0 = clock64();
    const char* q = p + (size_t)(s & 31) * 16384;
    if (MODE == 0) {
      dma16(q, base + (s % 3) * 16384 + wave * 2048);
      dma16(q + 1024, base + (s % 3) * 16384 + wave * 2048 + 1024);
    } else {
      u32x4 a = *(const u32x4*)q, b = *(const u32x4*)(q + 1024);
      __asm__ volatile("" :: "v"(a), "v"(b));
      acc += a ^ b;
    }
    long long t1 = clock64();
    issue += t1 - t0;
    __builtin_amdgcn_s_waitcnt((4 & 15) | (7 << 4) | (15 << 8));
    __builtin_amdgcn_s_barrier();
  }
  long long total = clock64() - total0;
  if (lane == 0) { clk[(blockIdx.x * 8 + wave) * 2] = issue; clk[(blockIdx.x * 8 + wave) * 2 + 1] = total; }
  out[blockIdx.x * 512 + threadIdx.x] = acc[0];
}
int main() {
  char* src; long long* clk; unsigned* out;
  hipMalloc(&src, (size_t)256 << 20); hipMalloc(&clk, 256 * 8 * 16); hipMalloc(&out, 256 * 512 * 4);
  hipMemset(src, 1, (size_t)256 << 20);
  static long long h[256 * 8 * 2];
  for (int mode = 0; mode < 2; ++mode) for (int rep = 0; rep < 2; ++rep) {
    int steps = 256;
    if (mode == 0) hipLaunchKernelGGL(k<0>, dim3(256), dim3(512), 48 * 1024, 0, src, clk, out, steps);
    else hipLaunchKernelGGL(k<1>, dim3(256), dim3(512), 48 * 1024, 0, src, clk, out, steps);
    hipDeviceSynchronize();
    hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
    double is = 0, to = 0; for (int i = 0; i < 256 * 8; ++i) { is += h[2 * i]; to += h[2 * i + 1]; }
    printf("%s: issue %.1f clk/step/wave, total %.1f clk/step\n", mode ? "plain" : "dma  ", is / (256 * 8) / steps, to / (256 * 8) / steps);
  }
  return 0;
}
