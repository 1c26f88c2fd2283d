// Lane layout of ds_read_b64_tr_b16 on gfx950 for three address patterns (prints the four
// 16-bit values each lane receives), and the LDS read rate of plain 16-byte reads at two
// strides.  The prefill reads its V^T fragments with this instruction.
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__global__ void tr_probe(short* out, int mode) {
  __shared__ short s[4096];
  int t = threadIdx.x;
  for (int i = t; i < 4096; i += 64) s[i] = (short)i;
  __syncthreads();
  // address: mode 0: lane*8 bytes (consecutive 64-bit); mode 1: row = lane, 256B stride
  int addr = mode == 0 ? t * 8 : (mode == 1 ? t * 256 : ((t % 16) * 256 + (t / 16) * 8));
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)((__attribute__((address_space(3))) char*)s + addr));
  for (int e = 0; e < 4; ++e) out[t * 4 + e] = v[e];
}
__global__ __launch_bounds__(256) void lds_bw3(float* out, long long* clk, int stride) {
  __shared__ u32x4 s[8192];
  int t = threadIdx.x;
  for (int i = t; i < 8192; i += 256) s[i] = u32x4{(unsigned)i, (unsigned)t, 2u, 3u};
  __syncthreads();
  u32x4 a0 = {0,0,0,0}, a1 = a0, a2 = a0, a3 = a0;
  int lane = t & 63, w = t >> 6;
  long long c0 = clock64();
  for (int i = 0; i < 1024; i += 4) {
    int b = (w * 2048 + i * 64 * stride) ;
    a0 += s[(b + lane) & 8191];
    a1 += s[(b + 64 + lane) & 8191];
    a2 += s[(b + 128 + lane) & 8191];
    a3 += s[(b + 192 + lane) & 8191];
    __asm__ volatile("" :: "v"(a0), "v"(a1), "v"(a2), "v"(a3));
  }
  long long c1 = clock64();
  u32x4 a = a0 + a1 + a2 + a3;
  out[blockIdx.x * 256 + t] = a[0] + a[1] + a[2] + a[3];
  if (t == 0) clk[blockIdx.x] = c1 - c0;
}
int main() {
  short* out; hipMalloc(&out, 4096 * 2); short h[256];
  for (int mode = 0; mode < 3; ++mode) {
    hipLaunchKernelGGL(tr_probe, dim3(1), dim3(64), 0, 0, out, mode);
    hipMemcpy(h, out, 512, hipMemcpyDeviceToHost);
    printf("mode %d:\n", mode);
    for (int l = 0; l < 64; ++l) { printf("L%02d:%4d %4d %4d %4d  ", l, h[l*4], h[l*4+1], h[l*4+2], h[l*4+3]); if (l % 4 == 3) printf("\n"); }
  }
  float* o2; long long* clk; hipMalloc(&o2, 1 << 22); hipMalloc(&clk, 1 << 16);
  long long hc[256];
  for (int st = 1; st <= 2; ++st) for (int rep = 0; rep < 2; ++rep) {
    hipLaunchKernelGGL(lds_bw3, dim3(256), dim3(256), 0, 0, o2, clk, st);
    hipDeviceSynchronize(); hipMemcpy(hc, clk, 8 * 256, hipMemcpyDeviceToHost);
    double avg = 0; for (int i = 0; i < 256; ++i) avg += hc[i]; avg /= 256;
    printf("lds_bw3 stride %d: %.0f clk -> %.1f B/clk/CU\n", st, avg, 256.0 * 16 * 1024 / avg);
  }
  return 0;
}
