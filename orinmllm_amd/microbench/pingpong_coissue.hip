// The prefill's ping-pong pattern on gfx950: 8 waves per workgroup (2 per SIMD); waves 0-3
// issue only MFMAs (4 independent v_mfma_f32_32x32x16_f16 accumulators, in VGPRs or, through
// inline asm, in AGPRs), optionally after ds_read_b128 fragment reads as the prefill's MFMA
// wave does (6 per 4 MFMAs), and waves 4-7 issue only VALU instructions of one kind on 16
// independent chains.  Prints the shader clocks per loop iteration of each side, alone and
// side by side: what a softmax wave's VALU work costs beside an MFMA wave.
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
template <int NM, int NV, int KIND, bool AG, int ND = 0>
__global__ void __launch_bounds__(512) k(float* out, long long* clk, int iters) {
  const int wave = threadIdx.x >> 6;
  __shared__ u32x4 lds[4096];
  for (int i = threadIdx.x; i < 4096; i += 512) lds[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
  __syncthreads();
  long long t0 = __builtin_amdgcn_s_memtime(), t1;
  float s = 0.f;
  if (wave < 4) {
    f32x16 acc[4] = {};
    f16x8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(threadIdx.x * 0.001f + i); b[i] = (_Float16)(i * 0.5f); }
    u32x4 fr[8] = {};
    t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < ND; ++j) {
        const int idx = ((threadIdx.x & 63) + 64 * ((wave + j + it) & 15)) & 4095;
        asm volatile("ds_read_b128 %0, %1" : "=v"(fr[j & 7]) : "v"((unsigned)(idx * 16)));
      }
      if (ND) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        if (AG)
          asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc[j & 3]) : "v"(a), "v"(b));
        else
          acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j & 3], 0, 0, 0);
      }
    }
    t1 = __builtin_amdgcn_s_memtime();
    for (int j = 0; j < 4; ++j) for (int i = 0; i < 16; ++i) s += acc[j][i];
    for (int j = 0; j < 8; ++j) s += (float)fr[j][0];
  } else {
    float x[16];
    for (int i = 0; i < 16; ++i) x[i] = threadIdx.x * 1e-3f + i;
    t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        float& y = x[j & 15];
        if (KIND == 0) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(y) : "v"(1.0001f), "v"(1e-7f));
        else if (KIND == 1) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(y) : "v"(1.0001f));
        else if (KIND == 2) asm volatile("v_exp_f32 %0, %0" : "+v"(y));
        else if (KIND == 3) asm volatile("v_cvt_pk_f16_f32 %0, %0, %0" : "+v"(y));
        else asm volatile("v_mov_b32 %0, %0" : "+v"(y));
      }
    }
    t1 = __builtin_amdgcn_s_memtime();
    for (int i = 0; i < 16; ++i) s += x[i];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if ((threadIdx.x & 63) == 0) clk[blockIdx.x * 8 + wave] = t1 - t0;
}

template <int NM, int NV, int KIND, bool AG, int ND = 0>
void run(const char* name, float* out, long long* clk) {
  const int iters = 2048;
  hipLaunchKernelGGL((k<NM, NV, KIND, AG, ND>), dim3(256), dim3(512), 0, 0, out, clk, iters);
  hipDeviceSynchronize();
  long long h[256 * 8];
  hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
  double m = 0, v = 0;
  for (int b = 0; b < 256; ++b)
    for (int w = 0; w < 8; ++w) (w < 4 ? m : v) += h[b * 8 + w];
  m /= 1024.0 * iters;
  v /= 1024.0 * iters;
  printf("%-34s MFMA waves %6.1f clk/iter, VALU waves %6.1f clk/iter\n", name, m, v);
}

int main() {
  float* out;
  long long* clk;
  hipMalloc(&out, 256 * 512 * 4);
  hipMalloc(&clk, 256 * 8 * 8);
  run<4, 0, 0, false>("4 mfma (VGPR acc) alone", out, clk);
  run<4, 0, 0, true>("4 mfma (AGPR acc) alone", out, clk);
  run<4, 0, 0, false, 6>("4 mfma + 6 ds_read_b128 alone", out, clk);
  run<0, 0, 0, false, 6>("6 ds_read_b128 alone", out, clk);
  run<0, 32, 4, false>("32 mov alone", out, clk);
  run<0, 32, 1, false>("32 mul alone", out, clk);
  run<0, 32, 0, false>("32 fma alone", out, clk);
  run<0, 32, 3, false>("32 cvt_pk alone", out, clk);
  run<0, 32, 2, false>("32 exp alone", out, clk);
  run<4, 32, 4, false>("4 mfma VGPR | 32 mov", out, clk);
  run<4, 32, 4, true>("4 mfma AGPR | 32 mov", out, clk);
  run<4, 32, 0, false>("4 mfma VGPR | 32 fma", out, clk);
  run<4, 32, 0, true>("4 mfma AGPR | 32 fma", out, clk);
  run<4, 32, 2, false>("4 mfma VGPR | 32 exp", out, clk);
  run<4, 32, 2, true>("4 mfma AGPR | 32 exp", out, clk);
  run<0, 32, 4, false, 6>("6 ds | 32 mov", out, clk);
  run<4, 32, 4, false, 6>("4 mfma + 6 ds | 32 mov", out, clk);
  run<4, 32, 1, false, 6>("4 mfma + 6 ds | 32 mul", out, clk);
  run<4, 32, 0, false, 6>("4 mfma + 6 ds | 32 fma", out, clk);
  run<4, 32, 3, false, 6>("4 mfma + 6 ds | 32 cvt_pk", out, clk);
  run<4, 32, 2, false, 6>("4 mfma + 6 ds | 32 exp", out, clk);
  return 0;
}
