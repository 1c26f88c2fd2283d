// Shared device helpers for the gfx950 attention kernels: element types, 16-byte
// vectors, wave-level reductions built on DPP and ds_bpermute, and exp2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace orin {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// bf16 -> fp16 on 16-bit pairs.  Exact for values in fp16's normal range (bf16 carries 8
// significant bits, fp16 11).  bf16 attention keeps its softmax weights in fp16 (2^-12
// rounding instead of bf16's 2^-9, which on a near-cancelling output is as large as the
// output tolerance) and converts V to fp16 for the weighted sum.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t x) {
  const float lo = __builtin_bit_cast(float, x << 16);
  const float hi = __builtin_bit_cast(float, x & 0xffff0000u);
  return __builtin_bit_cast(uint32_t, f16x2{(f16)lo, (f16)hi});
}
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(const u32x4& x) {
  return u32x4{bf16x2_to_f16x2(x[0]), bf16x2_to_f16x2(x[1]), bf16x2_to_f16x2(x[2]),
               bf16x2_to_f16x2(x[3])};
}

// Hardware base-2 exponential (v_exp_f32).  exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- Q/K producer arithmetic
// Shared by the Q/K producer (producers.hip, qk_norm_rope_kernel) and the prefill's fused
// Q load (fwd_pp.hip), so that both produce the same bits for the same row.
// Sum of squares of one 8-element chunk pair: elements lo[i] (first half of the head) and
// hi[i] (second half), nested as fma(lo, lo, fma(hi, hi, acc)) from i = 0.
__device__ __forceinline__ float qk_chunk_sumsq(const float* lo, const float* hi) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(lo[i], lo[i], __builtin_fmaf(hi[i], hi[i], ss));
  return ss;
}
// Row sum of the chunk sums c[0 .. N) in the order of an xor butterfly over N lanes
// (strides 1, 2, 4, ...): every lane of such a butterfly ends with this value.
template <int N>
__device__ __forceinline__ float qk_butterfly_sum(const float (&c)[N]) {
  float v[N];
#pragma unroll
  for (int l = 0; l < N; ++l) v[l] = c[l];
#pragma unroll
  for (int m = 1; m < N; m <<= 1) {
    float w[N];
#pragma unroll
    for (int l = 0; l < N; ++l) w[l] = v[l] + v[l ^ m];
#pragma unroll
    for (int l = 0; l < N; ++l) v[l] = w[l];
  }
  return v[0];
}
// 1 / rms of a head row: 1 / sqrt(sum(x^2) / d + eps) (rmsnorm_kernel.cu:483-545).
__device__ __forceinline__ float qk_rms_inv(float ss, int d, float eps) {
  return 1.0f / sqrtf(ss / (float)d + eps);
}
// Rotate-half RoPE of the pair (x_j, x_{j+d/2}) by the angle with cosine cv and sine sv
// (rope_kernel.cu:464-509).
__device__ __forceinline__ void qk_rope(float lo, float hi, float cv, float sv, float& ro,
                                        float& rh) {
  ro = __builtin_fmaf(cv, lo, -(sv * hi));
  rh = __builtin_fmaf(cv, hi, sv * lo);
  // Both results are fp32 values here: the empty asm keeps the compiler from fusing the fma
  // with a later conversion to 16 bits (v_fma_mix*_f16 rounds once, fma then convert twice),
  // a choice it makes per call site, so every kernel using this rounds alike.
  __asm__("" : "+v"(ro), "+v"(rh));
}

// ---------------------------------------------------------------- 16-byte lane chunk
// A lane chunk is 16 bytes of one K or V row: 8 halves or 4 floats.
template <typename T>
struct Chunk {
  static constexpr int kElems = 16 / sizeof(T);
  u32x4 raw;
};

// Dot product of two 16-byte chunks, accumulated in fp32 onto acc.
// fp16/bf16 use v_dot2_f32_{f16,bf16}: the products of two 16-bit floats are
// exact in fp32, only the additions round.
// Chunks are reinterpreted as whole vectors only: this toolchain mis-lowers
// __builtin_bit_cast applied to a single element of an ext_vector (it yields
// element 0 for every index).
__device__ __forceinline__ float chunk_dot(const Chunk<f16>& a, const Chunk<f16>& b,
                                           float acc) {
  const f16x8 x = __builtin_bit_cast(f16x8, a.raw), y = __builtin_bit_cast(f16x8, b.raw);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2(f16x2{x[2 * i], x[2 * i + 1]},
                                 f16x2{y[2 * i], y[2 * i + 1]}, acc, false);
  return acc;
}
__device__ __forceinline__ float chunk_dot(const Chunk<bf16>& a, const Chunk<bf16>& b,
                                           float acc) {
  const bf16x8 x = __builtin_bit_cast(bf16x8, a.raw), y = __builtin_bit_cast(bf16x8, b.raw);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{x[2 * i], x[2 * i + 1]},
                                          bf16x2{y[2 * i], y[2 * i + 1]}, acc,
                                          false);
  return acc;
}
// chunk_dot with a zero accumulator.  For 16-bit chunks the first product is the
// three-operand v_dot2 with an inline 0 (the compiler otherwise zeroes a register with a
// v_mov and accumulates into it with v_dot2c).
__device__ __forceinline__ float chunk_dot_first(const Chunk<f16>& a, const Chunk<f16>& b) {
  const f16x8 x = __builtin_bit_cast(f16x8, a.raw), y = __builtin_bit_cast(f16x8, b.raw);
  float acc;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(acc) : "v"(f16x2{x[0], x[1]}), "v"(f16x2{y[0], y[1]}));
#pragma unroll
  for (int i = 1; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2(f16x2{x[2 * i], x[2 * i + 1]},
                                 f16x2{y[2 * i], y[2 * i + 1]}, acc, false);
  return acc;
}
__device__ __forceinline__ float chunk_dot_first(const Chunk<bf16>& a, const Chunk<bf16>& b) {
  const bf16x8 x = __builtin_bit_cast(bf16x8, a.raw), y = __builtin_bit_cast(bf16x8, b.raw);
  float acc;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(bf16x2{x[0], x[1]}), "v"(bf16x2{y[0], y[1]}));
#pragma unroll
  for (int i = 1; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{x[2 * i], x[2 * i + 1]},
                                          bf16x2{y[2 * i], y[2 * i + 1]}, acc, false);
  return acc;
}
__device__ __forceinline__ float chunk_dot(const Chunk<float>& a, const Chunk<float>& b,
                                           float acc) {
  const f32x4 x = __builtin_bit_cast(f32x4, a.raw), y = __builtin_bit_cast(f32x4, b.raw);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(x[i], y[i], acc);
  return acc;
}
__device__ __forceinline__ float chunk_dot_first(const Chunk<float>& a, const Chunk<float>& b) {
  return chunk_dot(a, b, 0.f);
}

// Unpack a chunk into fp32 values.
__device__ __forceinline__ void chunk_unpack(const Chunk<f16>& c, float* out) {
  const f16x8 x = __builtin_bit_cast(f16x8, c.raw);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)x[i];
}
__device__ __forceinline__ void chunk_unpack(const Chunk<bf16>& c, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // bf16 -> fp32 is a 16-bit shift of the bit pattern.
    const uint32_t w = c.raw[i];
    out[2 * i] = __uint_as_float(w << 16);
    out[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
  }
}
__device__ __forceinline__ void chunk_unpack(const Chunk<float>& c, float* out) {
  const f32x4 x = __builtin_bit_cast(f32x4, c.raw);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = x[i];
}

template <typename T>
__device__ __forceinline__ Chunk<T> load_chunk(const T* p) {
  Chunk<T> c;
  c.raw = *reinterpret_cast<const u32x4*>(p);
  return c;
}

// Streaming load: the data is read once, so it should not displace reusable lines.
template <typename T>
__device__ __forceinline__ Chunk<T> load_chunk_nt(const T* p) {
  Chunk<T> c;
  c.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return c;
}

// ---------------------------------------------------------------- wave reductions
// DPP controls (CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each 8-lane half row
constexpr int kDppRowRor8 = 0x128;    // lane i <- lane (i+8) mod 16 inside a row

// No "old" operand (bound_ctrl set): the controls used here give every lane a valid
// source, and the compiler can fold the move into the consuming v_add / v_max as a DPP
// operand instead of zeroing a register first.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, true));
}

// Sum over each aligned group of 8 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float sum8(float x) {
  x += dpp_mov<kDppQuadXor1>(x);
  x += dpp_mov<kDppQuadXor2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  return x;
}

__device__ __forceinline__ float shfl_xor_f(float x, int mask) {
  int lane = __lane_id();
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, x)));
}

// x of lane l ^ 32: v_permlane32_swap_b32 on x and a copy of it.  The copy and the swap
// are one asm block with two wait states between them: on gfx950 a VALU write of a VGPR
// that v_permlane*_swap then reads needs two wait states, and the compiler's hazard check
// does not see VGPR writes made inside inline asm (a copy written by a separate asm
// statement could land right before the swap).  Lanes < 32 find their partner in the swapped
// copy, lanes >= 32 in the swapped original.
__device__ __forceinline__ float partner32(float x) {
  int a = __builtin_bit_cast(int, x), b;
  __asm__ volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane32_swap_b32 %0, %1"
                   : "+v"(a), "=&v"(b));
  return __builtin_bit_cast(float, (__lane_id() < 32) ? b : a);
}

// Max / sum across the 8 lane groups of a wave (lanes with equal lane%8).
__device__ __forceinline__ float max_across_groups8(float x) {
  x = fmaxf(x, dpp_mov<kDppRowRor8>(x));
  x = fmaxf(x, shfl_xor_f(x, 16));
  x = fmaxf(x, shfl_xor_f(x, 32));
  return x;
}
__device__ __forceinline__ float sum_across_groups8(float x) {
  x += dpp_mov<kDppRowRor8>(x);
  x += shfl_xor_f(x, 16);
  x += shfl_xor_f(x, 32);
  return x;
}

}  // namespace orin
