// Split-KV decode attention for gfx950.
//
// Replaces the reference's single-query attention kernels
// (kuiper/source/op/kernels/cuda/mha_kernel.cu:162-338,
//  flash_attention_kernel.cu:205-535 and :966-1175,
//  flash_attention2_kernel.cu:409-816) with one design:
//
//  * A workgroup (4 waves) owns one (row, kv head, split): it reads that split's
//    K/V once and serves the G query heads that share the kv head (GQA), so KV
//    bytes are read from HBM once per kv head instead of once per query head.
//  * Inside a wave, 8 lanes own one token: lane k of the group loads the 16-byte
//    chunks [128n + 16k, +16) of the token's K row (n < NV), so each load
//    instruction covers 8 tokens x 128 contiguous bytes.  q.k is a per-lane
//    dot2 followed by a 3-step DPP all-reduce over the 8 lanes.
//  * Each wave keeps its own online-softmax state (running max m, partial sum l,
//    accumulator acc) over 64-token tiles, so no barrier is needed per tile;
//    the 4 waves are merged once through LDS at the end.
//  * Splits are fixed-size ranges of logical token positions.  A row needing
//    more than one split writes (acc, m, l) partials to the workspace and
//    decode_combine merges them; a single-split row writes its output directly.
//  * The address of token t is computed by one of three maps (contiguous cache,
//    paged block table, varlen segment).  The arithmetic does not depend on the
//    map, so paged and contiguous decode of the same KV are bit-identical.
#include "common.h"
#include "kernels.h"

namespace orin {

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;

template <typename T, int D>
struct DecodeShape {
  static constexpr int kRowBytes = D * (int)sizeof(T);
  static_assert(kRowBytes % 128 == 0, "head row must be a multiple of 128 bytes");
  static constexpr int NV = kRowBytes / 128;           // 16-byte chunks per lane per token
  static constexpr int VEC = 16 / (int)sizeof(T);      // elements per chunk
  static constexpr int CH_STRIDE = 128 / (int)sizeof(T);  // elements between a lane's chunks
  static constexpr int STEPS = (16 / NV) < 2 ? 2 : (16 / NV);  // 8-token groups per wave tile
  static constexpr int TILE = STEPS * 8;               // tokens per wave tile
};

// Address of the K/V row of logical token `tok` of the current row, in elements,
// relative to the k/v base pointer (kv head offset excluded).
struct TokenMap {
  int mode;           // 0 contiguous, 1 paged
  long base;          // contiguous: element offset of token 0 of this row
  long tok_stride;    // elements between consecutive tokens (physical rows)
  const int* bt_row;  // paged: this row's block table
  int bs_log2;
  __device__ __forceinline__ long operator()(int tok) const {
    if (mode == 1) {
      long phys = ((long)bt_row[tok >> bs_log2] << bs_log2) + (tok & ((1 << bs_log2) - 1));
      return phys * tok_stride;
    }
    return base + (long)tok * tok_stride;
  }
};

__device__ __forceinline__ int row_len_raw(const DecodeArgs& a, int row) {
  if (a.cu_seqlens) {
    int lo = 0, hi = a.n_seg - 1;  // find s with cu[s] <= row < cu[s+1]
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (a.cu_seqlens[mid] <= row) lo = mid; else hi = mid - 1;
    }
    return a.cu_seqlens[lo + 1] - a.cu_seqlens[lo];
  }
  if (a.lens) return a.lens[row] + a.len_add;
  return a.len_base + row * a.len_step;
}

// Device-side lengths (gpu pos, context_lens) are clamped to what the launch covers.
__device__ __forceinline__ int row_len(const DecodeArgs& a, int row) {
  return min(row_len_raw(a, row), a.len_cap);
}

template <typename T, int D, int G>
__global__ void __launch_bounds__(kDecodeThreads)
decode_split_kernel(DecodeArgs a) {
  using S = DecodeShape<T, D>;
  constexpr int NV = S::NV, VEC = S::VEC, STEPS = S::STEPS, TILE = S::TILE;
  constexpr int EL = NV * VEC;  // fp32 accumulator elements per lane per head

  const int n_hg = a.kv_mul / G;
  int bid = blockIdx.x;
  const int split = bid % a.max_splits;
  bid /= a.max_splits;
  const int hg = bid % n_hg;
  bid /= n_hg;
  const int kvh = bid % a.Hkv;
  const int row = bid / a.Hkv;

  const int len = row_len(a, row);
  const int s0 = split * a.split_tokens;
  const int h0 = kvh * a.kv_mul + hg * G;
  const int nsplit = len > 0 ? (len + a.split_tokens - 1) / a.split_tokens : 0;

  T* out = reinterpret_cast<T*>(a.o) + (long)row * a.o_row_stride;
  if (len <= 0) {  // empty row: output zeros
    if (split == 0)
      for (int i = threadIdx.x; i < G * D; i += kDecodeThreads)
        out[(long)(h0 + i / D) * a.o_head_stride + i % D] = from_f32<T>(0.f);
    return;
  }
  if (split >= nsplit) return;
  const int s1 = min(s0 + a.split_tokens, len);

  TokenMap map;
  if (a.block_table) {
    map.mode = 1;
    map.bt_row = a.block_table + (long)row * a.bt_row_stride;
    map.bs_log2 = a.bs_log2;
    map.base = 0;
  } else {
    map.mode = 0;
    map.bt_row = nullptr;
    map.bs_log2 = 0;
    long base = (long)row * a.kv_row_stride;
    if (a.cu_seqlens) {
      int lo = 0, hi = a.n_seg - 1;
      while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (a.cu_seqlens[mid] <= row) lo = mid; else hi = mid - 1;
      }
      base = (long)a.cu_seqlens[lo] * a.kv_tok_stride;
    }
    map.base = base;
  }
  map.tok_stride = a.kv_tok_stride;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int k8 = lane & 7;   // chunk slot inside the token's row
  const int grp = lane >> 3; // token group (0..7)

  const T* kb = reinterpret_cast<const T*>(a.k) + (long)kvh * a.kv_head_stride + k8 * VEC;
  const T* vb = reinterpret_cast<const T*>(a.v) + (long)kvh * a.kv_head_stride + k8 * VEC;

  // q chunks for the G heads, same element mapping as K.
  Chunk<T> qc[G][NV];
  {
    const T* qb = reinterpret_cast<const T*>(a.q) + (long)row * a.q_row_stride + k8 * VEC;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int n = 0; n < NV; ++n)
        qc[g][n] = load_chunk(qb + (long)(h0 + g) * a.q_head_stride + n * S::CH_STRIDE);
  }

  float m[G], l[G], acc[G][EL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EL; ++e) acc[g][e] = 0.f;
  }

  const float c = a.scale_log2;
  for (int t0 = s0 + wave * TILE; t0 < s1; t0 += kDecodeWaves * TILE) {
    Chunk<T> kc[STEPS][NV], vc[STEPS][NV];
    bool valid[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      int tok = t0 + s * 8 + grp;
      valid[s] = tok < s1;
      long off = map(valid[s] ? tok : s1 - 1);
#pragma unroll
      for (int n = 0; n < NV; ++n) kc[s][n] = load_chunk(kb + off + n * S::CH_STRIDE);
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      int tok = t0 + s * 8 + grp;
      long off = map(tok < s1 ? tok : s1 - 1);
#pragma unroll
      for (int n = 0; n < NV; ++n) vc[s][n] = load_chunk(vb + off + n * S::CH_STRIDE);
    }

    float sc[STEPS][G];
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int n = 0; n < NV; ++n) d = chunk_dot(qc[g][n], kc[s][n], d);
        d = sum8(d);
        sc[s][g] = valid[s] ? d * c : -INFINITY;
      }

#pragma unroll
    for (int g = 0; g < G; ++g) {
      float tm = sc[0][g];
#pragma unroll
      for (int s = 1; s < STEPS; ++s) tm = fmaxf(tm, sc[s][g]);
      tm = max_across_groups8(tm);
      const float mn = fmaxf(m[g], tm);
      const float alpha = fast_exp2(m[g] - mn);
      m[g] = mn;
      float ls = 0.f;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        sc[s][g] = fast_exp2(sc[s][g] - mn);
        ls += sc[s][g];
      }
      l[g] = l[g] * alpha + ls;
#pragma unroll
      for (int e = 0; e < EL; ++e) acc[g][e] *= alpha;
    }

#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        float vf[VEC];
        chunk_unpack(vc[s][n], vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < VEC; ++i)
            acc[g][n * VEC + i] = __builtin_fmaf(sc[s][g], vf[i], acc[g][n * VEC + i]);
      }
    }
  }

  // Merge the 8 token groups of the wave (all groups share the wave's m).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = sum_across_groups8(l[g]);
#pragma unroll
    for (int e = 0; e < EL; ++e) acc[g][e] = sum_across_groups8(acc[g][e]);
  }

  // Merge the 4 waves through LDS: per wave [G][D] acc, then m, l.
  __shared__ float s_acc[kDecodeWaves][G][D];
  __shared__ float s_ml[kDecodeWaves][G][2];
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          s_acc[wave][g][n * S::CH_STRIDE + k8 * VEC + i] = acc[g][n * VEC + i];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_ml[wave][g][0] = m[g];
      s_ml[wave][g][1] = l[g];
    }
  }
  __syncthreads();

  const bool direct = (nsplit == 1);
  for (int i = threadIdx.x; i < G * D; i += kDecodeThreads) {
    const int g = i / D, dd = i % D;
    float M = s_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float f = fast_exp2(s_ml[w][g][0] - M);
      L += f * s_ml[w][g][1];
      o += f * s_acc[w][g][dd];
    }
    if (direct) {
      out[(long)(h0 + g) * a.o_head_stride + dd] = from_f32<T>(o / L);
    } else {
      float* p = a.ws + ((((long)row * a.Hq + h0 + g) * a.max_splits + split) * (D + 2));
      p[dd] = o;
      if (dd == 0) {
        p[D] = M;
        p[D + 1] = L;
      }
    }
  }
}

// Merge split partials of every (row, head) whose row needed more than one split.
template <typename T, int D>
__global__ void __launch_bounds__(64) decode_combine_kernel(DecodeArgs a) {
  const int h = blockIdx.x % a.Hq;
  const int row = blockIdx.x / a.Hq;
  const int len = row_len(a, row);
  const int nsplit = len > 0 ? (len + a.split_tokens - 1) / a.split_tokens : 0;
  if (nsplit <= 1) return;
  const float* p = a.ws + ((long)row * a.Hq + h) * a.max_splits * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p[s * (D + 2) + D]);
  float L = 0.f;
  for (int s = 0; s < nsplit; ++s)
    L += fast_exp2(p[s * (D + 2) + D] - M) * p[s * (D + 2) + D + 1];
  const float inv = 1.f / L;
  T* out = reinterpret_cast<T*>(a.o) + (long)row * a.o_row_stride + (long)h * a.o_head_stride;
  for (int dd = threadIdx.x; dd < D; dd += 64) {
    float o = 0.f;
    for (int s = 0; s < nsplit; ++s)
      o += fast_exp2(p[s * (D + 2) + D] - M) * p[s * (D + 2) + dd];
    out[dd] = from_f32<T>(o * inv);
  }
}

template <typename T, int D, int G>
hipError_t launch_decode_tg(const DecodeArgs& a, hipStream_t stream) {
  const long blocks = (long)a.n_rows * a.Hkv * (a.kv_mul / G) * a.max_splits;
  hipLaunchKernelGGL((decode_split_kernel<T, D, G>), dim3((unsigned)blocks), dim3(kDecodeThreads),
                     0, stream, a);
  if (a.max_splits > 1)
    hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3((unsigned)(a.n_rows * a.Hq)), dim3(64),
                       0, stream, a);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_decode_t(const DecodeArgs& a, int G, hipStream_t stream) {
  switch (G) {
    case 1: return launch_decode_tg<T, D, 1>(a, stream);
    case 2: return launch_decode_tg<T, D, 2>(a, stream);
    case 3: return launch_decode_tg<T, D, 3>(a, stream);
    case 4: return launch_decode_tg<T, D, 4>(a, stream);
    case 5: return launch_decode_tg<T, D, 5>(a, stream);
    case 6: return launch_decode_tg<T, D, 6>(a, stream);
    case 7: return launch_decode_tg<T, D, 7>(a, stream);
    case 8: return launch_decode_tg<T, D, 8>(a, stream);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_decode_d(const DecodeArgs& a, int G, hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_decode_t<T, 64>(a, G, stream);
    case 128: return launch_decode_t<T, 128>(a, G, stream);
    case 256: return launch_decode_t<T, 256>(a, G, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int decode_heads_per_block(int kv_mul) {
  for (int g = 8; g >= 1; --g)
    if (kv_mul % g == 0) return g;
  return 1;
}

bool decode_supports(int dtype, int head_size) {
  return (dtype == kF32 || dtype == kF16 || dtype == kBF16) &&
         (head_size == 64 || head_size == 128 || head_size == 256);
}

hipError_t launch_decode(const DecodeArgs& a, int dtype, hipStream_t stream) {
  const int G = decode_heads_per_block(a.kv_mul);
  switch (dtype) {
    case kF32: return launch_decode_d<float>(a, G, stream);
    case kF16: return launch_decode_d<f16>(a, G, stream);
    case kBF16: return launch_decode_d<bf16>(a, G, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace orin
