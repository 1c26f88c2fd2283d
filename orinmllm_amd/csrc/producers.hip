// The kernels either side of the attention hot path on gfx950: KV-cache writes and the
// Q/K producers.  All of them are HBM-bound element moves with a little fp32 math, so
// each workgroup streams 16-byte chunks with coalesced, vectorised loads and stores.
//
//  kv_append_kernel        kernel::copy_to_kv_cache_kernel{,_fp16}
//                          (kuiper/source/op/kernels/cuda/kv_cache_kernel.cu:13-57): one
//                          token's K or V row into a kuiper cache [layers, max_seq, kv_dim]
//                          at a position read from device memory (graph-capturable).
//  kv_scatter_kernel       rows of K and V into a paged pool through a slot mapping
//                          (the paged-cache counterpart of the cudaMemcpyAsync pair of
//                          qwen3.cpp:1220-1241).
//  kv_convert_kernel       one sequence between a contiguous kuiper layer cache and a
//                          paged pool (either direction).
//  qk_norm_rope_kernel     per-head RMSNorm (rmsnorm_kernel.cu:483-545, eps 1e-6) then
//                          rotate-half RoPE (rope_kernel.cu:464-509, sin/cos cache entry
//                          2j for pair (j, j+d/2)) of Q in place and of K, with the rotated
//                          K and the V rows written to the cache -- the rmsnorm x2 +
//                          batched_rope + two cudaMemcpyAsync of qwen3.cpp:1195-1241 in
//                          one pass.
//  vision_qkv_kernel       kernel::fused_split_rope_transpose_cu
//                          (vision_encoder_kernel.cu:662-773): split [N, 3*H*d] into
//                          head-major q/k/v [H, N, d] with the 2-D rotary on q and k.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace orin {

namespace {

constexpr int kProdThreads = 256;

// 16-byte copy of element range [i, i+VEC) when the row is 16-byte aligned.
template <typename T>
__device__ __forceinline__ void copy16(T* dst, const T* src) {
  *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
}

// ---------------------------------------------------------------- kuiper append
template <typename T>
__global__ void __launch_bounds__(kProdThreads)
kv_append_kernel(T* cache, const T* src, const int* pos, int kv_dim, long layer_off) {
  const int position = *reinterpret_cast<const volatile int*>(pos);
  T* dst = cache + layer_off + (long)position * kv_dim;
  constexpr int VEC = 16 / (int)sizeof(T);
  const int i = (blockIdx.x * kProdThreads + threadIdx.x) * VEC;
  if (kv_dim % VEC == 0) {
    if (i < kv_dim) copy16(dst + i, src + i);
  } else {
    for (int e = i; e < min(i + VEC, kv_dim); ++e) dst[e] = src[e];
  }
}

// ---------------------------------------------------------------- paged scatter
// Row r of k_src / v_src (row_elems = kv_heads * head_size elements) goes to pool slot
// slots[r] (block slots[r] / block_size, offset slots[r] % block_size); a negative slot
// skips the row.  Token-major pool: [blocks, block_size, kv_heads, head_size]; head-major:
// [blocks, kv_heads, block_size, head_size].  One 16-byte chunk per thread.
struct ScatterArgs {
  const void* k_src;
  const void* v_src;
  void* k_pool;
  void* v_pool;
  const int* slots;
  long src_row_stride;  // elements between source rows
  int n_rows, kv_heads, head_size, block_size, head_major;
};

template <typename T>
__global__ void __launch_bounds__(kProdThreads) kv_scatter_kernel(ScatterArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int chunks_per_head = a.head_size / VEC;
  const int chunks_per_row = a.kv_heads * chunks_per_head;
  const long idx = (long)blockIdx.x * kProdThreads + threadIdx.x;
  const int r = (int)(idx / chunks_per_row);
  if (r >= a.n_rows) return;
  const int c = (int)(idx % chunks_per_row);
  const int h = c / chunks_per_head, e = (c % chunks_per_head) * VEC;
  // The source rows do not depend on the slot: their loads go out with the slot's.
  const long src = (long)r * a.src_row_stride + (long)h * a.head_size + e;
  const u32x4 kx = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.k_src) + src);
  const u32x4 vx = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.v_src) + src);
  const int slot = a.slots[r];
  if (slot < 0) return;
  const long blk = slot / a.block_size, off = slot % a.block_size;
  const long dst = a.head_major
                       ? ((blk * a.kv_heads + h) * a.block_size + off) * a.head_size + e
                       : ((blk * a.block_size + off) * a.kv_heads + h) * a.head_size + e;
  *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.k_pool) + dst) = kx;
  *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.v_pool) + dst) = vx;
}

// ---------------------------------------------------------------- contiguous <-> paged
// Tokens [0, n_tokens) of one sequence: contiguous cache rows [n, kv_heads * head_size]
// and pool blocks block_table[t / block_size].  to_paged selects the direction.
struct ConvertArgs {
  void* contig;
  void* pool;
  const int* block_table;
  long contig_row_stride;
  int n_tokens, kv_heads, head_size, block_size, head_major, to_paged;
};

template <typename T>
__global__ void __launch_bounds__(kProdThreads) kv_convert_kernel(ConvertArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int chunks_per_head = a.head_size / VEC;
  const int chunks_per_row = a.kv_heads * chunks_per_head;
  const long idx = (long)blockIdx.x * kProdThreads + threadIdx.x;
  const int t = (int)(idx / chunks_per_row);
  if (t >= a.n_tokens) return;
  const int c = (int)(idx % chunks_per_row);
  const int h = c / chunks_per_head, e = (c % chunks_per_head) * VEC;
  const long blk = a.block_table[t / a.block_size], off = t % a.block_size;
  const long p = a.head_major ? ((blk * a.kv_heads + h) * a.block_size + off) * a.head_size + e
                              : ((blk * a.block_size + off) * a.kv_heads + h) * a.head_size + e;
  const long q = (long)t * a.contig_row_stride + (long)h * a.head_size + e;
  T* pool = reinterpret_cast<T*>(a.pool);
  T* contig = reinterpret_cast<T*>(a.contig);
  if (a.to_paged) copy16(pool + p, contig + q);
  else copy16(contig + q, pool + p);
}

// ---------------------------------------------------------------- Q/K norm + RoPE
// One (token, head) unit per LPU = D / (2 * VEC) lanes: lane l of a unit holds the 16-byte
// chunk l of each half of the head row, i.e. the RoPE pairs (VEC*l + i, VEC*l + i + D/2).
// Units 0..Hq-1 of a token are its query heads (rotated in place), units Hq..Hq+Hkv-1
// its key heads (rotated, written to the K cache); a key unit also copies the token's V
// head row to the V cache.
struct NormRopeArgs {
  void* q;                 // [S, Hq * d], in place
  const void* k;           // [S, Hkv * d]
  const void* v;           // [S, Hkv * d]
  const void* q_weight;    // [d] RMSNorm weights (T), null = no norm of Q
  const void* k_weight;    // [d], null = no norm of K
  const float* sin_cache;  // [max_pos, d] fp32; entry 2j rotates pair j
  const float* cos_cache;
  void* k_cache;           // row of token t: k_cache + (start + t) * cache_tok_stride
  void* v_cache;
  long cache_tok_stride;
  const int* pos_ptr;      // non-null: start position read from device memory
  int start_pos, seq_len, Hq, Hkv, head_size;
  float eps;
};

template <typename T>
__device__ __forceinline__ void unpack16(const u32x4& raw, float* out) {
  if constexpr (sizeof(T) == 4) {
    const f32x4 x = __builtin_bit_cast(f32x4, raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = x[i];
  } else {
    chunk_unpack(Chunk<T>{raw}, out);
  }
}

template <typename T>
__device__ __forceinline__ u32x4 pack16(const float* x) {
  constexpr int VEC = 16 / (int)sizeof(T);
  typedef T tv __attribute__((ext_vector_type(VEC)));
  tv r;
#pragma unroll
  for (int i = 0; i < VEC; ++i) r[i] = from_f32<T>(x[i]);
  return __builtin_bit_cast(u32x4, r);
}

template <typename T, int D>
__global__ void __launch_bounds__(kProdThreads) qk_norm_rope_kernel(NormRopeArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LPU = D / 2 / VEC;  // lanes per unit
  static_assert(LPU >= 1 && LPU <= kWave && (kWave % LPU) == 0, "unsupported head size");
  const int lane = threadIdx.x & 63;
  const int l = lane % LPU;
  const long unit = ((long)blockIdx.x * kProdThreads + threadIdx.x) / LPU;
  // Units per token: the Hq query heads (unless q is null: K/V only), then the Hkv key heads.
  const int nq = a.q ? a.Hq : 0;
  const int units = nq + a.Hkv;
  const int t = (int)(unit / units);
  const bool live = t < a.seq_len;
  const int u = (int)(unit % units);
  const bool is_q = u < nq;
  const int h = is_q ? u : u - nq;
  const int start = a.pos_ptr ? *a.pos_ptr : a.start_pos;
  const int pos = start + (live ? t : 0);

  float lo[VEC], hi[VEC];
  float ss = 0.f;
  const T* x = is_q ? reinterpret_cast<const T*>(a.q) + ((long)t * a.Hq + h) * D
                    : reinterpret_cast<const T*>(a.k) + ((long)t * a.Hkv + h) * D;
  if (live) {
    unpack16<T>(*reinterpret_cast<const u32x4*>(x + VEC * l), lo);
    unpack16<T>(*reinterpret_cast<const u32x4*>(x + D / 2 + VEC * l), hi);
    if constexpr (VEC == 8) {
      ss = qk_chunk_sumsq(lo, hi);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss = __builtin_fmaf(lo[i], lo[i], __builtin_fmaf(hi[i], hi[i], ss));
    }
  }
  // sum over the unit's LPU lanes (aligned groups; every lane runs the shuffles)
#pragma unroll
  for (int m = 1; m < LPU; m <<= 1) ss += shfl_xor_f(ss, m);
  if (!live) return;
  const T* w = reinterpret_cast<const T*>(is_q ? a.q_weight : a.k_weight);
  if (w) {
    const float inv = qk_rms_inv(ss, D, a.eps);
    float wl[VEC], wh[VEC];
    unpack16<T>(*reinterpret_cast<const u32x4*>(w + VEC * l), wl);
    unpack16<T>(*reinterpret_cast<const u32x4*>(w + D / 2 + VEC * l), wh);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      lo[i] = lo[i] * inv * wl[i];
      hi[i] = hi[i] * inv * wh[i];
    }
  }
  // table entries 2j for j = VEC*l .. VEC*l + VEC-1: floats [2 VEC l, 2 VEC l + 2 VEC)
  const float* sn = a.sin_cache + (long)pos * D + 2 * VEC * l;
  const float* cs = a.cos_cache + (long)pos * D + 2 * VEC * l;
  float ro[VEC], rh[VEC];
#pragma unroll
  for (int c4 = 0; c4 < VEC / 2; ++c4) {
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sn + 4 * c4);
    const f32x4 k4 = *reinterpret_cast<const f32x4*>(cs + 4 * c4);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = 2 * c4 + e;
      const float sv = s4[2 * e], cv = k4[2 * e];
      qk_rope(lo[i], hi[i], cv, sv, ro[i], rh[i]);
    }
  }
  T* out = is_q ? reinterpret_cast<T*>(a.q) + ((long)t * a.Hq + h) * D
                : reinterpret_cast<T*>(a.k_cache) + (long)pos * a.cache_tok_stride + (long)h * D;
  *reinterpret_cast<u32x4*>(out + VEC * l) = pack16<T>(ro);
  *reinterpret_cast<u32x4*>(out + D / 2 + VEC * l) = pack16<T>(rh);
  if (!is_q) {
    const T* vr = reinterpret_cast<const T*>(a.v) + ((long)t * a.Hkv + h) * D;
    T* vo = reinterpret_cast<T*>(a.v_cache) + (long)pos * a.cache_tok_stride + (long)h * D;
    copy16(vo + VEC * l, vr + VEC * l);
    copy16(vo + D / 2 + VEC * l, vr + D / 2 + VEC * l);
  }
}

// sin/cos cache of rope_kernel.cu:86-98 / 153-166: entry [p][i] = sin/cos(p * theta^(-i/d)).
__global__ void __launch_bounds__(kProdThreads)
rope_cache_kernel(float* sin_cache, float* cos_cache, int head_size, int max_pos, float theta) {
  const long idx = (long)blockIdx.x * kProdThreads + threadIdx.x;
  if (idx >= (long)head_size * max_pos) return;
  const int i = (int)(idx % head_size);
  const int p = (int)(idx / head_size);
  const float freq = 1.0f / powf(theta, (float)i / (float)head_size);
  float s, c;
  sincosf((float)p * freq, &s, &c);
  sin_cache[idx] = s;
  cos_cache[idx] = c;
}

// ---------------------------------------------------------------- vision split + rotary
// qkv [N, 3 * H * d] (q | k | v per token) -> head-major q/k/v [H, N, d]; q and k get
// x1' = x1 cos[j] - x2 sin[j], x2' = x1 sin[j + d/2] + x2 cos[j + d/2] with the
// [N, d] cos/sin tables in T.  One thread per (token, head, pair j).
template <typename T>
__global__ void __launch_bounds__(kProdThreads)
vision_qkv_kernel(const T* qkv, const T* cos_t, const T* sin_t, T* qo, T* ko, T* vo, int N, int H,
                  int d) {
  const int half = d / 2;
  const long idx = (long)blockIdx.x * kProdThreads + threadIdx.x;
  if (idx >= (long)N * H * half) return;
  const int j = (int)(idx % half);
  const long th = idx / half;
  const int h = (int)(th % H);
  const int t = (int)(th / H);
  const long hidden = (long)H * d;
  const T* row = qkv + (long)t * 3 * hidden + (long)h * d;
  const float c1 = to_f32(cos_t[(long)t * d + j]), s1 = to_f32(sin_t[(long)t * d + j]);
  const float c2 = to_f32(cos_t[(long)t * d + j + half]);
  const float s2 = to_f32(sin_t[(long)t * d + j + half]);
  const long o = ((long)h * N + t) * d;
  {
    const float x1 = to_f32(row[j]), x2 = to_f32(row[j + half]);
    qo[o + j] = from_f32<T>(__builtin_fmaf(x1, c1, -(x2 * s1)));
    qo[o + j + half] = from_f32<T>(__builtin_fmaf(x1, s2, x2 * c2));
  }
  {
    const float x1 = to_f32(row[hidden + j]), x2 = to_f32(row[hidden + j + half]);
    ko[o + j] = from_f32<T>(__builtin_fmaf(x1, c1, -(x2 * s1)));
    ko[o + j + half] = from_f32<T>(__builtin_fmaf(x1, s2, x2 * c2));
  }
  vo[o + j] = row[2 * hidden + j];
  vo[o + j + half] = row[2 * hidden + j + half];
}

// Vectorised form for d/2 % 4 == 0 (d = 64, 72, 80, 128 ...): a workgroup owns kVisTok
// consecutive tokens and every (q|k|v, head) of them; item (which, h, t, c) moves elements
// [4c, 4c+4) of both halves of one head row.  c runs fastest, then t, so a wave's stores
// for one head cover kVisTok contiguous output rows and its loads stay inside the
// workgroup's kVisTok input rows (read from HBM once, reused through L2).
constexpr int kVisTok = 8;

template <typename T>
union Chunk4 {
  typename std::conditional<sizeof(T) == 2, u32x2, u32x4>::type raw;
  T e[4];
};

template <typename T>
__device__ __forceinline__ Chunk4<T> load4(const T* p) {
  Chunk4<T> c;
  c.raw = *reinterpret_cast<const decltype(c.raw)*>(p);
  return c;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const Chunk4<T>& c) {
  *reinterpret_cast<decltype(c.raw)*>(p) = c.raw;
}

template <typename T>
__global__ void __launch_bounds__(kProdThreads)
vision_qkv4_kernel(const T* qkv, const T* cos_t, const T* sin_t, T* qo, T* ko, T* vo, int N, int H,
                   int d) {
  const int half = d / 2, chunks = half / 4;
  const int t0 = blockIdx.x * kVisTok;
  const int nt = min(kVisTok, N - t0);
  const long hidden = (long)H * d;
  const int per_head = nt * chunks;
  const int items = 3 * H * per_head;
  for (int i = threadIdx.x; i < items; i += kProdThreads) {
    const int wh = i / per_head;  // which * H + h
    const int r = i - wh * per_head;
    const int tl = r / chunks, j = (r - tl * chunks) * 4;
    const int which = wh / H, h = wh - which * H;
    const int t = t0 + tl;
    const T* src = qkv + (long)t * 3 * hidden + (long)which * hidden + (long)h * d + j;
    const long o = ((long)h * N + t) * d + j;
    T* dst = which == 0 ? qo : which == 1 ? ko : vo;
    Chunk4<T> x1 = load4(src), x2 = load4(src + half);
    if (which < 2) {
      const long tb = (long)t * d + j;
      const Chunk4<T> c1 = load4(cos_t + tb), s1 = load4(sin_t + tb);
      const Chunk4<T> c2 = load4(cos_t + tb + half), s2 = load4(sin_t + tb + half);
      Chunk4<T> y1, y2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = to_f32(x1.e[e]), b = to_f32(x2.e[e]);
        y1.e[e] = from_f32<T>(__builtin_fmaf(a, to_f32(c1.e[e]), -(b * to_f32(s1.e[e]))));
        y2.e[e] = from_f32<T>(__builtin_fmaf(a, to_f32(s2.e[e]), b * to_f32(c2.e[e])));
      }
      x1 = y1;
      x2 = y2;
    }
    store4(dst + o, x1);
    store4(dst + o + half, x2);
  }
}

unsigned grid_for(long items) { return (unsigned)((items + kProdThreads - 1) / kProdThreads); }

template <typename F>
hipError_t by_dtype(int dtype, F&& f) {
  switch (dtype) {
    case kF32: return f(float{});
    case kF16: return f(f16{});
    case kBF16: return f(bf16{});
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_kv_append(void* cache, const void* src, const int* pos, int kv_dim,
                            long layer_off, int dtype, hipStream_t stream) {
  return by_dtype(dtype, [&](auto z) {
    using T = decltype(z);
    constexpr int VEC = 16 / (int)sizeof(T);
    const long chunks = (kv_dim + VEC - 1) / VEC;
    hipLaunchKernelGGL(kv_append_kernel<T>, dim3(grid_for(chunks)), dim3(kProdThreads), 0, stream,
                       reinterpret_cast<T*>(cache), reinterpret_cast<const T*>(src), pos, kv_dim,
                       layer_off);
    return hipGetLastError();
  });
}

hipError_t launch_kv_scatter(const void* k_src, const void* v_src, void* k_pool, void* v_pool,
                             const int* slots, long src_row_stride, int n_rows, int kv_heads,
                             int head_size, int block_size, int head_major, int dtype,
                             hipStream_t stream) {
  ScatterArgs a{k_src, v_src, k_pool, v_pool, slots, src_row_stride,
                n_rows, kv_heads, head_size, block_size, head_major};
  return by_dtype(dtype, [&](auto z) {
    using T = decltype(z);
    const long chunks = (long)n_rows * kv_heads * (head_size / (16 / (int)sizeof(T)));
    if (chunks <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_scatter_kernel<T>, dim3(grid_for(chunks)), dim3(kProdThreads), 0,
                       stream, a);
    return hipGetLastError();
  });
}

hipError_t launch_kv_convert(void* contig, void* pool, const int* block_table,
                             long contig_row_stride, int n_tokens, int kv_heads, int head_size,
                             int block_size, int head_major, int to_paged, int dtype,
                             hipStream_t stream) {
  ConvertArgs a{contig, pool, block_table, contig_row_stride, n_tokens,
                kv_heads, head_size, block_size, head_major, to_paged};
  return by_dtype(dtype, [&](auto z) {
    using T = decltype(z);
    const long chunks = (long)n_tokens * kv_heads * (head_size / (16 / (int)sizeof(T)));
    if (chunks <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_convert_kernel<T>, dim3(grid_for(chunks)), dim3(kProdThreads), 0,
                       stream, a);
    return hipGetLastError();
  });
}

bool norm_rope_supports(int dtype, int head_size) {
  return (dtype == kF32 || dtype == kF16 || dtype == kBF16) &&
         (head_size == 64 || head_size == 128 || head_size == 256);
}

hipError_t launch_qk_norm_rope(void* q, const void* k, const void* v, const void* q_weight,
                               const void* k_weight, const float* sin_cache,
                               const float* cos_cache, void* k_cache, void* v_cache,
                               long cache_tok_stride, const int* pos_ptr, int start_pos,
                               int seq_len, int Hq, int Hkv, int head_size, float eps, int dtype,
                               hipStream_t stream) {
  NormRopeArgs a{q, k, v, q_weight, k_weight, sin_cache, cos_cache, k_cache, v_cache,
                 cache_tok_stride, pos_ptr, start_pos, seq_len, Hq, Hkv, head_size, eps};
  const long units = (long)seq_len * ((q ? Hq : 0) + Hkv);
  if (units <= 0) return hipSuccess;
  return by_dtype(dtype, [&](auto z) {
    using T = decltype(z);
    const long lpu = head_size / 2 / (16 / (long)sizeof(T));
    const unsigned grid = grid_for(units * lpu);
    if (head_size == 64)
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, 64>), dim3(grid), dim3(kProdThreads), 0, stream,
                         a);
    else if (head_size == 128)
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, 128>), dim3(grid), dim3(kProdThreads), 0, stream,
                         a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, 256>), dim3(grid), dim3(kProdThreads), 0, stream,
                         a);
    return hipGetLastError();
  });
}

hipError_t launch_rope_cache(float* sin_cache, float* cos_cache, int head_size, int max_pos,
                             float theta, hipStream_t stream) {
  const long n = (long)head_size * max_pos;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_cache_kernel, dim3(grid_for(n)), dim3(kProdThreads), 0, stream,
                     sin_cache, cos_cache, head_size, max_pos, theta);
  return hipGetLastError();
}

hipError_t launch_vision_qkv(const void* qkv, const void* cos_t, const void* sin_t, void* q,
                             void* k, void* v, int N, int H, int d, int dtype,
                             hipStream_t stream) {
  return by_dtype(dtype, [&](auto z) {
    using T = decltype(z);
    const long n = (long)N * H * (d / 2);
    if (n <= 0) return hipSuccess;
    if ((d / 2) % 4 == 0) {
      hipLaunchKernelGGL(vision_qkv4_kernel<T>, dim3((N + kVisTok - 1) / kVisTok),
                         dim3(kProdThreads), 0, stream, reinterpret_cast<const T*>(qkv),
                         reinterpret_cast<const T*>(cos_t), reinterpret_cast<const T*>(sin_t),
                         reinterpret_cast<T*>(q), reinterpret_cast<T*>(k),
                         reinterpret_cast<T*>(v), N, H, d);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(vision_qkv_kernel<T>, dim3(grid_for(n)), dim3(kProdThreads), 0, stream,
                       reinterpret_cast<const T*>(qkv), reinterpret_cast<const T*>(cos_t),
                       reinterpret_cast<const T*>(sin_t), reinterpret_cast<T*>(q),
                       reinterpret_cast<T*>(k), reinterpret_cast<T*>(v), N, H, d);
    return hipGetLastError();
  });
}

}  // namespace orin
