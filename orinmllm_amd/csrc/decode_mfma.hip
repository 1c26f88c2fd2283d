// Matrix-core decode attention for 16-bit KV caches on gfx950.
//
// Serves the same launches as decode.hip (the reference's single-query attention,
// kuiper/source/op/kernels/cuda/flash_attention_kernel.cu:966-1175 and mha_kernel.cu:162-338,
// plus the batched / paged decode) for fp16 / bf16 K and V, head sizes 64 and 128, and up
// to 16 query heads per kv head.
//
// Why a second decode kernel.  launch_decode sends it the launches whose rows are not split
// (one workgroup per (row, kv head)), where a single CU must stream a whole row: here the
// two contractions run on the matrix cores, the VALU work per 32-token tile is the softmax
// of 8 scores per lane, and the loads are whole coalesced rows.  Measured on the batch-32
// paged decode (fp16, d 128, lengths U[512, 4096]), whole rows: this kernel 0.64 of HBM,
// the dot-product kernel's 16-wave workgroups 0.59; a copy of this kernel with the
// arithmetic removed 0.67, so what remains is the rate at which one CU streams a row
// (~36 GB/s), not its arithmetic.  Split launches stay on the dot-product kernel (this one
// with 1024-token splits and the merge launch: 0.53-0.54).
//
// Work decomposition.  A workgroup of 4 waves owns one (row, kv head, split) and all G
// query heads of that kv head (G <= 16, padded to 16 columns).  Wave w takes the 32-token
// tiles w, w + 4, ... of the split, with its own online-softmax state; the waves are merged
// once through LDS at the end.  Per tile:
//   S^T[32 x 16] = K[32 x D] . Q^T[D x 16]        2 x D/32  v_mfma_f32_16x16x32
//   O^T[D x 16] += V^T[D x 32] . P^T[32 x 16]     D/16      v_mfma_f32_16x16x32 (fp16)
//                                                 2 x D/16  (bf16: P = hi + lo, both bf16)
//   K and V arrive as whole rows (one load instruction covers 1 KB of consecutive rows) and
//   are written to per-wave LDS tiles.  Lane (n, g) = (lane % 16, lane / 16) reads K row n
//   (and n + 16), 16-byte chunk 4 j + g, which is the A layout of QK^T MFMA j with the
//   contraction index permuted identically in Q^T.  The S^T accumulator leaves lane (n, g)
//   the scores of head n for tokens 4g .. 4g+3 and 16 + 4g .. +3, which is the B layout of
//   P^T in the PV MFMAs.  V^T fragments come from ds_read_b64_tr_b16, which hands lane
//   (n, g) the four tokens 4g .. 4g+3 of dimension n from the row-major tile.  K rows are
//   stored with chunk c of row r at c ^ r (d 64: c ^ (r / 2)), V rows at c ^ (2r & 14):
//   both fragment reads are then free of bank conflicts.  Each wave keeps the next tile's
//   loads in flight while it computes the current one.
//
// Numerics match decode.hip: scores and the normaliser l in fp32, weights P rounded to
// fp16 for fp16 caches.  For bf16 caches P is split into bf16 hi + lo (hi + lo carries 16
// significant bits) and V stays bf16, so V keeps bf16's full range.  Paged and contiguous
// launches of the same KV run the same arithmetic and give identical bits.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "decode_rows.h"

namespace orin {

namespace {

constexpr int kMWaves = 4;
constexpr int kMThreads = kMWaves * kWave;
constexpr int kMTile = 32;  // tokens per wave tile
// A wave keeps its running maximum while every weight stays at most 2^kMLazyLog2.
constexpr float kMLazyLog2 = 8.0f;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <typename T>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16<f16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<bf16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Packs two fp32 values into a 16-bit pair (round to nearest even).
template <typename T>
__device__ __forceinline__ uint32_t pack2m(float x, float y) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, T2{(T)x, (T)y});
}

__device__ __forceinline__ float xor16(float x) { return shfl_xor_f(x, 16); }
__device__ __forceinline__ float xor32(float x) { return shfl_xor_f(x, 32); }

template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(kMThreads) decode_mfma_kernel(DecodeArgs a) {
  constexpr int NQK = D / 32;  // QK^T MFMAs per 16-token half (16-byte K pieces per token)
  constexpr int NDT = D / 16;  // 16-wide output tiles of O^T
  constexpr bool kBf16 = std::is_same<T, bf16>::value;
  static_assert(D == 64 || D == 128, "head size 64 or 128");
  // Per-wave K and V tiles (32 rows of D elements each) while the loop runs; the merge
  // reuses the space.
  extern __shared__ __attribute__((aligned(16))) char smem[];

  int bid = blockIdx.x;
  const int kvh = bid % a.Hkv;
  bid /= a.Hkv;
  const int split = bid % a.max_splits;
  const int row = bid / a.max_splits;
  const int G = a.kv_mul;
  const int h0 = kvh * G;

  const int len = row_len(a, row);
  const int nsplit = len > 0 ? (len + a.split_tokens - 1) / a.split_tokens : 0;
  T* out = reinterpret_cast<T*>(a.o) + (long)row * a.o_row_stride;
  if (len > a.len_cap || len <= 0) {  // past the launch bound: NaN; empty row: zeros
    if (split == 0) {
      const float fill = len > 0 ? __builtin_nanf("") : 0.f;
      for (int i = threadIdx.x; i < G * D; i += kMThreads)
        out[(long)(h0 + i / D) * a.o_head_stride + i % D] = from_f32<T>(fill);
    }
    return;
  }
  if (split >= nsplit) return;
  const int s0 = split * a.split_tokens;
  const int s1 = min(s0 + a.split_tokens, len);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;  // head column / token within a 16-token half / V^T dimension
  const int g = lane >> 4;  // 16-byte piece group

  // ---------------------------------------------------------------- address map
  const long tok_bytes = a.kv_tok_stride * (long)sizeof(T);
  const char* kbase = reinterpret_cast<const char*>(a.k) + a.kv_head_stride * (long)sizeof(T) * kvh;
  const char* vbase = reinterpret_cast<const char*>(a.v) + a.kv_head_stride * (long)sizeof(T) * kvh;
  const __attribute__((address_space(4))) int* bt = nullptr;
  long blk_bytes = 0;
  int bmask = 0;
  if constexpr (PAGED) {
    bt = (const __attribute__((address_space(4))) int*)(a.block_table + (long)row * a.bt_row_stride);
    blk_bytes = a.block_stride * (long)sizeof(T);
    bmask = (1 << a.bs_log2) - 1;
  } else {
    // contiguous: token t of the row is at element base + t * kv_tok_stride
    const long base = a.cu_seqlens
                          ? (long)a.cu_seqlens[find_segment(a.cu_seqlens, a.n_seg, row)] * a.kv_tok_stride
                          : (long)row * a.kv_row_stride;
    kbase += base * (long)sizeof(T);
    vbase += base * (long)sizeof(T);
  }
  // Block ids of the four 8-token groups of the tile at t0 (paged): scalar loads.
  struct Blocks {
    int b[4];
  };
  auto tile_blocks = [&](int t0) __attribute__((always_inline)) {
    Blocks r;
#pragma unroll
    for (int q = 0; q < 4; ++q) r.b[q] = PAGED ? bt[min(t0 + 8 * q, s1 - 1) >> a.bs_log2] : 0;
    return r;
  };
  // Coalesced loads: instruction i of a tile covers rows RPI*i .. RPI*i + RPI-1 (whole rows,
  // RPI = 1 KB / row bytes), lane l row RPI*i + l / CPR, 16-byte chunk l % CPR.  Those rows
  // lie in one aligned 8-token group, so their block id is wave-uniform.
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int RPI = kWave / CPR;  // rows per load instruction
  constexpr int NLI = kMTile / RPI; // load instructions per tile (each of K and V)
  const int lrow = lane / CPR, lchunk = lane % CPR;
  // Row base (wave-uniform byte offset) and lane offset of load instruction i; rows past
  // the split read row s1 - 1.
  const uint32_t tok_b32 = (uint32_t)tok_bytes;
  auto row_base = [&](int t0, int i, const Blocks& bl) __attribute__((always_inline)) {
    const int rt = min(t0 + RPI * i, s1 - 1);
    if constexpr (PAGED) return (long)bl.b[(RPI * i) / 8] * blk_bytes + (long)(rt & bmask) * tok_bytes;
    return (long)rt * tok_bytes;
  };
  auto lane_off = [&](int t0, int i) __attribute__((always_inline)) {
    const int rt = min(t0 + RPI * i, s1 - 1);
    return (uint32_t)(min(t0 + RPI * i + lrow, s1 - 1) - rt) * tok_b32 + (uint32_t)(lchunk * 16);
  };

  // ---------------------------------------------------------------- Q^T operand
  // B operand of QK^T MFMA (h, j): lane (n, g) holds q[head h0 + n][32 j + 8 g .. +7]
  // (zero for columns n >= G).
  u32x4 qf[NQK];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (long)row * a.q_row_stride +
                  (long)(h0 + n) * a.q_head_stride + 8 * g;
#pragma unroll
    for (int j = 0; j < NQK; ++j)
      qf[j] = n < G ? *reinterpret_cast<const u32x4*>(qp + 32 * j) : u32x4{0u, 0u, 0u, 0u};
  }

  // ---------------------------------------------------------------- LDS K / V tiles
  // Per wave: K tile then V tile, 32 rows of D elements each.
  char* const kt = smem + wave * (2 * kMTile * D * 2);
  char* const vt = kt + kMTile * D * 2;
  // K: row r, chunk c at chunk c ^ fk(r); the fragment reads (16 rows, one chunk) are then
  // conflict-free.  V: chunk c ^ (2r & 14), conflict-free for the transposing reads.
  auto kt_chunk = [&](int r, int c) __attribute__((always_inline)) {
    const int f = (D == 128 ? r : (r >> 1)) & (CPR - 1);
    return r * (D * 2) + ((c ^ f) * 16);
  };
  auto vt_chunk = [&](int r, int c) __attribute__((always_inline)) {
    return r * (D * 2) + ((c ^ ((2 * r) & (CPR - 1) & 14)) * 16);
  };
  // ds_read_b64_tr_b16 address of lane (n, g) = (4e + q4 within the 16-lane group g):
  // row 16 hh + 4 g + e, dimensions 16 t + 4 q4 .. +3 (one half of a 16-byte chunk).
  const int tr_e = n >> 2, tr_q = n & 3;

  f32x4 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;  // head n: running maximum (log2 units), lane's weight sum
  const float c = a.scale_log2;

  // Loads of one tile: whole K and V rows, NLI 16-byte pieces per lane each.
  struct Regs {
    u32x4 k[NLI];
    u32x4 v[NLI];
  };
  auto load_tile = [&](Regs& r, int t0, const Blocks& bl) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      const long rb = row_base(t0, i, bl);
      const uint32_t lo = lane_off(t0, i);
      r.k[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kbase + rb + lo));
      r.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + rb + lo));
    }
  };

  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  typedef __attribute__((address_space(3))) char lds_char;
  auto compute_tile = [&](const Regs& r, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      *reinterpret_cast<lds_u32x4*>((lds_char*)(kt + kt_chunk(RPI * i + lrow, lchunk))) = r.k[i];
      *reinterpret_cast<lds_u32x4*>((lds_char*)(vt + vt_chunk(RPI * i + lrow, lchunk))) = r.v[i];
    }
    // K fragments: lane (n, g) reads row 16 h + n, chunk 4 j + g.
    u32x4 kf[2][NQK];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < NQK; ++j)
        kf[h][j] = *reinterpret_cast<const lds_u32x4*>((lds_char*)(kt + kt_chunk(16 * h + n, 4 * j + g)));
    // S^T halves: tokens 4g + i (h = 0) and 16 + 4g + i of head n.
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NQK; ++j) s[h] = mfma16<T>(kf[h][j], qf[j], s[h]);
    }
    float x[8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = t0 + 16 * h + 4 * g + i;
        x[4 * h + i] = tok < s1 ? s[h][i] * c : -INFINITY;
      }
    // Lazy running maximum: raised only when a weight would exceed 2^8 (and on the first
    // tile, m = -inf); the four lanes of a head column agree on m.
    bool raise = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) raise |= x[i] - m > kMLazyLog2;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      float tm = x[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) tm = fmaxf(tm, x[i]);
      tm = fmaxf(tm, xor16(tm));
      tm = fmaxf(tm, xor32(tm));
      const float mn = fmaxf(m, tm);
      const float alpha = fast_exp2(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) oacc[t][i] *= alpha;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = fast_exp2(x[i] - m);
      lsum += p[i];
    }
    // B operand P^T: items 0-3 = tokens 4g + i, items 4-7 = tokens 16 + 4g + i.
    u32x4 pb, pl;
    if constexpr (!kBf16) {
      pb = u32x4{pack2m<f16>(p[0], p[1]), pack2m<f16>(p[2], p[3]), pack2m<f16>(p[4], p[5]),
                 pack2m<f16>(p[6], p[7])};
    } else {
      float lo[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) lo[i] = p[i] - (float)(bf16)p[i];
      pb = u32x4{pack2m<bf16>(p[0], p[1]), pack2m<bf16>(p[2], p[3]), pack2m<bf16>(p[4], p[5]),
                 pack2m<bf16>(p[6], p[7])};
      pl = u32x4{pack2m<bf16>(lo[0], lo[1]), pack2m<bf16>(lo[2], lo[3]),
                 pack2m<bf16>(lo[4], lo[5]), pack2m<bf16>(lo[6], lo[7])};
    }
    // V^T tiles from LDS.  The writes above come first in this wave's LDS queue.
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      u32x2 part[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int rr = 16 * hh + 4 * g + tr_e;
        const int col = 16 * t + 4 * tr_q;  // element column
        const int off = vt_chunk(rr, col >> 3) + (col & 7) * 2;
        const s16x4 v4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)((__attribute__((address_space(3))) char*)(vt + off)));
        part[hh] = __builtin_bit_cast(u32x2, v4);
      }
      const u32x4 va = u32x4{part[0][0], part[0][1], part[1][0], part[1][1]};
      if constexpr (!kBf16) {
        oacc[t] = mfma16<f16>(va, pb, oacc[t]);
      } else {
        oacc[t] = mfma16<bf16>(va, pb, oacc[t]);
        oacc[t] = mfma16<bf16>(va, pl, oacc[t]);
      }
    }
  };

  // ---------------------------------------------------------------- tile loop
  constexpr int step = kMWaves * kMTile;
  // Wave w runs tiles t = w, w + 8, ... (n_w of them).  Block ids are requested one tile
  // ahead of the loads that use them.  Loads are issued unconditionally, two buffers deep,
  // so that every wait before a tile's use is the same vmcnt: past the end of the split
  // every lane's token clamps to s1 - 1 and the tile reads one 256-byte row.
  const int tw0 = s0 + wave * kMTile;
  const int n_w = tw0 < s1 ? (s1 - tw0 + step - 1) / step : 0;
  if (n_w > 0) {
    Regs ra, rb;
    load_tile(ra, tw0, tile_blocks(tw0));
    Blocks bn = tile_blocks(tw0 + step);
    for (int i = 0;; i += 2) {
      const int t0 = tw0 + i * step;
      load_tile(rb, t0 + step, bn);
      bn = tile_blocks(t0 + 2 * step);
      __builtin_amdgcn_sched_barrier(0);  // the next tile's loads go out before this tile's work
      compute_tile(ra, t0);
      if (i + 1 >= n_w) break;
      load_tile(ra, t0 + 2 * step, bn);
      bn = tile_blocks(t0 + 3 * step);
      __builtin_amdgcn_sched_barrier(0);
      compute_tile(rb, t0 + step);
      if (i + 2 >= n_w) break;
    }
  }

  // ---------------------------------------------------------------- merge the waves
  lsum += xor16(lsum);
  lsum += xor32(lsum);
  __syncthreads();  // every wave is done with its V tile
  float* s_m = reinterpret_cast<float*>(smem);      // [waves][16]
  float* s_l = s_m + kMWaves * 16;                  // [waves][16]
  float* s_o = s_l + kMWaves * 16;                  // [waves][G][D]
  if (g == 0) {
    s_m[wave * 16 + n] = m;
    s_l[wave * 16 + n] = lsum;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kMWaves; ++w) M = fmaxf(M, s_m[w * 16 + n]);
  const float f = m == -INFINITY ? 0.f : fast_exp2(m - M);
  if (n < G) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_o[(wave * G + n) * D + 16 * t + 4 * g + i] = oacc[t][i] * f;
  }
  __syncthreads();
  const bool direct = nsplit == 1;
  for (int i = threadIdx.x; i < G * D; i += kMThreads) {
    const int hn = i / D, dd = i % D;
    float Mh = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) Mh = fmaxf(Mh, s_m[w * 16 + hn]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      const float mw = s_m[w * 16 + hn];
      L += mw == -INFINITY ? 0.f : fast_exp2(mw - Mh) * s_l[w * 16 + hn];
      o += s_o[(w * G + hn) * D + dd];
    }
    if (direct) {
      out[(long)(h0 + hn) * a.o_head_stride + dd] = from_f32<T>(o / L);
    } else {
      float* pp = a.ws + ((((long)row * a.Hq + h0 + hn) * a.max_splits + split) * (D + 2));
      pp[dd] = o;
      if (dd == 0) {
        pp[D] = Mh;
        pp[D + 1] = L;
      }
    }
  }
}

template <typename T, int D, bool PAGED>
hipError_t launch_tp(const DecodeArgs& a, hipStream_t stream) {
  const long blocks = (long)a.n_rows * a.Hkv * a.max_splits;
  const size_t lds = decode_mfma_lds_bytes(D);
  const void* fn = (const void*)decode_mfma_kernel<T, D, PAGED>;
  // More than 64 KB of dynamic LDS must be granted per kernel (once per device).
  static unsigned long long configured = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 64 || !(__atomic_load_n(&configured, __ATOMIC_ACQUIRE) & (1ull << dev))) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    if (dev < 64) __atomic_fetch_or(&configured, 1ull << dev, __ATOMIC_RELEASE);
  }
  hipLaunchKernelGGL((decode_mfma_kernel<T, D, PAGED>), dim3((unsigned)blocks), dim3(kMThreads),
                     lds, stream, a);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_t(const DecodeArgs& a, hipStream_t stream) {
  return a.block_table ? launch_tp<T, D, true>(a, stream) : launch_tp<T, D, false>(a, stream);
}

}  // namespace

size_t decode_mfma_lds_bytes(int head_size) {
  const size_t tiles = (size_t)kMWaves * 2 * kMTile * head_size * 2;
  const size_t merge = (size_t)kMWaves * 16 * (2 + head_size) * sizeof(float);  // G <= 16
  return tiles > merge ? tiles : merge;
}

bool decode_mfma_supports(int dtype, int head_size, int kv_mul) {
  return (dtype == kF16 || dtype == kBF16) && (head_size == 64 || head_size == 128) &&
         kv_mul >= 1 && kv_mul <= 16;
}

hipError_t launch_decode_mfma(const DecodeArgs& a, int dtype, hipStream_t stream) {
  if (dtype == kF16)
    return a.head_size == 64 ? launch_t<f16, 64>(a, stream) : launch_t<f16, 128>(a, stream);
  return a.head_size == 64 ? launch_t<bf16, 64>(a, stream) : launch_t<bf16, 128>(a, stream);
}

}  // namespace orin
