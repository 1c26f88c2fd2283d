// Split-KV decode attention for gfx950.
//
// Replaces the reference's single-query attention kernels
// (kuiper/source/op/kernels/cuda/mha_kernel.cu:162-338,
//  flash_attention_kernel.cu:205-535 and :966-1175,
//  flash_attention2_kernel.cu:409-816) with one design:
//
//  * A workgroup (4 waves) owns one (row, kv head, head group, split): it reads that
//    split's K/V once and serves the G query heads that share the kv head (GQA), so KV
//    bytes are read from HBM once per kv head instead of once per query head.
//  * Scores: 8 lanes own one token.  Lane k of the group loads the 16-byte chunks
//    [128n + 16k, +16) of the token's K row (n < NV), so each load instruction covers
//    8 tokens x 128 contiguous bytes; q.k is a per-lane dot2 followed by a 3-step DPP
//    all-reduce over the 8 lanes.
//  * Values: each lane owns D/64 consecutive output elements for every token.  A V row
//    is one coalesced whole-wave load (D*sizeof(T)/64 bytes per lane) whose address is
//    wave-uniform; each softmax weight is broadcast from the lane group that computed
//    it with v_readlane (a scalar operand of the FMAs).  The accumulator is G * D/64 floats per lane and needs no
//    cross-lane reduction at the end.
//  * Each wave keeps its own online-softmax state over its tiles (no barrier per tile);
//    the 4 waves are merged once through LDS.  Each wave software-pipelines its tiles:
//    the next tile's K rows are requested once the current scores exist, its V rows
//    once the current PV is done.
//  * Splits are fixed-size ranges of logical token positions.  A row needing more than
//    one split writes (acc, m, l) partials to the workspace and decode_combine merges
//    them; a single-split row writes its output directly.
//  * Token addresses come from a contiguous map (optionally per varlen segment) or a
//    paged block table.  The arithmetic does not depend on the map, so paged and
//    contiguous decode of the same KV are bit-identical.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "decode_rows.h"

namespace orin {

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;
constexpr int kMaxCombineSplits = 1024;  // the host sizes splits so a row has at most this many
// A wave keeps its running maximum while every weight stays at most 2^kDecodeLazyLog2.
constexpr float kDecodeLazyLog2 = 8.0f;
// Whole-row mode: one 16-wave workgroup (a whole CU at 128 VGPRs) per (row, kv head, head
// group), no partials.  Only the shapes whose loop fits 128 VGPRs without spilling use it
// (16-bit K/V: head size 128 with up to 4 heads per group, 64 with up to 3; fp32: head
// size 64 with 1 head per group).
constexpr int kWideWaves = 16;
template <typename T, int D, int G>
constexpr bool wide_fits() {
  if (sizeof(T) == 4) return D == 64 && G == 1;
  return (D == 128 && G <= 4) || (D == 64 && G <= 3);
}

template <typename T, int D>
struct DecodeShape {
  static constexpr int kRowBytes = D * (int)sizeof(T);
  static_assert(kRowBytes % 128 == 0, "head row must be a multiple of 128 bytes");
  static constexpr int NV = kRowBytes / 128;              // K: 16-byte chunks per lane per token
  static constexpr int VEC = 16 / (int)sizeof(T);         // K: elements per chunk
  static constexpr int CH_STRIDE = 128 / (int)sizeof(T);  // K: elements between a lane's chunks
  static constexpr int STEPS = (NV == 2) ? 2 : (NV == 1 ? 4 : (NV >= 8 ? 1 : 8 / NV));
  static constexpr int TILE = STEPS * 8;                  // tokens per wave tile
  static constexpr int EPL = D / kWave;                   // V: elements per lane
  static constexpr int VB = EPL * (int)sizeof(T);         // V: bytes per lane per token
};

// Raw V fragment of one lane (VB bytes) and its conversion to fp32.
template <int VB>
struct VRaw;
template <>
struct VRaw<2> { typedef uint16_t type; };
template <>
struct VRaw<4> { typedef uint32_t type; };
template <>
struct VRaw<8> { typedef u32x2 type; };
template <>
struct VRaw<16> { typedef u32x4 type; };

template <typename T, int EPL, typename R>
__device__ __forceinline__ void v_unpack(const R& r, float* out) {
  if constexpr (sizeof(T) == 4) {
    typedef float fv __attribute__((ext_vector_type(EPL)));
    const fv x = __builtin_bit_cast(fv, r);
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = x[i];
  } else if constexpr (EPL == 1) {
    out[0] = (float)__builtin_bit_cast(T, r);
  } else {
    typedef T hv __attribute__((ext_vector_type(EPL)));
    const hv x = __builtin_bit_cast(hv, r);
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = (float)x[i];
  }
}

// Interleave two tokens' 16-bit V fragments: out[e] = (a.e, b.e) as a 16-bit pair.
template <int EPL>
__device__ __forceinline__ void pair_rows(uint16_t a, uint16_t b, uint32_t* out) {
  out[0] = (uint32_t)a | ((uint32_t)b << 16);
}
template <int EPL>
__device__ __forceinline__ void pair_rows(uint32_t a, uint32_t b, uint32_t* out) {
  out[0] = __builtin_amdgcn_perm(b, a, 0x05040100u);  // (a.lo, b.lo)
  out[1] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // (a.hi, b.hi)
}
template <int EPL>
__device__ __forceinline__ void pair_rows(u32x2 a, u32x2 b, uint32_t* out) {
  const uint32_t a0 = __builtin_bit_cast(u32x2, a).x, a1 = __builtin_bit_cast(u32x2, a).y;
  const uint32_t b0 = __builtin_bit_cast(u32x2, b).x, b1 = __builtin_bit_cast(u32x2, b).y;
  out[0] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(b0, a0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(b1, a1, 0x07060302u);
}

// acc + p.x*v.x + p.y*v.y on 16-bit pairs (fp32 accumulate).
template <typename T>
__device__ __forceinline__ float dot2(uint32_t p, uint32_t v, float acc);
template <>
__device__ __forceinline__ float dot2<f16>(uint32_t p, uint32_t v, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), __builtin_bit_cast(f16x2, v), acc,
                                false);
}
template <>
__device__ __forceinline__ float dot2<bf16>(uint32_t p, uint32_t v, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p),
                                         __builtin_bit_cast(bf16x2, v), acc, false);
}

// Address map of one row's KV sequence.  Offsets are in elements, relative to the
// k/v base pointer (kv head offset excluded).  A token's row is
//   contiguous: base + tok * tok_stride
//   paged:      blk * block_stride + (tok % block_size) * tok_stride,
//               blk = block_table[tok / block_size]
// Paged: every 8-token K step (and every single V token) lies inside one block
// (block_size >= 8, steps start at multiples of 8), so the block id is wave-uniform and
// read with a scalar load, which does not wait on the vector loads in flight.
template <bool PAGED>
struct TokenMap {
  long base;          // contiguous: element offset of token 0 of this row
  long tok_stride;    // elements between consecutive token rows
  long block_stride;  // paged: elements between consecutive pool blocks
  const __attribute__((address_space(4))) int* bt_row;  // paged: this row's block table
  int bs_log2;
  __device__ __forceinline__ int block_of(int tok) const {
    return PAGED ? bt_row[tok >> bs_log2] : 0;
  }
  // Element offset of the row of token `tok`, whose block id is `blk`.
  __device__ __forceinline__ long row_offset(int tok, int blk) const {
    if (PAGED)
      return (long)blk * block_stride + (long)(tok & ((1 << bs_log2) - 1)) * tok_stride;
    return (long)tok * tok_stride;
  }
};

template <typename T, int D, int G, bool PAGED, int NW>
__global__ void __launch_bounds__(NW * kWave)
decode_split_kernel(DecodeArgs a) {
  using S = DecodeShape<T, D>;
  constexpr int NV = S::NV, VEC = S::VEC, STEPS = S::STEPS, TILE = S::TILE, EPL = S::EPL;
  typedef typename VRaw<S::VB>::type VR;

  // Block order: kv head fastest, so the workgroups reading the Hkv interleaved head
  // slices of the same token rows run together (DRAM row locality); then head group,
  // split, row.
  const int n_hg = a.kv_mul / G;
  int bid = blockIdx.x;
  const int kvh = bid % a.Hkv;
  bid /= a.Hkv;
  const int hg = bid % n_hg;
  bid /= n_hg;
  const int split = bid % a.max_splits;
  const int row = bid / a.max_splits;

  const int len = row_len(a, row);
  const int s0 = split * a.split_tokens;
  const int h0 = kvh * a.kv_mul + hg * G;
  const int nsplit = len > 0 ? (len + a.split_tokens - 1) / a.split_tokens : 0;

  T* out = reinterpret_cast<T*>(a.o) + (long)row * a.o_row_stride;
  if (len > a.len_cap) {  // longer than the launch covers: NaN output
    if (split == 0)
      for (int i = threadIdx.x; i < G * D; i += NW * kWave)
        out[(long)(h0 + i / D) * a.o_head_stride + i % D] = from_f32<T>(__builtin_nanf(""));
    return;
  }
  if (len <= 0) {  // empty row: output zeros
    if (split == 0)
      for (int i = threadIdx.x; i < G * D; i += NW * kWave)
        out[(long)(h0 + i / D) * a.o_head_stride + i % D] = from_f32<T>(0.f);
    return;
  }
  if (split >= nsplit) return;
  const int s1 = min(s0 + a.split_tokens, len);

  TokenMap<PAGED> map;
  map.tok_stride = a.kv_tok_stride;
  map.block_stride = a.block_stride;
  map.bs_log2 = a.bs_log2;
  map.bt_row = (const __attribute__((address_space(4))) int*)(
      a.block_table + (PAGED ? (long)row * a.bt_row_stride : 0));
  map.base = 0;
  if (!PAGED) {
    map.base = a.cu_seqlens
                   ? (long)a.cu_seqlens[find_segment(a.cu_seqlens, a.n_seg, row)] * a.kv_tok_stride
                   : (long)row * a.kv_row_stride;
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k8 = lane & 7;    // K chunk slot inside the token's row
  const int grp = lane >> 3;  // K token group (0..7)

  // Wave-uniform bases; per-lane parts are 32-bit offsets added at the load.
  const T* kb = reinterpret_cast<const T*>(a.k) + (long)kvh * a.kv_head_stride + map.base;
  const T* vb = reinterpret_cast<const T*>(a.v) + (long)kvh * a.kv_head_stride + map.base;
  const int k_lane = k8 * VEC;
  const int v_lane = lane * EPL;

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

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  const float c = a.scale_log2;
  // Per-lane offsets (elements) inside an 8-token step, used when the whole tile lies
  // below s1: K token group grp, V token r.
  // Offsets are unsigned 32-bit byte offsets from a wave-uniform row base, so the loads use
  // the SGPR-base + VGPR-offset addressing form instead of 64-bit per-lane addresses.
  const uint32_t k_off = (uint32_t)(grp * (int)map.tok_stride + k_lane) * sizeof(T);
  uint32_t v_off[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) v_off[r] = (uint32_t)(r * (int)map.tok_stride + v_lane) * sizeof(T);

  // Block ids of the K steps / V tokens of the tile at t0.  In a tile that crosses s1,
  // tokens >= s1 read row s1-1 (finite data; their weights are 0).
  auto k_blocks = [&](int (&blk)[STEPS], int t0) {
#pragma unroll
    for (int s = 0; s < STEPS; ++s) blk[s] = map.block_of(min(t0 + s * 8, s1 - 1));
  };
  auto load_k = [&](Chunk<T> (&dst)[STEPS][NV], int t0, const int (&blk)[STEPS]) {
    const bool full = t0 + TILE <= s1;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int step_tok = min(t0 + s * 8, s1 - 1);  // uniform
      const char* rowp = reinterpret_cast<const char*>(kb + map.row_offset(step_tok, blk[s]));
      const uint32_t lo =
          full ? k_off
               : (uint32_t)((min(t0 + s * 8 + grp, s1 - 1) - step_tok) * (int)map.tok_stride +
                            k_lane) * sizeof(T);
#pragma unroll
      for (int n = 0; n < NV; ++n)
        dst[s][n] = load_chunk_nt(reinterpret_cast<const T*>(rowp + lo + n * S::CH_STRIDE * sizeof(T)));
    }
  };
  // V token j = 8s + r of the tile lies in the block of K step s; the step's row address
  // is uniform.
  auto load_v = [&](VR (&dst)[TILE], int t0, const int (&blk)[STEPS]) {
    const bool full = t0 + TILE <= s1;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int step_tok = min(t0 + s * 8, s1 - 1);
      const char* rowp = reinterpret_cast<const char*>(vb + map.row_offset(step_tok, blk[s]));
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint32_t off =
            full ? v_off[r]
                 : (uint32_t)((min(t0 + s * 8 + r, s1 - 1) - step_tok) * (int)map.tok_stride +
                              v_lane) * sizeof(T);
        dst[s * 8 + r] = __builtin_nontemporal_load(reinterpret_cast<const VR*>(rowp + off));
      }
    }
  };

  int t0 = s0 + wave * TILE;
  if (t0 < s1) {
    Chunk<T> kc[STEPS][NV];
    VR vr[TILE];
    int blk[STEPS], nblk[STEPS];
    k_blocks(blk, t0);
    load_k(kc, t0, blk);
    load_v(vr, t0, blk);
    while (true) {
      const int tn = t0 + NW * TILE;
      const bool more = tn < s1;
      if (more) k_blocks(nblk, tn);  // in flight while this tile's scores are computed

      float sc[STEPS][G];
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const bool valid = t0 + s * 8 + grp < s1;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float d = chunk_dot_first(qc[g][0], kc[s][0]);
#pragma unroll
          for (int n = 1; n < NV; ++n) d = chunk_dot(qc[g][n], kc[s][n], d);
          d = sum8(d);
          sc[s][g] = valid ? d * c : -INFINITY;
        }
      }
      if (more) load_k(kc, tn, nblk);

      // Weights 2^(s - m) against the wave's running maximum m, which is raised (and acc, l
      // rescaled) only when a weight would exceed 2^8, and on the wave's first tile (m =
      // -inf): the exact tile maximum and its lane-group reduction are skipped otherwise.
      bool raise = false;
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int s = 0; s < STEPS; ++s) raise |= sc[s][g] - m[g] > kDecodeLazyLog2;
      if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float tm = sc[0][g];
#pragma unroll
          for (int s = 1; s < STEPS; ++s) tm = fmaxf(tm, sc[s][g]);
          tm = max_across_groups8(tm);
          const float mn = fmaxf(m[g], tm);
          const float alpha = fast_exp2(m[g] - mn);
          m[g] = mn;
          l[g] *= alpha;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float ls = 0.f;
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          sc[s][g] = fast_exp2(sc[s][g] - m[g]);
          ls += sc[s][g];
        }
        l[g] += ls;
      }
      // Token j = 8s + r of the tile has its weights in lane group r (lane 8r); they are
      // broadcast with v_readlane into scalar registers.
      if constexpr (std::is_same<T, f16>::value) {
        // fp16 K/V: tokens 8(2u)+r and 8(2u+1)+r share one packed weight pair, so one
        // v_dot2 does two tokens.  The weights are rounded to fp16 (as P is in the MFMA
        // prefill); the normaliser l keeps the fp32 weights.
#pragma unroll
        for (int u = 0; u < STEPS / 2; ++u) {
          uint32_t pw[G];
#pragma unroll
          for (int g = 0; g < G; ++g)
            pw[g] = __builtin_bit_cast(uint32_t, f16x2{(f16)sc[2 * u][g], (f16)sc[2 * u + 1][g]});
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            uint32_t vp[EPL];
            pair_rows<EPL>(vr[16 * u + r], vr[16 * u + 8 + r], vp);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const uint32_t p2 = __builtin_amdgcn_readlane(pw[g], r * 8);
#pragma unroll
              for (int e = 0; e < EPL; ++e) acc[g][e] = dot2<f16>(p2, vp[e], acc[g][e]);
            }
          }
        }
      } else if constexpr (sizeof(T) == 2) {
        // bf16 K/V: the same token pairs, with each weight split into bf16 hi + lo (16
        // significant bits together) and two bf16 v_dot2 per pair, so V is used as stored
        // and keeps bf16's full range.
#pragma unroll
        for (int u = 0; u < STEPS / 2; ++u) {
          uint32_t ph[G], pl[G];
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float p0 = sc[2 * u][g], p1 = sc[2 * u + 1][g];
            const bf16 h0 = (bf16)p0, h1 = (bf16)p1;
            ph[g] = __builtin_bit_cast(uint32_t, bf16x2{h0, h1});
            pl[g] = __builtin_bit_cast(uint32_t, bf16x2{(bf16)(p0 - (float)h0), (bf16)(p1 - (float)h1)});
          }
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            uint32_t vp[EPL];
            pair_rows<EPL>(vr[16 * u + r], vr[16 * u + 8 + r], vp);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const uint32_t h2 = __builtin_amdgcn_readlane(ph[g], r * 8);
              const uint32_t l2 = __builtin_amdgcn_readlane(pl[g], r * 8);
#pragma unroll
              for (int e = 0; e < EPL; ++e)
                acc[g][e] = dot2<bf16>(l2, vp[e], dot2<bf16>(h2, vp[e], acc[g][e]));
            }
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < TILE; ++j) {
          float vf[EPL];
          v_unpack<T, EPL>(vr[j], vf);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float p = __builtin_bit_cast(
                float,
                __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc[j >> 3][g]), (j & 7) * 8));
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(p, vf[e], acc[g][e]);
          }
        }
      }
      if (!more) break;
      load_v(vr, tn, nblk);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) blk[s] = nblk[s];
      t0 = tn;
    }
  }

  // l: every lane of a token group holds the same partial sums; add the 8 groups.
#pragma unroll
  for (int g = 0; g < G; ++g) l[g] = sum_across_groups8(l[g]);

  // Merge the 4 waves through LDS.
  __shared__ float s_acc[NW][G][D];
  __shared__ float s_ml[NW][G][2];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) s_acc[wave][g][lane * EPL + e] = acc[g][e];
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_ml[wave][g][0] = m[g];
      s_ml[wave][g][1] = l[g];
    }
  }
  __syncthreads();

  const bool direct = (nsplit == 1);
  for (int i = threadIdx.x; i < G * D; i += NW * kWave) {
    const int g = i / D, dd = i % D;
    float M = s_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
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
// One wave per (row, head): the splits' (m, l) are staged in LDS by the lanes in
// parallel, then lane l forms outputs [l * D/64, (l + 1) * D/64) with the acc loads of
// eight splits in flight at a time.
template <typename T, int D>
__global__ void __launch_bounds__(64) decode_combine_kernel(DecodeArgs a) {
  constexpr int EPL = D / kWave;
  const int h = blockIdx.x % a.Hq;
  const int row = blockIdx.x / a.Hq;
  const int len = row_len(a, row);
  if (len > a.len_cap) return;  // the split kernel wrote NaN
  const int nsplit = len > 0 ? (len + a.split_tokens - 1) / a.split_tokens : 0;
  if (nsplit <= 1) return;
  const float* ph = a.ws + ((long)row * a.Hq + h) * a.max_splits * (D + 2);
  const float* pl = ph + threadIdx.x * EPL;
  // The first kFirst partial rows are loaded before (m, l), so both memory round trips
  // overlap instead of running one after the other.
  constexpr int kFirst = 16;
  float x0[kFirst][EPL];
#pragma unroll
  for (int u = 0; u < kFirst; ++u)
    if (u < nsplit)
#pragma unroll
      for (int e = 0; e < EPL; ++e) x0[u][e] = pl[u * (D + 2) + e];
  __shared__ float s_m[kMaxCombineSplits], s_l[kMaxCombineSplits];
  float M = -INFINITY;
  for (int sp = threadIdx.x; sp < nsplit; sp += kWave) {
    const float m = ph[sp * (D + 2) + D];
    s_m[sp] = m;
    s_l[sp] = ph[sp * (D + 2) + D + 1];
    M = fmaxf(M, m);
  }
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) M = fmaxf(M, shfl_xor_f(M, mask));
  __syncthreads();
  float L = 0.f, o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = 0.f;
#pragma unroll
  for (int u = 0; u < kFirst; ++u)
    if (u < nsplit) {
      const float f = fast_exp2(s_m[u] - M);
      L = __builtin_fmaf(f, s_l[u], L);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = __builtin_fmaf(f, x0[u][e], o[e]);
    }
  int sp = kFirst;
  for (; sp + 8 <= nsplit; sp += 8) {
    float x[8][EPL];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int e = 0; e < EPL; ++e) x[u][e] = pl[(sp + u) * (D + 2) + e];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float f = fast_exp2(s_m[sp + u] - M);
      L = __builtin_fmaf(f, s_l[sp + u], L);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = __builtin_fmaf(f, x[u][e], o[e]);
    }
  }
  for (; sp < nsplit; ++sp) {
    const float f = fast_exp2(s_m[sp] - M);
    L = __builtin_fmaf(f, s_l[sp], L);
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = __builtin_fmaf(f, pl[sp * (D + 2) + e], o[e]);
  }
  const float inv = 1.f / L;
  T* out = reinterpret_cast<T*>(a.o) + (long)row * a.o_row_stride + (long)h * a.o_head_stride;
#pragma unroll
  for (int e = 0; e < EPL; ++e) out[threadIdx.x * EPL + e] = from_f32<T>(o[e] * inv);
}

template <typename T, int D>
hipError_t launch_combine(const DecodeArgs& a, hipStream_t stream) {
  if (a.max_splits > 1)
    hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3((unsigned)(a.n_rows * a.Hq)), dim3(64),
                       0, stream, a);
  return hipGetLastError();
}

template <typename T, int D, int G>
hipError_t launch_decode_tg(const DecodeArgs& a, hipStream_t stream) {
  const long blocks = (long)a.n_rows * a.Hkv * (a.kv_mul / G) * a.max_splits;
  bool wide = false;
  if constexpr (wide_fits<T, D, G>()) wide = a.wide != 0;
  if (wide) {
    if constexpr (wide_fits<T, D, G>()) {
      if (a.block_table)
        hipLaunchKernelGGL((decode_split_kernel<T, D, G, true, kWideWaves>), dim3((unsigned)blocks),
                           dim3(kWideWaves * kWave), 0, stream, a);
      else
        hipLaunchKernelGGL((decode_split_kernel<T, D, G, false, kWideWaves>),
                           dim3((unsigned)blocks), dim3(kWideWaves * kWave), 0, stream, a);
    }
  } else if (a.block_table) {
    hipLaunchKernelGGL((decode_split_kernel<T, D, G, true, kDecodeWaves>), dim3((unsigned)blocks),
                       dim3(kDecodeThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((decode_split_kernel<T, D, G, false, kDecodeWaves>), dim3((unsigned)blocks),
                       dim3(kDecodeThreads), 0, stream, a);
  }
  return launch_combine<T, D>(a, stream);
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
  // Launches of whole rows that fill the device go to the matrix-core kernel, which streams
  // a row faster per CU; split launches stay on the dot-product kernel, whose small
  // workgroups balance ragged rows better.
  if (a.mfma && a.max_splits == 1 && decode_mfma_supports(dtype, a.head_size, a.kv_mul))
    return launch_decode_mfma(a, dtype, stream);
  const int G = decode_heads_per_block(a.kv_mul);
  switch (dtype) {
    case kF32: return launch_decode_d<float>(a, G, stream);
    case kF16: return launch_decode_d<f16>(a, G, stream);
    case kBF16: return launch_decode_d<bf16>(a, G, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace orin
