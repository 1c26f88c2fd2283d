// Ping-pong attention forward for head sizes 64-128 on gfx950 (fp16 / bf16 in, fp32 accumulate).
//
// Serves the same two paths as fwd.hip (causal GQA prefill over a kuiper KV cache,
// flash_attention_kernel.cu:554-905; bidirectional varlen attention,
// vision_encoder_kernel.cu:954-1021) when the grid is large enough to fill the chip
// with 256-query workgroups.
//
// Work decomposition.  A workgroup of 8 waves owns 256 query rows of one query head;
// each wave owns 32 rows (Q fragments in registers).  The waves form two groups of four,
// one wave of each group per SIMD.  Time is cut into steps separated by workgroup
// barriers; in every step one group runs its MFMA phase while the other runs its softmax
// phase, so the SIMD's matrix pipe and its VALU work for different waves at the same
// time:
//   MFMA phase M(t):  S(t+1)^T = K(t+1) . Q^T     (16 v_mfma_f32_32x32x16)
//                     O^T     += V(t)^T . P(t)^T  (16 v_mfma_f32_32x32x16)
//   softmax phase V(t): mask, exp2 of S' = s - m (the QK^T accumulators start at -m),
//                       P packed to fp16; the row maximum m is raised (and O, l
//                       rescaled) only when a tile's weights would exceed 2^8.
// Group 0 runs M at even steps, group 1 at odd steps.
//
// K/V tiles (64 keys) reach LDS through global_load_lds_dwordx4 (no register staging),
// in a ring of three stages (four for bf16); stage u holds K(u) and V(u-1) and is read in
// steps 2u and 2u+1.  Every wave moves 1/8 of a stage (four 1 KB transfers) and waits for
// its own transfers with vmcnt before the barrier that publishes them.  For bf16 inputs
// the V tile of each stage is converted to fp16 in LDS before it is read, so P and the PV
// MFMAs are fp16 (bf16's 2^-9 rounding of P would be as large as the output tolerance).
//   K rows are stored row-major with 16-byte chunk c of row r at chunk c ^ (r & 15):
//   the K fragment reads (one row per lane, same chunk) are then conflict-free.
//   V rows are stored row-major with chunk c of row r at chunk c ^ 4(r & 3) and read
//   with ds_read_b64_tr_b16, which transposes 16-bit elements across 16 lanes: each
//   read hands a lane four consecutive keys of one dimension, so V^T fragments come
//   straight from the row-major tile.
//
// Head sizes below 128 pad the QK contraction to a multiple of 16 (zero Q elements) and
// O^T to a multiple of 32 (rows never stored); K/V rows keep 256-byte LDS slots.
//
// Key split.  A causal launch with fewer 256-query blocks than CUs is bounded by its
// longest block; the host then cuts each block's keys before its diagonal into chunks
// (key_chunk_tiles), each run by its own workgroup, and fwd_pp_merge combines the
// chunks' partials (O / l in fp16 for fp16 inputs, fp32 otherwise; fp32 m and l) in a
// second launch.
#include "common.h"
#include "kernels.h"

#include <type_traits>


namespace orin {

namespace {

constexpr int PD = 128;            // largest head size; K/V rows occupy PD elements in LDS
constexpr int PBN = 64;            // keys per tile
constexpr int PNW = 8;             // waves per workgroup
constexpr int PBM = 32 * PNW;      // query rows per workgroup
constexpr int PTHREADS = PNW * kWave;
constexpr int PTILE_BYTES = PBN * PD * 2;              // 16 KB
// LDS ring depth: 3 stages for fp16; 4 for bf16, whose V tiles are converted to fp16 in
// LDS one step before the MFMA phases read them.  K ring, then V ring.
template <typename T>
constexpr int pp_stages() { return std::is_same<T, f16>::value ? 3 : 4; }
template <typename T>
constexpr int pp_lds_bytes() { return 2 * pp_stages<T>() * PTILE_BYTES; }  // 96 / 128 KB
constexpr int kXcdsPP = 8;
// A lane's 32 weights of one tile may sum to at most this before the row maximum is raised.
constexpr float kTileSumMax = 256.0f;
constexpr int PF = 3;  // LDS reads run this many MFMAs ahead of their use

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) const char* lds_ptr;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c);
template <>
__device__ __forceinline__ f32x16 mfma32<f16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<bf16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, T2{(T)x, (T)y});
}

template <typename T>
__device__ __forceinline__ float sum_pair(uint32_t p, float acc);
template <>
__device__ __forceinline__ float sum_pair<f16>(uint32_t p, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), f16x2{(f16)1.0f, (f16)1.0f}, acc,
                                false);
}
template <>
__device__ __forceinline__ float sum_pair<bf16>(uint32_t p, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p),
                                         bf16x2{(bf16)1.0f, (bf16)1.0f}, acc, false);
}


// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait for the K/V transfers of all but the `younger` most recent stages (four transfers
// per wave and stage).
__device__ __forceinline__ void wait_stage(int younger) {
  switch (younger) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<4>(); break;
    case 2: wait_vmcnt<8>(); break;
    default: wait_vmcnt<12>(); break;
  }
}

// Workgroup barrier that the scheduler may not move any instruction across.
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// One 16-byte global -> LDS transfer per lane (global_load_lds_dwordx4): lane l's data
// lands at LDS byte lds_addr + 16 l.  Issued from inline asm so that the compiler does
// not treat it as an LDS store to wait for before every later LDS read: the kernel
// orders these transfers itself (vmcnt wait + barrier before the stage is read).  An LDS
// DMA that reads M0 right after an SALU write of M0 needs one wait state on gfx9-family
// parts, which the compiler cannot insert inside the asm: hence the s_nop.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
  __asm__ volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                   :
                   : "v"(gptr), "s"(lds_addr)
                   : "memory", "m0");
}

// The same transfer from a wave-uniform base (SGPR pair) plus a 32-bit per-lane byte offset:
// the per-tile address arithmetic stays on the scalar unit.
__device__ __forceinline__ void dma16_s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(voff), "s"(sbase), "s"(lds_addr)
                   : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// LDS reads at a per-lane address plus a compile-time offset (folded into the
// instruction's offset field).
__device__ __forceinline__ u32x4 lds_read128(lds_ptr p, int byte_off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(p + byte_off);
}

__device__ __forceinline__ u32x2 lds_read_tr(lds_ptr p, int byte_off) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + byte_off));
  return __builtin_bit_cast(u32x2, v);
}

// Key split of causal query block qb (rows qb*PBM ..): `diag` = the first tile holding a
// key past the block's first query position.  The block's tiles are cut into
// ceil(tiles / C) chunks of near-equal length (C = the longest chunk the host allows),
// at most diag + 1 of them, with every cut at or before diag: each chunk but the last is
// unmasked, and the last holds tiles [diag, tiles), so every chunk shows each of the
// block's queries at least one key.
__host__ __device__ inline int pp_block_tiles(const FwdArgs& a, int qb) {
  return (a.start_pos + min((qb + 1) * PBM, a.n_q) + PBN - 1) / PBN;
}
__host__ __device__ inline int pp_block_diag(const FwdArgs& a, int qb) {
  return (a.start_pos + qb * PBM) / PBN;
}
__host__ __device__ inline int pp_block_chunks(const FwdArgs& a, int qb, int C) {
  const int diag = pp_block_diag(a, qb);
  if (diag <= 0) return 1;
  return min((pp_block_tiles(a, qb) + C - 1) / C, diag + 1);
}
// First tile of chunk c (0 <= c <= n, n = pp_block_chunks): the even cut c * tiles / n,
// clamped to diag - (n - 1 - c) so that the cuts stay strictly increasing and the last one
// is at most diag.  Both sequences rise by at least one per chunk (tiles >= n), so no
// chunk is empty.
__host__ __device__ inline int pp_chunk_lo(const FwdArgs& a, int qb, int n, int c) {
  const int tiles = pp_block_tiles(a, qb);
  if (c <= 0) return 0;
  if (c >= n) return tiles;
  return min((int)((long)c * tiles / n), pp_block_diag(a, qb) - (n - 1 - c));
}
// Work item `item` of a key-split launch, query blocks last to first: block qb, chunk c.
__host__ __device__ inline void pp_item(const FwdArgs& a, int item, int C, int* qb, int* c) {
  const int nqb = (a.n_q + PBM - 1) / PBM;
  for (int b = nqb - 1; b >= 0; --b) {
    const int n = pp_block_chunks(a, b, C);
    if (item < n) {
      *qb = b;
      *c = item;
      return;
    }
    item -= n;
  }
  *qb = -1;
  *c = 0;
}
__host__ __device__ inline int pp_items(const FwdArgs& a, int C) {
  const int nqb = (a.n_q + PBM - 1) / PBM;
  int n = 0;
  for (int b = 0; b < nqb; ++b) n += pp_block_chunks(a, b, C);
  return n;
}
// Workspace of a key split: normalised O rows (O / l) [items * Hq * PBM][head_size] in the
// partial type, then (m, l) [items * Hq * PBM][2] fp32.  The partial type is fp16 for fp16
// inputs (|O / l| <= max |V|, and fp16 keeps 11 bits: one more rounding of 2^-12 relative)
// and fp32 for bf16 inputs (a bf16 partial would add a rounding as large as the output's).
// Offsets in floats.
template <typename T>
using PartT = typename std::conditional<std::is_same<T, f16>::value, f16, float>::type;
__host__ __device__ inline long pp_ml_offset(const FwdArgs& a, int D, int part_bytes) {
  return (long)pp_items(a, a.key_chunk_tiles) * a.Hq * PBM * D * part_bytes / 4;
}

// Order of the MFMAs of one phase: QK steps (2 per 16-wide slice of the head) and PV steps
// (DT per 16-key chunk) alternate while both remain, so that consecutive MFMAs on one
// accumulator are at least two apart.
template <int NQK, int NPV>
struct PhaseOrder {
  int is_qk[NQK + NPV];
  int idx[NQK + NPV];
  constexpr PhaseOrder() : is_qk(), idx() {
    int q = 0, v = 0;
    for (int i = 0; i < NQK + NPV; ++i) {
      const bool take_qk = q < NQK && (v >= NPV || i % 2 == 0);
      is_qk[i] = take_qk;
      idx[i] = take_qk ? q++ : v++;
    }
  }
};

// Scheduling pins for one MFMA phase: the LDS reads of the first PF fragments, then per MFMA
// i the MFMA and the reads of fragment i + PF (one ds_read_b128 for a K fragment, two
// ds_read_b64_tr_b16 for a V fragment).  Without them the compiler sinks each read to just
// before its MFMA, which then waits out most of the LDS latency.
template <int NQK, int NPV, int I>
__device__ __forceinline__ void sgb_seq() {
  constexpr int N = NQK + NPV;
  if constexpr (I < N) {
    constexpr PhaseOrder<NQK, NPV> o{};
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (I + PF < N) __builtin_amdgcn_sched_group_barrier(0x100, o.is_qk[I + PF] ? 1 : 2, 0);
    sgb_seq<NQK, NPV, I + 1>();
  }
}
template <int NQK, int NPV, int I>
__device__ __forceinline__ void sgb_head() {
  if constexpr (I < PF) {
    constexpr PhaseOrder<NQK, NPV> o{};
    __builtin_amdgcn_sched_group_barrier(0x100, o.is_qk[I] ? 1 : 2, 0);
    sgb_head<NQK, NPV, I + 1>();
  }
}

// Fused Q producer on the Q fragments of one lane: qf[s] holds elements 16s + 8hf .. +7 of
// the lane's query row, so chunk c = 2s + hf (elements 8c .. 8c+7) of the first half of the
// head and its rotation partner (elements d/2 + 8c ..) are in qf[s] and qf[s + QS/2]; the
// partner lane (lane ^ 32) holds the other chunks.  Same arithmetic as qk_norm_rope_kernel
// (producers.hip), so the rounded row equals the one that producer writes.  The weight and
// table loads do not depend on the row and are issued first (rows past the end read the
// tables at position pos_ok and are left unchanged).
template <typename T, int D>
__device__ __forceinline__ void fuse_q_producer(const FwdArgs& a, u32x4 (&qf)[(D + 15) / 16],
                                                bool live, int pos, int pos_ok, int hf) {
  constexpr int QS = D / 16, H2 = QS / 2;  // chunks per lane in each half
  const int p = live ? pos : pos_ok;
  // table entries [p][2j], j = 16s + 8hf + i: four 16-byte loads per table and chunk
  const float* sn = a.rope_sin + (long)p * D + 16 * hf;
  const float* cn = a.rope_cos + (long)p * D + 16 * hf;
  f32x4 s4[H2][4], k4[H2][4];
#pragma unroll
  for (int s = 0; s < H2; ++s)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      s4[s][c4] = *reinterpret_cast<const f32x4*>(sn + 32 * s + 4 * c4);
      k4[s][c4] = *reinterpret_cast<const f32x4*>(cn + 32 * s + 4 * c4);
    }
  const T* w = reinterpret_cast<const T*>(a.q_norm_weight);
  u32x4 wl_raw[H2], wh_raw[H2];
  if (w) {
#pragma unroll
    for (int s = 0; s < H2; ++s) {
      wl_raw[s] = load_chunk(w + 16 * s + 8 * hf).raw;
      wh_raw[s] = load_chunk(w + D / 2 + 16 * s + 8 * hf).raw;
    }
  }
  float lo[H2][8], hi[H2][8], cs[2 * H2];
  float own[H2];
#pragma unroll
  for (int s = 0; s < H2; ++s) {
    chunk_unpack(Chunk<T>{qf[s]}, lo[s]);
    chunk_unpack(Chunk<T>{qf[s + H2]}, hi[s]);
    own[s] = qk_chunk_sumsq(lo[s], hi[s]);
  }
#pragma unroll
  for (int s = 0; s < H2; ++s) {
    const float other = partner32(own[s]);
    cs[2 * s + hf] = own[s];
    cs[2 * s + (hf ^ 1)] = other;
  }
  if (w) {
    const float inv = qk_rms_inv(qk_butterfly_sum(cs), D, a.eps);
#pragma unroll
    for (int s = 0; s < H2; ++s) {
      float wl[8], wh[8];
      chunk_unpack(Chunk<T>{wl_raw[s]}, wl);
      chunk_unpack(Chunk<T>{wh_raw[s]}, wh);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        lo[s][i] = lo[s][i] * inv * wl[i];
        hi[s][i] = hi[s][i] * inv * wh[i];
      }
    }
  }
  if (!live) return;  // rows past the end stay zero
  typedef T T8 __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int s = 0; s < H2; ++s) {
    T8 rl, rh;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int i = 2 * c4 + e;
        float ro, rv;
        qk_rope(lo[s][i], hi[s][i], k4[s][c4][2 * e], s4[s][c4][2 * e], ro, rv);
        rl[i] = from_f32<T>(ro);
        rh[i] = from_f32<T>(rv);
      }
    qf[s] = __builtin_bit_cast(u32x4, rl);
    qf[s + H2] = __builtin_bit_cast(u32x4, rh);
  }
}

// FQ: the fused Q producer variant (a.rope_sin set), a separate instance so that its
// registers do not weigh on the plain kernel.
template <typename T, bool CAUSAL, int D, bool FQ>
__global__ void __launch_bounds__(PTHREADS) fwd_pp_kernel(FwdArgs a) {
  static_assert(D % 8 == 0 && D <= PD, "head size: a multiple of 8 up to 128");
  constexpr int QS = (D + 15) / 16;  // 16-wide slices of the QK contraction (zero-padded)
  constexpr int DT = (D + 31) / 32;  // 32-wide output tiles of O^T
  constexpr int NCH = D / 8;         // valid 16-byte chunks of a K / V row
  // bf16: P stays fp16 (2^-12 rounding; bf16's 2^-9 would be as large as the output's),
  // so the PV product runs on fp16 MFMAs over V tiles converted to fp16 in LDS.
  constexpr bool kConvV = !std::is_same<T, f16>::value;
  constexpr int PSTAGES = pp_stages<T>();
  constexpr int PKREGION = PSTAGES * PTILE_BYTES;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int lq = lane & 31, hf = lane >> 5;

  // ------------------------------------------------------------ block -> (head, rows)
  int head, q_lo, q_n, seg_start, kv_end, pos_off;
  int t_lo = 0, t_hi_split = 0;  // key split: this workgroup's tiles [t_lo, t_hi_split)
  bool partial = false;          // key split: write fp32 partials, merged by a second launch
  const int C = a.key_chunk_tiles;
  if (CAUSAL && C > 0) {
    head = (int)blockIdx.x % a.Hq;
    int qb, c;
    pp_item(a, (int)blockIdx.x / a.Hq, C, &qb, &c);
    const int n_ch = pp_block_chunks(a, qb, C);
    t_lo = pp_chunk_lo(a, qb, n_ch, c);
    t_hi_split = pp_chunk_lo(a, qb, n_ch, c + 1);
    partial = n_ch > 1;
    q_lo = qb * PBM;
    q_n = a.n_q;
    seg_start = 0;
    pos_off = a.start_pos;
    kv_end = a.start_pos + min(q_lo + PBM, a.n_q);
  } else if (CAUSAL) {
    const int nqb = (a.n_q + PBM - 1) / PBM;
    int qb;
    if (a.Hkv % kXcdsPP == 0) {
      const int x = (int)blockIdx.x % kXcdsPP, i = (int)blockIdx.x / kXcdsPP;
      const int hpx = a.Hq / kXcdsPP;
      qb = nqb - 1 - i / hpx;
      const int hl = i % hpx;
      head = (x + kXcdsPP * (hl / a.kv_mul)) * a.kv_mul + hl % a.kv_mul;
    } else {
      qb = nqb - 1 - (int)blockIdx.x / a.Hq;
      head = (int)blockIdx.x % a.Hq;
    }
    q_lo = qb * PBM;
    q_n = a.n_q;
    seg_start = 0;
    pos_off = a.start_pos;
    kv_end = a.start_pos + min(q_lo + PBM, a.n_q);
  } else {
    const int nqb = (a.max_seqlen + PBM - 1) / PBM;
    head = (int)blockIdx.x % a.Hq;
    const int rest = (int)blockIdx.x / a.Hq;
    const int qb = rest % nqb, seg = rest / nqb;
    seg_start = a.cu_seqlens ? a.cu_seqlens[seg] : 0;
    q_n = a.cu_seqlens ? a.cu_seqlens[seg + 1] - seg_start : a.n_q;
    q_lo = qb * PBM;
    if (q_lo >= q_n) return;
    pos_off = 0;
    kv_end = q_n;
  }
  const int kvh = head / a.kv_mul;
  const long tok = a.kv_tok_stride;
  const T* kb = reinterpret_cast<const T*>(a.k) + (long)seg_start * tok + (long)kvh * a.kv_head_stride;
  const T* vb = reinterpret_cast<const T*>(a.v) + (long)seg_start * tok + (long)kvh * a.kv_head_stride;
  // Tiles run t = 0 .. n_tiles-1 locally; key tile t_lo + t globally.
  const int n_tiles = (C > 0 && CAUSAL) ? t_hi_split - t_lo : (kv_end + PBN - 1) / PBN;

  // Row slots interleave the groups (group 0: slots 0,2,4,6; group 1: 1,3,5,7) so both
  // groups reach the causal diagonal in the same tiles.
  const int slot = 2 * (wave & 3) + grp;
  const int wq0 = q_lo + 32 * slot;
  const int qi = wq0 + lq;
  const int wpos0 = pos_off + wq0;
  const int qpos = wpos0 + lq;

  // ------------------------------------------------------------ K/V transfer setup
  // Transfer i (0,1) of this wave covers rows 4b..4b+3 of a tile, b = 2*wave + i; lane l
  // moves 16-byte chunk (l%16) of row 4b + l/16 (physical position) whose logical chunk
  // follows the swizzle of each tile.
  int k_row[2], k_col[2], v_col[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 4 * (2 * wave + i) + (lane >> 4);
    const int pc = lane & 15;
    k_row[i] = row;
    // Chunks past the row (head sizes below 128) load chunk 0 of the same row instead:
    // finite values that meet zero Q elements (K) or fill O^T rows never stored (V).
    const int kc = pc ^ (row & 15), vc = pc ^ (4 * (row & 3));
    k_col[i] = 8 * (kc < NCH ? kc : 0);
    v_col[i] = 8 * (vc < NCH ? vc : 0);
  }
  char* const k_lds = smem;
  char* const v_lds = smem + PKREGION;
  const uint32_t k_base = __builtin_amdgcn_readfirstlane(lds_addr(smem));

  // Stage u = K(u) + V(u-1) into ring slot u % 3 (stage 0: K(0) only).  Rows past the
  // sequence read a valid row instead, so every stage after the first is exactly four
  // transfers per wave (the waits count them from the youngest stage) and the LDS rows the
  // MFMA phases read never hold non-finite garbage.
  // Addresses: a wave-uniform tile base (scalar) plus a per-lane byte offset
  // row_in_tile * row_bytes + column bytes (`fwd_pp_supports` keeps row_bytes below 2^24,
  // so one 24-bit multiply-add forms it).
  const uint32_t row_bytes = (uint32_t)tok * sizeof(T);
  // bf16 (plain instance): V is staged through registers, one buffer per ring slot, and
  // written to LDS converted to fp16 by the step that publishes it, instead of a transfer
  // to LDS converted there in place; the loads replace the V transfers one for one, so
  // every wait counts the same.  The ring slot is a compile-time tag at every issue and
  // conversion, so each load writes its slot's registers directly.  (The fused-Q instance
  // has no registers to spare and converts in LDS.)
  constexpr bool kRegV = kConvV && !FQ;
  u32x4 vbuf[kRegV ? PSTAGES : 1][2];
  // `sl_tag` = u % PSTAGES as a compile-time constant (used by the register staging).
  auto issue_stage = [&](int u, auto sl_tag) __attribute__((always_inline)) {
    const int sl = u % PSTAGES;
    // Tile bases are clamped into [0, kv_end - 1] so that the last valid row's offset from
    // its base is never negative: K(n_tiles) of the last stage starts past the sequence and
    // V(-1) before it; every row of such a tile reads a valid row.
    const int tk = (t_lo + u) * PBN, tv = tk - PBN;
    const int tk0 = tk < kv_end - 1 ? tk : kv_end - 1;
    const int tv0 = tv < 0 ? 0 : (tv < kv_end - 1 ? tv : kv_end - 1);
    const char* kt_base = reinterpret_cast<const char*>(kb + (long)tk0 * tok);
    const char* vt_base = reinterpret_cast<const char*>(vb + (long)tv0 * tok);
    const int k_last = kv_end - 1 - tk0, v_last = kv_end - 1 - tv0;  // >= 0
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int b = 2 * wave + i;
      const int rk = k_row[i] < k_last ? k_row[i] : k_last;
      const int rv = k_row[i] < v_last ? k_row[i] : v_last;
      dma16_s(kt_base, __umul24(rk, row_bytes) + k_col[i] * (uint32_t)sizeof(T),
              k_base + sl * PTILE_BYTES + b * 1024);
      if (u == 0) continue;  // V(-1): no MFMA phase reads it
      const uint32_t voff = __umul24(rv, row_bytes) + v_col[i] * (uint32_t)sizeof(T);
      if constexpr (kRegV)
        vbuf[decltype(sl_tag)::value % PSTAGES][i] =
            *reinterpret_cast<const u32x4*>(vt_base + voff);
      else
        dma16_s(vt_base, voff, k_base + PKREGION + sl * PTILE_BYTES + b * 1024);
    }
  };

  // ------------------------------------------------------------ fragment addresses
  // K fragment (kt, s): row kt*32 + lq, logical chunk 2s + hf.
  const lds_ptr lds0 = (lds_ptr)smem;
  lds_ptr k_p[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) k_p[s] = lds0 + lq * 256 + (((2 * s + hf) ^ (lane & 15)) * 16);
  // V^T fragment (chunk c of 16 keys, d-tile dt): two transposing reads.  Lane
  // L = 16g + 4e + q supplies row 16c + 4(g/2) + e (+8 for the second read) and
  // columns dt*32 + 16(g&1) + 4q .. +3.
  lds_ptr v_p[4];
  {
    const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
    const int row = 4 * (g >> 1) + e;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      v_p[dt] = lds0 + PKREGION + row * 256 + (((dt ^ e) * 4 + 2 * (g & 1) + (q >> 1)) * 16) +
                (q & 1) * 8;
  }

  // ------------------------------------------------------------ Q fragments
  u32x4 qf[QS];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (long)(seg_start + qi) * a.q_tok_stride +
                  (long)head * a.q_head_stride;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      u32x4 val = {0u, 0u, 0u, 0u};  // rows past the end and the zero padding of the head
      if (qi < q_n && 16 * s + 8 * hf < D) val = *reinterpret_cast<const u32x4*>(qp + 16 * s + 8 * hf);
      qf[s] = val;
    }
  }

  // Stages 0 .. PSTAGES-1 up front; wait for stage 0 (younger stages may stay in flight).
  issue_stage(0, std::integral_constant<int, 0>{});
  if (n_tiles >= 1) issue_stage(1, std::integral_constant<int, 1>{});
  if (n_tiles >= 2) issue_stage(2, std::integral_constant<int, 2>{});
  if (PSTAGES > 3 && n_tiles >= 3) issue_stage(3, std::integral_constant<int, 3 % PSTAGES>{});
  // The fused Q producer works while the first stages are in flight.
  if constexpr (FQ && CAUSAL && (D == 64 || D == 128))
    fuse_q_producer<T, D>(a, qf, qi < q_n, a.start_pos + qi, a.start_pos, hf);
  wait_stage(min(n_tiles, PSTAGES - 1));
  step_barrier();

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  f32x16 sacc[2];
  u32x4 pf[4];
  // Running row maximum m (raw score units) and its negation in every accumulator slot:
  // the QK^T MFMA chains start from `negm`, so S' = s - m leaves the matrix pipe and the
  // softmax needs no subtraction per score.
  const float c = a.scale_log2;
  float m_use = 0.f, l_run = 0.f;
  f32x16 negm;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = 0.f;

  auto active = [&](int t) __attribute__((always_inline)) {
    return !CAUSAL || (t_lo + t) * PBN <= wpos0 + 31;
  };

  // A operands of the MFMA phase.  K fragment (kt, s) of S^T = K . Q^T; V^T fragment
  // (chunk ck, d-tile dt) of O^T += V^T . P^T, from two transposing reads.
  // `sl_off` is the ring slot's byte offset (a compile-time constant at every call).
  auto k_frag = [&](int sl_off, int kt, int s) __attribute__((always_inline)) {
    return lds_read128(k_p[s], sl_off + kt * 8192);
  };
  auto v_frag = [&](int sl_off, int ck, int dt) __attribute__((always_inline)) {
    const u32x2 lo = lds_read_tr(v_p[dt], sl_off + ck * 16 * 256);
    const u32x2 hi = lds_read_tr(v_p[dt], sl_off + ck * 16 * 256 + 8 * 256);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  // S(0)^T = K(0) . Q^T (K(0) is in ring slot 0).
  auto qk0 = [&]() __attribute__((always_inline)) {
    sacc[0] = negm;
    sacc[1] = negm;
    constexpr int NQK = 2 * QS;
    u32x4 fr[PF + 1];
#pragma unroll
    for (int i = 0; i < PF; ++i) fr[i] = k_frag(0, i & 1, i >> 1);
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      if (i + PF < NQK) fr[(i + PF) % (PF + 1)] = k_frag(0, (i + PF) & 1, (i + PF) >> 1);
      sacc[i & 1] = mfma32<T>(fr[i % (PF + 1)], qf[i >> 1], sacc[i & 1]);
    }
  };

  // MFMA phase M(t): S(t+1)^T = K(t+1) . Q^T (when QK) and O^T += V(t)^T . P(t)^T, both
  // from ring slot (t+1) % 3.  The two products are interleaved (QK, PV, QK, ...) so that
  // consecutive MFMAs on one accumulator are at least two apart, and every A operand is
  // read from LDS three MFMAs before its use.
  auto mphase = [&](auto slot_tag, auto qk_tag) __attribute__((always_inline)) {
    constexpr bool QK = decltype(qk_tag)::value;
    constexpr int NQK = QK ? 2 * QS : 0, NPV = 4 * DT;
    constexpr int N = NQK + NPV;
    constexpr PhaseOrder<NQK, NPV> order{};
    constexpr int sl_off = decltype(slot_tag)::value * PTILE_BYTES;
    if (QK) {
      sacc[0] = negm;
      sacc[1] = negm;
    }
    // MFMA i: QK step j = (kt = j & 1, slice j >> 1) or PV step n = (chunk n / DT, d-tile
    // n % DT), in the order of PhaseOrder.
    auto fetch = [&](int i) __attribute__((always_inline)) {
      if (order.is_qk[i]) return k_frag(sl_off, order.idx[i] & 1, order.idx[i] >> 1);
      return v_frag(sl_off, order.idx[i] / DT, order.idx[i] % DT);
    };
    u32x4 fr[PF + 1];
#pragma unroll
    for (int i = 0; i < PF; ++i) fr[i] = fetch(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i + PF < N) fr[(i + PF) % (PF + 1)] = fetch(i + PF);
      if (order.is_qk[i]) {
        const int j = order.idx[i];
        sacc[j & 1] = mfma32<T>(fr[i % (PF + 1)], qf[j >> 1], sacc[j & 1]);
      } else {
        const int n = order.idx[i];
        oacc[n % DT] = mfma32<f16>(fr[i % (PF + 1)], pf[n / DT], oacc[n % DT]);
      }
    }
    sgb_head<NQK, NPV, 0>();
    sgb_seq<NQK, NPV, 0>();
  };

  // Softmax of S'(t) into P(t) (packed 16-bit).  Fast path: P = 2^(c*S') with the
  // running maximum m left as it is, valid while every weight stays at most 2^8 (checked
  // through each lane's sum of its 32 weights); otherwise (and on the first tile, where m
  // is not yet set) the row maximum is taken, m raised to it, O and l rescaled and P
  // recomputed.  The weights then never exceed 2^8 and the normaliser never underflows.
  auto softmax = [&](int t) __attribute__((always_inline)) {
    const int t0 = (t_lo + t) * PBN;
    const bool need_mask = CAUSAL ? (t0 + PBN - 1 > wpos0) : (t0 + PBN > kv_end);
    if (need_mask) {
      // Key t0 + 4hf + c (c a compile-time constant below 64) is masked when it lies
      // past `lim`, i.e. when c > lim - t0 - 4hf.
      const int rel = (CAUSAL ? qpos : kv_end - 1) - t0 - 4 * hf;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int cr = kt * 32 + 8 * (r >> 2) + (r & 3);
          sacc[kt][r] = cr > rel ? -INFINITY : sacc[kt][r];
        }
    }
    // The lane's weight sum in four partial sums: four short dependency chains instead of
    // one of 16 dot products.
    float lsp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const uint32_t pk =
            pack2<f16>(fast_exp2(sacc[kt][r] * c), fast_exp2(sacc[kt][r + 1] * c));
        pf[kt * 2 + (r >> 3)][(r & 7) >> 1] = pk;
        lsp[(r >> 1) & 3] = sum_pair<f16>(pk, lsp[(r >> 1) & 3]);
      }
    float ls = (lsp[0] + lsp[1]) + (lsp[2] + lsp[3]);
    const bool first = t == 0;
    if (__builtin_amdgcn_ballot_w64(first || !(ls <= kTileSumMax))) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
      mx = fmaxf(mx, partner32(mx));
      // raise m by `up`: to the row maximum on the first tile, else only upwards
      const float up = first ? (mx > -INFINITY ? mx : 0.f) : fmaxf(mx, 0.f);
      m_use += up;
#pragma unroll
      for (int r = 0; r < 16; ++r) negm[r] = -m_use;
      if (!first && __builtin_amdgcn_ballot_w64(up != 0.f)) {
        const float alpha = fast_exp2(-up * c);
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[d][r] *= alpha;
      }
      ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const uint32_t pk =
              pack2<f16>(fast_exp2((sacc[kt][r] - up) * c), fast_exp2((sacc[kt][r + 1] - up) * c));
          pf[kt * 2 + (r >> 3)][(r & 7) >> 1] = pk;
          ls = sum_pair<f16>(pk, ls);
        }
    }
    l_run += ls;
  };

  // Step bookkeeping shared by both groups.  Group 0 runs M(t) at step 2t+2 and softmax(t)
  // at step 2t+1, group 1 one step later; M(t) reads stage t+1.
  //  fp16: stage u is published by the barrier that ends step 2u-1 and issued at the
  //        start of step 2u-4 (three stages).
  //  bf16: stage u is published one step earlier (end of step 2u-2); at the end of step
  //        2u-1 every wave writes 1/8 of its V tile converted to fp16 (from its registers,
  //        or in place for the fused-Q instance; no phase reads stage u in that step), and
  //        the barrier ending that step publishes the result;
  //        it is issued at the start of step 2u-6 (four stages: the slot's previous stage
  //        was last read by group 1's M(u-5) at step 2u-7).
  const int last_step = 2 * n_tiles + 1;
  // `sl_tag`: the ring slot of the stage this step may issue (see the call sites).
  auto step_begin = [&](int k, auto sl_tag) __attribute__((always_inline)) {
    if (!(k & 1) && k >= 2) {
      const int u = k / 2 + PSTAGES - 1;
      if (u <= n_tiles) issue_stage(u, sl_tag);
    }
  };
  auto convert_v = [&](int u, auto sl_tag) __attribute__((always_inline)) {
    // wave w converts bytes [2048 w, 2048 w + 2048) of the stage's V tile
    lds_ptr base = lds0 + PKREGION + (u % PSTAGES) * PTILE_BYTES + wave * 2048 + lane * 16;
    u32x4 x[2];
    if constexpr (kRegV) {
      x[0] = vbuf[decltype(sl_tag)::value % PSTAGES][0];
      x[1] = vbuf[decltype(sl_tag)::value % PSTAGES][1];
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) x[j] = lds_read128(base, j * 1024);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
          const_cast<__attribute__((address_space(3))) char*>(base + j * 1024)) =
          bf16x8_to_f16x8(x[j]);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the writes land before the barrier
  };
  // `sl_tag`: the ring slot of the stage this step may convert (see the call sites).
  auto step_end = [&](int k, auto sl_tag) __attribute__((always_inline)) {
    if constexpr (kConvV) {
      if (!(k & 1)) {
        const int u = k / 2 + 1;
        if (u <= n_tiles) wait_stage(min(n_tiles, k / 2 + PSTAGES - 1) - u);
      } else {
        const int u = (k + 1) / 2;
        if (u <= n_tiles) convert_v(u, sl_tag);
      }
    } else if (k & 1) {
      const int u = (k + 1) / 2;
      if (u + 1 <= n_tiles) wait_vmcnt<4>();
      else wait_vmcnt<0>();
    }
    if (k < last_step) step_barrier();
  };

  // Ring-slot tags of the steps (stage u issued at even step 2u - 2(PSTAGES - 1), converted
  // at odd step 2u - 1, u % PSTAGES its slot): group 1's first step and both groups' QK(0)
  // step issue nothing and convert stage 1 (slot 1) at most; the softmax(0) step issues
  // stage PSTAGES (slot 0) in group 1 and converts stage 1 in group 0.
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  int k = 0;
  if (grp == 1) {  // group 1 starts one step late
    step_begin(k, S0{});
    step_end(k, S1{});
    ++k;
  }
  step_begin(k, S0{});
  qk0();
  step_end(k, S1{});
  ++k;
  step_begin(k, S0{});
  softmax(0);
  step_end(k, S1{});
  ++k;
  // Tile t's MFMA phase reads ring slot (t+1) % PSTAGES; the loop is unrolled by
  // PSTAGES so every LDS offset is a compile-time constant.  Tiles before the last one always run
  // the QK product of the next tile, also for a wave whose queries all precede it: one
  // MFMA-phase shape inside the loop keeps the accumulators in fixed registers.
  // In tile t (slot tag (t+1) % PSTAGES) group 0's MFMA step 2t+2 issues stage t +
  // PSTAGES (slot t % PSTAGES), group 1's softmax step 2t+4 issues stage t + PSTAGES + 1
  // (slot (t+1) % PSTAGES), and the odd step of each group converts stage t+2.
  auto tile = [&](int t, auto slot_tag) __attribute__((always_inline)) {
    constexpr int TG = decltype(slot_tag)::value;
    using SI = std::integral_constant<int, (TG + PSTAGES - 1) % PSTAGES>;
    using SC = std::integral_constant<int, (TG + 1) % PSTAGES>;
    step_begin(k, SI{});
    __builtin_amdgcn_s_setprio(1);
    if (active(t)) mphase(slot_tag, std::true_type{});
    __builtin_amdgcn_s_setprio(0);
    step_end(k, SC{});
    ++k;
    step_begin(k, slot_tag);
    if (active(t + 1)) softmax(t + 1);
    step_end(k, SC{});
    ++k;
  };
  const int n_loop = n_tiles - 1;
  for (int t = 0; t < n_loop; t += PSTAGES) {
    tile(t, std::integral_constant<int, 1>{});
    if (t + 1 < n_loop) tile(t + 1, std::integral_constant<int, 2>{});
    if (t + 2 < n_loop) tile(t + 2, std::integral_constant<int, 3 % PSTAGES>{});
    if (PSTAGES > 3 && t + 3 < n_loop) tile(t + 3, std::integral_constant<int, 4 % PSTAGES>{});
  }
  {  // last tile: PV only
    const int t = n_loop;
    step_begin(k, S0{});  // issues nothing: every stage is out
    __builtin_amdgcn_s_setprio(1);
    if (active(t)) {
      switch ((t + 1) % PSTAGES) {
        case 0: mphase(std::integral_constant<int, 0>{}, std::false_type{}); break;
        case 1: mphase(std::integral_constant<int, 1>{}, std::false_type{}); break;
        case 2: mphase(std::integral_constant<int, 2>{}, std::false_type{}); break;
        default: mphase(std::integral_constant<int, 3 % PSTAGES>{}, std::false_type{}); break;
      }
    }
    __builtin_amdgcn_s_setprio(0);
    step_end(k, S0{});  // converts nothing: stage n_tiles + 1 does not exist
    ++k;
  }
  if (grp == 0) {  // group 0 ends one step early
    step_begin(k, S0{});
    step_end(k, S0{});
    ++k;
  }

  // ------------------------------------------------------------ normalise and store
  const float l_tot = l_run + partner32(l_run);
  const float inv = 1.f / l_tot;
  if (partial) {
    // Partial of this key chunk per query row: O / l in the partial type, and (m, l) fp32.
    using PT = PartT<T>;
    const long row = (long)blockIdx.x * PBM + (qi - q_lo);
    if (qi < q_n) {
      PT* pr = reinterpret_cast<PT*>(a.ws) + row * D;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int d0 = t * 32 + 8 * rg + 4 * hf;
          if (d0 >= D) continue;
          const float o0 = oacc[t][4 * rg] * inv, o1 = oacc[t][4 * rg + 1] * inv;
          const float o2 = oacc[t][4 * rg + 2] * inv, o3 = oacc[t][4 * rg + 3] * inv;
          if constexpr (sizeof(PT) == 2)
            *reinterpret_cast<u32x2*>(pr + d0) = u32x2{pack2<T>(o0, o1), pack2<T>(o2, o3)};
          else
            *reinterpret_cast<f32x4*>(pr + d0) = f32x4{o0, o1, o2, o3};
        }
      if (hf == 0) {
        float* ml = a.ws + pp_ml_offset(a, D, sizeof(PT)) + row * 2;
        ml[0] = m_use * a.scale_log2;
        ml[1] = l_tot;
      }
    }
    return;
  }
  if (qi < q_n) {
    T* op = reinterpret_cast<T*>(a.o) + (long)(seg_start + qi) * a.o_tok_stride +
            (long)head * a.o_head_stride;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d0 = t * 32 + 8 * rg + 4 * hf;
        if (d0 >= D) continue;  // padding columns of O^T
        u32x2 pk = {pack2<T>(oacc[t][4 * rg] * inv, oacc[t][4 * rg + 1] * inv),
                    pack2<T>(oacc[t][4 * rg + 2] * inv, oacc[t][4 * rg + 3] * inv)};
        *reinterpret_cast<u32x2*>(op + d0) = pk;
      }
  }
}

// Merge the key-chunk partials of the split query blocks:
// O = sum_c w_c (O_c / l_c) / sum_c w_c with w_c = 2^(m_c - M) l_c.  A thread owns 8 dimensions of one row
// (16 rows per workgroup, a row's threads neighbours so a wave reads whole rows); every
// load it needs is issued before any is used.
constexpr int kMergeMaxChunks = 8;
constexpr int kMergeRows = 16;
template <typename T, int D>
__global__ void __launch_bounds__(kMergeRows * ((D + 7) / 8)) fwd_pp_merge(FwdArgs a) {
  constexpr int NP = (D + 7) / 8;  // 8-dimension parts of a row
  const int C = a.key_chunk_tiles;
  const int sub = (int)blockIdx.x % (PBM / kMergeRows);
  const int hb = (int)blockIdx.x / (PBM / kMergeRows);
  const int head = hb % a.Hq, qb = hb / a.Hq;
  const int n_ch = pp_block_chunks(a, qb, C);
  if (n_ch <= 1) return;
  const int part = (int)threadIdx.x % NP;
  const int r = sub * kMergeRows + (int)threadIdx.x / NP;
  const int qi = qb * PBM + r;
  if (qi >= a.n_q) return;
  const int nqb = (a.n_q + PBM - 1) / PBM;
  int item0 = 0;  // the items of blocks qb+1 .. nqb-1 come first
  for (int b = nqb - 1; b > qb; --b) item0 += pp_block_chunks(a, b, C);
  using PT = PartT<T>;
  const float* ml = a.ws + pp_ml_offset(a, D, sizeof(PT));
  const PT* po = reinterpret_cast<const PT*>(a.ws);
  const int d0 = 8 * part;
  float m[kMergeMaxChunks], l[kMergeMaxChunks];
  u32x4 x[kMergeMaxChunks][sizeof(PT) / 2];  // the 8 partial values of each chunk
#pragma unroll
  for (int c = 0; c < kMergeMaxChunks; ++c) {
    const long row = ((long)(item0 + min(c, n_ch - 1)) * a.Hq + head) * PBM + r;
    m[c] = c < n_ch ? ml[row * 2] : -INFINITY;
    l[c] = c < n_ch ? ml[row * 2 + 1] : 0.f;
#pragma unroll
    for (int j = 0; j < (int)sizeof(PT) / 2; ++j)
      x[c][j] = (c < n_ch && d0 < D)
                    ? *reinterpret_cast<const u32x4*>(po + row * D + d0 + j * (16 / sizeof(PT)))
                    : u32x4{0u, 0u, 0u, 0u};
  }
  float M = m[0];
#pragma unroll
  for (int c = 1; c < kMergeMaxChunks; ++c) M = fmaxf(M, m[c]);
  float W = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
  for (int c = 0; c < kMergeMaxChunks; ++c) {
    const float w = c < n_ch ? fast_exp2(m[c] - M) * l[c] : 0.f;
    W += w;
    float xv[8];
    if constexpr (sizeof(PT) == 2) {
      chunk_unpack(Chunk<f16>{x[c][0]}, xv);
    } else {
      const f32x4 lo = __builtin_bit_cast(f32x4, x[c][0]), hi = __builtin_bit_cast(f32x4, x[c][1]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[e] = lo[e];
        xv[e + 4] = hi[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(w, xv[e], o[e]);
  }
  const float inv = 1.f / W;
  if (d0 >= D) return;
  T* op = reinterpret_cast<T*>(a.o) + (long)qi * a.o_tok_stride + (long)head * a.o_head_stride;
  u32x4 pk = {pack2<T>(o[0] * inv, o[1] * inv), pack2<T>(o[2] * inv, o[3] * inv),
              pack2<T>(o[4] * inv, o[5] * inv), pack2<T>(o[6] * inv, o[7] * inv)};
  *reinterpret_cast<u32x4*>(op + d0) = pk;
}

template <typename T, bool CAUSAL, int D>
hipError_t launch_pp_d(const FwdArgs& a, hipStream_t stream) {
  long blocks;
  if (CAUSAL && a.key_chunk_tiles > 0) blocks = (long)pp_items(a, a.key_chunk_tiles) * a.Hq;
  else if (CAUSAL) blocks = (long)((a.n_q + PBM - 1) / PBM) * a.Hq;
  else blocks = (long)a.n_seg * ((a.max_seqlen + PBM - 1) / PBM) * a.Hq;
  if (blocks <= 0) return hipSuccess;
  constexpr bool kFusable = CAUSAL && (D == 64 || D == 128);
  const bool fq = kFusable && a.rope_sin != nullptr;
  const void* fn = fq ? (const void*)fwd_pp_kernel<T, CAUSAL, D, kFusable>
                      : (const void*)fwd_pp_kernel<T, CAUSAL, D, false>;
  static unsigned long long configured[2] = {0, 0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 64 || !(__atomic_load_n(&configured[fq], __ATOMIC_ACQUIRE) & (1ull << dev))) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, pp_lds_bytes<T>());
    if (e != hipSuccess) return e;
    if (dev < 64) __atomic_fetch_or(&configured[fq], 1ull << dev, __ATOMIC_RELEASE);
  }
  if (fq)
    hipLaunchKernelGGL((fwd_pp_kernel<T, CAUSAL, D, kFusable>), dim3((unsigned)blocks),
                       dim3(PTHREADS), pp_lds_bytes<T>(), stream, a);
  else
    hipLaunchKernelGGL((fwd_pp_kernel<T, CAUSAL, D, false>), dim3((unsigned)blocks),
                       dim3(PTHREADS), pp_lds_bytes<T>(), stream, a);
  if (CAUSAL && a.key_chunk_tiles > 0) {
    const int nqb = (a.n_q + PBM - 1) / PBM;
    hipLaunchKernelGGL((fwd_pp_merge<T, D>), dim3((unsigned)(nqb * a.Hq * (PBM / kMergeRows))),
                       dim3(kMergeRows * ((D + 7) / 8)), 0, stream, a);
  }
  return hipGetLastError();
}

template <typename T, bool CAUSAL>
hipError_t launch_pp_t(const FwdArgs& a, hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_pp_d<T, CAUSAL, 64>(a, stream);
    case 72: return launch_pp_d<T, CAUSAL, 72>(a, stream);
    case 80: return launch_pp_d<T, CAUSAL, 80>(a, stream);
    case 96: return launch_pp_d<T, CAUSAL, 96>(a, stream);
    case 128: return launch_pp_d<T, CAUSAL, 128>(a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool fwd_pp_supports(const FwdArgs& a, int dtype) {
  const int d = a.head_size;
  if (!(d == 64 || d == 72 || d == 80 || d == 96 || d == 128) || !(dtype == kF16 || dtype == kBF16))
    return false;
  // K/V rows and Q/O rows are read as 16-byte chunks.
  // K/V transfer offsets within a tile are formed with 24-bit multiplies.
  return a.kv_tok_stride % 8 == 0 && a.kv_head_stride % 8 == 0 && a.q_tok_stride % 8 == 0 &&
         a.q_head_stride % 8 == 0 && a.kv_tok_stride * 2 < (1 << 24);
}

int fwd_pp_key_split(const FwdArgs& a, int dtype, int n_cu, size_t* ws_bytes) {
  *ws_bytes = 0;
  if (!fwd_pp_supports(a, dtype) || a.n_q <= 0 || n_cu <= 0) return 0;
  const int nqb = (a.n_q + PBM - 1) / PBM;
  if ((long)nqb * a.Hq >= n_cu) return 0;  // the plain launch fills the device
  // Smallest chunk bound that keeps the launch to one workgroup per CU and each block to
  // at most kMergeMaxChunks chunks (both counts fall as C grows: binary search); no split
  // if that does not shorten the longest block by at least a third.
  const int longest = pp_block_tiles(a, nqb - 1);
  auto fits = [&](int C) {
    return (long)pp_items(a, C) * a.Hq <= n_cu && pp_block_chunks(a, nqb - 1, C) <= kMergeMaxChunks;
  };
  if (!fits(longest)) return 0;
  int lo = 1, hi = longest;
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    if (fits(mid)) hi = mid; else lo = mid + 1;
  }
  const int C = lo;
  int worst = 0;  // longest chunk of the launch
  for (int b = 0; b < nqb; ++b) {
    const int n = pp_block_chunks(a, b, C);
    for (int c = 0; c < n; ++c)
      worst = max(worst, pp_chunk_lo(a, b, n, c + 1) - pp_chunk_lo(a, b, n, c));
  }
  if (3 * worst > 2 * longest) return 0;
  const size_t rows = (size_t)pp_items(a, C) * a.Hq * PBM;
  const size_t part_bytes = dtype == kF16 ? 2 : 4;  // PartT
  *ws_bytes = rows * a.head_size * part_bytes + rows * 2 * sizeof(float);
  return C;
}

hipError_t launch_fwd_pp(const FwdArgs& a, int dtype, bool causal, hipStream_t stream) {
  if (dtype == kF16)
    return causal ? launch_pp_t<f16, true>(a, stream) : launch_pp_t<f16, false>(a, stream);
  return causal ? launch_pp_t<bf16, true>(a, stream) : launch_pp_t<bf16, false>(a, stream);
}

}  // namespace orin
