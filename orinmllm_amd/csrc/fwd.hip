// Tile-parallel attention forward on gfx950 MFMA (fp16 / bf16 in, fp32 accumulate).
//
// Serves two reference paths:
//  * causal GQA prefill over a kuiper KV cache [max_seq, Hkv*d]
//    (replaces flash_attention_prefill_kernel_fp16, flash_attention_kernel.cu:554-905,
//     and flash_attention2_prefill_kernel_fp16, flash_attention2_kernel.cu:68-257, 822-855);
//  * bidirectional varlen vision attention over q/k/v [H, N, d]
//    (replaces the cuBLAS QK^T / softmax / PV / transpose sequence of
//     vision_attention_pretransposed_cu, vision_encoder_kernel.cu:954-1021).
//
// Work decomposition.  A workgroup of 4 waves (one per SIMD) owns BM = 256 query rows
// of one query head; each wave owns 64 rows as two 32-row sub-blocks.  The Q rows sit
// in LDS for the whole kernel; key/value tiles of BN = 64 rows are staged in LDS
// (double-buffered, one barrier per tile) and shared by the 4 waves.  Every K or V fragment read from LDS feeds two MFMAs (one per
// sub-block), which halves LDS traffic per MFMA relative to one sub-block per wave.
//
// Per wave, sub-block and tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][q] = K . Q^T      A = K rows from LDS (one 16-byte ds_read per lane),
//                              B = Q fragment from LDS (one 16-byte ds_read per lane).
//   The 32x32 accumulator layout puts one query column in each lane (lane l holds
//   query l%32 and 16 key rows), so the row max / row sum of the online softmax are
//   in-lane reductions plus one v_permlane32_swap with lane l^32.
//   O^T[d][q] += V^T . P^T     B = P^T taken straight from the S^T accumulator
//                              registers (rounded to 16 bits), A = V^T from LDS.
//   V is transposed while it is written to LDS, with the 4-key blocks of every 16-key
//   group stored in the order the S^T accumulator hands them to lanes, so each A
//   fragment is again one 16-byte ds_read.  O^T keeps one query per lane, so the
//   online-softmax rescale is a per-lane scalar multiply.
//
// Softmax: exp2 with the scale folded into one FMA; the running max used in the
// exponent is only raised when a row's max grows by more than 2^8 (lazy rescale: the
// weights stay <= 256, exact in fp16/bf16 range, and O is rescaled only when some lane
// of the wave needs it); row sums come from v_dot2 on the packed 16-bit weights, so
// the normaliser is the sum of exactly the weights the PV MFMA used.
//
// Scheduling: causal blocks start longest-first.  When the kv heads split evenly over
// the 8 XCDs, block i (dispatched to XCD i % 8) serves a query head of kv head
// i % 8 + 8k, so a kv head's K/V stay in one XCD's L2.
#include "common.h"
#include "kernels.h"

namespace orin {

namespace {

constexpr int kFwdWaves = 4;
constexpr int kFwdThreads = kFwdWaves * kWave;
constexpr int BN = 64;                  // key rows per tile
constexpr int kXcds = 8;
#ifndef FWD_SUB
#define FWD_SUB 1
#endif
constexpr float kLazyRescale = 8.0f;    // log2 growth of the row max that forces a rescale

template <int D, int SUB>
struct FwdShape {
  // SUB 32-row query sub-blocks per wave; with SUB > 1 every K/V fragment read from LDS
  // feeds SUB MFMAs, and the Q rows live in LDS to leave registers for the accumulators.
  static constexpr int BM = 32 * SUB * kFwdWaves;  // query rows per workgroup
  static constexpr bool Q_IN_LDS = SUB > 1;
  static_assert(D % 8 == 0, "head size must be a multiple of 8");
  static constexpr int DK = (D + 15) / 16 * 16;  // contraction length of QK^T
  static constexpr int DO = (D + 31) / 32 * 32;  // output rows of O^T
  static constexpr int KS = DK / 16;             // MFMA k-steps for QK^T
  static constexpr int OT = DO / 32;             // 32-row output tiles
  static constexpr int DC = D / 8;               // 16-byte chunks per real row
  static constexpr int DKC = DK / 8;             // 16-byte chunks per LDS K row
  static constexpr int SK = DK + 8;              // LDS K row stride (elements)
  static constexpr int SV = BN + 8;              // LDS V^T row stride (elements)
  static constexpr int K_ELEMS = BN * SK;        // one K buffer
  static constexpr int V_ELEMS = DO * SV;        // one V^T buffer
  static constexpr int KCH = (BN * DKC + kFwdThreads - 1) / kFwdThreads;  // K chunks / thread
  static constexpr int VU_TOTAL = (BN / 4) * (DO / 8);                    // 4x8 V units
  static constexpr int VU = (VU_TOTAL + kFwdThreads - 1) / kFwdThreads;   // V units / thread
  static constexpr int SQ = DK + 8;              // LDS Q row stride (elements)
  static constexpr int Q_ELEMS = Q_IN_LDS ? BM * SQ : 0;  // the workgroup's Q rows
  static constexpr size_t LDS_BYTES = (2 * (K_ELEMS + V_ELEMS) + Q_ELEMS) * 2;
};

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

// Two floats rounded to T (round to nearest even), packed low | high << 16.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, T2{(T)x, (T)y});
}

// acc + p.x + p.y for a packed 16-bit pair (fp32 accumulate).
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

// x of lane l^32.  v_permlane32_swap exchanges the upper half of its first operand
// with the lower half of its second; with both holding x, one result has x[l^32] in
// the lower lanes and the other in the upper lanes.  The second operand is an opaque
// copy: this toolchain folds permlane32_swap(x, x) to {x, x}, which is wrong for the
// lanes that should receive the other half.
__device__ __forceinline__ float partner32(float x) {
  int y;
  __asm__("v_mov_b32 %0, %1" : "=v"(y) : "v"(__builtin_bit_cast(int, x)));
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), y, false, false);
  return __builtin_bit_cast(float, (__lane_id() < 32) ? r[1] : r[0]);
}
// Max / sum of x over lanes l and l^32 (every lane gets the result).
__device__ __forceinline__ float pair_max(float x) { return fmaxf(x, partner32(x)); }
__device__ __forceinline__ float pair_sum(float x) { return x + partner32(x); }

// Position of key k (0..63) inside an LDS V^T row: the 4-key blocks of each 16-key
// group are stored in the order (0, 2, 1, 3).
__device__ __forceinline__ int vt_pos(int k) {
  const int b = (k >> 2) & 3;
  const int pb = (b == 1) ? 2 : (b == 2) ? 1 : b;
  return (k & ~15) | (pb << 2) | (k & 3);
}

// Register staging of one K/V tile: global -> registers, then registers -> LDS.
template <typename T, int D>
struct TileStage {
  using S = FwdShape<D, 1>;
  u32x4 k[S::KCH];
  u32x4 v[S::VU][4];

  __device__ __forceinline__ void load(const T* kb, const T* vb, long tok_stride, int t0,
                                       int kv_end, int tid) {
    // Whole tile inside the sequence and no padded chunks: unconditional loads.
    if (t0 + BN <= kv_end && S::DC == S::DKC && S::VU_TOTAL % kFwdThreads == 0 &&
        (BN * S::DKC) % kFwdThreads == 0 && S::DC * 8 == S::DO) {
#pragma unroll
      for (int i = 0; i < S::KCH; ++i) {
        const int c = tid + i * kFwdThreads;
        const int row = c / S::DKC, ch = c % S::DKC;
        k[i] = *reinterpret_cast<const u32x4*>(kb + (long)(t0 + row) * tok_stride + ch * 8);
      }
#pragma unroll
      for (int i = 0; i < S::VU; ++i) {
        const int u = tid + i * kFwdThreads;
        const int kb4 = u % (BN / 4), db = u / (BN / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          v[i][r] = *reinterpret_cast<const u32x4*>(vb + (long)(t0 + kb4 * 4 + r) * tok_stride +
                                                    db * 8);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < S::KCH; ++i) {
      const int c = tid + i * kFwdThreads;
      const int row = c / S::DKC, ch = c % S::DKC;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (c < BN * S::DKC && ch < S::DC && t0 + row < kv_end)
        val = *reinterpret_cast<const u32x4*>(kb + (long)(t0 + row) * tok_stride + ch * 8);
      k[i] = val;
    }
#pragma unroll
    for (int i = 0; i < S::VU; ++i) {
      const int u = tid + i * kFwdThreads;
      const int kb4 = u % (BN / 4), db = u / (BN / 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x4 val = {0u, 0u, 0u, 0u};
        const int key = t0 + kb4 * 4 + r;
        if (u < S::VU_TOTAL && db < S::DC && key < kv_end)
          val = *reinterpret_cast<const u32x4*>(vb + (long)key * tok_stride + db * 8);
        v[i][r] = val;
      }
    }
  }

  __device__ __forceinline__ void store(T* sK, T* sV, int tid) const {
#pragma unroll
    for (int i = 0; i < S::KCH; ++i) {
      const int c = tid + i * kFwdThreads;
      if (c < BN * S::DKC) {
        const int row = c / S::DKC, ch = c % S::DKC;
        *reinterpret_cast<u32x4*>(sK + row * S::SK + ch * 8) = k[i];
      }
    }
#pragma unroll
    for (int i = 0; i < S::VU; ++i) {
      const int u = tid + i * kFwdThreads;
      if (u < S::VU_TOTAL) {
        const int kb4 = u % (BN / 4), db = u / (BN / 4);
        const int pos = vt_pos(kb4 * 4);
        // 4 keys x 8 dims -> 8 rows (dims) of 4 consecutive keys.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1, sh = (e & 1) * 16;
          const uint32_t x0 = (v[i][0][w] >> sh) & 0xffffu, x1 = (v[i][1][w] >> sh) & 0xffffu;
          const uint32_t x2 = (v[i][2][w] >> sh) & 0xffffu, x3 = (v[i][3][w] >> sh) & 0xffffu;
          u32x2 pk = {x0 | (x1 << 16), x2 | (x3 << 16)};
          *reinterpret_cast<u32x2*>(sV + (db * 8 + e) * S::SV + pos) = pk;
        }
      }
    }
  }
};

template <typename T, int D, int SUB, bool CAUSAL>
__global__ void __launch_bounds__(kFwdThreads, SUB == 1 ? 2 : 1) fwd_kernel(FwdArgs a) {
  using S = FwdShape<D, SUB>;
  constexpr int kSub = SUB;
  constexpr int BM = S::BM;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* sKbuf = reinterpret_cast<T*>(smem);
  T* sVbuf = sKbuf + 2 * S::K_ELEMS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lq = lane & 31, hf = lane >> 5;

  int head, q_lo, q_n, seg_start, kv_end, pos_off;
  if (CAUSAL) {
    const int nqb = (a.n_q + BM - 1) / BM;
    int qb;
    if (a.Hkv % kXcds == 0) {
      // XCD-aware: block i runs on XCD i % 8 and serves kv head i % 8 + 8k.
      const int x = (int)blockIdx.x % kXcds, i = (int)blockIdx.x / kXcds;
      const int hpx = a.Hq / kXcds;  // query heads per XCD
      qb = nqb - 1 - i / hpx;
      const int hl = i % hpx;
      head = (x + kXcds * (hl / a.kv_mul)) * a.kv_mul + hl % a.kv_mul;
    } else {
      qb = nqb - 1 - (int)blockIdx.x / a.Hq;
      head = (int)blockIdx.x % a.Hq;
    }
    q_lo = qb * BM;
    q_n = a.n_q;
    seg_start = 0;
    pos_off = a.start_pos;
    kv_end = a.start_pos + min(q_lo + BM, a.n_q);
  } else {
    const int nqb = (a.max_seqlen + BM - 1) / BM;
    head = (int)blockIdx.x % a.Hq;
    const int rest = (int)blockIdx.x / a.Hq;
    const int qb = rest % nqb, seg = rest / nqb;
    seg_start = a.cu_seqlens ? a.cu_seqlens[seg] : 0;
    q_n = a.cu_seqlens ? a.cu_seqlens[seg + 1] - seg_start : a.n_q;
    q_lo = qb * BM;
    if (q_lo >= q_n) return;
    pos_off = 0;
    kv_end = q_n;
  }
  const int kvh = head / a.kv_mul;
  const T* kb = reinterpret_cast<const T*>(a.k) + (long)seg_start * a.kv_tok_stride +
                (long)kvh * a.kv_head_stride;
  const T* vb = reinterpret_cast<const T*>(a.v) + (long)seg_start * a.kv_tok_stride +
                (long)kvh * a.kv_head_stride;

  // Q fragments: sub-block j, query row q_lo + wave*32*SUB + 32j + lq, dims
  // 16s + 8hf + 0..7.  With SUB > 1 the workgroup's Q rows go to LDS once (zero-padded
  // to DK and past q_n) and each wave reads its fragments per k-step, which keeps
  // registers free for the accumulators; with SUB == 1 they stay in registers.
  const int wq0 = q_lo + wave * 32 * kSub;  // first local query of the wave
  T* sQ = sVbuf + 2 * S::V_ELEMS;
  u32x4 qreg[S::Q_IN_LDS ? 1 : kSub][S::Q_IN_LDS ? 1 : S::KS];
  if constexpr (S::Q_IN_LDS) {
    for (int c = tid; c < BM * S::DKC; c += kFwdThreads) {
      const int row = c / S::DKC, ch = c % S::DKC;
      const int qi = q_lo + row;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (qi < q_n && ch < S::DC)
        val = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.q) +
                                              (long)(seg_start + qi) * a.q_tok_stride +
                                              (long)head * a.q_head_stride + ch * 8);
      *reinterpret_cast<u32x4*>(sQ + row * S::SQ + ch * 8) = val;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
      const int qi = wq0 + 32 * j + lq;
      const T* qp = reinterpret_cast<const T*>(a.q) + (long)(seg_start + qi) * a.q_tok_stride +
                    (long)head * a.q_head_stride;
#pragma unroll
      for (int s = 0; s < S::KS; ++s) {
        const int d0 = 16 * s + 8 * hf;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qi < q_n && d0 < D) val = *reinterpret_cast<const u32x4*>(qp + d0);
        qreg[S::Q_IN_LDS ? 0 : j][S::Q_IN_LDS ? 0 : s] = val;
      }
    }
  }
  const T* sQw = sQ + (wave * 32 * kSub + lq) * S::SQ + 8 * hf;

  f32x16 oacc[kSub][S::OT];
#pragma unroll
  for (int j = 0; j < kSub; ++j)
#pragma unroll
    for (int t = 0; t < S::OT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[j][t][r] = 0.f;
  float m_use[kSub], l_run[kSub];
#pragma unroll
  for (int j = 0; j < kSub; ++j) {
    m_use[j] = -INFINITY;
    l_run[j] = 0.f;
  }
  const float c = a.scale_log2;
  const int wpos0 = pos_off + wq0;  // position of the wave's first query

  const int n_tiles = (kv_end + BN - 1) / BN;
  TileStage<T, D> stage;
  stage.load(kb, vb, a.kv_tok_stride, 0, kv_end, tid);
  stage.store(sKbuf, sVbuf, tid);
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = it * BN;
    const T* sK = sKbuf + (it & 1) * S::K_ELEMS;
    const T* sV = sVbuf + (it & 1) * S::V_ELEMS;
    const bool more = it + 1 < n_tiles;
    if (more) stage.load(kb, vb, a.kv_tok_stride, t0 + BN, kv_end, tid);

    // Sub-block j is active if some of its queries see key t0 (causal).
    bool act[kSub];
#pragma unroll
    for (int j = 0; j < kSub; ++j) act[j] = !CAUSAL || t0 <= wpos0 + 32 * j + 31;

    if (act[kSub - 1]) {
      // S^T = K . Q^T for keys t0..t0+63 (two 32-key halves), both sub-blocks.
      f32x16 sacc[kSub][2];
#pragma unroll
      for (int j = 0; j < kSub; ++j)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[j][kt][r] = 0.f;
      // K fragments of k-step s+1 are read from LDS before the MFMAs of k-step s issue.
      u32x4 kf[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        kf[0][kt] = *reinterpret_cast<const u32x4*>(sK + (kt * 32 + lq) * S::SK + 8 * hf);
#pragma unroll
      for (int s = 0; s < S::KS; ++s) {
        if (s + 1 < S::KS) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
            kf[(s + 1) & 1][kt] = *reinterpret_cast<const u32x4*>(
                sK + (kt * 32 + lq) * S::SK + 16 * (s + 1) + 8 * hf);
        }
        u32x4 qf[kSub];
#pragma unroll
        for (int j = 0; j < kSub; ++j)
          qf[j] = S::Q_IN_LDS ? *reinterpret_cast<const u32x4*>(sQw + 32 * j * S::SQ + 16 * s)
                              : qreg[S::Q_IN_LDS ? 0 : j][S::Q_IN_LDS ? 0 : s];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < kSub; ++j)
            if (act[j]) sacc[j][kt] = mfma32<T>(kf[s & 1][kt], qf[j], sacc[j][kt]);
      }

      u32x4 pf[kSub][4];
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
        if (!act[j]) continue;
        // Mask (causal diagonal / segment tail) and the row max.
        const int qpos = wpos0 + 32 * j + lq;
        // Uniform per wave: only tiles on the diagonal / past the segment end mask.
        const bool need_mask = CAUSAL ? (t0 + BN - 1 > wpos0 + 32 * j) : (t0 + BN > kv_end);
        if (need_mask) {
          const int lim = CAUSAL ? qpos : kv_end - 1;  // last key this lane's query sees
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kp = t0 + kt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
              sacc[j][kt][r] = kp > lim ? -INFINITY : sacc[j][kt][r];
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[j][kt][r]);
        mx = pair_max(mx) * c;
        // Lazy rescale: raise the exponent offset only when the max grew by > 2^8.
        const float m_old = m_use[j];
        const float m_new = (mx > m_old + kLazyRescale) ? mx : m_old;
        m_use[j] = m_new;
        if (__builtin_amdgcn_ballot_w64(m_new != m_old)) {
          const float alpha = fast_exp2(m_old - m_new);  // 1 where unchanged
          l_run[j] *= alpha;
#pragma unroll
          for (int t = 0; t < S::OT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[j][t][r] *= alpha;
        }
        float ls = l_run[j];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float p0 = fast_exp2(__builtin_fmaf(sacc[j][kt][r], c, -m_new));
            const float p1 = fast_exp2(__builtin_fmaf(sacc[j][kt][r + 1], c, -m_new));
            const uint32_t pk = pack2<T>(p0, p1);
            pf[j][kt * 2 + (r >> 3)][(r & 7) >> 1] = pk;
            ls = sum_pair<T>(pk, ls);
          }
        l_run[j] = ls;
      }

      // O^T += V^T . P^T over the 4 16-key chunks of the tile; the V fragment of the
      // next (chunk, d-tile) is read from LDS before the current MFMAs issue.
      constexpr int NPV = 4 * S::OT;
      u32x4 vf[2];
      vf[0] = *reinterpret_cast<const u32x4*>(sV + lq * S::SV + 8 * hf);
#pragma unroll
      for (int n = 0; n < NPV; ++n) {
        const int ck = n / S::OT, t = n % S::OT;
        if (n + 1 < NPV) {
          const int ck1 = (n + 1) / S::OT, t1 = (n + 1) % S::OT;
          vf[(n + 1) & 1] = *reinterpret_cast<const u32x4*>(sV + (t1 * 32 + lq) * S::SV +
                                                            16 * ck1 + 8 * hf);
        }
#pragma unroll
        for (int j = 0; j < kSub; ++j)
          if (act[j]) oacc[j][t] = mfma32<T>(vf[n & 1], pf[j][ck], oacc[j][t]);
      }
    }

    if (more) {
      stage.store(sKbuf + ((it + 1) & 1) * S::K_ELEMS, sVbuf + ((it + 1) & 1) * S::V_ELEMS, tid);
      __syncthreads();
    }
  }

  // Normalise and store: lane holds dims t*32 + 8*(r/4) + 4*hf + r%4 of its query.
#pragma unroll
  for (int j = 0; j < kSub; ++j) {
    const int qi = wq0 + 32 * j + lq;
    const float inv = 1.f / pair_sum(l_run[j]);
    if (qi < q_n) {
      T* op = reinterpret_cast<T*>(a.o) + (long)(seg_start + qi) * a.o_tok_stride +
              (long)head * a.o_head_stride;
#pragma unroll
      for (int t = 0; t < S::OT; ++t)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int d0 = t * 32 + 8 * rg + 4 * hf;
          if (d0 < D) {
            u32x2 pk = {pack2<T>(oacc[j][t][4 * rg] * inv, oacc[j][t][4 * rg + 1] * inv),
                        pack2<T>(oacc[j][t][4 * rg + 2] * inv, oacc[j][t][4 * rg + 3] * inv)};
            *reinterpret_cast<u32x2*>(op + d0) = pk;
          }
        }
    }
  }
}

template <typename T, int D, int SUB, bool CAUSAL>
hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t stream) {
  constexpr int BM = FwdShape<D, SUB>::BM;
  long blocks;
  if (CAUSAL)
    blocks = (long)((a.n_q + BM - 1) / BM) * a.Hq;
  else
    blocks = (long)a.n_seg * ((a.max_seqlen + BM - 1) / BM) * a.Hq;
  if (blocks <= 0) return hipSuccess;
  constexpr size_t lds = FwdShape<D, SUB>::LDS_BYTES;
  // The dynamic-LDS limit is a per-device function attribute: set it once per device.
  static unsigned long long configured = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 64 || !(__atomic_load_n(&configured, __ATOMIC_ACQUIRE) & (1ull << dev))) {
    e = hipFuncSetAttribute((const void*)fwd_kernel<T, D, SUB, CAUSAL>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    if (dev < 64) __atomic_fetch_or(&configured, 1ull << dev, __ATOMIC_RELEASE);
  }
  hipLaunchKernelGGL((fwd_kernel<T, D, SUB, CAUSAL>), dim3((unsigned)blocks), dim3(kFwdThreads),
                     lds, stream, a);
  return hipGetLastError();
}

template <bool CAUSAL, typename T>
hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_fwd_t<T, 64, FWD_SUB, CAUSAL>(a, stream);
    case 72: return launch_fwd_t<T, 72, FWD_SUB, CAUSAL>(a, stream);
    case 80: return launch_fwd_t<T, 80, FWD_SUB, CAUSAL>(a, stream);
    case 96: return launch_fwd_t<T, 96, FWD_SUB, CAUSAL>(a, stream);
    case 128: return launch_fwd_t<T, 128, FWD_SUB, CAUSAL>(a, stream);
  }
  return hipErrorInvalidValue;
}

template <bool CAUSAL>
hipError_t launch_fwd(const FwdArgs& a, int dtype, hipStream_t stream) {
  if (dtype == kF16) return launch_fwd_d<CAUSAL, f16>(a, stream);
  if (dtype == kBF16) return launch_fwd_d<CAUSAL, bf16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool fwd_supports(int dtype, int head_size) {
  return (dtype == kF16 || dtype == kBF16) &&
         (head_size == 64 || head_size == 72 || head_size == 80 || head_size == 96 ||
          head_size == 128);
}

hipError_t launch_fwd_causal(const FwdArgs& a, int dtype, hipStream_t stream) {
  return launch_fwd<true>(a, dtype, stream);
}

hipError_t launch_fwd_varlen(const FwdArgs& a, int dtype, hipStream_t stream) {
  return launch_fwd<false>(a, dtype, stream);
}

}  // namespace orin
