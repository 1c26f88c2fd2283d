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
// Work decomposition.  A workgroup of NW = 4 waves owns BM = 32*NW query rows of one
// query head; each wave owns 32 rows whose Q fragments stay in registers.  Key/value tiles of BN = 64 rows are
// staged in LDS (double-buffered through registers, one barrier per tile) and shared by
// the waves.  Two waves share each SIMD, so one wave's softmax VALU work can fill the
// other's MFMA cycles.
//
// Per wave and tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][q] = K . Q^T      A = K rows from LDS (one 16-byte ds_read per lane, read
//                              one k-step ahead), B = Q fragment in registers.
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
// weights stay <= 256, inside fp16/bf16 range, and O is rescaled only when some lane
// of the wave needs it); row sums come from v_dot2 on the packed 16-bit weights, so
// the normaliser is the sum of exactly the weights the PV MFMA used.  The QK^T MFMAs
// run at raised wave priority (s_setprio 1), which measured faster than no priority
// change and than raising it around the PV MFMAs as well.
//
// Scheduling: causal blocks start longest-first.  When the kv heads split evenly over
// the 8 XCDs, block i (dispatched to XCD i % 8) serves a query head of kv head
// i % 8 + 8k, so a kv head's K/V stay in one XCD's L2.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace orin {

namespace {

constexpr int BN = 64;                // key rows per tile
constexpr int kXcds = 8;
constexpr float kLazyRescale = 8.0f;  // log2 growth of the row max that forces a rescale

template <int D, int NW>
struct FwdShape {
  static_assert(D % 8 == 0, "head size must be a multiple of 8");
  static_assert(NW == 2 || NW == 4, "2 or 4 waves per workgroup");
  static constexpr int THREADS = NW * kWave;
  static constexpr int BM = 32 * NW;             // query rows per workgroup
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
  static constexpr int KCH = (BN * DKC + THREADS - 1) / THREADS;  // K chunks / thread
  static constexpr int VU_TOTAL = (BN / 4) * (DO / 8);            // 4-key x 8-dim V units
  static constexpr int VU = (VU_TOTAL + THREADS - 1) / THREADS;   // V units / thread
  // Every thread's chunks are real data (no padding, no partial last pass).
  static constexpr bool EXACT = DC == DKC && DC * 8 == DO && VU_TOTAL % THREADS == 0 &&
                                (BN * DKC) % THREADS == 0;
  static constexpr size_t LDS_BYTES = 2 * (K_ELEMS + V_ELEMS) * 2;  // double-buffered
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
template <typename T, int D, int NW>
struct TileStage {
  using S = FwdShape<D, NW>;
  u32x4 k[S::KCH];
  u32x4 v[S::VU][4];

  __device__ __forceinline__ void load(const T* kb, const T* vb, long tok_stride, int t0,
                                       int kv_end, int tid) {
    if (S::EXACT && t0 + BN <= kv_end) {  // whole tile inside the sequence: no guards
#pragma unroll
      for (int i = 0; i < S::KCH; ++i) {
        const int c = tid + i * S::THREADS;
        const int row = c / S::DKC, ch = c % S::DKC;
        k[i] = *reinterpret_cast<const u32x4*>(kb + (long)(t0 + row) * tok_stride + ch * 8);
      }
#pragma unroll
      for (int i = 0; i < S::VU; ++i) {
        const int u = tid + i * S::THREADS;
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
      const int c = tid + i * S::THREADS;
      const int row = c / S::DKC, ch = c % S::DKC;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (c < BN * S::DKC && ch < S::DC && t0 + row < kv_end)
        val = *reinterpret_cast<const u32x4*>(kb + (long)(t0 + row) * tok_stride + ch * 8);
      k[i] = val;
    }
#pragma unroll
    for (int i = 0; i < S::VU; ++i) {
      const int u = tid + i * S::THREADS;
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
      const int c = tid + i * S::THREADS;
      if (c < BN * S::DKC) {
        const int row = c / S::DKC, ch = c % S::DKC;
        *reinterpret_cast<u32x4*>(sK + row * S::SK + ch * 8) = k[i];
      }
    }
#pragma unroll
    for (int i = 0; i < S::VU; ++i) {
      const int u = tid + i * S::THREADS;
      if (u < S::VU_TOTAL) {
        const int kb4 = u % (BN / 4), db = u / (BN / 4);
        const int pos = vt_pos(kb4 * 4);
        // 4 keys x 8 dims -> 8 rows (dims) of 4 consecutive keys; bf16 V is stored as
        // fp16 (the PV product runs on fp16 MFMAs with fp16 weights).
        u32x4 vv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          vv[r] = std::is_same<T, f16>::value ? v[i][r] : bf16x8_to_f16x8(v[i][r]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // element e of keys (0,1) and (2,3): one v_perm_b32 per packed pair
          const int w = e >> 1;
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          u32x2 pk = {__builtin_amdgcn_perm(vv[1][w], vv[0][w], sel),
                      __builtin_amdgcn_perm(vv[3][w], vv[2][w], sel)};
          *reinterpret_cast<u32x2*>(sV + (db * 8 + e) * S::SV + pos) = pk;
        }
      }
    }
  }
};

template <typename T, int D, int NW, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) fwd_kernel(FwdArgs a) {
  using S = FwdShape<D, NW>;
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

  // Q fragment of this lane: query row wq0 + lq, dims 16s + 8hf + 0..7 of k-step s.
  const int wq0 = q_lo + wave * 32;  // first local query of the wave
  const int qi = wq0 + lq;
  u32x4 qf[S::KS];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (long)(seg_start + qi) * a.q_tok_stride +
                  (long)head * a.q_head_stride;
#pragma unroll
    for (int s = 0; s < S::KS; ++s) {
      const int d0 = 16 * s + 8 * hf;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (qi < q_n && d0 < D) val = *reinterpret_cast<const u32x4*>(qp + d0);
      qf[s] = val;
    }
    // Settle the Q loads here: without this the loop-header wait merges them with the
    // next tile's prefetch and waits for all outstanding loads (vmcnt(0)) every tile.
#pragma unroll
    for (int s = 0; s < S::KS; ++s) __asm__ volatile("" : "+v"(qf[s]));
  }

  f32x16 oacc[S::OT];
#pragma unroll
  for (int t = 0; t < S::OT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_use = -INFINITY, l_run = 0.f;
  const float c = a.scale_log2;
  const int wpos0 = pos_off + wq0;  // position of the wave's first query
  const int qpos = wpos0 + lq;      // position of this lane's query

  const int n_tiles = (kv_end + BN - 1) / BN;
  TileStage<T, D, NW> stage;
  stage.load(kb, vb, a.kv_tok_stride, 0, kv_end, tid);
  stage.store(sKbuf, sVbuf, tid);
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = it * BN;
    const T* sK = sKbuf + (it & 1) * S::K_ELEMS;
    const T* sV = sVbuf + (it & 1) * S::V_ELEMS;
    const bool more = it + 1 < n_tiles;
    if (more) stage.load(kb, vb, a.kv_tok_stride, t0 + BN, kv_end, tid);

    // Causal: tiles wholly above this wave's diagonal contribute nothing.
    if (!CAUSAL || t0 <= wpos0 + 31) {
      // S^T = K . Q^T for keys t0..t0+63 (two 32-key halves); the K fragments of
      // k-step s+1 are read from LDS before the MFMAs of k-step s issue.
      f32x16 sacc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
      __builtin_amdgcn_s_setprio(1);
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
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) sacc[kt] = mfma32<T>(kf[s & 1][kt], qf[s], sacc[kt]);
      }
      __builtin_amdgcn_s_setprio(0);

      // Mask (wave-uniform test: only tiles on the diagonal / past the segment end).
      const bool need_mask = CAUSAL ? (t0 + BN - 1 > wpos0) : (t0 + BN > kv_end);
      if (need_mask) {
        const int lim = CAUSAL ? qpos : kv_end - 1;  // last key this lane's query sees
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kp = t0 + kt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            sacc[kt][r] = kp > lim ? -INFINITY : sacc[kt][r];
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
      mx = pair_max(mx) * c;
      // Lazy rescale: raise the exponent offset only when the max grew by > 2^8.
      const float m_old = m_use;
      const float m_new = (mx > m_old + kLazyRescale) ? mx : m_old;
      m_use = m_new;
      if (__builtin_amdgcn_ballot_w64(m_new != m_old)) {
        const float alpha = fast_exp2(m_old - m_new);  // 1 where unchanged
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < S::OT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      }
      u32x4 pf[4];
      float ls = l_run;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = fast_exp2(__builtin_fmaf(sacc[kt][r], c, -m_new));
          const float p1 = fast_exp2(__builtin_fmaf(sacc[kt][r + 1], c, -m_new));
          const uint32_t pk = pack2<f16>(p0, p1);
          pf[kt * 2 + (r >> 3)][(r & 7) >> 1] = pk;
          ls = sum_pair<f16>(pk, ls);
        }
      l_run = ls;

      // O^T += V^T . P^T over the 4 16-key chunks of the tile; the V fragment of the
      // next (chunk, d-tile) is read from LDS before the current MFMA issues.
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
        oacc[t] = mfma32<f16>(vf[n & 1], pf[ck], oacc[t]);
      }
    }

    if (more) {
      stage.store(sKbuf + ((it + 1) & 1) * S::K_ELEMS, sVbuf + ((it + 1) & 1) * S::V_ELEMS, tid);
      __syncthreads();
    }
  }

  // Normalise and store: the lane holds dims t*32 + 8*(r/4) + 4*hf + r%4 of its query.
  const float inv = 1.f / pair_sum(l_run);
  if (qi < q_n) {
    T* op = reinterpret_cast<T*>(a.o) + (long)(seg_start + qi) * a.o_tok_stride +
            (long)head * a.o_head_stride;
#pragma unroll
    for (int t = 0; t < S::OT; ++t)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d0 = t * 32 + 8 * rg + 4 * hf;
        if (d0 < D) {
          u32x2 pk = {pack2<T>(oacc[t][4 * rg] * inv, oacc[t][4 * rg + 1] * inv),
                      pack2<T>(oacc[t][4 * rg + 2] * inv, oacc[t][4 * rg + 3] * inv)};
          *reinterpret_cast<u32x2*>(op + d0) = pk;
        }
      }
  }
}

template <int BM, bool CAUSAL>
long fwd_blocks(const FwdArgs& a) {
  if (CAUSAL) return (long)((a.n_q + BM - 1) / BM) * a.Hq;
  return (long)a.n_seg * ((a.max_seqlen + BM - 1) / BM) * a.Hq;
}

template <typename T, int D, int NW, bool CAUSAL>
hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t stream) {
  using S = FwdShape<D, NW>;
  const long blocks = fwd_blocks<S::BM, CAUSAL>(a);
  if (blocks <= 0) return hipSuccess;
  // The dynamic-LDS limit is a per-device function attribute: set it once per device.
  static unsigned long long configured = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 64 || !(__atomic_load_n(&configured, __ATOMIC_ACQUIRE) & (1ull << dev))) {
    e = hipFuncSetAttribute((const void*)fwd_kernel<T, D, NW, CAUSAL>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::LDS_BYTES);
    if (e != hipSuccess) return e;
    if (dev < 64) __atomic_fetch_or(&configured, 1ull << dev, __ATOMIC_RELEASE);
  }
  hipLaunchKernelGGL((fwd_kernel<T, D, NW, CAUSAL>), dim3((unsigned)blocks), dim3(S::THREADS),
                     S::LDS_BYTES, stream, a);
  return hipGetLastError();
}

// 4-wave workgroups.  A 2-wave variant (BM = 64) for grids below two workgroups per CU
// measured no faster on Qwen3-VL-2B-sized prefill (12 heads, 2048 tokens): there the
// longest causal block, not the grid size, bounds the time.
template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd_w(const FwdArgs& a, hipStream_t stream) {
  return launch_fwd_t<T, D, 4, CAUSAL>(a, stream);
}

template <bool CAUSAL, typename T>
hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_fwd_w<T, 64, CAUSAL>(a, stream);
    case 72: return launch_fwd_w<T, 72, CAUSAL>(a, stream);
    case 80: return launch_fwd_w<T, 80, CAUSAL>(a, stream);
    case 96: return launch_fwd_w<T, 96, CAUSAL>(a, stream);
    case 128: return launch_fwd_w<T, 128, CAUSAL>(a, stream);
  }
  return hipErrorInvalidValue;
}

// Head sizes 64-128 go to the ping-pong kernel (256-query workgroups, one per CU) when its
// grid covers every CU at least once, or when the caller planned a key split for a causal
// launch that does not (fwd_pp_key_split).
template <bool CAUSAL>
bool use_pp(const FwdArgs& a, int dtype) {
  if (!fwd_pp_supports(a, dtype)) return false;
  if (CAUSAL && (a.key_chunk_tiles > 0 || a.rope_sin)) return true;
  const long blocks = CAUSAL ? (long)((a.n_q + 255) / 256) * a.Hq
                             : (long)a.n_seg * ((a.max_seqlen + 255) / 256) * a.Hq;
  return blocks >= 256;
}

template <bool CAUSAL>
hipError_t launch_fwd(const FwdArgs& a, int dtype, hipStream_t stream) {
  if (use_pp<CAUSAL>(a, dtype)) return launch_fwd_pp(a, dtype, CAUSAL, stream);
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
