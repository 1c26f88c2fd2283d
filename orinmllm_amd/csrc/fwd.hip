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
// Work decomposition.  A workgroup of 4 waves owns BM = 128 query rows of one
// query head; each wave owns 32 rows.  Key/value tiles of BN = 64 rows are staged
// in LDS once per workgroup and shared by the 4 waves.
//
// Per wave and tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][q] = K . Q^T      A = K rows from LDS (16-byte ds_read per lane),
//                              B = Q fragment held in registers for the whole kernel.
//   The 32x32 accumulator layout puts one query column in each lane (lane l holds
//   query l%32 and 16 key rows), so the row max / row sum of the online softmax are
//   in-lane reductions plus one exchange with lane l^32.
//   O^T[d][q] += V^T . P^T     B = P^T taken straight from the S^T accumulator
//                              registers (converted to 16-bit), A = V^T from LDS.
//   V is transposed while it is written to LDS, with the 4-key blocks of every
//   16-key group stored in the order the S^T accumulator hands them to lanes,
//   so each A fragment is again one 16-byte ds_read.
//   O^T keeps one query per lane too, so the online-softmax rescale is a
//   per-lane scalar multiply.
//
// Causal scheduling: blocks are numbered so that the query blocks with the most
// key tiles start first (longest-processing-time order across heads).
#include "common.h"
#include "kernels.h"

namespace orin {

namespace {

constexpr int kFwdWaves = 4;
constexpr int kFwdThreads = kFwdWaves * kWave;
constexpr int BM = 32 * kFwdWaves;  // query rows per workgroup
constexpr int BN = 64;              // key rows per tile

template <int D>
struct FwdShape {
  static_assert(D % 8 == 0, "head size must be a multiple of 8");
  static constexpr int DK = (D + 15) / 16 * 16;  // contraction length of QK^T
  static constexpr int DO = (D + 31) / 32 * 32;  // output rows of O^T
  static constexpr int KS = DK / 16;             // MFMA k-steps for QK^T
  static constexpr int OT = DO / 32;             // 32-row output tiles
  static constexpr int DC = D / 8;               // 16-byte chunks per real row
  static constexpr int DKC = DK / 8;             // 16-byte chunks per LDS K row
  static constexpr int SK = DK + 8;              // LDS K row stride (elements)
  static constexpr int SV = BN + 8;              // LDS V^T row stride (elements)
  static constexpr int KCH = (BN * DKC + kFwdThreads - 1) / kFwdThreads;  // K chunks / thread
  static constexpr int VU_TOTAL = (BN / 4) * (DO / 8);                    // 4x8 V units
  static constexpr int VU = (VU_TOTAL + kFwdThreads - 1) / kFwdThreads;   // V units / thread
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

template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  T a = from_f32<T>(x), b = from_f32<T>(y);
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

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
  using S = FwdShape<D>;
  u32x4 k[S::KCH];
  u32x4 v[S::VU][4];

  __device__ __forceinline__ void load(const T* kb, const T* vb, long tok_stride, int t0,
                                       int kv_end, int tid) {
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

template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kFwdThreads, 2) fwd_kernel(FwdArgs a) {
  using S = FwdShape<D>;
  __shared__ __attribute__((aligned(16))) T sK[BN * S::SK];
  __shared__ __attribute__((aligned(16))) T sV[S::DO * S::SV];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 31, hf = lane >> 5;

  int head, q_lo, q_n, seg_start, kv_end, pos_off;
  if (CAUSAL) {
    const int nqb = (a.n_q + BM - 1) / BM;
    const int qb = nqb - 1 - (int)blockIdx.x / a.Hq;
    head = (int)blockIdx.x % a.Hq;
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

  // Q fragment of this lane: query row q_lo + wave*32 + lq, dims 16s + 8hf + 0..7.
  const int qi = q_lo + wave * 32 + lq;  // local query index
  const bool q_valid = qi < q_n;
  u32x4 qf[S::KS];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (long)(seg_start + qi) * a.q_tok_stride +
                  (long)head * a.q_head_stride;
#pragma unroll
    for (int s = 0; s < S::KS; ++s) {
      const int d0 = 16 * s + 8 * hf;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (q_valid && d0 < D) val = *reinterpret_cast<const u32x4*>(qp + d0);
      qf[s] = val;
    }
  }

  f32x16 oacc[S::OT];
#pragma unroll
  for (int t = 0; t < S::OT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = a.scale_log2;
  const int qpos = pos_off + qi;                    // absolute position of this lane's query
  const int wave_q0 = pos_off + q_lo + wave * 32;   // first query position of the wave

  const int n_tiles = (kv_end + BN - 1) / BN;
  TileStage<T, D> stage;
  stage.load(kb, vb, a.kv_tok_stride, 0, kv_end, tid);

  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = it * BN;
    __syncthreads();  // previous tile fully consumed
    stage.store(sK, sV, tid);
    __syncthreads();
    if (it + 1 < n_tiles) stage.load(kb, vb, a.kv_tok_stride, t0 + BN, kv_end, tid);

    if (CAUSAL && t0 > wave_q0 + 31) continue;  // whole tile above this wave's diagonal

    // S^T = K . Q^T for keys t0..t0+63 (two 32-key halves).
    f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
#pragma unroll
    for (int s = 0; s < S::KS; ++s)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const u32x4 af =
            *reinterpret_cast<const u32x4*>(sK + (kt * 32 + lq) * S::SK + 16 * s + 8 * hf);
        sacc[kt] = mfma32<T>(af, qf[s], sacc[kt]);
      }

    // Scale, mask, online softmax (one query per lane, keys split with lane^32).
    const bool need_mask = CAUSAL ? (t0 + BN - 1 > wave_q0) : (t0 + BN > kv_end);
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = sacc[kt][r] * c;
        if (need_mask) {
          const int kp = t0 + kt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
          const bool dead = CAUSAL ? (kp > qpos) : (kp >= kv_end);
          x = dead ? -INFINITY : x;
        }
        sacc[kt][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    float ls = 0.f;
    u32x4 pf[4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(sacc[kt][r] - m_new);
        const float p1 = fast_exp2(sacc[kt][r + 1] - m_new);
        ls += p0 + p1;
        pf[kt * 2 + (r >> 3)][(r & 7) >> 1] = pack2<T>(p0, p1);
      }
    l_run = l_run * alpha + ls;
#pragma unroll
    for (int t = 0; t < S::OT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;

    // O^T += V^T . P^T over the 4 16-key chunks of the tile.
#pragma unroll
    for (int ck = 0; ck < 4; ++ck)
#pragma unroll
      for (int t = 0; t < S::OT; ++t) {
        const u32x4 af =
            *reinterpret_cast<const u32x4*>(sV + (t * 32 + lq) * S::SV + 16 * ck + 8 * hf);
        oacc[t] = mfma32<T>(af, pf[ck], oacc[t]);
      }
  }

  // Normalise and store: lane holds dims t*32 + 8*(r/4) + 4*hf + r%4 of its query.
  const float l_tot = l_run + shfl_xor_f(l_run, 32);
  const float inv = 1.f / l_tot;
  if (q_valid) {
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

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t stream) {
  long blocks;
  if (CAUSAL)
    blocks = (long)((a.n_q + BM - 1) / BM) * a.Hq;
  else
    blocks = (long)a.n_seg * ((a.max_seqlen + BM - 1) / BM) * a.Hq;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL>), dim3((unsigned)blocks), dim3(kFwdThreads), 0,
                     stream, a);
  return hipGetLastError();
}

template <bool CAUSAL, typename T>
hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_fwd_t<T, 64, CAUSAL>(a, stream);
    case 72: return launch_fwd_t<T, 72, CAUSAL>(a, stream);
    case 80: return launch_fwd_t<T, 80, CAUSAL>(a, stream);
    case 96: return launch_fwd_t<T, 96, CAUSAL>(a, stream);
    case 128: return launch_fwd_t<T, 128, CAUSAL>(a, stream);
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
