// Internal launch interface between the C-ABI layer (capi.hip) and the kernels.
#pragma once
#include <hip/hip_runtime.h>

namespace orin {

// Element type codes; values follow base::DataType (kuiper/include/base/base.h:58-64)
// with bf16 added.
enum { kF32 = 1, kF16 = 4, kBF16 = 5 };

// Decode / per-row attention.  Row r attends to tokens [0, len(r)) of its own
// KV sequence.  All strides are in elements.
struct DecodeArgs {
  const void* q;  // q(r, h, j) = q[r*q_row_stride + h*q_head_stride + j]
  long q_row_stride, q_head_stride;
  const void* k;  // k(r, t, g, j) = k[map_r(t) + g*kv_head_stride + j]
  const void* v;
  long kv_tok_stride, kv_head_stride, kv_row_stride;
  const int* block_table;  // paged: map_r(t) = bt[r][t>>bs_log2]*block_stride + (t&mask)*tok_stride
  long bt_row_stride;
  long block_stride;
  int bs_log2;
  const int* lens;  // len(r) = lens[r] + len_add  if lens
  int len_add;
  int len_base, len_step;  // len(r) = len_base + r*len_step otherwise
  int len_cap;             // the launch covers len(r) <= len_cap; longer rows output NaN
  const int* cu_seqlens;   // varlen: rows are tokens; row r attends its segment
  int n_seg;
  void* o;  // o(r, h, j) = o[r*o_row_stride + h*o_head_stride + j]
  long o_row_stride, o_head_stride;
  float* ws;  // [n_rows, Hq, max_splits, head_size + 2] fp32 partials (unused if max_splits == 1)
  int max_splits, split_tokens;
  int wide;  // dot-product kernel: 16-wave workgroups where the shape fits (decode.hip)
  int mfma;  // one split per row and a unit per CU or more: the matrix-core kernel where it
             // supports the shape (decode_mfma.hip)
  int n_rows, Hq, Hkv, kv_mul, head_size;
  float scale_log2;  // softmax scale * log2(e)
};

int decode_heads_per_block(int kv_mul);
bool decode_supports(int dtype, int head_size);
hipError_t launch_decode(const DecodeArgs& a, int dtype, hipStream_t stream);
// Matrix-core decode (decode_mfma.hip) for 16-bit caches, head sizes 64 / 128 and up to 16
// query heads per kv head: one workgroup per (row, kv head, split) serving all kv_mul heads.
// launch_decode routes the shapes it supports there.
bool decode_mfma_supports(int dtype, int head_size, int kv_mul);
size_t decode_mfma_lds_bytes(int head_size);
hipError_t launch_decode_mfma(const DecodeArgs& a, int dtype, hipStream_t stream);

// Tile-parallel attention forward on MFMA (fp16 / bf16): causal prefill over a
// kuiper-layout cache, or bidirectional varlen segments.
struct FwdArgs {
  const void* q;  // q(t, h, j) = q[t*q_tok_stride + h*q_head_stride + j]
  long q_tok_stride, q_head_stride;
  const void* k;  // k(t, g, j) = k[t*kv_tok_stride + g*kv_head_stride + j]
  const void* v;
  long kv_tok_stride, kv_head_stride;
  void* o;
  long o_tok_stride, o_head_stride;
  int n_q;        // query rows (causal: seq_len; varlen: total tokens)
  int start_pos;  // causal: query i sits at position start_pos + i
  const int* cu_seqlens;  // varlen (device), n_seg + 1 entries; null = one segment of n_q
  int n_seg, max_seqlen;
  int Hq, Hkv, kv_mul, head_size;
  float scale_log2;
  // Causal key split (fwd_pp.hip): > 0 cuts each query block's 64-key tiles into
  // near-equal chunks of at most this many tiles (the last chunk holds the diagonal
  // tiles); the chunks of a block write partials to ws (O / l rows, then fp32 (m, l)) and
  // a second launch merges them.  0 = off.
  int key_chunk_tiles;
  float* ws;
  // Fused Q producer (fwd_pp.hip, causal, head sizes 64 / 128): q holds the raw query rows;
  // row i is RMS-normalised (when q_norm_weight is non-null, with eps) and rotated with the
  // rope_sin / rope_cos tables (entry [p][2j] for pair (j, j + d/2)) at position
  // start_pos + i as it is loaded, with the arithmetic of launch_qk_norm_rope.  Null rope
  // tables = off.
  const void* q_norm_weight;
  const float* rope_sin;
  const float* rope_cos;
  float eps;
};

bool fwd_supports(int dtype, int head_size);
hipError_t launch_fwd_causal(const FwdArgs& a, int dtype, hipStream_t stream);
hipError_t launch_fwd_varlen(const FwdArgs& a, int dtype, hipStream_t stream);

// 8-wave ping-pong variant for head sizes 64, 72, 80, 96 and 128 (fwd_pp.hip).
bool fwd_pp_supports(const FwdArgs& a, int dtype);
hipError_t launch_fwd_pp(const FwdArgs& a, int dtype, bool causal, hipStream_t stream);
// Key split for a causal launch too small to fill the device with 256-query workgroups:
// returns the chunk size in tiles (0 = no split) and the fp32 workspace bytes it needs.
int fwd_pp_key_split(const FwdArgs& a, int dtype, int n_cu, size_t* ws_bytes);

// KV-cache writes and Q/K producers (producers.hip).
hipError_t launch_kv_append(void* cache, const void* src, const int* pos, int kv_dim,
                            long layer_off, int dtype, hipStream_t stream);
hipError_t launch_kv_scatter(const void* k_src, const void* v_src, void* k_pool, void* v_pool,
                             const int* slots, long src_row_stride, int n_rows, int kv_heads,
                             int head_size, int block_size, int head_major, int dtype,
                             hipStream_t stream);
hipError_t launch_kv_convert(void* contig, void* pool, const int* block_table,
                             long contig_row_stride, int n_tokens, int kv_heads, int head_size,
                             int block_size, int head_major, int to_paged, int dtype,
                             hipStream_t stream);
bool norm_rope_supports(int dtype, int head_size);
hipError_t launch_qk_norm_rope(void* q, const void* k, const void* v, const void* q_weight,
                               const void* k_weight, const float* sin_cache,
                               const float* cos_cache, void* k_cache, void* v_cache,
                               long cache_tok_stride, const int* pos_ptr, int start_pos,
                               int seq_len, int Hq, int Hkv, int head_size, float eps, int dtype,
                               hipStream_t stream);
hipError_t launch_rope_cache(float* sin_cache, float* cos_cache, int head_size, int max_pos,
                             float theta, hipStream_t stream);
hipError_t launch_vision_qkv(const void* qkv, const void* cos_t, const void* sin_t, void* q,
                             void* k, void* v, int N, int H, int d, int dtype, hipStream_t stream);

// Attention output projection (outproj.hip): out[b, k] = scale * sum_m in[b, m] * w[k, m].
// Returns 0, -1 (library error), -2 (dtype) or -3 (the stream is capturing and the device's
// handle was not prepared).
int output_projection(const void* input, const void* weight, void* output, int batch, int in_dim,
                      int out_dim, float scale, int dtype, hipStream_t stream, bool capturing);
// Creates the current device's rocBLAS handle and its workspace if missing (0 on success).
int output_projection_prepare();

}  // namespace orin
