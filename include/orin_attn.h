/*
 * orin_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Each entry point replaces one function of OrinMLLM's attention path
 * (paths relative to the OrinMLLM source tree) with the same argument meaning,
 * flattened to plain pointers: tensor::Tensor arguments become device pointers,
 * CudaConfig* becomes the stream the kernels are queued on (a hipStream_t,
 * NULL = the default stream), and the element type is an explicit code.
 *
 * Conventions shared by every entry point:
 *  - dim = head_num*head_size, kv_dim = kv_head_num*head_size; query head h reads
 *    kv head h / kv_mul (kuiper/source/op/kernels/cpu/mha_kernel.cpp:29).
 *  - KV caches are kuiper's [layers, max_seq_len, kv_dim]; the layer is selected
 *    with layer_index * max_seq_len * kv_dim, as the reference wrappers do.
 *  - softmax scale is 1/sqrt(head_size) unless an entry point takes `scale`
 *    (0 there also means 1/sqrt(head_size)).
 *  - Everything is asynchronous on `stream`; nothing synchronises the host.
 *  - The return value is ORIN_OK or a negative ORIN_ERR_* code.  Argument errors
 *    are detected before anything is queued.  The reference layers return
 *    base::error::InvalidArgument for non-positive sizes
 *    (kuiper/source/op/flash_attention.cpp:32-37) and do not check launches; the
 *    adapter maps ORIN_ERR_INVALID_ARG to InvalidArgument and the rest to
 *    InternalError.
 *  - Output may alias query (prefill is called with output == query by
 *    kuiper/source/model/qwen3_vl.cpp:2871-2878): every workgroup reads its own
 *    query rows before it writes the same rows.
 */
#ifndef ORIN_ATTN_H
#define ORIN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types: values follow base::DataType (kuiper/include/base/base.h:58-64),
 * which has fp32 = 1 and fp16 = 4; bf16 is new. */
#define ORIN_DTYPE_FP32 1
#define ORIN_DTYPE_FP16 4
#define ORIN_DTYPE_BF16 5

#define ORIN_OK 0
#define ORIN_ERR_INVALID_ARG (-1) /* non-positive size, null pointer, inconsistent heads */
#define ORIN_ERR_UNSUPPORTED (-2) /* dtype / head_size / block_size this build has no kernel for */
#define ORIN_ERR_WORKSPACE (-3)   /* workspace missing or too small */
#define ORIN_ERR_LAUNCH (-4)      /* the HIP runtime rejected a launch or allocation */

#define ORIN_ATTN_ABI_VERSION 1

int orin_attn_abi_version(void);
const char* orin_attn_status_string(int status);
/* Text of the last HIP error seen by this library in this thread ("" if none). */
const char* orin_attn_last_hip_error(void);

/* ------------------------------------------------------------------ decode (fp32 MHA) */

/*
 * kernel::mha_kernel_cu (kuiper/source/op/kernels/cuda/mha_kernel.cuh:4-8; the
 * MHAKernel typedef of kernels_interface.h:24-30, obtained from get_mha_kernel,
 * kernels_interfaces.cpp:63-72).  fp32.  Query position `pos` attends to cache rows
 * 0..pos of layer `layer_index`.  `seq_len` is the cache capacity (max_seq_len).
 * `score` is the caller's [head_num, seq_len] fp32 scratch (kScoreStorage): it is
 * used as split-KV workspace and its contents afterwards are unspecified.
 */
int orin_mha_kernel(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                    int32_t kv_dim, int32_t kv_mul, int32_t head_size, float* mha_out,
                    const float* query, float* score, const float* key_cache,
                    const float* value_cache, void* stream);

/*
 * kernel::mha_kernel_cu_gpu_pos (mha_kernel.cuh:13-19): as orin_mha_kernel with the
 * position read from device memory, so the launch can be captured into a HIP graph
 * and replayed while *pos_ptr changes.  The launch shape depends only on seq_len.
 */
int orin_mha_kernel_gpu_pos(const int32_t* pos_ptr, int32_t head_num, int32_t layer_index,
                            int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                            float* mha_out, const float* query, float* score,
                            const float* key_cache, const float* value_cache, void* stream);

/*
 * kernel::batched_mha_kernel_cu (mha_kernel.cuh:21-26): fp32 causal prefill of
 * seq_len query rows [seq_len, dim] at positions start_pos..start_pos+seq_len-1;
 * row i attends cache rows 0..start_pos+i.  `score` ([seq_len, head_num,
 * max_seq_len] in the reference) is not needed and may be NULL.
 */
int orin_batched_mha(int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t layer_index,
                     int32_t max_seq_len, int32_t dim, int32_t kv_dim, int32_t kv_mul,
                     int32_t head_size, float* mha_out, const float* query, float* score,
                     const float* key_cache, const float* value_cache, void* stream);

/* ------------------------------------------------------------------ flash attention */

/*
 * kernel::flash_attention_prefill_cu / flash_attention_prefill_fp16_cu /
 * flash_attention2_prefill_cu / flash_attention2_prefill_fp16_cu
 * (kuiper/source/op/kernels/cuda/flash_attention_kernel.cuh:27-80, 143-181).
 * Causal GQA prefill: query/output [seq_len, dim], caches [layers, max_seq_len, kv_dim];
 * row i attends 0..start_pos+i (flash_attention_kernel.cu:575-578).  dtype selects the
 * reference's fp32 or fp16 variant; bf16 is new.  fp16/bf16 run on MFMA.  A 16-bit launch
 * with fewer 256-query blocks than the device has CUs splits the keys of each block and
 * keeps the partials in the stream's library-owned workspace (see below).
 * bf16 range: the softmax weights and the weighted sum with V run in fp16 (V is converted
 * to fp16 on chip), so bf16 V must satisfy |v| <= 65504; a larger value turns non-finite
 * the outputs of every row that attends to it (and possibly of other rows whose 64-key
 * tile holds it).  V elements below 2^-14 in magnitude keep
 * fp16's subnormal spacing (absolute error at most 2^-25 each, hence in the output).  The
 * decode entry points use bf16 V as stored and have neither limit.
 */
int orin_flash_attention_prefill(int32_t start_pos, int32_t seq_len, int32_t head_num,
                                 int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                                 int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                                 const void* query, void* output, const void* key_cache,
                                 const void* value_cache, int32_t dtype, void* stream);

/*
 * The Qwen3 prefill producer fused into the attention (no single reference function: it
 * replaces, for the query, kernel::rmsnorm_kernel_cu_dim on the q heads,
 * rmsnorm_kernel.cu:483-545, and kernel::batched_rope_kernel_cu, rope_kernel.cu:377-427,
 * as called by kuiper/source/model/qwen3.cpp:1195-1215, and then
 * orin_flash_attention_prefill).  `query` holds the raw rows [seq_len, dim]; each query
 * head row i is RMS-normalised with q_norm_weight (NULL: no normalisation, the Qwen2 /
 * Llama producer) and rotated with sin_cache/cos_cache [max_seq_len, head_size] (entry
 * [p][2j] for the pair (j, j + head_size/2)) at position start_pos + i while the prefill
 * loads it, with the same arithmetic as orin_qk_norm_rope: the output equals
 * orin_qk_norm_rope on the query followed by orin_flash_attention_prefill, bit for bit, and
 * the query buffer is left unchanged.  Keys must already be in the cache (orin_qk_norm_rope
 * with query = NULL writes them).  fp16 / bf16, head_size 64 or 128; output must not
 * alias query.  bf16 V: the range limits of orin_flash_attention_prefill.
 */
int orin_flash_attention_prefill_qk_norm_rope(
    int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t kv_head_num, int32_t head_size,
    int32_t kv_mul, int32_t layer_index, int32_t max_seq_len, int32_t kv_dim, const void* query,
    void* output, const void* key_cache, const void* value_cache, const void* q_norm_weight,
    const float* sin_cache, const float* cos_cache, float eps, int32_t dtype, void* stream);

/*
 * kernel::flash_attention_decode_cu / flash_attention_decode_fp16_cu /
 * flash_attention2_decode_cu / flash_attention2_decode_fp16_cu
 * (flash_attention_kernel.cuh:50-63, 84-97, 186-216).  One query row [dim] at
 * position pos over cache rows 0..pos.  Split-KV partials go to the stream's
 * library-owned workspace (see orin_attn_workspace_reserve_stream).  bf16 caches: the
 * weights are split into bf16 hi + lo parts and V is used as stored (bf16's full range).
 */
int orin_flash_attention_decode(int32_t pos, int32_t head_num, int32_t kv_head_num,
                                int32_t head_size, int32_t kv_mul, int32_t layer_index,
                                int32_t max_seq_len, int32_t kv_dim, const void* query,
                                void* output, const void* key_cache, const void* value_cache,
                                int32_t dtype, void* stream);

/*
 * kernel::flash_attention_decode_fp16_gpu_pos_cu / flash_attention2_decode_fp16_gpu_pos_cu
 * (flash_attention_kernel.cuh:103-117, 222-234): the decode above with the position
 * read from device memory (HIP-graph capturable).  The launch shape and workspace
 * depend only on max_seq_len; reserve the capture stream's workspace before capturing.
 */
int orin_flash_attention_decode_gpu_pos(const int32_t* pos_ptr, int32_t head_num,
                                        int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                                        int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                                        const void* query, void* output, const void* key_cache,
                                        const void* value_cache, int32_t dtype, void* stream);

/*
 * No counterpart in the reference.  For callers that cannot allocate (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc): the gpu-pos flash
 * decode above, with its split partials in a fixed device array of
 * orin_flash_attention_decode_noalloc_max_bytes() bytes (4 MiB) that each GPU holds
 * until the process ends, instead of a library-owned buffer.  It allocates nothing and
 * needs no reserve; the launch and the result equal orin_flash_attention_decode_gpu_pos
 * bit for bit.  A launch whose partials would exceed the array (head_num * splits *
 * (head_size + 2) * 4 bytes; at 32 heads, d 128: a cache of more than 64512 rows) returns
 * ORIN_ERR_WORKSPACE and queues nothing.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time (other streams, concurrent graph replays) race.  Each call
 * writes every partial it reads, so the array needs no clearing between calls.
 */
int orin_flash_attention_decode_gpu_pos_noalloc(const int32_t* pos_ptr, int32_t head_num,
                                                int32_t kv_head_num, int32_t head_size,
                                                int32_t kv_mul, int32_t layer_index,
                                                int32_t max_seq_len, int32_t kv_dim,
                                                const void* query, void* output,
                                                const void* key_cache, const void* value_cache,
                                                int32_t dtype, void* stream);
size_t orin_flash_attention_decode_noalloc_max_bytes(void);

/*
 * Library-owned workspaces (no reference counterpart: kuiper's flash decode and prefill
 * take no workspace argument).  The flash decode entry points and the key split of a
 * small causal prefill keep their partials in buffers owned by this library, one per
 * (device, stream, use): calls on different streams never share bytes, so the entry
 * points are reentrant across streams; calls on one stream are ordered by it.
 *  - A buffer grows on demand (hipMalloc, no synchronisation).  The buffer it replaces is
 *    kept allocated, because a captured graph may still use its address, until
 *    orin_attn_workspace_release.
 *  - While `stream` is being captured nothing is allocated: a call whose buffer is missing
 *    or too small returns ORIN_ERR_WORKSPACE.  Reserve before capturing.
 *  - A graph uses the buffer of the stream it was captured on: do not replay it while
 *    other work that uses that stream's buffer runs.
 *
 * orin_flash_attention_decode_workspace_size: decode bytes for a cache of max_seq_len rows
 * (any kv_head_num).  orin_flash_attention_prefill_workspace_size: key-split bytes of one
 * causal prefill launch (0 when it does not split).  orin_attn_workspace_reserve_stream
 * allocates both on the current device for `stream` now.  orin_attn_workspace_reserve
 * reserves decode bytes for the NULL stream and makes every decode buffer created later on
 * this device at least that large.  orin_attn_workspace_reserve_stream also prepares the
 * device's output-projection handle (orin_batched_matmul), so that it can be captured.
 *  - Buffers are keyed by (device, stream handle) and live until released: a stream that is
 *    destroyed keeps its buffers (and a new stream that receives the same handle value
 *    reuses them).  orin_attn_workspace_release_stream(stream) synchronises `stream` and
 *    frees its buffers on the current device; orin_attn_workspace_release synchronises the
 *    device and frees every library-owned buffer of it.  Call either only when no captured
 *    graph that used those buffers will be replayed; both return ORIN_ERR_WORKSPACE, and
 *    free nothing, while one of the affected streams is being captured.
 *  - Allocations are made with the calling thread in relaxed capture mode, so they do not
 *    invalidate a capture that another thread runs in global mode.
 */
size_t orin_flash_attention_decode_workspace_size(int32_t head_num, int32_t head_size,
                                                  int32_t max_seq_len);
size_t orin_flash_attention_prefill_workspace_size(int32_t start_pos, int32_t seq_len,
                                                   int32_t head_num, int32_t kv_head_num,
                                                   int32_t head_size, int32_t dtype);
int orin_attn_workspace_reserve(size_t bytes);
int orin_attn_workspace_reserve_stream(size_t decode_bytes, size_t prefill_bytes, void* stream);
int orin_attn_workspace_release(void);
int orin_attn_workspace_release_stream(void* stream);

/* ------------------------------------------------------------------ batched decode */

/*
 * Batched decode over per-sequence contiguous caches.  No reference function: the
 * reference decodes one sequence (kuiper/source/model/qwen_base.cpp:675-781); this is
 * that decode applied to `batch` rows.  query/out [batch, head_num*head_size];
 * sequence b's token t, kv head g lives at
 *   cache + b*cache_batch_stride + t*cache_tok_stride + g*head_size   (elements).
 * context_lens (device, [batch]) gives each row's KV length; max_context_len bounds
 * them (it sets the launch shape).  A row whose length exceeds max_context_len (the host
 * cannot see device lengths) gets NaN outputs instead of attention over a truncated
 * prefix; the same holds for *pos_ptr >= max_seq_len in the gpu-pos entry points.
 * split_tokens: tokens per split (multiple of 64, else ORIN_ERR_INVALID_ARG), 0 =
 * automatic: whole rows (one split per row, no workspace) when batch * kv_head_num is at
 * least the device's CU count, else splits sized from max_context_len alone
 * (orin_attn_decode_split_tokens_for_total uses the batch's total length too).  Launches
 * of whole rows with batch * kv_head_num >= CUs run the matrix-core kernel where it
 * supports the shape (16-bit caches, head_size 64 or 128, at most 16 query heads per kv
 * head); the rest run the dot-product kernel.  Workspace: orin_attn_decode_workspace_size
 * bytes (may be NULL when that is 0).  bf16 caches: V is used as stored (the weights are
 * split into bf16 hi + lo parts), so bf16's full range is kept.
 */
size_t orin_attn_decode_workspace_size(int32_t batch, int32_t head_num, int32_t kv_head_num,
                                       int32_t head_size, int32_t max_context_len,
                                       int32_t split_tokens);
int32_t orin_attn_decode_split_tokens(int32_t batch, int32_t head_num, int32_t kv_head_num,
                                      int32_t max_context_len, int32_t split_tokens);
/*
 * Split size for a batched decode whose total KV length sum_context_len (the sum of the
 * rows' context lengths) the caller knows on the host -- a serving loop keeps it; no
 * reference counterpart.  A batch whose (row, kv head) units reach the CU count gets whole
 * rows, as the automatic choice does.  A smaller batch whose rows are all close to
 * max_context_len (sum >= 0.9 * batch * max_context_len) gets a few long splits per row
 * (one round of the workgroups the device holds at once), which streams faster than the
 * automatic choice; otherwise the automatic choice.  Pass the result as split_tokens (and
 * to orin_attn_decode_workspace_size).  Returns a multiple of 64, or 0 for invalid
 * arguments.
 */
int32_t orin_attn_decode_split_tokens_for_total(int32_t batch, int32_t head_num,
                                                int32_t kv_head_num, int32_t max_context_len,
                                                int64_t sum_context_len);
int orin_attn_decode(const void* query, const void* key_cache, const void* value_cache,
                     void* out, int32_t batch, int32_t head_num, int32_t kv_head_num,
                     int32_t head_size, int64_t cache_batch_stride, int64_t cache_tok_stride,
                     const int32_t* context_lens, int32_t max_context_len, int32_t dtype,
                     float scale, int32_t split_tokens, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Paged batched decode.  No reference function (the reference has no block-table
 * KV cache).  Block b of a pool holds block_size consecutive tokens of one sequence,
 * for all kv heads, in one of two layouts:
 *   ORIN_KV_LAYOUT_TOKEN_MAJOR  [num_blocks, block_size, kv_head_num, head_size]
 *                               (each token row is kuiper's kv_dim layout)
 *   ORIN_KV_LAYOUT_HEAD_MAJOR   [num_blocks, kv_head_num, block_size, head_size]
 *                               (each (block, kv head) is one contiguous run)
 * Sequence s's token t lives in pool block block_tables[s*max_blocks_per_seq +
 * t/block_size], row t % block_size.  block_size must be a power of two >= 8
 * (ORIN_ERR_UNSUPPORTED otherwise).  split_tokens must be a multiple of 64.  For equal
 * split_tokens the result is bit-identical to orin_attn_decode on a contiguous copy
 * of the same KV, in either layout.
 */
#define ORIN_KV_LAYOUT_TOKEN_MAJOR 0
#define ORIN_KV_LAYOUT_HEAD_MAJOR 1
int orin_attn_decode_paged(const void* query, const void* k_pool, const void* v_pool, void* out,
                           int32_t batch, int32_t head_num, int32_t kv_head_num,
                           int32_t head_size, const int32_t* block_tables,
                           int32_t max_blocks_per_seq, int32_t block_size, int32_t kv_layout,
                           const int32_t* context_lens, int32_t max_context_len, int32_t dtype,
                           float scale, int32_t split_tokens, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ vision */

/*
 * kernel::vision_attention_pretransposed_cu
 * (kuiper/source/op/kernels/cuda/vision_encoder_kernel.cuh:159-170): bidirectional
 * attention of num_tokens tokens over q/k/v [num_heads, num_tokens, head_dim] into
 * output [num_tokens, num_heads*head_dim].  The reference's out_transposed and scores
 * workspaces are not needed and may be NULL.  fp16 / bf16 (MFMA) or fp32.  bf16 V: the
 * range limits of orin_flash_attention_prefill (|v| <= 65504; subnormal spacing below
 * 2^-14).
 */
int orin_vision_attention_pretransposed(const void* q, const void* k, const void* v,
                                        void* output, void* out_transposed, void* scores,
                                        int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                        float softmax_scale, int32_t dtype, void* stream);

/*
 * Varlen form: tokens are packed segments (images) given by cu_seqlens (device,
 * n_seqs+1 entries, cu_seqlens[0] = 0, cu_seqlens[n_seqs] = num_tokens); every token
 * attends to all tokens of its own segment.  No reference function (the reference
 * builds cu_seqlens, kuiper/source/model/qwen3_vl.cpp:1561-1568, but attends over one
 * segment).  max_seqlen bounds the segment lengths.
 */
int orin_vision_attention_varlen(const void* q, const void* k, const void* v, void* output,
                                 const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                                 int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                 float softmax_scale, int32_t dtype, void* stream);

/* ------------------------------------------------------------------ output projection */

/*
 * kernel::batched_matmul_kernel_cu / batched_matmul_kernel_cu_pure_fp16
 * (kuiper/source/op/kernels/cuda/matmul_kernel.cuh:15-41), as the prefill runs the wo
 * projection on the attention output (kuiper/source/model/qwen_base.cpp:464-474):
 *   output[b, k] = scale * sum_m input[b, m] * weight[k, m]
 * input [batch_size, in_dim] (the attention output [tokens, head_num*head_size], as the
 * attention entry points store it), weight [out_dim, in_dim], output [batch_size, out_dim],
 * all row-major in `dtype` (fp32 / fp16 / bf16); fp32 accumulation.  A plain GEMM, run by
 * rocBLAS on `stream`.  The device's rocBLAS handle and its workspace are created by
 * orin_attn_workspace_reserve_stream or by the first call outside graph capture; a call on
 * a capturing stream of a device without them returns ORIN_ERR_WORKSPACE.
 */
int orin_batched_matmul(const void* input, const void* weight, void* output, int32_t batch_size,
                        int32_t in_dim, int32_t out_dim, float scale, int32_t dtype,
                        void* stream);

/* ------------------------------------------------------------------ KV-cache writes */

/*
 * kernel::copy_to_kv_cache_kernel / copy_to_kv_cache_kernel_fp16
 * (kuiper/source/op/kernels/cuda/kv_cache_kernel.cuh:24-33, kv_cache_kernel.cu:43-57):
 * kv_cache[layer_idx][*pos][0..kv_dim) = src[0..kv_dim) for a kuiper cache
 * [layers, seq_len, kv_dim].  The position is read from device memory when the kernel
 * runs, so a captured graph can be replayed with a new position.  fp32 / fp16 / bf16.
 */
int orin_copy_to_kv_cache(void* kv_cache, const void* src, const int32_t* pos, int32_t kv_dim,
                          int32_t layer_idx, int32_t seq_len, int32_t dtype, void* stream);

/*
 * Paged-cache write (no reference function: the reference's contiguous prefill copy is
 * the cudaMemcpyAsync pair of kuiper/source/model/qwen3.cpp:1220-1241).  Row r of k_src
 * and v_src ([n_rows, kv_head_num*head_size], row stride src_row_stride elements) is
 * stored at pool slot slot_mapping[r] (device int32: block * block_size + offset within
 * the block; a negative slot skips the row).  Pools use the layouts of
 * orin_attn_decode_paged (kv_layout).  head_size*sizeof(element) and src_row_stride
 * must be multiples of 16 bytes.
 */
int orin_kv_cache_write_paged(const void* k_src, const void* v_src, int64_t src_row_stride,
                              void* k_pool, void* v_pool, const int32_t* slot_mapping,
                              int32_t n_rows, int32_t kv_head_num, int32_t head_size,
                              int32_t block_size, int32_t kv_layout, int32_t dtype,
                              void* stream);

/*
 * Copy tokens [0, n_tokens) of one sequence between a contiguous cache
 * [n_tokens, kv_head_num*head_size] (row stride contig_row_stride elements, e.g. one
 * kuiper layer) and a paged pool through the sequence's block table (device int32).
 * direction ORIN_KV_TO_PAGED or ORIN_KV_TO_CONTIGUOUS.  No reference function.
 */
#define ORIN_KV_TO_PAGED 0
#define ORIN_KV_TO_CONTIGUOUS 1
int orin_kv_cache_convert(void* contig, int64_t contig_row_stride, void* pool,
                          const int32_t* block_table, int32_t n_tokens, int32_t kv_head_num,
                          int32_t head_size, int32_t block_size, int32_t kv_layout,
                          int32_t direction, int32_t dtype, void* stream);

/* ------------------------------------------------------------------ Q/K producers */

/*
 * kernel::sin_cos_cache_calc_cu (kuiper/source/op/kernels/cuda/rope_kernel.cu:86-98,
 * 153-166): sin_cache/cos_cache [max_seq_len, head_size] fp32 with entry [p][i] =
 * sin/cos(p * theta^(-i/head_size)) (the reference uses theta = 1e6).
 */
int orin_rope_sin_cos_cache(float* sin_cache, float* cos_cache, int32_t head_size,
                            int32_t max_seq_len, float theta, void* stream);

/*
 * The Qwen3 attention producer in one pass (replaces kernel::rmsnorm_kernel_cu_dim on
 * the q and k heads, rmsnorm_kernel.cu:483-545, then kernel::batched_rope_kernel_cu /
 * rope_kernel_cu_gpu_pos, rope_kernel.cu:377-427, 464-509, then the two cache copies of
 * kuiper/source/model/qwen3.cpp:1195-1241).  For tokens t < seq_len at positions
 * p = start + t (start = *pos_ptr if pos_ptr is non-NULL, else start_pos):
 *   query[t, h] <- rope(rmsnorm(query[t, h]) * q_norm_weight)         (in place)
 *   key_cache[layer][p][g] <- rope(rmsnorm(key[t, g]) * k_norm_weight)
 *   value_cache[layer][p][g] <- value[t, g]
 * rmsnorm(x) = x / sqrt(mean(x^2) + eps) in fp32; rope rotates pairs (j, j + d/2) with
 * sin_cache/cos_cache[p][2j].  A NULL weight skips that normalisation (Qwen2 / Llama).
 * query may be NULL: only the key and value rows are produced (for
 * orin_flash_attention_prefill_qk_norm_rope, which applies the query part itself).
 * head_size 64, 128 or 256; fp32 / fp16 / bf16 (weights in the same type).
 */
int orin_qk_norm_rope(void* query, const void* key, const void* value,
                      const void* q_norm_weight, const void* k_norm_weight,
                      const float* sin_cache, const float* cos_cache, void* key_cache,
                      void* value_cache, int32_t layer_index, int32_t max_seq_len,
                      int32_t start_pos, const int32_t* pos_ptr, int32_t seq_len,
                      int32_t head_num, int32_t kv_head_num, int32_t head_size, float eps,
                      int32_t dtype, void* stream);

/*
 * kernel::fused_split_rope_transpose_cu
 * (kuiper/source/op/kernels/cuda/vision_encoder_kernel.cu:662-773): qkv
 * [num_tokens, 3*num_heads*head_dim] -> q_trans/k_trans/v_trans [num_heads, num_tokens,
 * head_dim], with the 2-D rotary x1' = x1*cos[j] - x2*sin[j],
 * x2' = x1*sin[j+d/2] + x2*cos[j+d/2] (cos/sin [num_tokens, head_dim], same type) on
 * q and k.  fp16 / bf16 / fp32.
 */
int orin_vision_split_rope_transpose(const void* qkv, const void* cos_cache,
                                     const void* sin_cache, void* q_trans, void* k_trans,
                                     void* v_trans, int32_t num_tokens, int32_t num_heads,
                                     int32_t head_dim, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ORIN_ATTN_H */
