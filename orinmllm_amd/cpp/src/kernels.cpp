// kernel:: functions over the C ABI.  Each forwards its arguments unchanged (tensors
// become device pointers, the config its stream, the element type a dtype code) and
// records the C ABI's status for last_status().
#include "orin/kernels.h"

#include <string>

#include "orin_attn.h"

namespace orin {
namespace kernel {

namespace {

thread_local base::Status g_last;

int dtype_code(base::DataType t) {
  switch (t) {
    case base::DataType::kDataTypeFp32: return ORIN_DTYPE_FP32;
    case base::DataType::kDataTypeFp16: return ORIN_DTYPE_FP16;
    case base::DataType::kDataTypeBf16: return ORIN_DTYPE_BF16;
    default: return 0;  // rejected by the C ABI as unsupported
  }
}

void* stream_of(const CudaConfig* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

void record(const char* fn, int st) {
  if (st == ORIN_OK) {
    g_last = base::error::Success();
    return;
  }
  std::string msg = std::string(fn) + ": " + orin_attn_status_string(st);
  if (st == ORIN_ERR_LAUNCH) msg += std::string(" (") + orin_attn_last_hip_error() + ")";
  g_last = st == ORIN_ERR_INVALID_ARG ? base::error::InvalidArgument(msg)
                                      : base::error::InternalError(msg);
}

// Element type shared by all tensors of a call (0 if they disagree).
int common_dtype(std::initializer_list<const tensor::Tensor*> ts) {
  int code = -1;
  for (const tensor::Tensor* t : ts) {
    const int c = dtype_code(t->data_type());
    if (code == -1) code = c;
    else if (c != code) return 0;
  }
  return code < 0 ? 0 : code;
}

}  // namespace

const base::Status& last_status() { return g_last; }

MHAKernel get_mha_kernel(base::DeviceType device_type) {
  // The CPU attention is the test oracle (oracle/oracle.c), not a product path.
  return device_type == base::DeviceType::kDeviceCUDA ? &mha_kernel_cu : nullptr;
}

void mha_kernel_cu(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                   int32_t kv_dim, int32_t kv_mul, int32_t head_size, const tensor::Tensor& mha_out,
                   const tensor::Tensor& query_tensor, const tensor::Tensor& score_tensor,
                   const tensor::Tensor& key_cache_tensor,
                   const tensor::Tensor& value_cache_tensor, base::DeviceType,
                   CudaConfig* config) {
  record("mha_kernel_cu",
         orin_mha_kernel(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                         mha_out.ptr<float>(), query_tensor.ptr<const float>(),
                         score_tensor.ptr<float>(), key_cache_tensor.ptr<const float>(),
                         value_cache_tensor.ptr<const float>(), stream_of(config)));
}

void mha_kernel_cu_gpu_pos(const int32_t* pos_ptr, int32_t head_num, int32_t layer_index,
                           int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                           const tensor::Tensor& mha_out, const tensor::Tensor& query_tensor,
                           const tensor::Tensor& score_tensor,
                           const tensor::Tensor& key_cache_tensor,
                           const tensor::Tensor& value_cache_tensor, base::DeviceType,
                           CudaConfig* config) {
  record("mha_kernel_cu_gpu_pos",
         orin_mha_kernel_gpu_pos(pos_ptr, head_num, layer_index, seq_len, kv_dim, kv_mul,
                                 head_size, mha_out.ptr<float>(), query_tensor.ptr<const float>(),
                                 score_tensor.ptr<float>(), key_cache_tensor.ptr<const float>(),
                                 value_cache_tensor.ptr<const float>(), stream_of(config)));
}

void batched_mha_kernel_cu(int32_t start_pos, int32_t seq_len, int32_t head_num,
                           int32_t layer_index, int32_t max_seq_len, int32_t dim, int32_t kv_dim,
                           int32_t kv_mul, int32_t head_size, const tensor::Tensor& mha_out,
                           const tensor::Tensor& query_tensor, const tensor::Tensor& score_tensor,
                           const tensor::Tensor& key_cache_tensor,
                           const tensor::Tensor& value_cache_tensor, base::DeviceType,
                           CudaConfig* config) {
  record("batched_mha_kernel_cu",
         orin_batched_mha(start_pos, seq_len, head_num, layer_index, max_seq_len, dim, kv_dim,
                          kv_mul, head_size, mha_out.ptr<float>(), query_tensor.ptr<const float>(),
                          score_tensor.ptr<float>(), key_cache_tensor.ptr<const float>(),
                          value_cache_tensor.ptr<const float>(), stream_of(config)));
}

namespace {
void prefill(const char* fn, int32_t start_pos, int32_t seq_len, int32_t head_num,
             int32_t kv_head_num, int32_t head_size, int32_t kv_mul, int32_t layer_index,
             int32_t max_seq_len, int32_t kv_dim, const tensor::Tensor& query,
             const tensor::Tensor& output, const tensor::Tensor& key_cache,
             const tensor::Tensor& value_cache, CudaConfig* config) {
  record(fn, orin_flash_attention_prefill(
                 start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index,
                 max_seq_len, kv_dim, query.raw_ptr(), output.raw_ptr(), key_cache.raw_ptr(),
                 value_cache.raw_ptr(), common_dtype({&query, &output, &key_cache, &value_cache}),
                 stream_of(config)));
}
void decode(const char* fn, int32_t pos, const int32_t* pos_ptr, int32_t head_num,
            int32_t kv_head_num, int32_t head_size, int32_t kv_mul, int32_t layer_index,
            int32_t max_seq_len, int32_t kv_dim, const tensor::Tensor& query,
            const tensor::Tensor& output, const tensor::Tensor& key_cache,
            const tensor::Tensor& value_cache, CudaConfig* config) {
  const int dt = common_dtype({&query, &output, &key_cache, &value_cache});
  const int st =
      pos_ptr ? orin_flash_attention_decode_gpu_pos(
                    pos_ptr, head_num, kv_head_num, head_size, kv_mul, layer_index, max_seq_len,
                    kv_dim, query.raw_ptr(), output.raw_ptr(), key_cache.raw_ptr(),
                    value_cache.raw_ptr(), dt, stream_of(config))
              : orin_flash_attention_decode(pos, head_num, kv_head_num, head_size, kv_mul,
                                            layer_index, max_seq_len, kv_dim, query.raw_ptr(),
                                            output.raw_ptr(), key_cache.raw_ptr(),
                                            value_cache.raw_ptr(), dt, stream_of(config));
  record(fn, st);
}
}  // namespace

#define ORIN_FA_PREFILL_FWD                                                                \
  start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index, max_seq_len, \
      kv_dim, query, output, key_cache, value_cache, config
#define ORIN_FA_DECODE_FWD                                                                 \
  head_num, kv_head_num, head_size, kv_mul, layer_index, max_seq_len, kv_dim, query,      \
      output, key_cache, value_cache, config

void flash_attention_prefill_cu(ORIN_FA_PREFILL_ARGS) {
  prefill("flash_attention_prefill_cu", ORIN_FA_PREFILL_FWD);
}
void flash_attention_prefill_fp16_cu(ORIN_FA_PREFILL_ARGS) {
  prefill("flash_attention_prefill_fp16_cu", ORIN_FA_PREFILL_FWD);
}
void flash_attention2_prefill_cu(ORIN_FA_PREFILL_ARGS) {
  prefill("flash_attention2_prefill_cu", ORIN_FA_PREFILL_FWD);
}
void flash_attention2_prefill_fp16_cu(ORIN_FA_PREFILL_ARGS) {
  prefill("flash_attention2_prefill_fp16_cu", ORIN_FA_PREFILL_FWD);
}
void flash_attention_decode_cu(ORIN_FA_DECODE_ARGS) {
  decode("flash_attention_decode_cu", pos, nullptr, ORIN_FA_DECODE_FWD);
}
void flash_attention_decode_fp16_cu(ORIN_FA_DECODE_ARGS) {
  decode("flash_attention_decode_fp16_cu", pos, nullptr, ORIN_FA_DECODE_FWD);
}
void flash_attention2_decode_cu(ORIN_FA_DECODE_ARGS) {
  decode("flash_attention2_decode_cu", pos, nullptr, ORIN_FA_DECODE_FWD);
}
void flash_attention2_decode_fp16_cu(ORIN_FA_DECODE_ARGS) {
  decode("flash_attention2_decode_fp16_cu", pos, nullptr, ORIN_FA_DECODE_FWD);
}
void flash_attention_decode_fp16_gpu_pos_cu(ORIN_FA_DECODE_GPU_POS_ARGS) {
  decode("flash_attention_decode_fp16_gpu_pos_cu", 0, pos_ptr, ORIN_FA_DECODE_FWD);
}
void flash_attention2_decode_fp16_gpu_pos_cu(ORIN_FA_DECODE_GPU_POS_ARGS) {
  decode("flash_attention2_decode_fp16_gpu_pos_cu", 0, pos_ptr, ORIN_FA_DECODE_FWD);
}

void vision_attention_pretransposed_cu(const tensor::Tensor& q_trans,
                                       const tensor::Tensor& k_trans,
                                       const tensor::Tensor& v_trans, tensor::Tensor& output,
                                       tensor::Tensor& out_transposed, tensor::Tensor& scores,
                                       int num_tokens, int num_heads, int head_dim,
                                       float softmax_scale, const CudaConfig* config) {
  record("vision_attention_pretransposed_cu",
         orin_vision_attention_pretransposed(
             q_trans.raw_ptr(), k_trans.raw_ptr(), v_trans.raw_ptr(), output.raw_ptr(),
             out_transposed.raw_ptr(), scores.raw_ptr(), num_tokens, num_heads, head_dim,
             softmax_scale, common_dtype({&q_trans, &k_trans, &v_trans, &output}),
             stream_of(config)));
}

void batched_matmul_kernel_cu_pure_fp16(const tensor::Tensor& input,
                                         const tensor::Tensor& weight,
                                         const tensor::Tensor& output, int32_t batch_size,
                                         float scale, const CudaConfig* config) {
  if (weight.dims_size() != 2) {
    record("batched_matmul_kernel_cu_pure_fp16", ORIN_ERR_INVALID_ARG);
    return;
  }
  record("batched_matmul_kernel_cu_pure_fp16",
         orin_batched_matmul(input.raw_ptr(), weight.raw_ptr(), output.raw_ptr(), batch_size,
                             weight.get_dim(1), weight.get_dim(0), scale,
                             common_dtype({&input, &weight, &output}), stream_of(config)));
}

void fused_split_rope_transpose_cu(const tensor::Tensor& qkv, const tensor::Tensor& cos_cache,
                                   const tensor::Tensor& sin_cache, tensor::Tensor& q_trans,
                                   tensor::Tensor& k_trans, tensor::Tensor& v_trans,
                                   int num_tokens, int num_heads, int head_dim,
                                   hipStream_t stream) {
  record("fused_split_rope_transpose_cu",
         orin_vision_split_rope_transpose(
             qkv.raw_ptr(), cos_cache.raw_ptr(), sin_cache.raw_ptr(), q_trans.raw_ptr(),
             k_trans.raw_ptr(), v_trans.raw_ptr(), num_tokens, num_heads, head_dim,
             common_dtype({&qkv, &cos_cache, &sin_cache, &q_trans, &k_trans, &v_trans}),
             static_cast<void*>(stream)));
}

void copy_to_kv_cache_kernel(float* kv_cache, const float* src, const int32_t* pos,
                             int32_t kv_dim, int32_t layer_idx, int32_t seq_len,
                             hipStream_t stream) {
  record("copy_to_kv_cache_kernel",
         orin_copy_to_kv_cache(kv_cache, src, pos, kv_dim, layer_idx, seq_len, ORIN_DTYPE_FP32,
                               static_cast<void*>(stream)));
}

void copy_to_kv_cache_kernel_fp16(__half* kv_cache, const __half* src, const int32_t* pos,
                                  int32_t kv_dim, int32_t layer_idx, int32_t seq_len,
                                  hipStream_t stream) {
  record("copy_to_kv_cache_kernel_fp16",
         orin_copy_to_kv_cache(kv_cache, src, pos, kv_dim, layer_idx, seq_len, ORIN_DTYPE_FP16,
                               static_cast<void*>(stream)));
}

// rope_kernel.cu:86-98 uses theta = 1e6 (Qwen3).
void sin_cos_cache_calc_cu(int head_size, int max_seq_len, const tensor::Tensor& sin_cache,
                           const tensor::Tensor& cos_cache, hipStream_t stream) {
  record("sin_cos_cache_calc_cu",
         orin_rope_sin_cos_cache(sin_cache.ptr<float>(), cos_cache.ptr<float>(), head_size,
                                 max_seq_len, 1e6f, static_cast<void*>(stream)));
}

}  // namespace kernel
}  // namespace orin
