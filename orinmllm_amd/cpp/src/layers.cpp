// op:: attention layers over orin/kernels.h (kuiper/source/op/flash_attention.cpp,
// mha.cpp, misc_layers.cpp, vision_layers.cpp behave the same way; here forward()
// also reports the kernel call's status).
#include "orin/layers.h"

namespace orin {
namespace op {

using base::AttentionType;
using base::DeviceType;
using base::Status;

namespace {
const char kUseParams[] = "Use forward(...) with parameters";

kernel::CudaConfig* cfg(const std::shared_ptr<kernel::CudaConfig>& c) { return c.get(); }

bool dims_ok(int32_t head_num, int32_t kv_head_num, int32_t head_size) {
  return head_num > 0 && kv_head_num > 0 && head_size > 0;
}
}  // namespace

// ------------------------------------------------------------ MultiHeadAttention
MultiHeadAttention::MultiHeadAttention(DeviceType device_type, int32_t layer_index, int32_t kv_mul,
                                       int32_t kv_dim, int32_t seq_len, int32_t head_num,
                                       int32_t head_size)
    : Layer(device_type, "MultiHead"),
      layer_index_(layer_index),
      kv_mul_(kv_mul),
      kv_dim_(kv_dim),
      seq_len_(seq_len),
      head_num_(head_num),
      head_size_(head_size) {
  reset_input_size(5);
  reset_output_size(1);
}

// mha.cpp:46-56: the four inputs and the output must be non-empty tensors on this
// layer's device.
Status MultiHeadAttention::check() const {
  for (int i = 0; i < 4; ++i) {
    const tensor::Tensor& t = get_input(i);
    if (t.is_empty() || t.device_type() != device_type_)
      return base::error::InvalidArgument("The input tensor " + std::to_string(i) +
                                          " error in the mha layer.");
  }
  const tensor::Tensor& o = get_output(0);
  if (o.is_empty() || o.device_type() != device_type_)
    return base::error::InvalidArgument("The output tensor error in the mha layer.");
  return base::error::Success();
}

Status MultiHeadAttention::forward() {
  Status st = check();
  if (!st) return st;
  kernel::MHAKernel k = kernel::get_mha_kernel(device_type_);
  if (!k) return base::error::FunctionNotImplement("no attention kernel for this device type");
  k(pos_, head_num_, layer_index_, seq_len_, kv_dim_, kv_mul_, head_size_, get_output(0),
    get_input(0), get_input(1), get_input(2), get_input(3), device_type_, cfg(cuda_config_));
  return launched();
}

// ------------------------------------------------------------ MHAGpuPosLayer / BatchedMHALayer
MHAGpuPosLayer::MHAGpuPosLayer(DeviceType device_type) : Layer(device_type, "MHAGpuPos") {}
Status MHAGpuPosLayer::forward() { return base::error::InvalidArgument(kUseParams); }
Status MHAGpuPosLayer::forward(const int32_t* pos_ptr, int32_t head_num, int32_t layer_idx,
                               int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                               tensor::Tensor& mha_output, const tensor::Tensor& query,
                               tensor::Tensor& score_storage, const tensor::Tensor& key_cache,
                               const tensor::Tensor& val_cache) {
  kernel::mha_kernel_cu_gpu_pos(pos_ptr, head_num, layer_idx, seq_len, kv_dim, kv_mul, head_size,
                                mha_output, query, score_storage, key_cache, val_cache,
                                device_type_, cfg(cuda_config_));
  return launched();
}

BatchedMHALayer::BatchedMHALayer(DeviceType device_type) : Layer(device_type, "BatchedMHA") {}
Status BatchedMHALayer::forward() { return base::error::InvalidArgument(kUseParams); }
Status BatchedMHALayer::forward(int32_t start_pos, int32_t seq_len, int32_t head_num,
                                int32_t layer_idx, int32_t max_seq_len, int32_t dim,
                                int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                                tensor::Tensor& mha_output, const tensor::Tensor& query,
                                tensor::Tensor& score_storage, const tensor::Tensor& key_cache,
                                const tensor::Tensor& val_cache) {
  kernel::batched_mha_kernel_cu(start_pos, seq_len, head_num, layer_idx, max_seq_len, dim,
                                kv_dim, kv_mul, head_size, mha_output, query, score_storage,
                                key_cache, val_cache, device_type_, cfg(cuda_config_));
  return launched();
}

// ------------------------------------------------------------ FlashAttentionDecodeLayer
FlashAttentionDecodeLayer::FlashAttentionDecodeLayer(DeviceType device_type)
    : Layer(device_type, "FlashAttentionDecode") {
  reset_input_size(5);
  reset_output_size(0);
}

FlashAttentionDecodeLayer::FlashAttentionDecodeLayer(DeviceType device_type, int32_t head_num,
                                                     int32_t kv_head_num, int32_t head_size,
                                                     int32_t kv_mul, int32_t seq_len,
                                                     int32_t kv_dim, bool use_fp16)
    : FlashAttentionDecodeLayer(device_type) {
  set_dims(head_num, kv_head_num, head_size, kv_mul, seq_len, kv_dim);
  use_fp16_ = use_fp16;
}

void FlashAttentionDecodeLayer::set_dims(int32_t head_num, int32_t kv_head_num,
                                         int32_t head_size, int32_t kv_mul, int32_t seq_len,
                                         int32_t kv_dim) {
  head_num_ = head_num;
  kv_head_num_ = kv_head_num;
  head_size_ = head_size;
  kv_mul_ = kv_mul;
  seq_len_ = seq_len;
  kv_dim_ = kv_dim;
}

Status FlashAttentionDecodeLayer::check() const {
  if (!dims_ok(head_num_, kv_head_num_, head_size_))
    return base::error::InvalidArgument("Invalid attention parameters");
  return base::error::Success();
}

// flash_attention.cpp:40-112: the fp16 / fp32 and Flash1 / Flash2 branches pick kernels
// that are one implementation here; kAttentionMHA in fp32 goes through get_mha_kernel.
Status FlashAttentionDecodeLayer::forward() {
  Status st = check();
  if (!st) return st;
  const tensor::Tensor& q = get_input(0);
  const tensor::Tensor& o = get_input(1);
  const tensor::Tensor& kc = get_input(2);
  const tensor::Tensor& vc = get_input(3);
  kernel::CudaConfig* c = cfg(cuda_config_);
  if (use_fp16_ && use_gpu_pos_) {
    kernel::flash_attention_decode_fp16_gpu_pos_cu(get_input(4).ptr<const int32_t>(), head_num_,
                                                   kv_head_num_, head_size_, kv_mul_,
                                                   layer_index_, seq_len_, kv_dim_, q, o, kc, vc,
                                                   c);
  } else if (use_fp16_ || attention_type_ != AttentionType::kAttentionMHA) {
    kernel::flash_attention_decode_cu(pos_, head_num_, kv_head_num_, head_size_, kv_mul_,
                                      layer_index_, seq_len_, kv_dim_, q, o, kc, vc, c);
  } else {
    kernel::MHAKernel k = kernel::get_mha_kernel(device_type_);
    if (!k) return base::error::FunctionNotImplement("no attention kernel for this device type");
    k(pos_, head_num_, layer_index_, seq_len_, kv_dim_, kv_mul_, head_size_, o, q,
      tensor::Tensor(), kc, vc, device_type_, c);
  }
  return launched();
}

Status FlashAttentionDecodeLayer::forward(int32_t pos, int32_t head_num, int32_t kv_head_num,
                                          int32_t head_size, int32_t kv_mul, int32_t layer_idx,
                                          int32_t seq_len, int32_t kv_dim,
                                          const tensor::Tensor& query,
                                          const tensor::Tensor& mha_output,
                                          const tensor::Tensor& key_cache,
                                          const tensor::Tensor& val_cache) {
  kernel::flash_attention_decode_fp16_cu(pos, head_num, kv_head_num, head_size, kv_mul,
                                         layer_idx, seq_len, kv_dim, query, mha_output,
                                         key_cache, val_cache, cfg(cuda_config_));
  return launched();
}

// ------------------------------------------------------------ FlashAttentionPrefillLayer
FlashAttentionPrefillLayer::FlashAttentionPrefillLayer(DeviceType device_type)
    : Layer(device_type, "FlashAttentionPrefill") {
  reset_input_size(4);
  reset_output_size(0);
}

FlashAttentionPrefillLayer::FlashAttentionPrefillLayer(DeviceType device_type, int32_t head_num,
                                                       int32_t kv_head_num, int32_t head_size,
                                                       int32_t seq_len, bool use_fp16)
    : FlashAttentionPrefillLayer(device_type) {
  set_dims(head_num, kv_head_num, head_size, seq_len);
  use_fp16_ = use_fp16;
}

void FlashAttentionPrefillLayer::set_dims(int32_t head_num, int32_t kv_head_num,
                                          int32_t head_size, int32_t max_seq_len) {
  head_num_ = head_num;
  kv_head_num_ = kv_head_num;
  head_size_ = head_size;
  max_seq_len_ = max_seq_len;
}

Status FlashAttentionPrefillLayer::check() const {
  if (!dims_ok(head_num_, kv_head_num_, head_size_))
    return base::error::InvalidArgument("Invalid attention parameters");
  return base::error::Success();
}

Status FlashAttentionPrefillLayer::forward() {
  Status st = check();
  if (!st) return st;
  kernel::flash_attention_prefill_cu(start_pos_, cur_seq_len_, head_num_, kv_head_num_,
                                     head_size_, head_num_ / kv_head_num_, layer_idx_,
                                     max_seq_len_, kv_head_num_ * head_size_, get_input(0),
                                     get_input(1), get_input(2), get_input(3),
                                     cfg(cuda_config_));
  return launched();
}

Status FlashAttentionPrefillLayer::forward(int32_t start_pos, int32_t seq_len, int32_t head_num,
                                           int32_t kv_head_num, int32_t head_size,
                                           int32_t kv_mul, int32_t layer_idx,
                                           int32_t max_seq_len, int32_t kv_dim,
                                           const tensor::Tensor& query,
                                           const tensor::Tensor& output,
                                           const tensor::Tensor& key_cache,
                                           const tensor::Tensor& val_cache) {
  kernel::flash_attention_prefill_fp16_cu(start_pos, seq_len, head_num, kv_head_num, head_size,
                                          kv_mul, layer_idx, max_seq_len, kv_dim, query, output,
                                          key_cache, val_cache, cfg(cuda_config_));
  return launched();
}

// ------------------------------------------------------------ FlashAttentionDecodeGpuPosLayer
FlashAttentionDecodeGpuPosLayer::FlashAttentionDecodeGpuPosLayer(DeviceType device_type)
    : Layer(device_type, "FlashAttentionDecodeGpuPos") {}
Status FlashAttentionDecodeGpuPosLayer::forward() {
  return base::error::InvalidArgument(kUseParams);
}
Status FlashAttentionDecodeGpuPosLayer::forward(const int32_t* pos_gpu, int32_t head_num,
                                                int32_t kv_head_num, int32_t head_size,
                                                int32_t kv_mul, int32_t layer_idx,
                                                int32_t seq_len, int32_t kv_dim,
                                                const tensor::Tensor& query,
                                                const tensor::Tensor& mha_output,
                                                const tensor::Tensor& key_cache,
                                                const tensor::Tensor& val_cache) {
  kernel::flash_attention_decode_fp16_gpu_pos_cu(pos_gpu, head_num, kv_head_num, head_size,
                                                 kv_mul, layer_idx, seq_len, kv_dim, query,
                                                 mha_output, key_cache, val_cache,
                                                 cfg(cuda_config_));
  return launched();
}

// ------------------------------------------------------------ CopyToKVCacheLayer
CopyToKVCacheLayer::CopyToKVCacheLayer(DeviceType device_type)
    : Layer(device_type, "CopyToKVCache") {}
Status CopyToKVCacheLayer::forward() { return base::error::InvalidArgument(kUseParams); }
Status CopyToKVCacheLayer::forward(const tensor::Tensor& kv_cache, const tensor::Tensor& kv_data,
                                   const int32_t* pos_gpu, int32_t kv_dim, int32_t layer_idx,
                                   int32_t seq_len) {
  hipStream_t s = cuda_config_ ? cuda_config_->stream : nullptr;
  if (kv_cache.data_type() == base::DataType::kDataTypeFp16)
    kernel::copy_to_kv_cache_kernel_fp16(kv_cache.ptr<__half>(), kv_data.ptr<const __half>(),
                                         pos_gpu, kv_dim, layer_idx, seq_len, s);
  else
    kernel::copy_to_kv_cache_kernel(kv_cache.ptr<float>(), kv_data.ptr<const float>(), pos_gpu,
                                    kv_dim, layer_idx, seq_len, s);
  return launched();
}

// ------------------------------------------------------------ vision
FusedSplitRopeTransposeLayer::FusedSplitRopeTransposeLayer(DeviceType device_type)
    : Layer(device_type, "FusedSplitRopeTranspose") {}
Status FusedSplitRopeTransposeLayer::forward() {
  return base::error::InvalidArgument(kUseParams);
}
Status FusedSplitRopeTransposeLayer::forward(const tensor::Tensor& qkv,
                                             const tensor::Tensor& cos_cache,
                                             const tensor::Tensor& sin_cache,
                                             const tensor::Tensor& q_out,
                                             const tensor::Tensor& k_out,
                                             const tensor::Tensor& v_out, int32_t num_tokens,
                                             int32_t num_heads, int32_t head_dim,
                                             hipStream_t stream) {
  tensor::Tensor q = q_out, k = k_out, v = v_out;  // views: the data is shared
  kernel::fused_split_rope_transpose_cu(qkv, cos_cache, sin_cache, q, k, v, num_tokens,
                                        num_heads, head_dim, stream);
  return launched();
}

VisionAttentionLayer::VisionAttentionLayer(DeviceType device_type)
    : Layer(device_type, "VisionAttention") {}
Status VisionAttentionLayer::forward() { return base::error::InvalidArgument(kUseParams); }
Status VisionAttentionLayer::forward(const tensor::Tensor& q_transposed,
                                     const tensor::Tensor& k_transposed,
                                     const tensor::Tensor& v_transposed,
                                     const tensor::Tensor& attn_out,
                                     const tensor::Tensor& out_transposed,
                                     const tensor::Tensor& attn_scores, int32_t num_tokens,
                                     int32_t num_heads, int32_t head_dim, float scale,
                                     kernel::CudaConfig* cuda_config) {
  tensor::Tensor o = attn_out, ot = out_transposed, sc = attn_scores;
  kernel::vision_attention_pretransposed_cu(q_transposed, k_transposed, v_transposed, o, ot, sc,
                                            num_tokens, num_heads, head_dim, scale, cuda_config);
  return launched();
}

}  // namespace op
}  // namespace orin
