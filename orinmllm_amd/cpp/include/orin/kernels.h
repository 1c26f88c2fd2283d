// kernel:: free functions of the attention path with kuiper's signatures, running on
// the gfx950 kernels of liborin_attn.so through its C ABI (include/orin_attn.h).
//
// Like kuiper's kernels they return void and queue work on config->stream (nullptr =
// the default stream).  kuiper does not check its launches; here every call records its
// outcome, readable with last_status() on the calling thread: Success, InvalidArgument
// (a size, pointer or head count the C ABI rejected) or InternalError (unsupported
// shape or type, missing workspace, HIP launch failure).  Nothing falls back to a CPU
// implementation: get_mha_kernel(kDeviceCPU) returns nullptr.
#ifndef ORIN_HOST_KERNELS_H
#define ORIN_HOST_KERNELS_H

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "orin/base.h"
#include "orin/tensor.h"

namespace orin {
namespace kernel {

// kernel::CudaConfig (kuiper/include/base/cuda_config.h:17-33): the stream the path's
// kernels run on.  The cuBLAS handle, graph context and fp16 workspaces of kuiper's
// struct serve GEMMs outside this path.
struct CudaConfig {
  hipStream_t stream = nullptr;
};

// Outcome of the last kernel:: call on this thread.
const base::Status& last_status();

// kernels_interface.h:24-30 and kernels_interfaces.cpp:63-72.
typedef void (*MHAKernel)(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                          int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                          const tensor::Tensor& mha_out, const tensor::Tensor& query_tensor,
                          const tensor::Tensor& score_tensor,
                          const tensor::Tensor& key_cache_tensor,
                          const tensor::Tensor& value_cache_tensor, base::DeviceType device_type,
                          CudaConfig* config);
MHAKernel get_mha_kernel(base::DeviceType device_type);

// mha_kernel.cuh:4-26 (fp32).
void mha_kernel_cu(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                   int32_t kv_dim, int32_t kv_mul, int32_t head_size, const tensor::Tensor& mha_out,
                   const tensor::Tensor& query_tensor, const tensor::Tensor& score_tensor,
                   const tensor::Tensor& key_cache_tensor,
                   const tensor::Tensor& value_cache_tensor, base::DeviceType device_type,
                   CudaConfig* config);
void mha_kernel_cu_gpu_pos(const int32_t* pos_ptr, int32_t head_num, int32_t layer_index,
                           int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                           const tensor::Tensor& mha_out, const tensor::Tensor& query_tensor,
                           const tensor::Tensor& score_tensor,
                           const tensor::Tensor& key_cache_tensor,
                           const tensor::Tensor& value_cache_tensor,
                           base::DeviceType device_type, CudaConfig* config);
void batched_mha_kernel_cu(int32_t start_pos, int32_t seq_len, int32_t head_num,
                           int32_t layer_index, int32_t max_seq_len, int32_t dim, int32_t kv_dim,
                           int32_t kv_mul, int32_t head_size, const tensor::Tensor& mha_out,
                           const tensor::Tensor& query_tensor, const tensor::Tensor& score_tensor,
                           const tensor::Tensor& key_cache_tensor,
                           const tensor::Tensor& value_cache_tensor,
                           base::DeviceType device_type, CudaConfig* config);

// flash_attention_kernel.cuh:27-234.  The element type comes from the tensors (fp32,
// fp16 or bf16); the fp16 / FlashAttention-2 names are the same kernels.
#define ORIN_FA_PREFILL_ARGS                                                              \
  int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t kv_head_num,              \
      int32_t head_size, int32_t kv_mul, int32_t layer_index, int32_t max_seq_len,        \
      int32_t kv_dim, const tensor::Tensor &query, const tensor::Tensor &output,          \
      const tensor::Tensor &key_cache, const tensor::Tensor &value_cache, CudaConfig *config
#define ORIN_FA_DECODE_ARGS                                                               \
  int32_t pos, int32_t head_num, int32_t kv_head_num, int32_t head_size, int32_t kv_mul,  \
      int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,                           \
      const tensor::Tensor &query, const tensor::Tensor &output,                          \
      const tensor::Tensor &key_cache, const tensor::Tensor &value_cache, CudaConfig *config
#define ORIN_FA_DECODE_GPU_POS_ARGS                                                       \
  const int32_t *pos_ptr, int32_t head_num, int32_t kv_head_num, int32_t head_size,       \
      int32_t kv_mul, int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,           \
      const tensor::Tensor &query, const tensor::Tensor &output,                          \
      const tensor::Tensor &key_cache, const tensor::Tensor &value_cache, CudaConfig *config
void flash_attention_prefill_cu(ORIN_FA_PREFILL_ARGS);
void flash_attention_prefill_fp16_cu(ORIN_FA_PREFILL_ARGS);
void flash_attention2_prefill_cu(ORIN_FA_PREFILL_ARGS);
void flash_attention2_prefill_fp16_cu(ORIN_FA_PREFILL_ARGS);
void flash_attention_decode_cu(ORIN_FA_DECODE_ARGS);
void flash_attention_decode_fp16_cu(ORIN_FA_DECODE_ARGS);
void flash_attention2_decode_cu(ORIN_FA_DECODE_ARGS);
void flash_attention2_decode_fp16_cu(ORIN_FA_DECODE_ARGS);
void flash_attention_decode_fp16_gpu_pos_cu(ORIN_FA_DECODE_GPU_POS_ARGS);
void flash_attention2_decode_fp16_gpu_pos_cu(ORIN_FA_DECODE_GPU_POS_ARGS);

// vision_encoder_kernel.cuh:159-192.
void vision_attention_pretransposed_cu(const tensor::Tensor& q_trans,
                                       const tensor::Tensor& k_trans,
                                       const tensor::Tensor& v_trans, tensor::Tensor& output,
                                       tensor::Tensor& out_transposed, tensor::Tensor& scores,
                                       int num_tokens, int num_heads, int head_dim,
                                       float softmax_scale, const CudaConfig* config);
// matmul_kernel.cuh:37-41: output [batch, out] = scale * input [batch, in] . weight^T,
// weight [out, in] -- the wo projection after the batched attention (qwen_base.cpp:464-474).
void batched_matmul_kernel_cu_pure_fp16(const tensor::Tensor& input,
                                         const tensor::Tensor& weight,
                                         const tensor::Tensor& output, int32_t batch_size,
                                         float scale = 1.f, const CudaConfig* config = nullptr);
void fused_split_rope_transpose_cu(const tensor::Tensor& qkv, const tensor::Tensor& cos_cache,
                                   const tensor::Tensor& sin_cache, tensor::Tensor& q_trans,
                                   tensor::Tensor& k_trans, tensor::Tensor& v_trans,
                                   int num_tokens, int num_heads, int head_dim,
                                   hipStream_t stream);

// kv_cache_kernel.cuh:24-33 and rope_kernel.cuh:21-22.
void copy_to_kv_cache_kernel(float* kv_cache, const float* src, const int32_t* pos,
                             int32_t kv_dim, int32_t layer_idx, int32_t seq_len,
                             hipStream_t stream);
void copy_to_kv_cache_kernel_fp16(__half* kv_cache, const __half* src, const int32_t* pos,
                                  int32_t kv_dim, int32_t layer_idx, int32_t seq_len,
                                  hipStream_t stream);
void sin_cos_cache_calc_cu(int head_size, int max_seq_len, const tensor::Tensor& sin_cache,
                           const tensor::Tensor& cos_cache, hipStream_t stream);

}  // namespace kernel
}  // namespace orin

#endif  // ORIN_HOST_KERNELS_H
