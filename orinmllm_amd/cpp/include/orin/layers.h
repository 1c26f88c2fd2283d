// op:: attention layers of kuiper (kuiper/include/op/flash_attention.h,
// mha.h, misc_layers.h:27-62 and 167-200, vision_layers.h:76-111) over the kernel::
// functions of orin/kernels.h.  Same constructors, setters, input slots and forward
// overloads as the reference; check() rejects the same non-positive sizes
// (flash_attention.cpp:32-37).  Where kuiper's forward() returns Success without
// looking at the launch, these return the kernel call's status.
#ifndef ORIN_HOST_LAYERS_H
#define ORIN_HOST_LAYERS_H

#include <memory>
#include <string>
#include <vector>

#include "orin/base.h"
#include "orin/kernels.h"
#include "orin/tensor.h"

namespace orin {
namespace op {

// The part of kuiper's op::Layer (kuiper/include/op/layer.h) these layers use: typed
// input / output slots and the CUDA config shared with the model.
class Layer {
 public:
  Layer(base::DeviceType device_type, std::string name)
      : device_type_(device_type), name_(std::move(name)) {}
  virtual ~Layer() = default;

  virtual base::Status check() const = 0;
  virtual base::Status forward() = 0;

  void set_input(int32_t idx, const tensor::Tensor& t) { inputs_.at(idx) = t; }
  void set_output(int32_t idx, const tensor::Tensor& t) { outputs_.at(idx) = t; }
  const tensor::Tensor& get_input(int32_t idx) const { return inputs_.at(idx); }
  const tensor::Tensor& get_output(int32_t idx) const { return outputs_.at(idx); }
  size_t input_size() const { return inputs_.size(); }
  size_t output_size() const { return outputs_.size(); }
  void set_cuda_config(std::shared_ptr<kernel::CudaConfig> c) { cuda_config_ = std::move(c); }
  std::shared_ptr<kernel::CudaConfig> cuda_config() const { return cuda_config_; }
  base::DeviceType device_type() const { return device_type_; }
  const std::string& get_layer_name() const { return name_; }

 protected:
  void reset_input_size(size_t n) { inputs_.resize(n); }
  void reset_output_size(size_t n) { outputs_.resize(n); }
  // Status of the kernel call just made (see kernel::last_status).
  static base::Status launched() { return kernel::last_status(); }

  base::DeviceType device_type_;
  std::string name_;
  std::vector<tensor::Tensor> inputs_;
  std::vector<tensor::Tensor> outputs_;
  std::shared_ptr<kernel::CudaConfig> cuda_config_;
};

// mha.h:6-28.  Inputs: query, score, key_cache, value_cache; output 0: mha_out.
class MultiHeadAttention : public Layer {
 public:
  MultiHeadAttention(base::DeviceType device_type, int32_t layer_index, int32_t kv_mul,
                     int32_t kv_dim, int32_t seq_len, int32_t head_num, int32_t head_size);
  base::Status check() const override;
  base::Status forward() override;
  void set_pos(int32_t pos) { pos_ = pos; }
  void set_layer_idx(int32_t layer_idx) { layer_index_ = layer_idx; }

 private:
  int32_t layer_index_ = 0, pos_ = 0, kv_mul_ = 0, kv_dim_ = 0, seq_len_ = 0, head_num_ = 0,
          head_size_ = 0;
};

// misc_layers.h:27-40.
class MHAGpuPosLayer : public Layer {
 public:
  explicit MHAGpuPosLayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  base::Status forward(const int32_t* pos_ptr, int32_t head_num, int32_t layer_idx,
                       int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                       tensor::Tensor& mha_output, const tensor::Tensor& query,
                       tensor::Tensor& score_storage, const tensor::Tensor& key_cache,
                       const tensor::Tensor& val_cache);
};

// misc_layers.h:45-60.
class BatchedMHALayer : public Layer {
 public:
  explicit BatchedMHALayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  base::Status forward(int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t layer_idx,
                       int32_t max_seq_len, int32_t dim, int32_t kv_dim, int32_t kv_mul,
                       int32_t head_size, tensor::Tensor& mha_output, const tensor::Tensor& query,
                       tensor::Tensor& score_storage, const tensor::Tensor& key_cache,
                       const tensor::Tensor& val_cache);
};

// flash_attention.h:19-65.  Inputs: query, mha_output (written), key_cache, value_cache,
// pos (device int32 [1], read when use_gpu_pos).
class FlashAttentionDecodeLayer : public Layer {
 public:
  explicit FlashAttentionDecodeLayer(base::DeviceType device_type);
  FlashAttentionDecodeLayer(base::DeviceType device_type, int32_t head_num, int32_t kv_head_num,
                            int32_t head_size, int32_t kv_mul, int32_t seq_len, int32_t kv_dim,
                            bool use_fp16 = false);
  base::Status check() const override;
  base::Status forward() override;
  base::Status forward(int32_t pos, int32_t head_num, int32_t kv_head_num, int32_t head_size,
                       int32_t kv_mul, int32_t layer_idx, int32_t seq_len, int32_t kv_dim,
                       const tensor::Tensor& query, const tensor::Tensor& mha_output,
                       const tensor::Tensor& key_cache, const tensor::Tensor& val_cache);
  void set_layer_index(int32_t layer_index) { layer_index_ = layer_index; }
  void set_pos(int32_t pos) { pos_ = pos; }
  void set_use_gpu_pos(bool v) { use_gpu_pos_ = v; }
  void set_dims(int32_t head_num, int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                int32_t seq_len, int32_t kv_dim);
  void set_use_fp16(bool v) { use_fp16_ = v; }
  void set_attention_type(base::AttentionType t) { attention_type_ = t; }
  base::AttentionType get_attention_type() const { return attention_type_; }

 private:
  int32_t head_num_ = 0, kv_head_num_ = 0, head_size_ = 0, kv_mul_ = 0, seq_len_ = 0,
          kv_dim_ = 0, layer_index_ = 0, pos_ = 0;
  bool use_fp16_ = false, use_gpu_pos_ = false;
  base::AttentionType attention_type_ = base::AttentionType::kAttentionFlash1;
};

// flash_attention.h:76-118.  Inputs: query, output (written; may alias query),
// key_cache, value_cache.
class FlashAttentionPrefillLayer : public Layer {
 public:
  explicit FlashAttentionPrefillLayer(base::DeviceType device_type);
  FlashAttentionPrefillLayer(base::DeviceType device_type, int32_t head_num, int32_t kv_head_num,
                             int32_t head_size, int32_t seq_len, bool use_fp16 = false);
  base::Status check() const override;
  base::Status forward() override;
  base::Status forward(int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t kv_head_num,
                       int32_t head_size, int32_t kv_mul, int32_t layer_idx, int32_t max_seq_len,
                       int32_t kv_dim, const tensor::Tensor& query, const tensor::Tensor& output,
                       const tensor::Tensor& key_cache, const tensor::Tensor& val_cache);
  void set_cur_seq_len(int32_t v) { cur_seq_len_ = v; }
  void set_start_pos(int32_t v) { start_pos_ = v; }
  void set_layer_index(int32_t v) { layer_idx_ = v; }
  void set_dims(int32_t head_num, int32_t kv_head_num, int32_t head_size, int32_t max_seq_len);
  void set_use_fp16(bool v) { use_fp16_ = v; }
  void set_attention_type(base::AttentionType t) { attention_type_ = t; }
  base::AttentionType get_attention_type() const { return attention_type_; }

 private:
  int32_t head_num_ = 0, kv_head_num_ = 0, head_size_ = 0, max_seq_len_ = 0, cur_seq_len_ = 0,
          start_pos_ = 0, layer_idx_ = 0;
  bool use_fp16_ = false;
  base::AttentionType attention_type_ = base::AttentionType::kAttentionFlash1;
};

// misc_layers.h:183-200.
class FlashAttentionDecodeGpuPosLayer : public Layer {
 public:
  explicit FlashAttentionDecodeGpuPosLayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  void set_attention_type(base::AttentionType t) { attention_type_ = t; }
  base::AttentionType get_attention_type() const { return attention_type_; }
  base::Status forward(const int32_t* pos_gpu, int32_t head_num, int32_t kv_head_num,
                       int32_t head_size, int32_t kv_mul, int32_t layer_idx, int32_t seq_len,
                       int32_t kv_dim, const tensor::Tensor& query,
                       const tensor::Tensor& mha_output, const tensor::Tensor& key_cache,
                       const tensor::Tensor& val_cache);

 private:
  base::AttentionType attention_type_ = base::AttentionType::kAttentionFlash1;
};

// misc_layers.h:167-178.
class CopyToKVCacheLayer : public Layer {
 public:
  explicit CopyToKVCacheLayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  base::Status forward(const tensor::Tensor& kv_cache, const tensor::Tensor& kv_data,
                       const int32_t* pos_gpu, int32_t kv_dim, int32_t layer_idx,
                       int32_t seq_len);
};

// vision_layers.h:76-91.
class FusedSplitRopeTransposeLayer : public Layer {
 public:
  explicit FusedSplitRopeTransposeLayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  base::Status forward(const tensor::Tensor& qkv, const tensor::Tensor& cos_cache,
                       const tensor::Tensor& sin_cache, const tensor::Tensor& q_out,
                       const tensor::Tensor& k_out, const tensor::Tensor& v_out,
                       int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                       hipStream_t stream = nullptr);
};

// vision_layers.h:95-111.
class VisionAttentionLayer : public Layer {
 public:
  explicit VisionAttentionLayer(base::DeviceType device_type);
  base::Status check() const override { return base::error::Success(); }
  base::Status forward() override;
  base::Status forward(const tensor::Tensor& q_transposed, const tensor::Tensor& k_transposed,
                       const tensor::Tensor& v_transposed, const tensor::Tensor& attn_out,
                       const tensor::Tensor& out_transposed, const tensor::Tensor& attn_scores,
                       int32_t num_tokens, int32_t num_heads, int32_t head_dim, float scale,
                       kernel::CudaConfig* cuda_config = nullptr);
};

}  // namespace op
}  // namespace orin

#endif  // ORIN_HOST_LAYERS_H
