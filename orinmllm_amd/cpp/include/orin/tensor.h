// tensor::Tensor of the attention path: a non-owning view of device memory with an
// element type and dimensions.  It carries what the path's kernels read from kuiper's
// tensor::Tensor (kuiper/include/tensor/tensor.h:12-95: ptr<T>(), size(), get_dim(),
// dims_size(), data_type(), is_empty(), device_type()); the caller owns the memory,
// as kuiper's model owns its buffers.
#ifndef ORIN_HOST_TENSOR_H
#define ORIN_HOST_TENSOR_H

#include <cstddef>
#include <cstdint>
#include <vector>

#include "orin/base.h"

namespace orin {
namespace tensor {

class Tensor {
 public:
  Tensor() = default;
  Tensor(base::DataType data_type, std::vector<int32_t> dims, void* ptr,
         base::DeviceType device_type = base::DeviceType::kDeviceCUDA);

  template <typename T>
  T* ptr() const {
    return static_cast<T*>(ptr_);
  }
  void* raw_ptr() const { return ptr_; }

  size_t size() const { return size_; }
  size_t byte_size() const { return size_ * base::DataTypeSize(data_type_); }
  int32_t dims_size() const { return static_cast<int32_t>(dims_.size()); }
  int32_t get_dim(int32_t idx) const { return dims_.at(idx); }
  const std::vector<int32_t>& dims() const { return dims_; }
  base::DataType data_type() const { return data_type_; }
  base::DeviceType device_type() const { return device_type_; }
  bool is_empty() const { return ptr_ == nullptr || size_ == 0; }

 private:
  base::DataType data_type_ = base::DataType::kDataTypeUnknown;
  base::DeviceType device_type_ = base::DeviceType::kDeviceUnknown;
  std::vector<int32_t> dims_;
  size_t size_ = 0;
  void* ptr_ = nullptr;
};

}  // namespace tensor
}  // namespace orin

#endif  // ORIN_HOST_TENSOR_H
