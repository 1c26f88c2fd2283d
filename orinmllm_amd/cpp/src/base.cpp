#include "orin/base.h"
#include "orin/tensor.h"

namespace orin {
namespace base {

size_t DataTypeSize(DataType t) {
  switch (t) {
    case DataType::kDataTypeFp32:
    case DataType::kDataTypeInt32: return 4;
    case DataType::kDataTypeFp16:
    case DataType::kDataTypeBf16: return 2;
    case DataType::kDataTypeInt8: return 1;
    default: return 0;
  }
}

const char* AttentionTypeName(AttentionType t) {
  switch (t) {
    case AttentionType::kAttentionMHA: return "MHA";
    case AttentionType::kAttentionFlash1: return "FlashAttention1";
    case AttentionType::kAttentionFlash2: return "FlashAttention2";
  }
  return "Unknown";
}

std::ostream& operator<<(std::ostream& os, const Status& s) {
  return os << "status " << s.get_err_code() << ": " << s.get_err_msg();
}

namespace error {
Status Success(const std::string& msg) { return Status(kSuccess, msg); }
Status FunctionNotImplement(const std::string& msg) { return Status(kFunctionUnImplement, msg); }
Status InternalError(const std::string& msg) { return Status(kInternalError, msg); }
Status InvalidArgument(const std::string& msg) { return Status(kInvalidArgument, msg); }
}  // namespace error

}  // namespace base

namespace tensor {

Tensor::Tensor(base::DataType data_type, std::vector<int32_t> dims, void* ptr,
               base::DeviceType device_type)
    : data_type_(data_type), device_type_(device_type), dims_(std::move(dims)), ptr_(ptr) {
  size_ = dims_.empty() ? 0 : 1;
  for (int32_t d : dims_) size_ *= d > 0 ? static_cast<size_t>(d) : 0;
}

}  // namespace tensor
}  // namespace orin
