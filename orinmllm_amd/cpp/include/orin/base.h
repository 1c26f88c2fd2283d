// Host-side vocabulary of the attention path: device, element and attention types and
// the Status value the layers return.  Names and numeric values follow kuiper's
// base.h (kuiper/include/base/base.h:51-55 DeviceType, :58-64 DataType, :96-104
// StatusCode, :113-117 AttentionType, :127-190 Status and base::error) so that an
// adapter can pass them through unchanged; DataType gains kDataTypeBf16.
#ifndef ORIN_HOST_BASE_H
#define ORIN_HOST_BASE_H

#include <cstdint>
#include <ostream>
#include <string>

namespace orin {
namespace base {

enum class DeviceType : uint8_t {
  kDeviceUnknown = 0,
  kDeviceCPU = 1,
  kDeviceCUDA = 2,  // the GPU (HIP) device, named as in kuiper
};

enum class DataType : uint8_t {
  kDataTypeUnknown = 0,
  kDataTypeFp32 = 1,
  kDataTypeInt8 = 2,
  kDataTypeInt32 = 3,
  kDataTypeFp16 = 4,
  kDataTypeBf16 = 5,  // not in kuiper; the C ABI's ORIN_DTYPE_BF16
};

size_t DataTypeSize(DataType t);

enum class AttentionType : uint8_t {
  kAttentionMHA = 0,
  kAttentionFlash1 = 1,
  kAttentionFlash2 = 2,
};

const char* AttentionTypeName(AttentionType t);

enum StatusCode : uint8_t {
  kSuccess = 0,
  kFunctionUnImplement = 1,
  kPathNotValid = 2,
  kModelParseError = 3,
  kInternalError = 5,
  kKeyValueHasExist = 6,
  kInvalidArgument = 7,
};

class Status {
 public:
  Status(int code = kSuccess, std::string err_message = "")
      : code_(code), message_(std::move(err_message)) {}
  bool operator==(int code) const { return code_ == code; }
  bool operator!=(int code) const { return code_ != code; }
  explicit operator int() const { return code_; }
  explicit operator bool() const { return code_ == kSuccess; }
  int32_t get_err_code() const { return code_; }
  const std::string& get_err_msg() const { return message_; }
  void set_err_msg(const std::string& m) { message_ = m; }

 private:
  int code_ = kSuccess;
  std::string message_;
};

std::ostream& operator<<(std::ostream& os, const Status& s);

namespace error {
Status Success(const std::string& msg = "");
Status FunctionNotImplement(const std::string& msg = "");
Status InternalError(const std::string& msg = "");
Status InvalidArgument(const std::string& msg = "");
}  // namespace error

}  // namespace base
}  // namespace orin

#endif  // ORIN_HOST_BASE_H
