// The names a kuiper translation unit sees where the attention adapter is compiled
// (tensor::Tensor, base::DeviceType / DataType, kernel::CudaConfig, cudaStream_t and
// glog's CHECK_EQ; kuiper/include/tensor/tensor.h, base/base.h, base/cuda_config.h), bound
// to this repository's host mirror so that the kuiper-side adapter text compiles and
// links against liborin_attn.so here.  A failed CHECK_EQ prints its message and aborts,
// as LOG(FATAL) does.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <iostream>

#include "orin/base.h"
#include "orin/kernels.h"
#include "orin/tensor.h"

typedef hipStream_t cudaStream_t;
namespace tensor = orin::tensor;
namespace base = orin::base;
namespace kernel {
using orin::kernel::CudaConfig;
}

struct KuiperFatalStream {
  bool failed;
  ~KuiperFatalStream() {
    if (failed) {
      std::cerr << std::endl;
      std::abort();
    }
  }
  template <typename V>
  KuiperFatalStream& operator<<(const V& v) {
    if (failed) std::cerr << v;
    return *this;
  }
};
#define CHECK_EQ(a, b) KuiperFatalStream{!((a) == (b))} << "Check failed: " #a " == " #b " "
