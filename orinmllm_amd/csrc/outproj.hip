// Attention output projection: the step that consumes the attention output, as kuiper's
// prefill runs it (kuiper/source/model/qwen_base.cpp:464-474, wo through
// kernel::batched_matmul_kernel_cu_pure_fp16, matmul_kernel.cu:687-732):
//   out[b, k] = scale * sum_m in[b, m] * w[k, m]     (w is [out_dim, in_dim], row-major)
// The attention kernels already store their output as the row-major [tokens, heads*d]
// matrix this GEMM reads, so it runs straight on that buffer.  A plain dense GEMM is a
// library job: rocBLAS gemm_ex with fp32 accumulation (the reference uses an fp16 cuBLAS
// HGEMM).  One rocBLAS handle per device with a library-owned workspace
// (rocblas_set_workspace), created by output_projection_prepare (called from
// orin_attn_workspace_reserve_stream) or on the first call outside graph capture, so that a
// captured call allocates nothing; a capturing call on a device without a handle is
// refused.  The stream is set per call under a lock, so calls from several threads
// serialise only their enqueue.
#include <rocblas/rocblas.h>

#include <mutex>
#include <vector>

#include "kernels.h"

namespace orin {

namespace {

std::mutex g_blas_mu;
std::vector<rocblas_handle> g_blas;  // per device
constexpr size_t kBlasWorkspace = 32u << 20;

// Handle of the current device, created with its workspace if missing (g_blas_mu held).
rocblas_handle device_handle(int dev, bool create) {
  if ((int)g_blas.size() <= dev) g_blas.resize(dev + 1, nullptr);
  if (g_blas[dev] || !create) return g_blas[dev];
  rocblas_handle h = nullptr;
  if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
  void* ws = nullptr;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) {
    rocblas_destroy_handle(h);
    return nullptr;
  }
  const hipError_t e = hipMalloc(&ws, kBlasWorkspace);
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  if (e != hipSuccess || rocblas_set_workspace(h, ws, kBlasWorkspace) != rocblas_status_success) {
    if (ws) (void)hipFree(ws);
    rocblas_destroy_handle(h);
    return nullptr;
  }
  g_blas[dev] = h;  // kept, with its workspace, until the process ends
  return h;
}

}  // namespace

int output_projection_prepare() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(g_blas_mu);
  return device_handle(dev, true) ? 0 : -1;
}

int output_projection(const void* input, const void* weight, void* output, int batch, int in_dim,
                      int out_dim, float scale, int dtype, hipStream_t stream, bool capturing) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  rocblas_datatype t;
  switch (dtype) {
    case kF32: t = rocblas_datatype_f32_r; break;
    case kF16: t = rocblas_datatype_f16_r; break;
    case kBF16: t = rocblas_datatype_bf16_r; break;
    default: return -2;
  }
  std::lock_guard<std::mutex> lock(g_blas_mu);
  rocblas_handle h = device_handle(dev, !capturing);
  if (!h) return capturing ? -3 : -1;
  if (rocblas_set_stream(h, stream) != rocblas_status_success) return -1;
  const float alpha = scale, beta = 0.f;
  // Column-major view: out^T [out_dim, batch] = w^T' [out_dim, in_dim] . in^T [in_dim, batch],
  // with w stored as a column-major [in_dim, out_dim] matrix (transposed in the call).
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_transpose, rocblas_operation_none, out_dim, batch, in_dim, &alpha,
      weight, t, in_dim, input, t, in_dim, &beta, output, t, out_dim, output, t, out_dim,
      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  return st == rocblas_status_success ? 0 : -1;
}

}  // namespace orin
