// Parity of the C++ host mirror (orin::op layers and orin::kernel functions, the
// kuiper-shaped API over liborin_attn.so) against the CPU oracle (oracle/oracle.c,
// linked as the checker).  Run with --cpu-only for the cases that make no device call.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

#include "mini_test.h"
#include "orin/layers.h"

extern "C" {
void oracle_mha_kernel(int pos, int head_num, int layer_index, int seq_len, int kv_dim,
                       int kv_mul, int head_size, float* mha_out, const float* query,
                       float* score, const float* key_cache, const float* value_cache);
void oracle_prefill_causal(int start_pos, int S, int Hq, int Hkv, int d, float scale,
                           const float* q, const float* k_cache, const float* v_cache, float* o,
                           int nthreads);
void oracle_varlen_bidir(int N, int H, int d, float scale, const float* q, const float* k,
                         const float* v, const int* cu_seqlens, int n_seg, float* o,
                         int nthreads);
void oracle_vision_cos_sin(int grid_t, int grid_h, int grid_w, int merge, int d, float* cos_out,
                           float* sin_out);
void oracle_vision_rotary(float* x, int H, int N, int d, const float* cos_t, const float* sin_t);
}

using orin::base::DataType;
using orin::base::DeviceType;
using orin::base::Status;
using orin::tensor::Tensor;
namespace op = orin::op;
namespace kernel = orin::kernel;

namespace {

// ------------------------------------------------------------ host data helpers
std::vector<float> normal(size_t n, uint32_t seed) {
  std::mt19937 g(seed);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<float> v(n);
  for (float& x : v) x = nd(g);
  return v;
}

uint16_t to_bf16(float x) {  // round to nearest even
  uint32_t u;
  memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float from_bf16(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float x;
  memcpy(&x, &u, 4);
  return x;
}

// Values rounded to `dt` (what the device sees), and their device copy.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  explicit DevBuf(size_t b) : bytes(b) {
    if (hipMalloc(&p, b) != hipSuccess) p = nullptr;
  }
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
};

void quantize(std::vector<float>& x, DataType dt) {
  for (float& v : x) {
    if (dt == DataType::kDataTypeFp16) v = (float)(_Float16)v;
    else if (dt == DataType::kDataTypeBf16) v = from_bf16(to_bf16(v));
  }
}

void upload(DevBuf& b, const std::vector<float>& x, DataType dt) {
  if (dt == DataType::kDataTypeFp32) {
    (void)hipMemcpy(b.p, x.data(), x.size() * 4, hipMemcpyHostToDevice);
  } else {
    std::vector<uint16_t> h(x.size());
    for (size_t i = 0; i < x.size(); ++i) {
      if (dt == DataType::kDataTypeFp16) {
        _Float16 f = (_Float16)x[i];
        memcpy(&h[i], &f, 2);
      } else {
        h[i] = to_bf16(x[i]);
      }
    }
    (void)hipMemcpy(b.p, h.data(), h.size() * 2, hipMemcpyHostToDevice);
  }
}

std::vector<float> download(const DevBuf& b, size_t n, DataType dt) {
  std::vector<float> x(n);
  if (dt == DataType::kDataTypeFp32) {
    (void)hipMemcpy(x.data(), b.p, n * 4, hipMemcpyDeviceToHost);
  } else {
    std::vector<uint16_t> h(n);
    (void)hipMemcpy(h.data(), b.p, n * 2, hipMemcpyDeviceToHost);
    for (size_t i = 0; i < n; ++i) {
      if (dt == DataType::kDataTypeFp16) {
        _Float16 f;
        memcpy(&f, &h[i], 2);
        x[i] = (float)f;
      } else {
        x[i] = from_bf16(h[i]);
      }
    }
  }
  return x;
}

// A device tensor holding `x` rounded to dt; x is rounded in place.
struct DevTensor {
  DevBuf buf;
  Tensor t;
  DevTensor(std::vector<float>& x, std::vector<int32_t> dims, DataType dt)
      : buf(x.size() * orin::base::DataTypeSize(dt)) {
    quantize(x, dt);
    upload(buf, x, dt);
    t = Tensor(dt, std::move(dims), buf.p);
  }
  DevTensor(size_t n, std::vector<int32_t> dims, DataType dt)
      : buf(n * orin::base::DataTypeSize(dt)) {
    (void)hipMemset(buf.p, 0, buf.bytes);
    t = Tensor(dt, std::move(dims), buf.p);
  }
};

// Every element within atol + rtol*|ref| (the 16-bit bar of the Python suite is
// atol 2e-3, rtol 1e-2; fp32 uses 1e-5, 1e-4).
bool close(const std::vector<float>& got, const std::vector<float>& ref, float atol, float rtol,
           const char* what) {
  if (got.size() != ref.size()) return false;
  size_t bad = 0, worst = 0;
  float worst_err = 0.f;
  for (size_t i = 0; i < ref.size(); ++i) {
    const float e = std::fabs(got[i] - ref[i]);
    if (!(e <= atol + rtol * std::fabs(ref[i]))) ++bad;
    if (!(e <= worst_err)) {
      worst_err = e;
      worst = i;
    }
  }
  if (bad)
    printf("  %s: %zu of %zu elements outside tolerance; worst index %zu got %g want %g\n", what,
           bad, ref.size(), worst, got[worst], ref[worst]);
  return bad == 0;
}

bool gpu_ok() {
  int n = 0;
  return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

}  // namespace

// ============================================================ host-only cases

TEST(Status, ErrorHelpersCarryCodeAndMessage) {
  Status ok = orin::base::error::Success();
  Status bad = orin::base::error::InvalidArgument("x");
  EXPECT_TRUE(static_cast<bool>(ok));
  EXPECT_TRUE(!static_cast<bool>(bad));
  EXPECT_EQ(bad.get_err_code(), (int32_t)orin::base::kInvalidArgument);
  EXPECT_TRUE(bad.get_err_msg() == "x");
  EXPECT_EQ(orin::base::DataTypeSize(DataType::kDataTypeBf16), (size_t)2);
}

TEST(Layers, CheckRejectsNonPositiveDims) {
  // flash_attention.cpp:32-37: InvalidArgument before anything runs.
  op::FlashAttentionPrefillLayer pf(DeviceType::kDeviceCUDA, 0, 2, 128, 512, true);
  EXPECT_EQ(pf.check().get_err_code(), (int32_t)orin::base::kInvalidArgument);
  EXPECT_EQ(pf.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
  op::FlashAttentionDecodeLayer dc(DeviceType::kDeviceCUDA, 8, 2, -1, 4, 512, 256, true);
  EXPECT_EQ(dc.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
}

TEST(Layers, ParameterlessForwardIsRejected) {
  // misc_layers.cpp:60-62 and the other layers that take their arguments in forward(...).
  op::MHAGpuPosLayer a(DeviceType::kDeviceCUDA);
  op::VisionAttentionLayer b(DeviceType::kDeviceCUDA);
  op::FlashAttentionDecodeGpuPosLayer c(DeviceType::kDeviceCUDA);
  EXPECT_EQ(a.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
  EXPECT_EQ(b.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
  EXPECT_EQ(c.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
}

TEST(Kernels, NullTensorsAreInvalidArguments) {
  // The C ABI validates before queueing anything, so no device is needed.
  Tensor empty;
  kernel::flash_attention_prefill_fp16_cu(0, 16, 8, 2, 128, 4, 0, 64, 256, empty, empty, empty,
                                          empty, nullptr);
  EXPECT_EQ(kernel::last_status().get_err_code(), (int32_t)orin::base::kInvalidArgument);
  EXPECT_TRUE(kernel::get_mha_kernel(DeviceType::kDeviceCPU) == nullptr);
  EXPECT_TRUE(kernel::get_mha_kernel(DeviceType::kDeviceCUDA) != nullptr);
  op::MultiHeadAttention mha(DeviceType::kDeviceCUDA, 0, 1, 768, 256, 12, 64);
  EXPECT_EQ(mha.forward().get_err_code(), (int32_t)orin::base::kInvalidArgument);
}

// ============================================================ GPU cases

namespace {

// Causal prefill through FlashAttentionPrefillLayer (inputs set on the layer, as
// kuiper's Qwen models do) on layer 1 of a 2-layer cache, rows start_pos..start_pos+S-1.
void prefill_case(DataType dt, int start_pos, int S, bool direct) {
  ASSERT_TRUE(gpu_ok());
  const int Hq = 8, Hkv = 2, d = 128, max_seq = 512, layers = 2, layer = 1;
  const int dim = Hq * d, kv_dim = Hkv * d;
  std::vector<float> q = normal((size_t)S * dim, 1 + S);
  std::vector<float> kc = normal((size_t)layers * max_seq * kv_dim, 2 + S);
  std::vector<float> vc = normal((size_t)layers * max_seq * kv_dim, 3 + S);
  DevTensor qd(q, {S, dim}, dt), kd(kc, {layers, max_seq, kv_dim}, dt),
      vd(vc, {layers, max_seq, kv_dim}, dt), od((size_t)S * dim, {S, dim}, dt);
  auto cfg = std::make_shared<kernel::CudaConfig>();
  (void)hipStreamCreate(&cfg->stream);
  op::FlashAttentionPrefillLayer layer_op(DeviceType::kDeviceCUDA, Hq, Hkv, d, max_seq,
                                          dt != DataType::kDataTypeFp32);
  layer_op.set_cuda_config(cfg);
  Status st;
  if (direct) {
    st = layer_op.forward(start_pos, S, Hq, Hkv, d, Hq / Hkv, layer, max_seq, kv_dim, qd.t, od.t,
                          kd.t, vd.t);
  } else {
    layer_op.set_start_pos(start_pos);
    layer_op.set_cur_seq_len(S);
    layer_op.set_layer_index(layer);
    layer_op.set_input(0, qd.t);
    layer_op.set_input(1, od.t);
    layer_op.set_input(2, kd.t);
    layer_op.set_input(3, vd.t);
    st = layer_op.forward();
  }
  ASSERT_TRUE(static_cast<bool>(st));
  ASSERT_TRUE(hipStreamSynchronize(cfg->stream) == hipSuccess);
  std::vector<float> got = download(od.buf, (size_t)S * dim, dt);
  std::vector<float> ref((size_t)S * dim);
  const size_t loff = (size_t)layer * max_seq * kv_dim;
  oracle_prefill_causal(start_pos, S, Hq, Hkv, d, 1.f / std::sqrt((float)d), q.data(),
                        kc.data() + loff, vc.data() + loff, ref.data(), 8);
  (void)hipStreamDestroy(cfg->stream);
  EXPECT_TRUE(close(got, ref, 2e-3f, 1e-2f, "prefill"));
}

}  // namespace

TEST(GpuFlashAttentionPrefillLayer, Fp16CausalFromLayerInputs) {
  prefill_case(DataType::kDataTypeFp16, 0, 300, false);
}
TEST(GpuFlashAttentionPrefillLayer, Bf16CausalWithPrefixDirectForward) {
  prefill_case(DataType::kDataTypeBf16, 37, 200, true);
}

TEST(GpuFlashAttentionDecodeLayer, Fp16HostAndDevicePosition) {
  ASSERT_TRUE(gpu_ok());
  const DataType dt = DataType::kDataTypeFp16;
  const int Hq = 32, Hkv = 8, d = 128, max_seq = 1024, layers = 2, layer = 1, pos = 700;
  const int dim = Hq * d, kv_dim = Hkv * d;
  std::vector<float> q = normal(dim, 11);
  std::vector<float> kc = normal((size_t)layers * max_seq * kv_dim, 12);
  std::vector<float> vc = normal((size_t)layers * max_seq * kv_dim, 13);
  DevTensor qd(q, {dim}, dt), kd(kc, {layers, max_seq, kv_dim}, dt),
      vd(vc, {layers, max_seq, kv_dim}, dt), o1((size_t)dim, {dim}, dt), o2((size_t)dim, {dim}, dt);
  DevBuf posd(4);
  (void)hipMemcpy(posd.p, &pos, 4, hipMemcpyHostToDevice);
  auto cfg = std::make_shared<kernel::CudaConfig>();
  op::FlashAttentionDecodeLayer dec(DeviceType::kDeviceCUDA, Hq, Hkv, d, Hq / Hkv, max_seq,
                                    kv_dim, true);
  dec.set_cuda_config(cfg);
  dec.set_layer_index(layer);
  dec.set_pos(pos);
  dec.set_input(0, qd.t);
  dec.set_input(1, o1.t);
  dec.set_input(2, kd.t);
  dec.set_input(3, vd.t);
  ASSERT_TRUE(static_cast<bool>(dec.forward()));
  dec.set_use_gpu_pos(true);
  dec.set_input(1, o2.t);
  dec.set_input(4, Tensor(DataType::kDataTypeInt32, {1}, posd.p));
  ASSERT_TRUE(static_cast<bool>(dec.forward()));
  ASSERT_TRUE(hipDeviceSynchronize() == hipSuccess);
  std::vector<float> ref(dim), score((size_t)Hq * max_seq);
  oracle_mha_kernel(pos, Hq, layer, max_seq, kv_dim, Hq / Hkv, d, ref.data(), q.data(),
                    score.data(), kc.data(), vc.data());
  EXPECT_TRUE(close(download(o1.buf, dim, dt), ref, 2e-3f, 1e-2f, "host pos"));
  EXPECT_TRUE(close(download(o2.buf, dim, dt), ref, 2e-3f, 1e-2f, "device pos"));
}

TEST(GpuMultiHeadAttention, Fp32C1ThroughGetMhaKernel) {
  // 12 heads, d 64, query at position 255 of a 256-row cache.
  ASSERT_TRUE(gpu_ok());
  const DataType dt = DataType::kDataTypeFp32;
  const int H = 12, d = 64, seq = 256, pos = 255, kv_dim = H * d;
  std::vector<float> q = normal(kv_dim, 21), kc = normal((size_t)seq * kv_dim, 22),
                     vc = normal((size_t)seq * kv_dim, 23);
  DevTensor qd(q, {kv_dim}, dt), kd(kc, {1, seq, kv_dim}, dt), vd(vc, {1, seq, kv_dim}, dt),
      sd((size_t)H * seq, {H, seq}, dt), od((size_t)kv_dim, {kv_dim}, dt);
  op::MultiHeadAttention mha(DeviceType::kDeviceCUDA, 0, 1, kv_dim, seq, H, d);
  mha.set_cuda_config(std::make_shared<kernel::CudaConfig>());
  mha.set_pos(pos);
  mha.set_input(0, qd.t);
  mha.set_input(1, sd.t);
  mha.set_input(2, kd.t);
  mha.set_input(3, vd.t);
  mha.set_output(0, od.t);
  ASSERT_TRUE(static_cast<bool>(mha.forward()));
  ASSERT_TRUE(hipDeviceSynchronize() == hipSuccess);
  std::vector<float> ref(kv_dim), score((size_t)H * seq);
  oracle_mha_kernel(pos, H, 0, seq, kv_dim, 1, d, ref.data(), q.data(), score.data(), kc.data(),
                    vc.data());
  EXPECT_TRUE(close(download(od.buf, kv_dim, dt), ref, 1e-5f, 1e-4f, "fp32 mha"));
}

TEST(GpuVisionLayers, SplitRopeTransposeThenAttentionBf16) {
  ASSERT_TRUE(gpu_ok());
  const DataType dt = DataType::kDataTypeBf16;
  const int gh = 16, gw = 20, N = gh * gw, H = 4, d = 72;
  std::vector<float> qkv = normal((size_t)N * 3 * H * d, 31);
  std::vector<float> cs((size_t)N * d), sn((size_t)N * d);
  oracle_vision_cos_sin(1, gh, gw, 2, d, cs.data(), sn.data());
  DevTensor qkvd(qkv, {N, 3 * H * d}, dt), cd(cs, {N, d}, dt), sd(sn, {N, d}, dt);
  DevTensor qt((size_t)H * N * d, {H, N, d}, dt), kt((size_t)H * N * d, {H, N, d}, dt),
      vt((size_t)H * N * d, {H, N, d}, dt), out((size_t)N * H * d, {N, H * d}, dt);
  op::FusedSplitRopeTransposeLayer split(DeviceType::kDeviceCUDA);
  ASSERT_TRUE(static_cast<bool>(split.forward(qkvd.t, cd.t, sd.t, qt.t, kt.t, vt.t, N, H, d)));
  op::VisionAttentionLayer attn(DeviceType::kDeviceCUDA);
  kernel::CudaConfig cfg;
  ASSERT_TRUE(static_cast<bool>(attn.forward(qt.t, kt.t, vt.t, out.t, Tensor(), Tensor(), N, H,
                                              d, 1.f / std::sqrt((float)d), &cfg)));
  ASSERT_TRUE(hipDeviceSynchronize() == hipSuccess);
  // Oracle: split to [H, N, d], rotate q and k with the rounded tables, attend.
  std::vector<float> x[3];
  for (int w = 0; w < 3; ++w) {
    x[w].resize((size_t)H * N * d);
    for (int h = 0; h < H; ++h)
      for (int t = 0; t < N; ++t)
        for (int j = 0; j < d; ++j)
          x[w][((size_t)h * N + t) * d + j] = qkv[(size_t)t * 3 * H * d + (size_t)w * H * d + h * d + j];
  }
  oracle_vision_rotary(x[0].data(), H, N, d, cs.data(), sn.data());
  oracle_vision_rotary(x[1].data(), H, N, d, cs.data(), sn.data());
  // The device rounds the rotated q/k to bf16 before attention; the oracle does too.
  quantize(x[0], dt);
  quantize(x[1], dt);
  EXPECT_TRUE(close(download(vt.buf, (size_t)H * N * d, dt), x[2], 0.f, 0.f, "v passthrough"));
  std::vector<float> ref((size_t)N * H * d);
  const int cu[2] = {0, N};
  oracle_varlen_bidir(N, H, d, 1.f / std::sqrt((float)d), x[0].data(), x[1].data(), x[2].data(),
                      cu, 1, ref.data(), 8);
  EXPECT_TRUE(close(download(out.buf, (size_t)N * H * d, dt), ref, 2e-3f, 1e-2f, "vision"));
}

TEST(GpuCopyToKVCacheLayer, Fp16RowLandsAtDevicePosition) {
  ASSERT_TRUE(gpu_ok());
  const DataType dt = DataType::kDataTypeFp16;
  const int layers = 2, seq = 64, kv_dim = 1024, layer = 1, pos = 41;
  std::vector<float> row = normal(kv_dim, 41);
  DevTensor src(row, {kv_dim}, dt), cache((size_t)layers * seq * kv_dim, {layers, seq, kv_dim}, dt);
  DevBuf posd(4);
  (void)hipMemcpy(posd.p, &pos, 4, hipMemcpyHostToDevice);
  op::CopyToKVCacheLayer cp(DeviceType::kDeviceCUDA);
  ASSERT_TRUE(static_cast<bool>(cp.forward(cache.t, src.t, (const int32_t*)posd.p, kv_dim, layer, seq)));
  ASSERT_TRUE(hipDeviceSynchronize() == hipSuccess);
  std::vector<float> all = download(cache.buf, (size_t)layers * seq * kv_dim, dt);
  std::vector<float> want((size_t)layers * seq * kv_dim, 0.f);
  std::copy(row.begin(), row.end(), want.begin() + ((size_t)layer * seq + pos) * kv_dim);
  EXPECT_TRUE(close(all, want, 0.f, 0.f, "kv cache row"));
}

TEST(GpuKernels, Fp16WoProjectionMatchesFp32Reference) {
  // batched_matmul_kernel_cu_pure_fp16 (the wo projection): out = 0.5 * in . w^T.
  ASSERT_TRUE(gpu_ok());
  const DataType dt = DataType::kDataTypeFp16;
  const int B = 64, in_dim = 256, out_dim = 128;
  std::vector<float> xh = normal((size_t)B * in_dim, 51), wh = normal((size_t)out_dim * in_dim, 52);
  DevTensor x(xh, {B, in_dim}, dt), w(wh, {out_dim, in_dim}, dt);
  DevTensor o((size_t)B * out_dim, {B, out_dim}, dt);
  kernel::CudaConfig cfg;
  kernel::batched_matmul_kernel_cu_pure_fp16(x.t, w.t, o.t, B, 0.5f, &cfg);
  ASSERT_TRUE(static_cast<bool>(kernel::last_status()));
  ASSERT_TRUE(hipDeviceSynchronize() == hipSuccess);
  const std::vector<float>& xs = xh;  // rounded to fp16 by DevTensor
  const std::vector<float>& ws = wh;
  std::vector<float> ref((size_t)B * out_dim);
  for (int b = 0; b < B; ++b)
    for (int k = 0; k < out_dim; ++k) {
      double acc = 0;
      for (int m = 0; m < in_dim; ++m) acc += (double)xs[(size_t)b * in_dim + m] * ws[(size_t)k * in_dim + m];
      ref[(size_t)b * out_dim + k] = (float)(0.5 * acc);
    }
  EXPECT_TRUE(close(download(o.buf, (size_t)B * out_dim, dt), ref, 2e-2f, 1e-2f, "wo"));
}

int main(int argc, char** argv) { return mini_test::run_all(argc, argv); }
