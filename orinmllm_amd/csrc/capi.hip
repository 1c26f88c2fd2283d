// extern "C" entry points of liborin_attn.so (declared in include/orin_attn.h).
// Argument checking, the per-call launch shape (split-KV sizing) and the
// library-owned decode workspace live here; the kernels are in decode.hip and fwd.hip.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"
#include "orin_attn.h"

using namespace orin;

namespace {

thread_local std::string g_last_hip_error;

int hip_status(hipError_t e) {
  if (e == hipSuccess) return ORIN_OK;
  g_last_hip_error = hipGetErrorString(e);
  return ORIN_ERR_LAUNCH;
}

float resolve_scale(float scale, int head_size) {
  return scale > 0.f ? scale : 1.0f / sqrtf((float)head_size);
}

int round_up(long x, int m) { return (int)((x + m - 1) / m * m); }

// The combine kernel merges at most this many splits per row.
constexpr int kMaxSplits = 1024;

int device_cus();

// Tokens per split for a decode launch with `base_blocks` (row, kv head, head group)
// units and rows of up to max_len tokens.
//  * At least one unit per CU: whole rows (one split), so no partials and no merge launch.
//    Each unit is then one workgroup that streams its row (for 16-bit caches at head size
//    64 / 128 on the matrix-core kernel).  Batch 32 x 8 kv heads (fp16, d 128): every
//    length 4096 0.76-0.77 of HBM against 0.66 with 320-token splits; lengths U[512, 4096]
//    0.64 against 0.62-0.63 with 320-token splits plus their merge.
//  * Fewer units: aims at ~3328 workgroups (13 per CU, i.e. about 3.25 rounds of the 4
//    resident per CU; measured best on the batch-32 paged decode) with at least 256 tokens
//    (one 64-token tile per wave) per split.
int auto_split_tokens(long base_blocks, int max_len) {
  if (max_len <= 0) return 256;
  if (base_blocks >= device_cus()) return round_up(max_len, 64);
  const long target = 3328;
  long splits = (target + base_blocks - 1) / base_blocks;
  if (splits < 1) splits = 1;
  int st = round_up((max_len + splits - 1) / splits, 64);
  if (st < 256) st = 256;
  if (st >= max_len) st = round_up(max_len, 64);
  while ((max_len + st - 1) / st > kMaxSplits) st *= 2;
  return st;
}

long decode_base_blocks(int rows, int head_num, int kv_head_num) {
  const int kv_mul = head_num / kv_head_num;
  return (long)rows * kv_head_num * (kv_mul / decode_heads_per_block(kv_mul));
}

int n_splits(int max_len, int split_tokens) {
  return max_len <= 0 ? 1 : (max_len + split_tokens - 1) / split_tokens;
}

size_t ws_bytes(int rows, int head_num, int head_size, int splits) {
  return splits <= 1 ? 0 : (size_t)rows * head_num * splits * (head_size + 2) * sizeof(float);
}

bool heads_ok(int head_num, int kv_head_num, int kv_mul) {
  return head_num > 0 && kv_head_num > 0 && kv_mul > 0 && head_num == kv_head_num * kv_mul;
}

// Library-owned workspaces.  The kuiper-shaped flash decode and the causal prefill key
// split take no workspace argument, so the library keeps one grow-only buffer per
// (device, stream, kind): calls on different streams never share bytes, and the decode
// partials never share a buffer with the prefill key split.  A buffer that has to grow is
// retired, not freed: a captured graph may still hold its address, so it stays allocated
// until orin_attn_workspace_release.  Nothing here synchronises a stream or the device,
// and a stream that is capturing gets ORIN_ERR_WORKSPACE instead of an allocation.
enum WsKind { kWsDecode = 0, kWsPrefillSplit = 1 };

struct WsSlot {
  int dev;
  void* stream;
  int kind;
  void* ptr;
  size_t bytes;
};

std::mutex g_ws_mu;
std::vector<WsSlot> g_ws;                          // live buffers
struct WsRetired {
  int dev;
  void* stream;
  void* ptr;
};
std::vector<WsRetired> g_ws_retired;               // grown-out buffers kept for graphs
std::vector<size_t> g_ws_floor;                    // per device: minimum decode buffer size

// Grow geometrically so that a sequence of slightly larger calls retires few buffers.
size_t grown_size(size_t have, size_t need) {
  size_t n = have ? have : 1;
  while (n < need) n *= 2;
  return n < need ? need : n;
}

// hipMalloc with this thread in relaxed capture mode: a stream that another thread is
// capturing in global mode is then not invalidated by the allocation.
hipError_t relaxed_malloc(void** p, size_t bytes) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
  if (e != hipSuccess) return e;
  e = hipMalloc(p, bytes);
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  return e;
}

// True when `stream` is being captured (the null stream never is).
bool capturing(void* stream) {
  if (!stream) return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing((hipStream_t)stream, &cs) == hipSuccess &&
         cs != hipStreamCaptureStatusNone;
}

int library_workspace(int kind, hipStream_t stream, size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) return ORIN_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  WsSlot* slot = nullptr;
  for (auto& w : g_ws)
    if (w.dev == dev && w.stream == (void*)stream && w.kind == kind) slot = &w;
  if (slot && slot->bytes >= bytes) {
    *out = slot->ptr;
    return ORIN_OK;
  }
  // Allocation needed: refuse while this stream is being captured (the caller reserves
  // with orin_attn_workspace_reserve_stream before capturing).
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (stream != nullptr) {
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_status(e);
  }
  if (cs != hipStreamCaptureStatusNone) return ORIN_ERR_WORKSPACE;
  size_t want = grown_size(slot ? slot->bytes : 0, bytes);
  if (kind == kWsDecode && dev < (int)g_ws_floor.size() && g_ws_floor[dev] > want)
    want = g_ws_floor[dev];
  void* p = nullptr;
  e = relaxed_malloc(&p, want);
  if (e != hipSuccess) return hip_status(e);
  if (slot) {
    g_ws_retired.push_back({dev, slot->stream, slot->ptr});
    slot->ptr = p;
    slot->bytes = want;
  } else {
    g_ws.push_back({dev, (void*)stream, kind, p, want});
  }
  *out = p;
  return ORIN_OK;
}

// Compute units of the current device (cached per process; 256 if the query fails).
int device_cus() {
  static const int cached = [] {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    return cus;
  }();
  return cached;
}

DecodeArgs decode_defaults() {
  DecodeArgs a = {};
  a.max_splits = 1;
  a.split_tokens = 1 << 30;
  return a;
}

// Split size for a kuiper single-sequence decode whose workspace must fit in
// cap_bytes (0 = unlimited).
int kuiper_decode_split(int head_num, int kv_head_num, int head_size, int max_len,
                        size_t cap_bytes, bool capped) {
  int st = auto_split_tokens(decode_base_blocks(1, head_num, kv_head_num), max_len);
  while (capped && n_splits(max_len, st) > 1 &&
         ws_bytes(1, head_num, head_size, n_splits(max_len, st)) > cap_bytes)
    st *= 2;
  while (n_splits(max_len, st) > kMaxSplits) st *= 2;
  return st;
}

// max_len: the longest row the launch must cover (0 = rows are single-split by
// construction).  Rows are clamped to max_splits * split_tokens tokens.
int run_decode(DecodeArgs& a, int dtype, int max_len, hipStream_t stream) {
  a.max_splits = n_splits(max_len, a.split_tokens);
  if (a.max_splits <= 1) a.max_splits = 1;
  // Dot-product kernel: 16-wave workgroups (where the shape fits) when each (row, kv head,
  // head group) is one split, or when the launch has no more workgroups than the device has
  // CUs: 4-wave workgroups would then leave most wave slots idle.
  const long units = (long)a.n_rows * a.Hkv * (a.kv_mul / decode_heads_per_block(a.kv_mul));
  a.wide = a.max_splits == 1 || units * a.max_splits <= device_cus();
  // Whole rows of a launch with a (row, kv head) per CU or more: matrix-core kernel.  The
  // single-sequence (kuiper) decode never qualifies, so its result does not depend on
  // whether the launch was sized for the position or for the cache capacity.
  a.mfma = a.max_splits == 1 && (long)a.n_rows * a.Hkv >= device_cus();
  a.len_cap = max_len > 0 ? max_len : (1 << 30);
  return hip_status(launch_decode(a, dtype, stream));
}

}  // namespace

extern "C" {

int orin_attn_abi_version(void) { return ORIN_ATTN_ABI_VERSION; }

const char* orin_attn_status_string(int status) {
  switch (status) {
    case ORIN_OK: return "ok";
    case ORIN_ERR_INVALID_ARG: return "invalid argument";
    case ORIN_ERR_UNSUPPORTED: return "unsupported dtype/head_size/block_size";
    case ORIN_ERR_WORKSPACE: return "workspace missing or too small";
    case ORIN_ERR_LAUNCH: return "HIP launch or allocation error";
  }
  return "unknown status";
}

const char* orin_attn_last_hip_error(void) { return g_last_hip_error.c_str(); }

int orin_attn_workspace_reserve(size_t bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if ((int)g_ws_floor.size() <= dev) g_ws_floor.resize(dev + 1, 0);
    if (g_ws_floor[dev] < bytes) g_ws_floor[dev] = bytes;
  }
  void* p;
  return library_workspace(kWsDecode, nullptr, bytes, &p);
}

int orin_attn_workspace_reserve_stream(size_t decode_bytes, size_t prefill_bytes, void* stream) {
  void* p;
  int st = library_workspace(kWsDecode, (hipStream_t)stream, decode_bytes, &p);
  if (st != ORIN_OK) return st;
  st = library_workspace(kWsPrefillSplit, (hipStream_t)stream, prefill_bytes, &p);
  if (st != ORIN_OK) return st;
  // The output projection's rocBLAS handle and workspace, so that a capture of it on this
  // device allocates nothing.
  return output_projection_prepare() == 0 ? ORIN_OK : ORIN_ERR_LAUNCH;
}

// Frees the library-owned buffers of the current device that belong to `stream` (all
// streams when all_streams), after synchronising what may still use them.  Refused while
// one of those streams is being captured.
static int release_buffers(bool all_streams, void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto mine = [&](int d, void* s) { return d == dev && (all_streams || s == stream); };
  for (const auto& w : g_ws)
    if (mine(w.dev, w.stream) && capturing(w.stream)) return ORIN_ERR_WORKSPACE;
  e = all_streams ? hipDeviceSynchronize() : hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_status(e);
  for (auto it = g_ws.begin(); it != g_ws.end();) {
    if (mine(it->dev, it->stream)) {
      (void)hipFree(it->ptr);
      it = g_ws.erase(it);
    } else {
      ++it;
    }
  }
  for (auto it = g_ws_retired.begin(); it != g_ws_retired.end();) {
    if (mine(it->dev, it->stream)) {
      (void)hipFree(it->ptr);
      it = g_ws_retired.erase(it);
    } else {
      ++it;
    }
  }
  if (all_streams && dev < (int)g_ws_floor.size()) g_ws_floor[dev] = 0;
  return ORIN_OK;
}

int orin_attn_workspace_release(void) { return release_buffers(true, nullptr); }

int orin_attn_workspace_release_stream(void* stream) { return release_buffers(false, stream); }

// ------------------------------------------------------------------ fp32 MHA

static int mha_common(int32_t pos, const int32_t* pos_ptr, int32_t head_num, int32_t layer_index,
                      int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                      float* mha_out, const float* query, float* score, const float* key_cache,
                      const float* value_cache, void* stream) {
  if (head_size <= 0 || seq_len <= 0 || kv_dim <= 0 || layer_index < 0 || kv_dim % head_size)
    return ORIN_ERR_INVALID_ARG;
  const int kv_head_num = kv_dim / head_size;
  if (!heads_ok(head_num, kv_head_num, kv_mul)) return ORIN_ERR_INVALID_ARG;
  if (!mha_out || !query || !key_cache || !value_cache) return ORIN_ERR_INVALID_ARG;
  if (!pos_ptr && (pos < 0 || pos >= seq_len)) return ORIN_ERR_INVALID_ARG;
  if (!decode_supports(kF32, head_size)) return ORIN_ERR_UNSUPPORTED;
  const size_t cap = score ? (size_t)head_num * seq_len * sizeof(float) : 0;
  // Host position: size the split for pos+1 keys; device position: for the capacity.
  const int max_len = pos_ptr ? seq_len : pos + 1;
  DecodeArgs a = decode_defaults();
  a.split_tokens = kuiper_decode_split(head_num, kv_head_num, head_size, max_len, cap, true);
  const long layer_off = (long)layer_index * seq_len * kv_dim;
  a.q = query;
  a.q_row_stride = (long)head_num * head_size;
  a.q_head_stride = head_size;
  a.k = key_cache + layer_off;
  a.v = value_cache + layer_off;
  a.kv_tok_stride = kv_dim;
  a.kv_head_stride = head_size;
  if (pos_ptr) {
    a.lens = pos_ptr;
    a.len_add = 1;
  } else {
    a.len_base = pos + 1;
  }
  a.o = mha_out;
  a.o_row_stride = (long)head_num * head_size;
  a.o_head_stride = head_size;
  a.ws = score;
  a.n_rows = 1;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = kv_mul;
  a.head_size = head_size;
  a.scale_log2 = resolve_scale(0.f, head_size) * kLog2e;
  if (n_splits(max_len, a.split_tokens) > 1 && !score) return ORIN_ERR_WORKSPACE;
  return run_decode(a, kF32, max_len, (hipStream_t)stream);
}

int orin_mha_kernel(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                    int32_t kv_dim, int32_t kv_mul, int32_t head_size, float* mha_out,
                    const float* query, float* score, const float* key_cache,
                    const float* value_cache, void* stream) {
  return mha_common(pos, nullptr, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                    mha_out, query, score, key_cache, value_cache, stream);
}

int orin_mha_kernel_gpu_pos(const int32_t* pos_ptr, int32_t head_num, int32_t layer_index,
                            int32_t seq_len, int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                            float* mha_out, const float* query, float* score,
                            const float* key_cache, const float* value_cache, void* stream) {
  if (!pos_ptr) return ORIN_ERR_INVALID_ARG;
  return mha_common(0, pos_ptr, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                    mha_out, query, score, key_cache, value_cache, stream);
}

// Causal prefill on the per-row kernel (fp32, or any dtype the MFMA path lacks).
static int prefill_rows(int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t kv_head_num,
                        int32_t head_size, int32_t kv_mul, const void* query, void* output,
                        const void* k, const void* v, int32_t kv_dim, int dtype,
                        hipStream_t stream) {
  DecodeArgs a = decode_defaults();
  a.q = query;
  a.q_row_stride = (long)head_num * head_size;
  a.q_head_stride = head_size;
  a.k = k;
  a.v = v;
  a.kv_tok_stride = kv_dim;
  a.kv_head_stride = head_size;
  a.len_base = start_pos + 1;
  a.len_step = 1;
  a.o = output;
  a.o_row_stride = (long)head_num * head_size;
  a.o_head_stride = head_size;
  a.n_rows = seq_len;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = kv_mul;
  a.head_size = head_size;
  a.scale_log2 = resolve_scale(0.f, head_size) * kLog2e;
  return run_decode(a, dtype, 0, stream);
}

int orin_batched_mha(int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t layer_index,
                     int32_t max_seq_len, int32_t dim, int32_t kv_dim, int32_t kv_mul,
                     int32_t head_size, float* mha_out, const float* query, float* score,
                     const float* key_cache, const float* value_cache, void* stream) {
  (void)score;
  if (head_size <= 0 || seq_len <= 0 || max_seq_len <= 0 || kv_dim <= 0 || start_pos < 0 ||
      layer_index < 0 || kv_dim % head_size || dim != head_num * head_size ||
      start_pos + seq_len > max_seq_len)
    return ORIN_ERR_INVALID_ARG;
  const int kv_head_num = kv_dim / head_size;
  if (!heads_ok(head_num, kv_head_num, kv_mul)) return ORIN_ERR_INVALID_ARG;
  if (!mha_out || !query || !key_cache || !value_cache) return ORIN_ERR_INVALID_ARG;
  if (!decode_supports(kF32, head_size)) return ORIN_ERR_UNSUPPORTED;
  const long layer_off = (long)layer_index * max_seq_len * kv_dim;
  return prefill_rows(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, query,
                      mha_out, key_cache + layer_off, value_cache + layer_off, kv_dim, kF32,
                      (hipStream_t)stream);
}

// ------------------------------------------------------------------ flash attention

static size_t elem_size(int dtype) { return dtype == kF32 ? 4 : 2; }

static int prefill_common(int32_t start_pos, int32_t seq_len, int32_t head_num,
                          int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                          int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                          const void* query, void* output, const void* key_cache,
                          const void* value_cache, int32_t dtype, void* stream,
                          const void* q_norm_weight, const float* rope_sin,
                          const float* rope_cos, float eps) {
  if (head_size <= 0 || seq_len <= 0 || max_seq_len <= 0 || start_pos < 0 || layer_index < 0 ||
      kv_dim != kv_head_num * head_size || start_pos + seq_len > max_seq_len)
    return ORIN_ERR_INVALID_ARG;
  if (!heads_ok(head_num, kv_head_num, kv_mul)) return ORIN_ERR_INVALID_ARG;
  if (!query || !output || !key_cache || !value_cache) return ORIN_ERR_INVALID_ARG;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return ORIN_ERR_UNSUPPORTED;
  const size_t layer_off = (size_t)layer_index * max_seq_len * kv_dim * elem_size(dtype);
  const char* k = static_cast<const char*>(key_cache) + layer_off;
  const char* v = static_cast<const char*>(value_cache) + layer_off;
  const bool fused = rope_sin != nullptr;
  if (dtype == kF32) {
    if (fused || !decode_supports(kF32, head_size)) return ORIN_ERR_UNSUPPORTED;
    return prefill_rows(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, query,
                        output, k, v, kv_dim, kF32, (hipStream_t)stream);
  }
  if (!fwd_supports(dtype, head_size)) return ORIN_ERR_UNSUPPORTED;
  FwdArgs a = {};
  a.q = query;
  a.q_tok_stride = (long)head_num * head_size;
  a.q_head_stride = head_size;
  a.k = k;
  a.v = v;
  a.kv_tok_stride = kv_dim;
  a.kv_head_stride = head_size;
  a.o = output;
  a.o_tok_stride = (long)head_num * head_size;
  a.o_head_stride = head_size;
  a.n_q = seq_len;
  a.start_pos = start_pos;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = kv_mul;
  a.head_size = head_size;
  a.scale_log2 = resolve_scale(0.f, head_size) * kLog2e;
  if (fused) {
    // The fused Q producer runs in the ping-pong kernel's Q load (head sizes 64 and 128);
    // it reads the raw query while other rows' outputs are written, so no aliasing.
    if ((head_size != 64 && head_size != 128) || !fwd_pp_supports(a, dtype))
      return ORIN_ERR_UNSUPPORTED;
    if (query == output || !rope_cos || !(eps >= 0.f)) return ORIN_ERR_INVALID_ARG;
    a.q_norm_weight = q_norm_weight;
    a.rope_sin = rope_sin;
    a.rope_cos = rope_cos;
    a.eps = eps;
  }
  // Too few query blocks to fill the device: split their keys (library workspace).
  size_t split_bytes = 0;
  const int chunk = fwd_pp_key_split(a, dtype, device_cus(), &split_bytes);
  if (chunk > 0) {
    void* ws = nullptr;
    const int st = library_workspace(kWsPrefillSplit, (hipStream_t)stream, split_bytes, &ws);
    if (st != ORIN_OK) return st;
    a.key_chunk_tiles = chunk;
    a.ws = static_cast<float*>(ws);
  }
  return hip_status(launch_fwd_causal(a, dtype, (hipStream_t)stream));
}

int orin_flash_attention_prefill(int32_t start_pos, int32_t seq_len, int32_t head_num,
                                 int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                                 int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                                 const void* query, void* output, const void* key_cache,
                                 const void* value_cache, int32_t dtype, void* stream) {
  return prefill_common(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul,
                        layer_index, max_seq_len, kv_dim, query, output, key_cache, value_cache,
                        dtype, stream, nullptr, nullptr, nullptr, 0.f);
}

int orin_flash_attention_prefill_qk_norm_rope(
    int32_t start_pos, int32_t seq_len, int32_t head_num, int32_t kv_head_num, int32_t head_size,
    int32_t kv_mul, int32_t layer_index, int32_t max_seq_len, int32_t kv_dim, const void* query,
    void* output, const void* key_cache, const void* value_cache, const void* q_norm_weight,
    const float* sin_cache, const float* cos_cache, float eps, int32_t dtype, void* stream) {
  if (!sin_cache || !cos_cache) return ORIN_ERR_INVALID_ARG;
  return prefill_common(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul,
                        layer_index, max_seq_len, kv_dim, query, output, key_cache, value_cache,
                        dtype, stream, q_norm_weight, sin_cache, cos_cache, eps);
}

// Partials of orin_flash_attention_decode_gpu_pos_noalloc: a fixed device array, so that
// entry point never allocates.  In host code `scratch` names a host-side stand-in, not
// device memory: its device address is looked up once per device (noalloc_scratch) and
// only that address is passed to kernels.
static constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_ptr;  // per device: device address of `scratch`, or null

static int noalloc_scratch(void** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e);
    if (!p) return ORIN_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ORIN_OK;
}

// noalloc: take the partials from the device's static scratch array instead of the
// library-owned buffer (no allocation; ORIN_ERR_WORKSPACE if they do not fit).
static int flash_decode_common(int32_t pos, const int32_t* pos_ptr, int32_t head_num,
                               int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                               int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                               const void* query, void* output, const void* key_cache,
                               const void* value_cache, int32_t dtype, void* stream,
                               bool noalloc = false) {
  if (head_size <= 0 || max_seq_len <= 0 || layer_index < 0 || kv_dim != kv_head_num * head_size)
    return ORIN_ERR_INVALID_ARG;
  if (!heads_ok(head_num, kv_head_num, kv_mul)) return ORIN_ERR_INVALID_ARG;
  if (!query || !output || !key_cache || !value_cache) return ORIN_ERR_INVALID_ARG;
  if (!pos_ptr && (pos < 0 || pos >= max_seq_len)) return ORIN_ERR_INVALID_ARG;
  if (!decode_supports(dtype, head_size)) return ORIN_ERR_UNSUPPORTED;
  const int max_len = pos_ptr ? max_seq_len : pos + 1;
  DecodeArgs a = decode_defaults();
  a.split_tokens = kuiper_decode_split(head_num, kv_head_num, head_size, max_len, 0, false);
  const int splits = n_splits(max_len, a.split_tokens);
  const size_t need = ws_bytes(1, head_num, head_size, splits);
  void* ws = nullptr;
  int st;
  if (noalloc) {
    if (need > kNoAllocScratchBytes) return ORIN_ERR_WORKSPACE;
    st = noalloc_scratch(&ws);
  } else {
    st = library_workspace(kWsDecode, (hipStream_t)stream, need, &ws);
  }
  if (st != ORIN_OK) return st;
  const size_t layer_off = (size_t)layer_index * max_seq_len * kv_dim * elem_size(dtype);
  a.q = query;
  a.q_row_stride = (long)head_num * head_size;
  a.q_head_stride = head_size;
  a.k = static_cast<const char*>(key_cache) + layer_off;
  a.v = static_cast<const char*>(value_cache) + layer_off;
  a.kv_tok_stride = kv_dim;
  a.kv_head_stride = head_size;
  if (pos_ptr) {
    a.lens = pos_ptr;
    a.len_add = 1;
  } else {
    a.len_base = pos + 1;
  }
  a.o = output;
  a.o_row_stride = (long)head_num * head_size;
  a.o_head_stride = head_size;
  a.ws = static_cast<float*>(ws);
  a.n_rows = 1;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = kv_mul;
  a.head_size = head_size;
  a.scale_log2 = resolve_scale(0.f, head_size) * kLog2e;
  return run_decode(a, dtype, max_len, (hipStream_t)stream);
}

int orin_flash_attention_decode(int32_t pos, int32_t head_num, int32_t kv_head_num,
                                int32_t head_size, int32_t kv_mul, int32_t layer_index,
                                int32_t max_seq_len, int32_t kv_dim, const void* query,
                                void* output, const void* key_cache, const void* value_cache,
                                int32_t dtype, void* stream) {
  return flash_decode_common(pos, nullptr, head_num, kv_head_num, head_size, kv_mul, layer_index,
                             max_seq_len, kv_dim, query, output, key_cache, value_cache, dtype,
                             stream);
}

int orin_flash_attention_decode_gpu_pos(const int32_t* pos_ptr, int32_t head_num,
                                        int32_t kv_head_num, int32_t head_size, int32_t kv_mul,
                                        int32_t layer_index, int32_t max_seq_len, int32_t kv_dim,
                                        const void* query, void* output, const void* key_cache,
                                        const void* value_cache, int32_t dtype, void* stream) {
  if (!pos_ptr) return ORIN_ERR_INVALID_ARG;
  return flash_decode_common(0, pos_ptr, head_num, kv_head_num, head_size, kv_mul, layer_index,
                             max_seq_len, kv_dim, query, output, key_cache, value_cache, dtype,
                             stream);
}

int orin_flash_attention_decode_gpu_pos_noalloc(const int32_t* pos_ptr, int32_t head_num,
                                                int32_t kv_head_num, int32_t head_size,
                                                int32_t kv_mul, int32_t layer_index,
                                                int32_t max_seq_len, int32_t kv_dim,
                                                const void* query, void* output,
                                                const void* key_cache, const void* value_cache,
                                                int32_t dtype, void* stream) {
  if (!pos_ptr) return ORIN_ERR_INVALID_ARG;
  return flash_decode_common(0, pos_ptr, head_num, kv_head_num, head_size, kv_mul, layer_index,
                             max_seq_len, kv_dim, query, output, key_cache, value_cache, dtype,
                             stream, true);
}

size_t orin_flash_attention_decode_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

size_t orin_flash_attention_decode_workspace_size(int32_t head_num, int32_t head_size,
                                                  int32_t max_seq_len) {
  if (head_num <= 0 || head_size <= 0 || max_seq_len <= 0) return 0;
  // Worst case over kv_head_num: the split size shrinks as the unit count drops,
  // so size for kv_head_num = 1.
  const int st = auto_split_tokens(decode_base_blocks(1, 1, 1), max_seq_len);
  return ws_bytes(1, head_num, head_size, n_splits(max_seq_len, st));
}

size_t orin_flash_attention_prefill_workspace_size(int32_t start_pos, int32_t seq_len,
                                                   int32_t head_num, int32_t kv_head_num,
                                                   int32_t head_size, int32_t dtype) {
  if (seq_len <= 0 || start_pos < 0 || head_size <= 0 || kv_head_num <= 0 || head_num <= 0 ||
      head_num % kv_head_num || (dtype != kF16 && dtype != kBF16))
    return 0;
  FwdArgs a = {};
  a.q_tok_stride = a.o_tok_stride = (long)head_num * head_size;
  a.q_head_stride = a.o_head_stride = a.kv_head_stride = head_size;
  a.kv_tok_stride = (long)kv_head_num * head_size;
  a.n_q = seq_len;
  a.start_pos = start_pos;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = head_num / kv_head_num;
  a.head_size = head_size;
  size_t bytes = 0;
  (void)fwd_pp_key_split(a, dtype, device_cus(), &bytes);
  return bytes;
}

// ------------------------------------------------------------------ batched decode

int32_t orin_attn_decode_split_tokens(int32_t batch, int32_t head_num, int32_t kv_head_num,
                                      int32_t max_context_len, int32_t split_tokens) {
  if (split_tokens > 0) return split_tokens;
  if (batch <= 0 || kv_head_num <= 0 || head_num % kv_head_num) return 0;
  return auto_split_tokens(decode_base_blocks(batch, head_num, kv_head_num), max_context_len);
}

int32_t orin_attn_decode_split_tokens_for_total(int32_t batch, int32_t head_num,
                                                int32_t kv_head_num, int32_t max_context_len,
                                                int64_t sum_context_len) {
  if (batch <= 0 || max_context_len < 0 || sum_context_len < 0 ||
      !heads_ok(head_num, kv_head_num, kv_head_num > 0 ? head_num / kv_head_num : 0))
    return 0;
  const int automatic = orin_attn_decode_split_tokens(batch, head_num, kv_head_num,
                                                      max_context_len, 0);
  if (max_context_len == 0 || sum_context_len * 10 < (int64_t)batch * max_context_len * 9)
    return automatic;
  // Near-uniform rows.  A batch with a unit per CU or more already gets whole rows.
  const long base = decode_base_blocks(batch, head_num, kv_head_num);
  const long cus = device_cus();
  if (base >= cus) return automatic;
  // Otherwise one round of the 4-wave workgroups resident at once (4 per CU), e.g. at
  // batch 8, 8 kv heads, 4096 tokens 256-token splits.
  long per_row = cus * 4 / base;
  if (per_row < 1) per_row = 1;
  int st = round_up((max_context_len + per_row - 1) / per_row, 64);
  while (n_splits(max_context_len, st) > kMaxSplits) st *= 2;
  return st;
}

size_t orin_attn_decode_workspace_size(int32_t batch, int32_t head_num, int32_t kv_head_num,
                                       int32_t head_size, int32_t max_context_len,
                                       int32_t split_tokens) {
  const int st =
      orin_attn_decode_split_tokens(batch, head_num, kv_head_num, max_context_len, split_tokens);
  if (st <= 0 || head_size <= 0) return 0;
  return ws_bytes(batch, head_num, head_size, n_splits(max_context_len, st));
}

static int batched_decode(const void* query, const void* k, const void* v, void* out,
                          int32_t batch, int32_t head_num, int32_t kv_head_num, int32_t head_size,
                          int64_t batch_stride, int64_t tok_stride, int64_t head_stride,
                          int64_t block_stride, const int32_t* block_tables,
                          int32_t max_blocks, int32_t block_size, const int32_t* context_lens,
                          int32_t max_context_len, int32_t dtype, float scale,
                          int32_t split_tokens, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (batch <= 0 || head_size <= 0 || max_context_len < 0 || split_tokens < 0 ||
      kv_head_num <= 0 || head_num <= 0 || head_num % kv_head_num)
    return ORIN_ERR_INVALID_ARG;
  if (!query || !k || !v || !out || !context_lens) return ORIN_ERR_INVALID_ARG;
  if (!decode_supports(dtype, head_size)) return ORIN_ERR_UNSUPPORTED;
  int bs_log2 = 0;
  if (split_tokens % 64) return ORIN_ERR_INVALID_ARG;
  if (block_tables) {
    if (block_size <= 0 || max_blocks <= 0 || (long)max_blocks * block_size < max_context_len)
      return ORIN_ERR_INVALID_ARG;
    // Each 8-token step of the kernel must lie inside one block.
    if ((block_size & (block_size - 1)) || block_size < 8) return ORIN_ERR_UNSUPPORTED;
    while ((1 << bs_log2) < block_size) ++bs_log2;
  }
  const int st =
      orin_attn_decode_split_tokens(batch, head_num, kv_head_num, max_context_len, split_tokens);
  if (n_splits(max_context_len, st) > kMaxSplits) return ORIN_ERR_INVALID_ARG;
  const size_t need = ws_bytes(batch, head_num, head_size, n_splits(max_context_len, st));
  if (need > 0 && (!workspace || workspace_bytes < need)) return ORIN_ERR_WORKSPACE;
  DecodeArgs a = decode_defaults();
  a.split_tokens = st;
  a.q = query;
  a.q_row_stride = (long)head_num * head_size;
  a.q_head_stride = head_size;
  a.k = k;
  a.v = v;
  a.kv_tok_stride = tok_stride;
  a.kv_head_stride = head_stride;
  a.kv_row_stride = batch_stride;
  a.block_table = block_tables;
  a.block_stride = block_stride;
  a.bt_row_stride = max_blocks;
  a.bs_log2 = bs_log2;
  a.lens = context_lens;
  a.o = out;
  a.o_row_stride = (long)head_num * head_size;
  a.o_head_stride = head_size;
  a.ws = static_cast<float*>(workspace);
  a.n_rows = batch;
  a.Hq = head_num;
  a.Hkv = kv_head_num;
  a.kv_mul = head_num / kv_head_num;
  a.head_size = head_size;
  a.scale_log2 = resolve_scale(scale, head_size) * kLog2e;
  return run_decode(a, dtype, max_context_len, (hipStream_t)stream);
}

int orin_attn_decode(const void* query, const void* key_cache, const void* value_cache,
                     void* out, int32_t batch, int32_t head_num, int32_t kv_head_num,
                     int32_t head_size, int64_t cache_batch_stride, int64_t cache_tok_stride,
                     const int32_t* context_lens, int32_t max_context_len, int32_t dtype,
                     float scale, int32_t split_tokens, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (cache_tok_stride < (int64_t)kv_head_num * head_size || cache_batch_stride < 0)
    return ORIN_ERR_INVALID_ARG;
  return batched_decode(query, key_cache, value_cache, out, batch, head_num, kv_head_num,
                        head_size, cache_batch_stride, cache_tok_stride, head_size, 0, nullptr, 0, 0,
                        context_lens, max_context_len, dtype, scale, split_tokens, workspace,
                        workspace_bytes, stream);
}

int orin_attn_decode_paged(const void* query, const void* k_pool, const void* v_pool, void* out,
                           int32_t batch, int32_t head_num, int32_t kv_head_num,
                           int32_t head_size, const int32_t* block_tables,
                           int32_t max_blocks_per_seq, int32_t block_size, int32_t kv_layout,
                           const int32_t* context_lens, int32_t max_context_len, int32_t dtype,
                           float scale, int32_t split_tokens, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!block_tables || block_size <= 0 || kv_head_num <= 0) return ORIN_ERR_INVALID_ARG;
  const int64_t d = head_size, bs = block_size, hkv = kv_head_num;
  int64_t tok_stride, head_stride;
  if (kv_layout == ORIN_KV_LAYOUT_TOKEN_MAJOR) {
    tok_stride = hkv * d;  // [num_blocks, block_size, kv_heads, head_size]
    head_stride = d;
  } else if (kv_layout == ORIN_KV_LAYOUT_HEAD_MAJOR) {
    tok_stride = d;  // [num_blocks, kv_heads, block_size, head_size]
    head_stride = bs * d;
  } else {
    return ORIN_ERR_INVALID_ARG;
  }
  return batched_decode(query, k_pool, v_pool, out, batch, head_num, kv_head_num, head_size, 0,
                        tok_stride, head_stride, bs * hkv * d, block_tables, max_blocks_per_seq,
                        block_size, context_lens, max_context_len, dtype, scale, split_tokens,
                        workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------ vision

static int vision_common(const void* q, const void* k, const void* v, void* output,
                         const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                         int32_t num_tokens, int32_t num_heads, int32_t head_dim, float scale,
                         int32_t dtype, void* stream) {
  if (num_tokens <= 0 || num_heads <= 0 || head_dim <= 0 || !q || !k || !v || !output)
    return ORIN_ERR_INVALID_ARG;
  if (cu_seqlens && (n_seqs <= 0 || max_seqlen <= 0)) return ORIN_ERR_INVALID_ARG;
  const float sl2 = resolve_scale(scale, head_dim) * kLog2e;
  const long tok = head_dim, hs = (long)num_tokens * head_dim;
  if (dtype == kF16 || dtype == kBF16) {
    if (!fwd_supports(dtype, head_dim)) return ORIN_ERR_UNSUPPORTED;
    FwdArgs a = {};
    a.q = q;
    a.q_tok_stride = tok;
    a.q_head_stride = hs;
    a.k = k;
    a.v = v;
    a.kv_tok_stride = tok;
    a.kv_head_stride = hs;
    a.o = output;
    a.o_tok_stride = (long)num_heads * head_dim;
    a.o_head_stride = head_dim;
    a.n_q = num_tokens;
    a.cu_seqlens = cu_seqlens;
    a.n_seg = cu_seqlens ? n_seqs : 1;
    a.max_seqlen = cu_seqlens ? max_seqlen : num_tokens;
    a.Hq = num_heads;
    a.Hkv = num_heads;
    a.kv_mul = 1;
    a.head_size = head_dim;
    a.scale_log2 = sl2;
    return hip_status(launch_fwd_varlen(a, dtype, (hipStream_t)stream));
  }
  if (dtype != kF32) return ORIN_ERR_UNSUPPORTED;
  if (!decode_supports(kF32, head_dim)) return ORIN_ERR_UNSUPPORTED;
  DecodeArgs a = decode_defaults();
  a.q = q;
  a.q_row_stride = tok;
  a.q_head_stride = hs;
  a.k = k;
  a.v = v;
  a.kv_tok_stride = tok;
  a.kv_head_stride = hs;
  if (cu_seqlens) {
    a.cu_seqlens = cu_seqlens;
    a.n_seg = n_seqs;
  } else {
    a.len_base = num_tokens;
  }
  a.o = output;
  a.o_row_stride = (long)num_heads * head_dim;
  a.o_head_stride = head_dim;
  a.n_rows = num_tokens;
  a.Hq = num_heads;
  a.Hkv = num_heads;
  a.kv_mul = 1;
  a.head_size = head_dim;
  a.scale_log2 = sl2;
  return run_decode(a, kF32, 0, (hipStream_t)stream);
}

int orin_vision_attention_pretransposed(const void* q, const void* k, const void* v,
                                        void* output, void* out_transposed, void* scores,
                                        int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                        float softmax_scale, int32_t dtype, void* stream) {
  (void)out_transposed;
  (void)scores;
  return vision_common(q, k, v, output, nullptr, 1, num_tokens, num_tokens, num_heads, head_dim,
                       softmax_scale, dtype, stream);
}

int orin_vision_attention_varlen(const void* q, const void* k, const void* v, void* output,
                                 const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                                 int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                 float softmax_scale, int32_t dtype, void* stream) {
  if (!cu_seqlens) return ORIN_ERR_INVALID_ARG;
  return vision_common(q, k, v, output, cu_seqlens, n_seqs, max_seqlen, num_tokens, num_heads,
                       head_dim, softmax_scale, dtype, stream);
}


// ------------------------------------------------------------------ output projection

int orin_batched_matmul(const void* input, const void* weight, void* output, int32_t batch_size,
                        int32_t in_dim, int32_t out_dim, float scale, int32_t dtype,
                        void* stream) {
  if (!input || !weight || !output || batch_size <= 0 || in_dim <= 0 || out_dim <= 0)
    return ORIN_ERR_INVALID_ARG;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return ORIN_ERR_UNSUPPORTED;
  const int st = output_projection(input, weight, output, batch_size, in_dim, out_dim, scale,
                                   dtype, (hipStream_t)stream, capturing(stream));
  if (st == -2) return ORIN_ERR_UNSUPPORTED;
  if (st == -3) return ORIN_ERR_WORKSPACE;
  if (st != 0) {
    g_last_hip_error = "rocBLAS gemm_ex failed";
    return ORIN_ERR_LAUNCH;
  }
  return ORIN_OK;
}

// ------------------------------------------------------------------ KV-cache writes

static bool dtype_ok(int32_t dtype) {
  return dtype == ORIN_DTYPE_FP32 || dtype == ORIN_DTYPE_FP16 || dtype == ORIN_DTYPE_BF16;
}
static int elem_bytes(int32_t dtype) { return dtype == ORIN_DTYPE_FP32 ? 4 : 2; }

int orin_copy_to_kv_cache(void* kv_cache, const void* src, const int32_t* pos, int32_t kv_dim,
                          int32_t layer_idx, int32_t seq_len, int32_t dtype, void* stream) {
  if (!kv_cache || !src || !pos || kv_dim <= 0 || layer_idx < 0 || seq_len <= 0)
    return ORIN_ERR_INVALID_ARG;
  if (!dtype_ok(dtype)) return ORIN_ERR_UNSUPPORTED;
  return hip_status(launch_kv_append(kv_cache, src, pos, kv_dim,
                                     (long)layer_idx * seq_len * kv_dim, dtype,
                                     (hipStream_t)stream));
}

int orin_kv_cache_write_paged(const void* k_src, const void* v_src, int64_t src_row_stride,
                              void* k_pool, void* v_pool, const int32_t* slot_mapping,
                              int32_t n_rows, int32_t kv_head_num, int32_t head_size,
                              int32_t block_size, int32_t kv_layout, int32_t dtype,
                              void* stream) {
  if (!k_src || !v_src || !k_pool || !v_pool || !slot_mapping || n_rows < 0 ||
      kv_head_num <= 0 || head_size <= 0 || block_size <= 0 ||
      src_row_stride < (int64_t)kv_head_num * head_size)
    return ORIN_ERR_INVALID_ARG;
  if (kv_layout != ORIN_KV_LAYOUT_TOKEN_MAJOR && kv_layout != ORIN_KV_LAYOUT_HEAD_MAJOR)
    return ORIN_ERR_INVALID_ARG;
  if (!dtype_ok(dtype)) return ORIN_ERR_UNSUPPORTED;
  const int vec = 16 / elem_bytes(dtype);
  if (head_size % vec || src_row_stride % vec) return ORIN_ERR_UNSUPPORTED;
  return hip_status(launch_kv_scatter(k_src, v_src, k_pool, v_pool, slot_mapping,
                                      src_row_stride, n_rows, kv_head_num, head_size, block_size,
                                      kv_layout == ORIN_KV_LAYOUT_HEAD_MAJOR, dtype,
                                      (hipStream_t)stream));
}

int orin_kv_cache_convert(void* contig, int64_t contig_row_stride, void* pool,
                          const int32_t* block_table, int32_t n_tokens, int32_t kv_head_num,
                          int32_t head_size, int32_t block_size, int32_t kv_layout,
                          int32_t direction, int32_t dtype, void* stream) {
  if (!contig || !pool || !block_table || n_tokens < 0 || kv_head_num <= 0 || head_size <= 0 ||
      block_size <= 0 || contig_row_stride < (int64_t)kv_head_num * head_size)
    return ORIN_ERR_INVALID_ARG;
  if (kv_layout != ORIN_KV_LAYOUT_TOKEN_MAJOR && kv_layout != ORIN_KV_LAYOUT_HEAD_MAJOR)
    return ORIN_ERR_INVALID_ARG;
  if (direction != ORIN_KV_TO_PAGED && direction != ORIN_KV_TO_CONTIGUOUS)
    return ORIN_ERR_INVALID_ARG;
  if (!dtype_ok(dtype)) return ORIN_ERR_UNSUPPORTED;
  const int vec = 16 / elem_bytes(dtype);
  if (head_size % vec || contig_row_stride % vec) return ORIN_ERR_UNSUPPORTED;
  return hip_status(launch_kv_convert(contig, pool, block_table, contig_row_stride, n_tokens,
                                      kv_head_num, head_size, block_size,
                                      kv_layout == ORIN_KV_LAYOUT_HEAD_MAJOR,
                                      direction == ORIN_KV_TO_PAGED, dtype, (hipStream_t)stream));
}

// ------------------------------------------------------------------ Q/K producers

int orin_rope_sin_cos_cache(float* sin_cache, float* cos_cache, int32_t head_size,
                            int32_t max_seq_len, float theta, void* stream) {
  if (!sin_cache || !cos_cache || head_size <= 0 || max_seq_len <= 0 || !(theta > 0.f))
    return ORIN_ERR_INVALID_ARG;
  return hip_status(
      launch_rope_cache(sin_cache, cos_cache, head_size, max_seq_len, theta, (hipStream_t)stream));
}

int orin_qk_norm_rope(void* query, const void* key, const void* value,
                      const void* q_norm_weight, const void* k_norm_weight,
                      const float* sin_cache, const float* cos_cache, void* key_cache,
                      void* value_cache, int32_t layer_index, int32_t max_seq_len,
                      int32_t start_pos, const int32_t* pos_ptr, int32_t seq_len,
                      int32_t head_num, int32_t kv_head_num, int32_t head_size, float eps,
                      int32_t dtype, void* stream) {
  if (!key || !value || !sin_cache || !cos_cache || !key_cache || !value_cache)
    return ORIN_ERR_INVALID_ARG;
  if (seq_len <= 0 || head_num <= 0 || kv_head_num <= 0 || head_size <= 0 || layer_index < 0 ||
      max_seq_len <= 0 || start_pos < 0 || !(eps >= 0.f))
    return ORIN_ERR_INVALID_ARG;
  if (!pos_ptr && start_pos + seq_len > max_seq_len) return ORIN_ERR_INVALID_ARG;
  if (!norm_rope_supports(dtype, head_size)) return ORIN_ERR_UNSUPPORTED;
  const long kv_dim = (long)kv_head_num * head_size;
  const long layer_off = (long)layer_index * max_seq_len * kv_dim * elem_bytes(dtype);
  return hip_status(launch_qk_norm_rope(
      query, key, value, q_norm_weight, k_norm_weight, sin_cache, cos_cache,
      static_cast<char*>(key_cache) + layer_off, static_cast<char*>(value_cache) + layer_off,
      kv_dim, pos_ptr, start_pos, seq_len, head_num, kv_head_num, head_size, eps, dtype,
      (hipStream_t)stream));
}

int orin_vision_split_rope_transpose(const void* qkv, const void* cos_cache,
                                     const void* sin_cache, void* q_trans, void* k_trans,
                                     void* v_trans, int32_t num_tokens, int32_t num_heads,
                                     int32_t head_dim, int32_t dtype, void* stream) {
  if (!qkv || !cos_cache || !sin_cache || !q_trans || !k_trans || !v_trans || num_tokens <= 0 ||
      num_heads <= 0 || head_dim <= 0 || head_dim % 2)
    return ORIN_ERR_INVALID_ARG;
  if (!dtype_ok(dtype)) return ORIN_ERR_UNSUPPORTED;
  return hip_status(launch_vision_qkv(qkv, cos_cache, sin_cache, q_trans, k_trans, v_trans,
                                      num_tokens, num_heads, head_dim, dtype,
                                      (hipStream_t)stream));
}

}  // extern "C"
