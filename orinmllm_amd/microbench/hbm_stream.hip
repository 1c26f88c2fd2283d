// Streaming-read ceilings of HBM for the paged decode's access patterns on gfx950: 268 MB of
// 2 KB token rows (8 kv heads x 256 B at head size 128, fp16), read from 4 rotated pools so
// the 256 MB last-level cache cannot serve them.  dk_rd / dv_rd use the decode kernel's own
// instruction shapes (K: 8 tokens x 128 B per load; V: one 256 B row per wave load, 4 B per
// lane), slice_rd reads one 256 B head slice per workgroup, row_rd whole rows per
// workgroup; "nt" = nontemporal loads.  Prints time and GB/s per pattern.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
#define CHECK(x) do { hipError_t e = (x); if (e) { printf("err %s line %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

template <int U, bool NT>
__global__ __launch_bounds__(256) void slice_rd(const u32x4* buf, u32x4* out, int ch_tok, long ntok) {
  // WG: head h, token chunk; lane reads 16 B of a 256 B slice; 16 tokens per iteration
  const int h = blockIdx.x & 7;
  const long t0 = (long)(blockIdx.x >> 3) * ch_tok;
  const int t = threadIdx.x;
  u32x4 acc = {0, 0, 0, 0};
  const u32x4* base = buf + t0 * 128 + h * 16 + (t >> 4) * 128 + (t & 15);
  for (int i = 0; i < ch_tok; i += 16 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(base + (long)(i + 16 * u) * 128) : base[(long)(i + 16 * u) * 128];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  if (acc.x == 0x12345678) out[t] = acc;
}
template <int U, bool NT>
__global__ __launch_bounds__(256) void row_rd(const u32x4* buf, u32x4* out, int ch_tok, long ntok) {
  // WG: token chunk, all heads; 2 tokens per iteration (each 1 KB wave load = half a row)
  const long t0 = (long)blockIdx.x * (ch_tok / 8);
  const int t = threadIdx.x;
  u32x4 acc = {0, 0, 0, 0};
  const u32x4* base = buf + t0 * 128 + t;
  for (int i = 0; i < ch_tok / 8; i += 2 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(base + (long)(i + 2 * u) * 128) : base[(long)(i + 2 * u) * 128];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  if (acc.x == 0x12345678) out[t] = acc;
}

// decode K pattern: lane (grp = l>>3, k8 = l&7) loads 16 B at token grp, byte 128n + 16 k8
template <int U>
__global__ __launch_bounds__(256) void dk_rd(const u32x4* buf, u32x4* out, int ch_tok, long ntok) {
  const int h = blockIdx.x & 7;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long t0 = (long)(blockIdx.x >> 3) * ch_tok;
  u32x4 acc = {0, 0, 0, 0};
  const u32x4* base = buf + t0 * 128 + h * 16 + (l >> 3) * 128 + (l & 7);
  for (int i = w * 8; i < ch_tok; i += 32 * U) {
    u32x4 v[2 * U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[2 * u] = __builtin_nontemporal_load(base + (long)(i + 32 * u) * 128);
      v[2 * u + 1] = __builtin_nontemporal_load(base + (long)(i + 32 * u) * 128 + 8);
    }
#pragma unroll
    for (int u = 0; u < 2 * U; ++u) acc ^= v[u];
  }
  if (acc.x == 0x12345678) out[threadIdx.x] = acc;
}
// decode V pattern: whole wave loads one token's 256 B slice, 4 B per lane
template <int U>
__global__ __launch_bounds__(256) void dv_rd(const u32x4* buf, u32x4* out, int ch_tok, long ntok) {
  const int h = blockIdx.x & 7;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long t0 = (long)(blockIdx.x >> 3) * ch_tok;
  unsigned acc = 0;
  const unsigned* base = (const unsigned*)(buf + t0 * 128 + h * 16) + l;
  for (int i = w * 8; i < ch_tok; i += 32 * U) {
    unsigned v[8 * U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < 8; ++r) v[8 * u + r] = __builtin_nontemporal_load(base + (long)(i + 32 * u + r) * 512);
#pragma unroll
    for (int u = 0; u < 8 * U; ++u) acc ^= v[u];
  }
  if (acc == 0x12345678) out[threadIdx.x] = u32x4{acc, 0, 0, 0};
}

template <typename K>
void run(const char* name, K kern, int grid, const u32x4* buf, u32x4* out, int ch, long ntok, size_t bytes, int pools, size_t pool_elems) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a)); CHECK(hipEventCreate(&b));
  for (int w = 0; w < 4; ++w) hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, 0, buf + (w % pools) * pool_elems, out, ch, ntok);
  const int it = 20;
  CHECK(hipEventRecord(a));
  for (int w = 0; w < it; ++w) hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, 0, buf + (w % pools) * pool_elems, out, ch, ntok);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms; CHECK(hipEventElapsedTime(&ms, a, b));
  printf("%-28s ch %5d grid %7d : %7.2f us  %6.0f GB/s\n", name, ch, grid, ms * 1000 / it, bytes / (ms / it * 1e-3) / 1e9);
}

int main() {
  const long ntok = 32L * 4096 * 2 / 2 * 1;  // 131072 token rows x 2 KB = 268 MB (K+V of ~C4)
  const size_t bytes = ntok * 2048;
  const int pools = 4;
  const size_t pool_elems = bytes / 16;
  u32x4* buf; u32x4* out;
  CHECK(hipMalloc(&buf, bytes * pools)); CHECK(hipMalloc(&out, 4096));
  CHECK(hipMemset(buf, 1, bytes * pools));
  for (int ch : {256, 1024}) {
    int g = (int)(ntok / ch) * 8;
    run("dk U1", dk_rd<1>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("dk U2", dk_rd<2>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("dk U4", dk_rd<4>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("dv U1", dv_rd<1>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("dv U2", dv_rd<2>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("dv U4", dv_rd<4>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
  }
  for (int ch : {256, 1024}) {
    int g = (int)(ntok / ch) * 8;
    run("slice U4", slice_rd<4, false>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("slice U8", slice_rd<8, false>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("slice U8 nt", slice_rd<8, true>, g, buf, out, ch, ntok, bytes, pools, pool_elems);
    int gr = (int)(ntok / (ch / 8));
    run("row U4", row_rd<4, false>, gr, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("row U8", row_rd<8, false>, gr, buf, out, ch, ntok, bytes, pools, pool_elems);
    run("row U8 nt", row_rd<8, true>, gr, buf, out, ch, ntok, bytes, pools, pool_elems);
  }
  return 0;
}
