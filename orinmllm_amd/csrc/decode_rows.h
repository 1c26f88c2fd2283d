// Row lengths and segment lookup shared by the decode kernels (decode.hip, decode_mfma.hip).
#pragma once
#include "kernels.h"

namespace orin {

// Segment s with cu[s] <= row < cu[s+1] (binary search over n_seg segments).
__device__ __forceinline__ int find_segment(const int* cu, int n_seg, int row) {
  int lo = 0, hi = n_seg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Number of keys row `row` attends to.  A device-side length (gpu pos, context_lens) longer
// than the launch was sized for (len_cap, from the host's max_context_len / max_seq_len) is
// an argument error that the host cannot see; the kernels then write NaN for that row
// rather than attend over a truncated prefix.
__device__ __forceinline__ int row_len(const DecodeArgs& a, int row) {
  if (a.cu_seqlens) {
    const int s = find_segment(a.cu_seqlens, a.n_seg, row);
    return a.cu_seqlens[s + 1] - a.cu_seqlens[s];
  }
  if (a.lens) return a.lens[row] + a.len_add;
  return a.len_base + row * a.len_step;
}

}  // namespace orin
