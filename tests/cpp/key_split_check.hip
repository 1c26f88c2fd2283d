// Host-side check of the ping-pong prefill's causal key split (orinmllm_amd/csrc/fwd_pp.hip):
// the chunk bound the host chooses (fwd_pp_key_split), the chunk cuts of every query block
// (pp_block_chunks / pp_chunk_lo), the work-item order (pp_item) and the workspace size, over
// a grid of prefix lengths, sequence lengths, head counts, device sizes, element types and
// head sizes.  Runs on the CPU only (no HIP runtime call is made); exits non-zero on any
// failure.  Built and run by tests/test_key_split_host.py.
#include "fwd_pp.hip"

#include <stdio.h>

using namespace orin;

static int g_fails = 0;
#define EXPECT(cond, ...)                                \
  do {                                                   \
    if (!(cond)) {                                       \
      if (g_fails++ < 20) {                              \
        printf("FAIL %s: ", #cond);                      \
        printf(__VA_ARGS__);                             \
        printf("\n");                                    \
      }                                                  \
    }                                                    \
  } while (0)

int main() {
  long cases = 0, splits = 0;
  const int n_cus[] = {80, 256, 304};
  const int starts[] = {0, 1, 63, 64, 100, 1000, 4095, 20000};
  const int lens[] = {1, 2, 63, 64, 65, 255, 256, 257, 511, 700, 1024, 2048, 2049, 3000, 4096};
  const int heads[] = {1, 2, 4, 6, 8, 12, 16, 32};
  const int dtypes[] = {kF16, kBF16};
  const int dims[] = {64, 128};
  for (int n_cu : n_cus)
    for (int sp : starts)
      for (int nq : lens)
        for (int hq : heads)
          for (int dt : dtypes)
            for (int d : dims) {
              FwdArgs a = {};
              a.q_tok_stride = (long)hq * d;
              a.q_head_stride = d;
              a.kv_tok_stride = d;  // one kv head
              a.kv_head_stride = d;
              a.o_tok_stride = (long)hq * d;
              a.o_head_stride = d;
              a.n_q = nq;
              a.start_pos = sp;
              a.Hq = hq;
              a.Hkv = 1;
              a.kv_mul = hq;
              a.head_size = d;
              size_t bytes = 123;
              const int C = fwd_pp_key_split(a, dt, n_cu, &bytes);
              ++cases;
              const int nqb = (nq + PBM - 1) / PBM;
              if ((long)nqb * hq >= n_cu) {
                EXPECT(C == 0 && bytes == 0, "sp %d nq %d hq %d: full grid must not split", sp, nq, hq);
                continue;
              }
              if (C == 0) {
                EXPECT(bytes == 0, "sp %d nq %d hq %d: no split but %zu bytes", sp, nq, hq, bytes);
                continue;
              }
              ++splits;
              const long items = pp_items(a, C);
              // One workgroup per CU at most; the merge handles at most kMergeMaxChunks chunks.
              EXPECT(items * hq <= n_cu, "sp %d nq %d hq %d C %d: %ld items", sp, nq, hq, C, items);
              // C is the smallest bound that fits.
              if (C > 1)
                EXPECT(!((long)pp_items(a, C - 1) * hq <= n_cu &&
                         pp_block_chunks(a, nqb - 1, C - 1) <= kMergeMaxChunks),
                       "sp %d nq %d hq %d: C %d is not the smallest", sp, nq, hq, C);
              const size_t rows = (size_t)items * hq * PBM;
              EXPECT(bytes == rows * d * (dt == kF16 ? 2 : 4) + rows * 2 * sizeof(float),
                     "sp %d nq %d hq %d: workspace %zu", sp, nq, hq, bytes);
              for (int b = 0; b < nqb; ++b) {
                const int n = pp_block_chunks(a, b, C);
                const int tiles = pp_block_tiles(a, b);
                const int diag = pp_block_diag(a, b);
                // tiles / diag from their definitions: keys [0, last query + 1), and the
                // tile of the block's first query position.
                EXPECT(tiles == (sp + (b + 1 < nqb ? (b + 1) * PBM : nq) + PBN - 1) / PBN &&
                           diag == (sp + b * PBM) / PBN,
                       "block %d", b);
                EXPECT(n >= 1 && n <= kMergeMaxChunks, "block %d: %d chunks", b, n);
                EXPECT(pp_chunk_lo(a, b, n, 0) == 0 && pp_chunk_lo(a, b, n, n) == tiles,
                       "block %d: cuts do not cover [0, %d)", b, tiles);
                for (int c = 0; c < n; ++c) {
                  // Non-empty, and every chunk starts at or before the block's first diagonal
                  // tile, so each of its queries sees at least one key of the chunk.
                  EXPECT(pp_chunk_lo(a, b, n, c + 1) > pp_chunk_lo(a, b, n, c),
                         "sp %d nq %d hq %d block %d chunk %d empty", sp, nq, hq, b, c);
                  EXPECT(pp_chunk_lo(a, b, n, c) <= diag,
                         "sp %d nq %d hq %d block %d chunk %d starts past the diagonal", sp, nq, hq, b, c);
                }
              }
              // Work items: blocks last to first, each block's chunks in order.
              int eb = nqb - 1, ec = 0;
              for (long i = 0; i < items; ++i) {
                int qb = -2, c = -2;
                pp_item(a, (int)i, C, &qb, &c);
                EXPECT(qb == eb && c == ec, "item %ld -> (%d, %d), expected (%d, %d)", i, qb, c, eb, ec);
                if (++ec == pp_block_chunks(a, eb, C)) {
                  --eb;
                  ec = 0;
                }
              }
              int qb = 0, c = 0;
              pp_item(a, (int)items, C, &qb, &c);
              EXPECT(qb == -1, "item past the end maps to block %d", qb);
            }
  printf("cases %ld, key splits %ld, failures %d\n", cases, splits, g_fails);
  return g_fails != 0;
}
