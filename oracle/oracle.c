/*
 * oracle.c -- CPU restatement of OrinMLLM's attention arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (orinmllm_amd, liborin_attn.so)
 * never calls it.
 *
 * What it restates (paths relative to the OrinMLLM source tree):
 *   oracle_mha_kernel      kuiper/source/op/kernels/cpu/mha_kernel.cpp:5-62
 *                          (per-head loop :19, GQA map h/kv_mul :29, layer offset :10,
 *                          scale 1/sqrt(head_size) :11, score layout [head, seq_len] :20)
 *   dot_scaled             kuiper/source/op/kernels/cpu/matmul_kernel.cpp:37-40
 *                          (score = (q . k) * scale)
 *   softmax_inplace        kuiper/source/op/kernels/cpu/softmax_kernel.cpp:4-15
 *                          (max, exp(x - max), sum, divide)
 *   scale_sum              kuiper/source/op/kernels/cpu/scale_sum_kernel.cpp:5-22
 *                          (out += p_i * V_i, i = 0..pos in order, stride kv_dim)
 *   oracle_attn_rows       the same per-row arithmetic generalised to the GPU entry
 *                          points' semantics:
 *                            causal prefill row i attends 0..start_pos+i
 *                              (kuiper/source/op/kernels/cuda/flash_attention_kernel.cu:575-578)
 *                            paged decode: token t lives at block_table[t/bs]*bs + t%bs
 *                              (no reference function; defined as contiguous decode plus
 *                              an address map)
 *                            varlen bidirectional: each segment attends to itself only
 *                              (vision_encoder_kernel.cu:954-1021 for one segment)
 *   oracle_rope_rotate_half  kuiper/source/op/kernels/cuda/rope_kernel.cu:86-98, 464-509
 *                          (pairs (j, j+d/2), freq_j = theta^(-2j/d))
 *   oracle_rmsnorm_rows    kuiper/source/op/kernels/cuda/rmsnorm_kernel.cu:483-545 (eps 1e-6)
 *   oracle_vision_cos_sin  kuiper/source/model/qwen3_vl.cpp:1698-1831 ([h,w,h,w] layout)
 *   oracle_vision_rotary   kuiper/source/op/kernels/cuda/vision_encoder_kernel.cu:662-744
 *
 * Deviations of the reference that are deliberately NOT restated: the fp16
 * kernels' flush-to-zero of exp(s - m) for s - m <= -20
 * (flash_attention_kernel.cu:36) and the +1e-10 in the vision softmax
 * denominator (vision_encoder_kernel.cu:931).  The oracle is exact softmax.
 *
 * All arithmetic is float (the reference CPU path is Armadillo fvec/fmat);
 * dot products and the weighted V sum accumulate sequentially in key order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* matmul_kernel.cpp:37-40: output = (input * weight) * scale for a 1xd by dx1 product. */
static float dot_scaled(const float* q, const float* k, int n, float scale) {
  float acc = 0.f;
  for (int i = 0; i < n; ++i) acc += q[i] * k[i];
  return acc * scale;
}

/* softmax_kernel.cpp:8-14 */
static void softmax_inplace(float* x, int n) {
  float mx = x[0];
  for (int i = 1; i < n; ++i)
    if (x[i] > mx) mx = x[i];
  for (int i = 0; i < n; ++i) x[i] = expf(x[i] - mx);
  float sum = 0.f;
  for (int i = 0; i < n; ++i) sum += x[i];
  for (int i = 0; i < n; ++i) x[i] = x[i] / sum;
}

/* scale_sum_kernel.cpp:17-21: out += p[i] * v[i*stride ...], i = 0..pos in order. */
static void scale_sum(const float* v, const float* p, float* out, int pos, int size,
                      long stride) {
  for (int i = 0; i <= pos; ++i) {
    const float* vr = v + (long)i * stride;
    for (int j = 0; j < size; ++j) out[j] += p[i] * vr[j];
  }
}

/*
 * Exact restatement of kernel::mha_kernel (cpu/mha_kernel.cpp:5-62).
 * score: [head_num, seq_len] scratch, key/value cache: [layers, seq_len, kv_dim].
 */
void oracle_mha_kernel(int pos, int head_num, int layer_index, int seq_len, int kv_dim,
                       int kv_mul, int head_size, float* mha_out, const float* query,
                       float* score, const float* key_cache, const float* value_cache) {
  long layer_offset = (long)layer_index * seq_len * kv_dim;
  float scale = 1.f / sqrtf((float)head_size);
  for (int h = 0; h < head_num; ++h) {
    float* score_h = score + (long)h * seq_len;
    const float* q_h = query + (long)h * head_size;
    for (int t = 0; t <= pos; ++t) {
      long cache_offset = (long)t * kv_dim + (long)(h / kv_mul) * head_size;
      score_h[t] = dot_scaled(q_h, key_cache + layer_offset + cache_offset, head_size, scale);
    }
    softmax_inplace(score_h, pos + 1);
    float* out_h = mha_out + (long)h * head_size;
    memset(out_h, 0, sizeof(float) * head_size);
    const float* v_h = value_cache + layer_offset + (long)(h / kv_mul) * head_size;
    scale_sum(v_h, score_h, out_h, pos, head_size, kv_dim);
  }
}

/*
 * One query row, all heads: the mha_kernel per-head arithmetic with a general
 * address map.  Key/value element (token t, kv head g, j) lives at
 *   base[phys(t) * tok_stride + g * head_stride + j],
 * phys(t) = tok_map ? tok_map[t] : t.
 */
static void attn_row(int Hq, int kv_mul, int d, float scale, const float* q,
                     long q_head_stride, const float* k, const float* v, long tok_stride,
                     long head_stride, const int* tok_map, int kv_len, float* o,
                     long o_head_stride, float* score) {
  for (int h = 0; h < Hq; ++h) {
    const float* q_h = q + (long)h * q_head_stride;
    long hoff = (long)(h / kv_mul) * head_stride;
    for (int t = 0; t < kv_len; ++t) {
      long phys = tok_map ? (long)tok_map[t] : (long)t;
      score[t] = dot_scaled(q_h, k + phys * tok_stride + hoff, d, scale);
    }
    softmax_inplace(score, kv_len);
    float* o_h = o + (long)h * o_head_stride;
    for (int j = 0; j < d; ++j) o_h[j] = 0.f;
    for (int t = 0; t < kv_len; ++t) {
      long phys = tok_map ? (long)tok_map[t] : (long)t;
      const float* vr = v + phys * tok_stride + hoff;
      for (int j = 0; j < d; ++j) o_h[j] += score[t] * vr[j];
    }
  }
}

/*
 * General driver.  Row r:
 *   query  q + r*q_row_stride (+ h*q_head_stride)
 *   keys   k/v + row_kv_offset[r] (+ phys(t)*tok_stride + g*head_stride), t < row_kv_len[r]
 *   map    tok_map ? tok_map + r*map_stride : identity
 *   output o + r*o_row_stride (+ h*o_head_stride)
 * Rows are independent; nthreads > 1 runs them with OpenMP (the CPU baseline's
 * multi-core figure).  The result does not depend on nthreads.
 */
void oracle_attn_rows(int n_rows, int Hq, int Hkv, int d, float scale, const float* q,
                      long q_row_stride, long q_head_stride, const float* k, const float* v,
                      long tok_stride, long head_stride, const long* row_kv_offset,
                      const int* row_kv_len, const int* tok_map, long map_stride, float* o,
                      long o_row_stride, long o_head_stride, int nthreads) {
  int kv_mul = Hq / Hkv;
  int max_len = 1;
  for (int r = 0; r < n_rows; ++r)
    if (row_kv_len[r] > max_len) max_len = row_kv_len[r];
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads)
  {
    float* score = (float*)malloc(sizeof(float) * (size_t)max_len);
#pragma omp for schedule(dynamic, 1)
    for (int r = 0; r < n_rows; ++r) {
      long off = row_kv_offset ? row_kv_offset[r] : 0;
      attn_row(Hq, kv_mul, d, scale, q + (long)r * q_row_stride, q_head_stride, k + off,
               v + off, tok_stride, head_stride, tok_map ? tok_map + (long)r * map_stride : 0,
               row_kv_len[r], o + (long)r * o_row_stride, o_head_stride, score);
    }
    free(score);
  }
}

/*
 * Paged decode: B sequences, query [B, Hq*d]; pools [num_blocks, block_size, Hkv*d];
 * block_tables [B, max_blocks]; context_lens [B].  Expands the block table into a
 * per-token physical row map and calls oracle_attn_rows.
 */
void oracle_decode_paged(int B, int Hq, int Hkv, int d, float scale, const float* q,
                         const float* k_pool, const float* v_pool, const int* block_tables,
                         int max_blocks, int block_size, const int* context_lens, float* o,
                         int nthreads) {
  long map_stride = (long)max_blocks * block_size;
  int* map = (int*)malloc(sizeof(int) * (size_t)(B * map_stride));
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < context_lens[b]; ++t)
      map[b * map_stride + t] =
          block_tables[(long)b * max_blocks + t / block_size] * block_size + t % block_size;
  long kv_dim = (long)Hkv * d;
  oracle_attn_rows(B, Hq, Hkv, d, scale, q, (long)Hq * d, d, k_pool, v_pool, kv_dim, d, 0,
                   context_lens, map, map_stride, o, (long)Hq * d, d, nthreads);
  free(map);
}

/*
 * Causal prefill over a kuiper cache: query/output [S, Hq*d], cache [max_seq, Hkv*d]
 * (already offset to the layer).  Row i attends 0..start_pos+i
 * (flash_attention_kernel.cu:575-578).
 */
void oracle_prefill_causal(int start_pos, int S, int Hq, int Hkv, int d, float scale,
                           const float* q, const float* k_cache, const float* v_cache,
                           float* o, int nthreads) {
  int* lens = (int*)malloc(sizeof(int) * (size_t)S);
  for (int i = 0; i < S; ++i) lens[i] = start_pos + i + 1;
  long kv_dim = (long)Hkv * d;
  oracle_attn_rows(S, Hq, Hkv, d, scale, q, (long)Hq * d, d, k_cache, v_cache, kv_dim, d, 0,
                   lens, 0, 0, o, (long)Hq * d, d, nthreads);
  free(lens);
}

/*
 * Bidirectional varlen attention in the vision layout: q/k/v [H, N, d] head-major,
 * output [N, H*d]; cu_seqlens[n_seg+1].  Each token attends to every token of its
 * own segment.
 */
void oracle_varlen_bidir(int N, int H, int d, float scale, const float* q, const float* k,
                         const float* v, const int* cu_seqlens, int n_seg, float* o,
                         int nthreads) {
  long* off = (long*)malloc(sizeof(long) * (size_t)N);
  int* lens = (int*)malloc(sizeof(int) * (size_t)N);
  for (int s = 0; s < n_seg; ++s)
    for (int t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) {
      off[t] = (long)cu_seqlens[s] * d;
      lens[t] = cu_seqlens[s + 1] - cu_seqlens[s];
    }
  oracle_attn_rows(N, H, H, d, scale, q, d, (long)N * d, k, v, d, (long)N * d, off, lens, 0, 0,
                   o, (long)H * d, d, nthreads);
  free(off);
  free(lens);
}

/* ---------------------------------------------------------------- producers */

/*
 * Qwen rotate-half RoPE on x [S, H*d] in place, positions start_pos..start_pos+S-1
 * (rope_kernel.cu:86-98 builds sin/cos for freq index 2j; :464-509 rotates (j, j+d/2)).
 */
void oracle_rope_rotate_half(float* x, int S, int H, int d, int start_pos, float theta) {
  int half = d / 2;
  for (int i = 0; i < S; ++i) {
    float pos = (float)(start_pos + i);
    for (int h = 0; h < H; ++h) {
      float* v = x + (long)i * H * d + (long)h * d;
      for (int j = 0; j < half; ++j) {
        float freq = 1.0f / powf(theta, (float)(2 * j) / (float)d);
        float ang = pos * freq;
        float c = cosf(ang), s = sinf(ang);
        float v0 = v[j], v1 = v[j + half];
        v[j] = c * v0 - s * v1;
        v[j + half] = c * v1 + s * v0;
      }
    }
  }
}

/* Per-row RMSNorm: y = x / sqrt(mean(x^2) + eps) * w (rmsnorm_kernel.cu:483-545, eps 1e-6). */
void oracle_rmsnorm_rows(float* x, long rows, int d, float eps, const float* w) {
  for (long r = 0; r < rows; ++r) {
    float* v = x + r * d;
    float ss = 0.f;
    for (int j = 0; j < d; ++j) ss += v[j] * v[j];
    float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (int j = 0; j < d; ++j) v[j] = v[j] * inv * (w ? w[j] : 1.0f);
  }
}

/*
 * Vision 2-D rotary tables cos/sin [N, d] (qwen3_vl.cpp:1698-1831): theta 10000,
 * d/4 frequencies inv_freq_i = theta^(-2i/(d/2)); token order walks merge blocks;
 * the d-vector is laid out [h, w, h, w] in quarters.
 */
void oracle_vision_cos_sin(int grid_t, int grid_h, int grid_w, int merge, int d, float* cos_out,
                           float* sin_out) {
  int half = d / 2, quarter = d / 4;
  int idx = 0;
  for (int t = 0; t < grid_t; ++t)
    for (int bh = 0; bh < grid_h / merge; ++bh)
      for (int bw = 0; bw < grid_w / merge; ++bw)
        for (int lh = 0; lh < merge; ++lh)
          for (int lw = 0; lw < merge; ++lw) {
            int hp = bh * merge + lh, wp = bw * merge + lw;
            for (int j = 0; j < quarter; ++j) {
              float inv = 1.0f / powf(10000.0f, (float)(2 * j) / (float)half);
              float fh = (float)hp * inv, fw = (float)wp * inv;
              float* c = cos_out + (long)idx * d;
              float* s = sin_out + (long)idx * d;
              c[j] = cosf(fh);
              s[j] = sinf(fh);
              c[quarter + j] = cosf(fw);
              s[quarter + j] = sinf(fw);
              c[half + j] = cosf(fh);
              s[half + j] = sinf(fh);
              c[half + quarter + j] = cosf(fw);
              s[half + quarter + j] = sinf(fw);
            }
            ++idx;
          }
}

/*
 * Apply the vision rotary to x [H, N, d] in place (vision_encoder_kernel.cu:662-744):
 *   x1' = x1*cos[j] - x2*sin[j],  x2' = x1*sin[j+d/2] + x2*cos[j+d/2].
 */
void oracle_vision_rotary(float* x, int H, int N, int d, const float* cos_t,
                          const float* sin_t) {
  int half = d / 2;
  for (int h = 0; h < H; ++h)
    for (int t = 0; t < N; ++t) {
      float* v = x + ((long)h * N + t) * d;
      const float* c = cos_t + (long)t * d;
      const float* s = sin_t + (long)t * d;
      for (int j = 0; j < half; ++j) {
        float x1 = v[j], x2 = v[j + half];
        v[j] = x1 * c[j] - x2 * s[j];
        v[j + half] = x1 * s[j + half] + x2 * c[j + half];
      }
    }
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
