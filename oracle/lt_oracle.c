/* lt_oracle.c -- CPU restatement of LlamaTov's Q8_0 bs=1 decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the gfx950 path: it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and
 * by nothing else.  The product (llamatov_amd/) never links, imports or calls it.
 *
 * Each function restates the reference's algorithm in plain C, one scalar operation
 * at a time, in the reference's declared reduction order, and cites the reference
 * file:line it follows.  Transcendentals come from llamatov_amd/csrc/lt_numerics.h
 * (named textbook methods; the reference's CUDA intrinsics cannot be reproduced off
 * NVIDIA hardware) so that CPU and GPU agree bit for bit.  Build with
 * -ffp-contract=off: every fused multiply-add below is an explicit fmaf().
 *
 * Parity pins (what checks each function independently of this file) are listed in
 * tests/test_oracle_pins.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <omp.h>
#include "../llamatov_amd/csrc/lt_numerics.h"

#define OR_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------------
 * Q8_0 block codec.  A block is 34 bytes: fp16 scale d (little endian) then 32 int8.
 * Dequant y = q * d (bpd/llamatov_run.py:184-207).
 * ------------------------------------------------------------------------------- */
static inline uint16_t blk_scale(const uint8_t* blk) { return (uint16_t)(blk[0] | (blk[1] << 8)); }

/* Thread count of the OpenMP loops (the CPU baseline's 1-core and all-core figures). */
OR_API void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
OR_API int or_max_threads(void) { return omp_get_max_threads(); }

OR_API float or_half_to_float(uint16_t h) { return lt_half_to_float_bits(h); }
OR_API uint16_t or_float_to_half(float f) { return lt_float_to_half_bits(f); }
OR_API float or_expf(float x) { return lt_expf(x); }
/* Bit patterns start, start + stride, ... (count of them, mod 2^32) on which the device's
 * branch-free lt_expf_sel differs from lt_expf (0: the two forms agree). */
OR_API uint64_t or_expf_sel_mismatches(uint32_t start, uint32_t stride, uint64_t count) {
  uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t i = 0; i < (int64_t)count; i++) {
    const float x = lt_u2f(start + (uint32_t)((uint64_t)i * stride));
    if (lt_f2u(lt_expf_sel(x)) != lt_f2u(lt_expf(x))) bad++;
  }
  return bad;
}
OR_API void or_sincosf(float x, float* s, float* c) { lt_sincosf(x, s, c); }
OR_API float or_rsqrtf(float x) { return lt_rsqrtf(x); }

OR_API void or_dequant_rows(const uint8_t* W, int N, int K, float* out) {
  int nb = K / 32;
  for (int n = 0; n < N; n++)
    for (int b = 0; b < nb; b++) {
      const uint8_t* blk = W + ((size_t)n * nb + b) * 34;
      float d = lt_half_to_float_bits(blk_scale(blk));
      for (int i = 0; i < 32; i++) out[(size_t)n * K + b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

/* Weight quantizer (bpd/lib/fact_dispatch.py:255-282): per 32-block of a row,
 * d = fp16(amax/127) (1.0 if amax == 0), q = clip(rint(w / float(d16)), +-127). */
OR_API void or_quantize_rows(const float* W, int N, int K, uint8_t* out) {
  int nb = K / 32;
  for (int n = 0; n < N; n++)
    for (int b = 0; b < nb; b++) {
      const float* x = W + (size_t)n * K + b * 32;
      uint8_t* blk = out + ((size_t)n * nb + b) * 34;
      float amax = 0.0f;
      for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
      uint16_t d16 = lt_q8_scale_bits(amax);
      float dq = lt_half_to_float_bits(d16);
      blk[0] = (uint8_t)(d16 & 0xFF); blk[1] = (uint8_t)(d16 >> 8);
      for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)lt_q8_quant1(x[i], dq);
    }
}

/* Activation quant, engine convention (bpd/lib/dev_residency.py:799-808 serial,
 * :867-886 warp-parallel; numpy twin fact_dispatch.py:383-391). */
OR_API void or_quant_q8(const float* x, int K, int8_t* xq, uint16_t* xd) {
  int nb = K / 32;
  for (int b = 0; b < nb; b++) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[b * 32 + i]); if (a > amax) amax = a; }
    uint16_t d16 = lt_q8_scale_bits(amax);
    xd[b] = d16;
    float dq = lt_half_to_float_bits(d16);
    for (int i = 0; i < 32; i++) xq[b * 32 + i] = (int8_t)lt_q8_quant1(x[b * 32 + i], dq);
  }
}

/* SiLU(g)*u elementwise, v = (g/(1+exp(-g)))*u (bpd/lib/dev_residency.py:583). */
OR_API void or_silu_mul(const float* g, const float* u, int K, float* v) {
  for (int i = 0; i < K; i++) v[i] = lt_silu_mul(g[i], u[i]);
}

/* k_silu_mul_quant (bpd/lib/dev_residency.py:573-604): v = (g/(1+exp(-g)))*u, then quant. */
OR_API void or_silu_mul_quant(const float* g, const float* u, int K, int8_t* xq, uint16_t* xd) {
  float* v = (float*)malloc(sizeof(float) * (size_t)K);
  for (int i = 0; i < K; i++) v[i] = lt_silu_mul(g[i], u[i]);
  or_quant_q8(v, K, xq, xd);
  free(v);
}

/* Per-(row, block) int32 dots: isum = sum_i wq[i]*xq[i] (exact integer). */
OR_API void or_q8_block_dots(const uint8_t* W, const int8_t* xq, int N, int K, int32_t* isum) {
  int nb = K / 32;
  for (int n = 0; n < N; n++)
    for (int b = 0; b < nb; b++) {
      const uint8_t* blk = W + ((size_t)n * nb + b) * 34;
      int32_t s = 0;
      for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)blk[2 + i] * (int32_t)xq[b * 32 + i];
      isum[(size_t)n * nb + b] = s;
    }
}

/* Canonical Q8_0 GEMV order, reduction_order(q8_gemv_dp4a, lanes(32), strided,
 * accum(fma), tree(shfl_down,5)) (bpd/kernelgen/emitters/q8_0_from_facts.pl:466-516):
 *   lane L folds blocks b = L, L+32, ... with acc = fma(wd*xd, (float)isum, acc);
 *   the 32 partials merge s = 16,8,4,2,1: acc[t] += acc[t+s];
 *   Y = acc[0] (+ resid[row] as one fp32 add, the addres/bias epilogue :374-416). */
static float gemv_row(const uint8_t* W, const int8_t* xq, const uint16_t* xd, int row, int nb) {
  float lane[32];
  for (int L = 0; L < 32; L++) {
    float acc = 0.0f;
    for (int b = L; b < nb; b += 32) {
      const uint8_t* blk = W + ((size_t)row * nb + b) * 34;
      int32_t s = 0;
      for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)blk[2 + i] * (int32_t)xq[b * 32 + i];
      float wd = lt_half_to_float_bits(blk_scale(blk));
      float xdv = lt_half_to_float_bits(xd[b]);
      acc = fmaf(wd * xdv, (float)s, acc);
    }
    lane[L] = acc;
  }
  for (int s = 16; s > 0; s >>= 1)
    for (int t = 0; t < s; t++) lane[t] = lane[t] + lane[t + s];
  return lane[0];
}

OR_API void or_q8_gemv(const uint8_t* W, const int8_t* xq, const uint16_t* xd, const float* resid,
                       float* y, int N, int K) {
  int nb = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    float acc = gemv_row(W, xq, xd, n, nb);
    y[n] = resid ? acc + resid[n] : acc;
  }
}

/* ---------------------------------------------------------------------------------
 * ggml-compatible numerics (the optional profile that lets results be compared with
 * llama.cpp / Ollama): ggml's dispatched AVX quantizer and its two Q8_0 dot orders, as the
 * reference's CPU substrate restates them (bpd-substrate/bench/bpd_cpu.c:4005-4271,
 * bpd_gemm_q8_0_cpu.c:22-130; bpd/tests/q8_0_kernel/README.md:28-55).  AVX1 arithmetic:
 * separate multiply and add (no FMA), as on the reference's Ivy Bridge host.
 * ------------------------------------------------------------------------------- */

/* quantize_row_q8_0, AVX path (bpd_cpu.c:4083-4112): amax = max |x|; stored scale
 * d16 = fp16_rne(amax / 127.f); multiplier id = amax != 0 ? 127.f / amax : 0 (one division,
 * not 1/d); q = rint(x * id), ties to even.  |x * id| <= 127 * (1 + 2^-23) < 127.5, so the
 * int8 conversion never saturates. */
OR_API void or_quant_q8_ggml(const float* x, int K, int8_t* xq, uint16_t* xd) {
  int nb = K / 32;
  for (int b = 0; b < nb; b++) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[b * 32 + i]); if (a > amax) amax = a; }
    float d = amax / 127.0f;
    xd[b] = lt_float_to_half_bits(d);
    float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    for (int i = 0; i < 32; i++) {
      float t = x[b * 32 + i] * id;
      xq[b * 32 + i] = (int8_t)rintf(t);
    }
  }
}

/* The same quantizer writing 34-byte blocks (bpd_quant_q8_0_cpu's output format). */
OR_API void or_quant_q8_0_ggml_blocks(const float* x, int K, uint8_t* y) {
  int nb = K / 32;
  int8_t q[32];
  uint16_t d;
  for (int b = 0; b < nb; b++) {
    or_quant_q8_ggml(x + b * 32, 32, q, &d);
    y[b * 34] = (uint8_t)(d & 0xFF);
    y[b * 34 + 1] = (uint8_t)(d >> 8);
    memcpy(y + b * 34 + 2, q, 32);
  }
}

/* hsum_float_8 (bpd_cpu.c:4180-4186): (a4+a0 + a6+a2) + (a5+a1 + a7+a3). */
static float ggml_hsum8(const float* a) {
  float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
  float s0 = r0 + r2, s1 = r1 + r3;
  return s0 + s1;
}

/* Sum of the products of quants {4j..4j+3} of one block (exact integer). */
static int32_t quad_dot(const int8_t* w, const int8_t* x, int j) {
  int32_t s = 0;
  for (int i = 0; i < 4; i++) s += (int32_t)w[4 * j + i] * (int32_t)x[4 * j + i];
  return s;
}

/* ggml_vec_dot_q8_0_q8_0, AVX path (bpd_cpu.c:4188-4223): blocks in pairs (b, b+1); lane
 * 4h + j (h = 0, 1 the block of the pair, j = 0..3) holds the int dot of quants
 * {4j..4j+3} and {16+4j..16+4j+3} of block b+h, times delta = wd*xd of that block, added
 * to the lane's accumulator (mul, then add); hsum_float_8; an odd last block adds
 * (float)isum * (wd*xd) to the sum. */
static float dot_ggml_vec(const uint8_t* wrow, const int8_t* xq, const uint16_t* xd, int nb) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    for (int h = 0; h < 2; h++) {
      const uint8_t* blk = wrow + (size_t)(b + h) * 34;
      const int8_t* w = (const int8_t*)(blk + 2);
      const int8_t* x = xq + (size_t)(b + h) * 32;
      float delta = lt_half_to_float_bits(blk_scale(blk)) * lt_half_to_float_bits(xd[b + h]);
      for (int j = 0; j < 4; j++) {
        int32_t s = quad_dot(w, x, j) + quad_dot(w, x, j + 4);
        float p = delta * (float)s;
        acc[4 * h + j] = p + acc[4 * h + j];
      }
    }
  }
  float sum = ggml_hsum8(acc);
  for (; b < nb; b++) {
    const uint8_t* blk = wrow + (size_t)b * 34;
    const int8_t* w = (const int8_t*)(blk + 2);
    int32_t s = 0;
    for (int i = 0; i < 32; i++) s += (int32_t)w[i] * (int32_t)xq[(size_t)b * 32 + i];
    float delta = lt_half_to_float_bits(blk_scale(blk)) * lt_half_to_float_bits(xd[b]);
    float p = (float)s * delta;
    sum = sum + p;
  }
  return sum;
}

/* llamafile tinyBLAS_Q0_AVX cell (bpd_cpu.c:4344-4398, bpd_gemm_q8_0_cpu.c:82-130): per
 * block, lane j (0..7) holds the int dot of quants {4j..4j+3}, times scale = wd*xd, added
 * to the lane's accumulator (mul, then add); hsum_float_8 at the end. */
static float dot_ggml_llamafile(const uint8_t* wrow, const int8_t* xq, const uint16_t* xd, int nb) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; b++) {
    const uint8_t* blk = wrow + (size_t)b * 34;
    const int8_t* w = (const int8_t*)(blk + 2);
    const int8_t* x = xq + (size_t)b * 32;
    float scale = lt_half_to_float_bits(blk_scale(blk)) * lt_half_to_float_bits(xd[b]);
    for (int j = 0; j < 8; j++) {
      float p = scale * (float)quad_dot(w, x, j);
      acc[j] = p + acc[j];
    }
  }
  return ggml_hsum8(acc);
}

/* GEMV rows in a ggml order (0 = vec_dot, 1 = llamafile); y = dot (+ resid[row] as one
 * fp32 add, ggml's separate ADD node for the bias and the residual). */
OR_API void or_q8_gemv_ggml(const uint8_t* W, const int8_t* xq, const uint16_t* xd, const float* resid,
                            float* y, int N, int K, int order) {
  int nb = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    const uint8_t* wrow = W + (size_t)n * nb * 34;
    float v = order ? dot_ggml_llamafile(wrow, xq, xd, nb) : dot_ggml_vec(wrow, xq, xd, nb);
    y[n] = resid ? v + resid[n] : v;
  }
}

/* bpd_qmatmul_q8_0_cpu (bpd_cpu.c:4283-4305): X [M][K] fp32 quantized row by row, then
 * out[m][n] = vec_dot(W row n, X row m). */
OR_API void or_qmatmul_q8_0_ggml(const uint8_t* W, const float* X, float* out, int M, int N, int K) {
  int8_t* xq = (int8_t*)malloc((size_t)K);
  uint16_t* xd = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(K / 32));
  for (int m = 0; m < M; m++) {
    or_quant_q8_ggml(X + (size_t)m * K, K, xq, xd);
    or_q8_gemv_ggml(W, xq, xd, NULL, out + (size_t)m * N, N, K, 0);
  }
  free(xq);
  free(xd);
}

/* bpd_qmatmul_q8_0_llamafile_cpu (bpd_cpu.c:4419-4446) with its tile dispatcher
 * (bpd_gemm_q8_0_cpu.c:209-258, llamafile's mnpack): tokens go in groups of 4, then 2,
 * then 1; a token of a group of 1 (the last one when m_tokens is odd) takes the vec_dot
 * order, every other token the llamafile cell order.  out[token][row], ldc = m_weight. */
OR_API void or_qmatmul_q8_0_llamafile(const uint8_t* W, const float* X, float* out, int m_weight, int m_tokens,
                                      int K) {
  int8_t* xq = (int8_t*)malloc((size_t)K);
  uint16_t* xd = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(K / 32));
  for (int m = 0; m < m_tokens; m++) {
    int vec = (m_tokens & 1) && m == m_tokens - 1;
    or_quant_q8_ggml(X + (size_t)m * K, K, xq, xd);
    or_q8_gemv_ggml(W, xq, xd, NULL, out + (size_t)m * m_weight, m_weight, K, vec ? 0 : 1);
  }
  free(xq);
  free(xd);
}

/* ---------------------------------------------------------------------------------
 * Sampling beyond greedy (the extension the reference plans for its device argmax,
 * bpd/lib/dev_residency.py:186-191, 1795-1803).  The definition the device sampler
 * (lt_sample.hip) follows, restated with a full sort instead of its radix selects.
 * ------------------------------------------------------------------------------- */

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC 2011): 10 rounds, the key bumped by the
 * Weyl constants before every round but the first. */
OR_API void or_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3], k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; r++) {
    if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static uint32_t sample_order_key(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  if ((b << 1) == 0u) return 0x80000000u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static int cmp_desc_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

/* Rank by (logit desc, index asc) with -0 == +0; k = clamp(top_k, 1, 1024) (1 when
 * temperature <= 0 or 1/T is not finite), at most V; the top candidate when its logit is not
 * finite; e_i = lt_expf((l_i - l_0) * (1/T)); c_i sequential;
 * n = smallest count with c_{n-1} >= top_p * c_{k-1} (k when top_p >= 1);
 * u = (philox4x32_10({counter, 0}, seed).x >> 8) * 2^-24; first i < n with c_i > u*c_{n-1}. */
OR_API int or_sample(const float* logits, int V, float temperature, int top_k, float top_p, uint64_t seed,
                     uint64_t counter) {
  int k = top_k < 1 ? 1 : (top_k > 1024 ? 1024 : top_k);
  if (!(temperature > 0.0f) || !isfinite(1.0f / temperature)) k = 1;
  if (k > V) k = V;
  uint64_t* key = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  for (int i = 0; i < V; i++) key[i] = ((uint64_t)sample_order_key(logits[i]) << 32) | (uint32_t)~(uint32_t)i;
  qsort(key, (size_t)V, sizeof(uint64_t), cmp_desc_u64);
  if (!isfinite(logits[~(uint32_t)key[0]])) k = 1;
  int pick = 0;
  if (k > 1) {
    float invT = 1.0f / temperature;
    float l0 = logits[~(uint32_t)key[0]];
    float* c = (float*)malloc(sizeof(float) * (size_t)k);
    float acc = 0.0f;
    for (int i = 0; i < k; i++) {
      float li = logits[~(uint32_t)key[i]];
      float ci = (li - l0) * invT;
      /* -0 and +0 rank as one key; the logit difference only feeds exp, where they agree */
      acc = acc + lt_expf(ci);
      c[i] = acc;
    }
    int n = k;
    if (top_p < 1.0f) {
      float thr = top_p * c[k - 1];
      for (int i = 0; i < k; i++) if (c[i] >= thr) { n = i + 1; break; }
    }
    uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
    uint32_t kk[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)}, out[4];
    or_philox4x32_10(ctr, kk, out);
    float u = (float)(out[0] >> 8) * 0x1.0p-24f;
    float target = u * c[n - 1];
    pick = n - 1;
    for (int i = 0; i < n; i++) if (c[i] > target) { pick = i; break; }
    free(c);
  }
  int id = (int)~(uint32_t)key[pick];
  free(key);
  return id;
}

/* RMSNorm, reduction_order(rms_ss, lanes(256), strided, tree(pairwise,8))
 * (bpd/kernelgen/emitters/norm_softmax_from_facts.pl:49, block_row :83-108,
 * canonical_serial :117-144): p[t] = fma(x_j, x_j, p[t]) over j = t, t+256, ...;
 * tree s = 128..1; inv = rsqrt(p[0]/N + eps); y_j = (x_j*inv)*w_j. */
OR_API void or_rmsnorm(const float* x, const float* w, float* y, int N, float eps) {
  float p[256];
  for (int t = 0; t < 256; t++) {
    float acc = 0.0f;
    for (int j = t; j < N; j += 256) acc = fmaf(x[j], x[j], acc);
    p[t] = acc;
  }
  for (int s = 128; s > 0; s >>= 1)
    for (int t = 0; t < s; t++) p[t] = p[t] + p[t + s];
  float inv = lt_rsqrtf(p[0] / (float)N + eps);
  for (int j = 0; j < N; j++) y[j] = (x[j] * inv) * w[j];
}

/* RoPE inverse-frequency table: freq_j = theta^(-(2j)/hd) with the exponent formed
 * in binary32 as the reference does (bpd/kernelgen/emitters/rope_from_facts.pl:58)
 * and the power evaluated in binary64 then rounded once. */
OR_API void or_rope_freqs(int hd, float theta, float* freqs) {
  for (int j = 0; j < hd / 2; j++) {
    float e = -(2.0f * (float)j) / (float)hd;
    freqs[j] = (float)pow((double)theta, (double)e);
  }
}

/* NeoX half-split rotation in place over nheads contiguous heads
 * (rope_from_facts.pl:40-69; fused q|k launch dev_residency.py:722-741):
 *   ang = (float)pos * freq_j; c = cos(ang); s = sin(ang);
 *   x_j'      = fma(x_j, c, -(x_{j+h} * s))
 *   x_{j+h}'  = fma(x_j, s,  (x_{j+h} * c))
 * The reference's `x1*c - x2*s` / `x1*s + x2*c` are contracted by nvcc; this build
 * fixes the contraction as written above. */
OR_API void or_rope(float* x, int pos, int nheads, int hd, const float* freqs) {
  int half = hd / 2;
  for (int h = 0; h < nheads; h++)
    for (int j = 0; j < half; j++) {
      float ang = (float)pos * freqs[j];
      float s, c;
      lt_sincosf(ang, &s, &c);
      float* base = x + (size_t)h * hd;
      float x1 = base[j], x2 = base[j + half];
      base[j] = fmaf(x1, c, -(x2 * s));
      base[j + half] = fmaf(x1, s, x2 * c);
    }
}

static inline float kv_load(const void* cache, int kv_f16, size_t idx) {
  return kv_f16 ? lt_half_to_float_bits(((const uint16_t*)cache)[idx]) : ((const float*)cache)[idx];
}

/* Decode attention for one query token over a position-major cache [t][nkv][hd].
 *
 * nsplit == 1: the production masked single pass k_attn_decode_masked
 * (bpd/lib/dev_residency.py:1955-2008):
 *   s_t = (sum_i fma(q_i, K_t,i)) * scale for t < L (positions t >= L are masked and
 *   contribute exactly nothing: their exp is 0 and fmax against them is a no-op, so
 *   the result does not depend on MAXT);
 *   mx  = 64-lane strided fmax fold + 6-level tree;
 *   e_t = exp(s_t - mx);
 *   Z   = 64-lane strided sum fold + 6-level tree;
 *   out_d = (sum_{t<L} fma(e_t, V_t,d)) / Z.
 *
 * nsplit > 1: split-K flash-decode, the declared order attn_decode_split
 * (bpd/kernelgen/experimental/attn_decode_split.cu:14-91, bpd/lib/ir_param_axes.pl:303-341):
 *   contiguous ranges per = ceil(L/S); per split a local max, e_t = exp(s_t - m_s),
 *   Z_s by the same 64-lane strided fold + tree over the split's positions, O_s by a
 *   sequential fma fold; combine in ascending split order:
 *   M = max_s m_s; w_s = exp(m_s - M); Z = fma(w_s, Z_s, Z); O = fma(w_s, O_s, O);
 *   out = O / Z.  With S = 1 this reduces exactly to the single pass.
 * GQA: query head h reads kv head h / (nh/nkv). */
static float lane64_sum(const float* e, int n) {
  float red[64];
  for (int d = 0; d < 64; d++) {
    float ls = 0.0f;
    for (int t = d; t < n; t += 64) ls = ls + e[t];
    red[d] = ls;
  }
  for (int s = 32; s > 0; s >>= 1)
    for (int d = 0; d < s; d++) red[d] = red[d] + red[d + s];
  return red[0];
}

static float lane64_max(const float* sc, int n) {
  float red[64];
  for (int d = 0; d < 64; d++) {
    float m = -1e30f;
    for (int t = d; t < n; t += 64) m = fmaxf(m, sc[t]);
    red[d] = m;
  }
  for (int s = 32; s > 0; s >>= 1)
    for (int d = 0; d < s; d++) red[d] = fmaxf(red[d], red[d + s]);
  return red[0];
}

OR_API void or_attn_decode(const float* q, const void* kc, const void* vc, int L, float* out,
                           int nh, int nkv, int hd, float scale, int kv_f16, int nsplit) {
  int rep = nh / nkv;
  float* sc = (float*)malloc(sizeof(float) * (size_t)(L > 0 ? L : 1));
  float* Os = (float*)malloc(sizeof(float) * (size_t)hd * (size_t)nsplit);
  float* Ms = (float*)malloc(sizeof(float) * (size_t)nsplit);
  float* Zs = (float*)malloc(sizeof(float) * (size_t)nsplit);
  for (int h = 0; h < nh; h++) {
    int g = h / rep;
    const float* qh = q + (size_t)h * hd;
    for (int t = 0; t < L; t++) {
      float s = 0.0f;
      size_t base = ((size_t)t * nkv + g) * hd;
      for (int i = 0; i < hd; i++) s = fmaf(qh[i], kv_load(kc, kv_f16, base + i), s);
      sc[t] = s * scale;
    }
    if (nsplit <= 1) {
      float mx = lane64_max(sc, L);
      for (int t = 0; t < L; t++) sc[t] = lt_expf(sc[t] - mx);
      float Z = lane64_sum(sc, L);
      for (int d = 0; d < hd; d++) {
        float acc = 0.0f;
        for (int t = 0; t < L; t++) acc = fmaf(sc[t], kv_load(vc, kv_f16, ((size_t)t * nkv + g) * hd + d), acc);
        out[(size_t)h * hd + d] = acc / Z;
      }
      continue;
    }
    int per = (L + nsplit - 1) / nsplit;
    for (int sp = 0; sp < nsplit; sp++) {
      int p0 = sp * per, p1 = p0 + per;
      if (p1 > L) p1 = L;
      int n = p1 - p0;
      if (n <= 0) {
        Ms[sp] = -1e30f; Zs[sp] = 0.0f;
        for (int d = 0; d < hd; d++) Os[(size_t)sp * hd + d] = 0.0f;
        continue;
      }
      float m = lane64_max(sc + p0, n);
      float* e = (float*)malloc(sizeof(float) * (size_t)n);
      for (int t = 0; t < n; t++) e[t] = lt_expf(sc[p0 + t] - m);
      Ms[sp] = m;
      Zs[sp] = lane64_sum(e, n);
      for (int d = 0; d < hd; d++) {
        float acc = 0.0f;
        for (int t = 0; t < n; t++) acc = fmaf(e[t], kv_load(vc, kv_f16, ((size_t)(p0 + t) * nkv + g) * hd + d), acc);
        Os[(size_t)sp * hd + d] = acc;
      }
      free(e);
    }
    float M = -1e30f;
    for (int sp = 0; sp < nsplit; sp++) M = fmaxf(M, Ms[sp]);
    float w[4096];
    for (int sp = 0; sp < nsplit; sp++) w[sp] = lt_expf(Ms[sp] - M);
    float Z = 0.0f;
    for (int sp = 0; sp < nsplit; sp++) Z = fmaf(w[sp], Zs[sp], Z);
    for (int d = 0; d < hd; d++) {
      float acc = 0.0f;
      for (int sp = 0; sp < nsplit; sp++) acc = fmaf(w[sp], Os[(size_t)sp * hd + d], acc);
      out[(size_t)h * hd + d] = acc / Z;
    }
  }
  free(sc); free(Os); free(Ms); free(Zs);
}

/* Greedy argmax: the maximum, ties broken toward the lowest index
 * (bpd/lib/dev_residency.py:200-201, 218-224, two-stage :225-273). */
OR_API int or_argmax(const float* x, int n) {
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int i = 0; i < n; i++)
    if (x[i] > bv || (x[i] == bv && i < bi)) { bv = x[i]; bi = i; }
  return bi;
}

/* Embedding row of token `tok` from the Q8_0 token_embd (GGUF [vocab][E/32] blocks):
 * the host fp32 dequantized row the reference gathers (dev_residency.py:1357-1358). */
OR_API void or_embed_row(const uint8_t* emb, int tok, int E, float* x) {
  or_dequant_rows(emb + (size_t)tok * (E / 32) * 34, 1, E, x);
}

/* ---------------------------------------------------------------------------------
 * Whole decode step, the production chain of forward_pass_resident
 * (bpd/lib/dev_residency.py:1328-1593, logits :1596-1623):
 *   rms -> quant -> QKV gemv (+bias) -> rope(q|k, pos=len) -> append k,v at len, len++
 *   -> attention(L=len) -> quant -> o gemv + x -> rms -> quant -> gate|up gemv
 *   -> silu*mul+quant -> down gemv + xres;  final rms -> quant -> lm_head gemv.
 * ------------------------------------------------------------------------------- */
typedef struct {
  int n_layers, n_embd, n_ff, n_head, n_head_kv, head_dim, vocab, max_ctx, kv_f16, attn_nsplit;
  float eps, theta;
  const uint8_t* tok_embd;          /* [vocab][E/32] Q8_0 */
  const uint8_t* output;            /* lm_head [vocab][E/32] Q8_0 (== tok_embd when tied) */
  const float* output_norm;         /* [E] */
  const float* const* attn_norm;    /* [n_layers] -> [E] */
  const uint8_t* const* wqkv;       /* [n_layers] -> [(nh+2nkv)*hd][E/32] */
  const float* const* bqkv;         /* [n_layers] -> [(nh+2nkv)*hd] or NULL array */
  const uint8_t* const* wo;         /* [n_layers] -> [E][nh*hd/32] */
  const float* const* ffn_norm;     /* [n_layers] -> [E] */
  const uint8_t* const* wgu;        /* [n_layers] -> [2F][E/32], gate rows then up rows */
  const uint8_t* const* wdown;      /* [n_layers] -> [E][F/32] */
  int numerics;                     /* 0 = the engine's quantizer and GEMV order, 1 = ggml's
                                       (or_quant_q8_ggml, vec_dot order) for every GEMV */
} or_model;

/* The step's quantizer and GEMV under the model's numerics. */
static void step_quant(const or_model* m, const float* x, int K, int8_t* xq, uint16_t* xd) {
  if (m->numerics) or_quant_q8_ggml(x, K, xq, xd);
  else or_quant_q8(x, K, xq, xd);
}
static void step_gemv(const or_model* m, const uint8_t* W, const int8_t* xq, const uint16_t* xd,
                      const float* resid, float* y, int N, int K) {
  if (m->numerics) or_q8_gemv_ggml(W, xq, xd, resid, y, N, K, 0);
  else or_q8_gemv(W, xq, xd, resid, y, N, K);
}

typedef struct {
  int len;
  void** kc;   /* [n_layers] -> [max_ctx][nkv*hd] fp32 or fp16 */
  void** vc;
} or_state;

OR_API or_state* or_state_new(const or_model* m) {
  or_state* s = (or_state*)calloc(1, sizeof(or_state));
  size_t esz = m->kv_f16 ? 2 : 4;
  size_t n = (size_t)m->max_ctx * m->n_head_kv * m->head_dim * esz;
  s->kc = (void**)calloc((size_t)m->n_layers, sizeof(void*));
  s->vc = (void**)calloc((size_t)m->n_layers, sizeof(void*));
  for (int l = 0; l < m->n_layers; l++) { s->kc[l] = calloc(n, 1); s->vc[l] = calloc(n, 1); }
  return s;
}

OR_API void or_state_free(const or_model* m, or_state* s) {
  if (!s) return;
  for (int l = 0; l < m->n_layers; l++) { free(s->kc[l]); free(s->vc[l]); }
  free(s->kc); free(s->vc); free(s);
}

OR_API int or_state_len(const or_state* s) { return s->len; }

OR_API const void* or_state_kv(const or_state* s, int layer, int which) {
  return which ? s->vc[layer] : s->kc[layer];
}

static void kv_store(void* cache, int kv_f16, size_t idx, float v) {
  if (kv_f16) ((uint16_t*)cache)[idx] = lt_float_to_half_bits(v);
  else ((float*)cache)[idx] = v;
}

/* One token through the model; writes vocab logits.  Returns 0, or -1 if the cache is full. */
OR_API int or_decode_step(const or_model* m, or_state* st, int tok, float* logits) {
  const int E = m->n_embd, F = m->n_ff, nh = m->n_head, nkv = m->n_head_kv, hd = m->head_dim;
  const int QD = nh * hd, KD = nkv * hd, NQKV = QD + 2 * KD;
  if (st->len >= m->max_ctx) return -1;
  int Kmax = E > F ? E : F;
  if (QD > Kmax) Kmax = QD;
  float* x = (float*)malloc(sizeof(float) * E);
  float* h = (float*)malloc(sizeof(float) * E);
  float* xres = (float*)malloc(sizeof(float) * E);
  float* qkv = (float*)malloc(sizeof(float) * NQKV);
  float* att = (float*)malloc(sizeof(float) * QD);
  float* gu = (float*)malloc(sizeof(float) * 2 * (size_t)F);
  int8_t* xq = (int8_t*)malloc((size_t)Kmax);
  uint16_t* xd = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(Kmax / 32));
  float* freqs = (float*)malloc(sizeof(float) * (size_t)(hd / 2));
  or_rope_freqs(hd, m->theta, freqs);
  or_embed_row(m->tok_embd, tok, E, x);
  const int pos = st->len;
  float scale = (float)pow((double)hd, -0.5);   /* hd ** -0.5 (dev_residency.py:1423) */
  for (int l = 0; l < m->n_layers; l++) {
    or_rmsnorm(x, m->attn_norm[l], h, E, m->eps);
    step_quant(m, h, E, xq, xd);
    step_gemv(m, m->wqkv[l], xq, xd, m->bqkv ? m->bqkv[l] : NULL, qkv, NQKV, E);
    or_rope(qkv, pos, nh + nkv, hd, freqs);
    for (int i = 0; i < KD; i++) {
      kv_store(st->kc[l], m->kv_f16, (size_t)pos * KD + i, qkv[QD + i]);
      kv_store(st->vc[l], m->kv_f16, (size_t)pos * KD + i, qkv[QD + KD + i]);
    }
    or_attn_decode(qkv, st->kc[l], st->vc[l], pos + 1, att, nh, nkv, hd, scale, m->kv_f16,
                   m->attn_nsplit > 0 ? m->attn_nsplit : 1);
    step_quant(m, att, QD, xq, xd);
    step_gemv(m, m->wo[l], xq, xd, x, xres, E, QD);
    or_rmsnorm(xres, m->ffn_norm[l], h, E, m->eps);
    step_quant(m, h, E, xq, xd);
    step_gemv(m, m->wgu[l], xq, xd, NULL, gu, 2 * F, E);
    or_silu_mul(gu, gu + F, F, gu);
    step_quant(m, gu, F, xq, xd);
    step_gemv(m, m->wdown[l], xq, xd, xres, x, E, F);
  }
  st->len = pos + 1;
  or_rmsnorm(x, m->output_norm, h, E, m->eps);
  step_quant(m, h, E, xq, xd);
  step_gemv(m, m->output, xq, xd, NULL, logits, m->vocab, E);
  free(x); free(h); free(xres); free(qkv); free(att); free(gu); free(xq); free(xd); free(freqs);
  return 0;
}

/* Greedy generation: the prompt is fed token by token (the reference's device-uniform
 * prefill, dev_residency.py:1338-1356); the last prompt token's logits give the first
 * generated token; each generated token is fed back.  Writes n_gen token ids, and the
 * top-1/top-2 logit margin of each decision into margins (may be NULL). */
OR_API int or_generate(const or_model* m, or_state* st, const int* prompt, int n_prompt, int n_gen,
                       int* out, float* margins) {
  float* logits = (float*)malloc(sizeof(float) * (size_t)m->vocab);
  int rc = 0;
  for (int i = 0; i < n_prompt && rc == 0; i++) rc = or_decode_step(m, st, prompt[i], logits);
  for (int i = 0; i < n_gen && rc == 0; i++) {
    int t = or_argmax(logits, m->vocab);
    out[i] = t;
    if (margins) {
      float second = -INFINITY;
      for (int j = 0; j < m->vocab; j++) if (j != t && logits[j] > second) second = logits[j];
      margins[i] = logits[t] - second;
    }
    if (i + 1 < n_gen) rc = or_decode_step(m, st, t, logits);
  }
  free(logits);
  return rc;
}
