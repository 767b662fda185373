// lt_ggml.hip -- the ggml-compatible numerics profile: ggml's dispatched quantizer and its
// two Q8_0 dot orders on the device, so that results can be compared bit for bit with
// llama.cpp / Ollama on an AVX1 host.  The reference restates them on its CPU substrate
// (bpd-substrate/bench/bpd_cpu.c:4005-4271, bpd_gemm_q8_0_cpu.c:22-258); its engine path
// keeps its own quantizer and canonical GEMV order (lt_ops.hip, lt_fused.hip).
//
//   quantizer  d16 = fp16_rne(amax / 127.f), id = amax ? 127.f / amax : 0 (one division),
//              q = rint(x * id), ties to even (bpd_cpu.c:4083-4112)
//   vec_dot    blocks in pairs; lane 4h + j of 8 holds delta(b+h) * isum(quants 4j..4j+3 and
//              16+4j..16+4j+3 of block b+h), accumulated mul-then-add over the pairs; the
//              8 lanes close as (a4+a0 + a6+a2) + (a5+a1 + a7+a3); an odd last block adds
//              (float)isum * delta (bpd_cpu.c:4188-4223, ggml_vec_dot_q8_0_q8_0's AVX path)
//   llamafile  per block, lane j of 8 holds scale * isum(quants 4j..4j+3), accumulated
//              mul-then-add over all blocks; same 8-lane close (bpd_cpu.c:4344-4398,
//              tinyBLAS_Q0_AVX's cell)
//
// GPU mapping.  Only the float additions are ordered, so the GEMV splits in two phases:
// (1) a half-wave per row streams the row's blocks exactly as the engine GEMV does (lane L
// takes blocks L, L+32, ...; coalesced 34-byte blocks, v_dot4 on the re-aligned quants) and
// writes every lane product -- 4 per block (vec_dot) or 8 (llamafile), each one rounding --
// to LDS; (2) 8 lanes of the half-wave run the 8 sequential accumulator chains over LDS in
// the declared order, and the close is done with shuffles.  Integer sums and the fp16
// scale product wd*xd (exact in fp32) are order-free.
#include "lt_internal.h"
#include "lt_q8_device.h"

using namespace lt;

namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGgThreads = 256;
constexpr int kGgRows = kGgThreads / 32;      // one row per half-wave
constexpr int kGgUnroll = 4;                  // blocks in flight per lane
constexpr size_t kGgLdsMax = (size_t)160 * 1024;

// ---- quantizer ----------------------------------------------------------------------
// One half-wave per 32-element block.  kBlocks: write 34-byte Q8_0 blocks (fp16 scale little
// endian, then the 32 quants) instead of the split quants / scales.
template <bool kBlocks>
__global__ __launch_bounds__(kGgThreads) void k_quant_q8_ggml(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                              uint16_t* __restrict__ xd, uint8_t* __restrict__ yb,
                                                              int nb) {
  const int lane = threadIdx.x & 31;
  const int b = blockIdx.x * kGgRows + (threadIdx.x >> 5);
  const float v = b < nb ? x[(size_t)b * 32 + lane] : 0.0f;
  const float amax = halfwave_max(fabsf(v));   // every lane takes part in the DPP max
  if (b >= nb) return;
  const float d = amax / 127.0f;               // correctly rounded division
  const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
  const float t = v * id;
  const int q = (int)__builtin_rintf(t);
  const uint16_t h = lt_f2h(d);
  if constexpr (kBlocks) {
    uint8_t* blk = yb + (size_t)b * kBlockBytes;
    blk[2 + lane] = (uint8_t)(int8_t)q;
    if (lane == 0) {
      blk[0] = (uint8_t)(h & 0xFFu);
      blk[1] = (uint8_t)(h >> 8);
    }
  } else {
    xq[(size_t)b * 32 + lane] = (int8_t)q;
    if (lane == 0) xd[b] = h;
  }
}

// ---- GEMV -----------------------------------------------------------------------------
// grid (ceil(N / 8), tokens).  Token m reads xq + m*K, xd + m*nb and writes y + m*ldy.
template <int kOrder>
struct GgOrder {
  static constexpr int kLanes = kOrder == LT_GGML_VEC ? 4 : 8;   // products per block
};

template <int kOrder>
__global__ __launch_bounds__(kGgThreads) void k_gemv_ggml(const uint8_t* __restrict__ W,
                                                          const int8_t* __restrict__ xq,
                                                          const uint16_t* __restrict__ xd,
                                                          const float* __restrict__ resid, float* __restrict__ y,
                                                          int N, int K, int ldy) {
  constexpr int PL = GgOrder<kOrder>::kLanes;
  extern __shared__ __attribute__((aligned(16))) float sP[];   // [kGgRows][nb][PL]
  __shared__ float sTail[kGgRows];
  const int nb = K >> 5;
  const int lane = threadIdx.x & 31, hw = threadIdx.x >> 5;
  const int row = blockIdx.x * kGgRows + hw;
  const int m = blockIdx.y;
  const int8_t* xqm = xq + (size_t)m * K;
  const uint16_t* xdm = xd + (size_t)m * nb;
  float* prow = sP + (size_t)hw * nb * PL;
  const size_t last = (size_t)N * nb - 1;

  // (1) lane products, each with one rounding
  if (row < N) {
    for (int b0 = lane; b0 < nb; b0 += 32 * kGgUnroll) {
      BlockRegs r[kGgUnroll];
#pragma unroll
      for (int u = 0; u < kGgUnroll; u++) {
        const int b = b0 + 32 * u;
        if (b < nb) load_q8_block(W, (size_t)row * nb + b, last, r[u]);
      }
#pragma unroll
      for (int u = 0; u < kGgUnroll; u++) {
        const int b = b0 + 32 * u;
        if (b >= nb) break;
        const u32x4 x0 = *(const u32x4*)(xqm + (size_t)b * 32);
        const u32x4 x1 = *(const u32x4*)(xqm + (size_t)b * 32 + 16);
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int s[8];
#pragma unroll
        for (int j = 0; j < 8; j++) s[j] = __builtin_amdgcn_sdot4((int)r[u].q[j], (int)xw[j], 0, false);
        const float delta = lt_h2f(r[u].d) * lt_h2f(xdm[b]);   // exact: two fp16 significands
        float* pb = prow + (size_t)b * PL;
        if constexpr (kOrder == LT_GGML_VEC) {
          f32x4_t p;
          p.x = delta * (float)(s[0] + s[4]);
          p.y = delta * (float)(s[1] + s[5]);
          p.z = delta * (float)(s[2] + s[6]);
          p.w = delta * (float)(s[3] + s[7]);
          *(f32x4_t*)pb = p;
          if ((nb & 1) && b == nb - 1) {   // the odd last block: (float)isum * delta
            const int tot = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
            sTail[hw] = (float)tot * delta;
          }
        } else {
          f32x4_t p0, p1;
          p0.x = delta * (float)s[0]; p0.y = delta * (float)s[1];
          p0.z = delta * (float)s[2]; p0.w = delta * (float)s[3];
          p1.x = delta * (float)s[4]; p1.y = delta * (float)s[5];
          p1.z = delta * (float)s[6]; p1.w = delta * (float)s[7];
          *(f32x4_t*)pb = p0;
          *(f32x4_t*)(pb + 4) = p1;
        }
      }
    }
  }
  __syncthreads();

  // (2) the 8 accumulator chains (lane l < 8 of the half-wave), mul already done: add in
  // ascending pair (vec_dot) or block (llamafile) order
  float acc = 0.0f;
  if (row < N && lane < 8) {
    if constexpr (kOrder == LT_GGML_VEC) {
      const float* pl = prow + (lane >> 2) * 4 + (lane & 3);
      const int npairs = nb >> 1;
      for (int p = 0; p < npairs; p++) acc = pl[(size_t)p * 8] + acc;
    } else {
      const float* pl = prow + lane;
      for (int b = 0; b < nb; b++) acc = pl[(size_t)b * 8] + acc;
    }
  }
  // hsum_float_8: (a4+a0 + a6+a2) + (a5+a1 + a7+a3), lanes of this half-wave
  const int base = threadIdx.x & 32;
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; k++) a[k] = __shfl(acc, base + k, 64);
  if (row < N && lane == 0) {
    const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
    float v = (r0 + r2) + (r1 + r3);
    if constexpr (kOrder == LT_GGML_VEC) {
      if (nb & 1) v = v + sTail[hw];
    }
    y[(size_t)m * ldy + row] = resid ? v + resid[row] : v;
  }
}

size_t gemv_ggml_lds(int order, int K) {
  return (size_t)kGgRows * (K / 32) * (order == LT_GGML_VEC ? 4 : 8) * sizeof(float);
}

int check_ggml_gemv(const char* who, const void* W, int N, int K, int order) {
  LT_REQUIRE(W, "%s: null weights", who);
  LT_REQUIRE(lt_aligned(W, 4), "%s: weights must be 4-byte aligned", who);
  LT_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "%s: N=%d K=%d (K a positive multiple of 32)", who, N, K);
  LT_REQUIRE(order == LT_GGML_VEC || order == LT_GGML_LLAMAFILE, "%s: order=%d", who, order);
  LT_REQUIRE(gemv_ggml_lds(order, K) <= kGgLdsMax, "%s: K=%d exceeds the %s order's LDS limit (K <= %d)", who, K,
             order == LT_GGML_VEC ? "vec_dot" : "llamafile", order == LT_GGML_VEC ? 40960 : 20480);
  return LT_OK;
}

int launch_gemv_ggml(lt_ctx* ctx, int order, const void* W, const int8_t* xq, const uint16_t* xd,
                     const float* resid, float* y, int N, int K, int tokens, int ldy) {
  const dim3 grid((N + kGgRows - 1) / kGgRows, tokens);
  const size_t lds = gemv_ggml_lds(order, K);
  if (order == LT_GGML_VEC)
    k_gemv_ggml<LT_GGML_VEC><<<grid, kGgThreads, lds, ctx->stream>>>((const uint8_t*)W, xq, xd, resid, y, N, K, ldy);
  else
    k_gemv_ggml<LT_GGML_LLAMAFILE>
        <<<grid, kGgThreads, lds, ctx->stream>>>((const uint8_t*)W, xq, xd, resid, y, N, K, ldy);
  return lt_check_launch("k_gemv_ggml");
}

struct QmmWs {
  int8_t* xq;
  uint16_t* xd;
};

QmmWs qmm_ws_layout(void* ws, int M, int K) {
  QmmWs w;
  w.xq = (int8_t*)ws;
  w.xd = (uint16_t*)(((uintptr_t)ws + (size_t)M * K + 15) & ~(uintptr_t)15);
  return w;
}

}  // namespace

extern "C" {

int lt_quant_q8_ggml(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int K) {
  LT_REQUIRE(ctx && x && xq && xd, "lt_quant_q8_ggml: null argument");
  LT_REQUIRE(K > 0 && K % 32 == 0, "lt_quant_q8_ggml: K=%d must be a positive multiple of 32", K);
  const int nb = K / 32;
  k_quant_q8_ggml<false><<<(nb + kGgRows - 1) / kGgRows, kGgThreads, 0, ctx->stream>>>(x, xq, xd, nullptr, nb);
  return lt_check_launch("k_quant_q8_ggml");
}

int lt_quant_q8_0_ggml(lt_ctx* ctx, const float* x, uint8_t* y, int n_elements) {
  LT_REQUIRE(ctx && x && y, "lt_quant_q8_0_ggml: null argument");
  LT_REQUIRE(n_elements > 0 && n_elements % 32 == 0, "lt_quant_q8_0_ggml: n_elements=%d must be a positive multiple of 32",
             n_elements);
  const int nb = n_elements / 32;
  k_quant_q8_ggml<true><<<(nb + kGgRows - 1) / kGgRows, kGgThreads, 0, ctx->stream>>>(x, nullptr, nullptr, y, nb);
  return lt_check_launch("k_quant_q8_ggml<blocks>");
}

int lt_q8_gemv_ggml(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid, float* y,
                    int N, int K, int order) {
  LT_REQUIRE(ctx && xq && xd && y, "lt_q8_gemv_ggml: null argument");
  if (int rc = check_ggml_gemv("lt_q8_gemv_ggml", W, N, K, order)) return rc;
  LT_REQUIRE(lt_aligned(xq, 16), "lt_q8_gemv_ggml: xq must be 16-byte aligned");
  return launch_gemv_ggml(ctx, order, W, xq, xd, resid, y, N, K, 1, N);
}

size_t lt_qmatmul_q8_0_workspace_size(int M, int K) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  return (size_t)M * K + 16 + (size_t)M * (K / 32) * sizeof(uint16_t) + 16;
}

int lt_qmatmul_q8_0_ggml(lt_ctx* ctx, const void* W, const float* X, float* out, int M, int N, int K, void* ws,
                         size_t ws_bytes) {
  LT_REQUIRE(ctx && X && out && ws, "lt_qmatmul_q8_0_ggml: null argument");
  LT_REQUIRE(M > 0, "lt_qmatmul_q8_0_ggml: M=%d", M);
  if (int rc = check_ggml_gemv("lt_qmatmul_q8_0_ggml", W, N, K, LT_GGML_VEC)) return rc;
  LT_REQUIRE(lt_aligned(ws, 16) && ws_bytes >= lt_qmatmul_q8_0_workspace_size(M, K),
             "lt_qmatmul_q8_0_ggml: workspace must be 16-byte aligned and hold %zu bytes (got %zu)",
             lt_qmatmul_q8_0_workspace_size(M, K), ws_bytes);
  const QmmWs w = qmm_ws_layout(ws, M, K);
  if (int rc = lt_quant_q8_ggml(ctx, X, w.xq, w.xd, M * K)) return rc;   // rows are whole blocks
  return launch_gemv_ggml(ctx, LT_GGML_VEC, W, w.xq, w.xd, nullptr, out, N, K, M, N);
}

int lt_qmatmul_q8_0_llamafile(lt_ctx* ctx, const void* W, const float* X, float* out, int m_weight, int m_tokens,
                              int K, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && X && out && ws, "lt_qmatmul_q8_0_llamafile: null argument");
  LT_REQUIRE(m_tokens > 0, "lt_qmatmul_q8_0_llamafile: m_tokens=%d", m_tokens);
  if (int rc = check_ggml_gemv("lt_qmatmul_q8_0_llamafile", W, m_weight, K, LT_GGML_LLAMAFILE)) return rc;
  LT_REQUIRE(lt_aligned(ws, 16) && ws_bytes >= lt_qmatmul_q8_0_workspace_size(m_tokens, K),
             "lt_qmatmul_q8_0_llamafile: workspace must be 16-byte aligned and hold %zu bytes (got %zu)",
             lt_qmatmul_q8_0_workspace_size(m_tokens, K), ws_bytes);
  const QmmWs w = qmm_ws_layout(ws, m_tokens, K);
  if (int rc = lt_quant_q8_ggml(ctx, X, w.xq, w.xd, m_tokens * K)) return rc;
  // tokens in groups of 4, 2, 1 (llamafile's mnpack): only a group of one -- the last token
  // when m_tokens is odd -- takes the vec_dot order
  const int vec_tok = (m_tokens & 1) ? m_tokens - 1 : m_tokens;
  if (vec_tok > 0)
    if (int rc = launch_gemv_ggml(ctx, LT_GGML_LLAMAFILE, W, w.xq, w.xd, nullptr, out, m_weight, K, vec_tok, m_weight))
      return rc;
  if (vec_tok < m_tokens) {
    const int nb = K / 32;
    return launch_gemv_ggml(ctx, LT_GGML_VEC, W, w.xq + (size_t)vec_tok * K, w.xd + (size_t)vec_tok * nb, nullptr,
                            out + (size_t)vec_tok * m_weight, m_weight, K, 1, m_weight);
  }
  return LT_OK;
}

}  // extern "C"
