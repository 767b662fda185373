// lt_ops.hip -- gfx950 kernels and C-ABI launchers for the per-op Q8_0 decode path:
// activation quant, SiLU*mul+quant, RMSNorm (+quant), Q8_0 GEMV (+residual/bias),
// RoPE, KV append, embedding gather, argmax.
//
// Wave64 mapping of the reference's wave-32 orders: every order the reference defines
// over 32 lanes (the GEMV's lanes(32) strided fold + shfl_down tree, the quant's
// per-block amax) runs on one 32-lane half of a 64-lane wavefront, so two reference
// warps share one CDNA wave and the per-lane arithmetic and the tree pairing are the
// reference's.  Compile with -ffp-contract=off: every fma in this file is explicit.
#include "lt_q8_device.h"

namespace {

using namespace lt;

// ---------------------------------------------------------------------------------
// Byte fill (capturable replacement of a memset node).
// ---------------------------------------------------------------------------------
__global__ void k_fill_u8(uint8_t* dst, uint8_t v, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = v;
}

// ---------------------------------------------------------------------------------
// Activation quant: one 32-lane half-wave per 32-element block, lane = element
// (the warp-per-block k_quant_q8 of bpd/lib/dev_residency.py:867-886).  amax is a max
// and hence order-free; d16 and q use the shared lt_numerics.h quantizer.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_q8(const float* __restrict__ x,
                                                  int8_t* __restrict__ xq,
                                                  uint16_t* __restrict__ xd, int nb) {
  int b = blockIdx.x * 8 + (threadIdx.x >> 5);
  int lane = threadIdx.x & 31;
  if (b >= nb) return;  // uniform per half-wave
  float v = x[b * 32 + lane];
  quant_block_hw(v, lane, xq + b * 32, xd + b);
}

__global__ __launch_bounds__(256) void k_silu_mul_quant(const float* __restrict__ g,
                                                        const float* __restrict__ u,
                                                        int8_t* __restrict__ xq,
                                                        uint16_t* __restrict__ xd, int nb) {
  int b = blockIdx.x * 8 + (threadIdx.x >> 5);
  int lane = threadIdx.x & 31;
  if (b >= nb) return;
  int i = b * 32 + lane;
  float v = lt_silu_mul(g[i], u[i]);
  quant_block_hw(v, lane, xq + b * 32, xd + b);
}

// ---------------------------------------------------------------------------------
// Elementwise SiLU(g)*u and a + b (k_silu_mul / k_add, bpd/lib/dev_residency.py:545-555):
// the per-element expressions of the fused kernels, for callers that keep fp32 vectors.
// y may alias g or u (an in-place update: each thread reads its element before writing it),
// so none of the three pointers is declared restrict.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_silu_mul(const float* g, const float* u, float* y, int n) {
  int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = lt_silu_mul(g[i], u[i]);
}

__global__ __launch_bounds__(256) void k_add(const float* __restrict__ a, const float* __restrict__ b,
                                             float* __restrict__ y, int n) {
  int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
}

// ---------------------------------------------------------------------------------
// RMSNorm, order rms_ss lanes(256) strided + pairwise tree (norm_softmax_from_facts.pl:
// 49, 83-108).  Thread t of the 256-thread block is reference lane t.  The tree's first
// two levels (s = 128, 64) are formed explicitly from LDS by wave 0, the last six
// (s = 32..1) by shuffle-down inside that wave; the pairing is the reference's.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ float rms_inv_block256(const float* __restrict__ xr, int N, float eps,
                                                  float* red /* LDS [256] */, float* sinv) {
  const int t = threadIdx.x;
  float p = 0.0f;
  for (int j = t; j < N; j += 256) p = fmaf(xr[j], xr[j], p);
  red[t] = p;
  __syncthreads();
  if (t < 64) {
    float a = red[t] + red[t + 128];
    float b = red[t + 64] + red[t + 192];
    float c = a + b;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) c = c + __shfl_down(c, s, 64);
    if (t == 0) *sinv = lt_rsqrtf(c / (float)N + eps);
  }
  __syncthreads();
  return *sinv;
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x,
                                                 const float* __restrict__ w,
                                                 float* __restrict__ y, int N, float eps) {
  __shared__ float red[256];
  __shared__ float sinv;
  const float* xr = x + (size_t)blockIdx.x * N;
  float* yr = y + (size_t)blockIdx.x * N;
  float inv = rms_inv_block256(xr, N, eps, red, &sinv);
  for (int j = threadIdx.x; j < N; j += 256) yr[j] = (xr[j] * inv) * w[j];
}

// k_rms_quant: normalize into LDS, then quantize each 32-block on a half-wave.
__global__ __launch_bounds__(256) void k_rmsnorm_quant(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       int8_t* __restrict__ xq,
                                                       uint16_t* __restrict__ xd, int N,
                                                       float eps) {
  extern __shared__ float ybuf[];  // [N]
  __shared__ float red[256];
  __shared__ float sinv;
  float inv = rms_inv_block256(x, N, eps, red, &sinv);
  for (int j = threadIdx.x; j < N; j += 256) ybuf[j] = (x[j] * inv) * w[j];
  __syncthreads();
  int lane = threadIdx.x & 31;
  for (int b = threadIdx.x >> 5; b < N / 32; b += 8)
    quant_block_hw(ybuf[b * 32 + lane], lane, xq + b * 32, xd + b);
}

// k_rmsnorm_quant over T rows with block-major output (the prefill GEMM's activation layout):
// row t's block b goes to xq[(b*T + t)*32 ..], xd[b*T + t].  The same arithmetic as
// k_rmsnorm followed by k_quant_q8 per row: thread j's elements j, j+256, ... (NPT at most)
// are loaded at once into registers, with the weights, and folded in that order, then the
// block tree of rms_inv_block256.
template <int NPT, bool kRows = false>
__global__ __launch_bounds__(256) void k_rmsnorm_quant_bm(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          int8_t* __restrict__ xq,
                                                          uint16_t* __restrict__ xd, int T, int N,
                                                          float eps) {
  extern __shared__ __attribute__((aligned(16))) float ybuf[];  // [N]
  __shared__ float red[256];
  __shared__ float sinv;
  const int t = blockIdx.x, tid = threadIdx.x;
  const float* xr = x + (size_t)t * N;
  float xv[NPT], wv[NPT];
#pragma unroll
  for (int i = 0; i < NPT; i++) {
    const int j = tid + 256 * i;
    xv[i] = j < N ? xr[j] : 0.0f;
    wv[i] = j < N ? w[j] : 0.0f;
  }
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < NPT; i++)
    if (tid + 256 * i < N) p = fmaf(xv[i], xv[i], p);
  red[tid] = p;
  __syncthreads();
  if (tid < 64) {
    float a = red[tid] + red[tid + 128];
    float b = red[tid + 64] + red[tid + 192];
    float c = a + b;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) c = c + __shfl_down(c, s, 64);
    if (tid == 0) sinv = lt_rsqrtf(c / (float)N + eps);
  }
  __syncthreads();
  const float inv = sinv;
#pragma unroll
  for (int i = 0; i < NPT; i++)
    if (tid + 256 * i < N) ybuf[tid + 256 * i] = (xv[i] * inv) * wv[i];
  __syncthreads();
  // 8 lanes per block, 4 elements each (quant4: the quantizer of quant_block_hw)
  const int j = tid & 7;
  for (int b = tid >> 3; b < N / 32; b += 32) {
    const size_t ob = kRows ? (size_t)t * (N / 32) + b : (size_t)b * T + t;   // kRows: row-major
    const float4 v = *(const float4*)(ybuf + b * 32 + 4 * j);
    QScale sc;
    const uint32_t p = quant4(v.x, v.y, v.z, v.w, sc);
    ((uint32_t*)(xq + ob * 32))[j] = p;
    if (j == 0) xd[ob] = sc.h;
  }
}

// ---------------------------------------------------------------------------------
// Per-(row, block) int32 dots of the GEMV arithmetic (a debug hook; the GEMV itself is
// k_gemv_fused in lt_fused.hip).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q8_gemv_isums(const uint8_t* __restrict__ W,
                                                       const int8_t* __restrict__ xq,
                                                       int32_t* __restrict__ isum, int N, int K) {
  const int nb = K >> 5;
  const int lane = threadIdx.x & 31;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (row >= N) return;
  for (int b = lane; b < nb; b += 32) {
    BlockRegs r;
    load_q8_block(W, (size_t)row * nb + b, (size_t)N * nb - 1, r);
    u32x4 x0, x1;
    __builtin_memcpy(&x0, xq + b * 32, 16);
    __builtin_memcpy(&x1, xq + b * 32 + 16, 16);
    int8_t tmp[32];
    __builtin_memcpy(tmp, &x0, 16);
    __builtin_memcpy(tmp + 16, &x1, 16);
    isum[(size_t)row * nb + b] = dot_q8_block(r, tmp);
  }
}

// ---------------------------------------------------------------------------------
// RoPE, NeoX half split (rope_from_facts.pl:40-69).  Thread per (head, j).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope(float* __restrict__ x, const int* __restrict__ pos,
                                              int nheads, int hd, const float* __restrict__ freqs) {
  const int half = hd >> 1;
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nheads * half) return;
  const int j = gid % half;
  const int h = gid / half;
  const float ang = (float)(*pos) * freqs[j];
  float s, c;
  lt_sincosf(ang, &s, &c);
  float* base = x + (size_t)h * hd;
  const float x1 = base[j], x2 = base[j + half];
  base[j] = fmaf(x1, c, -(x2 * s));
  base[j + half] = fmaf(x1, s, x2 * c);
}

// ---------------------------------------------------------------------------------
// KV append at the device length then length += 1 (k_append_kv_incr,
// bpd/lib/dev_residency.py:303-315).  One workgroup; the barrier orders every row write
// before the increment.  A full cache (len >= maxt) is left untouched.
// ---------------------------------------------------------------------------------
template <bool kF16>
__global__ __launch_bounds__(256) void k_kv_append_incr(void* __restrict__ kc,
                                                        const float* __restrict__ k,
                                                        void* __restrict__ vc,
                                                        const float* __restrict__ v,
                                                        int* __restrict__ len, int width, int maxt) {
  const int L = *len;
  if (L < 0 || L >= maxt) return;  // uniform: every thread reads the same L
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    size_t off = (size_t)L * width + i;
    if (kF16) {
      ((uint16_t*)kc)[off] = lt_float_to_half_bits(k[i]);
      ((uint16_t*)vc)[off] = lt_float_to_half_bits(v[i]);
    } else {
      ((float*)kc)[off] = k[i];
      ((float*)vc)[off] = v[i];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *len = L + 1;
}

// ---------------------------------------------------------------------------------
// Embedding gather from Q8_0 token_embd: x = q * d (exact in fp32).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed_q8(const uint8_t* __restrict__ emb,
                                                  const int* __restrict__ tok,
                                                  float* __restrict__ x, int E, int vocab,
                                                  int* __restrict__ err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E) return;
  const int t = *tok;
  if (t < 0 || t >= vocab) {
    x[i] = 0.0f;
    if (err && i == 0) *err = 1;
    return;
  }
  const uint8_t* blk = emb + ((size_t)t * (E / 32) + (i >> 5)) * kBlockBytes;
  const uint16_t d = (uint16_t)(blk[0] | (blk[1] << 8));
  x[i] = (float)(int8_t)blk[2 + (i & 31)] * lt_h2f(d);
}

// ---------------------------------------------------------------------------------
// Argmax, ties to the lowest index (k_argmax_s1/_s2, bpd/lib/dev_residency.py:225-273).
// Stage 1: 256 workgroups over contiguous chunks; stage 2: one workgroup.
// ---------------------------------------------------------------------------------
constexpr int kArgmaxBlocks = 256;

__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void am_block_reduce(float& bv, int& bi, float* sv, int* si) {
  // wave-level then LDS across the 4 waves
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    float ov = __shfl_xor(bv, m, 64);
    int oi = __shfl_xor(bi, m, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; k++)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
  }
}

__global__ __launch_bounds__(256) void k_argmax_s1(const float* __restrict__ x, int n,
                                                   float* __restrict__ pval,
                                                   int* __restrict__ pidx) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const long chunk = ((long)n + kArgmaxBlocks - 1) / kArgmaxBlocks;
  const long lo = (long)blockIdx.x * chunk;
  long hi = lo + chunk;
  if (hi > n) hi = n;
  float bv = -__builtin_inff();
  int bi = 0x7FFFFFFF;
  for (long i = lo + threadIdx.x; i < hi; i += 256) {
    float v = x[i];
    if (am_better(v, (int)i, bv, bi)) { bv = v; bi = (int)i; }
  }
  am_block_reduce(bv, bi, sv, si);
  if (threadIdx.x == 0) { pval[blockIdx.x] = bv; pidx[blockIdx.x] = bi; }
}

// Stage 2 optionally appends the winner to a device token history (hist[*count] = id,
// *count += 1, while *count < cap) so back-to-back graph replays keep every token.
__global__ __launch_bounds__(256) void k_argmax_s2(const float* __restrict__ pval,
                                                   const int* __restrict__ pidx,
                                                   int* __restrict__ out, int* __restrict__ hist,
                                                   int* __restrict__ count, int cap) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float bv = pval[threadIdx.x];
  int bi = pidx[threadIdx.x];
  am_block_reduce(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    *out = bi;
    if (hist) {
      const int c = *count;
      if (c >= 0 && c < cap) {
        hist[c] = bi;
        *count = c + 1;
      }
    }
  }
}

// Row-wise argmax of a [rows][n] matrix (the batched decode step's vocab rows): one
// 1024-thread workgroup per row, 8 loads in flight per thread, the same total order (value,
// then lowest index) as the single-row argmax; optional per-row histories hist[r][cap].
__global__ __launch_bounds__(1024) void k_argmax_rows(const float* __restrict__ x, int n, int* __restrict__ out,
                                                      int* __restrict__ hist, int* __restrict__ count, int cap) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int r = blockIdx.x;
  const float* xr = x + (size_t)r * n;
  float bv = -__builtin_inff();
  int bi = 0x7FFFFFFF;
  for (int base = 0; base < n; base += 1024 * 8) {
    float v[8];
    int ix[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = base + k * 1024 + (int)threadIdx.x;
      v[k] = i < n ? xr[i] : -__builtin_inff();
      ix[k] = i < n ? i : 0x7FFFFFFF;
    }
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (am_better(v[k], ix[k], bv, bi)) { bv = v[k]; bi = ix[k]; }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 16; k++)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
    out[r] = bi;
    if (hist) {
      const int c = count[r];
      if (c >= 0 && c < cap) {
        hist[(size_t)r * cap + c] = bi;
        count[r] = c + 1;
      }
    }
  }
}

// The same argmax over kArgmaxSlices workgroups per row: slice s of row r takes a contiguous
// range and writes its (value, index) winner to ws; k_argmax_rows_fin reduces a row's slices
// in one wave.  The winner under the total order (value, then lowest index; NaN never wins)
// does not depend on how the row is cut, so the result is k_argmax_rows's.
constexpr int kArgmaxSlices = 8;

__global__ __launch_bounds__(1024) void k_argmax_rows_part(const float* __restrict__ x, int n, float* __restrict__ wv,
                                                           int* __restrict__ wi) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int r = blockIdx.y, sl = blockIdx.x;
  const int chunk = ((n + kArgmaxSlices - 1) / kArgmaxSlices + 1023) & ~1023;
  const int lo = sl * chunk, hi = lo + chunk < n ? lo + chunk : n;
  const float* xr = x + (size_t)r * n;
  float bv = -__builtin_inff();
  int bi = 0x7FFFFFFF;
  for (int base = lo; base < hi; base += 1024 * 4) {
    float v[4];
    int ix[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = base + k * 1024 + (int)threadIdx.x;
      v[k] = i < hi ? xr[i] : -__builtin_inff();
      ix[k] = i < hi ? i : 0x7FFFFFFF;
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (am_better(v[k], ix[k], bv, bi)) { bv = v[k]; bi = ix[k]; }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 16; k++)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
    wv[r * kArgmaxSlices + sl] = bv;
    wi[r * kArgmaxSlices + sl] = bi;
  }
}

__global__ __launch_bounds__(64) void k_argmax_rows_fin(const float* __restrict__ wv, const int* __restrict__ wi,
                                                        int* __restrict__ out, int* __restrict__ hist,
                                                        int* __restrict__ count, int cap) {
  const int r = blockIdx.x, l = threadIdx.x;
  float bv = l < kArgmaxSlices ? wv[r * kArgmaxSlices + l] : -__builtin_inff();
  int bi = l < kArgmaxSlices ? wi[r * kArgmaxSlices + l] : 0x7FFFFFFF;
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (l == 0) {
    out[r] = bi;
    if (hist) {
      const int c = count[r];
      if (c >= 0 && c < cap) {
        hist[(size_t)r * cap + c] = bi;
        count[r] = c + 1;
      }
    }
  }
}

inline int grid_for(long n, int per) { return (int)((n + per - 1) / per); }

// ---- numerics self-check (lt_selftest_numerics) ---------------------------------------
// Every non-NaN binary32 pattern: the hardware conversion lt_f2h against the portable
// round-to-nearest-even lt_float_to_half_bits.
__global__ __launch_bounds__(256) void k_check_f2h(unsigned long long* bad) {
  unsigned long long n = 0;
  const uint32_t stride = gridDim.x * 256u;
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < (1ull << 32); u += stride) {
    const float f = __builtin_bit_cast(float, (uint32_t)u);
    if (f == f && lt_f2h(f) != lt_float_to_half_bits(f)) n++;
  }
  if (n) atomicAdd(bad, n);
}

// Workgroup h (1 .. 0x7BFF): dq = fp16 h; x at and around every (k + 1/2) * dq and at
// k * dq for |k| <= 140; lt_q8_quotient against IEEE division.
__global__ __launch_bounds__(256) void k_check_quotient(unsigned long long* out) {
  const uint32_t h = blockIdx.x + 1u;
  const float dq = lt_h2f((uint16_t)h);
  const float r = 1.0f / dq;
  unsigned long long bits = 0, qbad = 0, cases = 0;
  for (int c = threadIdx.x; c < 281 * 8; c += 256) {
    const int k = c / 8 - 140, d = c % 8;
    float x;
    if (d == 7) {
      x = (float)k * dq;
    } else {
      const float base = ((float)k + 0.5f) * dq;
      x = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, base) + (uint32_t)(d - 3));
    }
    if (!(fabsf(x) <= 3.402823466e38f)) continue;
    cases++;
    const float want = x / dq;
    const float got = lt_q8_quotient(x, dq, r);
    if (fabsf(want) >= 1.17549435e-38f && fabsf(want) <= 3.402823466e38f &&
        __builtin_bit_cast(uint32_t, want) != __builtin_bit_cast(uint32_t, got))
      bits++;
    if (lt_q8_round_clamp(want) != lt_q8_round_clamp(got)) qbad++;
  }
  if (bits) atomicAdd(&out[0], bits);
  if (qbad) atomicAdd(&out[1], qbad);
  atomicAdd(&out[2], cases);
}

// Repack a Q8_0 matrix [N][nb] (34-byte blocks) into the planar layout (lt_q8_device.h):
// thread per block; its 32 quants go to the two 16-byte halves of its item slot, its scale to
// the scale plane.  Byte loads: the source blocks are only 2-byte aligned.
__global__ __launch_bounds__(256) void k_q8_to_planar(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                      uint32_t n_blocks, int nb) {
  const uint32_t gi = blockIdx.x * 256u + threadIdx.x;
  if (gi >= n_blocks) return;
  const uint8_t* b = src + (size_t)gi * kBlockBytes;
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
    w[j] = (uint32_t)b[2 + 4 * j] | ((uint32_t)b[3 + 4 * j] << 8) | ((uint32_t)b[4 + 4 * j] << 16) |
           ((uint32_t)b[5 + 4 * j] << 24);
  const uint32_t row = gi / (uint32_t)nb, blk = gi - row * (uint32_t)nb;
  const uint32_t k0 = blk & ~31u, lane = blk & 31u;
  const uint32_t m = (uint32_t)nb - k0 < 32u ? (uint32_t)nb - k0 : 32u;   // blocks of this item
  uint8_t* q = dst + ((size_t)row * (size_t)nb + k0) * 32u + lane * 16u;
  *(u32x4*)q = u32x4{w[0], w[1], w[2], w[3]};
  *(u32x4*)(q + m * 16u) = u32x4{w[4], w[5], w[6], w[7]};
  uint16_t* sc = (uint16_t*)(dst + (size_t)n_blocks * 32u);
  sc[gi] = (uint16_t)(b[0] | (b[1] << 8));
}

}  // namespace

extern "C" {

int lt_q8_to_planar(lt_ctx* ctx, const void* src, void* dst, int N, int K) {
  LT_REQUIRE(ctx && src && dst, "lt_q8_to_planar: null argument");
  LT_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && K <= 16384, "lt_q8_to_planar: N=%d K=%d (K a multiple of 32, <= 16384)",
             N, K);
  LT_REQUIRE((uint64_t)N * (uint64_t)(K / 32) * 34u < ((uint64_t)1 << 32), "lt_q8_to_planar: matrix must be below 4 GiB");
  LT_REQUIRE(lt_aligned(dst, 16), "lt_q8_to_planar: dst must be 16-byte aligned");
  LT_REQUIRE(src != dst, "lt_q8_to_planar: dst must not be src");
  const uint32_t n = (uint32_t)N * (uint32_t)(K / 32);
  k_q8_to_planar<<<(n + 255) / 256, 256, 0, ctx->stream>>>((const uint8_t*)src, (uint8_t*)dst, n, K / 32);
  return lt_check_launch("k_q8_to_planar");
}

int lt_fill_u8(lt_ctx* ctx, void* dst, uint8_t value, size_t nbytes) {
  LT_REQUIRE(ctx && (dst || !nbytes), "lt_fill_u8: null argument");
  if (!nbytes) return LT_OK;
  int grid = (int)((nbytes + 255) / 256);
  if (grid > 4096) grid = 4096;
  k_fill_u8<<<grid, 256, 0, ctx->stream>>>((uint8_t*)dst, value, nbytes);
  return lt_check_launch("k_fill_u8");
}

int lt_quant_q8(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int K) {
  LT_REQUIRE(ctx && x && xq && xd, "lt_quant_q8: null argument");
  LT_REQUIRE(K > 0 && K % 32 == 0, "lt_quant_q8: K=%d must be a positive multiple of 32", K);
  int nb = K / 32;
  k_quant_q8<<<grid_for(nb, 8), 256, 0, ctx->stream>>>(x, xq, xd, nb);
  return lt_check_launch("k_quant_q8");
}

int lt_silu_mul_quant(lt_ctx* ctx, const float* g, const float* u, int8_t* xq, uint16_t* xd, int K) {
  LT_REQUIRE(ctx && g && u && xq && xd, "lt_silu_mul_quant: null argument");
  LT_REQUIRE(K > 0 && K % 32 == 0, "lt_silu_mul_quant: K=%d must be a positive multiple of 32", K);
  int nb = K / 32;
  k_silu_mul_quant<<<grid_for(nb, 8), 256, 0, ctx->stream>>>(g, u, xq, xd, nb);
  return lt_check_launch("k_silu_mul_quant");
}

int lt_silu_mul(lt_ctx* ctx, const float* g, const float* u, float* y, int n) {
  LT_REQUIRE(ctx && g && u && y, "lt_silu_mul: null argument");
  LT_REQUIRE(n > 0, "lt_silu_mul: n=%d", n);
  k_silu_mul<<<(n + 255) / 256, 256, 0, ctx->stream>>>(g, u, y, n);
  return lt_check_launch("k_silu_mul");
}

int lt_add(lt_ctx* ctx, const float* a, const float* b, float* y, int n) {
  LT_REQUIRE(ctx && a && b && y, "lt_add: null argument");
  LT_REQUIRE(n > 0, "lt_add: n=%d", n);
  k_add<<<(n + 255) / 256, 256, 0, ctx->stream>>>(a, b, y, n);
  return lt_check_launch("k_add");
}

int lt_rmsnorm(lt_ctx* ctx, const float* x, const float* w, float* y, int M, int N, float eps) {
  LT_REQUIRE(ctx && x && w && y, "lt_rmsnorm: null argument");
  LT_REQUIRE(M > 0 && N > 0, "lt_rmsnorm: M=%d N=%d", M, N);
  k_rmsnorm<<<M, 256, 0, ctx->stream>>>(x, w, y, N, eps);
  return lt_check_launch("k_rmsnorm");
}

int lt_rmsnorm_quant(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd, int N,
                     float eps) {
  LT_REQUIRE(ctx && x && w && xq && xd, "lt_rmsnorm_quant: null argument");
  LT_REQUIRE(N > 0 && N % 32 == 0 && N <= 16384, "lt_rmsnorm_quant: N=%d (multiple of 32, <= 16384)", N);
  k_rmsnorm_quant<<<1, 256, (size_t)N * sizeof(float), ctx->stream>>>(x, w, xq, xd, N, eps);
  return lt_check_launch("k_rmsnorm_quant");
}

int lt_rmsnorm_quant_bm(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd, int T, int N,
                        float eps) {
  LT_REQUIRE(ctx && x && w && xq && xd, "lt_rmsnorm_quant_bm: null argument");
  LT_REQUIRE(T > 0 && N > 0 && N % 32 == 0 && N <= 16384, "lt_rmsnorm_quant_bm: T=%d N=%d (N multiple of 32, <= 16384)",
             T, N);
  LT_REQUIRE(lt_aligned(xq, 16) && lt_aligned(xd, 2), "lt_rmsnorm_quant_bm: misaligned argument");
  const size_t shm = (size_t)N * sizeof(float);
  if (N <= 1024) k_rmsnorm_quant_bm<4><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  else if (N <= 4096) k_rmsnorm_quant_bm<16><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  else k_rmsnorm_quant_bm<64><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  return lt_check_launch("k_rmsnorm_quant_bm");
}

int lt_rmsnorm_quant_rows(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd, int T, int N,
                          float eps) {
  LT_REQUIRE(ctx && x && w && xq && xd, "lt_rmsnorm_quant_rows: null argument");
  LT_REQUIRE(T > 0 && N > 0 && N % 32 == 0 && N <= 16384,
             "lt_rmsnorm_quant_rows: T=%d N=%d (N multiple of 32, <= 16384)", T, N);
  LT_REQUIRE(lt_aligned(xq, 16) && lt_aligned(xd, 2), "lt_rmsnorm_quant_rows: misaligned argument");
  const size_t shm = (size_t)N * sizeof(float);
  if (N <= 1024) k_rmsnorm_quant_bm<4, true><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  else if (N <= 4096) k_rmsnorm_quant_bm<16, true><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  else k_rmsnorm_quant_bm<64, true><<<T, 256, shm, ctx->stream>>>(x, w, xq, xd, T, N, eps);
  return lt_check_launch("k_rmsnorm_quant_rows");
}

int lt_q8_gemv_isums(lt_ctx* ctx, const void* W, const int8_t* xq, int32_t* isum, int N, int K) {
  LT_REQUIRE(ctx && W && xq && isum, "lt_q8_gemv_isums: null argument");
  LT_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "lt_q8_gemv_isums: N=%d K=%d", N, K);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(xq, 16), "lt_q8_gemv_isums: misaligned W or xq");
  k_q8_gemv_isums<<<grid_for(N, 8), 256, 0, ctx->stream>>>((const uint8_t*)W, xq, isum, N, K);
  return lt_check_launch("k_q8_gemv_isums");
}

int lt_rope_freqs(int hd, float theta, float* host_freqs) {
  LT_REQUIRE(host_freqs && hd > 0 && hd % 2 == 0, "lt_rope_freqs: hd=%d", hd);
  for (int j = 0; j < hd / 2; j++) {
    float e = -(2.0f * (float)j) / (float)hd;
    host_freqs[j] = (float)pow((double)theta, (double)e);
  }
  return LT_OK;
}

int lt_rope_qk(lt_ctx* ctx, float* qk, const int* pos, int nheads, int hd, const float* freqs) {
  LT_REQUIRE(ctx && qk && pos && freqs, "lt_rope_qk: null argument");
  LT_REQUIRE(nheads > 0 && hd > 0 && hd % 2 == 0, "lt_rope_qk: nheads=%d hd=%d", nheads, hd);
  int total = nheads * (hd / 2);
  k_rope<<<grid_for(total, 256), 256, 0, ctx->stream>>>(qk, pos, nheads, hd, freqs);
  return lt_check_launch("k_rope");
}

int lt_kv_append_incr(lt_ctx* ctx, void* kc, const float* k, void* vc, const float* v, int* len,
                      int width, int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && kc && k && vc && v && len, "lt_kv_append_incr: null argument");
  LT_REQUIRE(width > 0 && maxt > 0, "lt_kv_append_incr: width=%d maxt=%d", width, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_kv_append_incr: kv_dtype=%d", kv_dtype);
  if (kv_dtype == LT_KV_F16)
    k_kv_append_incr<true><<<1, 256, 0, ctx->stream>>>(kc, k, vc, v, len, width, maxt);
  else
    k_kv_append_incr<false><<<1, 256, 0, ctx->stream>>>(kc, k, vc, v, len, width, maxt);
  return lt_check_launch("k_kv_append_incr");
}

int lt_embed_q8(lt_ctx* ctx, const void* emb, const int* tok, float* x, int E, int vocab, int* err) {
  LT_REQUIRE(ctx && emb && tok && x, "lt_embed_q8: null argument");
  LT_REQUIRE(E > 0 && E % 32 == 0 && vocab > 0, "lt_embed_q8: E=%d vocab=%d", E, vocab);
  k_embed_q8<<<grid_for(E, 256), 256, 0, ctx->stream>>>((const uint8_t*)emb, tok, x, E, vocab, err);
  return lt_check_launch("k_embed_q8");
}

size_t lt_argmax_workspace_size(void) { return (size_t)kArgmaxBlocks * 8; }

static int argmax_impl(lt_ctx* ctx, const float* x, int n, int* out, int* hist, int* count, int cap,
                       void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && x && out && ws, "lt_argmax: null argument");
  LT_REQUIRE(n > 0, "lt_argmax: n=%d must be > 0", n);
  if (ws_bytes < lt_argmax_workspace_size())
    return lt_fail(LT_ENOMEM, "lt_argmax: workspace %zu < %zu bytes", ws_bytes, lt_argmax_workspace_size());
  LT_REQUIRE(lt_aligned(ws, 4), "lt_argmax: workspace must be 4-byte aligned");
  float* pval = (float*)ws;
  int* pidx = (int*)((char*)ws + kArgmaxBlocks * 4);
  k_argmax_s1<<<kArgmaxBlocks, 256, 0, ctx->stream>>>(x, n, pval, pidx);
  int rc = lt_check_launch("k_argmax_s1");
  if (rc) return rc;
  k_argmax_s2<<<1, 256, 0, ctx->stream>>>(pval, pidx, out, hist, count, cap);
  return lt_check_launch("k_argmax_s2");
}

int lt_argmax(lt_ctx* ctx, const float* x, int n, int* out, void* ws, size_t ws_bytes) {
  return argmax_impl(ctx, x, n, out, nullptr, nullptr, 0, ws, ws_bytes);
}

int lt_argmax_record(lt_ctx* ctx, const float* x, int n, int* out, int* hist, int* count, int cap,
                     void* ws, size_t ws_bytes) {
  LT_REQUIRE(hist && count && cap > 0, "lt_argmax_record: null history or cap=%d", cap);
  return argmax_impl(ctx, x, n, out, hist, count, cap, ws, ws_bytes);
}

int lt_argmax_rows(lt_ctx* ctx, const float* x, int rows, int n, int* out, int* hist, int* count, int cap) {
  LT_REQUIRE(ctx && x && out, "lt_argmax_rows: null argument");
  LT_REQUIRE(rows > 0 && n > 0, "lt_argmax_rows: rows=%d n=%d", rows, n);
  LT_REQUIRE(!hist || (count && cap > 0), "lt_argmax_rows: a history needs count and cap > 0");
  k_argmax_rows<<<rows, 1024, 0, ctx->stream>>>(x, n, out, hist, count, cap);
  return lt_check_launch("k_argmax_rows");
}

size_t lt_argmax_rows_workspace_size(int rows) { return rows > 0 ? (size_t)rows * kArgmaxSlices * 8u : 0; }

int lt_argmax_rows_ws(lt_ctx* ctx, const float* x, int rows, int n, int* out, int* hist, int* count, int cap,
                      void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && x && out && ws, "lt_argmax_rows_ws: null argument");
  LT_REQUIRE(rows > 0 && n > 0 && rows <= 65535, "lt_argmax_rows_ws: rows=%d n=%d", rows, n);
  LT_REQUIRE(!hist || (count && cap > 0), "lt_argmax_rows_ws: a history needs count and cap > 0");
  LT_REQUIRE(ws_bytes >= lt_argmax_rows_workspace_size(rows) && lt_aligned(ws, 4),
             "lt_argmax_rows_ws: workspace of %zu bytes, %zu needed (4-byte aligned)", ws_bytes,
             lt_argmax_rows_workspace_size(rows));
  float* wv = (float*)ws;
  int* wi = (int*)(wv + (size_t)rows * kArgmaxSlices);
  k_argmax_rows_part<<<dim3(kArgmaxSlices, rows), 1024, 0, ctx->stream>>>(x, n, wv, wi);
  if (int rc = lt_check_launch("k_argmax_rows_part")) return rc;
  k_argmax_rows_fin<<<rows, 64, 0, ctx->stream>>>(wv, wi, out, hist, count, cap);
  return lt_check_launch("k_argmax_rows_fin");
}

int lt_selftest_numerics(lt_ctx* ctx, unsigned long long* out) {
  LT_REQUIRE(ctx && out, "lt_selftest_numerics: null argument");
  unsigned long long* d = nullptr;
  LT_CHECK(hipMalloc(&d, 4 * sizeof(unsigned long long)));
  hipError_t e = hipMemsetAsync(d, 0, 4 * sizeof(unsigned long long), ctx->stream);
  if (e == hipSuccess) {
    k_check_f2h<<<4096, 256, 0, ctx->stream>>>(d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    k_check_quotient<<<0x7BFF, 256, 0, ctx->stream>>>(d + 1);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(out, d, 4 * sizeof(unsigned long long), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  hipFree(d);
  if (e != hipSuccess) return lt_fail_hip(e, "lt_selftest_numerics", __FILE__, __LINE__);
  return LT_OK;
}

}  // extern "C"
