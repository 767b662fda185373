// lt_attn.hip -- GQA decode attention over a position-major KV cache, fp32 or fp16.
//
// One workgroup per (split, group of HPW query heads sharing one KV head, sequence).
// A workgroup scores its contiguous range of positions for all HPW heads at once, so
// each K row is read once for the group; then it folds max and Z per head and the
// exp-weighted V sum per (head, dim).  The arithmetic of each head is exactly the
// reference's:
//   score  s_t = (sequential fma over i of q_i*K_t,i) * scale
//            (bpd/lib/dev_residency.py:1987-1991);
//   max    order-free (fmax);
//   e_t    = exp(s_t - m);
//   Z      64-lane strided sum fold over the range, then a 6-level shuffle-down tree
//            (the frozen RLANES = 64 order, dev_residency.py:1968-2000);
//   O_d    sequential fma fold over the range in ascending t.
// nsplit == 1 writes out = O/Z directly: the single-pass k_attn_decode_masked order
// (positions >= L contribute exactly nothing there, so maxt does not enter the result).
// nsplit > 1 writes per-split (m, Z, O) and k_attn_combine merges them in ascending
// split order, the declared order attn_decode_split (bpd/lib/ir_param_axes.pl:303-341,
// bpd/kernelgen/experimental/attn_decode_split.cu:37-91).
#include "lt_internal.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool kF16>
__device__ __forceinline__ void load8(const void* base, size_t idx, float v[8]) {
  if (kF16) {
    u32x4 w;
    __builtin_memcpy(&w, (const uint16_t*)base + idx, 16);
    uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = lt_h2f((uint16_t)(a[i] & 0xFFFFu));
      v[2 * i + 1] = lt_h2f((uint16_t)(a[i] >> 16));
    }
  } else {
    u32x4 w0, w1;
    __builtin_memcpy(&w0, (const float*)base + idx, 16);
    __builtin_memcpy(&w1, (const float*)base + idx + 4, 16);
    uint32_t a[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_bit_cast(float, a[i]);
  }
}

template <bool kF16>
__device__ __forceinline__ void load2(const void* base, size_t idx, float& a, float& b) {
  if (kF16) {
    uint32_t w;
    __builtin_memcpy(&w, (const uint16_t*)base + idx, 4);
    a = lt_h2f((uint16_t)(w & 0xFFFFu));
    b = lt_h2f((uint16_t)(w >> 16));
  } else {
    const float* p = (const float*)base + idx;
    a = p[0];
    b = p[1];
  }
}

// prefill != 0: the batch is T query tokens of one sequence sharing one cache, query b
// attending *len + b + 1 positions (causal); q rows are q_stride floats apart.
template <bool kF16, bool kSplit, int HPW>
__global__ __launch_bounds__(256) void k_attn_decode(
    const float* __restrict__ q, const void* __restrict__ kc, const void* __restrict__ vc,
    const int* __restrict__ len, float* __restrict__ out, float* __restrict__ wsm,
    float* __restrict__ wsz, float* __restrict__ wso, int nh, int nkv, int hd, float scale,
    int maxt, int nsplit, int per_max, int q_stride, int prefill) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* sq = lds;             // [HPW][hd]
  float* se = lds + HPW * hd;  // [HPW][per_max]
  __shared__ float s_mx[HPW];
  __shared__ float s_z[HPW];

  const int tid = threadIdx.x;
  const int sp = blockIdx.x;
  const int h0 = blockIdx.y * HPW;
  const int b = blockIdx.z;
  const int rep = nh / nkv;
  const int g = h0 / rep;

  int L = prefill ? len[0] + b + 1 : len[b];
  L = L < 0 ? 0 : (L > maxt ? maxt : L);
  const int per = (L + nsplit - 1) / nsplit;
  const int p0 = sp * per;
  int p1 = p0 + per;
  if (p1 > L) p1 = L;
  const int n = p1 > p0 ? p1 - p0 : 0;

  const size_t kvrow = (size_t)nkv * hd;
  const size_t seq_base = prefill ? 0 : (size_t)b * (size_t)maxt * kvrow;
  const size_t head_base = seq_base + (size_t)p0 * kvrow + (size_t)g * hd;

  for (int i = tid; i < HPW * hd; i += 256) sq[i] = q[(size_t)b * q_stride + (size_t)h0 * hd + i];
  __syncthreads();

  // scores: thread per position, HPW sequential-fma chains over i
  for (int t = tid; t < n; t += 256) {
    float acc[HPW];
#pragma unroll
    for (int r = 0; r < HPW; r++) acc[r] = 0.0f;
    const size_t rowi = head_base + (size_t)t * kvrow;
    for (int i0 = 0; i0 < hd; i0 += 8) {
      float kv[8];
      load8<kF16>(kc, rowi + i0, kv);
#pragma unroll
      for (int ii = 0; ii < 8; ii++)
#pragma unroll
        for (int r = 0; r < HPW; r++) acc[r] = fmaf(sq[r * hd + i0 + ii], kv[ii], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < HPW; r++) se[r * per_max + t] = acc[r] * scale;
  }
  __syncthreads();

  const int wave = tid >> 6, lane = tid & 63;
  for (int r = wave; r < HPW; r += 4) {
    float m = -1e30f;
    for (int t = lane; t < n; t += 64) m = fmaxf(m, se[r * per_max + t]);
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
    if (lane == 0) s_mx[r] = m;
  }
  __syncthreads();

  for (int r = 0; r < HPW; r++) {
    const float m = s_mx[r];
    for (int t = tid; t < n; t += 256) se[r * per_max + t] = lt_expf(se[r * per_max + t] - m);
  }
  __syncthreads();

  for (int r = wave; r < HPW; r += 4) {
    float ls = 0.0f;
    for (int t = lane; t < n; t += 64) ls = ls + se[r * per_max + t];
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) ls = ls + __shfl_down(ls, s, 64);
    if (lane == 0) s_z[r] = ls;
  }
  __syncthreads();

  // O: thread per (head, dim pair); two independent sequential chains over t
  const int hpairs = hd >> 1;
  for (int idx = tid; idx < HPW * hpairs; idx += 256) {
    const int r = idx / hpairs;
    const int d = (idx - r * hpairs) * 2;
    const float* e = se + r * per_max;
    float a0 = 0.0f, a1 = 0.0f;
    int t = 0;
    for (; t + 8 <= n; t += 8) {
      float v0[8], v1[8];
#pragma unroll
      for (int u = 0; u < 8; u++) load2<kF16>(vc, head_base + (size_t)(t + u) * kvrow + d, v0[u], v1[u]);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        a0 = fmaf(e[t + u], v0[u], a0);
        a1 = fmaf(e[t + u], v1[u], a1);
      }
    }
    for (; t < n; t++) {
      float x0, x1;
      load2<kF16>(vc, head_base + (size_t)t * kvrow + d, x0, x1);
      a0 = fmaf(e[t], x0, a0);
      a1 = fmaf(e[t], x1, a1);
    }
    const size_t hrow = (size_t)b * nh + h0 + r;
    if (!kSplit) {
      out[hrow * hd + d] = a0 / s_z[r];
      out[hrow * hd + d + 1] = a1 / s_z[r];
    } else {
      float* o = wso + (hrow * nsplit + sp) * hd + d;
      o[0] = a0;
      o[1] = a1;
    }
  }
  if (kSplit && tid < HPW) {
    const size_t hrow = (size_t)b * nh + h0 + tid;
    wsm[hrow * nsplit + sp] = s_mx[tid];
    wsz[hrow * nsplit + sp] = s_z[tid];
  }
}

__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ wsm,
                                                      const float* __restrict__ wsz,
                                                      const float* __restrict__ wso,
                                                      float* __restrict__ out, int nh, int hd,
                                                      int nsplit) {
  const size_t hrow = (size_t)blockIdx.y * nh + blockIdx.x;
  const float* m = wsm + hrow * nsplit;
  const float* z = wsz + hrow * nsplit;
  float M = -1e30f;
  for (int s = 0; s < nsplit; s++) M = fmaxf(M, m[s]);
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float Z = 0.0f, acc = 0.0f;
    for (int s = 0; s < nsplit; s++) {
      const float w = lt_expf(m[s] - M);
      Z = fmaf(w, z[s], Z);
      acc = fmaf(w, wso[(hrow * nsplit + s) * hd + d], acc);
    }
    out[hrow * hd + d] = acc / Z;
  }
}

template <bool kF16, bool kSplit>
hipError_t launch_attn(int hpw, dim3 grid, size_t shm, hipStream_t st, const float* q, const void* kc,
                       const void* vc, const int* len, float* out, float* wsm, float* wsz, float* wso,
                       int nh, int nkv, int hd, float scale, int maxt, int nsplit, int per_max,
                       int q_stride, int prefill) {
#define LT_ATTN_CASE(H)                                                                      \
  case H:                                                                                    \
    k_attn_decode<kF16, kSplit, H><<<grid, 256, shm, st>>>(q, kc, vc, len, out, wsm, wsz, wso, \
                                                           nh, nkv, hd, scale, maxt, nsplit,  \
                                                           per_max, q_stride, prefill);       \
    break;
  switch (hpw) {
    LT_ATTN_CASE(1)
    LT_ATTN_CASE(2)
    LT_ATTN_CASE(4)
    LT_ATTN_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef LT_ATTN_CASE
  return hipGetLastError();
}

}  // namespace

extern "C" {

size_t lt_attn_workspace_size(int batch, int nh, int hd, int nsplit) {
  if (nsplit <= 1 || batch <= 0 || nh <= 0 || hd <= 0) return 0;
  return lt_attn_ws_bytes(batch * nh, hd, nsplit);
}

static int attn_impl(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                     float* out, int batch, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                     int kv_dtype, void* ws, size_t ws_bytes, int q_stride, int prefill) {
  LT_REQUIRE(ctx && q && kc && vc && len && out, "lt_attn_decode: null argument");
  LT_REQUIRE(q_stride >= nh * hd, "lt_attn: q_stride=%d < nh*hd", q_stride);
  LT_REQUIRE(batch > 0 && nh > 0 && nkv > 0 && nh % nkv == 0, "lt_attn_decode: batch=%d nh=%d nkv=%d", batch, nh, nkv);
  LT_REQUIRE(hd > 0 && hd % 8 == 0 && hd <= 512, "lt_attn_decode: hd=%d (multiple of 8, <= 512)", hd);
  LT_REQUIRE(maxt > 0 && nsplit >= 1 && nsplit <= maxt, "lt_attn_decode: maxt=%d nsplit=%d", maxt, nsplit);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_attn_decode: kv_dtype=%d", kv_dtype);
  LT_REQUIRE(lt_aligned(kc, 16) && lt_aligned(vc, 16), "lt_attn_decode: K/V caches must be 16-byte aligned");
  const int rep = nh / nkv;
  int hpw = 1;
  if (nsplit > 1) {
    for (int c : {8, 4, 2})
      if (rep % c == 0) { hpw = c; break; }
  }
  const int per_max = (maxt + nsplit - 1) / nsplit;
  const size_t shm = (size_t)hpw * (hd + per_max) * sizeof(float);
  if (shm > 64 * 1024)
    return lt_fail(LT_EINVAL, "lt_attn_decode: %zu bytes of LDS for maxt=%d nsplit=%d; raise nsplit", shm, maxt, nsplit);
  dim3 grid(nsplit, nh / hpw, batch);
  float *wsm = nullptr, *wsz = nullptr, *wso = nullptr;
  if (nsplit > 1) {
    size_t need = lt_attn_workspace_size(batch, nh, hd, nsplit);
    LT_REQUIRE(ws != nullptr, "lt_attn_decode: nsplit=%d needs a workspace", nsplit);
    if (ws_bytes < need) return lt_fail(LT_ENOMEM, "lt_attn_decode: workspace %zu < %zu bytes", ws_bytes, need);
    LT_REQUIRE(lt_aligned(ws, 16), "lt_attn_decode: workspace must be 16-byte aligned");
    const AttnWs w = lt_attn_ws_layout(ws, batch * nh, hd, nsplit);
    wsm = w.m;
    wsz = w.z;
    wso = w.o;
  }
  hipError_t e;
  const bool f16 = kv_dtype == LT_KV_F16;
  if (nsplit == 1)
    e = f16 ? launch_attn<true, false>(hpw, grid, shm, ctx->stream, q, kc, vc, len, out, wsm, wsz, wso, nh, nkv, hd, scale, maxt, nsplit, per_max, q_stride, prefill)
            : launch_attn<false, false>(hpw, grid, shm, ctx->stream, q, kc, vc, len, out, wsm, wsz, wso, nh, nkv, hd, scale, maxt, nsplit, per_max, q_stride, prefill);
  else
    e = f16 ? launch_attn<true, true>(hpw, grid, shm, ctx->stream, q, kc, vc, len, out, wsm, wsz, wso, nh, nkv, hd, scale, maxt, nsplit, per_max, q_stride, prefill)
            : launch_attn<false, true>(hpw, grid, shm, ctx->stream, q, kc, vc, len, out, wsm, wsz, wso, nh, nkv, hd, scale, maxt, nsplit, per_max, q_stride, prefill);
  if (e != hipSuccess) return lt_fail_hip(e, "k_attn_decode launch", __FILE__, __LINE__);
  if (nsplit > 1) {
    k_attn_combine<<<dim3(nh, batch), hd < 256 ? hd : 256, 0, ctx->stream>>>(wsm, wsz, wso, out, nh, hd, nsplit);
    return lt_check_launch("k_attn_combine");
  }
  return LT_OK;
}

int lt_attn_decode(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                   float* out, int batch, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                   int kv_dtype, void* ws, size_t ws_bytes) {
  return attn_impl(ctx, q, kc, vc, len, out, batch, nh, nkv, hd, scale, maxt, nsplit, kv_dtype, ws, ws_bytes,
                   nh * hd, 0);
}

int lt_attn_prefill(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc, const int* len0,
                    float* out, int T, int nh, int nkv, int hd, float scale, int maxt, int nsplit, int kv_dtype,
                    void* ws, size_t ws_bytes) {
  return attn_impl(ctx, q, kc, vc, len0, out, T, nh, nkv, hd, scale, maxt, nsplit, kv_dtype, ws, ws_bytes,
                   q_stride, 1);
}

}  // extern "C"
