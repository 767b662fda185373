// lt_multi.hip -- the Q8_0 GEMV over several tokens at once, for the batched decode step at
// small batch: each weight block a workgroup loads is folded against every one of its tokens'
// quantized activations (2 to 8 tokens per workgroup, so a step of B tokens reads each weight
// matrix from HBM once and from L2 a few times; the prefill GEMM streams it once too, but it
// is tuned for hundreds of tokens and takes 5x the single-token time at B = 8).
//
// Per (row, token) the arithmetic is the single-token GEMV's, bit for bit: lane L of the
// row's half-wave folds blocks L, L+32, ... with acc = fma(wd*xd, (float)isum, acc) (exact
// int32 block dot by v_dot4), then the 5-level half-wave tree (the reference's lanes(32)
// strided accum(fma) tree(shfl_down,5), q8_0_from_facts.pl:466-476).
//
// Layout: row-major activation quants xq [T][K], xd [T][K/32] (lt_quant_q8 /
// lt_rmsnorm_quant_rows over the T rows); a workgroup of 8 half-waves takes 8 consecutive rows
// and NT tokens (gridDim.y covers T in groups of NT), stages the NT tokens' quants in LDS once
// (coalesced 16-byte loads, all in flight), and every half-wave streams its row's blocks --
// each re-aligned to dwords once (load_q8_block) -- against all of them (fold_block, the same
// fma as fold_raw).
#include <cstdlib>

#include "lt_internal.h"
#include "lt_q8_device.h"

using namespace lt;

namespace {

constexpr int kMtThreads = 256;
constexpr int kMtRows = kMtThreads / 32;
constexpr size_t kMtLdsMax = (size_t)150 * 1024;

enum MtEpi { MT_STORE = 0, MT_RESID = 1, MT_SILU = 2, MT_ROPE = 3 };

// MT_ROPE: the q|k|v rows of the next token of each of T sequences, then RoPE and the KV
// append of lt_rope_append_seqs (row t: sequence t, position len[t], its cache rows at
// kc/vc + t*maxt*nkv*hd elements)
struct MtRope {
  const int* len;
  const float* freqs;   // [hd/2]
  void* kc;
  void* vc;
  int nh, nkv, hd, maxt, f16;
};

// EPI: MT_STORE y[t][row] = v (+ add[row], a bias); MT_RESID y[t][row] = v + add[t][row];
// MT_SILU rows 2j, 2j+1 are gate j and up j (interleaved): y[t][j] = SiLU(g)*u, y [T][N/2];
// MT_ROPE the rows of 4 rotation pairs of one head (half-waves 0-3 rows j .. j+3 of the head,
// 4-7 rows j + hd/2 .. j + hd/2 + 3), v + add[row] (the bias), then q rotated into y[t][row],
// k rotated and v as they are into sequence t's cache row len[t], k and v also into y as
// they are.
template <int NT, int EPI>
__global__ __launch_bounds__(kMtThreads) void k_gemv_multi(const uint8_t* __restrict__ W,
                                                           const int8_t* __restrict__ xq,
                                                           const uint16_t* __restrict__ xd, int T,
                                                           const float* __restrict__ add, float* __restrict__ y,
                                                           int N, int K, MtRope R) {
  extern __shared__ __attribute__((aligned(16))) int8_t sxq[];   // [NT][K] quants, then [NT][nb] scales
  __shared__ float s_v[NT][kMtRows];
  const int nb = K >> 5;
  const int lane = threadIdx.x & 31, hw = threadIdx.x >> 5;
  // MT_ROPE: workgroup x holds pairs 4c .. 4c+3 of head x / (hd/8), c = x mod (hd/8)
  const int rq = EPI == MT_ROPE ? R.hd >> 3 : 1;
  const int rhead = EPI == MT_ROPE ? (int)blockIdx.x / rq : 0;
  const int rj0 = EPI == MT_ROPE ? ((int)blockIdx.x - rhead * rq) * 4 : 0;
  const int row = EPI == MT_ROPE ? rhead * R.hd + ((hw & 4) ? (R.hd >> 1) : 0) + rj0 + (hw & 3)
                                 : (int)blockIdx.x * kMtRows + hw;
  const int t0 = blockIdx.y * NT;
  const int nt = T - t0 < NT ? T - t0 : NT;
  uint16_t* sxd = (uint16_t*)(sxq + (size_t)NT * K);
  const size_t last = (size_t)N * nb - 1;
  const size_t g0 = (size_t)(row < N ? row : 0) * nb;   // the row's first global block index

  // this lane's first two blocks are requested before the activations are staged
  BlockRegs r0, r1;
  const bool has0 = row < N && lane < nb, has1 = row < N && lane + 32 < nb;
  if (has0) load_q8_block(W, g0 + lane, last, r0);
  if (has1) load_q8_block(W, g0 + lane + 32, last, r1);

  // the nt tokens' quants (nt*K contiguous bytes) and scales into LDS, every load in flight
  {
    const u32x4* src = (const u32x4*)(xq + (size_t)t0 * K);
    u32x4* dst = (u32x4*)sxq;
    const int n16 = nt * K / 16;
    for (int i = threadIdx.x; i < n16; i += kMtThreads) dst[i] = src[i];
    const uint16_t* dsrc = xd + (size_t)t0 * nb;
    for (int i = threadIdx.x; i < nt * nb; i += kMtThreads) sxd[i] = dsrc[i];
  }
  __syncthreads();

  float acc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++) acc[tt] = 0.0f;
  auto fold = [&](const BlockRegs& r, int b) {
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
      if (tt < nt) acc[tt] = fold_block(r, sxq + (size_t)tt * K + (size_t)b * 32, sxd[tt * nb + b], acc[tt]);
  };
  if (has0) fold(r0, lane);
  if (has1) fold(r1, lane + 32);
  // blocks past the first 64 of the row: two in flight per lane
  for (int b = lane + 64; b < nb && row < N; b += 64) {
    BlockRegs ra, rb;
    const bool hb = b + 32 < nb;
    load_q8_block(W, g0 + b, last, ra);
    if (hb) load_q8_block(W, g0 + b + 32, last, rb);
    fold(ra, b);
    if (hb) fold(rb, b + 32);
  }

  // the half-wave tree per token; lane 0 holds the row's value
  float v[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++) v[tt] = halfwave_tree_dpp(lane < nb ? acc[tt] : 0.0f);
  if constexpr (EPI == MT_SILU) {
    if (lane == 0)
#pragma unroll
      for (int tt = 0; tt < NT; tt++) s_v[tt][hw] = v[tt];
    __syncthreads();
    // 4 gate/up pairs per workgroup: thread (token tt, pair p)
    const int i = threadIdx.x;
    if (i < NT * (kMtRows / 2)) {
      const int tt = i / (kMtRows / 2), p = i - tt * (kMtRows / 2);
      const int j = blockIdx.x * (kMtRows / 2) + p;
      if (tt < nt && 2 * j + 1 < N) y[(size_t)(t0 + tt) * (N / 2) + j] = lt_silu_mul(s_v[tt][2 * p], s_v[tt][2 * p + 1]);
    }
  } else if constexpr (EPI == MT_ROPE) {
    // the biased rows into LDS, then thread (token tt, pair p) rotates rows j and j + hd/2
    // (k_rope_append_batch's arithmetic: sin/cos of pos * freqs[j], two fmas)
    if (lane == 0)
#pragma unroll
      for (int tt = 0; tt < NT; tt++) s_v[tt][hw] = add ? v[tt] + add[row] : v[tt];
    __syncthreads();
    const int i = threadIdx.x;
    if (i < NT * 4) {
      const int tt = i >> 2, p = i & 3;
      const int t = t0 + tt;
      if (tt < nt) {
        const int half = R.hd >> 1, j = rj0 + p;
        const int pos = R.len[t];
        float sn, cs;
        lt_sincosf((float)pos * R.freqs[j], &sn, &cs);
        const float x1 = s_v[tt][p], x2 = s_v[tt][p + 4];
        const int width = R.nkv * R.hd;
        const bool app = pos >= 0 && pos < R.maxt;
        const size_t cbase = ((size_t)t * R.maxt + (size_t)(app ? pos : 0)) * width;
        auto put = [&](void* c, size_t off, float val) {
          if (R.f16) ((uint16_t*)c)[off] = lt_float_to_half_bits(val);
          else ((float*)c)[off] = val;
        };
        const size_t o = (size_t)t * N + (size_t)rhead * R.hd + j;
        if (rhead < R.nh + R.nkv) {
          const float o1 = fmaf(x1, cs, -(x2 * sn));
          const float o2 = fmaf(x1, sn, x2 * cs);
          if (rhead < R.nh) {
            y[o] = o1;
            y[o + half] = o2;
          } else if (app) {
            const size_t off = cbase + (size_t)(rhead - R.nh) * R.hd + j;
            put(R.kc, off, o1);
            put(R.kc, off + half, o2);
          }
        } else if (app) {
          const size_t off = cbase + (size_t)(rhead - R.nh - R.nkv) * R.hd + j;
          put(R.vc, off, x1);
          put(R.vc, off + half, x2);
        }
        // k and v rows stay in y as the GEMV left them (as lt_rope_append_seqs leaves them)
        if (rhead >= R.nh) {
          y[o] = x1;
          y[o + half] = x2;
        }
      }
    }
  } else {
    if (lane == 0 && row < N) {
#pragma unroll
      for (int tt = 0; tt < NT; tt++) {
        if (tt < nt) {
          const size_t o = (size_t)(t0 + tt) * N + row;
          float r = v[tt];
          if (EPI == MT_STORE && add) r = r + add[row];
          if (EPI == MT_RESID) r = r + add[o];
          y[o] = r;
        }
      }
    }
  }
}

// Tokens per workgroup (a power of two; fewer tokens = more workgroups, each re-reading its rows
// from L2): 4, or 2 for matrices of at most 2048 rows at up to 8 tokens (down 896 x 4864 at
// T = 8: 6.5 us with 2, 7.9 with 4, 11.2 with 8; gate|up 9728 x 896 within 5% across 4 and 8);
// never more than T needs, and within the LDS budget.  LT_MULTI_NT=n sets it, for sweeps.
int mt_tokens(int K, int T, int N) {
  static const int env = [] {
    const char* s = getenv("LT_MULTI_NT");
    const int v = s ? atoi(s) : 0;
    return v == 1 || v == 2 || v == 4 || v == 8 ? v : 0;
  }();
  const size_t per = (size_t)K + (size_t)(K / 32) * 2;
  int nt = env ? env : (T <= 8 && N <= 2048 ? 2 : 4);
  while (nt > 1 && ((size_t)nt * per > kMtLdsMax || nt / 2 >= T)) nt /= 2;
  return (size_t)nt * per > kMtLdsMax ? 0 : nt;
}

template <int EPI>
hipError_t launch_mt(int nt, dim3 grid, size_t shm, hipStream_t st, const uint8_t* W, const int8_t* xq,
                     const uint16_t* xd, int T, const float* add, float* y, int N, int K, MtRope R = MtRope{}) {
  switch (nt) {
    case 8: k_gemv_multi<8, EPI><<<grid, kMtThreads, shm, st>>>(W, xq, xd, T, add, y, N, K, R); break;
    case 4: k_gemv_multi<4, EPI><<<grid, kMtThreads, shm, st>>>(W, xq, xd, T, add, y, N, K, R); break;
    case 2: k_gemv_multi<2, EPI><<<grid, kMtThreads, shm, st>>>(W, xq, xd, T, add, y, N, K, R); break;
    default: k_gemv_multi<1, EPI><<<grid, kMtThreads, shm, st>>>(W, xq, xd, T, add, y, N, K, R); break;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" {

int lt_q8_gemv_multi(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, int T, const float* add,
                     float* y, int N, int K, int epi) {
  LT_REQUIRE(ctx && W && xq && xd && y, "lt_q8_gemv_multi: null argument");
  LT_REQUIRE(T > 0 && N > 0 && K > 0 && K % 32 == 0, "lt_q8_gemv_multi: T=%d N=%d K=%d", T, N, K);
  LT_REQUIRE(epi == MT_STORE || epi == MT_RESID || epi == MT_SILU, "lt_q8_gemv_multi: epi=%d", epi);
  LT_REQUIRE(epi != MT_RESID || add, "lt_q8_gemv_multi: the residual epilogue needs add");
  LT_REQUIRE(epi != MT_SILU || N % 2 == 0, "lt_q8_gemv_multi: SiLU rows come in gate/up pairs (N=%d)", N);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(xq, 16), "lt_q8_gemv_multi: W 4-byte and xq 16-byte aligned");
  const int nt = mt_tokens(K, T, N);
  LT_REQUIRE(nt > 0, "lt_q8_gemv_multi: K=%d: one token's quants exceed the LDS budget", K);
  const size_t shm = (size_t)nt * ((size_t)K + (size_t)(K / 32) * 2);
  const dim3 grid((N + kMtRows - 1) / kMtRows, (T + nt - 1) / nt);
  const uint8_t* w = (const uint8_t*)W;
  hipError_t e;
  if (epi == MT_STORE) e = launch_mt<MT_STORE>(nt, grid, shm, ctx->stream, w, xq, xd, T, add, y, N, K);
  else if (epi == MT_RESID) e = launch_mt<MT_RESID>(nt, grid, shm, ctx->stream, w, xq, xd, T, add, y, N, K);
  else e = launch_mt<MT_SILU>(nt, grid, shm, ctx->stream, w, xq, xd, T, add, y, N, K);
  if (e != hipSuccess) return lt_fail_hip(e, "k_gemv_multi", __FILE__, __LINE__);
  return LT_OK;
}

int lt_q8_gemv_multi_rope(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, int T,
                          const float* bias, float* qkv, int N, int K, const int* len, int nh, int nkv, int hd,
                          const float* freqs, void* kc, void* vc, int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && W && xq && xd && qkv && len && freqs && kc && vc, "lt_q8_gemv_multi_rope: null argument");
  LT_REQUIRE(T > 0 && K > 0 && K % 32 == 0 && nh > 0 && nkv > 0 && hd > 0 && hd % 8 == 0 && hd <= 256 &&
                 maxt > 0 && N == (nh + 2 * nkv) * hd,
             "lt_q8_gemv_multi_rope: T=%d N=%d K=%d nh=%d nkv=%d hd=%d maxt=%d (N = (nh + 2 nkv) hd, hd a multiple "
             "of 8)", T, N, K, nh, nkv, hd, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_q8_gemv_multi_rope: kv_dtype=%d", kv_dtype);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(xq, 16), "lt_q8_gemv_multi_rope: W 4-byte and xq 16-byte aligned");
  const int nt = mt_tokens(K, T, N);
  LT_REQUIRE(nt > 0, "lt_q8_gemv_multi_rope: K=%d: one token's quants exceed the LDS budget", K);
  const size_t shm = (size_t)nt * ((size_t)K + (size_t)(K / 32) * 2);
  // one workgroup per 4 rotation pairs of a head: (nh + 2 nkv) * hd / 8 = N / 8 workgroups
  const dim3 grid(N / kMtRows, (T + nt - 1) / nt);
  MtRope R{len, freqs, kc, vc, nh, nkv, hd, maxt, kv_dtype == LT_KV_F16 ? 1 : 0};
  const hipError_t e =
      launch_mt<MT_ROPE>(nt, grid, shm, ctx->stream, (const uint8_t*)W, xq, xd, T, bias, qkv, N, K, R);
  if (e != hipSuccess) return lt_fail_hip(e, "k_gemv_multi", __FILE__, __LINE__);
  return LT_OK;
}

}  // extern "C"
