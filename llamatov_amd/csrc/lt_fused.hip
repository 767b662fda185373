// lt_fused.hip -- the fused decode-step kernels of libllamatov_hip.so.
//
// A decode token on MI355X is bound by the fixed cost of each launch (a replayed graph
// node costs ~1.5 us even when empty), so the step is cut to five launches per layer
// instead of thirteen, each one a reference op chain fused without changing a bit:
//
//   lt_q8_gemv_rms / _embed_rms   rmsnorm -> quant -> QKV GEMV (+bias)
//   lt_attn_step                  RoPE(q,k) -> KV append -> masked attention
//   lt_q8_gemv_attn_out           split-K merge -> quant -> O GEMV (+x), length bump
//   lt_q8_gemv_rms_silu           rmsnorm -> quant -> gate|up GEMV -> SiLU(g)*u
//   lt_q8_gemv_quant              quant -> down GEMV (+xres)
// and per token lt_q8_gemv_rms_argmax (final norm -> quant -> vocab GEMV -> argmax).
//
// Every workgroup of a fused GEMV builds the quantized activation itself, in LDS (the
// prologue), before it streams its rows of the weight matrix; the prologue's inputs are
// a few KB and stay in L2, so the redundancy costs far less than a launch.  The
// weight loads of a workgroup's first rows are issued before the prologue, so the
// prologue runs under their HBM latency.  The arithmetic of each stage is the per-op
// kernel's (lt_ops.hip, lt_attn.hip) operation for operation.
#include "lt_q8_device.h"

#include <cstdlib>
#include <mutex>

namespace {

using namespace lt;

enum Pro { PRO_STAGE = 0, PRO_QUANT = 1, PRO_RMS = 2, PRO_EMBED_RMS = 3, PRO_MERGE = 4 };
enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_ARGMAX = 3, EPI_SWIGLU = 4, EPI_ROPE_KV = 5 };

struct GemvParams {
  const uint8_t* W;
  int N, K;
  // row mapping: half-wave hw of workgroup w takes rows w*row0 + hw + step*i, i < max_rows
  int row0, step, max_rows;
  // prologue sources
  const float* x;          // PRO_QUANT / PRO_RMS input, PRO_MERGE single-split input
  const float* nw;         // norm weight
  float eps;
  const int8_t* xq;        // PRO_STAGE
  const uint16_t* xd;
  const uint8_t* emb;      // PRO_EMBED_RMS: Q8_0 token_embd [vocab][K/32]
  const int* tok;
  int vocab;
  float* x_out;            // PRO_EMBED_RMS: block 0 stores the embedding row here
  int* err;
  const float* wsm;        // PRO_MERGE split partials
  const float* wsz;
  const float* wso;
  int nh, hd, nsplit;
  int* len;                // PRO_MERGE: block 0 bumps *len (when < maxt)
  int maxt;
  // epilogue
  const float* resid;      // EPI_RESID
  float* y;
  int8_t* yq;              // EPI_SILU: the quantized SiLU(g)*u vector
  uint16_t* yd;
  float* pval;             // EPI_ARGMAX per-workgroup partials
  int* pidx;
  // EPI_ROPE_KV: RoPE of the q and k heads at position *lenr (freqs [hd/2]), the k and v rows
  // written into the caches at row *lenr (row stride nkv*hd; fp16 when kv_f16)
  const float* freqs;
  void* kc;
  void* vc;
  const int* lenr;
  int nkv, kv_f16;
  int planar;              // W is in the planar layout (lt_q8_to_planar)
  int* len_bump;           // any PRO but PRO_MERGE: block 0 bumps *len_bump (when < maxt) at its end
};

constexpr int kThreads = 256;
constexpr int kHalfWaves = kThreads / 32;
constexpr int kResidPre = 4;   // residuals prefetched per half-wave
constexpr int kSiluRows = 64;  // gate|up rows per workgroup: one 32-element quant block

__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// ---- prologues: the quantized activation, written as per-block records in LDS ---------
//
// Each prologue leaves, for every 32-element block b, the activation record rec[b] that
// fold_raw reads (both byte phases and the fp32 scale).  Its global inputs are loaded
// before the weight loads are issued (loads complete in issue order, so the prologue never
// waits behind the weights), and its arithmetic runs while the weights are in flight.

// Quantize one 32-element block held one element per lane of a half-wave (k_quant_q8's
// quantizer) and write it into the block's record: byte l+2 of phase E and byte 44+l of
// phase O hold q of element l; the other bytes of the two phases are zero; dwords 9 and 19
// hold the scale as fp32.
__device__ __forceinline__ void quant_to_rec(float v, int lane, uint32_t* recw) {
  const QScale sc = q8_scale(halfwave_max(fabsf(v)));
  const int8_t q = (int8_t)q8_quant(v, sc);
  uint8_t* rb = (uint8_t*)recw;
  rb[2 + lane] = (uint8_t)q;
  rb[44 + lane] = (uint8_t)q;
  if (lane == 0) {
    ((uint16_t*)rb)[0] = 0;          // E bytes 0, 1
    recw[kRecPhase] = 0u;            // O dword 0
    recw[9] = __builtin_bit_cast(uint32_t, sc.dq);
    recw[kRecPhase + 9] = __builtin_bit_cast(uint32_t, sc.dq);
  }
  if (lane == 31) ((uint16_t*)rb)[17] = 0;   // E bytes 34, 35
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// A buffer resource over n floats: loads past the end return zeros without touching
// memory, so the prologue loads are unconditional (no branches, exact load counters).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const float* p, int n) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, n * 4, 0x00020000);
}

// Two register layouts of the prologue's fp32 input:
//  - strided: slot s of thread t holds element s*256 + t (the rms_ss order's lanes);
//  - vector:  group v of thread t holds elements 4t + 1024v .. +3, so a 32-element block
//    lives on 8 consecutive lanes (quant4 / q4_to_rec).
// KS = ceil(K/256) strided slots (held by the first 256 threads); a workgroup of NT
// threads covers 4*NT elements per vector group; KV groups are held at once (all of them
// up to 4), the rest are processed KV at a time.
template <int KS, int NT = kThreads>
struct Slots {
  static constexpr int NV = (KS * 256 + 4 * NT - 1) / (4 * NT);   // vector groups in all
  static constexpr int KV = NV < 4 ? NV : 4;
  float s[KS];       // strided x (sum of squares only)
  f32x4 x[KV];       // vector x
  f32x4 w[KV];       // vector norm weight
};

template <int KS, int NT>
__device__ __forceinline__ void load_vgroups(const float* __restrict__ x, const float* __restrict__ w, int K,
                                             int v0, Slots<KS, NT>& S) {
  const __amdgpu_buffer_rsrc_t rx = f32_rsrc(x, K);
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < Slots<KS, NT>::KV; v++)
    S.x[v] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (t + NT * (v0 + v)) * 16, 0, 0));
  if (w) {
    const __amdgpu_buffer_rsrc_t rw = f32_rsrc(w, K);
#pragma unroll
    for (int v = 0; v < Slots<KS, NT>::KV; v++)
      S.w[v] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (t + NT * (v0 + v)) * 16, 0, 0));
  }
}

// kStrided: also load the strided copy of x for the sum of squares (threads < 256).
template <int KS, bool kStrided, int NT = kThreads>
__device__ __forceinline__ void load_slots(const float* __restrict__ x, const float* __restrict__ w, int K,
                                           Slots<KS, NT>& S) {
  if (kStrided) {
    const __amdgpu_buffer_rsrc_t rx = f32_rsrc(x, K);
    const int t = threadIdx.x;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const int off = (NT == 256 || t < 256) ? (s * 256 + t) * 4 : (int)0x80000000;
      S.s[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
    }
  }
  load_vgroups<KS, NT>(x, w, K, 0, S);
}

// Quantize the vector groups into records (optionally normalized: y = (x*inv)*w).  The
// groups past the first KV are loaded here (K > 16*NT).
template <int KS, bool kNorm, int NT = kThreads, bool kPL = false>
__device__ __forceinline__ void slots_to_rec(Slots<KS, NT>& S, const float* __restrict__ x,
                                             const float* __restrict__ w, float inv, int K, uint32_t* rec) {
  const int t = threadIdx.x;
  const int j = t & 7;
  const int nb = K >> 5;
  constexpr int KV = Slots<KS, NT>::KV;
#pragma unroll
  for (int v0 = 0; v0 < Slots<KS, NT>::NV; v0 += KV) {
    if (v0 > 0) load_vgroups<KS, NT>(x, kNorm ? w : nullptr, K, v0, S);
    uint32_t p[KV];
    QScale sc[KV];
#pragma unroll
    for (int v = 0; v < KV; v++) {
      f32x4 y = S.x[v];
      if (kNorm) {
        y.x = (y.x * inv) * S.w[v].x;
        y.y = (y.y * inv) * S.w[v].y;
        y.z = (y.z * inv) * S.w[v].z;
        y.w = (y.w * inv) * S.w[v].w;
      }
      p[v] = quant4(y.x, y.y, y.z, y.w, sc[v]);
    }
#pragma unroll
    for (int v = 0; v < KV; v++) {
      const int b = (t >> 3) + (NT / 8) * (v0 + v);
      if constexpr (kPL) {   // planar folds read phase O and the scale only
        if (b < nb) {
          rec[b * kRecDwords + kRecPhase + 1 + j] = p[v];
          if (j == 0) rec[b * kRecDwords + kRecPhase + 9] = __builtin_bit_cast(uint32_t, sc[v].dq);
        }
      } else {
        q4_to_rec(p[v], sc[v].dq, j, b < nb, rec + b * kRecDwords);
      }
    }
  }
}

// The slots of an fp32 row already in LDS (the embedding prologue), norm weight from
// global memory.
template <int KS>
__device__ __forceinline__ void lds_slots(const float* xrow, const float* __restrict__ w, int K, Slots<KS>& S) {
  const int t = threadIdx.x;
#pragma unroll
  for (int s = 0; s < KS; s++) S.s[s] = s * kThreads + t < K ? xrow[s * kThreads + t] : 0.0f;
#pragma unroll
  for (int v = 0; v < Slots<KS>::KV; v++) {
    const int e = 4 * (t + kThreads * v);
    S.x[v] = e < K ? *(const f32x4*)(xrow + e) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const __amdgpu_buffer_rsrc_t rw = f32_rsrc(w, K);
#pragma unroll
  for (int v = 0; v < Slots<KS>::KV; v++)
    S.w[v] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (t + kThreads * v) * 16, 0, 0));
}

// rms_ss order (norm_softmax_from_facts.pl:49, 83-108): thread t folds x[t], x[t+256], ...
// by fma, then the pairwise tree 128..1; inv = rsqrt(ss/N + eps).  Slots past K hold
// zeros, which leave the fold unchanged (p + 0*0 == p for p >= 0).
template <int KS, int NT>
__device__ __forceinline__ float rms_inv(const Slots<KS, NT>& S, int K, float eps, float* red, float* sinv) {
  const int t = threadIdx.x;
  float p = 0.0f;
#pragma unroll
  for (int s = 0; s < KS; s++) p = fmaf(S.s[s], S.s[s], p);
  if (NT == 256 || t < 256) red[t] = p;
  __syncthreads();
  if (t < 64) {
    float a = red[t] + red[t + 128];
    float b = red[t + 64] + red[t + 192];
    const float c = wave_tree_dpp(a + b);
    if (t == 0) *sinv = lt_rsqrtf(c / (float)K + eps);
  }
  __syncthreads();
  return *sinv;
}

// rms_inv over a single (vector) load of x: the vector groups go to LDS (xs, KS*256 floats)
// and each thread reads its strided slots back, so x is read from L2 once per workgroup; the
// fold and the tree are rms_inv's.  All vector groups are held (KS*256 <= 4*4*NT).
template <int KS>
__device__ __forceinline__ float rms_inv_lds(Slots<KS>& S, int K, float eps, float* red, float* sinv, float* xs) {
  static_assert(Slots<KS>::NV == Slots<KS>::KV, "every vector group in registers");
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < Slots<KS>::KV; v++) *(f32x4*)(xs + 4 * (t + kThreads * v)) = S.x[v];
  __syncthreads();
#pragma unroll
  for (int s = 0; s < KS; s++) S.s[s] = xs[s * kThreads + t];
  return rms_inv<KS, kThreads>(S, K, eps, red, sinv);
}

// Split-K merge of the attention partials (the declared combine, ascending split order,
// bpd/kernelgen/experimental/attn_decode_split.cu:37-91: M = max m_s, w_s = exp(m_s - M),
// Z = sum fma(w_s, Z_s), O = sum fma(w_s, O_s), out = O/Z), then the quant.
__device__ __forceinline__ void pro_merge_quant(const GemvParams& P, uint32_t* rec) {
  const int lane = threadIdx.x & 31;
  const int S = P.nsplit;
  for (int b = threadIdx.x >> 5; b < P.K / 32; b += kHalfWaves) {
    const int j = b * 32 + lane;
    const int h = j / P.hd;
    const int d = j - h * P.hd;
    const float* m = P.wsm + (size_t)h * S;
    const float* z = P.wsz + (size_t)h * S;
    float M = -1e30f;
    for (int s = 0; s < S; s++) M = fmaxf(M, m[s]);
    float Z = 0.0f, acc = 0.0f;
    for (int s = 0; s < S; s++) {
      const float w = lt_expf_sel(m[s] - M);
      Z = fmaf(w, z[s], Z);
      acc = fmaf(w, P.wso[((size_t)h * S + s) * P.hd + d], acc);
    }
    quant_to_rec(acc / Z, lane, rec + b * kRecDwords);
  }
}

// Staged int8 quants + fp16 scales: copied through LDS, then laid out as records.
constexpr int kStageChunks = 4;   // 16-byte chunks of xq per thread of a 256-thread workgroup (K <= 16384)

template <int NT = kThreads>
struct StageRegs {
  static constexpr int C = kStageChunks * 256 / NT;   // chunks per thread
  static constexpr int DS = 2 * 256 / NT > 0 ? 2 * 256 / NT : 1;   // scales per thread
  u32x4 c[C];
  uint16_t d[DS];
};

template <int NT = kThreads>
__device__ __forceinline__ void load_stage(const int8_t* __restrict__ xq, const uint16_t* __restrict__ xd,
                                           int K, StageRegs<NT>& R) {
  // buffer loads: chunks past K and scales past K/32 read zeros, with no branches
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)xq, 0, K, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)xd, 0, (K / 32) * 2, 0x00020000);
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::C; k++)
    R.c[k] = __builtin_amdgcn_raw_buffer_load_b128(rq, (threadIdx.x + NT * k) * 16, 0, 0);
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::DS; k++)
    R.d[k] = __builtin_amdgcn_raw_buffer_load_b16(rd, (threadIdx.x + NT * k) * 2, 0, 0);
}

template <int NT = kThreads>
__device__ __forceinline__ void stage_to_rec(const StageRegs<NT>& R, int K, uint8_t* sxq, uint32_t* rec) {
  u32x4* dst = (u32x4*)sxq;
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::C; k++) {
    const int i = threadIdx.x + NT * k;
    if (i < K / 16) dst[i] = R.c[k];
  }
  __syncthreads();
  const uint32_t* X = (const uint32_t*)sxq;   // 8 dwords per block
  const int nb = K >> 5;
  for (int i = threadIdx.x; i < nb * 9; i += NT) {
    const int b = i / 9;
    const int j = i - b * 9;
    uint32_t* r = rec + b * kRecDwords;
    const uint32_t lo = j > 0 ? X[b * 8 + j - 1] : 0u;
    const uint32_t hi = j < 8 ? X[b * 8 + j] : 0u;
    r[j] = __builtin_amdgcn_perm(hi, lo, 0x05040302u);
    r[kRecPhase + j] = lo;
  }
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::DS; k++) {
    const int b = threadIdx.x + NT * k;
    if (b < nb) {
      const uint32_t xdf = __builtin_bit_cast(uint32_t, lt_h2f(R.d[k]));
      rec[b * kRecDwords + 9] = xdf;
      rec[b * kRecDwords + kRecPhase + 9] = xdf;
    }
  }
}

// The planar folds' records straight from the staged registers: 16-byte chunk i is half
// (i & 1) of block i / 2, i.e. dwords kRecPhase+1+4(i&1) .. +3 of its record (phase O), and
// the scale goes to dword kRecPhase+9; no LDS copy of xq, no extra barrier.
template <int NT = kThreads>
__device__ __forceinline__ void stage_to_rec_pl(const StageRegs<NT>& R, int K, uint32_t* rec) {
  const int nb = K >> 5;
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::C; k++) {
    const int i = threadIdx.x + NT * k;
    if (i < K / 16) {
      uint32_t* r = rec + (i >> 1) * kRecDwords + kRecPhase + 1 + 4 * (i & 1);
      r[0] = R.c[k].x; r[1] = R.c[k].y; r[2] = R.c[k].z; r[3] = R.c[k].w;
    }
  }
#pragma unroll
  for (int k = 0; k < StageRegs<NT>::DS; k++) {
    const int b = threadIdx.x + NT * k;
    if (b < nb) rec[b * kRecDwords + kRecPhase + 9] = __builtin_bit_cast(uint32_t, lt_h2f(R.d[k]));
  }
}

// ---- the fused GEMV ----------------------------------------------------------------
//
// Half-wave hw (0..7) of workgroup w takes rows w*row0 + hw + step*i (i < max_rows): one
// group of 8 rows per workgroup, or (large N) a contiguous block of row0 rows per
// workgroup, walked 8 rows at a time.  Each
// row is the canonical Q8_0 dot: lane L folds blocks L, L+32, ... by fma, then the 5-level
// shfl_down tree (q8_0_from_facts.pl:466-516).
//
// A half-wave walks the flattened sequence of items (row i, block slot k), k < nk =
// ceil(nb/32), lane L's block of item (i, k) being L + 32k.  It keeps D items in flight: a
// ring of D block registers, each refilled with item m + D right after item m is folded,
// so every lane streams D blocks ahead across row boundaries.  The weights are read with
// buffer loads: items past the half-wave's last one get an out-of-range offset and read
// zeros without touching memory, so the loop issues every load unconditionally (the
// compiler's load counters stay exact and the loads pipeline).
constexpr uint32_t kNoBlock = 0x80000000u;
// Staged streaming (kStg): a workgroup whose 64 rows are contiguous and one 32-block item
// each (K <= 1024) reads its whole region -- at most 64 x 32 blocks -- as coalesced
// non-temporal 16-byte loads (kStgLoads per thread, issued before the prologue), parks it
// in LDS, and every half-wave then folds its rows' blocks from there: the same raw dwords
// and arithmetic as the per-lane block loads, with whole cache lines per load instruction.
// It is used when the whole grid is resident at once (the 0.5B gate|up GEMV: every load
// of the launch is in flight from its start); a grid of several rounds (the vocab GEMV)
// streams better through the per-lane ring, which overlaps loads and folds.
constexpr int kStgRows = 64;
constexpr int kStgLoads = (kStgRows * 32 * (int)kBlockBytes + 4095) / 4096;   // 17
constexpr uint32_t kStgBytes = (uint32_t)kStgLoads * 4096u + 16u;   // + the last block's 9th dword
// Planar weights (kPL, lt_q8_to_planar): the same ring and item order, each
// item read as two coalesced non-temporal 16-byte loads per lane plus its scale (lt_q8_device.h,
// fold_planar); every other stage is unchanged.

template <int KS, Pro PRO, Epi EPI, int D, bool kStg = false, bool kPL = false>
__global__ __launch_bounds__(kThreads) void k_gemv_fused(GemvParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int K = P.K;
  const int nb = K >> 5;
  float* red = (float*)smem;                                  // [256] + sinv + pad
  float* sinv = red + kThreads;
  uint32_t* rec = (uint32_t*)(red + kThreads + 4);            // [nb][kRecDwords]
  uint8_t* sxq = (uint8_t*)(rec + ((nb * kRecDwords + 3) & ~3));   // [K]: PRO_STAGE staging (16-aligned)
  float* xrow = (float*)(sxq + ((K + 15) & ~15));             // [K]: PRO_EMBED_RMS row
  __shared__ float s_rows[kSiluRows];

  const int hw = threadIdx.x >> 5;
  const int lane = threadIdx.x & 31;
  // @phase gemv 0

  // (1) the prologue's global inputs
  Slots<KS> S;
  StageRegs<> SR;
  int tok = 0;
  // planar RMS prologues with every vector group held read x once (rms_inv_lds)
  constexpr bool kXLds = kPL && PRO == PRO_RMS && KS <= 16;
  if constexpr (PRO == PRO_RMS) load_slots<KS, !kXLds>(P.x, P.nw, K, S);
  else if constexpr (PRO == PRO_QUANT) load_slots<KS, false>(P.x, nullptr, K, S);
  else if constexpr (PRO == PRO_STAGE) load_stage(P.xq, P.xd, K, SR);
  else if constexpr (PRO == PRO_MERGE) { if (P.nsplit == 1) load_stage(P.xq, P.xd, K, SR); }
  else if constexpr (PRO == PRO_EMBED_RMS) tok = *P.tok;

  // (2) the weights
  // EPI_ROPE_KV: workgroup w holds 4 rotation pairs of one head (head w / (hd/8), pairs
  // 4c .. 4c+3 with c = w % (hd/8)): half-waves 0-3 take rows j, half-waves 4-7 rows j + hd/2
  auto row_of = [&](int h) {
    if constexpr (EPI == EPI_ROPE_KV) {
      const int hq = P.hd >> 3;
      const int head = blockIdx.x / hq;
      return head * P.hd + ((h & 4) ? (P.hd >> 1) : 0) + (blockIdx.x - head * hq) * 4 + (h & 3);
    } else {
      return blockIdx.x * P.row0 + h;
    }
  };
  const int rbase = row_of(hw);
  const int step = P.step;
  const int nk = (nb + 31) >> 5;
  auto rows_from = [&](int r0) {
    int n = P.N > r0 ? (P.N - r0 + step - 1) / step : 0;
    return n < P.max_rows ? n : P.max_rows;
  };
  const int nrows = rows_from(rbase);
  const int total = nrows * nk;
  // the even half-wave of a wave has the most rows: its count makes the loop wave-uniform
  const int trips = (rows_from(row_of(hw & ~1)) * nk + D - 1) / D;
  const uint32_t row_step_bytes = (uint32_t)step * (uint32_t)nb * (uint32_t)kBlockBytes;
  constexpr uint32_t kSlotBytes = 32u * kBlockBytes;
  const uint32_t lane_bytes = (uint32_t)lane * (uint32_t)kBlockBytes;
  const uint32_t mat_bytes = (uint32_t)P.N * (uint32_t)nb * (uint32_t)kBlockBytes;
  // the final even block's 9th dword reaches 2 bytes past the matrix: that dword starts
  // inside it, so it lies in the same mapped page; its 2 extra bytes meet zero activations
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)P.W, 0, (int)((mat_bytes + 3u) & ~3u), 0x00020000);

  // staged: the workgroup's region (rows past N read zeros)
  u32x4 stg[kStg ? kStgLoads : 1];
  if constexpr (kStg) {
    const int r0 = blockIdx.x * kStgRows;
    const int nr = P.N - r0 < kStgRows ? P.N - r0 : kStgRows;
    const uint32_t region = (uint32_t)nr * (uint32_t)nb * (uint32_t)kBlockBytes;
    const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.W + (size_t)r0 * (size_t)nb * kBlockBytes), 0, (int)((region + 3u) & ~3u), 0x00020000);
#pragma unroll
    for (int i = 0; i < kStgLoads; i++)
      stg[i] = __builtin_amdgcn_raw_buffer_load_b128(srsrc, (int)(threadIdx.x * 16u + (uint32_t)i * 4096u), 0, 2);
  }
  RawBlock ring[D];
  int is = 0, ik = 0;                                                   // next item to issue
  uint32_t issue_row = (uint32_t)rbase * (uint32_t)nb * (uint32_t)kBlockBytes;
  // planar: the row's first block index row*nb (an item starts at (row*nb + 32k)*32 bytes, its
  // second halves 16m bytes on, m its blocks), and the scale plane after the N*nb*32 quant bytes
  uint32_t issue_blk = (uint32_t)rbase * (uint32_t)nb;
  const uint32_t scale_base = (uint32_t)P.N * (uint32_t)nb * 32u;
  auto issue = [&](RawBlock& r) {
    const bool real = is < total && lane + 32 * ik < nb;
    if constexpr (kPL) {
      const uint32_t k0 = 32u * (uint32_t)ik;
      const uint32_t m = (uint32_t)nb - k0 < 32u ? (uint32_t)nb - k0 : 32u;
      const uint32_t qo = real ? (issue_blk + k0) * 32u + (uint32_t)lane * 16u : kNoBlock;
      const uint32_t so = real ? scale_base + (issue_blk + k0 + (uint32_t)lane) * 2u : kNoBlock;
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)qo, 0, 2);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)(qo + m * 16u), 0, 2);
      r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
      r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
      r.w[8] = __builtin_amdgcn_raw_buffer_load_b16(wrsrc, (int)so, 0, 2);
    } else {
      const uint32_t off = real ? issue_row + lane_bytes + (uint32_t)ik * kSlotBytes : kNoBlock;
      const uint32_t o4 = off & ~3u;
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)o4, 0, 0);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)(o4 + 16u), 0, 0);
      r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
      r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
      r.w[8] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(o4 + 32u), 0, 0);
    }
    is++;
    if (++ik == nk) { ik = 0; issue_row += row_step_bytes; issue_blk += (uint32_t)step * (uint32_t)nb; }
  };
  if constexpr (!kStg) {
#pragma unroll
    for (int d = 0; d < D; d++) issue(ring[d]);
  }
  // the epilogue's residuals (or biases), fetched with the weights
  float rpre[kResidPre];
  if constexpr (EPI == EPI_RESID || EPI == EPI_ROPE_KV) {
    const __amdgpu_buffer_rsrc_t rres = f32_rsrc(P.resid, P.resid ? P.N : 0);
#pragma unroll
    for (int i = 0; i < kResidPre; i++) {   // buffer loads: no branches, exact load counters
      const int off = (lane == 0 && i < nrows) ? (rbase + step * i) * 4 : (int)kNoBlock;
      rpre[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rres, off, 0, 0));
    }
  }
  // EPI_ROPE_KV: the rotation of this workgroup's 4 pairs at position *lenr (k_rope's
  // arithmetic), evaluated under the weight loads
  __shared__ float s_rot[8];
  __shared__ int s_pos;
  if constexpr (EPI == EPI_ROPE_KV) {
    if (threadIdx.x < 4) {
      const int pos = *P.lenr;
      const int j = (blockIdx.x - (blockIdx.x / (P.hd >> 3)) * (P.hd >> 3)) * 4 + threadIdx.x;
      float sn, cs;
      lt_sincosf((float)pos * P.freqs[j], &sn, &cs);
      s_rot[threadIdx.x] = sn;
      s_rot[4 + threadIdx.x] = cs;
      if (threadIdx.x == 0) s_pos = pos;
    }
  }
  // @phase gemv 1

  // (3) the prologue's arithmetic, under the weight loads
  if constexpr (PRO == PRO_RMS) {
    float inv;
    if constexpr (kXLds) inv = rms_inv_lds<KS>(S, K, P.eps, red, sinv, (float*)sxq);
    else inv = rms_inv<KS>(S, K, P.eps, red, sinv);
    // @phase gemv 5
    slots_to_rec<KS, true, kThreads, kPL>(S, P.x, P.nw, inv, K, rec);
  } else if constexpr (PRO == PRO_QUANT) {
    slots_to_rec<KS, false, kThreads, kPL>(S, P.x, nullptr, 0.0f, K, rec);
  } else if constexpr (PRO == PRO_STAGE) {
    if constexpr (kPL) stage_to_rec_pl(SR, K, rec);
    else stage_to_rec(SR, K, sxq, rec);
  } else if constexpr (PRO == PRO_MERGE) {
    if (P.nsplit > 1) pro_merge_quant(P, rec);
    else if constexpr (kPL) stage_to_rec_pl(SR, K, rec);
    else stage_to_rec(SR, K, sxq, rec);
    if (P.len && blockIdx.x == 0 && threadIdx.x == 0) {
      const int L = *P.len;
      if (L >= 0 && L < P.maxt) *P.len = L + 1;
    }
  } else if constexpr (PRO == PRO_EMBED_RMS) {
    // embedding row of the device token (x = q*d, exact); workgroup 0 keeps it as the
    // layer's residual
    const bool bad = tok < 0 || tok >= P.vocab;
    for (int j = threadIdx.x; j < K; j += kThreads) {
      float v = 0.0f;
      if (!bad) {
        const uint8_t* blk = P.emb + ((size_t)tok * (K / 32) + (j >> 5)) * kBlockBytes;
        const uint16_t dd = (uint16_t)(blk[0] | (blk[1] << 8));
        v = (float)(int8_t)blk[2 + (j & 31)] * lt_h2f(dd);
      }
      xrow[j] = v;
      if (blockIdx.x == 0) P.x_out[j] = v;
    }
    if (bad && blockIdx.x == 0 && threadIdx.x == 0 && P.err) *P.err = 1;
    __syncthreads();
    static_assert(KS <= 16, "the embedding prologue holds every vector group (K <= 4096)");
    lds_slots<KS>(xrow, P.nw, K, S);
    const float inv = rms_inv<KS>(S, K, P.eps, red, sinv);
    slots_to_rec<KS, true, kThreads, kPL>(S, nullptr, P.nw, inv, K, rec);
  }
  // staged: the region into LDS, after the prologue's buffers (the host sizes the launch's
  // LDS the same way)
  const uint32_t stage_off = (uint32_t)(kThreads + 4) * 4u + (uint32_t)((nb * kRecDwords + 3) & ~3) * 4u +
                             ((PRO == PRO_STAGE || PRO == PRO_MERGE) ? (uint32_t)((K + 15) & ~15) : 0u) +
                             (PRO == PRO_EMBED_RMS ? (uint32_t)((K + 15) & ~15) + (uint32_t)K * 4u : 0u);
  const uint32_t* stage = (const uint32_t*)(smem + stage_off);
  if constexpr (kStg) {
#pragma unroll
    for (int i = 0; i < kStgLoads; i++) *(u32x4*)(smem + stage_off + threadIdx.x * 16u + (uint32_t)i * 4096u) = stg[i];
  }
  __syncthreads();
  // @phase gemv 2

  // (4) stream the rows
  float bv = -__builtin_inff();
  int bi = 0x7FFFFFFF;
  float acc = 0.0f;
  int fm = 0, fi = 0, fk = 0;         // item being folded: index, row, slot
  uint32_t fold_row = (uint32_t)rbase * (uint32_t)nb * (uint32_t)kBlockBytes;
  // a finished row: the tree (the row value lands on lane 0 of the half-wave), then the
  // epilogue for row rbase + step * fi
  auto finish_row = [&](float a, int ri) {
    const float v = halfwave_tree_dpp(a);
    const int row = rbase + step * ri;
    if constexpr (EPI == EPI_ROPE_KV) {   // one row per half-wave: the biased value to LDS
      if (lane == 0 && ri < nrows) s_rows[hw] = P.resid ? v + rpre[0] : v;
      return;
    }
    if constexpr (EPI == EPI_SWIGLU) {
      // rows 2j (gate j) and 2j + 1 (up j) sit on the two half-waves of one wave, which
      // finish them together: lane 0 takes the up value from lane 32
      const float u = __shfl_xor(v, 32, 64);
      if ((threadIdx.x & 63) == 0 && ri < nrows) P.y[row >> 1] = lt_silu_mul(v, u);
      return;
    }
    if (lane == 0 && ri < nrows) {
      if constexpr (EPI == EPI_SILU) {
        s_rows[row - blockIdx.x * kSiluRows] = v;
      } else {
        float o = v;
        if constexpr (EPI == EPI_RESID) {
          float rv = 0.0f;
          if (ri < kResidPre) {
#pragma unroll
            for (int i = 0; i < kResidPre; i++)   // static indices keep rpre in registers
              if (ri == i) rv = rpre[i];
          } else {
            rv = P.resid[row];
          }
          o = v + rv;
        }
        P.y[row] = o;
        if (EPI == EPI_ARGMAX && am_better(o, row, bv, bi)) { bv = o; bi = row; }
      }
    }
  };
  if constexpr (kStg) {
    // row hw + 8i of the region: lane L folds block L from LDS (lanes past nb fold lane 0's
    // block and discard it)
    const int lb = lane < nb ? lane : 0;
#pragma unroll
    for (int i = 0; i < kStgRows / 8; i++) {
      const uint32_t off = (uint32_t)(hw + 8 * i) * (uint32_t)nb * (uint32_t)kBlockBytes + (uint32_t)lb * kBlockBytes;
      RawBlock r;
#pragma unroll
      for (int k = 0; k < 9; k++) r.w[k] = stage[(off >> 2) + k];
      const float folded = fold_raw(r, (off & 2u) != 0, rec + lb * kRecDwords, 0.0f);
      finish_row(lane < nb ? folded : 0.0f, i);
    }
  } else {
    // all trips but the last refill the ring; the last one only drains it
    auto fold_item = [&](RawBlock& r, bool refill) {
      const int b = lane + 32 * fk;
      float folded;
      if constexpr (kPL) {
        folded = fold_planar(r, rec + (b < nb ? b : 0) * kRecDwords, acc);
      } else {
        const bool odd = ((fold_row + lane_bytes + (uint32_t)fk * kSlotBytes) & 2u) != 0;
        folded = fold_raw(r, odd, rec + (b < nb ? b : 0) * kRecDwords, acc);
      }
      acc = (fm < total && b < nb) ? folded : acc;
      if (refill) issue(r);
      fm++;
      if (++fk == nk) {                   // row end: the same item for both half-waves
        finish_row(acc, fi);
        acc = 0.0f;
        fk = 0;
        fi++;
        fold_row += row_step_bytes;
      }
    };
    for (int t = 0; t + 1 < trips; t++) {
#pragma unroll
      for (int d = 0; d < D; d++) fold_item(ring[d], true);
    }
    if (trips > 0) {
#pragma unroll
      for (int d = 0; d < D; d++) fold_item(ring[d], false);
    }
  }

  // @phase gemv 3
  if constexpr (EPI == EPI_ROPE_KV) {
    // x1 = row j, x2 = row j + hd/2: q and k heads rotate (fma(x1, c, -(x2*s)),
    // fma(x1, s, x2*c)), v heads pass; all rows go to y; k and v rows also to the caches at
    // row *lenr (a full cache is left unchanged)
    __syncthreads();
    if (threadIdx.x < 4) {
      const int i = threadIdx.x;
      const int hq = P.hd >> 3;
      const int head = blockIdx.x / hq;
      const int half = P.hd >> 1;
      const int j = (blockIdx.x - head * hq) * 4 + i;
      const int r1 = head * P.hd + j;
      float x1 = s_rows[i], x2 = s_rows[i + 4];
      if (head < P.nh + P.nkv) {
        const float sn = s_rot[i], cs = s_rot[4 + i];
        const float y1 = fmaf(x1, cs, -(x2 * sn));
        const float y2 = fmaf(x1, sn, x2 * cs);
        x1 = y1;
        x2 = y2;
      }
      P.y[r1] = x1;
      P.y[r1 + half] = x2;
      const int L = s_pos;
      if (head >= P.nh && L >= 0 && L < P.maxt) {
        const bool isv = head >= P.nh + P.nkv;
        const size_t off = (size_t)L * P.nkv * P.hd + (size_t)(head - P.nh - (isv ? P.nkv : 0)) * P.hd + j;
        if (P.kv_f16) {
          uint16_t* c = (uint16_t*)(isv ? P.vc : P.kc);
          c[off] = lt_f2h(x1);
          c[off + half] = lt_f2h(x2);
        } else {
          float* c = (float*)(isv ? P.vc : P.kc);
          c[off] = x1;
          c[off + half] = x2;
        }
      }
    }
  }
  if constexpr (PRO != PRO_MERGE) {
    if (P.len_bump && blockIdx.x == 0 && threadIdx.x == 0) {
      const int L = *P.len_bump;
      if (L >= 0 && L < P.maxt) *P.len_bump = L + 1;
    }
  }
  if constexpr (EPI == EPI_SILU) {
    // the workgroup's 64 rows are the gate/up pairs of one 32-element block: SiLU(g)*u
    // one pair per lane of half-wave 0, then k_silu_mul_quant's quantizer
    __syncthreads();
    if (hw == 0) {
      const float v = lt_silu_mul(s_rows[2 * lane], s_rows[2 * lane + 1]);
      quant_block_hw(v, lane, P.yq + blockIdx.x * 32, P.yd + blockIdx.x);
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    __shared__ float sv[kHalfWaves];
    __shared__ int si[kHalfWaves];
    if (lane == 0) { sv[hw] = bv; si[hw] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = sv[0];
      int ix = si[0];
      for (int k = 1; k < kHalfWaves; k++)
        if (am_better(sv[k], si[k], v, ix)) { v = sv[k]; ix = si[k]; }
      P.pval[blockIdx.x] = v;
      P.pidx[blockIdx.x] = ix;
    }
  }
  // @phase gemv 4
}

// ---- attention recomputed in the O projection's prologue ----------------------------
//
// k_attn_o: one launch for k_attn_decode_masked (nsplit 1) -> quant -> O GEMV + residual
// (bpd/lib/dev_residency.py:1420-1440), for at most AoLayout::kRows / nkv attended rows, where the
// attention is a few microseconds of arithmetic: every workgroup computes the attention
// output of all heads itself (q and the cache rows are small and come from L2), quantizes
// it into the GEMV's activation records, and folds its 32 rows of the O matrix.  The O
// weights, q, the length and the first kAoFirstL cache rows of K and V are all requested at
// kernel start, so the launch waits for memory once (twice past kAoFirstL rows).  Each
// value is the oracle's: scores are sequential fma chains over the head dims times scale;
// max and Z are the 64-lane strided folds plus trees; exps by lt_expf; out = (sequential
// fma chain over positions) / Z; then the engine quantizer and the canonical GEMV order.
struct AttnOParams {
  const float* qkv;      // roped q of the nh heads at [0, nh*hd)
  const void* kc;        // caches [maxt][nkv*hd] (fp16 or fp32); this token's row is at *len
  const void* vc;
  const int* len;        // rows before this token's (attention covers *len + 1 rows)
  int nh, nkv, maxt;
  int maxL;              // rows the launch can attend: AoLayout::kRows / nkv
  float scale;
  const uint8_t* W;      // O projection: N rows of K = nh*hd (K <= 1024: one 32-block item per row)
  const float* resid;
  float* y;
  int N;
};

constexpr int kAoThreads = 1024;
constexpr int kAoRows = kAoThreads / 32;   // one O row per half-wave
constexpr int kAoWaves = kAoThreads / 64;
constexpr int kAoHd = 64;                  // head size: a wave's lanes are one head's dims
constexpr int kAoFirstL = 128;             // rows requested before the length is known
constexpr int kAoMaxHpw = 4;               // heads per thread (scores) and per wave (O chains)

template <bool kF16>
struct AoLayout {
  static constexpr int kEsz = kF16 ? 2 : 4;
  static constexpr int kRows = kF16 ? 512 : 256;    // staged (position, KV group) rows
  static constexpr int kRowB = kAoHd * kEsz;        // one cache row of one KV group, bytes
  static constexpr int kKRowB = kRowB + 16;         // staged K row: a 16-byte pad keeps a wave's rows on distinct banks
  static constexpr size_t kKBytes = (size_t)kRows * kKRowB;   // K, group-major
  // V position-major, [maxL][nkv][hd]: a wave's 64 lanes read one row's 64 dims at once
  static __host__ __device__ size_t vbytes(int nkv, int maxL) { return (size_t)nkv * maxL * kRowB; }
};
constexpr size_t kAoLdsMax = (size_t)160 * 1024;   // LDS of one gfx950 workgroup

template <bool kF16>
size_t attn_o_lds_bytes(int nh, int nkv, int maxL) {
  const int K = nh * kAoHd, nb = K / 32;
  return (size_t)K * 4 + AoLayout<kF16>::kKBytes + AoLayout<kF16>::vbytes(nkv, maxL) + (size_t)nh * maxL * 4 + 64 +
         (size_t)((nb * kRecDwords + 3) & ~3) * 4;
}

template <bool kF16>
__device__ __forceinline__ float kv_elem(const uint8_t* p) {
  if constexpr (kF16) return lt_h2f(*(const uint16_t*)p);
  else return *(const float*)p;
}

// The cache rows [r0, r1) of K (group-major, padded rows) and V (position-major) into LDS:
// 16-byte pieces, loaded first and stored after, so every load of the round is in flight.
// A call stages at most kRows (position, group) rows.
template <bool kF16>
__device__ __forceinline__ void ao_stage(const AttnOParams& P, int r0, int r1, uint8_t* sK, uint8_t* sV) {
  using Lo = AoLayout<kF16>;
  constexpr int PPR = Lo::kRowB / 16;               // pieces per (position, group) row
  constexpr int kMaxPer = (Lo::kRows * PPR + kAoThreads - 1) / kAoThreads;   // per thread, per tensor
  const int nkv = P.nkv;
  const int npieces = (r1 - r0) * nkv * PPR;
  const uint8_t* kc = (const uint8_t*)P.kc + (size_t)r0 * nkv * Lo::kRowB;
  const uint8_t* vc = (const uint8_t*)P.vc + (size_t)r0 * nkv * Lo::kRowB;
  u32x4 kb[kMaxPer], vb[kMaxPer];
#pragma unroll
  for (int k = 0; k < kMaxPer; k++) {
    const int i = threadIdx.x + k * kAoThreads;
    if (i < npieces) {
      kb[k] = *(const u32x4*)(kc + (size_t)i * 16);
      vb[k] = *(const u32x4*)(vc + (size_t)i * 16);
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxPer; k++) {
    const int i = threadIdx.x + k * kAoThreads;
    if (i < npieces) {
      const int rr = i / PPR, pc = i - rr * PPR;      // rr = (t - r0) * nkv + g
      const int t = r0 + rr / nkv, g = rr - (rr / nkv) * nkv;
      *(u32x4*)(sK + ((size_t)g * P.maxL + t) * Lo::kKRowB + pc * 16) = kb[k];
      *(u32x4*)(sV + ((size_t)t * nkv + g) * Lo::kRowB + pc * 16) = vb[k];
    }
  }
}

template <bool kF16>
__global__ __launch_bounds__(kAoThreads) void k_attn_o(AttnOParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  using Lo = AoLayout<kF16>;
  constexpr int HD = kAoHd;
  const int nh = P.nh, nkv = P.nkv, rep = nh / nkv, K = nh * HD, nb = K >> 5, maxt = P.maxt;
  float* sq = (float*)smem;                                    // [K] roped q
  const int maxL = P.maxL;
  uint8_t* sK = (uint8_t*)(sq + K);                            // [nkv][maxL] padded K rows
  uint8_t* sV = sK + Lo::kKBytes;                              // [maxL][nkv] V rows
  float* sS = (float*)(sV + Lo::vbytes(nkv, maxL));            // [nh][maxL] scores, then exps
  float* sZ = sS + (size_t)nh * maxL;                          // [16]
  uint32_t* rec = (uint32_t*)(sZ + 16);                        // [nb][kRecDwords]
  __shared__ int s_len;
  const int tid = threadIdx.x, lane = tid & 31, hw = tid >> 5, wl = tid & 63, wv = tid >> 6;

  // (1) every request that does not depend on the length: this half-wave's O row, its
  // residual, q, the length, and the first kAoFirstL rows of K and V
  const int row = blockIdx.x * kAoRows + hw;
  const uint32_t mat_bytes = (uint32_t)P.N * (uint32_t)nb * (uint32_t)kBlockBytes;
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)P.W, 0, (int)((mat_bytes + 3u) & ~3u), 0x00020000);
  const uint32_t off = (row < P.N && lane < nb) ? (uint32_t)row * (uint32_t)nb * kBlockBytes + (uint32_t)lane * kBlockBytes
                                                : kNoBlock;
  RawBlock rw;
  {
    const uint32_t o4 = off & ~3u;
    const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)o4, 0, 0);
    const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)(o4 + 16u), 0, 0);
    rw.w[0] = v0.x; rw.w[1] = v0.y; rw.w[2] = v0.z; rw.w[3] = v0.w;
    rw.w[4] = v1.x; rw.w[5] = v1.y; rw.w[6] = v1.z; rw.w[7] = v1.w;
    rw.w[8] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(o4 + 32u), 0, 0);
  }
  const bool odd = (off & 2u) != 0;
  const __amdgpu_buffer_rsrc_t rres = f32_rsrc(P.resid, P.resid ? P.N : 0);
  const float rv = __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(rres, (lane == 0 && row < P.N) ? row * 4 : (int)kNoBlock, 0, 0));
  if (tid == 0) s_len = *P.len;
  for (int i = tid; i < K; i += kAoThreads) sq[i] = P.qkv[i];
  int first = maxt < kAoFirstL ? maxt : kAoFirstL;
  if (first > maxL) first = maxL;
  ao_stage<kF16>(P, 0, first, sK, sV);
  __syncthreads();
  const int len0 = s_len;
  const int L = len0 < 0 ? 0 : (len0 < maxt ? len0 + 1 : maxt);
  if (L > maxL) {   // outside the launch's contract (the host checks): poison the rows
    if (lane == 0 && row < P.N) P.y[row] = __builtin_nanf("");
    return;
  }
  if (L > first) {
    ao_stage<kF16>(P, first, L, sK, sV);
    __syncthreads();
  }

  // (2) scores: thread (t, g, part) takes the K row of position t, group g (each value
  // converted once) and runs the chains of heads part*hpt .. of the group; a wave's lanes
  // are 64 positions of one (g, part), so every q read is a broadcast
  const int parts = kAoThreads / (maxL * nkv) > 0 ? kAoThreads / (maxL * nkv) : 1;
  const int hpt = (rep + parts - 1) / parts;
  for (int i = tid; i < maxL * nkv * parts; i += kAoThreads) {
    const int t = i % maxL, gp = i / maxL;
    const int g = gp % nkv, part = gp / nkv;
    const int h0 = g * rep + part * hpt;
    const int nhh = t < L ? (rep - part * hpt < hpt ? rep - part * hpt : hpt) : 0;
    if (nhh <= 0) continue;
    const uint8_t* kr = sK + ((size_t)g * maxL + t) * Lo::kKRowB;
    float sc[kAoMaxHpw] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e0 = 0; e0 < HD; e0 += 16) {   // 16 dims at a time; each head's chain ascends
      float kk[16];
#pragma unroll
      for (int u = 0; u < 16 * Lo::kEsz / 16; u++) {   // 16-byte reads of the row
        const u32x4 w = *(const u32x4*)(kr + e0 * Lo::kEsz + u * 16);
        if constexpr (kF16) {
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 8; j++) kk[u * 8 + j] = lt_h2f((uint16_t)(ww[j >> 1] >> (16 * (j & 1))));
        } else {
          // not __builtin_bit_cast(float, w.y): this hipcc lowers a bit_cast of a vector
          // element to element 0 (every kk would be w.x)
          kk[u * 4 + 0] = __uint_as_float(w.x);
          kk[u * 4 + 1] = __uint_as_float(w.y);
          kk[u * 4 + 2] = __uint_as_float(w.z);
          kk[u * 4 + 3] = __uint_as_float(w.w);
        }
      }
#pragma unroll
      for (int k = 0; k < kAoMaxHpw; k++) {
        if (k < nhh) {
          const float* qh = sq + (h0 + k) * HD + e0;
#pragma unroll
          for (int e = 0; e < 16; e += 4) {
            const f32x4 q4 = *(const f32x4*)(qh + e);
            sc[k] = fmaf(q4.x, kk[e], sc[k]);
            sc[k] = fmaf(q4.y, kk[e + 1], sc[k]);
            sc[k] = fmaf(q4.z, kk[e + 2], sc[k]);
            sc[k] = fmaf(q4.w, kk[e + 3], sc[k]);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kAoMaxHpw; k++)
      if (k < nhh) sS[(h0 + k) * maxL + t] = sc[k] * P.scale;
  }
  __syncthreads();

  // (3) softmax statistics, one wave per head: m and Z folded over lanes t mod 64
  for (int h = wv; h < nh; h += kAoWaves) {
    float* sh = sS + h * maxL;
    float m = -1e30f;
    for (int t = wl; t < L; t += 64) m = fmaxf(m, sh[t]);
    m = wave_max(m);
    float z = 0.0f;
    for (int t = wl; t < L; t += 64) {
      const float e = lt_expf_sel(sh[t] - m);
      sh[t] = e;
      z = z + e;
    }
    z = wave_tree_dpp(z);
    if (wl == 0) sZ[h] = z;
  }
  __syncthreads();

  // (4) O chains: wave (g, part) takes heads part*hpw .. of group g, lane = head dim; the
  // wave reads one staged V row (64 dims) per position, 8 positions per round, each value
  // converted once for the wave's heads
  const int wpg0 = kAoWaves / nkv;
  const int wpg = wpg0 < rep ? wpg0 : rep;                    // waves per KV group
  const int hpw = (rep + wpg - 1) / wpg;
  const int og = wv / wpg, opart = wv - og * wpg;
  const int oh0 = og * rep + opart * hpw;
  const int onh = og < nkv ? (rep - opart * hpw < hpw ? rep - opart * hpw : hpw) : 0;
  float acc[kAoMaxHpw] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (onh > 0) {
    const uint8_t* vr = sV + (size_t)og * Lo::kRowB + wl * Lo::kEsz;
    const size_t vstride = (size_t)nkv * Lo::kRowB;
    int t = 0;
    for (; t + 8 <= L; t += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = kv_elem<kF16>(vr + (t + j) * vstride);
#pragma unroll
      for (int k = 0; k < kAoMaxHpw; k++)
        if (k < onh) {
          const f32x4 e0 = *(const f32x4*)(sS + (oh0 + k) * maxL + t);
          const f32x4 e1 = *(const f32x4*)(sS + (oh0 + k) * maxL + t + 4);
          acc[k] = fmaf(e0.x, v[0], acc[k]);
          acc[k] = fmaf(e0.y, v[1], acc[k]);
          acc[k] = fmaf(e0.z, v[2], acc[k]);
          acc[k] = fmaf(e0.w, v[3], acc[k]);
          acc[k] = fmaf(e1.x, v[4], acc[k]);
          acc[k] = fmaf(e1.y, v[5], acc[k]);
          acc[k] = fmaf(e1.z, v[6], acc[k]);
          acc[k] = fmaf(e1.w, v[7], acc[k]);
        }
    }
    for (; t < L; t++) {
      const float v = kv_elem<kF16>(vr + t * vstride);
#pragma unroll
      for (int k = 0; k < kAoMaxHpw; k++)
        if (k < onh) acc[k] = fmaf(sS[(oh0 + k) * maxL + t], v, acc[k]);
    }
  }
  // (5) out = O / Z, quantized into the GEMV's records (half-wave = one 32-element block)
#pragma unroll
  for (int k = 0; k < kAoMaxHpw; k++)
    if (k < onh) quant_to_rec(acc[k] / sZ[oh0 + k], lane, rec + (2 * (oh0 + k) + (wl >> 5)) * kRecDwords);
  __syncthreads();

  // (6) the O row: lane L folds block L, the half-wave tree, + residual
  const float folded = fold_raw(rw, odd, rec + (lane < nb ? lane : 0) * kRecDwords, 0.0f);
  const float v = halfwave_tree_dpp(lane < nb ? folded : 0.0f);
  if (lane == 0 && row < P.N) P.y[row] = P.resid ? v + rv : v;
}

// Reduce G argmax partials (ties to the lowest index) and publish the token; optionally
// append it to the device history (hist[*count] = id, *count += 1 while < cap).  1024
// threads; each issues all of its partial loads before comparing.
constexpr int kFinThreads = 1024;
constexpr int kFinPer = 8;   // partials per thread per round

__global__ __launch_bounds__(kFinThreads) void k_argmax_finalize(const float* __restrict__ pval,
                                                                 const int* __restrict__ pidx, int G,
                                                                 int* __restrict__ out, int* __restrict__ hist,
                                                                 int* __restrict__ count, int cap) {
  __shared__ float sv[kFinThreads / 64];
  __shared__ int si[kFinThreads / 64];
  // the history count is requested first (only this launch writes it), so the final write
  // does not wait for a load issued after the reduction
  const int c0 = hist ? *count : 0;
  float bv = -__builtin_inff();
  int bi = 0x7FFFFFFF;
  for (int base = 0; base < G; base += kFinThreads * kFinPer) {
    float v[kFinPer];
    int ix[kFinPer];
#pragma unroll
    for (int k = 0; k < kFinPer; k++) {
      const int i = base + k * kFinThreads + threadIdx.x;
      v[k] = i < G ? pval[i] : -__builtin_inff();
      ix[k] = i < G ? pidx[i] : 0x7FFFFFFF;
    }
#pragma unroll
    for (int k = 0; k < kFinPer; k++)
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
    for (int k = 1; k < kFinThreads / 64; k++)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
    *out = bi;
    if (hist) {
      const int c = c0;
      if (c >= 0 && c < cap) {
        hist[c] = bi;
        *count = c + 1;
      }
    }
  }
}

inline int grid_for(long n, int per) { return (int)((n + per - 1) / per); }

// Row mapping.  The gate|up GEMV takes 64 contiguous rows per workgroup (one quant block
// of its SiLU output).  Otherwise each workgroup takes one group of 8 rows when the groups
// fit in one wave of resident workgroups; larger matrices get contiguous blocks of rows:
// 64 per workgroup when a row is a single 32-block item (K <= 1024), else blocks sized so
// about half a resident wave of workgroups covers the matrix (LT_GEMV_ROWS=R forces R
// contiguous rows per workgroup, for tuning sweeps).
int env_rows() {
  static const int env = [] {   // read once (thread-safe initialization)
    const char* s = getenv("LT_GEMV_ROWS");
    const int r = s ? atoi(s) : 0;
    return r < 0 || r % 8 ? 0 : r;
  }();
  return env;
}

// Resident workgroups of a kernel at an LDS size, cached per (kernel, LDS size).
template <typename Kern>
int resident_wgs(Kern kern, size_t shm, int num_cus) {
  constexpr int kCache = 32;
  static const void* cached_k[kCache];
  static size_t cached_shm[kCache];
  static int cached_n[kCache];
  static int used = 0;
  static std::mutex mu;   // launches may come from several host threads
  std::lock_guard<std::mutex> lock(mu);
  const void* key = (const void*)kern;
  for (int i = 0; i < used; i++)
    if (cached_k[i] == key && cached_shm[i] == shm) return cached_n[i];
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, shm) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int n = per_cu * (num_cus > 0 ? num_cus : 1);
  if (used < kCache) { cached_k[used] = key; cached_shm[used] = shm; cached_n[used] = n; used++; }
  return n;
}

// LT_GEMV_STAGE=0 keeps the 64-row mapping on per-lane block loads (for comparisons).
bool use_stage() {
  static const bool on = [] {
    const char* s = getenv("LT_GEMV_STAGE");
    return !(s && s[0] == '0');
  }();
  return on;
}

template <int KS, Pro PRO, Epi EPI, int D>
hipError_t launch_gemv_k(GemvParams P, size_t shm, hipStream_t st, int num_cus, int* grid_out) {
  auto kern = k_gemv_fused<KS, PRO, EPI, D>;
  const int groups = (P.N + 7) / 8;
  const int nk = (P.K / 32 + 31) / 32;   // items (32-block groups) per row
  const bool one_item = nk == 1;
  int grid;
  bool stg = false;   // the 64-row mapping with one item per row: staged streaming
  if (EPI == EPI_SILU) {
    P.row0 = kSiluRows; P.step = 8; P.max_rows = kSiluRows / 8;
    grid = P.N / kSiluRows;
    stg = one_item;
  } else if (EPI == EPI_ROPE_KV) {
    P.row0 = 8; P.step = 8; P.max_rows = 1;   // the row mapping is the kernel's own (4 pairs of a head)
    grid = P.N / 8;
  } else if (env_rows() > 0) {
    const int R = env_rows();
    P.row0 = R; P.step = 8; P.max_rows = R / 8;
    grid = (P.N + R - 1) / R;
  } else {
    const int cap = resident_wgs(kern, shm, num_cus);
    if (P.N >= 4096 && nk >= 2 && nk <= 4 && (P.N <= 8192 || groups > cap)) {
      // 2 to 4 items per row (K = 2048 .. 4096), 4096 to 8192 rows or more rows than one
      // resident round of 8-row workgroups: 16 rows per workgroup, 2 per half-wave (8 items:
      // the ring full).  Measured against 8 rows per workgroup (or the region walk past the
      // resident cap): 4096 x 4096 7.19 -> 6.38 us, the same with the RMS prologue 8.80 ->
      // 7.31, 6144 x 4096 10.86 -> 9.70, 128256 x 4096 96.6 -> 92.1; 14336 x 4096 (one
      // resident round) stays on 8 rows (13.54 against 13.78)
      P.row0 = 16; P.step = 8; P.max_rows = 2;
      grid = (P.N + 15) / 16;
    } else if (groups <= cap) {
      P.row0 = 8; P.step = 8; P.max_rows = 1;
      grid = groups;
    } else if (one_item) {
      // rows of one item (K <= 1024): 64 contiguous rows per workgroup, streamed staged
      P.row0 = kStgRows; P.step = 8; P.max_rows = kStgRows / 8;
      grid = (P.N + kStgRows - 1) / kStgRows;
      stg = true;
    } else {
      // workgroups walking contiguous blocks of rows (their half-waves 8 rows apart), about
      // half a resident wave of them: every workgroup streams one region of the matrix
      const int wgs = cap / 2 > 0 ? cap / 2 : 1;
      const int per = (P.N + wgs - 1) / wgs;
      P.row0 = (per + 7) & ~7; P.step = 8; P.max_rows = P.row0 / 8;
      grid = (P.N + P.row0 - 1) / P.row0;
    }
  }
  if (grid_out) *grid_out = grid;
  if constexpr (D == 8 && KS <= 4) {
    if (stg && use_stage()) {
      auto skern = k_gemv_fused<KS, PRO, EPI, D, true>;
      if (grid <= resident_wgs(skern, shm + kStgBytes, num_cus)) {
        skern<<<grid, kThreads, shm + kStgBytes, st>>>(P);
        return hipGetLastError();
      }
    }
  }
  kern<<<grid, kThreads, shm, st>>>(P);
  return hipGetLastError();
}

// Planar weights: a ring of 4 items (the probes of this layout on the box: 4 beats 8 by
// occupancy, 8 waves per SIMD against 4) and one row per half-wave -- 8 rows per workgroup,
// 16 for matrices of 64k rows or more, 64 for the gate|up SiLU block.  Measured by rows per
// half-wave 1 / 2 / 4 (14336 x 4096: 11.4 / 12.3 / 12.2 us; 4096 x 14336: 11.2 / 11.8 us;
// 4096 x 4096: 5.2 / 5.3 us; 128256 x 4096 at 2: 82.7 us).
template <int KS, Pro PRO, Epi EPI>
hipError_t launch_gemv_pl(GemvParams P, size_t shm, hipStream_t st, int* grid_out) {
  int grid;
  if (EPI == EPI_SILU) {
    P.row0 = kSiluRows; P.step = 8; P.max_rows = kSiluRows / 8;
    grid = P.N / kSiluRows;
  } else if (env_rows() > 0) {
    const int R = env_rows();
    P.row0 = R; P.step = 8; P.max_rows = R / 8;
    grid = (P.N + R - 1) / R;
  } else if (PRO == PRO_RMS || PRO == PRO_EMBED_RMS) {
    // every workgroup of an RMSNorm prologue reads x (twice) and the norm weight and
    // normalizes and quantizes the whole row: about 384 workgroups (8 .. 64 rows each)
    // balance that against the streaming.  Measured against 8 rows (16 from 64k rows):
    // 6144 x 4096 8.27 -> 7.63 us, 4096 x 4096 6.42 -> 6.15, 128256 x 4096 90.1 -> 85.0
    int R = ((P.N + 383) / 384 + 7) & ~7;
    R = R < 8 ? 8 : (R > kSiluRows ? kSiluRows : R);
    P.row0 = R; P.step = 8; P.max_rows = R / 8;
    grid = (P.N + R - 1) / R;
  } else {
    // a staged prologue is a copy: short-lived 8-row workgroups stream best (16 from 64k rows)
    const int R = P.N >= 65536 ? 16 : 8;
    P.row0 = R; P.step = 8; P.max_rows = R / 8;
    grid = (P.N + R - 1) / R;
  }
  if (grid_out) *grid_out = grid;
  k_gemv_fused<KS, PRO, EPI, 4, false, true><<<grid, kThreads, shm, st>>>(P);
  return hipGetLastError();
}

template <Pro PRO, Epi EPI>
hipError_t launch_gemv(const GemvParams& P, lt_ctx* ctx, int* grid_out) {
  const int nb = P.K / 32;
  size_t shm = (kThreads + 4) * sizeof(float) + (size_t)((nb * kRecDwords + 3) & ~3) * 4;
  if (PRO == PRO_STAGE || PRO == PRO_MERGE) shm += (size_t)((P.K + 15) & ~15);
  if (PRO == PRO_EMBED_RMS) shm += (size_t)((P.K + 15) & ~15) + (size_t)P.K * sizeof(float);
  if (PRO == PRO_RMS && P.planar && P.K <= 4096) shm += (size_t)16 * kThreads * sizeof(float);   // rms_inv_lds's xs
  hipStream_t st = ctx->stream;
  const int ncu = ctx->num_cus;
  // ring depth: 2 when a half-wave has at most 2 blocks to stream, else 8 (4 for the
  // register-heavy K > 4096 prologues)
  const int nk = (P.K / 32 + 31) / 32;
  if constexpr (EPI != EPI_ROPE_KV) {
    if (P.planar) {
      if constexpr (PRO == PRO_STAGE) return launch_gemv_pl<1, PRO, EPI>(P, shm, st, grid_out);
      else if constexpr (PRO == PRO_EMBED_RMS) return launch_gemv_pl<16, PRO, EPI>(P, shm, st, grid_out);
      else return P.K <= 4096 ? launch_gemv_pl<16, PRO, EPI>(P, shm, st, grid_out)
                              : launch_gemv_pl<64, PRO, EPI>(P, shm, st, grid_out);
    }
  }
  const bool shallow = EPI != EPI_SILU && (env_rows() == 0 || EPI == EPI_ROPE_KV) && (P.N + 7) / 8 <= 1024 &&
                       nk <= 2;
  if constexpr (PRO == PRO_STAGE) {
    return shallow ? launch_gemv_k<1, PRO, EPI, 2>(P, shm, st, ncu, grid_out)
                   : launch_gemv_k<1, PRO, EPI, 8>(P, shm, st, ncu, grid_out);
  } else {
    if (P.K <= 1024) {
      return shallow ? launch_gemv_k<4, PRO, EPI, 2>(P, shm, st, ncu, grid_out)
                     : launch_gemv_k<4, PRO, EPI, 8>(P, shm, st, ncu, grid_out);
    }
    if (P.K <= 4096) return launch_gemv_k<16, PRO, EPI, 8>(P, shm, st, ncu, grid_out);
    if constexpr (PRO == PRO_EMBED_RMS) return hipErrorInvalidValue;   // K <= 4096 (entry check)
    else if (P.K <= 5120) return launch_gemv_k<20, PRO, EPI, 8>(P, shm, st, ncu, grid_out);
    else return launch_gemv_k<64, PRO, EPI, 4>(P, shm, st, ncu, grid_out);
  }
}

int check_gemv(const char* fn, const void* W, int N, int K) {
  LT_REQUIRE(W, "%s: null weight", fn);
  LT_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && K <= 16384, "%s: N=%d K=%d (K multiple of 32, <= 16384)", fn, N, K);
  LT_REQUIRE((uint64_t)N * (uint64_t)(K / 32) * 34u < ((uint64_t)1 << 32),
             "%s: a %d x %d Q8_0 matrix must be below 4 GiB (split it by rows)", fn, N, K);
  LT_REQUIRE(lt_aligned(W, 4), "%s: W must be 4-byte aligned", fn);
  return LT_OK;
}

// Rows the fused attention + O launch attends at most (0: the geometry is outside it).
template <bool kF16>
int attn_o_max_len(int nh, int nkv, int hd) {
  using Lo = AoLayout<kF16>;
  if (nh <= 0 || nkv <= 0 || nh % nkv || hd != kAoHd || nh * hd > 1024) return 0;   // one block item per O row
  const int rep = nh / nkv;
  const int maxL = Lo::kRows / nkv / 8 * 8;
  if (maxL < 8 || attn_o_lds_bytes<kF16>(nh, nkv, maxL) > kAoLdsMax) return 0;
  const int wpg0 = kAoWaves / nkv;
  const int wpg = wpg0 < rep ? wpg0 : rep;
  if (wpg < 1 || (rep + wpg - 1) / wpg > kAoMaxHpw) return 0;
  const int parts = kAoThreads / (maxL * nkv) > 0 ? kAoThreads / (maxL * nkv) : 1;
  if ((rep + parts - 1) / parts > kAoMaxHpw) return 0;
  return maxL;
}

// The planar entry points (the *_pl twins): K a multiple of 32, and a 16-byte aligned
// planar copy (lt_q8_to_planar).
int check_planar(const char* fn, const void* W, int K) {
  LT_REQUIRE(K % 32 == 0, "%s: K=%d: the planar layout needs K a multiple of 32", fn, K);
  LT_REQUIRE(lt_aligned(W, 16), "%s: the planar weight must be 16-byte aligned", fn);
  return LT_OK;
}

int finish(hipError_t e, const char* kernel) {
  if (e != hipSuccess) return lt_fail_hip(e, kernel, __FILE__, __LINE__);
  return LT_OK;
}

}  // namespace

extern "C" {

static int lt_q8_gemv_impl(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid,
               float* y, int N, int K, bool pl) {
  LT_REQUIRE(ctx && xq && xd && y, "lt_q8_gemv: null argument");
  if (int rc = check_gemv("lt_q8_gemv", W, N, K)) return rc;
  LT_REQUIRE(lt_aligned(xq, 16), "lt_q8_gemv: xq must be 16-byte aligned");
  LT_REQUIRE(lt_aligned(xd, 2), "lt_q8_gemv: xd must be 2-byte aligned");
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_pl", W, K)) return rc;
  }
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.xq = xq; P.xd = xd; P.resid = resid; P.y = y;
  hipError_t e = resid ? launch_gemv<PRO_STAGE, EPI_RESID>(P, ctx, nullptr)
                       : launch_gemv<PRO_STAGE, EPI_STORE>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<stage>");
}

int lt_q8_gemv(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid,
               float* y, int N, int K) {
  return lt_q8_gemv_impl(ctx, W, xq, xd, resid, y, N, K, false);
}

int lt_q8_gemv_pl(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid,
               float* y, int N, int K) {
  return lt_q8_gemv_impl(ctx, W, xq, xd, resid, y, N, K, true);
}

static int lt_q8_gemv_rms_impl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                   const float* resid, float* y, int N, int K, bool pl) {
  LT_REQUIRE(ctx && x && nw && y, "lt_q8_gemv_rms: null argument");
  if (int rc = check_gemv("lt_q8_gemv_rms", W, N, K)) return rc;
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_rms_pl", W, K)) return rc;
  }
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.resid = resid; P.y = y;
  hipError_t e = resid ? launch_gemv<PRO_RMS, EPI_RESID>(P, ctx, nullptr)
                       : launch_gemv<PRO_RMS, EPI_STORE>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<rms>");
}

int lt_q8_gemv_rms(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                   const float* resid, float* y, int N, int K) {
  return lt_q8_gemv_rms_impl(ctx, x, nw, eps, W, resid, y, N, K, false);
}

int lt_q8_gemv_rms_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                   const float* resid, float* y, int N, int K) {
  return lt_q8_gemv_rms_impl(ctx, x, nw, eps, W, resid, y, N, K, true);
}

static int lt_q8_gemv_embed_rms_impl(lt_ctx* ctx, const void* emb, const int* tok, int vocab, float* x_out, int* err,
                         const float* nw, float eps, const void* W, const float* resid, float* y, int N, int K, bool pl) {
  LT_REQUIRE(ctx && emb && tok && x_out && nw && y, "lt_q8_gemv_embed_rms: null argument");
  LT_REQUIRE(vocab > 0, "lt_q8_gemv_embed_rms: vocab=%d", vocab);
  LT_REQUIRE(K <= 4096, "lt_q8_gemv_embed_rms: K=%d (<= 4096)", K);
  if (int rc = check_gemv("lt_q8_gemv_embed_rms", W, N, K)) return rc;
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_embed_rms_pl", W, K)) return rc;
  }
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.emb = (const uint8_t*)emb; P.tok = tok; P.vocab = vocab;
  P.x_out = x_out; P.err = err; P.nw = nw; P.eps = eps; P.resid = resid; P.y = y;
  hipError_t e = resid ? launch_gemv<PRO_EMBED_RMS, EPI_RESID>(P, ctx, nullptr)
                       : launch_gemv<PRO_EMBED_RMS, EPI_STORE>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<embed_rms>");
}

int lt_q8_gemv_embed_rms(lt_ctx* ctx, const void* emb, const int* tok, int vocab, float* x_out, int* err,
                         const float* nw, float eps, const void* W, const float* resid, float* y, int N, int K) {
  return lt_q8_gemv_embed_rms_impl(ctx, emb, tok, vocab, x_out, err, nw, eps, W, resid, y, N, K, false);
}

int lt_q8_gemv_embed_rms_pl(lt_ctx* ctx, const void* emb, const int* tok, int vocab, float* x_out, int* err,
                         const float* nw, float eps, const void* W, const float* resid, float* y, int N, int K) {
  return lt_q8_gemv_embed_rms_impl(ctx, emb, tok, vocab, x_out, err, nw, eps, W, resid, y, N, K, true);
}

int lt_q8_gemv_quant(lt_ctx* ctx, const float* x, const void* W, const float* resid, float* y, int N, int K) {
  LT_REQUIRE(ctx && x && y, "lt_q8_gemv_quant: null argument");
  if (int rc = check_gemv("lt_q8_gemv_quant", W, N, K)) return rc;
  GemvParams P{};
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.x = x; P.resid = resid; P.y = y;
  hipError_t e = resid ? launch_gemv<PRO_QUANT, EPI_RESID>(P, ctx, nullptr)
                       : launch_gemv<PRO_QUANT, EPI_STORE>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<quant>");
}

static int lt_q8_gemv_attn_out_impl(lt_ctx* ctx, const int8_t* xq, const uint16_t* xd, const void* ws, size_t ws_bytes,
                        int nsplit, int nh, int hd, const void* W, const float* resid, float* y, int N, int K,
                        int* len, int maxt, bool pl) {
  LT_REQUIRE(ctx && y, "lt_q8_gemv_attn_out: null argument");
  if (int rc = check_gemv("lt_q8_gemv_attn_out", W, N, K)) return rc;
  LT_REQUIRE(nh > 0 && hd > 0 && nh * hd == K, "lt_q8_gemv_attn_out: nh*hd=%d*%d must equal K=%d", nh, hd, K);
  LT_REQUIRE(nsplit >= 1, "lt_q8_gemv_attn_out: nsplit=%d", nsplit);
  LT_REQUIRE(!len || maxt > 0, "lt_q8_gemv_attn_out: maxt=%d", maxt);
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_attn_out_pl", W, K)) return rc;
  }
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.nsplit = nsplit; P.nh = nh; P.hd = hd;
  P.resid = resid; P.y = y; P.len = len; P.maxt = maxt;
  if (nsplit == 1) {
    LT_REQUIRE(xq && xd && lt_aligned(xq, 16), "lt_q8_gemv_attn_out: nsplit=1 needs the quantized attention (xq 16-byte aligned)");
    P.xq = xq;
    P.xd = xd;
  } else {
    const size_t need = lt_attn_workspace_size(1, nh, hd, nsplit);
    LT_REQUIRE(ws && lt_aligned(ws, 16), "lt_q8_gemv_attn_out: nsplit=%d needs a 16-byte aligned workspace", nsplit);
    if (ws_bytes < need) return lt_fail(LT_ENOMEM, "lt_q8_gemv_attn_out: workspace %zu < %zu bytes", ws_bytes, need);
    const AttnWs w = lt_attn_ws_layout(const_cast<void*>(ws), nh, hd, nsplit);
    P.wsm = w.m;
    P.wsz = w.z;
    P.wso = w.o;
  }
  hipError_t e = resid ? launch_gemv<PRO_MERGE, EPI_RESID>(P, ctx, nullptr)
                       : launch_gemv<PRO_MERGE, EPI_STORE>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<merge>");
}

int lt_q8_gemv_attn_out(lt_ctx* ctx, const int8_t* xq, const uint16_t* xd, const void* ws, size_t ws_bytes,
                        int nsplit, int nh, int hd, const void* W, const float* resid, float* y, int N, int K,
                        int* len, int maxt) {
  return lt_q8_gemv_attn_out_impl(ctx, xq, xd, ws, ws_bytes, nsplit, nh, hd, W, resid, y, N, K, len, maxt, false);
}

int lt_q8_gemv_attn_out_pl(lt_ctx* ctx, const int8_t* xq, const uint16_t* xd, const void* ws, size_t ws_bytes,
                        int nsplit, int nh, int hd, const void* W, const float* resid, float* y, int N, int K,
                        int* len, int maxt) {
  return lt_q8_gemv_attn_out_impl(ctx, xq, xd, ws, ws_bytes, nsplit, nh, hd, W, resid, y, N, K, len, maxt, true);
}

static int lt_q8_gemv_rms_silu_impl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu, int8_t* vq,
                        uint16_t* vd, int F, int K, bool pl) {
  LT_REQUIRE(ctx && x && nw && vq && vd, "lt_q8_gemv_rms_silu: null argument");
  LT_REQUIRE(F > 0 && F % 32 == 0, "lt_q8_gemv_rms_silu: F=%d (multiple of 32)", F);
  if (int rc = check_gemv("lt_q8_gemv_rms_silu", Wgu, 2 * F, K)) return rc;
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_rms_silu_pl", Wgu, K)) return rc;
  }
  P.W = (const uint8_t*)Wgu; P.N = 2 * F; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.yq = vq; P.yd = vd;
  return finish(launch_gemv<PRO_RMS, EPI_SILU>(P, ctx, nullptr), "k_gemv_fused<rms,silu>");
}

int lt_q8_gemv_rms_silu(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu, int8_t* vq,
                        uint16_t* vd, int F, int K) {
  return lt_q8_gemv_rms_silu_impl(ctx, x, nw, eps, Wgu, vq, vd, F, K, false);
}

int lt_q8_gemv_rms_silu_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu, int8_t* vq,
                        uint16_t* vd, int F, int K) {
  return lt_q8_gemv_rms_silu_impl(ctx, x, nw, eps, Wgu, vq, vd, F, K, true);
}

int lt_q8_gemv_rms_swiglu(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu, float* v,
                          int F, int K) {
  LT_REQUIRE(ctx && x && nw && v, "lt_q8_gemv_rms_swiglu: null argument");
  LT_REQUIRE(F > 0 && F % 4 == 0, "lt_q8_gemv_rms_swiglu: F=%d (multiple of 4)", F);
  if (int rc = check_gemv("lt_q8_gemv_rms_swiglu", Wgu, 2 * F, K)) return rc;
  GemvParams P{};
  P.W = (const uint8_t*)Wgu; P.N = 2 * F; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.y = v;
  return finish(launch_gemv<PRO_RMS, EPI_SWIGLU>(P, ctx, nullptr), "k_gemv_fused<rms,swiglu>");
}

int lt_q8_gemv_rms_rope_kv(lt_ctx* ctx, const float* x, const void* emb, const int* tok, int vocab, float* x_out,
                           int* err, const float* nw, float eps, const void* W, const float* bias, float* qkv, int K,
                           const float* freqs, void* kc, void* vc, const int* len, int nh, int nkv, int hd,
                           int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && nw && qkv && freqs && kc && vc && len, "lt_q8_gemv_rms_rope_kv: null argument");
  LT_REQUIRE(emb ? (tok && x_out && vocab > 0 && K <= 4096) : x != nullptr,
             "lt_q8_gemv_rms_rope_kv: needs x, or emb + tok + x_out + vocab with K <= 4096");
  LT_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && hd > 0 && hd % 8 == 0 && maxt > 0,
             "lt_q8_gemv_rms_rope_kv: nh=%d nkv=%d hd=%d maxt=%d", nh, nkv, hd, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_q8_gemv_rms_rope_kv: kv_dtype=%d", kv_dtype);
  const int N = (nh + 2 * nkv) * hd;
  if (int rc = check_gemv("lt_q8_gemv_rms_rope_kv", W, N, K)) return rc;
  GemvParams P{};
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.resid = bias; P.y = qkv;
  P.emb = (const uint8_t*)emb; P.tok = tok; P.vocab = vocab; P.x_out = x_out; P.err = err;
  P.freqs = freqs; P.kc = kc; P.vc = vc; P.lenr = len; P.nh = nh; P.nkv = nkv; P.hd = hd; P.maxt = maxt;
  P.kv_f16 = kv_dtype == LT_KV_F16;
  hipError_t e = emb ? launch_gemv<PRO_EMBED_RMS, EPI_ROPE_KV>(P, ctx, nullptr)
                     : launch_gemv<PRO_RMS, EPI_ROPE_KV>(P, ctx, nullptr);
  return finish(e, "k_gemv_fused<rms,rope_kv>");
}

int lt_q8_gemv_rms_silu_len(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu, int8_t* vq,
                            uint16_t* vd, int F, int K, int* len, int maxt) {
  LT_REQUIRE(ctx && x && nw && vq && vd && len, "lt_q8_gemv_rms_silu_len: null argument");
  LT_REQUIRE(F > 0 && F % 32 == 0 && maxt > 0, "lt_q8_gemv_rms_silu_len: F=%d maxt=%d", F, maxt);
  if (int rc = check_gemv("lt_q8_gemv_rms_silu_len", Wgu, 2 * F, K)) return rc;
  GemvParams P{};
  P.W = (const uint8_t*)Wgu; P.N = 2 * F; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.yq = vq; P.yd = vd;
  P.len_bump = len; P.maxt = maxt;
  return finish(launch_gemv<PRO_RMS, EPI_SILU>(P, ctx, nullptr), "k_gemv_fused<rms,silu,len>");
}

int lt_attn_o_max_len(int nh, int nkv, int hd, int kv_dtype) {
  if (kv_dtype == LT_KV_F16) return attn_o_max_len<true>(nh, nkv, hd);
  if (kv_dtype == LT_KV_F32) return attn_o_max_len<false>(nh, nkv, hd);
  return 0;
}

int lt_q8_gemv_attn_o(lt_ctx* ctx, const float* qkv, const void* kc, const void* vc, const int* len, int nh, int nkv,
                      int hd, float scale, int maxt, int kv_dtype, const void* W, const float* resid, float* y,
                      int N) {
  LT_REQUIRE(ctx && qkv && kc && vc && len && y, "lt_q8_gemv_attn_o: null argument");
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_q8_gemv_attn_o: kv_dtype=%d", kv_dtype);
  const int maxL = lt_attn_o_max_len(nh, nkv, hd, kv_dtype);
  LT_REQUIRE(maxL > 0 && maxt > 0,
             "lt_q8_gemv_attn_o: nh=%d nkv=%d hd=%d kv_dtype=%d is outside the fused kernel (hd 64, nh*hd <= 1024); "
             "use lt_attn_step + lt_q8_gemv_attn_out", nh, nkv, hd, kv_dtype);
  LT_REQUIRE(lt_aligned(kc, 16) && lt_aligned(vc, 16), "lt_q8_gemv_attn_o: caches must be 16-byte aligned");
  if (int rc = check_gemv("lt_q8_gemv_attn_o", W, N, nh * hd)) return rc;
  AttnOParams P{};
  P.qkv = qkv; P.kc = kc; P.vc = vc; P.len = len; P.nh = nh; P.nkv = nkv; P.maxt = maxt; P.scale = scale;
  P.W = (const uint8_t*)W; P.resid = resid; P.y = y; P.N = N; P.maxL = maxL;
  const int grid = (N + kAoRows - 1) / kAoRows;
  if (kv_dtype == LT_KV_F16)
    k_attn_o<true><<<grid, kAoThreads, attn_o_lds_bytes<true>(nh, nkv, maxL), ctx->stream>>>(P);
  else
    k_attn_o<false><<<grid, kAoThreads, attn_o_lds_bytes<false>(nh, nkv, maxL), ctx->stream>>>(P);
  return finish(hipGetLastError(), "k_attn_o");
}

size_t lt_q8_gemv_argmax_workspace_size(int N) {
  if (N <= 0) return 0;
  const int env = env_rows();
  const int G = grid_for(N, env > 0 ? env : 8);   // the most workgroups a launch can use
  return (size_t)G * 8 + 64;
}

static int lt_q8_gemv_rms_argmax_impl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                          float* logits, int N, int K, int* out, int* hist, int* count, int cap,
                          void* ws, size_t ws_bytes, bool pl) {
  LT_REQUIRE(ctx && x && nw && logits && out && ws, "lt_q8_gemv_rms_argmax: null argument");
  LT_REQUIRE(!hist || (count && cap > 0), "lt_q8_gemv_rms_argmax: history needs count and cap > 0");
  if (int rc = check_gemv("lt_q8_gemv_rms_argmax", W, N, K)) return rc;
  const size_t need = lt_q8_gemv_argmax_workspace_size(N);
  if (ws_bytes < need) return lt_fail(LT_ENOMEM, "lt_q8_gemv_rms_argmax: workspace %zu < %zu bytes", ws_bytes, need);
  LT_REQUIRE(lt_aligned(ws, 4), "lt_q8_gemv_rms_argmax: workspace must be 4-byte aligned");
  GemvParams P{};
  P.planar = pl;
  if (pl) {
    if (int rc = check_planar("lt_q8_gemv_rms_argmax_pl", W, K)) return rc;
  }
  P.W = (const uint8_t*)W; P.N = N; P.K = K; P.x = x; P.nw = nw; P.eps = eps; P.y = logits;
  const int env = env_rows();
  const int G = grid_for(N, env > 0 ? env : 8);
  P.pval = (float*)ws;
  P.pidx = (int*)((char*)ws + (size_t)G * 4);
  int grid = 0;
  if (int rc = finish(launch_gemv<PRO_RMS, EPI_ARGMAX>(P, ctx, &grid), "k_gemv_fused<rms,argmax>")) return rc;
  k_argmax_finalize<<<1, kFinThreads, 0, ctx->stream>>>(P.pval, P.pidx, grid, out, hist, count, cap);
  return lt_check_launch("k_argmax_finalize");
}

int lt_q8_gemv_rms_argmax(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                          float* logits, int N, int K, int* out, int* hist, int* count, int cap,
                          void* ws, size_t ws_bytes) {
  return lt_q8_gemv_rms_argmax_impl(ctx, x, nw, eps, W, logits, N, K, out, hist, count, cap, ws, ws_bytes, false);
}

int lt_q8_gemv_rms_argmax_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                          float* logits, int N, int K, int* out, int* hist, int* count, int cap,
                          void* ws, size_t ws_bytes) {
  return lt_q8_gemv_rms_argmax_impl(ctx, x, nw, eps, W, logits, N, K, out, hist, count, cap, ws, ws_bytes, true);
}

}  // extern "C"
