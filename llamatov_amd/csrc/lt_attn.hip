// lt_attn.hip -- GQA attention over a position-major KV cache (fp32 or fp16): the decode
// step's fused RoPE + KV append + attention, batched decode, and causal prefill, all on
// one workgroup kernel with split-K over the context and a deterministic merge launch.
//
// One workgroup per (split, group of HPW query heads sharing one KV head, sequence or
// query token).  A workgroup scores its contiguous range of positions for all HPW heads
// at once, so each K row is read once for the group; then it folds max and Z per head and
// the exp-weighted V sum per (head, dim).  The arithmetic of each head is exactly the
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
// nsplit > 1 splits the context into contiguous ceil(L/nsplit) ranges, writes per-split
// (m, Z, O), and k_attn_merge combines them in ascending split order, the declared order
// attn_decode_split (bpd/lib/ir_param_axes.pl:303-341,
// bpd/kernelgen/experimental/attn_decode_split.cu:37-91).
//
// Latency structure: the thread's K row and the first V chunk are loaded before any
// arithmetic; V is staged through LDS in chunks (double-buffered through registers) so
// the sequential per-dimension chains read LDS; every load of a row that may lie past
// the range is a buffer load (out-of-range offsets read zeros), so loads never sit
// behind branches.
#include <cstdlib>
#include <type_traits>

#include "lt_q8_device.h"

#include <mutex>

namespace {

using namespace lt;

constexpr uint32_t kNoRow = 0x80000000u;   // out-of-range buffer offset: reads zeros
constexpr int kVChunkFloats = 8192;        // 32 KB of staged V per chunk

// AM_PREFILL_RM (k_attn_w1 only): a causal prefill row whose nsplit splits are all computed
// by one wave and merged in registers (no partials, no merge launch)
enum AttnMode { AM_STEP = 0, AM_DECODE = 1, AM_PREFILL = 2, AM_PREFILL_RM = 3 };

struct AttnArgs {
  const float* qkv;     // AM_STEP: q|k|v of the new token (q, k un-roped)
  const float* freqs;   // AM_STEP: RoPE frequencies [hd/2]
  const float* q;       // AM_DECODE / AM_PREFILL: query rows, q_stride floats apart
  int q_stride;
  void* kc;
  void* vc;
  const int* len;       // STEP: *len = position of the new token; DECODE: len[b]; PREFILL: len[0]
  float* out;           // [rows][nh*hd] (optional for STEP)
  int8_t* oq;           // AM_STEP / AM_DECODE: quantized output (optional)
  uint16_t* od;
  int obm;              // > 0: oq / od block-major over obm rows (q8_out_block)
  float* wsm;           // nsplit > 1: partials
  float* wsz;
  float* wso;
  int nh, nkv, hd;
  float scale;
  int maxt, nsplit, per_max;
  int inwg;             // 1: this workgroup computes all nsplit splits of its row and merges them
  int xcd_groups;       // k_attn_w1, one split, one row: workgroup i serves KV group i % 8 (slot i / 8)
};

constexpr int kMaxInWgSplits = 16;   // splits one workgroup can hold (partial outputs in registers)

// Where block g of the quantized output goes (g counts the blocks of the [rows][nh*hd] output
// row by row): row-major, or with obm > 0 block-major over obm rows -- quants [nh*hd/32][obm]
// [32], scales [nh*hd/32][obm], the tiled GEMM's activation layout.
__device__ __forceinline__ size_t q8_out_block(int obm, int nh, int hd, size_t g) {
  if (obm <= 0) return g;
  const size_t nbr = (size_t)(nh * hd / 32);
  const size_t row = g / nbr;
  return (g - row * nbr) * (size_t)obm + row;
}

template <bool kF16>
__device__ __forceinline__ float kv_round(float v) {
  return kF16 ? lt_half_to_float_bits(lt_float_to_half_bits(v)) : v;
}

template <bool kF16, int HPW, int MODE>
__global__ __launch_bounds__(256) void k_attn(AttnArgs A) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int hd = A.hd;
  const int per_max = A.per_max;
  const int nsplit = A.nsplit;
  float* sq = lds;                      // [HPW][hd] q (roped in STEP mode)
  float* sk = sq + HPW * hd;            // [hd] STEP: new k (roped, cache-rounded)
  float* sv = sk + hd;                  // [hd] STEP: new v (cache-rounded)
  float* se = sv + hd;                  // [HPW][per_max] scores, then exps
  float* svt = se + HPW * per_max;      // [kVChunkFloats] staged V (then the output)
  __shared__ float s_ms[HPW * kMaxInWgSplits];   // per (head, split): max, then exp weight
  __shared__ float s_zs[HPW * kMaxInWgSplits];   // per (head, split): Z
  __shared__ float s_z[HPW];                     // per head: the final Z

  const int tid = threadIdx.x;
  const int sp = blockIdx.x;
  const int h0 = blockIdx.y * HPW;
  const int b = blockIdx.z;
  const int rep = A.nh / A.nkv;
  const int g = h0 / rep;
  const int half = hd >> 1;
  const int qd = A.nh * hd;
  const int kvd = A.nkv * hd;
  const size_t kvrow = (size_t)kvd;
  constexpr int kEpu = kF16 ? 8 : 4;               // elements per 16-byte unit
  constexpr int kUpt = kVChunkFloats / kEpu / 256;  // V units per thread per chunk
  constexpr int kKU = 16;                           // K units prefetched per thread
  const int upr = hd / kEpu;                        // units per position row
  const int cpos = kVChunkFloats / hd;              // positions per V chunk

  // @phase attn 0
  // the inputs that do not depend on the length first
  const int nrope = (HPW + 1) * half;
  float x1 = 0.0f, x2 = 0.0f, vnew = 0.0f, fr = 0.0f;
  if (MODE == AM_STEP) {
    if (tid < nrope) {
      const int r = tid / half;
      const int j = tid - r * half;
      const float* src = r < HPW ? A.qkv + (size_t)(h0 + r) * hd : A.qkv + qd + (size_t)g * hd;
      x1 = src[j];
      x2 = src[j + half];
      fr = A.freqs[j];
    }
    if (tid < hd) vnew = A.qkv[qd + kvd + (size_t)g * hd + tid];
  }
  // DECODE / PREFILL: the q rows into registers now, into LDS after the K/V loads issue
  constexpr int kQpt = (HPW * 256 + 255) / 256;   // q values per thread (hd <= 256)
  float qreg[kQpt];
  if (MODE != AM_STEP) {
    const float* qs = A.q + (size_t)b * A.q_stride + (size_t)h0 * hd;
#pragma unroll
    for (int k = 0; k < kQpt; k++) qreg[k] = tid + 256 * k < HPW * hd ? qs[tid + 256 * k] : 0.0f;
  }

  // context: positions [0, nctx); position Lnew (STEP only) comes from registers
  int Lnew = -1, nctx;
  bool valid = true;
  if (MODE == AM_STEP) {
    Lnew = *A.len;
    valid = Lnew >= 0 && Lnew < A.maxt;
    nctx = valid ? Lnew + 1 : 0;
  } else {
    const int L = MODE == AM_PREFILL ? A.len[0] + b + 1 : A.len[b];
    nctx = L < 0 ? 0 : (L > A.maxt ? A.maxt : L);
  }
  const bool inwg = MODE == AM_PREFILL && A.inwg != 0;
  const int nsub = inwg ? nsplit : 1;            // splits inside this workgroup's range
  const int per = inwg ? nctx : (nctx + nsplit - 1) / nsplit;
  const int p0 = sp * per;
  int p1 = p0 + per;
  if (p1 > nctx) p1 = nctx;
  const int n = p1 > p0 ? p1 - p0 : 0;
  const size_t seq_base = MODE == AM_DECODE ? (size_t)b * (size_t)A.maxt * kvrow : 0;
  const size_t head_base = seq_base + (size_t)p0 * kvrow + (size_t)g * hd;
  const int cache_rows = MODE == AM_DECODE ? (int)gridDim.z * A.maxt : A.maxt;
  const int ebytes = kF16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.kc, 0, (int)((size_t)cache_rows * kvrow * ebytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.vc, 0, (int)((size_t)cache_rows * kvrow * ebytes), 0x00020000);

  // @phase attn 1
  // this thread's first K row and the first V chunk, under the prologue's arithmetic
  const bool kpre = upr <= kKU;
  u32x4 kraw[kKU];
  if (kpre) {
    const bool real = tid < n && p0 + tid != Lnew;
#pragma unroll
    for (int u = 0; u < kKU; u++) {
      const int off = (real && u < upr) ? (int)((head_base + (size_t)tid * kvrow + u * kEpu) * ebytes) : (int)kNoRow;
      kraw[u] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, off, 0, 0);
    }
  }
  auto load_vchunk = [&](int c0, u32x4* dst) {
    const int cn = n - c0 < cpos ? n - c0 : cpos;
#pragma unroll
    for (int k = 0; k < kUpt; k++) {
      const int u = tid + 256 * k;
      const int t = u / upr;
      const bool real = t < cn && p0 + c0 + t != Lnew;
      const size_t e = head_base + (size_t)(c0 + t) * kvrow + (size_t)(u - t * upr) * kEpu;
      dst[k] = __builtin_amdgcn_raw_buffer_load_b128(vrsrc, real ? (int)(e * ebytes) : (int)kNoRow, 0, 0);
    }
  };
  u32x4 vraw[kUpt];
  load_vchunk(0, vraw);

  if (MODE == AM_STEP) {
    // RoPE (the arithmetic of k_rope, rope_from_facts.pl:40-69) of the q heads and of the
    // group's k; v rounded through the cache's type
    const float pos = (float)(valid ? Lnew : 0);
    for (int i = tid; i < nrope; i += 256) {
      const int r = i / half;
      const int j = i - r * half;
      if (i != tid) {
        const float* src = r < HPW ? A.qkv + (size_t)(h0 + r) * hd : A.qkv + qd + (size_t)g * hd;
        x1 = src[j];
        x2 = src[j + half];
        fr = A.freqs[j];
      }
      float s, c;
      lt_sincosf(pos * fr, &s, &c);
      const float o1 = fmaf(x1, c, -(x2 * s));
      const float o2 = fmaf(x1, s, x2 * c);
      if (r < HPW) {
        sq[r * hd + j] = o1;
        sq[r * hd + j + half] = o2;
      } else {
        sk[j] = kv_round<kF16>(o1);
        sk[j + half] = kv_round<kF16>(o2);
      }
    }
    if (tid < hd) sv[tid] = kv_round<kF16>(vnew);
  } else {
#pragma unroll
    for (int k = 0; k < kQpt; k++)
      if (tid + 256 * k < HPW * hd) sq[tid + 256 * k] = qreg[k];
  }
  __syncthreads();
  // @phase attn 2

  if (MODE == AM_STEP && valid && sp == 0 && (h0 % rep) == 0 && tid < hd) {
    // the new row into the cache (k_append_kv_incr, dev_residency.py:303-315)
    const size_t off = (size_t)Lnew * kvrow + (size_t)g * hd + tid;
    if (kF16) {
      ((uint16_t*)A.kc)[off] = lt_float_to_half_bits(sk[tid]);
      ((uint16_t*)A.vc)[off] = lt_float_to_half_bits(sv[tid]);
    } else {
      ((float*)A.kc)[off] = sk[tid];
      ((float*)A.vc)[off] = sv[tid];
    }
  }

  // scores: thread per position, HPW sequential fma chains over i
  for (int t = tid; t < n; t += 256) {
    float acc[HPW];
#pragma unroll
    for (int r = 0; r < HPW; r++) acc[r] = 0.0f;
    const bool fresh = p0 + t == Lnew;
    if (fresh) {
      for (int i = 0; i < hd; i++) {
        const float kv = sk[i];
#pragma unroll
        for (int r = 0; r < HPW; r++) acc[r] = fmaf(sq[r * hd + i], kv, acc[r]);
      }
    } else if (kpre) {
      u32x4 kr[kKU];
      if (t == tid) {
#pragma unroll
        for (int u = 0; u < kKU; u++) kr[u] = kraw[u];
      } else {   // positions past the first 256: loaded here, all 16 pieces at once
#pragma unroll
        for (int u = 0; u < kKU; u++) {
          const int off = (u < upr) ? (int)((head_base + (size_t)t * kvrow + u * kEpu) * ebytes) : (int)kNoRow;
          kr[u] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, off, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < kKU; u++) {
        if (u < upr) {
          const uint32_t a[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
          if (kF16) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const float k0 = lt_h2f((uint16_t)(a[q] & 0xFFFFu));
              const float k1 = lt_h2f((uint16_t)(a[q] >> 16));
              const int i = u * 8 + 2 * q;
#pragma unroll
              for (int r = 0; r < HPW; r++) {
                acc[r] = fmaf(sq[r * hd + i], k0, acc[r]);
                acc[r] = fmaf(sq[r * hd + i + 1], k1, acc[r]);
              }
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const float k0 = __builtin_bit_cast(float, a[q]);
              const int i = u * 4 + q;
#pragma unroll
              for (int r = 0; r < HPW; r++) acc[r] = fmaf(sq[r * hd + i], k0, acc[r]);
            }
          }
        }
      }
    } else {
      // rows wider than the prefetch (fp32 with hd > 64): 16-byte pieces in order
      const size_t rowi = head_base + (size_t)t * kvrow;
      for (int u = 0; u < upr; u++) {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(krsrc, (int)((rowi + u * kEpu) * ebytes), 0, 0);
        const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float k0 = __builtin_bit_cast(float, a[q]);
          const int i = u * 4 + q;
#pragma unroll
          for (int r = 0; r < HPW; r++) acc[r] = fmaf(sq[r * hd + i], k0, acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < HPW; r++) se[r * per_max + t] = acc[r] * A.scale;
  }
  __syncthreads();

  // @phase attn 3
  // softmax of each split (the whole range, or nsub splits of length spl inside it)
  const int wave = tid >> 6, wl = tid & 63;
  const int spl = nsub > 1 ? ((n + nsub - 1) / nsub > 0 ? (n + nsub - 1) / nsub : 1) : (n > 0 ? n : 1);
  for (int q = wave; q < HPW * nsub; q += 4) {
    const int r = q / nsub, sub = q - r * nsub;
    const int t0 = sub * spl, t1 = t0 + spl < n ? t0 + spl : n;
    float m = -1e30f;
    for (int t = t0 + wl; t < t1; t += 64) m = fmaxf(m, se[r * per_max + t]);
    m = wave_max(m);
    if (wl == 0) s_ms[q] = m;
  }
  __syncthreads();
  for (int r = 0; r < HPW; r++)
    for (int t = tid; t < n; t += 256)
      se[r * per_max + t] = lt_expf_sel(se[r * per_max + t] - s_ms[r * nsub + t / spl]);
  __syncthreads();
  for (int q = wave; q < HPW * nsub; q += 4) {
    const int r = q / nsub, sub = q - r * nsub;
    const int t0 = sub * spl, t1 = t0 + spl < n ? t0 + spl : n;
    float ls = 0.0f;
    for (int t = t0 + wl; t < t1; t += 64) ls = ls + se[r * per_max + t];
    ls = wave_tree_dpp(ls);   // the frozen 64-lane tree, s = 32 .. 1
    if (wl == 0) s_zs[q] = ls;
  }

  // @phase attn 4
  // O: thread per (head, dim); each a sequential fma chain over t, V staged in LDS in
  // chunks of cpos positions, the next chunk's loads in flight under this chunk's chains
  const int nout = HPW * hd;
  float acc0 = 0.0f, acc1 = 0.0f;   // thread handles outputs tid and tid + 256
  float po0[kMaxInWgSplits], po1[kMaxInWgSplits];   // in-workgroup splits' outputs
#pragma unroll
  for (int i = 0; i < kMaxInWgSplits; i++) { po0[i] = 0.0f; po1[i] = 0.0f; }
  for (int c0 = 0; c0 < n; c0 += cpos) {
    const int cn = n - c0 < cpos ? n - c0 : cpos;
    if (c0 > 0) __syncthreads();   // the previous chunk's readers are done with svt
#pragma unroll
    for (int k = 0; k < kUpt; k++) {
      const int u = tid + 256 * k;
      const int t = u / upr;
      if (t < cn) {
        const int c = u - t * upr;
        float* dst = svt + t * hd + c * kEpu;
        if (p0 + c0 + t == Lnew) {
#pragma unroll
          for (int q = 0; q < kEpu; q++) dst[q] = sv[c * kEpu + q];
        } else {
          const uint32_t a[4] = {vraw[k].x, vraw[k].y, vraw[k].z, vraw[k].w};
          if (kF16) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
              dst[2 * q] = lt_h2f((uint16_t)(a[q] & 0xFFFFu));
              dst[2 * q + 1] = lt_h2f((uint16_t)(a[q] >> 16));
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++) dst[q] = __builtin_bit_cast(float, a[q]);
          }
        }
      }
    }
    if (c0 + cpos < n) load_vchunk(c0 + cpos, vraw);
    __syncthreads();
    // ascending t; where an inner split ends the chain is saved as that split's O and
    // restarts from 0
    for (int t = 0; t < cn;) {
      int tend = cn;
      if (nsub > 1) {
        const int nextb = ((c0 + t) / spl + 1) * spl;   // the next split boundary
        if (nextb - c0 < cn) tend = nextb - c0;
      }
      if (tid < nout) {
        const int r = tid / hd, d = tid - r * hd;
        const float* e = se + r * per_max + c0;
        for (int u = t; u < tend; u++) acc0 = fmaf(e[u], svt[u * hd + d], acc0);
      }
      if (tid + 256 < nout) {
        const int o = tid + 256;
        const int r = o / hd, d = o - r * hd;
        const float* e = se + r * per_max + c0;
        for (int u = t; u < tend; u++) acc1 = fmaf(e[u], svt[u * hd + d], acc1);
      }
      t = tend;
      const int g1 = c0 + t;   // positions folded so far
      if (nsub > 1 && g1 % spl == 0 && g1 < n) {   // an inner boundary: split g1/spl - 1 ends
        const int ended = g1 / spl - 1;
#pragma unroll
        for (int i = 0; i < kMaxInWgSplits; i++)
          if (i == ended) { po0[i] = acc0; po1[i] = acc1; }
        acc0 = 0.0f;
        acc1 = 0.0f;
      }
    }
  }
  if (nsub > 1) {
    // the last nonempty split ends at n; then merge the splits in ascending order (the
    // declared combine, attn_decode_split.cu:37-91)
    const int last = n > 0 ? (n - 1) / spl : 0;
#pragma unroll
    for (int i = 0; i < kMaxInWgSplits; i++)
      if (i == last && n > 0) { po0[i] = acc0; po1[i] = acc1; }
    __syncthreads();   // s_ms / s_zs complete
    if (tid < HPW) {
      float M = -1e30f;
      for (int q = 0; q < nsub; q++) M = fmaxf(M, s_ms[tid * nsub + q]);
      float Z = 0.0f;
      for (int q = 0; q < nsub; q++) {
        const float w = lt_expf_sel(s_ms[tid * nsub + q] - M);
        s_ms[tid * nsub + q] = w;
        Z = fmaf(w, s_zs[tid * nsub + q], Z);
      }
      s_z[tid] = Z;
    }
    __syncthreads();
    acc0 = 0.0f;
    acc1 = 0.0f;
    const int r0 = (tid < nout ? tid : 0) / hd;
    const int r1 = (tid + 256 < nout ? tid + 256 : 0) / hd;
#pragma unroll
    for (int i = 0; i < kMaxInWgSplits; i++) {
      if (i < nsub) {
        acc0 = fmaf(s_ms[r0 * nsub + i], po0[i], acc0);
        acc1 = fmaf(s_ms[r1 * nsub + i], po1[i], acc1);
      }
    }
  } else if (tid < HPW) {
    s_z[tid] = s_zs[tid];
  }
  __syncthreads();
  const size_t hrow0 = (size_t)b * A.nh + h0;   // output / partial row of head h0
  for (int k = 0; k < 2; k++) {
    const int o = tid + 256 * k;
    if (o >= nout) break;
    const int r = o / hd, d = o - r * hd;
    const float a = k ? acc1 : acc0;
    if (nsplit == 1 || inwg) {
      const float v = valid ? a / s_z[r] : 0.0f;
      if (A.out) A.out[hrow0 * hd + o] = v;
      svt[o] = v;
    } else {
      A.wso[((hrow0 + r) * nsplit + sp) * hd + d] = a;
    }
  }
  if (nsplit > 1 && !inwg) {
    if (tid < HPW) {
      A.wsm[(hrow0 + tid) * nsplit + sp] = s_ms[tid];
      A.wsz[(hrow0 + tid) * nsplit + sp] = s_z[tid];
    }
    return;   // k_attn_merge combines the partials
  }
  // @phase attn 5
  if ((MODE == AM_STEP || MODE == AM_DECODE) && A.oq) {
    // the workgroup's heads are whole 32-element blocks of the row's attention vector:
    // quantize them for the O projection (k_quant_q8's quantizer)
    __syncthreads();
    const int lane = tid & 31;
    const size_t o0 = hrow0 * hd;
    for (int q = tid >> 5; q < nout / 32; q += 8) {
      const size_t gb = q8_out_block(A.obm, A.nh, A.hd, (o0 >> 5) + q);
      quant_block_hw(svt[q * 32 + lane], lane, A.oq + gb * 32, A.od + gb);
    }
  }
  // @phase attn 6
}

// Single-wave attention for batched decode (AM_DECODE), causal prefill (AM_PREFILL: query
// row b of one sequence is a decode of *len + b + 1 positions of the shared cache) and the
// decode step (AM_STEP: RoPE of q and the new k, the KV append and the quantized output
// fused in, as k_attn does): one wave per workgroup, (split, HPW heads of one KV group,
// sequence or query row).  The same
// per-split arithmetic as k_attn, laid out so nothing waits on a barrier or on LDS-staged V:
//   scores   one lane per position (K row from LDS), the heads' sequential fma chains over
//            i, times scale, into LDS position-major [t][HPW];
//   max      per head over the split (fmax, order-free);
//   Z        lane l folds e_t over its positions l, l+64, ... in ascending order, then the
//            64-lane tree (the frozen strided order);
//   O        lane l owns dims [l*DPL, l*DPL + DPL) of every head: HPW*DPL sequential fma
//            chains over t ascending, reading V rows straight from HBM (a wave reads one
//            whole row per load) and the HPW exps of row t by one broadcast LDS read.
// In a step the new position's K and V rows come from the RoPE'd registers (rounded
// through the cache's type): they replace the loaded rows in the LDS K round and in the V
// ring, so no workgroup depends on another's append.
// Loads run as rings: each V row slot is refilled with the next row as soon as it is
// consumed, and a K round is in flight while the previous one is scored.  Every load is
// unconditional (past the range a buffer offset reads zeros, or the row is clamped) and
// tails are masked by selects, so waits stay partial.  Every K/V row is read once per KV
// group.  Bit-identical to k_attn's results.
constexpr int kVRingDw = 32;       // V dwords in flight per lane, batched decode (many waves)
constexpr int kVRingDwStep = 56;   // the decode step (few waves): a deep ring (under the 63 loads a wave can count), issued before the scores

template <bool kF16, int HPW, int DPL, int MODE>
// (occupancy hint: 3 waves per SIMD where a K row is at most 16 units and at most 4 heads
// share the wave, else 2 -- 8 heads' exps and outputs need the registers -- and 1 for the
// step's deep ring)
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(
    MODE == AM_STEP ? 1 : (kF16 ? DPL * 8 : DPL * 16) <= 16 && HPW <= 4 ? 3 : 2))) void k_attn_w1(AttnArgs A) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  constexpr bool kStep = MODE == AM_STEP;
  constexpr bool kRM = MODE == AM_PREFILL_RM;
  constexpr int HD = 64 * DPL;
  constexpr int kEb = kF16 ? 2 : 4;                 // bytes per cache element
  constexpr int KU = HD * kEb / 16;                 // 16-byte units per K row
  constexpr int kVB = DPL * kEb;                    // V bytes per lane per row (2 .. 16)
  constexpr int VD = kVB < 4 ? 1 : kVB / 4;         // registers per V row
  constexpr int OPL = DPL;                          // outputs per lane per head
  constexpr int kEg = 8;                            // exps read per group in the O loop
  constexpr int kVRing = (kStep ? kVRingDwStep : kVRingDw) / VD / kEg * kEg;   // V rows in flight
  // K/V cache policy: a batched decode whose waves hold 4 or more heads (in practice all heads
  // of a KV group) reads each cache row once, so its loads are non-temporal (C4 batch 8 at 16k:
  // 105 -> 90 us); with fewer heads per wave, in a step or in a prefill, rows are re-read from
  // L2 (the group's other heads, the later query rows) and keep the default policy
  constexpr int kKvPolicy = MODE == AM_DECODE && HPW >= 4 ? 2 : 0;
  const int per_up = (A.per_max + kVRing - 1) / kVRing * kVRing;   // per_max rounded to whole rings
  const int srow = per_up + kEg;                    // the spare score row
  // The step with 64 fp16 dims (a V row is 128 bytes): V streams in chunks of kCR rows, one
  // 16-byte load per lane (8 lanes per row), kNC chunks in flight, and each chunk passes
  // through 1 KB of LDS to the lanes' dims -- 8x fewer load instructions than a row per
  // load, so a whole short context is in flight at once.
  constexpr bool kChunk = kStep && kF16 && DPL == 1;
  // kK2 (the chunked step): K rounds are requested two ahead (round r + 2 while round r is
  // scored, rounds 0 and 1 at the start), so a context of two or three rounds waits for one
  // round trip instead of one per round; 16 chunks in flight instead of 24 make the room
  constexpr bool kK2 = kChunk;
  constexpr int kCR = 8;                            // rows per chunk (one exp group)
  constexpr int kNC = kK2 ? 16 : 24;                // chunks in flight
  static_assert(!kChunk || kCR == kEg, "k_attn_w1: a V chunk is one exp group");
  constexpr int kPR = HPW >= 2 ? 32 : 64;           // positions per score round
  static_assert(KU >= 8 && KU <= 32, "k_attn_w1: unsupported head size / cache type");
  float* sq = lds;                                  // [HPW][HD] q (roped in a step); then the outputs
  u32x4* sk = (u32x4*)(lds + HPW * HD);             // [kPR][KU + 1] one round of K rows, padded
  u32x4* sfk = sk + kPR * (KU + 1);                 // step: the new K row, then the new V row (cache format)
  // [per_up + kEg + 1 (+ 64 in kRM: the Z trees' reads past a split)][HPW]: rows (zero past n), spare
  float* se = (float*)(sfk + (kStep ? 2 * KU : 0));
  constexpr int kRmPad = kRM ? 64 : 0;
  uint32_t* sv = (uint32_t*)(se + ((per_up + kEg + 1 + kRmPad) * HPW + 3) / 4 * 4);   // kChunk: 2 x 1 KB
  float* srm = (float*)sv;                          // kRM: [3][nsplit*HPW] m_s, Z_s, w_s; then [HPW] Z
  const int l = threadIdx.x;
  const int sp = blockIdx.x;
  // xcd_groups: workgroups are dealt to the 8 XCDs round-robin by id, so id i runs on XCD
  // i % 8; giving XCD g all the workgroups of KV group g keeps the group's K/V rows in one L2
  // (fetched from HBM once, not once per head); ids whose XCD has no group exit at once
  int h0 = blockIdx.y * HPW;
  if (A.xcd_groups) {
    const int x = (int)(blockIdx.y & 7u), k = (int)(blockIdx.y >> 3);
    if (x >= A.nkv) return;
    h0 = x * (A.nh / A.nkv) + k * HPW;
  }
  // kRM: the longest rows first (a row's work grows with its position)
  const int b = kRM ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  const int rep = A.nh / A.nkv;
  const int g = h0 / rep;
  const int kvrow = A.nkv * HD;                     // elements per cache position

  // the step's length first, then the new token's inputs: waiting for the length (which
  // places the cache reads) does not wait for the inputs, and waiting for the inputs
  // never waits for cache rows
  const int len0 = kStep ? *A.len : MODE == AM_PREFILL || kRM ? A.len[0] + b + 1 : A.len[b];
  constexpr int kHalf = HD / 2;
  constexpr int kRopeIt = ((HPW + 1) * kHalf + 63) / 64;
  // Lane l's rotary pair index in RoPE iteration it is (l + 64·it) mod kHalf: with kHalf
  // = 32 or 64 always the same, with 128 one of two -- so each lane evaluates sin/cos for
  // kJ angles only, shared by every head it rotates (the same function of the same value)
  constexpr int kJ = kHalf <= 64 ? 1 : kHalf / 64;
  float rx1[kRopeIt], rx2[kRopeIt], rfq[kJ], rv[DPL];
  if (kStep) {
#pragma unroll
    for (int it = 0; it < kRopeIt; it++) {
      const int i0 = l + 64 * it < (HPW + 1) * kHalf ? l + 64 * it : 0;
      const int r = i0 / kHalf, j = i0 - r * kHalf;
      const float* src = r < HPW ? A.qkv + (size_t)(h0 + r) * HD : A.qkv + (size_t)A.nh * HD + (size_t)g * HD;
      rx1[it] = src[j];
      rx2[it] = src[j + kHalf];
    }
#pragma unroll
    for (int q = 0; q < kJ; q++) rfq[q] = A.freqs[(l % kHalf) + 64 * q];
#pragma unroll
    for (int k = 0; k < DPL; k++) rv[k] = A.qkv[(size_t)A.nh * HD + kvrow + (size_t)g * HD + l + 64 * k];
  }

  int Lnew = -1, nctx;
  bool valid = true;
  if (kStep) {
    Lnew = len0;
    valid = Lnew >= 0 && Lnew < A.maxt;
    nctx = valid ? Lnew + 1 : 0;
  } else {
    nctx = len0 < 0 ? 0 : (len0 > A.maxt ? A.maxt : len0);
  }
  const int per = kRM ? nctx : (nctx + A.nsplit - 1) / A.nsplit;   // kRM: the whole row, split later
  const int p0 = sp * per;
  const int p1 = p0 + per < nctx ? p0 + per : nctx;
  const int n = p1 > p0 ? p1 - p0 : 0;
  const int tnew = kStep ? Lnew - p0 : -1;          // the new position within this split (if 0 <= tnew < n)
  const uint32_t rows = MODE == AM_DECODE ? (uint32_t)gridDim.z * (uint32_t)A.maxt : (uint32_t)A.maxt;
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.kc, 0, (int)(rows * (uint32_t)kvrow * kEb), 0x00020000);
  // byte offset of (position p0 of this split, head group g) and the row pitch
  const uint32_t seq0 = MODE == AM_DECODE ? (uint32_t)b * (uint32_t)A.maxt : 0u;   // the sequence's first row
  const uint32_t base = (seq0 + (uint32_t)p0) * (uint32_t)kvrow * kEb + (uint32_t)g * HD * kEb;
  const uint32_t pitch = (uint32_t)kvrow * kEb;
  // The V rows read from the cache are the split's first nv rows (a step's new row, the
  // split's last, is folded from registers): a buffer that ends right after them makes
  // every later row read zeros with no per-row test.
  const int nv = kStep && n > 0 && tnew == n - 1 ? n - 1 : n;
  const __amdgpu_buffer_rsrc_t vrsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.vc, 0, (int)(base + (uint32_t)nv * pitch), 0x00020000);

  // 2 bytes per lane (fp16, 64 dims): lanes 2i and 2i+1 load the same dword of the row and
  // take its low / high half
  auto load_v = [&](int t, uint32_t* dst) {
    const int off = (int)(base + (uint32_t)t * pitch + (kVB == 2 ? (uint32_t)(l >> 1) * 4 : (uint32_t)l * kVB));
    if (kVB == 2 || kVB == 4) {
      dst[0] = __builtin_amdgcn_raw_buffer_load_b32(vrsrc, off, 0, kKvPolicy);
    } else if (kVB == 8) {
      const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(vrsrc, off, 0, kKvPolicy);
      dst[0] = w.x; dst[1] = w.y;
    } else {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(vrsrc, off, 0, kKvPolicy);
      dst[0] = w.x; dst[1] = w.y; dst[2] = w.z; dst[3] = w.w;
    }
  };

  // chunk c: rows c*kCR + l/8, bytes (l%8)*16 of each (rows past nv read zeros)
  auto load_chunk = [&](int c, u32x4& dst) {
    const uint32_t off = base + (uint32_t)(c * kCR + (l >> 3)) * pitch + (uint32_t)(l & 7) * 16u;
    dst = __builtin_amdgcn_raw_buffer_load_b128(vrsrc, (int)off, 0, kKvPolicy);
  };

  // @phase attn 0
  // Scores run in rounds of kPR positions.  With HPW >= 2 the two half-waves take half of
  // the heads each for the same 32 positions (lane l: position t0 + l%32, heads
  // hb .. hb+kHL-1), which halves a round's K footprint; with HPW = 1 a round is 64
  // positions.  K rounds are read coalesced: load i of a round brings rows
  // i*(64/KU) + l/KU, unit l%KU (whole rows per instruction); they pass through LDS rows
  // padded by one 16-byte unit, so the lane-per-row reads below (lanes 4 banks apart) are
  // bank-conflict free and every LDS address is a base plus an immediate.
  constexpr int kHL = HPW >= 2 ? HPW / 2 : 1;       // heads per lane
  constexpr int kRpi = 64 / KU;                     // rows per load instruction
  constexpr int kNI = kPR * KU / 64;                // load instructions per round
  const int lr = l % kPR;                           // this lane's row within a round
  const int hb = HPW >= 2 ? (l / 32) * kHL : 0;     // this lane's first head
  const int kl_row = l / KU, kl_unit = l % KU;
  u32x4 kb[kNI];
  // Rows past the split's end are clamped to its last row: their scores only reach the
  // spare LDS row, which no later pass reads (V rows past the end read zeros instead).
  const int nlast = n > 0 ? n - 1 : 0;
  const uint32_t k_last = base + (uint32_t)nlast * pitch + (uint32_t)kl_unit * 16;
  auto load_round = [&](int t0, u32x4* dst) {
    uint32_t off = base + (uint32_t)(t0 + kl_row) * pitch + (uint32_t)kl_unit * 16;
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      dst[i] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, (int)(off < k_last ? off : k_last), 0, kKvPolicy);
      off += kRpi * pitch;
    }
  };
  // a step's V ring, then the first K round: in flight before anything else (the ring's
  // loads are the oldest, so waiting for a ring row never waits for K)
  // (the fences keep the ring's loads in the order its rows are consumed, so each row
  // waits for its own load only)
  uint32_t v[kVRing][VD];
  u32x4 vch[kChunk ? kNC : 1];
  if (kChunk) {
#pragma unroll
    for (int k = 0; k < kNC; k++) {
      load_chunk(k, vch[k]);
      asm volatile("" ::: "memory");
    }
  } else if (kStep) {
#pragma unroll
    for (int k = 0; k < kVRing; k++) {
      load_v(k, v[k]);
      asm volatile("" ::: "memory");
    }
  }
  load_round(0, kb);
  u32x4 kb2[kK2 ? kNI : 1];
  if constexpr (kK2) load_round(kPR, kb2);          // past n: clamped rows (scores reach the spare row)
  uint32_t fv[VD];                                  // step: this lane's part of the new V row
  if (kStep) {
    // RoPE (the arithmetic of k_rope, rope_from_facts.pl:40-69) of the q heads and the
    // group's k; k and v rounded through the cache's type
    const float pos = (float)(valid ? Lnew : 0);
    float snq[kJ], csq[kJ];
#pragma unroll
    for (int q = 0; q < kJ; q++) lt_sincosf(pos * rfq[q], &snq[q], &csq[q]);
#pragma unroll
    for (int it = 0; it < kRopeIt; it++) {
      const int i = l + 64 * it;
      if (i < (HPW + 1) * kHalf) {
        const int r = i / kHalf, j = i - r * kHalf;
        const float sn = snq[kJ == 1 ? 0 : it % kJ], cs = csq[kJ == 1 ? 0 : it % kJ];
        const float o1 = fmaf(rx1[it], cs, -(rx2[it] * sn));
        const float o2 = fmaf(rx1[it], sn, rx2[it] * cs);
        if (r < HPW) {
          sq[r * HD + j] = o1;
          sq[r * HD + j + kHalf] = o2;
        } else if (kF16) {
          ((uint16_t*)sfk)[j] = lt_float_to_half_bits(o1);
          ((uint16_t*)sfk)[j + kHalf] = lt_float_to_half_bits(o2);
        } else {
          ((float*)sfk)[j] = o1;
          ((float*)sfk)[j + kHalf] = o2;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < DPL; k++) {
      if (kF16) ((uint16_t*)(sfk + KU))[l + 64 * k] = lt_float_to_half_bits(rv[k]);
      else ((float*)(sfk + KU))[l + 64 * k] = rv[k];
    }
  } else {
    const float* qs = A.q + (size_t)b * A.q_stride + (size_t)h0 * HD;
#pragma unroll
    for (int k = 0; k < HPW * DPL; k++) sq[l + 64 * k] = qs[l + 64 * k];
  }
  __syncthreads();
  if (kStep) {
    // this lane's dims of the new V row, in the V ring's register format
    const uint32_t* fvr = (const uint32_t*)(sfk + KU);
    if (kVB == 2) fv[0] = fvr[l >> 1];
    else {
#pragma unroll
      for (int w = 0; w < VD; w++) fv[w] = fvr[l * VD + w];
    }
    if (valid && sp == 0 && h0 % rep == 0 && l < KU) {
      // the new row into the cache (k_append_kv_incr, dev_residency.py:303-315)
      const size_t off = ((size_t)Lnew * kvrow + (size_t)g * HD) * kEb;
      *(u32x4*)((char*)A.kc + off + l * 16) = sfk[l];
      *(u32x4*)((char*)A.vc + off + l * 16) = sfk[KU + l];
    }
  }

  // @phase attn 1
  auto score_round = [&](int t0, u32x4* buf, auto prefetch) {
    // this round's rows into LDS (the previous round's reads were issued before these
    // writes, and one wave's LDS operations complete in order), the new row over its
    // loaded copy, then the next round's loads into the same registers
#pragma unroll
    for (int i = 0; i < kNI; i++) sk[(i * kRpi + kl_row) * (KU + 1) + kl_unit] = buf[i];
    if (kStep) {
      const int tr = tnew - t0;
      if (tr >= 0 && tr < kPR && l < KU) sk[tr * (KU + 1) + l] = sfk[l];
    }
    asm volatile("" ::: "memory");
    // prefetch: the round decltype(prefetch)::value rounds ahead into the same registers (0: none)
    if constexpr (decltype(prefetch)::value > 0) load_round(t0 + decltype(prefetch)::value * kPR, buf);
    // passes of kHg heads over this lane's K row in LDS (K unit u with q of unit u, kQu dims
    // per head)
    constexpr int kHg = kHL < 2 ? kHL : 2;
    constexpr int kQu = kF16 ? 8 : 4;
    // stored unconditionally (lanes past the range write the spare row), so the
    // chains are computed in place rather than sunk into branches
    const int t = t0 + lr;
    const int ts = t < n ? t : srow;
    // units in flight: kUD - 1 units' K and q reads ahead of the unit being folded (one
    // head per lane has the registers for 3 ahead; each unit's fmas are tied to the reads
    // before them through the chains, so the compiler cannot hoist them above the reads and
    // wait out one LDS round trip per unit)
    constexpr int kUD = kHg == 1 ? 4 : 2;
#pragma unroll
    for (int g0 = 0; g0 < kHL; g0 += kHg) {
      float acc[kHg];
      float qb[kUD][kHg][kQu];
      u32x4 kb_[kUD];
      auto read_unit = [&](int u, int slot) {
        kb_[slot] = sk[lr * (KU + 1) + u];
#pragma unroll
        for (int r = 0; r < kHg; r++)
#pragma unroll
          for (int i = 0; i < kQu; i++) qb[slot][r][i] = sq[(hb + g0 + r) * HD + u * kQu + i];
      };
#pragma unroll
      for (int r = 0; r < kHg; r++) acc[r] = 0.0f;
#pragma unroll
      for (int u = 0; u < kUD - 1 && u < KU; u++) read_unit(u, u);
#pragma unroll
      for (int u = 0; u < KU; u++) {
        if (u + kUD - 1 < KU) read_unit(u + kUD - 1, (u + kUD - 1) % kUD);
#pragma unroll
        for (int r = 0; r < kHg; r++) asm volatile("" : "+v"(acc[r]) : : "memory");
        const int sl = u % kUD;
        uint32_t a[4] = {kb_[sl].x, kb_[sl].y, kb_[sl].z, kb_[sl].w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
          if (kF16) {
            const float k0 = lt_h2f((uint16_t)(a[c] & 0xFFFFu));
            const float k1 = lt_h2f((uint16_t)(a[c] >> 16));
#pragma unroll
            for (int r = 0; r < kHg; r++) {
              acc[r] = fmaf(qb[sl][r][2 * c], k0, acc[r]);
              acc[r] = fmaf(qb[sl][r][2 * c + 1], k1, acc[r]);
            }
          } else {
            const float k0 = __builtin_bit_cast(float, a[c]);
#pragma unroll
            for (int r = 0; r < kHg; r++) acc[r] = fmaf(qb[sl][r][c], k0, acc[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kHg; r++) se[ts * HPW + hb + g0 + r] = acc[r] * A.scale;
    }
  };
  // the last round loads nothing ahead: loads still pending when the O loop reuses their
  // registers would make it wait for them
  int t0s = 0;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  if constexpr (kK2) {
    // round r in kb (r even) or kb2 (r odd); each refilled with round r + 2 while one exists
    for (; t0s + 3 * kPR < n; t0s += 2 * kPR) {
      score_round(t0s, kb, P2{});
      score_round(t0s + kPR, kb2, P2{});
    }
    if (t0s + 2 * kPR < n) {                        // three rounds left
      score_round(t0s, kb, P2{});
      score_round(t0s + kPR, kb2, P0{});
      score_round(t0s + 2 * kPR, kb, P0{});
    } else if (t0s + kPR < n) {                     // two
      score_round(t0s, kb, P0{});
      score_round(t0s + kPR, kb2, P0{});
    } else if (n > 0) {
      score_round(t0s, kb, P0{});
    }
  } else {
    for (; t0s + kPR < n; t0s += kPR) score_round(t0s, kb, P1{});
    if (n > 0) score_round(t0s, kb, P0{});
  }
  // @phase attn 2
  // batched decode: the first kVRing V rows go out now, under the softmax
  if (!kStep) {
#pragma unroll
    for (int k = 0; k < kVRing; k++) {
      load_v(k, v[k]);
      asm volatile("" ::: "memory");
    }
  }
  __syncthreads();
  float m[HPW], zs[HPW];
  const int rm_np = A.nsplit * HPW;                 // kRM: (split, head) pairs
  const int rm_per = kRM ? (n + A.nsplit - 1) / A.nsplit : 0;   // kRM: positions per split (<= 64)
  if constexpr (kRM) {
    // One lane per (split s, head r), the arithmetic of a split's workgroup and of
    // k_attn_merge: m_s = max of the split's scores, its exps in place, Z_s = the lane fold
    // (one position per lane: 0 + e_j = e_j) through the 64-lane tree of wave_tree_dpp
    // evaluated serially (b_j = z_j + z_{j+32}, then halves 16 .. 1), then
    // w_s = exp(m_s - M) with M = max m_s, and Z = sum over s ascending of fma(w_s, Z_s).
    for (int pi = l; pi < rm_np; pi += 64) {
      const int s_ = pi / HPW, r = pi - s_ * HPW;
      const int q0 = s_ * rm_per;
      const int ns = q0 < n ? (q0 + rm_per < n ? rm_per : n - q0) : 0;
      float* e = se + (ns > 0 ? q0 : 0) * HPW + r;
      float mx = -1e30f;
      for (int t = 0; t < ns; t++) mx = fmaxf(mx, e[t * HPW]);
      for (int t = 0; t < ns; t++) e[t * HPW] = lt_expf_sel(e[t * HPW] - mx);
      float bt[32];
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const float lo = e[j * HPW], hi = e[(j + 32) * HPW];
        bt[j] = (j < ns ? lo : 0.0f) + (j + 32 < ns ? hi : 0.0f);
      }
#pragma unroll
      for (int w = 16; w >= 1; w /= 2)
#pragma unroll
        for (int j = 0; j < w; j++) bt[j] = bt[j] + bt[j + w];
      srm[pi] = mx;
      srm[rm_np + pi] = bt[0];
    }
    __syncthreads();
    for (int pi = l; pi < rm_np; pi += 64) {
      const int r = pi % HPW;
      float M = -1e30f;
      for (int q = 0; q < A.nsplit; q++) M = fmaxf(M, srm[q * HPW + r]);
      srm[2 * rm_np + pi] = lt_expf_sel(srm[pi] - M);
    }
    __syncthreads();
    if (l < HPW) {
      float Z = 0.0f;
      for (int q = 0; q < A.nsplit; q++) Z = fmaf(srm[2 * rm_np + q * HPW + l], srm[rm_np + q * HPW + l], Z);
      srm[3 * rm_np + l] = Z;
    }
  } else {
  // max (order-free: from the stored scores), exps and Z
#pragma unroll
  for (int r = 0; r < HPW; r++) m[r] = -1e30f;
  for (int t = l; t < n; t += 64) {
#pragma unroll
    for (int r = 0; r < HPW; r++) m[r] = fmaxf(m[r], se[t * HPW + r]);
  }
#pragma unroll
  for (int r = 0; r < HPW; r++) {
    m[r] = wave_max(m[r]);
    zs[r] = 0.0f;
  }
  for (int t = l; t < n; t += 64) {
#pragma unroll
    for (int r = 0; r < HPW; r++) {
      const float e = lt_expf_sel(se[t * HPW + r] - m[r]);
      se[t * HPW + r] = e;
      zs[r] = zs[r] + e;
    }
  }
#pragma unroll
  for (int r = 0; r < HPW; r++) zs[r] = wave_tree_dpp(zs[r]);   // lane 0: Z of head r
  }
  // exps of 0 up to the O loop's last ring (those rows read zeros from V)
  {
    const int n_up = (n + kVRing - 1) / kVRing * kVRing;
    for (int i = n * HPW + l; i < n_up * HPW; i += 64) se[i] = 0.0f;
  }
  __syncthreads();

  // @phase attn 3
  // O: ascending t; row slot k is refilled with row t + kVRing once row t is folded.  Past
  // n the exps come from the zero row and the rows read zeros, so fma(0, 0, o) leaves o
  // unchanged (o is never -0: it starts at +0 and +0 + -0 = +0).
  float o[HPW][OPL];
#pragma unroll
  for (int r = 0; r < HPW; r++)
#pragma unroll
    for (int k = 0; k < OPL; k++) o[r][k] = 0.0f;
  // kRM: a[r][k] = sum over splits s ascending of fma(w_s, O_s), each split's chain O_s
  // restarting from 0 at its first row (the trailing empty splits add fma(0, 0, a) = a);
  // rm_nb = rows folded when the current split rm_s ends (-1 after the last)
  float a[kRM ? HPW : 1][kRM ? OPL : 1];
#pragma unroll
  for (int r = 0; r < (kRM ? HPW : 1); r++)
#pragma unroll
    for (int k = 0; k < (kRM ? OPL : 1); k++) a[r][k] = 0.0f;
  int rm_s = 0, rm_nb = kRM ? (n < rm_per ? n : rm_per) : -1;
  auto rm_merge = [&]() {
#pragma unroll
    for (int r = 0; r < (kRM ? HPW : 1); r++) {
      const float w = srm[2 * rm_np + rm_s * HPW + r];
#pragma unroll
      for (int k = 0; k < (kRM ? OPL : 1); k++) {
        a[r][k] = fmaf(w, o[r][k], a[r][k]);
        o[r][k] = 0.0f;
      }
    }
    rm_s++;
    rm_nb = rm_nb == n ? -1 : (rm_nb + rm_per < n ? rm_nb + rm_per : n);
  };
  // The exps of a group of kEg rows are read one group ahead (the per-row fence below keeps
  // the ring in registers and would otherwise make every row wait for its LDS read).
  static_assert(kVRing % kEg == 0, "k_attn_w1: ring of whole exp groups");
  auto read_e = [&](int t, float (*dst)[HPW]) {
#pragma unroll
    for (int j = 0; j < kEg; j++)
#pragma unroll
      for (int r = 0; r < HPW; r++) dst[j][r] = se[(t + j) * HPW + r];
  };
  auto fold_row = [&](const float* e, const uint32_t* x) {
    if (kF16 && kVB == 2) {
      const float x0 = lt_h2f((uint16_t)(l & 1 ? x[0] >> 16 : x[0] & 0xFFFFu));
#pragma unroll
      for (int r = 0; r < HPW; r++) o[r][0] = fmaf(e[r], x0, o[r][0]);
    } else {
#pragma unroll
      for (int w = 0; w < VD; w++) {
        if (kF16) {
          const float x0 = lt_h2f((uint16_t)(x[w] & 0xFFFFu));
          const float x1 = lt_h2f((uint16_t)(x[w] >> 16));
#pragma unroll
          for (int r = 0; r < HPW; r++) {
            o[r][2 * w] = fmaf(e[r], x0, o[r][2 * w]);
            o[r][2 * w + 1] = fmaf(e[r], x1, o[r][2 * w + 1]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < HPW; r++) o[r][w] = fmaf(e[r], __builtin_bit_cast(float, x[w]), o[r][w]);
        }
      }
    }
  };
  float ec[kEg][HPW], en[kEg][HPW];
  read_e(0, ec);
  if constexpr (kChunk) {
    // chunk c: through LDS buffer c % 2 (a wave's LDS operations complete in order, so a
    // buffer is rewritten only after the reads of the chunk before), its kCR rows folded
    // in order, its register slot refilled with chunk c + kNC.  (Writing and reading chunk
    // c + 1 during chunk c's fold measured slower, with the look-ahead conditional or not.)
    const int nch = (n + kCR - 1) / kCR;
    for (int c0 = 0; c0 < nch; c0 += kNC) {
#pragma unroll
      for (int k = 0; k < kNC; k++) {
        const int c = c0 + k;
        if (c >= nch) break;
        read_e((c + 1) * kCR, en);
        u32x4 x = vch[k];
        asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w) : : "memory");
        uint32_t* buf = sv + (k & 1) * 256;
        *(u32x4*)&buf[l * 4] = x;
        load_chunk(c + kNC, vch[k]);
        const uint16_t* b16 = (const uint16_t*)buf;
#pragma unroll
        for (int j = 0; j < kCR; j++) {
          const float x0 = lt_h2f(b16[j * 64 + l]);
#pragma unroll
          for (int r = 0; r < HPW; r++) o[r][0] = fmaf(ec[j][r], x0, o[r][0]);
        }
#pragma unroll
        for (int j = 0; j < kEg; j++)
#pragma unroll
          for (int r = 0; r < HPW; r++) ec[j][r] = en[j][r];
      }
    }
  } else
  for (int t0 = 0; t0 < n; t0 += kVRing) {
#pragma unroll
    for (int k0 = 0; k0 < kVRing; k0 += kEg) {
      read_e(t0 + k0 + kEg, en);
#pragma unroll
      for (int j = 0; j < kEg; j++) {
        const int k = k0 + j;
        uint32_t x[VD];
#pragma unroll
        for (int w = 0; w < VD; w++) x[w] = v[k][w];
        // row t0+k is consumed here
        if (VD == 1) asm volatile("" : "+v"(x[0]) : : "memory");
        else if (VD == 2) asm volatile("" : "+v"(x[0]), "+v"(x[1]) : : "memory");
        else asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[VD > 2 ? 2 : 0]), "+v"(x[VD > 3 ? 3 : 0]) : : "memory");
        // the refill after the fold: the fenced value is dead by then, so the new row can
        // land in the same registers and the ring needs no copies at the loop's back edge
        fold_row(ec[j], x);
        load_v(t0 + k + kVRing, v[k]);
        if constexpr (kRM) {
          if (t0 + k + 1 == rm_nb) rm_merge();
        }
      }
#pragma unroll
      for (int j = 0; j < kEg; j++)
#pragma unroll
        for (int r = 0; r < HPW; r++) ec[j][r] = en[j][r];
    }
  }
  if (kStep && nv < n) {
    // the new row, last in its split
    float e[HPW];
#pragma unroll
    for (int r = 0; r < HPW; r++) e[r] = se[(n - 1) * HPW + r];
    fold_row(e, fv);
  }

  // @phase attn 4
  // outputs: dims [l*OPL, l*OPL + OPL) of each head
  const size_t hrow0 = (size_t)b * A.nh + h0;
  if constexpr (kRM) {
#pragma unroll
    for (int r = 0; r < HPW; r++) {
      const float z = srm[3 * rm_np + r];
#pragma unroll
      for (int k = 0; k < OPL; k++) A.out[(hrow0 + r) * HD + l * OPL + k] = a[r][k] / z;
    }
  } else if (A.nsplit == 1) {
#pragma unroll
    for (int r = 0; r < HPW; r++) {
      const float z = __shfl(zs[r], 0, 64);
#pragma unroll
      for (int k = 0; k < OPL; k++) {
        const float val = valid ? o[r][k] / z : 0.0f;
        if (A.out) A.out[(hrow0 + r) * HD + l * OPL + k] = val;
        if (kStep || (MODE == AM_DECODE && A.oq)) sq[r * HD + l * OPL + k] = val;
      }
    }
    if ((kStep || MODE == AM_DECODE) && A.oq) {
      // the workgroup's heads are whole 32-element blocks of the row's attention vector:
      // quantize them for the O projection (k_quant_q8's quantizer)
      __syncthreads();
      const int lane = l & 31;
      const size_t o0 = hrow0 * HD;
      for (int qb = l >> 5; qb < HPW * HD / 32; qb += 2) {
        const size_t gb = q8_out_block(A.obm, A.nh, A.hd, (o0 >> 5) + qb);
        quant_block_hw(sq[qb * 32 + lane], lane, A.oq + gb * 32, A.od + gb);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < HPW; r++)
#pragma unroll
      for (int k = 0; k < OPL; k++) A.wso[((hrow0 + r) * A.nsplit + sp) * HD + l * OPL + k] = o[r][k];
    if (l == 0) {
#pragma unroll
      for (int r = 0; r < HPW; r++) {
        A.wsm[(hrow0 + r) * A.nsplit + sp] = m[r];
        A.wsz[(hrow0 + r) * A.nsplit + sp] = zs[r];
      }
    }
  }
}

// Batched decode (AM_DECODE) with one wave per query head of a KV group: a workgroup of NW
// waves takes one split of one KV group (all its NW query heads) of one sequence.  Each K round
// (64 positions) is loaded once by the whole workgroup into padded LDS rows; wave w scores its
// head against it (lane = position), then runs its head's softmax and O chains exactly as
// k_attn_w1 with one head per wave does -- the same per-head arithmetic (scores as fma chains
// over the dims in ascending order times scale; max order-free; exps by lt_expf_sel; Z the
// 64-lane strided fold plus tree; O per dim a chain over positions in ascending order), so
// bit-identical to it, with the group's heads on NW waves instead of one wave's serial chains.
// V is staged the same way, in chunks of 32 rows through a double-buffered LDS area, so each
// cache row is read from HBM once per workgroup.

template <bool kF16, int NW, int DPL>
__global__ __launch_bounds__(64 * NW) void k_attn_dec(AttnArgs A) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  constexpr int HD = 64 * DPL;
  constexpr int kEb = kF16 ? 2 : 4;
  constexpr int KU = HD * kEb / 16;                 // 16-byte units per K row
  constexpr int kPR = 64;                           // positions per K round
  constexpr int kNT = 64 * NW;
  constexpr int kLPT = (kPR * KU + kNT - 1) / kNT;  // K loads per thread per round
  static_assert(KU >= 8 && KU <= 32, "k_attn_dec: unsupported head size / cache type");
  const int per_up = (A.per_max + 63) / 64 * 64;
  const int SE = per_up + 64;                       // a head's exps row (the spare past the end)
  float* sq = lds;                                  // [NW][HD]
  u32x4* sk = (u32x4*)(sq + NW * HD);               // [kPR][KU + 1]
  float* se = (float*)(sk + kPR * (KU + 1));        // [NW][SE]
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int sp = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int h = g * NW + w;                         // this wave's query head (NW = nh / nkv)
  const int kvrow = A.nkv * HD;
  const int len0 = A.len[b];
  const int nctx = len0 < 0 ? 0 : (len0 > A.maxt ? A.maxt : len0);
  const int per = (nctx + A.nsplit - 1) / A.nsplit;
  const int p0 = sp * per;
  const int p1 = p0 + per < nctx ? p0 + per : nctx;
  const int n = p1 > p0 ? p1 - p0 : 0;
  const uint32_t pitch = (uint32_t)kvrow * kEb;
  const uint32_t base = ((uint32_t)b * (uint32_t)A.maxt + (uint32_t)p0) * pitch + (uint32_t)g * HD * kEb;
  // rows past the split's end read zeros (the resources end after its n rows)
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.kc, 0, (int)(base + (uint32_t)n * pitch), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc =
      __builtin_amdgcn_make_buffer_rsrc(A.vc, 0, (int)(base + (uint32_t)n * pitch), 0x00020000);
  constexpr int kKvPolicy = 2;                      // every cache row is read once per workgroup

  // K round loads: unit i = tid + kNT*j of the round is row i / KU, unit i % KU
  auto load_round = [&](int t0, u32x4* dst) {
#pragma unroll
    for (int j = 0; j < kLPT; j++) {
      const int i = tid + kNT * j;
      const int r = i / KU, u = i - r * KU;
      const uint32_t off = kPR * KU % kNT == 0 || i < kPR * KU ? base + (uint32_t)(t0 + r) * pitch + (uint32_t)u * 16u : kNoRow;
      dst[j] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, (int)off, 0, kKvPolicy);
    }
  };
  float qv[DPL];
  {
    const float* qrow = A.q + (size_t)b * A.q_stride + (size_t)h * HD;
#pragma unroll
    for (int k = 0; k < DPL; k++) qv[k] = qrow[l + 64 * k];
  }
  u32x4 kb[kLPT];
  load_round(0, kb);
  // V in chunks of kVC rows, loaded once by the whole workgroup (16-byte units, coalesced)
  // into a double-buffered LDS area, two chunks in flight: chunks 0 and 1 are requested after
  // the last K round (requested with the first one they slow the K rounds down: 32k at batch
  // 1 33 us against 30), chunk c + 2 while chunk c is folded.  The loop body is straight-line
  // (no per-chunk tests), which lets the compiler wait for chunk c alone, not c + 1 too.
  constexpr int kVC = 32;                           // rows per chunk
  constexpr int kVU = kVC * KU;                     // 16-byte units per chunk
  constexpr int kVLT = (kVU + kNT - 1) / kNT;       // V loads per thread per chunk
  u32x4* sv = (u32x4*)(se + NW * SE);               // [2][kVC][KU] raw cache rows
  auto load_chunk = [&](int c, u32x4* dst) {
#pragma unroll
    for (int j = 0; j < kVLT; j++) {
      const int i = tid + kNT * j;
      const int r = i / KU, u = i - r * KU;
      const uint32_t off = kVU % kNT == 0 || i < kVU ? base + (uint32_t)(c * kVC + r) * pitch + (uint32_t)u * 16u : kNoRow;
      dst[j] = __builtin_amdgcn_raw_buffer_load_b128(vrsrc, (int)off, 0, kKvPolicy);
    }
  };
  // chunks come in pairs (a last odd chunk gets a zero partner: its rows are past the split's
  // end, so its loads read zeros without touching memory, and their exps are 0)
  const int nch = ((n + kVC - 1) / kVC + 1) & ~1;
  u32x4 vb0[kVLT], vb1[kVLT];
  // this wave's query row (requested before the cache rows, so storing it waits for it alone)
#pragma unroll
  for (int k = 0; k < DPL; k++) sq[w * HD + l + 64 * k] = qv[k];
  const int srow = SE - 1;                          // spare slot for positions past n
  for (int t0 = 0; t0 < n; t0 += kPR) {
#pragma unroll
    for (int j = 0; j < kLPT; j++) {
      const int i = tid + kNT * j;
      if (kPR * KU % kNT == 0 || i < kPR * KU) sk[(i / KU) * (KU + 1) + (i % KU)] = kb[j];
    }
    __syncthreads();
    if (t0 + kPR < n) load_round(t0 + kPR, kb);
    constexpr int kQu = kF16 ? 8 : 4;               // q values per K unit
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const u32x4 kc = sk[l * (KU + 1) + u];
      const uint32_t a4[4] = {kc.x, kc.y, kc.z, kc.w};
      const float* qu = sq + w * HD + u * kQu;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (kF16) {
          acc = fmaf(qu[2 * c], lt_h2f((uint16_t)(a4[c] & 0xFFFFu)), acc);
          acc = fmaf(qu[2 * c + 1], lt_h2f((uint16_t)(a4[c] >> 16)), acc);
        } else {
          acc = fmaf(qu[c], __uint_as_float(a4[c]), acc);
        }
      }
    }
    const int t = t0 + l;
    se[w * SE + (t < n ? t : srow)] = acc * A.scale;
    __syncthreads();                                // the next round rewrites sk
  }

  load_chunk(0, vb0);
  load_chunk(1, vb1);
  // softmax of this wave's head (under the first V chunks' loads)
  float* e = se + w * SE;
  float m = -1e30f;
  for (int t = l; t < n; t += 64) m = fmaxf(m, e[t]);
  m = wave_max(m);
  float zs = 0.0f;
  for (int t = l; t < n; t += 64) {
    const float x = lt_expf_sel(e[t] - m);
    e[t] = x;
    zs = zs + x;
  }
  zs = wave_tree_dpp(zs);                           // lane 0: Z
  const int n_up = nch * kVC;
  for (int t = n + l; t < n_up; t += 64) e[t] = 0.0f;   // past n: exps of 0 (rows read zeros)

  // O: lane l owns dims [l*DPL, l*DPL + DPL) of the head; rows in ascending order (o is never
  // -0, so the zero rows past n leave it unchanged)
  float o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; k++) o[k] = 0.0f;
  auto fold_chunk = [&](int c, u32x4 (&vb)[kVLT]) {
    u32x4* buf = sv + (c & 1) * kVU;
#pragma unroll
    for (int j = 0; j < kVLT; j++) {
      const int i = tid + kNT * j;
      if (kVU % kNT == 0 || i < kVU) buf[i] = vb[j];
    }
    __syncthreads();                                // chunk c in LDS (and every wave's exps)
    load_chunk(c + 2, vb);                          // past the split: zeros, no traffic
    const uint8_t* rows = (const uint8_t*)buf;
#pragma unroll 8
    for (int r = 0; r < kVC; r++) {
      const float ek = e[c * kVC + r];
      const uint8_t* row = rows + r * KU * 16;
      if (kF16) {
        if (DPL == 1) {
          const uint32_t x = ((const uint32_t*)row)[l >> 1];
          o[0] = fmaf(ek, lt_h2f((uint16_t)((l & 1) ? (x >> 16) : (x & 0xFFFFu))), o[0]);
        } else {
          const uint32_t x = ((const uint32_t*)row)[l];
          o[0] = fmaf(ek, lt_h2f((uint16_t)(x & 0xFFFFu)), o[0]);
          o[1] = fmaf(ek, lt_h2f((uint16_t)(x >> 16)), o[1]);
        }
      } else {
#pragma unroll
        for (int d = 0; d < DPL; d++) o[d] = fmaf(ek, ((const float*)row)[l * DPL + d], o[d]);
      }
    }
  };
  for (int c = 0; c < nch; c += 2) {
    fold_chunk(c, vb0);
    fold_chunk(c + 1, vb1);
  }

  const size_t hrow = (size_t)b * A.nh + h;
  if (A.nsplit == 1) {
    const float z = __shfl(zs, 0, 64);
#pragma unroll
    for (int k = 0; k < DPL; k++) {
      const float val = o[k] / z;
      if (A.out) A.out[hrow * HD + l * DPL + k] = val;
      sq[w * HD + l * DPL + k] = val;
    }
    if (A.oq) {
      // the head's HD values are whole 32-element blocks of the row's attention vector
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int lane = l & 31;
      const size_t o0 = hrow * HD;
      for (int qb = l >> 5; qb < HD / 32; qb += 2) {
        const size_t gb = q8_out_block(A.obm, A.nh, A.hd, (o0 >> 5) + qb);
        quant_block_hw(sq[w * HD + qb * 32 + lane], lane, A.oq + gb * 32, A.od + gb);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < DPL; k++) A.wso[(hrow * A.nsplit + sp) * HD + l * DPL + k] = o[k];
    if (l == 0) {
      A.wsm[hrow * A.nsplit + sp] = m;
      A.wsz[hrow * A.nsplit + sp] = zs;
    }
  }
}

// Split-K merge, one workgroup per (query head, row): the declared combine in ascending
// split order (attn_decode_split.cu:37-91): M = max m_s, w_s = exp(m_s - M),
// Z = sum fma(w_s, Z_s), O_d = sum fma(w_s, O_s,d), out = O/Z; optionally the quant of
// the head's hd/32 blocks.  Every partial is fetched by independent buffer loads issued at
// the start (kMergeQ >= nsplit: one memory round trip); the exps run one per thread.  Every
// thread then runs the max and the two sequential chains (Z and its dimension's O) itself,
// fully unrolled, so the broadcast LDS reads of m, w and Z_s are batched rather than paid
// one round trip per split.  len (STEP) marks an out-of-range position: the output is then
// 0, as in the single pass.
template <int kMergeQ>   // split outputs prefetched per thread (>= nsplit)
__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ wsm, const float* __restrict__ wsz,
                                                    const float* __restrict__ wso, const int* __restrict__ len,
                                                    int maxt, float* __restrict__ out, int8_t* __restrict__ oq,
                                                    uint16_t* __restrict__ od, int nh, int hd, int nsplit) {
  __shared__ __attribute__((aligned(16))) float sm[kMergeQ];
  __shared__ __attribute__((aligned(16))) float sz[kMergeQ];
  __shared__ __attribute__((aligned(16))) float sw[kMergeQ];
  __shared__ float sout[256];
  const size_t hrow = (size_t)blockIdx.y * nh + blockIdx.x;
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t orsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wso + hrow * nsplit * hd), 0, nsplit * hd * 4, 0x00020000);
  // every load in range and unconditional (dim clamped to hd-1, split to nsplit-1; the
  // surplus values are never folded), so no load waits behind a branch
  float po[kMergeQ];
  const int dcl = tid < hd ? tid : hd - 1;
#pragma unroll
  for (int q = 0; q < kMergeQ; q++) {
    const int sq_ = q < nsplit ? q : nsplit - 1;
    po[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(orsrc, dcl * 4, sq_ * hd * 4, 0));
  }
  // splits past nsplit: m = -inf (no effect on the max), never folded into Z or O
  if (tid < kMergeQ) {
    sm[tid] = tid < nsplit ? wsm[hrow * nsplit + tid] : -INFINITY;
    sz[tid] = tid < nsplit ? wsz[hrow * nsplit + tid] : 0.0f;
  }
  bool valid = true;
  if (len) {
    const int L = *len;
    valid = L >= 0 && L < maxt;
  }
  __syncthreads();
  float M = -1e30f;   // fmax is exact and order-free
#pragma unroll
  for (int q = 0; q < kMergeQ; q += 4) {
    const float4 m4 = *(const float4*)(sm + q);
    M = fmaxf(M, fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w)));
  }
  if (tid < nsplit) sw[tid] = lt_expf_sel(sm[tid] - M);
  __syncthreads();
  float Z = 0.0f, a = 0.0f;
#pragma unroll
  for (int q = 0; q < kMergeQ; q++) {
    if (q < nsplit) {
      const float w = sw[q];
      Z = fmaf(w, sz[q], Z);
      a = fmaf(w, po[q], a);
    }
  }
  if (tid < hd) {
    const float v = valid ? a / Z : 0.0f;
    if (out) out[hrow * hd + tid] = v;
    sout[tid] = v;
  }
  if (oq) {
    __syncthreads();
    const int lane = tid & 31;
    const size_t o0 = hrow * hd;
    for (int q = tid >> 5; q < hd / 32; q += 8)
      quant_block_hw(sout[q * 32 + lane], lane, oq + o0 + q * 32, od + (o0 >> 5) + q);
  }
}

// The same merge for head sizes that are a multiple of 32, one wave per (32-dim slice of a
// query head, row): lane l owns dim l % 32 of the slice (the two half-waves compute the same
// values; the first one writes them).  The slice's partial outputs of every split
// (kMergeQ x 128 bytes) arrive by 16-byte loads, eight splits per instruction, all in
// flight at once (kMergeQ / 8 <= 16 loads per lane; many small workgroups spread the
// fetch over many CUs), and pass through LDS to the lanes' dims; m and Z of split s come
// from lane s mod 64.  Splits past nsplit are padded with w = 0, Z_s = 0 and O_s = 0, so
// the unrolled chains need no per-split test (which would put every step in its own
// block and serialize the LDS reads): fma(0, 0, c) = c for every c that is not -0, and
// neither chain is ever -0 (both start at +0, and an exact cancellation rounds to +0).
// The declared chains over the splits in ascending order, as k_attn_merge runs them --
// bit-identical to it.
template <int kMergeQ>   // >= nsplit, a multiple of 8
__global__ __launch_bounds__(64) void k_attn_merge32(const float* __restrict__ wsm, const float* __restrict__ wsz,
                                                     const float* __restrict__ wso, const int* __restrict__ len,
                                                     int maxt, float* __restrict__ out, int8_t* __restrict__ oq,
                                                     uint16_t* __restrict__ od, int nh, int hd, int nsplit) {
  constexpr int kM = kMergeQ < 64 ? 64 : kMergeQ;   // m/Z slots: a whole wave's worth
  constexpr int kLd = kMergeQ / 8;                  // 16-byte loads per lane
  __shared__ __attribute__((aligned(16))) float so[kMergeQ * 32];
  __shared__ __attribute__((aligned(16))) float sw[kM];
  __shared__ __attribute__((aligned(16))) float sz[kM];
  const int l = threadIdx.x;
  const int slices = hd >> 5;
  const int c = (int)blockIdx.x % slices;
  const size_t hrow = (size_t)blockIdx.y * nh + (size_t)blockIdx.x / slices;
  // the slice's partials: split s, dims c*32 .. c*32+31 at wso[(hrow*nsplit + s)*hd + c*32]
  const __amdgpu_buffer_rsrc_t orsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wso + hrow * nsplit * hd), 0, nsplit * hd * 4, 0x00020000);
  // m and Z first: loads complete in order, so the max and the exps then overlap the
  // partial outputs' fetch
  float mv[kM / 64], zv[kM / 64];
#pragma unroll
  for (int j = 0; j < kM / 64; j++) {
    const int sp = l + 64 * j;
    const int sc = sp < nsplit ? sp : nsplit - 1;
    mv[j] = wsm[hrow * nsplit + sc];
    zv[j] = wsz[hrow * nsplit + sc];
  }
  asm volatile("" ::: "memory");
  u32x4 po[kLd];
#pragma unroll
  for (int i = 0; i < kLd; i++) {
    const int sp = 8 * i + (l >> 3);
    const int sc = sp < nsplit ? sp : nsplit - 1;   // in range; replaced by zeros below
    po[i] = __builtin_amdgcn_raw_buffer_load_b128(orsrc, (sc * hd + c * 32 + (l & 7) * 4) * 4, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < kM / 64; j++) {
    const int sp = l + 64 * j;
    if (sp >= nsplit) {
      mv[j] = -INFINITY;
      zv[j] = 0.0f;
    }
  }
  bool valid = true;
  if (len) {
    const int L = *len;
    valid = L >= 0 && L < maxt;
  }
  float M = -1e30f;   // fmax is exact and order-free
#pragma unroll
  for (int j = 0; j < kM / 64; j++) M = fmaxf(M, mv[j]);
  M = wave_max(M);
#pragma unroll
  for (int j = 0; j < kM / 64; j++) {
    const int sp = l + 64 * j;
    sw[sp] = sp < nsplit ? lt_expf_sel(mv[j] - M) : 0.0f;
    sz[sp] = zv[j];
  }
#pragma unroll
  for (int i = 0; i < kLd; i++) {
    const int sp = 8 * i + (l >> 3);
    const u32x4 z4 = {0u, 0u, 0u, 0u};
    *(u32x4*)(so + sp * 32 + (l & 7) * 4) = sp < nsplit ? po[i] : z4;
  }
  __syncthreads();
  const int d = l & 31;
  float Z = 0.0f, a = 0.0f;
#pragma unroll
  for (int q = 0; q < kMergeQ; q++) {
    const float w = sw[q];
    Z = fmaf(w, sz[q], Z);
    a = fmaf(w, so[q * 32 + d], a);
  }
  if (l < 32) {
    const float v = valid ? a / Z : 0.0f;
    const size_t o0 = hrow * hd + (size_t)c * 32;
    if (out) out[o0 + l] = v;
    if (oq) quant_block_hw(v, l, oq + o0, od + (o0 >> 5));
  }
}

template <bool kF16, int MODE>
hipError_t launch_attn_k(int hpw, dim3 grid, size_t shm, hipStream_t st, const AttnArgs& A) {
#define LT_ATTN_CASE(H)                                    \
  case H:                                                  \
    k_attn<kF16, H, MODE><<<grid, 256, shm, st>>>(A);      \
    break;
  switch (hpw) {
    LT_ATTN_CASE(1)
    LT_ATTN_CASE(2)
    LT_ATTN_CASE(4)
    LT_ATTN_CASE(7)
    LT_ATTN_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef LT_ATTN_CASE
  return hipGetLastError();
}

// The merge with a prefetch depth covering nsplit (<= 128, checked by the callers): one wave
// per 32-dim slice where the head size allows (LT_ATTN_MERGE32=0 keeps k_attn_merge, for
// comparisons).
void launch_merge(dim3 grid, hipStream_t st, const float* wsm, const float* wsz, const float* wso, const int* len,
                  int maxt, float* out, int8_t* oq, uint16_t* od, int nh, int hd, int nsplit) {
  static const bool m32 = [] {
    const char* s = getenv("LT_ATTN_MERGE32");
    return !(s && s[0] == '0');
  }();
  if (m32 && hd % 32 == 0) {
    const dim3 g(grid.x * (hd / 32), grid.y);
    if (nsplit <= 8)
      k_attn_merge32<8><<<g, 64, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
    else if (nsplit <= 16)
      k_attn_merge32<16><<<g, 64, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
    else if (nsplit <= 32)
      k_attn_merge32<32><<<g, 64, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
    else if (nsplit <= 64)
      k_attn_merge32<64><<<g, 64, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
    else
      k_attn_merge32<128><<<g, 64, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
    return;
  }
  if (nsplit <= 16)
    k_attn_merge<16><<<grid, 256, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
  else if (nsplit <= 32)
    k_attn_merge<32><<<grid, 256, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
  else if (nsplit <= 64)
    k_attn_merge<64><<<grid, 256, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
  else
    k_attn_merge<128><<<grid, 256, 0, st>>>(wsm, wsz, wso, len, maxt, out, oq, od, nh, hd, nsplit);
}

template <bool kF16, int MODE>
hipError_t launch_w1(int hpw, int dpl, dim3 grid, size_t shm, hipStream_t st, const AttnArgs& A) {
#define LT_W1_CASE(H, D)                                            \
  if (hpw == H && dpl == D) {                                       \
    k_attn_w1<kF16, H, D, MODE><<<grid, 64, shm, st>>>(A);          \
    return hipGetLastError();                                       \
  }
  LT_W1_CASE(1, 1) LT_W1_CASE(2, 1) LT_W1_CASE(4, 1) LT_W1_CASE(8, 1)
  LT_W1_CASE(1, 2) LT_W1_CASE(2, 2) LT_W1_CASE(4, 2) LT_W1_CASE(8, 2)
  if constexpr (kF16) {
    LT_W1_CASE(1, 4) LT_W1_CASE(2, 4) LT_W1_CASE(4, 4) LT_W1_CASE(8, 4)
  }
#undef LT_W1_CASE
  return hipErrorInvalidValue;
}

// LT_ATTN_PREFILL_RM=0 keeps a prefill with splits on partials + k_attn_merge (for
// comparisons); the default merges each row's splits in its own wave where they fit.
bool use_rm() {
  static const bool on = [] {
    const char* s = getenv("LT_ATTN_PREFILL_RM");
    return !(s && s[0] == '0');
  }();
  return on;
}

// LT_ATTN_W1=0 keeps every mode on k_attn (for comparisons); the default is k_attn_w1
// wherever its head sizes and LDS budget apply.
bool use_w1() {
  static const bool on = [] {
    const char* s = getenv("LT_ATTN_W1");
    return !(s && s[0] == '0');
  }();
  return on;
}

// Launches the attention (and the merge when nsplit > 1) for `rows` query rows with hpw
// heads per workgroup.
int launch_attn(lt_ctx* ctx, int mode, bool f16, int hpw, int rows, AttnArgs A, void* ws, size_t ws_bytes,
                const char* what) {
  LT_REQUIRE(A.nsplit <= 128, "%s: nsplit=%d (at most 128)", what, A.nsplit);
  // the single-wave kernel (every mode): all heads of a KV group share its K/V reads
  const int rep = A.nh / A.nkv;
  int h = rep % 8 == 0 ? 8 : rep % 4 == 0 ? 4 : rep % 2 == 0 ? 2 : 1;
  const int per_max = (A.maxt + A.nsplit - 1) / A.nsplit;
  if (mode == AM_STEP) {
    // A step is one token: with splits of at most 256 rows its single-wave workgroups are
    // bound by their own serial work (RoPE, scores, exps and the O chains of HPW heads), so
    // one head per wave (rep workgroups per KV group, each re-reading the group's rows from
    // L2) is fastest (8B decode 432 -> 450 tok/s); longer splits keep the heads together.
    // LT_ATTN_STEP_HPW=H caps the heads per wave instead (sweeps).
    static const int cap = [] {
      const char* s = getenv("LT_ATTN_STEP_HPW");
      return s ? atoi(s) : 0;
    }();
    const int c = cap > 0 ? cap : per_max <= 256 ? 1 : 8;
    while (h > c && h > 1) h /= 2;
  } else if (mode == AM_DECODE) {
    // LT_ATTN_DECODE_HPW=H caps a batched decode's heads per wave (sweeps)
    static const int dcap = [] {
      const char* s = getenv("LT_ATTN_DECODE_HPW");
      return s ? atoi(s) : 0;
    }();
    while (dcap > 0 && h > dcap && h > 1) h /= 2;
  } else if (mode == AM_PREFILL) {
    // LT_ATTN_PREFILL_HPW=H caps a prefill's heads per wave (sweeps)
    static const int pcap = [] {
      const char* s = getenv("LT_ATTN_PREFILL_HPW");
      return s ? atoi(s) : 0;
    }();
    while (pcap > 0 && h > pcap && h > 1) h /= 2;
  }
  const int dpl = A.hd / 64;
  const size_t ku = (size_t)A.hd * (f16 ? 2 : 4) / 16;
  const size_t kpr = h >= 2 ? 32 : 64;              // positions per score round
  const int vb = dpl * (f16 ? 2 : 4);               // V bytes per lane per row
  const int ring = (mode == AM_STEP ? kVRingDwStep : kVRingDw) / (vb < 4 ? 1 : vb / 4) / 8 * 8;   // V rows in flight
  const size_t per_up = (size_t)(per_max + ring - 1) / ring * ring;
  const size_t w1_shm = ((size_t)h * A.hd + (kpr * (ku + 1) + (mode == AM_STEP ? 2 * ku : 0)) * 4 +
                         ((per_up + 8 + 1) * h + 3) / 4 * 4) * sizeof(float) +
                        (mode == AM_STEP && f16 && dpl == 1 ? 2048 : 0);   // the step's V chunk buffers
  // fp16: 64, 128 or 256 dims; fp32: 64 or 128 (a K row of 8 to 32 16-byte units)
  const bool w1 = use_w1() && A.hd % 64 == 0 &&
                  (f16 ? (dpl == 1 || dpl == 2 || dpl == 4) : (dpl == 1 || dpl == 2)) && w1_shm <= 64 * 1024;
  // a prefill row's splits in one wave (AM_PREFILL_RM): at most 64 positions per split (each
  // lane of a split's Z tree then holds one position) and the whole row's scores in LDS
  const size_t per_up_rm = (size_t)(A.maxt + ring - 1) / ring * ring;
  const size_t rm_shm = ((size_t)h * A.hd + kpr * (ku + 1) * 4 + ((per_up_rm + 8 + 1 + 64) * h + 3) / 4 * 4 +
                         3 * (size_t)A.nsplit * h + h) * sizeof(float);
  if (w1 && mode == AM_PREFILL && A.nsplit > 1 && per_max <= 64 && rm_shm <= 64 * 1024 && use_rm()) {
    A.per_max = A.maxt;
    const dim3 grid(1, A.nh / h, rows);
    const hipError_t e = f16 ? launch_w1<true, AM_PREFILL_RM>(h, dpl, grid, rm_shm, ctx->stream, A)
                             : launch_w1<false, AM_PREFILL_RM>(h, dpl, grid, rm_shm, ctx->stream, A);
    if (e != hipSuccess) return lt_fail_hip(e, what, __FILE__, __LINE__);
    return lt_check_launch("k_attn_w1");
  }
  if (A.nsplit > 1 && (w1 || !(mode == AM_PREFILL && A.nsplit <= kMaxInWgSplits &&
                               ((size_t)hpw * A.hd + 2 * A.hd + (size_t)hpw * A.maxt + kVChunkFloats) *
                                       sizeof(float) <= 64 * 1024))) {
    const size_t need = lt_attn_ws_bytes(rows * A.nh, A.hd, A.nsplit);
    LT_REQUIRE(ws && lt_aligned(ws, 16), "%s: nsplit=%d needs a 16-byte aligned workspace", what, A.nsplit);
    if (ws_bytes < need) return lt_fail(LT_ENOMEM, "%s: workspace %zu < %zu bytes", what, ws_bytes, need);
    const AttnWs w = lt_attn_ws_layout(ws, rows * A.nh, A.hd, A.nsplit);
    A.wsm = w.m;
    A.wsz = w.z;
    A.wso = w.o;
  }
  // decode with 2, 4, 7 or 8 query heads per KV group on a grid of at most 4 workgroups per CU
  // (batch 1): one wave per head, K and V staged once per workgroup through LDS.  On larger
  // grids its LDS footprint (3 workgroups per CU at 16k) loses to the single-wave kernel's
  // occupancy (batch 8 at 16k: 105 us against 92).  LT_ATTN_DEC=0 keeps the single-wave
  // kernel, LT_ATTN_DEC=2 takes this one at any grid size, for comparisons.
  static const int dec_env = [] {
    const char* s = getenv("LT_ATTN_DEC");
    return s ? atoi(s) : 1;
  }();
  const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const bool dec_on = dec_env == 2 || (dec_env == 1 && (size_t)A.nsplit * A.nkv * rows <= (size_t)4 * cus);
  if (dec_on && mode == AM_DECODE && (rep == 2 || rep == 4 || rep == 7 || rep == 8) && A.hd % 64 == 0 &&
      (dpl == 1 || dpl == 2)) {
    const size_t per_up = (size_t)(per_max + 63) / 64 * 64;
    const size_t dec_shm = ((size_t)rep * A.hd + 64 * (ku + 1) * 4 + (size_t)rep * (per_up + 64)) * sizeof(float) +
                           2 * 32 * ku * 16;
    if (dec_shm <= 64 * 1024) {
      A.per_max = per_max;
      const dim3 grid(A.nsplit, A.nkv, rows);
      hipError_t e = hipErrorInvalidValue;
#define LT_DEC_CASE(F, NW, D)                                                          \
  if (f16 == F && rep == NW && dpl == D) {                                             \
    k_attn_dec<F, NW, D><<<grid, 64 * NW, dec_shm, ctx->stream>>>(A);                  \
    e = hipGetLastError();                                                             \
  }
      LT_DEC_CASE(true, 2, 1) LT_DEC_CASE(true, 4, 1) LT_DEC_CASE(true, 7, 1) LT_DEC_CASE(true, 8, 1)
      LT_DEC_CASE(true, 2, 2) LT_DEC_CASE(true, 4, 2) LT_DEC_CASE(true, 8, 2)
      LT_DEC_CASE(false, 2, 1) LT_DEC_CASE(false, 4, 1) LT_DEC_CASE(false, 7, 1) LT_DEC_CASE(false, 8, 1)
      LT_DEC_CASE(false, 2, 2) LT_DEC_CASE(false, 4, 2) LT_DEC_CASE(false, 8, 2)
#undef LT_DEC_CASE
      if (e != hipSuccess) return lt_fail_hip(e, what, __FILE__, __LINE__);
      if (A.nsplit > 1) {
        launch_merge(dim3(A.nh, rows), ctx->stream, A.wsm, A.wsz, A.wso, nullptr, A.maxt, A.out, A.oq, A.od, A.nh,
                     A.hd, A.nsplit);
        return lt_check_launch("k_attn_merge");
      }
      return lt_check_launch("k_attn_dec");
    }
  }
  if (w1) {
    A.per_max = per_max;
    dim3 grid(A.nsplit, A.nh / h, rows);
    // one step row, one split, several workgroups per KV group, at most 8 groups: place each
    // group's workgroups on one XCD (LT_ATTN_XCD=0 keeps the plain order, for comparison)
    static const bool xcd = [] {
      const char* s = getenv("LT_ATTN_XCD");
      return !(s && s[0] == '0');
    }();
    if (xcd && mode == AM_STEP && A.nsplit == 1 && rows == 1 && A.nkv <= 8 && A.nh / A.nkv > h) {
      A.xcd_groups = 1;
      grid.y = 8 * (A.nh / A.nkv / h);
    }
    hipError_t e;
    if (mode == AM_STEP)
      e = f16 ? launch_w1<true, AM_STEP>(h, dpl, grid, w1_shm, ctx->stream, A)
              : launch_w1<false, AM_STEP>(h, dpl, grid, w1_shm, ctx->stream, A);
    else if (mode == AM_DECODE)
      e = f16 ? launch_w1<true, AM_DECODE>(h, dpl, grid, w1_shm, ctx->stream, A)
              : launch_w1<false, AM_DECODE>(h, dpl, grid, w1_shm, ctx->stream, A);
    else
      e = f16 ? launch_w1<true, AM_PREFILL>(h, dpl, grid, w1_shm, ctx->stream, A)
              : launch_w1<false, AM_PREFILL>(h, dpl, grid, w1_shm, ctx->stream, A);
    if (e != hipSuccess) return lt_fail_hip(e, what, __FILE__, __LINE__);
    if (A.nsplit > 1) {
      launch_merge(dim3(A.nh, rows), ctx->stream, A.wsm, A.wsz, A.wso, mode == AM_STEP ? A.len : nullptr, A.maxt,
                   A.out, A.oq, A.od, A.nh, A.hd, A.nsplit);
      return lt_check_launch("k_attn_merge");
    }
    return lt_check_launch("k_attn_w1");
  }
  auto shm_for = [&](int per_max) {
    return ((size_t)hpw * A.hd + 2 * A.hd + (size_t)hpw * per_max + kVChunkFloats) * sizeof(float);
  };
  // prefill: every query row's splits inside one workgroup when they fit (no merge launch)
  A.inwg = mode == AM_PREFILL && A.nsplit > 1 && A.nsplit <= kMaxInWgSplits && shm_for(A.maxt) <= 64 * 1024;
  A.per_max = A.inwg ? A.maxt : (A.maxt + A.nsplit - 1) / A.nsplit;
  const size_t shm = shm_for(A.per_max);
  if (shm > 64 * 1024)
    return lt_fail(LT_EINVAL, "%s: %zu bytes of LDS for maxt=%d nsplit=%d; raise nsplit", what, shm, A.maxt,
                   A.nsplit);
  const dim3 grid(A.inwg ? 1 : A.nsplit, A.nh / hpw, rows);
  hipError_t e;
  if (mode == AM_STEP)
    e = f16 ? launch_attn_k<true, AM_STEP>(hpw, grid, shm, ctx->stream, A)
            : launch_attn_k<false, AM_STEP>(hpw, grid, shm, ctx->stream, A);
  else if (mode == AM_DECODE)
    e = f16 ? launch_attn_k<true, AM_DECODE>(hpw, grid, shm, ctx->stream, A)
            : launch_attn_k<false, AM_DECODE>(hpw, grid, shm, ctx->stream, A);
  else
    e = f16 ? launch_attn_k<true, AM_PREFILL>(hpw, grid, shm, ctx->stream, A)
            : launch_attn_k<false, AM_PREFILL>(hpw, grid, shm, ctx->stream, A);
  if (e != hipSuccess) return lt_fail_hip(e, what, __FILE__, __LINE__);
  if (A.nsplit > 1 && !A.inwg) {
    launch_merge(dim3(A.nh, rows), ctx->stream, A.wsm, A.wsz, A.wso, mode == AM_STEP ? A.len : nullptr, A.maxt,
                 A.out, A.oq, A.od, A.nh, A.hd, A.nsplit);
    return lt_check_launch("k_attn_merge");
  }
  return lt_check_launch("k_attn");
}

// Heads per workgroup: short caches are latency-bound (one head per workgroup keeps each
// thread's chains short); large caches are bandwidth-bound (the heads of a KV group share
// one workgroup so every K/V row is read once).
int pick_hpw(int nh, int nkv, int hd, size_t cache_bytes) {
  const int rep = nh / nkv;
  if (cache_bytes > ((size_t)4 << 20))
    for (int c : {8, 7, 4, 2})
      if (rep % c == 0 && c * hd <= 512) return c;
  return 1;
}

int check_common(int nh, int nkv, int hd, int maxt, int nsplit, int kv_dtype, const void* kc, const void* vc,
                 size_t cache_bytes, const char* what) {
  LT_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0, "%s: nh=%d nkv=%d", what, nh, nkv);
  LT_REQUIRE(hd > 0 && hd % 8 == 0 && hd <= 256, "%s: hd=%d (multiple of 8, <= 256)", what, hd);
  LT_REQUIRE(maxt > 0 && nsplit >= 1 && nsplit <= maxt, "%s: maxt=%d nsplit=%d", what, maxt, nsplit);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "%s: kv_dtype=%d", what, kv_dtype);
  LT_REQUIRE(lt_aligned(kc, 16) && lt_aligned(vc, 16), "%s: K/V caches must be 16-byte aligned", what);
  LT_REQUIRE(cache_bytes < ((size_t)1 << 31), "%s: %zu bytes of K (or V) cache (at most 2 GiB)", what, cache_bytes);
  return LT_OK;
}

size_t cache_bytes_of(int rows, int maxt, int nkv, int hd, int kv_dtype) {
  return (size_t)rows * maxt * nkv * hd * (kv_dtype == LT_KV_F16 ? 2 : 4);
}

}  // namespace

// Scratch of lt_attn_decode_noalloc: the split-K partials (m, Z, O per split) in a
// file-scope device array instead of a caller workspace.  Each GPU holds its own copy at
// its own address until the process ends; host code never uses the array's name as an
// address (it is a host-side stand-in): lt_init looks the device address up once per
// context, with its device current, and the entry point passes that address.  Every
// split's partials are written before the merge reads them, so nothing needs clearing.
// Calls that overlap on one GPU (two contexts' streams) share the array and race.
constexpr size_t kAttnScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kAttnScratchBytes];

void lt_attn_scratch_bind(lt_ctx* ctx) {
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  ctx->attn_scratch_err = e;
  ctx->attn_scratch = e == hipSuccess ? p : nullptr;
  ctx->attn_scratch_bytes = e == hipSuccess ? kAttnScratchBytes : 0;
}

// One context per GPU may use the scratch: the first whose call needs it claims it, later
// contexts on that GPU are refused (their streams are not ordered with the owner's, so their
// calls would race on the one array), and lt_free_ctx gives it back.
namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
lt_ctx* g_scratch_owner[kScratchMaxDevices] = {};
}  // namespace

static int claim_scratch(lt_ctx* ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (ctx->device < 0 || ctx->device >= kScratchMaxDevices)
    return lt_fail(LT_ESTATE, "lt_attn_decode_noalloc: device %d has no scratch slot", ctx->device);
  lt_ctx*& owner = g_scratch_owner[ctx->device];
  if (!owner) owner = ctx;
  if (owner != ctx)
    return lt_fail(LT_ESTATE,
                   "lt_attn_decode_noalloc: device %d's scratch belongs to another context (calls from two "
                   "contexts would race on it); free that context first, or call lt_attn_decode with a workspace",
                   ctx->device);
  return LT_OK;
}

void lt_attn_scratch_release(lt_ctx* ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (ctx->device >= 0 && ctx->device < kScratchMaxDevices && g_scratch_owner[ctx->device] == ctx)
    g_scratch_owner[ctx->device] = nullptr;
}

extern "C" {

size_t lt_attn_workspace_size(int batch, int nh, int hd, int nsplit) {
  if (nsplit <= 1 || batch <= 0 || nh <= 0 || hd <= 0) return 0;
  return lt_attn_ws_bytes(batch * nh, hd, nsplit);
}

int lt_attn_decode(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                   float* out, int batch, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                   int kv_dtype, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && q && kc && vc && len && out, "lt_attn_decode: null argument");
  LT_REQUIRE(batch > 0, "lt_attn_decode: batch=%d", batch);
  const size_t cb = cache_bytes_of(batch, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_decode")) return rc;
  AttnArgs A = {};
  A.q = q; A.q_stride = nh * hd; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len; A.out = out;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  return launch_attn(ctx, AM_DECODE, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb / batch), batch, A, ws,
                     ws_bytes, "lt_attn_decode");
}

int lt_attn_decode_rows(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc, const int* len,
                        float* out, int batch, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                        int kv_dtype, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && q && kc && vc && len && out, "lt_attn_decode_rows: null argument");
  LT_REQUIRE(batch > 0 && q_stride >= nh * hd, "lt_attn_decode_rows: batch=%d q_stride=%d", batch, q_stride);
  const size_t cb = cache_bytes_of(batch, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_decode_rows")) return rc;
  AttnArgs A = {};
  A.q = q; A.q_stride = q_stride; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len; A.out = out;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  return launch_attn(ctx, AM_DECODE, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb / batch), batch, A, ws,
                     ws_bytes, "lt_attn_decode_rows");
}

int lt_attn_decode_rows_q8(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc, const int* len,
                           float* out, int8_t* oq, uint16_t* od, int batch, int nh, int nkv, int hd, float scale,
                           int maxt, int nsplit, int kv_dtype, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && q && kc && vc && len && oq && od, "lt_attn_decode_rows_q8: null argument");
  LT_REQUIRE(batch > 0 && q_stride >= nh * hd, "lt_attn_decode_rows_q8: batch=%d q_stride=%d", batch, q_stride);
  LT_REQUIRE(hd % 32 == 0, "lt_attn_decode_rows_q8: hd=%d (the quant blocks are 32 elements of one head)", hd);
  const size_t cb = cache_bytes_of(batch, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_decode_rows_q8")) return rc;
  AttnArgs A = {};
  A.q = q; A.q_stride = q_stride; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len; A.out = out;
  A.oq = oq; A.od = od;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  return launch_attn(ctx, AM_DECODE, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb / batch), batch, A, ws,
                     ws_bytes, "lt_attn_decode_rows_q8");
}

int lt_attn_decode_rows_q8_bm(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc,
                              const int* len, float* out, int8_t* oq, uint16_t* od, int batch, int nh, int nkv, int hd,
                              float scale, int maxt, int kv_dtype) {
  const char* fn = "lt_attn_decode_rows_q8_bm";
  LT_REQUIRE(ctx && q && kc && vc && len && oq && od, "%s: null argument", fn);
  LT_REQUIRE(batch > 0 && q_stride >= nh * hd, "%s: batch=%d q_stride=%d", fn, batch, q_stride);
  LT_REQUIRE(hd % 32 == 0, "%s: hd=%d (the quant blocks are 32 elements of one head)", fn, hd);
  const size_t cb = cache_bytes_of(batch, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, 1, kv_dtype, kc, vc, cb, fn)) return rc;
  AttnArgs A = {};
  A.q = q; A.q_stride = q_stride; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len; A.out = out;
  A.oq = oq; A.od = od; A.obm = batch;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = 1;
  return launch_attn(ctx, AM_DECODE, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb / batch), batch, A, nullptr,
                     0, fn);
}

int lt_attn_decode_noalloc(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                           float* out, int batch, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                           int kv_dtype) {
  LT_REQUIRE(ctx && q && kc && vc && len && out, "lt_attn_decode_noalloc: null argument");
  LT_REQUIRE(batch > 0, "lt_attn_decode_noalloc: batch=%d", batch);
  const size_t cb = cache_bytes_of(batch, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_decode_noalloc")) return rc;
  const size_t need = lt_attn_workspace_size(batch, nh, hd, nsplit);
  if (need > 0) {
    if (!ctx->attn_scratch)
      return lt_fail(LT_ESTATE, "lt_attn_decode_noalloc: the device scratch is not bound (%s)",
                     hipGetErrorString(ctx->attn_scratch_err));
    if (need > ctx->attn_scratch_bytes)
      return lt_fail(LT_EINVAL,
                     "lt_attn_decode_noalloc: batch=%d nh=%d hd=%d nsplit=%d needs %zu bytes of split partials, "
                     "more than the %zu-byte device scratch; lower nsplit or batch, or call lt_attn_decode "
                     "with a workspace", batch, nh, hd, nsplit, need, ctx->attn_scratch_bytes);
    if (int rc = claim_scratch(ctx)) return rc;
  }
  AttnArgs A = {};
  A.q = q; A.q_stride = nh * hd; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len; A.out = out;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  return launch_attn(ctx, AM_DECODE, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb / batch), batch, A,
                     ctx->attn_scratch, ctx->attn_scratch_bytes, "lt_attn_decode_noalloc");
}

int lt_attn_prefill(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc, const int* len0,
                    float* out, int T, int nh, int nkv, int hd, float scale, int maxt, int nsplit, int kv_dtype,
                    void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && q && kc && vc && len0 && out, "lt_attn_prefill: null argument");
  LT_REQUIRE(T > 0 && q_stride >= nh * hd, "lt_attn_prefill: T=%d q_stride=%d", T, q_stride);
  const size_t cb = cache_bytes_of(1, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_prefill")) return rc;
  AttnArgs A = {};
  A.q = q; A.q_stride = q_stride; A.kc = (void*)kc; A.vc = (void*)vc; A.len = len0; A.out = out;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  // the T query rows of one sequence re-read the same rows: the heads of a KV group share
  // each workgroup whenever the group divides
  return launch_attn(ctx, AM_PREFILL, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, (size_t)1 << 30), T, A, ws,
                     ws_bytes, "lt_attn_prefill");
}

int lt_attn_step(lt_ctx* ctx, const float* qkv, const float* freqs, void* kc, void* vc, const int* len,
                 float* out, int8_t* xq, uint16_t* xd, int nh, int nkv, int hd, float scale, int maxt, int nsplit,
                 int kv_dtype, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && qkv && freqs && kc && vc && len, "lt_attn_step: null argument");
  const size_t cb = cache_bytes_of(1, maxt, nkv, hd, kv_dtype);
  if (int rc = check_common(nh, nkv, hd, maxt, nsplit, kv_dtype, kc, vc, cb, "lt_attn_step")) return rc;
  LT_REQUIRE(out || xq, "lt_attn_step: needs out or xq/xd");
  LT_REQUIRE(!xq || (xd && hd % 32 == 0), "lt_attn_step: quantized output needs xd and hd %% 32 == 0");
  AttnArgs A = {};
  A.qkv = qkv; A.freqs = freqs; A.kc = kc; A.vc = vc; A.len = len; A.out = out; A.oq = xq; A.od = xd;
  A.nh = nh; A.nkv = nkv; A.hd = hd; A.scale = scale; A.maxt = maxt; A.nsplit = nsplit;
  return launch_attn(ctx, AM_STEP, kv_dtype == LT_KV_F16, pick_hpw(nh, nkv, hd, cb), 1, A, ws, ws_bytes,
                     "lt_attn_step");
}

}  // extern "C"
