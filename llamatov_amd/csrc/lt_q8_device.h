// lt_q8_device.h -- device building blocks of the Q8_0 kernels, shared by the per-op
// kernels (lt_ops.hip) and the fused decode-step kernels (lt_fused.hip).
//
// Wave64 mapping of the reference's wave-32 orders: every order the reference defines
// over 32 lanes (the GEMV's lanes(32) strided fold + shfl_down tree,
// q8_0_from_facts.pl:466-476; the quant's per-block amax, dev_residency.py:867-886) runs
// on one 32-lane half of a 64-lane wavefront, so two reference warps share one CDNA
// wave and the per-lane arithmetic and the tree pairing are the reference's.
#pragma once

#include "lt_internal.h"

namespace lt {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 16-byte vector with 4-byte alignment: global_load_dwordx4 needs only dword alignment.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kBlockBytes = 34;

// One Q8_0 block in registers: the 32 quants re-aligned to dwords, and the fp16 scale.
struct BlockRegs {
  uint32_t q[8];
  uint16_t d;
};

// Block gi (global index row*nb + b) starts at byte 34*gi of the 4-aligned matrix, so it
// is 4-aligned for even gi and 2 mod 4 for odd gi.  The lane loads the 9 aligned dwords
// that cover the block (dwordx4, dwordx4, dword) and re-aligns the quants with
// v_perm_b32.  An even block's 9th dword ends 2 bytes past the block; for the matrix's
// final block (gi == last) those bytes lie outside the allocation, so that one block
// reads its last 2 bytes as a ushort.
__device__ __forceinline__ void load_q8_block(const uint8_t* __restrict__ W, size_t gi, size_t last,
                                              BlockRegs& r) {
  const size_t off = gi * kBlockBytes;
  const uint32_t* p = (const uint32_t*)(W + (off & ~(size_t)3));
  const u32x4_a4 v0 = *(const u32x4_a4*)p;
  const u32x4_a4 v1 = *(const u32x4_a4*)(p + 4);
  const uint32_t w8 = (gi == last && !(gi & 1u)) ? (uint32_t)*(const uint16_t*)(W + off + 32) : p[8];
  const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, w8};
  const bool odd = (gi & 1u) != 0;
  const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
  r.d = odd ? (uint16_t)(w[0] >> 16) : (uint16_t)(w[0] & 0xFFFFu);
#pragma unroll
  for (int i = 0; i < 8; i++) r.q[i] = __builtin_amdgcn_perm(w[i + 1], w[i], sel);
}

// isum = sum of 32 int8 products by 8 x v_dot4_i32_i8 (exact; order-free).
__device__ __forceinline__ int dot_q8_block(const BlockRegs& r, const int8_t* sx /* 16B aligned */) {
  u32x4 x0, x1;
  __builtin_memcpy(&x0, sx, 16);
  __builtin_memcpy(&x1, sx + 16, 16);
  int s = 0;
  s = __builtin_amdgcn_sdot4((int)r.q[0], (int)x0.x, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[1], (int)x0.y, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[2], (int)x0.z, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[3], (int)x0.w, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[4], (int)x1.x, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[5], (int)x1.y, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[6], (int)x1.z, s, false);
  s = __builtin_amdgcn_sdot4((int)r.q[7], (int)x1.w, s, false);
  return s;
}

// One step of a lane's canonical fold: acc = fma(wd*xd, (float)isum, acc).  wd*xd is a
// product of two binary16 values (exact in binary32) and |isum| < 2^24 (exact), so each
// block contributes with exactly one rounding (q8_0_from_facts.pl:357, 408, 505).
__device__ __forceinline__ float fold_block(const BlockRegs& r, const int8_t* sxq_blk, uint16_t xd16,
                                            float acc) {
  const int isum = dot_q8_block(r, sxq_blk);
  return fmaf(lt_h2f(r.d) * lt_h2f(xd16), (float)isum, acc);
}

// The reference's 5-level shfl_down tree over the 32 lanes of a half-wave; lane 0 of the
// half-wave ends with the row value.
__device__ __forceinline__ float halfwave_tree(float acc) {
#pragma unroll
  for (int s = 16; s > 0; s >>= 1) acc = acc + __shfl_down(acc, s, 32);
  return acc;
}

}  // namespace lt

namespace lt {

// ---- wave-level reductions through DPP / ds_swizzle (no LDS traffic) -----------------
// DPP controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_shl:n = 0x100 + n,
// row_mirror = 0x140, row_half_mirror = 0x141.  ds_swizzle bitmask mode offset
// and_mask | or_mask << 5 | xor_mask << 10: 0x401F reads lane ^ 16 within 32 lanes.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// Maximum over the 32 lanes of a half-wave, returned to every lane (max is exact and
// order-free, so any combining pattern gives the same value).
__device__ __forceinline__ float halfwave_max(float a) {
  a = fmaxf(a, dpp_f<0xB1>(a));   // lane ^ 1
  a = fmaxf(a, dpp_f<0x4E>(a));   // lane ^ 2
  a = fmaxf(a, dpp_f<0x141>(a));  // mirror within 8: quads combine
  a = fmaxf(a, dpp_f<0x140>(a));  // mirror within 16: halves of the row combine
  a = fmaxf(a, swz_xor16(a));     // the two 16-lane rows of the half-wave
  return a;
}

// The reference's shfl_down tree over 32 lanes (s = 16, 8, 4, 2, 1: acc[t] += acc[t+s] for
// t < s, q8_0_from_facts.pl:466-476) with lane t reading lane t + s through ds_swizzle
// (s = 16) and DPP row_shl (s < 16, inside the first 16-lane row).  Lane 0 ends with the
// sum; other lanes hold values the tree never reads.
__device__ __forceinline__ float halfwave_tree_dpp(float acc) {
  acc = acc + swz_xor16(acc);
  acc = acc + dpp_f<0x108>(acc);
  acc = acc + dpp_f<0x104>(acc);
  acc = acc + dpp_f<0x102>(acc);
  acc = acc + dpp_f<0x101>(acc);
  return acc;
}

// The 64-lane versions (order: s = 32 first, then the half-wave tree): lane t < 32 reads
// lane t + 32 through ds_bpermute, the rest by swizzle/DPP.  Sum: lane 0 ends with the
// total of the reference's 6-level shfl_down tree; max: every lane ends with the maximum.
__device__ __forceinline__ float wave_tree_dpp(float acc) {
  acc = acc + __shfl_down(acc, 32, 64);
  return halfwave_tree_dpp(acc);
}
__device__ __forceinline__ float wave_max(float a) {
  a = fmaxf(a, __shfl_xor(a, 32, 64));
  return halfwave_max(a);
}

// ---- the engine quantizer without per-element division -----------------------------
// d16 = fp16(amax/127) (1 if not amax > 0) by the hardware conversion v_cvt_f16_f32
// (round to nearest even, gradual underflow, overflow to inf: the bits of
// lt_float_to_half_bits for every non-NaN input; amax/127 is never NaN), and
// q = clamp(rint(x / dq), +-127) with x / dq formed as lt_q8_quotient from one reciprocal
// per block.  The one case the quotient does not cover, dq = 0 (every |x| of the block
// below 127 * 2^-25), is x / 0 = +-inf or NaN: +-127 or 0.  Bit-identical to
// lt_q8_scale_bits + lt_q8_quant1.
__device__ __forceinline__ uint16_t lt_f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

struct QScale {
  uint16_t h;   // fp16 scale bits
  float dq;     // the scale as fp32
  float r;      // RN(1 / dq)
};

__device__ __forceinline__ QScale q8_scale(float amax) {
  QScale s;
  s.h = lt_f2h(amax > 0.0f ? amax / 127.0f : 1.0f);
  s.dq = lt_h2f(s.h);
  s.r = 1.0f / s.dq;
  return s;
}

__device__ __forceinline__ int q8_quant_zero_scale(float x) { return x > 0.0f ? 127 : (x < 0.0f ? -127 : 0); }

__device__ __forceinline__ int q8_quant(float x, const QScale& s) {
  int q = lt_q8_round_clamp(lt_q8_quotient(x, s.dq, s.r));
  if (__builtin_expect(s.h == 0, 0)) q = q8_quant_zero_scale(x);
  return q;
}

// quant_block_halfwave with the DPP max and the division-free quantizer.
__device__ __forceinline__ void quant_block_hw(float v, int lane, int8_t* xq_blk, uint16_t* xd_slot) {
  const QScale s = q8_scale(halfwave_max(fabsf(v)));
  if (lane == 0) *xd_slot = s.h;
  xq_blk[lane] = (int8_t)q8_quant(v, s);
}

// Maximum over the 8 lanes 8g .. 8g+7 (half of a DPP row): order-free.
__device__ __forceinline__ float group8_max(float a) {
  a = fmaxf(a, dpp_f<0xB1>(a));   // lane ^ 1
  a = fmaxf(a, dpp_f<0x4E>(a));   // lane ^ 2
  a = fmaxf(a, dpp_f<0x141>(a));  // mirror within 8: the two quads combine
  return a;
}

// One 32-element block held 4 consecutive elements per lane on 8 consecutive lanes (lane
// j = lane & 7 holds elements 4j .. 4j+3): returns the block's scale and this lane's four
// quants packed little-endian (element 4j+i in byte i).
__device__ __forceinline__ uint32_t quant4(float x0, float x1, float x2, float x3, QScale& s) {
  const float a = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
  s = q8_scale(group8_max(a));
  auto pack = [](int q0, int q1, int q2, int q3) {
    return ((uint32_t)q0 & 0xFFu) | (((uint32_t)q1 & 0xFFu) << 8) | (((uint32_t)q2 & 0xFFu) << 16) |
           ((uint32_t)q3 << 24);
  };
  uint32_t p = pack(lt_q8_round_clamp(lt_q8_quotient(x0, s.dq, s.r)), lt_q8_round_clamp(lt_q8_quotient(x1, s.dq, s.r)),
                    lt_q8_round_clamp(lt_q8_quotient(x2, s.dq, s.r)), lt_q8_round_clamp(lt_q8_quotient(x3, s.dq, s.r)));
  if (__builtin_expect(s.h == 0, 0))   // the whole block is below 127 * 2^-25: x / 0
    p = pack(q8_quant_zero_scale(x0), q8_quant_zero_scale(x1), q8_quant_zero_scale(x2), q8_quant_zero_scale(x3));
  return p;
}

// ---- raw 34-byte block loads dotted against a phase-matched activation ---------------
// Block gi starts at byte 34*gi.  The lane loads the 9 aligned dwords covering it
// (dwordx4, dwordx4, dword) from the 4-aligned base and leaves them as they are:
//   even gi: w0 = (d_lo, d_hi, q0, q1), w1..w7 = q2..q29 in fours, w8 = (q30, q31, *, *)
//   odd gi:  w0 = (*, *, d_lo, d_hi),   w1..w8 = q0..q31 in fours.
// The activation record of each block therefore exists in two phases (ActRec), and the
// 9 v_dot4_i32_i8 with the matching phase give exactly the block's isum: the bytes that
// are not quants meet zeros.
struct RawBlock {
  uint32_t w[9];
};

// The block at byte offset off (off = 34*gi; matrices are below 4 GiB, so offsets are
// 32-bit): odd blocks are exactly those with off % 4 == 2.  All three loads are
// unconditional (so the compiler's load counters stay exact and the loads pipeline).  For
// the matrix's final block, when even, the 9th dword reaches 2 bytes past the last block:
// that dword starts at a 4-aligned address inside the allocation, so it lies in the same
// mapped page, and its 2 extra bytes meet zero activations in the dot.
__device__ __forceinline__ void load_q8_raw(const uint8_t* __restrict__ W, uint32_t off, RawBlock& r) {
  const uint32_t* p = (const uint32_t*)(W + (off & ~3u));
  const u32x4_a4 v0 = *(const u32x4_a4*)p;
  const u32x4_a4 v1 = *(const u32x4_a4*)(p + 4);
  r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
  r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
  r.w[8] = p[8];
}

// Per-block activation record in LDS, kRecDwords = 25 dwords: phase E (even blocks) at
// dwords 0..8 with the scale xd (as fp32) at dword 9; phase O (odd blocks) at dwords
// 10..18, xd again at 19.
//   E_j = bytes (x[4j-2], x[4j-1], x[4j], x[4j+1]),  O_0 = 0,  O_j = (x[4j-4] .. x[4j-1]),
// with x outside 0..31 read as 0.  Lane L reads the record of block L (+32k): the odd
// stride puts the 32 lanes of a half-wave on 32 distinct LDS banks (25L + 10*(L&1) never
// collides mod 32 or mod 64), so the activation reads are conflict-free.
constexpr int kRecDwords = 25;
constexpr int kRecPhase = 10;

__device__ __forceinline__ float fold_raw(const RawBlock& r, bool odd, const uint32_t* rec, float acc) {
  const uint32_t* a = rec + (odd ? kRecPhase : 0);
  int s = 0;
#pragma unroll
  for (int j = 0; j < 9; j++) s = __builtin_amdgcn_sdot4((int)r.w[j], (int)a[j], s, false);
  const float xdv = __builtin_bit_cast(float, a[9]);
  const uint16_t d16 = (uint16_t)(odd ? (r.w[0] >> 16) : (r.w[0] & 0xFFFFu));
  return fmaf(lt_h2f(d16) * xdv, (float)s, acc);
}

// fold_raw in two steps, so a caller can have every record read in flight before the first
// dot: rec_regs copies the 10 dwords of the block's phase into registers, fold_regs is
// fold_raw's arithmetic on them (the same 9 v_dot4_i32_i8, scale product and fma).
__device__ __forceinline__ void rec_regs(const uint32_t* rec, bool odd, uint32_t (&a)[10]) {
  const uint32_t* p = rec + (odd ? kRecPhase : 0);
#pragma unroll
  for (int j = 0; j < 10; j++) a[j] = p[j];
}
__device__ __forceinline__ float fold_regs(const RawBlock& r, bool odd, const uint32_t (&a)[10], float acc) {
  int s = 0;
#pragma unroll
  for (int j = 0; j < 9; j++) s = __builtin_amdgcn_sdot4((int)r.w[j], (int)a[j], s, false);
  const float xdv = __builtin_bit_cast(float, a[9]);
  const uint16_t d16 = (uint16_t)(odd ? (r.w[0] >> 16) : (r.w[0] & 0xFFFFu));
  return fmaf(lt_h2f(d16) * xdv, (float)s, acc);
}

// Planar Q8_0 layout (K % 32 == 0): the quants of item (row r, slot k) -- blocks 32k ..
// 32k+m-1 of row r, m = min(32, nb - 32k) -- are 32m contiguous bytes at (r*nb + 32k)*32,
// first the leading 16 quants of each of the m blocks (16 bytes per block, in block order),
// then their trailing 16; the fp16 scales follow the whole quant plane as [N][nb].  With
// K % 1024 == 0 every item is 1024 bytes at (r*nk + k)*1024.  A half-wave reads a whole item
// with two coalesced loads of 16m bytes and one of 2m, and every cache line of a full item
// is consumed by a single load instruction.  Lane L
// holds block 32k+L as w[0..7] = quants 0..31 in fours and w[8] = the scale bits.  Against
// the activation record's phase O (dwords kRecPhase+1 .. kRecPhase+8 hold quants 0..31,
// kRecPhase+9 the scale) the 8 v_dot4_i32_i8 give the same exact isum as fold_raw's 9, and
// the fma is the same.
__device__ __forceinline__ float fold_planar(const RawBlock& r, const uint32_t* rec, float acc) {
  const uint32_t* a = rec + kRecPhase + 1;
  int s = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) s = __builtin_amdgcn_sdot4((int)r.w[j], (int)a[j], s, false);
  const float xdv = __builtin_bit_cast(float, a[8]);
  return fmaf(lt_h2f((uint16_t)(r.w[8] & 0xFFFFu)) * xdv, (float)s, acc);
}

// Build the activation records of nb blocks from the staged quants sxq[32*nb] (int8) and
// scales sxd[nb] (fp16 bits); called by every thread of the workgroup.
// Write a block quantized by quant4 into its record: lane j of the block's 8-lane group
// holds quants 4j .. 4j+3 in p.  Phase O (dwords kRecPhase+1 ..) takes p as it is; phase E
// is shifted by 2 bytes, so its dword j joins the previous lane's upper two quants (DPP
// row_shr:1) with this lane's lower two; its dword 0 starts with two zero bytes and dword 8
// holds the last two quants.  Every lane executes the DPP; `write` selects the lanes whose
// block exists.
__device__ __forceinline__ void q4_to_rec(uint32_t p, float dq, int j, bool write, uint32_t* rec) {
  const uint32_t prev = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)p, 0x111, 0xF, 0xF, true);
  const uint32_t e = j == 0 ? (p << 16) : __builtin_amdgcn_alignbyte(p, prev, 2);
  if (write) {
    rec[j] = e;
    rec[kRecPhase + 1 + j] = p;
    if (j == 7) rec[8] = p >> 16;
    if (j == 0) {
      const uint32_t d = __builtin_bit_cast(uint32_t, dq);
      rec[9] = d;
      rec[kRecPhase] = 0u;
      rec[kRecPhase + 9] = d;
    }
  }
}

__device__ __forceinline__ void build_act_records(const int8_t* sxq, const uint16_t* sxd, int nb,
                                                  uint32_t* rec, int tid, int nthreads) {
  const uint32_t* X = (const uint32_t*)sxq;   // 8 dwords per block
  for (int i = tid; i < nb * 10; i += nthreads) {
    const int b = i / 10;
    const int j = i - b * 10;
    uint32_t* r = rec + b * kRecDwords;
    if (j == 9) {
      const uint32_t xd = __builtin_bit_cast(uint32_t, lt_h2f(sxd[b]));
      r[9] = xd;
      r[kRecPhase + 9] = xd;
    } else {
      const uint32_t lo = j > 0 ? X[b * 8 + j - 1] : 0u;
      const uint32_t hi = j < 8 ? X[b * 8 + j] : 0u;
      r[j] = __builtin_amdgcn_perm(hi, lo, 0x05040302u);
      r[kRecPhase + j] = lo;
    }
  }
}

}  // namespace lt
