// lt_prefill.hip -- the batched (prefill) path: a tiled int8-MFMA Q8_0 GEMM and the
// batched RoPE / KV append that go with it.
//
// The reference prefills one token at a time through the decode GEMV and requires any
// batched prefill to stay "device-uniform": every element bit-identical to the
// single-token path (bpd/lib/dev_residency.py:1338-1356).  The GEMM here meets that
// exactly.  For a 32-row x 32-token tile, one v_mfma_i32_32x32x32_i8 per Q8_0 block gives
// the exact int32 block dots isum[n][t]; the fp32 arithmetic then replays the GEMV's
// canonical order (q8_0_from_facts.pl:466-516) per element:
//   leaf L (0..31) = fma-fold over blocks L, L+32, ... of wd*xd*isum (one rounding each),
//   result = the 5-level pairwise tree over the 32 leaves.
// The leaves are visited in bit-reversed order, which is the post-order of that tree, so a
// stack of 5 partial sums per element replays the pairing with every addition in place.
#include "lt_q8_device.h"

#include <cstdlib>
#include <type_traits>

namespace {

using namespace lt;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kGemmWaves = 4;                  // waves per workgroup: 4 x 32 tokens share 32 rows
constexpr int kGemmTokens = 32 * kGemmWaves;   // tokens per workgroup
constexpr int kDepth = 4;                      // blocks in flight per wave
constexpr uint32_t kNoBlk = 0x80000000u;       // out-of-range buffer offset: reads zeros

// GE_ROPE (leaf-split kernel only): the q|k|v rows of the next token of each of T sequences
// in the rope-pair order of lt_q8_tiles_rope, + bias, then RoPE and the KV append
enum GemmEpi { GE_STORE = 0, GE_BIAS = 1, GE_RESID = 2, GE_SILU = 3, GE_ROPE = 4 };

struct GemmParams {
  const uint8_t* W;      // Q8_0 blocks [N][K/32]; tiled: [ceil(N/32)][K/32][32 rows][34 B]
  const int8_t* Xq;      // [T][K]; tiled: block-major [K/32][T][32]
  const uint16_t* Xd;    // [T][K/32] fp16 bits; tiled: [K/32][T]
  const float* bias;     // [N] (GE_BIAS)
  const float* resid;    // [T][N] (GE_RESID)
  float* Y;              // [T][N], or [T][N/2] for GE_SILU
  int8_t* Yq;            // the leaf-split SiLU + quant variant: block-major quants of Y, [N/64][T][32]
  uint16_t* Yd;          //   and their scales [N/64][T]
  int T, N, K;
  int nrt, ntt;          // row tiles (32 rows), token tiles (kGemmTokens)
  // GE_ROPE: row t is sequence t at position len[t]; its cache rows at kc / vc + t*maxt*nkv*hd
  // elements (fp16 when f16)
  const int* len;
  const float* freqs;    // [hd/2]
  void* kc;
  void* vc;
  int nh, nkv, hd, maxt, f16;
};

// C layout of v_mfma_i32_32x32x32_i8: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4,
// column l%32.  A lane l supplies row l%32, B lane l column l%32, each the 16 bytes
// 16*(l/32) .. +16 of the block (the same half of k for A and B).
__device__ __forceinline__ int c_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// The tile-major copy's 1088-byte tile block: the 32 rows' quants, 32 bytes each (row r at
// 32r), then the 32 rows' fp16 scales (row r at kTileQ + 2r).
constexpr uint32_t kTileQ = 32u * 32u;
constexpr uint32_t kTileBlk = kTileQ + 64u;
static_assert(kTileBlk == 32u * kBlockBytes, "a tile block holds 32 Q8_0 blocks");

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// kTiled: the weights in the tile-major copy and the activations block-major (block b of
// 32 consecutive tokens is 1 KB of quants and 64 bytes of scales, each contiguous), so
// both operands of a block are coalesced, aligned loads; the arithmetic and the order are
// those of the row-major layouts.
// kSL: how the tiled kernel walks the leaves.  0: one dynamic loop over the block sequence
// (any K).  1..3: K a multiple of 2048 (an even number bpl of blocks per leaf) -- leaves in
// groups of 4 with the group's structure static: the tree's levels 0 and 1 are the
// accumulators themselves (no parking copies), the ring slot indices are static, and only the
// group's last leaf closes levels 2..4 (in LDS) with a short dynamic loop.  1: a 2-slot load
// ring (3 waves per SIMD); 2: a 4-slot ring with the MFMAs one block ahead of the fold (up to
// 256 registers, 2 waves per SIMD; bpl % 4 == 0 -- with bpl % 4 == 2 the allocation spills).
template <GemmEpi EPI, bool kTiled, int kSL = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kSL >= 2 ? 2 : 3))) void k_q8_gemm(GemmParams P) {
  static_assert(kSL == 0 || kTiled, "k_q8_gemm: grouped leaves use the tiled layouts");
  __shared__ float s_st[kGemmWaves][3][16 * 64];   // tree levels 2..4 of each wave's 32 x 32 tile
  const int wave = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int h = l >> 5;
  const int c = l & 31;

  // XCD-aware tile order: workgroups are dispatched round robin over the 8 XCDs, so the
  // token tiles of one row tile get ids 8 apart and share an XCD (and its L2).
  const int g = blockIdx.x;
  const int rt = (g / (8 * P.ntt)) * 8 + (g & 7);
  const int tt = (g >> 3) % P.ntt;
  if (rt >= P.nrt) return;   // uniform per workgroup
  const int n0 = rt * 32;
  const int t0 = tt * kGemmTokens + wave * 32;
  const int nb = P.K >> 5;
  // B lane: token t0 + c (clamped; results of clamped tokens are discarded)
  const int btok = t0 + c < P.T ? t0 + c : P.T - 1;

  // Operands of one block, raw as loaded (so the loads stay in flight until the block is
  // folded).  Every load is unconditional: past the last block they read zeros.
  //   row-major: the A lane's 5 dwords around its 16 quant bytes (a block's quants begin 2
  //     bytes in), the dword holding its row's scale, the B lane's 16 quant bytes and the
  //     dword holding its token's scale;
  //   tiled: the A and B lanes' 16 quant bytes and (lanes of the first k half) the row's
  //     and the token's scale as 16-bit loads; the block's part of each offset is the
  //     wave-uniform soffset, the lane's part a constant.
  struct Ops {
    v4i w03, bq;
    uint32_t w4, wdw, xdw;
  };
  // row-major addressing: block b of the A lane's row (clamped) at row_off + 34b, of the
  // B lane's token at xrow_off + 32b, its scale at xd_off + 2b
  const int arow = n0 + c < P.N ? n0 + c : P.N - 1;
  const uint32_t row_off = (uint32_t)arow * (uint32_t)nb * (uint32_t)kBlockBytes;
  const uint32_t xrow_off = (uint32_t)btok * (uint32_t)P.K + 16u * (uint32_t)h;
  const uint32_t xd_off = (uint32_t)btok * (uint32_t)nb * 2u;
  // the 5th dword can lie past the matrix: buffer loads bound it (out-of-range dwords read
  // as zero)
  const uint32_t mat_bytes = kTiled ? (uint32_t)nb * kTileBlk : (uint32_t)P.N * (uint32_t)nb * (uint32_t)kBlockBytes;
  // tiled: the resources cover this row tile's blocks; lanes of the second k half aim their
  // scale loads out of range (the scale MFMA's k = 4..7 terms must be zero)
  const uint8_t* wbase = kTiled ? P.W + (size_t)rt * (size_t)nb * kTileBlk : P.W;
  const uint32_t aq_v = (uint32_t)c * 32u + 16u * (uint32_t)h;
  const uint32_t ad_v = h ? kNoBlk : kTileQ + 2u * (uint32_t)c;
  const uint32_t bq_v = (uint32_t)btok * 32u + 16u * (uint32_t)h;
  const uint32_t bd_v = h ? kNoBlk : (uint32_t)btok * 2u;
  const uint32_t x_bytes = (uint32_t)P.T * (uint32_t)P.K;
  const uint32_t xd_bytes = (uint32_t)P.T * (uint32_t)nb * 2u;
  // scale loads in chain pairs (grouped walks): lanes of the second k half fetch the scales
  // of the next block of the leaf's chain (32 blocks on) instead of reading zeros
  const uint32_t ad2_v = kTileQ + 2u * (uint32_t)c + (h ? 32u * kTileBlk : 0u);
  const uint32_t bd2_v = (uint32_t)btok * 2u + (h ? 64u * (uint32_t)P.T : 0u);
  // smode: 0 the block's own scales (second k half zero), 1 the chain pair's, 2 none
  auto load_ops = [&](int b, bool real, Ops& o, int smode = 0) {
    if constexpr (kTiled) {
      // past the last block: resources of no records (every load reads zeros)
      const __amdgpu_buffer_rsrc_t wr =
          __builtin_amdgcn_make_buffer_rsrc((void*)wbase, 0, real ? (int)mat_bytes : 0, 0x00020000);
      const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)P.Xq, 0, real ? (int)x_bytes : 0, 0x00020000);
      const __amdgpu_buffer_rsrc_t xdr =
          __builtin_amdgcn_make_buffer_rsrc((void*)P.Xd, 0, real ? (int)((xd_bytes + 3u) & ~3u) : 0, 0x00020000);
      const int bb = real ? b : 0;
      const int sa = (int)((uint32_t)bb * kTileBlk);
      const int sq = (int)((uint32_t)bb * (uint32_t)P.T * 32u);
      const int sd = (int)((uint32_t)bb * (uint32_t)P.T * 2u);
      o.w03 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)aq_v, sa, 0));
      if (smode != 2) o.wdw = __builtin_amdgcn_raw_buffer_load_b16(wr, (int)(smode ? ad2_v : ad_v), sa, 0);
      o.bq = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)bq_v, sq, 0));
      if (smode != 2) o.xdw = __builtin_amdgcn_raw_buffer_load_b16(xdr, (int)(smode ? bd2_v : bd_v), sd, 0);
    } else {
      const __amdgpu_buffer_rsrc_t wr =
          __builtin_amdgcn_make_buffer_rsrc((void*)P.W, 0, (int)((mat_bytes + 3u) & ~3u), 0x00020000);
      const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)P.Xq, 0, (int)x_bytes, 0x00020000);
      const __amdgpu_buffer_rsrc_t xdr =
          __builtin_amdgcn_make_buffer_rsrc((void*)P.Xd, 0, (int)((xd_bytes + 3u) & ~3u), 0x00020000);
      const uint32_t off = row_off + (uint32_t)b * kBlockBytes;
      const uint32_t base = real ? (off + 2u + 16u * (uint32_t)h) & ~3u : kNoBlk;
      o.w03 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)base, 0, 0));
      o.w4 = __builtin_amdgcn_raw_buffer_load_b32(wr, (int)(base + 16u), 0, 0);
      o.wdw = __builtin_amdgcn_raw_buffer_load_b32(wr, real ? (int)(off & ~3u) : (int)kNoBlk, 0, 0);
      o.bq = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, real ? (int)(xrow_off + 32u * (uint32_t)b) : (int)kNoBlk, 0, 0));
      o.xdw = __builtin_amdgcn_raw_buffer_load_b32(
          xdr, real ? (int)((xd_off + 2u * (uint32_t)b) & ~3u) : (int)kNoBlk, 0, 0);
    }
  };
  // fold block b into the leaf's 16 running sums: exact MFMA dots isum, the exact scale
  // products wd*xd as an MFMA outer product (A lane: its row's wd in k = 0, zero in the
  // other k; B lane: its token's xd in k = 0; a product of two fp16 values is exact in fp32
  // and the zero terms add nothing), then v = fma(wd*xd, isum, v) per element
  auto fold_ops = [&](const Ops& o, int b, float (&v)[16]) {
    const v16i z = {};
    const v16f zf = {};
    v16i isum;
    v16f sc;
    if constexpr (kTiled) {
      isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.w03, o.bq, z, 0, 0, 0);
      // the 16-bit loads zero-extend: {scale, 0, 0, 0} as fp16 (zeros in the other k half)
      const u32x2 aw = {o.wdw, 0u}, bw = {o.xdw, 0u};
      sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(h4, aw), __builtin_bit_cast(h4, bw), zf, 0, 0, 0);
    } else {
      const uint32_t off = row_off + (uint32_t)b * kBlockBytes;
      const uint32_t sh = (off + 2u + 16u * (uint32_t)h) & 3u;   // 0 or 2
      v4i a;
      a.x = (int)__builtin_amdgcn_alignbyte((uint32_t)o.w03.y, (uint32_t)o.w03.x, sh);
      a.y = (int)__builtin_amdgcn_alignbyte((uint32_t)o.w03.z, (uint32_t)o.w03.y, sh);
      a.z = (int)__builtin_amdgcn_alignbyte((uint32_t)o.w03.w, (uint32_t)o.w03.z, sh);
      a.w = (int)__builtin_amdgcn_alignbyte(o.w4, (uint32_t)o.w03.w, sh);
      const float wd = lt_h2f((uint16_t)((off & 2u) ? (o.wdw >> 16) : (o.wdw & 0xFFFFu)));
      const float xd = lt_h2f((uint16_t)(((xd_off + 2u * (uint32_t)b) & 2u) ? (o.xdw >> 16) : (o.xdw & 0xFFFFu)));
      isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, o.bq, z, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(h == 0 ? wd : 0.0f, h == 0 ? xd : 0.0f, zf, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; r++) v[r] = fmaf(sc[r], (float)isum[r], v[r]);
  };

  // The blocks in post-order: leaf i (0..31) is lane L = bitrev5(i) and holds blocks
  // L, L+32, ... < nb (leaves with L >= nb hold none).  A producer cursor walks that
  // sequence kDepth blocks ahead of the consumer, refilling a ring of prefetched operands.
  auto leaf_lane = [](int i) { return (int)(__builtin_bitreverse32((uint32_t)i) >> 27); };
  int pi = 0, pb = 0;   // producer: leaf, next block (pb = -1: done)
  auto produce = [&](Ops& o) {
    load_ops(pb >= 0 ? pb : 0, pb >= 0, o);
    if (pb >= 0) {
      pb += 32;
      while (pb >= nb) {           // next non-empty leaf
        if (++pi == 32) { pb = -1; break; }
        pb = leaf_lane(pi);
      }
    }
  };
  float v[16];   // the tile's row values once every leaf is folded
  if constexpr (kSL == 0) {
  Ops ring[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; d++) produce(ring[d]);

  // pending partial sums of the tree: levels 0 and 1 in registers; levels 2..4, parked at
  // most once per 4 leaves, in LDS
  float st[2][16];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    v[r] = 0.0f;
  }
#pragma unroll
  for (int l2 = 0; l2 < 2; l2++)
#pragma unroll
    for (int r = 0; r < 16; r++) st[l2][r] = 0.0f;
  // combine leaf i into the stack: it closes every level whose bit is set in i (its
  // trailing ones: left subtree (the parked sum) + right subtree v, the reference tree's
  // pairing, level by level from the bottom) and parks the sum at the first clear level.
  // i is uniform, so these are scalar branches around static register indices.
  auto close_leaf = [&](int i) {
    const int t1 = __builtin_ctz(~(unsigned)i);   // trailing ones, 0..5
#pragma unroll
    for (int lvl = 0; lvl < 2; lvl++) {
      if (lvl < t1) {
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = st[lvl][r] + v[r];
      }
    }
#pragma unroll
    for (int lvl = 2; lvl < 5; lvl++) {
      if (lvl < t1) {
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = s_st[wave][lvl - 2][r * 64 + l] + v[r];
      }
    }
    switch (t1) {
      case 0:
#pragma unroll
        for (int r = 0; r < 16; r++) st[0][r] = v[r];
        break;
      case 1:
#pragma unroll
        for (int r = 0; r < 16; r++) st[1][r] = v[r];
        break;
      case 2:
      case 3:
      case 4:
#pragma unroll
        for (int r = 0; r < 16; r++) s_st[wave][t1 - 2][r * 64 + l] = v[r];
        break;
      default:   // i == 31: every level closed, v is the row value (kept in v)
        break;
    }
  };
  int ci = 0, cb = 0;   // consumer: leaf, block
  // tiled: the MFMAs run one block ahead of the fold (two result sets, A and B, alternate
  // with the slot's parity, so nothing is copied), and a fold never waits for its own MFMAs
  static_assert(kDepth % 2 == 0, "k_q8_gemm: the A/B result sets alternate over an even ring");
  v16i isA, isB;
  v16f scA, scB;
  auto mfma_tiled = [&](const Ops& o, v16i& isum, v16f& sc) {
    const v16i z = {};
    const v16f zf = {};
    isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.w03, o.bq, z, 0, 0, 0);
    // the 16-bit loads zero-extend: {scale, 0, 0, 0} as fp16 (zeros in the other k half)
    const u32x2 aw = {o.wdw, 0u}, bw = {o.xdw, 0u};
    sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(h4, aw), __builtin_bit_cast(h4, bw), zf, 0, 0, 0);
  };
  if constexpr (kTiled) mfma_tiled(ring[0], isA, scA);
  for (int s0 = 0; s0 < nb; s0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; d++) {
      // every slot folds and refills (loads on all paths keep the load counters exact):
      // past the last block a slot holds zeros, and v + 0*0 leaves v unchanged
      if constexpr (kTiled) {
        // slot d + 1 holds the next block (slot 0 was refilled with it at d = 0)
        if (d % 2 == 0) {
          mfma_tiled(ring[(d + 1) % kDepth], isB, scB);
#pragma unroll
          for (int r = 0; r < 16; r++) v[r] = fmaf(scA[r], (float)isA[r], v[r]);
        } else {
          mfma_tiled(ring[(d + 1) % kDepth], isA, scA);
#pragma unroll
          for (int r = 0; r < 16; r++) v[r] = fmaf(scB[r], (float)isB[r], v[r]);
        }
      } else {
        fold_ops(ring[d], cb, v);
      }
      produce(ring[d]);
      if (s0 + d < nb) {
        cb += 32;
        if (cb >= nb) {            // leaf ci is complete; close it and any empty leaves after it
          close_leaf(ci);
          while (++ci < 32 && (cb = leaf_lane(ci)) >= nb) {
#pragma unroll
            for (int r = 0; r < 16; r++) v[r] = 0.0f;
            close_leaf(ci);
          }
          if (ci < 32) {           // after leaf 31, v holds the row values
#pragma unroll
            for (int r = 0; r < 16; r++) v[r] = 0.0f;
          }
        }
      }
    }
  }

  } else {
    // groups of 4 leaves (post-order leaf i = 4g + j holds blocks bitrev5(i) + 32k, k < bpl):
    //   j = 0 -> va (parked at level 0 as it is);  j = 1 -> vb, closes level 0 (va + vb) and
    //   parks at level 1;  j = 2 -> va (level 0);  j = 3 -> vc, closes levels 0 (va + vc),
    //   1 (vb + vc) and 2 .. t1-1 from LDS, parks at t1 = 2 + ctz(~g) (leaf 31: the row value)
    // The block at sequence position p lives in ring slot p % kRD (a leaf starts at position
    // i·bpl, slot (i·bpl) % kRD); a slot is refilled with position p + kRD once its MFMAs are
    // issued.  With kRD = 4 the MFMAs of position p + 1 run before position p's fold (result
    // sets A / B by the parity of p).
    // The scales come in chain pairs: the slot of an even chain position k (bpl and kRD are
    // even, so slot parity is chain parity) loads the rows' and tokens' scales of blocks k
    // (lanes h = 0, the scale MFMA's k-slot 0) and k + 1 (lanes h = 1, k-slot 4) -- one load
    // each for two blocks; block k's scale MFMA keeps the h = 0 halves and k + 1's the h = 1
    // halves, the other half masked to zero, so each is the single product wd * xd.
    constexpr int kRD = kSL == 1 ? 2 : 4;
    const int bpl = nb >> 5;
    const uint32_t m_lo = h ? 0u : 0xFFFFFFFFu, m_hi = ~m_lo;
    Ops ring[kRD];
#pragma unroll
    for (int d = 0; d < kRD; d++) load_ops(32 * d, true, ring[d], (d & 1) ? 2 : 1);   // leaf 0's first kRD blocks
    const v16i z = {};
    const v16f zf = {};
    // block o's MFMAs with the scale pair's dwords sw (rows) and sx (tokens) masked by m
    auto mfma_t = [&](const Ops& o, uint32_t sw, uint32_t sx, uint32_t m, v16i& isum, v16f& sc) {
      isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.w03, o.bq, z, 0, 0, 0);
      const u32x2 aw = {sw & m, 0u}, bw = {sx & m, 0u};
      sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(h4, aw), __builtin_bit_cast(h4, bw), zf, 0, 0, 0);
    };
    v16i isA, isB;
    v16f scA, scB;
    uint32_t pw = 0u, px = 0u;   // kRD == 2: the pair's scales for the odd slot
    if constexpr (kRD == 4) mfma_t(ring[0], ring[0].wdw, ring[0].xdw, m_lo, isA, scA);
    // one block from ring slot sl, which is then refilled with the block kRD positions on; a
    // leaf's first block (kFirst) folds into +0.0 as an fma operand, so no register is zeroed
    auto step = [&](auto S, auto F, float (&acc)[16], int rb, bool rreal) {
      constexpr int sl = decltype(S)::value;
      constexpr bool kFirst = decltype(F)::value;
      auto fold = [&](const v16f& sc, const v16i& isum) {
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = fmaf(sc[r], (float)isum[r], kFirst ? 0.0f : acc[r]);
      };
      if constexpr (kRD == 2) {
        v16i isum;
        v16f sc;
        if constexpr (sl == 0) {
          pw = ring[0].wdw;
          px = ring[0].xdw;
          mfma_t(ring[0], pw, px, m_lo, isum, sc);
          load_ops(rb, rreal, ring[0], 1);
        } else {
          mfma_t(ring[1], pw, px, m_hi, isum, sc);
          load_ops(rb, rreal, ring[1], 2);
        }
        fold(sc, isum);
      } else if constexpr ((sl & 1) == 0) {
        // the odd block sl + 1 from this slot's pair, before the slot is refilled
        mfma_t(ring[(sl + 1) & 3], ring[sl].wdw, ring[sl].xdw, m_hi, isB, scB);
        load_ops(rb, rreal, ring[sl], 1);
        fold(scA, isA);
      } else {
        mfma_t(ring[(sl + 1) & 3], ring[(sl + 1) & 3].wdw, ring[(sl + 1) & 3].xdw, m_lo, isA, scA);
        load_ops(rb, rreal, ring[sl], 2);
        fold(scB, isB);
      }
    };
    auto leaf = [&](auto J, int i, float (&acc)[16]) {
      constexpr int j = decltype(J)::value;
      static_assert(j >= 0 && j < 4, "k_q8_gemm: leaf within a group");   // (i·bpl) % kRD == 0
      const int L = leaf_lane(i);
      const int Ln = i < 31 ? leaf_lane(i + 1) : 0;
      // position (i, k) + kRD: the same leaf or the next one (past leaf 31: zeros)
      using first = std::true_type;
      using next = std::false_type;
      auto ref = [&](int k, auto S, auto F) {
        const bool same = k + kRD < bpl;
        step(S, F, acc, same ? L + 32 * (k + kRD) : Ln + 32 * (k + kRD - bpl), same || i < 31);
      };
      // bpl >= kRD: the first kRD blocks are peeled (the leaf's first block starts the chain)
      if constexpr (kRD == 2) {
        ref(0, std::integral_constant<int, 0>{}, first{});
        ref(1, std::integral_constant<int, 1>{}, next{});
        for (int k = 2; k < bpl; k += 2) {
          ref(k, std::integral_constant<int, 0>{}, next{});
          ref(k + 1, std::integral_constant<int, 1>{}, next{});
        }
      } else {
        ref(0, std::integral_constant<int, 0>{}, first{});
        ref(1, std::integral_constant<int, 1>{}, next{});
        ref(2, std::integral_constant<int, 2>{}, next{});
        ref(3, std::integral_constant<int, 3>{}, next{});
        for (int k = 4; k + 4 <= bpl; k += 4) {
          ref(k, std::integral_constant<int, 0>{}, next{});
          ref(k + 1, std::integral_constant<int, 1>{}, next{});
          ref(k + 2, std::integral_constant<int, 2>{}, next{});
          ref(k + 3, std::integral_constant<int, 3>{}, next{});
        }
      }
    };
    float va[16], vb[16], vc[16];
    for (int g = 0; g < 8; g++) {
      leaf(std::integral_constant<int, 0>{}, 4 * g, va);
      leaf(std::integral_constant<int, 1>{}, 4 * g + 1, vb);
#pragma unroll
      for (int r = 0; r < 16; r++) vb[r] = va[r] + vb[r];
      leaf(std::integral_constant<int, 2>{}, 4 * g + 2, va);
      leaf(std::integral_constant<int, 3>{}, 4 * g + 3, vc);
#pragma unroll
      for (int r = 0; r < 16; r++) vc[r] = va[r] + vc[r];
#pragma unroll
      for (int r = 0; r < 16; r++) vc[r] = vb[r] + vc[r];
      const int t1 = 2 + __builtin_ctz(~(unsigned)g);   // 2 .. 5
      for (int lvl = 2; lvl < t1; lvl++) {
#pragma unroll
        for (int r = 0; r < 16; r++) vc[r] = s_st[wave][lvl - 2][r * 64 + l] + vc[r];
      }
      if (t1 < 5) {
#pragma unroll
        for (int r = 0; r < 16; r++) s_st[wave][t1 - 2][r * 64 + l] = vc[r];
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) v[r] = vc[r];
  }

  // the wave's tile through its own (now free) tree level-2 buffer, then stores along the
  // rows: each token's 32 rows (16 SiLU outputs) are one contiguous run of Y.  Element (token
  // q, row e) sits at 32q + (e ^ q): both the column writes and the row reads are free of
  // bank conflicts.
  float* tile = s_st[wave][0];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int e = c_row(r, h);
    tile[32 * c + (e ^ c)] = v[r];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if constexpr (EPI == GE_SILU) {
    // output j of token q is rows 2j (gate) and 2j+1 (up); 4 tokens per pass
    const int F = P.N >> 1;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int q = 4 * k + (l >> 4), j = l & 15;
      const int t = t0 + q, n = n0 + 2 * j;         // N is even: n < N means n + 1 < N
      if (t < P.T && n < P.N)
        P.Y[(size_t)t * F + (n >> 1)] = lt_silu_mul(tile[32 * q + ((2 * j) ^ q)], tile[32 * q + ((2 * j + 1) ^ q)]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int q = 2 * k + h, t = t0 + q, n = n0 + c;
      if (t < P.T && n < P.N) {
        float o = tile[32 * q + (c ^ q)];
        if constexpr (EPI == GE_BIAS) o = o + P.bias[n];
        if constexpr (EPI == GE_RESID) o = o + P.resid[(size_t)t * P.N + n];
        P.Y[(size_t)t * P.N + n] = o;
      }
    }
  }
}

// Leaf-split tiled GEMM, for launches with few tiles (the batched decode step: tens of
// tokens).  A workgroup of kW waves (4, 8 or 16) takes one 32-row x 32-token tile, so a launch
// has kW times the waves of a one-wave-per-tile walk, and each wave folds 32/kW of the
// tile's leaves.  The GEMV's tree (halfwave_tree_dpp) pairs lanes l and l+16, then +8, +4,
// +2, +1, so the leaves L = w, w+kW, ..., w+32-kW form the subtree of its partial at level
// log2(32/kW) -- with kW = 4 the 8 leaves of d_w:
//   b(L) = a(L) + a(L+16),  c(L) = b(L) + b(L+8),  d_w = c(w) + c(w+4);
// wave w folds its leaves (the fma chains over blocks L, L+32, ... as in k_q8_gemm) in that
// subtree's post-order -- L = w + kW * bitrev(i) (kW = 4: w, w+16, w+8, w+24, w+4, w+20,
// w+12, w+28) -- closing each pair in place, and wave 0 adds the remaining levels from LDS,
// the tree's pairings over the waves' partials (kW = 4: (d0 + d2) + (d1 + d3); kW = 16: the
// same pairs level by level on every wave).  Every element is the single-token GEMV's, bit
// for bit.  The combined tile then goes through LDS to an epilogue over every thread.
//
// kQ (SiLU gate|up only): a workgroup of two such halves takes two adjacent row tiles -- 64
// interleaved rows, the gate/up pairs of one 32-element block of the SiLU output -- and, after
// each half's tree, quantizes every token's block (the activation quantizer, q8_scale /
// q8_quant, one half-wave per token) into block-major Yq / Yd, the down projection's input:
// bit-identical to the SiLU output quantized by lt_quant_q8_bm, with no fp32 round trip.
//
// kP > 0 (K at most kP * 1024): every leaf is padded to kP blocks -- the blocks past the
// matrix read zeros through resources of no records, and fma(0, 0, a) = a for the leaf
// values, which are never -0 -- so the wave's kNL * kP slots, the ring over them and the
// leaf closes are all fixed at compile time: no per-slot branches, and the tree's pairings
// are register additions the compiler schedules freely.  kP = 0: the leaf lengths are read
// at run time (any K).
template <GemmEpi EPI, int kW, bool kQ = false, int kP = 0>
__global__ __launch_bounds__(64 * kW * (kQ ? 2 : 1)) void k_q8_gemm_ls(GemmParams P) {
  static_assert(kW == 4 || kW == 8 || kW == 16, "k_q8_gemm_ls: 4, 8 or 16 waves per tile");
  static_assert(!(kQ && kW == 16), "k_q8_gemm_ls: the quantizing variant has 8 waves per half");
  static_assert(!kQ || (EPI == GE_SILU && kW == 4), "k_q8_gemm_ls: the quantizing variant is SiLU, 4 waves per tile");
  constexpr int kNL = 32 / kW;                      // leaves per wave
  __shared__ float s_d[kQ ? 2 : 1][kW - 1][16 * 64];   // the partials of waves 1 .. kW-1 (per half)
  // the wave index through readfirstlane: everything derived from it (the leaves, the block
  // offsets, the buffer resources) is then wave-uniform, and no buffer load is a waterfall
  const int wall = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = kQ ? wall / kW : 0;
  const int wave = kQ ? wall - half * kW : wall;
  const int l = threadIdx.x & 63;
  const int h = l >> 5;
  const int c = l & 31;
  // XCD-aware tile order, as k_q8_gemm's: the token tiles of one row tile share an XCD (kQ:
  // of one pair of row tiles)
  const int g = blockIdx.x;
  const int rtg = (g / (8 * P.ntt)) * 8 + (g & 7);
  const int tt = (g >> 3) % P.ntt;
  if (kQ ? 2 * rtg >= P.nrt : rtg >= P.nrt) return;   // uniform per workgroup
  const int rt = kQ ? 2 * rtg + half : rtg;
  const int n0 = rt * 32;
  const int t0 = tt * 32;
  const int nb = P.K >> 5;
  const int btok = t0 + c < P.T ? t0 + c : P.T - 1;

  struct Ops {
    v4i w03, bq;
    uint32_t wdw, xdw;
  };
  const uint8_t* wbase = P.W + (size_t)rt * (size_t)nb * kTileBlk;
  const uint32_t mat_bytes = (uint32_t)nb * kTileBlk;
  const uint32_t aq_v = (uint32_t)c * 32u + 16u * (uint32_t)h;
  const uint32_t ad_v = h ? kNoBlk : kTileQ + 2u * (uint32_t)c;
  const uint32_t bq_v = (uint32_t)btok * 32u + 16u * (uint32_t)h;
  const uint32_t bd_v = h ? kNoBlk : (uint32_t)btok * 2u;
  const uint32_t x_bytes = (uint32_t)P.T * (uint32_t)P.K;
  const uint32_t xd_bytes = (uint32_t)P.T * (uint32_t)nb * 2u;
  // block b's operands (b < 0: resources of no records, every load reads zeros)
  auto load_ops = [&](int b, Ops& o) {
    const bool real = b >= 0;
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void*)wbase, 0, real ? (int)mat_bytes : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)P.Xq, 0, real ? (int)x_bytes : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t xdr =
        __builtin_amdgcn_make_buffer_rsrc((void*)P.Xd, 0, real ? (int)((xd_bytes + 3u) & ~3u) : 0, 0x00020000);
    const int bb = real ? b : 0;
    const int sa = (int)((uint32_t)bb * kTileBlk);
    const int sq = (int)((uint32_t)bb * (uint32_t)P.T * 32u);
    const int sd = (int)((uint32_t)bb * (uint32_t)P.T * 2u);
    o.w03 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)aq_v, sa, 0));
    o.wdw = __builtin_amdgcn_raw_buffer_load_b16(wr, (int)ad_v, sa, 0);
    o.bq = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)bq_v, sq, 0));
    o.xdw = __builtin_amdgcn_raw_buffer_load_b16(xdr, (int)bd_v, sd, 0);
  };
  // the wave's leaves in its subtree's post-order: L = wave + kW * bitrev(i) over
  // log2(kNL) bits (kW = 4: offsets 0, 16, 8, 24, 4, 20, 12, 28)
  auto leaf_of = [&](int i) {
    const int k = (int)(__builtin_bitreverse32((uint32_t)i) >> (32 - __builtin_ctz(kNL)));
    return wave + kW * k;
  };
  float a[16], s0[16], s1[16], s2[16];
#pragma unroll
  for (int r = 0; r < 16; r++) { a[r] = 0.0f; s0[r] = 0.0f; s1[r] = 0.0f; s2[r] = 0.0f; }
  // close the leaf at post-order position i (a holds its value): the subtree's pairings
  // (static register arrays in every branch: a pointer to one would put them in scratch)
  auto close_leaf = [&](int i) {
    if constexpr (kNL == 2) {
      if (i == 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) s0[r] = a[r];
      } else {
#pragma unroll
        for (int r = 0; r < 16; r++) s0[r] = s0[r] + a[r];
      }
#pragma unroll
      for (int r = 0; r < 16; r++) a[r] = 0.0f;
      return;
    }
    if constexpr (kNL == 4) {
      switch (i) {
        case 0:
#pragma unroll
          for (int r = 0; r < 16; r++) s0[r] = a[r];
          break;
        case 1:
#pragma unroll
          for (int r = 0; r < 16; r++) s0[r] = s0[r] + a[r];
          break;
        case 2:
#pragma unroll
          for (int r = 0; r < 16; r++) s1[r] = a[r];
          break;
        default:   // 3
#pragma unroll
          for (int r = 0; r < 16; r++) { s1[r] = s1[r] + a[r]; s0[r] = s0[r] + s1[r]; }
          break;
      }
#pragma unroll
      for (int r = 0; r < 16; r++) a[r] = 0.0f;
      return;
    }
    switch (i) {
      case 0:
#pragma unroll
        for (int r = 0; r < 16; r++) s0[r] = a[r];
        break;
      case 2:
      case 4:
#pragma unroll
        for (int r = 0; r < 16; r++) s1[r] = a[r];
        break;
      case 6:
#pragma unroll
        for (int r = 0; r < 16; r++) s2[r] = a[r];
        break;
      case 1:
#pragma unroll
        for (int r = 0; r < 16; r++) s0[r] = s0[r] + a[r];
        break;
      case 3:
#pragma unroll
        for (int r = 0; r < 16; r++) { s1[r] = s1[r] + a[r]; s0[r] = s0[r] + s1[r]; }
        break;
      case 5:
#pragma unroll
        for (int r = 0; r < 16; r++) s1[r] = s1[r] + a[r];
        break;
      default:   // 7
#pragma unroll
        for (int r = 0; r < 16; r++) { s2[r] = s2[r] + a[r]; s1[r] = s1[r] + s2[r]; s0[r] = s0[r] + s1[r]; }
        break;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) a[r] = 0.0f;
  };
  if constexpr (kP > 0) {
    constexpr int kS = kNL * kP;                    // slots of the wave
    constexpr int kRmax = kW == 16 ? 4 : 8;         // 16 waves: at most 128 registers a wave
    constexpr int kRS = kS < kRmax ? kS : kRmax;    // blocks in flight
    // slot j: block j % kP of the leaf at post-order position j / kP (-1: past the matrix)
    auto blk = [&](int j) {
      const int b = leaf_of(j / kP) + 32 * (j % kP);
      return b < nb ? b : -1;
    };
    Ops ring[kRS];
#pragma unroll
    for (int j = 0; j < kRS; j++) load_ops(blk(j), ring[j]);
    const v16i z = {};
    const v16f zf = {};
#pragma unroll
    for (int j = 0; j < kS; j++) {
      Ops& o = ring[j % kRS];
      const v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.w03, o.bq, z, 0, 0, 0);
      const u32x2 aw = {o.wdw, 0u}, bw = {o.xdw, 0u};
      const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(h4, aw), __builtin_bit_cast(h4, bw), zf,
                                                             0, 0, 0);
      if (j + kRS < kS) load_ops(blk(j + kRS), o);
#pragma unroll
      for (int r = 0; r < 16; r++) a[r] = fmaf(sc[r], (float)isum[r], a[r]);
      if (j % kP == kP - 1) close_leaf(j / kP);
    }
  } else {
    // producer: position pi (0..kNL-1) of the post-order, next block pb (-1: done)
    int pi = 0, pb = wave;
    while (pb >= nb) {                                // leading empty leaves
      if (++pi == kNL) { pb = -1; break; }
      pb = leaf_of(pi);
    }
    const int first_pi = pi;
    auto produce = [&](Ops& o) {
      load_ops(pb, o);
      if (pb >= 0) {
        pb += 32;
        while (pb >= nb) {
          if (++pi == kNL) { pb = -1; break; }
          pb = leaf_of(pi);
        }
      }
    };
    // blocks of the wave: every leaf's count
    int total = 0;
#pragma unroll
    for (int i = 0; i < kNL; i++) {
      const int L = wave + kW * i;
      total += L < nb ? (nb - L + 31) / 32 : 0;
    }
    constexpr int kR = 4;                             // blocks in flight
    Ops ring[kR];
#pragma unroll
    for (int d = 0; d < kR; d++) produce(ring[d]);
    // leading empty leaves close with a = 0
    for (int i = 0; i < first_pi; i++) close_leaf(i);
    int ci = first_pi, cb = ci < kNL ? leaf_of(ci) : 0;   // consumer: position, block
    const v16i z = {};
    const v16f zf = {};
    // whole groups of kR slots, every slot folded: past the wave's last block a slot holds
    // zeros (fma(0, 0, a) = a, and a is +0 once every leaf is closed), so the body has no
    // per-slot test and each fold waits for its own slot's loads only
    for (int s = 0; s < total; s += kR) {
#pragma unroll
      for (int d = 0; d < kR; d++) {
        const v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(ring[d].w03, ring[d].bq, z, 0, 0, 0);
        const u32x2 aw = {ring[d].wdw, 0u}, bw = {ring[d].xdw, 0u};
        const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(h4, aw), __builtin_bit_cast(h4, bw), zf,
                                                               0, 0, 0);
        produce(ring[d]);
#pragma unroll
        for (int r = 0; r < 16; r++) a[r] = fmaf(sc[r], (float)isum[r], a[r]);
        if (ci < kNL) {                               // uniform
          cb += 32;
          if (cb >= nb) {                             // the leaf is complete; close it and any empty ones after
            close_leaf(ci);
            while (++ci < kNL && (cb = leaf_of(ci)) >= nb) close_leaf(ci);
          }
        }
      }
    }
    // empty leaves at the end (a wave with no blocks at all closes everything here)
    for (; ci < kNL; ci++) close_leaf(ci);
  }
  // s0 = the wave's subtree partial; the remaining levels on wave 0: pairs (w, w + s) for
  // s = kW/2, ..., 1, each into the lower wave's value
  if constexpr (kW == 16) {
    // the levels on every wave, one barrier each (wave 0 alone would hold 15 partials): at
    // level s, waves s .. 2s-1 publish their values and wave w < s adds wave w + s's into its
    // own -- the same pairs in the same order
#pragma unroll
    for (int st = kW / 2; st >= 1; st /= 2) {
      if (wave >= st && wave < 2 * st) {
#pragma unroll
        for (int r = 0; r < 16; r++) s_d[half][wave - 1][r * 64 + l] = s0[r];
      }
      __syncthreads();
      if (wave < st) {
#pragma unroll
        for (int r = 0; r < 16; r++) s0[r] = s0[r] + s_d[half][wave + st - 1][r * 64 + l];
      }
    }
  } else {
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < 16; r++) s_d[half][wave - 1][r * 64 + l] = s0[r];
    }
    __syncthreads();
  }
  auto combine = [&](float (&v)[16]) {
    if constexpr (kW == 16) {
#pragma unroll
      for (int r = 0; r < 16; r++) v[r] = s0[r];
      return;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      float t[kW];
      t[0] = s0[r];
#pragma unroll
      for (int w = 1; w < kW; w++) t[w] = s_d[half][w - 1][r * 64 + l];
#pragma unroll
      for (int st = kW / 2; st >= 1; st /= 2)
#pragma unroll
        for (int w = 0; w < st; w++) t[w] = t[w] + t[w + st];
      v[r] = t[0];
    }
  };
  if constexpr (kQ) {
    // every wave stays to the end (the barriers below are the whole workgroup's)
    __shared__ float s_raw[2][32][33];              // [half][token][row of the half's tile] (+1 pad)
    __shared__ float s_o[32][33];                   // [token][SiLU element of the block] (+1 pad)
    if (wave == 0) {
      float v[16];
      combine(v);
#pragma unroll
      for (int r = 0; r < 16; r++) s_raw[half][c][c_row(r, h)] = v[r];
    }
    __syncthreads();
    // the SiLU products over every wave: rows 2j (gate) and 2j+1 (up) of a half are the
    // block's element half*16 + j
    for (int i = threadIdx.x; i < 2 * 32 * 16; i += 2 * 64 * kW) {
      const int hf = i >> 9, tq = (i >> 4) & 31, pr = i & 15;
      s_o[tq][hf * 16 + pr] = lt_silu_mul(s_raw[hf][tq][2 * pr], s_raw[hf][tq][2 * pr + 1]);
    }
    __syncthreads();
    // half-wave q quantizes tokens q and q + 16 of the tile (lane = element of the block)
    const int q = threadIdx.x >> 5, e = threadIdx.x & 31;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int tq = q + 16 * k, t = t0 + tq;
      if (t < P.T)   // uniform per half-wave
        quant_block_hw(s_o[tq][e], e, P.Yq + ((size_t)rtg * P.T + t) * 32, P.Yd + (size_t)rtg * P.T + t);
    }
    return;
  }
  if constexpr (EPI == GE_SILU) {
    // the tile through LDS, then the SiLU products spread over every wave (each one's exp and
    // division are binary64 work): output j of token q is rows 2j (gate) and 2j+1 (up)
    __shared__ float s_o[32][33];                   // [token][row of the tile] (+1 pad)
    if (wave == 0) {
      float v[16];
      combine(v);
#pragma unroll
      for (int r = 0; r < 16; r++) s_o[c][c_row(r, h)] = v[r];
    }
    __syncthreads();
    const int F = P.N >> 1;
    for (int i = threadIdx.x; i < 32 * 16; i += 64 * kW) {
      const int tq = i >> 4, pr = i & 15;
      const int t = t0 + tq, n = n0 + 2 * pr;       // N is even: n < N means n + 1 < N
      if (t < P.T && n < P.N) P.Y[(size_t)t * F + (n >> 1)] = lt_silu_mul(s_o[tq][2 * pr], s_o[tq][2 * pr + 1]);
    }
    return;
  }
  if constexpr (EPI == GE_ROPE) {
    // the tile through LDS, then one rotation pair per thread: pair p of token q is rows
    // 2p, 2p+1 of the tile -- below nqk, rows j and j + hd/2 of one head, rotated with
    // k_rope_append_batch's arithmetic (sin / cos of pos * freqs[j], two fmas); q rotated
    // into Y, k rotated into the cache and as it was into Y, v into the cache and Y
    __shared__ float s_o[32][33];                   // [token][row of the tile] (+1 pad)
    if (wave == 0) {
      float v[16];
      combine(v);
#pragma unroll
      for (int r = 0; r < 16; r++) s_o[c][c_row(r, h)] = v[r];
    }
    __syncthreads();
    const int half = P.hd >> 1, nqk = (P.nh + P.nkv) * P.hd, width = P.nkv * P.hd;
    auto put = [&](void* cache, size_t off, float val) {
      if (P.f16) ((uint16_t*)cache)[off] = lt_float_to_half_bits(val);
      else ((float*)cache)[off] = val;
    };
    for (int i = threadIdx.x; i < 32 * 16; i += 64 * kW) {
      const int tq = i >> 4, pr = i & 15;
      const int t = t0 + tq, n = n0 + 2 * pr;       // N is even: n < N means n + 1 < N
      if (t >= P.T || n >= P.N) continue;
      const int pos = P.len[t];
      const bool app = pos >= 0 && pos < P.maxt;
      const size_t cbase = ((size_t)t * P.maxt + (size_t)(app ? pos : 0)) * width;
      float* yt = P.Y + (size_t)t * P.N;
      const float v0 = s_o[tq][2 * pr], v1 = s_o[tq][2 * pr + 1];
      if (n < nqk) {
        const int head = n / P.hd, j = (n - head * P.hd) >> 1;
        const int ra = head * P.hd + j, rb = ra + half;
        const float x1 = P.bias ? v0 + P.bias[ra] : v0;
        const float x2 = P.bias ? v1 + P.bias[rb] : v1;
        float sn, cs;
        lt_sincosf((float)pos * P.freqs[j], &sn, &cs);
        const float o1 = fmaf(x1, cs, -(x2 * sn));
        const float o2 = fmaf(x1, sn, x2 * cs);
        if (head < P.nh) {
          yt[ra] = o1;
          yt[rb] = o2;
        } else {
          yt[ra] = x1;
          yt[rb] = x2;
          if (app) {
            const size_t off = cbase + (size_t)(head - P.nh) * P.hd + j;
            put(P.kc, off, o1);
            put(P.kc, off + half, o2);
          }
        }
      } else {
        const float x1 = P.bias ? v0 + P.bias[n] : v0;
        const float x2 = P.bias ? v1 + P.bias[n + 1] : v1;
        yt[n] = x1;
        yt[n + 1] = x2;
        if (app) {
          put(P.vc, cbase + (size_t)(n - nqk), x1);
          put(P.vc, cbase + (size_t)(n - nqk) + 1, x2);
        }
      }
    }
    return;
  }
  // the tile through LDS, then the epilogue over every wave, element (token q, row e) on
  // thread 32q + e: each token's 32 rows are one 128-byte run of Y (and of the residual)
  __shared__ float s_o[32][33];                     // [token][row of the tile] (+1 pad)
  if (wave == 0) {
    float v[16];
    combine(v);
#pragma unroll
    for (int r = 0; r < 16; r++) s_o[c][c_row(r, h)] = v[r];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * 32; i += 64 * kW) {
    const int tq = i >> 5, e = i & 31;
    const int t = t0 + tq, n = n0 + e;
    if (t < P.T && n < P.N) {
      float o = s_o[tq][e];
      if constexpr (EPI == GE_BIAS) o = o + P.bias[n];
      if constexpr (EPI == GE_RESID) o = o + P.resid[(size_t)t * P.N + n];
      P.Y[(size_t)t * P.N + n] = o;
    }
  }
}

// RoPE of T rows of q|k at positions *pos0 + t (k_rope's arithmetic per token).
__global__ __launch_bounds__(256) void k_rope_batch(float* __restrict__ x, int T, int row_stride,
                                                    const int* __restrict__ pos0, int nheads, int hd,
                                                    const float* __restrict__ freqs) {
  const int half = hd >> 1;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long per_tok = (long)nheads * half;
  if (gid >= per_tok * T) return;
  const int t = (int)(gid / per_tok);
  const int rem = (int)(gid - (long)t * per_tok);
  const int hh = rem / half;
  const int j = rem - hh * half;
  const float ang = (float)(*pos0 + t) * freqs[j];
  float s, cc;
  lt_sincosf(ang, &s, &cc);
  float* base = x + (size_t)t * row_stride + (size_t)hh * hd;
  const float x1 = base[j], x2 = base[j + half];
  base[j] = fmaf(x1, cc, -(x2 * s));
  base[j + half] = fmaf(x1, s, x2 * cc);
}

// KV append of T rows (k_append_kv_incr per token): rows *len .. *len+T-1 (those below
// maxt).  The length is bumped by k_len_add, after the attention that reads it.
template <bool kF16>
__global__ __launch_bounds__(256) void k_kv_append_batch(void* __restrict__ kc, void* __restrict__ vc,
                                                         const float* __restrict__ src, int src_stride,
                                                         int k_off, int v_off, int T,
                                                         const int* __restrict__ len, int width, int maxt) {
  const int t = blockIdx.x;
  const int L = *len + t;
  if (L < 0 || L >= maxt) return;  // uniform per workgroup
  const float* row = src + (size_t)t * src_stride;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const size_t off = (size_t)L * width + i;
    if (kF16) {
      ((uint16_t*)kc)[off] = lt_float_to_half_bits(row[k_off + i]);
      ((uint16_t*)vc)[off] = lt_float_to_half_bits(row[v_off + i]);
    } else {
      ((float*)kc)[off] = row[k_off + i];
      ((float*)vc)[off] = row[v_off + i];
    }
  }
}

// Embedding rows of T device token ids from Q8_0 token_embd (x = q*d, exact); a token
// outside [0, vocab) gives a zero row and sets *err.
__global__ __launch_bounds__(256) void k_embed_batch(const uint8_t* __restrict__ emb, const int* __restrict__ toks,
                                                     float* __restrict__ x, int E, int vocab, int* __restrict__ err) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E) return;
  const int tk = toks[t];
  float v = 0.0f;
  if (tk < 0 || tk >= vocab) {
    if (err && i == 0) *err = 1;
  } else {
    const uint8_t* blk = emb + ((size_t)tk * (E / 32) + (i >> 5)) * kBlockBytes;
    const uint16_t d = (uint16_t)(blk[0] | (blk[1] << 8));
    v = (float)(int8_t)blk[2 + (i & 31)] * lt_h2f(d);
  }
  x[(size_t)t * E + i] = v;
}

// k_rope_batch of the q and k heads of one row of q|k|v, then k_kv_append_batch of its k
// and v, in one workgroup per token: the hd/2 angles of the row's position are evaluated
// once (lt_sincosf of the same products) into LDS and shared by every head; gridDim.y
// workgroups share a token's pairs and V elements.  The roped k goes to the cache only (not
// back into the row).  kSeqs: row t is the next token of sequence t -- position len[t], cache
// rows of sequence t at [t][maxt][nkv*hd] -- instead of token t of one sequence at *len + t.
template <bool kF16, bool kSeqs>
__global__ __launch_bounds__(256) void k_rope_append_batch(float* __restrict__ qkv, int row_stride,
                                                           const int* __restrict__ len, int nh, int nkv, int hd,
                                                           const float* __restrict__ freqs, void* __restrict__ kc,
                                                           void* __restrict__ vc, int maxt) {
  __shared__ float s_sn[128], s_cs[128];
  const int t = blockIdx.x;
  const int half = hd >> 1;
  const int pos = kSeqs ? len[t] : *len + t;
  if (kSeqs) {
    const size_t seq = (size_t)t * maxt * nkv * hd * (kF16 ? 2 : 4);
    kc = (uint8_t*)kc + seq;
    vc = (uint8_t*)vc + seq;
  }
  for (int j = threadIdx.x; j < half; j += 256) lt_sincosf((float)pos * freqs[j], &s_sn[j], &s_cs[j]);
  __syncthreads();
  float* row = qkv + (size_t)t * row_stride;
  const bool app = pos >= 0 && pos < maxt;
  const int width = nkv * hd;
  auto put = [&](void* c, size_t off, float v) {
    if (kF16) ((uint16_t*)c)[off] = lt_float_to_half_bits(v);
    else ((float*)c)[off] = v;
  };
  const int i0 = threadIdx.x + 256 * blockIdx.y, istep = 256 * gridDim.y;
  for (int i = i0; i < (nh + nkv) * half; i += istep) {
    const int hh = i / half, j = i - hh * half;
    float* base = row + (size_t)hh * hd;
    const float x1 = base[j], x2 = base[j + half];
    const float sn = s_sn[j], cs = s_cs[j];
    const float o1 = fmaf(x1, cs, -(x2 * sn));
    const float o2 = fmaf(x1, sn, x2 * cs);
    if (hh < nh) {
      base[j] = o1;
      base[j + half] = o2;
    } else if (app) {
      const size_t off = (size_t)pos * width + (size_t)(hh - nh) * hd + j;
      put(kc, off, o1);
      put(kc, off + half, o2);
    }
  }
  if (app) {
    const float* v = row + (size_t)(nh + nkv) * hd;
    for (int i = i0; i < width; i += istep) put(vc, (size_t)pos * width + i, v[i]);
  }
}

// n consecutive lengths each advanced by T (clamped to maxt)
__global__ void k_len_add_n(int* __restrict__ len, int n, int T, int maxt) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int L = len[i] + T;
    len[i] = L < maxt ? L : maxt;
  }
}

__global__ void k_len_add(int* __restrict__ len, int T, int maxt) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int L = *len + T;
    *len = L < maxt ? L : maxt;
  }
}

// The tile-major copy of a Q8_0 matrix: tile rt, block b holds the quants of rows
// 32*rt .. 32*rt+31 of block b (32 bytes each), then their fp16 scales (rows past N are
// zero).  One 2-byte unit per thread, written in order.  nqk > 0: the rope-pair order --
// within each of the first nqk rows' heads of hd rows, row 2j + e of the copy is row
// j + e*hd/2 of the head (the two rows RoPE rotates together are adjacent); rows from nqk
// on keep their places.
__global__ __launch_bounds__(256) void k_q8_tiles(const uint16_t* __restrict__ W, uint16_t* __restrict__ Wt, int N,
                                                  int nb, uint32_t units, int hd, int nqk) {
  constexpr uint32_t kUnits = kBlockBytes / 2;             // 17 per block
  constexpr uint32_t kTileUnits = kTileBlk / 2;            // 544 per tile block
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < units; i += gridDim.x * 256u) {
    const uint32_t chunk = i / kTileUnits, j = i - chunk * kTileUnits;
    const uint32_t rt = chunk / (uint32_t)nb, b = chunk - rt * (uint32_t)nb;
    // units 0..511: row j/16's quant pair j%16 (block unit 1 + j%16); 512..543: the scale
    // of row j-512 (block unit 0)
    const uint32_t r = j < 512u ? j >> 4 : j - 512u;
    const uint32_t u = j < 512u ? 1u + (j & 15u) : 0u;
    uint32_t row = rt * 32u + r;
    if ((int)row < nqk) {
      const uint32_t head = row / (uint32_t)hd, q = row - head * (uint32_t)hd;
      row = head * (uint32_t)hd + (q >> 1) + (q & 1u) * ((uint32_t)hd >> 1);
    }
    Wt[i] = row < (uint32_t)N ? W[((size_t)row * nb + b) * kUnits + u] : (uint16_t)0;
  }
}
__global__ __launch_bounds__(256) void k_quant_q8_bm(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                     uint16_t* __restrict__ xd, int T, int nbk) {
  // 8 lanes per output block (4 consecutive elements each, one 16-byte load), 32 blocks
  // per workgroup; consecutive blocks of the output are consecutive tokens of one block column
  const long ob = (long)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  if (ob >= (long)T * nbk) return;   // uniform per 8-lane group
  const int b = (int)(ob / T), t = (int)(ob - (long)b * T);
  const float4 v = *(const float4*)(x + ((size_t)t * nbk + b) * 32 + 4 * j);
  QScale s;
  const uint32_t p = quant4(v.x, v.y, v.z, v.w, s);
  ((uint32_t*)(xq + ob * 32))[j] = p;
  if (j == 0) xd[ob] = s.h;
}

int check_gemm(const char* fn, const void* W, const int8_t* Xq, const uint16_t* Xd, const float* Y, int T, int N,
               int K) {
  LT_REQUIRE(W && Xq && Xd && Y, "%s: null argument", fn);
  LT_REQUIRE(T > 0 && N > 0 && K > 0 && K % 32 == 0, "%s: T=%d N=%d K=%d (K multiple of 32)", fn, T, N, K);
  LT_REQUIRE((uint64_t)N * (uint64_t)(K / 32) * 34u < ((uint64_t)1 << 31),
             "%s: a %d x %d Q8_0 matrix must be below 2 GiB (split it by rows)", fn, N, K);
  LT_REQUIRE((uint64_t)T * (uint64_t)K < ((uint64_t)1 << 31), "%s: T=%d x K=%d activation quants above 2 GiB", fn, T,
             K);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(Xq, 16) && lt_aligned(Xd, 2), "%s: misaligned argument", fn);
  return LT_OK;
}

// LT_GEMM_LS=0 keeps every launch on k_q8_gemm (for comparisons), 1 sends every tiled launch
// to the leaf-split kernel.  By default a tiled launch takes it when it holds at most kLsMaxT
// tokens, or when k_q8_gemm's grid (kGemmTokens-token tiles) would hold fewer than kLsFill
// workgroups per CU: there the leaf-split kernel's 32-token tiles, four waves each, fill the
// chip.  Measured per launch, k_q8_gemm / leaf-split (us): 896 x 4864 at T = 512 40.5 / 15.4,
// 1152 x 896 at 512 19.7 / 10.6, 9728 x 896 at 128 22.1 / 18.4 but at 256 28.3 / 31.7,
// 4096 x 4096 at 256 30.6 / 27.7 but at 512 40.7 / 46.6, 151936 x 896 at 128 169 / 206.
constexpr int kLsMaxT = 64;
constexpr int kLsFill = 2;
int ls_mode() {
  const char* s = getenv("LT_GEMM_LS");
  return s ? atoi(s) : -1;
}

// A leaf-split launch: the compile-time schedule (k_q8_gemm_ls's kP, blocks per leaf) when a
// wave's slots, (32 / kW) * kP, number at most 20 -- 4 waves per tile: K <= 2048, 8 waves:
// K <= 5120 -- else the run-time walk.  LT_GEMM_LS_STATIC=0 forces the run-time walk (read at
// every launch).  Measured at T = 64, run-time / compile-time walk (us): 9728 x 896 11.2 /
// 8.0, 151936 x 896 115 / 83, 1152 x 896 5.5 / 4.2, 896 x 4864 (8 waves) 8.7 / 7.9, 4096 x
// 4096 (8 waves) 9.7 / 9.4; but with 32 slots, 6144 x 4096 (4 waves) 15.6 / 16.7.
template <GemmEpi EPI, int kW, bool kQ>
void launch_ls(lt_ctx* ctx, const GemmParams& P, unsigned grid) {
  constexpr unsigned kThreads = 64u * kW * (kQ ? 2u : 1u);
  const char* senv = getenv("LT_GEMM_LS_STATIC");
  const int bpl = (senv && atoi(senv) == 0) ? 0 : (P.K / 32 + 31) / 32;
  if (bpl == 1) {
    k_q8_gemm_ls<EPI, kW, kQ, 1><<<grid, kThreads, 0, ctx->stream>>>(P);
  } else if (bpl == 2) {
    k_q8_gemm_ls<EPI, kW, kQ, 2><<<grid, kThreads, 0, ctx->stream>>>(P);
  } else if constexpr (kW >= 8) {
    if (bpl == 3) k_q8_gemm_ls<EPI, kW, kQ, 3><<<grid, kThreads, 0, ctx->stream>>>(P);
    else if (bpl == 4) k_q8_gemm_ls<EPI, kW, kQ, 4><<<grid, kThreads, 0, ctx->stream>>>(P);
    else if (bpl == 5) k_q8_gemm_ls<EPI, kW, kQ, 5><<<grid, kThreads, 0, ctx->stream>>>(P);
    else k_q8_gemm_ls<EPI, kW, kQ, 0><<<grid, kThreads, 0, ctx->stream>>>(P);
  } else {
    k_q8_gemm_ls<EPI, kW, kQ, 0><<<grid, kThreads, 0, ctx->stream>>>(P);
  }
}

template <GemmEpi EPI, bool kTiled>
int launch_gemm(lt_ctx* ctx, GemmParams P) {
  P.nrt = (P.N + 31) / 32;
  if constexpr (kTiled) {
    const int mode = ls_mode();
    const long wgs = (long)((P.nrt + 7) / 8) * 8 * ((P.T + kGemmTokens - 1) / kGemmTokens);
    const long fill = (long)kLsFill * (ctx->num_cus > 0 ? ctx->num_cus : 256);
    if (mode == 1 || (mode < 0 && (P.T <= kLsMaxT || wgs < fill))) {
      P.ntt = (P.T + 31) / 32;
      const long gls = (long)((P.nrt + 7) / 8) * 8 * P.ntt;
      // 8 waves per tile when the launch holds at most one tile per CU, 16 when in addition
      // each leaf holds 3 to 5 blocks (K 2049 .. 5120; LT_GEMM_LS_W=4 / 8 / 16 forces one,
      // read at every launch).  Measured at T = 64, 4 / 8 waves (us): 896 x 4864 13.4 / 8.9,
      // 896 x 896 7.9 / 5.6, 4096 x 4096 13.1 / 10.3, 4096 x 14336 29.4 / 24.7, but 6144 x
      // 4096 15.2 / 17.4 and 9728 x 896 10.8 / 14.0 (384 and 608 tiles); 8 / 16 waves on the
      // compile-time schedule: 896 x 4864 7.95 / 7.58, 4096 x 4096 9.52 / 9.12, 896 x 896
      // 4.19 / 4.26.
      const char* wenv = getenv("LT_GEMM_LS_W");
      const int wforce = wenv ? atoi(wenv) : 0;
      const long cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
      const int bpl = (P.K / 32 + 31) / 32;
      const int w = wforce ? wforce : gls > cus ? 4 : (bpl >= 3 && bpl <= 5) ? 16 : 8;
      if (w == 16) launch_ls<EPI, 16, false>(ctx, P, (unsigned)gls);
      else if (w == 8) launch_ls<EPI, 8, false>(ctx, P, (unsigned)gls);
      else launch_ls<EPI, 4, false>(ctx, P, (unsigned)gls);
      return lt_check_launch("k_q8_gemm_ls");
    }
  }
  P.ntt = (P.T + kGemmTokens - 1) / kGemmTokens;
  const long grid = (long)((P.nrt + 7) / 8) * 8 * P.ntt;
  if constexpr (kTiled) {
    // K a multiple of 2048 (an even number of blocks per leaf, bpl): grouped leaves -- with a
    // 2-slot ring when the launch holds 3 or more waves per SIMD (the other waves hide the
    // latency), else (bpl % 4 == 0) with a 4-slot ring and pipelined MFMAs in 256 registers.
    // LT_GEMM_GROUPED=0 / 1 / 2 forces the dynamic walk / the 2-slot / the 4-slot walk where
    // K allows it (read at every launch).
    if (P.K % 2048 == 0) {
      const int bpl = P.K / 1024;
      const long waves = (long)P.nrt * ((P.T + 31) / 32);
      const bool big = waves >= 12L * (ctx->num_cus > 0 ? ctx->num_cus : 256);
      const char* force = getenv("LT_GEMM_GROUPED");
      const int walk = force ? atoi(force) : big ? 1 : bpl % 4 == 0 ? 2 : 0;
      if (walk == 1) {
        k_q8_gemm<EPI, true, 1><<<(unsigned)grid, 256, 0, ctx->stream>>>(P);
        return lt_check_launch("k_q8_gemm");
      }
      if (walk == 2 && bpl % 4 == 0) {
        k_q8_gemm<EPI, true, 2><<<(unsigned)grid, 256, 0, ctx->stream>>>(P);
        return lt_check_launch("k_q8_gemm");
      }
    }
  }
  k_q8_gemm<EPI, kTiled><<<(unsigned)grid, 256, 0, ctx->stream>>>(P);
  return lt_check_launch("k_q8_gemm");
}

size_t tiles_bytes(int N, int K) { return (size_t)((N + 31) / 32) * 32 * (size_t)(K / 32) * kBlockBytes; }

template <bool kTiled>
int gemm_entry(const char* fn, lt_ctx* ctx, const void* W, const int8_t* Xq, const uint16_t* Xd, const float* bias,
               const float* resid, float* Y, int T, int N, int K) {
  LT_REQUIRE(ctx, "%s: null ctx", fn);
  if (int rc = check_gemm(fn, W, Xq, Xd, Y, T, N, K)) return rc;
  LT_REQUIRE(!(bias && resid), "%s: give bias or resid, not both", fn);
  if (kTiled) LT_REQUIRE(tiles_bytes(N, K) < ((size_t)1 << 31), "%s: tile copy of %d x %d above 2 GiB", fn, N, K);
  GemmParams P{};
  P.W = (const uint8_t*)W; P.Xq = Xq; P.Xd = Xd; P.bias = bias; P.resid = resid; P.Y = Y;
  P.T = T; P.N = N; P.K = K;
  if (bias) return launch_gemm<GE_BIAS, kTiled>(ctx, P);
  if (resid) return launch_gemm<GE_RESID, kTiled>(ctx, P);
  return launch_gemm<GE_STORE, kTiled>(ctx, P);
}

// q|k|v of the next token of T sequences on the leaf-split kernel with the RoPE + KV-append
// epilogue (k_q8_gemm_ls<GE_ROPE, ...>): the weights in lt_q8_tiles_rope's order, 8 waves per
// tile when the launch holds at most one tile per CU.
int launch_gemm_rope(lt_ctx* ctx, GemmParams P) {
  P.nrt = (P.N + 31) / 32;
  P.ntt = (P.T + 31) / 32;
  const long gls = (long)((P.nrt + 7) / 8) * 8 * P.ntt;
  const long cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  if (gls <= cus) launch_ls<GE_ROPE, 8, false>(ctx, P, (unsigned)gls);
  else launch_ls<GE_ROPE, 4, false>(ctx, P, (unsigned)gls);
  return lt_check_launch("k_q8_gemm_ls");
}

// The leaf-split SiLU GEMM with the quant of its output fused (k_q8_gemm_ls<GE_SILU, 4, true>):
// every launch on it, whatever T (its grid: pairs of row tiles x 32-token tiles).
int launch_gemm_silu_q(lt_ctx* ctx, GemmParams P) {
  P.nrt = (P.N + 31) / 32;
  P.ntt = (P.T + 31) / 32;
  const int npair = P.nrt / 2;
  const long gls = (long)((npair + 7) / 8) * 8 * P.ntt;
  launch_ls<GE_SILU, 4, true>(ctx, P, (unsigned)gls);
  return lt_check_launch("k_q8_gemm_ls");
}

template <bool kTiled>

int gemm_silu_entry(const char* fn, lt_ctx* ctx, const void* Wgu, const int8_t* Xq, const uint16_t* Xd, float* V,
                    int T, int F, int K) {
  LT_REQUIRE(ctx && F > 0, "%s: null ctx or F=%d", fn, F);
  if (int rc = check_gemm(fn, Wgu, Xq, Xd, V, T, 2 * F, K)) return rc;
  if (kTiled) LT_REQUIRE(tiles_bytes(2 * F, K) < ((size_t)1 << 31), "%s: tile copy above 2 GiB", fn);
  GemmParams P{};
  P.W = (const uint8_t*)Wgu; P.Xq = Xq; P.Xd = Xd; P.Y = V;
  P.T = T; P.N = 2 * F; P.K = K;
  return launch_gemm<GE_SILU, kTiled>(ctx, P);
}

}  // namespace

extern "C" {

int lt_q8_gemm(lt_ctx* ctx, const void* W, const int8_t* Xq, const uint16_t* Xd, const float* bias,
               const float* resid, float* Y, int T, int N, int K) {
  return gemm_entry<false>("lt_q8_gemm", ctx, W, Xq, Xd, bias, resid, Y, T, N, K);
}

int lt_q8_gemm_silu(lt_ctx* ctx, const void* Wgu, const int8_t* Xq, const uint16_t* Xd, float* V, int T, int F,
                    int K) {
  return gemm_silu_entry<false>("lt_q8_gemm_silu", ctx, Wgu, Xq, Xd, V, T, F, K);
}

size_t lt_q8_tiles_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) return 0;
  return tiles_bytes(N, K);
}

int lt_q8_tiles(lt_ctx* ctx, const void* W, void* Wt, int N, int K) {
  LT_REQUIRE(ctx && W && Wt, "lt_q8_tiles: null argument");
  LT_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "lt_q8_tiles: N=%d K=%d", N, K);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(Wt, 16), "lt_q8_tiles: misaligned argument");
  const size_t units = tiles_bytes(N, K) / 2;
  LT_REQUIRE(units < ((size_t)1 << 32), "lt_q8_tiles: %d x %d too large", N, K);
  const unsigned grid = (unsigned)(units / 256 < 65536 ? (units + 255) / 256 : 65536);
  k_q8_tiles<<<grid, 256, 0, ctx->stream>>>((const uint16_t*)W, (uint16_t*)Wt, N, K / 32, (uint32_t)units, 1, 0);
  return lt_check_launch("k_q8_tiles");
}

int lt_q8_tiles_rope(lt_ctx* ctx, const void* W, void* Wt, int N, int K, int nh, int nkv, int hd) {
  LT_REQUIRE(ctx && W && Wt, "lt_q8_tiles_rope: null argument");
  LT_REQUIRE(K > 0 && K % 32 == 0 && nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && N == (nh + 2 * nkv) * hd,
             "lt_q8_tiles_rope: N=%d K=%d nh=%d nkv=%d hd=%d (N = (nh + 2 nkv) hd, hd even)", N, K, nh, nkv, hd);
  LT_REQUIRE(lt_aligned(W, 4) && lt_aligned(Wt, 16), "lt_q8_tiles_rope: misaligned argument");
  const size_t units = tiles_bytes(N, K) / 2;
  LT_REQUIRE(units < ((size_t)1 << 32), "lt_q8_tiles_rope: %d x %d too large", N, K);
  const unsigned grid = (unsigned)(units / 256 < 65536 ? (units + 255) / 256 : 65536);
  k_q8_tiles<<<grid, 256, 0, ctx->stream>>>((const uint16_t*)W, (uint16_t*)Wt, N, K / 32, (uint32_t)units, hd,
                                            (nh + nkv) * hd);
  return lt_check_launch("k_q8_tiles");
}

int lt_quant_q8_bm(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int T, int K) {
  LT_REQUIRE(ctx && x && xq && xd, "lt_quant_q8_bm: null argument");
  LT_REQUIRE(T > 0 && K > 0 && K % 32 == 0, "lt_quant_q8_bm: T=%d K=%d", T, K);
  LT_REQUIRE(lt_aligned(xq, 16) && lt_aligned(xd, 2), "lt_quant_q8_bm: misaligned argument");
  const long nblk = (long)T * (K / 32);
  LT_REQUIRE(lt_aligned(x, 16), "lt_quant_q8_bm: x must be 16-byte aligned");
  k_quant_q8_bm<<<(unsigned)((nblk + 31) / 32), 256, 0, ctx->stream>>>(x, xq, xd, T, K / 32);
  return lt_check_launch("k_quant_q8_bm");
}

int lt_q8_gemm_t(lt_ctx* ctx, const void* Wt, const int8_t* Xq, const uint16_t* Xd, const float* bias,
                 const float* resid, float* Y, int T, int N, int K) {
  return gemm_entry<true>("lt_q8_gemm_t", ctx, Wt, Xq, Xd, bias, resid, Y, T, N, K);
}

int lt_q8_gemm_silu_t(lt_ctx* ctx, const void* Wgut, const int8_t* Xq, const uint16_t* Xd, float* V, int T, int F,
                      int K) {
  return gemm_silu_entry<true>("lt_q8_gemm_silu_t", ctx, Wgut, Xq, Xd, V, T, F, K);
}

int lt_q8_gemm_silu_quant_t(lt_ctx* ctx, const void* Wgut, const int8_t* Xq, const uint16_t* Xd, int8_t* Vq,
                            uint16_t* Vd, int T, int F, int K) {
  const char* fn = "lt_q8_gemm_silu_quant_t";
  LT_REQUIRE(ctx && Vq && Vd, "%s: null argument", fn);
  LT_REQUIRE(F > 0 && F % 32 == 0, "%s: F=%d (a multiple of 32: whole quant blocks)", fn, F);
  if (int rc = check_gemm(fn, Wgut, Xq, Xd, (const float*)Vq, T, 2 * F, K)) return rc;
  LT_REQUIRE(tiles_bytes(2 * F, K) < ((size_t)1 << 31), "%s: tile copy above 2 GiB", fn);
  LT_REQUIRE((uint64_t)T * (uint64_t)F < ((uint64_t)1 << 31), "%s: T=%d x F=%d output quants above 2 GiB", fn, T, F);
  LT_REQUIRE((void*)Vq != (const void*)Xq && (const void*)Vd != (const void*)Xd,
             "%s: the output quants must not overwrite the input quants", fn);
  GemmParams P{};
  P.W = (const uint8_t*)Wgut; P.Xq = Xq; P.Xd = Xd; P.Yq = Vq; P.Yd = Vd;
  P.T = T; P.N = 2 * F; P.K = K;
  return launch_gemm_silu_q(ctx, P);
}

int lt_q8_gemm_rope_t(lt_ctx* ctx, const void* Wt, const int8_t* Xq, const uint16_t* Xd, int T, const float* bias,
                      float* qkv, int N, int K, const int* len, int nh, int nkv, int hd, const float* freqs, void* kc,
                      void* vc, int maxt, int kv_dtype) {
  const char* fn = "lt_q8_gemm_rope_t";
  LT_REQUIRE(ctx && len && freqs && kc && vc, "%s: null argument", fn);
  if (int rc = check_gemm(fn, Wt, Xq, Xd, qkv, T, N, K)) return rc;
  LT_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && maxt > 0 && N == (nh + 2 * nkv) * hd,
             "%s: N=%d nh=%d nkv=%d hd=%d maxt=%d (N = (nh + 2 nkv) hd, hd even)", fn, N, nh, nkv, hd, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "%s: kv_dtype=%d", fn, kv_dtype);
  LT_REQUIRE(tiles_bytes(N, K) < ((size_t)1 << 31), "%s: tile copy of %d x %d above 2 GiB", fn, N, K);
  GemmParams P{};
  P.W = (const uint8_t*)Wt; P.Xq = Xq; P.Xd = Xd; P.bias = bias; P.Y = qkv;
  P.T = T; P.N = N; P.K = K;
  P.len = len; P.freqs = freqs; P.kc = kc; P.vc = vc;
  P.nh = nh; P.nkv = nkv; P.hd = hd; P.maxt = maxt; P.f16 = kv_dtype == LT_KV_F16 ? 1 : 0;
  return launch_gemm_rope(ctx, P);
}

int lt_rope_batch(lt_ctx* ctx, float* qk, int T, int row_stride, const int* pos0, int nheads, int hd,
                  const float* freqs) {
  LT_REQUIRE(ctx && qk && pos0 && freqs, "lt_rope_batch: null argument");
  LT_REQUIRE(T > 0 && nheads > 0 && hd > 0 && hd % 2 == 0 && row_stride >= nheads * hd,
             "lt_rope_batch: T=%d nheads=%d hd=%d row_stride=%d", T, nheads, hd, row_stride);
  const long total = (long)T * nheads * (hd / 2);
  k_rope_batch<<<(unsigned)((total + 255) / 256), 256, 0, ctx->stream>>>(qk, T, row_stride, pos0, nheads, hd, freqs);
  return lt_check_launch("k_rope_batch");
}

int lt_kv_append_batch(lt_ctx* ctx, void* kc, void* vc, const float* src, int src_stride, int k_off, int v_off,
                       int T, const int* len, int width, int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && kc && vc && src && len, "lt_kv_append_batch: null argument");
  LT_REQUIRE(T > 0 && width > 0 && maxt > 0, "lt_kv_append_batch: T=%d width=%d maxt=%d", T, width, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_kv_append_batch: kv_dtype=%d", kv_dtype);
  if (kv_dtype == LT_KV_F16)
    k_kv_append_batch<true><<<T, 256, 0, ctx->stream>>>(kc, vc, src, src_stride, k_off, v_off, T, len, width, maxt);
  else
    k_kv_append_batch<false><<<T, 256, 0, ctx->stream>>>(kc, vc, src, src_stride, k_off, v_off, T, len, width, maxt);
  return lt_check_launch("k_kv_append_batch");
}

int lt_embed_q8_batch(lt_ctx* ctx, const void* emb, const int* toks, float* x, int T, int E, int vocab, int* err) {
  LT_REQUIRE(ctx && emb && toks && x, "lt_embed_q8_batch: null argument");
  LT_REQUIRE(T > 0 && E > 0 && E % 32 == 0 && vocab > 0, "lt_embed_q8_batch: T=%d E=%d vocab=%d", T, E, vocab);
  k_embed_batch<<<dim3((E + 255) / 256, T), 256, 0, ctx->stream>>>((const uint8_t*)emb, toks, x, E, vocab, err);
  return lt_check_launch("k_embed_batch");
}

int lt_rope_append_batch(lt_ctx* ctx, float* qkv, int T, int row_stride, const int* len, int nh, int nkv, int hd,
                         const float* freqs, void* kc, void* vc, int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && qkv && len && freqs && kc && vc, "lt_rope_append_batch: null argument");
  LT_REQUIRE(T > 0 && nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && hd <= 256 && maxt > 0 &&
                 row_stride >= (nh + 2 * nkv) * hd,
             "lt_rope_append_batch: T=%d nh=%d nkv=%d hd=%d row_stride=%d maxt=%d", T, nh, nkv, hd, row_stride, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_rope_append_batch: kv_dtype=%d", kv_dtype);
  if (kv_dtype == LT_KV_F16)
    k_rope_append_batch<true, false><<<dim3(T, 4), 256, 0, ctx->stream>>>(qkv, row_stride, len, nh, nkv, hd, freqs,
                                                                           kc, vc, maxt);
  else
    k_rope_append_batch<false, false><<<dim3(T, 4), 256, 0, ctx->stream>>>(qkv, row_stride, len, nh, nkv, hd, freqs,
                                                                            kc, vc, maxt);
  return lt_check_launch("k_rope_append_batch");
}

int lt_rope_append_seqs(lt_ctx* ctx, float* qkv, int B, int row_stride, const int* len, int nh, int nkv, int hd,
                        const float* freqs, void* kc, void* vc, int maxt, int kv_dtype) {
  LT_REQUIRE(ctx && qkv && len && freqs && kc && vc, "lt_rope_append_seqs: null argument");
  LT_REQUIRE(B > 0 && nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && hd <= 256 && maxt > 0 &&
                 row_stride >= (nh + 2 * nkv) * hd,
             "lt_rope_append_seqs: B=%d nh=%d nkv=%d hd=%d row_stride=%d maxt=%d", B, nh, nkv, hd, row_stride, maxt);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_rope_append_seqs: kv_dtype=%d", kv_dtype);
  if (kv_dtype == LT_KV_F16)
    k_rope_append_batch<true, true><<<dim3(B, 4), 256, 0, ctx->stream>>>(qkv, row_stride, len, nh, nkv, hd, freqs,
                                                                          kc, vc, maxt);
  else
    k_rope_append_batch<false, true><<<dim3(B, 4), 256, 0, ctx->stream>>>(qkv, row_stride, len, nh, nkv, hd, freqs,
                                                                           kc, vc, maxt);
  return lt_check_launch("k_rope_append_batch<seqs>");
}

int lt_len_add_n(lt_ctx* ctx, int* len, int n, int T, int maxt) {
  LT_REQUIRE(ctx && len && n > 0 && T >= 0 && maxt > 0, "lt_len_add_n: bad argument");
  k_len_add_n<<<1, 256, 0, ctx->stream>>>(len, n, T, maxt);
  return lt_check_launch("k_len_add_n");
}

int lt_len_add(lt_ctx* ctx, int* len, int T, int maxt) {
  LT_REQUIRE(ctx && len && T >= 0 && maxt > 0, "lt_len_add: bad argument");
  k_len_add<<<1, 64, 0, ctx->stream>>>(len, T, maxt);
  return lt_check_launch("k_len_add");
}

}  // extern "C"
