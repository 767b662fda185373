// lt_step.hip -- the whole decode step of a small model in one persistent launch.
//
// The five-launch step (lt_fused.hip, lt_attn.hip) spends most of a layer at kernel
// boundaries: each launch begins with a node gap and a dependent memory round trip before its
// first weight byte arrives, and streams its weights only after that.  Here one launch of one
// workgroup per CU runs every layer.  The reference chain of a layer
// (bpd/lib/dev_residency.py:1380-1477) is cut into five phases at the points where an op needs
// the whole output of the previous one:
//
//   A  rmsnorm -> quant -> QKV GEMV + bias -> RoPE(q, k) -> KV append     (8-row units)
//   B  masked attention over the cache and the new row -> quant            (one head each)
//   C  O GEMV + residual                                                   (8-row units)
//   D  rmsnorm -> quant -> gate|up GEMV -> SiLU(g)*u -> quant              (64-row units)
//   E  down GEMV + residual                                                (8-row units)
//
// A phase's outputs reach the consuming workgroups through device memory as 64-bit words that
// carry the step's tag next to a 32-bit payload (flag in data, as in RCCL's LL protocol).  Each
// word is written by one relaxed agent-scope atomic store and read by relaxed agent-scope
// atomic loads (device-coherent accesses: they do not stop in the non-coherent per-XCD L2), and
// a consumer re-reads its words until every tag is the step's.  A 64-bit atomic store is seen
// whole or not at all, so a matching tag vouches for its payload: no release/acquire fence, L2
// writeback or invalidate is ever issued.  Every producer writes one contiguous run of words
// (words of one cache line shared by many producers measured slower to exchange).
//
// A workgroup's weights are requested one or two phases before they are used, into registers,
// per lane in the GEMV's raw 34-byte block pattern, so the HBM stream runs under the exchanges
// and a phase's critical path is its exchange plus its arithmetic.  The arithmetic of every op
// is the per-op kernels' (lt_ops.hip, lt_attn.hip, lt_fused.hip) operation for operation, so
// the step is bit-identical to them and to the oracle.
//
// Every wait is bounded: a poll that does not see its tags within kSpin rounds, or that sees
// another workgroup's failure, records an error and its workgroup leaves the step, so the
// launch always drains.  The launch needs all of its workgroups resident at once (one per CU,
// checked on the host from the kernel's occupancy before every launch).
#include "lt_q8_device.h"

namespace {

using namespace lt;

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kT = 256;                 // threads per workgroup
constexpr int kHd = 64;                 // head size
constexpr int kMaxE = 1024;             // n_embd and n_head*hd: one 32-block item per row
constexpr int kMaxNb = kMaxE / 32;
constexpr int kDownItems = 5;           // n_ff <= 5120: at most 5 blocks per lane per down row
constexpr int kMaxF = kDownItems * 1024;
constexpr int kMaxNbF = kMaxF / 32;
constexpr int kGuRows = 64;             // gate|up rows per unit: the gate/up pairs of one quant block
constexpr uint32_t kSpin = 1u << 17;    // poll rounds before a wait is declared failed (>= ~60 ms)
constexpr uint32_t kNone = 0x80000000u; // buffer offset past every matrix: reads zeros
constexpr int kLdsMax = 160 * 1024;     // LDS of one gfx950 workgroup

// error codes written to *err (the plan's error word; 1 = token out of range)
constexpr int kErrTimeout = 2;
constexpr int kErrLength = 3;

// ---- device-coherent tagged words -------------------------------------------------------
__device__ __forceinline__ void xput(uint64_t* p, uint32_t tag, uint32_t v) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t xget(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int iget(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t uget(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void uput(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct StepState {
  uint32_t serial;     // steps completed: this step's tag is serial + 1
  uint32_t arrived;    // workgroups done with this step (reset by the last one)
  uint32_t fail;       // nonzero once a workgroup gave up on a wait (cleared by the host)
  uint32_t pad[61];
};
static_assert(sizeof(StepState) == 256, "StepState keeps the exchange words 256-byte aligned");

struct StepParams {
  const lt_step_layer* layers;
  int n_layers;
  int E, F, nh, nkv;
  float eps, scale;
  const float* freqs;      // RoPE inverse frequencies [hd/2]
  int* lens;               // [n_layers]: cache length of each layer = position of the new token
  int maxt;
  const uint8_t* emb;      // Q8_0 token_embd [vocab][E/32] (layer 0 input), or null with x_in
  const int* tok;
  int vocab;
  const float* x_in;       // host-written input row (when emb is null)
  float* x_out;            // the last layer's output row
  int* err;
  StepState* st;
  uint64_t* xw;            // exchange words
  int offA, offB, offC, offD, offE, lstride;   // per-layer word offsets and stride
  int nmax;                // attended rows the launch's LDS stages
};

// The layer descriptors are read through the constant address space: scalar loads into
// SGPRs, so the buffer resources built from them are uniform.  (Read as ordinary global
// memory they land in VGPRs, every buffer load of a weight becomes a waterfall loop, and each
// waits for all loads in flight first -- the prefetches included.)
__device__ __forceinline__ lt_step_layer layer_desc(const lt_step_layer* layers, int l) {
  static_assert(sizeof(lt_step_layer) == 9 * sizeof(uint64_t), "lt_step_layer: nine pointers");
#if defined(__HIP_DEVICE_COMPILE__)
  typedef const __attribute__((address_space(4))) uint64_t* ConstWords;
  const ConstWords q = (ConstWords)(layers + l);
  lt_step_layer d;
  d.attn_norm = (const float*)q[0];
  d.wqkv = (const void*)q[1];
  d.bqkv = (const float*)q[2];
  d.wo = (const void*)q[3];
  d.ffn_norm = (const float*)q[4];
  d.wgu = (const void*)q[5];
  d.wdown = (const void*)q[6];
  d.kc = (void*)q[7];
  d.vc = (void*)q[8];
  return d;
#else
  return layers[l];
#endif
}

// Words of one layer's exchange regions.
struct XLayout {
  int offA, offB, offC, offD, offE, lstride;
};
inline int up16(int n) { return (n + 15) & ~15; }
inline XLayout x_layout(int E, int F, int nh, int nkv) {
  XLayout x;
  const int nqkv = (nh + 2 * nkv) * kHd;
  x.offA = 0;                                   // q|k|v after RoPE, 8 words per unit
  x.offB = x.offA + up16(nqkv);                 // attention output: 9 words per 32-block
  x.offC = x.offB + up16(nh * kHd / 32 * 9);    // x after the attention residual
  x.offD = x.offC + up16(E);                    // SiLU(g)*u quantized: 9 words per block
  x.offE = x.offD + up16(F / 32 * 9);           // x after the FFN residual
  x.lstride = x.offE + up16(E);
  return x;
}

// Poll words [0, n) of p: thread t takes words t + kT*k.  False when the tags do not all
// match within kSpin rounds, or another workgroup has failed.
template <int PER>
__device__ __forceinline__ bool xpoll(const uint64_t* p, int n, uint32_t tag, const uint32_t* fail, uint32_t (&v)[PER]) {
  uint32_t spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int i = (int)threadIdx.x + kT * k;
      if (i < n) {
        const uint64_t x = xget(p + i);
        v[k] = (uint32_t)x;
        ok &= (uint32_t)(x >> 32) == tag;
      } else {
        v[k] = 0u;
      }
    }
    if (ok) return true;
    if (++spins >= kSpin) return false;
    if ((spins & 31u) == 0u && uget(fail) != 0u) return false;
  }
}

// one word per calling thread
__device__ __forceinline__ bool xpoll1(const uint64_t* p, uint32_t tag, const uint32_t* fail, uint32_t& v) {
  uint32_t spins = 0;
  for (;;) {
    const uint64_t x = xget(p);
    v = (uint32_t)x;
    if ((uint32_t)(x >> 32) == tag) return true;
    if (++spins >= kSpin) return false;
    if ((spins & 31u) == 0u && uget(fail) != 0u) return false;
  }
}

// ---- workgroup barriers over LDS only ------------------------------------------------------
// __syncthreads() carries a workgroup-scope fence over all memory, which on this target waits
// for every load in flight (s_waitcnt vmcnt(0)) -- the prefetched weights of the next phases
// included.  The phases only synchronize through LDS, so their barriers fence LDS alone and
// the weight loads stay in flight across them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// True on every thread when p holds on any thread of the workgroup (a barrier).  The four
// wave flags alternate between two slot sets, so one call's writes never meet the previous
// call's reads.
__device__ __forceinline__ bool wg_any(bool p, int* slots, int& parity) {
  const bool wave = __ballot(p) != 0ull;
  int* s = slots + 4 * parity;
  parity ^= 1;
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = wave ? 1 : 0;
  lds_barrier();
  return (s[0] | s[1] | s[2] | s[3]) != 0;
}

// ---- weights: the lane's raw 34-byte block in 9 aligned dwords (buffer loads; an offset of
// kNone reads zeros without touching memory) -------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mat_rsrc(const void* W, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(W), 0, (int)((bytes + 3u) & ~3u), 0x00020000);
}

__device__ __forceinline__ void issue_block(__amdgpu_buffer_rsrc_t rs, uint32_t off, RawBlock& r) {
  const uint32_t o4 = off & ~3u;
  const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o4, 0, 0);
  const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(o4 + 16u), 0, 0);
  r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
  r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
  r.w[8] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(o4 + 32u), 0, 0);
}

__device__ __forceinline__ float f32_at(__amdgpu_buffer_rsrc_t rs, int i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, i < 0 ? (int)kNone : i * 4, 0, 0));
}

// byte offset of block b of row `row` in a matrix of nb blocks per row (kNone when absent)
__device__ __forceinline__ uint32_t blk_off(int row, int nb, int b, bool real) {
  return real ? ((uint32_t)row * (uint32_t)nb + (uint32_t)b) * (uint32_t)kBlockBytes : kNone;
}

// element i of a Q8_0 row (y = q*d, exact)
__device__ __forceinline__ float q8_elem(const uint8_t* row, int i) {
  const uint8_t* blk = row + (size_t)(i >> 5) * kBlockBytes;
  const uint16_t d = (uint16_t)(blk[0] | (blk[1] << 8));
  return (float)(int8_t)blk[2 + (i & 31)] * lt_h2f(d);
}

// halfwave_tree_dpp on 8 values at once, level by level: the same pairing for each value, the
// cross-lane reads of the 8 values in flight together.
__device__ __forceinline__ void halfwave_tree_dpp8(float (&a)[8]) {
  float b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) b[i] = swz_xor16(a[i]);
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = a[i] + b[i];
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = a[i] + dpp_f<0x108>(a[i]);
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = a[i] + dpp_f<0x104>(a[i]);
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = a[i] + dpp_f<0x102>(a[i]);
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = a[i] + dpp_f<0x101>(a[i]);
}

// ---- the pieces of the fused GEMV prologues ---------------------------------------------
// rms_ss order (norm_softmax_from_facts.pl:49, 83-108): thread t folds x[t], x[t+256], ... by
// fma (slots past K hold 0, which leave the fold unchanged), then the pairwise tree 128..1;
// inv = rsqrt(ss/N + eps).  red: kT floats.
__device__ __forceinline__ float rms_inv4(const float (&s)[4], int K, float eps, float* red) {
  float p = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) p = fmaf(s[k], s[k], p);
  red[threadIdx.x] = p;
  lds_barrier();
  // every wave evaluates the last levels and the rsqrt itself (no second barrier)
  const int t = threadIdx.x & 63;
  const float a = red[t] + red[t + 128];
  const float b = red[t + 64] + red[t + 192];
  const float c = __shfl(wave_tree_dpp(a + b), 0, 64);
  return lt_rsqrtf(c / (float)K + eps);
}

// The normalized row y = (x*inv)*w quantized into the GEMV's activation records: thread t
// takes elements 4t .. 4t+3 (8 lanes per 32-element block; quant4 / q4_to_rec).  Every
// thread runs the group max (DPP), the ones past K on zeros that are never written.
__device__ __forceinline__ void norm_to_rec(const float* xs, const f32x4& w4, float inv, int K, uint32_t* rec) {
  const int t = threadIdx.x;
  const int e = 4 * t;
  const f32x4 x = e < K ? *(const f32x4*)(xs + e) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  QScale sc;
  const uint32_t p = quant4((x.x * inv) * w4.x, (x.y * inv) * w4.y, (x.z * inv) * w4.z, (x.w * inv) * w4.w, sc);
  q4_to_rec(p, sc.dq, t & 7, (t >> 3) < (K >> 5), rec + (t >> 3) * kRecDwords);
}

// 9 exchange words of one quantized 32-element block: 8 words of 4 quants (element 4j+i in
// byte i of word j) and the fp16 scale.  The block's 32 values sit one per lane of a
// half-wave; every lane of the wave calls this, lanes j < 9 of each half-wave return a word.
__device__ __forceinline__ uint32_t block_word(int q, uint16_t h, int lane) {
  const int j = lane < 8 ? lane : 0;
  const int base = (threadIdx.x & 32) + 4 * j;
  const uint32_t b0 = (uint32_t)__shfl(q, base, 64) & 0xFFu;
  const uint32_t b1 = (uint32_t)__shfl(q, base + 1, 64) & 0xFFu;
  const uint32_t b2 = (uint32_t)__shfl(q, base + 2, 64) & 0xFFu;
  const uint32_t b3 = (uint32_t)__shfl(q, base + 3, 64) & 0xFFu;
  const uint32_t hw = (uint32_t)__shfl((int)h, threadIdx.x & 32, 64) & 0xFFFFu;
  return lane < 8 ? (b0 | (b1 << 8) | (b2 << 16) | (b3 << 24)) : hw;
}

// Poll the 9 exchange words of quantized blocks (thread b takes block b) and write each
// block's activation record directly -- the records build_act_records makes from staged
// quants, formed here in registers: phase O dword j is quant word j-1 (0 for j = 0), phase E
// dword j joins the upper two bytes of word j-1 with the lower two of word j (words -1 and
// 8 read as 0), and both phases carry the fp16 scale widened to fp32.  No barrier inside.
__device__ __forceinline__ bool poll_blocks_to_rec(const uint64_t* X, int nb, uint32_t tag, const uint32_t* fail,
                                                   uint32_t* rec) {
  bool ok = true;
  for (int b = threadIdx.x; b < nb; b += kT) {
    uint32_t w[9];
    const uint64_t* p = X + b * 9;
    uint32_t spins = 0;
    for (;;) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < 9; j++) {
        const uint64_t x = xget(p + j);
        w[j] = (uint32_t)x;
        all &= (uint32_t)(x >> 32) == tag;
      }
      if (all) break;
      if (++spins >= kSpin || ((spins & 31u) == 0u && uget(fail) != 0u)) {
        ok = false;
        break;
      }
    }
    uint32_t* r = rec + b * kRecDwords;
    const uint32_t xd = __builtin_bit_cast(uint32_t, lt_h2f((uint16_t)w[8]));
#pragma unroll
    for (int j = 0; j < 9; j++) {
      const uint32_t lo = j > 0 ? w[j - 1] : 0u;
      const uint32_t hi = j < 8 ? w[j] : 0u;
      r[j] = __builtin_amdgcn_perm(hi, lo, 0x05040302u);
      r[kRecPhase + j] = lo;
    }
    r[9] = xd;
    r[kRecPhase + 9] = xd;
  }
  return ok;
}

// ---- LDS ----------------------------------------------------------------------------------
// The first kLdsSlots bytes hold wg_any's flags; each role's layout follows.
constexpr int kLdsSlots = 64;
// GEMV roles (phases A, C, D, E): x, the norm tree, activation records, staged quants, rows.
constexpr int kLdsX = 0;                                   // float [kMaxE]
constexpr int kLdsRed = kLdsX + kMaxE * 4;                 // float [kT + 16]
constexpr int kLdsRec = kLdsRed + (kT + 16) * 4;           // uint32 [kMaxNbF][kRecDwords]
constexpr int kLdsSxq = kLdsRec + kMaxNbF * kRecDwords * 4;   // int8 [kMaxF]
constexpr int kLdsSxd = kLdsSxq + kMaxF;                   // fp16 [kMaxNbF]
constexpr int kLdsRow = kLdsSxd + kMaxNbF * 2;             // float [kGuRows]
constexpr int kLdsGemv = kLdsRow + kGuRows * 4;
static_assert(kLdsRec % 16 == 0 && kLdsSxq % 16 == 0, "LDS alignment");

// Attention (phase B; its workgroups have no GEMV role): scores/exps [nmax], q [64],
// wave maxima [4], then K rows padded by 16 bytes [nmax], V rows [nmax].
template <bool kF16>
struct AttnLds {
  static constexpr int kEsz = kF16 ? 2 : 4;
  static constexpr int kRow = kHd * kEsz;          // bytes of one cache row of one KV group
  static constexpr int kKRow = kRow + 16;          // the pad puts a wave's rows on distinct banks
  // V is staged transposed, one row of nmax positions per head dim, so a lane reads 8
  // positions of its dim in one 16-byte read; the 16-byte pad puts the 16 lanes of a read
  // phase on distinct banks (nmax is a multiple of 64)
  static __host__ __device__ int vt_pitch(int nmax) { return nmax * kEsz + 16; }
  static __host__ __device__ int k_off(int nmax) { return nmax * 4 + kHd * 4 + 32; }
  static __host__ __device__ int v_off(int nmax) { return k_off(nmax) + nmax * kKRow; }
  static __host__ __device__ int bytes(int nmax) { return kLdsSlots + v_off(nmax) + kHd * vt_pitch(nmax); }
};

template <bool kF16>
__device__ __forceinline__ float kv_at(const uint8_t* p) {
  if constexpr (kF16) return lt_h2f(*(const uint16_t*)p);
  else return *(const float*)p;
}

// ---- phase B: one query head per workgroup, every layer ---------------------------------
template <bool kF16>
__device__ __forceinline__ bool attn_worker(const StepParams& P, uint8_t* smem, int head, uint32_t tag) {
  using AL = AttnLds<kF16>;
  int* slots = (int*)smem;   // wg_any's flags
  int par = 0;
  smem += kLdsSlots;
  const int t = threadIdx.x;
  const int lane = t & 31;
  const int nh = P.nh, nkv = P.nkv, NL = P.n_layers;
  const uint32_t* fail = &P.st->fail;
  for (int l = 0; l < NL; l++) {
    const lt_step_layer Ly = layer_desc(P.layers, l);
    uint64_t* X = P.xw + (size_t)l * P.lstride;
    uint64_t* XA = X + P.offA;
    uint64_t* XB = X + P.offB;
    const int L = iget(P.lens + l);
    const bool lvalid = L >= 0 && L < P.maxt;
    lds_barrier();   // wave 0 may still be reading the previous layer's V rows and exps
    float* ss = (float*)smem;                              // [nmax] scores, then exps
    float* sq = ss + P.nmax;                               // [64]
    float* smx = sq + kHd;                                 // [4] wave maxima, then [1] Z
    uint8_t* sK = smem + AL::k_off(P.nmax);
    uint8_t* sV = smem + AL::v_off(P.nmax);                // [hd][vpitch]: V transposed
    const int vpitch = AL::vt_pitch(P.nmax);
    const int g = head / (nh / nkv);
    const int n = L + 1;
    const bool ok_len = lvalid && n <= P.nmax;
    if (t == 0 && !ok_len && P.err) *P.err = kErrLength;
    // the cached rows [0, L) of group g into LDS (16-byte units, 8 per thread in flight)
    {
      constexpr int kUR = AL::kRow / 16;
      const int units = ok_len ? L * kUR : 0;
      const uint8_t* kc = (const uint8_t*)Ly.kc + (size_t)g * AL::kRow;
      const uint8_t* vc = (const uint8_t*)Ly.vc + (size_t)g * AL::kRow;
      const size_t pitch = (size_t)nkv * AL::kRow;
      for (int base = 0; base < units; base += kT * 8) {
        u32x4 kk[8], vv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int i = base + t + kT * j;
          if (i < units) {
            const int r = i / kUR, u = i - r * kUR;
            kk[j] = *(const u32x4*)(kc + r * pitch + u * 16);
            vv[j] = *(const u32x4*)(vc + r * pitch + u * 16);
          }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int i = base + t + kT * j;
          if (i < units) {
            const int r = i / kUR, u = i - r * kUR;
            *(u32x4*)(sK + r * AL::kKRow + u * 16) = kk[j];
            // V transposed: the unit's dims each to their own row, at position r
            const uint32_t a[4] = {vv[j].x, vv[j].y, vv[j].z, vv[j].w};
            constexpr int kPer = 16 / AL::kEsz;
#pragma unroll
            for (int k = 0; k < kPer; k++) {
              uint8_t* dst = sV + (u * kPer + k) * vpitch + r * AL::kEsz;
              if constexpr (kF16) *(uint16_t*)dst = (uint16_t)(a[k >> 1] >> (16 * (k & 1)));
              else *(uint32_t*)dst = a[k];
            }
          }
        }
      }
    }
    // q of the head, k and v of the group (the new row, rounded through the cache's type)
    uint32_t qv = 0u;
    bool ok = true;
    if (t < 3 * kHd) {
      const int part = t / kHd, d = t - part * kHd;
      const int hh = part == 0 ? head : (part == 1 ? nh + g : nh + nkv + g);
      const int wi = (hh * 8 + (d & 31) / 4) * 8 + (d & 3) + (d >= kHd / 2 ? 4 : 0);
      ok = xpoll1(XA + wi, tag, fail, qv);
    }
    if (wg_any(!ok, slots, par)) return false;
    if (t < kHd) {
      sq[t] = __uint_as_float(qv);
    } else if (t < 3 * kHd && ok_len) {
      const int d = (t - kHd) & (kHd - 1);
      uint8_t* dst = t < 2 * kHd ? sK + L * AL::kKRow + d * AL::kEsz : sV + d * vpitch + L * AL::kEsz;
      if constexpr (kF16) *(uint16_t*)dst = lt_f2h(__uint_as_float(qv));
      else *(float*)dst = __uint_as_float(qv);
    }
    lds_barrier();
    // scores: position p on thread p % 256, the sequential fma chain over the head dims
    // times scale; then the maximum (order-free)
    float m = -1e30f;
    if (ok_len) {
      float q[kHd];
#pragma unroll
      for (int i = 0; i < kHd; i += 4) {
        const f32x4 q4 = *(const f32x4*)(sq + i);
        q[i] = q4.x; q[i + 1] = q4.y; q[i + 2] = q4.z; q[i + 3] = q4.w;
      }
      for (int p = t; p < n; p += kT) {
        const u32x4* kr = (const u32x4*)(sK + p * AL::kKRow);
        // the whole K row's reads in flight before the first fma (read unit by unit, each
        // later unit waits out its own LDS round trip)
        u32x4 krow[AL::kRow / 16];
#pragma unroll
        for (int u = 0; u < AL::kRow / 16; u++) krow[u] = kr[u];
        asm volatile("" ::: "memory");
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < AL::kRow / 16; u++) {
          const u32x4 k4 = krow[u];
          const uint32_t a[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
          for (int c = 0; c < 4; c++) {
            if constexpr (kF16) {
              acc = fmaf(q[8 * u + 2 * c], lt_h2f((uint16_t)(a[c] & 0xFFFFu)), acc);
              acc = fmaf(q[8 * u + 2 * c + 1], lt_h2f((uint16_t)(a[c] >> 16)), acc);
            } else {
              acc = fmaf(q[4 * u + c], __uint_as_float(a[c]), acc);
            }
          }
        }
        const float s = acc * P.scale;
        ss[p] = s;
        m = fmaxf(m, s);
      }
    }
    m = wave_max(m);
    if ((t & 63) == 0) smx[t >> 6] = m;
    lds_barrier();
    m = fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3]));
    if (ok_len)
      for (int p = t; p < n; p += kT) ss[p] = lt_expf_sel(ss[p] - m);
    lds_barrier();
    // Z on wave 1 while wave 0 runs the O chains: lane l folds the exps of positions l, l+64,
    // ... in order, then the 64-lane tree
    if (t >= 64 && t < 128) {
      float z = 0.0f;
      if (ok_len)
        for (int p = t - 64; p < n; p += 64) z = z + ss[p];
      z = wave_tree_dpp(z);
      if (t == 64) smx[4] = z;
    }
    float o = 0.0f;
    if (t < 64) {
      // O: lane d's sequential fma chain over the positions
      if (ok_len) {
        // groups of 8 positions: the exps in two 16-byte reads, the lane's V values in one
        // (fp16) or two (fp32) from the transposed rows; two groups' reads in flight ahead of
        // the chain (a wave alone on its SIMD would otherwise wait out an LDS round trip per
        // group).  V stays raw cache bits until its fma; a look-ahead past the last group
        // re-reads that group and is discarded.
        const uint8_t* vrow = sV + t * vpitch;
        const int ng = n >> 3;
        struct Grp {
          f32x4 e0, e1;
          u32x4 v0, v1;
        };
        auto rd = [&](int gi, Grp& g) {
          const int p0 = (gi < ng ? gi : ng - 1) * 8;
          g.e0 = *(const f32x4*)(ss + p0);
          g.e1 = *(const f32x4*)(ss + p0 + 4);
          g.v0 = *(const u32x4*)(vrow + p0 * AL::kEsz);
          if constexpr (!kF16) g.v1 = *(const u32x4*)(vrow + p0 * AL::kEsz + 16);
        };
        auto fold8 = [&](const Grp& g) {
          const float e[8] = {g.e0.x, g.e0.y, g.e0.z, g.e0.w, g.e1.x, g.e1.y, g.e1.z, g.e1.w};
          const uint32_t v[8] = {g.v0.x, g.v0.y, g.v0.z, g.v0.w, g.v1.x, g.v1.y, g.v1.z, g.v1.w};
#pragma unroll
          for (int j = 0; j < 8; j++) {
            if constexpr (kF16) o = fmaf(e[j], lt_h2f((uint16_t)(v[j >> 1] >> (16 * (j & 1)))), o);
            else o = fmaf(e[j], __uint_as_float(v[j]), o);
          }
        };
        // kRot register groups in rotation (kRot - 1 groups' reads in flight).  Whole
        // rotations run without an exit (an exit inside one makes every fold wait for all
        // reads in flight), then the last ng % kRot groups, already read into slots 0, 1, 2
        constexpr int kRot = 4;
        if (ng > 0) {
          Grp g[kRot];
#pragma unroll
          for (int k = 0; k < kRot - 1; k++) rd(k, g[k]);
          const int ngf = ng & ~(kRot - 1);
#pragma unroll 1
          for (int gi = 0; gi < ngf; gi += kRot) {
#pragma unroll
            for (int k = 0; k < kRot; k++) {
              rd(gi + k + kRot - 1, g[(k + kRot - 1) % kRot]);
              // the chain value through an empty statement after the reads: the fold
              // cannot be hoisted above them, so kRot - 1 groups stay in flight
              asm volatile("" : "+v"(o) : : "memory");
              fold8(g[k]);
            }
          }
          const int rem = ng - ngf;
          static_assert(kRot == 4, "the tail takes slots 0 .. 2");
          if (rem > 0) fold8(g[0]);
          if (rem > 1) fold8(g[1]);
          if (rem > 2) fold8(g[2]);
        }
        for (int p = ng * 8; p < n; p++) o = fmaf(ss[p], kv_at<kF16>(vrow + p * AL::kEsz), o);
      }
    }
    lds_barrier();
    if (t < 64) {
      const float z = smx[4];
      const float out = ok_len ? o / z : 0.0f;
      // quantized for the O projection: the head's two 32-element blocks, one per half-wave
      const QScale sc = q8_scale(halfwave_max(fabsf(out)));
      const uint32_t word = block_word(q8_quant(out, sc), sc.h, lane);
      if (lane < 9) xput(XB + (2 * head + (t >> 5)) * 9 + lane, tag, word);
    }
  }
  return true;
}

// ---- phases A, C, D, E: the GEMV units of every layer ----------------------------------------
template <bool kF16>
__device__ __forceinline__ bool gemv_worker(const StepParams& P, uint8_t* smem, int w, uint32_t tag) {
  int* slots = (int*)smem;   // wg_any's flags
  int par = 0;
  smem += kLdsSlots;
  const int t = threadIdx.x;
  const int hw = t >> 5;
  const int lane = t & 31;
  const int G = gridDim.x;
  const int E = P.E, F = P.F, nh = P.nh, nkv = P.nkv, NL = P.n_layers;
  const int nbE = E >> 5, nbO = (nh * kHd) >> 5, nbF = F >> 5;
  const int nA = (nh + 2 * nkv) * kHd / 8, nC = E / 8, nD = F / 32, nE = E / 8;
  const uint32_t* fail = &P.st->fail;

  // roles: workgroups 0 .. nh-1 attend one query head each; the others take the GEMV units,
  // A and D counted from the bottom, C and E from the top (so the heavy D and E units sit on
  // different workgroups as far as they can)
  const int wr = w - nh;
  const int rr = G - 1 - w;
  const int uA = wr >= 0 && wr < nA ? wr : -1;
  const int uD = wr >= 0 && wr < nD ? wr : -1;
  const int uC = wr >= 0 && rr < nC ? rr : -1;
  const int uE = wr >= 0 && rr < nE ? rr : -1;

  float* xs = (float*)(smem + kLdsX);
  float* red = (float*)(smem + kLdsRed);
  uint32_t* rec = (uint32_t*)(smem + kLdsRec);
  uint8_t* sxq = smem + kLdsSxq;
  uint16_t* sxd = (uint16_t*)(smem + kLdsSxd);
  float* srow = (float*)(smem + kLdsRow);


  // layer inputs at layer 0: the embedding row of the device token (or the host row)
  int tok = 0;
  bool bad_tok = false;
  if (P.emb && (uA >= 0 || uC >= 0)) {
    tok = *P.tok;
    bad_tok = tok < 0 || tok >= P.vocab;
  }
  const uint8_t* emb_row = P.emb ? P.emb + (size_t)(bad_tok ? 0 : tok) * nbE * kBlockBytes : nullptr;
  auto x0_elem = [&](int i) -> float {
    if (P.emb) return bad_tok ? 0.0f : q8_elem(emb_row, i);
    return P.x_in[i];
  };
  if (bad_tok && uA == 0 && t == 0 && P.err) *P.err = 1;

  // prefetched weights: this workgroup's QKV row, O row, 8 gate|up rows, down row
  RawBlock wA, wC, wD[8], wE[kDownItems];
  const int arow = uA >= 0 ? (uA >> 3) * kHd + ((hw & 4) ? kHd / 2 : 0) + (uA & 7) * 4 + (hw & 3) : 0;
  auto issue_A = [&](int l) {
    const lt_step_layer Ly = layer_desc(P.layers, l);
    const __amdgpu_buffer_rsrc_t rs = mat_rsrc(Ly.wqkv, (uint32_t)(nA * 8) * (uint32_t)nbE * kBlockBytes);
    issue_block(rs, blk_off(arow, nbE, lane, lane < nbE), wA);
  };
  auto issue_CDE = [&](int l) {
    const lt_step_layer Ly = layer_desc(P.layers, l);
    if (uC >= 0) {
      const __amdgpu_buffer_rsrc_t rs = mat_rsrc(Ly.wo, (uint32_t)E * (uint32_t)nbO * kBlockBytes);
      issue_block(rs, blk_off(uC * 8 + hw, nbO, lane, lane < nbO), wC);
    }
    if (uD >= 0) {
      const __amdgpu_buffer_rsrc_t rs = mat_rsrc(Ly.wgu, (uint32_t)(2 * F) * (uint32_t)nbE * kBlockBytes);
#pragma unroll
      for (int i = 0; i < 8; i++) issue_block(rs, blk_off(uD * kGuRows + hw + 8 * i, nbE, lane, lane < nbE), wD[i]);
    }
    if (uE >= 0) {
      const __amdgpu_buffer_rsrc_t rs = mat_rsrc(Ly.wdown, (uint32_t)E * (uint32_t)nbF * kBlockBytes);
#pragma unroll
      for (int k = 0; k < kDownItems; k++)
        issue_block(rs, blk_off(uE * 8 + hw, nbF, lane + 32 * k, lane + 32 * k < nbF), wE[k]);
    }
  };
  if (uA >= 0) issue_A(0);

  for (int l = 0; l < NL; l++) {
    const lt_step_layer Ly = layer_desc(P.layers, l);
    uint64_t* X = P.xw + (size_t)l * P.lstride;
    uint64_t* XA = X + P.offA;
    uint64_t* XB = X + P.offB;
    uint64_t* XC = X + P.offC;
    uint64_t* XD = X + P.offD;
    uint64_t* XE = X + P.offE;
    const uint64_t* XEp = P.xw + (size_t)(l > 0 ? l - 1 : 0) * P.lstride + P.offE;
    const int L = uA >= 0 ? iget(P.lens + l) : 0;
    const bool lvalid = L >= 0 && L < P.maxt;

    // ---------------- A: rmsnorm -> quant -> QKV + bias -> RoPE -> KV append ----------------
    if (uA >= 0) {
      const int ahead = uA >> 3, ac = uA & 7;
      const __amdgpu_buffer_rsrc_t rb = mat_rsrc(Ly.bqkv, Ly.bqkv ? (uint32_t)(nA * 8) * 4u : 0u);
      const float bias = f32_at(rb, lane == 0 ? arow : -1);
      const __amdgpu_buffer_rsrc_t rn = mat_rsrc(Ly.attn_norm, (uint32_t)E * 4u);
      const f32x4 nw4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rn, t * 16, 0, 0));
      // the rotation of pair j = 4*ac + t at position L (k_rope's arithmetic), under the poll
      float sn = 0.0f, cs = 1.0f;
      if (t < 8) lt_sincosf((float)L * P.freqs[ac * 4 + (t & 3)], &sn, &cs);
      float xv[4];
      bool ok = true;
      if (l == 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = t + kT * k < E ? x0_elem(t + kT * k) : 0.0f;
      } else {
        uint32_t v[4];
        ok = xpoll<4>(XEp, E, tag, fail, v);
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = __uint_as_float(v[k]);
      }
      if (wg_any(!ok, slots, par)) return false;
      // x into LDS before the norm's reduction: its barrier also publishes xs (the last
      // reads of xs, the previous phase's norm_to_rec, ended at a barrier since)
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (t + kT * k < E) xs[t + kT * k] = xv[k];
      const float inv = rms_inv4(xv, E, P.eps, red);
      norm_to_rec(xs, nw4, inv, E, rec);
      lds_barrier();
      // the record's reads all in flight before the first dot (fold_raw, read by read, waits
      // out one LDS round trip per two dots)
      const bool oddA = (blk_off(arow, nbE, lane, true) & 2u) != 0;
      uint32_t ra[10];
      rec_regs(rec + (lane < nbE ? lane : 0) * kRecDwords, oddA, ra);
      asm volatile("" ::: "memory");
      const float folded = fold_regs(wA, oddA, ra, 0.0f);
      const float rv = halfwave_tree_dpp(lane < nbE ? folded : 0.0f);
      if (lane == 0) srow[hw] = Ly.bqkv ? rv + bias : rv;
      lds_barrier();
      if (t < 8) {
        // thread i takes pair i & 3 (rows j and j + hd/2) and keeps its first (i < 4) or
        // second output: the unit's 8 words go out in one store instruction
        const int i = t & 3;
        const int j = ac * 4 + i;
        float x1 = srow[i], x2 = srow[i + 4];
        if (ahead < nh + nkv) {   // q and k heads rotate, v heads pass
          const float y1 = fmaf(x1, cs, -(x2 * sn));
          const float y2 = fmaf(x1, sn, x2 * cs);
          x1 = y1;
          x2 = y2;
        }
        const float y = t < 4 ? x1 : x2;
        xput(XA + uA * 8 + t, tag, __float_as_uint(y));
        if (ahead >= nh && lvalid) {   // the k and v rows into the caches at row L
          const bool isv = ahead >= nh + nkv;
          const size_t off = (size_t)L * nkv * kHd + (size_t)(ahead - nh - (isv ? nkv : 0)) * kHd + j +
                             (t < 4 ? 0 : kHd / 2);
          void* c = isv ? Ly.vc : Ly.kc;
          if constexpr (kF16) ((uint16_t*)c)[off] = lt_f2h(y);
          else ((float*)c)[off] = y;
        }
      }
    }
    // this layer's C, D and E weights, after phase A's arithmetic: a load issued earlier would
    // make the compiler's conservative waits in that arithmetic wait for it
    issue_CDE(l);

    // ---------------- C: O GEMV + residual ----------------
    if (uC >= 0) {
      const int row = uC * 8 + hw;
      lds_barrier();   // every wave is done reading the previous phase's records
      bool ok = poll_blocks_to_rec(XB, nbO, tag, fail, rec);
      float xres = 0.0f;
      if (lane == 0) {
        if (l == 0) {
          xres = x0_elem(row);
        } else {
          uint32_t r;
          ok = ok && xpoll1(XEp + row, tag, fail, r);
          xres = __uint_as_float(r);
        }
      }
      if (wg_any(!ok, slots, par)) return false;
      const bool oddC = (blk_off(row, nbO, lane, true) & 2u) != 0;
      uint32_t ra[10];
      rec_regs(rec + (lane < nbO ? lane : 0) * kRecDwords, oddC, ra);
      asm volatile("" ::: "memory");
      const float folded = fold_regs(wC, oddC, ra, 0.0f);
      const float rv = halfwave_tree_dpp(lane < nbO ? folded : 0.0f);
      // the unit's 8 rows leave in one store instruction (a word per half-wave measured
      // ~0.6 us slower to exchange)
      if (lane == 0) srow[hw] = rv + xres;
      lds_barrier();
      if (t < 8) xput(XC + uC * 8 + t, tag, __float_as_uint(srow[t]));
    }
    if (uA >= 0 && l + 1 < NL) issue_A(l + 1);

    // ---------------- D: rmsnorm -> quant -> gate|up -> SiLU(g)*u -> quant ----------------
    if (uD >= 0) {
      const __amdgpu_buffer_rsrc_t rn = mat_rsrc(Ly.ffn_norm, (uint32_t)E * 4u);
      const f32x4 nw4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rn, t * 16, 0, 0));
      uint32_t v[4];
      const bool ok = xpoll<4>(XC, E, tag, fail, v);
      if (wg_any(!ok, slots, par)) return false;
      float xv[4];
#pragma unroll
      for (int k = 0; k < 4; k++) xv[k] = __uint_as_float(v[k]);
      // x into LDS before the norm's reduction: its barrier also publishes xs (the last
      // reads of xs, the previous phase's norm_to_rec, ended at a barrier since)
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (t + kT * k < E) xs[t + kT * k] = xv[k];
      const float inv = rms_inv4(xv, E, P.eps, red);
      norm_to_rec(xs, nw4, inv, E, rec);
      lds_barrier();
      const uint32_t* ra = rec + (lane < nbE ? lane : 0) * kRecDwords;
      // the 8 rows' folds first, then their trees level by level (one row at a time would
      // wait out each tree's cross-lane latencies in turn)
      float f[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int row = uD * kGuRows + hw + 8 * i;
        const float folded = fold_raw(wD[i], (blk_off(row, nbE, lane, true) & 2u) != 0, ra, 0.0f);
        f[i] = lane < nbE ? folded : 0.0f;
      }
      halfwave_tree_dpp8(f);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) srow[hw + 8 * i] = f[i];
      }
      lds_barrier();
      if (t < 64) {
        // rows 2j (gate j) and 2j+1 (up j): SiLU(g)*u one pair per lane of half-wave 0, then
        // k_silu_mul_quant's quantizer (the values of half-wave 1 are never stored)
        const float s = lt_silu_mul(srow[2 * lane], srow[2 * lane + 1]);
        const QScale sc = q8_scale(halfwave_max(fabsf(s)));
        const uint32_t word = block_word(q8_quant(s, sc), sc.h, lane);
        if (t < 9) xput(XD + uD * 9 + t, tag, word);
      }
    }

    // ---------------- E: down GEMV + residual ----------------
    if (uE >= 0) {
      const int row = uE * 8 + hw;
      lds_barrier();   // every wave is done reading the previous phase's records
      bool ok = poll_blocks_to_rec(XD, nbF, tag, fail, rec);
      float xres = 0.0f;
      if (lane == 0) {
        uint32_t r;
        ok = ok && xpoll1(XC + row, tag, fail, r);
        xres = __uint_as_float(r);
      }
      if (wg_any(!ok, slots, par)) return false;
      // every item's record read first (all in flight together), then the folds in block
      // order; a lane past the row's last block folds block 0's record and keeps acc (a
      // select, not a branch: the items' reads and dots interleave)
      uint32_t ra[kDownItems][10];
      bool oddE[kDownItems];
#pragma unroll
      for (int k = 0; k < kDownItems; k++) {
        const int b = lane + 32 * k;
        const int bb = b < nbF ? b : 0;
        oddE[k] = (blk_off(row, nbF, bb, true) & 2u) != 0;
        rec_regs(rec + bb * kRecDwords, oddE[k], ra[k]);
      }
      asm volatile("" ::: "memory");
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < kDownItems; k++) {
        const float f = fold_regs(wE[k], oddE[k], ra[k], acc);
        acc = lane + 32 * k < nbF ? f : acc;
      }
      const float rv = halfwave_tree_dpp(acc);
      if (lane == 0) srow[hw] = rv + xres;
      lds_barrier();
      if (t < 8) {
        const float y = srow[t];
        xput(XE + uE * 8 + t, tag, __float_as_uint(y));
        if (l == NL - 1) P.x_out[uE * 8 + t] = y;
      }
    }
  }
  return true;
}

// ---- the kernel ---------------------------------------------------------------------------
template <bool kF16>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_decode_step(StepParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int t = threadIdx.x;
  const int G = gridDim.x;
  const int NL = P.n_layers;
  const uint32_t tag = uget(&P.st->serial) + 1u;
  // the attention workgroups and the GEMV workgroups run separate code (no register of one
  // is live in the other)
  const bool ok = (int)blockIdx.x < P.nh ? attn_worker<kF16>(P, smem, blockIdx.x, tag)
                                         : gemv_worker<kF16>(P, smem, blockIdx.x, tag);
  const bool failed = !ok;
  __syncthreads();
  if (t == 0) {
    if (failed) {
      uput(&P.st->fail, 1u);
      if (P.err) *P.err = kErrTimeout;
    }
    // the last workgroup to finish advances the caches' lengths and the step serial (every
    // other workgroup has finished reading both)
    const uint32_t prev = __hip_atomic_fetch_add(&P.st->arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)G - 1u) {
      for (int l = 0; l < NL; l++) {
        const int L = iget(P.lens + l);
        if (L >= 0 && L < P.maxt) P.lens[l] = L + 1;
      }
      uput(&P.st->arrived, 0u);
      uput(&P.st->serial, tag);
    }
  }
}

// ---- host side ----------------------------------------------------------------------------
bool step_geometry_ok(int E, int F, int nh, int nkv, int hd) {
  return hd == kHd && E > 0 && E % 32 == 0 && E <= kMaxE && nh > 0 && nkv > 0 && nh % nkv == 0 &&
         nh * kHd <= kMaxE && F > 0 && F % 32 == 0 && F <= kMaxF;
}

int step_nmax(int kv_dtype, int maxt) {
  const int fixed = kLdsGemv;   // the GEMV roles' LDS (the attention region aliases it)
  (void)fixed;
  int cap = 0;
  for (int n = 64; n <= 4096; n += 64) {
    const int b = kv_dtype == LT_KV_F16 ? AttnLds<true>::bytes(n) : AttnLds<false>::bytes(n);
    if (b > kLdsMax) break;
    cap = n;
  }
  const int want = (maxt + 63) / 64 * 64;
  return want < cap ? want : cap;
}

int step_lds_bytes(int kv_dtype, int nmax) {
  const int a = kv_dtype == LT_KV_F16 ? AttnLds<true>::bytes(nmax) : AttnLds<false>::bytes(nmax);
  return a > kLdsSlots + kLdsGemv ? a : kLdsSlots + kLdsGemv;
}

// 0 when the device cannot hold the whole grid at once
int step_grid(lt_ctx* ctx, int kv_dtype, int lds) {
  int per_cu = 0;
  const hipError_t e = kv_dtype == LT_KV_F16
                           ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_step<true>, kT, lds)
                           : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_step<false>, kT, lds);
  if (e != hipSuccess || per_cu < 1 || ctx->num_cus < 1) return 0;
  return ctx->num_cus;   // one workgroup per CU
}

bool step_roles_fit(int G, int E, int F, int nh, int nkv) {
  const int gp = G - nh;
  const int nA = (nh + 2 * nkv) * kHd / 8, nC = E / 8, nD = F / 32;
  return gp > 0 && nA <= gp && nC <= gp && nD <= gp;
}

}  // namespace

extern "C" {

size_t lt_decode_step_workspace_size(int n_layers, int E, int F, int nh, int nkv, int hd) {
  if (n_layers <= 0 || !step_geometry_ok(E, F, nh, nkv, hd)) return 0;
  const XLayout x = x_layout(E, F, nh, nkv);
  return sizeof(StepState) + (size_t)n_layers * (size_t)x.lstride * 8u;
}

int lt_decode_step_max_len(lt_ctx* ctx, int n_layers, int E, int F, int nh, int nkv, int hd, int kv_dtype, int maxt) {
  if (!ctx || n_layers <= 0 || maxt <= 0 || !step_geometry_ok(E, F, nh, nkv, hd)) return 0;
  if (kv_dtype != LT_KV_F16 && kv_dtype != LT_KV_F32) return 0;
  const int nmax = step_nmax(kv_dtype, maxt);
  if (nmax <= 0) return 0;
  const int G = step_grid(ctx, kv_dtype, step_lds_bytes(kv_dtype, nmax));
  if (G <= 0 || !step_roles_fit(G, E, F, nh, nkv)) return 0;
  return nmax < maxt ? nmax : maxt;
}

int lt_decode_step(lt_ctx* ctx, const lt_step_layer* layers, int n_layers, int E, int F, int nh, int nkv, int hd,
                   float eps, float scale, const float* freqs, int* lens, int maxt, int kv_dtype, const void* emb,
                   const int* tok, int vocab, const float* x_in, float* x_out, int* err, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && layers && freqs && lens && x_out && err && ws, "lt_decode_step: null argument");
  LT_REQUIRE(n_layers > 0 && maxt > 0, "lt_decode_step: n_layers=%d maxt=%d", n_layers, maxt);
  LT_REQUIRE(step_geometry_ok(E, F, nh, nkv, hd),
             "lt_decode_step: E=%d F=%d nh=%d nkv=%d hd=%d outside the persistent step (hd 64, E and nh*hd <= 1024, "
             "F <= 5120, multiples of 32)", E, F, nh, nkv, hd);
  LT_REQUIRE(kv_dtype == LT_KV_F32 || kv_dtype == LT_KV_F16, "lt_decode_step: kv_dtype=%d", kv_dtype);
  LT_REQUIRE(emb ? (tok != nullptr && vocab > 0) : x_in != nullptr,
             "lt_decode_step: needs emb + tok + vocab, or x_in");
  LT_REQUIRE(lt_aligned(ws, 256), "lt_decode_step: workspace must be 256-byte aligned");
  const size_t need = lt_decode_step_workspace_size(n_layers, E, F, nh, nkv, hd);
  if (ws_bytes < need) return lt_fail(LT_ENOMEM, "lt_decode_step: workspace %zu < %zu bytes", ws_bytes, need);
  const int nmax = step_nmax(kv_dtype, maxt);
  const int lds = step_lds_bytes(kv_dtype, nmax);
  const int G = step_grid(ctx, kv_dtype, lds);
  LT_REQUIRE(G > 0 && step_roles_fit(G, E, F, nh, nkv),
             "lt_decode_step: the device cannot hold the step's grid (%d CUs) at once for this geometry; use the "
             "five-launch step", ctx->num_cus);
  const XLayout x = x_layout(E, F, nh, nkv);
  StepParams P{};
  P.layers = layers; P.n_layers = n_layers; P.E = E; P.F = F; P.nh = nh; P.nkv = nkv;
  P.eps = eps; P.scale = scale; P.freqs = freqs; P.lens = lens; P.maxt = maxt;
  P.emb = (const uint8_t*)emb; P.tok = tok; P.vocab = vocab; P.x_in = x_in; P.x_out = x_out; P.err = err;
  P.st = (StepState*)ws;
  P.xw = (uint64_t*)((char*)ws + sizeof(StepState));
  P.offA = x.offA; P.offB = x.offB; P.offC = x.offC; P.offD = x.offD; P.offE = x.offE; P.lstride = x.lstride;
  P.nmax = nmax;
  if (kv_dtype == LT_KV_F16)
    k_decode_step<true><<<G, kT, lds, ctx->stream>>>(P);
  else
    k_decode_step<false><<<G, kT, lds, ctx->stream>>>(P);
  return lt_check_launch("k_decode_step");
}

}  // extern "C"
