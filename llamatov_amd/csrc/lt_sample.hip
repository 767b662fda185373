// lt_sample.hip -- sampling beyond greedy on the device: temperature, top-k and top-p (nucleus)
// over the vocab logits, with a counter-based generator, so the token loop stays on the GPU
// and inside a captured graph.  The reference's device argmax is the k = 1 case of this
// primitive and is planned to grow into it (bpd/lib/dev_residency.py:186-191, 1795-1803);
// its semantics here are the usual ones, fixed bit for bit so that a CPU restatement can
// reproduce every draw:
//
//   order       candidates rank by logit, larger first, ties to the lower index (the argmax
//               rule); -0 and +0 tie
//   top-k       the first k = clamp(top_k, 1, LT_SAMPLE_MAX_K) candidates (k = 1 when
//               temperature <= 0 or 1/temperature is not finite: greedy; a non-finite top
//               logit also draws the top candidate)
//   weights     e_i = lt_expf((l_i - l_0) * invT), invT = 1 / temperature (fp32, rounded once)
//   cumulative  c_i = c_{i-1} + e_i, sequential in rank order (c_{-1} = 0)
//   top-p       n = the smallest i + 1 with c_i >= top_p * c_{k-1} (n = k when top_p >= 1)
//   draw        u = (philox4x32_10({counter, 0, 0}, seed).x >> 8) * 2^-24 in [0, 1),
//               pick the first i < n with c_i > u * c_{n-1} (else n - 1); counter += 1
//
// Philox4x32-10 is Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as
// 1, 2, 3" (SC 2011), with its published multipliers and key increments.
//
// Two launches.  (1) k_sample_chunks: one 1024-thread workgroup per 8192 logits finds its
// chunk's top k by a 4-pass 8-bit radix select on order-preserving keys (LDS histograms;
// the crossing digit found by one wave with a shuffle scan) and compacts them in index
// order, so ties at the threshold keep the lowest indices.  (2) k_sample_final: one
// workgroup sorts the chunk survivors by (logit, -index) with a bitonic network in LDS and
// keeps the first k -- all of them when they are at most 1024; otherwise it first selects
// the global top k the same way as the chunks (a second radix select on the index resolves
// ties that straddle the threshold) and sorts those.  It evaluates the weights in parallel,
// runs the sequential cumulative sum on one thread (its inputs read in batches), and finds
// the nucleus cut and the draw as minimum indices over the threads.
#include "lt_internal.h"
#include "lt_q8_device.h"

using namespace lt;

namespace {

constexpr int kSmThreads = 1024;
constexpr int kSmWaves = kSmThreads / 64;
constexpr int kSmPer = 8;                          // logits per thread in a chunk (contiguous)
constexpr int kSmChunk = kSmThreads * kSmPer;      // 8192
constexpr int kSmMaxChunks = 32;                   // V <= 262144
constexpr int kSmMaxK = LT_SAMPLE_MAX_K;           // 1024 = kSmThreads

static_assert(kSmMaxK == kSmThreads, "one final candidate slot per thread");

// Order-preserving key of a logit: larger logit -> larger key; -0 and +0 share one key.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  if ((b << 1) == 0u) return 0x80000000u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ int sample_k(const lt_sample_params* P, int V) {
  int k = P->top_k;
  k = k < 1 ? 1 : (k > kSmMaxK ? kSmMaxK : k);
  // greedy when the temperature is not positive, or so small that 1/T is not finite (its
  // weights would be exp(0 * inf) = NaN)
  if (!(P->temperature > 0.0f) || !__builtin_isfinite(1.0f / P->temperature)) k = 1;
  return k < V ? k : V;
}

constexpr int kSmCopies = 16;    // pass-0 histogram copies (lane mod 16)
constexpr int kSmCopyStride = 257;   // rows 257 apart: equal digits of different copies in different banks

struct SmShared {
  int hist[256];
  int hist16[kSmCopies * kSmCopyStride];
  int wave_sum[kSmWaves];
  int sel_digit, sel_rem;
};

// Exclusive prefix sum of v over the workgroup's threads in thread order; *total gets the sum.
__device__ int block_excl_scan(int v, SmShared& S, int* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) S.wave_sum[wv] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSmWaves; w++) {
    const int s = S.wave_sum[w];
    before += w < wv ? s : 0;
    all += s;
  }
  __syncthreads();   // wave_sum is reused by the next scan
  *total = all;
  return before + x - v;
}

// After the histogram of this pass is complete: the digit (largest first) at which the count
// of larger-or-equal digits reaches `rem`, and the rank left inside it.  Wave 0 only; lane j
// holds digits 255-4j .. 252-4j.
__device__ void find_digit(SmShared& S, int rem) {
  const int lane = threadIdx.x & 63;
  int c[4];
#pragma unroll
  for (int q = 0; q < 4; q++) c[q] = S.hist[255 - 4 * lane - q];
  const int mine = c[0] + c[1] + c[2] + c[3];
  int x = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  int run = x - mine;   // elements with a larger digit than this lane's first
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (run < rem && run + c[q] >= rem) {
      S.sel_digit = 255 - 4 * lane - q;
      S.sel_rem = rem - run;
    }
    run += c[q];
  }
}

// Radix select over N keys per thread (those with live[j]): returns the key T of rank `rem`
// (1 = largest) among them and sets *rem_out to T's rank among the keys equal to T.
template <int N>
__device__ uint32_t radix_select(const uint32_t (&key)[N], const bool (&live)[N], int rem, SmShared& S,
                                 int* rem_out) {
  uint32_t prefix = 0, mask = 0;
  // pass 0 (the top byte: mostly the exponent, so a few digits hold most keys) counts into
  // 16 copies of the histogram, one per lane mod 16, so lanes of one atomic instruction
  // with the same digit hit different banks; the copies are then summed (integer counts:
  // the same histogram)
#pragma unroll
  for (int i = threadIdx.x; i < kSmCopies * kSmCopyStride; i += kSmThreads) S.hist16[i] = 0;
  __syncthreads();
  {
    int* h = S.hist16 + (threadIdx.x & (kSmCopies - 1)) * kSmCopyStride;
#pragma unroll
    for (int j = 0; j < N; j++)
      if (live[j]) atomicAdd(&h[key[j] >> 24], 1);
  }
  __syncthreads();
  if (threadIdx.x < 256) {
    int c = 0;
#pragma unroll
    for (int q = 0; q < kSmCopies; q++) c += S.hist16[q * kSmCopyStride + threadIdx.x];
    S.hist[threadIdx.x] = c;
  }
#pragma unroll 1
  for (int pass = 0; pass < 4; pass++) {
    const int shift = 24 - 8 * pass;
    if (pass > 0) {
      if (threadIdx.x < 256) S.hist[threadIdx.x] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < N; j++)
        if (live[j] && (key[j] & mask) == prefix) atomicAdd(&S.hist[(key[j] >> shift) & 255u], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) find_digit(S, rem);
    __syncthreads();
    prefix |= (uint32_t)S.sel_digit << shift;
    mask |= 255u << shift;
    rem = S.sel_rem;
  }
  *rem_out = rem;
  return prefix;
}

struct SmWs {
  float* val;   // [chunks][kSmMaxK]
  int* idx;     // [chunks][kSmMaxK]
  int* cnt;     // [chunks]
};

__host__ __device__ inline SmWs sm_ws_layout(void* ws, int chunks) {
  SmWs w;
  w.val = (float*)ws;
  w.idx = (int*)(w.val + (size_t)chunks * kSmMaxK);
  w.cnt = w.idx + (size_t)chunks * kSmMaxK;
  return w;
}

__global__ __launch_bounds__(kSmThreads) void k_sample_chunks(const float* __restrict__ logits, int V,
                                                             const lt_sample_params* __restrict__ P, SmWs ws) {
  __shared__ SmShared S;
  const int g = blockIdx.x;
  const int base = g * kSmChunk + threadIdx.x * kSmPer;
  const int nvalid = V - g * kSmChunk < kSmChunk ? V - g * kSmChunk : kSmChunk;
  const int kloc = sample_k(P, V) < nvalid ? sample_k(P, V) : nvalid;
  float v[kSmPer];
  uint32_t key[kSmPer];
  bool live[kSmPer];
#pragma unroll
  for (int j = 0; j < kSmPer; j++) {
    live[j] = base + j < V;
    v[j] = live[j] ? logits[base + j] : 0.0f;
    key[j] = order_key(v[j]);
  }
  int rem;
  const uint32_t T = radix_select<kSmPer>(key, live, kloc, S, &rem);
  // compaction in index order: keys above T, then the first `rem` keys equal to T
  int ngt = 0, neq = 0;
#pragma unroll
  for (int j = 0; j < kSmPer; j++) {
    ngt += live[j] && key[j] > T;
    neq += live[j] && key[j] == T;
  }
  int tot;
  const int ex = block_excl_scan(ngt | (neq << 16), S, &tot);
  int ogt = ex & 0xFFFF, oeq = ex >> 16;
  const int gt_total = kloc - rem;
  float* ov = ws.val + (size_t)g * kSmMaxK;
  int* oi = ws.idx + (size_t)g * kSmMaxK;
#pragma unroll
  for (int j = 0; j < kSmPer; j++) {
    if (!live[j]) continue;
    if (key[j] > T) {
      ov[ogt] = v[j];
      oi[ogt] = base + j;
      ogt++;
    } else if (key[j] == T) {
      if (oeq < rem) {
        ov[gt_total + oeq] = v[j];
        oi[gt_total + oeq] = base + j;
      }
      oeq++;
    }
  }
  if (threadIdx.x == 0) ws.cnt[g] = kloc;
}

// Philox4x32-10 (Salmon et al., SC 2011).
__device__ __forceinline__ uint32_t philox_x(uint64_t counter, uint64_t seed) {
  uint32_t c0 = (uint32_t)counter, c1 = (uint32_t)(counter >> 32), c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; r++) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

__global__ __launch_bounds__(kSmThreads) void k_sample_final(lt_sample_params* __restrict__ P, SmWs ws, int chunks,
                                                            int V, int* __restrict__ out, int* __restrict__ hist,
                                                            int* __restrict__ count, int cap) {
  __shared__ SmShared S;
  __shared__ unsigned long long s_key[kSmMaxK];
  __shared__ __attribute__((aligned(16))) float s_e[kSmMaxK];   // exps in rank order
  __shared__ float s_c[kSmMaxK];                                // their running sums
  const int t = threadIdx.x;
  const int kc = sample_k(P, V);   // candidates
  // the chunks' survivor counts (every load at once), then their total M
  int cnts[kSmMaxChunks];
  int M = 0;
#pragma unroll
  for (int r = 0; r < kSmMaxChunks; r++) {
    cnts[r] = r < chunks ? ws.cnt[r] : 0;
    M += cnts[r];
  }
  // Sort keys: (order key, -index) as one 64-bit value, larger first, distinct for distinct
  // candidates; padding = 0, below every candidate.  The first k of that order are the
  // selection in either path.
  int P2 = 1;
  if (M <= kSmThreads) {
    // at most one survivor per thread: thread t takes the t-th survivor in chunk order and
    // every survivor is sorted (no selection pass)
    while (P2 < M) P2 <<= 1;
    // its chunk r is the first whose running end exceeds t; `before` is that chunk's start
    int r = 0, before = 0, end = 0;
#pragma unroll
    for (int q = 0; q < kSmMaxChunks; q++) {
      end += cnts[q];
      if (end <= t) {
        r = q + 1;
        before = end;
      }
    }
    if (t < M) {
      const size_t slot = (size_t)r * kSmMaxK + (size_t)(t - before);
      s_key[t] = ((unsigned long long)order_key(ws.val[slot]) << 32) | (uint32_t)~(uint32_t)ws.idx[slot];
    } else if (t < P2) {
      s_key[t] = 0ull;
    }
    __syncthreads();
  } else {
    // candidate r of this thread: chunk r, slot t
    uint32_t key[kSmMaxChunks], nidx[kSmMaxChunks];
    bool live[kSmMaxChunks];
#pragma unroll
    for (int r = 0; r < kSmMaxChunks; r++) {
      live[r] = t < cnts[r];
      const float v = live[r] ? ws.val[(size_t)r * kSmMaxK + t] : 0.0f;
      key[r] = order_key(v);
      nidx[r] = live[r] ? ~(uint32_t)ws.idx[(size_t)r * kSmMaxK + t] : 0u;   // larger = lower index
    }
    int rem;
    const uint32_t T = radix_select<kSmMaxChunks>(key, live, kc, S, &rem);
    // keys equal to T: all of them, or (when the tie straddles rank k) the rem lowest indices
    bool eq[kSmMaxChunks];
    int neq = 0;
#pragma unroll
    for (int r = 0; r < kSmMaxChunks; r++) {
      eq[r] = live[r] && key[r] == T;
      neq += eq[r];
    }
    int eq_total;
    (void)block_excl_scan(neq, S, &eq_total);
    uint32_t NT = 0u;   // every equal key qualifies
    if (eq_total > rem) {
      int rem2;
      NT = radix_select<kSmMaxChunks>(nidx, eq, rem, S, &rem2);
    }
    int nsel = 0;
    bool sel[kSmMaxChunks];
#pragma unroll
    for (int r = 0; r < kSmMaxChunks; r++) {
      sel[r] = live[r] && (key[r] > T || (key[r] == T && nidx[r] >= NT));
      nsel += sel[r];
    }
    int total;
    int o = block_excl_scan(nsel, S, &total);
    while (P2 < kc) P2 <<= 1;
    if (t < P2) s_key[t] = 0ull;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kSmMaxChunks; r++)
      if (sel[r]) s_key[o++] = ((unsigned long long)key[r] << 32) | nidx[r];
    __syncthreads();
  }
  // The bitonic network over P2 slots, one key per thread in a register: in each stage the
  // thread with the lower index of a pair keeps the larger key in a descending block (the
  // smaller in an ascending one) and its partner the other.  Partners less than 64 apart
  // are in the same wave and trade keys by shuffles; farther ones through LDS.
  auto sort_reg = [&](unsigned long long x, int P2n) {
    for (int size = 2; size <= P2n; size <<= 1)
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        unsigned long long y;
        if (stride >= 64) {
          s_key[t] = x;
          __syncthreads();
          y = s_key[t ^ stride];
          __syncthreads();
        } else {
          y = __shfl_xor(x, stride, 64);
        }
        const bool desc = (t & size) == 0;
        const bool lower = (t & stride) == 0;
        const unsigned long long hi = x > y ? x : y, lo = x > y ? y : x;
        x = desc == lower ? hi : lo;
      }
    return x;
  };
  if (P2 <= 64) {
    if (t < 64) {
      const unsigned long long x = sort_reg(t < P2 ? s_key[t] : 0ull, P2);
      if (t < P2) s_key[t] = x;
    }
  } else {
    const unsigned long long x = sort_reg(t < P2 ? s_key[t] : 0ull, P2);
    if (t < P2) s_key[t] = x;
  }
  __syncthreads();
  // weights
  const float temp = P->temperature;
  const float invT = temp > 0.0f ? 1.0f / temp : 0.0f;
  const float l0 = key_logit((uint32_t)(s_key[0] >> 32));
  // a non-finite top logit (its differences would be inf - inf) draws greedily: the top
  // candidate; k below is the weighted count
  const int k = __builtin_isfinite(l0) ? kc : 1;
  // exps of the k candidates, zeros up to the next multiple of 16 (c + 0 = c: the sum
  // is never -0, as every e >= +0)
  if (t < ((k + 15) & ~15)) {
    float e = 0.0f;
    if (t < k) {
      const float l = key_logit((uint32_t)(s_key[t] >> 32));
      e = lt_expf_sel((l - l0) * invT);
    }
    s_e[t] = e;
  }
  if (t == 0) S.sel_digit = k;   // the nucleus size n (k when top_p >= 1)
  __syncthreads();
  const float topp = P->top_p;
  if (k > 1) {
    // c_i = c_{i-1} + e_i in rank order on one thread; the exps come in 16 at a time from
    // an array the sums are not written to, so the reads are batched ahead of the chain
    if (t == 0) {
      float c = 0.0f;
      for (int i = 0; i < k; i += 16) {
        float e[16];
#pragma unroll
        for (int j = 0; j < 16; j += 4) {
          const float4 v = *(const float4*)&s_e[i + j];
          e[j] = v.x; e[j + 1] = v.y; e[j + 2] = v.z; e[j + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
          c = c + e[j];
          s_c[i + j] = c;
        }
      }
    }
    __syncthreads();
    // n = the smallest i + 1 with c_i >= top_p * c_{k-1}: c is nondecreasing, so the first
    // such i is the minimum over the candidates that satisfy it
    if (topp < 1.0f) {
      const float thr = topp * s_c[k - 1];
      if (t < k && s_c[t] >= thr) atomicMin(&S.sel_digit, t + 1);
      __syncthreads();
    }
  }
  if (t == 0) {
    int pick = 0;
    if (k > 1) {
      const int n = S.sel_digit;
      const uint32_t x = philox_x(P->counter, P->seed);
      const float u = (float)(x >> 8) * 0x1.0p-24f;
      S.sel_rem = n - 1;   // the first i < n with c_i > u * c_{n-1}, else n - 1
      S.wave_sum[0] = __float_as_int(u * s_c[n - 1]);
    }
  }
  __syncthreads();
  if (k > 1) {
    const int n = S.sel_digit;
    const float target = __int_as_float(S.wave_sum[0]);
    if (t < n && s_c[t] > target) atomicMin(&S.sel_rem, t);
    __syncthreads();
  }
  if (t == 0) {
    const int pick = k > 1 ? S.sel_rem : 0;
    const int id = (int)~(uint32_t)s_key[pick];
    *out = id;
    P->counter = P->counter + 1ull;
    if (hist) {
      const int cn = *count;
      if (cn >= 0 && cn < cap) {
        hist[cn] = id;
        *count = cn + 1;
      }
    }
  }
}

int sm_chunks(int V) { return (V + kSmChunk - 1) / kSmChunk; }

}  // namespace

extern "C" {

size_t lt_sample_workspace_size(int V) {
  if (V <= 0 || sm_chunks(V) > kSmMaxChunks) return 0;
  return (size_t)sm_chunks(V) * (kSmMaxK * 8 + 4) + 64;
}

int lt_sample(lt_ctx* ctx, const float* logits, int V, lt_sample_params* params, int* out_tok, int* hist, int* count,
              int cap, void* ws, size_t ws_bytes) {
  LT_REQUIRE(ctx && logits && params && out_tok && ws, "lt_sample: null argument");
  LT_REQUIRE(V > 0 && sm_chunks(V) <= kSmMaxChunks, "lt_sample: V=%d (1 .. %d)", V, kSmMaxChunks * kSmChunk);
  LT_REQUIRE(!hist || (count && cap > 0), "lt_sample: a history needs count and cap > 0");
  LT_REQUIRE(lt_aligned(params, 8) && lt_aligned(ws, 16), "lt_sample: params 8-byte and ws 16-byte aligned");
  LT_REQUIRE(ws_bytes >= lt_sample_workspace_size(V), "lt_sample: workspace of %zu bytes, needs %zu", ws_bytes,
             lt_sample_workspace_size(V));
  const int chunks = sm_chunks(V);
  const SmWs w = sm_ws_layout(ws, chunks);
  k_sample_chunks<<<chunks, kSmThreads, 0, ctx->stream>>>(logits, V, params, w);
  if (int rc = lt_check_launch("k_sample_chunks")) return rc;
  k_sample_final<<<1, kSmThreads, 0, ctx->stream>>>(params, w, chunks, V, out_tok, hist, count, cap);
  return lt_check_launch("k_sample_final");
}

}  // extern "C"
