/* llamatov_hip.h -- C ABI of libllamatov_hip.so, the gfx950 (MI355X) implementation of
 * LlamaTov's Q8_0 bs=1 decode hot path.
 *
 * The reference boundary is Python ctypes -> CUDA driver API -> extern "C" kernels
 * (bpd/lib/fact_dispatch.py:36-72; launch pattern bpd/lib/dev_residency.py:558-566).
 * Each entry point below replaces one reference kernel launch (or driver call) and
 * keeps its argument meaning; the reference launcher each one replaces is cited.
 *
 * Conventions
 *  - Every function returns int: 0 = success, otherwise an LT_E* code (negative) or a
 *    positive hipError_t.  lt_last_error() returns the message of the last failure on
 *    the calling thread.
 *  - All tensor pointers are raw device pointers (from lt_malloc or any HIP allocation)
 *    unless the name says host.  Sizes are element counts.
 *  - Q8_0 weights are GGUF Q8_0 blocks, row-major [N][K/32], 34 bytes each
 *    (fp16 scale little-endian, then 32 int8), starting at a 4-byte aligned address.
 *  - Activation quant: int8 xq[K] plus fp16 scales xd[K/32] (uint16 bit patterns).
 *  - Work is enqueued on the context's stream, asynchronously; lt_sync() waits.
 *    Between lt_graph_begin and lt_graph_end the launches are recorded into a HIP
 *    graph instead of executed.
 *  - Not re-entrant per context: one host thread drives one lt_ctx.
 */
#ifndef LLAMATOV_HIP_H
#define LLAMATOV_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define LT_API __attribute__((visibility("default")))
#else
#define LT_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define LT_OK 0
#define LT_EINVAL (-1)     /* bad argument: null pointer, bad size, misalignment */
#define LT_ESTATE (-2)     /* call not valid in the current state (e.g. nested capture) */
#define LT_ENOMEM (-3)     /* workspace too small */

#define LT_KV_F32 0        /* KV cache element type: fp32 (reference DeviceKVCache, elem_bytes=4) */
#define LT_KV_F16 1        /* fp16, round-to-nearest-even on store, exact widen on load */

typedef struct lt_ctx lt_ctx;
typedef struct lt_graph lt_graph;

/* ---- runtime (replaces fact_dispatch._ctx/_libcuda and the cuMem* calls,
 *      bpd/lib/fact_dispatch.py:46-72; DevTensor bpd/lib/dev_residency.py:387-415) ---- */
LT_API int lt_version(void);
LT_API int lt_last_error(char* buf, size_t n);
LT_API int lt_device_count(int* n);
LT_API int lt_init(int device, lt_ctx** out);
LT_API int lt_free_ctx(lt_ctx* ctx);
LT_API int lt_malloc(lt_ctx* ctx, void** ptr, size_t nbytes);
LT_API int lt_free(lt_ctx* ctx, void* ptr);
LT_API int lt_memcpy_h2d(lt_ctx* ctx, void* dst, const void* host_src, size_t nbytes);
LT_API int lt_memcpy_d2h(lt_ctx* ctx, void* host_dst, const void* src, size_t nbytes);
LT_API int lt_memcpy_d2d(lt_ctx* ctx, void* dst, const void* src, size_t nbytes);
/* Stream-ordered byte fill by a kernel (capturable, unlike a memset node). */
LT_API int lt_fill_u8(lt_ctx* ctx, void* dst, uint8_t value, size_t nbytes);
LT_API int lt_sync(lt_ctx* ctx);

/* ---- op launchers -------------------------------------------------------------------- */

/* Activation quant, k_quant_q8 (bpd/lib/dev_residency.py:867-886, launcher _launch_quant
 * :891-904): per 32-block d16 = fp16(amax/127) (1.0 if amax == 0),
 * q = clamp(rint(x/float(d16)), +-127).  K % 32 == 0. */
LT_API int lt_quant_q8(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int K);

/* k_silu_mul_quant (bpd/lib/dev_residency.py:573-604, _launch_silu_quant :606-613):
 * v = (g/(1+exp(-g)))*u then lt_quant_q8's quantizer.  K % 32 == 0. */
LT_API int lt_silu_mul_quant(lt_ctx* ctx, const float* g, const float* u, int8_t* xq, uint16_t* xd, int K);

/* k_silu_mul (bpd/lib/dev_residency.py:545-551, silu_mul_dev :632-637):
 * y = (g/(1+exp(-g)))*u elementwise, n elements; y may be g or u (in place). */
LT_API int lt_silu_mul(lt_ctx* ctx, const float* g, const float* u, float* y, int n);

/* k_add (bpd/lib/dev_residency.py:552-555, add_dev :639-642): y = a + b elementwise. */
LT_API int lt_add(lt_ctx* ctx, const float* a, const float* b, float* y, int n);

/* k_rmsnorm block_row over M rows of N (norm_softmax_from_facts.pl:83-108, launcher
 * rms_norm_dev bpd/lib/dev_residency.py:746-781): 256-lane strided fma sum of squares,
 * pairwise tree, inv = rsqrt(ss/N + eps), y = (x*inv)*w.  eps is an argument here
 * (the reference bakes it into the cubin). */
LT_API int lt_rmsnorm(lt_ctx* ctx, const float* x, const float* w, float* y, int M, int N, float eps);

/* k_rms_quant (bpd/kernelgen/emitters/fused_rms_quant.pl:31-78, _launch_rms_quant
 * bpd/lib/dev_residency.py:624-629): lt_rmsnorm of one row followed by lt_quant_q8,
 * without writing the normalized row. */
LT_API int lt_rmsnorm_quant(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd,
                     int N, float eps);

/* Q8_0 GEMV, k_q8_0_gemv tiled_v4 / k_q8_0_gemv_addres tiled_v4_addres
 * (q8_0_from_facts.pl:212-253, 374-416; launchers q8_linear_dev, q8_linear_add_residual_dev,
 * q8_linear_dev_bias bpd/lib/dev_residency.py:905-1045, 1177-1193):
 *   y[n] = canonical-order sum over blocks of fma(wd*xd, isum, .)  (+ resid[n] if non-null).
 * resid doubles as the bias vector (the reference's bias fold).  K % 32 == 0. */
LT_API int lt_q8_gemv(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd,
               const float* resid, float* y, int N, int K);

/* Debug hook: per-(row, block) int32 dots isum[N][K/32] of the same kernel arithmetic. */
LT_API int lt_q8_gemv_isums(lt_ctx* ctx, const void* W, const int8_t* xq, int32_t* isum, int N, int K);

/* RoPE over nheads contiguous heads in place (k_rope, rope_from_facts.pl:40-69; fused q|k
 * launcher rope_dev_qk_fused bpd/lib/dev_residency.py:722-741).  The position is read on
 * the device from *pos (the cache length before the append, so the launch is capturable).
 * freqs[hd/2] is the device inverse-frequency table from lt_rope_freqs (the reference
 * evaluates powf(theta, -2j/hd) per thread; the table is that value rounded once). */
LT_API int lt_rope_qk(lt_ctx* ctx, float* qk, const int* pos, int nheads, int hd, const float* freqs);

/* Host helper, no GPU work: freqs[j] = theta^(-(2j)/hd), exponent formed in binary32. */
LT_API int lt_rope_freqs(int hd, float theta, float* host_freqs);

/* k_append_kv_incr (bpd/lib/dev_residency.py:303-315, DeviceKVCache.append_at_len_incr
 * :508-521): kc[*len][:] = k, vc[*len][:] = v (width = nkv*hd elements), then *len += 1.
 * kv_dtype LT_KV_F32 or LT_KV_F16 (fp16 RNE store).  maxt is the cache capacity in
 * positions; a full cache (*len >= maxt) is left unchanged (the reference does not check). */
LT_API int lt_kv_append_incr(lt_ctx* ctx, void* kc, const float* k, void* vc, const float* v,
                      int* len, int width, int maxt, int kv_dtype);

/* Decode attention over a position-major cache [t][nkv][hd] per sequence
 * (k_attn_decode_masked bpd/lib/dev_residency.py:1955-2031; split-K design
 * bpd/kernelgen/experimental/attn_decode_split.cu:14-91 with the declared order
 * bpd/lib/ir_param_axes.pl:303-341).
 *   q   [batch][nh*hd] fp32,  out [batch][nh*hd] fp32,
 *   kc, vc  [batch][maxt][nkv*hd] (kv_dtype), len[batch] device ints (valid positions).
 * nsplit == 1: the single-pass order of k_attn_decode_masked.  nsplit > 1 (<= 128):
 * split-K with contiguous ceil(L/nsplit) ranges and an ascending-split combine (a second
 * launch).  The result does not depend on maxt.  hd % 8 == 0, hd <= 256; each cache below
 * 2 GiB.  ws must hold lt_attn_workspace_size(...) bytes (0 for nsplit == 1). */
LT_API int lt_attn_decode(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                   float* out, int batch, int nh, int nkv, int hd, float scale, int maxt,
                   int nsplit, int kv_dtype, void* ws, size_t ws_bytes);
/* Bytes of split-K workspace (0 for nsplit == 1). */
LT_API size_t lt_attn_workspace_size(int batch, int nh, int hd, int nsplit);

/* lt_attn_decode without a workspace argument and without allocating: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The split-K partials live in a
 * file-scope device array of 16 MiB (one per GPU, held until the process ends), so
 * lt_attn_workspace_size(batch, nh, hd, nsplit) must be at most 16 MiB (else LT_EINVAL, nothing
 * launched).  Same results as lt_attn_decode, bit for bit.  The array is per GPU, so one
 * context per GPU may use it: the first call that needs it (nsplit > 1) claims it for its
 * context, a call from another context on that GPU is refused with LT_ESTATE (the two streams
 * would race on it), and lt_free_ctx releases it.  Calls on one context are stream-ordered. */
LT_API int lt_attn_decode_noalloc(lt_ctx* ctx, const float* q, const void* kc, const void* vc, const int* len,
                                  float* out, int batch, int nh, int nkv, int hd, float scale, int maxt,
                                  int nsplit, int kv_dtype);

/* Greedy argmax over n logits, ties to the lowest index (k_argmax_s1/_s2,
 * bpd/lib/dev_residency.py:225-273, argmax_dev :1074-1110).  ws must hold
 * lt_argmax_workspace_size() bytes.  out is a device int. */
LT_API int lt_argmax(lt_ctx* ctx, const float* x, int n, int* out, void* ws, size_t ws_bytes);
LT_API size_t lt_argmax_workspace_size(void);

/* lt_argmax that also appends the winner to a device token history: hist[*count] = id,
 * *count += 1 while *count < cap.  Lets a captured decode step be replayed back to back
 * (greedy decoding needs no host round trip per token; the reference reads each id back,
 * GraphRunner.replay_token bpd/lib/dev_residency.py:1795-1818). */
LT_API int lt_argmax_record(lt_ctx* ctx, const float* x, int n, int* out, int* hist, int* count, int cap,
                     void* ws, size_t ws_bytes);

/* Embedding row of the device token id *tok from Q8_0 token_embd [vocab][E/32]:
 * x = q*d (replaces the host gather emb.T[tok] + cuMemcpyHtoD into _RESID_IN,
 * bpd/lib/dev_residency.py:1357-1358, 1806-1809).  Rejects *tok outside [0, vocab)
 * by writing zeros and setting *err (device int, may be null) to 1. */
LT_API int lt_embed_q8(lt_ctx* ctx, const void* emb, const int* tok, float* x, int E, int vocab, int* err);

/* ---- fused decode-step launchers --------------------------------------------------------
 * Each one is a chain of the reference's per-op launches fused into one kernel with the
 * arithmetic of each op unchanged (every output bit equals the per-op chain's).  A replayed
 * graph node costs ~1.5 us on MI355X, so the step uses five launches per layer instead of
 * thirteen.  Every workgroup quantizes the activation into its own LDS (the prologue). */

/* rms_norm_dev -> quant -> k_q8_0_gemv_addres: q8_linear_dev with rms_src
 * (bpd/lib/dev_residency.py:905-985 with _launch_rms_quant :624-629, the QKV launch of
 * forward_pass_resident :1380-1395 with the bias fold of q8_linear_dev_bias :1177-1193).
 * y = Q8GEMV(W, quant(rmsnorm(x)*nw)) (+ resid[n] if non-null).  K % 32 == 0, K <= 16384. */
LT_API int lt_q8_gemv_rms(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                          const float* resid, float* y, int N, int K);

/* lt_q8_gemv_rms on the embedding row of the device token *tok (Q8_0 token_embd
 * [vocab][K/32]; replaces the host gather + cuMemcpyHtoD into _RESID_IN,
 * bpd/lib/dev_residency.py:1357-1358, 1806-1809).  Workgroup 0 also stores the row into
 * x_out (the layer's residual).  A token outside [0, vocab) gives a zero row and sets
 * *err = 1 (err may be null).  K <= 8192. */
LT_API int lt_q8_gemv_embed_rms(lt_ctx* ctx, const void* emb, const int* tok, int vocab, float* x_out,
                                int* err, const float* nw, float eps, const void* W, const float* resid,
                                float* y, int N, int K);

/* quant -> GEMV (+resid): the reference's k_q8_0_gemv_qfused / tiled_v4_qfused
 * (q8_0_from_facts.pl:316-365, dev_residency.py:914-930).  Used for the down projection
 * on the SiLU*up vector written by lt_q8_gemv_rms_silu. */
LT_API int lt_q8_gemv_quant(lt_ctx* ctx, const float* x, const void* W, const float* resid, float* y,
                            int N, int K);

/* O projection after lt_attn_step (q8_linear_add_residual_dev on the attention output,
 * bpd/lib/dev_residency.py:1426-1440): GEMV (+resid) of the attention output, K = nh*hd.
 * nsplit == 1: the input is the quantized attention output (xq, xd) lt_attn_step wrote.
 * nsplit > 1: the split partials in ws are first merged in ascending split order
 * (bpd/kernelgen/experimental/attn_decode_split.cu:37-91) and quantized.  If len is
 * non-null, workgroup 0 then does *len += 1 (while *len < maxt): the length bump of
 * k_append_kv_incr (:303-315), deferred to this launch because lt_attn_step's workgroups
 * all read *len. */
LT_API int lt_q8_gemv_attn_out(lt_ctx* ctx, const int8_t* xq, const uint16_t* xd, const void* ws, size_t ws_bytes,
                               int nsplit, int nh, int hd, const void* W, const float* resid, float* y, int N,
                               int K, int* len, int maxt);

/* rms_norm_dev -> quant -> gate|up GEMV -> SiLU(g)*u -> quant (gateup_fused_dev +
 * k_silu_mul_quant, bpd/lib/dev_residency.py:1321-1326, 573-604; tiled_v4_silu
 * q8_0_from_facts.pl:423-464).  Wgu holds 2F rows INTERLEAVED: row 2j = gate row j,
 * row 2j+1 = up row j.  v_j = (g_j / (1 + exp(-g_j))) * u_j is quantized like
 * lt_quant_q8 into vq[F] / vd[F/32], the input of the down projection.  F % 32 == 0. */
LT_API int lt_q8_gemv_rms_silu(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu,
                               int8_t* vq, uint16_t* vd, int F, int K);

/* rmsnorm -> quant -> gate|up GEMV -> v = SiLU(g)*u in fp32 (the chain of
 * lt_q8_gemv_rms_silu without the final quant; the down GEMV quantizes v in its prologue,
 * lt_q8_gemv_quant).  Wgu holds 2F rows interleaved (row 2j = gate j, row 2j+1 = up j);
 * v is fp32 [F], each element (g/(1+exp(-g)))*u as k_silu_mul computes it
 * (bpd/lib/dev_residency.py:545-551, gate|up GEMV :1321-1326).  F % 4 == 0. */
LT_API int lt_q8_gemv_rms_swiglu(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu,
                                 float* v, int F, int K);

/* ---- the four-launch step (no reference counterparts: each replaces a run of the
 * launches above with the same bits) ----------------------------------------------------
 * lt_q8_gemv_rms_rope_kv: lt_q8_gemv_rms (or lt_q8_gemv_embed_rms when emb is given: x is
 * then ignored and the embedding row of *tok is written to x_out) of the q|k|v rows
 * N = (nh + 2*nkv)*hd with the bias, then lt_rope_qk of the q and k heads at position *len
 * and the k and v rows written into the caches at row *len (what lt_attn_step's append
 * does), qkv receiving every row (q and k rotated).  *len is read, not changed. */
LT_API int lt_q8_gemv_rms_rope_kv(lt_ctx* ctx, const float* x, const void* emb, const int* tok, int vocab,
                                  float* x_out, int* err, const float* nw, float eps, const void* W,
                                  const float* bias, float* qkv, int K, const float* freqs, void* kc, void* vc,
                                  const int* len, int nh, int nkv, int hd, int maxt, int kv_dtype);

/* lt_attn_step's masked attention (nsplit 1) over *len + 1 cache rows for the roped q in
 * qkv, its quant, and the O GEMV + resid (y = O . Q8(attention) + resid), in one launch: every
 * workgroup recomputes the attention of all heads (k_attn_decode_masked's order,
 * bpd/lib/dev_residency.py:1955-2031) before folding its 32 O rows.  *len is read, not
 * changed.  It attends at most lt_attn_o_max_len(nh, nkv, hd, kv_dtype) rows (0: the geometry
 * is outside the kernel; hd must be 64 and nh*hd <= 1024); a launch that finds more rows
 * writes NaN rows (callers check the length on the host). */
LT_API int lt_attn_o_max_len(int nh, int nkv, int hd, int kv_dtype);
LT_API int lt_q8_gemv_attn_o(lt_ctx* ctx, const float* qkv, const void* kc, const void* vc, const int* len, int nh,
                             int nkv, int hd, float scale, int maxt, int kv_dtype, const void* W, const float* resid,
                             float* y, int N);

/* lt_q8_gemv_rms_silu, then *len += 1 (when < maxt) after the layer's attention has read it. */
LT_API int lt_q8_gemv_rms_silu_len(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu,
                                   int8_t* vq, uint16_t* vd, int F, int K, int* len, int maxt);

/* ---- the persistent step: every layer of forward_pass_resident's fully-device branch
 * (bpd/lib/dev_residency.py:1380-1477; the layers of GraphRunner's captured step, :1739-1765)
 * in one launch, with the same bits as the five- and per-op launches -----------------------
 * One workgroup per CU runs all layers.  Each layer passes through five phases (rmsnorm ->
 * quant -> QKV + bias -> RoPE -> KV append; masked attention -> quant; O + residual; rmsnorm ->
 * quant -> gate|up -> SiLU(g)*u -> quant; down + residual), their outputs exchanged between
 * workgroups through ws as words tagged with the step's serial (no fences).  Layer l reads its
 * position from lens[l], appends the new k/v rows at that row and attends lens[l] + 1 rows;
 * after the step every lens[l] < maxt is incremented.  Layer 0 takes the embedding row of *tok
 * from the Q8_0 token_embd emb [vocab][E/32] (out-of-range token: a zero row and *err = 1), or
 * x_in[E] when emb is null; the last layer's output row goes to x_out[E] (the input of
 * lt_q8_gemv_rms_argmax).  Errors found on the device go to *err: 2 = an exchange wait ran out
 * (bounded; the launch still ends), 3 = a length outside [0, lt_decode_step_max_len).
 * Geometry: hd = 64, E and nh*hd at most 1024, n_ff F at most 5120, multiples of 32.
 * lt_decode_step_max_len returns the rows the step attends at most (0: the geometry, the
 * cache type or the device's residency rules the step out); callers take the five-launch step
 * past it.  ws holds lt_decode_step_workspace_size(...) bytes, 256-byte aligned, zero-filled
 * before the plan's first step and kept across steps (a step's tag is one more than the last;
 * clear ws or its first 256 bytes' fail word after an error).  One step at a time per ws. */
typedef struct lt_step_layer {
  const float* attn_norm;   /* fp32 [E] */
  const void* wqkv;         /* Q8_0 [(nh + 2*nkv)*hd][E/32]: q, k, v rows */
  const float* bqkv;        /* fp32 [(nh + 2*nkv)*hd] or NULL */
  const void* wo;           /* Q8_0 [E][nh*hd/32] */
  const float* ffn_norm;    /* fp32 [E] */
  const void* wgu;          /* Q8_0 [2F][E/32], rows interleaved: 2j = gate j, 2j+1 = up j */
  const void* wdown;        /* Q8_0 [E][F/32] */
  void* kc;                 /* caches [maxt][nkv*hd], fp16 or fp32 per kv_dtype */
  void* vc;
} lt_step_layer;
LT_API size_t lt_decode_step_workspace_size(int n_layers, int E, int F, int nh, int nkv, int hd);
LT_API int lt_decode_step_max_len(lt_ctx* ctx, int n_layers, int E, int F, int nh, int nkv, int hd, int kv_dtype,
                                  int maxt);
/* layers: a device array of n_layers descriptors */
LT_API int lt_decode_step(lt_ctx* ctx, const lt_step_layer* layers, int n_layers, int E, int F, int nh, int nkv,
                          int hd, float eps, float scale, const float* freqs, int* lens, int maxt, int kv_dtype,
                          const void* emb, const int* tok, int vocab, const float* x_in, float* x_out, int* err,
                          void* ws, size_t ws_bytes);

/* Final norm -> quant -> vocab GEMV -> greedy argmax (_compute_folded_logits
 * bpd/lib/dev_residency.py:1596-1623 + argmax_dev :1074-1110): writes logits[N], then the
 * index of the maximum (ties to the lowest index) to *out, appending it to hist like
 * lt_argmax_record when hist is non-null.  ws holds lt_q8_gemv_argmax_workspace_size(N). */
LT_API int lt_q8_gemv_rms_argmax(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                                 float* logits, int N, int K, int* out, int* hist, int* count, int cap,
                                 void* ws, size_t ws_bytes);
LT_API size_t lt_q8_gemv_argmax_workspace_size(int N);

/* ---- the planar weight layout (no counterpart in the reference, whose GEMVs read GGUF
 * blocks; a residency choice of this library) ----------------------------------------------
 * lt_q8_to_planar repacks a Q8_0 matrix [N][K/32] of 34-byte blocks into dst (the same
 * N*K/32*34 bytes, 16-byte aligned, not overlapping src): per row and group of up to 32
 * blocks (the row's last group holds K/32 mod 32 blocks when that is not 0), the leading 16
 * quants of the group's blocks, then their trailing 16 (1024 bytes for a full group), and
 * after all N rows the fp16 scales [N][K/32].  Every load instruction of a GEMV over it reads
 * aligned, contiguous bytes.  The *_pl entry points are their namesakes above over such a
 * copy (W or Wgu planar; K % 32 == 0, else LT_EINVAL): the same arguments, arithmetic and
 * bits. */
LT_API int lt_q8_to_planar(lt_ctx* ctx, const void* src, void* dst, int N, int K);
LT_API int lt_q8_gemv_pl(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid,
                         float* y, int N, int K);
LT_API int lt_q8_gemv_rms_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                             const float* resid, float* y, int N, int K);
LT_API int lt_q8_gemv_embed_rms_pl(lt_ctx* ctx, const void* emb, const int* tok, int vocab, float* x_out, int* err,
                                   const float* nw, float eps, const void* W, const float* resid, float* y, int N,
                                   int K);
LT_API int lt_q8_gemv_attn_out_pl(lt_ctx* ctx, const int8_t* xq, const uint16_t* xd, const void* ws,
                                  size_t ws_bytes, int nsplit, int nh, int hd, const void* W, const float* resid,
                                  float* y, int N, int K, int* len, int maxt);
LT_API int lt_q8_gemv_rms_silu_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* Wgu,
                                  int8_t* vq, uint16_t* vd, int F, int K);
LT_API int lt_q8_gemv_rms_argmax_pl(lt_ctx* ctx, const float* x, const float* nw, float eps, const void* W,
                                    float* logits, int N, int K, int* out, int* hist, int* count, int cap,
                                    void* ws, size_t ws_bytes);

/* RoPE(q, k) -> KV append -> decode attention for one token of one sequence
 * (rope_dev_qk_fused + DeviceKVCache.append_at_len_incr + attn_decode_from_cache_masked,
 * bpd/lib/dev_residency.py:1396-1425).  qkv = [q (nh*hd) | k (nkv*hd) | v (nkv*hd)] before
 * RoPE (bias included); the new token is position L = *len; K/V row L is written to the
 * cache and attention runs over L+1 positions.  *len is not changed here (see
 * lt_q8_gemv_attn_out).  The output goes to out[nh*hd] fp32 (if non-null) and quantized to
 * xq[nh*hd] / xd[nh*hd/32] (if non-null; hd % 32 == 0).  nsplit > 1 (<= 128) splits the
 * context into contiguous ceil((L+1)/nsplit) ranges; each split's partials go to ws
 * (lt_attn_workspace_size(1, nh, hd, nsplit) bytes) and a second launch merges them in
 * ascending split order (the declared combine,
 * bpd/kernelgen/experimental/attn_decode_split.cu:37-91), so the output is final either
 * way; lt_q8_gemv_attn_out then takes it with nsplit = 1. */
LT_API int lt_attn_step(lt_ctx* ctx, const float* qkv, const float* freqs, void* kc, void* vc, const int* len,
                        float* out, int8_t* xq, uint16_t* xd, int nh, int nkv, int hd, float scale, int maxt,
                        int nsplit, int kv_dtype, void* ws, size_t ws_bytes);

/* ---- batched prefill -----------------------------------------------------------------
 * The reference prefills token by token through the decode GEMV and requires a batched
 * prefill to be device-uniform: bit-identical per element to the single-token path
 * (bpd/lib/dev_residency.py:1338-1356).  These launchers meet that: the prefill KV cache
 * and logits equal the token-by-token ones bit for bit. */

/* Tiled int8-MFMA Q8_0 GEMM (no reference counterpart): Y[t][n] for T tokens, each element
 * bit-identical to lt_q8_gemv on token t (exact MFMA block dots, then the GEMV's canonical
 * fp32 fold and tree).  Xq [T][K] int8, Xd [T][K/32] fp16 bits (lt_quant_q8 over T*K
 * elements), Y [T][N]; bias [N] broadcast over tokens, or resid [T][N] (at most one).
 * K % 32 == 0; the matrix must be below 2 GiB. */
LT_API int lt_q8_gemm(lt_ctx* ctx, const void* W, const int8_t* Xq, const uint16_t* Xd, const float* bias,
                      const float* resid, float* Y, int T, int N, int K);

/* lt_q8_gemm on an interleaved gate|up matrix (2F rows, row 2j = gate j, row 2j+1 = up j)
 * followed by V[t][j] = SiLU(g)*u ((g / (1 + exp(-g))) * u), V [T][F]. */
LT_API int lt_q8_gemm_silu(lt_ctx* ctx, const void* Wgu, const int8_t* Xq, const uint16_t* Xd, float* V, int T,
                           int F, int K);

/* The coalesced layouts of the prefill GEMM (no reference counterpart; same results):
 * - the tile-major copy of a Q8_0 matrix W [N][K/32] (GGUF blocks): the 1088-byte tile
 *   block (rt, b) at Wt + (rt*K/32 + b)*1088 holds the 32 quant bytes of rows 32*rt + r,
 *   r = 0..31, at 32*r, then their fp16 scales at 1024 + 2*r; rows past N are zero.
 *   lt_q8_tiles_bytes(N, K) bytes, built on the device by lt_q8_tiles (Wt 16-byte aligned);
 * - block-major activation quants: lt_quant_q8_bm writes token t's block b of x [T][K] (the
 *   lt_quant_q8 quantizer) to Xq[b][t][32] and Xd[b][t] (x 16-byte aligned, Xq 16, Xd 2). */
LT_API size_t lt_q8_tiles_bytes(int N, int K);
LT_API int lt_q8_tiles(lt_ctx* ctx, const void* W, void* Wt, int N, int K);
LT_API int lt_quant_q8_bm(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int T, int K);
/* lt_rmsnorm of T rows of x [T][N] followed by lt_quant_q8_bm of the result, in one launch
 * (the same arithmetic; the normalized rows are not stored). */
LT_API int lt_rmsnorm_quant_bm(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd, int T,
                               int N, float eps);

/* lt_q8_gemm / lt_q8_gemm_silu on those layouts (Wt from lt_q8_tiles, Xq/Xd from
 * lt_quant_q8_bm): every block's operands are contiguous runs, so each element is the same
 * bits with far fewer cache lines touched per block.  The tile copy must be below 2 GiB. */
LT_API int lt_q8_gemm_t(lt_ctx* ctx, const void* Wt, const int8_t* Xq, const uint16_t* Xd, const float* bias,
                        const float* resid, float* Y, int T, int N, int K);
LT_API int lt_q8_gemm_silu_t(lt_ctx* ctx, const void* Wgut, const int8_t* Xq, const uint16_t* Xd, float* V, int T,
                             int F, int K);
/* lt_q8_gemm_silu_t followed by lt_quant_q8_bm of its output, in one launch (no fp32 output):
 * Vq [F/32][T][32], Vd [F/32][T], bit-identical to the two calls; F a multiple of 32, Vq/Vd
 * not the input's buffers.  For launches of tens of tokens (the batched decode step: its
 * leaf-split kernel), any T accepted. */
LT_API int lt_q8_gemm_silu_quant_t(lt_ctx* ctx, const void* Wgut, const int8_t* Xq, const uint16_t* Xd, int8_t* Vq,
                                   uint16_t* Vd, int T, int F, int K);

/* The q|k|v projection of the batched decode step with RoPE and the KV append in its
 * epilogue (no reference counterpart: lt_q8_gemm_t with the bias followed by
 * lt_rope_append_seqs, in one launch; qkv [T][N] and the cache rows bit-identical to those two
 * calls).  Wt is lt_q8_tiles_rope's copy of the q|k|v matrix W [N][K/32]: the tile-major copy
 * with the rows of each q and k head of hd in the rope-pair order -- row 2j + e of the head
 * is row j + e*hd/2 of W -- so the two rows RoPE rotates together land in one lane; v rows keep
 * their places.  N = (nh + 2 nkv) hd, hd even; row t of Xq / Xd (block-major) is sequence t at
 * position len[t], its cache rows at kc / vc + t*maxt*nkv*hd elements. */
LT_API int lt_q8_tiles_rope(lt_ctx* ctx, const void* W, void* Wt, int N, int K, int nh, int nkv, int hd);
LT_API int lt_q8_gemm_rope_t(lt_ctx* ctx, const void* Wt, const int8_t* Xq, const uint16_t* Xd, int T,
                             const float* bias, float* qkv, int N, int K, const int* len, int nh, int nkv, int hd,
                             const float* freqs, void* kc, void* vc, int maxt, int kv_dtype);

/* RoPE (lt_rope_qk's arithmetic) of T rows of q|k, row t at position *pos0 + t; rows are
 * row_stride floats apart and hold nheads contiguous heads of hd. */
LT_API int lt_rope_batch(lt_ctx* ctx, float* qk, int T, int row_stride, const int* pos0, int nheads, int hd,
                         const float* freqs);

/* KV rows of T tokens into the cache at *len .. *len + T - 1 (k = src[t*src_stride + k_off ..],
 * v = src[t*src_stride + v_off ..], width elements each; fp32 or fp16 RNE).  *len is not
 * changed (lt_len_add bumps it after the attention that reads it). */
LT_API int lt_kv_append_batch(lt_ctx* ctx, void* kc, void* vc, const float* src, int src_stride, int k_off,
                              int v_off, int T, const int* len, int width, int maxt, int kv_dtype);

/* *len += T, capped at maxt. */
LT_API int lt_len_add(lt_ctx* ctx, int* len, int T, int maxt);

/* lt_rope_batch of the nh q and nkv k heads of T rows of q|k|v (row_stride floats apart),
 * then lt_kv_append_batch of their k and v (k_off = nh*hd, v_off = (nh+nkv)*hd, width
 * nkv*hd), in one launch (no reference counterpart; the same q rows and cache rows).  The
 * roped k is written to the cache only, not back into the rows.  hd even, at most 256. */
LT_API int lt_rope_append_batch(lt_ctx* ctx, float* qkv, int T, int row_stride, const int* len, int nh, int nkv,
                                int hd, const float* freqs, void* kc, void* vc, int maxt, int kv_dtype);
/* lt_len_add of len[0 .. n-1] in one launch (the prefill's per-layer lengths after its last
 * layer; no reference counterpart). */
LT_API int lt_len_add_n(lt_ctx* ctx, int* len, int n, int T, int maxt);

/* Causal attention of T query tokens of one sequence over its cache (k_attn_decode_masked's
 * order per query): query t (q + t*q_stride) attends *len0 + t + 1 positions; out [T][nh*hd].
 * nsplit and ws as lt_attn_decode with batch = T. */
LT_API int lt_attn_prefill(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc,
                           const int* len0, float* out, int T, int nh, int nkv, int hd, float scale, int maxt,
                           int nsplit, int kv_dtype, void* ws, size_t ws_bytes);

/* Embedding rows of T device token ids (lt_embed_q8 per token), x [T][E]. */
LT_API int lt_embed_q8_batch(lt_ctx* ctx, const void* emb, const int* toks, float* x, int T, int E, int vocab,
                             int* err);

/* ---- batched decode (bs > 1): B independent sequences, one token of each per step ----
 * The reference notes batched decode as future work of its device-uniform prefill
 * (bpd/lib/dev_residency.py:1344-1350); no reference signature.  The step reuses the
 * prefill's GEMM (lt_q8_gemm_t over the B rows) and these three per-sequence entries; row b
 * of every result is bit-identical to sequence b decoded alone. */

/* lt_rope_append_batch with row t the next token of sequence t: position len[t], cache rows
 * of sequence t at kc/vc + t*maxt*nkv*hd elements ([B][maxt][nkv*hd]). */
LT_API int lt_rope_append_seqs(lt_ctx* ctx, float* qkv, int B, int row_stride, const int* len, int nh, int nkv,
                               int hd, const float* freqs, void* kc, void* vc, int maxt, int kv_dtype);

/* lt_attn_decode with the query rows q_stride floats apart (the q|k|v rows of the GEMM
 * output), same results. */
LT_API int lt_attn_decode_rows(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc,
                               const int* len, float* out, int batch, int nh, int nkv, int hd, float scale, int maxt,
                               int nsplit, int kv_dtype, void* ws, size_t ws_bytes);

/* lt_attn_decode_rows writing each row's attention vector also (or only: out may be null) as
 * Q8_0 activation quants, oq [batch][nh*hd] and od [batch][nh*hd/32]: bit-identical to
 * lt_quant_q8 of the fp32 rows (the batched decode's input to the O projection; hd a multiple
 * of 32). */
LT_API int lt_attn_decode_rows_q8(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc,
                                  const int* len, float* out, int8_t* oq, uint16_t* od, int batch, int nh, int nkv,
                                  int hd, float scale, int maxt, int nsplit, int kv_dtype, void* ws,
                                  size_t ws_bytes);
/* The same with one split (no workspace) and the quants block-major, oq [nh*hd/32][batch][32]
 * and od [nh*hd/32][batch]: lt_quant_q8_bm of the fp32 rows, the tiled GEMM's input (no
 * reference counterpart: the batched step's O projection on the GEMM). */
LT_API int lt_attn_decode_rows_q8_bm(lt_ctx* ctx, const float* q, int q_stride, const void* kc, const void* vc,
                                     const int* len, float* out, int8_t* oq, uint16_t* od, int batch, int nh,
                                     int nkv, int hd, float scale, int maxt, int kv_dtype);

/* lt_rmsnorm_quant over T rows with row-major output (xq [T][N], xd [T][N/32]): row t is
 * bit-identical to lt_rmsnorm_quant of that row alone. */
LT_API int lt_rmsnorm_quant_rows(lt_ctx* ctx, const float* x, const float* w, int8_t* xq, uint16_t* xd, int T,
                                 int N, float eps);

/* The Q8_0 GEMV over T tokens at once (W [N][K/32] GGUF blocks; row-major quants xq [T][K],
 * xd [T][K/32]): each weight block read once per group of up to 8 tokens; y[t][row] is
 * bit-identical to lt_q8_gemv of token t.  epi: LT_MULTI_STORE (y [T][N], plus add[row] when
 * add is given: a bias), LT_MULTI_RESID (y = v + add[t][row]), LT_MULTI_SILU (rows 2j / 2j+1
 * are gate j / up j: y[t][j] = SiLU(g)*u, y [T][N/2]). */
#define LT_MULTI_STORE 0
#define LT_MULTI_RESID 1
#define LT_MULTI_SILU 2
LT_API int lt_q8_gemv_multi(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, int T,
                            const float* add, float* y, int N, int K, int epi);

/* lt_q8_gemv_multi (LT_MULTI_STORE with the bias) over the q|k|v rows of the next token of T
 * sequences followed by lt_rope_append_seqs of its output, in one launch: qkv [T][N] as the two
 * calls leave it (q rotated, k and v as computed), the same cache rows written; N = (nh +
 * 2 nkv) hd, hd a multiple of 8. */
LT_API int lt_q8_gemv_multi_rope(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, int T,
                                 const float* bias, float* qkv, int N, int K, const int* len, int nh, int nkv,
                                 int hd, const float* freqs, void* kc, void* vc, int maxt, int kv_dtype);

/* out[r] = argmax of row r of x [rows][n] (ties to the lowest index, as lt_argmax); with
 * hist, also hist[r][count[r]] = out[r], count[r] += 1 while < cap. */
LT_API int lt_argmax_rows(lt_ctx* ctx, const float* x, int rows, int n, int* out, int* hist, int* count, int cap);
/* lt_argmax_rows over 8 workgroups per row (no reference counterpart; the same results):
 * each takes a contiguous slice and writes its winner to ws, then one wave per row reduces
 * the slices.  ws: lt_argmax_rows_workspace_size(rows) bytes, 4-byte aligned; rows <= 65535. */
LT_API size_t lt_argmax_rows_workspace_size(int rows);
LT_API int lt_argmax_rows_ws(lt_ctx* ctx, const float* x, int rows, int n, int* out, int* hist, int* count, int cap,
                             void* ws, size_t ws_bytes);

/* ---- ggml-compatible numerics (the optional profile; the reference's CPU substrate,
 *      bpd-substrate/bench/bpd_cpu.c:4005-4446 and bpd_gemm_q8_0_cpu.c:22-258) ----
 * Quantizer: d16 = fp16_rne(amax / 127.f), id = amax != 0 ? 127.f / amax : 0,
 * q = rint(x * id) with ties to even (ggml's dispatched AVX quantize_row_q8_0).  Dot orders:
 * LT_GGML_VEC = ggml_vec_dot_q8_0_q8_0's AVX path (block pairs, 8 lanes, mul then add,
 * hsum_float_8, scalar odd tail); LT_GGML_LLAMAFILE = llamafile tinyBLAS_Q0_AVX's cell
 * (per block, 8 lanes of 4 quants, mul then add, hsum_float_8). */
#define LT_GGML_VEC 0
#define LT_GGML_LLAMAFILE 1

/* The quantizer into the engine's split layout (xq [K] int8, xd [K/32] fp16 bits), for the
 * profile's decode step.  No reference counterpart of this layout: bpd_quant_q8_0_cpu's
 * arithmetic (bpd_cpu.c:4083-4112) with the engine's activation buffers. */
LT_API int lt_quant_q8_ggml(lt_ctx* ctx, const float* x, int8_t* xq, uint16_t* xd, int K);

/* bpd_quant_q8_0_cpu(x, y, n_elements) (bpd_cpu.c:4083): n_elements fp32 -> n_elements/32
 * 34-byte Q8_0 blocks at y. */
LT_API int lt_quant_q8_0_ggml(lt_ctx* ctx, const float* x, uint8_t* y, int n_elements);

/* y[n] = dot(W row n, (xq, xd)) in ggml order `order` (+ resid[n] as one fp32 add, ggml's
 * separate ADD node), N rows of K.  The row's lane products live in LDS: K <= 40960
 * (LT_GGML_VEC) or 20480 (LT_GGML_LLAMAFILE).  xq 16-byte aligned, W 4-byte aligned. */
LT_API int lt_q8_gemv_ggml(lt_ctx* ctx, const void* W, const int8_t* xq, const uint16_t* xd, const float* resid,
                           float* y, int N, int K, int order);

/* Workspace of the two qmatmul entries: the quantized activation rows. */
LT_API size_t lt_qmatmul_q8_0_workspace_size(int M, int K);

/* bpd_qmatmul_q8_0_cpu(W_q8_0, X_f32, out, M, N, K) (bpd_cpu.c:4283-4305): X [M][K] fp32,
 * out[m][n] = vec_dot(W row n, quantized X row m).  ws 16-byte aligned. */
LT_API int lt_qmatmul_q8_0_ggml(lt_ctx* ctx, const void* W, const float* X, float* out, int M, int N, int K,
                                void* ws, size_t ws_bytes);

/* bpd_qmatmul_q8_0_llamafile_cpu(W_q8_0, X_f32, out, m_weight, m_tokens, K)
 * (bpd_cpu.c:4419-4446 with bpd_gemm_q8_0_cpu.c:209-258): out[token][row] (ldc = m_weight);
 * tokens grouped 4/2/1 as llamafile's mnpack, the llamafile cell order except for a group of
 * one token (the last when m_tokens is odd), which takes the vec_dot order -- with ggml's
 * odd-block tail, which the reference dispatcher's single-token path omits. */
LT_API int lt_qmatmul_q8_0_llamafile(lt_ctx* ctx, const void* W, const float* X, float* out, int m_weight,
                                     int m_tokens, int K, void* ws, size_t ws_bytes);

/* ---- sampling beyond greedy (temperature, top-k, top-p) on the device ----
 * The reference's device argmax (k_argmax / replay_token, bpd/lib/dev_residency.py:186-191,
 * 1795-1818) is the k = 1 case, planned there to extend to top-k/top-p/temperature; there is
 * no reference signature.  Semantics (exact, reproduced by the CPU restatement): candidates
 * ranked by logit (ties to the lower index, -0 == +0); the first k = clamp(top_k, 1,
 * LT_SAMPLE_MAX_K) of them (k = 1 when temperature <= 0 or 1/temperature is not finite, and
 * the top candidate drawn when its logit is not finite); e_i = exp((l_i - l_0) / T) with the
 * division as one multiply by the fp32 reciprocal; c_i the sequential cumulative sum; n the
 * smallest count with c_{n-1} >= top_p * c_{k-1} (all k when top_p >= 1); u from
 * Philox4x32-10 (counter {counter, 0}, key seed): u = (x0 >> 8) * 2^-24; the token is the
 * first i < n with c_i > u * c_{n-1}.  Every call advances params->counter by one. */
#define LT_SAMPLE_MAX_K 1024

/* Sampling state, kept in DEVICE memory (8-byte aligned): the host may rewrite it between
 * launches or graph replays; the kernel reads it and advances counter. */
typedef struct lt_sample_params {
  float temperature;
  int top_k;
  float top_p;
  int reserved;
  unsigned long long seed;
  unsigned long long counter;
} lt_sample_params;

/* Workspace of lt_sample for a vocabulary of V (0 when V is outside 1 .. 262144). */
LT_API size_t lt_sample_workspace_size(int V);

/* Draw one token from logits[V] into *out_tok; with hist, also append it (hist[*count] = id,
 * *count += 1 while < cap), as lt_argmax_record does.  Two launches, graph-capturable. */
LT_API int lt_sample(lt_ctx* ctx, const float* logits, int V, lt_sample_params* params, int* out_tok, int* hist,
                     int* count, int cap, void* ws, size_t ws_bytes);

/* ---- numerics self-check (no reference counterpart: a diagnostic of this build) ----
 * Runs on the device and writes 4 counters to host memory: out[0] = non-NaN binary32
 * patterns whose hardware fp16 conversion (the quantizer's scale) differs from
 * round-to-nearest-even with gradual underflow (all 2^32 - 2^24 + 2 of them are tried),
 * out[1] = quantizer quotients x / dq formed without division that differ in any bit from
 * the device's IEEE division (normal quotients), out[2] = those that quantize differently,
 * out[3] = quotient cases tried (every positive finite fp16 dq, x at and around every
 * (k + 1/2) * dq for |k| <= 140).  Synchronous; 0 or an error code. */
LT_API int lt_selftest_numerics(lt_ctx* ctx, unsigned long long* out);

/* ---- graphs (replaces cuStreamBeginCapture/EndCapture/GraphInstantiate/GraphLaunch,
 *      GraphRunner.capture / replay, bpd/lib/dev_residency.py:1732-1818) ---- */
LT_API int lt_graph_begin(lt_ctx* ctx);
LT_API int lt_graph_end(lt_ctx* ctx, lt_graph** out);
LT_API int lt_graph_launch(lt_ctx* ctx, lt_graph* g);
LT_API int lt_graph_free(lt_graph* g);

/* ---- measurement: HIP events on the context's stream (replaces the reference's
 *      time.time() around cuLaunchKernel loops, bpd/kernelgen/referee/gemv_sweep.py:69-85) ---- */
LT_API int lt_event_create(lt_ctx* ctx, void** ev);
LT_API int lt_event_record(lt_ctx* ctx, void* ev);
LT_API int lt_event_elapsed_ms(void* start, void* stop, float* ms);
LT_API int lt_event_destroy(void* ev);

#ifdef __cplusplus
}
#endif

#endif /* LLAMATOV_HIP_H */
