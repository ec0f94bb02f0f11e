/*
 * alpacca_amd.h - C ABI of the MI355X (gfx950) quantized linear-layer library.
 *
 * One shared library, libalpacca_amd.so, holds GGUF-quantized weight matrices
 * in HBM and runs the hot path on them: the M=1 decode matvec, the batched
 * prefill matmul and the row gather used for embedding lookups.  Every entry
 * point takes plain pointers and sizes; no PyTorch or HIP C++ types appear in
 * the signatures (a stream is passed as an opaque hipStream_t cast to void*).
 *
 * Reference seam being replaced: the Python class QuantMatrix of the Alpacca
 * engine (alpacca/qmatrix.py:64) and its native tier kernels.matvec_codes
 * (alpacca/kernels.py:89-104).  Each declaration below names the reference
 * interface it stands in for.
 *
 * Status codes: every function returns AQ_OK or one of the AQ_ERR_* codes;
 * aq_last_error() then returns a message for the calling thread.  The host
 * mirror maps AQ_ERR_VALUE -> ValueError, AQ_ERR_INDEX -> IndexError and
 * AQ_ERR_RUNTIME -> RuntimeError, the exception types the reference raises
 * (qmatrix.py:78-96, :189-191, :216-217, :236-237).
 *
 * Threading: a matrix is immutable after aq_matrix_create.  Calls on
 * different streams may run concurrently; each host thread owns its own
 * staging buffers, so concurrent calls must come from different host threads
 * (or pass device pointers, which use no staging).
 */
#ifndef ALPACCA_AMD_H
#define ALPACCA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define AQ_OK 0
#define AQ_ERR_VALUE 1   /* bad argument (ValueError)                      */
#define AQ_ERR_INDEX 2   /* row index out of range (IndexError)            */
#define AQ_ERR_RUNTIME 3 /* HIP / device failure (RuntimeError)            */

/* ---- dtype ids: the ggml tensor type ids of GGUF (alpacca/gguf.py:36-43) - */
#define AQ_Q4_0 2
#define AQ_Q4_1 3
#define AQ_Q5_0 6
#define AQ_Q5_1 7
#define AQ_Q8_0 8
#define AQ_Q4_K 12
#define AQ_Q5_K 13
#define AQ_Q6_K 14
/* Dense matrices: the reference keeps F32/F16/BF16 weights (and anything it
 * cannot quantize-matvec) as dense float32 (alpacca/model.py:269-281,
 * quants.py:517-523).  Here they stay in HBM as stored (4 or 2 bytes per
 * value), in blocks of 32 values along K (cols must be a multiple of 32),
 * and run the fp32 matvec kernel (aq_matvec; not the aq_matvec_multi /
 * aq_matvec_fused launches), the MFMA matmul and the row gather. */
#define AQ_F32 0
#define AQ_F16 1
#define AQ_BF16 30

/* ---- HBM layouts --------------------------------------------------------
 * AQ_LAYOUT_RAW:   the GGUF super-blocks verbatim (only for Q4_K and Q5_K,
 *                  whose 144/176-byte blocks keep every field 16-B aligned).
 * AQ_LAYOUT_SPLIT: each block's fields (quant payload, high bits, scales,
 *                  fp16 d) moved into separate planes, each 16-B aligned, so
 *                  that a wavefront reads every field with coalesced loads.
 *                  Lossless: a byte permutation of the same data.
 * AQ_LAYOUT_AUTO:  the layout the library measures fastest for the dtype. */
#define AQ_LAYOUT_AUTO 0
#define AQ_LAYOUT_RAW 1
#define AQ_LAYOUT_SPLIT 2

/* ---- flags for pointer arguments ---------------------------------------- */
#define AQ_IN_DEVICE 1   /* input pointer (x / X / idx) is device memory      */
#define AQ_OUT_DEVICE 2  /* output pointer (y / Y / out) is device memory     */
#define AQ_MATVEC_FP32 4 /* aq_matvec: fp32 FMA kernel instead of the default
                            integer-dot kernel (x kept as exact fp32)       */
/* aq_matvec_fused: what the kernel uses as x, and what it does with y      */
#define AQ_X_RMSNORM 8     /* x_eff = x * inv * norm_w, inv = 1/sqrt(mean(x^2)+eps) */
#define AQ_X_SWIGLU 16     /* x_eff = x / (1 + exp(-x)) * x2                    */
#define AQ_Y_ACCUMULATE 32 /* y_i += W_i x_eff instead of y_i = W_i x_eff        */
/* the rows of W_i are (gate, up) pairs: y_i[j] = silu(u[2j]) * u[2j+1] with
 * u = W_i x_eff (rows/2 outputs; rows of at most 32 lane units: K <= 2048
 * for the K-quants, K <= 1024 for the 32-element formats; one dtype) */
#define AQ_Y_SWIGLU_PAIRS 64

/* ---- matmul_t precision -------------------------------------------------- */
#define AQ_PREC_AUTO 0   /* float32 accuracy (the reference's own float32
                            matmul, qmatrix.py:196-211); BF16 is opt-in      */
#define AQ_PREC_FP32 1   /* float32 accuracy: Q4_K as exact integer weights
                            (sc*code) on fp16 MFMA with X in two fp16 pieces
                            (22 bits) and fp32 scales; other formats fp32
                            MFMA over exactly decoded weights.  The same bits
                            for any M                                        */
#define AQ_PREC_BF16 2   /* weights and X rounded to bf16, MFMA, fp32 accum.   */
#define AQ_PREC_INT8 3   /* Q8_0 only: X quantized to int8 per 32-element block
                            (d = absmax/127, q = rint(x/d)), exact int8 MFMA
                            block dots, scaled by d_x*d_w in fp32           */

typedef struct aq_matrix aq_matrix;

/* Library version string. */
const char *aq_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char *aq_last_error(void);

/* Select and initialise a HIP device for the calling thread.
 * No reference counterpart (the reference is CPU-only); the host mirror calls
 * it once before the first QuantMatrix is built. */
int aq_init(int device);

/* Number of visible HIP devices (0 on a host without a GPU). */
int aq_device_count(int *count);

/* Block geometry of a dtype: (block_elements, block_bytes, sub_block_len,
 * affine).  Replaces the lookup in QUANT_GEOMETRY (alpacca/quants.py:317-326). */
int aq_geometry(int dtype, int *block_elems, int *block_bytes, int *sub_len,
                int *affine);

/* Upload `rows` x `cols` raw GGUF blocks (row-major, blocks along cols) to
 * HBM once.  The caller keeps ownership of `blocks` and may free it (or close
 * the mmap it points into) as soon as the call returns.
 * Replaces QuantMatrix.__init__ (alpacca/qmatrix.py:77-119) including its
 * validation: AQ_ERR_VALUE for an unknown dtype, cols not a multiple of the
 * block size, or nbytes != rows*cols/block_elems*block_bytes. */
int aq_matrix_create(const void *blocks, size_t nbytes, int dtype, int64_t rows,
                     int64_t cols, int layout, aq_matrix **out);

/* Free the device copy.  Replaces QuantMatrix.__del__ (qmatrix.py:121-126). */
int aq_matrix_destroy(aq_matrix *m);

/* Shape, dtype, layout and device_bytes, the size of the matrix's one HBM
 * allocation: the GGUF blocks (RAW), or the SPLIT planes each padded to a
 * multiple of 256 bytes; never less than 256.
 * Replaces QuantMatrix.shape / storage_nbytes (qmatrix.py:130-141). */
int aq_matrix_info(const aq_matrix *m, int64_t *rows, int64_t *cols, int *dtype,
                   int *layout, size_t *device_bytes);

/* y[rows] = W x[cols], fp32 in and out, fused dequantize-and-dot.  The
 * default kernel splits each 32-element group of x into three int8 pieces
 * (24 bits relative to the group maximum) and accumulates exact int32 dot
 * products; AQ_MATVEC_FP32 selects the fp32-FMA kernel.  Any column count
 * (a multiple of the block) runs: x is staged in LDS, so rows wider than one
 * launch can stage run as column windows whose products are added in K
 * order.
 * Replaces QuantMatrix.matvec (qmatrix.py:148-171) and the fused native kernel
 * kernels.matvec_codes (kernels.py:89-104).  With a host pointer on either
 * side the call is synchronous; with AQ_IN_DEVICE|AQ_OUT_DEVICE it only
 * enqueues on `stream`. */
int aq_matvec(const aq_matrix *m, const float *x, float *y, int flags,
              void *stream);

/* y_i = W_i x for n (1..8) matrices that share x: one kernel launch whose
 * workgroups split the rows of all n matrices evenly.  The matrices must have
 * one column count and either one dtype and layout, or two dtypes of the
 * pairs (Q4_K, Q6_K), (Q5_K, Q6_K), (Q4_K, Q5_K) with the matrices of the
 * first dtype first (each dtype one layout): a Q4_K_M layer's q/k (Q4_K) and
 * v (Q6_K) in one launch.  x and every y_i are device pointers
 * (AQ_IN_DEVICE | AQ_OUT_DEVICE required) and the call only enqueues on
 * `stream`.  Wide rows run as column windows as in aq_matvec.  The
 * reference has no single call for this: its decode step
 * runs QuantMatrix.matvec once per projection on the same input
 * (alpacca/model.py:529-531 q/k/v, :549-550 gate/up); this entry point is the
 * fused form of those calls. */
int aq_matvec_multi(const aq_matrix *const *ms, int n, const float *x,
                    float *const *ys, int flags, void *stream);

/* aq_matvec_multi with the elementwise work around the decode matvecs folded
 * into the same launch: AQ_X_RMSNORM (x_eff = RMSNorm(x) * norm_w, the
 * tensor.rmsnorm before q/k/v and gate/up, model.py:528 and :548),
 * AQ_X_SWIGLU (x_eff = silu(x) * x2, the SwiGLU before ffn_down,
 * model.py:551), AQ_Y_ACCUMULATE (y_i += W_i x_eff, the residual adds of
 * model.py:546 and :552) and AQ_Y_SWIGLU_PAIRS (the SwiGLU after gate/up,
 * model.py:549-551, applied to interleaved gate/up rows in the store).  x_eff is rounded operation by operation as the
 * reference's NumPy expressions are.  Device pointers only; enqueue only.
 * Matrices as for aq_matvec_multi (two dtypes only without AQ_X_SWIGLU);
 * the outputs must not overlap x, x2 or norm_w.  AQ_X_RMSNORM needs all of x
 * in one launch: AQ_ERR_VALUE for rows wider than one launch stages (the
 * message names the limit, > 45,000 columns on gfx950).
 * The reference has no single call for these; each replaces the reference
 * calls it names plus the matvecs of aq_matvec_multi. */
int aq_matvec_fused(const aq_matrix *const *ms, int n, const float *x,
                    const float *x2, const float *norm_w, float eps,
                    float *const *ys, int flags, void *stream);

/* Y[M, rows] = X[M, cols] W^T.  Replaces QuantMatrix.matmul_t
 * (qmatrix.py:184-211); AQ_ERR_VALUE for M < 0.  `precision` is one of
 * AQ_PREC_*.  AQ_PREC_AUTO keeps float32 accuracy: the exact-integer fp16
 * kernels (weights as exact fp16 integers, X in two fp16 pieces) from 8
 * rows of X for Q4_K and Q5_K and from 64 rows for Q6_K, Q8_0, Q4_0, Q4_1,
 * Q5_0 and Q5_1 (K a multiple of 256 for the last five), K split over
 * workgroups where that fills the GPU; fewer rows on the integer decode
 * matvec with several rows of X sharing one weight stream (the accuracy of
 * aq_matvec; up to 32 rows, 63 for matrices of 2^24 weights or more), the
 * rest (dense matrices among them) on fp32 MFMA.  AQ_PREC_FP32 gives every
 * M the same bits (the batched prefill step's precision); AQ_PREC_BF16 is
 * an opt-in. */
int aq_matmul_t(const aq_matrix *m, const float *X, int64_t M, float *Y,
                int precision, int flags, void *stream);

/* The batched step's gate/up product and SwiGLU in one call, for a matrix
 * whose rows are interleaved (gate, up) pairs: Z = X W^T as aq_matmul_t,
 * then out[M, rows/2] = silu(Z[:, 2p]) * Z[:, 2p+1] rounded as
 * aq_swiglu_pairs.  Replaces the reference's gate and up matmul_t and the
 * SwiGLU after them (model.py:511-513).  Where the exact-integer fp16
 * kernel runs the product without a split of K (Q4_K and Q5_K at
 * AQ_PREC_FP32, or at AQ_PREC_AUTO when the tiles fill the GPU) the pairs
 * are formed in its store and Z is not written; otherwise Z (M x rows, the
 * caller's scratch) holds the product and the pairs kernel follows.  The
 * same bits either way.  Device pointers only (AQ_IN_DEVICE | AQ_OUT_DEVICE
 * required); enqueue only.  AQ_ERR_VALUE for an odd row count. */
int aq_matmul_t_swiglu(const aq_matrix *m, const float *X, int64_t M, float *Z, float *out,
                       int precision, int flags, void *stream);

/* out[n, cols] = decoded rows idx[0..n) of W, bit-identical to the reference
 * decoder (quants.py:498-528).  Replaces QuantMatrix.row / rows_at
 * (qmatrix.py:215-246): AQ_ERR_INDEX when an index is negative or >= rows
 * (checked on the host; device-resident indices are clamped to the valid
 * range instead, since a kernel cannot raise). */
int aq_dequant_rows(const aq_matrix *m, const int64_t *idx, int64_t n,
                    float *out, int flags, void *stream);

/* Wait for all work queued on `stream` (NULL: the default stream). */
int aq_synchronize(void *stream);

/* Free the library's scratch memory for `stream` (split-K partials, matmul
 * X pieces, decode attention partials), after the stream's queued work;
 * scratch that a HIP graph captured on the stream may still use is kept
 * until the process exits, so the graph replays unchanged.  Call it before
 * destroying a stream the library has run on.
 * Graph capture: a call that needs scratch allocates it on first use of a
 * size, and nothing is allocated while the stream is capturing.  Run each
 * such call once eagerly, at the shapes the graph will use, before capture
 * (the call then fails with AQ_ERR_RUNTIME and says so), or use
 * aq_attention_rope_noalloc.  No reference counterpart (the reference holds
 * no device memory). */
int aq_release_workspace(void *stream);

/* ==== decode step: the callers around the quantized matvec ==============
 *
 * The reference's decode step (Model._forward_np, alpacca/model.py:520-555)
 * wraps the seven matvecs of a layer in RMSNorm, rotary embeddings, the KV
 * cache, attention, SwiGLU and residual adds, and ends with a greedy argmax.
 * The entry points below run those on the device.  Every pointer is device
 * memory and every call only enqueues on `stream`, so a whole step can be
 * captured once as a HIP graph and replayed per token: the token and its
 * position live in an aq_decode_state in device memory, read and advanced by
 * the kernels themselves.
 *
 * KV cache of one layer: k_cache / v_cache are [n_kv][n_ctx][head_dim] fp32
 * (the reference keeps [n_ctx][n_kv][head_dim], model.py:368-371; a head-major
 * cache lets attention stream each head's positions contiguously).
 */

/* Device-resident state of a decode loop (caller allocates it in device
 * memory, zero-initialised).  `key` is scratch of the argmax and must be 0
 * between steps (aq_greedy_advance leaves it 0). */
typedef struct aq_decode_state {
  int64_t token;   /* token the next step embeds                             */
  uint64_t key;    /* argmax scratch                                         */
  int32_t pos;     /* position of `token`: the KV slot the step writes       */
  int32_t fed;     /* prompt tokens consumed                                 */
  int32_t count;   /* tokens chosen by argmax                                */
  int32_t done;    /* reserved, 0                                            */
} aq_decode_state;

/* out[r, :] = x[r, :] * inv_r * w with inv_r = 1/sqrt(mean(x[r, :]^2) + eps),
 * for r < rows (n elements per row).  out may equal x.
 * Replaces tensor.rmsnorm (alpacca/tensor.py:163-172). */
int aq_rmsnorm(const float *x, const float *w, int64_t rows, int64_t n,
               float eps, float *out, void *stream);

/* x += y, then out = aq_rmsnorm(x) over the same rows, in one launch: the
 * batched step's residual add followed by the next RMSNorm (model.py:507
 * then :509; :514 then the next layer's :487).  x and out are bit-identical
 * to aq_add followed by aq_rmsnorm.  out must not alias x or y. */
int aq_add_rmsnorm(float *x, const float *y, const float *w, int64_t rows, int64_t n,
                   float eps, float *out, void *stream);

/* Rotary embedding of T tokens at positions p0 .. p0+T-1, where p0 =
 * state->pos when `state` is not NULL and `pos0` otherwise: q [T][n_head *
 * head_dim] is rotated in place; k [T][n_kv * head_dim] is rotated and stored
 * with v [T][n_kv * head_dim] into the caches at those positions.  cos_tab /
 * sin_tab are [n_ctx][n_rot/2] fp32 (cos/sin of pos * inv_freq, computed by
 * the caller).  neox = 0: pairs (2i, 2i+1) ("norm", llama); 1: (i, i+n_rot/2).
 * Replaces Model._rope_np / _rope_batch_np (alpacca/model.py:400-434) and
 * the cache stores of model.py:533-540 / :495-503.  AQ_ERR_VALUE when
 * p0 + T > n_ctx (checked only for a host position; the kernels skip
 * positions past the cache). */
int aq_rope_kv(float *q, const float *k, const float *v, int64_t T, int n_head,
               int n_kv, int head_dim, int n_rot, int neox,
               const float *cos_tab, const float *sin_tab,
               const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
               float *k_cache, float *v_cache, void *stream);

/* Grouped-query attention of one query token per head (q [n_head *
 * head_dim], already rotated) at position p (state->pos, or pos0 when state
 * is NULL) over cache positions 0..p: out [n_head * head_dim].  Query head h
 * uses kv head h / (n_head / n_kv).  head_dim 64 or 128, n_head / n_kv in
 * {1, 2, 4, 8}.  Replaces Model._attention_np (alpacca/model.py:447-455). */
int aq_attention(const float *q, const float *k_cache, const float *v_cache,
                 int n_head, int n_kv, int head_dim, int64_t n_ctx,
                 const aq_decode_state *state, int64_t pos0, float *out,
                 void *stream);

/* Causal attention of T consecutive query tokens (q [T][n_head * head_dim],
 * already rotated) at positions p0 .. p0+T-1 (p0 = state->pos, or pos0 when
 * state is NULL): token t attends to cache positions 0 .. p0+t, whose k and
 * v must already be stored (aq_rope_kv with the same T).  out [T][n_head *
 * head_dim].  Replaces Model._attention_batch_np (alpacca/model.py:457-467);
 * aq_attention is the T = 1 case. */
int aq_attention_batch(const float *q, const float *k_cache, const float *v_cache,
                       int64_t T, int n_head, int n_kv, int head_dim, int64_t n_ctx,
                       const aq_decode_state *state, int64_t pos0, float *out,
                       void *stream);

/* aq_rope_kv (T = 1) followed by aq_attention, with the rotation folded into
 * the attention kernel: q and k are rotated in registers, k and v stored at
 * position p, and the attention of the q heads over positions 0..p written
 * to out (two launches instead of three); q, k, v are left as they are.  Results are identical to the two calls (the same operations in the
 * same order).  n_rot must be a multiple of 8 for neox.  Replaces
 * model.py:533-544 (_rope_np of q and k, the cache stores, _attention_np). */
int aq_attention_rope(float *q, const float *k, const float *v, int n_head,
                      int n_kv, int head_dim, int n_rot, int neox,
                      const float *cos_tab, const float *sin_tab,
                      const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
                      float *k_cache, float *v_cache, float *out, void *stream);

/* The decode attention's partial scratch for one call of aq_attention_rope,
 * aq_attention_rope_noalloc (T = 1) or the chunked form of
 * aq_attention_batch (T > 1): *scratch_bytes is what the library sizes for
 * it, *launch_bytes the extent that call's launch grid writes (the launchers
 * refuse a smaller scratch with AQ_ERR_VALUE).  Host only: no device is
 * touched.  AQ_ERR_VALUE for an unsupported shape.  No counterpart in the
 * reference (it has no device scratch): for callers that bring their own
 * scratch, and for tests that the two sizes agree. */
int aq_attention_scratch_info(int n_head, int n_kv, int head_dim, int64_t n_ctx,
                              int64_t T, size_t *scratch_bytes, size_t *launch_bytes);

/* aq_attention_rope without device allocation: the same kernels and the same
 * results, with the per-split attention partials in the library's static
 * device scratch (8 MiB per device, held until the process exits) instead of
 * the per-stream workspace that aq_attention_rope allocates.  AQ_ERR_VALUE
 * when the partials, n_head * S * (head_dim + 4) floats with
 * S = min(32, max(1, ceil(n_ctx / chunk) / 2)) splits and chunk = 64
 * (head_dim 64) or 32 (head_dim 128), exceed the
 * scratch: any cache length up to 496 query heads at head_dim 128 and 963 at
 * head_dim 64.  Every call on a device shares that device's
 * scratch, so calls that overlap on one device (different streams) race;
 * nothing in it needs clearing between calls.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). */
int aq_attention_rope_noalloc(float *q, const float *k, const float *v, int n_head,
                              int n_kv, int head_dim, int n_rot, int neox,
                              const float *cos_tab, const float *sin_tab,
                              const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
                              float *k_cache, float *v_cache, float *out, void *stream);

/* out = gate / (1 + exp(-gate)) * up, n elements (model.py:549-551). */
int aq_swiglu(const float *gate, const float *up, int64_t n, float *out,
              void *stream);

/* aq_swiglu over interleaved pairs: out[i] = silu(gate_up[2i]) *
 * gate_up[2i + 1], i < n, rounded as aq_swiglu.  The batched step's form of
 * model.py:549-551 when ffn_gate and ffn_up are stored as one matrix with
 * their rows interleaved (one matmul_t gives the pairs). */
int aq_swiglu_pairs(const float *gate_up, int64_t n, float *out, void *stream);

/* x += y, n elements: the residual adds of model.py:546 and :552. */
int aq_add(float *x, const float *y, int64_t n, void *stream);

/* x[r, :] += b for r < rows (n elements per row, b of n): the q/k/v bias
 * adds of a batch (q + bq over all tokens, model.py:491-496), one launch per
 * projection; each element rounded as x + b in fp32. */
int aq_add_rows(float *x, const float *b, int64_t rows, int64_t n, void *stream);

/* End of a decode step: state->pos += 1 and the token of the next step is
 * chosen.  While state->fed < n_prompt it is the next prompt token
 * (prompt[state->fed++]: the prompt loop of Model.prefill,
 * alpacca/model.py:633-640); after that, when take_argmax != 0, it is the
 * first index of the maximum of logits[0..n) (tensor.argmax,
 * alpacca/tensor.py:187-194, as the greedy sampler uses it,
 * alpacca/sample.py:44-45), also appended to history[state->count++] while
 * count < capacity (history may be NULL). */
int aq_greedy_advance(const float *logits, int64_t n, aq_decode_state *state,
                      const int64_t *prompt, int64_t n_prompt, int64_t *history,
                      int64_t capacity, int take_argmax, void *stream);

/* aq_greedy_advance with the repetition penalty of the reference's greedy
 * sampler: Sampler.sample at temperature <= 0 (alpacca/sample.py:36-45, the
 * decode loop of tests/bench.py:78-90) and Sampler.accept (sample.py:31-34).
 * window (device memory, caller-owned, 1 + last_n int64): window[0] counts
 * the tokens accepted so far, the i-th of them is window[1 + i % last_n];
 * every token this call makes state->token (a prompt token or the chosen
 * one) is accepted.  The chosen token is the first index of the maximum of
 * logits[0..n) taken as double, where each distinct token t among the last
 * min(window[0], last_n) accepted counts as logits[t] / penalty when
 * logits[t] > 0 and as logits[t] * penalty otherwise (double arithmetic, as
 * the reference's Python floats); penalty 0 or 1 leaves the logits as they
 * are.  Window tokens outside [0, n) are skipped.  last_n >= 1; penalty
 * finite. */
int aq_greedy_advance_penalized(const float *logits, int64_t n, aq_decode_state *state,
                                const int64_t *prompt, int64_t n_prompt, int64_t *history,
                                int64_t capacity, int64_t *window, int64_t last_n,
                                double penalty, int take_argmax, void *stream);

/* ==== calibration ========================================================
 *
 * Reads rows * row_bytes bytes of device memory at p (row_bytes <= 4096):
 * `waves` waves (a multiple of 4), wave w reading rows w, w + waves, ... with
 * `inflight` (1, 2 or 4) rows in flight, 16 bytes per lane per load, results
 * folded into a value that is almost never stored to *sink.  No counterpart
 * in the reference: it measures how fast one launch of a given size can read
 * HBM on this part, the ceiling that bench.py reports beside the decode
 * matvec's roofline fraction.  Enqueues only. */
int aq_stream_read(const void *p, int64_t rows, int row_bytes, int waves, int inflight,
                   unsigned *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ALPACCA_AMD_H */
