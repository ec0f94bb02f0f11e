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

/* ---- matmul_t precision -------------------------------------------------- */
#define AQ_PREC_AUTO 0   /* M < 64: FP32; M >= 64: BF16                        */
#define AQ_PREC_FP32 1   /* fp32 FMA over exactly decoded weights              */
#define AQ_PREC_BF16 2   /* weights and X rounded to bf16, MFMA, fp32 accum.   */

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

/* Shape, dtype, layout and the HBM bytes of the quantized representation.
 * Replaces QuantMatrix.shape / storage_nbytes (qmatrix.py:130-141). */
int aq_matrix_info(const aq_matrix *m, int64_t *rows, int64_t *cols, int *dtype,
                   int *layout, size_t *device_bytes);

/* y[rows] = W x[cols], fp32 in and out, fused dequantize-and-dot.  The
 * default kernel splits each 32-element group of x into three int8 pieces
 * (24 bits relative to the group maximum) and accumulates exact int32 dot
 * products; AQ_MATVEC_FP32 selects the fp32-FMA kernel.
 * Replaces QuantMatrix.matvec (qmatrix.py:148-171) and the fused native kernel
 * kernels.matvec_codes (kernels.py:89-104).  With host pointers the call is
 * synchronous; with AQ_IN_DEVICE|AQ_OUT_DEVICE it only enqueues on `stream`. */
int aq_matvec(const aq_matrix *m, const float *x, float *y, int flags,
              void *stream);

/* y_i = W_i x for n (1..8) matrices that share x: one kernel launch whose
 * workgroups split the rows of all n matrices evenly.  The matrices must have
 * one dtype, one column count and one layout; x and every y_i are device
 * pointers (AQ_IN_DEVICE | AQ_OUT_DEVICE required) and the call only enqueues
 * on `stream`.  The reference has no single call for this: its decode step
 * runs QuantMatrix.matvec once per projection on the same input
 * (alpacca/model.py:529-531 q/k/v, :549-550 gate/up); this entry point is the
 * fused form of those calls. */
int aq_matvec_multi(const aq_matrix *const *ms, int n, const float *x,
                    float *const *ys, int flags, void *stream);

/* Y[M, rows] = X[M, cols] W^T.  Replaces QuantMatrix.matmul_t
 * (qmatrix.py:184-211); AQ_ERR_VALUE for M < 0.  `precision` is one of
 * AQ_PREC_*. */
int aq_matmul_t(const aq_matrix *m, const float *X, int64_t M, float *Y,
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

#ifdef __cplusplus
}
#endif

#endif /* ALPACCA_AMD_H */
