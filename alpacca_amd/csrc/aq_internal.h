// aq_internal.h - types shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/alpacca_amd.h"
#include "aq_formats.h"

// A quantized matrix resident in HBM (the object behind aq_matrix*).
struct aq_matrix {
  int dtype;
  int layout;           // AQ_LAYOUT_RAW or AQ_LAYOUT_SPLIT (never AUTO)
  int device;           // HIP device that holds `dev`
  int64_t rows, cols;   // N (outputs) x K (inputs)
  int64_t nb_row;       // blocks per row
  int64_t nb_pitch;     // blocks from one row to the next (nb_row, except in
                        // a column window of a wider matrix)
  size_t raw_bytes;     // GGUF bytes: rows * nb_row * block_bytes
  uint8_t *dev;         // one hipMalloc holding every plane
  size_t dev_bytes;
  aq::Planes planes;
};

namespace aq {

// F32 / F16 / BF16 matrices (dense values, fp32 kernels only)
inline bool is_dense(int dtype) {
  return dtype == AQ_F32 || dtype == AQ_F16 || dtype == AQ_BF16;
}

// Columns [nb0 * block_elems, (nb0 + nb) * block_elems) of m as a matrix of
// its own: the same rows and row pitch, plane pointers moved to block nb0.
// Only the matvec launchers take such a window (they address row r at
// block r * nb_pitch); it owns nothing and lives as long as m.
inline aq_matrix column_window(const aq_matrix &m, int64_t nb0, int64_t nb) {
  aq_matrix v = m;
  v.nb_row = nb;
  v.cols = m.cols / m.nb_row * nb;
  for (int k = 0; k < 4; ++k)
    if (v.planes.p[k]) v.planes.p[k] += nb0 * v.planes.stride[k];
  return v;
}

// Per-device facts queried once by aq_init.
struct DeviceInfo {
  int cus;            // compute units
  size_t lds_max;     // max dynamic LDS per workgroup
};
const DeviceInfo &device_info(int device);

// Raise kernel `kern`'s dynamic-LDS limit to `bytes` on the current device
// (hipFuncSetAttribute applies per device), once per (kernel, device);
// thread-safe.
hipError_t set_dynamic_lds(const void *kern, int bytes);

// Kernel launchers (aq_matvec.hip, aq_dequant.hip, aq_matmul.hip).  All
// pointers are device pointers; they only enqueue work on `s`.
hipError_t launch_matvec(const aq_matrix *m, const float *x, float *y,
                         hipStream_t s, bool accumulate = false);
hipError_t launch_dequant_rows(const aq_matrix *m, const int64_t *idx,
                               int64_t n, float *out, hipStream_t s);
hipError_t launch_matmul_t(const aq_matrix *m, const float *X, int64_t M,
                           float *Y, int precision, hipStream_t s);
// Y[i] = sum_z P[z * n + i] over z < splits, in z order (aq_matmul.hip)
hipError_t sum_splits(const float *P, int splits, int64_t n, float *Y, hipStream_t s);
// matmul_t with the weights as exact integers on fp16 matrix cores and X in
// two fp16 pieces per element after a per-row power-of-two scale (22 bits;
// aq_matmul_h.hip); mm_h_supported says which matrices it takes.
// m_invariant: the same bits for every M (no split of the K range).
// ysw: rows are interleaved (gate, up) pairs; where the launch can form the
// pairs in its store (Q4_K / Q5_K without a split) it writes silu(gate) * up
// (M x rows/2) there instead of Y and sets *fused_sw, else it writes Y and
// clears it.
bool mm_h_supported(const aq_matrix *m);
hipError_t launch_matmul_h(const aq_matrix *m, const float *X, int64_t M, float *Y,
                           bool m_invariant, hipStream_t s, float *ysw = nullptr,
                           bool *fused_sw = nullptr);

// Device scratch memory for work on stream `s` of `device`, at least `bytes`
// long (nullptr when it cannot be allocated).  One buffer per (device,
// stream): work on one stream is ordered, so the buffer is reused by the next
// call on that stream.  Sizes grow geometrically.  While the stream is
// capturing a HIP graph nothing is allocated: a buffer too small then gives
// nullptr (and the C ABI reports that the call must first run eagerly).  An
// outgrown buffer is freed after the stream's queued work, unless it was
// handed out during a capture: such a buffer is kept until the process
// exits, so the graph stays valid.
void *workspace(int device, hipStream_t s, size_t bytes);
// Drop the workspace of stream `s` (all devices), as workspace() drops an
// outgrown buffer; the next call on the stream allocates anew.
void release_workspace(hipStream_t s);

// Largest K (columns) the matvec kernel accepts: x is staged whole in LDS.
int64_t matvec_max_cols(int dtype, int device);

// Integer-dot decode matvec (aq_matvec_i8.hip): LDS bytes of the prepared x
// of one row, the largest K it accepts, and the launcher (x -> y).
size_t matvec_i8_scratch_bytes(int dtype, int64_t nb_row);
int64_t matvec_i8_max_cols(int dtype, int device);
hipError_t launch_matvec_i8(const aq_matrix *m, const float *x, float *y,
                            hipStream_t s);
// Fused forms of the decode matvec: what is staged as x, and whether the
// result is added to y.
struct MatvecFusion {
  enum Mode { kPlain = 0, kNorm = 1, kSwiglu = 2 };
  int mode;
  const float *x2;      // kSwiglu: x_eff = x / (1 + exp(-x)) * x2
  const float *norm_w;  // kNorm: x_eff = x * inv * norm_w
  float eps;            // kNorm: inv = 1 / sqrt(mean(x^2) + eps)
  bool accumulate;      // y += W x_eff
  bool swiglu_pairs;    // rows are (gate, up) pairs: y[j] = silu(row 2j) * row 2j+1
};
// n (<= 8) matrices of one dtype, K and layout sharing x: one launch
// (fu may be NULL: plain y = W x).
hipError_t launch_matvec_i8_multi(const aq_matrix *const *ms, int n,
                                  const float *x, float *const *ys,
                                  hipStream_t s, const MatvecFusion *fu);
// Y[v, :] = W X[v, :] for v < M with the integer kernel: passes of up to 8
// x vectors share one weight stream (X rows ldx floats apart, Y rows ldy
// apart); rows wider than a pass can stage run as column windows.
hipError_t launch_matvec_i8_batch(const aq_matrix *m, const float *X, int64_t M, int64_t ldx,
                                  float *Y, int64_t ldy, hipStream_t s);
// Pairs of dtypes one multi launch may mix (matrices of dtype0 first).
bool matvec_mixed_supported(int dtype0, int dtype1);
// rows of this dtype and width run two per wave (at most 32 lane units)
bool matvec_pair_rows(int dtype, int64_t nb_row);

// Decode-step kernels (aq_decode.hip).  Device pointers; enqueue only.
bool attention_supported(int head_dim, int group);
size_t attention_scratch_bytes(int n_kv, int head_dim, int group, int64_t n_ctx, int64_t T);
// Bytes of partial scratch one attention launch writes, from the grid it
// launches (the launchers refuse a smaller part_bytes with
// hipErrorInvalidValue).
size_t attention_launch_extent_bytes(int n_kv, int head_dim, int group, int64_t n_ctx,
                                     int64_t T);
hipError_t launch_rmsnorm(const float *x, const float *w, int64_t rows,
                          int64_t n, float eps, float *out, hipStream_t s);
hipError_t launch_add_rmsnorm(float *x, const float *y, const float *w, int64_t rows,
                              int64_t n, float eps, float *out, hipStream_t s);
hipError_t launch_rope_kv(float *q, const float *k, const float *v, int64_t T,
                          int n_head, int n_kv, int hd, int n_rot, int neox,
                          const float *cos_t, const float *sin_t,
                          const aq_decode_state *st, int64_t pos0, int64_t n_ctx,
                          float *kc, float *vc, hipStream_t s);
// T > 1 query tokens at positions pos..pos+T-1 (causal), one launch, no
// scratch (k_attn_prefill)
hipError_t launch_attention_prefill(const float *q, const float *kc, const float *vc,
                                    int n_head, int n_kv, int hd, int64_t n_ctx,
                                    const aq_decode_state *st, int64_t pos0, int64_t T,
                                    float *out, hipStream_t s);
hipError_t launch_attention(const float *q, const float *kc, const float *vc,
                            int n_head, int n_kv, int hd, int64_t n_ctx,
                            const aq_decode_state *st, int64_t pos0, int64_t T, float *part,
                            size_t part_bytes, float *out, hipStream_t s);
hipError_t launch_attention_rope(const float *q, const float *k, const float *v,
                                 int n_head, int n_kv, int hd, int n_rot, int neox,
                                 const float *cos_t, const float *sin_t, int64_t n_ctx,
                                 const aq_decode_state *st, int64_t pos0, float *kc,
                                 float *vc, float *part, size_t part_bytes, float *out,
                                 hipStream_t s);
// out[i] = silu(g[i * stride]) * u[i * stride], i < n
hipError_t launch_swiglu(const float *g, const float *u, int64_t stride, int64_t n,
                         float *out, hipStream_t s);

hipError_t launch_add(float *x, const float *y, int64_t n, hipStream_t s);
hipError_t launch_add_rows(float *x, const float *b, int64_t rows, int64_t n, hipStream_t s);
// window: NULL, or the repetition window (1 + last_n int64: count, ring);
// penalize != 0 applies `penalty` to the window's tokens before the argmax.
hipError_t launch_greedy_advance(const float *logits, int64_t n,
                                 aq_decode_state *st, const int64_t *prompt,
                                 int64_t n_prompt, int64_t *hist, int64_t cap,
                                 int take_argmax, int64_t *window, int64_t last_n,
                                 int penalize, double penalty, hipStream_t s);

}  // namespace aq
