// aq_dequant.hip - decode whole rows to fp32 (embedding lookups).
//
// Replaces QuantMatrix.row / rows_at (alpacca/qmatrix.py:215-246), whose
// values are those of quants.dequantize (quants.py:498-528): code * d_eff
// (+ m_eff).  One thread decodes one chunk of one requested row and writes
// its two 16-element runs with 16-byte stores.
#include "aq_internal.h"

namespace aq {
namespace {

template <class F>
__global__ void __launch_bounds__(256)
    k_dequant_rows(Planes P, int64_t rows, int nb_row,
                   const int64_t *__restrict__ idx, int64_t n,
                   float *__restrict__ out) {
  const int64_t n_chunks = (int64_t)nb_row * F::CPB;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * n_chunks) return;
  const int64_t i = gid / n_chunks;
  const int ch = (int)(gid - i * n_chunks);
  int64_t r = idx[i];
  r = r < 0 ? 0 : (r >= rows ? rows - 1 : r);  // device indices: clamp
  const int b = ch / F::CPB, j = ch - b * F::CPB;
  const typename F::Raw raw = F::load(P, r * nb_row + b, j);
  float v[F::ELEMS];
  F::decode(raw, j, v);
  float *o = out + i * (int64_t)nb_row * F::BE + (int64_t)b * F::BE;
#pragma unroll
  for (int q = 0; q < F::ELEMS / 4; ++q)
    *reinterpret_cast<float4 *>(o + F::xoff(j, 4 * q)) =
        make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

template <class F>
hipError_t launch_fmt(const aq_matrix *m, const int64_t *idx, int64_t n,
                      float *out, hipStream_t s) {
  const int64_t total = n * m->nb_row * F::CPB;
  if (total == 0) return hipSuccess;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(k_dequant_rows<F>, dim3((unsigned)grid), dim3(256), 0, s,
                     m->planes, m->rows, (int)m->nb_row, idx, n, out);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dequant_rows(const aq_matrix *m, const int64_t *idx,
                               int64_t n, float *out, hipStream_t s) {
  switch (m->dtype) {
    case AQ_Q4_K: return launch_fmt<Q4K>(m, idx, n, out, s);
    case AQ_Q5_K: return launch_fmt<Q5K>(m, idx, n, out, s);
    case AQ_Q6_K: return launch_fmt<Q6K>(m, idx, n, out, s);
    case AQ_Q8_0: return launch_fmt<Q80>(m, idx, n, out, s);
    case AQ_Q4_0: return launch_fmt<Q40>(m, idx, n, out, s);
    case AQ_Q4_1: return launch_fmt<Q41>(m, idx, n, out, s);
    case AQ_Q5_0: return launch_fmt<Q50>(m, idx, n, out, s);
    case AQ_Q5_1: return launch_fmt<Q51>(m, idx, n, out, s);
    case AQ_F32: return launch_fmt<F32D>(m, idx, n, out, s);
    case AQ_F16: return launch_fmt<F16D>(m, idx, n, out, s);
    case AQ_BF16: return launch_fmt<BF16D>(m, idx, n, out, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aq
