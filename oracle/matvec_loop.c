/* CPU baseline - TEST INFRASTRUCTURE (see oracle/__init__.py).
 *
 * C/OpenMP transliteration of the reference's fused native-tier loop
 * _matvec_codes (jtiro232/Alpacca alpacca/kernels.py:49-69), which Numba
 * compiles with parallel=True, fastmath=True: per output row, a float32 dot
 * of the int8 codes of each sub-block with x, times the sub-block scale, plus
 * (affine formats) sum_s m_eff[r,s] * xsum[s].  Rows are spread over OpenMP
 * threads as Numba's prange spreads them.  Inputs are the unpacked form the
 * reference keeps in RAM (codes int8 (rows, n_sub, sub_len), d/m float32
 * (rows, n_sub)); unpacking is not timed, as in the reference.
 */
#include <stdint.h>

void matvec_codes(const int8_t *q3, const float *d, const float *m,
                  const float *xs, const float *xsums, int affine,
                  int64_t rows, int64_t nsub, int64_t sub_len, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float acc = 0.0f;
    const int8_t *qr = q3 + r * nsub * sub_len;
    for (int64_t s = 0; s < nsub; ++s) {
      float dot = 0.0f;
      const int8_t *qb = qr + s * sub_len;
      const float *xb = xs + s * sub_len;
      for (int64_t j = 0; j < sub_len; ++j) dot += (float)qb[j] * xb[j];
      acc += d[r * nsub + s] * dot;
    }
    if (affine) {
      float macc = 0.0f;
      for (int64_t s = 0; s < nsub; ++s) macc += m[r * nsub + s] * xsums[s];
      acc += macc;
    }
    out[r] = acc;
  }
}
