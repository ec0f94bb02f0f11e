// aq_matmul.hip - batched prefill Y = X W^T on gfx950 matrix cores.
//
// Replaces QuantMatrix.matmul_t (alpacca/qmatrix.py:184-211), which
// dequantizes ~4 MiB f32 row tiles of W and multiplies them with OpenBLAS.
// Here each workgroup decodes a 128-row x 64-slot tile of W straight from the
// quantized blocks into LDS and runs MFMA against the matching 128 x 64 tile
// of X:
//   BF16: both tiles rounded to bf16, v_mfma_f32_16x16x32_bf16, fp32 accum.
//   FP32: both tiles kept fp32, v_mfma_f32_16x16x4_f32 (fp32 products,
//         fp32 accumulation) - the precision of the reference's SGEMM.
//
// K order.  The contraction runs over "slots" (chunk j, slot t) instead of
// natural element order: each chunk's decoded values land contiguously in
// LDS, and X is gathered with the same slot -> element map (xoff), so both
// operands see one consistent permutation of K and the sum is unchanged.
//
// Wave layout: 4 waves as 2 x 2, each owning a 64 x 64 block of Y as 4 x 4
// MFMA tiles of 16 x 16.  For a 16x16 tile, lane l holds A row l%16, B column
// l%16 and D[4*(l/16) + r][l%16], r = 0..3.
#include "aq_internal.h"

namespace aq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));

constexpr int BM = 128;  // rows of X (and Y) per workgroup
constexpr int BN = 128;  // rows of W (columns of Y) per workgroup
constexpr int BK = 64;   // K slots per stage

__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return bf16_rne(a) | (bf16_rne(b) << 16);
}

template <bool BF16>
struct TileTraits;
template <>
struct TileTraits<true> {
  static constexpr int LD = BK + 8;  // bf16 elements per LDS row (144 B)
  using T = uint16_t;
};
template <>
struct TileTraits<false> {
  static constexpr int LD = BK + 4;  // floats per LDS row (272 B)
  using T = float;
};

template <class F, bool BF16>
__global__ void __launch_bounds__(256)
    k_matmul_t(Planes P, int64_t N, int nb_row, const float *__restrict__ X,
               int64_t M, float *__restrict__ Y) {
  using TT = TileTraits<BF16>;
  using T = typename TT::T;
  constexpr int LD = TT::LD;
  constexpr int CPS = BK / F::ELEMS;  // chunks per stage
  __shared__ __attribute__((aligned(16))) T As[BM * LD];
  __shared__ __attribute__((aligned(16))) T Bs[BN * LD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K = (int64_t)nb_row * F::BE;
  const int n_chunks = nb_row * F::CPB;
  const int n_stages = (n_chunks + CPS - 1) / CPS;

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int st = 0; st < n_stages; ++st) {
    // ---- X tile: BM rows x BK slots, 8 float4 per thread ----
#pragma unroll
    for (int it = 0; it < (BM * BK / 4) / 256; ++it) {
      const int idx = it * 256 + tid;
      const int row = idx / (BK / 4), quad = idx % (BK / 4);
      const int slot = 4 * quad;
      const int ch = st * CPS + slot / F::ELEMS, t = slot % F::ELEMS;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m0 + row < M && ch < n_chunks) {
        const int b = ch / F::CPB, j = ch - b * F::CPB;
        v = *reinterpret_cast<const float4 *>(
            X + (m0 + row) * K + (int64_t)b * F::BE + F::xoff(j, t));
      }
      if constexpr (BF16) {
        *reinterpret_cast<uint2 *>(&As[row * LD + slot]) =
            make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
      } else {
        *reinterpret_cast<float4 *>(&As[row * LD + slot]) = v;
      }
    }
    // ---- W tile: BN rows x CPS chunks decoded exactly, then stored ----
    for (int item = tid; item < BN * CPS; item += 256) {
      const int row = item / CPS, c = item % CPS;
      const int ch = st * CPS + c;
      float v[F::ELEMS];
      if (ch < n_chunks) {
        int64_t n = n0 + row;
        n = n < N ? n : N - 1;
        const int b = ch / F::CPB, j = ch - b * F::CPB;
        F::decode(F::load(P, n * nb_row + b, j), j, v);
      } else {
#pragma unroll
        for (int t = 0; t < F::ELEMS; ++t) v[t] = 0.f;
      }
      T *dst = &Bs[row * LD + c * F::ELEMS];
      if constexpr (BF16) {
#pragma unroll
        for (int q = 0; q < F::ELEMS / 8; ++q)
          *reinterpret_cast<uint4 *>(dst + 8 * q) = make_uint4(
              pack_bf16(v[8 * q], v[8 * q + 1]), pack_bf16(v[8 * q + 2], v[8 * q + 3]),
              pack_bf16(v[8 * q + 4], v[8 * q + 5]), pack_bf16(v[8 * q + 6], v[8 * q + 7]));
      } else {
#pragma unroll
        for (int q = 0; q < F::ELEMS / 4; ++q)
          *reinterpret_cast<float4 *>(dst + 4 * q) =
              make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      }
    }
    __syncthreads();

    // ---- MFMA over the stage ----
    const int r16 = lane & 15, kq = lane >> 4;
    if constexpr (BF16) {
#pragma unroll
      for (int kk = 0; kk < BK; kk += 32) {
        bf16x8 a[4], b[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
          a[tm] = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const uint4 *>(
                          &As[(wm * 64 + tm * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
        for (int tn = 0; tn < 4; ++tn)
          b[tn] = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const uint4 *>(
                          &Bs[(wn * 64 + tn * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
          for (int tn = 0; tn < 4; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                a[tm], b[tn], acc[tm][tn], 0, 0, 0);
      }
    } else {
#pragma unroll 4
      for (int kk = 0; kk < BK; kk += 4) {
        float a[4], b[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
          a[tm] = As[(wm * 64 + tm * 16 + r16) * LD + kk + kq];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn)
          b[tn] = Bs[(wn * 64 + tn * 16 + r16) * LD + kk + kq];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
          for (int tn = 0; tn < 4; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                a[tm], b[tn], acc[tm][tn], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- store: D[4*(l/16) + r][l%16] of each 16x16 tile ----
  const int col = lane & 15, rq = lane >> 4;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm)
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int64_t n = n0 + wn * 64 + tn * 16 + col;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * 64 + tm * 16 + 4 * rq + r;
        if (m < M && n < N) Y[m * N + n] = acc[tm][tn][r];
      }
    }
}

template <class F>
hipError_t launch_fmt(const aq_matrix *m, const float *X, int64_t M, float *Y,
                      int precision, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const dim3 grid((unsigned)((m->rows + BN - 1) / BN),
                  (unsigned)((M + BM - 1) / BM));
  if (precision == AQ_PREC_BF16)
    hipLaunchKernelGGL((k_matmul_t<F, true>), grid, dim3(256), 0, s, m->planes,
                       m->rows, (int)m->nb_row, X, M, Y);
  else
    hipLaunchKernelGGL((k_matmul_t<F, false>), grid, dim3(256), 0, s,
                       m->planes, m->rows, (int)m->nb_row, X, M, Y);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_matmul_t(const aq_matrix *m, const float *X, int64_t M,
                           float *Y, int precision, hipStream_t s) {
  switch (m->dtype) {
    case AQ_Q4_K: return launch_fmt<Q4K>(m, X, M, Y, precision, s);
    case AQ_Q5_K: return launch_fmt<Q5K>(m, X, M, Y, precision, s);
    case AQ_Q6_K: return launch_fmt<Q6K>(m, X, M, Y, precision, s);
    case AQ_Q8_0: return launch_fmt<Q80>(m, X, M, Y, precision, s);
    case AQ_Q4_0: return launch_fmt<Q40>(m, X, M, Y, precision, s);
    case AQ_Q4_1: return launch_fmt<Q41>(m, X, M, Y, precision, s);
    case AQ_Q5_0: return launch_fmt<Q50>(m, X, M, Y, precision, s);
    case AQ_Q5_1: return launch_fmt<Q51>(m, X, M, Y, precision, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aq
