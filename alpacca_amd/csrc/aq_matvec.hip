// aq_matvec.hip - decode matvec y = W x (M = 1) over GGUF blocks in HBM.
//
// Replaces the fused loop of the reference's native tier
// (alpacca/kernels.py:49-69) and the einsum matvec (alpacca/qmatrix.py:160-171):
// y[r] = sum over sub-blocks of d_eff * (codes . x) (+ m_eff * sum(x)), here
// computed straight from the quantized blocks without an unpacked copy.
//
// Mapping.  A workgroup has 4 waves.  Lane l of a wave handles chunk
// 64g + l of a row (a chunk = 16 payload bytes, see aq_formats.h), so one
// wave-wide load reads 1 KB of contiguous payload.  Each lane keeps its x
// slots in registers and applies them to R rows at once; KW waves split the
// chunk groups of the same rows (KW > 1 when there are too few rows to fill
// the chip) and combine through LDS in a fixed order, so results are
// deterministic.  Workgroups loop over row tiles (grid = resident slots).
//
// x lives in LDS for the whole kernel, stored chunk-major and interleaved so
// that the 64 lanes reading slot quad q of 64 consecutive chunks touch 1 KB of
// consecutive LDS (no bank conflicts).  The per-chunk sums of x over slots
// [0,16) and [16,32) are precomputed once per workgroup: the formats with an
// offset (mins, the -8/-16/-32 code bias) need them for every row.
#include <stdlib.h>

#include "aq_internal.h"

namespace aq {
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// Sum over the 64 lanes of a wave (result is wave-uniform).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror: 8-lane sums
  v += dpp_f32<0x140>(v);  // row_mirror: 16-lane sums
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

constexpr int WG = 256;

template <class F, int R, int KW>
__global__ void __launch_bounds__(WG)
    k_matvec(Planes P, int64_t N, int nb_row, int nb_pitch, const float *__restrict__ x,
             float *__restrict__ y, int accumulate) {
  extern __shared__ float4 smem4[];
  constexpr int Q = F::ELEMS / 4;  // float4 quads per chunk
  constexpr int RG = 4 / KW;       // row groups per workgroup
  constexpr int RPT = RG * R;      // rows per tile
  const int n_chunks = nb_row * F::CPB;
  const int n_groups = (n_chunks + 63) >> 6;
  float4 *xl = smem4;
  float2 *xsl = reinterpret_cast<float2 *>(xl + (size_t)n_groups * Q * 64);
  float *red = reinterpret_cast<float *>(xsl + (size_t)n_groups * 64);

  // ---- stage x (chunk-major, lane-interleaved) and the half-chunk sums ----
  for (int p = threadIdx.x; p < n_chunks * Q; p += WG) {
    const int ch = p / Q, q = p - ch * Q;
    const int b = ch / F::CPB, j = ch - b * F::CPB;
    xl[((ch >> 6) * Q + q) * 64 + (ch & 63)] =
        *reinterpret_cast<const float4 *>(x + (int64_t)b * F::BE +
                                          F::xoff(j, 4 * q));
  }
  __syncthreads();
  for (int ch = threadIdx.x; ch < n_chunks; ch += WG) {
    const float4 *src = xl + (size_t)(ch >> 6) * Q * 64 + (ch & 63);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const float4 v = src[q * 64];
      const float s = (v.x + v.y) + (v.z + v.w);
      if (q < 4)
        s0 += s;
      else
        s1 += s;
    }
    xsl[ch] = make_float2(s0, s1);
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kw = wave % KW, rg = wave / KW;
  const int64_t n_tiles = (N + RPT - 1) / RPT;
  // groups per wave per tile; at least 1 so that every wave reaches the end
  // of each tile (the host never launches KW > n_groups)
  const int gpw = max(1, (n_groups - kw + KW - 1) / KW);
  const int64_t my_tiles =
      blockIdx.x < n_tiles ? (n_tiles - 1 - blockIdx.x) / gridDim.x + 1 : 0;

  using Raw = typename F::Raw;
  // step (ti, gi): this wave's gi-th chunk group of its ti-th row tile
  auto fetch = [&](int64_t ti, int gi, Raw *dst) {
    const int g = kw + gi * KW;
    const int64_t tile = blockIdx.x + ti * gridDim.x;
    int ch = g * 64 + lane;
    ch = ch < n_chunks ? ch : n_chunks - 1;
    const int b = ch / F::CPB, j = ch - b * F::CPB;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      int64_t r = tile * RPT + rg * R + i;
      r = r < N ? r : N - 1;
      dst[i] = F::load(P, r * nb_pitch + b, j);
    }
  };
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.f;
  auto compute = [&](int64_t ti, int gi, const Raw *w) {
    const int g = kw + gi * KW;
    const int ch = g * 64 + lane;
    if (ch < n_chunks) {
      float xv[F::ELEMS];
      const float4 *src = xl + (size_t)g * Q * 64 + lane;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const float4 v = src[q * 64];
        xv[4 * q] = v.x;
        xv[4 * q + 1] = v.y;
        xv[4 * q + 2] = v.z;
        xv[4 * q + 3] = v.w;
      }
      const float2 xs = xsl[ch];
      const int j = ch % F::CPB;
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] += F::dot(w[i], j, xv, xs.x, xs.y);
    }
    if (gi == gpw - 1) {
      // end of this wave's share of a row tile: reduce and store
      const int64_t r0 = (blockIdx.x + ti * gridDim.x) * RPT + rg * R;
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = wave_sum(acc[i]);
      if constexpr (KW == 1) {
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < R; ++i)
            if (r0 + i < N) y[r0 + i] = accumulate ? y[r0 + i] + acc[i] : acc[i];
        }
      } else {
        __syncthreads();  // previous tile's partials have been consumed
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < R; ++i) red[wave * R + i] = acc[i];
        }
        __syncthreads();
        if (kw == 0 && lane == 0) {
#pragma unroll
          for (int i = 0; i < R; ++i) {
            float t = 0.f;
#pragma unroll
            for (int k = 0; k < KW; ++k) t += red[(rg * KW + k) * R + i];
            if (r0 + i < N) y[r0 + i] = accumulate ? y[r0 + i] + t : t;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = 0.f;
    }
  };
  auto advance = [&](int64_t &ti, int &gi) {
    if (++gi == gpw) {
      gi = 0;
      ++ti;
    }
  };

  // two register buffers, used alternately: the loads of step s+1 are in
  // flight while step s computes
  Raw bufA[R], bufB[R];
  int64_t ti = 0, nti = 0;
  int gi = 0, ngi = 0;
  if (my_tiles > 0) {
    fetch(nti, ngi, bufA);
    advance(nti, ngi);
  }
  while (ti < my_tiles) {
    if (nti < my_tiles) {
      fetch(nti, ngi, bufB);
      advance(nti, ngi);
    }
    compute(ti, gi, bufA);
    advance(ti, gi);
    if (ti >= my_tiles) break;
    if (nti < my_tiles) {
      fetch(nti, ngi, bufA);
      advance(nti, ngi);
    }
    compute(ti, gi, bufB);
    advance(ti, gi);
  }
}

template <class F>
size_t matvec_lds_bytes(int64_t nb_row) {
  const int64_t n_chunks = nb_row * F::CPB;
  const int64_t n_groups = (n_chunks + 63) / 64;
  return (size_t)n_groups * (F::ELEMS / 4) * 64 * 16 + (size_t)n_groups * 64 * 8 +
         4 * 4 * 4;
}

template <class F, int R, int KW>
hipError_t launch_cfg(const aq_matrix *m, const float *x, float *y,
                      hipStream_t s, bool accumulate) {
  const size_t lds = matvec_lds_bytes<F>(m->nb_row);
  auto kern = k_matvec<F, R, KW>;
  // LDS above 64 KiB
  hipError_t e = set_dynamic_lds(reinterpret_cast<const void *>(kern),
                                 (int)device_info(m->device).lds_max);
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, WG, lds);
  if (e != hipSuccess) return e;
  if (per_cu < 1) per_cu = 1;
  if (const char *env = getenv("AQ_MATVEC_WPC")) {  // tuning: cap WGs per CU
    const int w = atoi(env);
    if (w > 0 && w < per_cu) per_cu = w;
  }
  constexpr int RPT = (4 / KW) * R;
  const int64_t n_tiles = (m->rows + RPT - 1) / RPT;
  int64_t grid = (int64_t)device_info(m->device).cus * per_cu;
  if (grid > n_tiles) grid = n_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(WG), lds, s, m->planes,
                     m->rows, (int)m->nb_row, (int)m->nb_pitch, x, y, accumulate ? 1 : 0);
  return hipGetLastError();
}

// Pick rows-per-lane R and K-split KW: the largest R, then the smallest KW,
// that still gives every compute unit two row tiles.
template <class F>
hipError_t launch_fmt(const aq_matrix *m, const float *x, float *y,
                      hipStream_t s, bool acc) {
  const int64_t n_groups = (m->nb_row * F::CPB + 63) / 64;
  const int64_t want = 2 * (int64_t)device_info(m->device).cus;
  const int64_t N = m->rows;
  auto tiles = [&](int R, int KW) { return (N + (4 / KW) * R - 1) / ((4 / KW) * R); };
  if (tiles(4, 1) >= want) return launch_cfg<F, 4, 1>(m, x, y, s, acc);
  if (n_groups >= 2 && tiles(4, 2) >= want) return launch_cfg<F, 4, 2>(m, x, y, s, acc);
  if (n_groups >= 4 && tiles(4, 4) >= want) return launch_cfg<F, 4, 4>(m, x, y, s, acc);
  if (tiles(2, 1) >= want) return launch_cfg<F, 2, 1>(m, x, y, s, acc);
  if (n_groups >= 2 && tiles(2, 2) >= want) return launch_cfg<F, 2, 2>(m, x, y, s, acc);
  if (n_groups >= 4 && tiles(2, 4) >= want) return launch_cfg<F, 2, 4>(m, x, y, s, acc);
  if (n_groups >= 4) return launch_cfg<F, 1, 4>(m, x, y, s, acc);
  if (n_groups >= 2) return launch_cfg<F, 1, 2>(m, x, y, s, acc);
  return launch_cfg<F, 1, 1>(m, x, y, s, acc);
}

}  // namespace

int64_t matvec_max_cols(int dtype, int device) {
  const size_t lds = device_info(device).lds_max;
  // bytes of LDS per column: x (4) + half-chunk sums (8 per chunk) + padding
  // of the last 64-chunk group; solve conservatively per format.
  int64_t be = 256;
  switch (dtype) {
    case AQ_Q4_0: case AQ_Q4_1: case AQ_Q5_0: case AQ_Q5_1: case AQ_Q8_0:
    case AQ_F32: case AQ_F16: case AQ_BF16:
      be = 32;
      break;
    default:
      break;
  }
  int64_t k = 0;
  for (int64_t cand = be; cand <= (int64_t)1 << 20; cand += be) {
    size_t need = 0;
    const int64_t nb = cand / be;
    switch (dtype) {
      case AQ_Q4_K: need = matvec_lds_bytes<Q4K>(nb); break;
      case AQ_Q5_K: need = matvec_lds_bytes<Q5K>(nb); break;
      case AQ_Q6_K: need = matvec_lds_bytes<Q6K>(nb); break;
      case AQ_Q8_0: need = matvec_lds_bytes<Q80>(nb); break;
      case AQ_Q4_0: need = matvec_lds_bytes<Q40>(nb); break;
      case AQ_Q4_1: need = matvec_lds_bytes<Q41>(nb); break;
      case AQ_Q5_0: need = matvec_lds_bytes<Q50>(nb); break;
      case AQ_Q5_1: need = matvec_lds_bytes<Q51>(nb); break;
      case AQ_F32: need = matvec_lds_bytes<F32D>(nb); break;
      case AQ_F16: need = matvec_lds_bytes<F16D>(nb); break;
      case AQ_BF16: need = matvec_lds_bytes<BF16D>(nb); break;
      default: return 0;
    }
    if (need > lds) break;
    k = cand;
  }
  return k;
}

hipError_t launch_matvec(const aq_matrix *m, const float *x, float *y,
                         hipStream_t s, bool acc) {
  switch (m->dtype) {
    case AQ_Q4_K: return launch_fmt<Q4K>(m, x, y, s, acc);
    case AQ_Q5_K: return launch_fmt<Q5K>(m, x, y, s, acc);
    case AQ_Q6_K: return launch_fmt<Q6K>(m, x, y, s, acc);
    case AQ_Q8_0: return launch_fmt<Q80>(m, x, y, s, acc);
    case AQ_Q4_0: return launch_fmt<Q40>(m, x, y, s, acc);
    case AQ_Q4_1: return launch_fmt<Q41>(m, x, y, s, acc);
    case AQ_Q5_0: return launch_fmt<Q50>(m, x, y, s, acc);
    case AQ_Q5_1: return launch_fmt<Q51>(m, x, y, s, acc);
    case AQ_F32: return launch_fmt<F32D>(m, x, y, s, acc);
    case AQ_F16: return launch_fmt<F16D>(m, x, y, s, acc);
    case AQ_BF16: return launch_fmt<BF16D>(m, x, y, s, acc);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aq
