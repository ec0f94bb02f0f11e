// aq_matmul_h.hip - batched Y = X W^T on fp16 matrix cores with the weights
// kept as exact integers.
//
// Replaces QuantMatrix.matmul_t (alpacca/qmatrix.py:184-211) at float32
// accuracy.  The reference dequantizes f32 row tiles (w = d*sc*code -
// dmin*mn) and multiplies them with SGEMM.  Here the decode stops before
// the fp32 scales: per 32-element sub-block the product sc*code of a Q4_K
// weight is an integer of at most 945 (6-bit scale, 4-bit code), exact in
// fp16 as the subnormal sc*code * 2^-24, and the 6-bit min mn is exact too.
// The super-block scales d and dmin (fp16 fields, exact in fp32) are applied
// once per 256 weights in fp32:
//
//   Y[m][n] = sum_b  d[n][b] * P[m][n][b] - dmin[n][b] * Q[m][n][b]
//   P = sum_{k in b} (sc*code)[n][k] * x[m][k]     (v_mfma_f32_16x16x32_f16)
//   Q = sum_{sb in b} mn[n][sb] * S[m][sb]         (v_mfma_f32_16x16x16f16)
//
// with S the sub-block sums of x.  x itself is cut into fp16 pieces after a
// per-row power-of-two scale 2^e (the row maximum lands in [2^14, 2^15), so
// nothing overflows fp16): NP = 2 pieces carry 22 bits of every element
// (hi = fp16(x 2^e), lo = fp16(x 2^e - hi)), NP = 1 only hi (11 bits).  The
// products of 10-bit integers with fp16 pieces are exact in fp32, so the only
// roundings are the fp32 sums inside the matrix core, the scale products and
// the final 2^-e (exact).  The sub-block sums are formed in fp32 from the
// unscaled x and carried as two fp16 pieces at 2^(e-5).
//
// Q5_K runs the Q4_K kernel with the fifth code bit (sc*code <= 1953, still
// an exact half).  The per-32 block formats (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1)
// run k_mm_h_b32: one 16x16x32 product per block with the code exact, d per
// block in fp32.  Q6_K runs a kernel of its own (k_mm_h_q6k, below): q - 32 as exact fp16
// integers on v_mfma_f32_16x16x16f16, one 16-element scale group per
// instruction, and d * sc applied per group in fp32.
//
// Data flow (one workgroup: WGM x WGN waves, each MT x NT tiles of 16 x 16):
// the X pieces of the workgroup's rows are staged in LDS, 64 columns (two
// sub-blocks) per stage, double-buffered; every wave loads the weight bytes
// of its own NT x 16 rows straight into registers (8 bytes of codes per lane
// and stage, the 16-byte block header once per super-block) and builds the
// fp16 B operand there, so W never passes through LDS.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "aq_internal.h"

namespace aq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kStageK = 64;        // columns of X per LDS stage
constexpr int kXsSmall = 16;       // stages a whole-split X staging holds (one row of tiles)
constexpr int kLdA = kStageK + 16;  // halves per LDS row (160 B)

// ---- X preparation ---------------------------------------------------------
// One workgroup per row of X.  e[m] = 15 - E with max|x| = f 2^E, f in
// [0.5, 1) (0 for an all-zero row); piece planes xp[0] (hi) and xp[1] (lo),
// M x K halves each; xs[(m * (K / 256) + b) * 16 + j] = hi (j < 8) and lo
// (j >= 8) of the sum of sub-block j of super-block b, times 2^(e - 5).
// Sums are formed per 8 elements ((x0 + x1) + (x2 + x3)) + (...) and then
// over the four 8-element runs of a sub-block in pairs - one fixed order, the
// same for every M.  Thread t takes the 8-element runs j = 8 t + 2048 i.
// CH > 0 (K <= 2048 CH): all of the thread's runs are loaded at once and kept
// in registers, so the row is read in one memory round trip; CH = 0 reads
// the row twice (the maximum, then the pieces).
__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float run_max(const float (&v)[8]) {
  float mx = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mx = fmaxf(mx, fabsf(v[i]));
    nan = nan || !(v[i] == v[i]);
  }
  // a NaN anywhere makes the row's scale NaN-safe below (isfinite test)
  return nan ? INFINITY : mx;
}
__device__ __forceinline__ void load_run(const float *p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
// pieces and the sub-block sum of the run at column j.  Q6: the pieces in
// the Q6_K kernel's order - in every 64 columns, column 16k + 4q + i at
// position 32 (k / 2) + 8q + 4 (k % 2) + i (the 4-column units of the
// 16-column groups transposed per pair of groups), so that the units one
// lane takes from groups 0, 1 and from 2, 3 of a stage are 8 consecutive
// halves each, at the offsets the Q4_K kernel's fragment reads use
template <int NP, bool Q6 = false>
__device__ __forceinline__ void emit_run(const float (&v)[8], int64_t m, int64_t j, int64_t K,
                                         int e, int t, uint16_t *__restrict__ xp, int64_t plane,
                                         uint16_t *__restrict__ xs) {
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float s0 = __builtin_amdgcn_ldexpf(v[2 * i], e);
    const float s1 = __builtin_amdgcn_ldexpf(v[2 * i + 1], e);
    const _Float16 h0 = (_Float16)s0, h1 = (_Float16)s1;
    const _Float16 l0 = (_Float16)(s0 - (float)h0), l1 = (_Float16)(s1 - (float)h1);
    hi[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
            ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    lo[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
            ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
  }
  if constexpr (Q6) {
    const int64_t c = j & 63, k = c >> 4, q0 = (c & 15) >> 2;  // units q0, q0 + 1 of group k
    const int64_t d0 = m * K + (j - c) + 32 * (k >> 1) + 8 * q0 + 4 * (k & 1), d1 = d0 + 8;
    *reinterpret_cast<uint2 *>(xp + d0) = make_uint2(hi[0], hi[1]);
    *reinterpret_cast<uint2 *>(xp + d1) = make_uint2(hi[2], hi[3]);
    if (NP > 1) {
      *reinterpret_cast<uint2 *>(xp + plane + d0) = make_uint2(lo[0], lo[1]);
      *reinterpret_cast<uint2 *>(xp + plane + d1) = make_uint2(lo[2], lo[3]);
    }
  } else {
    *reinterpret_cast<uint4 *>(xp + m * K + j) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    if (NP > 1)
      *reinterpret_cast<uint4 *>(xp + plane + m * K + j) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }
  if (xs) {
    // sub-block sum: this thread's 8 elements, then the four threads of
    // the sub-block (lanes 4q .. 4q+3 hold one sub-block: j = 8t)
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    const float s1 = __shfl_xor(s, 1);
    s = (t & 1) ? s1 + s : s + s1;  // (s0 + s1) in both lanes of the pair
    const float s2 = __shfl_xor(s, 2);
    s = (t & 2) ? s2 + s : s + s2;  // (s01 + s23) in all four lanes
    if ((t & 3) == 0) {
      const int64_t nsb = K / 256;
      const float ss = __builtin_amdgcn_ldexpf(s, e - 5);
      const _Float16 h = (_Float16)ss, l = (_Float16)(ss - (float)h);
      const int64_t sb = j / 32, b = sb / 8, r = sb % 8;
      xs[(m * nsb + b) * 16 + r] = __builtin_bit_cast(uint16_t, h);
      xs[(m * nsb + b) * 16 + 8 + r] = __builtin_bit_cast(uint16_t, l);
    }
  }
}
template <int NP, int CH, bool Q6 = false>
__global__ void __launch_bounds__(256)
    k_x_h_pieces(const float *__restrict__ X, int64_t K, uint16_t *__restrict__ xp,
                 int64_t plane, int32_t *__restrict__ xe, uint16_t *__restrict__ xs) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const float *xr = X + m * K;
  const int t = threadIdx.x;
  float v[CH > 0 ? CH : 1][8];
  float mx = 0.f;
  if constexpr (CH > 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t j = 8 * (int64_t)t + 2048 * c;
      if (j < K) load_run(xr + j, v[c]);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c)
      if (8 * (int64_t)t + 2048 * c < K) mx = fmaxf(mx, run_max(v[c]));
  } else {
    for (int64_t j = 8 * (int64_t)t; j < K; j += 2048) {
      load_run(xr + j, v[0]);
      mx = fmaxf(mx, run_max(v[0]));
    }
  }
  mx = wave_max(mx);
  if ((t & 63) == 0) red[t >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // a non-finite row keeps e = 0: its infinities and NaNs reach the outputs
  const int e = (mx > 0.f && mx < INFINITY) ? 15 - __builtin_amdgcn_frexp_expf(mx) : 0;
  if (t == 0) xe[m] = e;
  if constexpr (CH > 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t j = 8 * (int64_t)t + 2048 * c;
      if (j < K) emit_run<NP, Q6>(v[c], m, j, K, e, t, xp, plane, xs);
    }
  } else {
    for (int64_t j = 8 * (int64_t)t; j < K; j += 2048) {
      load_run(xr + j, v[0]);
      emit_run<NP, Q6>(v[0], m, j, K, e, t, xp, plane, xs);
    }
  }
}

// X pieces of an M x K matrix (K a multiple of 256); Q6: in the Q6_K
// kernel's column order
template <int NP, bool Q6 = false>
void launch_x_h_pieces(const float *X, int64_t M, int64_t K, uint16_t *xp, int64_t plane,
                       int32_t *xe, uint16_t *xs, hipStream_t s) {
#define AQ_XH(ch) \
  hipLaunchKernelGGL((k_x_h_pieces<NP, ch, Q6>), dim3((unsigned)M), dim3(256), 0, s, X, K, xp, \
                     plane, xe, xs)
  if (K <= 2048) AQ_XH(1);
  else if (K <= 4096) AQ_XH(2);
  else if (K <= 8192) AQ_XH(4);
  else if (K <= 16384) AQ_XH(8);
  else AQ_XH(0);
#undef AQ_XH
}

// ---- the B operand: sc * code as fp16 subnormals, from packed code bytes ---
// sc * code of a Q4_K weight is an integer m below 1024 (6-bit scale, 4-bit
// code), and the fp16 half whose bits are m is the subnormal m 2^-24: exact,
// and exactly multiplied by the matrix core (fp16 subnormal inputs are
// kept).  A byte permute puts two codes (low nibbles, or high nibbles
// shifted down) into the low bytes of two halves with zero high bytes, and
// one packed 16-bit integer multiply by (sc, sc) gives the two B values.
// The 2^24 goes with the super-block scale d.
__device__ __forceinline__ uint32_t fma_h2(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_bit_cast(
      uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b),
                                          __builtin_bit_cast(h2, c)));
}
__device__ __forceinline__ uint32_t mul_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}
// 8 values from two words of codes (one per byte, below 16), in byte order,
// times sc2 = (sc, sc)
__device__ __forceinline__ void sc_codes8(uint32_t c0, uint32_t c1, uint32_t sc2, uint32_t *o) {
  o[0] = mul_u16x2(__builtin_amdgcn_perm(0u, c0, 0x0C010C00u), sc2);
  o[1] = mul_u16x2(__builtin_amdgcn_perm(0u, c0, 0x0C030C02u), sc2);
  o[2] = mul_u16x2(__builtin_amdgcn_perm(0u, c1, 0x0C010C00u), sc2);
  o[3] = mul_u16x2(__builtin_amdgcn_perm(0u, c1, 0x0C030C02u), sc2);
}

// The SwiGLU of a (gate, up) pair, rounded operation by operation as the
// reference's NumPy expression (model.py:513) and the library's elementwise
// SwiGLU kernel are.
__device__ __forceinline__ float swiglu_pair(float g, float u) {
#pragma clang fp contract(off)
  return g / (1.0f + expf(-g)) * u;
}

// byte-granular buffer loads (offsets past the resource read zeros)
__device__ __forceinline__ uint2 rsrc_u2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
// Lane group g (lanes 16 g .. 16 g + 15) holds words (w0 .. w3) = row g of a
// 4 x 4 matrix T of words (per lane of the group); afterwards it holds
// column g: w_j = T[j][g].  Two stages of gfx950 row swaps, which exchange
// the odd rows of their first operand with the even rows of the second:
// 32-lane rows swap the off-diagonal 2 x 2 blocks, then 16-lane rows
// transpose within the blocks.  Every lane of the wave must be active.
__device__ __forceinline__ void transpose_groups(uint32_t &w0, uint32_t &w1, uint32_t &w2,
                                                 uint32_t &w3) {
  const auto a = __builtin_amdgcn_permlane32_swap(w0, w2, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w1, w3, false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  w0 = c[0];
  w1 = c[1];
  w2 = d[0];
  w3 = d[1];
}

// Lane group g holds chunk (0, 2, 1, 3)[g] of a 64-byte run as (v.x, v.y,
// v.z, v.w); afterwards (v.x, v.y) are bytes 8 g .. 8 g + 7 of the run's
// first 32 bytes and (v.z, v.w) those of its second 32: two 16-lane row
// swaps (odd lane groups' first words for even groups' second words).
// Every lane of the wave must be active.
__device__ __forceinline__ void pair_words(uint4 &v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v.x, v.z, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(v.y, v.w, false, false);
  v.x = a[0];
  v.z = a[1];
  v.y = b[0];
  v.w = b[1];
}
// the chunk of a 64-byte run that lane group g loads for pair_words
__device__ __forceinline__ uint32_t pair_chunk(int g) {
  return 16u * (uint32_t)(((g & 1) << 1) | (g >> 1));
}

__device__ __forceinline__ uint4 rsrc_u4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// ---- main kernel (Q4_K) --------------------------------------------------------
// Lane l of a 16 x 16 tile: A row l%16 and B column l%16 with k = 8 (l/16) ..
// +7 of each 32-column sub-block (the same k set for A and B, so the matrix
// core sums over every k), D rows 4 (l/16) .. +3 of column l%16.  Q4_K
// sub-block 2c is the low nibbles of qs[32c, 32c + 32), 2c+1 the high nibbles
// (quants.py:136-161): lane group g takes bytes 32c + 8g .. +7, i.e. elements
// 8g .. 8g+7 of both sub-blocks, in natural order.  One loop iteration is a
// super-block (four stages c = 0..3, each two sub-blocks), so every index
// into the register sets is a compile-time one.
//
// XS > 0: the whole split's X pieces (at most XS stages) are staged into LDS
// before the loop, behind one barrier, and the stage loop has neither X
// loads nor barriers: for a few rows of X a stage's work is much shorter
// than the X round trip, which the two-stage form then waits for every stage.
//
// FX (with XS, one 16-row tile of 256 threads): the workgroup makes its X
// pieces itself from the fp32 rows Xf, with a power-of-two scale e per row
// over the split's own columns (the split's maximum in [2^14, 2^15)), and
// writes its partial as acc 2^-e: no separate preparation launch.  The
// pieces of an element are its pieces under the whole-row scale shifted by
// a power of two (exact unless the element falls among fp16 subnormals,
// where the split's larger scale keeps more of its bits), and the sub-block
// sums are formed in the preparation kernel's order, so the outputs are
// those of the two-launch form.  The sub-block sums and the exponents live
// in the padding columns 64..79 of the staged rows, which the matrix-core
// reads never touch: super-block bb's sums at As[4 bb][0][r][64..79] (hi
// 0..7, lo 8..15), row r's exponent at As[0][1][r][64..65].
//
// Q5 (Q5_K): the same kernel with a fifth code bit from the qh plane: bit 2c
// (low nibbles) and 2c+1 (high nibbles) of qh byte l for element l of
// sub-blocks 2c, 2c+1 (quants.py:164-193), so a lane's bits for a whole
// super-block are qh bytes 8g .. 8g+7, loaded with the header.  sc*code is
// then at most 63 * 31 = 1953: below 2048, the fp16 half whose bits are that
// integer m is still m 2^-24 exactly (a normal half from 1024 on).
template <int NP, int MT, int NT, int WGM, int WGN, int XS = 0, bool FX = false, bool Q5 = false>
__global__ void __launch_bounds__(64 * WGM * WGN)
    k_mm_h_q4k(const uint8_t *qs, const uint8_t *hd, uint32_t qs_stride, uint32_t hd_stride,
               int64_t N, int nb_row, const uint16_t *__restrict__ xp, int64_t plane,
               const int32_t *__restrict__ xe, const uint16_t *__restrict__ xs, int64_t M,
               float *__restrict__ Y, int sb_per_split, const float *__restrict__ Xf,
               const uint8_t *qhp, uint32_t qh_stride, float *__restrict__ Ysw) {
  constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
  constexpr int BM = WGM * MT * 16, BN = WGN * NT * 16;
  // fused X staging: 256 threads per set of stages (XH sets, interleaved)
  constexpr int XH = THREADS / 256;
  static_assert(!FX || (XS > 0 && BM == 16 && (THREADS == 256 || THREADS == 512) && NP == 2 &&
                        XS % XH == 0),
                "the fused X staging is laid out for one 16-row tile of 256 or 512 threads");
  __shared__ __attribute__((aligned(16))) uint16_t As[XS > 0 ? XS : 2][NP][BM * kLdA];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K = (int64_t)nb_row * 256;
  const int b_begin = (int)blockIdx.z * sb_per_split;
  const int b_end = std::min(b_begin + sb_per_split, nb_row);
  Y += (int64_t)blockIdx.z * M * N;

  // weights: one buffer resource per plane, over the rows that exist (the
  // launcher keeps them below 2^31 bytes)
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(qs), 0, (int)(N * nb_row * qs_stride), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(hd), 0, (int)(N * nb_row * hd_stride), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t r5 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(qhp), 0, Q5 ? (int)(N * nb_row * qh_stride) : 0, kRsrcWord3);
  // X pieces and sums: rows past M read zeros
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(xp), 0, (int)(2 * NP * plane), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(xs), 0, (int)(M * nb_row * 32), kRsrcWord3);
  constexpr uint32_t kNone = 0x7fffffffu;  // an offset past every resource

  uint32_t rowq[NT], rowh[NT], row5[NT];  // byte offsets of this lane's rows (block 0)
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t n = n0 + (wn * NT + j) * 16 + c16;
    // (+ the 16-byte chunk this lane group loads of a stage pair: w_load)
    rowq[j] = n < N ? (uint32_t)(n * nb_row * qs_stride) + pair_chunk(g) : kNone;
    rowh[j] = n < N ? (uint32_t)(n * nb_row * hd_stride) : kNone;
    row5[j] = Q5 && n < N ? (uint32_t)(n * nb_row * qh_stride) + 8 * g : kNone;
  }

  // staging of one 64-column stage of X: BM rows x 8 uint4 per piece
  constexpr int SQ = BM * 8 * NP;                    // uint4 per stage
  constexpr int SPT = (SQ + THREADS - 1) / THREADS;  // per thread
  const int n_st = 4 * (b_end - b_begin);
  uint4 sreg[2][SPT];
  auto stage_load = [&](int stg, uint4 *dst) {  // stage stg of the split (zeros past it)
    const int64_t k0 = (int64_t)b_begin * 256 + 64 * (int64_t)stg;
    const bool live = stg < n_st;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
      const int64_t row = m0 + r;
      const bool ok = live && q < SQ && row < M;
      dst[i] = rsrc_u4(rx, ok ? (uint32_t)(2 * ((int64_t)p * plane + row * K + k0 + 8 * s)) : kNone);
    }
  };
  auto stage_store = [&](const uint4 *src, int buf) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      if (SQ % THREADS == 0 || q < SQ) {
        const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
        *reinterpret_cast<uint4 *>(&As[buf][p][r * kLdA + 8 * s]) = src[i];
      }
    }
  };
  // code bytes of split stage stg (zeros past the split)
  // code bytes of split stages 2 pr and 2 pr + 1 (zeros past the split): the
  // pair's 64 bytes of a row are four 16-byte chunks, lane group g loads
  // chunk (0, 2, 1, 3)[g], and two 16-lane row swaps (pair_words) leave each
  // lane group its 8 bytes of either stage (bytes 8 g .. 8 g + 7 of each
  // stage's 32) in place of two 8-byte loads per pair
  auto w_load = [&](int pr, uint4 *dst) {
    const int stg = 2 * pr, b = b_begin + stg / 4, c = stg % 4;
#pragma unroll
    for (int j = 0; j < NT; ++j)
      dst[j] = rsrc_u4(rq, stg < n_st && rowq[j] != kNone
                               ? rowq[j] + (uint32_t)b * qs_stride + 32 * c : kNone);
  };
  auto h_load = [&](int b, uint4 *dst, uint2 *dq5) {  // header (and Q5's qh bytes)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      dst[j] = rsrc_u4(rh, b < b_end && rowh[j] != kNone ? rowh[j] + (uint32_t)b * hd_stride
                                                         : kNone);
      if constexpr (Q5)
        dq5[j] = rsrc_u2(r5, b < b_end && row5[j] != kNone ? row5[j] + (uint32_t)b * qh_stride
                                                           : kNone);
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Loads run well ahead of their use, since a stage's own work is shorter
  // than a memory round trip: the code bytes of stages s + 3, s + 4 are
  // issued as soon as stages s - 1, s have turned theirs into B operands (two
  // register sets of a stage pair each),
  // the X pieces of stage s + 2 at the start of stage s (two register sets,
  // stored to LDS at the end of stage s + 1), the next super-block's header
  // and this one's sub-block sums at its first stage.
  uint4 hdr[NT], hdn[NT];
  uint4 wq[2][NT];
  uint2 xsv[MT], q5r[NT], q5n[NT];
  h_load(b_begin, hdr, q5r);
  w_load(0, wq[0]);
  w_load(1, wq[1]);
  if constexpr (FX) {
    // thread t: row t / 16 % 16, columns 4 (t % 16) .. +3 of stages
    // XH i + t / 256 (every stage with 256 threads, every other with 512)
    const int r = (tid >> 4) & 15, q = tid & 15, hs = tid >> 8;
    const int64_t row = m0 + r;
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(Xf), 0, (int)(M * K * 4), kRsrcWord3);
    constexpr int XT = XS / XH;  // stages per thread
    f32x4 xv[XT];
#pragma unroll
    for (int i = 0; i < XT; ++i) {
      const int st = XH * i + hs;
      xv[i] = __builtin_bit_cast(
          f32x4, rsrc_u4(rf, st < n_st && row < M
                                 ? (uint32_t)(4 * (row * K + (int64_t)b_begin * 256 + 64 * st + 4 * q))
                                 : kNone));
    }
    float mx = 0.f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < XT; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        mx = fmaxf(mx, fabsf(xv[i][k]));
        nan = nan || !(xv[i][k] == xv[i][k]);
      }
    if (nan) mx = INFINITY;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if constexpr (XH > 1) {  // the row's two halves meet in a padding slot of stage 1's lo piece
      float *slot = reinterpret_cast<float *>(&As[1][1][r * kLdA + 64]);
      if (q == 0) slot[hs] = mx;
      __syncthreads();
      mx = fmaxf(slot[0], slot[1]);
    }
    // a non-finite row keeps e = 0: its infinities and NaNs reach the outputs
    const int e = (mx > 0.f && mx < INFINITY) ? 15 - __builtin_amdgcn_frexp_expf(mx) : 0;
    if (q == 0 && hs == 0) *reinterpret_cast<int32_t *>(&As[0][1][r * kLdA + 64]) = e;
#pragma unroll
    for (int i = 0; i < XT; ++i) {  // (stages past the split: zeros, never read)
      const int st = XH * i + hs;
      uint32_t hi[2], lo[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float s0 = __builtin_amdgcn_ldexpf(xv[i][2 * k], e);
        const float s1 = __builtin_amdgcn_ldexpf(xv[i][2 * k + 1], e);
        const _Float16 h0 = (_Float16)s0, h1 = (_Float16)s1;
        const _Float16 l0 = (_Float16)(s0 - (float)h0), l1 = (_Float16)(s1 - (float)h1);
        hi[k] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        lo[k] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      }
      *reinterpret_cast<uint2 *>(&As[st][0][r * kLdA + 4 * q]) = make_uint2(hi[0], hi[1]);
      *reinterpret_cast<uint2 *>(&As[st][1][r * kLdA + 4 * q]) = make_uint2(lo[0], lo[1]);
      // sub-block sum in the preparation kernel's order: per 8-element run
      // ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)) (two threads), then
      // the four runs in pairs (threads q ^ 2, then q ^ 4)
      float a = (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);
      a = a + __shfl_xor(a, 1);
      a = a + __shfl_xor(a, 2);
      a = a + __shfl_xor(a, 4);
      if ((q & 7) == 0) {
        const float ss = __builtin_amdgcn_ldexpf(a, e - 5);
        const _Float16 h = (_Float16)ss, l = (_Float16)(ss - (float)h);
        const int r8 = 2 * (st % 4) + (q >> 3);
        As[st & ~3][0][r * kLdA + 64 + r8] = __builtin_bit_cast(uint16_t, h);
        As[st & ~3][0][r * kLdA + 72 + r8] = __builtin_bit_cast(uint16_t, l);
      }
    }
  } else if constexpr (XS > 0) {
    // every stage's loads first, then the stores (the launcher keeps n_st <= XS)
    uint4 sall[XS][SPT];
#pragma unroll
    for (int st = 0; st < XS; ++st) stage_load(st, sall[st]);
#pragma unroll
    for (int st = 0; st < XS; ++st)
      if (st < n_st) stage_store(sall[st], st);
  } else {
    stage_load(0, sreg[0]);
    stage_load(1, sreg[1]);
    stage_store(sreg[0], 0);
  }
  __syncthreads();

  // one super-block; hdr holds its header, hdn receives the next one (the
  // loop runs two super-blocks per iteration with the two sets swapped, so
  // no copy ties a pending load to the loop edge)
  auto superblock = [&](int b, uint4 (&hdr)[NT], uint4 (&hdn)[NT], uint2 (&q5r)[NT],
                        uint2 (&q5n)[NT]) {
    h_load(b + 1, hdn, q5n);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int64_t row = m0 + (wm * MT + i) * 16 + c16;
      if constexpr (FX)
        xsv[i] = *reinterpret_cast<const uint2 *>(&As[4 * (b - b_begin)][0][c16 * kLdA + 64 + 4 * g]);
      else
        xsv[i] = rsrc_u2(rs, row < M ? (uint32_t)(((row * nb_row + b) * 16 + 4 * g) * 2) : kNone);
    }
    f32x4 P[MT][NT];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int stg = 4 * (b - b_begin) + c;
      if constexpr (XS == 0) stage_load(stg + 2, sreg[c & 1]);
      // B operands of the two sub-blocks 2c, 2c+1 of every n-tile
      uint32_t blo[NT][4], bhi[NT][4];
      if (c % 2 == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) pair_words(wq[c >> 1][j]);
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        uint32_t sc, mn;
        kquant_scale_pair(hdr[j].y, hdr[j].z, hdr[j].w, c, sc, mn);
        const uint4 &wp = wq[c >> 1][j];
        const uint2 w = c % 2 == 0 ? uint2{wp.x, wp.y} : uint2{wp.z, wp.w};
        const uint32_t sl = sc & 0xFFu, sh = sc >> 8;
        uint32_t l0 = w.x & 0x0F0F0F0Fu, l1 = w.y & 0x0F0F0F0Fu;
        uint32_t h0 = (w.x >> 4) & 0x0F0F0F0Fu, h1 = (w.y >> 4) & 0x0F0F0F0Fu;
        if constexpr (Q5) {  // the fifth bit: 16 when set
          l0 |= ((q5r[j].x >> (2 * c)) & 0x01010101u) << 4;
          l1 |= ((q5r[j].y >> (2 * c)) & 0x01010101u) << 4;
          h0 |= ((q5r[j].x >> (2 * c + 1)) & 0x01010101u) << 4;
          h1 |= ((q5r[j].y >> (2 * c + 1)) & 0x01010101u) << 4;
        }
        sc_codes8(l0, l1, sl | (sl << 16), blo[j]);
        sc_codes8(h0, h1, sh | (sh << 16), bhi[j]);
      }
      if (c % 2 == 1) w_load((stg + 3) / 2, wq[c >> 1]);  // stages stg + 3, stg + 4
      const int buf = XS > 0 ? stg : c & 1;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = (wm * MT + i) * 16 + c16;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const h8 alo = *reinterpret_cast<const h8 *>(&As[buf][p][r * kLdA + 8 * g]);
          const h8 ahi = *reinterpret_cast<const h8 *>(&As[buf][p][r * kLdA + 32 + 8 * g]);
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            const f32x4 c0 = (c == 0 && p == 0) ? f32x4{0.f, 0.f, 0.f, 0.f} : P[i][j];
            P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                alo, __builtin_bit_cast(h8, u32x4{blo[j][0], blo[j][1], blo[j][2], blo[j][3]}),
                c0, 0, 0, 0);
            P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                ahi, __builtin_bit_cast(h8, u32x4{bhi[j][0], bhi[j][1], bhi[j][2], bhi[j][3]}),
                P[i][j], 0, 0, 0);
          }
        }
      }
      if constexpr (XS == 0) {
        stage_store(sreg[(c + 1) & 1], buf ^ 1);  // stage stg + 1, loaded at stage stg - 1
        __syncthreads();
      }
    }
    // super-block end: the min term and the fp32 scales
    float d[NT], dm32[NT];
    h4 bm[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      d[j] = f16_bits_to_f32(hdr[j].x) * 16777216.f;  // P is in units of 2^-24
      dm32[j] = -32.f * f16_bits_to_f32(hdr[j].x >> 16);  // S carries 2^(e-5)
      uint32_t sc0, mn0, sc1, mn1;
      kquant_scale_pair(hdr[j].y, hdr[j].z, hdr[j].w, 2 * (g & 1), sc0, mn0);
      kquant_scale_pair(hdr[j].y, hdr[j].z, hdr[j].w, 2 * (g & 1) + 1, sc1, mn1);
      const uint32_t mn4 = mn0 | (mn1 << 16);  // mn of sub-blocks 4(g&1) .. +3, one per byte
      bm[j] = __builtin_bit_cast(
          h4, uint2{fma_h2(__builtin_amdgcn_perm(0x64646464u, mn4, 0x05010400u), 0x3c003c00u,
                           0xe400e400u),
                    fma_h2(__builtin_amdgcn_perm(0x64646464u, mn4, 0x05030402u), 0x3c003c00u,
                           0xe400e400u)});
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const h4 as = __builtin_bit_cast(h4, xsv[i]);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const f32x4 q = __builtin_amdgcn_mfma_f32_16x16x16f16(as, bm[j], f32x4{0.f, 0.f, 0.f, 0.f},
                                                              0, 0, 0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          acc[i][j][rr] = fmaf(d[j], P[i][j][rr], acc[i][j][rr]);
          acc[i][j][rr] = fmaf(dm32[j], q[rr], acc[i][j][rr]);
        }
      }
    }
  };
  int b = b_begin;
  for (; b + 1 < b_end; b += 2) {
    superblock(b, hdr, hdn, q5r, q5n);
    superblock(b + 1, hdn, hdr, q5n, q5r);
  }
  if (b < b_end) superblock(b, hdr, hdn, q5r, q5n);
  // Y = acc 2^-e (per row), rows past M and columns past N not stored.
  // Ysw (an unsplit launch over interleaved gate/up rows, N even): the pair
  // of columns 2p, 2p+1 sits in lanes c16, c16 ^ 1 of one row, and the
  // M x N/2 output takes silu(gate) * up at column p instead.  Of each two
  // rows rr, rr + 1 the even lane forms row rr's pair and the odd lane row
  // rr + 1's, one exchanged value each (gate of rr + 1 one way, up of rr the
  // other).
  const bool odd = c16 & 1;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    int64_t row[4];
    bool live[4];
    int ex[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      row[rr] = m0 + (wm * MT + i) * 16 + 4 * g + rr;
      live[rr] = row[rr] < M;
      ex[rr] = FX ? *reinterpret_cast<const int32_t *>(&As[0][1][(4 * g + rr) * kLdA + 64])
                  : (live[rr] ? xe[row[rr]] : 0);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t n = n0 + (wn * NT + j) * 16 + c16;
      float v[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) v[rr] = __builtin_amdgcn_ldexpf(acc[i][j][rr], -ex[rr]);
      if (Ysw) {
#pragma unroll
        for (int rr = 0; rr < 4; rr += 2) {
          const float mine = odd ? v[rr] : v[rr + 1];  // what the partner lane needs
          const float got = __shfl_xor(mine, 1);
          const int r = odd ? rr + 1 : rr;
          const float out = odd ? swiglu_pair(got, v[rr + 1]) : swiglu_pair(v[rr], got);
          if (live[r] && n < N) Ysw[row[r] * (N >> 1) + (n >> 1)] = out;
        }
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (live[rr] && n < N) Y[row[rr] * N + n] = v[rr];
      }
    }
  }
}


// ---- main kernel (Q6_K) ------------------------------------------------------
// Q6_K weights are d * sc * (q - 32) with a 6-bit code q, an int8 scale sc
// per 16 elements and an fp16 d per 256 (quants.py:196-224): (q - 32) is an
// exact small fp16 integer, but sc * (q - 32) reaches 4096 in magnitude, past
// the exact integers of the B operand.  So the scale stays out of B: every
// 16-element scale group is one v_mfma_f32_16x16x16f16 per X piece (K = 16:
// lane group g holds elements 4g .. 4g+3 of the group), P_G = sum x (q - 32)
// with exact products, and the group's d * sc (exact in fp32) is applied to
// P_G by one fma per output in fp32.  B from the packed codes: a byte
// permute puts code bytes under 0x64 (the half 1024 + q) and one packed fp16
// fma by (1, -1056) leaves q - 32 exactly.
//
// Elements 16G + 4g .. +3 of super-block group G (half hf = G / 8, nibble
// h = G / 4 % 2, k = G % 4 = 2u + kk) are the low (h = 0) or high (h = 1)
// nibbles of ql bytes 64 hf + 16 k + 4g .. +3, with two high bits from qh
// bytes 32 hf + 16 kk + 4g .. +3 at shift 2u + 4h (the layout of
// quants.py:447-466): per half a lane loads four ql words and two qh words,
// which serve both of the half's stages.  Stage c of a super-block (64
// columns) holds groups 4c .. 4c+3, so c = 2 hf + h.
template <int NP, int MT, int NT, int WGM, int WGN>
__global__ void __launch_bounds__(64 * WGM * WGN)
    k_mm_h_q6k(const uint8_t *ql, const uint8_t *qh, const uint8_t *scl, const uint8_t *dp,
               int64_t N, int nb_row, const uint16_t *__restrict__ xp, int64_t plane,
               const int32_t *__restrict__ xe, int64_t M, float *__restrict__ Y,
               int sb_per_split) {
  constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
  constexpr int BM = WGM * MT * 16, BN = WGN * NT * 16;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NP][BM * kLdA];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K = (int64_t)nb_row * 256;
  const int b_begin = (int)blockIdx.z * sb_per_split;
  const int b_end = std::min(b_begin + sb_per_split, nb_row);
  Y += (int64_t)blockIdx.z * M * N;

  // the four planes (dense, SPLIT layout), over the rows that exist (the
  // launcher keeps them below 2^31 bytes); X pieces: rows past M read zeros
  const int64_t nblk = N * nb_row;
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(ql), 0, (int)(nblk * 128), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(qh), 0, (int)(nblk * 64), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(scl), 0, (int)(nblk * 16), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(dp), 0, (int)(nblk * 2), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(xp), 0, (int)(2 * NP * plane), kRsrcWord3);
  constexpr uint32_t kNone = 0x7fffffffu;

  int64_t blk0[NT];  // first block of this lane's rows (-1 past N)
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t n = n0 + (wn * NT + j) * 16 + c16;
    blk0[j] = n < N ? n * nb_row : -1;
  }

  // the weight words of one super-block for every n-tile, in two register
  // sets (set S of wl/wh/wsc/wd; S is always a compile-time index).  Lane
  // group g needs word g of each 16-byte chunk of a 64-byte run (ql bytes
  // 64 hf + 16 k + 4 g, qh bytes 16 c + 4 g): it loads chunk g whole (one
  // 16-byte load) and the four lane groups transpose their words
  // (transpose_groups), in place of four 4-byte loads at 16-byte strides.
  uint32_t wl[2][NT][8], wh[2][NT][4], wsc[2][NT][4], wd[2][NT];
  auto w_load = [&](int b, auto set) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bool ok = b < b_end && blk0[j] >= 0;
      const uint32_t blk = ok ? (uint32_t)(blk0[j] + b) : 0u;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint4 cl = rsrc_u4(rl, ok ? blk * 128 + 64 * hf + 16 * g : kNone);
        wl[S][j][4 * hf + 0] = cl.x;
        wl[S][j][4 * hf + 1] = cl.y;
        wl[S][j][4 * hf + 2] = cl.z;
        wl[S][j][4 * hf + 3] = cl.w;
      }
      const uint4 ch = rsrc_u4(rh, ok ? blk * 64 + 16 * g : kNone);
      wh[S][j][0] = ch.x;
      wh[S][j][1] = ch.y;
      wh[S][j][2] = ch.z;
      wh[S][j][3] = ch.w;
      const u32x4 sv = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? (int)(blk * 16) : (int)kNone, 0, 0));
#pragma unroll
      for (int q = 0; q < 4; ++q) wsc[S][j][q] = sv[q];
      wd[S][j] = __builtin_amdgcn_raw_buffer_load_b16(rd, ok ? (int)(blk * 2) : (int)kNone, 0, 0);
    }
  };

  // staging of one 64-column stage of X: BM rows x 8 uint4 per piece
  constexpr int SQ = BM * 8 * NP;
  constexpr int SPT = (SQ + THREADS - 1) / THREADS;
  const int n_st = 4 * (b_end - b_begin);
  uint4 sreg[2][SPT];
  auto stage_load = [&](int stg, uint4 *dst) {
    const int64_t k0 = (int64_t)b_begin * 256 + 64 * (int64_t)stg;
    const bool live = stg < n_st;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
      const int64_t row = m0 + r;
      const bool ok = live && q < SQ && row < M;
      dst[i] = rsrc_u4(rx, ok ? (uint32_t)(2 * ((int64_t)p * plane + row * K + k0 + 8 * s)) : kNone);
    }
  };
  auto stage_store = [&](const uint4 *src, int buf) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      if (SQ % THREADS == 0 || q < SQ) {
        const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
        *reinterpret_cast<uint4 *>(&As[buf][p][r * kLdA + 8 * s]) = src[i];
      }
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // X pieces two stages ahead (two register sets), the next super-block's
  // weight words at the start of each super-block (set 1, moved to set 0)
  w_load(b_begin, std::integral_constant<int, 0>{});
  stage_load(0, sreg[0]);
  stage_load(1, sreg[1]);
  stage_store(sreg[0], 0);
  __syncthreads();

  auto superblock = [&](int b, auto set) {
    constexpr int S = decltype(set)::value;
    w_load(b + 1, std::integral_constant<int, 1 - S>{});
    // set S's 16-byte chunks into each lane group's words (w_load)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      transpose_groups(wl[S][j][0], wl[S][j][1], wl[S][j][2], wl[S][j][3]);
      transpose_groups(wl[S][j][4], wl[S][j][5], wl[S][j][6], wl[S][j][7]);
      transpose_groups(wh[S][j][0], wh[S][j][1], wh[S][j][2], wh[S][j][3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int stg = 4 * (b - b_begin) + c;
      stage_load(stg + 2, sreg[c & 1]);
      const int hf = c >> 1, h = c & 1, buf = c & 1;
      // B operands and scales of the stage's four groups
      h4 bop[4][NT];
      float dsc[4][NT];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int u = k >> 1, kk = k & 1, G = 4 * c + k;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const uint32_t codes = ((wl[S][j][4 * hf + k] >> (4 * h)) & 0x0F0F0F0Fu) |
                                 (((wh[S][j][2 * hf + kk] >> (2 * u + 4 * h)) & 0x03030303u) << 4);
          bop[k][j] = __builtin_bit_cast(
              h4, uint2{fma_h2(__builtin_amdgcn_perm(0x64646464u, codes, 0x05010400u),
                               0x3c003c00u, 0xe420e420u),
                        fma_h2(__builtin_amdgcn_perm(0x64646464u, codes, 0x05030402u),
                               0x3c003c00u, 0xe420e420u)});
          dsc[k][j] = f16_bits_to_f32(wd[S][j] & 0xFFFFu) * sbyte(wsc[S][j][G >> 2], G & 3);
        }
      }
      // X pieces in the transposed order: lane group g's units of groups 0,
      // 1 are halves 8g .. 8g+7 of the stage row, of groups 2, 3 halves
      // 32 + 8g .. +7 (two 16-byte reads)
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = (wm * MT + i) * 16 + c16;
        f32x4 P[4][NT];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const h8 a0 = *reinterpret_cast<const h8 *>(&As[buf][p][r * kLdA + 8 * g]);
          const h8 a1 = *reinterpret_cast<const h8 *>(&As[buf][p][r * kLdA + 32 + 8 * g]);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const h8 &ak = k < 2 ? a0 : a1;
            const h4 a = (k & 1) ? h4{ak[4], ak[5], ak[6], ak[7]} : h4{ak[0], ak[1], ak[2], ak[3]};
#pragma unroll
            for (int j = 0; j < NT; ++j)
              P[k][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                  a, bop[k][j], p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : P[k][j], 0, 0, 0);
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              acc[i][j][rr] = fmaf(dsc[k][j], P[k][j][rr], acc[i][j][rr]);
      }
      stage_store(sreg[(c + 1) & 1], buf ^ 1);  // stage stg + 1, loaded at stage stg - 1
      __syncthreads();
    }
  };
  // One super-block per iteration, the prefetched set moved into the working
  // one at the loop edge: a super-block's work is several memory round trips
  // long, so the wait that move implies costs nothing, and the loop unrolled
  // by two (two sets in turn, as the Q4_K kernel runs) spilled registers.
  for (int b = b_begin; b < b_end; ++b) {
    superblock(b, std::integral_constant<int, 0>{});
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int q = 0; q < 8; ++q) wl[0][j][q] = wl[1][j][q];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        wh[0][j][q] = wh[1][j][q];
        wsc[0][j][q] = wsc[1][j][q];
      }
      wd[0][j] = wd[1][j];
    }
  }
  // Y = acc 2^-e (per row), rows past M and columns past N not stored
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int64_t row = m0 + (wm * MT + i) * 16 + 4 * g + rr;
      if (row >= M) continue;
      const int e = xe[row];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t n = n0 + (wn * NT + j) * 16 + c16;
        if (n < N) Y[row * N + n] = __builtin_amdgcn_ldexpf(acc[i][j][rr], -e);
      }
    }
  }
}

// ---- main kernel (per-32 block formats: Q8_0, Q4_0, Q4_1, Q5_0, Q5_1) --------
// A 32-element block is one v_mfma_f32_16x16x32_f16 per X piece (lane group g
// holds elements 8g .. 8g+7, natural order) and the block's d is applied to
// that product by one fma per output in fp32.  B is the block's code, exact:
// with an offset (Q8_0: the int8 code as q + 128 after flipping its sign
// bit, offset 128; Q4_0: nibble - 8; Q5_0: code - 16) a byte permute puts
// the code under 0x64 (the half 1024 + code) and one packed fp16 fma by
// (1, -(1024 + offset)) leaves code - offset; the min formats (Q4_1, Q5_1:
// d code + m) use the code itself as a subnormal half (bits = code, value
// code 2^-24, with 2^24 put into d), and their m term is summed per 8 blocks
// by one v_mfma_f32_16x16x16f16 of the blocks' x sums against their m, as
// the Q4_K kernel's min term (quants.py:50-124).  Codes: Q8_0 bytes 8g .. +7
// of qs; nibble formats bytes 8 (g & 1) .. +7, low nibbles for g < 2, high
// for g >= 2; Q5 formats bits 8g .. 8g+7 of qh as the fifth bit.  Groups of 8
// blocks (256 columns, the X preparation's unit), four stages each.
template <int QSB, bool NIB, bool HIGH, bool MIN, int OFF>
struct B32Fmt {
  static constexpr int kQsBytes = QSB;      // code bytes per block
  static constexpr bool kNib = NIB;         // 4-bit codes (two per byte)
  static constexpr bool kHigh = HIGH;       // fifth bit plane (u32 per block)
  static constexpr bool kMin = MIN;         // scale plane holds d and m
  static constexpr int kOff = OFF;          // code offset (0 with a min)
  static constexpr uint32_t kXor = QSB == 32 ? 0x80808080u : 0u;  // int8 -> q + 128
};
using B32Q80 = B32Fmt<32, false, false, false, 128>;
using B32Q40 = B32Fmt<16, true, false, false, 8>;
using B32Q41 = B32Fmt<16, true, false, true, 0>;
using B32Q50 = B32Fmt<16, true, true, false, 16>;
using B32Q51 = B32Fmt<16, true, true, true, 0>;

template <class F, int NP, int MT, int NT, int WGM, int WGN>
__global__ void __launch_bounds__(64 * WGM * WGN)
    k_mm_h_b32(const uint8_t *qsp, const uint8_t *qhp, const uint8_t *sp, int64_t N,
               int nb_row, const uint16_t *__restrict__ xp, int64_t plane,
               const int32_t *__restrict__ xe, const uint16_t *__restrict__ xs, int64_t M,
               float *__restrict__ Y, int sg_per_split) {
  constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
  constexpr int BM = WGM * MT * 16, BN = WGN * NT * 16;
  constexpr int SB = F::kMin ? 4 : 2;  // scale bytes per block
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NP][BM * kLdA];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K = (int64_t)nb_row * 32;
  const int nsg = nb_row / 8;  // groups of 8 blocks per row
  const int s_begin = (int)blockIdx.z * sg_per_split;
  const int s_end = std::min(s_begin + sg_per_split, nsg);
  Y += (int64_t)blockIdx.z * M * N;

  const int64_t nblk = N * nb_row;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(qsp), 0, (int)(nblk * F::kQsBytes), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(qhp), 0, F::kHigh ? (int)(nblk * 4) : 0, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(sp), 0, (int)(nblk * SB), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(xp), 0, (int)(2 * NP * plane), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rxs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(xs), 0, F::kMin ? (int)(M * (K / 256) * 32) : 0, kRsrcWord3);
  constexpr uint32_t kNone = 0x7fffffffu;

  int64_t blk0[NT];  // first block of this lane's rows (-1 past N)
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t n = n0 + (wn * NT + j) * 16 + c16;
    blk0[j] = n < N ? n * nb_row : -1;
  }
  const uint32_t qoff = F::kNib ? 8 * (g & 1) : 8 * g;  // this lane's code bytes in a block

  // staging of one 64-column stage of X: BM rows x 8 uint4 per piece
  constexpr int SQ = BM * 8 * NP;
  constexpr int SPT = (SQ + THREADS - 1) / THREADS;
  const int n_st = 4 * (s_end - s_begin);
  uint4 sreg[2][SPT];
  auto stage_load = [&](int stg, uint4 *dst) {
    const int64_t k0 = (int64_t)s_begin * 256 + 64 * (int64_t)stg;
    const bool live = stg < n_st;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
      const int64_t row = m0 + r;
      const bool ok = live && q < SQ && row < M;
      dst[i] = rsrc_u4(rx, ok ? (uint32_t)(2 * ((int64_t)p * plane + row * K + k0 + 8 * s)) : kNone);
    }
  };
  auto stage_store = [&](const uint4 *src, int buf) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int q = tid + i * THREADS;
      if (SQ % THREADS == 0 || q < SQ) {
        const int p = q / (BM * 8), r = (q / 8) % BM, s = q % 8;
        *reinterpret_cast<uint4 *>(&As[buf][p][r * kLdA + 8 * s]) = src[i];
      }
    }
  };
  // the code words of the two blocks of split stage stg
  // (Q8_0: a stage's two 32-byte blocks are one 64-byte run, loaded as one
  // 16-byte chunk per lane group and turned into each group's words by
  // pair_words at the stage's start)
  uint2 wq[4][NT][2];
  auto w_load = [&](int stg, int c) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bool ok = stg < n_st && blk0[j] >= 0;
      const uint32_t blk = ok ? (uint32_t)(blk0[j] + (int64_t)s_begin * 8 + 2 * stg) : 0u;
      if constexpr (F::kQsBytes == 32) {
        const uint4 v = rsrc_u4(rq, ok ? blk * 32 + pair_chunk(g) : kNone);
        wq[c][j][0] = make_uint2(v.x, v.y);
        wq[c][j][1] = make_uint2(v.z, v.w);
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e)
          wq[c][j][e] = rsrc_u2(rq, ok ? (blk + e) * F::kQsBytes + qoff : kNone);
      }
    }
  };
  // the scales (d, or d | m << 16) and fifth-bit words of a group's 8 blocks:
  // 16 or 32 bytes each per row, loaded whole (one or two 16-byte loads) a
  // group ahead into `nx`, moved into `cu` at the group's end (indices stay
  // static, so the sets stay in registers)
  constexpr int GSQ = SB * 8 / 16, GHQ = F::kHigh ? 2 : 1;
  struct GroupWords {
    uint4 s[NT][GSQ];
    uint4 h[NT][GHQ];
  };
  GroupWords gcu, gnx;
  auto g_load = [&](int sg, GroupWords &gw) {  // group sg of the row (zeros past the split)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bool ok = sg < s_end && blk0[j] >= 0;
      const uint32_t blk = ok ? (uint32_t)(blk0[j] + (int64_t)sg * 8) : 0u;
#pragma unroll
      for (int q = 0; q < GSQ; ++q) gw.s[j][q] = rsrc_u4(rs, ok ? blk * SB + 16 * q : kNone);
      if constexpr (F::kHigh) {
#pragma unroll
        for (int q = 0; q < GHQ; ++q) gw.h[j][q] = rsrc_u4(rh, ok ? blk * 4 + 16 * q : kNone);
      }
    }
  };
  auto u4_word = [](const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; };
  // block b (0..7) of the current group: its scale word (d in the low half,
  // m in the high half for the min formats) and fifth-bit word
  auto scale_word = [&](int j, int b) -> uint32_t {
    if constexpr (SB == 2) {
      const uint32_t w = u4_word(gcu.s[j][0], b >> 1);
      return (b & 1) ? w >> 16 : w & 0xFFFFu;
    } else {
      return u4_word(gcu.s[j][b >> 2], b & 3);
    }
  };
  auto high_word = [&](int j, int b) -> uint32_t { return u4_word(gcu.h[j][b >> 2], b & 3); };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < 4; ++c) w_load(c, c);
  g_load(s_begin, gcu);
  stage_load(0, sreg[0]);
  stage_load(1, sreg[1]);
  stage_store(sreg[0], 0);
  __syncthreads();

  for (int sg = s_begin; sg < s_end; ++sg) {
    g_load(sg + 1, gnx);
    uint2 xsv[MT];
    if constexpr (F::kMin) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int64_t row = m0 + (wm * MT + i) * 16 + c16;
        xsv[i] = rsrc_u2(rxs, row < M ? (uint32_t)(((row * nsg + sg) * 16 + 4 * g) * 2) : kNone);
      }
    }
    uint32_t mv[NT][4];  // the group's 8 m halves, two per word (min formats)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int stg = 4 * (sg - s_begin) + c;
      stage_load(stg + 2, sreg[c & 1]);
      const int buf = c & 1;
      h8 bop[2][NT];
      float dsc[2][NT];
      if constexpr (F::kQsBytes == 32) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          uint4 v = make_uint4(wq[c][j][0].x, wq[c][j][0].y, wq[c][j][1].x, wq[c][j][1].y);
          pair_words(v);
          wq[c][j][0] = make_uint2(v.x, v.y);
          wq[c][j][1] = make_uint2(v.z, v.w);
        }
      }
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          uint32_t c0 = wq[c][j][e].x, c1 = wq[c][j][e].y;
          if constexpr (F::kNib) {
            const int sh = 4 * (g >> 1);
            c0 = (c0 >> sh) & 0x0F0F0F0Fu;
            c1 = (c1 >> sh) & 0x0F0F0F0Fu;
          }
          if constexpr (F::kHigh) {
            const uint32_t hb = (high_word(j, 2 * c + e) >> (8 * g)) & 0xFFu;
            c0 |= spread4_to_bit4(hb & 15u);
            c1 |= spread4_to_bit4(hb >> 4);
          }
          c0 ^= F::kXor;
          c1 ^= F::kXor;
          uint32_t o[4];
          if constexpr (F::kOff == 0) {
            o[0] = __builtin_amdgcn_perm(0u, c0, 0x0C010C00u);
            o[1] = __builtin_amdgcn_perm(0u, c0, 0x0C030C02u);
            o[2] = __builtin_amdgcn_perm(0u, c1, 0x0C010C00u);
            o[3] = __builtin_amdgcn_perm(0u, c1, 0x0C030C02u);
            dsc[e][j] = f16_bits_to_f32(scale_word(j, 2 * c + e) & 0xFFFFu) * 16777216.f;
          } else {
            constexpr uint32_t kSub = (0xE400u | F::kOff) * 0x10001u;  // -(1024 + offset), twice
            o[0] = fma_h2(__builtin_amdgcn_perm(0x64646464u, c0, 0x05010400u), 0x3c003c00u, kSub);
            o[1] = fma_h2(__builtin_amdgcn_perm(0x64646464u, c0, 0x05030402u), 0x3c003c00u, kSub);
            o[2] = fma_h2(__builtin_amdgcn_perm(0x64646464u, c1, 0x05010400u), 0x3c003c00u, kSub);
            o[3] = fma_h2(__builtin_amdgcn_perm(0x64646464u, c1, 0x05030402u), 0x3c003c00u, kSub);
            dsc[e][j] = f16_bits_to_f32(scale_word(j, 2 * c + e) & 0xFFFFu);
          }
          bop[e][j] = __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
          if constexpr (F::kMin) {  // m of block 2c + e into half (2c + e) % 2 of word c
            const uint32_t mh = scale_word(j, 2 * c + e) >> 16;
            mv[j][c] = e == 0 ? mh : (mv[j][c] | (mh << 16));
          }
        }
      w_load(stg + 4, c);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = (wm * MT + i) * 16 + c16;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          f32x4 P[NT];
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const h8 a = *reinterpret_cast<const h8 *>(&As[buf][p][r * kLdA + 32 * e + 8 * g]);
#pragma unroll
            for (int j = 0; j < NT; ++j)
              P[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  a, bop[e][j], p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : P[j], 0, 0, 0);
          }
#pragma unroll
          for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              acc[i][j][rr] = fmaf(dsc[e][j], P[j][rr], acc[i][j][rr]);
        }
      }
      stage_store(sreg[(c + 1) & 1], buf ^ 1);  // stage stg + 1, loaded at stage stg - 1
      __syncthreads();
    }
    if constexpr (F::kMin) {
      // m term: A = the x sums of the group's blocks (hi 0..7, lo 8..15, at
      // 2^(e-5)), B = m of blocks 4 (g & 1) .. +3 (lane group g holds k = 4g .. 4g+3)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const h4 bm = __builtin_bit_cast(
            h4, (g & 1) ? uint2{mv[j][2], mv[j][3]} : uint2{mv[j][0], mv[j][1]});
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const f32x4 q = __builtin_amdgcn_mfma_f32_16x16x16f16(
              __builtin_bit_cast(h4, xsv[i]), bm, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) acc[i][j][rr] = fmaf(32.f, q[rr], acc[i][j][rr]);
        }
      }
    }
    gcu = gnx;  // the next group's words (loaded at this group's start)
  }
  // Y = acc 2^-e (per row), rows past M and columns past N not stored
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int64_t row = m0 + (wm * MT + i) * 16 + 4 * g + rr;
      if (row >= M) continue;
      const int e = xe[row];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t n = n0 + (wn * NT + j) * 16 + c16;
        if (n < N) Y[row * N + n] = __builtin_amdgcn_ldexpf(acc[i][j][rr], -e);
      }
    }
  }
}
}  // namespace

// Workspace bytes of the X pieces of an M x K matrix (NP planes, the
// exponents and the sub-block sums), each 256-B aligned.
size_t mm_h_x_bytes(int64_t M, int64_t K, int np) {
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  return al((size_t)np * M * K * 2) + al((size_t)M * 4) + al((size_t)M * (K / 256) * 32);
}

bool mm_h_supported(const aq_matrix *m) {
  // 32-bit buffer offsets over each plane
  const double nblk = (double)m->rows * m->nb_row;
  if (m->nb_pitch != m->nb_row) return false;
  if (m->dtype == AQ_Q4_K || m->dtype == AQ_Q5_K) {
    const int np = m->dtype == AQ_Q4_K ? 2 : 3;
    for (int k = 0; k < np; ++k)
      if (nblk * (double)m->planes.stride[k] >= 2147483648.0) return false;
    return true;
  }
  // per-32 block formats: the dense planes of the SPLIT layout (codes, then
  // qh for Q5_0/Q5_1, then d or d|m), whole 256-column groups
  const int dt = m->dtype;
  if (dt == AQ_Q8_0 || dt == AQ_Q4_0 || dt == AQ_Q4_1 || dt == AQ_Q5_0 || dt == AQ_Q5_1) {
    const bool high = dt == AQ_Q5_0 || dt == AQ_Q5_1, mn = dt == AQ_Q4_1 || dt == AQ_Q5_1;
    const int64_t qsb = dt == AQ_Q8_0 ? 32 : 16;
    return m->layout == AQ_LAYOUT_SPLIT && m->cols % 256 == 0 && m->planes.stride[0] == qsb &&
           (!high || m->planes.stride[1] == 4) && m->planes.stride[high ? 2 : 1] == (mn ? 4 : 2) &&
           nblk * (double)qsb < 2147483648.0;
  }
  // Q6_K: the dense planes of the SPLIT layout (ql, qh, scales, d)
  return m->dtype == AQ_Q6_K && m->layout == AQ_LAYOUT_SPLIT && m->planes.stride[0] == 128 &&
         m->planes.stride[1] == 64 && m->planes.stride[2] == 16 && m->planes.stride[3] == 2 &&
         nblk * 128.0 < 2147483648.0;
}

// The per-32 block format kernels of one format: shapes 64 x 256, 64 x 128,
// 32 x 128 and the small batches' 16 x 128 and 32 x 256 (8 waves of one and
// of 2 x 2 tiles)
template <class F>
const void *b32_kernel(int shape) {
  constexpr int NP = 2;
  switch (shape) {
    case 1: return reinterpret_cast<const void *>(k_mm_h_b32<F, NP, 4, 2, 1, 4>);
    case 2: return reinterpret_cast<const void *>(k_mm_h_b32<F, NP, 2, 2, 1, 4>);
    case 3: return reinterpret_cast<const void *>(k_mm_h_b32<F, NP, 1, 1, 1, 8>);
    case 4: return reinterpret_cast<const void *>(k_mm_h_b32<F, NP, 2, 2, 1, 8>);
    default: return reinterpret_cast<const void *>(k_mm_h_b32<F, NP, 4, 2, 1, 8>);
  }
}

// The Q6_K kernels: the same shapes but 32 x 256 (which spills registers)
inline const void *q6_kernel(int shape) {
  constexpr int NP = 2;
  switch (shape) {
    case 1: return reinterpret_cast<const void *>(k_mm_h_q6k<NP, 4, 2, 1, 4>);
    case 2: return reinterpret_cast<const void *>(k_mm_h_q6k<NP, 2, 2, 1, 4>);
    case 3: return reinterpret_cast<const void *>(k_mm_h_q6k<NP, 1, 1, 1, 8>);
    default: return reinterpret_cast<const void *>(k_mm_h_q6k<NP, 4, 2, 1, 8>);
  }
}

// The Q4_K / Q5_K kernel instantiations the launcher picks from
template <bool Q5>
struct Q45Kernels {
  static constexpr int NP = 2;
  const void *big = reinterpret_cast<const void *>(k_mm_h_q4k<NP, 4, 2, 1, 8, 0, false, Q5>);
  const void *xs = reinterpret_cast<const void *>(k_mm_h_q4k<NP, 1, 1, 1, 8, kXsSmall, true, Q5>);
  const void *mt1 = reinterpret_cast<const void *>(k_mm_h_q4k<NP, 1, 2, 1, 4, 0, false, Q5>);
  const void *mt2 = reinterpret_cast<const void *>(k_mm_h_q4k<NP, 2, 2, 1, 8, 0, false, Q5>);
  const void *mt3 = reinterpret_cast<const void *>(k_mm_h_q4k<NP, 3, 2, 1, 8, 0, false, Q5>);
};

// Y (M x rows) = X W^T with X in two fp16 pieces.  m_invariant: no split
// of the super-blocks, so every output is the same sequence of operations
// for any M (the batched prefill step gives the same bits in any chunk
// size); otherwise the super-blocks are split over workgroups when the
// tiles leave CUs idle, and the partials added in split order.
hipError_t launch_matmul_h(const aq_matrix *m, const float *X, int64_t M, float *Y,
                           bool m_invariant, hipStream_t s, float *ysw, bool *fused_sw) {
  constexpr int NP = 2;
  if (M == 0 || m->rows == 0) return hipSuccess;
  if (!mm_h_supported(m)) return hipErrorInvalidValue;
  // the X pieces through 32-bit buffer offsets: callers split larger batches
  if ((double)M * m->cols * 2 * NP >= 2147483648.0) return hipErrorInvalidValue;
  const int64_t K = m->cols, N = m->rows;
  const int nb = (int)m->nb_row;
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t xb = mm_h_x_bytes(M, K, NP);
  // Tile shapes (waves along M x N, each MT x NT tiles of 16 x 16): above 48
  // rows of X one row of 8 waves of 4 x 2 tiles (64 x 256).  Every stage
  // each CU pulls the workgroup's X pieces (BM rows) and weight bytes (BN
  // rows) through its L1, so the tile is as wide along N as the registers of
  // two waves per SIMD allow: 14336 x 4096 at M = 512 takes 178 us at 64 x
  // 256, 203 us at 128 x 128 (2 x 4 waves of 4 x 2), 227 us at 64 x 256 as 1
  // x 4 waves of 4 x 4 (one wave per SIMD), 276 us at 32 x 512.  Up to 16
  // rows 16 x 128 (M = 16 on 14336 x 4096, graph-replayed, X prepared by its
  // own launch: 24.9 us against 26.2 us at 16 x 256 and 25.2 us at 16 x 64,
  // with the best K-split of each): with the fused X staging one row of 8
  // waves of one tile (19.6-19.9 us against 22.2-22.6 us as 4 waves of 1 x 2
  // tiles, M = 8 18.0-18.3 against 22.1-22.2 us: two waves per SIMD became
  // four), otherwise 4 waves of 1 x 2 tiles; up to 48 rows 8 waves of
  // ceil(M / 16) x 2 tiles (32 x 256 and 48 x 256; two waves per SIMD where 4
  // waves of ceil(M / 16) x 4 tiles held one: M = 32 29.8-30.0 against
  // 31.7-31.8 us, M = 48 35.1-35.2 against 37.0-37.2 us; 4 x 4 tiles spill
  // registers).  The arithmetic of an output is the same in every shape.
  //
  // Q6_K (k_mm_h_q6k) runs 64 x 256 (8 waves of 4 x 2 tiles), split for
  // AUTO; without a split (m_invariant) a shape whose tiles leave CUs idle
  // gives way to 64 x 128 or 32 x 128 (4 waves of 4 x 2 or 2 x 2 tiles):
  // 512 x 2048 at M = 2048 115 -> 59 us, 4096 x 14336 at M = 512 709 -> 489
  // us, graph-replayed.  The arithmetic of an output is the same in every
  // shape here too.  The per-32 block formats (k_mm_h_b32) take the same
  // shapes by the same rule.  Up to 48 rows both take small-batch tiles
  // (q6_shape below): 16 x 128 as 8 waves of one tile up to 16 rows, 32 x
  // 256 as 8 waves of 2 x 2 (Q6_K, whose 8-wave 32-row tile spills
  // registers: 32 x 128) up to 32, 64 x 256 up to 48.
  const int dt = m->dtype;
  const bool b32 =
      dt == AQ_Q8_0 || dt == AQ_Q4_0 || dt == AQ_Q4_1 || dt == AQ_Q5_0 || dt == AQ_Q5_1;
  const bool q6 = dt == AQ_Q6_K;
  const bool tiled = q6 || b32;  // the Q6_K and per-32 kernels
  const bool small = M <= 48;
  const int mt_small = (int)std::min<int64_t>(3, (M + 15) / 16);
  const int cus = device_info(m->device).cus;
  auto n_tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  // shape of the Q6_K / per-32 kernels: 0 = 64 x 256, 1 = 64 x 128, 2 = 32 x
  // 128, 3 = 16 x 128 (8 waves), 4 = 32 x 256 (8 waves; per-32 formats).  Up
  // to 16 rows 3, up to 32 rows 4 (Q6_K: 2), up to 48 rows 0 (the 48-row
  // 8-wave tiles spill registers); above, 64 x 256 unless its tiles leave
  // CUs idle in an unsplit launch
  const int q6_shape = !tiled                                    ? 0
                       : M <= 16                                 ? 3
                       : M <= 32                                 ? (q6 ? 2 : 4)
                       : small || !m_invariant || n_tiles(64, 256) >= cus ? 0
                       : n_tiles(64, 128) >= cus                 ? 1
                                                                 : 2;
  // Q4_K / Q5_K above 48 rows without a split: where 64 x 256 tiles leave
  // CUs idle, the 32 x 256 or 16 x 128 shape of the small batches
  const int q45_shape = small || tiled || !m_invariant || n_tiles(64, 256) >= cus ? 0
                        : n_tiles(32, 256) >= cus                               ? 2
                                                                               : 1;
  const int mt_eff = q45_shape ? q45_shape : mt_small;  // the small family's MT
  const bool small_shape = (small && !tiled) || q45_shape > 0;  // the Q4_K / Q5_K small family
  const int BM = small_shape ? 16 * mt_eff : q6_shape == 3 ? 16
                                           : q6_shape == 2 || q6_shape == 4 ? 32 : 64;
  const int BN = (small_shape && mt_eff == 1) || (q6_shape >= 1 && q6_shape <= 3) ? 128 : 256;
  // up to 16 rows the split's X is staged whole when it has at most
  // kXsSmall stages (80 KB of LDS, two workgroups per CU), its pieces made
  // in the workgroup from the fp32 rows (no preparation launch)
  const bool q5 = m->dtype == AQ_Q5_K;
  const Q45Kernels<false> k4;
  const Q45Kernels<true> k5;
  const void *kern_xs = q5 ? k5.xs : k4.xs;
  const void *kq6 = q6_kernel(q6_shape);
  const void *kb32 = dt == AQ_Q8_0   ? b32_kernel<B32Q80>(q6_shape)
                     : dt == AQ_Q4_0 ? b32_kernel<B32Q40>(q6_shape)
                     : dt == AQ_Q4_1 ? b32_kernel<B32Q41>(q6_shape)
                     : dt == AQ_Q5_0 ? b32_kernel<B32Q50>(q6_shape)
                                     : b32_kernel<B32Q51>(q6_shape);
  const void *kern =
      q6              ? kq6
      : b32           ? kb32
      : !small_shape  ? (q5 ? k5.big : k4.big)
      : mt_eff == 1   ? kern_xs
      : mt_eff == 2   ? (q5 ? k5.mt2 : k4.mt2)
                      : (q5 ? k5.mt3 : k4.mt3);
  // 256 threads for the 4-wave kernels (16 x 128 with X prepared by its own
  // launch, the two smaller Q6_K / per-32 shapes), 512 for the rest; a
  // function of the kernel, since the fused staging may give way below
  auto threads_of = [&](const void *k) {
    return k == k4.mt1 || k == k5.mt1 || q6_shape == 1 || q6_shape == 2 ? 256 : 512;
  };
  const int threads = threads_of(kern);
  const int64_t tiles = n_tiles(BM, BN);
  // Split K when the tiles leave CUs idle (AQ_PREC_AUTO only): at 48 rows
  // or fewer up to as many workgroups as the CUs hold at once, at most two
  // per CU (M = 16: 4 splits 24.9 us, 8 splits 27.2 us; M = 32, one
  // workgroup per CU: 4 splits 31.3 us, 8 splits 38.3 us); above, one per CU.
  int splits = 1;
  int64_t want = cus;
  if (small) {
    int per_cu = 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0) != hipSuccess)
      per_cu = 1;
    want = (int64_t)std::min(std::max(per_cu, 1), 2) * cus;
  }
  if (!m_invariant && tiles < want)
    splits = (int)std::min<int64_t>(std::max<int64_t>(1, want / tiles), 16);
  // (units of the split: super-blocks, or groups of 8 blocks of 32)
  const int units = b32 ? nb / 8 : nb;
  splits = std::min(splits, std::max(1, units / 2));
  const int per = (units + splits - 1) / splits;
  splits = (units + per - 1) / per;
  // the same arithmetic with X prepared by its own launch and staged per
  // stage: splits longer than kXsSmall stages, or on request
  // (AQ_MATMUL_X_PREP, which tests compare the fused staging with)
  if (kern == kern_xs && (4 * per > kXsSmall || getenv("AQ_MATMUL_X_PREP")))
    kern = q5 ? k5.mt1 : k4.mt1;
  const bool fused = kern == kern_xs;
  const int threads_launch = threads_of(kern);
  const size_t part = splits > 1 ? (size_t)splits * M * N * 4 : 0;
  uint8_t *ws = static_cast<uint8_t *>(workspace(m->device, s, xb + part));
  if (!ws) return hipErrorOutOfMemory;
  uint16_t *xp = reinterpret_cast<uint16_t *>(ws);
  int32_t *xe = reinterpret_cast<int32_t *>(ws + al((size_t)NP * M * K * 2));
  uint16_t *xs = reinterpret_cast<uint16_t *>(ws + al((size_t)NP * M * K * 2) + al((size_t)M * 4));
  float *dst = splits > 1 ? reinterpret_cast<float *>(ws + xb) : Y;
  const int64_t plane = M * K;
  // (Q6_K needs no sub-block sums)
  // (Q6_K in its own column order, without sums; the per-32 formats with
  // sums only for the min formats)
  const bool mins = dt == AQ_Q4_1 || dt == AQ_Q5_1;
  if (q6)
    launch_x_h_pieces<NP, true>(X, M, K, xp, plane, xe, nullptr, s);
  else if (b32)
    launch_x_h_pieces<NP>(X, M, K, xp, plane, xe, mins ? xs : nullptr, s);
  else if (!fused)
    launch_x_h_pieces<NP>(X, M, K, xp, plane, xe, xs, s);
  // planes: Q4_K qs, header; Q5_K qs, qh, header; Q6_K ql, qh, scales, d
  const uint8_t *qs = m->planes.p[0], *hd = m->planes.p[q5 ? 2 : 1];
  const uint32_t qst = (uint32_t)m->planes.stride[0], hst = (uint32_t)m->planes.stride[q5 ? 2 : 1];
  const uint8_t *a_q5 = m->planes.p[1];
  uint32_t a_q5st = (uint32_t)m->planes.stride[1];
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)splits);
  uint32_t a_qst = qst, a_hst = hst;
  int64_t a_n = N, a_plane = plane;
  int a_nb = nb, a_per = per;
  const float *a_xf = fused ? X : nullptr;
  const uint8_t *sc6 = m->planes.p[2], *d6 = m->planes.p[3];
  // the SwiGLU pairs in the store: Q4_K / Q5_K launches without a split
  float *a_sw = ysw && !tiled && splits == 1 && N % 2 == 0 ? ysw : nullptr;
  if (fused_sw) *fused_sw = a_sw != nullptr;
  void *args[] = {&qs, &hd, &a_qst, &a_hst, &a_n,  &a_nb,   &xp,  &a_plane, &xe,
                  &xs, &M,  &dst,   &a_per, &a_xf, &a_q5, &a_q5st, &a_sw};
  void *args6[] = {&qs, &hd, &sc6, &d6, &a_n, &a_nb, &xp, &a_plane, &xe, &M, &dst, &a_per};
  // per-32 formats: codes, qh (Q5_0/Q5_1; else unused), d or d|m
  const bool high = dt == AQ_Q5_0 || dt == AQ_Q5_1;
  const uint8_t *bq = m->planes.p[0], *bh = m->planes.p[high ? 1 : 0],
                *bs = m->planes.p[high ? 2 : 1];
  void *argsb[] = {&bq, &bh, &bs, &a_n, &a_nb, &xp, &a_plane, &xe, &xs, &M, &dst, &a_per};
  (void)hipLaunchKernel(kern, grid, dim3(threads_launch), q6 ? args6 : b32 ? argsb : args, 0, s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return sum_splits(dst, splits, M * N, Y, s);
}

}  // namespace aq
