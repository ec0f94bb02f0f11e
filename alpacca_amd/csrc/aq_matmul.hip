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
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "aq_internal.h"

namespace aq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));

constexpr int BM = 128;  // rows of X (and Y) per workgroup
constexpr int BN = 128;  // rows of W (columns of Y) per workgroup
constexpr int BK = 64;   // K slots per stage
// bf16 per LDS row of the bf16 kernels' tiles: 160 B rows leave 13 % of the
// LDS cycles in bank conflicts (144 B: 36 %, 176 B: 36 %, 192 B: 50 %,
// measured with SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE on the Q4_K prefill)
constexpr int kBfLD = BK + 16;

// two floats -> two bf16 (round to nearest even), one v_cvt_pk_bf16_f32
// (a vector conversion; two scalar ones would become two conversions and a
// v_perm)
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// byte k of x as a float (v_cvt_f32_ubyte<k>: the compiler would extract the
// byte with a separate bit-field op first)
template <int K>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float r;
  if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// One chunk (F::ELEMS slots) decoded and packed to bf16 pairs: o[i] holds
// slots 2i and 2i+1.  The values are F::decode's (bit-exact fp32) rounded to
// bf16; Q4_K converts its nibbles with the byte-lane conversions.
template <class F>
struct ChunkBF16 {
  __device__ static void run(const typename F::Raw &r, int j, uint32_t *o) {
    float v[F::ELEMS];
    F::decode(r, j, v);
#pragma unroll
    for (int i = 0; i < F::ELEMS / 2; ++i) o[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
  }
};
template <>
struct ChunkBF16<Q4K> {
  __device__ static void run(const Q4K::Raw &r, int j, uint32_t *o) {
    uint32_t sc, mn;
    kquant_scale_pair(r.h.y, r.h.z, r.h.w, j >> 1, sc, mn);
    const float d = f16_bits_to_f32(r.h.x), dm = f16_bits_to_f32(r.h.x >> 16);
    const float d0 = d * ubyte(sc, 0), d1 = d * ubyte(sc, 1);
    const float m0 = -(dm * ubyte(mn, 0)), m1 = -(dm * ubyte(mn, 1));
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // slots 4i..4i+3: low nibbles of the word's bytes; 16+4i..: high nibbles
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      o[2 * i] = pack_bf16(fmaf(ubyte_f32<0>(lo), d0, m0), fmaf(ubyte_f32<1>(lo), d0, m0));
      o[2 * i + 1] = pack_bf16(fmaf(ubyte_f32<2>(lo), d0, m0), fmaf(ubyte_f32<3>(lo), d0, m0));
      o[8 + 2 * i] = pack_bf16(fmaf(ubyte_f32<0>(hi), d1, m1), fmaf(ubyte_f32<1>(hi), d1, m1));
      o[9 + 2 * i] = pack_bf16(fmaf(ubyte_f32<2>(hi), d1, m1), fmaf(ubyte_f32<3>(hi), d1, m1));
    }
  }
};

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
               int64_t M, float *__restrict__ Y, int stages_per_split) {
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
  // stages [s_begin, s_end) of split blockIdx.z; partials to Y + z M N
  const int s_begin = (int)blockIdx.z * stages_per_split;
  const int s_end = s_begin + stages_per_split < n_stages ? s_begin + stages_per_split : n_stages;
  Y += (int64_t)blockIdx.z * M * N;

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int st = s_begin; st < s_end; ++st) {
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

// ---- bf16 path: X converted once, then a software-pipelined MFMA kernel ----
// Pre-pass: X (M x K fp32, row-major) -> Xb (M x K bf16) with every block's
// elements in the decoder's slot order (chunk j, slot t), so the main kernel's
// X tiles are plain copies and W tiles decode contiguously.  Four
// consecutive slots are four consecutive elements in every format.
template <class F>
__global__ void __launch_bounds__(256)
    k_x_bf16_slots(const float *__restrict__ X, int64_t M, int nb_row,
                   uint2 *__restrict__ Xb) {
  const int64_t K = (int64_t)nb_row * F::BE;
  const int64_t quads = M * (K / 4);
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < quads;
       q += (int64_t)gridDim.x * 256) {
    const int64_t m = q / (K / 4);
    const int64_t e = 4 * (q - m * (K / 4));  // slot-order position in the row
    const int64_t b = e / F::BE;
    const int r = (int)(e - b * F::BE), j = r / F::ELEMS, t = r % F::ELEMS;
    const float4 v = *reinterpret_cast<const float4 *>(X + m * K + b * F::BE + F::xoff(j, t));
    Xb[q] = make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
  }
}

// Main kernel: BM x BN output tile per workgroup, WM x WN waves, each owning a
// (BM/WM) x (BN/WN) block of Y as 16x16 MFMA tiles.  Two LDS stages: while the
// waves run the MFMAs of stage s, the global loads of stage s+1 are already in
// registers; they are stored (X) and decoded (W) into the other LDS stage
// before the one barrier of the iteration.  Every load is unconditional (the
// last iteration re-reads its own stage, clamped), so the compiler can keep
// the prefetch registers live across the MFMAs.
//
// Split K (gridDim.z > 1): workgroup z takes stages [z*S, min((z+1)*S, n)) of
// the contraction and writes its partial tile to Y + z*M*N; k_sum_splits
// adds the partials in order of z.
template <class F, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN)
    k_matmul_bf16(Planes P, int64_t N, int nb_row, const uint4 *__restrict__ Xb,
                  int64_t M, float *__restrict__ Y, int stages_per_split) {
  constexpr int NT = 64 * WM * WN;
  constexpr int LD = kBfLD;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int CPS = BK / F::ELEMS;         // chunks per stage
  constexpr int XIT = (BM * BK / 8 + NT - 1) / NT;   // uint4 (8 bf16) of X per thread
  constexpr int WIT = (BN * CPS + NT - 1) / NT;      // W chunks per thread
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t *As = smem;                       // [2][BM * LD]
  uint16_t *Bs = smem + 2 * BM * LD;         // [2][BN * LD]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K8 = (int64_t)nb_row * (F::BE / 8);  // uint4 per row of Xb
  const int n_chunks = nb_row * F::CPB;
  const int n_all = (n_chunks + CPS - 1) / CPS;
  const int s_begin = (int)blockIdx.z * stages_per_split;
  const int s_end = s_begin + stages_per_split < n_all ? s_begin + stages_per_split : n_all;
  Y += (int64_t)blockIdx.z * M * N;

  // per-thread load bases, computed once: the X row of each of the thread's
  // uint4 slots, and the planes of the W row of each of its chunk items
  uint4 xr[XIT];
  typename F::Raw wr[WIT];
  const uint4 *xrow[XIT];
  int xq[XIT];
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    int idx = it * NT + tid;
    idx = idx < BM * BK / 8 ? idx : BM * BK / 8 - 1;
    int64_t m = m0 + idx / (BK / 8);
    m = m < M ? m : M - 1;
    xrow[it] = Xb + m * K8;
    xq[it] = idx % (BK / 8);
  }
  Planes wrow[WIT];
  int wc[WIT];
#pragma unroll
  for (int it = 0; it < WIT; ++it) {
    int item = it * NT + tid;
    item = item < BN * CPS ? item : BN * CPS - 1;
    int64_t n = n0 + item / CPS;
    n = n < N ? n : N - 1;
#pragma unroll
    for (int k = 0; k < F::NPL; ++k) {
      wrow[it].p[k] = P.p[k] + n * nb_row * P.stride[k];
      wrow[it].stride[k] = P.stride[k];
    }
    wc[it] = item % CPS;
  }
  auto fetch = [&](int st) {
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      int k8 = st * (BK / 8) + xq[it];
      k8 = k8 < (int)K8 ? k8 : (int)K8 - 1;
      xr[it] = xrow[it][k8];
    }
#pragma unroll
    for (int it = 0; it < WIT; ++it) {
      int ch = st * CPS + wc[it];
      ch = ch < n_chunks ? ch : n_chunks - 1;
      const int b = ch / F::CPB, j = ch - b * F::CPB;
      wr[it] = F::load(wrow[it], b, j);
    }
  };
  auto store = [&](int st, int buf) {
    uint16_t *A = As + buf * BM * LD, *B = Bs + buf * BN * LD;
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int idx = it * NT + tid;
      if (BM * BK / 8 % NT == 0 || idx < BM * BK / 8) {
        // rows past M hold copies of row M-1 (their outputs are not stored);
        // slots past K must be zero
        const int row = idx / (BK / 8), q = idx % (BK / 8);
        const bool ok = (int64_t)st * (BK / 8) + q < K8;
        *reinterpret_cast<uint4 *>(&A[row * LD + 8 * q]) = ok ? xr[it] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int it = 0; it < WIT; ++it) {
      const int item = it * NT + tid;
      if (BN * CPS % NT == 0 || item < BN * CPS) {
        const int row = item / CPS, c = item % CPS;
        const int ch = st * CPS + c;
        const int j = ch % F::CPB;
        uint32_t o[F::ELEMS / 2];
        ChunkBF16<F>::run(wr[it], j, o);
        const bool ok = ch < n_chunks;  // a clamped chunk past K stores zeros
        uint16_t *dst = &B[row * LD + c * F::ELEMS];
#pragma unroll
        for (int q = 0; q < F::ELEMS / 8; ++q)
          *reinterpret_cast<uint4 *>(dst + 8 * q) =
              ok ? make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3])
                 : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  fetch(s_begin);
  store(s_begin, 0);
  __syncthreads();
  const int r16 = lane & 15, kq = lane >> 4;
  for (int st = s_begin; st < s_end; ++st) {
    const int nxt = st + 1 < s_end ? st + 1 : st;
    fetch(nxt);  // unconditional: the last iteration re-reads its own stage
    // keep the scheduler from sinking the loads below the MFMAs (they would
    // then be waited for right away instead of flying during the MFMAs)
    __builtin_amdgcn_sched_barrier(0);
    const int cur = (st - s_begin) & 1;
    const uint16_t *A = As + cur * BM * LD, *B = Bs + cur * BN * LD;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 a[TM], b[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(
                        &A[(wm * TM * 16 + tm * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        b[tn] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(
                        &B[(wn * TN * 16 + tn * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // unconditional too (a conditional use would let the compiler sink the
    // loads into it); after the last stage it rewrites an unread buffer
    store(nxt, cur ^ 1);
    __syncthreads();
  }

  const int col = lane & 15, rq = lane >> 4;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int64_t n = n0 + wn * TN * 16 + tn * 16 + col;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * TM * 16 + tm * 16 + 4 * rq + r;
        if (m < M && n < N) Y[m * N + n] = acc[tm][tn][r];
      }
    }
}

// Workgroup barrier that waits for this wave's LDS operations only: global
// loads issued for later stages stay in flight (__syncthreads() would wait
// for them too: s_waitcnt vmcnt(0) lgkmcnt(0)).  LDS is coherent within the
// workgroup, so completed LDS stores are visible to every wave after it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // gfx9 encoding: lgkmcnt(0), vmcnt/expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Pipelined form of k_matmul_bf16 (same tiles, same LDS layout, same
// results), used for the 256 x 128 tiles: the global loads run two stages
// ahead in two register sets and the stage barrier waits for LDS only, so
// the decode and LDS store of stage s+1 (into the LDS buffer nobody reads
// during stage s) never wait for a load still in flight.
//
// The waves that own W chunks and the waves that do not (for the 32-slot
// chunk formats, waves 4-7 of the 256 x 128 tile) run separate copies of
// the loop: a per-thread "has a chunk" test inside the step would put the
// decode in its own basic block and leave the others' W loads unconsumed,
// which costs the loop conservative waits.  When K is a multiple of the
// 64-slot stage (RAGGED = false) the K-edge masks are compiled out.  Measured
// on M = 512, 14336 x 4096 Q4_K: 92.5 us against 102 us with both in one
// loop.  What bounds it is per-SIMD issue: in a stage every wave reads its
// A/B fragments (128 x 1 KB of LDS per CU), runs its MFMAs, then decodes and
// stores; with the waves in step the MFMA unit idles during the decode
// (MFMA busy ~28 %, VALU/MFMA co-execution ~18 % of that).
template <class F, int BM, int BN, int WM, int WN, bool RAGGED>
__global__ void __launch_bounds__(64 * WM * WN)
    k_matmul_bf16p(Planes P, int64_t N, int nb_row, const uint4 *__restrict__ Xb,
                   int64_t M, float *__restrict__ Y, int stages_per_split) {
  constexpr int NT = 64 * WM * WN;
  constexpr int LD = kBfLD;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int CPS = BK / F::ELEMS;         // chunks per stage
  constexpr int XIT = BM * BK / 8 / NT;      // uint4 (8 bf16) of X per thread
  constexpr int WIT = (BN * CPS + NT - 1) / NT;      // W chunks per thread
  static_assert(BM * BK / 8 % NT == 0, "the X tile divides over the threads");
  static_assert(BN * CPS % 64 == 0, "W chunks fill whole waves");
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t *As = smem;                       // [2][BM * LD]
  uint16_t *Bs = smem + 2 * BM * LD;         // [2][BN * LD]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t K8 = (int64_t)nb_row * (F::BE / 8);  // uint4 per row of Xb
  const int n_chunks = nb_row * F::CPB;
  const int n_all = (n_chunks + CPS - 1) / CPS;
  const int s_begin = (int)blockIdx.z * stages_per_split;
  const int s_end = s_begin + stages_per_split < n_all ? s_begin + stages_per_split : n_all;
  Y += (int64_t)blockIdx.z * M * N;
  if (s_begin >= s_end) return;  // not launched so (no empty split); keeps the loops' barrier
                                 // counts equal regardless

  const uint4 *xrow[XIT];
  int xq[XIT];
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int idx = it * NT + tid;
    int64_t m = m0 + idx / (BK / 8);
    m = m < M ? m : M - 1;
    xrow[it] = Xb + m * K8;
    xq[it] = idx % (BK / 8);
  }
  Planes wrow[WIT];
  int wc[WIT];
#pragma unroll
  for (int it = 0; it < WIT; ++it) {
    int item = it * NT + tid;
    item = item < BN * CPS ? item : BN * CPS - 1;
    int64_t n = n0 + item / CPS;
    n = n < N ? n : N - 1;
#pragma unroll
    for (int k = 0; k < F::NPL; ++k) {
      wrow[it].p[k] = P.p[k] + n * nb_row * P.stride[k];
      wrow[it].stride[k] = P.stride[k];
    }
    wc[it] = item % CPS;
  }
  struct Regs {
    uint4 x[XIT];
    typename F::Raw w[WIT];
  };
  // WITHW: this thread's waves own W chunks (all of them: the chunks fill
  // whole waves and threads past the last chunk run the other loop)
  auto fetch = [&](int st, Regs &R, auto withw) {
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      int k8 = st * (BK / 8) + xq[it];
      if constexpr (RAGGED) k8 = k8 < (int)K8 ? k8 : (int)K8 - 1;
      R.x[it] = xrow[it][k8];
    }
    if constexpr (decltype(withw)::value) {
#pragma unroll
      for (int it = 0; it < WIT; ++it) {
        int ch = st * CPS + wc[it];
        if constexpr (RAGGED) ch = ch < n_chunks ? ch : n_chunks - 1;
        const int b = ch / F::CPB, j = ch - b * F::CPB;
        R.w[it] = F::load(wrow[it], b, j);
      }
    }
  };
  auto store = [&](int st, int buf, const Regs &R, auto withw) {
    uint16_t *A = As + buf * BM * LD, *B = Bs + buf * BN * LD;
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      // rows past M hold copies of row M-1 (their outputs are not stored);
      // slots past K must be zero
      const int idx = it * NT + tid;
      const int row = idx / (BK / 8), q = idx % (BK / 8);
      uint4 v = R.x[it];
      if constexpr (RAGGED)
        if ((int64_t)st * (BK / 8) + q >= K8) v = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4 *>(&A[row * LD + 8 * q]) = v;
    }
    if constexpr (decltype(withw)::value) {
#pragma unroll
      for (int it = 0; it < WIT; ++it) {
        const int item = it * NT + tid;
        const int row = item / CPS, c = item % CPS;
        const int ch = st * CPS + c;
        uint32_t o[F::ELEMS / 2];
        ChunkBF16<F>::run(R.w[it], ch % F::CPB, o);  // a clamped chunk past K: zeroed below
        uint16_t *dst = &B[row * LD + c * F::ELEMS];
#pragma unroll
        for (int q = 0; q < F::ELEMS / 8; ++q) {
          uint4 v = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
          if constexpr (RAGGED)
            if (ch >= n_chunks) v = make_uint4(0u, 0u, 0u, 0u);
          *reinterpret_cast<uint4 *>(dst + 8 * q) = v;
        }
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, kq = lane >> 4;
  auto mfma = [&](int cur) {
    const uint16_t *A = As + cur * BM * LD, *B = Bs + cur * BN * LD;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 a[TM], b[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(
                        &A[(wm * TM * 16 + tm * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        b[tn] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(
                        &B[(wn * TN * 16 + tn * 16 + r16) * LD + kk + 8 * kq]));
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
    }
  };

  // one stage: loads of stage st+2 into F_, MFMAs on LDS buffer (st - s_begin) & 1,
  // decode + store of stage st+1 (in S_) into the other buffer, barrier.
  // Clamped stages past the end re-read and re-store data nobody uses.
  auto run = [&](auto withw) {
    auto step = [&](int st, Regs &F_, const Regs &S_) {
      const int n1 = st + 1 < s_end ? st + 1 : st;
      const int n2 = st + 2 < s_end ? st + 2 : s_end - 1;
      fetch(n2, F_, withw);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out first
      const int cur = (st - s_begin) & 1;
      mfma(cur);
      store(n1, cur ^ 1, S_, withw);
      lds_barrier();
    };
    Regs R0, R1;
    fetch(s_begin, R0, withw);
    fetch(s_begin + 1 < s_end ? s_begin + 1 : s_begin, R1, withw);
    store(s_begin, 0, R0, withw);
    __syncthreads();
    for (int st = s_begin;;) {
      step(st, R0, R1);
      if (++st >= s_end) break;
      step(st, R1, R0);
      if (++st >= s_end) break;
    }
  };
  // Q4_K with whole stages (splits start on a super-block: the launcher keeps
  // them 4-stage aligned): a decoding thread loads its chunk of all 4 stages
  // of a super-block at once (4 x 16 B of one row's qs plus the header),
  // two stages before the first of them is decoded, instead of 32 B of the
  // same lines per stage — the lines are then fetched from L2 once per
  // super-block, not once per stage.  Two group register sets alternate; the
  // loop is unrolled over two super-blocks so every register index is static.
  constexpr bool kGroupW = std::is_same<F, Q4K>::value && !RAGGED && WIT == 1 && CPS == 2;
  struct WGroup {
    uint4 h, q[4];
  };
  auto run_grouped = [&]() {
    const int c = wc[0];
    auto fetch_group = [&](int g, WGroup &G) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const Q4K::Raw r = Q4K::load(wrow[0], g, 2 * s4 + c);
        G.q[s4] = r.q;
        if (s4 == 0) G.h = r.h;
      }
    };
    auto store_w = [&](int buf, const WGroup &G, int s4) {
      uint16_t *B = Bs + buf * BN * LD;
      const int row = tid / CPS;
      uint32_t o[Q4K::ELEMS / 2];
      Q4K::Raw r;
      r.q = G.q[s4];
      r.h = G.h;
      ChunkBF16<Q4K>::run(r, 2 * s4 + c, o);
      uint16_t *dst = &B[row * LD + c * Q4K::ELEMS];
#pragma unroll
      for (int q = 0; q < Q4K::ELEMS / 8; ++q)
        *reinterpret_cast<uint4 *>(dst + 8 * q) =
            make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    };
    const int g_last = (s_end - 1) >> 2;
    // step I of the 8-step body (st = s_begin + 8k + I): X of st+2 into F_,
    // MFMAs on st, X and W of st+1 (chunk (I+1) % 4 of group set
    // ((I+1) / 4) % 2) stored; at I = 2 and 6 the super-block of st+2 goes
    // into the set the other one left
    auto stepg = [&](auto I, int st, Regs &F_, const Regs &S_, WGroup &G0, WGroup &G1) {
      constexpr int i = decltype(I)::value;
      const int n1 = st + 1 < s_end ? st + 1 : st;
      const int n2 = st + 2 < s_end ? st + 2 : s_end - 1;
      fetch(n2, F_, std::false_type{});
      if constexpr ((i + 2) % 4 == 0) {
        const int g = (st + 2) >> 2;
        fetch_group(g < g_last ? g : g_last, ((i + 2) / 4) % 2 ? G1 : G0);
      }
      __builtin_amdgcn_sched_barrier(0);  // the loads go out first
      const int cur = (st - s_begin) & 1;
      mfma(cur);
      store(n1, cur ^ 1, S_, std::false_type{});
      store_w(cur ^ 1, ((i + 1) / 4) % 2 ? G1 : G0, (i + 1) % 4);
      // The compiler puts the stage's MFMAs in one run and the decode after
      // it; every wave of the CU reaches both at about the same time, so the
      // MFMA unit idles through the decode.  Per 32-slot slice: its fragment
      // reads, then each MFMA followed by two VALU ops of the decode
      // (M = 512 Q4_K: 14336 x 4096 84 -> 80 us, 4096 x 14336 89 -> 85 us;
      // one or three VALU per MFMA, or the next slice's reads moved among
      // the MFMAs, measured the same or slower).
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);  // LDS reads
#pragma unroll
        for (int k = 0; k < TM * TN; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
        }
      }
      lds_barrier();
    };
    Regs R0, R1;
    WGroup GA, GB;
    fetch(s_begin, R0, std::false_type{});
    fetch(s_begin + 1 < s_end ? s_begin + 1 : s_begin, R1, std::false_type{});
    fetch_group(s_begin >> 2, GA);
    store(s_begin, 0, R0, std::false_type{});
    store_w(0, GA, 0);
    __syncthreads();
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using I5 = std::integral_constant<int, 5>;
    using I6 = std::integral_constant<int, 6>;
    using I7 = std::integral_constant<int, 7>;
    for (int st = s_begin;;) {
      stepg(I0{}, st, R0, R1, GA, GB);
      if (++st >= s_end) break;
      stepg(I1{}, st, R1, R0, GA, GB);
      if (++st >= s_end) break;
      stepg(I2{}, st, R0, R1, GA, GB);
      if (++st >= s_end) break;
      stepg(I3{}, st, R1, R0, GA, GB);
      if (++st >= s_end) break;
      stepg(I4{}, st, R0, R1, GA, GB);
      if (++st >= s_end) break;
      stepg(I5{}, st, R1, R0, GA, GB);
      if (++st >= s_end) break;
      stepg(I6{}, st, R0, R1, GA, GB);
      if (++st >= s_end) break;
      stepg(I7{}, st, R1, R0, GA, GB);
      if (++st >= s_end) break;
    }
  };
  if (BN * CPS % NT == 0 || tid < BN * CPS - (WIT - 1) * NT) {
    if constexpr (kGroupW) run_grouped();
    else run(std::true_type{});
  } else {
    run(std::false_type{});
  }

  const int col = lane & 15, rq = lane >> 4;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int64_t n = n0 + wn * TN * 16 + tn * 16 + col;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * TM * 16 + tm * 16 + 4 * rq + r;
        if (m < M && n < N) Y[m * N + n] = acc[tm][tn][r];
      }
    }
}

// Y[i] = sum_z P[z][i], z = 0 .. splits-1 in order (float4 when n % 4 == 0).
// The partials of up to kSumBatch splits are loaded together and then added
// in split order (the same additions as one at a time, one memory round trip
// per batch instead of one per split).
constexpr int kSumBatch = 8;
__global__ void __launch_bounds__(256)
    k_sum_splits(const float *__restrict__ P, int splits, int64_t n, float *__restrict__ Y) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  if ((n & 3) == 0) {
    const float4 *P4 = reinterpret_cast<const float4 *>(P);
    float4 *Y4 = reinterpret_cast<float4 *>(Y);
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
      float4 a = P4[i];
      for (int z0 = 1; z0 < splits; z0 += kSumBatch) {
        float4 b[kSumBatch];
#pragma unroll
        for (int k = 0; k < kSumBatch; ++k)
          if (z0 + k < splits) b[k] = P4[(z0 + k) * n4 + i];
#pragma unroll
        for (int k = 0; k < kSumBatch; ++k) {
          if (z0 + k < splits) {
            a.x += b[k].x;
            a.y += b[k].y;
            a.z += b[k].z;
            a.w += b[k].w;
          }
        }
      }
      Y4[i] = a;
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
      float a = P[i];
      for (int z = 1; z < splits; ++z) a += P[z * n + i];
      Y[i] = a;
    }
  }
}

// PIPE: the pipelined kernel, RAGGED: K not a multiple of the stage (PIPE only)
template <class F, int BM, int BN, int WM, int WN, bool PIPE, bool RAGGED = true>
hipError_t launch_bf16(const aq_matrix *m, const uint4 *Xb, int64_t M, float *Y,
                       int splits, int stages_per_split, hipStream_t s) {
  auto kern = [] {
    if constexpr (PIPE) return k_matmul_bf16p<F, BM, BN, WM, WN, RAGGED>;
    else return k_matmul_bf16<F, BM, BN, WM, WN>;
  }();
  const size_t lds = 2 * (size_t)(BM + BN) * kBfLD * sizeof(uint16_t);
  hipError_t e = set_dynamic_lds(reinterpret_cast<const void *>(kern), (int)lds);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((m->rows + BN - 1) / BN), (unsigned)((M + BM - 1) / BM),
                  (unsigned)splits);
  hipLaunchKernelGGL(kern, grid, dim3(64 * WM * WN), lds, s, m->planes, m->rows,
                     (int)m->nb_row, Xb, M, Y, stages_per_split);
  return hipGetLastError();
}

// ---- int8 path: Q8_0 weights against int8 activations ----------------------
// X is quantized per 32-element block: d = absmax / 127 and q = rint(x / d)
// (q = 0 when the block is all zeros).  One thread per block.
__global__ void __launch_bounds__(256)
    k_x_q8(const float *__restrict__ X, int64_t n_blocks, uint4 *__restrict__ Xq,
           float *__restrict__ Xd) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= n_blocks) return;
  const float4 *src = reinterpret_cast<const float4 *>(X + 32 * b);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 f = src[i];
    v[4 * i] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float d = amax / 127.0f;
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = d > 0.f ? (int)rintf(v[4 * i + k] / d) : 0;
      word |= ((uint32_t)q & 0xFFu) << (8 * k);
    }
    w[i] = word;
  }
  Xq[2 * b] = make_uint4(w[0], w[1], w[2], w[3]);
  Xq[2 * b + 1] = make_uint4(w[4], w[5], w[6], w[7]);
  Xd[b] = d;
}

// Y[m, n] = sum_b dx[m, b] dw[n, b] sum_{i in block b} qx[m, i] qw[n, i]:
// one v_mfma_i32_16x16x32_i8 per 16 x 16 tile and 32-element block gives the
// exact integer block dot; it is converted once and scaled by dx * dw into
// an fp32 accumulator.  128 x 64 output tiles, 4 waves as 2 x 2 (64 x 32
// each: 4 x 2 MFMA tiles), two blocks (64 bytes of K) per stage, two LDS
// stages with the next stage's loads in registers during the MFMAs.  Lane
// l's operand: row (or column) l % 16, bytes 8 (l / 16) .. +7 of the block;
// result D[4 (l / 16) + r][l % 16].  The stages may be split over
// blockIdx.z (stages_per_split each, partials to Y + z M N, added in split
// order by k_sum_splits) so that a 512 x 4096 product runs several waves per
// SIMD instead of one.
constexpr int Q8_BM = 128, Q8_BN = 64, Q8_LD = 64 + 8;  // int8 row stride in LDS
__global__ void __launch_bounds__(256)
    k_matmul_q8(const uint8_t *__restrict__ Wq, const uint16_t *__restrict__ Wd, int64_t N,
                int nb_row, const uint4 *__restrict__ Xq, const float *__restrict__ Xd,
                int64_t M, float *__restrict__ Y, int stages_per_split) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) uint8_t As[2][Q8_BM * Q8_LD];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][Q8_BN * Q8_LD];
  __shared__ float dxs[2][Q8_BM][2], dws[2][Q8_BN][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t n0 = (int64_t)blockIdx.x * Q8_BN, m0 = (int64_t)blockIdx.y * Q8_BM;
  const int n_stages = (nb_row + 1) / 2;
  const int s_begin = (int)blockIdx.z * stages_per_split;
  const int s_end = s_begin + stages_per_split < n_stages ? s_begin + stages_per_split : n_stages;
  Y += (int64_t)blockIdx.z * M * N;
  const int64_t row16 = (int64_t)nb_row * 2;  // uint4 per row of Xq

  // per-thread load slots: X rows (two uint4 each of two rows), W row, scales
  const int xr0 = tid >> 2, xq = tid & 3;  // rows xr0 and xr0 + 64, uint4 xq of the stage
  const int64_t xm0 = m0 + xr0 < M ? m0 + xr0 : M - 1;
  const int64_t xm1 = m0 + xr0 + 64 < M ? m0 + xr0 + 64 : M - 1;
  const int wr = tid >> 2;  // W row of this thread's uint4
  const int64_t wn_row = n0 + wr < N ? n0 + wr : N - 1;
  uint4 rx0, rx1, rw;
  float rdx = 0.f;
  uint32_t rdw = 0;
  auto fetch = [&](int st) {
    const int b0 = 2 * st;  // first block of the stage
    // X: uint4 q of the stage's 64 bytes = block b0 + q / 2, half q % 2
    const int qb = b0 + (xq >> 1);
    const bool okx = qb < nb_row;
    const int64_t ix = 2 * (int64_t)(okx ? qb : nb_row - 1) + (xq & 1);
    rx0 = Xq[xm0 * row16 + ix];
    rx1 = Xq[xm1 * row16 + ix];
    if (!okx) rx0 = rx1 = make_uint4(0u, 0u, 0u, 0u);
    const int64_t iw = (wn_row * nb_row + (okx ? qb : nb_row - 1)) * 2 + (xq & 1);
    rw = reinterpret_cast<const uint4 *>(Wq)[iw];
    if (!okx) rw = make_uint4(0u, 0u, 0u, 0u);
    // scales: thread t < 256 -> dx of row t / 2, block b0 + t % 2;
    // t < 128 -> dw of row t / 2, block b0 + t % 2
    const int sb = b0 + (tid & 1);
    const bool oks = sb < nb_row;
    const int64_t sm = m0 + (tid >> 1) < M ? m0 + (tid >> 1) : M - 1;
    rdx = oks ? Xd[sm * nb_row + sb] : 0.f;
    const int64_t sn = n0 + (tid >> 1 & 63) < N ? n0 + (tid >> 1 & 63) : N - 1;
    rdw = oks ? Wd[sn * nb_row + sb] : 0u;
  };
  auto store = [&](int buf) {
    *reinterpret_cast<uint4 *>(&As[buf][xr0 * Q8_LD + 16 * xq]) = rx0;
    *reinterpret_cast<uint4 *>(&As[buf][(xr0 + 64) * Q8_LD + 16 * xq]) = rx1;
    *reinterpret_cast<uint4 *>(&Bs[buf][wr * Q8_LD + 16 * xq]) = rw;
    dxs[buf][tid >> 1][tid & 1] = rdx;
    if (tid < 2 * Q8_BN) dws[buf][tid >> 1][tid & 1] = f16_bits_to_f32(rdw);
  };

  f32x4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(s_begin);
  store(0);
  __syncthreads();
  const int r16 = lane & 15, kq = lane >> 4;
  for (int st = s_begin; st < s_end; ++st) {
    const int cur = (st - s_begin) & 1;
    const int nxt = st + 1 < s_end ? st + 1 : st;
    fetch(nxt);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *A = As[cur], *B = Bs[cur];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      long a[4], b[2];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        a[tm] = *reinterpret_cast<const long *>(&A[(wm * 64 + tm * 16 + r16) * Q8_LD + 32 * kb + 8 * kq]);
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
        b[tn] = *reinterpret_cast<const long *>(&B[(wn * 32 + tn * 16 + r16) * Q8_LD + 32 * kb + 8 * kq]);
      float dw[2];
#pragma unroll
      for (int tn = 0; tn < 2; ++tn) dw[tn] = dws[cur][wn * 32 + tn * 16 + r16][kb];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        float dx[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) dx[r] = dxs[cur][wm * 64 + tm * 16 + 4 * kq + r][kb];
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
          const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[tm], b[tn], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[tm][tn][r] = fmaf((float)d[r], dx[r] * dw[tn], acc[tm][tn][r]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    store(cur ^ 1);
    __syncthreads();
  }
  const int col = lane & 15, rq = lane >> 4;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
      const int64_t n = n0 + wn * 32 + tn * 16 + col;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t mm = m0 + wm * 64 + tm * 16 + 4 * rq + r;
        if (mm < M && n < N) Y[mm * N + n] = acc[tm][tn][r];
      }
    }
}

hipError_t launch_q8(const aq_matrix *m, const float *X, int64_t M, float *Y, hipStream_t s) {
  const int64_t nb = m->nb_row;
  // stage split: about two 4-wave workgroups per CU, each split at least 8
  // stages long (AQ_MATMUL_SPLIT overrides; measured on 512 x 4096 x 4096:
  // 96 us unsplit, 65 us in 2 splits, 70 in 4, 79 in 8)
  const int cus = device_info(m->device).cus;
  const int n_stages = (int)((nb + 1) / 2);
  const int64_t tiles = ((m->rows + Q8_BN - 1) / Q8_BN) * ((M + Q8_BM - 1) / Q8_BM);
  int splits = 1;
  if (tiles < 2 * (int64_t)cus) {
    splits = (int)std::min<int64_t>(8, std::max<int64_t>(1, 2 * (int64_t)cus / tiles));
    splits = std::min(splits, std::max(1, n_stages / 8));
  }
  if (const char *env = getenv("AQ_MATMUL_SPLIT")) {
    const int v = atoi(env);
    if (v >= 1 && v <= 16) splits = std::min(v, n_stages);
  }
  const int per = (n_stages + splits - 1) / splits;
  splits = (n_stages + per - 1) / per;  // no empty split
  const size_t q_bytes = ((size_t)M * nb * 32 + 255) & ~(size_t)255;
  const size_t d_bytes = ((size_t)M * nb * 4 + 255) & ~(size_t)255;
  const size_t part_bytes = splits > 1 ? (size_t)splits * M * m->rows * 4 : 0;
  uint8_t *ws = static_cast<uint8_t *>(workspace(m->device, s, q_bytes + d_bytes + part_bytes));
  if (!ws) return hipErrorOutOfMemory;
  uint4 *xq = reinterpret_cast<uint4 *>(ws);
  float *xd = reinterpret_cast<float *>(ws + q_bytes);
  float *dst = splits > 1 ? reinterpret_cast<float *>(ws + q_bytes + d_bytes) : Y;
  const int64_t blocks = M * nb;
  hipLaunchKernelGGL(k_x_q8, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, X, blocks,
                     xq, xd);
  const dim3 grid((unsigned)((m->rows + Q8_BN - 1) / Q8_BN), (unsigned)((M + Q8_BM - 1) / Q8_BM),
                  (unsigned)splits);
  hipLaunchKernelGGL(k_matmul_q8, grid, dim3(256), 0, s, m->planes.p[0],
                     reinterpret_cast<const uint16_t *>(m->planes.p[1]), m->rows, (int)nb, xq, xd,
                     M, dst, per);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const int64_t n = M * m->rows;
  const int64_t swg = std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)swg), dim3(256), 0, s, dst, splits, n, Y);
  return hipGetLastError();
}

template <class F>
hipError_t launch_fmt(const aq_matrix *m, const float *X, int64_t M, float *Y,
                      int precision, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const dim3 grid((unsigned)((m->rows + BN - 1) / BN),
                  (unsigned)((M + BM - 1) / BM));
  if (precision == AQ_PREC_BF16) {
    // Tiles: 256 x 128 (half the W decoding of 128-row tiles; the pipelined
    // kernel) when they fill
    // three quarters of the CUs or more; otherwise 256 x 128 tiles with the
    // K stages split over up to 8 workgroups so that about one workgroup per
    // CU runs, each split at least 8 stages long, or 128 x 64 tiles when
    // even that leaves the CUs short.  AQ_MATMUL_SPLIT overrides the split.
    const int cus = device_info(m->device).cus;
    const int n_stages = (int)((m->nb_row * F::CPB * F::ELEMS + BK - 1) / BK);
    const int64_t big = ((M + 255) / 256) * ((m->rows + 127) / 128);
    int splits = 1;
    if (big * 4 < (int64_t)cus * 3) {
      splits = (int)std::min<int64_t>(8, std::max<int64_t>(1, cus / big));
      splits = std::min(splits, std::max(1, n_stages / 8));
    }
    bool forced = false;
    if (const char *env = getenv("AQ_MATMUL_SPLIT")) {
      const int v = atoi(env);
      if (v >= 1 && v <= 16) {
        splits = std::min(v, n_stages);
        forced = true;
      }
    }
    const bool small_tiles = !forced && big * splits * 4 < (int64_t)cus * 3;
    if (small_tiles) splits = 1;
    int per = (n_stages + splits - 1) / splits;
    // Q4_K: splits start on a super-block (4 stages), see k_matmul_bf16p
    if (std::is_same<F, Q4K>::value) per = (per + 3) & ~3;
    splits = (n_stages + per - 1) / per;  // no empty split
    const size_t xb_bytes = ((size_t)M * m->cols * 2 + 255) & ~(size_t)255;
    const size_t part_bytes = splits > 1 ? (size_t)splits * M * m->rows * 4 : 0;
    uint8_t *ws = static_cast<uint8_t *>(workspace(m->device, s, xb_bytes + part_bytes));
    if (!ws) return hipErrorOutOfMemory;
    uint2 *xb = reinterpret_cast<uint2 *>(ws);
    float *dst = splits > 1 ? reinterpret_cast<float *>(ws + xb_bytes) : Y;
    const int64_t quads = M * (m->cols / 4);
    const int64_t wg = std::min<int64_t>((quads + 255) / 256, 8192);
    hipLaunchKernelGGL(k_x_bf16_slots<F>, dim3((unsigned)wg), dim3(256), 0, s, X, M,
                       (int)m->nb_row, xb);
    const uint4 *x8 = reinterpret_cast<const uint4 *>(xb);
    hipError_t e =
        small_tiles         ? launch_bf16<F, 128, 64, 2, 2, false>(m, x8, M, dst, 1, n_stages, s)
        : m->cols % BK != 0 ? launch_bf16<F, 256, 128, 4, 2, true, true>(m, x8, M, dst, splits, per, s)
                            : launch_bf16<F, 256, 128, 4, 2, true, false>(m, x8, M, dst, splits, per, s);
    if (e != hipSuccess || splits == 1) return e;
    const int64_t n = M * m->rows;
    const int64_t swg = std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096);
    hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)swg), dim3(256), 0, s, dst, splits, n, Y);
    return hipGetLastError();
  }
  // fp32: K stages split over up to 4 workgroups when the N tiles are few
  // (about cus / 4 per column of tiles), each split >= 8 stages; the split
  // depends on N and K only, so every output sums in the same order for any
  // M (a batched prefill gives the same results in any chunk size)
  const int cus = device_info(m->device).cus;
  const int n_stages = (int)((m->nb_row * F::CPB * F::ELEMS + BK - 1) / BK);
  const int64_t ntiles = (m->rows + BN - 1) / BN;
  int splits = (int)std::min<int64_t>(4, std::max<int64_t>(1, cus / (4 * ntiles)));
  splits = std::min(splits, std::max(1, n_stages / 8));
  const int per = (n_stages + splits - 1) / splits;
  splits = (n_stages + per - 1) / per;  // no empty split
  float *dst = Y;
  if (splits > 1) {
    dst = static_cast<float *>(workspace(m->device, s, (size_t)splits * M * m->rows * 4));
    if (!dst) return hipErrorOutOfMemory;
  }
  const dim3 grid3(grid.x, grid.y, (unsigned)splits);
  hipLaunchKernelGGL((k_matmul_t<F, false>), grid3, dim3(256), 0, s, m->planes,
                     m->rows, (int)m->nb_row, X, M, dst, per);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const int64_t n = M * m->rows;
  const int64_t swg = std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)swg), dim3(256), 0, s, dst, splits, n, Y);
  return hipGetLastError();
}

}  // namespace

hipError_t sum_splits(const float *P, int splits, int64_t n, float *Y, hipStream_t s) {
  const int64_t swg = std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)swg), dim3(256), 0, s, P, splits, n, Y);
  return hipGetLastError();
}

hipError_t launch_matmul_t(const aq_matrix *m, const float *X, int64_t M,
                           float *Y, int precision, hipStream_t s) {
  if (precision == AQ_PREC_INT8) {
    if (m->dtype != AQ_Q8_0 || m->layout != AQ_LAYOUT_SPLIT) return hipErrorInvalidValue;
    return M ? launch_q8(m, X, M, Y, s) : hipSuccess;
  }
  switch (m->dtype) {
    case AQ_Q4_K: return launch_fmt<Q4K>(m, X, M, Y, precision, s);
    case AQ_Q5_K: return launch_fmt<Q5K>(m, X, M, Y, precision, s);
    case AQ_Q6_K: return launch_fmt<Q6K>(m, X, M, Y, precision, s);
    case AQ_Q8_0: return launch_fmt<Q80>(m, X, M, Y, precision, s);
    case AQ_Q4_0: return launch_fmt<Q40>(m, X, M, Y, precision, s);
    case AQ_Q4_1: return launch_fmt<Q41>(m, X, M, Y, precision, s);
    case AQ_Q5_0: return launch_fmt<Q50>(m, X, M, Y, precision, s);
    case AQ_Q5_1: return launch_fmt<Q51>(m, X, M, Y, precision, s);
    case AQ_F32: return launch_fmt<F32D>(m, X, M, Y, precision, s);
    case AQ_F16: return launch_fmt<F16D>(m, X, M, Y, precision, s);
    case AQ_BF16: return launch_fmt<BF16D>(m, X, M, Y, precision, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aq
