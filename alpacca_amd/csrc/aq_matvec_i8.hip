// aq_matvec_i8.hip - decode matvec y = W x on integer dot products.
//
// Same contract as the reference's matvec (alpacca/qmatrix.py:148-171,
// alpacca/kernels.py:49-69): y[r] = sum_i w[r,i] x[i] with w the decoded
// GGUF weights, fp32 output.  One persistent kernel per call:
//
//  * each workgroup converts x (fp32) into LDS: per 32-element group three
//    int8 pieces, the group scale and two fp32 half sums, laid out in the
//    format's unit order (aq_units.h); the first weight loads of every wave
//    are already in flight meanwhile;
//  * wave w of W then takes rows w, w + W, ... (over the concatenated rows of
//    up to 8 matrices that share x).  Lane l takes unit 64s + l of a row
//    (64 weights each for the K-quants, 32 for the classic formats), decodes
//    the codes with a few bit operations and accumulates exact int32 dot4
//    chains against the pieces.  The loads of the next rows are issued
//    before the current ones compute, so HBM streams while the VALU works.
//    Sub-block scales, mins and code offsets are applied in fp32.
//
// Why integers: at 8 TB/s a Q4_K weight arrives every ~0.07 ns per GPU, which
// leaves ~2.8 VALU ops per weight.  Converting a nibble to fp32 and FMA-ing it
// already costs 2; the dot4 path costs ~1.6 in total (3 dot4 per 4 weights,
// unpacking and scales amortized over 64 weights).
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <initializer_list>

#include "aq_internal.h"
#include "aq_units.h"

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
__device__ __forceinline__ float row_sums(float v) {  // per 16-lane row
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sums(v);
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// low bytes of four words, packed (v_perm_b32 twice, then once more)
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b,
                                                   uint32_t c, uint32_t d) {
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// ---- x -> LDS: four threads per 32-element group, 8 elements each ----
// Thread q4 of a group converts elements 8*q4 .. 8*q4+7; the group maximum and
// the two half sums are combined across the four lanes with DPP.
//
// The group scale is a power of two, 2^e with e = exponent(M) - 6
// (M = m * 2^exponent, m in [0.5, 1)), so t = x / 2^e = ldexp(x, -e) is exact
// and |t| < 64.  The pieces are t = a + (254 b + c) / 254^2 rounded to
// nearest: a = rint(t), b = rint(254 (t - a)), c = rint(254 (254 (t - a) - b)),
// each in [-127, 127]; the representation error is at most 2^e / (2 * 254^2)
// <= M / 4.1e6.  Rounding uses the 1.5 * 2^23 trick: the low byte of the bits
// of t + 1.5 * 2^23 is rint(t) in two's complement.  A NaN or an infinity in
// the group makes its half sums non-finite, which carries into every row's
// result.
template <int CTRL>
__device__ __forceinline__ float dpp_q(float v) {  // within a quad of lanes
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, false));
}
struct Slice {
  float4 lo, hi;
};
// xg must be a valid group address even for an inactive slice (its values
// are then replaced by zeros): the load itself is unconditional.
__device__ __forceinline__ Slice load_slice(const float *__restrict__ xg, int q4,
                                            bool active) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const global_ptr<const f4> p = as_global(reinterpret_cast<const f4 *>(xg)) + 2 * q4;
  const f4 va = p[0], vb = p[1];
  const float4 a = make_float4(va.x, va.y, va.z, va.w), b = make_float4(vb.x, vb.y, vb.z, vb.w);
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  return Slice{active ? a : z, active ? b : z};
}
__device__ __forceinline__ void prep_slice(const Slice &sl, int q4, uint4 *dst,
                                           bool active) {
  const float v[8] = {sl.lo.x, sl.lo.y, sl.lo.z, sl.lo.w,
                      sl.hi.x, sl.hi.y, sl.hi.z, sl.hi.w};
  float M = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) M = fmaxf(M, fabsf(v[i]));
  const float part = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  // quad reductions: max over 4 lanes, pair sums of the two 16-element halves
  M = fmaxf(M, dpp_q<0xB1>(M));
  M = fmaxf(M, dpp_q<0x4E>(M));
  const float half = part + dpp_q<0xB1>(part);      // lanes 0,1: lo; 2,3: hi
  const float other = dpp_q<0x4E>(half);            // the other half's sum
  const int e = __builtin_amdgcn_frexp_expf(M) - 6;
  constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
  uint32_t ra[8], rb[8], rc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = __builtin_amdgcn_ldexpf(v[i], -e);
    const float xa = t + kMagic;
    const float u = (t - (xa - kMagic)) * 254.f;
    const float xb = u + kMagic;
    const float xc = (u - (xb - kMagic)) * 254.f + kMagic;
    ra[i] = __builtin_bit_cast(uint32_t, xa);
    rb[i] = __builtin_bit_cast(uint32_t, xb);
    rc[i] = __builtin_bit_cast(uint32_t, xc);
  }
  if (!active) return;
  // quad (q4 >> 1) of each piece, dwords 2*(q4 & 1) .. +1
  uint2 *d2 = reinterpret_cast<uint2 *>(dst);
  const int hq = q4 >> 1, w = q4 & 1;
  d2[((0 + hq) * 64) * 2 + w] = make_uint2(pack_low_bytes(ra[0], ra[1], ra[2], ra[3]),
                                           pack_low_bytes(ra[4], ra[5], ra[6], ra[7]));
  d2[((2 + hq) * 64) * 2 + w] = make_uint2(pack_low_bytes(rb[0], rb[1], rb[2], rb[3]),
                                           pack_low_bytes(rb[4], rb[5], rb[6], rb[7]));
  d2[((4 + hq) * 64) * 2 + w] = make_uint2(pack_low_bytes(rc[0], rc[1], rc[2], rc[3]),
                                           pack_low_bytes(rc[4], rc[5], rc[6], rc[7]));
  if (q4 == 0)
    dst[6 * 64] = make_uint4((uint32_t)e, __builtin_bit_cast(uint32_t, half),
                             __builtin_bit_cast(uint32_t, other), 0u);
}

constexpr int kMaxSeg = 8;

// Up to kMaxSeg matrices (same dtype, K and layout) sharing one x run in one
// launch.  The waves are split between them in proportion to their rows:
// segment m owns waves [wstart[m], wstart[m] + wcount[m]) and wave
// wstart[m] + j takes rows j, j + wcount[m], ... of matrix m, so a wave never
// changes matrix.  Unused entries have wstart = the total wave count.
struct MvSeg {
  const uint8_t *p[4];  // plane bases (words 0-7)
  float *y;             // words 8-9
  int wstart;           // word 10
  int wcount;           // word 11
  int rows;             // word 12
  int pad[3];
};
static_assert(sizeof(MvSeg) == 64, "segment table entry is four 16-byte words");
struct MvArgs {
  MvSeg seg[kMaxSeg];  // first kernel argument: at offset 0 of the kernarg segment
  uint32_t stride[2][4];  // plane strides (bytes per block) of format 0 and (mixed) format 1
  int nb_row;
  int nb_pitch;  // blocks from one row to the next (> nb_row in a column window)
  int n_waves;
  int wg_split;  // mixed launches: workgroups below this run format 0, the rest format 1
  const float *x2;  // kXSwiglu: the "up" input
  const float *nw;  // kXNorm: the RMSNorm weights
  float eps;        // kXNorm
  int accumulate;   // y += W x instead of y = W x
  int swiglu_pairs; // row pairs (gate, up): y[p] = silu(row 2p) * row 2p+1
  int pad0;         // (the word before ldx, read with eps .. swiglu_pairs)
  // several x vectors (MX > 1, one matrix): vector v is x + v * ldx and its
  // product goes to y + v * ldy; vectors from mvalid on repeat the last valid
  // one and are not stored
  int64_t ldx, ldy;
  int mvalid;
};

// What the kernel stages as x (a template parameter: the plain kernel keeps
// its exact load schedule).
constexpr int kXPlain = 0;
constexpr int kXNorm = 1;    // x * inv * nw, inv = 1 / sqrt(mean(x^2) + eps)
constexpr int kXSwiglu = 2;  // x / (1 + exp(-x)) * x2

__device__ __forceinline__ float slice_sumsq(const Slice &a) {
  return ((a.lo.x * a.lo.x + a.lo.y * a.lo.y) + (a.lo.z * a.lo.z + a.lo.w * a.lo.w)) +
         ((a.hi.x * a.hi.x + a.hi.y * a.hi.y) + (a.hi.z * a.hi.z + a.hi.w * a.hi.w));
}
// Elementwise forms, rounded operation by operation as the reference's NumPy
// expressions are (tensor.py:163-172: arr * inv * weight; model.py:549-551:
// gate / (1.0 + exp(-gate)) * up).
__device__ __forceinline__ float4 norm4(float4 v, float inv, float4 w) {
#pragma clang fp contract(off)
  return make_float4((v.x * inv) * w.x, (v.y * inv) * w.y, (v.z * inv) * w.z,
                     (v.w * inv) * w.w);
}
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  return g / (1.0f + expf(-g)) * u;
}
__device__ __forceinline__ float4 swiglu4(float4 g, float4 u) {
  return make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z),
                     silu_mul(g.w, u.w));
}

// Every kernel argument that the start of the kernel needs, read in one
// scalar batch and pinned in scalar registers before any of it is used: the
// x pointer, the row geometry, the plane strides of format fmt, the x2 /
// RMSNorm weight pointers and the segment-table words of entries 0-2 (for
// the scalar selection in mv_body).  Read where they were used, they made
// three dependent round trips to the kernel-argument memory before the first
// weight load.  The strides of all four planes, the unused wg_split and pad0
// are kept too: they share multi-word loads with the values used, and a dead
// register of a pending load that the compiler reuses costs a wait for the
// whole batch.
struct MvStart {
  uint32_t e[3][13];
  uint32_t w3;
  int nb_row, nb_pitch, n_waves, wg_split;
  uint32_t stride[4];
  const float *xa, *xb;
  float eps;
  int accumulate, swiglu_pairs, pad0;
};
template <int NPL, int XM>
__device__ __forceinline__ void mv_start(const MvArgs &A, const float *x, int fmt, MvStart &S) {
  using AS4U = const __attribute__((address_space(4))) uint32_t;
  AS4U *kt = (AS4U *)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int kSW = sizeof(MvSeg) / 4;  // words per entry
  // the words used: plane pointers 0 .. 2 NPL - 1, y (8, 9), wstart, wcount,
  // rows (10 - 12)
  auto used = [](int j) { return j < 2 * NPL || j >= 8; };
  S.w3 = kt[3 * kSW + 10];
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int j = 0; j < 13; ++j) S.e[q][j] = used(j) ? kt[q * kSW + j] : 0u;
  S.nb_row = A.nb_row;
  S.nb_pitch = A.nb_pitch;
  S.n_waves = A.n_waves;
  S.wg_split = A.wg_split;
#pragma unroll
  for (int k = 0; k < 4; ++k) S.stride[k] = A.stride[fmt][k];
  S.xa = x;
  S.xb = XM == kXSwiglu ? A.x2 : XM == kXNorm ? A.nw : x;
  S.eps = A.eps;
  S.accumulate = A.accumulate;
  S.swiglu_pairs = A.swiglu_pairs;
  S.pad0 = A.pad0;
  asm volatile("" : "+s"(S.nb_row), "+s"(S.nb_pitch), "+s"(S.n_waves), "+s"(S.wg_split),
               "+s"(S.w3));
  asm volatile("" : "+s"(S.xa), "+s"(S.xb), "+s"(S.eps), "+s"(S.accumulate),
               "+s"(S.swiglu_pairs), "+s"(S.pad0));
#pragma unroll
  for (int k = 0; k < 4; ++k) asm volatile("" : "+s"(S.stride[k]));
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int j = 0; j < 13; ++j)
      if (used(j)) asm volatile("" : "+s"(S.e[q][j]));
  __builtin_amdgcn_sched_barrier(0);  // the batch is complete here
}

// One-segment launches (k_matvec_i8_one): what the x loads and the first
// weight fetches need comes as leading scalar arguments, preloaded into
// scalar registers at wave launch (the file is built with kernel argument
// preloading), so those loads go out with no argument load ahead of them:
// x and the second input, the first two plane pointers, the rows, nb_row |
// nb_pitch << 16, the first two plane strides and wcount | n_waves << 16.
// The rest (y, planes past the second, eps and the flags) is read from the
// argument struct behind them, at byte kOneArgOff of the kernel-argument
// segment, and awaited where it is first used.
constexpr int kOneArgOff = 64;
template <int NPL, int XM>
__device__ __forceinline__ void mv_start_one(const MvArgs &A, const float *x, const float *xb,
                                             const uint8_t *p0, const uint8_t *p1, int rows,
                                             uint32_t nbp, uint32_t stride0, uint32_t stride1,
                                             uint32_t wn, MvStart &S) {
  using AS4U = const __attribute__((address_space(4))) uint32_t;
  AS4U *kt = (AS4U *)((const __attribute__((address_space(4))) uint8_t *)
                          __builtin_amdgcn_kernarg_segment_ptr() + kOneArgOff);
  asm volatile("" : "+s"(x), "+s"(xb), "+s"(p0), "+s"(p1), "+s"(rows), "+s"(nbp), "+s"(stride0),
               "+s"(stride1), "+s"(wn));
  const uint64_t q0 = (uint64_t)p0, q1 = (uint64_t)p1;
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int j = 0; j < 13; ++j) S.e[q][j] = 0u;
  S.e[0][0] = (uint32_t)q0;
  S.e[0][1] = (uint32_t)(q0 >> 32);
  S.e[0][2] = (uint32_t)q1;
  S.e[0][3] = (uint32_t)(q1 >> 32);
#pragma unroll
  for (int j = 4; j < 8; ++j)
    if (j < 2 * NPL) S.e[0][j] = kt[j];  // planes past the second (y: after the fetches)
  S.e[0][11] = wn & 0xffffu;
  S.e[0][12] = (uint32_t)rows;
  S.w3 = 0;
  S.nb_row = (int)(nbp & 0xffffu);
  S.nb_pitch = (int)(nbp >> 16);
  S.n_waves = (int)(wn >> 16);
  S.wg_split = 0;
  S.stride[0] = stride0;
  S.stride[1] = stride1;
  S.stride[2] = NPL > 2 ? A.stride[0][2] : 0u;
  S.stride[3] = NPL > 3 ? A.stride[0][3] : 0u;
  S.xa = x;
  S.xb = XM == kXPlain ? x : xb;
  S.eps = 0.f;  // y, eps and the flags: read by mv_body after the first fetches
  S.accumulate = 0;
  S.swiglu_pairs = 0;
  S.pad0 = 0;
}

// ---- decode matvec ----
// A wave works through "iterations": iteration it = (chunk c, step s) covers
// RC of its rows (chunk c) at 64-unit step s.  The loads of iterations
// it+1 .. it+PD-1 are in flight while iteration it computes (PD register
// buffers in rotation, every fetch unconditional), so the compiler can count
// outstanding loads exactly.  The loads of the first PD iterations are
// issued before x is staged, so the staging runs under their latency.
// SINGLE: a row is one step, and the lane's x pieces stay in registers for
// the whole kernel.  WG threads share one staged x.
//
// PAIR (rows of at most 32 units, so SINGLE): the wave takes row pairs:
// lanes 0-31 row 2p, lanes 32-63 row 2p+1, read through one buffer resource
// that spans both rows, and every "row" of the loop below is a pair.
//
// The body runs one format, whose plane strides mv_start read (a mixed
// launch runs two formats, each in whole workgroups: k_matvec_i8_mixed);
// `block` is the workgroup's index in the launch's wave numbering.
//
// MX > 1 (small batches, one matrix, plain x): MX x vectors share the weight
// stream.  Each is staged into its own LDS region; a lane decodes its unit
// once (U::decode) and applies it to every vector (U::dotx), so the weights
// are read and unpacked once for MX products.
template <class U, int RC, int PD, bool SINGLE, int WG, int XM, bool PAIR, int MX = 1,
          bool ONE = false>
__device__ __forceinline__ void mv_body(const MvArgs &A, const MvStart &S, int block) {
  static_assert(!PAIR || (SINGLE && RC == 1), "pair mode: one step, one pair per iteration");
  static_assert(MX == 1 || (XM == kXPlain && RC == 1), "several x vectors: plain x, one row");
  extern __shared__ uint4 xl[];
  using F = typename U::F;
  using Raw = typename U::Raw;
  constexpr int GPB = F::BE / 32;  // 32-element groups per block
  const int nb_row = S.nb_row, nb_pitch = S.nb_pitch, n_waves = S.n_waves;
  const uint32_t w3 = S.w3;
  const float *const xa = S.xa, *const xb = S.xb;
  uint32_t pstride[F::NPL];
#pragma unroll
  for (int k = 0; k < F::NPL; ++k) pstride[k] = S.stride[k];
  // copied out with constant indices only, so that S stays in registers
  uint32_t e[3][13];
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int j = 0; j < 13; ++j) e[q][j] = S.e[q][j];
  const int units = nb_row * U::UPB;
  const int n_steps = SINGLE ? 1 : (units + 63) >> 6;
  // uint4 of one staged x vector (all of its steps)
  const int xregion = ((units + 63) >> 6) * U::GPU * XQ * 64;
  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform values are pinned to scalar registers with readfirstlane
  const int w = block * (WG / 64) + __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool live = w < n_waves;
  // x staging: four threads per 32-element group, WG threads per pass.  The
  // x loads of the first passes are issued before the weight prologue, so
  // waiting for them does not wait for the weights (loads complete in order).
  const int n_groups = nb_row * GPB;
  const int n_pass = (n_groups * 4 + WG - 1) / WG;
  auto slice_src = [&](int t, bool &active, int &gg) {
    const int g = t >> 2;
    active = g < n_groups;
    gg = active ? g : n_groups - 1;
  };
  auto slice_dst = [&](int gg) {
    const int blk = gg / GPB;
    int ub, k;
    U::group_slot(gg - blk * GPB, ub, k);
    const int u = blk * U::UPB + ub;
    return xl + ((u >> 6) * U::GPU + k) * XQ * 64 + (u & 63);
  };
  // the x loads of the first kPre passes go out before the weight prologue
  // (their preps run unconditionally, so the compiler cannot sink a load
  // below the prologue into a conditional use; a pass past the last one is
  // all inactive lanes)
  constexpr int kPre = SINGLE ? 1 : 2;
  Slice pre[kPre], pre2[kPre];
  bool pact[kPre];
  int pgg[kPre];
#pragma unroll
  for (int q = 0; q < kPre; ++q) {
    slice_src(tid + q * WG, pact[q], pgg[q]);  // inactive past the last pass
    pre[q] = load_slice(xa + 32 * (int64_t)pgg[q], tid & 3, pact[q]);
    if constexpr (XM != kXPlain) pre2[q] = load_slice(xb + 32 * (int64_t)pgg[q], tid & 3, pact[q]);
  }

  __builtin_amdgcn_sched_barrier(0);  // the x loads go out before the table is read

  // The wave's segment-table entry (13 words).  Launches of up to three
  // segments (every decode-step launch) select among entries 0-2, loaded as
  // scalars in the kernel's first scalar batch: one scalar round trip, which
  // does not queue behind the vector loads of the workgroup that arrived on
  // the CU first (lane-indexed vector loads of the table did: ~2 us from a
  // wave's start to its first weight load against ~0.8 us).  Waves of larger
  // launches past entry 3's start read the table with vector loads (lane q
  // holds entry q & 7) and pick the entry by a ballot.
  uint32_t sw[13];
  if (ONE || w < (int)e[1][10]) {  // entry 0 (every wave of a one-matrix launch): no selection
#pragma unroll
    for (int j = 0; j < 13; ++j) sw[j] = e[0][j];
  } else if (w < (int)w3) {  // entry 3 starts past this wave: entry 1 or 2
    const bool two = w >= (int)e[2][10];
#pragma unroll
    for (int j = 0; j < 13; ++j) sw[j] = two ? e[2][j] : e[1][j];
  } else {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    using KU4 = const __attribute__((address_space(4))) u32x4;
    const __attribute__((address_space(4))) uint8_t *ent =
        (const __attribute__((address_space(4))) uint8_t *)__builtin_amdgcn_kernarg_segment_ptr() +
        sizeof(MvSeg) * (lane & (kMaxSeg - 1));
    const u32x4 te0 = *(KU4 *)ent;
    const u32x4 te1 = F::NPL > 2 ? *(KU4 *)(ent + 16) : u32x4{0u, 0u, 0u, 0u};
    const u32x4 te2 = *(KU4 *)(ent + 32);
    const uint32_t te3 = *(const __attribute__((address_space(4))) uint32_t *)(ent + 48);
    const int m = __builtin_popcountll(
        __ballot(lane >= 1 && lane < kMaxSeg && w >= (int)te2.z));
#pragma unroll
    for (int j = 0; j < 13; ++j) {
      const uint32_t v = j < 4 ? te0[j & 3] : j < 8 ? te1[j & 3] : j < 12 ? te2[j & 3] : te3;
      sw[j] = (uint32_t)__builtin_amdgcn_readlane((int)v, m);
    }
  }
  auto seg_word = [&](int j) -> uint32_t { return sw[j]; };
  auto seg_ptr = [&](int j) -> uint64_t {
    return (uint64_t)seg_word(j) | ((uint64_t)seg_word(j + 1) << 32);
  };
  const int wl = w - (int)seg_word(10), W = (int)seg_word(11);
  const int seg_rows = (int)seg_word(12);
  const int seg_items = PAIR ? (seg_rows + 1) >> 1 : seg_rows;  // rows or row pairs
  global_ptr<float> yseg = as_global(reinterpret_cast<float *>(seg_ptr(8)));
  int accumulate = S.accumulate, swiglu_pairs = S.swiglu_pairs;
  float eps = S.eps;

  // fetch: RC rows of chunk c at step st.  A row past the wave's last row
  // (or any row of a wave with no rows) is "dead": its buffer has no bytes,
  // so the loads return zeros without touching memory and every fetch can
  // be issued unconditionally (a fetch under a branch lets the register
  // allocator reuse the in-flight buffer's registers, which forces a full
  // drain of the weight stream at every iteration).
  uint32_t row_bytes[F::NPL], row_pitch[F::NPL];
#pragma unroll
  for (int k = 0; k < F::NPL; ++k) {
    row_bytes[k] = (uint32_t)nb_row * pstride[k];
    row_pitch[k] = (uint32_t)nb_pitch * pstride[k];
  }
  const unsigned ul = (unsigned)lane;
  auto fetch = [&](int c, int st, Raw *dst) {
#pragma unroll
    for (int j = 0; j < RC; ++j) {
      const int i = c * RC + j;
      // the wave's i-th row, dead past the segment (the same test as
      // i >= n_rows without its division, so that the first fetches do not
      // wait for it)
      const int r = wl + i * W;
      const bool dead = !live || r >= seg_items;
      RowSrc src;
      // PAIR: item r is rows 2r and 2r+1 (the second may not exist)
      const int r0 = PAIR ? 2 * r : r;
      const int nr = PAIR ? (seg_rows - r0 < 2 ? 1 : 2) : 1;
#pragma unroll
      for (int k = 0; k < F::NPL; ++k) {
        src.rs[k] = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<uint8_t *>(seg_ptr(2 * k) + (uint64_t)(uint32_t)r0 * row_pitch[k]), 0,
            dead ? 0 : (nr - 1) * (int)row_pitch[k] + (int)row_bytes[k], kRsrcWord3);
        src.stride[k] = pstride[k];
        src.base[k] = PAIR ? (ul >> 5) * row_pitch[k] : 0u;
      }
      // lanes past the row's last unit read past its bytes: zeros (in PAIR
      // mode the low half's surplus lanes read the second row: unused)
      const unsigned u = PAIR ? (ul & 31u) : (unsigned)(st * 64) + ul;
      const unsigned b = u / U::UPB, ub = u - b * U::UPB;
      dst[j] = U::load(src, b, ub);
    }
  };
  // iteration counters: (c, st) of the iteration computed, (fc, fs) fetched
  int c = 0, st = 0, fc = 0, fs = 0;
  auto next = [&](int &cc, int &ss) {
    if (++ss == n_steps) {
      ss = 0;
      ++cc;
    }
  };
  Raw buf[PD][RC];
#pragma unroll
  for (int p = 0; p < PD; ++p) {
    fetch(fc, fs, buf[p]);
    next(fc, fs);
  }
  // the wave's row count (a division) only after the first fetches are out
  __builtin_amdgcn_sched_barrier(0);
  // ONE: y, eps and the flags from the argument struct, loaded here and
  // awaited under the first fetches' latency (read where they are used,
  // each would be a round trip of its own after the x staging; read at the
  // start, their wait would come before the fetches)
  if constexpr (ONE) {
    using AS4U = const __attribute__((address_space(4))) uint32_t;
    AS4U *kt = (AS4U *)((const __attribute__((address_space(4))) uint8_t *)
                            __builtin_amdgcn_kernarg_segment_ptr() + kOneArgOff);
    yseg = as_global(reinterpret_cast<float *>((uint64_t)kt[8] | (uint64_t)kt[9] << 32));
    // (through the segment pointer: the struct's fields would be loaded
    // ahead of the fetches)
    accumulate = (int)kt[offsetof(MvArgs, accumulate) / 4];
    swiglu_pairs = (int)kt[offsetof(MvArgs, swiglu_pairs) / 4];
    eps = __builtin_bit_cast(float, kt[offsetof(MvArgs, eps) / 4]);
    asm volatile("" : "+s"(yseg), "+s"(accumulate), "+s"(swiglu_pairs), "+s"(eps));
  }
  const int n_rows = live ? (seg_items - wl + W - 1) / W : 1;
  const int n_chunks = (n_rows + RC - 1) / RC;
  const int n_iters = n_chunks * n_steps;
  // i-th row of this wave (clamped to the last)
  auto row_of = [&](int i) { return wl + (i < n_rows ? i : n_rows - 1) * W; };

  // kXNorm: the sum of squares of all of x (slices are disjoint; inactive
  // ones are zeros), reduced over the workgroup, then the fp32 factor formed
  // in double as the reference forms it (tensor.py:168-170)
  float inv = 1.f;
  if constexpr (XM == kXNorm) {
    __shared__ float red[WG / 64];
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kPre; ++q) ss += slice_sumsq(pre[q]);
    for (int pass = kPre; pass < n_pass; ++pass) {
      const int t = tid + pass * WG;
      bool act;
      int gg;
      slice_src(t, act, gg);
      ss += slice_sumsq(load_slice(xa + 32 * (int64_t)gg, t & 3, act));
    }
    // DPP row sums and four lane reads (six __shfl_xor would be six LDS
    // round trips in a row on the way to the first product)
    ss = wave_sum(ss);
    if (lane == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < WG / 64; ++i) tot += red[i];
    inv = (float)(1.0 / sqrt((double)tot / (double)(nb_row * F::BE) + (double)eps));
  }
  auto finish = [&](const Slice &a, const Slice &b) -> Slice {
    if constexpr (XM == kXSwiglu) return Slice{swiglu4(a.lo, b.lo), swiglu4(a.hi, b.hi)};
    else if constexpr (XM == kXNorm) return Slice{norm4(a.lo, inv, b.lo), norm4(a.hi, inv, b.hi)};
    else return a;
  };
#pragma unroll
  for (int q = 0; q < kPre; ++q)
    prep_slice(finish(pre[q], pre2[q]), tid & 3, slice_dst(pgg[q]), pact[q]);
  for (int pass = kPre; pass < n_pass; ++pass) {
    const int t = tid + pass * WG;
    bool act;
    int gg;
    slice_src(t, act, gg);
    const Slice a = load_slice(xa + 32 * (int64_t)gg, t & 3, act);
    Slice b = a;
    if constexpr (XM != kXPlain) b = load_slice(xb + 32 * (int64_t)gg, t & 3, act);
    prep_slice(finish(a, b), t & 3, slice_dst(gg), act);
  }
  // vectors 1 .. MX-1 into their own regions (after the weight prologue)
  for (int v = 1; v < MX; ++v) {
    const float *xv = xa + (int64_t)(v < A.mvalid ? v : A.mvalid - 1) * A.ldx;
    for (int pass = 0; pass < n_pass; ++pass) {
      const int t = tid + pass * WG;
      bool act;
      int gg;
      slice_src(t, act, gg);
      prep_slice(load_slice(xv + 32 * (int64_t)gg, t & 3, act), t & 3,
                 slice_dst(gg) + v * xregion, act);
    }
  }
  __syncthreads();
  if (!live) return;

  GroupX gx[U::GPU];
  if constexpr (SINGLE && MX == 1) {
#pragma unroll
    for (int k = 0; k < U::GPU; ++k)
#pragma unroll
      for (int q = 0; q < XQ; ++q) gx[k].q[q] = xl[(k * XQ + q) * 64 + (PAIR ? lane & 31 : lane)];
  }
  float acc[RC][MX];
#pragma unroll
  for (int j = 0; j < RC; ++j)
#pragma unroll
    for (int v = 0; v < MX; ++v) acc[j][v] = 0.f;
  auto load_gx = [&](int st, int v) {
#pragma unroll
    for (int k = 0; k < U::GPU; ++k)
#pragma unroll
      for (int q = 0; q < XQ; ++q)
        gx[k].q[q] = xl[v * xregion + ((st * U::GPU + k) * XQ + q) * 64 +
                        (PAIR ? lane & 31 : lane)];
  };

  // Row results wait in registers - lane i & 63 of the wave holds the result
  // of its row i - and go out as one vector store per 64 rows and after the
  // wave's last row.  Stores and loads share the vmcnt counter and complete
  // out of order with each other, so while a store is pending the compiler
  // makes the next use of any loaded register wait for every outstanding
  // load: a store per row drained the weight pipeline once per row.
  // res[v][0] is row i's value (PAIR: row 2p's, or the SwiGLU pair's), and
  // res[v][1] row 2p+1's.
  float res[MX][2];
#pragma unroll
  for (int v = 0; v < MX; ++v) res[v][0] = res[v][1] = 0.f;
  // rows (last & ~63) .. last, one per lane
  auto flush = [&](int last) {
    const int i = (last & ~63) + lane;
    if (i > last) return;
    const int p = row_of(i);
#pragma unroll
    for (int v = 0; v < MX; ++v) {
      if (MX > 1 && v >= A.mvalid) continue;
      const global_ptr<float> yv = MX == 1 ? yseg : yseg + v * A.ldy;
      if constexpr (PAIR) {
        if (swiglu_pairs) {
          yv[p] = accumulate ? yv[p] + res[v][0] : res[v][0];
        } else {
          const global_ptr<float> yp = yv + 2 * p;
          yp[0] = accumulate ? yp[0] + res[v][0] : res[v][0];
          if (2 * p + 1 < seg_rows) yp[1] = accumulate ? yp[1] + res[v][1] : res[v][1];
        }
      } else {
        yv[p] = accumulate ? yv[p] + res[v][0] : res[v][0];
      }
    }
  };

  auto compute = [&](int c, int st, const Raw *wv) {
    if constexpr (!SINGLE && MX == 1) load_gx(st, 0);
    const int u = PAIR ? lane & 31 : st * 64 + lane;
    if (u < units) {
      const int ub = (int)((unsigned)u % U::UPB);
      if constexpr (MX == 1) {
#pragma unroll
        for (int j = 0; j < RC; ++j) acc[j][0] += U::dot(wv[j], ub, gx);
      } else {
        const typename U::Dec dec = U::decode(wv[0], ub);
#pragma unroll
        for (int v = 0; v < MX; ++v) {
          load_gx(st, v);
          acc[0][v] += U::dotx(dec, gx);
        }
      }
    }
    if (st == n_steps - 1) {
#pragma unroll
      for (int j = 0; j < RC; ++j) {
        const int i = c * RC + j;
#pragma unroll
        for (int v = 0; v < MX; ++v) {
          float r0, r1 = 0.f;
          if constexpr (PAIR) {
            const float s = row_sums(acc[j][v]);
            const float t0 = lane_f32(s, 0) + lane_f32(s, 16);
            const float t1 = lane_f32(s, 32) + lane_f32(s, 48);
            // gate row 2p, up row 2p+1 (the host checks rows are even)
            r0 = swiglu_pairs ? silu_mul(t0, t1) : t0;
            r1 = t1;
          } else {
            r0 = wave_sum(acc[j][v]);
          }
          acc[j][v] = 0.f;
          if (lane == (i & 63)) {
            res[v][0] = r0;
            res[v][1] = r1;
          }
        }
        if (i < n_rows && ((i & 63) == 63 || i == n_rows - 1)) flush(i);
      }
    }
  };

  // PD register buffers used in rotation: while one is computed, the loads
  // of the next PD - 1 iterations are in flight
  for (int it = 0; it < n_iters; it += PD) {
#pragma unroll
    for (int p = 0; p < PD; ++p) {
      if (p == 0 || it + p < n_iters) {
        compute(c, st, buf[p]);
        next(c, st);
      }
      fetch(fc, fs, buf[p]);
      next(fc, fs);
    }
  }
}

template <class U, int RC, int PD, bool SINGLE, int WG, int XM, bool PAIR = false, int MX = 1>
__global__ void __launch_bounds__(WG)
    k_matvec_i8(MvArgs A, const float *__restrict__ x) {
  MvStart S;
  mv_start<U::F::NPL, XM>(A, x, 0, S);
  mv_body<U, RC, PD, SINGLE, WG, XM, PAIR, MX>(A, S, (int)blockIdx.x);
}

template <class U, int RC, int PD, bool SINGLE, int WG, int XM, bool PAIR = false>
__global__ void __launch_bounds__(WG)
    k_matvec_i8_one(const float *__restrict__ x, const float *__restrict__ xb,
                    const uint8_t *p0, const uint8_t *p1, int rows, uint32_t nbp,
                    uint32_t stride0, uint32_t stride1, uint32_t wn, int pad0, int pad1,
                    int pad2, MvArgs A) {
  static_assert(kOneArgOff == 64, "the leading arguments fill 16 dwords");
  MvStart S;
  mv_start_one<U::F::NPL, XM>(A, x, xb, p0, p1, rows, nbp, stride0, stride1, wn, S);
  mv_body<U, RC, PD, SINGLE, WG, XM, PAIR, 1, true>(A, S, (int)blockIdx.x);
}

// Two formats sharing x (q/k in Q4_K and v in Q6_K, say): the segments of
// format 0 come first and own workgroups [0, wg_split), those of format 1
// the rest.  Grid row y runs format y (workgroup wg_split + x for format 1),
// so the branch needs no kernel argument and each body reads its own
// arguments in one batch; workgroups past their format's share end at once.
// Every branch is uniform over a workgroup, so each body's barriers are met
// by all of its threads.
template <class U, class U2, bool SINGLE, int WG, int XM, bool PAIR>
__global__ void __launch_bounds__(WG)
    k_matvec_i8_mixed(MvArgs A, const float *__restrict__ x) {
  MvStart S;
  if (blockIdx.y == 0) {
    mv_start<U::F::NPL, XM>(A, x, 0, S);
    if ((int)blockIdx.x >= S.wg_split) return;
    mv_body<U, 1, 2, SINGLE, WG, XM, PAIR>(A, S, (int)blockIdx.x);
  } else {
    mv_start<U2::F::NPL, XM>(A, x, 1, S);
    const int block = S.wg_split + (int)blockIdx.x;
    if (block * (WG / 64) >= S.n_waves) return;
    mv_body<U2, 1, 2, SINGLE, WG, XM, PAIR>(A, S, block);
  }
}

template <class U>
size_t lds_bytes(int64_t nb_row) {
  return xprep_bytes<U>(nb_row);
}

// Every wave that the GPU can hold at once gets an equal share of whole rows
// (to within one), so the launch is a single round with no tail.  The wave
// budget is the occupancy of the kernel (VGPRs, LDS), optionally capped by
// AQ_MATVEC_WPC (waves per CU, tuning).
int env_choice(const char *name, std::initializer_list<int> allowed, int dflt) {
  if (const char *env = getenv(name)) {
    const int v = atoi(env);
    for (int a : allowed)
      if (v == a) return v;
  }
  return dflt;
}

// Launch one matvec kernel (signature (MvArgs, const float *)): the wave
// budget is the kernel's occupancy on all CUs (optionally capped by
// AQ_MATVEC_WPC, waves per CU), split between the segments in proportion to
// their work items (rows, or row pairs in PAIR mode), every segment getting
// at least one wave and at most one per item, so the launch is one round with
// no tail.  Segments [n1, nseg) are a second format (n1 < nseg): they start
// on a workgroup boundary, the last segment of the first format taking the
// padding waves (a wave past its segment's items has no rows).
hipError_t launch_waves(const void *kern, MvArgs &A, int nseg, int n1, bool pair, size_t lds,
                        int wg, int device, const float *x, hipStream_t s, int wpc_cap = 0,
                        const float *one_xb = nullptr, bool one = false) {
  // the dynamic LDS may use what the kernel's static LDS leaves free
  hipFuncAttributes fa;
  hipError_t e = hipFuncGetAttributes(&fa, kern);
  if (e != hipSuccess) return e;
  e = set_dynamic_lds(kern, (int)(device_info(device).lds_max - fa.sharedSizeBytes));
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, wg, lds);
  if (e != hipSuccess) return e;
  const int wpg = wg / 64;  // waves per workgroup
  int wpc = (per_cu < 1 ? 1 : per_cu) * wpg;
  if (wpc_cap > 0 && wpc_cap < wpc) wpc = wpc_cap;
  if (const char *env = getenv("AQ_MATVEC_WPC")) {
    const int w = atoi(env);
    if (w > 0 && w < (per_cu < 1 ? 1 : per_cu) * wpg) wpc = w;
  }
  auto items = [&](int i) -> int64_t {
    return pair ? ((int64_t)A.seg[i].rows + 1) / 2 : (int64_t)A.seg[i].rows;
  };
  int64_t total = 0;
  for (int i = 0; i < nseg; ++i) total += items(i);
  int64_t target = (int64_t)device_info(device).cus * wpc;
  if (target > total) target = total;
  int waves = 0, last1 = -1;
  A.wg_split = 0;
  for (int i = 0; i < nseg; ++i) {
    if (i == n1 && n1 > 0) {  // second format: pad to a workgroup boundary
      const int pad = (wpg - waves % wpg) % wpg;
      if (last1 >= 0) A.seg[last1].wcount += pad;
      waves += last1 >= 0 ? pad : 0;
      A.wg_split = waves / wpg;
    }
    const int64_t rows = items(i);
    int64_t c = rows ? (target * rows + total / 2) / total : 0;
    if (rows && c < 1) c = 1;
    if (c > rows) c = rows;
    A.seg[i].wstart = waves;
    A.seg[i].wcount = (int)c;
    waves += (int)c;
    if (i < n1 && c > 0) last1 = i;
  }
  if (n1 >= nseg) A.wg_split = (waves + wpg - 1) / wpg;
  for (int i = nseg; i < kMaxSeg; ++i) A.seg[i].wstart = waves;
  A.n_waves = waves;
  const int64_t grid = (waves + wpg - 1) / wpg;
  if (one) {  // k_matvec_i8_one: the leading words, then the struct
    if (A.n_waves > 0xffff) return hipErrorInvalidValue;  // packed in 16 bits
    const uint8_t *p0 = A.seg[0].p[0], *p1 = A.seg[0].p[1];
    int rows = A.seg[0].rows, pad = 0;
    uint32_t nbp = (uint32_t)A.nb_row | (uint32_t)A.nb_pitch << 16;
    uint32_t st0 = A.stride[0][0], st1 = A.stride[0][1];
    uint32_t wn = (uint32_t)A.seg[0].wcount | (uint32_t)A.n_waves << 16;
    void *oargs[] = {&x, &one_xb, &p0, &p1, &rows, &nbp, &st0, &st1, &wn, &pad, &pad, &pad, &A};
    return hipLaunchKernel(kern, dim3((unsigned)grid), dim3(wg), oargs, lds, s);
  }
  void *args[] = {&A, &x};
  if (n1 < nseg) {  // two formats: grid row y runs format y (k_matvec_i8_mixed)
    const int64_t wide = std::max<int64_t>(A.wg_split, grid - A.wg_split);
    return hipLaunchKernel(kern, dim3((unsigned)wide, 2u), dim3(wg), args, lds, s);
  }
  return hipLaunchKernel(kern, dim3((unsigned)grid), dim3(wg), args, lds, s);
}

template <class U, int RC, int PD, bool SINGLE, int WG, int XM = kXPlain, bool PAIR = false,
          int MX = 1>
hipError_t launch_cfg(MvArgs &A, int nseg, int device, const float *x,
                      hipStream_t s, int wpc_cap = 0) {
  // one matrix, one x vector, formats of at most two planes (a third plane's
  // pointer would be awaited before the first fetch anyway), row geometry
  // that packs into 16-bit halves (the wave count always does: at most 32
  // waves on each of 256 CUs)
  if constexpr (MX == 1 && U::F::NPL <= 2)
    if (nseg == 1 && A.nb_row <= 0xffff && A.nb_pitch <= 0xffff)
      return launch_waves(
          reinterpret_cast<const void *>(k_matvec_i8_one<U, RC, PD, SINGLE, WG, XM, PAIR>), A,
          nseg, nseg, PAIR, lds_bytes<U>(A.nb_row), WG, device, x, s, wpc_cap,
          XM == kXSwiglu ? A.x2 : XM == kXNorm ? A.nw : x, true);
  return launch_waves(
      reinterpret_cast<const void *>(k_matvec_i8<U, RC, PD, SINGLE, WG, XM, PAIR, MX>), A, nseg,
      nseg, PAIR, MX * lds_bytes<U>(A.nb_row), WG, device, x, s, wpc_cap);
}

// MX x vectors per launch (small batches): row pairs for rows of at most 32
// units, else one row per wave, one or several steps.
template <class U, int MX>
hipError_t launch_batch_cfg(MvArgs &A, int device, const float *x, hipStream_t s) {
  const int64_t units = (int64_t)A.nb_row * U::UPB;
  if (units <= 32) return launch_cfg<U, 1, 2, true, 512, kXPlain, true, MX>(A, 1, device, x, s);
  if (units <= 64) return launch_cfg<U, 1, 2, true, 512, kXPlain, false, MX>(A, 1, device, x, s);
  return launch_cfg<U, 1, 2, false, 1024, kXPlain, false, MX>(A, 1, device, x, s);
}
template <class U>
hipError_t launch_batch(MvArgs &A, int mx, int device, const float *x, hipStream_t s) {
  switch (mx) {
    case 2: return launch_batch_cfg<U, 2>(A, device, x, s);
    case 4: return launch_batch_cfg<U, 4>(A, device, x, s);
    case 8: return launch_batch_cfg<U, 8>(A, device, x, s);
    default: return hipErrorInvalidValue;
  }
}

template <class U, class U2, bool SINGLE, int WG, int XM, bool PAIR>
hipError_t launch_mixed_cfg(MvArgs &A, int nseg, int n1, int device, const float *x,
                            hipStream_t s) {
  const size_t lds = std::max(lds_bytes<U>(A.nb_row), lds_bytes<U2>(A.nb_row));
  return launch_waves(reinterpret_cast<const void *>(k_matvec_i8_mixed<U, U2, SINGLE, WG, XM, PAIR>),
                      A, nseg, n1, PAIR, lds, WG, device, x, s);
}

// Rows of several steps run 1024-thread workgroups (one staged copy of the
// long x per CU) when the launch has at least 16 rows per CU; with fewer, that
// leaves CUs without a workgroup, so 512 threads (ffn_down 2048 x 8192 Q4_K:
// 4.8 against 6.0 us; 4096 x 14336: 10.3 us with 1024 against 11.8 with 512).
int64_t launch_rows(const MvArgs &A, int nseg) {
  int64_t rows = 0;
  for (int i = 0; i < nseg; ++i) rows += A.seg[i].rows;
  return rows;
}
bool wide_workgroups(int64_t rows, int device) {
  return rows >= 16 * (int64_t)device_info(device).cus;
}
// Single-step rows (and row pairs): 512-thread workgroups, or 256 when the
// launch has fewer than 8 items (rows, or row pairs in pair mode) per CU, so
// that every CU still gets a workgroup.
bool small_workgroups(const MvArgs &A, int nseg, bool pair, int device) {
  int64_t items = 0;
  for (int i = 0; i < nseg; ++i) items += pair ? (A.seg[i].rows + 1) / 2 : A.seg[i].rows;
  return items < 8 * (int64_t)device_info(device).cus;
}

// Mixed launches: the default configuration of each shape (row pairs, one
// step, several steps) for plain and RMSNorm-staged x.
template <class U, class U2>
hipError_t launch_i8_mixed(MvArgs &A, int nseg, int n1, int device, const float *x, int xm,
                           hipStream_t s) {
  const int64_t units = std::max<int64_t>((int64_t)A.nb_row * U::UPB, (int64_t)A.nb_row * U2::UPB);
  const bool single = units <= 64;
  const bool pair = units <= 32 && env_choice("AQ_MATVEC_PAIR", {0, 1}, 1);
  const bool wide = wide_workgroups(launch_rows(A, nseg), device);
  const bool small = single && small_workgroups(A, nseg, pair, device);
  if (xm == kXSwiglu) return hipErrorInvalidValue;
  if (xm == kXNorm) {  // fixed workgroup sizes: see launch_i8
    if (pair) return launch_mixed_cfg<U, U2, true, 512, kXNorm, true>(A, nseg, n1, device, x, s);
    return single ? launch_mixed_cfg<U, U2, true, 512, kXNorm, false>(A, nseg, n1, device, x, s)
                  : launch_mixed_cfg<U, U2, false, 1024, kXNorm, false>(A, nseg, n1, device, x, s);
  }
  if (pair)
    return small ? launch_mixed_cfg<U, U2, true, 256, kXPlain, true>(A, nseg, n1, device, x, s)
                 : launch_mixed_cfg<U, U2, true, 512, kXPlain, true>(A, nseg, n1, device, x, s);
  if (single)
    return small ? launch_mixed_cfg<U, U2, true, 256, kXPlain, false>(A, nseg, n1, device, x, s)
                 : launch_mixed_cfg<U, U2, true, 512, kXPlain, false>(A, nseg, n1, device, x, s);
  return wide ? launch_mixed_cfg<U, U2, false, 1024, kXPlain, false>(A, nseg, n1, device, x, s)
              : launch_mixed_cfg<U, U2, false, 512, kXPlain, false>(A, nseg, n1, device, x, s);
}


// Rows per iteration (RC), pipeline depth (PD: register buffers, so PD
// iterations' loads are in flight) and workgroup size (WG).  Defaults: one
// row per iteration, two buffers; 512 threads for single-step rows (256 when
// the launch has fewer than 8 rows or row pairs per CU) and for launches of
// several-step rows with fewer than 16 rows per CU, 1024 (one staged copy of
// the longer x per CU) otherwise.  AQ_MATVEC_RC (1, 2),
// AQ_MATVEC_PD (2, 3, 4) and AQ_MATVEC_WG (256, 512, 1024) override them for
// tuning; the instantiated combinations are RC = 1, PD = 2 with any WG,
// RC = 1, PD = 3 or 4 with WG = 512 or 1024, and RC = 2, PD = 2, WG = 512;
// any other request runs the defaults.
template <class U>
hipError_t launch_i8(MvArgs &A, int nseg, int device, const float *x, int xm,
                     hipStream_t s) {
  const int64_t steps = ((int64_t)A.nb_row * U::UPB + 63) / 64;
  const bool single = steps == 1;
  // rows of at most 32 units run as row pairs (all 64 lanes busy) unless
  // AQ_MATVEC_PAIR=0
  const bool pair = (int64_t)A.nb_row * U::UPB <= 32 &&
                    (A.swiglu_pairs || env_choice("AQ_MATVEC_PAIR", {0, 1}, 1));
  // The RMSNorm-staged form keeps fixed workgroup sizes (512 for single-step
  // rows, 1024 otherwise): its sum of squares is reduced over the workgroup,
  // so the workgroup size sets the rounding, and a launch of several matrices
  // must give the bits of one launch per matrix.
  const bool small = single && xm != kXNorm && small_workgroups(A, nseg, pair, device);
  if (pair) {
    if (xm == kXNorm) return launch_cfg<U, 1, 2, true, 512, kXNorm, true>(A, nseg, device, x, s);
    if (xm == kXSwiglu)
      return small ? launch_cfg<U, 1, 2, true, 256, kXSwiglu, true>(A, nseg, device, x, s)
                   : launch_cfg<U, 1, 2, true, 512, kXSwiglu, true>(A, nseg, device, x, s);
    return small ? launch_cfg<U, 1, 2, true, 256, kXPlain, true>(A, nseg, device, x, s)
                 : launch_cfg<U, 1, 2, true, 512, kXPlain, true>(A, nseg, device, x, s);
  }
  const int64_t rows = launch_rows(A, nseg);
  const bool wide = wide_workgroups(rows, device);
  if (xm == kXNorm)  // fused forms: the default configuration only
    return single ? launch_cfg<U, 1, 2, true, 512, kXNorm>(A, nseg, device, x, s)
                  : launch_cfg<U, 1, 2, false, 1024, kXNorm>(A, nseg, device, x, s);
  if (xm == kXSwiglu) {
    if (single)
      return small ? launch_cfg<U, 1, 2, true, 256, kXSwiglu>(A, nseg, device, x, s)
                   : launch_cfg<U, 1, 2, true, 512, kXSwiglu>(A, nseg, device, x, s);
    return wide ? launch_cfg<U, 1, 2, false, 1024, kXSwiglu>(A, nseg, device, x, s)
                : launch_cfg<U, 1, 2, false, 512, kXSwiglu>(A, nseg, device, x, s);
  }
  // Single-step rows of launches with 4096 to 32768 rows: at most 8 waves
  // per CU, with three rows in flight per wave from 16384 rows and two below
  // (gate/up 2 x 14336 x 4096: 14.5 against 15.3 us with two rows and the
  // full occupancy, interleaved repeats; the 8B step, whose q/k/v and
  // attn_output launches have 6144 and 4096 rows, 0.2480 ms with two rows
  // for those against 0.2527-0.2553 ms with three and 0.2500-0.2505 with
  // two for gate/up too; Q5_K 4096 x 4096 5.8 against 6.3 us, 14336 x 4096
  // 10.5 against 11.7 us).  Smaller launches keep two rows and the
  // occupancy (Q5_K 1024 x 4096: 4.5 against 5.0 us), as do larger ones (the
  // Q6_K 128256 x 4096 head: 81.4 against 83.7 us) and rows of several steps
  // (down 4096 x 14336: 10.2 against 11.6 us).
  const bool deep = single && rows >= 4096 && rows <= 32768;
  const bool deep3 = deep && rows >= 16384;
  const int RC = env_choice("AQ_MATVEC_RC", {1, 2}, 1);
  const int PD = env_choice("AQ_MATVEC_PD", {2, 3, 4}, deep3 ? 3 : 2);
  const int WG = env_choice("AQ_MATVEC_WG", {256, 512, 1024},
                            small ? 256 : single || !wide ? 512 : 1024);
  const int cap = deep ? 8 : 0;
#define AQ_CFG(rc, pd, wg)                                                        \
  if (RC == rc && PD == pd && WG == wg)                                           \
    return single ? launch_cfg<U, rc, pd, true, wg>(A, nseg, device, x, s, cap)   \
                  : launch_cfg<U, rc, pd, false, wg>(A, nseg, device, x, s, cap);
  AQ_CFG(1, 2, 256) AQ_CFG(1, 2, 512) AQ_CFG(1, 2, 1024)
  AQ_CFG(1, 3, 512) AQ_CFG(1, 3, 1024)
  AQ_CFG(1, 4, 512) AQ_CFG(1, 4, 1024)
  AQ_CFG(2, 2, 512)
#undef AQ_CFG
  // a combination that is not instantiated: the default configuration
  if (deep3) return launch_cfg<U, 1, 3, true, 512>(A, nseg, device, x, s, cap);
  if (deep) return launch_cfg<U, 1, 2, true, 512>(A, nseg, device, x, s, cap);
  if (single)
    return small ? launch_cfg<U, 1, 2, true, 256>(A, nseg, device, x, s)
                 : launch_cfg<U, 1, 2, true, 512>(A, nseg, device, x, s);
  return wide ? launch_cfg<U, 1, 2, false, 1024>(A, nseg, device, x, s)
              : launch_cfg<U, 1, 2, false, 512>(A, nseg, device, x, s);
}

}  // namespace

size_t matvec_i8_scratch_bytes(int dtype, int64_t nb_row) {
  switch (dtype) {
    case AQ_Q4_K: return xprep_bytes<UQ4K>(nb_row);
    case AQ_Q5_K: return xprep_bytes<UQ5K>(nb_row);
    case AQ_Q6_K: return xprep_bytes<UQ6K>(nb_row);
    case AQ_Q8_0: return xprep_bytes<UQ80>(nb_row);
    case AQ_Q4_0: return xprep_bytes<UQ40>(nb_row);
    case AQ_Q4_1: return xprep_bytes<UQ41>(nb_row);
    case AQ_Q5_0: return xprep_bytes<UQ50>(nb_row);
    case AQ_Q5_1: return xprep_bytes<UQ51>(nb_row);
    default: return 0;
  }
}

// The widest row whose `vectors` prepared x vectors fit in LDS.
static int64_t max_cols_for(int dtype, int device, int vectors) {
  // 256 B stay free for the static LDS of the fused kernels (kXNorm)
  const size_t lds = device_info(device).lds_max - 256;
  const int64_t be = (dtype == AQ_Q4_K || dtype == AQ_Q5_K || dtype == AQ_Q6_K) ? 256 : 32;
  // prepared bytes per column: 7 quads per 32 columns, rounded to whole
  // 64-unit steps
  int64_t k = 0;
  for (int64_t nb = 1;; ++nb) {
    if (vectors * matvec_i8_scratch_bytes(dtype, nb) > lds) break;
    k = nb * be;
  }
  return k;
}

int64_t matvec_i8_max_cols(int dtype, int device) { return max_cols_for(dtype, device, 1); }

namespace {
template <class U>
hipError_t batch_pass(MvArgs &A, int mx, int device, const float *x, hipStream_t s) {
  if (mx == 1) return launch_i8<U>(A, 1, device, x, kXPlain, s);
  return launch_batch<U>(A, mx, device, x, s);
}
}  // namespace

hipError_t launch_matvec_i8_batch(const aq_matrix *m, const float *X, int64_t M, int64_t ldx,
                                  float *Y, int64_t ldy, hipStream_t s) {
  if (M <= 0 || m->rows == 0) return hipSuccess;
  if (m->rows >= INT32_MAX) return hipErrorInvalidValue;
  const int be = (int)(m->cols / m->nb_row);
  // the most vectors whose whole rows fit in LDS (column windows multiply the
  // launches and leave each wave one short row: slower than more passes)
  int cap = 8;
  while (cap > 2 && max_cols_for(m->dtype, m->device, cap) < m->cols) cap /= 2;
  if (max_cols_for(m->dtype, m->device, cap) < m->cols) cap = 8;  // windows either way
  for (int64_t v0 = 0; v0 < M;) {
    // 8 vectors per pass while 5 or more are left, then 4, 2 or 1 (at most cap)
    const int64_t left = M - v0;
    int mx = left >= 5 ? 8 : left >= 3 ? 4 : (int)left;
    if (mx > cap) mx = cap;
    const int mvalid = (int)(left < mx ? left : mx);
    // rows wider than mx staged vectors fit run as column windows (added in
    // K order, the first window stores)
    const int64_t kmax = max_cols_for(m->dtype, m->device, mx);
    const int64_t wnb = kmax / be;
    if (wnb < 1) return hipErrorInvalidValue;
    const int64_t n_win = (m->nb_row + wnb - 1) / wnb;
    for (int64_t i = 0, nb0 = 0; i < n_win; ++i) {
      const int64_t nb = (m->nb_row - nb0 + (n_win - i) - 1) / (n_win - i);
      const aq_matrix v = column_window(*m, nb0, nb);
      MvArgs A{};
      for (int k = 0; k < 4; ++k) {
        A.seg[0].p[k] = v.planes.p[k];
        A.stride[0][k] = A.stride[1][k] = (uint32_t)v.planes.stride[k];
      }
      A.seg[0].y = Y + v0 * ldy;
      A.seg[0].rows = (int)v.rows;
      for (int k = 1; k < kMaxSeg; ++k) {
        A.seg[k] = A.seg[0];
        A.seg[k].rows = 0;
      }
      A.nb_row = (int)v.nb_row;
      A.nb_pitch = (int)v.nb_pitch;
      A.accumulate = i > 0 ? 1 : 0;
      A.ldx = ldx;
      A.ldy = ldy;
      A.mvalid = mvalid;
      const float *x = X + v0 * ldx + nb0 * be;
      hipError_t e;
      switch (m->dtype) {
        case AQ_Q4_K: e = batch_pass<UQ4K>(A, mx, m->device, x, s); break;
        case AQ_Q5_K: e = batch_pass<UQ5K>(A, mx, m->device, x, s); break;
        case AQ_Q6_K: e = batch_pass<UQ6K>(A, mx, m->device, x, s); break;
        case AQ_Q8_0: e = batch_pass<UQ80>(A, mx, m->device, x, s); break;
        case AQ_Q4_0: e = batch_pass<UQ40>(A, mx, m->device, x, s); break;
        case AQ_Q4_1: e = batch_pass<UQ41>(A, mx, m->device, x, s); break;
        case AQ_Q5_0: e = batch_pass<UQ50>(A, mx, m->device, x, s); break;
        case AQ_Q5_1: e = batch_pass<UQ51>(A, mx, m->device, x, s); break;
        default: return hipErrorInvalidValue;
      }
      if (e != hipSuccess) return e;
      nb0 += nb;
    }
    v0 += mvalid;
  }
  return hipSuccess;
}

hipError_t launch_matvec_i8_multi(const aq_matrix *const *ms, int n,
                                  const float *x, float *const *ys,
                                  hipStream_t s, const MatvecFusion *fu) {
  if (n < 1 || n > kMaxSeg) return hipErrorInvalidValue;
  MvArgs A{};
  int xm = kXPlain;
  if (fu) {
    xm = fu->mode == MatvecFusion::kNorm ? kXNorm
         : fu->mode == MatvecFusion::kSwiglu ? kXSwiglu : kXPlain;
    A.x2 = fu->x2;
    A.nw = fu->norm_w;
    A.eps = fu->eps;
    A.accumulate = fu->accumulate ? 1 : 0;
    A.swiglu_pairs = fu->swiglu_pairs ? 1 : 0;
  }
  A.nb_row = (int)ms[0]->nb_row;
  A.nb_pitch = (int)ms[0]->nb_pitch;
  // matrices [0, n1) share the first dtype, [n1, n) the second (if any)
  int n1 = n;
  for (int i = 1; i < n; ++i)
    if (ms[i]->dtype != ms[0]->dtype) {
      n1 = i;
      break;
    }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    for (int k = 0; k < 4; ++k) A.seg[i].p[k] = ms[i]->planes.p[k];
    A.seg[i].y = ys[i];
    A.seg[i].rows = (int)ms[i]->rows;
    total += ms[i]->rows;
    if (total >= INT32_MAX) return hipErrorInvalidValue;
  }
  for (int k = 0; k < 4; ++k) {
    A.stride[0][k] = (uint32_t)ms[0]->planes.stride[k];
    A.stride[1][k] = (uint32_t)ms[n1 < n ? n1 : 0]->planes.stride[k];
  }
  for (int i = n; i < kMaxSeg; ++i) {
    A.seg[i] = A.seg[0];
    A.seg[i].rows = 0;
  }
  if (total == 0) return hipSuccess;
  const int dev = ms[0]->device;
  if (n1 < n) {
    const int d0 = ms[0]->dtype, d1 = ms[n1]->dtype;
    if (d0 == AQ_Q4_K && d1 == AQ_Q6_K) return launch_i8_mixed<UQ4K, UQ6K>(A, n, n1, dev, x, xm, s);
    if (d0 == AQ_Q5_K && d1 == AQ_Q6_K) return launch_i8_mixed<UQ5K, UQ6K>(A, n, n1, dev, x, xm, s);
    if (d0 == AQ_Q4_K && d1 == AQ_Q5_K) return launch_i8_mixed<UQ4K, UQ5K>(A, n, n1, dev, x, xm, s);
    return hipErrorInvalidValue;
  }
  switch (ms[0]->dtype) {
    case AQ_Q4_K: return launch_i8<UQ4K>(A, n, dev, x, xm, s);
    case AQ_Q5_K: return launch_i8<UQ5K>(A, n, dev, x, xm, s);
    case AQ_Q6_K: return launch_i8<UQ6K>(A, n, dev, x, xm, s);
    case AQ_Q8_0: return launch_i8<UQ80>(A, n, dev, x, xm, s);
    case AQ_Q4_0: return launch_i8<UQ40>(A, n, dev, x, xm, s);
    case AQ_Q4_1: return launch_i8<UQ41>(A, n, dev, x, xm, s);
    case AQ_Q5_0: return launch_i8<UQ50>(A, n, dev, x, xm, s);
    case AQ_Q5_1: return launch_i8<UQ51>(A, n, dev, x, xm, s);
    default: return hipErrorInvalidValue;
  }
}

bool matvec_pair_rows(int dtype, int64_t nb_row) {
  int upb = 0;
  switch (dtype) {
    case AQ_Q4_K: case AQ_Q5_K: case AQ_Q6_K: upb = 4; break;
    case AQ_Q8_0: case AQ_Q4_0: case AQ_Q4_1: case AQ_Q5_0: case AQ_Q5_1: upb = 1; break;
    default: return false;
  }
  return nb_row * upb <= 32;
}

bool matvec_mixed_supported(int dtype0, int dtype1) {
  return (dtype0 == AQ_Q4_K && dtype1 == AQ_Q6_K) || (dtype0 == AQ_Q5_K && dtype1 == AQ_Q6_K) ||
         (dtype0 == AQ_Q4_K && dtype1 == AQ_Q5_K);
}

hipError_t launch_matvec_i8(const aq_matrix *m, const float *x, float *y,
                            hipStream_t s) {
  return launch_matvec_i8_multi(&m, 1, x, &y, s, nullptr);
}

}  // namespace aq
