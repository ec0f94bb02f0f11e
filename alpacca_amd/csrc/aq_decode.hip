// aq_decode.hip - the kernels around the quantized matvec in a decode step
// (alpacca/model.py:520-555): RMSNorm, rotary embedding + KV-cache store,
// grouped-query attention over the fp32 KV cache, SwiGLU, residual add, and
// greedy selection with the chosen token fed back on the device.
//
// Position and token live in device memory (aq_decode_state), so one decode
// step is a fixed sequence of launches that a HIP graph can capture once and
// replay for every token: nothing in it depends on host-side values that
// change from token to token.
//
// KV cache layout (per layer): [n_kv][n_ctx][head_dim] fp32.  A (kv head,
// chunk of positions) is one contiguous run of memory, so the attention
// kernel streams it with fully coalesced 16-byte loads.
#include <math.h>

#include "aq_internal.h"

namespace aq {
namespace {

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, false));
}
// sum over each row of 16 lanes, left in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppf<0x141>(v);  // row_half_mirror
  v += dppf<0x140>(v);  // row_mirror
  return v;
}

// ---- RMSNorm (tensor.py:163-172) -------------------------------------------
// out = x * inv * w with inv = 1 / sqrt(mean(x^2) + eps); one workgroup per
// row.  The sum of squares is fp32; the scalar is formed in double and
// rounded to fp32 once, as the reference forms it in Python floats and then
// multiplies the float32 array by it.  out may alias x.
constexpr int kNormWG = 256;
__global__ void __launch_bounds__(kNormWG)
    k_rmsnorm(const float *x, const float *__restrict__ w, int64_t n, float eps,
              float *out) {
#pragma clang fp contract(off)
  __shared__ float red[kNormWG / 64];
  const int64_t row = blockIdx.x;
  x += row * n;
  out += row * n;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kNormWG) ss = fmaf(x[i], x[i], ss);
  ss = row16_sum(ss);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormWG / 64; ++i) tot += red[i];
  const float inv = (float)(1.0 / sqrt((double)tot / (double)n + (double)eps));
  for (int64_t i = threadIdx.x; i < n; i += kNormWG) out[i] = (x[i] * inv) * w[i];
}

// The batched step's residual add and the RMSNorm that follows it
// (model.py:507 then :509, and :514 then the next layer's :487) in one pass:
// x = x + y is stored, and out = rmsnorm(x) * w.  Each thread visits the
// elements k_rmsnorm's thread of the same index visits, in the same order,
// and the sum, the scalar and the products are k_rmsnorm's, so x and out are
// bit-identical to k_add followed by k_rmsnorm.  The second loop reads back
// the thread's own stores.  out must not alias x or y.
__global__ void __launch_bounds__(kNormWG)
    k_add_rmsnorm(float *x, const float *__restrict__ y, const float *__restrict__ w, int64_t n,
                  float eps, float *__restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float red[kNormWG / 64];
  const int64_t row = blockIdx.x;
  x += row * n;
  y += row * n;
  out += row * n;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kNormWG) {
    const float v = x[i] + y[i];
    x[i] = v;
    ss = fmaf(v, v, ss);
  }
  ss = row16_sum(ss);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormWG / 64; ++i) tot += red[i];
  const float inv = (float)(1.0 / sqrt((double)tot / (double)n + (double)eps));
  for (int64_t i = threadIdx.x; i < n; i += kNormWG) out[i] = (x[i] * inv) * w[i];
}

// ---- rotary embedding + KV store (model.py:400-434, :533-540, :495-503) ---
// One thread per (token t, head, pair i).  Heads 0..n_head-1 are q (rotated
// in place), the next n_kv are k (rotated and stored into the cache); the k
// threads also copy v into the cache.  Pair i < n_rot/2 rotates elements
// (2i, 2i+1) ("norm", llama) or (i, i + n_rot/2) ("neox") by the angle
// pos * inv_freq[i] from the host-computed fp32 tables; dimensions past
// n_rot are left as they are.  Products and differences are rounded
// separately (no fused multiply-add: contraction is off in these kernels),
// as NumPy evaluates x0*c - x1*s.
__global__ void __launch_bounds__(256)
    k_rope_kv(float *__restrict__ q, const float *__restrict__ k,
              const float *__restrict__ v, int64_t T, int n_head, int n_kv,
              int hd, int n_rot, int neox, const float *__restrict__ cos_t,
              const float *__restrict__ sin_t, const aq_decode_state *st,
              int64_t pos0, int64_t n_ctx, float *__restrict__ kc,
              float *__restrict__ vc) {
#pragma clang fp contract(off)
  const int pairs = hd / 2, half = n_rot / 2;
  const int64_t per_tok = (int64_t)(n_head + n_kv) * pairs;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= T * per_tok) return;
  const int64_t t = gid / per_tok;
  const int r = (int)(gid - t * per_tok);
  const int h = r / pairs, i = r - h * pairs;
  const int64_t pos = (st ? (int64_t)st->pos : pos0) + t;
  if (pos < 0 || pos >= n_ctx) return;
  int a, b;
  if (i < half) {
    a = neox ? i : 2 * i;
    b = neox ? i + half : 2 * i + 1;
  } else {  // past n_rot: untouched pair of dimensions
    a = n_rot + 2 * (i - half);
    b = a + 1;
  }
  const bool is_q = h < n_head;
  const float *src = is_q ? q + (t * n_head + h) * hd : k + (t * n_kv + (h - n_head)) * hd;
  float x0 = src[a], x1 = src[b];
  if (i < half) {
    const float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
    const float r0 = x0 * c - x1 * s;
    const float r1 = x0 * s + x1 * c;
    x0 = r0;
    x1 = r1;
  }
  if (is_q) {
    float *dst = q + (t * n_head + h) * hd;
    dst[a] = x0;
    dst[b] = x1;
  } else {
    const int kvh = h - n_head;
    const int64_t off = ((int64_t)kvh * n_ctx + pos) * hd;
    kc[off + a] = x0;
    kc[off + b] = x1;
    const float *vs = v + (t * n_kv + kvh) * hd;
    vc[off + a] = vs[a];
    vc[off + b] = vs[b];
  }
}

// ---- attention over the KV cache (model.py:447-455) ------------------------
// k_attn_partial runs calls of several query tokens (one token per call runs
// k_attn_split below).  Split over positions: workgroup (chunk, kv head) takes CH consecutive
// positions of one kv head for the G query heads that share it, in three
// phases:
//  1. scores: lane l of a wave holds dimensions 4*(l % LPP) .. +3 of position
//     slot l / LPP (a wave reads PPW whole cache rows, 1 KB, per load), so a
//     score is a four-term dot plus a reduction over LPP lanes; the scaled
//     scores go to LDS;
//  2. softmax statistics: one wave per query head takes the chunk's CH
//     scores (a lane each), their maximum m, the weights e^(s - m) (one exp
//     per score) and their sum l;
//  3. the weighted sum of the V rows the lanes already hold, reduced over the
//     slots and waves: the chunk's numerators.
// The partial (numerators, m, l) of every chunk is merged by k_attn_combine:
// the reference's max-subtracted softmax followed by the weighted sum of V,
// reassociated over chunks.
constexpr int kAttnIt = 4;  // positions per slot per workgroup
constexpr int kAttnQT = 16;  // query tokens per workgroup (batched, non-rotating form)
template <int HD>
struct AttnGeom {
  static constexpr int LPP = HD / 4;            // lanes per position
  static constexpr int PPW = 64 / LPP;          // positions per wave per step
  static constexpr int CH = 4 * kAttnIt * PPW;  // positions per workgroup (<= 64)
  static constexpr int PS = HD + 4;             // floats per partial: num, m, l, pad
};

// four floats through a global-memory pointer (HIP's float4 struct has no
// assignment to or from other address spaces)
typedef float f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4(global_ptr<const float> p) {
  const f4v v = *reinterpret_cast<global_ptr<const f4v>>(p);
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st4(global_ptr<float> p, float4 x) {
  *reinterpret_cast<global_ptr<f4v>>(p) = f4v{x.x, x.y, x.z, x.w};
}
// e^x of a softmax weight (x = s - max <= 0) as 2^(x log2 e) on the
// hardware's exp2 (v_exp_f32): the rounded product adds a relative error of
// about |x| 2^-24 ln 2, under 1e-6 for the |x| <= 17 whose weights count
// against the largest (e^-17 < 5e-8), where the full-precision expf spent ~10
// instructions per weight (1B decode step 1613 -> 1678 tok/s, the golden
// traces unchanged).  x = -inf gives 0.
__device__ __forceinline__ float exp_w(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}
__device__ __forceinline__ float exp_shift(float m, float mx) {
  return m == -INFINITY ? 0.f : exp_w(m - mx);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float wave_add(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// v of lanes l and l ^ OFF (OFF = 16 or 32), lower lane's first, in both
// lanes of the couple: gfx950's row swap with v as both operands (a VALU
// operation; __shfl_xor goes through LDS).  A commutative op on the pair
// gives the same bits as v op __shfl_xor(v, OFF).
template <int OFF>
__device__ __forceinline__ float2 lane_pair(float v) {
  static_assert(OFF == 16 || OFF == 32, "row swaps of 16 or 32 lanes");
  const unsigned u = __float_as_uint(v);
  const auto r = OFF == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int OFF>
__device__ __forceinline__ float add_xor(float v) {
  const float2 p = lane_pair<OFF>(v);
  return p.x + p.y;
}
template <int OFF>
__device__ __forceinline__ float max_xor(float v) {
  const float2 p = lane_pair<OFF>(v);
  return fmaxf(p.x, p.y);
}

// Rotation of four consecutive dimensions j0 = 4*d4 .. j0+3 of one head
// vector at position pos, as k_rope_kv rotates them (products and
// differences rounded separately).  "neox" pairs (i, i + n_rot/2) need
// n_rot % 8 == 0 so that the partner four-group is aligned.
//
// The table values come first (rope_cs), all loaded at once with indices
// clamped into the row, so that a kernel rotating several heads at one
// position reads them once and in one round trip (loaded where each pair is
// rotated, under its lane's condition, they were a chain of dependent loads);
// values of pairs a lane does not rotate are loaded but never applied.
struct RopeCS {
  float c[4], s[4];
};
__device__ __forceinline__ RopeCS rope_cs(int d4, int64_t pos, int n_rot, int neox,
                                          const float *__restrict__ cos_t,
                                          const float *__restrict__ sin_t) {
  RopeCS r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r.c[e] = 1.f;
    r.s[e] = 0.f;
  }
  const int half = n_rot / 2;
  if (half == 0) return r;  // no rotation (and an empty table)
  const float *cr = cos_t + pos * half, *sr = sin_t + pos * half;
  const int j0 = 4 * d4;
  if (!neox) {  // pairs j0 / 2 and j0 / 2 + 1
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int i = j0 / 2 + p < half ? j0 / 2 + p : half - 1;
      r.c[p] = cr[i];
      r.s[p] = sr[i];
    }
  } else {  // pairs (i, i + half) for the four dimensions of the lane
    const bool lo = j0 < half;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i0 = lo ? j0 + e : j0 + e - half;
      const int i = i0 < half ? i0 : half - 1;
      r.c[e] = cr[i];
      r.s[e] = sr[i];
    }
  }
  return r;
}
// The head vector's four dimensions of the lane (x) and, for "neox", the
// partner four-group (y, loaded by every lane: it lies in the row for any d4).
// (y is loaded by every lane, and without a branch: the lane's own group
// again when there is no partner)
__device__ __forceinline__ void rope_src(const float *__restrict__ src, int d4, int n_rot,
                                         int neox, float4 &x, float4 &y) {
  const int half = n_rot / 2;
  const int yi = neox && half > 0 ? (4 * d4 < half ? d4 + half / 4 : d4 - half / 4) : d4;
  x = reinterpret_cast<const float4 *>(src)[d4];
  y = reinterpret_cast<const float4 *>(src)[yi];
}
__device__ __forceinline__ float4 rope4_xy(float4 x, float4 y4, int d4, int n_rot, int neox,
                                           const RopeCS &cs) {
#pragma clang fp contract(off)
  const int half = n_rot / 2;
  const float v[4] = {x.x, x.y, x.z, x.w};
  float r[4] = {x.x, x.y, x.z, x.w};
  const int j0 = 4 * d4;
  if (!neox) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int i = j0 / 2 + p;
      if (i < half) {
        const float c = cs.c[p], s = cs.s[p];
        r[2 * p] = v[2 * p] * c - v[2 * p + 1] * s;
        r[2 * p + 1] = v[2 * p] * s + v[2 * p + 1] * c;
      }
    }
  } else if (j0 < n_rot) {
    const bool lo = j0 < half;
    const float y[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = cs.c[e], s = cs.s[e];
      r[e] = lo ? v[e] * c - y[e] * s : y[e] * s + v[e] * c;
    }
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}
__device__ __forceinline__ float4 rope4(const float *__restrict__ src, int d4, int64_t pos,
                                        int n_rot, int neox, const float *__restrict__ cos_t,
                                        const float *__restrict__ sin_t) {
  float4 x, y;
  rope_src(src, d4, n_rot, neox, x, y);
  return rope4_xy(x, y, d4, n_rot, neox, rope_cs(d4, pos, n_rot, neox, cos_t, sin_t));
}

// ROPE = false: q is already rotated and k/v of the position are in the
// cache (aq_attention, aq_attention_batch).  ROPE = true: q, k, v are the raw
// projections of one token; q is rotated in registers and the workgroup
// whose chunk holds the position rotates k, stores k and v and uses them
// from registers (aq_attention_rope).
//
// A workgroup holds one chunk of CH cached positions of one kv head in
// registers and runs QT consecutive query tokens of a batch against it
// (token t at position pos + t sees positions <= pos + t), so a batched
// prefill reads each chunk from L2 once per QT tokens instead of once per
// token.  Tokens whose range ends before the chunk leave no partial (the
// combine reads only the chunks a token reaches).
template <int HD, int G, bool ROPE, int QT>
__global__ void __launch_bounds__(256)
    k_attn_partial(const float *__restrict__ q, const float *__restrict__ k,
                   const float *__restrict__ v, int n_rot, int neox,
                   const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                   const aq_decode_state *st, int64_t pos0, int64_t n_ctx, float scale,
                   float *kc, float *vc, float *__restrict__ part, int n_chunks, int64_t T) {
  static_assert(!ROPE || QT == 1, "the rotating form runs one token");
  using AG = AttnGeom<HD>;
  constexpr int LPP = AG::LPP, PPW = AG::PPW, CH = AG::CH, PS = AG::PS;
  __shared__ float sc[G][CH];          // scores, then weights
  __shared__ float stat[G][2];         // m, l of each head
  __shared__ float red[4][G][HD];      // per-wave numerators
  const int kvh = blockIdx.y, chunk = blockIdx.x;
  const int64_t t0 = (int64_t)blockIdx.z * QT;
  const int64_t pbase0 = st ? (int64_t)st->pos : pos0;  // position of token 0
  // the tile's last token inside the batch and the cache
  int64_t t_end = t0 + QT < T ? t0 + QT : T;
  if (pbase0 + t_end > n_ctx) t_end = n_ctx - pbase0;
  if (t_end <= t0 || pbase0 + t0 < 0) return;  // nothing to do (uniform)
  const int64_t L_max = pbase0 + t_end;  // positions seen by the tile's last token
  if ((int64_t)chunk * CH >= L_max) return;  // whole workgroup: uniform exit
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = lane / LPP, d4 = lane % LPP;

  const float4 *kb = reinterpret_cast<const float4 *>(kc + (int64_t)kvh * n_ctx * HD);
  const float4 *vb = reinterpret_cast<const float4 *>(vc + (int64_t)kvh * n_ctx * HD);
  const int pw = wave * (kAttnIt * PPW) + slot;  // position of iteration 0 in the chunk
  const int64_t pbase = (int64_t)chunk * CH + pw;
  float4 kr[kAttnIt], vr[kAttnIt];
#pragma unroll
  for (int it = 0; it < kAttnIt; ++it) {
    const int64_t p = pbase + it * PPW;
    const int64_t pc = p < L_max ? p : L_max - 1;  // in bounds; masked below
    kr[it] = kb[pc * LPP + d4];
    vr[it] = vb[pc * LPP + d4];
  }
  if constexpr (ROPE) {
    // The chunk that holds the token's position: the LPP lanes that own it
    // rotate k, store k and v into the cache and use the new values from
    // registers (what they loaded there above is the old cache content), so
    // this workgroup waits for one round of loads like the others.
    const int64_t pos = pbase0 + t0;
    if ((int64_t)(chunk + 1) * CH >= pos + 1) {
#pragma unroll
      for (int it = 0; it < kAttnIt; ++it) {
        if (pbase + it * PPW != pos) continue;
        kr[it] = rope4(k + (int64_t)kvh * HD, d4, pos, n_rot, neox, cos_t, sin_t);
        vr[it] = reinterpret_cast<const float4 *>(v + (int64_t)kvh * HD)[d4];
        const int64_t off = ((int64_t)kvh * n_ctx + pos) * HD;
        reinterpret_cast<float4 *>(kc + off)[d4] = kr[it];
        reinterpret_cast<float4 *>(vc + off)[d4] = vr[it];
      }
    }
  }
  for (int64_t t = t0; t < t_end; ++t) {
    const int64_t L = pbase0 + t + 1;
    if ((int64_t)chunk * CH >= L) continue;  // the token does not reach this chunk
    const float *qt = q + t * gridDim.y * G * HD;
    float4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float *qh = qt + (int64_t)(kvh * G + g) * HD;
      if constexpr (ROPE) qv[g] = rope4(qh, d4, L - 1, n_rot, neox, cos_t, sin_t);
      else qv[g] = reinterpret_cast<const float4 *>(qh)[d4];
    }
    // 1. scores
#pragma unroll
    for (int it = 0; it < kAttnIt; ++it) {
      const bool valid = pbase + it * PPW < L;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = qv[g].x * kr[it].x + qv[g].y * kr[it].y + qv[g].z * kr[it].z +
                  qv[g].w * kr[it].w;
        s = row16_sum(s);
        if constexpr (LPP == 32) s += __shfl_xor(s, 16);
        if (d4 == 0) sc[g][pw + it * PPW] = valid ? s * scale : -INFINITY;
      }
    }
    __syncthreads();
    // 2. softmax statistics, one wave per head (CH <= 64 positions a lane each)
    for (int g = wave; g < G; g += 4) {
      const float s = lane < CH ? sc[g][lane] : -INFINITY;
      const float m = wave_max(s);  // position 0 of the chunk is always valid
      const float e = s == -INFINITY ? 0.f : exp_w(s - m);
      const float l = wave_add(e);
      if (lane < CH) sc[g][lane] = e;
      if (lane == 0) {
        stat[g][0] = m;
        stat[g][1] = l;
      }
    }
    __syncthreads();
    // 3. weighted sum of V
    float4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int it = 0; it < kAttnIt; ++it) {
        const float w = sc[g][pw + it * PPW];
        acc[g].x = fmaf(w, vr[it].x, acc[g].x);
        acc[g].y = fmaf(w, vr[it].y, acc[g].y);
        acc[g].z = fmaf(w, vr[it].z, acc[g].z);
        acc[g].w = fmaf(w, vr[it].w, acc[g].w);
      }
#pragma unroll
      for (int off = LPP; off < 64; off *= 2) {
        acc[g].x += __shfl_xor(acc[g].x, off);
        acc[g].y += __shfl_xor(acc[g].y, off);
        acc[g].z += __shfl_xor(acc[g].z, off);
        acc[g].w += __shfl_xor(acc[g].w, off);
      }
      if (slot == 0) reinterpret_cast<float4 *>(&red[wave][g][0])[d4] = acc[g];
    }
    __syncthreads();
    float *pt = part + t * gridDim.y * n_chunks * G * PS;
    for (int i = threadIdx.x; i < G * HD; i += 256) {
      const int g = i / HD, d = i - g * HD;
      float *pp = pt + (((int64_t)kvh * n_chunks + chunk) * G + g) * PS;
      pp[d] = (red[0][g][d] + red[1][g][d]) + (red[2][g][d] + red[3][g][d]);
      if (d == 0) {
        pp[HD] = stat[g][0];
        pp[HD + 1] = stat[g][1];
      }
    }
    if (QT > 1) __syncthreads();  // sc, stat and red are rewritten by the next token
  }
}

// ---- attention of one query token, split over positions (the decode step) --
// Workgroup (split j, kv head) takes chunks j, j + S, j + 2S, ... (S splits,
// CH positions per chunk) of positions 0..p.  Wave w of it owns positions
// w*WPOS .. w*WPOS + WPOS - 1 of every chunk and keeps its own online-softmax
// state per query head over all of them: a running maximum m, the sum l of
// e^(s - m) and the numerators o = sum e^(s - m) V, rescaled by e^(m - m')
// whenever the maximum grows.  The loads of the next chunk are issued before
// the current one is computed (two register sets), nothing inside the loop
// synchronizes the workgroup, and the kSplitWaves waves' states are merged once at
// the end through LDS into the split's partial (numerators, m, l), which
// k_attn_combine merges over the splits.  The result differs from the
// reference's softmax only by the reassociation of these sums.
//
// ROPE: q is rotated in registers; the workgroup whose chunk holds p rotates
// k, stores k and v at p and uses them from registers (no other workgroup
// reads position p).
// waves per split workgroup: 4 (four positions per slot and chunk).  With
// the full-precision expf 8 waves ran the decode step faster (1598 -> 1618
// tok/s); with the weights on the hardware exp2 4 do (1720 against 1697).
constexpr int kSplitWaves = 4;
constexpr int kAttnSplits = 32;      // most splits per kv head
constexpr int kAttnSplitChunks = 2;  // chunks per split of a full cache, below that
// splits of a cache of n_chunks chunks
inline int attn_splits(int64_t n_chunks) {
  const int64_t s = n_chunks / kAttnSplitChunks;
  return (int)(s < 1 ? 1 : s > kAttnSplits ? kAttnSplits : s);
}
// Arguments: the first 14 dwords (kc .. rot) are what the start needs and
// arrive preloaded in scalar registers (the file is built with kernel
// argument preloading); rot = n_rot | neox << 16.
template <int HD, int G, bool ROPE>
__global__ void __launch_bounds__(64 * kSplitWaves)
    k_attn_split(float *kc, float *vc, const aq_decode_state *st,
                 const float *__restrict__ q, const float *__restrict__ k,
                 const float *__restrict__ v, int n_ctx32, int rot, int64_t pos0,
                 const float *__restrict__ cos_t, const float *__restrict__ sin_t, float scale,
                 float *__restrict__ part) {
  // every fused multiply-add is written out, so the rotating and the plain
  // instances round the same way (the compiler would contract each
  // differently)
#pragma clang fp contract(off)
  using AG = AttnGeom<HD>;
  constexpr int LPP = AG::LPP, PPW = AG::PPW, CH = AG::CH, PS = AG::PS;
  constexpr int SIT = CH / (kSplitWaves * PPW);  // positions per slot and chunk
  constexpr int WPOS = SIT * PPW;  // positions of a chunk per wave
  __shared__ float wst[kSplitWaves][G][HD + 2];  // per wave and head: o[HD], m, l
  // The preloaded arguments (pinned in scalar registers), then every load
  // that does not depend on the position - the split's first chunk (j < S <=
  // the cache's chunks, so it lies in the cache), q, k and v - and only then
  // the position, whose round trip runs under theirs (with the rest of the
  // arguments'), and the rope table values at it, in one round trip for all
  // the heads.  Read where they were used, the arguments, the position and
  // the table values made a chain of about ten dependent round trips before
  // the first score.  Pointers are pinned as global-memory pointers: a
  // pinned generic pointer would turn every access through it into a flat
  // one.
  global_ptr<const float> gq = as_global(q), gk = as_global(k), gv = as_global(v);
  global_ptr<float> gkc = as_global(kc), gvc = as_global(vc);
  asm volatile("" : "+s"(gq), "+s"(gk), "+s"(gv), "+s"(gkc), "+s"(gvc), "+s"(n_ctx32), "+s"(rot),
               "+s"(st));
  const int64_t n_ctx = n_ctx32;
  const int n_rot = rot & 0xffff, neox = rot >> 16;
  const int j = blockIdx.x, S = gridDim.x, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = lane / LPP, d4 = lane % LPP;
  float *kh = (float *)gkc + (int64_t)kvh * n_ctx * HD, *vh = (float *)gvc + (int64_t)kvh * n_ctx * HD;
  const int pw = wave * WPOS + slot;  // this lane's position in a chunk, load 0
  // chunk c through buffer resources over its bytes: positions past the
  // cache read zeros (masked below), and a chunk past the last active one has
  // resources of zero bytes, so the loop below issues every load
  // unconditionally (a load under a branch would make the compiler wait for
  // the other register set's loads too) without touching memory
  float4 kr0[SIT], vr0[SIT], kr1[SIT], vr1[SIT];
  int n_act = 0;  // chunks below the position, known after its load
  auto load = [&](int c, float4 *kr, float4 *vr) {
    const bool live = c == j || c < n_act;
    const int64_t p0 = (int64_t)(live ? c : j) * CH;
    const int64_t np = n_ctx - p0 < CH ? n_ctx - p0 : CH;
    const int bytes = live ? (int)(np * HD * sizeof(float)) : 0;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(kh + p0 * HD, 0, bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(vh + p0 * HD, 0, bytes, kRsrcWord3);
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int off = ((pw + it * PPW) * HD + 4 * d4) * (int)sizeof(float);
      kr[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
      vr[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    }
  };
  load(j, kr0, vr0);
  float4 qv[G], qy[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const global_ptr<const float> qh = gq + (int64_t)(kvh * G + g) * HD;
    if constexpr (ROPE) rope_src((const float *)qh, d4, n_rot, neox, qv[g], qy[g]);
    else qv[g] = ld4(qh + 4 * d4);
  }
  // the new k (rotated) and v of position p, loaded with q by every lane: the
  // lanes that own p use them inside the loop without a memory round trip of
  // their own there (the kernel ends with its slowest workgroup, the one
  // whose chunk holds p)
  float4 k_new = make_float4(0.f, 0.f, 0.f, 0.f), v_new = k_new, k_y = k_new;
  if constexpr (ROPE) {
    rope_src((const float *)(gk + (int64_t)kvh * HD), d4, n_rot, neox, k_new, k_y);
    v_new = ld4(gv + (int64_t)kvh * HD + 4 * d4);
  }
  // the position word, without a branch (the cache's first word when there is
  // no state) and through the constant address space, so that it is a scalar
  // load: its wait is not the vector loads' counter, which would wait for the
  // whole first chunk (the state is written by an earlier kernel only)
  using CI32 = const __attribute__((address_space(4))) int32_t;
  const int32_t pos_word = *(CI32 *)(st ? &st->pos : reinterpret_cast<const int32_t *>(kc));
  // the arguments past the preloaded ones, awaited with the position
  global_ptr<const float> gcos = as_global(cos_t), gsin = as_global(sin_t);
  global_ptr<float> gpart = as_global(part);
  asm volatile("" : "+s"(gcos), "+s"(gsin), "+s"(gpart), "+s"(pos0), "+s"(scale));
  const int64_t pos = st ? (int64_t)pos_word : pos0;
  if (pos < 0 || pos >= n_ctx) return;  // uniform: no position of the cache
  const int64_t L = pos + 1;
  n_act = (int)((L + CH - 1) / CH);
  if (j >= n_act) return;  // uniform: this split has no chunk
  if constexpr (ROPE) {
    const RopeCS cs = rope_cs(d4, pos, n_rot, neox, (const float *)gcos, (const float *)gsin);
#pragma unroll
    for (int g = 0; g < G; ++g) qv[g] = rope4_xy(qv[g], qy[g], d4, n_rot, neox, cs);
    k_new = rope4_xy(k_new, k_y, d4, n_rot, neox, cs);
  }
  float m[G], l[G];
  float4 o[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  auto compute = [&](int c, float4 *kr, float4 *vr) {
    if constexpr (ROPE) {
      // the chunk that holds position p: its owner lanes store the new k
      // and v into the cache and use them (what they loaded is the old cache
      // content)
      if ((int64_t)c * CH <= pos && pos < (int64_t)(c + 1) * CH) {
#pragma unroll
        for (int it = 0; it < SIT; ++it) {
          if ((int64_t)c * CH + pw + it * PPW != pos) continue;
          kr[it] = k_new;
          vr[it] = v_new;
          const int64_t off = ((int64_t)kvh * n_ctx + pos) * HD;
          st4(gkc + off + 4 * d4, kr[it]);
          st4(gvc + off + 4 * d4, vr[it]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[SIT];
      float mc = -INFINITY;
#pragma unroll
      for (int it = 0; it < SIT; ++it) {
        float d = fmaf(qv[g].w, kr[it].w,
                       fmaf(qv[g].z, kr[it].z, fmaf(qv[g].y, kr[it].y, qv[g].x * kr[it].x)));
        d = row16_sum(d);
        if constexpr (LPP == 32) d = add_xor<16>(d);
        const bool valid = (int64_t)c * CH + pw + it * PPW < L;
        s[it] = valid ? d * scale : -INFINITY;
        mc = fmaxf(mc, s[it]);
      }
      // the maximum over the wave's slots (lane groups of LPP)
      if constexpr (LPP == 16) mc = max_xor<16>(mc);
      mc = max_xor<32>(mc);
      const float mn = fmaxf(m[g], mc);
      const float corr = exp_shift(m[g], mn);
      float es = 0.f;
      float4 acc = make_float4(o[g].x * corr, o[g].y * corr, o[g].z * corr, o[g].w * corr);
#pragma unroll
      for (int it = 0; it < SIT; ++it) {
        const float e = s[it] == -INFINITY ? 0.f : exp_w(s[it] - mn);
        es += e;
        acc.x = fmaf(e, vr[it].x, acc.x);
        acc.y = fmaf(e, vr[it].y, acc.y);
        acc.z = fmaf(e, vr[it].z, acc.z);
        acc.w = fmaf(e, vr[it].w, acc.w);
      }
      l[g] = fmaf(l[g], corr, es);
      o[g] = acc;
      m[g] = mn;
    }
  };
  // two register sets in turn: the loads of chunk c + S are in flight while
  // chunk c is computed
  for (int c = j;;) {
    load(c + S, kr1, vr1);
    compute(c, kr0, vr0);
    if ((c += S) >= n_act) break;
    load(c + S, kr0, vr0);
    compute(c, kr1, vr1);
    if ((c += S) >= n_act) break;
  }
  // the wave's state summed over its slots (lanes of a slot hold the same
  // l; o holds a slot's share), then the workgroup's waves merged through LDS
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if constexpr (LPP == 16) {
      o[g] = make_float4(add_xor<16>(o[g].x), add_xor<16>(o[g].y), add_xor<16>(o[g].z),
                         add_xor<16>(o[g].w));
      l[g] = add_xor<16>(l[g]);
    }
    o[g] = make_float4(add_xor<32>(o[g].x), add_xor<32>(o[g].y), add_xor<32>(o[g].z),
                       add_xor<32>(o[g].w));
    l[g] = add_xor<32>(l[g]);
    if (slot == 0) reinterpret_cast<float4 *>(&wst[wave][g][0])[d4] = o[g];
    if (lane == 0) {
      wst[wave][g][HD] = m[g];
      wst[wave][g][HD + 1] = l[g];
    }
  }
  __syncthreads();
  const global_ptr<float> pp = gpart + ((int64_t)kvh * S + j) * G * PS;
  for (int i = threadIdx.x; i < G * HD; i += 64 * kSplitWaves) {
    const int g = i / HD, d = i - g * HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) M = fmaxf(M, wst[w][g][HD]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) {
      const float e = exp_shift(wst[w][g][HD], M);
      num = fmaf(wst[w][g][d], e, num);
      den = fmaf(wst[w][g][HD + 1], e, den);
    }
    pp[g * PS + d] = num;
    if (d == 0) {
      pp[g * PS + HD] = M;
      pp[g * PS + HD + 1] = den;
    }
  }
}

// Batched causal attention (the prefill form, T > 1 query tokens): one
// workgroup per (4 waves x 16 query rows, kv head).  A wave owns NTG = 16
// (token, head) rows - 16 / G consecutive tokens times the G query heads of
// the kv head - and keeps for each row the running max m, sum l and
// numerator o of an online softmax over the chunks of 64 cached positions.
// The workgroup stages each chunk once in LDS (K transposed, V row-major).
// Every lane holds a 4 x 4 register block: rows 4*rg..4*rg+3 (rg = lane/16)
// times positions 4*cq..4*cq+3 for the scores, times dimensions 4*cq.. (+64k)
// for the values (cq = lane % 16), so each 16 FMAs take two 16-byte LDS reads
// shared by 16-lane groups:
//   scores  s = q . K^T                 (q rows from LDS, K^T from LDS)
//   softmax m' = max(m, row max s), e = exp(s - m'), l = l e^(m-m') + row sum e
//           (row reductions over the 16 lanes of a row group)
//   values  o = o e^(m-m') + e V        (e through LDS, V from LDS)
// The output is o / l.  No partials and no second launch; positions past a
// token's own are masked, so each token sees exactly positions 0..pos.
constexpr int kPfRows = 16;  // (token, head) rows per wave
template <int HD, int G>
__global__ void __launch_bounds__(256)
    k_attn_prefill(const float *__restrict__ q, const float *__restrict__ kc,
                   const float *__restrict__ vc, const aq_decode_state *st, int64_t pos0,
                   int64_t n_ctx, int64_t T, float scale, float *__restrict__ out) {
  constexpr int NTG = kPfRows, TPW = NTG / G, TPB = 4 * TPW, CH = 64, DPL = HD / 64;
  static_assert(NTG % G == 0 && HD % 64 == 0, "rows per wave, dimension blocks");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *Kt = lds;                     // [HD][CH]
  float *Vs = Kt + HD * CH;            // [CH][HD]
  float *qs = Vs + CH * HD;            // [4 waves][HD][NTG]
  float *ws = qs + 4 * HD * NTG;       // [4 waves][CH][NTG]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> 4, cq = lane & 15;
  const int kvh = blockIdx.y, n_head = gridDim.y * G;
  const int64_t tw = (int64_t)blockIdx.x * TPB + wave * TPW;  // this wave's first token
  const int64_t pb = st ? (int64_t)st->pos : pos0;            // position of token 0
  float *qw = qs + wave * HD * NTG, *ww = ws + wave * CH * NTG;
  // the wave's query rows into LDS (tokens past T: zeros, never stored)
#pragma unroll
  for (int r = 0; r < NTG; ++r) {
    const int64_t t = tw + r / G;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const int d = lane + 64 * k;
      qw[d * NTG + r] = t < T ? q[(t * n_head + kvh * G + r % G) * HD + d] : 0.f;
    }
  }
  int64_t t_last = (int64_t)blockIdx.x * TPB + TPB - 1;
  t_last = t_last < T ? t_last : T - 1;
  const int n_c = (int)((pb + t_last + 1 + CH - 1) / CH);  // chunks the last token reaches
  // this lane's rows: 4*rg + i; the last position each may see
  int64_t lim[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lim[i] = pb + tw + (4 * rg + i) / G;
  float m[4], l[4], o[4][DPL][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[i][k][j] = 0.f;
  }
  const float4 *kb = reinterpret_cast<const float4 *>(kc + (int64_t)kvh * n_ctx * HD);
  const float4 *vb = reinterpret_cast<const float4 *>(vc + (int64_t)kvh * n_ctx * HD);
  for (int c = 0; c < n_c; ++c) {
    __syncthreads();  // the previous chunk is consumed (and the q rows are staged)
    for (int i = threadIdx.x; i < CH * (HD / 4); i += 256) {
      const int p = i / (HD / 4), d4 = i - p * (HD / 4);
      int64_t pg = (int64_t)c * CH + p;
      pg = pg < n_ctx ? pg : n_ctx - 1;  // in bounds; such positions are masked
      const float4 kv = kb[pg * (HD / 4) + d4], vv = vb[pg * (HD / 4) + d4];
      Kt[(4 * d4 + 0) * CH + p] = kv.x;
      Kt[(4 * d4 + 1) * CH + p] = kv.y;
      Kt[(4 * d4 + 2) * CH + p] = kv.z;
      Kt[(4 * d4 + 3) * CH + p] = kv.w;
      reinterpret_cast<float4 *>(Vs)[p * (HD / 4) + d4] = vv;
    }
    __syncthreads();
    // scores of rows 4rg+i at positions 4cq+j of the chunk
    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[i][j] = 0.f;
    for (int d = 0; d < HD; ++d) {
      const float4 qq = reinterpret_cast<const float4 *>(qw + d * NTG)[rg];
      const float4 kk = reinterpret_cast<const float4 *>(Kt + d * CH)[cq];
      const float qa[4] = {qq.x, qq.y, qq.z, qq.w}, ka[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[i][j] = fmaf(qa[i], ka[j], sc[i][j]);
    }
    // online softmax per row; row reductions over the 16 lanes of the group
    float e[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t pg = (int64_t)c * CH + 4 * cq + j;
        sc[i][j] = pg <= lim[i] ? sc[i][j] * scale : -INFINITY;
        mx = fmaxf(mx, sc[i][j]);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      const float mn = fmaxf(m[i], mx);
      const float corr = exp_shift(m[i], mn);
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[i][j] = sc[i][j] == -INFINITY ? 0.f : exp_w(sc[i][j] - mn);
        sum += e[i][j];
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off);
      l[i] = l[i] * corr + sum;
      m[i] = mn;
#pragma unroll
      for (int k = 0; k < DPL; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) o[i][k][j] *= corr;
    }
    // weights to LDS: position 4cq+j, rows 4rg..4rg+3 (read back by the wave)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      reinterpret_cast<float4 *>(ww + (4 * cq + j) * NTG)[rg] =
          make_float4(e[0][j], e[1][j], e[2][j], e[3][j]);
    // values: rows 4rg+i, dimensions 64k + 4cq + j
    for (int p = 0; p < CH; ++p) {
      const float4 w4 = reinterpret_cast<const float4 *>(ww + p * NTG)[rg];
      const float wa[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const float4 vv = reinterpret_cast<const float4 *>(Vs + p * HD + 64 * k)[cq];
        const float va[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[i][k][j] = fmaf(wa[i], va[j], o[i][k][j]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * rg + i;
    const int64_t t = tw + r / G;
    if (t < T) {
      const float inv = 1.f / l[i];
#pragma unroll
      for (int k = 0; k < DPL; ++k)
        reinterpret_cast<float4 *>(out + (t * n_head + kvh * G + r % G) * HD + 64 * k)[cq] =
            make_float4(o[i][k][0] * inv, o[i][k][1] * inv, o[i][k][2] * inv, o[i][k][3] * inv);
    }
  }
}

// The same batched causal attention on fp32 matrix cores
// (v_mfma_f32_16x16x4f32), the default form: the fp32 products and sums of
// the VALU kernel above at twice its speed (552 -> 268 us per layer of the
// 1B model's 2048-token prefill).  The grid, the rows of a wave (16 (token, head)
// rows, 16 / G tokens times the G heads) and the online softmax over
// 64-position chunks are k_attn_prefill's.  Per chunk, staged in LDS (K
// row-major, V transposed):
//   S^T (positions x rows) = K Q^T: lane l holds row l % 16's scores at
//     positions 16 pt + 4 (l / 16) + r (four 16-position tiles pt, r = 0..3);
//     the k index of lane group c = l / 16 in step s is dimension c HD/4 + s,
//     so a lane's q fragment and K reads are HD/4 consecutive floats;
//   the row's maximum and sum over the chunk: the lane's 16 scores, then the
//     four lanes of the row (xor 16, xor 32);
//   O^T (dimensions x rows) += V^T P^T: the weights are the B operand as the
//     lanes hold them (step (pt, r) takes position 16 pt + 4 c + r in lane
//     group c), V^T the A operand, so the rescale of O by e^(m - m') is a
//     lane's own row.
// The output is O / l.  Positions past a token's own are masked.
template <int HD, int G, int NW>
__global__ void __launch_bounds__(64 * NW)
    k_attn_prefill_mfma(const float *__restrict__ q, const float *__restrict__ kc,
                        const float *__restrict__ vc, const aq_decode_state *st, int64_t pos0,
                        int64_t n_ctx, int64_t T, float scale, float *__restrict__ out) {
  constexpr int NTG = kPfRows, TPW = NTG / G, TPB = NW * TPW, CH = 64, NT = 64 * NW;
  constexpr int KS = HD / 4;          // k steps of S^T (dimensions per lane)
  constexpr int NHT = HD / 16;        // 16-dimension tiles of O^T
  constexpr int LK = HD + 4, LV = CH + 4;  // LDS row strides (floats)
  constexpr int F4 = CH * HD / 4;     // float4 of K (and of V) per chunk
  constexpr int PT = F4 / NT;         // per thread
  static_assert(F4 % NT == 0 && KS % 4 == 0, "the chunk divides over the threads");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *Ks = lds;            // [CH][LK]
  float *Vt = Ks + CH * LK;   // [HD][LV]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, cg = lane >> 4;
  const int kvh = blockIdx.y, n_head = gridDim.y * G;
  const int64_t tw = (int64_t)blockIdx.x * TPB + wave * TPW;  // this wave's first token
  const int64_t pb = st ? (int64_t)st->pos : pos0;            // position of token 0
  // this lane's row (r16): token, head, last position it may see
  const int64_t t_row = tw + r16 / G;
  const int h_row = kvh * G + r16 % G;
  const int64_t lim = pb + t_row;
  // q fragment: dimensions cg*KS .. cg*KS + KS - 1 of the row (zeros past T)
  float qf[KS];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t_row < T) v = reinterpret_cast<const float4 *>(q + (t_row * n_head + h_row) * HD + cg * KS)[j];
    qf[4 * j] = v.x;
    qf[4 * j + 1] = v.y;
    qf[4 * j + 2] = v.z;
    qf[4 * j + 3] = v.w;
  }
  int64_t t_last = (int64_t)blockIdx.x * TPB + TPB - 1;
  t_last = t_last < T ? t_last : T - 1;
  const int n_c = (int)((pb + t_last + 1 + CH - 1) / CH);  // chunks the last token reaches
  // (native 4-vectors: HIP's float4 struct kept these arrays in scratch)
  typedef float f4v_ __attribute__((ext_vector_type(4)));
  const f4v_ *kb = reinterpret_cast<const f4v_ *>(kc + (int64_t)kvh * n_ctx * HD);
  const f4v_ *vb = reinterpret_cast<const f4v_ *>(vc + (int64_t)kvh * n_ctx * HD);
  // float4 i of a chunk: position i / (HD/4), dimensions 4 (i % (HD/4)) ..
  f4v_ rk[PT], rv[PT];
#define AQ_PF_FETCH(c)                                                          \
  _Pragma("unroll") for (int j = 0; j < PT; ++j) {                             \
    const int i = tid + NT * j;                                                 \
    int64_t pg = (int64_t)(c) * CH + i / (HD / 4);                              \
    pg = pg < n_ctx ? pg : n_ctx - 1; /* in bounds; such positions are masked */ \
    rk[j] = kb[pg * (HD / 4) + i % (HD / 4)];                                   \
    rv[j] = vb[pg * (HD / 4) + i % (HD / 4)];                                   \
  }
  f4v_ o[NHT];
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) o[ht] = f4v_{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  AQ_PF_FETCH(0)
  for (int c = 0; c < n_c; ++c) {
    __syncthreads();  // the previous chunk is consumed
#pragma unroll
    for (int j = 0; j < PT; ++j) {  // stage: K row-major, V transposed
      const int i = tid + NT * j;
      const int p = i / (HD / 4), d4 = i % (HD / 4);
      *reinterpret_cast<f4v_ *>(&Ks[p * LK + 4 * d4]) = rk[j];
      Vt[(4 * d4 + 0) * LV + p] = rv[j][0];
      Vt[(4 * d4 + 1) * LV + p] = rv[j][1];
      Vt[(4 * d4 + 2) * LV + p] = rv[j][2];
      Vt[(4 * d4 + 3) * LV + p] = rv[j][3];
    }
    __syncthreads();
    if (c + 1 < n_c) {  // the next chunk's loads fly during this one
      AQ_PF_FETCH(c + 1)
    }
    // scores S^T of the four 16-position tiles
    f4v_ sc[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
      sc[pt] = f4v_{0.f, 0.f, 0.f, 0.f};
      const float *kr = &Ks[(pt * 16 + r16) * LK + cg * KS];
#pragma unroll
      for (int j = 0; j < KS / 4; ++j) {
        const float4 kv = reinterpret_cast<const float4 *>(kr)[j];
        sc[pt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qf[4 * j], sc[pt], 0, 0, 0);
        sc[pt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qf[4 * j + 1], sc[pt], 0, 0, 0);
        sc[pt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qf[4 * j + 2], sc[pt], 0, 0, 0);
        sc[pt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qf[4 * j + 3], sc[pt], 0, 0, 0);
      }
    }
    // lane (r16, cg) of tile pt holds S^T[16 pt + 4 cg + r][row r16]
    float mx = -INFINITY;
#pragma unroll
    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t pg = (int64_t)c * CH + pt * 16 + 4 * cg + r;
        sc[pt][r] = pg <= lim ? sc[pt][r] * scale : -INFINITY;
        mx = fmaxf(mx, sc[pt][r]);
      }
    mx = max_xor<16>(mx);
    mx = max_xor<32>(mx);
    const float mn = fmaxf(m, mx);
    const float corr = exp_shift(m, mn);
    float sum = 0.f;
#pragma unroll
    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = sc[pt][r] == -INFINITY ? 0.f : exp_w(sc[pt][r] - mn);
        sc[pt][r] = e;
        sum += e;
      }
    sum = add_xor<16>(sum);
    sum = add_xor<32>(sum);
    l = l * corr + sum;
    m = mn;
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      o[ht] *= corr;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const float4 vv = *reinterpret_cast<const float4 *>(&Vt[(ht * 16 + r16) * LV + pt * 16 + 4 * cg]);
        o[ht] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, sc[pt][0], o[ht], 0, 0, 0);
        o[ht] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, sc[pt][1], o[ht], 0, 0, 0);
        o[ht] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, sc[pt][2], o[ht], 0, 0, 0);
        o[ht] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, sc[pt][3], o[ht], 0, 0, 0);
      }
    }
  }
#undef AQ_PF_FETCH
  // lane (r16, cg) of tile ht holds O^T[16 ht + 4 cg + r][row r16]
  if (t_row < T) {
    const float inv = 1.f / l;
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht)
      reinterpret_cast<float4 *>(out + (t_row * n_head + h_row) * HD + ht * 16)[cg] =
          make_float4(o[ht][0] * inv, o[ht][1] * inv, o[ht][2] * inv, o[ht][3] * inv);
  }
}

template <int HD, int G>
hipError_t prefill_attn_launch(const float *q, const float *kc, const float *vc, int n_kv,
                               int64_t n_ctx, const aq_decode_state *st, int64_t pos0,
                               int64_t T, float scale, float *out, hipStream_t s) {
  constexpr int TPB = 4 * (kPfRows / G);
  const dim3 grid((unsigned)((T + TPB - 1) / TPB), (unsigned)n_kv);
  // matrix cores (the default; 4-wave workgroups: 26.6 ms for the 1B model's
  // 2048-token prefill against 27.4 ms with 8 waves and 27.8 ms with 2), or
  // the VALU kernel when AQ_ATTN_PREFILL_VALU is set (31.2 ms)
  if (!getenv("AQ_ATTN_PREFILL_VALU")) {
    const size_t lds = (size_t)(64 * (HD + 4) + HD * (64 + 4)) * sizeof(float);
    hipError_t e =
        set_dynamic_lds(reinterpret_cast<const void *>(k_attn_prefill_mfma<HD, G, 4>), (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attn_prefill_mfma<HD, G, 4>), grid, dim3(256), lds, s, q, kc, vc, st,
                       pos0, n_ctx, T, scale, out);
    return hipGetLastError();
  }
  const size_t lds = (size_t)(2 * 64 * HD + 4 * HD * kPfRows + 4 * 64 * kPfRows) * sizeof(float);
  hipError_t e = set_dynamic_lds(reinterpret_cast<const void *>(k_attn_prefill<HD, G>), (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_attn_prefill<HD, G>), grid, dim3(256), lds, s, q, kc, vc, st, pos0, n_ctx,
                     T, scale, out);
  return hipGetLastError();
}

// One workgroup of HD threads per query head merges the partials of the
// active chunks: out = sum_c num_c e^(m_c - M) / sum_c l_c e^(m_c - M).  The
// head's partials (PS floats per chunk, chunk stride G*PS) are staged into
// LDS a tile at a time with all loads in flight, then merged from LDS.
constexpr int kCombineTile = 64;  // chunks per LDS tile
constexpr int kCombineDirect = 32;  // most partials merged from registers (kAttnSplits)
template <int HD, int G>
__global__ void __launch_bounds__(HD)
    k_attn_combine(const float *__restrict__ part, const aq_decode_state *st,
                   int64_t pos0, int64_t n_ctx, int n_chunks, int max_parts, int heads,
                   float *__restrict__ out) {
  // partials of n_chunks slots per kv head, of which the first
  // min(max_parts, chunks below the position) were written: one per chunk
  // (k_attn_partial, max_parts = n_chunks) or one per split (k_attn_split)
  using AG = AttnGeom<HD>;
  constexpr int CH = AG::CH, PS = AG::PS;
  __shared__ __attribute__((aligned(16))) float tile[kCombineTile * PS];
  // The kernel arguments (all of them preloaded in scalar registers; heads
  // is the grid's x size, passed so that no dispatch-packet read is needed),
  // pinned (pointers as global-memory pointers, so that their accesses stay
  // global ones), then the position word, without a branch (the partials'
  // first word when there is no state) and through the constant address
  // space, so that it is a scalar load whose wait is not the partials' (read
  // where they were used, the arguments and the position each made a round
  // trip of their own).
  global_ptr<const float> gpart = as_global(part);
  global_ptr<float> gout = as_global(out);
  asm volatile("" : "+s"(gpart), "+s"(gout), "+s"(st), "+s"(pos0), "+s"(n_ctx), "+s"(n_chunks),
               "+s"(max_parts), "+s"(heads));
  using CI32 = const __attribute__((address_space(4))) int32_t;
  const int32_t pos_word = *(CI32 *)(st ? &st->pos : reinterpret_cast<const int32_t *>(part));
  const int head = blockIdx.x, kvh = head / G, g = head - kvh * G, d = threadIdx.x;
  const int t = blockIdx.y;  // query token of the batch
  gpart += (int64_t)t * heads * n_chunks * PS;
  gout += (int64_t)t * heads * HD;
  // the slots below the position (those the partial kernel wrote)
  auto active_slots = [&]() {
    int64_t L = (st ? (int64_t)pos_word : pos0) + t + 1;
    L = L < n_ctx ? L : n_ctx;
    const int n = (int)((L + CH - 1) / CH);
    return n < max_parts ? n : max_parts;
  };
  const global_ptr<const float> pp = gpart + ((int64_t)kvh * n_chunks * G + g) * PS;
  float M = -INFINITY, num = 0.f, den = 0.f;
  if (max_parts <= kCombineDirect) {
    // Up to kCombineDirect partial slots (every decode-step call): each
    // thread loads its numerator and every slot's m and l at once, through a
    // buffer resource over the max_parts slots (the loads do not wait for the
    // position; slots past the active ones are not used, those past
    // max_parts read zeros), and merges the active ones in slot order - the
    // same operations as the staged form below, without the LDS round trip.
    const int bytes = (int)(((max_parts - 1) * G * PS + PS) * sizeof(float));
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void *)(const float *)pp, 0, bytes, kRsrcWord3);
    uint32_t nv[kCombineDirect], mv[kCombineDirect], lv[kCombineDirect];  // float bits
#pragma unroll
    for (int c = 0; c < kCombineDirect; ++c) {
      const int o = c * G * PS * (int)sizeof(float);
      nv[c] = __builtin_amdgcn_raw_buffer_load_b32(rp, o + d * (int)sizeof(float), 0, 0);
      mv[c] = __builtin_amdgcn_raw_buffer_load_b32(rp, o + HD * (int)sizeof(float), 0, 0);
      lv[c] = __builtin_amdgcn_raw_buffer_load_b32(rp, o + (HD + 1) * (int)sizeof(float), 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before the position is awaited
    const int n_act = active_slots();
    float mt = M;
#pragma unroll
    for (int c = 0; c < kCombineDirect; ++c)
      if (c < n_act) mt = fmaxf(mt, __builtin_bit_cast(float, mv[c]));
    const float r = exp_shift(M, mt);
    num *= r;
    den *= r;
#pragma unroll
    for (int c = 0; c < kCombineDirect; ++c) {
      if (c < n_act) {
        const float e = exp_shift(__builtin_bit_cast(float, mv[c]), mt);
        num = fmaf(__builtin_bit_cast(float, nv[c]), e, num);
        den = fmaf(__builtin_bit_cast(float, lv[c]), e, den);
      }
    }
    gout[(int64_t)head * HD + d] = num / den;
    return;
  }
  const int n_act = active_slots();
  for (int c0 = 0; c0 < n_act; c0 += kCombineTile) {
    const int nc = n_act - c0 < kCombineTile ? n_act - c0 : kCombineTile;
    __syncthreads();  // the previous tile has been consumed
    // PS / 4 float4 per chunk; chunk c of the head at pp + (c0 + c) * G * PS
#pragma unroll 4
    for (int i = threadIdx.x; i < nc * (PS / 4); i += HD) {
      const int c = i / (PS / 4), f = i - c * (PS / 4);
      reinterpret_cast<float4 *>(tile)[i] = ld4(pp + (int64_t)(c0 + c) * G * PS + 4 * f);
    }
    __syncthreads();
    float mt = M;
#pragma unroll 8
    for (int c = 0; c < nc; ++c) mt = fmaxf(mt, tile[c * PS + HD]);
    const float r = exp_shift(M, mt);
    num *= r;
    den *= r;
#pragma unroll 8
    for (int c = 0; c < nc; ++c) {
      const float e = exp_shift(tile[c * PS + HD], mt);
      num = fmaf(tile[c * PS + d], e, num);
      den = fmaf(tile[c * PS + HD + 1], e, den);
    }
    M = mt;
  }
  gout[(int64_t)head * HD + d] = num / den;
}

// ---- SwiGLU (model.py:549-551) and residual add (model.py:546, :552) ------
// element i of gate and up at g[i * stride], u[i * stride] (stride 2 with
// u = g + 1: the interleaved (gate, up) pairs of one matmul_t)
__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                         int64_t stride, int64_t n, float *__restrict__ out) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const float gv = g[i * stride];
    out[i] = gv / (1.0f + expf(-gv)) * u[i * stride];
  }
}
__global__ void k_add(float *x, const float *y, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    x[i] = x[i] + y[i];
}
// x[r, :] += b for every row r: the bias adds of a batch (model.py:491-496)
__global__ void k_add_rows(float *x, const float *__restrict__ b, int64_t rows, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    float *xr = x + r * n;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256)
      xr[i] = xr[i] + b[i];
  }
}

// ---- greedy selection (tensor.py:187-194) with on-device feedback ---------
// The key orders (value, -index): larger value wins, and among equal values
// the lower index, which is np.argmax's first maximum.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - i);
}
__device__ __forceinline__ float argmax_key_value(unsigned long long k) {
  const uint32_t b = (uint32_t)(k >> 32);
  return __uint_as_float((b & 0x80000000u) ? (b & 0x7FFFFFFFu) : ~b);
}
__device__ __forceinline__ int64_t argmax_key_index(unsigned long long k) {
  return (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
}

// End of a step: k_argmax folds every workgroup's slice of the logits into
// st->key (atomicMax), then k_advance (one wave) moves the state on.  Two
// launches: the kernel boundary orders them without device-scope fences.
//
// Repetition penalty (sample.py:36-45): the window's tokens are left out of
// k_argmax (each workgroup marks the ones in its 512-element slice in an
// LDS bitmap) and k_advance takes their penalized values in double - the
// reference divides or multiplies Python floats - and merges the two
// maxima.  A penalty only moves a window token's value, so the maximum over
// everything is the larger of the two, the lower index on a tie.
constexpr int kArgSlice = 512;  // logits per k_argmax workgroup (256 x 2): ~250 workgroups
                                // for a 128K vocabulary

__global__ void __launch_bounds__(256)
    k_argmax(const float *__restrict__ v, int64_t n, aq_decode_state *st,
             const int64_t *__restrict__ window, int64_t last_n) {
  __shared__ uint32_t skip[kArgSlice / 32];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kArgSlice;
  if (window) {
    if (tid < kArgSlice / 32) skip[tid] = 0;
    __syncthreads();
    const int64_t seen = window[0];
    const int64_t cnt = seen < last_n ? seen : last_n;
    for (int64_t j = tid; j < cnt; j += 256) {
      const int64_t t = window[1 + j] - base;
      if (t >= 0 && t < kArgSlice) atomicOr(&skip[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
  }
  unsigned long long best = 0;
#pragma unroll
  for (int k = 0; k < kArgSlice / 256; ++k) {
    const int e = k * 256 + tid;
    const int64_t i = base + e;
    if (i < n && !(window && ((skip[e >> 5] >> (e & 31)) & 1u))) {
      const unsigned long long key = argmax_key(v[i], (uint32_t)i);
      best = key > best ? key : best;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off);
    best = o > best ? o : best;
  }
  // one atomic per workgroup: the waves' maxima meet in LDS first
  __shared__ unsigned long long wbest[4];
  if ((tid & 63) == 0) wbest[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int i = 1; i < 4; ++i) best = wbest[i] > best ? wbest[i] : best;
    if (best) atomicMax(&st->key, best);
  }
}

// (a, ia) := the larger of (a, ia) and (b, ib), the lower index on a tie.
__device__ __forceinline__ void max_first(double &a, int64_t &ia, double b, int64_t ib) {
  if (b > a || (b == a && ib < ia)) {
    a = b;
    ia = ib;
  }
}

__global__ void __launch_bounds__(64)
    k_advance(aq_decode_state *st, const int64_t *__restrict__ prompt, int64_t n_prompt,
              int64_t *hist, int64_t cap, int take_argmax, const float *__restrict__ logits,
              int64_t n, int64_t *window, int64_t last_n, int penalize, double penalty) {
  const int lane = threadIdx.x;
  const int32_t f = st->fed;
  int64_t next = 0;
  if (f < n_prompt) {  // the prompt continues
    next = prompt[f];
  } else if (take_argmax) {
    const unsigned long long k = st->key;
    double bv = -__builtin_inf();
    int64_t bi = INT64_MAX;
    if (k) {  // 0: every logit is in the window
      bv = (double)argmax_key_value(k);
      bi = argmax_key_index(k);
    }
    if (penalize) {
      const int64_t seen = window[0];
      const int64_t cnt = seen < last_n ? seen : last_n;
      double pv = -__builtin_inf();
      int64_t pi = INT64_MAX;
      for (int64_t j = lane; j < cnt; j += 64) {
        const int64_t t = window[1 + j];
        if (t < 0 || t >= n) continue;
        const double x = (double)logits[t];
        max_first(pv, pi, x > 0.0 ? x / penalty : x * penalty, t);
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const double ov = __shfl_xor(pv, off);
        const int64_t oi = __shfl_xor(pi, off);
        max_first(pv, pi, ov, oi);
      }
      max_first(bv, bi, pv, pi);
    }
    next = bi;
  }
  if (lane != 0) return;
  if (f < n_prompt) {
    st->fed = f + 1;
  } else if (take_argmax) {
    const int32_t c = st->count;
    if (hist && c < cap) hist[c] = next;
    st->count = c + 1;
  }
  if (f < n_prompt || take_argmax) {
    st->token = next;
    if (window) {  // Sampler.accept (sample.py:31-34)
      const int64_t seen = window[0] > 0 ? window[0] : 0;
      window[1 + seen % last_n] = next;
      window[0] = seen + 1;
    }
  }
  st->key = 0;
  st->done = 0;
  st->pos += 1;
}

// The grid of one decode-attention launch and the extent of the partial
// scratch it writes, in floats.  One query token: k_attn_split, grid (S, n_kv),
// workgroup (j, kvh) writes the G partials of slot kvh * S + j.  Several:
// k_attn_partial, grid (n_chunks, n_kv, token tiles), workgroup (c, kvh) of
// token t writes slot (t * n_kv + kvh) * n_chunks + c.  A slot is G partials
// of PS floats.  attn_launch sizes nothing itself: it refuses a scratch
// smaller than this extent.
struct AttnGrid {
  int64_t n_chunks, slots_per_head;  // slots per (token, kv head)
  int64_t extent;                    // floats written: T * n_kv * slots * G * PS
};
template <int HD>
AttnGrid attn_grid(int n_kv, int G, int64_t n_ctx, int64_t T) {
  constexpr int CH = AttnGeom<HD>::CH, PS = AttnGeom<HD>::PS;
  AttnGrid a;
  a.n_chunks = (n_ctx + CH - 1) / CH;
  a.slots_per_head = T == 1 ? attn_splits(a.n_chunks) : a.n_chunks;
  a.extent = T * n_kv * a.slots_per_head * G * PS;
  return a;
}

template <int HD, int G, bool ROPE>
hipError_t attn_launch(const float *q, const float *k, const float *v, int n_rot, int neox,
                       const float *cos_t, const float *sin_t, int n_kv, int64_t n_ctx,
                       const aq_decode_state *st, int64_t pos0, int64_t T, float scale,
                       float *kc, float *vc, float *part, size_t part_bytes, float *out,
                       hipStream_t s) {
  constexpr int QT = ROPE ? 1 : kAttnQT;
  const AttnGrid ag = attn_grid<HD>(n_kv, G, n_ctx, T);
  // the partials this launch writes must fit the scratch it was handed
  if ((size_t)ag.extent * sizeof(float) > part_bytes) return hipErrorInvalidValue;
  const int n_chunks = (int)ag.n_chunks;
  if (T == 1) {  // one token: splits with per-wave online softmax
    if (n_ctx > INT32_MAX) return hipErrorInvalidValue;  // the split kernel takes an int
    const int S = (int)ag.slots_per_head;
    hipLaunchKernelGGL((k_attn_split<HD, G, ROPE>), dim3((unsigned)S, (unsigned)n_kv),
                       dim3(64 * kSplitWaves), 0, s, kc, vc, st, q, k, v, (int)n_ctx,
                       n_rot | neox << 16, pos0, cos_t, sin_t, scale, part);
    hipLaunchKernelGGL((k_attn_combine<HD, G>), dim3((unsigned)(n_kv * G), 1u), dim3(HD), 0, s,
                       part, st, pos0, n_ctx, S, S, n_kv * G, out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((k_attn_partial<HD, G, ROPE, QT>),
                     dim3((unsigned)n_chunks, (unsigned)n_kv, (unsigned)((T + QT - 1) / QT)),
                     dim3(256), 0, s, q, k, v, n_rot, neox, cos_t, sin_t, st, pos0, n_ctx, scale,
                     kc, vc, part, n_chunks, T);
  hipLaunchKernelGGL((k_attn_combine<HD, G>), dim3((unsigned)(n_kv * G), (unsigned)T), dim3(HD),
                     0, s, part, st, pos0, n_ctx, n_chunks, n_chunks, n_kv * G, out);
  return hipGetLastError();
}

}  // namespace

bool attention_supported(int head_dim, int group) {
  return (head_dim == 64 || head_dim == 128) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

size_t attention_scratch_bytes(int n_kv, int head_dim, int group, int64_t n_ctx, int64_t T) {
  const int ch = head_dim == 64 ? AttnGeom<64>::CH : AttnGeom<128>::CH;
  const int64_t n_chunks = (n_ctx + ch - 1) / ch;
  // one token: a partial per split; several: a partial per chunk and token
  const int64_t parts = T == 1 ? attn_splits(n_chunks) : n_chunks;
  return (size_t)T * n_kv * parts * group * (head_dim + 4) * sizeof(float);
}

size_t attention_launch_extent_bytes(int n_kv, int head_dim, int group, int64_t n_ctx,
                                     int64_t T) {
  const AttnGrid a = head_dim == 64 ? attn_grid<64>(n_kv, group, n_ctx, T)
                                    : attn_grid<128>(n_kv, group, n_ctx, T);
  return (size_t)a.extent * sizeof(float);
}

hipError_t launch_rmsnorm(const float *x, const float *w, int64_t rows,
                          int64_t n, float eps, float *out, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(kNormWG), 0, s, x, w, n,
                     eps, out);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float *x, const float *y, const float *w, int64_t rows,
                              int64_t n, float eps, float *out, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_add_rmsnorm, dim3((unsigned)rows), dim3(kNormWG), 0, s, x, y, w, n,
                     eps, out);
  return hipGetLastError();
}

hipError_t launch_rope_kv(float *q, const float *k, const float *v, int64_t T,
                          int n_head, int n_kv, int hd, int n_rot, int neox,
                          const float *cos_t, const float *sin_t,
                          const aq_decode_state *st, int64_t pos0, int64_t n_ctx,
                          float *kc, float *vc, hipStream_t s) {
  const int64_t n = T * (int64_t)(n_head + n_kv) * (hd / 2);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rope_kv, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, q,
                     k, v, T, n_head, n_kv, hd, n_rot, neox, cos_t, sin_t, st, pos0,
                     n_ctx, kc, vc);
  return hipGetLastError();
}

hipError_t launch_attention(const float *q, const float *kc, const float *vc,
                            int n_head, int n_kv, int hd, int64_t n_ctx,
                            const aq_decode_state *st, int64_t pos0, int64_t T, float *part,
                            size_t part_bytes, float *out, hipStream_t s) {
  const int G = n_head / n_kv;
  const float scale = (float)(1.0 / sqrt((double)hd));
#define AQ_ATT(hdv, gv)                                                              \
  if (hd == hdv && G == gv)                                                          \
    return attn_launch<hdv, gv, false>(q, nullptr, nullptr, 0, 0, nullptr, nullptr,  \
                                       n_kv, n_ctx, st, pos0, T, scale,              \
                                       const_cast<float *>(kc), const_cast<float *>(vc), \
                                       part, part_bytes, out, s);
  AQ_ATT(64, 1) AQ_ATT(64, 2) AQ_ATT(64, 4) AQ_ATT(64, 8)
  AQ_ATT(128, 1) AQ_ATT(128, 2) AQ_ATT(128, 4) AQ_ATT(128, 8)
#undef AQ_ATT
  return hipErrorInvalidValue;
}

hipError_t launch_attention_prefill(const float *q, const float *kc, const float *vc,
                                    int n_head, int n_kv, int hd, int64_t n_ctx,
                                    const aq_decode_state *st, int64_t pos0, int64_t T,
                                    float *out, hipStream_t s) {
  const int G = n_head / n_kv;
  const float scale = (float)(1.0 / sqrt((double)hd));
#define AQ_ATT(hdv, gv)                                                                   \
  if (hd == hdv && G == gv)                                                               \
    return prefill_attn_launch<hdv, gv>(q, kc, vc, n_kv, n_ctx, st, pos0, T, scale, out, s);
  AQ_ATT(64, 1) AQ_ATT(64, 2) AQ_ATT(64, 4) AQ_ATT(64, 8)
  AQ_ATT(128, 1) AQ_ATT(128, 2) AQ_ATT(128, 4) AQ_ATT(128, 8)
#undef AQ_ATT
  return hipErrorInvalidValue;
}

hipError_t launch_attention_rope(const float *q, const float *k, const float *v,
                                 int n_head, int n_kv, int hd, int n_rot, int neox,
                                 const float *cos_t, const float *sin_t, int64_t n_ctx,
                                 const aq_decode_state *st, int64_t pos0, float *kc,
                                 float *vc, float *part, size_t part_bytes, float *out,
                                 hipStream_t s) {
  const int G = n_head / n_kv;
  const float scale = (float)(1.0 / sqrt((double)hd));
#define AQ_ATT(hdv, gv)                                                               \
  if (hd == hdv && G == gv)                                                           \
    return attn_launch<hdv, gv, true>(q, k, v, n_rot, neox, cos_t, sin_t, n_kv, n_ctx, \
                                      st, pos0, 1, scale, kc, vc, part, part_bytes, out, s);
  AQ_ATT(64, 1) AQ_ATT(64, 2) AQ_ATT(64, 4) AQ_ATT(64, 8)
  AQ_ATT(128, 1) AQ_ATT(128, 2) AQ_ATT(128, 4) AQ_ATT(128, 8)
#undef AQ_ATT
  return hipErrorInvalidValue;
}

hipError_t launch_swiglu(const float *g, const float *u, int64_t stride, int64_t n,
                         float *out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int64_t wg = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  hipLaunchKernelGGL(k_swiglu, dim3((unsigned)wg), dim3(256), 0, s, g, u, stride, n, out);
  return hipGetLastError();
}

hipError_t launch_add(float *x, const float *y, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int64_t wg = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  hipLaunchKernelGGL(k_add, dim3((unsigned)wg), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_add_rows(float *x, const float *b, int64_t rows, int64_t n, hipStream_t s) {
  if (n == 0 || rows == 0) return hipSuccess;
  const int64_t gx = (n + 255) / 256 < 64 ? (n + 255) / 256 : 64;
  const int64_t gy = rows < 1024 ? rows : 1024;
  hipLaunchKernelGGL(k_add_rows, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, x, b,
                     rows, n);
  return hipGetLastError();
}

hipError_t launch_greedy_advance(const float *logits, int64_t n,
                                 aq_decode_state *st, const int64_t *prompt,
                                 int64_t n_prompt, int64_t *hist, int64_t cap,
                                 int take_argmax, int64_t *window, int64_t last_n,
                                 int penalize, double penalty, hipStream_t s) {
  if (take_argmax) {
    const int64_t wg = (n + kArgSlice - 1) / kArgSlice;
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)wg), dim3(256), 0, s, logits, n, st,
                       penalize ? window : nullptr, last_n);
  }
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, st, prompt, n_prompt, hist, cap,
                     take_argmax, logits, n, window, last_n, take_argmax && penalize ? 1 : 0,
                     penalty);
  return hipGetLastError();
}

}  // namespace aq
