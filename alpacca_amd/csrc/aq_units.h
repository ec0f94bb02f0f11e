// aq_units.h - the integer-dot view of each GGUF format used by the decode
// matvec (aq_matvec_i8.hip).
//
// x preparation.  x is cut into groups of 32 consecutive elements.  Group g
// with M = max|x_i| gets the power-of-two scale 2^e, e = exponent(M) - 6
// (so 2^e <= M / 32 and t_i = x_i / 2^e is exact with |t_i| < 64), and each
// element is written as three int8 pieces a, b, c in [-127, 127]:
//     x_i ~= 2^e * (a_i + (254 * b_i + c_i) / 254^2)
// (a = rint(t), b = rint(254 * rem), c = rint(254 * rem')).  The
// representation error is at most 2^e / (2 * 254^2) <= 2.5e-7 * M, so the
// matvec error normalized by ||W_r||*||x|| stays below sqrt(32) * 2.5e-7
// < 1.5e-6 whatever x is.  A dot product of 32 int codes with the pieces is
// then three exact int32 dot4 chains (v_dot4_i32_i8), combined once in fp32.
// The group also carries fp32 sums of x over its two 16-element halves (for
// mins and code offsets; NaN or infinite when the group holds a NaN or an
// infinity) and e.
//
// Lane units.  One lane handles one "unit" per step: 64 weights of a K-quant
// super-block (two 32-element groups) or one 32-element block of the classic
// formats.  The prepared x of unit u, group slot k, quad q (16 bytes) lives at
// uint4 index ((u/64 * GPU + k) * 7 + q) * 64 + u%64, so that the 64 lanes of a
// wave reading the same (k, q) of 64 consecutive units touch 1 KB of
// consecutive memory.  Quads: 0,1 = a (elements 0-15, 16-31), 2,3 = b, 4,5 =
// c, 6 = {s, sum x[0:16), sum x[16:32), 0}.
//
// Block layouts follow alpacca/quants.py:50-224 (see aq_formats.h).
#pragma once

#include "aq_formats.h"

namespace aq {

constexpr int XQ = 7;  // quads per prepared group

struct GroupX {
  uint4 q[XQ];
  // the group scale is 2^e; scaled(v) = v * 2^e, exact up to the final rounding
  __device__ int e() const { return (int)q[6].x; }
  __device__ float scaled(float v) const { return __builtin_amdgcn_ldexpf(v, e()); }
  __device__ float sum_lo() const { return __builtin_bit_cast(float, q[6].y); }
  __device__ float sum_hi() const { return __builtin_bit_cast(float, q[6].z); }
  __device__ float sum() const { return sum_lo() + sum_hi(); }
};

__device__ __forceinline__ int dot4(uint32_t w, uint32_t p, int acc) {
  return __builtin_amdgcn_sdot4((int)w, (int)p, acc, false);
}
__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
// Piece-weighted sum of n (4 or 8) code words starting at element 16*h of the
// group, as a float in units of s: A + (254 B + C) / 254^2.
template <int NW>
__device__ __forceinline__ float piece_dot(const uint32_t *w, const GroupX &gx,
                                           int h) {
  int A = 0, B = 0, C = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int qd = h + (i >> 2), wd = i & 3;
    A = dot4(w[i], word(gx.q[0 + qd], wd), A);
    B = dot4(w[i], word(gx.q[2 + qd], wd), B);
    C = dot4(w[i], word(gx.q[4 + qd], wd), C);
  }
  const int bc = __mul24(B, 254) + C;  // |B| < 2^23: one v_mad_i32_i24
  return fmaf((float)bc, 1.0f / 64516.0f, (float)A);
}

// opaque copy: stops the compiler from re-deriving a masked word from its
// source (it would otherwise fold mask+shift into per-byte bitfield extracts)
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// One row of a matrix as buffer resources, one per plane (wave-uniform, in
// scalar registers).  A load at an offset past the row's bytes returns zeros
// without a memory access; a row marked dead has no bytes at all.  The
// decode matvec relies on both: lanes past the last unit and fetches past a
// wave's last row cost no traffic, so every fetch can be issued
// unconditionally.
struct RowSrc {
  __amdgpu_buffer_rsrc_t rs[4];
  uint32_t stride[4];
  uint32_t base[4];  // per-lane byte offset added to every block offset
  template <class T>
  __device__ __forceinline__ T get(int k, uint32_t off) const {
    if constexpr (sizeof(T) == 16)
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(rs[k], (int)off, 0, 0));
    else if constexpr (sizeof(T) == 8)
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(rs[k], (int)off, 0, 0));
    else if constexpr (sizeof(T) == 4)
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(rs[k], (int)off, 0, 0));
    else
      return (T)__builtin_amdgcn_raw_buffer_load_b16(rs[k], (int)off, 0, 0);
  }
  __device__ __forceinline__ uint32_t at(int k, uint32_t b) const {
    return b * stride[k] + base[k];
  }
};

// Each group's piece dot is multiplied by the weight scales first and by the
// group's 2^e last (one ldexp), so no intermediate leaves the normal float
// range unless the true partial product does: x near the top or the bottom of
// the float range costs no precision.  Non-finite x reaches the result through
// the group sums, which are NaN or infinite for such a group (Q8_0 adds
// 0 * sum for that reason).
//
// Every unit type splits its work in two: decode() turns the loaded bytes of
// a lane unit into int8 code words and fp32 scale products (the part that
// depends on the weights only), dotx() applies them to one prepared x.  A
// launch over several x vectors decodes once and calls dotx() per vector;
// dot() = dotx(decode()) is the one-vector form.  Products are formed in the
// same order either way, so the results are the same bits.
//
// Q4_K / Q5_K: d*sc*P0*2^e0 + d*sc'*P1*2^e1 - dmin*(mn*sum0 + mn'*sum1).
struct KQuantDec {
  uint32_t lo[8], hi[8];  // codes of the unit's two groups
  float ds0, ds1;         // d * sc of the two sub-blocks
  float dm0, dm1;         // dmin * mn of the two sub-blocks
};
__device__ __forceinline__ void kquant_scales(const uint4 &h, int ub, KQuantDec &o) {
  uint32_t sc, mn;
  kquant_scale_pair(h.y, h.z, h.w, ub, sc, mn);
  const float d = f16_bits_to_f32(h.x), dm = f16_bits_to_f32(h.x >> 16);
  o.ds0 = d * ubyte(sc, 0);
  o.ds1 = d * ubyte(sc, 1);
  o.dm0 = dm * ubyte(mn, 0);
  o.dm1 = dm * ubyte(mn, 1);
}
__device__ __forceinline__ float kquant_dotx(const KQuantDec &o, const GroupX *gx) {
  const float p0 = piece_dot<8>(o.lo, gx[0], 0), p1 = piece_dot<8>(o.hi, gx[1], 0);
  const float m = fmaf(o.dm0, gx[0].sum(), o.dm1 * gx[1].sum());
  return (gx[0].scaled(o.ds0 * p0) + gx[1].scaled(o.ds1 * p1)) - m;
}

// ---------------------------------------------------------------------------
// Q4_K: unit c in 0..3 = qs[32c, 32c+32): low nibbles are group 2c
// (sub-block 2c), high nibbles group 2c+1; both groups are contiguous runs of
// 32 elements (64c..64c+31, 64c+32..64c+63).
struct UQ4K {
  using F = Q4K;
  static constexpr int UPB = 4, GPU = 2;
  __host__ __device__ static void group_slot(int gi, int &ub, int &k) {
    ub = gi >> 1;
    k = gi & 1;
  }
  struct Raw {
    uint4 q0, q1, h;
  };
  using Dec = KQuantDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int ub) {
    Raw r;
    const uint32_t qs = s.at(0, b) + 32 * ub;
    r.q0 = s.get<uint4>(0, qs);
    r.q1 = s.get<uint4>(0, qs + 16);
    r.h = s.get<uint4>(1, s.at(1, b));
    return r;
  }
  __device__ static Dec decode(const Raw &r, int ub) {
    Dec o;
    kquant_scales(r.h, ub, o);
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w,
                           r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o.lo[i] = opaque(w[i] & 0x0F0F0F0Fu);
      o.hi[i] = opaque((w[i] >> 4) & 0x0F0F0F0Fu);
    }
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return kquant_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

// Q5_K: as Q4_K; the fifth bit of element l of group 2c (2c+1) is bit 2c
// (2c+1) of qh[l].
struct UQ5K {
  using F = Q5K;
  static constexpr int UPB = 4, GPU = 2;
  __host__ __device__ static void group_slot(int gi, int &ub, int &k) {
    ub = gi >> 1;
    k = gi & 1;
  }
  struct Raw {
    uint4 q0, q1, h0, h1, h;
  };
  using Dec = KQuantDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int ub) {
    Raw r;
    const uint32_t qs = s.at(0, b) + 32 * ub;
    r.q0 = s.get<uint4>(0, qs);
    r.q1 = s.get<uint4>(0, qs + 16);
    const uint32_t qh = s.at(1, b);
    r.h0 = s.get<uint4>(1, qh);
    r.h1 = s.get<uint4>(1, qh + 16);
    r.h = s.get<uint4>(2, s.at(2, b));
    return r;
  }
  __device__ static Dec decode(const Raw &r, int ub) {
    Dec o;
    kquant_scales(r.h, ub, o);
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w,
                           r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t b[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w,
                           r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o.lo[i] = (w[i] & 0x0F0F0F0Fu) | (((b[i] >> (2 * ub)) & 0x01010101u) << 4);
      o.hi[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) |
                (((b[i] >> (2 * ub + 1)) & 0x01010101u) << 4);
    }
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return kquant_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

// Q6_K: unit (hf, v), ub = 2hf + v: ql[64hf+32v, +32) and qh[32hf, +32).
// Low nibbles (+ qh bits 2v) are group 4hf+v (elements 128hf+32v+l), high
// nibbles (+ qh bits 4+2v) group 4hf+2+v; each group spans two 16-element
// sub-blocks with int8 scales sc[8hf+2v(+1)] and sc[8hf+4+2v(+1)]; code = q-32.
struct UQ6K {
  using F = Q6K;
  static constexpr int UPB = 4, GPU = 2;
  __host__ __device__ static void group_slot(int gi, int &ub, int &k) {
    const int hf = gi >> 2, r = gi & 3;
    k = r >> 1;
    ub = 2 * hf + (r & 1);
  }
  struct Raw {
    uint4 l0, l1, h0, h1;
    uint2 sc;
    uint32_t d;
  };
  struct Dec {
    uint32_t lo[8], hi[8];
    float d;
    float c00, c01, c10, c11;  // 16-element halves: group 0 (c00, c01), group 1
    float e00, e01, e10, e11;  // -32 * d * c: the code offset's share
  };
  __device__ static Raw load(const RowSrc &s, uint32_t b, int ub) {
    Raw r;
    const int hf = ub >> 1;
    const uint32_t ql = s.at(0, b) + 32 * ub;
    r.l0 = s.get<uint4>(0, ql);
    r.l1 = s.get<uint4>(0, ql + 16);
    const uint32_t qh = s.at(1, b) + 32 * hf;
    r.h0 = s.get<uint4>(1, qh);
    r.h1 = s.get<uint4>(1, qh + 16);
    r.sc = s.get<uint2>(2, s.at(2, b) + 8 * hf);
    r.d = s.get<uint16_t>(3, s.at(3, b));
    return r;
  }
  __device__ static Dec decode(const Raw &r, int ub) {
    Dec o;
    const int v = ub & 1;
    const uint32_t w[8] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w,
                           r.l1.x, r.l1.y, r.l1.z, r.l1.w};
    const uint32_t b[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w,
                           r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o.lo[i] = (w[i] & 0x0F0F0F0Fu) | (((b[i] >> (2 * v)) & 0x03030303u) << 4);
      o.hi[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) |
                (((b[i] >> (4 + 2 * v)) & 0x03030303u) << 4);
    }
    const int sh = 16 * v;
    o.c00 = sbyte(r.sc.x >> sh, 0);
    o.c01 = sbyte(r.sc.x >> sh, 1);
    o.c10 = sbyte(r.sc.y >> sh, 0);
    o.c11 = sbyte(r.sc.y >> sh, 1);
    o.d = f16_bits_to_f32(r.d);
    const float dd = -32.f * o.d;
    o.e00 = dd * o.c00;
    o.e01 = dd * o.c01;
    o.e10 = dd * o.c10;
    o.e11 = dd * o.c11;
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) {
    const float p0 = fmaf(o.c00, piece_dot<4>(o.lo, gx[0], 0), o.c01 * piece_dot<4>(o.lo + 4, gx[0], 1));
    const float p1 = fmaf(o.c10, piece_dot<4>(o.hi, gx[1], 0), o.c11 * piece_dot<4>(o.hi + 4, gx[1], 1));
    const float m = fmaf(o.e00, gx[0].sum_lo(), o.e01 * gx[0].sum_hi()) +
                    fmaf(o.e10, gx[1].sum_lo(), o.e11 * gx[1].sum_hi());
    return (gx[0].scaled(o.d * p0) + gx[1].scaled(o.d * p1)) + m;
  }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

// Q8_0: unit = block = group; codes are the int8 qs themselves.
struct UQ80 {
  using F = Q80;
  static constexpr int UPB = 1, GPU = 1;
  __host__ __device__ static void group_slot(int, int &ub, int &k) {
    ub = 0;
    k = 0;
  }
  struct Raw {
    uint4 q0, q1;
    uint32_t d;
  };
  struct Dec {
    uint32_t w[8];
    float d;
  };
  __device__ static Raw load(const RowSrc &s, uint32_t b, int) {
    Raw r;
    const uint32_t qs = s.at(0, b);
    r.q0 = s.get<uint4>(0, qs);
    r.q1 = s.get<uint4>(0, qs + 16);
    r.d = s.get<uint16_t>(1, s.at(1, b));
    return r;
  }
  __device__ static Dec decode(const Raw &r, int) {
    return Dec{{r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w},
               f16_bits_to_f32(r.d)};
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) {
    return fmaf(0.f, gx[0].sum(), gx[0].scaled(o.d * piece_dot<8>(o.w, gx[0], 0)));
  }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

// classic 4/5-bit formats: codes of elements 0-15 (low nibbles) then 16-31
__device__ __forceinline__ void nibble_codes(const uint4 &q, uint32_t *c) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = opaque(w[i] & 0x0F0F0F0Fu);
    c[4 + i] = opaque((w[i] >> 4) & 0x0F0F0F0Fu);
  }
}
__device__ __forceinline__ void add_qh_bits(uint32_t qh, uint32_t *c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] |= spread4_to_bit4((qh >> (4 * i)) & 15u);
    c[4 + i] |= spread4_to_bit4((qh >> (16 + 4 * i)) & 15u);
  }
}

// decoded classic block: codes, scale d and the per-element offset m
// (-8 d or -16 d for Q4_0 / Q5_0, the stored m for Q4_1 / Q5_1)
struct ClassicDec {
  uint32_t c[8];
  float d, m;
};
__device__ __forceinline__ float classic_dotx(const ClassicDec &o, const GroupX *gx) {
  return fmaf(o.m, gx[0].sum(), gx[0].scaled(o.d * piece_dot<8>(o.c, gx[0], 0)));
}

struct UQ40 {
  using F = Q40;
  static constexpr int UPB = 1, GPU = 1;
  __host__ __device__ static void group_slot(int, int &ub, int &k) {
    ub = 0;
    k = 0;
  }
  struct Raw {
    uint4 q;
    uint32_t d;
  };
  using Dec = ClassicDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int) {
    return Raw{s.get<uint4>(0, s.at(0, b)), s.get<uint16_t>(1, s.at(1, b))};
  }
  __device__ static Dec decode(const Raw &r, int) {
    Dec o;
    nibble_codes(r.q, o.c);
    o.d = f16_bits_to_f32(r.d);
    o.m = -8.f * o.d;
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return classic_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

struct UQ41 {
  using F = Q41;
  static constexpr int UPB = 1, GPU = 1;
  __host__ __device__ static void group_slot(int, int &ub, int &k) {
    ub = 0;
    k = 0;
  }
  struct Raw {
    uint4 q;
    uint32_t dm;
  };
  using Dec = ClassicDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int) {
    return Raw{s.get<uint4>(0, s.at(0, b)), s.get<uint32_t>(1, s.at(1, b))};
  }
  __device__ static Dec decode(const Raw &r, int) {
    Dec o;
    nibble_codes(r.q, o.c);
    o.d = f16_bits_to_f32(r.dm);
    o.m = f16_bits_to_f32(r.dm >> 16);
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return classic_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

struct UQ50 {
  using F = Q50;
  static constexpr int UPB = 1, GPU = 1;
  __host__ __device__ static void group_slot(int, int &ub, int &k) {
    ub = 0;
    k = 0;
  }
  struct Raw {
    uint4 q;
    uint32_t qh, d;
  };
  using Dec = ClassicDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int) {
    return Raw{s.get<uint4>(0, s.at(0, b)), s.get<uint32_t>(1, s.at(1, b)),
               s.get<uint16_t>(2, s.at(2, b))};
  }
  __device__ static Dec decode(const Raw &r, int) {
    Dec o;
    nibble_codes(r.q, o.c);
    add_qh_bits(r.qh, o.c);
    o.d = f16_bits_to_f32(r.d);
    o.m = -16.f * o.d;
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return classic_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

struct UQ51 {
  using F = Q51;
  static constexpr int UPB = 1, GPU = 1;
  __host__ __device__ static void group_slot(int, int &ub, int &k) {
    ub = 0;
    k = 0;
  }
  struct Raw {
    uint4 q;
    uint32_t qh, dm;
  };
  using Dec = ClassicDec;
  __device__ static Raw load(const RowSrc &s, uint32_t b, int) {
    return Raw{s.get<uint4>(0, s.at(0, b)), s.get<uint32_t>(1, s.at(1, b)),
               s.get<uint32_t>(2, s.at(2, b))};
  }
  __device__ static Dec decode(const Raw &r, int) {
    Dec o;
    nibble_codes(r.q, o.c);
    add_qh_bits(r.qh, o.c);
    o.d = f16_bits_to_f32(r.dm);
    o.m = f16_bits_to_f32(r.dm >> 16);
    return o;
  }
  __device__ static float dotx(const Dec &o, const GroupX *gx) { return classic_dotx(o, gx); }
  __device__ static float dot(const Raw &r, int ub, const GroupX *gx) {
    return dotx(decode(r, ub), gx);
  }
};

// bytes of the prepared x of one row (all units, padded to whole steps)
template <class U>
__host__ __device__ inline size_t xprep_bytes(int64_t nb_row) {
  const int64_t units = nb_row * U::UPB;
  const int64_t steps = (units + 63) / 64;
  return (size_t)steps * 64 * U::GPU * XQ * 16;
}

}  // namespace aq
