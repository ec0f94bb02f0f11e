// aq_formats.h - GGUF block formats as the gfx950 kernels see them.
//
// A block of each format is cut into "chunks": the unit one lane handles in
// one step.  A chunk is 16 bytes of quant payload (32 weights for the 4/5/6-bit
// formats, 16 for Q8_0) plus whatever scale/high-bit bytes those weights need.
// Each format struct below gives
//   xoff(j, t)   element offset inside the block of slot t of chunk j; slots
//                [0,16) and [16,32) are each a run of 16 consecutive elements
//   load()       the chunk's bytes, straight from HBM into registers
//   decode()     the chunk's 32 (16) values in slot order, bit-identical to the
//                reference decoder: code * d_eff (+ m_eff) in fp32, where
//                d_eff/m_eff are formed exactly from the fp16 fields
//                (alpacca/quants.py:338-504)
//   dot()        sum_t value[t] * xv[t] for the matvec, given xs0/xs1 = the
//                sums of xv over slots [0,16) / [16,32)
//
// Field planes.  A matrix lives in HBM as up to four planes; plane k holds one
// field of every block, `stride[k]` bytes per block.  With the SPLIT layout
// each plane is a dense array of that field (all 16-B aligned); with the RAW
// layout every plane points into the verbatim GGUF bytes at the field's
// offset with stride = block bytes (used only where that keeps 16-B
// alignment: Q4_K and Q5_K).  Field offsets follow the block layouts of
// alpacca/quants.py:50-224.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aq {

// Global-memory (address space 1) views of device pointers.  Loads and stores
// through them compile to global_* instructions.  Through a generic pointer
// that the compiler cannot trace to a kernel argument they become flat_*
// instructions, and while a flat access is outstanding the compiler makes the
// next use of any loaded register wait for every outstanding vector load
// (vmcnt(0)): one y store per row would drain a kernel's whole load pipeline.
template <class T>
using global_ptr = __attribute__((address_space(1))) T *;
template <class T>
__device__ __forceinline__ global_ptr<T> as_global(T *p) {
  return (global_ptr<T>)p;
}
template <class T>
__device__ __forceinline__ global_ptr<const T> as_global(const T *p) {
  return (global_ptr<const T>)p;
}

// buffer resource word 3 for gfx9-family raw (unswizzled, untyped) buffers.
// A load past a resource's byte count returns zeros without touching memory,
// so a resource of zero bytes makes an unconditional load a no-op.
constexpr int kRsrcWord3 = 0x00020000;

struct Planes {
  const uint8_t *p[4];
  int64_t stride[4];
};

struct FieldSpec {
  int raw_off;  // offset of the field inside the GGUF block
  int bytes;    // bytes of the field per block
};

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}
// byte k of v as float (v_cvt_f32_ubyteN)
__device__ __forceinline__ float ubyte(uint32_t v, int k) {
  return (float)((v >> (8 * k)) & 0xFFu);
}
// signed byte k of v as float
__device__ __forceinline__ float sbyte(uint32_t v, int k) {
  return (float)((int32_t)(v << (24 - 8 * k)) >> 24);
}

template <class T>
__device__ __forceinline__ T ld(const uint8_t *p) {
  return *reinterpret_cast<const T *>(p);
}

// 6-bit scale/min pairs of Q4_K / Q5_K for sub-blocks 2c and 2c+1
// (alpacca/quants.py:127-133).  s0/s1/s2 = scale bytes 0-3 / 4-7 / 8-11.
// Returns sc = sc[2c] | sc[2c+1] << 8 and mn likewise.
__device__ __forceinline__ void kquant_scale_pair(uint32_t s0, uint32_t s1,
                                                  uint32_t s2, int c,
                                                  uint32_t &sc, uint32_t &mn) {
  const int sh = 16 * (c & 1);
  if (c < 2) {
    sc = (s0 >> sh) & 0x3F3Fu;
    mn = (s1 >> sh) & 0x3F3Fu;
  } else {
    const uint32_t lo4 = s2 >> sh;  // bytes 8+2c', 9+2c'
    sc = (lo4 & 0x0F0Fu) | (((s0 >> sh) >> 2) & 0x3030u);
    mn = ((lo4 >> 4) & 0x0F0Fu) | (((s1 >> sh) >> 2) & 0x3030u);
  }
}

// spread the low 4 bits of b to bit 4 of each byte (b0 -> bit 4, b1 -> 12...)
__device__ __forceinline__ uint32_t spread4_to_bit4(uint32_t b) {
  return ((b * 0x00204081u) & 0x01010101u) << 4;
}

// ---------------------------------------------------------------------------
// Q4_K: 144 B / 256 = d, dmin (fp16), 12 B packed 6-bit scales/mins, 128 B qs.
// Chunk j = qs[16j, 16j+16): c = j/2, h = j%2; low nibbles are elements
// 64c+16h+t of sub-block 2c, high nibbles 64c+32+16h+t of sub-block 2c+1
// (quants.py:136-161, 417-427).
struct Q4K {
  static constexpr int BE = 256, BB = 144, SUB = 32, CPB = 8, ELEMS = 32;
  static constexpr int NPL = 2;
  static constexpr bool RAW_OK = true;
  static constexpr FieldSpec FIELDS[NPL] = {{16, 128}, {0, 16}};
  __host__ __device__ static int xoff(int j, int t) {
    return 64 * (j >> 1) + 16 * (j & 1) + (t & 15) + ((t >> 4) << 5);
  }
  struct Raw {
    uint4 q, h;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0] + 16 * j);
    r.h = ld<uint4>(P.p[1] + blk * P.stride[1]);
    return r;
  }
  __device__ static void decode(const Raw &r, int j, float *v) {
    uint32_t sc, mn;
    kquant_scale_pair(r.h.y, r.h.z, r.h.w, j >> 1, sc, mn);
    const float d = f16_bits_to_f32(r.h.x), dm = f16_bits_to_f32(r.h.x >> 16);
    const float d0 = d * ubyte(sc, 0), d1 = d * ubyte(sc, 1);
    const float m0 = -(dm * ubyte(mn, 0)), m1 = -(dm * ubyte(mn, 1));
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b = (w[i] >> (8 * k)) & 0xFFu;
        v[4 * i + k] = fmaf((float)(b & 15u), d0, m0);
        v[16 + 4 * i + k] = fmaf((float)(b >> 4), d1, m1);
      }
    }
  }
  __device__ static float dot(const Raw &r, int j, const float *xv, float xs0,
                              float xs1) {
    uint32_t sc, mn;
    kquant_scale_pair(r.h.y, r.h.z, r.h.w, j >> 1, sc, mn);
    const float d = f16_bits_to_f32(r.h.x), dm = f16_bits_to_f32(r.h.x >> 16);
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t l = w[i] & 0x0F0F0F0Fu;
      const uint32_t h = w[i] & 0xF0F0F0F0u;  // 16 * high nibble per byte
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lo = fmaf(ubyte(l, k), xv[4 * i + k], lo);
        hi = fmaf(ubyte(h, k), xv[16 + 4 * i + k], hi);
      }
    }
    const float s0 = d * ubyte(sc, 0), s1 = d * ubyte(sc, 1) * 0.0625f;
    return fmaf(s0, lo, s1 * hi) -
           dm * fmaf(ubyte(mn, 0), xs0, ubyte(mn, 1) * xs1);
  }
};

// ---------------------------------------------------------------------------
// Q5_K: 176 B / 256 = d, dmin, 12 B scales, 32 B qh, 128 B qs.  As Q4_K with
// bit 2c (low nibbles) / 2c+1 (high nibbles) of qh[16h+t] as the fifth bit
// (quants.py:164-193, 430-444).
struct Q5K {
  static constexpr int BE = 256, BB = 176, SUB = 32, CPB = 8, ELEMS = 32;
  static constexpr int NPL = 3;
  static constexpr bool RAW_OK = true;
  static constexpr FieldSpec FIELDS[NPL] = {{48, 128}, {16, 32}, {0, 16}};
  __host__ __device__ static int xoff(int j, int t) { return Q4K::xoff(j, t); }
  struct Raw {
    uint4 q, qh, h;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0] + 16 * j);
    r.qh = ld<uint4>(P.p[1] + blk * P.stride[1] + 16 * (j & 1));
    r.h = ld<uint4>(P.p[2] + blk * P.stride[2]);
    return r;
  }
  // 5-bit codes of the chunk: lo[i] / hi[i] hold 4 codes each (one per byte)
  __device__ static void codes(const Raw &r, int j, uint32_t *lo,
                               uint32_t *hi) {
    const int c = j >> 1;
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t b[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = (w[i] & 0x0F0F0F0Fu) | (((b[i] >> (2 * c)) & 0x01010101u) << 4);
      hi[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) |
              (((b[i] >> (2 * c + 1)) & 0x01010101u) << 4);
    }
  }
  __device__ static void decode(const Raw &r, int j, float *v) {
    uint32_t sc, mn;
    kquant_scale_pair(r.h.y, r.h.z, r.h.w, j >> 1, sc, mn);
    const float d = f16_bits_to_f32(r.h.x), dm = f16_bits_to_f32(r.h.x >> 16);
    const float d0 = d * ubyte(sc, 0), d1 = d * ubyte(sc, 1);
    const float m0 = -(dm * ubyte(mn, 0)), m1 = -(dm * ubyte(mn, 1));
    uint32_t lo[4], hi[4];
    codes(r, j, lo, hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[4 * i + k] = fmaf(ubyte(lo[i], k), d0, m0);
        v[16 + 4 * i + k] = fmaf(ubyte(hi[i], k), d1, m1);
      }
    }
  }
  __device__ static float dot(const Raw &r, int j, const float *xv, float xs0,
                              float xs1) {
    uint32_t sc, mn;
    kquant_scale_pair(r.h.y, r.h.z, r.h.w, j >> 1, sc, mn);
    const float d = f16_bits_to_f32(r.h.x), dm = f16_bits_to_f32(r.h.x >> 16);
    uint32_t lo[4], hi[4];
    codes(r, j, lo, hi);
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a = fmaf(ubyte(lo[i], k), xv[4 * i + k], a);
        b = fmaf(ubyte(hi[i], k), xv[16 + 4 * i + k], b);
      }
    }
    return d * fmaf(ubyte(sc, 0), a, ubyte(sc, 1) * b) -
           dm * fmaf(ubyte(mn, 0), xs0, ubyte(mn, 1) * xs1);
  }
};

// ---------------------------------------------------------------------------
// Q6_K: 210 B / 256 = ql[128], qh[64], int8 scales[16], d (fp16).
// Chunk j = ql[16j, 16j+16): hf = j/4, k = j%4, u = k/2, kk = k%2.  Low
// nibbles are elements 128hf+32u+16kk+t (sub-block 8hf+k), high nibbles
// 128hf+64+32u+16kk+t (sub-block 8hf+4+k); the two high bits come from
// qh[32hf+16kk+t] at shift 2u (low) and 4+2u (high); code = q - 32
// (quants.py:196-224, 447-466).  Only the SPLIT layout: 210-B blocks break
// 16-B alignment.
struct Q6K {
  static constexpr int BE = 256, BB = 210, SUB = 16, CPB = 8, ELEMS = 32;
  static constexpr int NPL = 4;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {
      {0, 128}, {128, 64}, {192, 16}, {208, 2}};
  __host__ __device__ static int xoff(int j, int t) {
    const int hf = j >> 2, k = j & 3;
    return 128 * hf + 32 * (k >> 1) + 16 * (k & 1) + (t & 15) + ((t >> 4) << 6);
  }
  struct Raw {
    uint4 ql, qh;
    uint2 sc;
    uint32_t d;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    Raw r;
    const int hf = j >> 2;
    r.ql = ld<uint4>(P.p[0] + blk * P.stride[0] + 16 * j);
    r.qh = ld<uint4>(P.p[1] + blk * P.stride[1] + 32 * hf + 16 * (j & 1));
    r.sc = ld<uint2>(P.p[2] + blk * P.stride[2] + 8 * hf);
    r.d = ld<uint16_t>(P.p[3] + blk * P.stride[3]);
    return r;
  }
  // unsigned 6-bit codes (q, before the -32)
  __device__ static void codes(const Raw &r, int j, uint32_t *lo,
                               uint32_t *hi) {
    const int u = (j >> 1) & 1;
    const uint32_t w[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
    const uint32_t b[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = (w[i] & 0x0F0F0F0Fu) | (((b[i] >> (2 * u)) & 0x03030303u) << 4);
      hi[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) |
              (((b[i] >> (4 + 2 * u)) & 0x03030303u) << 4);
    }
  }
  __device__ static void decode(const Raw &r, int j, float *v) {
    const int k = j & 3;
    const float d = f16_bits_to_f32(r.d);
    const float d0 = d * sbyte(r.sc.x, k), d1 = d * sbyte(r.sc.y, k);
    uint32_t lo[4], hi[4];
    codes(r, j, lo, hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        v[4 * i + kk] = (float)((int)((lo[i] >> (8 * kk)) & 0xFFu) - 32) * d0;
        v[16 + 4 * i + kk] =
            (float)((int)((hi[i] >> (8 * kk)) & 0xFFu) - 32) * d1;
      }
    }
  }
  __device__ static float dot(const Raw &r, int j, const float *xv, float xs0,
                              float xs1) {
    const int k = j & 3;
    const float d = f16_bits_to_f32(r.d);
    uint32_t lo[4], hi[4];
    codes(r, j, lo, hi);
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        a = fmaf(ubyte(lo[i], kk), xv[4 * i + kk], a);
        b = fmaf(ubyte(hi[i], kk), xv[16 + 4 * i + kk], b);
      }
    }
    return d * fmaf(sbyte(r.sc.x, k), fmaf(-32.f, xs0, a),
                    sbyte(r.sc.y, k) * fmaf(-32.f, xs1, b));
  }
};

// ---------------------------------------------------------------------------
// Q8_0: 34 B / 32 = d (fp16), int8 qs[32] (quants.py:50-60, 346-349).
// Chunk j = qs[16j, 16j+16) = elements 16j+t.
struct Q80 {
  static constexpr int BE = 32, BB = 34, SUB = 32, CPB = 2, ELEMS = 16;
  static constexpr int NPL = 2;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {{2, 32}, {0, 2}};
  __host__ __device__ static int xoff(int j, int t) { return 16 * j + t; }
  struct Raw {
    uint4 q;
    uint32_t d;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0] + 16 * j);
    r.d = ld<uint16_t>(P.p[1] + blk * P.stride[1]);
    return r;
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const float d = f16_bits_to_f32(r.d);
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * i + k] = sbyte(w[i], k) * d;
  }
  __device__ static float dot(const Raw &r, int, const float *xv, float,
                              float) {
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a = fmaf(sbyte(w[i], k), xv[4 * i + k], a);
        b = fmaf(sbyte(w[i + 1], k), xv[4 * i + 4 + k], b);
      }
    }
    return f16_bits_to_f32(r.d) * (a + b);
  }
};

// ---------------------------------------------------------------------------
// The classic 32-element formats: one chunk per block, slot t < 16 is element
// t (low nibble of qs[t]), slot 16+t is element 16+t (high nibble).
__host__ __device__ inline int xoff32(int, int t) { return t; }

// sum over the 16 low / high nibbles of a 16-byte qs vector with xv
__device__ __forceinline__ void nibble_dots(const uint4 &q, const float *xv,
                                            float &lo, float &hi) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  lo = 0.f;
  hi = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t l = w[i] & 0x0F0F0F0Fu, h = w[i] & 0xF0F0F0F0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo = fmaf(ubyte(l, k), xv[4 * i + k], lo);
      hi = fmaf(ubyte(h, k), xv[16 + 4 * i + k], hi);
    }
  }
  hi *= 0.0625f;
}

// Q4_0: 18 B / 32 = d, qs[16]; code = nibble - 8 (quants.py:63-74, 352-359).
struct Q40 {
  static constexpr int BE = 32, BB = 18, SUB = 32, CPB = 1, ELEMS = 32;
  static constexpr int NPL = 2;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {{2, 16}, {0, 2}};
  __host__ __device__ static int xoff(int j, int t) { return xoff32(j, t); }
  struct Raw {
    uint4 q;
    uint32_t d;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0]);
    r.d = ld<uint16_t>(P.p[1] + blk * P.stride[1]);
    return r;
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const float d = f16_bits_to_f32(r.d);
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b = (w[i] >> (8 * k)) & 0xFFu;
        v[4 * i + k] = (float)((int)(b & 15u) - 8) * d;
        v[16 + 4 * i + k] = (float)((int)(b >> 4) - 8) * d;
      }
  }
  __device__ static float dot(const Raw &r, int, const float *xv, float xs0,
                              float xs1) {
    float lo, hi;
    nibble_dots(r.q, xv, lo, hi);
    return f16_bits_to_f32(r.d) * ((lo + hi) - 8.f * (xs0 + xs1));
  }
};

// Q4_1: 20 B / 32 = d, m, qs[16]; value = d * nibble + m (quants.py:77-89).
struct Q41 {
  static constexpr int BE = 32, BB = 20, SUB = 32, CPB = 1, ELEMS = 32;
  static constexpr int NPL = 2;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {{4, 16}, {0, 4}};
  __host__ __device__ static int xoff(int j, int t) { return xoff32(j, t); }
  struct Raw {
    uint4 q;
    uint32_t dm;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0]);
    r.dm = ld<uint32_t>(P.p[1] + blk * P.stride[1]);
    return r;
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const float d = f16_bits_to_f32(r.dm), m = f16_bits_to_f32(r.dm >> 16);
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b = (w[i] >> (8 * k)) & 0xFFu;
        v[4 * i + k] = fmaf((float)(b & 15u), d, m);
        v[16 + 4 * i + k] = fmaf((float)(b >> 4), d, m);
      }
  }
  __device__ static float dot(const Raw &r, int, const float *xv, float xs0,
                              float xs1) {
    float lo, hi;
    nibble_dots(r.q, xv, lo, hi);
    return fmaf(f16_bits_to_f32(r.dm), lo + hi,
                f16_bits_to_f32(r.dm >> 16) * (xs0 + xs1));
  }
};

// 5-bit codes of Q5_0/Q5_1: bit t of the u32 qh is the fifth bit of element t
// (quants.py:92-124, 372-399).
__device__ __forceinline__ void q5_codes(const uint4 &q, uint32_t qh,
                                         uint32_t *lo, uint32_t *hi) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo[i] = (w[i] & 0x0F0F0F0Fu) | spread4_to_bit4((qh >> (4 * i)) & 15u);
    hi[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) |
            spread4_to_bit4((qh >> (16 + 4 * i)) & 15u);
  }
}
__device__ __forceinline__ void code_dots(const uint32_t *lo,
                                          const uint32_t *hi, const float *xv,
                                          float &a, float &b) {
  a = 0.f;
  b = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a = fmaf(ubyte(lo[i], k), xv[4 * i + k], a);
      b = fmaf(ubyte(hi[i], k), xv[16 + 4 * i + k], b);
    }
}

// Q5_0: 22 B / 32 = d, u32 qh, qs[16]; code = q - 16.
struct Q50 {
  static constexpr int BE = 32, BB = 22, SUB = 32, CPB = 1, ELEMS = 32;
  static constexpr int NPL = 3;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {{6, 16}, {2, 4}, {0, 2}};
  __host__ __device__ static int xoff(int j, int t) { return xoff32(j, t); }
  struct Raw {
    uint4 q;
    uint32_t qh, d;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0]);
    r.qh = ld<uint32_t>(P.p[1] + blk * P.stride[1]);
    r.d = ld<uint16_t>(P.p[2] + blk * P.stride[2]);
    return r;
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const float d = f16_bits_to_f32(r.d);
    uint32_t lo[4], hi[4];
    q5_codes(r.q, r.qh, lo, hi);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[4 * i + k] = (float)((int)((lo[i] >> (8 * k)) & 0xFFu) - 16) * d;
        v[16 + 4 * i + k] = (float)((int)((hi[i] >> (8 * k)) & 0xFFu) - 16) * d;
      }
  }
  __device__ static float dot(const Raw &r, int, const float *xv, float xs0,
                              float xs1) {
    uint32_t lo[4], hi[4];
    q5_codes(r.q, r.qh, lo, hi);
    float a, b;
    code_dots(lo, hi, xv, a, b);
    return f16_bits_to_f32(r.d) * ((a + b) - 16.f * (xs0 + xs1));
  }
};

// Q5_1: 24 B / 32 = d, m, u32 qh, qs[16]; value = d * q + m.
struct Q51 {
  static constexpr int BE = 32, BB = 24, SUB = 32, CPB = 1, ELEMS = 32;
  static constexpr int NPL = 3;
  static constexpr bool RAW_OK = false;
  static constexpr FieldSpec FIELDS[NPL] = {{8, 16}, {4, 4}, {0, 4}};
  __host__ __device__ static int xoff(int j, int t) { return xoff32(j, t); }
  struct Raw {
    uint4 q;
    uint32_t qh, dm;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int) {
    Raw r;
    r.q = ld<uint4>(P.p[0] + blk * P.stride[0]);
    r.qh = ld<uint32_t>(P.p[1] + blk * P.stride[1]);
    r.dm = ld<uint32_t>(P.p[2] + blk * P.stride[2]);
    return r;
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const float d = f16_bits_to_f32(r.dm), m = f16_bits_to_f32(r.dm >> 16);
    uint32_t lo[4], hi[4];
    q5_codes(r.q, r.qh, lo, hi);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[4 * i + k] = fmaf(ubyte(lo[i], k), d, m);
        v[16 + 4 * i + k] = fmaf(ubyte(hi[i], k), d, m);
      }
  }
  __device__ static float dot(const Raw &r, int, const float *xv, float xs0,
                              float xs1) {
    uint32_t lo[4], hi[4];
    q5_codes(r.q, r.qh, lo, hi);
    float a, b;
    code_dots(lo, hi, xv, a, b);
    return fmaf(f16_bits_to_f32(r.dm), a + b,
                f16_bits_to_f32(r.dm >> 16) * (xs0 + xs1));
  }
};

// ---------------------------------------------------------------------------
// Dense values (F32, F16, BF16): a "block" is 32 values along K, a chunk 8
// of them (16 B for the 2-byte types, 32 B for F32); decode is the exact
// conversion to fp32 (quants.py:517-523) and dot an fp32 FMA chain.
__host__ __device__ inline int xoff8(int j, int t) { return 8 * j + t; }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, (b & 0xFFFFu) << 16);
}
__device__ __forceinline__ float dot8(const float *v, const float *xv) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int t = 0; t < 8; t += 2) {
    a = fmaf(v[t], xv[t], a);
    b = fmaf(v[t + 1], xv[t + 1], b);
  }
  return a + b;
}

template <bool BF>
struct Half16 {  // F16 (BF = false) and BF16 (BF = true)
  static constexpr int BE = 32, BB = 64, SUB = 32, CPB = 4, ELEMS = 8;
  static constexpr int NPL = 1;
  static constexpr bool RAW_OK = true;
  static constexpr FieldSpec FIELDS[NPL] = {{0, 64}};
  __host__ __device__ static int xoff(int j, int t) { return xoff8(j, t); }
  struct Raw {
    uint4 q;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    return Raw{ld<uint4>(P.p[0] + blk * P.stride[0] + 16 * j)};
  }
  __device__ static float cvt(uint32_t h) {
    return BF ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = cvt(w[i]);
      v[2 * i + 1] = cvt(w[i] >> 16);
    }
  }
  __device__ static float dot(const Raw &r, int j, const float *xv, float, float) {
    float v[8];
    decode(r, j, v);
    return dot8(v, xv);
  }
};
using F16D = Half16<false>;
using BF16D = Half16<true>;

struct F32D {
  static constexpr int BE = 32, BB = 128, SUB = 32, CPB = 4, ELEMS = 8;
  static constexpr int NPL = 1;
  static constexpr bool RAW_OK = true;
  static constexpr FieldSpec FIELDS[NPL] = {{0, 128}};
  __host__ __device__ static int xoff(int j, int t) { return xoff8(j, t); }
  struct Raw {
    uint4 a, b;
  };
  __device__ static Raw load(const Planes &P, int64_t blk, int j) {
    const uint8_t *p = P.p[0] + blk * P.stride[0] + 32 * j;
    return Raw{ld<uint4>(p), ld<uint4>(p + 16)};
  }
  __device__ static void decode(const Raw &r, int, float *v) {
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(float, w[i]);
  }
  __device__ static float dot(const Raw &r, int j, const float *xv, float, float) {
    float v[8];
    decode(r, j, v);
    return dot8(v, xv);
  }
};

}  // namespace aq
