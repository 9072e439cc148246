// Device helpers shared by the gfx950 kernels of the KV compression engine.
//
// Numerics follow KVServe's modular torch pipeline, where every elementwise op is
// computed in fp32 and rounded to bf16 (round-to-nearest-even) before the next op:
//   transform  y   = bf16( FWHT_fp32(x * s) * (1/sqrt(D)) )  hadamard_func.py:161-197
//   scale      sc  = bf16( max(bf16(mx - mn), 1e-5) / (L - 1) ) quantizer_func.py:56
//   quantize   q   = bf16( bf16(y - mn) / sc )                   quantizer_func.py:60-62
//              sym = clamp(rint(q), 0, L)                        quantizer_func.py:65
//   dequantize x~  = bf16( bf16(sym * sc) + mn )                 quantizer_func.py:108-112
// The FWHT runs radix-2 in natural (Sylvester) order, one stage per index bit,
// lowest bit first, all in fp32, with a single bf16 rounding after the scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvmi {

// ---------------------------------------------------------------- global memory
// The buffers of a job are pointers read out of a descriptor in device memory, so
// the compiler cannot prove they are global and would emit flat_* instructions.  A
// flat load also counts against the LDS wait counter: every LDS wait would then
// drain the outstanding HBM loads.  All HBM accesses of the paged kernels go
// through these address-space-1 accessors (global_* instructions) instead.
#define KVMI_GLOBAL __attribute__((address_space(1)))
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ T gld(const T* p) {
  return *(const KVMI_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ void gst(T* p, T v) {
  *(KVMI_GLOBAL T*)p = v;
}
// Read-only data through the constant address space: a wave-uniform address becomes
// a scalar load (counted by lgkmcnt, so waiting for it does not drain the streaming
// vector loads).  Only for buffers no kernel of the launch writes.
template <class T>
__device__ __forceinline__ T cld(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}
__device__ __forceinline__ uint4 gld(const uint4* p) {
  const u32x4v v = *(const KVMI_GLOBAL u32x4v*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void gst(uint4* p, uint4 v) {
  const u32x4v w = {v.x, v.y, v.z, v.w};
  *(KVMI_GLOBAL u32x4v*)p = w;
}
// Streaming store (global_store ... nt): output written once and not read again by
// this kernel; it is not allocated in the caches on the way, which measured ~5 %
// more bandwidth for a read-mostly kernel's write stream on gfx950.
__device__ __forceinline__ void gst_stream(uint4* p, uint4 v) {
  const u32x4v w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, (KVMI_GLOBAL u32x4v*)p);
}
__device__ __forceinline__ uint2 gld(const uint2* p) {
  const u32x2v v = *(const KVMI_GLOBAL u32x2v*)p;
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ void gst(uint2* p, uint2 v) {
  const u32x2v w = {v.x, v.y};
  *(KVMI_GLOBAL u32x2v*)p = w;
}

// ---------------------------------------------------------------- bf16 <-> fp32
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16 bits, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  __bf16 b = (__bf16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// Value of x rounded to bf16, returned as fp32.
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16_bits(x)); }

// Order-preserving map fp32 -> uint32 (for integer atomics on min / max).
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// bf16 value of 1e-5, the clamp_min floor of the scale (quantizer_func.py:56).
__device__ __forceinline__ float scale_floor() { return round_bf16(1e-5f); }

// Scale and reciprocal of a min/max pair, both already bf16 values.
__device__ __forceinline__ float quant_scale(float mn, float mx, int levels) {
  float d = round_bf16(mx - mn);
  float fl = scale_floor();
  d = d < fl ? fl : d;  // clamp_(min=1e-5) on a bf16 tensor
  return round_bf16(d / (float)(levels - 1));
}

// One quantized symbol of a bf16 value y (held as fp32) given bf16 mn and
// rcp = 1/sc.  bf16(t * rcp) equals bf16(t / sc) for bf16 t and sc: the exact
// quotient of two 8-bit significands lies at least 2^-17 (relative) away from
// every bf16 rounding midpoint, while t * rcp is within 2^-22 of it.
__device__ __forceinline__ float quant_value(float y, float mn, float rcp, float lv) {
  float t = round_bf16(y - mn);
  float q = round_bf16(t * rcp);
  float r = __builtin_rintf(q);
  return r < lv ? r : lv;  // q >= 0 always (y >= mn), so only the upper clamp acts
}

__device__ __forceinline__ float dequant_value(float sym, float mn, float sc) {
  return round_bf16(round_bf16(sym * sc) + mn);
}

// ---------------------------------------------------------------- FWHT
// Each row of D elements is held by a quad of 4 lanes: lane q of the quad owns the
// contiguous elements [q*E, (q+1)*E), E = D/4.  The low log2(E) index bits are
// transformed in registers; the two top bits cross lanes through DPP quad_perm.
template <int E>
__device__ __forceinline__ void fwht_in_lane(float (&v)[E]) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if (!(i & h)) {
        float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Butterfly with the quad partner: the lane whose quad bit is 0 holds the lower
// element a and gets a + b; the other holds b and gets a - b = partner - own.
template <int E>
__device__ __forceinline__ void fwht_cross_quad(float (&v)[E], int q) {
  const float s1 = (q & 1) ? -1.0f : 1.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) v[i] = __builtin_fmaf(v[i], s1, dpp_f<0xB1>(v[i]));  // quad_perm [1,0,3,2]
  const float s2 = (q & 2) ? -1.0f : 1.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) v[i] = __builtin_fmaf(v[i], s2, dpp_f<0x4E>(v[i]));  // quad_perm [2,3,0,1]
}

template <int E>
__device__ __forceinline__ void fwht_row(float (&v)[E], int q) {
  fwht_in_lane<E>(v);
  fwht_cross_quad<E>(v, q);
}

// Value of lane (lane ^ J): DPP for J = 1, 2 (quad_perm) and 8 (row_ror:8 within a
// 16-lane row), ds_swizzle bit masks for 4 and 16, bpermute beyond.
template <int J>
__device__ __forceinline__ float lane_xor(float x) {
  if constexpr (J == 1) {
    return dpp_f<0xB1>(x);
  } else if constexpr (J == 2) {
    return dpp_f<0x4E>(x);
  } else if constexpr (J == 8) {
    return dpp_f<0x128>(x);
  } else if constexpr (J == 4 || J == 16) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1F | (J << 10)));
  } else {
    return __shfl_xor(x, J, 64);
  }
}

// Min / max of a value across the 4 lanes of a quad.
__device__ __forceinline__ float quad_min(float x) {
  x = fminf(x, dpp_f<0xB1>(x));
  return fminf(x, dpp_f<0x4E>(x));
}
__device__ __forceinline__ float quad_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  return fmaxf(x, dpp_f<0x4E>(x));
}

// ---------------------------------------------------------------- row segment I/O
// A lane's E bf16 elements are E/2 dwords, loaded as 16-byte vectors.
template <int E>
__device__ __forceinline__ void load_bf16_seg(const uint16_t* __restrict__ p, uint32_t (&w)[E / 2]) {
  const uint4* p4 = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < E / 8; ++i) {
    uint4 t = gld(p4 + i);
    w[4 * i + 0] = t.x;
    w[4 * i + 1] = t.y;
    w[4 * i + 2] = t.z;
    w[4 * i + 3] = t.w;
  }
}
template <int E>
__device__ __forceinline__ void store_bf16_seg(uint16_t* __restrict__ p, const uint32_t (&w)[E / 2]) {
  uint4* p4 = reinterpret_cast<uint4*>(p);
#pragma unroll
  for (int i = 0; i < E / 8; ++i) gst(p4 + i, make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]));
}

// Signs of the lane's E (<= 32) elements: bit i of sb set = element i negated.
// Flipping the bf16 sign bit is the exact product x * (-1).
template <int E>
__device__ __forceinline__ void apply_sign_bf16(uint32_t (&w)[E / 2], uint32_t sb) {
#pragma unroll
  for (int i = 0; i < E / 2; ++i) {
    uint32_t s = sb >> (2 * i);
    w[i] ^= ((s & 1u) << 15) | ((s & 2u) << 30);
  }
}

template <int E>
__device__ __forceinline__ void unpack_bf16(const uint32_t (&w)[E / 2], float (&v)[E]) {
#pragma unroll
  for (int i = 0; i < E / 2; ++i) {
    v[2 * i] = bf_lo(w[i]);
    v[2 * i + 1] = bf_hi(w[i]);
  }
}

// ---------------------------------------------------------------- bit packing
// E symbols packed LSB-first into NW = E*BITS/32 (rounded up) words.
template <int E, int BITS>
struct Packed {
  static constexpr int kBitsTotal = E * BITS;
  static constexpr int kWords = (kBitsTotal + 31) / 32;
  static constexpr int kBytes = kBitsTotal / 8;
  uint32_t w[kWords];
};

template <int E, int BITS>
__device__ __forceinline__ void pack_syms(const uint32_t (&s)[E], Packed<E, BITS>& out) {
#pragma unroll
  for (int i = 0; i < Packed<E, BITS>::kWords; ++i) out.w[i] = 0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int bit = j * BITS, wi = bit >> 5, sh = bit & 31;
    out.w[wi] |= s[j] << sh;
    if (sh + BITS > 32) out.w[wi + 1] |= s[j] >> (32 - sh);
  }
}

template <int E, int BITS>
__device__ __forceinline__ void unpack_syms(const Packed<E, BITS>& in, uint32_t (&s)[E]) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int bit = j * BITS, wi = bit >> 5, sh = bit & 31;
    uint32_t v = in.w[wi] >> sh;
    if (sh + BITS > 32) v |= in.w[wi + 1] << (32 - sh);
    s[j] = v & mask;
  }
}

// Store / load the kBytes bytes of a packed segment.  Segments start at a multiple
// of their own size, which is a multiple of 2 bytes (E >= 16), so 16-bit accesses
// are always aligned; whole dwords are used when the size allows it.
template <int E, int BITS>
__device__ __forceinline__ void store_packed(uint8_t* __restrict__ p, const Packed<E, BITS>& v) {
  constexpr int NB = Packed<E, BITS>::kBytes;
  if constexpr (NB % 16 == 0) {
    uint4* p4 = reinterpret_cast<uint4*>(p);
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) gst(p4 + i, make_uint4(v.w[4 * i], v.w[4 * i + 1], v.w[4 * i + 2], v.w[4 * i + 3]));
  } else if constexpr (NB % 4 == 0) {
    uint32_t* p32 = reinterpret_cast<uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < NB / 4; ++i) gst(p32 + i, v.w[i]);
  } else {
    uint16_t* p16 = reinterpret_cast<uint16_t*>(p);
#pragma unroll
    for (int i = 0; i < NB / 2; ++i) gst(p16 + i, (uint16_t)(v.w[i >> 1] >> ((i & 1) * 16)));
  }
}

template <int E, int BITS>
__device__ __forceinline__ void load_packed(const uint8_t* __restrict__ p, Packed<E, BITS>& v) {
  constexpr int NB = Packed<E, BITS>::kBytes;
  if constexpr (NB % 16 == 0) {
    const uint4* p4 = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      uint4 t = gld(p4 + i);
      v.w[4 * i] = t.x;
      v.w[4 * i + 1] = t.y;
      v.w[4 * i + 2] = t.z;
      v.w[4 * i + 3] = t.w;
    }
  } else if constexpr (NB % 4 == 0) {
    const uint32_t* p32 = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < NB / 4; ++i) v.w[i] = gld(p32 + i);
  } else {
    const uint16_t* p16 = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int i = 0; i < Packed<E, BITS>::kWords; ++i) v.w[i] = 0;
#pragma unroll
    for (int i = 0; i < NB / 2; ++i) v.w[i >> 1] |= (uint32_t)gld(p16 + i) << ((i & 1) * 16);
  }
}

}  // namespace kvmi
