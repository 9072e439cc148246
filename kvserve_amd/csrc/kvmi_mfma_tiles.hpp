// Device helpers of the MFMA paged kernels (gfx950): Hadamard tiles, rounding
// chains, bit packers, lane reductions and the per-tile K / V work shared by the
// two-pass kernels (kvmi_mfma.hip) and the one-pass compress (kvmi_compress.hip).
//
// Paged compress / decompress kernels with the Hadamard transform on MFMA (gfx950).
//
// The D-point transform of a row is a dense product with the +-1 Sylvester matrix,
// issued as v_mfma_f32_32x32x16_bf16 tiles: bf16 inputs times +-1 are exact and the
// products accumulate in fp32 (the reference runs its FWHT in fp32 with one bf16
// rounding at the end, hadamard_func.py:97-99).  Element index e (7 bits at D=128,
// 6 at D=64) is split as
//     e = HALF*hl + 16*c + 8*kt + j      (HALF = D/2, hl = lane half, j = 0..7)
// so a lane always holds one contiguous half-row: the 16-byte MFMA operand of
// k-tile (c, kt) is uint4 number 2c+kt of that half-row.  The output element f has
// the same split, and the Sylvester sign of (e, f) factorises into a sign per
// 32x16 tile (chunk bits c, c') times one of two 32x16 base tiles (kt = 0, 1):
//   H[e][f] = (-1)^(popc(c & c')) * Hb_kt[m(f)][k(e)],
// so output chunk c' accumulates 2*NC MFMAs with +Hb or -Hb.  One accumulator
// (16 fp32 per lane) is live at a time.
//
// Orientation T (encode, decode): A = Hb, B = X^T -> lane holds output half-row of
// its row.  Orientation N (K statistics): A = X, B = Hb^T -> lane holds 16 rows of
// one output channel, so per-channel min/max reduce in registers.
//
// Rademacher signs are applied by flipping bf16 sign bits (exact): on the input
// before the forward transform and on the output after the inverse one, from an LDS
// table of per-(head, element pair) masks.
//
// Work split: a workgroup of 4 wave64s owns a run of whole blocks of one (request,
// layer) job; a tile is 32 consecutive pool rows (32/H tokens x H heads,
// token-major, as the cache stores them), and wave w takes tiles w, w+4, ... of the
// run.  Because 32 % H == 0 and S*H % 32 == 0, a tile never crosses a block, lane l
// always holds head (l % 32) % H, and the H heads of a token sit in H neighbouring
// lanes.  Each wave issues the loads of its next section (K or V half of a tile)
// before it computes the current one.
//
// Per-element VALU work is kept to the rounding chain the reference fixes:
//   encode  y = bf16(acc*s); t = bf16(y - mn); q = bf16(t * rcp); sym = rint(q)
//   decode  x = bf16(bf16(sym*sc) + mn)  ->  MFMA  ->  out = bf16(acc*s) ^ sign
// with each bf16 rounding one v_cvt_pk_bf16_f32, and symbols packed four to a
// dword by v_cvt_pk_u8_f32 before the bit-width shuffle.
#pragma once

#include <atomic>


#include "kvmi_common.hpp"

namespace kvmi {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMW = 256;  // threads per workgroup
constexpr int kWaves = kMW / 64;
constexpr int kTok = 32;  // rows per tile (MFMA M / N)
constexpr int kMH = 8;    // heads per shard served by these kernels (8 % H == 0)

__device__ __forceinline__ bf16x8 as_b8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Keeps the scheduler from interleaving work across output chunks (or K / V
// sections), which would keep several chunks' accumulators and constants alive.
__device__ __forceinline__ void chunk_fence() { __builtin_amdgcn_sched_barrier(0); }

// A per-lane LDS offset the compiler must re-read every iteration: the per-head
// tables are loop-invariant for a lane, and hoisting their reads out of the tile
// loop would pin ~160 VGPRs for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
// A value the instruction selector may not look through (keeps byte extracts of a
// masked word as v_cvt_f32_ubyteN instead of re-deriving them from the source).
__device__ __forceinline__ uint32_t barrier_u(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// Software pipelining: the loads of the next tile are issued before the current one
// is computed.  Pinning a buffer where its tile's work starts keeps the compiler from
// hoisting that work (e.g. the sign flips) above the previous tile's, which would
// make the previous tile wait for these loads.
__device__ __forceinline__ void pin(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ f32x16 mfma(uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_b8(a), as_b8(b), c, 0, 0, 0);
}

// Base tile kt of the 32-point factor as this lane's MFMA operand (8 bf16 = uint4).
// orient_n == false: A[m][k], lane = m + 32*(k/8); output bits (f_top, f3, f2, f1, f0)
//   = (m2, m4, m3, m1, m0) so that lane l ends up with row l%32, outputs
//   HALF*hl + 16*c' + i in accumulator register i.
// orient_n == true:  B[k][n], lane = n + 32*(k/8); output channel bits
//   (f_top, f3, f2, f1, f0) = (n4, n3, n2, n1, n0).
// Input bits (e_top, e3, e2, e1, e0) = (k/8, kt, j2, j1, j0) in both.
__device__ __forceinline__ uint4 hadamard_tile(int l, int kt, bool orient_n, bool negate) {
  const int hl = l >> 5, r = l & 31;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t v = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int j = 2 * p + s;
      int par;
      if (!orient_n)
        par = ((r >> 2) & hl) ^ ((r >> 4) & kt) ^ ((r >> 3) & (j >> 2)) ^ ((r >> 1) & (j >> 1) & 1) ^ (r & j & 1);
      else
        par = (hl & (r >> 4)) ^ (kt & (r >> 3)) ^ ((j >> 2) & (r >> 2)) ^ ((j >> 1) & (r >> 1) & 1) ^ (j & r & 1);
      par = (par ^ (negate ? 1 : 0)) & 1;
      v |= (uint32_t)(par ? 0xBF80u : 0x3F80u) << (16 * s);
    }
    w[p] = v;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ uint4 hadamard_tile(int kt, bool orient_n, bool negate) {
  return hadamard_tile((int)(threadIdx.x & 63), kt, orient_n, negate);
}

// Base tile kt for the split of decode_kt_kernel (D = 128, orientation T):
//   input  e = 16*s + 8*hl + j    (k-step s = 2*t + kt, lane half hl = k/8, j = 0..7)
//   output f = 32*c' + 16*m2 + i  (chunk c', MFMA row bit m2 = lane half, i = register)
// so a lane's outputs of chunk c' are 16 consecutive elements and chunks 0-1 / 2-3 are
// the two 128-byte halves of a row.  popc(f & e) = popc(c' & t) + the in-tile part
// (m2 & kt) ^ (m4 & kh) ^ (m3 & j2) ^ (m1 & j1) ^ (m0 & j0) (i = 8 m4 + 4 m3 + 2 m1 + m0),
// so transform_T over k-step operands x[2t + kt] gives this split's outputs.
__device__ __forceinline__ uint4 hadamard_tile_d(int kt, bool negate) {
  const int l = (int)(threadIdx.x & 63), kh = l >> 5, m = l & 31;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t v = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int j = 2 * p + s;
      int par = ((m >> 2) & kt) ^ ((m >> 4) & kh) ^ ((m >> 3) & (j >> 2)) ^ ((m >> 1) & (j >> 1) & 1) ^ (m & j & 1);
      par = (par ^ (negate ? 1 : 0)) & 1;
      v |= (uint32_t)(par ? 0xBF80u : 0x3F80u) << (16 * s);
    }
    w[p] = v;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 xor4(uint4 a, uint4 b) { return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w); }

// A bf16-pair constant held in an SGPR.  Left to itself the compiler encodes the
// pair (1.0, 0) = 0x00003F80 as the inline constant "1.0" of v_dot2c_f32_bf16, which
// the hardware reads as the f32 1.0 = 0x3F800000, i.e. the pair (0, 1.0).  The asm
// is not volatile, so the value is materialised once and shared.
__device__ __forceinline__ bf16x2v sgpr_pair(uint32_t v) {
  asm("" : "+s"(v));
  return __builtin_bit_cast(bf16x2v, v);
}

// lo(bf16 pair) + c and hi(bf16 pair) + c by v_dot2_f32_bf16 against (1, 0) / (0, 1).
// On gfx950 the sum is exact when it fits fp32 and is otherwise rounded toward -inf
// (measured: ~0.015 % of random bf16 + bf16-valued operand pairs differ from the fp32
// add by one ulp).  Used only where both terms are bf16 values and the sum is rounded
// to bf16 next: then the fp32 sum is exact when the exponents differ by at most 15, and
// otherwise the smaller term is below 2^-15 of the larger, so both roundings of the
// sum land on the larger term in bf16 -- the result equals bf16(fl(a + c)).
__device__ __forceinline__ float add_lo(uint32_t pk, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pk), sgpr_pair(0x00003F80u), c, false);
}
__device__ __forceinline__ float add_hi(uint32_t pk, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pk), sgpr_pair(0x3F800000u), c, false);
}

// (rbf(c0 - lo(pk)), rbf(c1 - hi(pk))) for a bf16 pair pk and bf16-valued c0, c1: the
// differences by v_dot2_f32_bf16 against (-1, 0) / (0, -1), each rounded to bf16 by
// v_cvt_pk_bf16_f32 with a zero low half (see rbf).  The same argument as for add_lo
// holds (both terms bf16 values, the sum rounded to bf16 next).  A dot instruction's
// result may be read by another VALU instruction only 3 wait states after it: the
// compiler pads that for the instructions it emits itself, not for the reads inside an
// asm statement, so the pair is written out with its padding (the second dot and an
// s_nop 1 before the first read, the s_nop and the first conversion before the second).
// Outputs are early-clobber: the first difference is written before the second dot
// reads pk and c1.
__device__ __forceinline__ void rsub_rbf_pair(uint32_t pk, float c0, float c1, float& t0, float& t1) {
  asm("v_dot2_f32_bf16 %0, %2, %3, %5\n\t"
      "v_dot2_f32_bf16 %1, %2, %4, %6\n\t"
      "s_nop 1\n\t"
      "v_cvt_pk_bf16_f32 %0, 0, %0\n\t"
      "v_cvt_pk_bf16_f32 %1, 0, %1"
      : "=&v"(t0), "=&v"(t1)
      : "v"(pk), "s"(sgpr_pair(0x0000BF80u)), "s"(sgpr_pair(0xBF800000u)), "v"(c0), "v"(c1));
}

// fp32 value of x rounded to bf16 (round to nearest even) in one instruction:
// v_cvt_pk_bf16_f32 with a zero low half leaves bf16(x) << 16, which is that value.
__device__ __forceinline__ float rbf(float x) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
  return r;
}

// Rounded-to-nearest-even integer in [0, 255] of a float, as byte BYTE of `acc`
// (v_cvt_pk_u8_f32 rounds half to even and saturates, checked on gfx950).
template <int BYTE>
__device__ __forceinline__ uint32_t cvt_u8(float x, uint32_t acc) {
  return __builtin_amdgcn_cvt_pk_u8_f32(x, BYTE, acc);
}

// Byte BYTE of w as a float (v_cvt_f32_ubyteN).
template <int BYTE>
__device__ __forceinline__ float ubyte(uint32_t w) {
  return (float)((w >> (8 * BYTE)) & 0xffu);
}

// q = bf16(bf16(bf16(a * s) - mn) * rcp): the quantizer's value before rint
// (quantizer_func.py:60-62; bf16(t * rcp) == bf16(t / sc) for bf16 t and sc, the
// exact quotient being >= 2^-17 (relative) away from every bf16 midpoint).
__device__ __forceinline__ float quant_q(float a, float s, float mn, float rcp) {
  return rbf(rbf(rbf(a * s) - mn) * rcp);
}

// Streaming bit packer for one lane's HALF symbols (compile-time positions).
template <int HALF, int BITS>
struct LanePack {
  static constexpr int kWords = (HALF * BITS + 31) / 32;
  static constexpr int kBytes = HALF * BITS / 8;
  uint32_t w[kWords];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = 0;
  }
  __device__ __forceinline__ void put(int idx, uint32_t s) {  // idx compile-time after unrolling
    const int bit = idx * BITS, wi = bit >> 5, sh = bit & 31;
    w[wi] |= s << sh;
    if (sh + BITS > 32) w[wi + 1] |= s >> (32 - sh);
  }
  __device__ __forceinline__ uint32_t get(int idx) const {
    const int bit = idx * BITS, wi = bit >> 5, sh = bit & 31;
    uint32_t v = w[wi] >> sh;
    if (sh + BITS > 32) v |= w[wi + 1] << (32 - sh);
    return v & ((1u << BITS) - 1u);
  }
  // kBytes is a multiple of 4 (HALF >= 32), and of 8 when HALF == 64.
  __device__ __forceinline__ void store(uint8_t* p) const {
    if constexpr (kBytes % 16 == 0) {
      uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 16; ++i) gst(q + i, make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]));
    } else if constexpr (kBytes % 8 == 0) {
      uint2* q = reinterpret_cast<uint2*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 8; ++i) gst(q + i, make_uint2(w[2 * i], w[2 * i + 1]));
    } else {
      uint32_t* q = reinterpret_cast<uint32_t*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 4; ++i) gst(q + i, w[i]);
    }
  }
  // Store into LDS (p aligned to the largest of 16, 8, 4 that divides kBytes).
  __device__ __forceinline__ void store_lds(uint8_t* p) const {
    if constexpr (kBytes % 16 == 0) {
      uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 16; ++i) q[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    } else if constexpr (kBytes % 8 == 0) {
      uint2* q = reinterpret_cast<uint2*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 8; ++i) q[i] = make_uint2(w[2 * i], w[2 * i + 1]);
    } else {
      uint32_t* q = reinterpret_cast<uint32_t*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 4; ++i) q[i] = w[i];
    }
  }
  __device__ __forceinline__ void load(const uint8_t* p) {
    if constexpr (kBytes % 16 == 0) {
      const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 16; ++i) {
        uint4 t = gld(q + i);
        w[4 * i] = t.x;
        w[4 * i + 1] = t.y;
        w[4 * i + 2] = t.z;
        w[4 * i + 3] = t.w;
      }
    } else if constexpr (kBytes % 8 == 0) {
      const uint2* q = reinterpret_cast<const uint2*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 8; ++i) {
        uint2 t = gld(q + i);
        w[2 * i] = t.x;
        w[2 * i + 1] = t.y;
      }
    } else {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 4; ++i) w[i] = gld(q + i);
    }
    if constexpr (kWords * 4 > kBytes) w[kWords - 1] &= 0xffffffffu >> (32 - 8 * (kBytes % 4));
  }
};

// Byte lanes of the symbols that cannot fit BITS bits (v_cvt_pk_u8_f32 saturates at
// 255, so a symbol >= 2^BITS always shows in these bits of the OR of all bytes).
template <int BITS>
constexpr uint32_t overflow_mask() {
  return 0x01010101u * (0xffu & ~((1u << BITS) - 1u));
}

// Shared per-workgroup tables for up to HM heads (8, or 32 for the wide-head kernels).
template <int HM>
struct TablesT {
  uint32_t smask[HM][64 + 4];  // bf16 sign-flip masks per (head, element pair), padded rows
  float2 kc[HM][128 + 4];      // K (min, -1/scale) [encode] or (min, scale) [decode], by source head
  uint8_t prof[2][3][HM];      // the job's profile bytes (kvmi_layer_job::profile)
  int posk[HM], posv[HM], gfirst[HM];
};
using Tables = TablesT<kMH>;
constexpr int kWideH = 32;  // head capacity of the wide-head kernels (H = 16 or 32)

// Decode tables of the K-table decode: the per-channel K pairs are replaced by the
// table of dequantized values (decode_kt_kernel).
struct DecTables {
  uint32_t smask[kMH][64 + 4];
  uint8_t prof[2][3][kMH];
  int posk[kMH], posv[kMH], gfirst[kMH];
};

// Stage the profile bytes into LDS (one load per thread, no dependent chains).  With
// paired virtual heads (kPairedHeads) the job's profile is the real one, [2][3][H / 2]:
// virtual position 2j + b is half b of position j, whose source head is 2 order[j] + b.
template <class TT>
__device__ __forceinline__ void stage_profile(TT& T, const uint8_t* profile, int H, bool paired = false) {
  if (threadIdx.x < 6u * H) {
    const int i = threadIdx.x, part = i / (3 * H), f = (i / H) % 3, k = i % H;
    if (paired) {
      const int hr = H / 2;
      const uint8_t b = gld(profile + part * 3 * hr + f * hr + (k >> 1));
      T.prof[part][f][k] = f == 0 ? (uint8_t)(2 * b + (k & 1)) : b;
    } else {
      T.prof[part][f][k] = gld(profile + i);
    }
  }
}

// Fill the sign-mask table: word p of head h flips elements 2p and 2p+1.
template <class TT>
__device__ __forceinline__ void fill_signs(TT& T, const uint32_t* signs, int H, int D) {
  for (int i = threadIdx.x; i < H * (D / 2); i += (int)blockDim.x) {
    const int h = i / (D / 2), p = i % (D / 2);
    const uint32_t s = gld(signs + h * (D / 32) + (2 * p) / 32) >> ((2 * p) & 31);
    T.smask[h][p] = ((s & 1u) << 15) | ((s & 2u) << 30);
  }
}

// Output positions of each source head and the first head of each V group, from
// the staged profile (after a barrier).
template <class TT>
__device__ __forceinline__ void fill_positions(TT& T, int H) {
  if (threadIdx.x < (unsigned)H) {
    const int h = threadIdx.x;
    for (int k = 0; k < H; ++k) {
      if (T.prof[0][0][k] == h) T.posk[h] = k;
      if (T.prof[1][0][k] == h) T.posv[h] = k;
    }
    // first output position of V group h (if any) -> its source head
    T.gfirst[h] = -1;
    for (int k = H - 1; k >= 0; --k)
      if (T.prof[1][2][k] == h) T.gfirst[h] = T.prof[1][0][k];
  }
}

// K constants by source head from kmeta (stored by output position j, whose source
// head is order[j]).  DIV: store (min, -1/scale) (the quantizer's form) instead of (min, scale).
template <bool DIV, class TT>
__device__ __forceinline__ void fill_kconst(TT& T, const uint16_t* kmeta, int H, int D) {
  const int HD = H * D;
  for (int i = threadIdx.x; i < HD; i += (int)blockDim.x) {
    const int j = i / D, e = i % D, hs = T.prof[0][0][j];
    const float m = bf16_to_f32(gld(kmeta + i));
    const float sc = bf16_to_f32(gld(kmeta + HD + i));
    T.kc[hs][e] = make_float2(m, DIV ? -1.0f / sc : sc);
  }
}

// The run of tokens [tok0, tok_end) of a workgroup and its tile count.  Runs are
// whole blocks and tiles never straddle blocks, so every row of every tile exists.
struct Run {
  int tok0, tok_end, tiles, nwg;
};
__device__ __forceinline__ Run wg_run(const kvmi_layer_job& job, const Geo& g) {
  Run u;
  const int ntok = job.num_blocks * g.S;
  const int run = g.bpw * g.S;
  u.nwg = (ntok + run - 1) / run;
  u.tok0 = blockIdx.x * run;
  u.tok_end = min(ntok, u.tok0 + run);
  u.tiles = u.tok_end > u.tok0 ? (u.tok_end - u.tok0) * g.H / kTok : 0;
  return u;
}

// Pool row of the first row of tile t (wave-uniform); lane r's row is that + r, its
// token tile_tok(..) + r / H.
__device__ __forceinline__ int tile_tok(int tok0, int H, int t) { return tok0 + t * (kTok / H); }
__device__ __forceinline__ int64_t tile_row0(const kvmi_layer_job& job, int S, int H, int ta) {
  return ((int64_t)cld(job.block_ids + ta / S) * S + (ta % S)) * H;
}

// Load (and sign) the lane's half-row of bf16 inputs of pool row `row`.
template <int NC>
__device__ __forceinline__ void load_half_row(const uint16_t* __restrict__ pool, int64_t row, int hl,
                                              uint4 (&x)[2 * NC]) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const uint4* src = reinterpret_cast<const uint4*>(pool + row * D + HALF * hl);
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) x[u] = gld(src + u);
}
// Coalesced load of the 32 rows of a tile (contiguous in the pool, from row `row0`):
// instruction v reads 1 KiB, lane l the 16-byte piece 64 v + l of the tile.  Random
// 32 KiB blocks read this way stream at ~5.8 TB/s on MI355X, against ~4.2 TB/s when
// each lane reads its own half-row (every instruction then touches 64 cache lines).
template <int NC>
__device__ __forceinline__ void load_tile(const uint16_t* __restrict__ pool, int64_t row0, uint4 (&x)[2 * NC]) {
  const uint4* src = reinterpret_cast<const uint4*>(pool + row0 * (32 * NC)) + (threadIdx.x & 63);
#pragma unroll
  for (int v = 0; v < 2 * NC; ++v) x[v] = gld(src + 64 * v);
}

// uint4 of a wave's buffer for tile_to_half_rows: 32 rows at a pitch of 4NC + 1 pieces.
template <int NC>
constexpr int tile_buf_q() { return kTok * (4 * NC + 1); }

// Rearrange a tile loaded by load_tile into the MFMA layout (lane (r, hl): half-row hl
// of row r, as load_half_row) through the wave's LDS buffer `buf` (tile_buf_q<NC>()
// uint4).  Rows sit at a pitch of 4NC + 1 pieces, so the lanes that write one row and
// the lanes that read one piece of consecutive rows fall on distinct banks, and every
// access is a per-lane base plus a compile-time offset.  LDS executes a wave's
// operations in order, so no barrier is needed; the buffer belongs to this wave.
template <int NC>
__device__ __forceinline__ void tile_to_half_rows(uint4* buf, uint4 (&x)[2 * NC]) {
  constexpr int PR = 4 * NC, PP = PR + 1;  // pieces per row, pitch
  const int l = threadIdx.x & 63, r = l & 31, hl = l >> 5;
  // piece 64 v + l of the tile: row (64 v + l) / PR = (64 / PR) v + l / PR, piece l % PR
  uint4* wr = buf + (l / PR) * PP + l % PR;
#pragma unroll
  for (int v = 0; v < 2 * NC; ++v) wr[(64 / PR) * PP * v] = x[v];
  const uint4* rd = buf + r * PP + 2 * NC * hl;
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) x[u] = rd[u];
}

// The same from a sign-mask table laid out like Tables::smask.
template <int NC>
__device__ __forceinline__ void sign_half_row(const uint32_t (*smask)[64 + 4], int h, int hl, uint4 (&x)[2 * NC]) {
  constexpr int HALF = 16 * NC;
  const uint4* sm = reinterpret_cast<const uint4*>(&smask[0][0] + opaque(h * (64 + 4) + (HALF / 2) * hl));
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) x[u] = xor4(x[u], sm[u]);
}
template <int NC, class TT>
__device__ __forceinline__ void sign_half_row(const TT& T, int h, int hl, uint4 (&x)[2 * NC]) {
  constexpr int HALF = 16 * NC;
  const uint4* sm = reinterpret_cast<const uint4*>(&T.smask[0][0] + opaque(h * (64 + 4) + (HALF / 2) * hl));
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) x[u] = xor4(x[u], sm[u]);
}

// Paired virtual heads: the 256-point transform of a row from the 128-point transforms
// a_lo, a_hi of its halves, y_lo = a_lo + a_hi and y_hi = a_lo - a_hi (the Sylvester
// matrix's last stage; the inverse has the same form).  Orientation T holds the two
// halves of a row in the lane pair (2i, 2i + 1): fma(+-1, a, partner) is the one
// rounding of the sum or difference.
__device__ __forceinline__ void pair_butterfly_T(f32x16& acc) {
  const float sgn = (threadIdx.x & 1) ? -1.f : 1.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float partner = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[i]), 0xB1, 0xF, 0xF, false));
    acc[i] = __builtin_fmaf(sgn, acc[i], partner);
  }
}
// Orientation N holds them in registers 2i and 2i + 1 of a lane (rows m and m ^ 1).
__device__ __forceinline__ void pair_butterfly_N(f32x16& acc) {
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const float a = acc[i], b = acc[i + 1];
    acc[i] = a + b;
    acc[i + 1] = a - b;
  }
}

// Forward / inverse transform, orientation T, output chunk cp (unscaled fp32).
// The input chunks are visited in the order cp ^ k, so the chains of different
// output chunks share no prefix (a shared prefix would keep extra accumulators live).
template <int NC>
__device__ __forceinline__ f32x16 transform_T(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                              int cp) {
  f32x16 acc = {};
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = cp ^ k;
    const bool neg = __builtin_popcount(c & cp) & 1;
    acc = mfma(neg ? hn[0] : hp[0], x[2 * c], acc);
    acc = mfma(neg ? hn[1] : hp[1], x[2 * c + 1], acc);
  }
  return acc;
}

// Pack the 16 quantized values q of output chunk cp into the lane's packer (rint,
// saturate, and OR the bytes into `over` for the width check).  Widths 2, 4, 8 pack
// byte lanes: dword d_m holds the symbols i with i % P == m (P = 8/BITS symbols per
// byte), and the chunk's words are OR_m d_m << (m*BITS).
template <int HALF, int BITS>
__device__ __forceinline__ void pack_chunk(const float (&q)[16], int cp, LanePack<HALF, BITS>& pk, uint32_t& over) {
  if constexpr (BITS == 2 || BITS == 4 || BITS == 8) {
    constexpr int P = 8 / BITS, W = BITS / 2;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int m = 0; m < P; ++m) {
        uint32_t d = cvt_u8<0>(q[P * (4 * j) + m], 0u);
        d = cvt_u8<1>(q[P * (4 * j + 1) + m], d);
        d = cvt_u8<2>(q[P * (4 * j + 2) + m], d);
        d = cvt_u8<3>(q[P * (4 * j + 3) + m], d);
        over |= d;
        word |= d << (m * BITS);
      }
      pk.w[cp * W + j] = word;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t sym = cvt_u8<0>(q[i], 0u);
      over |= sym;
      pk.put(16 * cp + i, sym);
    }
  }
}

// Quantize output chunk cp (16 accumulators of the lane's half-row) with per-element
// (min, -1/scale) pairs from the LDS table at kq (K: per-channel statistics).
template <int HALF, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_chunk_k(const f32x16& acc, int cp, float s, const float2* kq, float lv,
                                              LanePack<HALF, BITS>& pk, uint32_t& over) {
  float q[16];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const float4 c = *reinterpret_cast<const float4*>(kq + i);
    // y pair rounded by one v_cvt_pk_bf16_f32; with c = (mn, -1/scale), and negation
    // commuting with round-to-nearest-even: rbf(rbf(mn - y) * -rcp) == rbf(rbf(y - mn) * rcp)
    const uint32_t y2 = pack_bf16x2(acc[i] * s, acc[i + 1] * s);
    float t0, t1;
    rsub_rbf_pair(y2, c.x, c.z, t0, t1);
    q[i] = rbf(t0 * c.y);
    q[i + 1] = rbf(t1 * c.w);
    if constexpr (CLAMP) {
      q[i] = fminf(q[i], lv);
      q[i + 1] = fminf(q[i + 1], lv);
    }
  }
  pack_chunk<HALF, BITS>(q, cp, pk, over);
}

// Quantize output chunk cp from its 16 transformed values y, kept as 8 bf16 pairs,
// with the row's (mn, 1/scale) (V: per-token statistics).
template <int HALF, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_chunk_v(const uint32_t* ypk, int cp, float mn, float rcp, float lv,
                                              LanePack<HALF, BITS>& pk, uint32_t& over) {
  const float nrcp = -rcp;
  float q[16];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    float t0, t1;
    rsub_rbf_pair(ypk[i / 2], mn, mn, t0, t1);
    q[i] = rbf(t0 * nrcp);
    q[i + 1] = rbf(t1 * nrcp);
    if constexpr (CLAMP) {
      q[i] = fminf(q[i], lv);
      q[i + 1] = fminf(q[i + 1], lv);
    }
  }
  pack_chunk<HALF, BITS>(q, cp, pk, over);
}

// The 8 symbols of operand u (elements 8u .. 8u+7 of the half-row) as floats.
template <int HALF, int BITS>
__device__ __forceinline__ void syms8(const LanePack<HALF, BITS>& pk, int u, float (&s)[8]) {
  if constexpr (BITS == 4) {
    const uint32_t w = pk.w[u];
    const uint32_t lo = barrier_u(w & 0x0F0F0F0Fu), hi = barrier_u((w >> 4) & 0x0F0F0F0Fu);
    s[0] = ubyte<0>(lo);
    s[1] = ubyte<0>(hi);
    s[2] = ubyte<1>(lo);
    s[3] = ubyte<1>(hi);
    s[4] = ubyte<2>(lo);
    s[5] = ubyte<2>(hi);
    s[6] = ubyte<3>(lo);
    s[7] = ubyte<3>(hi);
  } else if constexpr (BITS == 8) {
    const uint32_t a = pk.w[2 * u], b = pk.w[2 * u + 1];
    s[0] = ubyte<0>(a);
    s[1] = ubyte<1>(a);
    s[2] = ubyte<2>(a);
    s[3] = ubyte<3>(a);
    s[4] = ubyte<0>(b);
    s[5] = ubyte<1>(b);
    s[6] = ubyte<2>(b);
    s[7] = ubyte<3>(b);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = (float)pk.get(8 * u + j);
  }
}

// Dequantized bf16 MFMA operands of the lane's half-row: x~ = bf16(bf16(sym*sc) + mn)
// (quantizer_func.py:108-112).  KQ: per-element (min, scale) pairs from the LDS
// table at kd; otherwise the row's (mn, sc).
template <int NC, int BITS, bool KQ>
__device__ __forceinline__ void dequant_half_row(const LanePack<16 * NC, BITS>& pk, const float2* kd, float mn,
                                                 float sc, uint4 (&x)[2 * NC]) {
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) {
    float sy[8];
    syms8<16 * NC, BITS>(pk, u, sy);
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (KQ) {
        // per-element constants: the pair's sums come straight out of v_dot2
        const float4 c = *reinterpret_cast<const float4*>(&kd[8 * u + 2 * p]);
        const uint32_t spk = pack_bf16x2(sy[2 * p] * c.y, sy[2 * p + 1] * c.w);
        w[p] = pack_bf16x2(add_lo(spk, c.x), add_hi(spk, c.z));
      } else {
        // one row minimum: plain adds (v_dot2c would need a copy of it per element)
        w[p] = pack_bf16x2(rbf(sy[2 * p] * sc) + mn, rbf(sy[2 * p + 1] * sc) + mn);
      }
    }
    x[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------- V by table lookup
// A V row has one (mn, sc) pair, so at widths 2 and 4 its dequantized values
// x~(q) = bf16(bf16(q * sc) + mn) take 2^BITS values: the wave stages them per row in
// LDS and each element becomes one LDS read instead of the convert / multiply / round /
// add / round chain.  Layout of a wave's table (32 rows): entry (row r, symbol q) at
// byte (r / 8) * G + 16 * q + 2 * (r % 8), G = 16 * 2^BITS + 16 (the pad turns each
// group of 8 rows by four banks).  The address of a symbol is then the row's base
// plus 16 * q, formed from the packed word with one byte-select add per element.
template <int BITS>
constexpr bool kVTable = BITS == 2 || BITS == 4;
template <int BITS>
constexpr int vtab_group() { return 16 * (1 << BITS) + 16; }
template <int BITS>
constexpr int vtab_bytes() { return 4 * vtab_group<BITS>(); }

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_u8*)p; }
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t a) { return *(const lds_u16*)(uintptr_t)a; }
__device__ __forceinline__ void lds_write_u16(uint32_t a, uint32_t v) { *(lds_u16*)(uintptr_t)a = (uint16_t)v; }

// base + byte B of packed (v_add_u32 with an SDWA byte select: one instruction).
template <int B>
__device__ __forceinline__ uint32_t add_byte(uint32_t packed, uint32_t base) {
  uint32_t r;
  if constexpr (B == 0)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
        : "=v"(r) : "v"(packed), "v"(base));
  else if constexpr (B == 1)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:DWORD"
        : "=v"(r) : "v"(packed), "v"(base));
  else if constexpr (B == 2)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:DWORD"
        : "=v"(r) : "v"(packed), "v"(base));
  else
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:DWORD"
        : "=v"(r) : "v"(packed), "v"(base));
  return r;
}

// 16 * (symbol of element e) in the byte lanes of word w, for the elements e of w
// with e % P == M (P symbols per byte; byte b holds element P * b + M).
template <int BITS, int M>
__device__ __forceinline__ uint32_t sym16(uint32_t w) {
  constexpr int sh = 4 - BITS * M;
  constexpr uint32_t mask = 0x01010101u * (((1u << BITS) - 1u) << 4);
  return (sh >= 0 ? (w << sh) : (w >> -sh)) & mask;
}

// Fill the table of the lane's row (lanes r and r + 32 take half the symbols each).
template <int BITS>
__device__ __forceinline__ void fill_v_table(uint32_t row_base, float mn, float sc) {
  constexpr int EH = (1 << BITS) / 2;
  const int hl = (threadIdx.x >> 5) & 1;
#pragma unroll
  for (int k = 0; k < EH; k += 2) {
    const float q0 = (float)(EH * hl + k);
    const uint32_t w = pack_bf16x2(rbf(q0 * sc) + mn, rbf((q0 + 1.f) * sc) + mn);
    const uint32_t a = row_base + 16u * (uint32_t)(EH * hl + k);
    lds_write_u16(a, w);
    lds_write_u16(a + 16u, w >> 16);
  }
}

// Dequantized bf16 MFMA operands of the lane's half-row of a V section from the
// wave's table at `tab` (filled here): the values of dequant_half_row<NC, BITS, false>.
template <int NC, int BITS>
__device__ __forceinline__ void dequant_v_table(const LanePack<16 * NC, BITS>& pk, float mn, float sc, void* tab,
                                                uint4 (&x)[2 * NC]) {
  static_assert(kVTable<BITS>, "table lookup serves widths 2 and 4");
  const int r = threadIdx.x & 31;
  const uint32_t row_base = lds_addr(tab) + (uint32_t)((r >> 3) * vtab_group<BITS>() + 2 * (r & 7));
  fill_v_table<BITS>(row_base, mn, sc);
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) {
    uint32_t w[4];
    if constexpr (BITS == 4) {
      // word u: elements 8u + 2b in the low nibbles of byte b, 8u + 2b + 1 in the high
      const uint32_t ev = sym16<4, 0>(pk.w[u]), od = sym16<4, 1>(pk.w[u]);
      w[0] = lds_read_u16(add_byte<0>(ev, row_base)) | lds_read_u16(add_byte<0>(od, row_base)) << 16;
      w[1] = lds_read_u16(add_byte<1>(ev, row_base)) | lds_read_u16(add_byte<1>(od, row_base)) << 16;
      w[2] = lds_read_u16(add_byte<2>(ev, row_base)) | lds_read_u16(add_byte<2>(od, row_base)) << 16;
      w[3] = lds_read_u16(add_byte<3>(ev, row_base)) | lds_read_u16(add_byte<3>(od, row_base)) << 16;
    } else {
      // word u / 2: element 4b + m in bits 2m of byte b; x[u] takes bytes 2(u % 2), +1
      const uint32_t pw = pk.w[u / 2];
      const uint32_t s0 = sym16<2, 0>(pw), s1 = sym16<2, 1>(pw), s2 = sym16<2, 2>(pw), s3 = sym16<2, 3>(pw);
      if (u % 2 == 0) {
        w[0] = lds_read_u16(add_byte<0>(s0, row_base)) | lds_read_u16(add_byte<0>(s1, row_base)) << 16;
        w[1] = lds_read_u16(add_byte<0>(s2, row_base)) | lds_read_u16(add_byte<0>(s3, row_base)) << 16;
        w[2] = lds_read_u16(add_byte<1>(s0, row_base)) | lds_read_u16(add_byte<1>(s1, row_base)) << 16;
        w[3] = lds_read_u16(add_byte<1>(s2, row_base)) | lds_read_u16(add_byte<1>(s3, row_base)) << 16;
      } else {
        w[0] = lds_read_u16(add_byte<2>(s0, row_base)) | lds_read_u16(add_byte<2>(s1, row_base)) << 16;
        w[1] = lds_read_u16(add_byte<2>(s2, row_base)) | lds_read_u16(add_byte<2>(s3, row_base)) << 16;
        w[2] = lds_read_u16(add_byte<3>(s0, row_base)) | lds_read_u16(add_byte<3>(s1, row_base)) << 16;
        w[3] = lds_read_u16(add_byte<3>(s2, row_base)) | lds_read_u16(add_byte<3>(s3, row_base)) << 16;
      }
    }
    x[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------- K by table lookup
// K table of decode_kt_kernel (D = 128, 4-bit symbols): the 16 dequantized values
// bf16(bf16(q * sc) + mn) of every (source head hs, channel c) at byte
// c * kKtabRow + 16 * q + 2 * hs.  kKtabRow = 272 turns the banks of channels eight
// apart (the two lane halves of one k-step) by 32.
constexpr int kKtabRow = 16 * 16 + 16;

// Fill the table from the K metadata (stored by output position j, whose source head
// is prof[0][0][j]); after the profile is staged.
template <class TT>
__device__ __forceinline__ void fill_k_table(uint8_t* ktab, const TT& T, const uint16_t* kmeta, int H, int D) {
  const int HD = H * D;
  const uint32_t base = lds_addr(ktab);
  for (int i = threadIdx.x; i < HD; i += (int)blockDim.x) {
    const int j = i / D, c = i % D, hs = T.prof[0][0][j];
    const float mn = bf16_to_f32(gld(kmeta + i));
    const float sc = bf16_to_f32(gld(kmeta + HD + i));
    const uint32_t a = base + (uint32_t)(c * kKtabRow + 2 * hs);
#pragma unroll
    for (int q = 0; q < 16; q += 2) {
      const uint32_t w = pack_bf16x2(rbf((float)q * sc) + mn, rbf((float)(q + 1) * sc) + mn);
      lds_write_u16(a + 16u * q, w);
      lds_write_u16(a + 16u * (q + 1), w >> 16);
    }
  }
}

// Dequantized bf16 MFMA operands of a K section of decode_kt_kernel: word W[s] holds
// the symbols of elements 16 s + 8 hl + (0..7) (nibble j = element j), `base` is the
// table address of the lane's (source head, channel 8 hl).
__device__ __forceinline__ void dequant_k_table(const uint32_t (&W)[8], uint32_t base, uint4 (&x)[8]) {
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t ev = sym16<4, 0>(W[s]), od = sym16<4, 1>(W[s]);
    constexpr int R = kKtabRow;
    const uint32_t o = (uint32_t)(16 * s * R);
    const uint32_t w0 = lds_read_u16(add_byte<0>(ev, base) + o) | lds_read_u16(add_byte<0>(od, base) + o + R) << 16;
    const uint32_t w1 = lds_read_u16(add_byte<1>(ev, base) + o + 2 * R) | lds_read_u16(add_byte<1>(od, base) + o + 3 * R) << 16;
    const uint32_t w2 = lds_read_u16(add_byte<2>(ev, base) + o + 4 * R) | lds_read_u16(add_byte<2>(od, base) + o + 5 * R) << 16;
    const uint32_t w3 = lds_read_u16(add_byte<3>(ev, base) + o + 6 * R) | lds_read_u16(add_byte<3>(od, base) + o + 7 * R) << 16;
    x[s] = make_uint4(w0, w1, w2, w3);
  }
}

// ---------------------------------------------------------------- tables at any width
// Widths whose symbols do not sit in byte lanes (3 bits) address the tables with a
// bit-field extract and a shift-add per element instead of the byte-select adds.

// v * 16 + base in one v_lshl_add_u32 (left to itself the compiler folds the shift
// into the extract that feeds it and spends a third instruction on the add).
__device__ __forceinline__ uint32_t lshl4_add(uint32_t v, uint32_t base) {
  uint32_t r;
  asm("v_lshl_add_u32 %0, %1, 4, %2" : "=v"(r) : "v"(v), "v"(base));
  return r;
}

// base + 16 * (symbol idx of the lane's packed half-row); idx is compile-time.
template <int HALF, int BITS>
__device__ __forceinline__ uint32_t sym_addr16(const LanePack<HALF, BITS>& pk, int idx, uint32_t base) {
  const int bit = idx * BITS, wi = bit >> 5, sh = bit & 31;
  uint32_t v;
  if (sh + BITS <= 32)
    v = __builtin_amdgcn_ubfe(pk.w[wi], (uint32_t)sh, (uint32_t)BITS);
  else  // the symbol straddles two words
    v = __builtin_amdgcn_alignbit(pk.w[wi + 1], pk.w[wi], (uint32_t)sh) & ((1u << BITS) - 1u);
  return lshl4_add(v, base);
}

// Dequantized V operands from the wave's row table (filled here) for the widths the
// byte-select lookup of dequant_v_table does not serve: the values of
// dequant_half_row<NC, BITS, false>.
template <int NC, int BITS>
__device__ __forceinline__ void dequant_v_table_bfe(const LanePack<16 * NC, BITS>& pk, float mn, float sc, void* tab,
                                                    uint4 (&x)[2 * NC]) {
  const int r = threadIdx.x & 31;
  const uint32_t row_base = lds_addr(tab) + (uint32_t)((r >> 3) * vtab_group<BITS>() + 2 * (r & 7));
  fill_v_table<BITS>(row_base, mn, sc);
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int e = 8 * u + 2 * p;
      w[p] = lds_read_u16(sym_addr16<16 * NC, BITS>(pk, e, row_base)) |
             lds_read_u16(sym_addr16<16 * NC, BITS>(pk, e + 1, row_base)) << 16;
    }
    x[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// K table of decode_mfma_kernel at D = 64 and widths up to 4: the 2^BITS dequantized
// values of every (source head hs, channel c) at byte c * ktab_row + 16 * q + 2 * hs.
template <int BITS>
constexpr int ktab_row() { return 16 * (1 << BITS) + 16; }

template <int BITS, class TT>
__device__ __forceinline__ void fill_k_table_w(uint8_t* ktab, const TT& T, const uint16_t* kmeta, int H, int D) {
  const int HD = H * D;
  const uint32_t base = lds_addr(ktab);
  for (int i = threadIdx.x; i < HD; i += (int)blockDim.x) {
    const int j = i / D, c = i % D, hs = T.prof[0][0][j];
    const float mn = bf16_to_f32(gld(kmeta + i));
    const float sc = bf16_to_f32(gld(kmeta + HD + i));
    const uint32_t a = base + (uint32_t)(c * ktab_row<BITS>() + 2 * hs);
#pragma unroll
    for (int q = 0; q < (1 << BITS); q += 2) {
      const uint32_t w = pack_bf16x2(rbf((float)q * sc) + mn, rbf((float)(q + 1) * sc) + mn);
      lds_write_u16(a + 16u * q, w);
      lds_write_u16(a + 16u * (q + 1), w >> 16);
    }
  }
}

// Dequantized K operands of the lane's half-row from that table; `kbase` is the
// address of (the lane's source head, channel HALF * hl): element e of the half-row
// is channel HALF * hl + e.
template <int NC, int BITS>
__device__ __forceinline__ void dequant_k_table_w(const LanePack<16 * NC, BITS>& pk, uint32_t kbase,
                                                  uint4 (&x)[2 * NC]) {
  constexpr int R = ktab_row<BITS>();
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int e = 8 * u + 2 * p;
      w[p] = lds_read_u16(sym_addr16<16 * NC, BITS>(pk, e, kbase) + (uint32_t)(e * R)) |
             lds_read_u16(sym_addr16<16 * NC, BITS>(pk, e + 1, kbase) + (uint32_t)((e + 1) * R)) << 16;
    }
    x[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// DPP lane exchange of a float (no bound_ctrl; every lane is enabled).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Min / max over the H lanes of a token (aligned groups of H in 1, 2, 4, 8, 16, 32):
// quad_perm xor 1, xor 2, row_half_mirror (lane i <-> 7 - i of each 8), row_mirror
// (lane i <-> 15 - i of each 16), then lane xor 16 through ds_bpermute.
__device__ __forceinline__ void token_minmax(float& a, float& b, int H) {
  if (H >= 2) {
    a = fminf(a, dpp<0xB1>(a));
    b = fmaxf(b, dpp<0xB1>(b));
  }
  if (H >= 4) {
    a = fminf(a, dpp<0x4E>(a));
    b = fmaxf(b, dpp<0x4E>(b));
  }
  if (H >= 8) {
    a = fminf(a, dpp<0x141>(a));
    b = fmaxf(b, dpp<0x141>(b));
  }
  if (H >= 16) {
    a = fminf(a, dpp<0x140>(a));
    b = fmaxf(b, dpp<0x140>(b));
  }
  if (H >= 32) {
    const int src = (int)((threadIdx.x & 63) ^ 16) << 2;
    a = fminf(a, __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(a))));
    b = fmaxf(b, __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(b))));
  }
}
// Min / max of x over lanes l and l ^ 32.  v_permlane32_swap exchanges the upper 32
// lanes of its first operand with the lower 32 lanes of its second; with x in both,
// result 0 holds x of lane l % 32 and result 1 x of lane 32 + l % 32.
__device__ __forceinline__ float halves_min(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ============================================================== tile helpers
// K statistics of one signed tile, orientation N: output register i of chunk c holds
// row m = 8*(i/4) + 4*hl + i%4 of the tile and channel f(r, c) = HALF*(r>>4) + 16*c +
// (r & 15); row m has head m % H, which depends only on s = i%4 (32 % H == 0 and
// H <= 8).  Running min / max per (s, c) of the unscaled accumulators.
template <int NC>
__device__ __forceinline__ void kstats_tile(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                            float (&mn)[4][NC], float (&mx)[4][NC], bool paired = false) {
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 acc = {};
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c = cp ^ k;
      const bool neg = __builtin_popcount(c & cp) & 1;
      acc = mfma(x[2 * c], neg ? hn[0] : hp[0], acc);
      acc = mfma(x[2 * c + 1], neg ? hn[1] : hp[1], acc);
    }
    if (paired) pair_butterfly_N(acc);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      mn[a][cp] = fminf(fminf(mn[a][cp], acc[a]), fminf(acc[a + 4], fminf(acc[a + 8], acc[a + 12])));
      mx[a][cp] = fmaxf(fmaxf(mx[a][cp], acc[a]), fmaxf(acc[a + 4], fmaxf(acc[a + 8], acc[a + 12])));
    }
    chunk_fence();
  }
}

// Push a wave's running K min / max into the workgroup's LDS keys [2][H][D] (by
// source head and channel).  Scaling by 1/sqrt(D) > 0 is monotone, so it commutes
// with min / max (and so does the bf16 rounding applied when the keys are finalised).
template <int NC>
__device__ __forceinline__ void push_lkeys(uint32_t* lkey, const float (&mn)[4][NC], const float (&mx)[4][NC],
                                           int H, float scale) {
  constexpr int D = 32 * NC;
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31, HD = H * D;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int h = (4 * hl + a) % H;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int f = (16 * NC) * (r >> 4) + 16 * c + (r & 15);
      atomicMin(&lkey[h * D + f], f2key(mn[a][c] * scale));
      atomicMax(&lkey[HD + h * D + f], f2key(mx[a][c] * scale));
    }
  }
}

// The lane's fixed V / K profile values within a job (after fill_positions).
struct LaneProfile {
  int jk, jv, gv;
  float lvk, lvv;
  bool rep_lane;  // writes the V metadata of (group, token)
};
template <class TT>
__device__ __forceinline__ LaneProfile lane_profile(const TT& T, int hme, int hl) {
  LaneProfile p;
  p.jk = T.posk[hme];
  p.jv = T.posv[hme];
  p.gv = T.prof[1][2][p.jv];
  p.lvk = (float)T.prof[0][1][p.jk];
  p.lvv = (float)T.prof[1][1][p.jv];
  p.rep_lane = hl == 0 && T.gfirst[p.gv] == hme;
  return p;
}

// K section of a signed tile (orientation T): transform and quantize with the
// per-channel (min, 1/scale) pairs at kq into pkd.
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_k_tile(const uint4 (&xk)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                             const float2* kq, float s, float lvk, LanePack<16 * NC, BITS>& pkd,
                                             uint32_t& over, bool paired = false) {
  pkd.clear();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 acc = transform_T<NC>(xk, hp, hn, cp);
    if (paired) pair_butterfly_T(acc);
    quant_chunk_k<16 * NC, BITS, CLAMP>(acc, cp, s, kq + 16 * cp, lvk, pkd, over);
    chunk_fence();
  }
}

// V section of a signed tile (per-token statistics over the heads of a group):
// transform once, keeping y = bf16(acc * s) as bf16 pairs, reduce the group's
// min / max over the token's lanes, write the (group, token) metadata from the
// representative lane and quantize into pkd.
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_v_tile(const uint4 (&xv)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                             const LaneProfile& lp, const kvmi_layer_job& job, int ntok, int tok,
                                             int G, int H, float s, LanePack<16 * NC, BITS>& pkd, uint32_t& over) {
  constexpr int HALF = 16 * NC;
  uint32_t ypk[HALF / 2];
  float amn = __builtin_inff(), amx = -__builtin_inff();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    const f32x16 acc = transform_T<NC>(xv, hp, hn, cp);
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      amn = fminf(fminf(amn, acc[i]), fminf(acc[i + 1], fminf(acc[i + 2], acc[i + 3])));
      amx = fmaxf(fmaxf(amx, acc[i]), fmaxf(acc[i + 1], fmaxf(acc[i + 2], acc[i + 3])));
    }
#pragma unroll
    for (int i = 0; i < 16; i += 2) ypk[8 * cp + i / 2] = pack_bf16x2(acc[i] * s, acc[i + 1] * s);
    chunk_fence();
  }
  // y = bf16(fl(acc * s)) is monotone in acc (s > 0): the row's min / max of y
  // are those of acc pushed through the same rounding.
  amn = halves_min(amn);
  amx = halves_max(amx);
  float mn = 0.f, mx = 0.f;
  for (int gg = 0; gg < G; ++gg) {
    float a = lp.gv == gg ? amn : __builtin_inff();
    float b = lp.gv == gg ? amx : -__builtin_inff();
    token_minmax(a, b, H);
    if (lp.gv == gg) {
      mn = a;
      mx = b;
    }
  }
  mn = rbf(mn * s);
  mx = rbf(mx * s);
  const float sc = quant_scale(mn, mx, (int)lp.lvv);
  const float rcp = 1.0f / sc;
  if (lp.rep_lane) {
    gst(job.vmeta + (int64_t)lp.gv * ntok + tok, (uint16_t)f32_to_bf16_bits(mn));
    gst(job.vmeta + (int64_t)(G + lp.gv) * ntok + tok, (uint16_t)f32_to_bf16_bits(sc));
  }
  pkd.clear();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    quant_chunk_v<HALF, BITS, CLAMP>(ypk + 8 * cp, cp, mn, rcp, lp.lvv, pkd, over);
    chunk_fence();
  }
}

// V section of a signed tile like quant_v_tile, with the rounded outputs y parked in
// LDS between the statistics and the quantization instead of in registers (or a second
// transform): `ylane` is the lane's slot of a wave buffer of 2*NC x 64 uint4 (stride 64
// uint4, so every access of the wave is 1 KB of consecutive LDS).
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_v_tile_lds(const uint4 (&xv)[2 * NC], const uint4 (&hp)[2],
                                                 const uint4 (&hn)[2], const LaneProfile& lp,
                                                 const kvmi_layer_job& job, int ntok, int tok, int G, int H,
                                                 float s, uint4* ylane, LanePack<16 * NC, BITS>& pkd,
                                                 uint32_t& over, bool paired = false) {
  constexpr int HALF = 16 * NC;
  float amn = __builtin_inff(), amx = -__builtin_inff();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 acc = transform_T<NC>(xv, hp, hn, cp);
    if (paired) pair_butterfly_T(acc);
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      amn = fminf(fminf(amn, acc[i]), fminf(acc[i + 1], fminf(acc[i + 2], acc[i + 3])));
      amx = fmaxf(fmaxf(amx, acc[i]), fmaxf(acc[i + 1], fmaxf(acc[i + 2], acc[i + 3])));
    }
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) w[i / 2] = pack_bf16x2(acc[i] * s, acc[i + 1] * s);
    ylane[(2 * cp) * 64] = make_uint4(w[0], w[1], w[2], w[3]);
    ylane[(2 * cp + 1) * 64] = make_uint4(w[4], w[5], w[6], w[7]);
    chunk_fence();
  }
  amn = halves_min(amn);
  amx = halves_max(amx);
  float mn = 0.f, mx = 0.f;
  for (int gg = 0; gg < G; ++gg) {
    float a = lp.gv == gg ? amn : __builtin_inff();
    float b = lp.gv == gg ? amx : -__builtin_inff();
    token_minmax(a, b, H);
    if (lp.gv == gg) {
      mn = a;
      mx = b;
    }
  }
  mn = rbf(mn * s);
  mx = rbf(mx * s);
  const float sc = quant_scale(mn, mx, (int)lp.lvv);
  const float rcp = 1.0f / sc;
  if (lp.rep_lane) {
    gst(job.vmeta + (int64_t)lp.gv * ntok + tok, (uint16_t)f32_to_bf16_bits(mn));
    gst(job.vmeta + (int64_t)(G + lp.gv) * ntok + tok, (uint16_t)f32_to_bf16_bits(sc));
  }
  pkd.clear();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    const uint4 a = ylane[(2 * cp) * 64], b = ylane[(2 * cp + 1) * 64];
    const uint32_t ypk[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    quant_chunk_v<HALF, BITS, CLAMP>(ypk, cp, mn, rcp, lp.lvv, pkd, over);
    chunk_fence();
  }
}

// V section of a signed tile (per-token statistics over the heads of a group) like
// quant_v_tile, with the transform run twice (statistics, then quantization) instead
// of keeping the rounded outputs in registers: the same values, 32 fewer VGPRs.
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_v_tile_twice(const uint4 (&xv)[2 * NC], const uint4 (&hp)[2],
                                                   const uint4 (&hn)[2], const LaneProfile& lp,
                                                   const kvmi_layer_job& job, int ntok, int tok, int G, int H,
                                                   float s, LanePack<16 * NC, BITS>& pkd, uint32_t& over) {
  constexpr int HALF = 16 * NC;
  float amn = __builtin_inff(), amx = -__builtin_inff();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    const f32x16 acc = transform_T<NC>(xv, hp, hn, cp);
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      amn = fminf(fminf(amn, acc[i]), fminf(acc[i + 1], fminf(acc[i + 2], acc[i + 3])));
      amx = fmaxf(fmaxf(amx, acc[i]), fmaxf(acc[i + 1], fmaxf(acc[i + 2], acc[i + 3])));
    }
    chunk_fence();
  }
  amn = halves_min(amn);
  amx = halves_max(amx);
  float mn = 0.f, mx = 0.f;
  for (int gg = 0; gg < G; ++gg) {
    float a = lp.gv == gg ? amn : __builtin_inff();
    float b = lp.gv == gg ? amx : -__builtin_inff();
    token_minmax(a, b, H);
    if (lp.gv == gg) {
      mn = a;
      mx = b;
    }
  }
  mn = rbf(mn * s);
  mx = rbf(mx * s);
  const float sc = quant_scale(mn, mx, (int)lp.lvv);
  const float rcp = 1.0f / sc;
  if (lp.rep_lane) {
    gst(job.vmeta + (int64_t)lp.gv * ntok + tok, (uint16_t)f32_to_bf16_bits(mn));
    gst(job.vmeta + (int64_t)(G + lp.gv) * ntok + tok, (uint16_t)f32_to_bf16_bits(sc));
  }
  pkd.clear();
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    const f32x16 acc = transform_T<NC>(xv, hp, hn, cp);
    float q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      q[i] = quant_q(acc[i], s, mn, rcp);
      if constexpr (CLAMP) q[i] = fminf(q[i], lp.lvv);
    }
    pack_chunk<HALF, BITS>(q, cp, pkd, over);
    chunk_fence();
  }
}

// Counters in LDS between the waves of a workgroup.  Everything these counters
// publish (keys, constants, tables) lives in LDS, and the LDS executes each wave's
// operations in order: a wave that sees another wave's increment also sees that
// wave's earlier LDS writes.  So the only ordering needed is the compiler's (and a
// wait for the wave's own LDS operations); a workgroup-scope fence would also wait for
// every outstanding global load and store of the wave, i.e. for the prefetched tiles.
__device__ __forceinline__ void lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Spin (the whole wave) until an LDS counter reaches `target`.  Bounded: after about
// half a second it gives up and returns false.
constexpr uint32_t kMaxLdsPolls = 1u << 22;
__device__ __forceinline__ bool lds_wait(uint32_t* ctr, uint32_t target) {
  bool ok = false;
  for (uint32_t polls = 0; polls < kMaxLdsPolls; ++polls) {
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
      ok = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  lds_order();
  return ok;
}
__device__ __forceinline__ void lds_signal(uint32_t* ctr) {
  lds_order();
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

}  // namespace
}  // namespace kvmi
