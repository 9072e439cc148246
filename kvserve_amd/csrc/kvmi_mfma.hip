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
// Work split: a workgroup of 4 wave64s owns a run of tokens of one (request, layer)
// job; a tile is 32 consecutive pool rows (32/H tokens x H heads, token-major, as
// the cache stores them), and wave w takes tiles w, w+4, ... of the run.  Because
// 32 % H == 0, lane l always holds head (l % 32) % H, and the H heads of a token sit
// in H neighbouring lanes of one wave.
#include "kvmi_common.hpp"

namespace kvmi {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMW = 256;  // threads per workgroup
constexpr int kWaves = kMW / 64;
constexpr int kTok = 32;  // tokens per tile (MFMA rows)

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
__device__ __forceinline__ uint4 hadamard_tile(int kt, bool orient_n, bool negate) {
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
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

__device__ __forceinline__ uint4 xor4(uint4 a, uint4 b) { return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w); }

// A bf16-pair constant held in an SGPR.  Left to itself the compiler encodes the
// pair (1.0, 0) = 0x00003F80 as the inline constant "1.0" of v_dot2c_f32_bf16, which
// the hardware reads as the f32 1.0 = 0x3F800000, i.e. the pair (0, 1.0).  The asm
// is not volatile, so the value is materialised once and shared.
__device__ __forceinline__ bf16x2v sgpr_pair(uint32_t v) {
  asm("" : "+s"(v));
  return __builtin_bit_cast(bf16x2v, v);
}

// RN(lo(bf16 pair) + c) and RN(hi(bf16 pair) + c): v_dot2_f32_bf16 against (1, 0) /
// (0, 1) is exactly one fp32 rounding of the sum (checked on gfx950 hardware).
__device__ __forceinline__ float add_lo(uint32_t pk, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pk), sgpr_pair(0x00003F80u), c, false);
}
__device__ __forceinline__ float add_hi(uint32_t pk, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pk), sgpr_pair(0x3F800000u), c, false);
}

// Rounded-to-nearest-even integer in [0, 255] of a float, as one byte of `acc`
// (v_cvt_pk_u8_f32 rounds half to even and saturates, checked on gfx950).
template <int BYTE>
__device__ __forceinline__ uint32_t cvt_u8(float x, uint32_t acc) {
  return __builtin_amdgcn_cvt_pk_u8_f32(x, BYTE, acc);
}

// Symbols of an element pair (y0, y1) given per-element (mn, rcp):
//   t = bf16(y - mn); q = bf16(t * rcp); sym = clamp(rint(q), 0, L)
// with y rounded to bf16 first.  Returns the two rounded q values (fp32).
__device__ __forceinline__ void quant_pair(float y0, float y1, float mn0, float mn1, float rcp0, float rcp1,
                                           float& q0, float& q1) {
  const uint32_t ypk = pack_bf16x2(y0, y1);
  const uint32_t tpk = pack_bf16x2(add_lo(ypk, -mn0), add_hi(ypk, -mn1));
  const uint32_t qpk = pack_bf16x2(bf_lo(tpk) * rcp0, bf_hi(tpk) * rcp1);
  q0 = bf_lo(qpk);
  q1 = bf_hi(qpk);
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
        uint4 t = q[i];
        w[4 * i] = t.x;
        w[4 * i + 1] = t.y;
        w[4 * i + 2] = t.z;
        w[4 * i + 3] = t.w;
      }
    } else if constexpr (kBytes % 8 == 0) {
      const uint2* q = reinterpret_cast<const uint2*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 8; ++i) {
        uint2 t = q[i];
        w[2 * i] = t.x;
        w[2 * i + 1] = t.y;
      }
    } else {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
      for (int i = 0; i < kBytes / 4; ++i) w[i] = q[i];
    }
    if constexpr (kWords * 4 > kBytes) w[kWords - 1] &= 0xffffffffu >> (32 - 8 * (kBytes % 4));
  }
};

// Shared per-workgroup tables.
struct Tables {
  uint32_t smask[kMaxH][64 + 4];  // bf16 sign-flip masks per (head, element pair), padded rows
  float2 kc[kMaxH][128 + 4];      // K (min, 1/scale) [encode] or (min, scale) [decode], by source head
  int posk[kMaxH], posv[kMaxH], gfirst[kMaxH];
};

// Fill the sign-mask table: word p of head h flips elements 2p and 2p+1.
__device__ __forceinline__ void fill_signs(Tables& T, const uint32_t* signs, int H, int D, bool transform) {
  for (int i = threadIdx.x; i < H * (D / 2); i += kMW) {
    const int h = i / (D / 2), p = i % (D / 2);
    uint32_t m = 0;
    if (transform) {
      const uint32_t s = signs[h * (D / 32) + (2 * p) / 32] >> ((2 * p) & 31);
      m = ((s & 1u) << 15) | ((s & 2u) << 30);
    }
    T.smask[h][p] = m;
  }
}

__device__ __forceinline__ void fill_positions(Tables& T, const Profile& pk, const Profile& pv, int H) {
  if (threadIdx.x < (unsigned)H) {
    const int h = threadIdx.x;
    for (int k = 0; k < H; ++k) {
      if (pk.order[k] == h) T.posk[h] = k;
      if (pv.order[k] == h) T.posv[h] = k;
    }
    // first output position of V group h (if any) -> its source head
    T.gfirst[h] = -1;
    for (int k = H - 1; k >= 0; --k)
      if (pv.group[k] == h) T.gfirst[h] = pv.order[k];
  }
}

// Tile coordinates: row r of tile t of the workgroup's run.
struct Tile {
  int h;           // source head (fixed per lane: r % H)
  int tok;         // token (within the job) of this lane's row
  bool active;     // row exists
  int64_t row;     // pool row index (block * S*H + t_in_block*H + h)
};
// tok_end = end of this workgroup's token run (never past the request).
__device__ __forceinline__ Tile tile_row(const kvmi_layer_job& job, int S, int H, int tok0, int tok_end, int t, int r) {
  Tile x;
  const int R = t * kTok + r;  // row within the run
  x.h = R % H;
  x.tok = tok0 + R / H;
  x.active = x.tok < tok_end;
  x.row = 0;
  if (x.active) {
    const int b = x.tok / S;
    x.row = ((int64_t)job.block_ids[b] * S + (x.tok % S)) * H + x.h;
  }
  return x;
}

// Load (and sign) the lane's half-row of bf16 inputs.
template <int NC>
__device__ __forceinline__ void load_half_row(const uint16_t* __restrict__ pool, const Tile& tl, int hl,
                                              const Tables& T, uint4 (&x)[2 * NC]) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  if (tl.active) {
    const uint4* src = reinterpret_cast<const uint4*>(pool + tl.row * D + HALF * hl);
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) x[u] = src[u];
  } else {
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) x[u] = make_uint4(0, 0, 0, 0);
  }
  const int off = opaque(tl.h * (64 + 4) + (HALF / 2) * hl);
  const uint4* sm = reinterpret_cast<const uint4*>(&T.smask[0][0] + off);
#pragma unroll
  for (int u = 0; u < 2 * NC; ++u) x[u] = xor4(x[u], sm[u]);
}

// Forward / inverse transform, orientation T, output chunk cp (unscaled fp32).
template <int NC>
__device__ __forceinline__ f32x16 transform_T(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                              int cp) {
  f32x16 acc = {};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const bool neg = __builtin_popcount(c & cp) & 1;
    acc = mfma(neg ? hn[0] : hp[0], x[2 * c], acc);
    acc = mfma(neg ? hn[1] : hp[1], x[2 * c + 1], acc);
  }
  return acc;
}

// ============================================================== K statistics (orientation N)
template <int NC>
__global__ __launch_bounds__(kMW) void kstats_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                          int32_t* __restrict__ err) {
  constexpr int D = 32 * NC;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H;
  const int ntok = job.num_blocks * S;
  const int run = g.bpw * S;  // tokens per workgroup (multiple of 32)
  const int nwg = (ntok + run - 1) / run;
  if ((int)blockIdx.x >= nwg) return;
  const int tok0 = blockIdx.x * run;
  const int tok_end = min(ntok, tok0 + run);
  const int tiles = ((tok_end - tok0) * H + kTok - 1) / kTok;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
  const bool transform = true;  // MFMA kernels serve the transform profile only

  __shared__ Tables T;
  __shared__ uint32_t lkey[2 * kMaxHD];
  __shared__ int last;
  fill_signs(T, job.signs, H, D, transform);
  for (int i = threadIdx.x; i < H * D; i += kMW) {
    lkey[i] = 0xffffffffu;
    lkey[H * D + i] = 0u;
  }
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, true, false);
  hp[1] = hadamard_tile(1, true, false);
  hn[0] = hadamard_tile(0, true, true);
  hn[1] = hadamard_tile(1, true, true);
  // Output register i of chunk c holds row m = 8*(i/4) + 4*hl + i%4 of the tile and
  // channel f(r, c) = HALF*(r>>4) + 16*c + (r & 15); row m has head m % H, which
  // depends only on s = i%4 (32 % H == 0 and H <= 8).  Running min/max per (s, c).
  float mn[4][NC], mx[4][NC];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      mn[a][c] = __builtin_inff();
      mx[a][c] = -__builtin_inff();
    }
  const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool);
  for (int t = wave; t < tiles; t += kWaves) {
    const Tile tl = tile_row(job, S, H, tok0, tok_end, t, r);
    uint4 x[2 * NC];
    load_half_row<NC>(pool, tl, hl, T, x);
    const int valid = min(kTok, (tok_end - tok0) * H - t * kTok);  // rows of this tile that exist
#pragma unroll
    for (int cp = 0; cp < NC; ++cp) {
      f32x16 acc = {};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const bool neg = __builtin_popcount(c & cp) & 1;
        acc = mfma(x[2 * c], neg ? hn[0] : hp[0], acc);
        acc = mfma(x[2 * c + 1], neg ? hn[1] : hp[1], acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i / 4) + 4 * hl + (i % 4);
        if (m < valid) {
          mn[i % 4][cp] = fminf(mn[i % 4][cp], acc[i]);
          mx[i % 4][cp] = fmaxf(mx[i % 4][cp], acc[i]);
        }
      }
      chunk_fence();
    }
  }
  // Push per (head, channel): scaling by 1/sqrt(D) > 0 is monotone, so it commutes
  // with min / max (and so does the bf16 rounding applied by the finaliser).
  const int HD = H * D;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int h = (4 * hl + a) % H;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int f = (16 * NC) * (r >> 4) + 16 * c + (r & 15);
      const float smn = mn[a][c] * g.scale;
      const float smx = mx[a][c] * g.scale;
      if (smn <= smx) {  // at least one row of this head went through the slot
        atomicMin(&lkey[h * D + f], f2key(smn));
        atomicMax(&lkey[HD + h * D + f], f2key(smx));
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kMW) {
    if (lkey[i] != 0xffffffffu) atomicMin(&job.kstats[i], lkey[i]);
    if (lkey[HD + i] != 0u) atomicMax(&job.kstats[HD + i], lkey[HD + i]);
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = (atomicAdd(job.counter, 1u) == (unsigned)(nwg - 1)) ? 1 : 0;
  __syncthreads();
  if (!last) return;
  __threadfence();
  const Profile pk = part_profile(job.profile, 0, H);
  for (int i = threadIdx.x; i < HD; i += kMW) {
    const float kmn = round_bf16(key2f(__hip_atomic_exchange(&job.kstats[i], 0xffffffffu, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)));
    const float kmx =
        round_bf16(key2f(__hip_atomic_exchange(&job.kstats[HD + i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
    const int hs = i / D, e = i % D;
    int j = 0;
    for (int k = 0; k < H; ++k)
      if (pk.order[k] == hs) j = k;
    const float sc = quant_scale(kmn, kmx, pk.levels[j]);
    job.kmeta[j * D + e] = (uint16_t)f32_to_bf16_bits(kmn);
    job.kmeta[HD + j * D + e] = (uint16_t)f32_to_bf16_bits(sc);
  }
  if (threadIdx.x == 0) __hip_atomic_exchange(job.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Quantize and pack one lane's output half-row (HALF = 16*NC values in NC chunks of
// 16) computed on the fly by transform_T.  KQ: per-element (min, 1/scale) from the
// LDS table; otherwise one (mn, rcp) for the whole row.
template <int NC, int BITS, bool CLAMP, bool KQ>
__device__ __forceinline__ uint32_t quantize_half_row(const uint4 (&x)[2 * NC], const uint4 (&hp)[2],
                                                      const uint4 (&hn)[2], float scale, const float2* kq_row,
                                                      float mn, float rcp, float lv, LanePack<16 * NC, BITS>& pk) {
  pk.clear();
  uint32_t over = 0;
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    float y[16];
    const f32x16 acc = transform_T<NC>(x, hp, hn, cp);
#pragma unroll
    for (int i = 0; i < 16; ++i) y[i] = acc[i] * scale;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      float m0 = mn, m1 = mn, r0 = rcp, r1 = rcp;
      if (KQ) {
        const float4 c = *reinterpret_cast<const float4*>(&kq_row[16 * cp + i]);
        m0 = c.x;
        r0 = c.y;
        m1 = c.z;
        r1 = c.w;
      }
      float q0, q1;
      quant_pair(y[i], y[i + 1], m0, m1, r0, r1, q0, q1);
      if (CLAMP) {
        q0 = fminf(q0, lv);
        q1 = fminf(q1, lv);
      }
      const uint32_t s0 = cvt_u8<0>(q0, 0u), s1 = cvt_u8<0>(q1, 0u);
      over |= s0 | s1;
      pk.put(16 * cp + i, s0);
      pk.put(16 * cp + i + 1, s1);
    }
    chunk_fence();
  }
  return over;
}

// ============================================================== encode (orientation T)
template <int NC, int BITS, bool CLAMP>
__global__ __launch_bounds__(kMW) void encode_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                          int32_t* __restrict__ err) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int ntok = job.num_blocks * S;
  const int run = g.bpw * S;
  const int nwg = (ntok + run - 1) / run;
  if ((int)blockIdx.x >= nwg) return;
  const int tok0 = blockIdx.x * run;
  const int tok_end = min(ntok, tok0 + run);
  const int tiles = ((tok_end - tok0) * H + kTok - 1) / kTok;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
  const bool transform = true;  // MFMA kernels serve the transform profile only
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);

  __shared__ Tables T;
  fill_signs(T, job.signs, H, D, transform);
  fill_positions(T, pk, pv, H);
  if (threadIdx.x == 0 && job.write_header && blockIdx.x == 0 && !(g.flags & KVMI_F_NO_HEADER))
    write_stream_header(job.stream, BITS, job.chunk_symbols);
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kMW) {
    const int hs = i / D, e = i % D, j = T.posk[hs];
    const float m = bf16_to_f32(job.kmeta[j * D + e]);
    const float sc = bf16_to_f32(job.kmeta[HD + j * D + e]);
    T.kc[hs][e] = make_float2(m, 1.0f / sc);
  }
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, false, false);
  hp[1] = hadamard_tile(1, false, false);
  hn[0] = hadamard_tile(0, false, true);
  hn[1] = hadamard_tile(1, false, true);
  const uint16_t* poolK = reinterpret_cast<const uint16_t*>(job.pool);
  const uint16_t* poolV = poolK + job.pool_part_stride;
  uint32_t over = 0;

  // V statistic groups of this lane's head and of the H heads of its token
  const int hme = r % H;
  const int jk = T.posk[hme], jv = T.posv[hme];
  const int gv = pv.group[jv];
  const float lvk = (float)pk.levels[jk], lvv = (float)pv.levels[jv];
  const bool rep_lane = hl == 0 && T.gfirst[gv] == hme;  // writes the V metadata of (group, token)
  for (int t = wave; t < tiles; t += kWaves) {
    const Tile tl = tile_row(job, S, H, tok0, tok_end, t, r);
    // ---------------- K: per-channel statistics from the kstats pass
    {
      uint4 x[2 * NC];
      load_half_row<NC>(poolK, tl, hl, T, x);
      LanePack<HALF, BITS> pkd;
      const float2* kq_row = &T.kc[0][0] + opaque(hme * (128 + 4) + HALF * hl);
      over |= quantize_half_row<NC, BITS, CLAMP, true>(x, hp, hn, g.scale, kq_row, 0.f, 0.f, lvk, pkd);
      if (tl.active) pkd.store(seg_addr<BITS>(job, g, 0, jk, tl.tok, HALF * hl));
    }
    chunk_fence();
    // ---------------- V: per-token statistics over the heads of a group
    uint4 x[2 * NC];
    load_half_row<NC>(poolV, tl, hl, T, x);
    uint32_t ypk[HALF / 2];
    float lmn = __builtin_inff(), lmx = -__builtin_inff();
#pragma unroll
    for (int cp = 0; cp < NC; ++cp) {
      float y[16];
      const f32x16 acc = transform_T<NC>(x, hp, hn, cp);
#pragma unroll
      for (int i = 0; i < 16; ++i) y[i] = acc[i] * g.scale;
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const uint32_t p = pack_bf16x2(y[i], y[i + 1]);
        ypk[(16 * cp + i) / 2] = p;
        lmn = fminf(lmn, fminf(bf_lo(p), bf_hi(p)));
        lmx = fmaxf(lmx, fmaxf(bf_lo(p), bf_hi(p)));
      }
      chunk_fence();
    }
    // whole row, then the heads of this token that share the group: lanes
    // (r / H) * H .. + H - 1 of this half hold the token's H heads
    lmn = fminf(lmn, __shfl_xor(lmn, 32));
    lmx = fmaxf(lmx, __shfl_xor(lmx, 32));
    float mn = __builtin_inff(), mx = -__builtin_inff();
    for (int gg = 0; gg < G; ++gg) {
      float a = gv == gg ? lmn : __builtin_inff();
      float b = gv == gg ? lmx : -__builtin_inff();
      for (int step = 1; step < H; step <<= 1) {
        a = fminf(a, __shfl_xor(a, step));
        b = fmaxf(b, __shfl_xor(b, step));
      }
      if (gv == gg) {
        mn = a;
        mx = b;
      }
    }
    const float sc = quant_scale(mn, mx, pv.levels[jv]);
    const float rcp = 1.0f / sc;
    if (tl.active && rep_lane) {
      job.vmeta[(int64_t)gv * ntok + tl.tok] = (uint16_t)f32_to_bf16_bits(mn);
      job.vmeta[(int64_t)(G + gv) * ntok + tl.tok] = (uint16_t)f32_to_bf16_bits(sc);
    }
    LanePack<HALF, BITS> pkd;
    pkd.clear();
#pragma unroll
    for (int i = 0; i < HALF; i += 2) {
      const uint32_t p = ypk[i / 2];
      const uint32_t tpk = pack_bf16x2(add_lo(p, -mn), add_hi(p, -mn));
      const uint32_t qpk = pack_bf16x2(bf_lo(tpk) * rcp, bf_hi(tpk) * rcp);
      float q0 = bf_lo(qpk), q1 = bf_hi(qpk);
      if (CLAMP) {
        q0 = fminf(q0, lvv);
        q1 = fminf(q1, lvv);
      }
      const uint32_t s0 = cvt_u8<0>(q0, 0u), s1 = cvt_u8<0>(q1, 0u);
      over |= s0 | s1;
      pkd.put(i, s0);
      pkd.put(i + 1, s1);
    }
    if (tl.active) pkd.store(seg_addr<BITS>(job, g, 1, jv, tl.tok, HALF * hl));
  }
  if (over >> BITS) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
}

// ============================================================== decode (orientation T)
template <int NC, int BITS>
__global__ __launch_bounds__(kMW) void decode_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                          int32_t* __restrict__ err) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int ntok = job.num_blocks * S;
  const int run = g.bpw * S;
  const int nwg = (ntok + run - 1) / run;
  if ((int)blockIdx.x >= nwg) return;
  const int tok0 = blockIdx.x * run;
  const int tok_end = min(ntok, tok0 + run);
  const int tiles = ((tok_end - tok0) * H + kTok - 1) / kTok;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
  const bool transform = true;  // MFMA kernels serve the transform profile only
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);

  __shared__ Tables T;
  __shared__ int ok;
  if (threadIdx.x == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  fill_signs(T, job.signs, H, D, transform);
  fill_positions(T, pk, pv, H);
  __syncthreads();
  if (!ok) return;
  for (int i = threadIdx.x; i < HD; i += kMW) {
    const int hs = i / D, e = i % D, j = T.posk[hs];
    T.kc[hs][e] = make_float2(bf16_to_f32(job.kmeta[j * D + e]), bf16_to_f32(job.kmeta[HD + j * D + e]));
  }
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, false, false);
  hp[1] = hadamard_tile(1, false, false);
  hn[0] = hadamard_tile(0, false, true);
  hn[1] = hadamard_tile(1, false, true);
  uint16_t* poolK = reinterpret_cast<uint16_t*>(job.pool);
  uint16_t* poolV = poolK + job.pool_part_stride;

  for (int t2 = wave; t2 < 2 * tiles; t2 += kWaves) {
    const int part = t2 / tiles, t = t2 % tiles;
    const Tile tl = tile_row(job, S, H, tok0, tok_end, t, r);
    const int j = part ? T.posv[tl.h] : T.posk[tl.h];
    // every lane takes part in the MFMAs (rows are independent columns of B);
    // rows past the run end decode zero symbols and are not stored
    LanePack<HALF, BITS> pkd;
    pkd.clear();
    if (tl.active) pkd.load(seg_addr<BITS>(job, g, part, j, tl.tok, HALF * hl));
    float vmn = 0.f, vsc = 0.f;
    if (part && tl.active) {
      const int gv = pv.group[j];
      vmn = bf16_to_f32(job.vmeta[(int64_t)gv * ntok + tl.tok]);
      vsc = bf16_to_f32(job.vmeta[(int64_t)(G + gv) * ntok + tl.tok]);
    }
    const float2* kd = &T.kc[0][0] + opaque(tl.h * (128 + 4) + HALF * hl);
    // dequantize into bf16 MFMA operands: x~ = bf16(bf16(q * scale) + min)
    uint4 x[2 * NC];
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) {
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int e = 8 * u + 2 * p;
        float m0 = vmn, m1 = vmn, s0 = vsc, s1 = vsc;
        if (!part) {
          const float4 c = *reinterpret_cast<const float4*>(&kd[e]);
          m0 = c.x;
          s0 = c.y;
          m1 = c.z;
          s1 = c.w;
        }
        const uint32_t spk = pack_bf16x2((float)pkd.get(e) * s0, (float)pkd.get(e + 1) * s1);
        w[p] = pack_bf16x2(add_lo(spk, m0), add_hi(spk, m1));
      }
      x[u] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    chunk_fence();
    uint16_t* dst = (part ? poolV : poolK) + tl.row * D + HALF * hl;
    const uint4* sm = reinterpret_cast<const uint4*>(&T.smask[0][0] + opaque(tl.h * (64 + 4) + (HALF / 2) * hl));
    {
#pragma unroll
      for (int cp = 0; cp < NC; ++cp) {
        const f32x16 acc = transform_T<NC>(x, hp, hn, cp);
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = pack_bf16x2(acc[2 * i] * g.scale, acc[2 * i + 1] * g.scale);
        const uint4 a = xor4(make_uint4(w[0], w[1], w[2], w[3]), sm[2 * cp]);
        const uint4 b = xor4(make_uint4(w[4], w[5], w[6], w[7]), sm[2 * cp + 1]);
        if (tl.active) {
          reinterpret_cast<uint4*>(dst)[2 * cp] = a;
          reinterpret_cast<uint4*>(dst)[2 * cp + 1] = b;
        }
        chunk_fence();
      }
    }
  }
}

// ============================================================== launch
// Tokens per workgroup: whole 32-token groups and whole blocks.
int mfma_run_blocks(const Geo& g, int32_t max_blocks, int target_wgs_per_job) {
  // blocks per workgroup: a multiple of the blocks that make up 32 tokens
  const int unit = (kTok + g.S - 1) / g.S;  // S divides 32 or 32 divides S*? (S*H % 32 == 0 checked)
  int bpw = unit;
  if (target_wgs_per_job > 0) {
    const int want = (max_blocks + target_wgs_per_job - 1) / target_wgs_per_job;
    bpw = ((want + unit - 1) / unit) * unit;
    if (bpw < unit) bpw = unit;
  }
  return bpw;
}

template <int NC, int BITS>
void launch_enc(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  if (g.flags & KVMI_F_CLAMP_LEVELS)
    hipLaunchKernelGGL((encode_mfma_kernel<NC, BITS, true>), grid, dim3(kMW), 0, st, g, jobs, err);
  else
    hipLaunchKernelGGL((encode_mfma_kernel<NC, BITS, false>), grid, dim3(kMW), 0, st, g, jobs, err);
}
template <int NC, int BITS>
void launch_dec(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  hipLaunchKernelGGL((decode_mfma_kernel<NC, BITS>), grid, dim3(kMW), 0, st, g, jobs, err);
}

#define KVMI_MFMA_BITS(FN, NC, g, grid, jobs, err, st) \
  switch ((g).bits) {                                  \
    case 1: FN<NC, 1>(g, grid, jobs, err, st); break;  \
    case 2: FN<NC, 2>(g, grid, jobs, err, st); break;  \
    case 3: FN<NC, 3>(g, grid, jobs, err, st); break;  \
    case 4: FN<NC, 4>(g, grid, jobs, err, st); break;  \
    case 5: FN<NC, 5>(g, grid, jobs, err, st); break;  \
    case 6: FN<NC, 6>(g, grid, jobs, err, st); break;  \
    case 7: FN<NC, 7>(g, grid, jobs, err, st); break;  \
    default: FN<NC, 8>(g, grid, jobs, err, st); break; \
  }

}  // namespace

int mfma_kstats(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st) {
  Geo g = g0;
  g.bpw = mfma_run_blocks(g, max_blocks, 8);  // <= ~8 workgroups per job: few global atomics
  const int ntok = max_blocks * g.S, run = g.bpw * g.S;
  dim3 grid((unsigned)((ntok + run - 1) / run), (unsigned)num_jobs);
  if (g.D == 64)
    hipLaunchKernelGGL((kstats_mfma_kernel<2>), grid, dim3(kMW), 0, st, g, jobs, err);
  else
    hipLaunchKernelGGL((kstats_mfma_kernel<4>), grid, dim3(kMW), 0, st, g, jobs, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int mfma_encode(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st) {
  Geo g = g0;
  g.bpw = mfma_run_blocks(g, max_blocks, 0);
  const int ntok = max_blocks * g.S, run = g.bpw * g.S;
  dim3 grid((unsigned)((ntok + run - 1) / run), (unsigned)num_jobs);
  if (g.D == 64) {
    KVMI_MFMA_BITS(launch_enc, 2, g, grid, jobs, err, st)
  } else {
    KVMI_MFMA_BITS(launch_enc, 4, g, grid, jobs, err, st)
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int mfma_decode(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st) {
  Geo g = g0;
  g.bpw = mfma_run_blocks(g, max_blocks, 0);
  const int ntok = max_blocks * g.S, run = g.bpw * g.S;
  dim3 grid((unsigned)((ntok + run - 1) / run), (unsigned)num_jobs);
  if (g.D == 64) {
    KVMI_MFMA_BITS(launch_dec, 2, g, grid, jobs, err, st)
  } else {
    KVMI_MFMA_BITS(launch_dec, 4, g, grid, jobs, err, st)
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

}  // namespace kvmi
