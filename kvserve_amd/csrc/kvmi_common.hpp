// Definitions shared by the paged codec kernels (register-FWHT and MFMA variants).
#pragma once

#include "kvmi_device.hpp"
#include "../../include/kvserve_amd.h"

namespace kvmi {

constexpr int kMaxHeads = 64;     // heads per worker shard (profile and finalize tables)
constexpr int kMaxRowSlots = 8192; // H * next_pow2(D): the generic row kernels' pass holds a whole token
constexpr int kMaxQuadH = 16;     // heads of the quad-per-row kernels' LDS tables
constexpr int kMaxQuadHD = kMaxQuadH * 128;

__host__ __device__ constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Quantization axis of a part (0 = K, 1 = V): the default is K per channel and V per
// token; the KVMI_F_* axis flags select the others.
enum Axis { kAxChannel = 0, kAxToken = 1, kAxTensor = 2 };
constexpr uint32_t kAxisFlags = KVMI_F_K_TOKEN | KVMI_F_K_TENSOR | KVMI_F_V_CHANNEL | KVMI_F_V_TENSOR;
// Internal (never part of a caller's geometry): head_dim 256 served by the D = 128 MFMA
// kernels as 2H "virtual heads" of 128 channels, virtual head 2h + b being half b of
// head h.  Pool rows, sign bits, K metadata and K keys have the same bytes in both
// views; the permuted stream and the profile are mapped (seg_addr, stage_profile), and
// the 256-point transform is rebuilt from the two 128-point ones by one butterfly.
constexpr uint32_t kPairedHeads = 1u << 30;
__host__ __device__ inline int part_axis(uint32_t flags, int part) {
  if (part == 0) return (flags & KVMI_F_K_TOKEN) ? kAxToken : (flags & KVMI_F_K_TENSOR) ? kAxTensor : kAxChannel;
  return (flags & KVMI_F_V_CHANNEL) ? kAxChannel : (flags & KVMI_F_V_TENSOR) ? kAxTensor : kAxToken;
}

// Launch geometry (kernel argument).
struct Geo {
  int S, H, D, bits;
  uint32_t flags;
  int G;
  int bpw;      // paged blocks per workgroup
  float scale;  // fp32 value of 1/sqrt(D)
};

struct Profile {  // decoded kvmi_layer_job::profile for one part
  const KVMI_GLOBAL uint8_t* order;
  const KVMI_GLOBAL uint8_t* levels;
  const KVMI_GLOBAL uint8_t* group;
};
__device__ __forceinline__ Profile part_profile(const uint8_t* p, int part, int H) {
  const KVMI_GLOBAL uint8_t* b = (const KVMI_GLOBAL uint8_t*)p + part * 3 * H;
  return Profile{b, b + H, b + 2 * H};
}

// Where row r (0-based, token-major) of a workgroup's block run lives.
struct RowPos {
  int64_t pool_row;  // row index in the pool part: physical block * S*H + within
  int tok;           // token index within the job (logical block * S + token in block)
  bool active;
};
__device__ __forceinline__ RowPos row_pos(const kvmi_layer_job& job, int blk0, int64_t rows, int64_t r, int S,
                                          int H) {
  RowPos p;
  p.active = r < rows;
  if (!p.active) {
    p.pool_row = 0;
    p.tok = 0;
    return p;
  }
  const int rpb = S * H;
  const int b = blk0 + (int)(r / rpb);
  const int within = (int)(r % rpb);
  p.pool_row = (int64_t)gld(job.block_ids + b) * rpb + within;
  p.tok = b * S + within / H;
  return p;
}

// Byte address of the packed symbols of (part, output head position j, token tok)
// starting at element e0 of the row, in the permuted [l,2,H',B,S,D] or native
// [l,2,B,S,H',D] symbol order.  Callers keep e0*BITS a multiple of 8.
// PAIRED: j is a paired virtual head (kPairedHeads); the permuted order is then
// [H/2][tokens][2 halves x D].
template <int BITS, bool PAIRED = false>
__device__ __forceinline__ uint8_t* seg_addr(const kvmi_layer_job& job, const Geo& g, int part, int j, int tok,
                                             int e0) {
  const int64_t D = g.D;
  const int64_t ntok = (int64_t)job.num_blocks * g.S;
  int64_t ts, hs, ps;
  if (g.flags & KVMI_F_NATIVE_LAYOUT) {  // the same bytes for paired virtual heads
    ts = (int64_t)g.H * D;
    hs = D;
    ps = ntok * g.H * D;
  } else if (PAIRED) {  // [H/2][tokens][2 halves x D]
    ts = 2 * D;
    ps = ntok * g.H * D;
    return job.stream + ((g.flags & KVMI_F_NO_HEADER) ? 0 : KVMI_HEADER_BYTES) +
           ((job.symbol_offset + part * ps + (j >> 1) * (2 * ntok * D) + (j & 1) * D + tok * ts + e0) * BITS) / 8;
  } else {
    ts = D;
    hs = ntok * D;
    ps = (int64_t)g.H * hs;
  }
  const int64_t sym = job.symbol_offset + part * ps + j * hs + tok * ts + e0;
  const int64_t base = (g.flags & KVMI_F_NO_HEADER) ? 0 : KVMI_HEADER_BYTES;
  return job.stream + base + (sym * BITS) / 8;
}

// The 16-byte header of a chunk stream (streams are 16-byte aligned).
__device__ __forceinline__ bool header_matches(const uint8_t* in, int bits, int64_t chunk_symbols) {
  const uint4 hw = gld(reinterpret_cast<const uint4*>(in));
  const uint64_t n = (uint64_t)chunk_symbols;
  return hw.x == KVMI_MAGIC && hw.y == (uint32_t)bits && hw.z == (uint32_t)(n & 0xffffffffu) &&
         hw.w == (uint32_t)(n >> 32);
}

__device__ __forceinline__ void write_stream_header(uint8_t* out, int bits, int64_t chunk_symbols) {
  uint32_t* o = reinterpret_cast<uint32_t*>(out);
  gst(o, (uint32_t)KVMI_MAGIC);
  gst(o + 1, (uint32_t)bits);
  gst(o + 2, (uint32_t)((uint64_t)chunk_symbols & 0xffffffffu));
  gst(o + 3, (uint32_t)((uint64_t)chunk_symbols >> 32));
}

// Host-side validation of a launch geometry; fills the kernel argument.
inline int check_geo(const kvmi_geometry* geom, int32_t num_jobs, int32_t max_blocks, Geo* out) {
  if (!geom || num_jobs < 0 || max_blocks < 0) return KVMI_EINVAL;
  const int S = geom->block_size, H = geom->num_heads, D = geom->head_dim, bits = geom->bits;
  if (S < 1 || H < 1 || H > kMaxHeads) return KVMI_EINVAL;
  // D even up to 256; below 16 or not a multiple of 16 its power-of-two chunks go below
  // one 16-channel lane (the row kernels' SM variants), and every packed row must then
  // still be whole bytes (D * bits a multiple of 8)
  if (D < 2 || D > 256 || D % 2 || H * next_pow2(D) > kMaxRowSlots) return KVMI_EINVAL;
  if (bits < 1 || bits > 8 || (D * bits) % 8) return KVMI_EINVAL;
  if (geom->max_groups < 1 || geom->max_groups > H) return KVMI_EINVAL;
  if ((geom->flags & KVMI_F_NO_HEADER) && bits != 8) return KVMI_EINVAL;
  if (geom->flags & ~(KVMI_F_NO_TRANSFORM | KVMI_F_NATIVE_LAYOUT | KVMI_F_NO_HEADER | KVMI_F_VALU_FWHT |
                      KVMI_F_CLAMP_LEVELS | KVMI_F_TWO_PASS | KVMI_F_ROW_FWHT | kAxisFlags))
    return KVMI_EINVAL;
  if ((geom->flags & KVMI_F_K_TOKEN) && (geom->flags & KVMI_F_K_TENSOR)) return KVMI_EINVAL;
  if ((geom->flags & KVMI_F_V_CHANNEL) && (geom->flags & KVMI_F_V_TENSOR)) return KVMI_EINVAL;
  out->S = S;
  out->H = H;
  out->D = D;
  out->bits = bits;
  out->flags = geom->flags;
  out->G = geom->max_groups;
  out->scale = (float)(1.0 / __builtin_sqrt((double)D));
  out->bpw = 1;
  return KVMI_OK;
}

// Kernel families, by geometry:
//  * MFMA (kvmi_mfma.hip): the transform profile with D in {64, 128}, H dividing 8
//    (or H = 16 or 32 with a power-of-two S, and 16-byte stream runs) and S*H a
//    multiple of 32, unless the caller forces the register FWHT (KVMI_F_VALU_FWHT);
//  * quad-per-row register FWHT (kvmi_codec.hip): D in {64, 128}, H dividing 128,
//    H <= 16;
//  * generic rows (kvmi_rows.hip): every other geometry check_geo admits (D even up
//    to 256 with whole-byte packed rows, split into power-of-two chunks when it is not
//    one, chunks below 16 channels included; H up to 64), every non-default
//    quantization axis, and any geometry when the caller forces them (KVMI_F_ROW_FWHT).
inline bool mfma_eligible(const Geo& g) {
  // The encoder writes each stream run (32/H tokens of one head) in 16-byte pieces, so
  // a run's packed bytes (32/H) * D * bits / 8 must be a multiple of 16: at 32 heads
  // that excludes D = 64 at odd widths (24-byte runs at 3 bits).
  const bool runs16 = ((32 / g.H) * g.D * g.bits / 8) % 16 == 0;
  const bool heads = (8 % g.H) == 0 || ((g.H == 16 || g.H == 32) && (g.S & (g.S - 1)) == 0 && runs16);
  return !(g.flags & (KVMI_F_VALU_FWHT | KVMI_F_ROW_FWHT | KVMI_F_NO_TRANSFORM | kAxisFlags)) &&
         (g.D == 64 || g.D == 128) && heads && ((g.S * g.H) % 32) == 0;
}
// head_dim 256 on the MFMA kernels (the transform profile, default axes, up to 16
// heads): fills *v with the virtual-head view (2H heads of 128, scale still 1/16).
inline bool paired_view(const Geo& g, Geo* v) {
  if (g.D != 256 || g.H > 16 || (g.flags & (KVMI_F_VALU_FWHT | KVMI_F_ROW_FWHT | KVMI_F_NO_TRANSFORM | kAxisFlags)))
    return false;
  Geo w = g;
  w.H = 2 * g.H;
  w.D = 128;
  w.flags |= kPairedHeads;
  if (!mfma_eligible(w)) return false;
  *v = w;
  return true;
}
inline bool quad_eligible(const Geo& g) {
  return !(g.flags & (KVMI_F_ROW_FWHT | kAxisFlags)) && (g.D == 64 || g.D == 128) && g.H <= kMaxQuadH &&
         (128 % g.H) == 0;
}
int rows_kstats(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);
int rows_encode(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);
int rows_decode(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);
int rows_hadamard(const void* in, void* out, int64_t rows, int32_t H, int32_t D, const uint32_t* signs,
                  int32_t inverse, hipStream_t st);
int mfma_kstats(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);
int mfma_encode(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);
int mfma_decode(const Geo& g, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st);

}  // namespace kvmi
