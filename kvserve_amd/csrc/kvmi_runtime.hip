// Fixed-profile runtime numerics (kvserve_v1/compression/runtime/pipeline.py:264-804,
// runtime/csrc/kvs_compress.cu) on gfx950 -- a second numerics mode next to the
// modular profile of kvmi_mfma.hip / kvmi_codec.hip:
//
//   transform   y = rn(FWHT_bf16(x * s) * D^-1/2), every butterfly stage rounded to
//               bf16 (torch.add / torch.sub on bf16, pipeline.py:309-338), stages in
//               increasing index-bit order
//   params      min, max of the section (axis channel / token / tensor);
//               scale = rn(rn(max(rn(max - min), 1e-5)) / (L - 1)), inverse = rn(1 / scale)
//   quantize    q = clamp(rint(rn(rn(y - min) * inverse)), 0, L - 1)     (pipeline.py:414-466)
//   dequantize  y~ = rn(rn(q * scale) + min)                            (pipeline.py:652-684)
//   inverse     x~ = rn(FWHT_bf16(y~) * D^-1/2) * s, scattered to the cache (:686-703)
//
// Cache: per layer an HND view [blocks, heads, kernel_tokens, channels] (the KV part
// is a channel window of it).  Canonical rows [block, token] x [H, D] in output-head
// order; one workgroup per (layer, row), one 64-lane slice per head row.
#include "kvmi_device.hpp"
#include "../../include/kvserve_amd.h"

namespace kvmi {
namespace {

static_assert(sizeof(kvmi_rt_geometry) == 32 && sizeof(kvmi_rt_section) == 32 && sizeof(kvmi_rt_layer) == 136,
              "kvmi_rt_* layouts are part of the C-ABI");

constexpr int kRtThreads = 256;
constexpr int kRtWaves = kRtThreads / 64;

__device__ __forceinline__ float rn(float x) { return round_bf16(x); }

__device__ __forceinline__ float ld_bf16(const uint16_t* p) { return bf16_to_f32(gld(p)); }
__device__ __forceinline__ void st_bf16(uint16_t* p, float v) { gst(p, (uint16_t)f32_to_bf16_bits(v)); }

// Normalized FWHT of one head row held as EPL values per lane (element lane*EPL + k),
// or one value per lane when D < 64 (element lane % D).  Every stage rounds to bf16.
template <int D>
__device__ __forceinline__ void fwht_bf16(float (&v)[D >= 64 ? D / 64 : 1], uint32_t lane, float scale) {
  constexpr int EPL = D >= 64 ? D / 64 : 1;
  constexpr int LB = D >= 64 ? 64 : D;  // lanes per row
#pragma unroll
  for (int m = 1; m < EPL; m <<= 1) {
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      if (k & m) continue;
      const float a = v[k], b = v[k | m];
      v[k] = rn(a + b);
      v[k | m] = rn(a - b);
    }
  }
#pragma unroll
  for (int m = 1; m < LB; m <<= 1) {
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const float o = __shfl_xor(v[k], m, 64);
      v[k] = rn((lane & m) ? o - v[k] : v[k] + o);
    }
  }
#pragma unroll
  for (int k = 0; k < EPL; ++k) v[k] = rn(v[k] * scale);
}

struct RtIdx {
  uint32_t layer;
  uint64_t row;  // canonical row = physical block * kernel_tokens + token
  uint64_t blk;  // index into block_ids
  uint32_t tok;
};

// rows * layers <= 2^31 (checked on the host): 32-bit index arithmetic throughout
__device__ __forceinline__ RtIdx rt_idx(uint64_t rows) {
  RtIdx r;
  const uint32_t n = (uint32_t)rows;
  r.layer = blockIdx.x / n;
  r.row = blockIdx.x - r.layer * n;
  return r;
}

// ------------------------------------------------------------------ transform
// gather (head order) * signs -> [FWHT] -> canonical bf16 rows.  to_packed: into the
// payload at each layer's u8_offset (elements); else into the compact scratch, layer l
// at dst + l * rows * H * D.
template <int D>
__global__ __launch_bounds__(kRtThreads) void rt_transform_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                                  const int64_t* __restrict__ block_ids, uint64_t rows,
                                                                  uint16_t* __restrict__ dst, bool to_packed,
                                                                  float scale) {
  constexpr int EPL = D >= 64 ? D / 64 : 1;
  constexpr int HPW = D >= 64 ? 1 : 64 / D;  // head rows per wave pass
  const RtIdx ix = rt_idx(rows);
  const kvmi_rt_layer L = layers[ix.layer];
  const uint32_t blk = (uint32_t)ix.row / (uint32_t)g.kernel_tokens;
  const uint32_t tok = (uint32_t)ix.row - blk * (uint32_t)g.kernel_tokens;
  const int64_t pb = gld(block_ids + blk);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint16_t* cache = static_cast<const uint16_t*>(L.cache);
  const uint16_t* signs = static_cast<const uint16_t*>(L.signs);
  const uint64_t cols = (uint64_t)g.num_heads * D;
  uint16_t* out = to_packed ? dst + L.u8_offset + ix.row * cols : dst + ((uint64_t)ix.layer * rows + ix.row) * cols;
  for (int h0 = (int)wave * HPW; h0 < g.num_heads; h0 += kRtWaves * HPW) {
    const int h = h0 + (D >= 64 ? 0 : (int)(lane / D));
    const bool live = h < g.num_heads && (D >= 64 || lane < (uint32_t)(HPW * D));
    const int hc = live ? gld(L.head_order + h) : 0;
    const uint16_t* src = cache + pb * L.block_stride + (int64_t)hc * L.head_stride + (int64_t)tok * L.token_stride +
                          L.channel_offset;
    float v[EPL];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
      float x = live ? ld_bf16(src + d) : 0.0f;
      if (signs && live) x = rn(x * ld_bf16(signs + (int64_t)h * D + d));
      v[k] = x;
    }
    if (g.flags & KVMI_RT_TRANSFORM) fwht_bf16<D>(v, lane, scale);
    if (live) {
#pragma unroll
      for (int k = 0; k < EPL; ++k) {
        const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
        st_bf16(out + (int64_t)h * D + d, v[k]);
      }
    }
  }
}

// ------------------------------------------------------------------ parameters
struct QP {
  float mn, mx, scale, inv;
};

__device__ __forceinline__ QP quant_params(float mn, float mx, int levels) {
  QP p;
  p.mn = rn(mn);
  p.mx = rn(mx);
  float raw = rn(p.mx - p.mn);
  if (raw < 1e-5f) raw = rn(1e-5f);
  p.scale = rn(raw / (float)(levels - 1));
  p.inv = rn(1.0f / p.scale);
  return p;
}

// aux arena: section minima / scales at their offsets; the second half holds the
// maxima / inverses at the same offsets (the reference's temporary region).
__device__ __forceinline__ void put_params(uint8_t* aux, uint64_t half, const kvmi_rt_section& s, uint64_t i,
                                           const QP& p) {
  st_bf16(reinterpret_cast<uint16_t*>(aux + s.aux_min_offset) + i, p.mn);
  st_bf16(reinterpret_cast<uint16_t*>(aux + s.aux_scale_offset) + i, p.scale);
  st_bf16(reinterpret_cast<uint16_t*>(aux + half + s.aux_min_offset) + i, p.mx);
  st_bf16(reinterpret_cast<uint16_t*>(aux + half + s.aux_scale_offset) + i, p.inv);
}

// channel axis: one thread per (layer, section column), looping over the rows
__global__ __launch_bounds__(kRtThreads) void rt_params_channel_kernel(kvmi_rt_geometry g,
                                                                       const kvmi_rt_layer* __restrict__ layers,
                                                                       uint64_t rows, const uint16_t* __restrict__ canon,
                                                                       uint8_t* __restrict__ aux, uint64_t half) {
  const uint32_t cols = (uint32_t)g.num_heads * (uint32_t)g.head_dim;
  const uint32_t per_layer = (cols + kRtThreads - 1) / kRtThreads;
  const uint32_t layer = blockIdx.x / per_layer;
  const uint32_t c = (blockIdx.x % per_layer) * kRtThreads + threadIdx.x;
  if (c >= cols) return;
  const kvmi_rt_layer L = layers[layer];
  const int h = (int)(c / (uint32_t)g.head_dim);
#pragma unroll
  for (int si = 0; si < 2; ++si) {
    if (si >= L.num_sections) break;
    const kvmi_rt_section s = si ? L.sections[1] : L.sections[0];
    if (s.axis != 0 || h < s.head_start || h >= s.head_start + s.head_count) continue;
    const uint16_t* base = canon + (uint64_t)layer * rows * cols + c;
    float mn = INFINITY, mx = -INFINITY;
    for (uint64_t r = 0; r < rows; ++r) {
      const float v = ld_bf16(base + r * cols);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    put_params(aux, half, s, c - (uint32_t)s.head_start * (uint32_t)g.head_dim, quant_params(mn, mx, s.levels));
  }
}

// token axis: one wave per (layer, row) and section
__global__ __launch_bounds__(64) void rt_params_token_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                             uint64_t rows, const uint16_t* __restrict__ canon,
                                                             uint8_t* __restrict__ aux, uint64_t half) {
  const RtIdx ix = rt_idx(rows);
  const kvmi_rt_layer L = layers[ix.layer];
  const uint32_t lane = threadIdx.x;
  const uint32_t cols = (uint32_t)g.num_heads * (uint32_t)g.head_dim;
  const uint16_t* row = canon + ((uint64_t)ix.layer * rows + ix.row) * cols;
#pragma unroll
  for (int si = 0; si < 2; ++si) {
    if (si >= L.num_sections) break;
    const kvmi_rt_section s = si ? L.sections[1] : L.sections[0];
    if (s.axis != 1) continue;
    float mn = INFINITY, mx = -INFINITY;
    const uint32_t c0 = (uint32_t)s.head_start * g.head_dim, c1 = c0 + (uint32_t)s.head_count * g.head_dim;
    for (uint32_t c = c0 + lane; c < c1; c += 64) {
      const float v = ld_bf16(row + c);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      mn = fminf(mn, __shfl_xor(mn, o, 64));
      mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if (lane == 0) put_params(aux, half, s, ix.row, quant_params(mn, mx, s.levels));
  }
}

// tensor axis: one workgroup per (layer, section)
__global__ __launch_bounds__(kRtThreads) void rt_params_tensor_kernel(kvmi_rt_geometry g,
                                                                      const kvmi_rt_layer* __restrict__ layers,
                                                                      uint64_t rows, const uint16_t* __restrict__ canon,
                                                                      uint8_t* __restrict__ aux, uint64_t half) {
  __shared__ float smn[kRtThreads], smx[kRtThreads];
  const uint32_t layer = blockIdx.x / 2, si = blockIdx.x % 2;
  const kvmi_rt_layer L = layers[layer];
  if ((int)si >= L.num_sections) return;  // uniform per workgroup
  const kvmi_rt_section s = si ? L.sections[1] : L.sections[0];
  if (s.axis != 2) return;
  const uint32_t cols = (uint32_t)g.num_heads * (uint32_t)g.head_dim;
  const uint32_t c0 = (uint32_t)s.head_start * g.head_dim, w = (uint32_t)s.head_count * g.head_dim;
  float mn = INFINITY, mx = -INFINITY;
  for (uint64_t i = threadIdx.x; i < rows * w; i += kRtThreads) {
    const float v = ld_bf16(canon + ((uint64_t)layer * rows + i / w) * cols + c0 + i % w);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  smn[threadIdx.x] = mn;
  smx[threadIdx.x] = mx;
  __syncthreads();
  for (int o = kRtThreads / 2; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) {
      smn[threadIdx.x] = fminf(smn[threadIdx.x], smn[threadIdx.x + o]);
      smx[threadIdx.x] = fmaxf(smx[threadIdx.x], smx[threadIdx.x + o]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) put_params(aux, half, s, 0, quant_params(smn[0], smx[0], s.levels));
}

// ------------------------------------------------------------------ quantize
__device__ __forceinline__ int section_of(const kvmi_rt_layer& L, int h) {
  return (L.num_sections > 1 && h >= L.sections[1].head_start) ? 1 : 0;
}

__device__ __forceinline__ uint64_t param_index(const kvmi_rt_section& s, uint64_t row, int h, int d, int D) {
  if (s.axis == 0) return (uint64_t)(h - s.head_start) * D + d;
  if (s.axis == 1) return row;
  return 0;
}

__global__ __launch_bounds__(kRtThreads) void rt_quantize_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                                 uint64_t rows, const uint16_t* __restrict__ canon,
                                                                 const uint8_t* __restrict__ aux, uint64_t half,
                                                                 uint8_t* __restrict__ packed) {
  const RtIdx ix = rt_idx(rows);
  const kvmi_rt_layer L = layers[ix.layer];
  const int D = g.head_dim;
  const uint32_t cols = (uint32_t)g.num_heads * (uint32_t)D;
  const uint16_t* row = canon + ((uint64_t)ix.layer * rows + ix.row) * cols;
  uint8_t* out = packed + L.u8_offset + ix.row * cols;
  for (uint32_t c = threadIdx.x; c < cols; c += kRtThreads) {
    const int h = (int)(c / (uint32_t)D), d = (int)(c % (uint32_t)D);
    const kvmi_rt_section s = L.sections[section_of(L, h)];
    const uint64_t pi = param_index(s, ix.row, h, d, D);
    const float mn = ld_bf16(reinterpret_cast<const uint16_t*>(aux + s.aux_min_offset) + pi);
    const float inv = ld_bf16(reinterpret_cast<const uint16_t*>(aux + half + s.aux_scale_offset) + pi);
    float q = rintf(rn(rn(ld_bf16(row + c) - mn) * inv));
    q = fminf(fmaxf(q, 0.0f), (float)(s.levels - 1));
    gst(out + c, (uint8_t)q);
  }
}

// ------------------------------------------------------------------ decode
// packed (u8 symbols, or bf16 rows when not quantized) -> [dequantize] -> [inverse
// FWHT] * signs -> cache, rows written back through the head order.
template <int D>
__global__ __launch_bounds__(kRtThreads) void rt_decode_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                               const int64_t* __restrict__ block_ids, uint64_t rows,
                                                               const uint8_t* __restrict__ packed,
                                                               const uint8_t* __restrict__ aux, float scale) {
  constexpr int EPL = D >= 64 ? D / 64 : 1;
  constexpr int HPW = D >= 64 ? 1 : 64 / D;
  const RtIdx ix = rt_idx(rows);
  const kvmi_rt_layer L = layers[ix.layer];
  const uint32_t blk = (uint32_t)ix.row / (uint32_t)g.kernel_tokens;
  const uint32_t tok = (uint32_t)ix.row - blk * (uint32_t)g.kernel_tokens;
  const int64_t pb = gld(block_ids + blk);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint16_t* cache = static_cast<uint16_t*>(L.cache);
  const uint16_t* signs = static_cast<const uint16_t*>(L.signs);
  const uint32_t cols = (uint32_t)g.num_heads * D;
  const bool quant = g.flags & KVMI_RT_QUANTIZE;
  for (int h0 = (int)wave * HPW; h0 < g.num_heads; h0 += kRtWaves * HPW) {
    const int h = h0 + (D >= 64 ? 0 : (int)(lane / D));
    const bool live = h < g.num_heads && (D >= 64 || lane < (uint32_t)(HPW * D));
    float v[EPL];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
      const uint64_t c = (uint64_t)h * D + d;
      float y = 0.0f;
      if (live) {
        if (quant) {
          const kvmi_rt_section s = L.sections[section_of(L, h)];
          const uint64_t pi = param_index(s, ix.row, h, d, D);
          const float mn = ld_bf16(reinterpret_cast<const uint16_t*>(aux + s.aux_min_offset) + pi);
          const float sc = ld_bf16(reinterpret_cast<const uint16_t*>(aux + s.aux_scale_offset) + pi);
          const float q = (float)gld(packed + L.u8_offset + ix.row * cols + c);
          y = rn(rn(q * sc) + mn);
        } else {
          y = ld_bf16(reinterpret_cast<const uint16_t*>(packed) + L.u8_offset + ix.row * cols + c);
        }
      }
      v[k] = y;
    }
    if (g.flags & KVMI_RT_TRANSFORM) fwht_bf16<D>(v, lane, scale);
    if (live) {
      const int hc = gld(L.head_order + h);
      uint16_t* dst = cache + pb * L.block_stride + (int64_t)hc * L.head_stride + (int64_t)tok * L.token_stride +
                      L.channel_offset;
#pragma unroll
      for (int k = 0; k < EPL; ++k) {
        const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
        float x = v[k];
        if (signs) x = rn(x * ld_bf16(signs + (int64_t)h * D + d));
        st_bf16(dst + d, x);
      }
    }
  }
}

// standalone normalized FWHT of bf16 rows with per-stage rounding
template <int D>
__global__ __launch_bounds__(kRtThreads) void rt_hadamard_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                                 int64_t rows, float scale) {
  constexpr int EPL = D >= 64 ? D / 64 : 1;
  constexpr int RPW = D >= 64 ? 1 : 64 / D;  // rows per wave
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = ((int64_t)blockIdx.x * kRtWaves + wave) * RPW + (D >= 64 ? 0 : (int64_t)(lane / D));
  const bool live = r < rows;
  float v[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
    v[k] = live ? ld_bf16(in + r * D + d) : 0.0f;
  }
  fwht_bf16<D>(v, lane, scale);
  if (live) {
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int d = D >= 64 ? (int)lane * EPL + k : (int)(lane % D);
      st_bf16(out + r * D + d, v[k]);
    }
  }
}

// ================================================================== row kernels
// One wave per canonical row (all heads of one token of one layer).  A head row of D
// channels spans LH = D / E lanes holding E contiguous channels each; a wave pass
// covers HPW = 64 / LH heads and P passes cover the row.  Loads and stores are E-wide
// vectors, the FWHT runs in registers (in-lane stages, then lane xor stages), and the
// transformed rows never leave the chip: the token axis reduces inside the wave, the
// channel / tensor axes take a statistics pass (per-workgroup partials) and a small
// reduction before the quantizing pass.
template <int D>
struct RowGeo {
  static constexpr int E = D <= 8 ? D : (D / 64 > 8 ? D / 64 : 8);
  static constexpr int LH = D / E;
  static constexpr int HPW = 64 / LH;
};

constexpr int kStatRows = 64;     // rows per workgroup of the statistics pass
constexpr int kMaxRowCols = 2048; // H * D held by one wave (<= 32 values per lane)

template <int E>
__device__ __forceinline__ void ld_seg(const uint16_t* p, float (&v)[E], bool vec) {
  if (vec) {
    if constexpr (E >= 8) {
#pragma unroll
      for (int i = 0; i < E / 8; ++i) {
        const uint4 t = gld(reinterpret_cast<const uint4*>(p) + i);
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) v[8 * i + 2 * j] = bf_lo(w[j]), v[8 * i + 2 * j + 1] = bf_hi(w[j]);
      }
    } else if constexpr (E == 4) {
      const uint2 t = gld(reinterpret_cast<const uint2*>(p));
      v[0] = bf_lo(t.x), v[1] = bf_hi(t.x), v[2] = bf_lo(t.y), v[3] = bf_hi(t.y);
    } else if constexpr (E == 2) {
      const uint32_t t = gld(reinterpret_cast<const uint32_t*>(p));
      v[0] = bf_lo(t), v[1] = bf_hi(t);
    } else {
      v[0] = ld_bf16(p);
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = ld_bf16(p + k);
  }
}

template <int E>
__device__ __forceinline__ void st_seg(uint16_t* p, const float (&v)[E], bool vec) {
  if (vec) {
    if constexpr (E >= 8) {
#pragma unroll
      for (int i = 0; i < E / 8; ++i)
        gst(reinterpret_cast<uint4*>(p) + i,
            make_uint4(pack_bf16x2(v[8 * i], v[8 * i + 1]), pack_bf16x2(v[8 * i + 2], v[8 * i + 3]),
                       pack_bf16x2(v[8 * i + 4], v[8 * i + 5]), pack_bf16x2(v[8 * i + 6], v[8 * i + 7])));
    } else if constexpr (E == 4) {
      gst(reinterpret_cast<uint2*>(p), make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])));
    } else if constexpr (E == 2) {
      gst(reinterpret_cast<uint32_t*>(p), pack_bf16x2(v[0], v[1]));
    } else {
      st_bf16(p, v[0]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) st_bf16(p + k, v[k]);
  }
}

// E u8 symbols, packed 4 per dword
template <int E>
__device__ __forceinline__ void ld_sym(const uint8_t* p, uint32_t (&w)[(E + 3) / 4]) {
  if constexpr (E >= 8) {
#pragma unroll
    for (int i = 0; i < E / 8; ++i) {
      const uint2 t = gld(reinterpret_cast<const uint2*>(p) + i);
      w[2 * i] = t.x, w[2 * i + 1] = t.y;
    }
  } else if constexpr (E == 4) {
    w[0] = gld(reinterpret_cast<const uint32_t*>(p));
  } else {
    w[0] = 0;
#pragma unroll
    for (int k = 0; k < E; ++k) w[0] |= (uint32_t)gld(p + k) << (8 * k);
  }
}

template <int E>
__device__ __forceinline__ void st_sym(uint8_t* p, const uint32_t (&w)[(E + 3) / 4]) {
  if constexpr (E >= 8) {
#pragma unroll
    for (int i = 0; i < E / 8; ++i) gst(reinterpret_cast<uint2*>(p) + i, make_uint2(w[2 * i], w[2 * i + 1]));
  } else if constexpr (E == 4) {
    gst(reinterpret_cast<uint32_t*>(p), w[0]);
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) gst(p + k, (uint8_t)(w[0] >> (8 * k)));
  }
}

// Signs of a head row: bf16 +-1, applied as the exact sign flip x * s.
template <int E>
__device__ __forceinline__ void mul_signs(float (&v)[E], const uint16_t* s) {
  float sg[E];
  ld_seg<E>(s, sg, true);
#pragma unroll
  for (int k = 0; k < E; ++k) v[k] = __uint_as_float(__float_as_uint(v[k]) ^ (__float_as_uint(sg[k]) & 0x80000000u));
}

// x and y rounded to bf16 with one conversion instruction
__device__ __forceinline__ void rn2(float& x, float& y) {
  const uint32_t p = pack_bf16x2(x, y);
  x = bf_lo(p);
  y = bf_hi(p);
}

// Butterfly stages across lanes J, 2J, .. < LH: the lane with bit J clear holds the
// lower element a and gets a + b, the other gets a - b = partner - own; fma(v, +-1, o)
// is that sum with one fp32 rounding, then bf16.
template <int J, int LH, int P, int E>
__device__ __forceinline__ void fwht_cross(float (&v)[P][E], uint32_t lane) {
  if constexpr (J < LH) {
    const float sgn = (lane & J) ? -1.0f : 1.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
#pragma unroll
      for (int k = 0; k < E; ++k) v[p][k] = __builtin_fmaf(v[p][k], sgn, lane_xor<J>(v[p][k]));
#pragma unroll
      for (int k = 0; k < E; k += 2) rn2(v[p][k], v[p][k + 1]);
    }
    fwht_cross<J * 2, LH, P, E>(v, lane);
  }
}

template <int D, int P>
__device__ __forceinline__ void fwht_rows(float (&v)[P][RowGeo<D>::E], uint32_t lane, float scale) {
  constexpr int E = RowGeo<D>::E, LH = RowGeo<D>::LH;
  static_assert(E % 2 == 0, "pairs of elements per lane");
#pragma unroll
  for (int m = 1; m < E; m <<= 1) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
#pragma unroll
      for (int k = 0; k < E; ++k) {
        if (k & m) continue;
        const float a = v[p][k], b = v[p][k | m];
        v[p][k] = a + b;
        v[p][k | m] = a - b;
        rn2(v[p][k], v[p][k | m]);
      }
    }
  }
  fwht_cross<1, LH, P, E>(v, lane);
#pragma unroll
  for (int p = 0; p < P; ++p) {
#pragma unroll
    for (int k = 0; k < E; k += 2) {
      v[p][k] *= scale;
      v[p][k + 1] *= scale;
      rn2(v[p][k], v[p][k + 1]);
    }
  }
}

struct RowLane {
  uint32_t lane, slot, sub;  // lane, head slot of the pass, lane within the head row
};

template <int D>
__device__ __forceinline__ RowLane row_lane() {
  RowLane r;
  r.lane = threadIdx.x & 63;
  r.slot = r.lane / RowGeo<D>::LH;
  r.sub = r.lane % RowGeo<D>::LH;
  return r;
}

// Rows whose loads a wave issues together: 4 rows of one pass, fewer for wider rows
// (the values of R rows x P passes stay in registers).
template <int P>
constexpr int rows_per_wave() { return P >= 4 ? 1 : 4 / P; }

// Per-wave constants of one layer: the cache head of each pass (-1: no head in this
// slot) and the signs of the lane's channels.
template <int D, int P>
struct LayerLanes {
  int hc[P];
  float sg[P][RowGeo<D>::E];
};

template <int D, int P>
__device__ __forceinline__ void layer_lanes(const kvmi_rt_geometry& g, const kvmi_rt_layer& L, const RowLane& rl,
                                            LayerLanes<D, P>& c) {
  constexpr int E = RowGeo<D>::E, HPW = RowGeo<D>::HPW;
  const uint16_t* signs = static_cast<const uint16_t*>(L.signs);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int h = p * HPW + (int)rl.slot;
    c.hc[p] = h < g.num_heads ? gld(L.head_order + h) : -1;
    if (signs && h < g.num_heads) {
      ld_seg<E>(signs + (int64_t)h * D + rl.sub * E, c.sg[p], true);
    } else {
#pragma unroll
      for (int k = 0; k < E; ++k) c.sg[p][k] = 1.0f;
    }
  }
}

// Physical block and token of row row0 + lane (lanes < n), for the rows a wave
// handles; lane j's pair is broadcast when row j is processed.
struct RowRef {
  int64_t pb;
  uint32_t tok;
};

__device__ __forceinline__ RowRef row_ref(const kvmi_rt_geometry& g, const int64_t* block_ids, uint32_t row0,
                                          uint32_t n, uint32_t lane) {
  RowRef r = {0, 0};
  if (lane < n) {
    const uint32_t row = row0 + lane, kt = (uint32_t)g.kernel_tokens;
    const uint32_t blk = row / kt;
    r.tok = row - blk * kt;
    r.pb = gld(block_ids + blk);
  }
  return r;
}

// gather -> signs -> [FWHT] of rows row0 .. row0 + n - 1 (n <= R) into v, in output-head
// order; `pbl` holds the rows' physical blocks in lanes 0 .. n - 1.  The cache loads of
// all R rows are issued before any of them is used.
template <int D, int P, int R>
__device__ __forceinline__ void load_rows(const kvmi_rt_geometry& g, const kvmi_rt_layer& L,
                                          const LayerLanes<D, P>& c, const RowRef& ref, uint32_t n,
                                          const RowLane& rl, float (&v)[R][P][RowGeo<D>::E], bool vec, float scale) {
  constexpr int E = RowGeo<D>::E;
  const uint16_t* base = static_cast<const uint16_t*>(L.cache) + L.channel_offset + rl.sub * E;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int64_t pb = __shfl(ref.pb, j, 64);
    const uint32_t tok = (uint32_t)__shfl((int)ref.tok, j, 64);
    const uint16_t* row = base + pb * L.block_stride + (int64_t)tok * L.token_stride;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if ((uint32_t)j < n && c.hc[p] >= 0) {
        ld_seg<E>(row + (int64_t)c.hc[p] * L.head_stride, v[j][p], vec);
      } else {
#pragma unroll
        for (int k = 0; k < E; ++k) v[j][p][k] = 0.0f;
      }
    }
  }
  if (L.signs) {
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int k = 0; k < E; ++k)
          v[j][p][k] = __uint_as_float(__float_as_uint(v[j][p][k]) ^ (__float_as_uint(c.sg[p][k]) & 0x80000000u));
  }
  if (g.flags & KVMI_RT_TRANSFORM) {
#pragma unroll
    for (int j = 0; j < R; ++j) fwht_rows<D, P>(v[j], rl.lane, scale);
  }
}

__device__ __forceinline__ float wave_min(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fminf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

// Statistics pass: per-workgroup min / max of every column of the layer's rows
// [r0, r0 + kStatRows), written as fp32 partials [layer][workgroup][2][cols].  Each
// wave takes kStatRows / 4 consecutive rows, rows_per_wave at a time.
template <int D, int P>
__global__ __launch_bounds__(kRtThreads) void rt_stats_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                              const int64_t* __restrict__ block_ids, uint64_t rows,
                                                              float* __restrict__ partial, uint32_t wgs_per_layer,
                                                              bool vec, float scale) {
  constexpr int E = RowGeo<D>::E, HPW = RowGeo<D>::HPW, R = rows_per_wave<P>();
  constexpr uint32_t kWaveRows = kStatRows / kRtWaves;
  static_assert(kWaveRows <= 64 && kWaveRows % R == 0, "one block id per lane");
  __shared__ float smn[kMaxRowCols], smx[kMaxRowCols];
  const uint32_t layer = blockIdx.x / wgs_per_layer, wg = blockIdx.x % wgs_per_layer;
  const kvmi_rt_layer L = layers[layer];
  const RowLane rl = row_lane<D>();
  const uint32_t wave = threadIdx.x >> 6;
  LayerLanes<D, P> c;
  layer_lanes<D, P>(g, L, rl, c);
  const uint32_t nrows = (uint32_t)rows;
  const uint32_t r0 = wg * kStatRows + wave * kWaveRows;
  const uint32_t nw = r0 < nrows ? min(kWaveRows, nrows - r0) : 0u;
  const RowRef all = row_ref(g, block_ids, r0, nw, rl.lane);
  float mn[P][E], mx[P][E];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int k = 0; k < E; ++k) mn[p][k] = INFINITY, mx[p][k] = -INFINITY;
  for (uint32_t i = 0; i < nw; i += R) {
    const uint32_t n = min((uint32_t)R, nw - i);
    RowRef ref;  // lane j: row r0 + i + j
    ref.pb = __shfl(all.pb, (int)((rl.lane + i) & 63u), 64);
    ref.tok = (uint32_t)__shfl((int)all.tok, (int)((rl.lane + i) & 63u), 64);
    float v[R][P][E];
    load_rows<D, P, R>(g, L, c, ref, n, rl, v, vec, scale);
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if ((uint32_t)j >= n) break;
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int k = 0; k < E; ++k) mn[p][k] = fminf(mn[p][k], v[j][p][k]), mx[p][k] = fmaxf(mx[p][k], v[j][p][k]);
    }
  }
  const uint32_t cols = (uint32_t)g.num_heads * D;
  for (uint32_t w = 0; w < (uint32_t)kRtWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int h = p * HPW + (int)rl.slot;
        if (h >= g.num_heads) continue;
#pragma unroll
        for (int k = 0; k < E; ++k) {
          const uint32_t col = (uint32_t)h * D + rl.sub * E + k;
          smn[col] = w ? fminf(smn[col], mn[p][k]) : mn[p][k];
          smx[col] = w ? fmaxf(smx[col], mx[p][k]) : mx[p][k];
        }
      }
    }
    __syncthreads();
  }
  float* out = partial + ((uint64_t)layer * wgs_per_layer + wg) * 2 * cols;
  for (uint32_t col = threadIdx.x; col < cols; col += kRtThreads) {
    gst(out + col, smn[col]);
    gst(out + cols + col, smx[col]);
  }
}

// Reduce the partials of one layer into the channel / tensor section parameters.
__global__ __launch_bounds__(kRtThreads) void rt_stats_reduce_kernel(kvmi_rt_geometry g,
                                                                     const kvmi_rt_layer* __restrict__ layers,
                                                                     const float* __restrict__ partial,
                                                                     uint32_t wgs_per_layer, uint8_t* __restrict__ aux,
                                                                     uint64_t half) {
  __shared__ float tmn[2][kRtThreads], tmx[2][kRtThreads];
  const uint32_t layer = blockIdx.x;
  const kvmi_rt_layer L = layers[layer];
  const uint32_t D = (uint32_t)g.head_dim, cols = (uint32_t)g.num_heads * D;
  float smin[2] = {INFINITY, INFINITY}, smax[2] = {-INFINITY, -INFINITY};
  const float* base = partial + (uint64_t)layer * wgs_per_layer * 2 * cols;
  for (uint32_t c = threadIdx.x; c < cols; c += kRtThreads) {
    float mn = INFINITY, mx = -INFINITY;
    uint32_t w = 0;
    for (; w + 8 <= wgs_per_layer; w += 8) {  // eight partials in flight
      float a[8], b[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        a[u] = gld(base + (uint64_t)(w + u) * 2 * cols + c);
        b[u] = gld(base + (uint64_t)(w + u) * 2 * cols + cols + c);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) mn = fminf(mn, a[u]), mx = fmaxf(mx, b[u]);
    }
    for (; w < wgs_per_layer; ++w) {
      mn = fminf(mn, gld(base + (uint64_t)w * 2 * cols + c));
      mx = fmaxf(mx, gld(base + (uint64_t)w * 2 * cols + cols + c));
    }
    const int h = (int)(c / D);
    const int si = section_of(L, h);
    if (si >= L.num_sections) continue;
    const kvmi_rt_section s = si ? L.sections[1] : L.sections[0];
    if (s.axis == 0) put_params(aux, half, s, c - (uint32_t)s.head_start * D, quant_params(mn, mx, s.levels));
    if (s.axis == 2) {
      if (si) {
        smin[1] = fminf(smin[1], mn), smax[1] = fmaxf(smax[1], mx);
      } else {
        smin[0] = fminf(smin[0], mn), smax[0] = fmaxf(smax[0], mx);
      }
    }
  }
  const bool tensor = (L.num_sections > 0 && L.sections[0].axis == 2) || (L.num_sections > 1 && L.sections[1].axis == 2);
  if (!tensor) return;  // uniform per workgroup
#pragma unroll
  for (int si = 0; si < 2; ++si) tmn[si][threadIdx.x] = smin[si], tmx[si][threadIdx.x] = smax[si];
  __syncthreads();
  for (int o = kRtThreads / 2; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o)
      for (int si = 0; si < 2; ++si) {
        tmn[si][threadIdx.x] = fminf(tmn[si][threadIdx.x], tmn[si][threadIdx.x + o]);
        tmx[si][threadIdx.x] = fmaxf(tmx[si][threadIdx.x], tmx[si][threadIdx.x + o]);
      }
    __syncthreads();
  }
  if (threadIdx.x == 0)
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      if (si >= L.num_sections) break;
      const kvmi_rt_section s = si ? L.sections[1] : L.sections[0];
      if (s.axis == 2) put_params(aux, half, s, 0, quant_params(tmn[si][0], tmx[si][0], s.levels));
    }
}

// Quantization parameters of a lane's channels for a channel / tensor section (read
// from aux, constant over the layer's rows), or unused for a token section.
template <int D, int P>
struct LaneParams {
  float mn[P][RowGeo<D>::E], inv[P][RowGeo<D>::E];
};

// Encode pass: a wave takes rows_per_wave consecutive rows of one layer.  Quantized:
// token sections reduce inside the wave, channel / tensor sections read their
// parameters from aux; the u8 symbols land at the layer's u8_offset.  Not quantized:
// the bf16 rows are the payload.
template <int D, int P>
__global__ __launch_bounds__(kRtThreads) void rt_row_encode_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                                   const int64_t* __restrict__ block_ids, uint64_t rows,
                                                                   uint32_t num_layers, uint8_t* __restrict__ packed,
                                                                   uint8_t* __restrict__ aux, uint64_t half, bool vec,
                                                                   float scale) {
  constexpr int E = RowGeo<D>::E, HPW = RowGeo<D>::HPW, R = rows_per_wave<P>();
  const uint32_t nrows = (uint32_t)rows, groups = (nrows + R - 1) / R;
  const uint32_t task = blockIdx.x * kRtWaves + (threadIdx.x >> 6);
  if (task >= groups * num_layers) return;  // wave-uniform
  const uint32_t layer = task / groups;
  const uint32_t row0 = (task - layer * groups) * R;
  const uint32_t n = min((uint32_t)R, nrows - row0);
  const kvmi_rt_layer L = layers[layer];
  const RowLane rl = row_lane<D>();
  LayerLanes<D, P> c;
  layer_lanes<D, P>(g, L, rl, c);
  const RowRef ref = row_ref(g, block_ids, row0, n, rl.lane);
  float v[R][P][E];
  load_rows<D, P, R>(g, L, c, ref, n, rl, v, vec, scale);
  const uint64_t cols = (uint64_t)g.num_heads * D;
  if (!(g.flags & KVMI_RT_QUANTIZE)) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if ((uint32_t)j >= n) break;
      uint16_t* out = reinterpret_cast<uint16_t*>(packed) + L.u8_offset + (row0 + j) * cols + rl.sub * E;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int h = p * HPW + (int)rl.slot;
        if (h < g.num_heads) st_seg<E>(out + (int64_t)h * D, v[j][p], true);
      }
    }
    return;
  }
  // channel / tensor parameters of the lane's channels
  LaneParams<D, P> lp;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int h = p * HPW + (int)rl.slot;
    const kvmi_rt_section s = (h < g.num_heads && section_of(L, h)) ? L.sections[1] : L.sections[0];
    if (h >= g.num_heads || s.axis == 1) {
#pragma unroll
      for (int k = 0; k < E; ++k) lp.mn[p][k] = 0.0f, lp.inv[p][k] = 0.0f;
      continue;
    }
    const uint64_t pi = s.axis == 0 ? (uint64_t)(h - s.head_start) * D + rl.sub * E : 0;
    const uint16_t* pmn = reinterpret_cast<const uint16_t*>(aux + s.aux_min_offset) + pi;
    const uint16_t* pinv = reinterpret_cast<const uint16_t*>(aux + half + s.aux_scale_offset) + pi;
    if (s.axis == 0) {
      ld_seg<E>(pmn, lp.mn[p], true);
      ld_seg<E>(pinv, lp.inv[p], true);
    } else {
      const float a = ld_bf16(pmn), b = ld_bf16(pinv);
#pragma unroll
      for (int k = 0; k < E; ++k) lp.mn[p][k] = a, lp.inv[p][k] = b;
    }
  }
  const bool tok0 = L.num_sections > 0 && L.sections[0].axis == 1;
  const bool tok1 = L.num_sections > 1 && L.sections[1].axis == 1;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if ((uint32_t)j >= n) break;
    const uint64_t row = row0 + j;
    // token-axis statistics of the row, per section (two named sections: a local
    // array indexed by a run-time section number would live in scratch memory)
    QP tp0 = {}, tp1 = {};
    if (tok0 || tok1) {
      float tmin0 = INFINITY, tmin1 = INFINITY, tmax0 = -INFINITY, tmax1 = -INFINITY;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int h = p * HPW + (int)rl.slot;
        if (h >= g.num_heads) continue;
        float a = INFINITY, b = -INFINITY;
#pragma unroll
        for (int k = 0; k < E; ++k) a = fminf(a, v[j][p][k]), b = fmaxf(b, v[j][p][k]);
        if (section_of(L, h)) {
          tmin1 = fminf(tmin1, a), tmax1 = fmaxf(tmax1, b);
        } else {
          tmin0 = fminf(tmin0, a), tmax0 = fmaxf(tmax0, b);
        }
      }
      if (tok0) {
        tp0 = quant_params(wave_min(tmin0), wave_max(tmax0), L.sections[0].levels);
        if (rl.lane == (uint32_t)j) put_params(aux, half, L.sections[0], row, tp0);
      }
      if (tok1) {
        tp1 = quant_params(wave_min(tmin1), wave_max(tmax1), L.sections[1].levels);
        if (rl.lane == (uint32_t)j) put_params(aux, half, L.sections[1], row, tp1);
      }
    }
    uint8_t* out = packed + L.u8_offset + row * cols + rl.sub * E;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int h = p * HPW + (int)rl.slot;
      if (h >= g.num_heads) continue;
      const bool second = section_of(L, h);
      const kvmi_rt_section s = second ? L.sections[1] : L.sections[0];
      const bool token = s.axis == 1;
      const QP& t = second ? tp1 : tp0;
      const float top = (float)(s.levels - 1);
      uint32_t w[(E + 3) / 4];
#pragma unroll
      for (int i = 0; i < (E + 3) / 4; ++i) w[i] = 0;
#pragma unroll
      for (int k = 0; k < E; k += 2) {
        float a = v[j][p][k] - (token ? t.mn : lp.mn[p][k]);
        float b = v[j][p][k + 1] - (token ? t.mn : lp.mn[p][k + 1]);
        rn2(a, b);
        a *= token ? t.inv : lp.inv[p][k];
        b *= token ? t.inv : lp.inv[p][k + 1];
        rn2(a, b);
        a = fminf(fmaxf(rintf(a), 0.0f), top);
        b = fminf(fmaxf(rintf(b), 0.0f), top);
        w[k / 4] |= ((uint32_t)a | ((uint32_t)b << 8)) << (8 * (k % 4));
      }
      st_sym<E>(out + (int64_t)h * D, w);
    }
  }
}

// Decode pass: a wave takes rows_per_wave consecutive rows of one layer: symbols (or
// bf16 rows) -> dequantize -> [FWHT] -> signs -> the cache, through the head order.
template <int D, int P>
__global__ __launch_bounds__(kRtThreads) void rt_row_decode_kernel(kvmi_rt_geometry g, const kvmi_rt_layer* __restrict__ layers,
                                                                   const int64_t* __restrict__ block_ids, uint64_t rows,
                                                                   uint32_t num_layers, const uint8_t* __restrict__ packed,
                                                                   const uint8_t* __restrict__ aux, bool vec, float scale) {
  constexpr int E = RowGeo<D>::E, HPW = RowGeo<D>::HPW, R = rows_per_wave<P>();
  const uint32_t nrows = (uint32_t)rows, groups = (nrows + R - 1) / R;
  const uint32_t task = blockIdx.x * kRtWaves + (threadIdx.x >> 6);
  if (task >= groups * num_layers) return;  // wave-uniform
  const uint32_t layer = task / groups;
  const uint32_t row0 = (task - layer * groups) * R;
  const uint32_t n = min((uint32_t)R, nrows - row0);
  const kvmi_rt_layer L = layers[layer];
  const RowLane rl = row_lane<D>();
  const uint64_t cols = (uint64_t)g.num_heads * D;
  const bool quant = g.flags & KVMI_RT_QUANTIZE;
  LayerLanes<D, P> c;
  layer_lanes<D, P>(g, L, rl, c);
  const RowRef ref = row_ref(g, block_ids, row0, n, rl.lane);
  float v[R][P][E];
  if (!quant) {
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int h = p * HPW + (int)rl.slot;
        if ((uint32_t)j < n && h < g.num_heads) {
          ld_seg<E>(reinterpret_cast<const uint16_t*>(packed) + L.u8_offset + (row0 + j) * cols + (uint64_t)h * D +
                        rl.sub * E, v[j][p], true);
        } else {
#pragma unroll
          for (int k = 0; k < E; ++k) v[j][p][k] = 0.0f;
        }
      }
  } else {
    // symbols of all rows first, then the parameters
    uint32_t w[R][P][(E + 3) / 4];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int h = p * HPW + (int)rl.slot;
        if ((uint32_t)j < n && h < g.num_heads) {
          ld_sym<E>(packed + L.u8_offset + (row0 + j) * cols + (uint64_t)h * D + rl.sub * E, w[j][p]);
        } else {
#pragma unroll
          for (int i = 0; i < (E + 3) / 4; ++i) w[j][p][i] = 0;
        }
      }
    // token parameters: lane j holds row row0 + j's (min, scale) of each section
    float tmn0 = 0.0f, tsc0 = 0.0f, tmn1 = 0.0f, tsc1 = 0.0f;
    if (rl.lane < n) {
      if (L.num_sections > 0 && L.sections[0].axis == 1) {
        tmn0 = ld_bf16(reinterpret_cast<const uint16_t*>(aux + L.sections[0].aux_min_offset) + row0 + rl.lane);
        tsc0 = ld_bf16(reinterpret_cast<const uint16_t*>(aux + L.sections[0].aux_scale_offset) + row0 + rl.lane);
      }
      if (L.num_sections > 1 && L.sections[1].axis == 1) {
        tmn1 = ld_bf16(reinterpret_cast<const uint16_t*>(aux + L.sections[1].aux_min_offset) + row0 + rl.lane);
        tsc1 = ld_bf16(reinterpret_cast<const uint16_t*>(aux + L.sections[1].aux_scale_offset) + row0 + rl.lane);
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int h = p * HPW + (int)rl.slot;
      const bool live = h < g.num_heads;
      const bool second = live && section_of(L, h);
      const kvmi_rt_section s = second ? L.sections[1] : L.sections[0];
      float mn[E], sc[E];
      if (live && s.axis != 1) {
        const uint64_t pi = s.axis == 0 ? (uint64_t)(h - s.head_start) * D + rl.sub * E : 0;
        const uint16_t* pmn = reinterpret_cast<const uint16_t*>(aux + s.aux_min_offset) + pi;
        const uint16_t* psc = reinterpret_cast<const uint16_t*>(aux + s.aux_scale_offset) + pi;
        if (s.axis == 0) {
          ld_seg<E>(pmn, mn, true);
          ld_seg<E>(psc, sc, true);
        } else {
          const float a = ld_bf16(pmn), b = ld_bf16(psc);
#pragma unroll
          for (int k = 0; k < E; ++k) mn[k] = a, sc[k] = b;
        }
      }
#pragma unroll
      for (int j = 0; j < R; ++j) {
        // row j's parameters of both sections from lane j, then this lane's section
        const float m0 = __shfl(tmn0, j, 64), m1 = __shfl(tmn1, j, 64);
        const float s0 = __shfl(tsc0, j, 64), s1 = __shfl(tsc1, j, 64);
        const float rmn = second ? m1 : m0, rsc = second ? s1 : s0;
#pragma unroll
        for (int k = 0; k < E; k += 2) {
          const bool tok = live && s.axis == 1;
          float a = (float)((w[j][p][k / 4] >> (8 * (k % 4))) & 0xffu) * (tok ? rsc : sc[k]);
          float b = (float)((w[j][p][k / 4] >> (8 * (k % 4) + 8)) & 0xffu) * (tok ? rsc : sc[k + 1]);
          rn2(a, b);
          a += tok ? rmn : mn[k];
          b += tok ? rmn : mn[k + 1];
          rn2(a, b);
          v[j][p][k] = a;
          v[j][p][k + 1] = b;
        }
      }
    }
  }
  if (g.flags & KVMI_RT_TRANSFORM) {
#pragma unroll
    for (int j = 0; j < R; ++j) fwht_rows<D, P>(v[j], rl.lane, scale);
  }
  const uint16_t* signs = static_cast<const uint16_t*>(L.signs);
  uint16_t* base = static_cast<uint16_t*>(L.cache) + L.channel_offset + rl.sub * E;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if ((uint32_t)j >= n) break;
    const int64_t pb = __shfl(ref.pb, j, 64);
    const uint32_t tok = (uint32_t)__shfl((int)ref.tok, j, 64);
    uint16_t* row = base + pb * L.block_stride + (int64_t)tok * L.token_stride;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (c.hc[p] < 0) continue;
      if (signs) {
#pragma unroll
        for (int k = 0; k < E; ++k)
          v[j][p][k] = __uint_as_float(__float_as_uint(v[j][p][k]) ^ (__float_as_uint(c.sg[p][k]) & 0x80000000u));
      }
      st_seg<E>(row + (int64_t)c.hc[p] * L.head_stride, v[j][p], vec);
    }
  }
}

float rt_scale(int D) { return (float)(1.0 / __builtin_sqrt((double)D)); }

template <class F>
int rt_dispatch(int D, F&& f) {
  switch (D) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    case 256: return f(std::integral_constant<int, 256>{});
    case 512: return f(std::integral_constant<int, 512>{});
    case 1024: return f(std::integral_constant<int, 1024>{});
    case 2048: return f(std::integral_constant<int, 2048>{});
    default: return KVMI_EINVAL;
  }
}

// head sizes served by the row kernels (the others take the generic path)
bool rt_row_head_dim(int D) { return D >= 8 && D <= 256; }

// P passes of HPW heads cover a row; the row kernels hold E * P <= 32 values per lane
// and row; wider rows take the generic path
int rt_row_passes(int D, int H) {
  if (!rt_row_head_dim(D)) return 0;
  int E = D <= 8 ? D : (D / 64 > 8 ? D / 64 : 8);
  const int hpw = 64 / (D / E);
  const int need = (H + hpw - 1) / hpw;
  int P = 1;
  while (P < need) P <<= 1;
  if (P > 4 || E * P > 32 || (int64_t)H * D > kMaxRowCols) return 0;
  return P;
}

template <class F>
int rt_row_dispatch(int D, int P, F&& f) {
  auto passes = [&](auto Dc) {
    switch (P) {
      case 1: return f(Dc, std::integral_constant<int, 1>{});
      case 2: return f(Dc, std::integral_constant<int, 2>{});
      case 4: return f(Dc, std::integral_constant<int, 4>{});
      default: return (int)KVMI_EINVAL;
    }
  };
  switch (D) {
    case 8: return passes(std::integral_constant<int, 8>{});
    case 16: return passes(std::integral_constant<int, 16>{});
    case 32: return passes(std::integral_constant<int, 32>{});
    case 64: return passes(std::integral_constant<int, 64>{});
    case 128: return passes(std::integral_constant<int, 128>{});
    case 256: return passes(std::integral_constant<int, 256>{});
    default: return (int)KVMI_EINVAL;
  }
}

int64_t stat_wgs(uint64_t rows) { return (int64_t)((rows + kStatRows - 1) / kStatRows); }

bool rt_geometry_ok(const kvmi_rt_geometry* g) {
  return g && g->num_heads >= 1 && g->num_heads <= 1024 && g->head_dim >= 1 && g->head_dim <= 2048 &&
         (g->head_dim & (g->head_dim - 1)) == 0 && g->kernel_tokens >= 1;
}

}  // namespace
}  // namespace kvmi

using namespace kvmi;

extern "C" int64_t kvmi_rt_scratch_bytes(int32_t num_layers, int64_t rows, int32_t num_heads, int32_t head_dim) {
  if (num_layers < 0 || rows < 0 || num_heads < 0 || head_dim < 0) return -1;
  const int64_t cols = (int64_t)num_heads * head_dim;
  const int64_t canon = (int64_t)num_layers * rows * cols * 2;
  const int64_t stats = (int64_t)num_layers * stat_wgs((uint64_t)rows) * 2 * cols * 4;
  return canon > stats ? canon : stats;
}

extern "C" int kvmi_rt_encode(const kvmi_rt_geometry* geom, const kvmi_rt_layer* layers, int32_t num_layers,
                              const int64_t* block_ids, int64_t num_blocks, void* canon, uint8_t* packed,
                              uint8_t* aux, int64_t aux_half_bytes, kvmi_stream_t stream) {
  if (!rt_geometry_ok(geom) || num_layers < 0 || num_blocks < 0) return KVMI_EINVAL;
  if (num_layers == 0 || num_blocks == 0) return KVMI_OK;
  if (!layers || !block_ids || !packed) return KVMI_EINVAL;
  const kvmi_rt_geometry g = *geom;
  const bool quant = g.flags & KVMI_RT_QUANTIZE;
  if (quant && (!canon || !aux || aux_half_bytes <= 0)) return KVMI_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint64_t rows = (uint64_t)num_blocks * (uint64_t)g.kernel_tokens;
  const uint64_t grid = rows * (uint64_t)num_layers;
  if (grid > 0x7fffffffull) return KVMI_EINVAL;
  const float scale = rt_scale(g.head_dim);
  const uint64_t half = (uint64_t)aux_half_bytes;
  const int P = (g.flags & KVMI_RT_GENERIC) ? 0 : rt_row_passes(g.head_dim, g.num_heads);
  const bool vec = g.flags & KVMI_RT_ALIGNED;
  if (P) {
    int rc = rt_row_dispatch(g.head_dim, P, [&](auto Dc, auto Pc) {
      constexpr int D = decltype(Dc)::value, PP = decltype(Pc)::value;
      if (quant && (g.axes & 5u)) {
        const uint32_t wpl = (uint32_t)stat_wgs(rows);
        float* partial = static_cast<float*>(canon);
        hipLaunchKernelGGL((rt_stats_kernel<D, PP>), dim3(wpl * (uint32_t)num_layers), dim3(kRtThreads), 0, s, g,
                           layers, block_ids, rows, partial, wpl, vec, scale);
        hipLaunchKernelGGL(rt_stats_reduce_kernel, dim3((uint32_t)num_layers), dim3(kRtThreads), 0, s, g, layers,
                           (const float*)partial, wpl, aux, half);
      }
      constexpr int R = rows_per_wave<PP>();
      const uint64_t tasks = (rows + R - 1) / R * (uint64_t)num_layers;
      const uint32_t wgs = (uint32_t)((tasks + kRtWaves - 1) / kRtWaves);
      hipLaunchKernelGGL((rt_row_encode_kernel<D, PP>), dim3(wgs), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                         (uint32_t)num_layers, packed, aux, half, vec, scale);
      return (int)KVMI_OK;
    });
    if (rc != KVMI_OK) return rc;
    return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
  }
  // generic path: transformed rows through the scratch
  uint16_t* dst = quant ? static_cast<uint16_t*>(canon) : reinterpret_cast<uint16_t*>(packed);
  int rc = rt_dispatch(g.head_dim, [&](auto Dc) {
    constexpr int D = decltype(Dc)::value;
    hipLaunchKernelGGL(rt_transform_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                       dst, !quant, scale);
    return KVMI_OK;
  });
  if (rc != KVMI_OK) return rc;
  if (!quant) return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
  const uint32_t cols = (uint32_t)g.num_heads * (uint32_t)g.head_dim;
  const uint32_t per_layer = (cols + kRtThreads - 1) / kRtThreads;
  if (g.axes & 1u)
    hipLaunchKernelGGL(rt_params_channel_kernel, dim3(per_layer * (uint32_t)num_layers), dim3(kRtThreads), 0, s, g,
                       layers, rows, dst, aux, half);
  if (g.axes & 2u)
    hipLaunchKernelGGL(rt_params_token_kernel, dim3((uint32_t)grid), dim3(64), 0, s, g, layers, rows, dst, aux, half);
  if (g.axes & 4u)
    hipLaunchKernelGGL(rt_params_tensor_kernel, dim3(2u * (uint32_t)num_layers), dim3(kRtThreads), 0, s, g, layers,
                       rows, dst, aux, half);
  hipLaunchKernelGGL(rt_quantize_kernel, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, rows, dst, aux, half,
                     packed);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_rt_decode(const kvmi_rt_geometry* geom, const kvmi_rt_layer* layers, int32_t num_layers,
                              const int64_t* block_ids, int64_t num_blocks, const uint8_t* packed, const uint8_t* aux,
                              kvmi_stream_t stream) {
  if (!rt_geometry_ok(geom) || num_layers < 0 || num_blocks < 0) return KVMI_EINVAL;
  if (num_layers == 0 || num_blocks == 0) return KVMI_OK;
  if (!layers || !block_ids || !packed) return KVMI_EINVAL;
  const kvmi_rt_geometry g = *geom;
  if ((g.flags & KVMI_RT_QUANTIZE) && !aux) return KVMI_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint64_t rows = (uint64_t)num_blocks * (uint64_t)g.kernel_tokens;
  const uint64_t grid = rows * (uint64_t)num_layers;
  if (grid > 0x7fffffffull) return KVMI_EINVAL;
  const float scale = rt_scale(g.head_dim);
  const int P = (g.flags & KVMI_RT_GENERIC) ? 0 : rt_row_passes(g.head_dim, g.num_heads);
  int rc;
  if (P) {
    const bool vec = g.flags & KVMI_RT_ALIGNED;
    rc = rt_row_dispatch(g.head_dim, P, [&](auto Dc, auto Pc) {
      constexpr int D = decltype(Dc)::value, PP = decltype(Pc)::value;
      constexpr int R = rows_per_wave<PP>();
      const uint64_t tasks = (rows + R - 1) / R * (uint64_t)num_layers;
      const uint32_t wgs = (uint32_t)((tasks + kRtWaves - 1) / kRtWaves);
      hipLaunchKernelGGL((rt_row_decode_kernel<D, PP>), dim3(wgs), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                         (uint32_t)num_layers, packed, aux, vec, scale);
      return (int)KVMI_OK;
    });
  } else {
    rc = rt_dispatch(g.head_dim, [&](auto Dc) {
      constexpr int D = decltype(Dc)::value;
      hipLaunchKernelGGL(rt_decode_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                         packed, aux, scale);
      return KVMI_OK;
    });
  }
  if (rc != KVMI_OK) return rc;
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_rt_hadamard(const void* in, void* out, int64_t rows, int32_t head_dim, kvmi_stream_t stream) {
  if (rows < 0 || head_dim < 1 || head_dim > 2048 || (head_dim & (head_dim - 1)) || !in || !out) return KVMI_EINVAL;
  const uint64_t bytes = (uint64_t)rows * head_dim * 2;
  const uintptr_t a = reinterpret_cast<uintptr_t>(in), b = reinterpret_cast<uintptr_t>(out);
  if (a != b && a < b + bytes && b < a + bytes) return KVMI_EINVAL;  // partial overlap
  if (rows == 0) return KVMI_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t rpw = head_dim >= 64 ? 1 : 64 / head_dim;
  const int64_t per_block = kRtWaves * rpw;
  const int64_t grid = (rows + per_block - 1) / per_block;
  if (grid > 0x7fffffffll) return KVMI_EINVAL;
  const float scale = rt_scale(head_dim);
  int rc = rt_dispatch(head_dim, [&](auto Dc) {
    constexpr int D = decltype(Dc)::value;
    hipLaunchKernelGGL(rt_hadamard_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s,
                       static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, scale);
    return KVMI_OK;
  });
  if (rc != KVMI_OK) return rc;
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}
