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

__device__ __forceinline__ RtIdx rt_idx(uint64_t rows) {
  RtIdx r;
  r.layer = (uint32_t)(blockIdx.x / rows);
  r.row = blockIdx.x % rows;
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
  const uint64_t blk = ix.row / (uint64_t)g.kernel_tokens;
  const uint32_t tok = (uint32_t)(ix.row % (uint64_t)g.kernel_tokens);
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
  for (int si = 0; si < L.num_sections; ++si) {
    const kvmi_rt_section s = L.sections[si];
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
  for (int si = 0; si < L.num_sections; ++si) {
    const kvmi_rt_section s = L.sections[si];
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
  if ((int)si >= L.num_sections || L.sections[si].axis != 2) return;  // uniform per workgroup
  const kvmi_rt_section s = L.sections[si];
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
  const uint64_t blk = ix.row / (uint64_t)g.kernel_tokens;
  const uint32_t tok = (uint32_t)(ix.row % (uint64_t)g.kernel_tokens);
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

bool rt_geometry_ok(const kvmi_rt_geometry* g) {
  return g && g->num_heads >= 1 && g->num_heads <= 1024 && g->head_dim >= 1 && g->head_dim <= 2048 &&
         (g->head_dim & (g->head_dim - 1)) == 0 && g->kernel_tokens >= 1;
}

}  // namespace
}  // namespace kvmi

using namespace kvmi;

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
  // not quantized: the canonical rows are the payload (bf16)
  uint16_t* dst = quant ? static_cast<uint16_t*>(canon) : reinterpret_cast<uint16_t*>(packed);
  const float scale = rt_scale(g.head_dim);
  if (!quant) {
    int rc = rt_dispatch(g.head_dim, [&](auto Dc) {
      constexpr int D = decltype(Dc)::value;
      hipLaunchKernelGGL(rt_transform_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, block_ids,
                         rows, dst, true, scale);
      return KVMI_OK;
    });
    if (rc != KVMI_OK) return rc;
    return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
  }
  int rc = rt_dispatch(g.head_dim, [&](auto Dc) {
    constexpr int D = decltype(Dc)::value;
    hipLaunchKernelGGL(rt_transform_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                       dst, false, scale);
    return KVMI_OK;
  });
  if (rc != KVMI_OK) return rc;
  const uint64_t half = (uint64_t)aux_half_bytes;
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
  int rc = rt_dispatch(g.head_dim, [&](auto Dc) {
    constexpr int D = decltype(Dc)::value;
    hipLaunchKernelGGL(rt_decode_kernel<D>, dim3((uint32_t)grid), dim3(kRtThreads), 0, s, g, layers, block_ids, rows,
                       packed, aux, scale);
    return KVMI_OK;
  });
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
