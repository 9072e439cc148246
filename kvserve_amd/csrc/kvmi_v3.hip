// Fused Hadamard quantizer with fp32 statistics (quantizer_config.impl
// "tilelang_fused"): the arithmetic of KVHadamardQuantOp.compress_v3 /
// decompress_v3 (kvserve_v1/tilelang_ops/kv_hadamard_quant.py:1519-1599,
// :1645-1750) on one dense layer [2, R, H, D] (R rows = blocks * block_size).
//
// A head-row (one token of one head, D contiguous bf16) is held by a quad of lanes,
// lane q owning elements [q*E, (q+1)*E), E = D/4; a 256-thread workgroup covers 64
// consecutive head-rows per pass, and since 64 % H == 0 a lane always sees the same
// head.  The FWHT is the reference's radix-2 butterfly in fp32 (natural order, lowest
// index bit first: fwht_row), so y = FWHT(x*s) * (1/sqrt(D)) is bit-identical to the
// TileLang kernels' values (:521-596).
//
// Compress is three launches:
//   kstats: y of every K head-row; per-lane running min / max per channel, reduced
//           over the workgroup in LDS (order-preserving keys) into a per-workgroup
//           partial [wg][2][H][D];
//   kfinal: K min / max over the partials, scale = max(max - min, 1e-5) / (L - 1);
//   quant:  y again, had = bf16(y); K with the channel constants; V with the
//           per-head-row min / max over D (:652-659) reduced over the heads of its
//           group (equal L, :1143-1163) in LDS -- a pass holds 64 / H whole rows, so
//           V is read once; q = clamp(roundf((had - min) / scale), 0, L) as uint8.
// Decompress is one launch: x = fma(q, scale16, min16), fp32 butterflies,
// bf16((y * (1/sqrt(D))) * s) (:685-716).
#include <mutex>

#include "kvmi_common.hpp"

namespace kvmi {
namespace {

constexpr int kV3WG = 256;
constexpr int kV3Rows = kV3WG / 4;  // head-rows per pass
constexpr int kV3MaxH = 64;
constexpr int kV3KGrid = 256;       // most workgroups of the K statistics pass (partials)
constexpr int kV3Ahead = 4;         // K statistics: passes loaded before any is transformed

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Sign bits of lane q's E elements of head h (bit i set = element i negated).
template <int D>
__device__ __forceinline__ uint32_t v3_lane_signs(const uint32_t* signs, int h, int q) {
  constexpr int E = D / 4;
  const uint32_t* sg = signs + h * (D / 32);
  if constexpr (E == 32) {
    return gld(sg + q);
  } else {  // E == 16
    return (gld(sg + (q >> 1)) >> ((q & 1) * 16)) & 0xffffu;
  }
}

// y = FWHT_fp32(x * s) * (1/sqrt(D)) of the lane's E elements (w: their bf16 pairs).
template <int D>
__device__ __forceinline__ void v3_transform_w(uint32_t (&w)[D / 8], uint32_t sb, float scale, int q,
                                               float (&y)[D / 4]) {
  constexpr int E = D / 4;
  apply_sign_bf16<E>(w, sb);
  unpack_bf16<E>(w, y);
  fwht_row<E>(y, q);
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] *= scale;
}
template <int D>
__device__ __forceinline__ void v3_transform(const uint16_t* src, uint32_t sb, float scale, int q,
                                             float (&y)[D / 4]) {
  uint32_t w[D / 8];
  load_bf16_seg<D / 4>(src, w);
  v3_transform_w<D>(w, sb, scale, q, y);
}

// clamp(roundf((had - mn) / sc), 0, L) as an integer (roundf: ties away from zero;
// the division is the correctly rounded fp32 one).
__device__ __forceinline__ uint32_t v3_symbol(float had, float mn, float sc, float lv) {
  return (uint32_t)fminf(fmaxf(__builtin_roundf((had - mn) / sc), 0.0f), lv);
}

struct V3Shape {
  int64_t rows;  // R
  int H;
  float scale;   // fp32 1/sqrt(D)
};

// ------------------------------------------------------------------ K statistics
// One partial per workgroup: the grid must not exceed kV3KGrid.  With about one
// workgroup per CU a lane loads kV3Ahead passes before transforming any of them, so
// that enough bytes are in flight; the LDS holds the layer's 2 * H * D keys (dynamic
// size).  (Up to 1024 workgroups of 2 passes ahead measured faster on 128 Ki-row layers
// and slower on 8 Ki-row ones, where the partials cost more than the overlap gains.)
template <int D>
__global__ __launch_bounds__(kV3WG) void v3_kstats_kernel(V3Shape sh, const uint16_t* __restrict__ x,
                                                          const uint32_t* __restrict__ signs,
                                                          uint32_t* __restrict__ kpart) {
  constexpr int E = D / 4;
  const int H = sh.H, HD = H * D;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3, h = Q % H;
  const int64_t hrows = sh.rows * H;
  const uint32_t sb = v3_lane_signs<D>(signs, h, q);
  const int64_t passes = (hrows + kV3Rows - 1) / kV3Rows;
  // [2][H * D] keys; channel c = seg * E + k sits at seg * E + (k + seg) % E, so that the
  // lanes of one atomic instruction (same k, different segments) use different banks.
  extern __shared__ uint32_t lkey[];
  for (int i = tid; i < HD; i += kV3WG) {
    lkey[i] = 0xffffffffu;
    lkey[HD + i] = 0u;
  }
  float mn[E], mx[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    mn[i] = __builtin_inff();
    mx[i] = -__builtin_inff();
  }
  bool any = false;
  const int64_t stride = gridDim.x;
  for (int64_t p0 = blockIdx.x; p0 < passes; p0 += kV3Ahead * stride) {
    uint32_t w[kV3Ahead][E / 2];
#pragma unroll
    for (int u = 0; u < kV3Ahead; ++u) {
      const int64_t hr = (p0 + u * stride) * kV3Rows + Q;
      if (hr < hrows) load_bf16_seg<E>(x + hr * D + q * E, w[u]);
    }
#pragma unroll
    for (int u = 0; u < kV3Ahead; ++u) {
      const int64_t hr = (p0 + u * stride) * kV3Rows + Q;
      if (hr >= hrows) continue;  // a quad's lanes share hr: the quad shuffles stay whole
      any = true;
      float y[E];
      v3_transform_w<D>(w[u], sb, sh.scale, q, y);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        mn[i] = fminf(mn[i], y[i]);
        mx[i] = fmaxf(mx[i], y[i]);
      }
    }
  }
  __syncthreads();
  if (any) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int seg = h * 4 + q, slot = seg * E + ((i + seg) & (E - 1));
      atomicMin(&lkey[slot], f2key(mn[i]));
      atomicMax(&lkey[HD + slot], f2key(mx[i]));
    }
  }
  __syncthreads();
  uint32_t* out = kpart + (int64_t)blockIdx.x * 2 * HD;
  for (int i = tid; i < HD; i += kV3WG) {
    const int seg = i / E, slot = seg * E + ((i + seg) & (E - 1));
    gst(out + i, lkey[slot]);
    gst(out + HD + i, lkey[HD + slot]);
  }
}

// K statistics over the partials -> kmeta [2][H][D] = (min, scale).  A workgroup
// takes 4 channels: lane j = tid & 3 of every quad reads channel 4 * blockIdx.x + j
// of the partials s, s + 64, ... (s = tid >> 2, so every load of a lane is
// independent), then the 64 slices are reduced across the wave and the 4 waves.
__global__ __launch_bounds__(kV3WG) void v3_kfinal_kernel(int HD, int D, int nparts, const uint32_t* __restrict__ kpart,
                                                          const float* __restrict__ levels, float* __restrict__ kmeta) {
  const int j = threadIdx.x & 3, s = threadIdx.x >> 2;
  // The 8 workgroups whose channels share a 128-byte line of the partials take ids
  // equal mod 8, i.e. the same XCD under round-robin dispatch, so that one L2 fetch
  // serves them all (when the grid is a multiple of 64; else the plain order).
  const int wg = blockIdx.x;
  const int grp = (gridDim.x % 64 == 0) ? 8 * ((wg % 8) + 8 * (wg / 64)) + (wg / 8) % 8 : wg;
  const int c = grp * 4 + j;
  uint32_t a = 0xffffffffu, b = 0u;
  if (c < HD) {
    for (int w = s; w < nparts; w += kV3WG / 4) {
      a = min(a, gld(kpart + (int64_t)w * 2 * HD + c));
      b = max(b, gld(kpart + (int64_t)w * 2 * HD + HD + c));
    }
  }
#pragma unroll
  for (int m = 4; m < 64; m <<= 1) {  // lanes of equal j within the wave
    a = min(a, (uint32_t)__shfl_xor((int)a, m));
    b = max(b, (uint32_t)__shfl_xor((int)b, m));
  }
  __shared__ uint32_t la[kV3WG / 64][4], lb[kV3WG / 64][4];
  const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
  if (ln < 4) {
    la[wv][ln] = a;
    lb[wv][ln] = b;
  }
  __syncthreads();
  if (threadIdx.x >= 4 || c >= HD) return;
#pragma unroll
  for (int v = 1; v < kV3WG / 64; ++v) {
    a = min(a, la[v][j]);
    b = max(b, lb[v][j]);
  }
  const float mn = key2f(a), mx = key2f(b);
  const float lv = gld(levels + c / D);
  gst(kmeta + c, mn);
  gst(kmeta + HD + c, fmaxf(mx - mn, 1e-5f) / (lv - 1.0f));
}

// ------------------------------------------------------------------ quantize
// Symbols leave through streaming stores: 3-4 % faster compress than cached stores
// (the same stores for dequant's bf16 output were 1.6x slower, so that one stays cached).
template <int E>
__device__ __forceinline__ void v3_store_symbols(uint8_t* p, const uint32_t (&sym)[E]) {
  uint32_t w[E / 4];
#pragma unroll
  for (int i = 0; i < E / 4; ++i)
    w[i] = sym[4 * i] | (sym[4 * i + 1] << 8) | (sym[4 * i + 2] << 16) | (sym[4 * i + 3] << 24);
  uint4* o = reinterpret_cast<uint4*>(p);
#pragma unroll
  for (int i = 0; i < E / 16; ++i) gst_stream(o + i, make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]));
}

// blockIdx.y = part (0 = K, 1 = V).  hrows is a multiple of H and 64 % H == 0, so a
// pass of 64 consecutive head-rows holds whole rows, each entirely inside or entirely
// past the layer; lanes past it load and store nothing but still reach the V branch's
// barriers (the pass count is uniform over the workgroup).
template <int D>
__global__ __launch_bounds__(kV3WG) void v3_quant_kernel(V3Shape sh, const uint16_t* __restrict__ x,
                                                         const uint32_t* __restrict__ signs,
                                                         const float* __restrict__ levels,
                                                         const int32_t* __restrict__ vgroup,
                                                         const float* __restrict__ kmeta, uint8_t* __restrict__ qout,
                                                         float* __restrict__ vmeta) {
  constexpr int E = D / 4;
  const int part = blockIdx.y;
  const int H = sh.H, HD = H * D;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3, h = Q % H;
  const int64_t hrows = sh.rows * H;
  const uint16_t* src = x + part * hrows * D;
  uint8_t* dst = qout + part * hrows * D;
  const uint32_t sb = v3_lane_signs<D>(signs, h, q);
  const float lv = gld(levels + part * H + h);
  const int64_t passes = (hrows + kV3Rows - 1) / kV3Rows;
  // heads of this head's V group (equal L), as a bit set over the row's heads
  uint64_t same = 0;
  if (part == 1) {
    const int grp = gld(vgroup + h);
    for (int k = 0; k < H; ++k)
      if (gld(vgroup + k) == grp) same |= (uint64_t)1 << k;
  }
  __shared__ float lmn[kV3Rows], lmx[kV3Rows];
  const int row0 = Q - h;  // this pass's LDS slot of head 0 of the lane's row
  for (int64_t p = blockIdx.x; p < passes; p += gridDim.x) {
    const int64_t hr = p * kV3Rows + Q;
    const bool live = hr < hrows;
    float y[E];
    if (live) {
      v3_transform<D>(src + hr * D + q * E, sb, sh.scale, q, y);
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) y[i] = 0.0f;
    }
    uint32_t sym[E];
    if (part == 0) {
      if (!live) continue;
      const float* kmn = kmeta + h * D + q * E;
#pragma unroll
      for (int i = 0; i < E; ++i) sym[i] = v3_symbol(round_bf16(y[i]), gld(kmn + i), gld(kmn + HD + i), lv);
    } else {
      float mn = y[0], mx = y[0];
#pragma unroll
      for (int i = 1; i < E; ++i) {
        mn = fminf(mn, y[i]);
        mx = fmaxf(mx, y[i]);
      }
      mn = quad_min(mn);
      mx = quad_max(mx);
      __syncthreads();  // the previous pass's readers are done
      if (q == 0) {
        lmn[Q] = mn;
        lmx[Q] = mx;
      }
      __syncthreads();
      if (!live) continue;  // no barrier follows in this pass
      // the row's statistics over the heads of this head's group
      float gmn = __builtin_inff(), gmx = -__builtin_inff();
      for (uint64_t m = same; m; m &= m - 1) {
        const int k = __builtin_ctzll(m);
        gmn = fminf(gmn, lmn[row0 + k]);
        gmx = fmaxf(gmx, lmx[row0 + k]);
      }
      const float sc = fmaxf(gmx - gmn, 1e-5f) / (lv - 1.0f);
      if (q == 0) {
        gst(vmeta + hr, gmn);
        gst(vmeta + hrows + hr, sc);
      }
#pragma unroll
      for (int i = 0; i < E; ++i) sym[i] = v3_symbol(round_bf16(y[i]), gmn, sc, lv);
    }
    v3_store_symbols<E>(dst + hr * D + q * E, sym);
  }
}

// ------------------------------------------------------------------ dequantize
template <int E>
__device__ __forceinline__ void v3_load_symbols(const uint8_t* p, uint32_t (&w)[E / 4]) {
  const uint4* s4 = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < E / 16; ++i) {
    const uint4 t = gld(s4 + i);
    w[4 * i] = t.x;
    w[4 * i + 1] = t.y;
    w[4 * i + 2] = t.z;
    w[4 * i + 3] = t.w;
  }
}

// fp32 butterflies of the lane's reconstructed values, bf16((y * (1/sqrt(D))) * s) as
// E/2 words: the sign is exact after rounding.
template <int D>
__device__ __forceinline__ void v3_inverse_words(float (&v)[D / 4], uint32_t sb, float scale, int q,
                                                 uint32_t (&o)[D / 8]) {
  constexpr int E = D / 4;
  fwht_row<E>(v, q);
#pragma unroll
  for (int i = 0; i < E / 2; ++i) o[i] = pack_bf16x2(v[2 * i] * scale, v[2 * i + 1] * scale);
  apply_sign_bf16<E>(o, sb);
}

// The output leaves through a per-wave LDS stage: lane l puts its W = E/2 words at row
// l (rows padded to W + 4 words against bank conflicts), then the wave stores 16-byte
// chunk f = c * 64 + lane, i.e. chunk f % (W/4) of lane f / (W/4)'s segment, so that
// consecutive lanes store consecutive bytes of each head-row (a lane's own segment at
// a 2E-byte lane stride writes at a far lower rate).
template <int W>
__device__ __forceinline__ void v3_stage_put(uint32_t* ws, int lane, const uint32_t (&o)[W]) {
  uint4* row = reinterpret_cast<uint4*>(ws + lane * (W + 4));
#pragma unroll
  for (int i = 0; i < W / 4; ++i) row[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// K passes are head-major: a pass is 64 rows of one head, so the quads of a wave read
// the same channel constants (one broadcast line per lane position, not one copy per
// quad).  V passes are 64 consecutive head-rows.  Every lane takes part in the staged
// store (a chunk is written only if its head-row exists), so no lane leaves a pass
// early.
template <int D>
__global__ __launch_bounds__(kV3WG) void v3_dequant_kernel(V3Shape sh, const uint8_t* __restrict__ qin,
                                                           const uint32_t* __restrict__ signs,
                                                           const uint16_t* __restrict__ kmeta16,
                                                           const uint16_t* __restrict__ vmeta16,
                                                           uint16_t* __restrict__ out) {
  constexpr int E = D / 4, W = E / 2, CH = W / 4;  // words and 16-byte chunks of a segment
  const int part = blockIdx.y;
  const int H = sh.H, HD = H * D;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3, lane = tid & 63, qw = (tid >> 6) * 16;
  const int64_t hrows = sh.rows * H;
  const uint8_t* src = qin + part * hrows * D;
  uint16_t* dst = out + part * hrows * D;
  __shared__ __align__(16) uint32_t stage[kV3WG / 64][64 * (W + 4)];
  uint32_t* ws = stage[tid >> 6];
  if (part == 0) {
    const int64_t kpasses = (sh.rows + kV3Rows - 1) / kV3Rows * H;
    for (int64_t p = blockIdx.x; p < kpasses; p += gridDim.x) {
      const int hk = (int)(p % H);
      const int64_t r0 = (p / H) * kV3Rows;  // row of quad 0 of the pass
      const int64_t r = r0 + Q;
      if (r < sh.rows) {
        const int64_t hr = r * H + hk;
        uint32_t w[E / 4];
        v3_load_symbols<E>(src + hr * D + q * E, w);
        const uint4* mn = reinterpret_cast<const uint4*>(kmeta16 + hk * D + q * E);  // 16-byte aligned
        const uint4* sc = reinterpret_cast<const uint4*>(kmeta16 + HD + hk * D + q * E);
        float v[E];
#pragma unroll
        for (int i8 = 0; i8 < E / 8; ++i8) {
          const uint4 m4 = gld(mn + i8), c4 = gld(sc + i8);
          const uint32_t mw[4] = {m4.x, m4.y, m4.z, m4.w}, cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int i = 8 * i8 + k;
            const float sym = (float)((w[i / 4] >> (8 * (i % 4))) & 0xffu);
            v[i] = __builtin_fmaf(sym, f16_to_f32((uint16_t)(cw[k / 2] >> (16 * (k & 1)))),
                                  f16_to_f32((uint16_t)(mw[k / 2] >> (16 * (k & 1)))));
          }
        }
        uint32_t o[W];
        v3_inverse_words<D>(v, v3_lane_signs<D>(signs, hk, q), sh.scale, q, o);
        v3_stage_put<W>(ws, lane, o);
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int f = c * 64 + lane, sl = f / CH, k = f % CH;  // source lane, its chunk
        const int64_t rs = r0 + qw + (sl >> 2);
        if (rs < sh.rows) {
          const uint4 t = *reinterpret_cast<const uint4*>(ws + sl * (W + 4) + 4 * k);
          gst(reinterpret_cast<uint4*>(dst + (rs * H + hk) * D + (sl & 3) * E + 8 * k), t);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }
  const uint32_t sb = v3_lane_signs<D>(signs, Q % H, q);
  const int64_t passes = (hrows + kV3Rows - 1) / kV3Rows;
  for (int64_t p = blockIdx.x; p < passes; p += gridDim.x) {
    const int64_t h0 = p * kV3Rows;  // head-row of quad 0 of the pass
    const int64_t hr = h0 + Q;
    if (hr < hrows) {
      uint32_t w[E / 4];
      v3_load_symbols<E>(src + hr * D + q * E, w);
      const float mn = f16_to_f32(gld(vmeta16 + hr)), sc = f16_to_f32(gld(vmeta16 + hrows + hr));
      float v[E];
#pragma unroll
      for (int i = 0; i < E; ++i) v[i] = __builtin_fmaf((float)((w[i / 4] >> (8 * (i % 4))) & 0xffu), sc, mn);
      uint32_t o[W];
      v3_inverse_words<D>(v, sb, sh.scale, q, o);
      v3_stage_put<W>(ws, lane, o);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int f = c * 64 + lane, sl = f / CH, k = f % CH;
      const int64_t hs = h0 + qw + (sl >> 2);
      if (hs < hrows) {
        const uint4 t = *reinterpret_cast<const uint4*>(ws + sl * (W + 4) + 4 * k);
        gst(reinterpret_cast<uint4*>(dst + hs * D + (sl & 3) * E + 8 * k), t);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------------------------ launch
// rows * H <= 2^29 head-rows: at most 2^23 workgroups of 256 threads, so the grid stays
// below HIP's 2^32 work-items per dimension.
int v3_check(int64_t rows, int32_t H, int32_t D) {
  if (rows < 0 || H < 1 || H > kV3MaxH || (kV3Rows % H) != 0 || (D != 64 && D != 128)) return KVMI_EINVAL;
  if (rows * H > (int64_t)1 << 29) return KVMI_EINVAL;
  return KVMI_OK;
}

// One pass per workgroup (at most 2^23 workgroups, see v3_check): capping the grid at
// 4096 and looping measured 12-14 % slower for dequant at 128-512 Ki rows.
unsigned v3_grid(int64_t rows, int H) {
  const int64_t passes = (rows * H + kV3Rows - 1) / kV3Rows;
  return (unsigned)(passes > 0 ? passes : 1);
}

// Workgroups of the K statistics pass, i.e. the K partials one call writes and reads.
unsigned v3_kgrid(int64_t rows, int H) {
  const unsigned g = v3_grid(rows, H);
  return g < (unsigned)kV3KGrid ? g : (unsigned)kV3KGrid;
}

// The three launches of compress with the K partials at `kpart`
// (v3_kgrid(rows, H) * 2 * H * D uint32; every one is written before it is read).
int v3_compress_launch(const void* x, int64_t rows, int32_t H, int32_t D, const uint32_t* signs,
                       const float* levels, const int32_t* vgroup, uint8_t* q, float* kmeta, float* vmeta,
                       uint32_t* kpart, hipStream_t st) {
  V3Shape sh{rows, H, (float)(1.0 / __builtin_sqrt((double)D))};
  const unsigned g = v3_grid(rows, H);
  const unsigned gk = v3_kgrid(rows, H);
  const size_t klds = (size_t)2 * H * D * 4;
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  const unsigned gf = (unsigned)((H * D + 3) / 4);  // 4 channels per workgroup
  if (D == 64)
    hipLaunchKernelGGL((v3_kstats_kernel<64>), dim3(gk), dim3(kV3WG), klds, st, sh, xs, signs, kpart);
  else
    hipLaunchKernelGGL((v3_kstats_kernel<128>), dim3(gk), dim3(kV3WG), klds, st, sh, xs, signs, kpart);
  hipLaunchKernelGGL(v3_kfinal_kernel, dim3(gf), dim3(kV3WG), 0, st, H * D, D, (int)gk, kpart, levels, kmeta);
  if (D == 64)
    hipLaunchKernelGGL((v3_quant_kernel<64>), dim3(g, 2), dim3(kV3WG), 0, st, sh, xs, signs, levels, vgroup, kmeta,
                       q, vmeta);
  else
    hipLaunchKernelGGL((v3_quant_kernel<128>), dim3(g, 2), dim3(kV3WG), 0, st, sh, xs, signs, levels, vgroup, kmeta,
                       q, vmeta);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int v3_compress_args(const void* x, int64_t rows, int32_t H, int32_t D, const uint32_t* signs, const float* levels,
                     const int32_t* vgroup, const uint8_t* q, const float* kmeta, const float* vmeta) {
  if (!x || !signs || !levels || !vgroup || !q || !kmeta || !vmeta) return KVMI_EINVAL;
  if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)kmeta) & 15) return KVMI_EINVAL;  // 16-byte vectors
  return KVMI_OK;
}

// ------------------------------------------------------------------ no-allocation variant
// The K partials of kvmi_v3_compress_noalloc live in this fixed device array (one copy
// per GPU, held until the process ends).  Host code never passes the array's name to a
// kernel: the name is a host-side stand-in, and the device address of each GPU's copy
// comes from hipGetSymbolAddress (with that GPU current), once per device.
static __device__ __align__(256) uint8_t scratch[KVMI_V3_NOALLOC_SCRATCH_BYTES];

// Calls on one GPU share its array, so they are put in one order: each call's launches
// wait (hipStreamWaitEvent) for the event recorded after the previous call's launches on
// that GPU, whichever stream or host thread made it, and the mutex keeps the wait, the
// launches and the record of one call together.  Launches enqueued under graph capture
// take no part (an event of an eager call cannot be waited on inside a capture): a
// replayed graph is ordered only by the stream it is launched on.
constexpr int kMaxScratchDevices = 64;
struct NoAllocSlot {
  void* ptr = nullptr;         // device address of this GPU's copy of `scratch`
  hipEvent_t done = nullptr;   // recorded after the last eager call's launches
  bool recorded = false;
};
std::mutex g_scratch_mu;
NoAllocSlot g_scratch[kMaxScratchDevices];

// The current GPU's slot, set up on its first use (null on failure); g_scratch_mu held.
NoAllocSlot* noalloc_slot() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return nullptr;
  NoAllocSlot& sl = g_scratch[dev];
  if (!sl.ptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    if (hipEventCreateWithFlags(&sl.done, hipEventDisableTiming) != hipSuccess) return nullptr;
    sl.ptr = p;
  }
  return &sl;
}

}  // namespace
}  // namespace kvmi

extern "C" int64_t kvmi_v3_scratch_bytes(int64_t rows, int32_t num_heads, int32_t head_dim) {
  using namespace kvmi;
  if (v3_check(rows, num_heads, head_dim)) return -1;
  return (int64_t)kV3KGrid * 2 * num_heads * head_dim * 4;
}

extern "C" int kvmi_v3_compress(const void* x, int64_t rows, int32_t num_heads, int32_t head_dim,
                                const uint32_t* signs, const float* levels, const int32_t* vgroup, uint8_t* q,
                                float* kmeta, float* vmeta, void* workspace, kvmi_stream_t stream) {
  using namespace kvmi;
  int rc = v3_check(rows, num_heads, head_dim);
  if (rc) return rc;
  if (rows == 0) return KVMI_OK;
  rc = v3_compress_args(x, rows, num_heads, head_dim, signs, levels, vgroup, q, kmeta, vmeta);
  if (rc) return rc;
  if (!workspace) return KVMI_EINVAL;
  return v3_compress_launch(x, rows, num_heads, head_dim, signs, levels, vgroup, q, kmeta, vmeta,
                            static_cast<uint32_t*>(workspace), reinterpret_cast<hipStream_t>(stream));
}

extern "C" int kvmi_v3_compress_noalloc(const void* x, int64_t rows, int32_t num_heads, int32_t head_dim,
                                        const uint32_t* signs, const float* levels, const int32_t* vgroup,
                                        uint8_t* q, float* kmeta, float* vmeta, kvmi_stream_t stream) {
  using namespace kvmi;
  int rc = v3_check(rows, num_heads, head_dim);
  if (rc) return rc;
  if (rows == 0) return KVMI_OK;
  rc = v3_compress_args(x, rows, num_heads, head_dim, signs, levels, vgroup, q, kmeta, vmeta);
  if (rc) return rc;
  // K partials of this call: v3_kgrid workgroups x 2 x H x D keys
  const int64_t need = (int64_t)v3_kgrid(rows, num_heads) * 2 * num_heads * head_dim * 4;
  if (need > KVMI_V3_NOALLOC_SCRATCH_BYTES) return KVMI_ENOSPC;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  NoAllocSlot* sl = noalloc_slot();
  if (!sl) return KVMI_ELAUNCH;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) return KVMI_ELAUNCH;
  const bool ordered = cap == hipStreamCaptureStatusNone;
  if (ordered && sl->recorded && hipStreamWaitEvent(st, sl->done, 0) != hipSuccess) return KVMI_ELAUNCH;
  rc = v3_compress_launch(x, rows, num_heads, head_dim, signs, levels, vgroup, q, kmeta, vmeta,
                          static_cast<uint32_t*>(sl->ptr), st);
  if (rc == KVMI_OK && ordered) {
    if (hipEventRecord(sl->done, st) != hipSuccess) return KVMI_ELAUNCH;
    sl->recorded = true;
  }
  return rc;
}

extern "C" int kvmi_v3_decompress(const uint8_t* q, int64_t rows, int32_t num_heads, int32_t head_dim,
                                  const uint32_t* signs, const uint16_t* kmeta16, const uint16_t* vmeta16, void* out,
                                  kvmi_stream_t stream) {
  using namespace kvmi;
  int rc = v3_check(rows, num_heads, head_dim);
  if (rc) return rc;
  if (rows == 0) return KVMI_OK;
  if (!q || !signs || !kmeta16 || !vmeta16 || !out) return KVMI_EINVAL;
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)kmeta16) & 15) return KVMI_EINVAL;  // 16-byte vectors
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  V3Shape sh{rows, num_heads, (float)(1.0 / __builtin_sqrt((double)head_dim))};
  const unsigned g = v3_grid(rows, num_heads);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (head_dim == 64)
    hipLaunchKernelGGL((v3_dequant_kernel<64>), dim3(g, 2), dim3(kV3WG), 0, st, sh, q, signs, kmeta16, vmeta16, o);
  else
    hipLaunchKernelGGL((v3_dequant_kernel<128>), dim3(g, 2), dim3(kV3WG), 0, st, sh, q, signs, kmeta16, vmeta16, o);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}
