// Generic-geometry paged compress / decompress kernels for gfx950 (register FWHT).
//
// They serve the geometries the MFMA and quad-per-row kernels do not: any H up to 64
// and any D that is a multiple of 16 up to 256, with H * next_pow2(D) <= 8192.  A D
// that is not a power of two is transformed as the reference does it
// (hadamard_func.py:50-103): split into descending power-of-two chunks, each chunk
// transformed on its own with scale 1/sqrt(chunk).
//
// Row mapping.  A row (one token x one KV head, D contiguous bf16) is held by LPR =
// next_pow2(D/16) lanes, lane `sub` owning the 16 contiguous channels [16 sub, 16 sub
// + 16); lanes with 16 sub >= D only pad the row.  A workgroup of 512 threads holds
// P = 512 / LPR row slots and processes RP = floor(P / H) * H rows per pass (whole
// tokens), so slot i always sees head i % H: its signs, its K statistics and its K
// quantization constants stay in registers across passes.  A chunk of c channels
// spans c/16 lanes and starts at a lane index that is a multiple of c/16, so its
// cross-lane butterflies are lane-xor exchanges inside the chunk; the FWHT stage order
// is the oracle's (index bits from the lowest up: 4 in-lane, then across lanes).
//
// Compress is kstats (this file) + kstats_finalize (kvmi_codec.hip) + encode; decode
// is one launch -- the same passes, metadata and stream layout as the other families.
#include "kvmi_common.hpp"

namespace kvmi {
namespace {

constexpr int kRWG = 512;  // threads per workgroup
constexpr int kSeg = 16;   // channels per lane

// fp32 values of 1/sqrt(c) for c = 16, 32, .., 256 (computed in double on the host and
// rounded once, as the reference passes the Python float 1/sqrt(size)).
struct ChunkScales {
  float s[5];
};

// A lane's place in its row: segment, whether it holds channels, and the chunk that
// contains them (lanes of the chunk, scale).
struct Lane {
  int slot, sub;
  bool seg_ok;
  int chunk_lanes;
  float scale;
};

template <int LPR>
__device__ __forceinline__ Lane lane_of(int D, const ChunkScales& cs) {
  Lane l;
  l.slot = threadIdx.x / LPR;
  l.sub = threadIdx.x % LPR;
  const int c0 = l.sub * kSeg;
  l.seg_ok = c0 < D;
  l.chunk_lanes = 1;
  l.scale = cs.s[0];
  int start = 0;  // first channel of the chunk of size c (chunks descend, as D's bits)
#pragma unroll
  for (int b = 8; b >= 4; --b) {
    const int c = 1 << b;
    if (!(D & c)) continue;
    if (c0 >= start && c0 < start + c) {
      l.chunk_lanes = c / kSeg;
      l.scale = cs.s[b - 4];
    }
    start += c;
  }
  return l;
}

// Butterfly stages across lanes J, 2J, .. < LPR, each applied only inside the lane's
// chunk (J < chunk lanes).  The lane with bit J clear holds the lower element a and
// gets a + b, the other gets a - b = partner - own: one fp32 rounding either way.
template <int J, int LPR>
__device__ __forceinline__ void cross_stages(float (&v)[kSeg], int sub, int chunk_lanes) {
  if constexpr (J < LPR) {
    const float sgn = (sub & J) ? -1.0f : 1.0f;
    const bool on = J < chunk_lanes;
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      const float r = __builtin_fmaf(v[i], sgn, lane_xor<J>(v[i]));
      v[i] = on ? r : v[i];
    }
    cross_stages<J * 2, LPR>(v, sub, chunk_lanes);
  }
}

template <int LPR>
__device__ __forceinline__ void fwht_seg(float (&v)[kSeg], const Lane& l) {
  fwht_in_lane<kSeg>(v);
  cross_stages<1, LPR>(v, l.sub, l.chunk_lanes);
}

template <int LPR>
__device__ __forceinline__ float row_min(float x) {
  if constexpr (LPR > 1) x = fminf(x, lane_xor<1>(x));
  if constexpr (LPR > 2) x = fminf(x, lane_xor<2>(x));
  if constexpr (LPR > 4) x = fminf(x, lane_xor<4>(x));
  if constexpr (LPR > 8) x = fminf(x, lane_xor<8>(x));
  return x;
}
template <int LPR>
__device__ __forceinline__ float row_max(float x) {
  if constexpr (LPR > 1) x = fmaxf(x, lane_xor<1>(x));
  if constexpr (LPR > 2) x = fmaxf(x, lane_xor<2>(x));
  if constexpr (LPR > 4) x = fmaxf(x, lane_xor<4>(x));
  if constexpr (LPR > 8) x = fmaxf(x, lane_xor<8>(x));
  return x;
}

// Sign bits of the lane's 16 channels of head h (signs: [H][ceil(D/32)] words).
__device__ __forceinline__ uint32_t seg_signs(const uint32_t* signs, int h, int D, const Lane& l) {
  if (!l.seg_ok) return 0u;
  const uint32_t w = gld(signs + h * ((D + 31) / 32) + (l.sub >> 1));
  return (w >> ((l.sub & 1) * 16)) & 0xffffu;
}

// Load the lane's 16 channels, apply signs + chunked FWHT + scale (unless transform
// is off) and return fp32 values (ROUND: rounded to bf16).  Padding lanes load nothing.
template <int LPR, bool ROUND>
__device__ __forceinline__ void load_transform(const uint16_t* src, const Lane& l, uint32_t sb, bool transform,
                                               float (&y)[kSeg]) {
  uint32_t w[kSeg / 2];
  if (l.seg_ok) {
    load_bf16_seg<kSeg>(src, w);
  } else {
#pragma unroll
    for (int i = 0; i < kSeg / 2; ++i) w[i] = 0u;
  }
  if (transform) apply_sign_bf16<kSeg>(w, sb);
  unpack_bf16<kSeg>(w, y);
  if (transform) {
    fwht_seg<LPR>(y, l);
#pragma unroll
    for (int i = 0; i < kSeg; ++i) y[i] = ROUND ? round_bf16(y[i] * l.scale) : y[i] * l.scale;
  }
}

struct Pass {
  int RP;    // rows per pass (whole tokens)
  bool on;   // this lane's slot is used
  int h;     // its head
};
template <int LPR>
__device__ __forceinline__ Pass pass_of(int H, const Lane& l) {
  constexpr int P = kRWG / LPR;
  Pass p;
  p.RP = (P / H) * H;
  p.on = l.slot < p.RP;
  p.h = l.slot % H;
  return p;
}

// ============================================================== K statistics
template <int LPR>
__global__ __launch_bounds__(kRWG) void rows_kstats_kernel(Geo g, ChunkScales cs,
                                                           const kvmi_layer_job* __restrict__ jobs) {
  extern __shared__ uint32_t lkey[];  // [2][H*D]: min keys, then max keys
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) return;
  const int H = g.H, S = g.S, D = g.D, HD = H * D;
  const int blk0 = blockIdx.x * g.bpw;
  const int64_t rows = (int64_t)(min(B, blk0 + g.bpw) - blk0) * S * H;
  const Lane l = lane_of<LPR>(D, cs);
  const Pass ps = pass_of<LPR>(H, l);
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? seg_signs(job.signs, ps.h, D, l) : 0u;

  for (int i = threadIdx.x; i < HD; i += kRWG) {
    lkey[i] = 0xffffffffu;
    lkey[HD + i] = 0u;
  }
  float mn[kSeg], mx[kSeg];
#pragma unroll
  for (int i = 0; i < kSeg; ++i) {
    mn[i] = __builtin_inff();
    mx[i] = -__builtin_inff();
  }
  const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool);
  bool any = false;
  for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
    if (ps.on && rp.active) {
      float y[kSeg];
      load_transform<LPR, false>(pool + rp.pool_row * D + l.sub * kSeg, l, sb, transform, y);
      any = true;
#pragma unroll
      for (int i = 0; i < kSeg; ++i) {
        mn[i] = fminf(mn[i], y[i]);
        mx[i] = fmaxf(mx[i], y[i]);
      }
    }
  }
  __syncthreads();
  // channel c = seg * 16 + i (seg = c / 16) sits at seg * 16 + (i + seg) % 16, so that
  // the lanes of one atomic instruction (same i, different segments) use different banks
  if (any && l.seg_ok) {
    const int seg = (ps.h * D) / kSeg + l.sub;
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      const int slot = seg * kSeg + ((i + seg) & (kSeg - 1));
      atomicMin(&lkey[slot], f2key(mn[i]));
      atomicMax(&lkey[HD + slot], f2key(mx[i]));
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kRWG) {
    const int seg = i / kSeg, slot = seg * kSeg + ((i + seg) & (kSeg - 1));
    const uint32_t kmn = lkey[slot], kmx = lkey[HD + slot];
    if (kmn != 0xffffffffu) atomicMin(&job.kstats[i], kmn);
    if (kmx != 0u) atomicMax(&job.kstats[HD + i], kmx);
  }
}

// Source head -> output position of both parts, in LDS.
__device__ __forceinline__ void positions(const kvmi_layer_job& job, int H, int* posk, int* posv) {
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);
  if ((int)threadIdx.x < H) {
    posk[gld(pk.order + threadIdx.x)] = threadIdx.x;
    posv[gld(pv.order + threadIdx.x)] = threadIdx.x;
  }
}

// ============================================================== encode
template <int LPR, int BITS>
__global__ __launch_bounds__(kRWG) void rows_encode_kernel(Geo g, ChunkScales cs,
                                                           const kvmi_layer_job* __restrict__ jobs,
                                                           int32_t* __restrict__ err) {
  constexpr int P = kRWG / LPR;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) {
    // a job without blocks still heads its chunk (the stream of N = 0 symbols)
    if (nwg == 0 && blockIdx.x == 0 && threadIdx.x == 0 && job.write_header && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
    return;
  }
  const int H = g.H, S = g.S, D = g.D, HD = H * D, G = g.G;
  const int blk0 = blockIdx.x * g.bpw;
  const int64_t rows = (int64_t)(min(B, blk0 + g.bpw) - blk0) * S * H;
  const Lane l = lane_of<LPR>(D, cs);
  const Pass ps = pass_of<LPR>(H, l);
  const int tid = threadIdx.x;
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? seg_signs(job.signs, ps.h, D, l) : 0u;
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);

  __shared__ int posk[kMaxHeads], posv[kMaxHeads];
  __shared__ float2 rowmm[P];  // V row (min, max) by slot
  __shared__ float2 tokq[P];   // V (min, 1/scale) by (token of pass, group)
  positions(job, H, posk, posv);
  if (tid == 0 && job.write_header && blockIdx.x == 0 && !(g.flags & KVMI_F_NO_HEADER))
    write_stream_header(job.stream, BITS, job.chunk_symbols);
  int ngroups = 1;
  for (int k = 0; k < H; ++k) ngroups = max(ngroups, (int)gld(pv.group + k) + 1);
  __syncthreads();

  const int jk = posk[ps.h], jv = posv[ps.h];
  // K constants of the lane's 16 channels: (min, 1/scale) of output position jk
  float kmn[kSeg], krc[kSeg];
  {
    const int e0 = l.seg_ok ? l.sub * kSeg : 0;
    uint32_t wm[kSeg / 2], ws[kSeg / 2];
    load_bf16_seg<kSeg>(job.kmeta + jk * D + e0, wm);
    load_bf16_seg<kSeg>(job.kmeta + HD + jk * D + e0, ws);
#pragma unroll
    for (int i = 0; i < kSeg / 2; ++i) {
      kmn[2 * i] = bf_lo(wm[i]);
      kmn[2 * i + 1] = bf_hi(wm[i]);
      krc[2 * i] = 1.0f / bf_lo(ws[i]);
      krc[2 * i + 1] = 1.0f / bf_hi(ws[i]);
    }
  }
  const float lk = (float)gld(pk.levels + jk);
  const float lvv = (float)gld(pv.levels + jv);
  const int gv = gld(pv.group + jv);
  const int tpp = ps.RP / H;  // tokens per pass
  const uint16_t* poolK = reinterpret_cast<const uint16_t*>(job.pool);
  const uint16_t* poolV = poolK + job.pool_part_stride;
  const int64_t ntok = (int64_t)B * S;
  uint32_t over = 0;

  for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
    const bool act = ps.on && rp.active;  // uniform over the lanes of a row
    // ---------------- K: per-channel statistics from the kstats pass
    if (act) {
      float y[kSeg];
      load_transform<LPR, true>(poolK + rp.pool_row * D + l.sub * kSeg, l, sb, transform, y);
      if (l.seg_ok) {
        uint32_t s[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          s[i] = (uint32_t)quant_value(y[i], kmn[i], krc[i], lk);
          over |= s[i];
        }
        Packed<kSeg, BITS> pkd;
        pack_syms<kSeg, BITS>(s, pkd);
        store_packed<kSeg, BITS>(seg_addr<BITS>(job, g, 0, jk, rp.tok, l.sub * kSeg), pkd);
      }
    }
    // ---------------- V: per-token statistics over the heads of a group
    float y[kSeg];
    if (act) {
      load_transform<LPR, true>(poolV + rp.pool_row * D + l.sub * kSeg, l, sb, transform, y);
      float lmn = __builtin_inff(), lmx = -__builtin_inff();
      if (l.seg_ok) {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          lmn = fminf(lmn, y[i]);
          lmx = fmaxf(lmx, y[i]);
        }
      }
      lmn = row_min<LPR>(lmn);
      lmx = row_max<LPR>(lmx);
      if (l.sub == 0) rowmm[l.slot] = make_float2(lmn, lmx);
    }
    __syncthreads();
    if (tid < tpp * G) {
      const int tp = tid / G, gg = tid % G;
      const int64_t rr = r0 + (int64_t)tp * H;
      if (gg < ngroups && rr < rows) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
        int lv = 2;
        for (int k = 0; k < H; ++k) {
          if (gld(pv.group + k) == gg) {
            const float2 m = rowmm[tp * H + gld(pv.order + k)];
            mn = fminf(mn, m.x);
            mx = fmaxf(mx, m.y);
            lv = gld(pv.levels + k);
          }
        }
        const float sc = quant_scale(mn, mx, lv);
        tokq[tid] = make_float2(mn, 1.0f / sc);
        const RowPos tpz = row_pos(job, blk0, rows, rr, S, H);
        gst(job.vmeta + (int64_t)gg * ntok + tpz.tok, (uint16_t)f32_to_bf16_bits(mn));
        gst(job.vmeta + (int64_t)(G + gg) * ntok + tpz.tok, (uint16_t)f32_to_bf16_bits(sc));
      }
    }
    __syncthreads();
    if (act && l.seg_ok) {
      const float2 c = tokq[(l.slot / H) * G + gv];
      uint32_t s[kSeg];
#pragma unroll
      for (int i = 0; i < kSeg; ++i) {
        s[i] = (uint32_t)quant_value(y[i], c.x, c.y, lvv);
        over |= s[i];
      }
      Packed<kSeg, BITS> pkd;
      pack_syms<kSeg, BITS>(s, pkd);
      store_packed<kSeg, BITS>(seg_addr<BITS>(job, g, 1, jv, rp.tok, l.sub * kSeg), pkd);
    }
    __syncthreads();
  }
  if (over >> BITS) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
}

// ============================================================== decode
template <int LPR, int BITS>
__global__ __launch_bounds__(kRWG) void rows_decode_kernel(Geo g, ChunkScales cs,
                                                           const kvmi_layer_job* __restrict__ jobs,
                                                           int32_t* __restrict__ err) {
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) return;
  const int H = g.H, S = g.S, D = g.D, HD = H * D, G = g.G;
  const int tid = threadIdx.x;
  __shared__ int posk[kMaxHeads], posv[kMaxHeads];
  __shared__ int ok;
  if (tid == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  positions(job, H, posk, posv);
  __syncthreads();
  if (!ok) return;

  const int blk0 = blockIdx.x * g.bpw;
  const int64_t rows = (int64_t)(min(B, blk0 + g.bpw) - blk0) * S * H;
  const Lane l = lane_of<LPR>(D, cs);
  const Pass ps = pass_of<LPR>(H, l);
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? seg_signs(job.signs, ps.h, D, l) : 0u;
  const int jk = posk[ps.h], jv = posv[ps.h];
  const Profile pv = part_profile(job.profile, 1, H);
  const int gv = gld(pv.group + jv);
  float kmn[kSeg], ksc[kSeg];
  {
    const int e0 = l.seg_ok ? l.sub * kSeg : 0;
    uint32_t wm[kSeg / 2], ws[kSeg / 2];
    load_bf16_seg<kSeg>(job.kmeta + jk * D + e0, wm);
    load_bf16_seg<kSeg>(job.kmeta + HD + jk * D + e0, ws);
    unpack_bf16<kSeg>(wm, kmn);
    unpack_bf16<kSeg>(ws, ksc);
  }
  uint16_t* poolK = reinterpret_cast<uint16_t*>(job.pool);
  uint16_t* poolV = poolK + job.pool_part_stride;
  const int64_t ntok = (int64_t)B * S;

  for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
    if (!(ps.on && rp.active)) continue;  // rows are whole: every lane of a row agrees
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      uint32_t s[kSeg];
      if (l.seg_ok) {
        Packed<kSeg, BITS> pkd;
        load_packed<kSeg, BITS>(seg_addr<BITS>(job, g, part, part ? jv : jk, rp.tok, l.sub * kSeg), pkd);
        unpack_syms<kSeg, BITS>(pkd, s);
      } else {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) s[i] = 0u;
      }
      float x[kSeg];
      if (part == 0) {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) x[i] = dequant_value((float)s[i], kmn[i], ksc[i]);
      } else {
        const float mn = bf16_to_f32(gld(job.vmeta + (int64_t)gv * ntok + rp.tok));
        const float sc = bf16_to_f32(gld(job.vmeta + (int64_t)(G + gv) * ntok + rp.tok));
#pragma unroll
        for (int i = 0; i < kSeg; ++i) x[i] = dequant_value((float)s[i], mn, sc);
      }
      uint32_t w[kSeg / 2];
      if (transform) {
        fwht_seg<LPR>(x, l);
#pragma unroll
        for (int i = 0; i < kSeg / 2; ++i) w[i] = pack_bf16x2(x[2 * i] * l.scale, x[2 * i + 1] * l.scale);
        apply_sign_bf16<kSeg>(w, sb);
      } else {
#pragma unroll
        for (int i = 0; i < kSeg / 2; ++i) w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
      }
      if (l.seg_ok) store_bf16_seg<kSeg>((part ? poolV : poolK) + rp.pool_row * D + l.sub * kSeg, w);
    }
  }
}

// ============================================================== unit transform
// Contiguous rows [rows, D], row r of head r % H: forward = signs then chunked FWHT,
// inverse = chunked FWHT then signs (hadamard_func.py:161-231).  One row per LPR lanes.
template <int LPR>
__global__ __launch_bounds__(kRWG) void rows_hadamard_kernel(const uint16_t* __restrict__ in,
                                                             uint16_t* __restrict__ out, int64_t rows, int H, int D,
                                                             const uint32_t* __restrict__ signs, int inverse,
                                                             ChunkScales cs) {
  const Lane l = lane_of<LPR>(D, cs);
  const int64_t r = (int64_t)blockIdx.x * (kRWG / LPR) + l.slot;
  if (r >= rows) return;  // the lanes of a row share r
  const uint32_t sb = seg_signs(signs, (int)(r % H), D, l);
  uint32_t w[kSeg / 2];
  if (l.seg_ok) {
    load_bf16_seg<kSeg>(in + r * D + l.sub * kSeg, w);
  } else {
#pragma unroll
    for (int i = 0; i < kSeg / 2; ++i) w[i] = 0u;
  }
  if (!inverse) apply_sign_bf16<kSeg>(w, sb);
  float v[kSeg];
  unpack_bf16<kSeg>(w, v);
  fwht_seg<LPR>(v, l);
#pragma unroll
  for (int i = 0; i < kSeg / 2; ++i) w[i] = pack_bf16x2(v[2 * i] * l.scale, v[2 * i + 1] * l.scale);
  if (inverse) apply_sign_bf16<kSeg>(w, sb);
  if (l.seg_ok) store_bf16_seg<kSeg>(out + r * D + l.sub * kSeg, w);
}

// ============================================================== host side
ChunkScales chunk_scales() {
  ChunkScales cs;
  for (int b = 4; b <= 8; ++b) cs.s[b - 4] = (float)(1.0 / __builtin_sqrt((double)(1 << b)));
  return cs;
}

// Blocks per workgroup: enough for one pass of whole tokens; kstats also caps a job
// at ~16 workgroups, which keeps the global atomics per channel few.
int rows_per_pass(const Geo& g) { return (kRWG / next_pow2(g.D / kSeg) / g.H) * g.H; }
void set_rows_bpw(Geo* g, int32_t max_blocks, bool stats) {
  const int rpb = g->S * g->H, rp = rows_per_pass(*g);
  g->bpw = rpb >= rp ? 1 : (rp + rpb - 1) / rpb;
  if (stats) g->bpw = max(g->bpw, (max_blocks + 15) / 16);
}

template <int LPR>
void launch_kstats(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, hipStream_t st) {
  const size_t lds = (size_t)2 * g.H * g.D * sizeof(uint32_t);
  hipLaunchKernelGGL((rows_kstats_kernel<LPR>), grid, dim3(kRWG), lds, st, g, chunk_scales(), jobs);
}
template <int LPR, int BITS>
void launch_encode(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  hipLaunchKernelGGL((rows_encode_kernel<LPR, BITS>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
}
template <int LPR, int BITS>
void launch_decode(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  hipLaunchKernelGGL((rows_decode_kernel<LPR, BITS>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
}

template <template <int, int> class F, int LPR>
struct ByBits {
  template <class... A>
  static void run(int bits, A... a) {
    switch (bits) {
      case 1: F<LPR, 1>::go(a...); break;
      case 2: F<LPR, 2>::go(a...); break;
      case 3: F<LPR, 3>::go(a...); break;
      case 4: F<LPR, 4>::go(a...); break;
      case 5: F<LPR, 5>::go(a...); break;
      case 6: F<LPR, 6>::go(a...); break;
      case 7: F<LPR, 7>::go(a...); break;
      default: F<LPR, 8>::go(a...); break;
    }
  }
};
template <int LPR, int BITS>
struct Enc {
  static void go(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
    launch_encode<LPR, BITS>(g, grid, jobs, err, st);
  }
};
template <int LPR, int BITS>
struct Dec {
  static void go(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
    launch_decode<LPR, BITS>(g, grid, jobs, err, st);
  }
};

template <template <int, int> class F>
void by_lanes(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  switch (next_pow2(g.D / kSeg)) {
    case 1: ByBits<F, 1>::run(g.bits, g, grid, jobs, err, st); break;
    case 2: ByBits<F, 2>::run(g.bits, g, grid, jobs, err, st); break;
    case 4: ByBits<F, 4>::run(g.bits, g, grid, jobs, err, st); break;
    case 8: ByBits<F, 8>::run(g.bits, g, grid, jobs, err, st); break;
    default: ByBits<F, 16>::run(g.bits, g, grid, jobs, err, st); break;
  }
}

}  // namespace

int rows_hadamard(const void* in, void* out, int64_t rows, int32_t H, int32_t D, const uint32_t* signs,
                  int32_t inverse, hipStream_t st) {
  const int lpr = next_pow2(D / kSeg);
  const int64_t grid = (rows + kRWG / lpr - 1) / (kRWG / lpr);
  if (grid > 0x7fffffffLL) return KVMI_EINVAL;
  const uint16_t* i16 = static_cast<const uint16_t*>(in);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  const dim3 gr((unsigned)grid), bl(kRWG);
  const ChunkScales cs = chunk_scales();
  switch (lpr) {
    case 1: hipLaunchKernelGGL((rows_hadamard_kernel<1>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 2: hipLaunchKernelGGL((rows_hadamard_kernel<2>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 4: hipLaunchKernelGGL((rows_hadamard_kernel<4>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 8: hipLaunchKernelGGL((rows_hadamard_kernel<8>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    default: hipLaunchKernelGGL((rows_hadamard_kernel<16>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs); break;
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int rows_kstats(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t*,
                hipStream_t st) {
  Geo g = g0;
  set_rows_bpw(&g, max_blocks, true);
  const dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  switch (next_pow2(g.D / kSeg)) {
    case 1: launch_kstats<1>(g, grid, jobs, st); break;
    case 2: launch_kstats<2>(g, grid, jobs, st); break;
    case 4: launch_kstats<4>(g, grid, jobs, st); break;
    case 8: launch_kstats<8>(g, grid, jobs, st); break;
    default: launch_kstats<16>(g, grid, jobs, st); break;
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int rows_encode(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st) {
  Geo g = g0;
  set_rows_bpw(&g, max_blocks, false);
  const dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  by_lanes<Enc>(g, grid, jobs, err, st);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int rows_decode(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t* err,
                hipStream_t st) {
  Geo g = g0;
  set_rows_bpw(&g, max_blocks, false);
  const dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  by_lanes<Dec>(g, grid, jobs, err, st);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

}  // namespace kvmi
