// Generic-geometry paged compress / decompress kernels for gfx950 (register FWHT).
//
// They serve the geometries the MFMA and quad-per-row kernels do not: any H up to 64
// and any D that is a multiple of 16 up to 256, with H * next_pow2(D) <= 8192.  A D
// that is not a power of two is transformed as the reference does it
// (hadamard_func.py:50-103): split into descending power-of-two chunks, each chunk
// transformed on its own with scale 1/sqrt(chunk).
//
// Row mapping.  A row (one token x one KV head, D contiguous bf16) is held by LPR =
// next_pow2(ceil(D/16)) lanes, lane `sub` owning the 16 contiguous channels [16 sub,
// 16 sub + 16); lanes with 16 sub >= D only pad the row.
//
// D not a multiple of 16 (the SM variants, D even and D * bits a multiple of 8): D's
// chunks below 16 channels (8, 4, 2, 1: its low four bits, descending) all sit in the
// last, partial lane from its first channel on, each at an offset that is a multiple of
// its size (hadamard_func.py:63-64: 100 = 64 + 32 + 4).  That lane runs only the
// in-lane stages that stay inside an element's chunk, scales each element by its own
// chunk's 1/sqrt(c) and treats the channels past D as padding (never loaded, stored or
// counted in statistics).  Rows are then only 4-byte aligned in the caches (200 bytes
// at D = 100) and whole bytes but not words in the stream (50 bytes at 4 bits), so the
// SM variants move bf16 in 4-byte pieces and packed symbols byte by byte.  A workgroup of 512 threads holds
// P = 512 / LPR row slots and processes RP = floor(P / H) * H rows per pass (whole
// tokens), so slot i always sees head i % H: its signs, its K statistics and its K
// quantization constants stay in registers across passes.  A chunk of c channels
// spans c/16 lanes and starts at a lane index that is a multiple of c/16, so its
// cross-lane butterflies are lane-xor exchanges inside the chunk; the FWHT stage order
// is the oracle's (index bits from the lowest up: 4 in-lane, then across lanes).
//
// Every quantization axis runs here (quantizer_func.py:41-49): a part on the channel
// or tensor axis takes its statistics in a pass of its own over the job (reduced per
// (head, channel) or per group) before encode; a part on the token axis takes them
// inside encode, per token over the heads of a group.  Compress is stats + finalize
// (both parts) + encode; decode is one launch.
#include "kvmi_common.hpp"

namespace kvmi {
namespace {

constexpr int kRWG = 512;  // threads per workgroup
constexpr int kSeg = 16;   // channels per lane

// fp32 values of 1/sqrt(c) for c = 1, 2, 4, .., 256 (index log2 c; computed in double
// on the host and rounded once, as the reference passes the Python float 1/sqrt(size)).
struct ChunkScales {
  float s[9];
};

// A lane's place in its row: segment, whether it holds channels, and the chunk that
// contains them (lanes of the chunk, scale); `nvalid` channels of the segment are
// inside the row (16 but in the partial lane of a D with D % 16 != 0).
struct Lane {
  int slot, sub;
  bool seg_ok;
  int chunk_lanes;
  float scale;
  int nvalid;
  bool partial;
};

template <int LPR>
__device__ __forceinline__ Lane lane_of(int D, const ChunkScales& cs) {
  Lane l;
  l.slot = threadIdx.x / LPR;
  l.sub = threadIdx.x % LPR;
  const int c0 = l.sub * kSeg;
  l.seg_ok = c0 < D;
  l.nvalid = min(max(D - c0, 0), kSeg);
  l.partial = l.nvalid > 0 && l.nvalid < kSeg;
  l.chunk_lanes = 1;
  l.scale = cs.s[4];
  int start = 0;  // first channel of the chunk of size c (chunks descend, as D's bits)
#pragma unroll
  for (int b = 8; b >= 4; --b) {
    const int c = 1 << b;
    if (!(D & c)) continue;
    if (c0 >= start && c0 < start + c) {
      l.chunk_lanes = c / kSeg;
      l.scale = cs.s[b];
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

// Size of the chunk below 16 channels that holds element i of the partial lane (0 for
// padding): the chunks are the set bits of low = D % 16, descending, from element 0.
__device__ __forceinline__ int small_chunk(int i, int low) {
  int start = 0;
#pragma unroll
  for (int b = 3; b >= 0; --b) {
    const int c = 1 << b;
    if (!(low & c)) continue;
    if (i >= start && i < start + c) return c;
    start += c;
  }
  return 0;
}
// The scale of element i: its chunk's, which differs per element only in the partial lane.
template <bool SM>
__device__ __forceinline__ float elem_scale(const Lane& l, int i, int D, const ChunkScales& cs) {
  if constexpr (!SM) return l.scale;
  const int c = small_chunk(i, D & (kSeg - 1));  // wave-uniform
  return l.partial ? cs.s[c ? __builtin_ctz((unsigned)c) : 0] : l.scale;
}

template <int LPR, bool SM = false>
__device__ __forceinline__ void fwht_seg(float (&v)[kSeg], const Lane& l, int D = 0) {
  if constexpr (SM) {
    // in-lane stages, in the partial lane only inside an element's own chunk (a chunk is
    // aligned to its size, so i and i + h share it when its size exceeds h)
    const int low = D & (kSeg - 1);
#pragma unroll
    for (int h = 1; h < kSeg; h <<= 1) {
#pragma unroll
      for (int i = 0; i < kSeg; ++i) {
        if (!(i & h)) {
          const bool on = !l.partial || small_chunk(i, low) > h;
          const float a = v[i], b = v[i + h];
          v[i] = on ? a + b : a;
          v[i + h] = on ? a - b : b;
        }
      }
    }
  } else {
    fwht_in_lane<kSeg>(v);
  }
  cross_stages<1, LPR>(v, l.sub, l.chunk_lanes);
}

// bf16 segments and packed symbols of the SM variants: 4-byte pieces of the lane's
// `nvalid` channels (D is even), and the packed bytes one at a time.
__device__ __forceinline__ void load_bf16_n(const uint16_t* __restrict__ p, int nvalid, uint32_t (&w)[kSeg / 2]) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < kSeg / 2; ++i) w[i] = 2 * i < nvalid ? gld(q + i) : 0u;
}
__device__ __forceinline__ void store_bf16_n(uint16_t* __restrict__ p, int nvalid, const uint32_t (&w)[kSeg / 2]) {
  uint32_t* q = reinterpret_cast<uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < kSeg / 2; ++i)
    if (2 * i < nvalid) gst(q + i, w[i]);
}
template <int BITS>
__device__ __forceinline__ void store_packed_n(uint8_t* __restrict__ p, int nvalid, const Packed<kSeg, BITS>& v) {
  const int nb = nvalid * BITS / 8;
#pragma unroll
  for (int k = 0; k < Packed<kSeg, BITS>::kBytes; ++k)
    if (k < nb) gst(p + k, (uint8_t)(v.w[k / 4] >> (8 * (k % 4))));
}
template <int BITS>
__device__ __forceinline__ void load_packed_n(const uint8_t* __restrict__ p, int nvalid, Packed<kSeg, BITS>& v) {
  const int nb = nvalid * BITS / 8;
#pragma unroll
  for (int i = 0; i < Packed<kSeg, BITS>::kWords; ++i) v.w[i] = 0u;
#pragma unroll
  for (int k = 0; k < Packed<kSeg, BITS>::kBytes; ++k)
    if (k < nb) v.w[k / 4] |= (uint32_t)gld(p + k) << (8 * (k % 4));
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
template <int LPR, bool ROUND, bool SM>
__device__ __forceinline__ void load_transform(const uint16_t* src, const Lane& l, uint32_t sb, bool transform,
                                               float (&y)[kSeg], int D, const ChunkScales& cs) {
  uint32_t w[kSeg / 2];
  if (l.seg_ok) {
    if constexpr (SM)
      load_bf16_n(src, l.nvalid, w);
    else
      load_bf16_seg<kSeg>(src, w);
  } else {
#pragma unroll
    for (int i = 0; i < kSeg / 2; ++i) w[i] = 0u;
  }
  if (transform) apply_sign_bf16<kSeg>(w, sb);
  unpack_bf16<kSeg>(w, y);
  if (transform) {
    fwht_seg<LPR, SM>(y, l, D);
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      const float sc = elem_scale<SM>(l, i, D, cs);
      y[i] = ROUND ? round_bf16(y[i] * sc) : y[i] * sc;
    }
  }
}
// Element i of the lane is a channel of the row (all 16 unless SM and the partial lane).
template <bool SM>
__device__ __forceinline__ bool elem_ok(const Lane& l, int i) {
  return SM ? i < l.nvalid : l.seg_ok;
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

// ============================================================== per-part context
// What a lane needs to quantize its head of one part: the part's axis, the output
// position and statistic group of its head, the level count, the cache half and the
// metadata table (laid out by the axis: channel [2][H][D], token [2][G][ntok],
// tensor [2][G]).
struct PartCtx {
  int axis, j, grp;
  float level;
  Profile prof;
  uint16_t* meta;
};

__device__ __forceinline__ PartCtx part_ctx(const Geo& g, const kvmi_layer_job& job, int part, const int* pos,
                                            int h) {
  PartCtx c;
  c.axis = part_axis(g.flags, part);
  c.prof = part_profile(job.profile, part, g.H);
  c.j = pos[h];
  c.grp = gld(c.prof.group + c.j);
  c.level = (float)gld(c.prof.levels + c.j);
  c.meta = part ? job.vmeta : job.kmeta;
  return c;
}

// Source head -> output position of both parts, in LDS; statistic groups per part.
__device__ __forceinline__ void positions(const kvmi_layer_job& job, int H, int* posk, int* posv) {
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);
  if ((int)threadIdx.x < H) {
    posk[gld(pk.order + threadIdx.x)] = threadIdx.x;
    posv[gld(pv.order + threadIdx.x)] = threadIdx.x;
  }
}
__device__ __forceinline__ int group_count(const Profile& p, int H) {
  int n = 1;
  for (int k = 0; k < H; ++k) n = max(n, (int)gld(p.group + k) + 1);
  return n;
}

// The lane's quantization constants of a channel- or tensor-axis part: (min, x) per
// channel, x = 1/scale (encode) or scale (decode).
template <bool RCP, bool SM>
__device__ __forceinline__ void part_consts(const Geo& g, const PartCtx& c, const Lane& l, float (&mn)[kSeg],
                                            float (&x)[kSeg]) {
  if (c.axis == kAxChannel) {
    const int HD = g.H * g.D, e0 = l.seg_ok ? l.sub * kSeg : 0;
    uint32_t wm[kSeg / 2], ws[kSeg / 2];
    if constexpr (SM) {  // padding channels: (0, 1)
      load_bf16_n(c.meta + c.j * g.D + e0, l.nvalid, wm);
      load_bf16_n(c.meta + HD + c.j * g.D + e0, l.nvalid, ws);
#pragma unroll
      for (int i = 0; i < kSeg / 2; ++i)
        if (2 * i >= l.nvalid) ws[i] = 0x3F803F80u;
    } else {
      load_bf16_seg<kSeg>(c.meta + c.j * g.D + e0, wm);
      load_bf16_seg<kSeg>(c.meta + HD + c.j * g.D + e0, ws);
    }
    unpack_bf16<kSeg>(wm, mn);
    unpack_bf16<kSeg>(ws, x);
  } else if (c.axis == kAxTensor) {
    const float m = bf16_to_f32(gld(c.meta + c.grp)), s = bf16_to_f32(gld(c.meta + g.G + c.grp));
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      mn[i] = m;
      x[i] = s;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSeg; ++i) mn[i] = x[i] = 1.0f;  // token axis: per-token, not per-lane
  }
  if (RCP) {
#pragma unroll
    for (int i = 0; i < kSeg; ++i) x[i] = 1.0f / x[i];
  }
}

// ============================================================== statistics
// Pass 1 of compress for every part on the channel or tensor axis: min / max over all
// tokens of the job, per (head, channel) or per group, reduced through LDS atomics and
// then global atomics on order-preserving keys (part p at kstats + p * 2*H*D).
template <int LPR, bool SM>
__global__ __launch_bounds__(kRWG) void rows_stats_kernel(Geo g, ChunkScales cs,
                                                          const kvmi_layer_job* __restrict__ jobs) {
  extern __shared__ uint32_t lkey[];  // [2][H*D]: min keys, then max keys (one part at a time)
  __shared__ int pos[2][kMaxHeads];
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
  positions(job, H, pos[0], pos[1]);

#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int axis = part_axis(g.flags, part);
    if (axis == kAxToken) continue;  // uniform: per-token statistics are taken in encode
    float mn[kSeg], mx[kSeg];
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      mn[i] = __builtin_inff();
      mx[i] = -__builtin_inff();
    }
    const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool) + part * job.pool_part_stride;
    bool any = false;
    for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
      const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
      if (ps.on && rp.active) {
        float y[kSeg];
        load_transform<LPR, false, SM>(pool + rp.pool_row * D + l.sub * kSeg, l, sb, transform, y, D, cs);
        any = true;
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          if (SM && i >= l.nvalid) continue;  // padding channels
          mn[i] = fminf(mn[i], y[i]);
          mx[i] = fmaxf(mx[i], y[i]);
        }
      }
    }
    __syncthreads();  // the previous part's flush has read the LDS keys; positions are visible
    const int nkeys = axis == kAxChannel ? HD : g.G;
    for (int i = threadIdx.x; i < nkeys; i += kRWG) {
      lkey[i] = 0xffffffffu;
      lkey[HD + i] = 0u;
    }
    __syncthreads();
    if (axis == kAxChannel) {
      // channel c = seg * 16 + i (seg = c / 16) sits at seg * 16 + (i + seg) % 16, so
      // that the lanes of one atomic (same i, different segments) use different banks
      if (any && l.seg_ok) {
        const int seg = (ps.h * D) / kSeg + l.sub;
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          if (SM && i >= l.nvalid) continue;
          // SM: rows are not whole segments, so keys sit at their channel index
          const int slot = SM ? ps.h * D + l.sub * kSeg + i : seg * kSeg + ((i + seg) & (kSeg - 1));
          atomicMin(&lkey[slot], f2key(mn[i]));
          atomicMax(&lkey[HD + slot], f2key(mx[i]));
        }
      }
    } else {
      float a = __builtin_inff(), b = -__builtin_inff();
      if (l.seg_ok) {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          if (SM && i >= l.nvalid) continue;
          a = fminf(a, mn[i]);
          b = fmaxf(b, mx[i]);
        }
      }
      if (any) {  // rows are whole: every lane of a row has the same `any`
        a = row_min<LPR>(a);
        b = row_max<LPR>(b);
        if (l.sub == 0) {
          const Profile pr = part_profile(job.profile, part, H);
          const int grp = gld(pr.group + pos[part][ps.h]);
          atomicMin(&lkey[grp], f2key(a));
          atomicMax(&lkey[HD + grp], f2key(b));
        }
      }
    }
    __syncthreads();
    uint32_t* keys = job.kstats + part * 2 * HD;
    for (int i = threadIdx.x; i < nkeys; i += kRWG) {
      const int slot = axis == kAxChannel && !SM ? (i / kSeg) * kSeg + ((i + i / kSeg) & (kSeg - 1)) : i;
      const uint32_t kmn = lkey[slot], kmx = lkey[HD + slot];
      if (kmn != 0xffffffffu) atomicMin(&keys[i], kmn);
      if (kmx != 0u) atomicMax(&keys[HD + i], kmx);
    }
  }
}

// Pass 1b, one workgroup per job: keys -> metadata of every channel- or tensor-axis
// part (bf16 min and scale), keys re-initialised.  Its own launch, so every
// workgroup's atomics of pass 1 are visible without a device-wide fence.
__global__ __launch_bounds__(kRWG) void rows_finalize_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs) {
  const kvmi_layer_job job = jobs[blockIdx.x];
  if (job.num_blocks <= 0) return;  // nothing accumulated: the metadata is left as it is
  const int H = g.H, D = g.D, HD = H * D;
  __shared__ int pos[kMaxHeads];
  __shared__ uint8_t lev[kMaxHeads];
  __shared__ uint8_t glev[kMaxHeads];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int axis = part_axis(g.flags, part);
    if (axis == kAxToken) continue;
    const Profile pr = part_profile(job.profile, part, H);
    __syncthreads();  // the previous part is done with the tables
    if ((int)threadIdx.x < H) {
      const int k = threadIdx.x;
      pos[gld(pr.order + k)] = k;
      lev[k] = gld(pr.levels + k);
      glev[gld(pr.group + k)] = gld(pr.levels + k);  // one level count per group
    }
    __syncthreads();
    uint32_t* keys = job.kstats + part * 2 * HD;
    uint16_t* meta = part ? job.vmeta : job.kmeta;
    if (axis == kAxChannel) {
      for (int i = threadIdx.x; i < HD; i += kRWG) {
        const int j = pos[i / D], e = i % D;
        const float kmn = round_bf16(key2f(gld(keys + i)));
        const float kmx = round_bf16(key2f(gld(keys + HD + i)));
        gst(meta + j * D + e, (uint16_t)f32_to_bf16_bits(kmn));
        gst(meta + HD + j * D + e, (uint16_t)f32_to_bf16_bits(quant_scale(kmn, kmx, lev[j])));
        gst(keys + i, 0xffffffffu);
        gst(keys + HD + i, 0u);
      }
    } else {
      const int ng = group_count(pr, H);
      for (int i = threadIdx.x; i < ng; i += kRWG) {
        const float kmn = round_bf16(key2f(gld(keys + i)));
        const float kmx = round_bf16(key2f(gld(keys + HD + i)));
        gst(meta + i, (uint16_t)f32_to_bf16_bits(kmn));
        gst(meta + g.G + i, (uint16_t)f32_to_bf16_bits(quant_scale(kmn, kmx, glev[i])));
        gst(keys + i, 0xffffffffu);
        gst(keys + HD + i, 0u);
      }
    }
  }
}

// ============================================================== encode
// Per-token statistics of one part over the heads of each group (token axis): row
// min / max -> LDS, then one thread per (token of the pass, group) forms (min, 1/scale)
// and writes the part's token table.  Every thread of the workgroup calls this.
template <int LPR, bool SM>
__device__ __forceinline__ float2 token_stats(const Geo& g, const kvmi_layer_job& job, const PartCtx& c,
                                              const Lane& l, const Pass& ps, const float (&y)[kSeg], bool act,
                                              int64_t r0, int64_t rows, int blk0, int ngroups, float2* rowmm,
                                              float2* tokq) {
  const int H = g.H, G = g.G, tid = threadIdx.x;
  if (act) {
    float lmn = __builtin_inff(), lmx = -__builtin_inff();
    if (l.seg_ok) {
#pragma unroll
      for (int i = 0; i < kSeg; ++i) {
        if (SM && i >= l.nvalid) continue;
        lmn = fminf(lmn, y[i]);
        lmx = fmaxf(lmx, y[i]);
      }
    }
    lmn = row_min<LPR>(lmn);
    lmx = row_max<LPR>(lmx);
    if (l.sub == 0) rowmm[l.slot] = make_float2(lmn, lmx);
  }
  __syncthreads();
  const int tpp = ps.RP / H;  // tokens per pass
  if (tid < tpp * G) {
    const int tp = tid / G, gg = tid % G;
    const int64_t rr = r0 + (int64_t)tp * H;
    if (gg < ngroups && rr < rows) {
      float mn = __builtin_inff(), mx = -__builtin_inff();
      int lv = 2;
      for (int k = 0; k < H; ++k) {
        if (gld(c.prof.group + k) == gg) {
          const float2 m = rowmm[tp * H + gld(c.prof.order + k)];
          mn = fminf(mn, m.x);
          mx = fmaxf(mx, m.y);
          lv = gld(c.prof.levels + k);
        }
      }
      const float sc = quant_scale(mn, mx, lv);
      tokq[tid] = make_float2(mn, 1.0f / sc);
      const int64_t ntok = (int64_t)job.num_blocks * g.S;
      const RowPos tpz = row_pos(job, blk0, rows, rr, g.S, H);
      gst(c.meta + (int64_t)gg * ntok + tpz.tok, (uint16_t)f32_to_bf16_bits(mn));
      gst(c.meta + (int64_t)(G + gg) * ntok + tpz.tok, (uint16_t)f32_to_bf16_bits(sc));
    }
  }
  __syncthreads();
  const float2 q = act ? tokq[(l.slot / H) * G + c.grp] : make_float2(0.0f, 1.0f);
  __syncthreads();  // rowmm / tokq are reused by the next call
  return q;
}

template <int LPR, int BITS, bool SM>
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
  const int H = g.H, S = g.S, D = g.D;
  const int blk0 = blockIdx.x * g.bpw;
  const int64_t rows = (int64_t)(min(B, blk0 + g.bpw) - blk0) * S * H;
  const Lane l = lane_of<LPR>(D, cs);
  const Pass ps = pass_of<LPR>(H, l);
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? seg_signs(job.signs, ps.h, D, l) : 0u;

  __shared__ int pos[2][kMaxHeads];
  __shared__ float2 rowmm[P];  // row (min, max) by slot
  __shared__ float2 tokq[P];   // (min, 1/scale) by (token of pass, group)
  positions(job, H, pos[0], pos[1]);
  if (threadIdx.x == 0 && job.write_header && blockIdx.x == 0 && !(g.flags & KVMI_F_NO_HEADER))
    write_stream_header(job.stream, BITS, job.chunk_symbols);
  __syncthreads();

  PartCtx ctx[2];
  float cmn[2][kSeg], crc[2][kSeg];
  int ngroups[2];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    ctx[part] = part_ctx(g, job, part, pos[part], ps.h);
    part_consts<true, SM>(g, ctx[part], l, cmn[part], crc[part]);
    ngroups[part] = group_count(ctx[part].prof, H);
  }
  uint32_t over = 0;

  for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
    const bool act = ps.on && rp.active;  // uniform over the lanes of a row
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const PartCtx& c = ctx[part];
      const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool) + part * job.pool_part_stride;
      float y[kSeg];
      if (act) load_transform<LPR, true, SM>(pool + rp.pool_row * D + l.sub * kSeg, l, sb, transform, y, D, cs);
      if (c.axis == kAxToken) {  // uniform over the workgroup
        const float2 q =
            token_stats<LPR, SM>(g, job, c, l, ps, y, act, r0, rows, blk0, ngroups[part], rowmm, tokq);
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          cmn[part][i] = q.x;
          crc[part][i] = q.y;
        }
      }
      if (act && l.seg_ok) {
        uint32_t s[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
          s[i] = (uint32_t)quant_value(y[i], cmn[part][i], crc[part][i], c.level);
          if (!SM || i < l.nvalid) over |= s[i];  // padding symbols are not stored
        }
        Packed<kSeg, BITS> pkd;
        pack_syms<kSeg, BITS>(s, pkd);
        if constexpr (SM)
          store_packed_n<BITS>(seg_addr<BITS>(job, g, part, c.j, rp.tok, l.sub * kSeg), l.nvalid, pkd);
        else
          store_packed<kSeg, BITS>(seg_addr<BITS>(job, g, part, c.j, rp.tok, l.sub * kSeg), pkd);
      }
    }
  }
  if (over >> BITS) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
}

// ============================================================== decode
template <int LPR, int BITS, bool SM>
__global__ __launch_bounds__(kRWG) void rows_decode_kernel(Geo g, ChunkScales cs,
                                                           const kvmi_layer_job* __restrict__ jobs,
                                                           int32_t* __restrict__ err) {
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) return;
  const int H = g.H, S = g.S, D = g.D, G = g.G;
  __shared__ int pos[2][kMaxHeads];
  __shared__ int ok;
  if (threadIdx.x == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  positions(job, H, pos[0], pos[1]);
  __syncthreads();
  if (!ok) return;

  const int blk0 = blockIdx.x * g.bpw;
  const int64_t rows = (int64_t)(min(B, blk0 + g.bpw) - blk0) * S * H;
  const Lane l = lane_of<LPR>(D, cs);
  const Pass ps = pass_of<LPR>(H, l);
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? seg_signs(job.signs, ps.h, D, l) : 0u;
  PartCtx ctx[2];
  float cmn[2][kSeg], csc[2][kSeg];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    ctx[part] = part_ctx(g, job, part, pos[part], ps.h);
    part_consts<false, SM>(g, ctx[part], l, cmn[part], csc[part]);
  }
  const int64_t ntok = (int64_t)B * S;

  for (int64_t r0 = 0; r0 < rows; r0 += ps.RP) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + l.slot, S, H);
    if (!(ps.on && rp.active)) continue;  // rows are whole: every lane of a row agrees
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const PartCtx& c = ctx[part];
      uint32_t s[kSeg];
      if (l.seg_ok) {
        Packed<kSeg, BITS> pkd;
        if constexpr (SM)
          load_packed_n<BITS>(seg_addr<BITS>(job, g, part, c.j, rp.tok, l.sub * kSeg), l.nvalid, pkd);
        else
          load_packed<kSeg, BITS>(seg_addr<BITS>(job, g, part, c.j, rp.tok, l.sub * kSeg), pkd);
        unpack_syms<kSeg, BITS>(pkd, s);
      } else {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) s[i] = 0u;
      }
      float x[kSeg];
      if (c.axis == kAxToken) {
        const float mn = bf16_to_f32(gld(c.meta + (int64_t)c.grp * ntok + rp.tok));
        const float sc = bf16_to_f32(gld(c.meta + (int64_t)(G + c.grp) * ntok + rp.tok));
#pragma unroll
        for (int i = 0; i < kSeg; ++i) x[i] = dequant_value((float)s[i], mn, sc);
      } else {
#pragma unroll
        for (int i = 0; i < kSeg; ++i) x[i] = dequant_value((float)s[i], cmn[part][i], csc[part][i]);
      }
      uint32_t w[kSeg / 2];
      if (transform) {
        fwht_seg<LPR, SM>(x, l, D);
#pragma unroll
        for (int i = 0; i < kSeg / 2; ++i)
          w[i] = pack_bf16x2(x[2 * i] * elem_scale<SM>(l, 2 * i, D, cs), x[2 * i + 1] * elem_scale<SM>(l, 2 * i + 1, D, cs));
        apply_sign_bf16<kSeg>(w, sb);
      } else {
#pragma unroll
        for (int i = 0; i < kSeg / 2; ++i) w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
      }
      uint16_t* dst = reinterpret_cast<uint16_t*>(job.pool) + part * job.pool_part_stride + rp.pool_row * D +
                      l.sub * kSeg;
      if (l.seg_ok) {
        if constexpr (SM)
          store_bf16_n(dst, l.nvalid, w);
        else
          store_bf16_seg<kSeg>(dst, w);
      }
    }
  }
}

// ============================================================== unit transform
// Contiguous rows [rows, D], row r of head r % H: forward = signs then chunked FWHT,
// inverse = chunked FWHT then signs (hadamard_func.py:161-231).  One row per LPR lanes.
template <int LPR, bool SM>
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
    if constexpr (SM)
      load_bf16_n(in + r * D + l.sub * kSeg, l.nvalid, w);
    else
      load_bf16_seg<kSeg>(in + r * D + l.sub * kSeg, w);
  } else {
#pragma unroll
    for (int i = 0; i < kSeg / 2; ++i) w[i] = 0u;
  }
  if (!inverse) apply_sign_bf16<kSeg>(w, sb);
  float v[kSeg];
  unpack_bf16<kSeg>(w, v);
  fwht_seg<LPR, SM>(v, l, D);
#pragma unroll
  for (int i = 0; i < kSeg / 2; ++i)
    w[i] = pack_bf16x2(v[2 * i] * elem_scale<SM>(l, 2 * i, D, cs), v[2 * i + 1] * elem_scale<SM>(l, 2 * i + 1, D, cs));
  if (inverse) apply_sign_bf16<kSeg>(w, sb);
  if (l.seg_ok) {
    if constexpr (SM)
      store_bf16_n(out + r * D + l.sub * kSeg, l.nvalid, w);
    else
      store_bf16_seg<kSeg>(out + r * D + l.sub * kSeg, w);
  }
}

// ============================================================== host side
ChunkScales chunk_scales() {
  ChunkScales cs;
  for (int b = 0; b <= 8; ++b) cs.s[b] = (float)(1.0 / __builtin_sqrt((double)(1 << b)));
  return cs;
}
// lanes per row: next_pow2(ceil(D / 16))
int row_lanes(int D) { return next_pow2((D + kSeg - 1) / kSeg); }

// Blocks per workgroup: enough for one pass of whole tokens; kstats also caps a job
// at ~16 workgroups, which keeps the global atomics per channel few.
int rows_per_pass(const Geo& g) { return (kRWG / row_lanes(g.D) / g.H) * g.H; }
void set_rows_bpw(Geo* g, int32_t max_blocks, bool stats) {
  const int rpb = g->S * g->H, rp = rows_per_pass(*g);
  g->bpw = rpb >= rp ? 1 : (rp + rpb - 1) / rpb;
  if (stats) g->bpw = max(g->bpw, (max_blocks + 15) / 16);
}

// The SM variants (D % 16 != 0) are separate instantiations, so the others keep their code.
template <int LPR>
void launch_stats(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, hipStream_t st) {
  const size_t lds = (size_t)2 * g.H * g.D * sizeof(uint32_t);
  if (g.D % kSeg)
    hipLaunchKernelGGL((rows_stats_kernel<LPR, true>), grid, dim3(kRWG), lds, st, g, chunk_scales(), jobs);
  else
    hipLaunchKernelGGL((rows_stats_kernel<LPR, false>), grid, dim3(kRWG), lds, st, g, chunk_scales(), jobs);
}
template <int LPR, int BITS>
void launch_encode(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  if (g.D % kSeg)
    hipLaunchKernelGGL((rows_encode_kernel<LPR, BITS, true>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
  else
    hipLaunchKernelGGL((rows_encode_kernel<LPR, BITS, false>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
}
template <int LPR, int BITS>
void launch_decode(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  if (g.D % kSeg)
    hipLaunchKernelGGL((rows_decode_kernel<LPR, BITS, true>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
  else
    hipLaunchKernelGGL((rows_decode_kernel<LPR, BITS, false>), grid, dim3(kRWG), 0, st, g, chunk_scales(), jobs, err);
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
  switch (row_lanes(g.D)) {
    case 1: ByBits<F, 1>::run(g.bits, g, grid, jobs, err, st); break;
    case 2: ByBits<F, 2>::run(g.bits, g, grid, jobs, err, st); break;
    case 4: ByBits<F, 4>::run(g.bits, g, grid, jobs, err, st); break;
    case 8: ByBits<F, 8>::run(g.bits, g, grid, jobs, err, st); break;
    default: ByBits<F, 16>::run(g.bits, g, grid, jobs, err, st); break;
  }
}

template <int LPR>
void launch_hadamard(dim3 gr, dim3 bl, hipStream_t st, const uint16_t* i16, uint16_t* o16, int64_t rows, int H, int D,
                     const uint32_t* signs, int inverse, const ChunkScales& cs) {
  if (D % kSeg)
    hipLaunchKernelGGL((rows_hadamard_kernel<LPR, true>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs);
  else
    hipLaunchKernelGGL((rows_hadamard_kernel<LPR, false>), gr, bl, 0, st, i16, o16, rows, H, D, signs, inverse, cs);
}

}  // namespace

int rows_hadamard(const void* in, void* out, int64_t rows, int32_t H, int32_t D, const uint32_t* signs,
                  int32_t inverse, hipStream_t st) {
  const int lpr = row_lanes(D);
  const int64_t grid = (rows + kRWG / lpr - 1) / (kRWG / lpr);
  if (grid > 0x7fffffffLL) return KVMI_EINVAL;
  const uint16_t* i16 = static_cast<const uint16_t*>(in);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  const dim3 gr((unsigned)grid), bl(kRWG);
  const ChunkScales cs = chunk_scales();
  switch (lpr) {
    case 1: launch_hadamard<1>(gr, bl, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 2: launch_hadamard<2>(gr, bl, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 4: launch_hadamard<4>(gr, bl, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    case 8: launch_hadamard<8>(gr, bl, st, i16, o16, rows, H, D, signs, inverse, cs); break;
    default: launch_hadamard<16>(gr, bl, st, i16, o16, rows, H, D, signs, inverse, cs); break;
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

int rows_kstats(const Geo& g0, const kvmi_layer_job* jobs, int32_t num_jobs, int32_t max_blocks, int32_t*,
                hipStream_t st) {
  Geo g = g0;
  set_rows_bpw(&g, max_blocks, true);
  const dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  if (part_axis(g.flags, 0) == kAxToken && part_axis(g.flags, 1) == kAxToken) return KVMI_OK;  // nothing to reduce
  switch (row_lanes(g.D)) {
    case 1: launch_stats<1>(g, grid, jobs, st); break;
    case 2: launch_stats<2>(g, grid, jobs, st); break;
    case 4: launch_stats<4>(g, grid, jobs, st); break;
    case 8: launch_stats<8>(g, grid, jobs, st); break;
    default: launch_stats<16>(g, grid, jobs, st); break;
  }
  if (hipGetLastError() != hipSuccess) return KVMI_ELAUNCH;
  hipLaunchKernelGGL(rows_finalize_kernel, dim3((unsigned)num_jobs), dim3(kRWG), 0, st, g, jobs);
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
