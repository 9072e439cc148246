// Fused paged compress / decompress kernels for gfx950, register FWHT, one quad of
// lanes per row (D in {64, 128}, H dividing 128, H <= 16; other geometries run the
// generic row kernels of kvmi_rows.hip, the transform profile mostly the MFMA kernels).
//
// Work unit: a workgroup of 512 threads (8 wave64s) owns a run of paged blocks of
// one (request, layer) job.  The run's rows (one row = one token x one KV head =
// D contiguous bf16) are processed 128 at a time; row r of a pass is held by the
// quad of lanes 4r..4r+3, lane q of the quad owning elements [q*D/4, (q+1)*D/4).
// Rows of a pass are contiguous in the pool (a block is [S, H, D] row-major), so
// every wave reads 16 consecutive rows.  Because 128 % H == 0, a lane always sees
// the same KV head, which keeps sign bits and per-channel K statistics in place.
//
// Compress is three launches:
//   kstats: gather + transform of K, per-channel running min/max per lane,
//           workgroup reduction through LDS atomics, device reduction through
//           global atomics;
//   kstats finalize: one workgroup per job turns the keys into the job's K
//           metadata and re-initialises them (a launch of its own, so no
//           device-wide fence is needed between the workgroups of the first);
//   encode: gather + transform of K and V, K quantized with the per-channel
//           metadata, V with per-(token, group) statistics reduced through LDS;
//           symbols bitpacked straight into the chunk stream.
// Decompress is one launch: header check, unpack, dequantize, inverse transform,
// sign and scatter into the pool.
#include "kvmi_common.hpp"

static_assert(sizeof(kvmi_layer_job) == 104, "kvmi_layer_job layout is part of the ABI");
static_assert(sizeof(kvmi_geometry) == 32, "kvmi_geometry layout is part of the ABI");

namespace kvmi {
namespace {

constexpr int kWG = 512;
constexpr int kRows = kWG / 4;  // rows per pass

// Sign bits of lane q's E elements for head h.
template <int D>
__device__ __forceinline__ uint32_t lane_signs(const uint32_t* signs, int h, int q) {
  constexpr int E = D / 4;
  const uint32_t* sg = signs + h * (D / 32);
  if constexpr (E == 32) {
    return gld(sg + q);
  } else {  // E == 16
    return (gld(sg + (q >> 1)) >> ((q & 1) * 16)) & 0xffffu;
  }
}

// Load one row segment, apply signs + FWHT + scale (unless NO_TRANSFORM) and return
// the fp32 values.  ROUND: round the result to bf16 values.
template <int D, bool ROUND>
__device__ __forceinline__ void load_transform(const uint16_t* __restrict__ src, uint32_t sb, bool transform,
                                               float scale, int q, float (&y)[D / 4]) {
  constexpr int E = D / 4;
  uint32_t w[E / 2];
  load_bf16_seg<E>(src, w);
  if (transform) {
    apply_sign_bf16<E>(w, sb);
    unpack_bf16<E>(w, y);
    fwht_row<E>(y, q);
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = ROUND ? round_bf16(y[i] * scale) : y[i] * scale;
  } else {
    unpack_bf16<E>(w, y);
  }
}

// ============================================================== K statistics
template <int D>
__global__ __launch_bounds__(kWG) void kstats_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                     int32_t* __restrict__ err) {
  constexpr int E = D / 4;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) return;
  const int H = g.H, S = g.S, HD = H * D;
  const int blk0 = blockIdx.x * g.bpw;
  const int blk1 = min(B, blk0 + g.bpw);
  const int64_t rows = (int64_t)(blk1 - blk0) * S * H;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3;
  const int h = Q % H;
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? lane_signs<D>(job.signs, h, q) : 0u;

  __shared__ uint32_t lkey[2 * kMaxQuadHD];
  for (int i = tid; i < HD; i += kWG) {
    lkey[i] = 0xffffffffu;
    lkey[HD + i] = 0u;
  }

  float mn[E], mx[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    mn[i] = __builtin_inff();
    mx[i] = -__builtin_inff();
  }
  const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool);
  for (int64_t r0 = 0; r0 < rows; r0 += kRows) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + Q, S, H);
    if (rp.active) {
      float y[E];
      load_transform<D, false>(pool + rp.pool_row * D + q * E, sb, transform, g.scale, q, y);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        mn[i] = fminf(mn[i], y[i]);
        mx[i] = fmaxf(mx[i], y[i]);
      }
    }
  }
  __syncthreads();
  // channel c = seg * E + k (seg = h * 4 + q) sits at seg * E + (k + seg) % E, so that
  // the lanes of one atomic instruction (same k, different segments) use different banks
  if (Q < (int)((rows < kRows) ? rows : kRows)) {
    const int seg = h * 4 + q;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int slot = seg * E + ((i + seg) & (E - 1));
      atomicMin(&lkey[slot], f2key(mn[i]));
      atomicMax(&lkey[HD + slot], f2key(mx[i]));
    }
  }
  __syncthreads();
  for (int i = tid; i < HD; i += kWG) {
    const int seg = i / E, slot = seg * E + ((i + seg) & (E - 1));
    atomicMin(&job.kstats[i], lkey[slot]);
    atomicMax(&job.kstats[HD + i], lkey[HD + slot]);
  }
}

// Pass 1b: per job, turn the accumulated keys into kmeta (bf16 min and scale of
// every K channel, by output position) and re-initialise the keys.  A kernel of its
// own: the launch boundary makes every workgroup's atomics of pass 1a visible, with
// no device-wide fence inside the accumulating kernels.
__global__ __launch_bounds__(kWG) void kstats_finalize_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs) {
  const kvmi_layer_job job = jobs[blockIdx.x];
  if (job.num_blocks <= 0) return;  // nothing accumulated: kmeta is left as it is
  const int H = g.H, D = g.D, HD = H * D;
  __shared__ int pos[kMaxHeads];
  __shared__ uint8_t lev[kMaxHeads];
  if (threadIdx.x < (unsigned)H) {
    const int k = threadIdx.x;
    pos[gld(job.profile + k)] = k;  // order[k] = source head at output position k
    lev[k] = gld(job.profile + H + k);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kWG) {
    const int hs = i / D, e = i % D, j = pos[hs];
    const float kmn = round_bf16(key2f(gld(job.kstats + i)));
    const float kmx = round_bf16(key2f(gld(job.kstats + HD + i)));
    const float sc = quant_scale(kmn, kmx, lev[j]);
    gst(job.kmeta + j * D + e, (uint16_t)f32_to_bf16_bits(kmn));
    gst(job.kmeta + HD + j * D + e, (uint16_t)f32_to_bf16_bits(sc));
    gst(job.kstats + i, 0xffffffffu);
    gst(job.kstats + HD + i, 0u);
  }
}

// ============================================================== encode
template <int D, int BITS>
__global__ __launch_bounds__(kWG) void encode_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                     int32_t* __restrict__ err) {
  constexpr int E = D / 4;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) {
    // a job without blocks still heads its chunk (the stream of N = 0 symbols)
    if (nwg == 0 && blockIdx.x == 0 && threadIdx.x == 0 && job.write_header && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
    return;
  }
  const int H = g.H, S = g.S, HD = H * D, G = g.G;
  const int blk0 = blockIdx.x * g.bpw;
  const int blk1 = min(B, blk0 + g.bpw);
  const int64_t rows = (int64_t)(blk1 - blk0) * S * H;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3;
  const int h = Q % H;
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? lane_signs<D>(job.signs, h, q) : 0u;
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);

  __shared__ float2 kq[kMaxQuadHD];     // (min, 1/scale) by source head and channel
  __shared__ int posk[kMaxQuadH], posv[kMaxQuadH];
  __shared__ float2 rowmm[kRows];   // V row (min, max)
  __shared__ float2 tokq[kRows];    // V (min, 1/scale) by (token of pass, group)
  __shared__ int ngv;

  if (tid < H) {
    for (int k = 0; k < H; ++k) {
      if (pk.order[k] == tid) posk[tid] = k;
      if (pv.order[k] == tid) posv[tid] = k;
    }
  }
  if (tid == 0) {
    int m = 0;
    for (int k = 0; k < H; ++k) m = max(m, (int)pv.group[k]);
    ngv = m + 1;
    if (job.write_header && blockIdx.x == 0 && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
  }
  __syncthreads();
  for (int i = tid; i < HD; i += kWG) {
    const int hs = i / D, e = i % D, j = posk[hs];
    const float m = bf16_to_f32(gld(job.kmeta + j * D + e));
    const float sc = bf16_to_f32(gld(job.kmeta + HD + j * D + e));
    kq[i] = make_float2(m, 1.0f / sc);
  }
  __syncthreads();

  const int jk = posk[h], jv = posv[h];
  const float lk = (float)pk.levels[jk];
  const float lvv = (float)pv.levels[jv];
  const int gv = pv.group[jv];
  const int ngroups = ngv;
  const int tpp = kRows / H;  // tokens per pass
  const uint16_t* poolK = reinterpret_cast<const uint16_t*>(job.pool);
  const uint16_t* poolV = poolK + job.pool_part_stride;
  const int64_t ntok = (int64_t)B * S;
  uint32_t over = 0;

  for (int64_t r0 = 0; r0 < rows; r0 += kRows) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + Q, S, H);
    // ---------------- K: per-channel statistics from the kstats pass
    if (rp.active) {
      float y[E];
      load_transform<D, true>(poolK + rp.pool_row * D + q * E, sb, transform, g.scale, q, y);
      uint32_t s[E];
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float2 c = kq[h * D + q * E + i];
        s[i] = (uint32_t)quant_value(y[i], c.x, c.y, lk);
        over |= s[i];
      }
      Packed<E, BITS> pkd;
      pack_syms<E, BITS>(s, pkd);
      store_packed<E, BITS>(seg_addr<BITS>(job, g, 0, jk, rp.tok, q * (D / 4)), pkd);
    }
    // ---------------- V: per-token statistics over the heads of a group
    float y[E];
    if (rp.active) {
      load_transform<D, true>(poolV + rp.pool_row * D + q * E, sb, transform, g.scale, q, y);
      float lmn = y[0], lmx = y[0];
#pragma unroll
      for (int i = 1; i < E; ++i) {
        lmn = fminf(lmn, y[i]);
        lmx = fmaxf(lmx, y[i]);
      }
      lmn = quad_min(lmn);
      lmx = quad_max(lmx);
      if (q == 0) rowmm[Q] = make_float2(lmn, lmx);
    }
    __syncthreads();
    if (tid < tpp * G) {
      const int tp = tid / G, gg = tid % G;
      const int64_t rr = r0 + (int64_t)tp * H;
      if (gg < ngroups && rr < rows) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
        int lv = 2;
        for (int k = 0; k < H; ++k) {
          if (pv.group[k] == gg) {
            const float2 m = rowmm[tp * H + pv.order[k]];
            mn = fminf(mn, m.x);
            mx = fmaxf(mx, m.y);
            lv = pv.levels[k];
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
    if (rp.active) {
      const float2 c = tokq[(Q / H) * G + gv];
      uint32_t s[E];
#pragma unroll
      for (int i = 0; i < E; ++i) {
        s[i] = (uint32_t)quant_value(y[i], c.x, c.y, lvv);
        over |= s[i];
      }
      Packed<E, BITS> pkd;
      pack_syms<E, BITS>(s, pkd);
      store_packed<E, BITS>(seg_addr<BITS>(job, g, 1, jv, rp.tok, q * (D / 4)), pkd);
    }
    __syncthreads();
  }
  if (over >> BITS) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
}

// ============================================================== decode
template <int D, int BITS>
__global__ __launch_bounds__(kWG) void decode_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                     int32_t* __restrict__ err) {
  constexpr int E = D / 4;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int B = job.num_blocks;
  const int nwg = (B + g.bpw - 1) / g.bpw;
  if ((int)blockIdx.x >= nwg) return;
  const int H = g.H, S = g.S, HD = H * D, G = g.G;
  const int tid = threadIdx.x, Q = tid >> 2, q = tid & 3;

  __shared__ float2 kd[kMaxQuadHD];  // (min, scale) by source head and channel
  __shared__ int posk[kMaxQuadH], posv[kMaxQuadH];
  __shared__ int ok;
  const Profile pk = part_profile(job.profile, 0, H);
  const Profile pv = part_profile(job.profile, 1, H);
  if (tid == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  if (tid < H) {
    for (int k = 0; k < H; ++k) {
      if (pk.order[k] == tid) posk[tid] = k;
      if (pv.order[k] == tid) posv[tid] = k;
    }
  }
  __syncthreads();
  if (!ok) return;
  for (int i = tid; i < HD; i += kWG) {
    const int hs = i / D, e = i % D, j = posk[hs];
    kd[i] = make_float2(bf16_to_f32(gld(job.kmeta + j * D + e)), bf16_to_f32(gld(job.kmeta + HD + j * D + e)));
  }
  __syncthreads();

  const int blk0 = blockIdx.x * g.bpw;
  const int blk1 = min(B, blk0 + g.bpw);
  const int64_t rows = (int64_t)(blk1 - blk0) * S * H;
  const int h = Q % H;
  const bool transform = !(g.flags & KVMI_F_NO_TRANSFORM);
  const uint32_t sb = transform ? lane_signs<D>(job.signs, h, q) : 0u;
  const int jk = posk[h], jv = posv[h];
  const int gv = pv.group[jv];
  uint16_t* poolK = reinterpret_cast<uint16_t*>(job.pool);
  uint16_t* poolV = poolK + job.pool_part_stride;
  const int64_t ntok = (int64_t)B * S;

  for (int64_t r0 = 0; r0 < rows; r0 += kRows) {
    const RowPos rp = row_pos(job, blk0, rows, r0 + Q, S, H);
    if (!rp.active) continue;  // quads are whole: DPP partners share activity
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const int j = part ? jv : jk;
      Packed<E, BITS> pkd;
      load_packed<E, BITS>(seg_addr<BITS>(job, g, part, j, rp.tok, q * (D / 4)), pkd);
      uint32_t s[E];
      unpack_syms<E, BITS>(pkd, s);
      float x[E];
      if (part == 0) {
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const float2 c = kd[h * D + q * E + i];
          x[i] = dequant_value((float)s[i], c.x, c.y);
        }
      } else {
        const float mn = bf16_to_f32(gld(job.vmeta + (int64_t)gv * ntok + rp.tok));
        const float sc = bf16_to_f32(gld(job.vmeta + (int64_t)(G + gv) * ntok + rp.tok));
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = dequant_value((float)s[i], mn, sc);
      }
      uint32_t w[E / 2];
      if (transform) {
        fwht_row<E>(x, q);
#pragma unroll
        for (int i = 0; i < E / 2; ++i) w[i] = pack_bf16x2(x[2 * i] * g.scale, x[2 * i + 1] * g.scale);
        apply_sign_bf16<E>(w, sb);
      } else {
#pragma unroll
        for (int i = 0; i < E / 2; ++i) w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
      }
      store_bf16_seg<E>((part ? poolV : poolK) + rp.pool_row * D + q * E, w);
    }
  }
}

// ============================================================== host side
template <int D, int BITS>
void launch_encode_db(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  hipLaunchKernelGGL((encode_kernel<D, BITS>), grid, dim3(kWG), 0, st, g, jobs, err);
}
template <int D, int BITS>
void launch_decode_db(const Geo& g, dim3 grid, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  hipLaunchKernelGGL((decode_kernel<D, BITS>), grid, dim3(kWG), 0, st, g, jobs, err);
}

#define KVMI_DISPATCH_BITS(FN, D, g, grid, jobs, err, st) \
  switch ((g).bits) {                                     \
    case 1: FN<D, 1>(g, grid, jobs, err, st); break;      \
    case 2: FN<D, 2>(g, grid, jobs, err, st); break;      \
    case 3: FN<D, 3>(g, grid, jobs, err, st); break;      \
    case 4: FN<D, 4>(g, grid, jobs, err, st); break;      \
    case 5: FN<D, 5>(g, grid, jobs, err, st); break;      \
    case 6: FN<D, 6>(g, grid, jobs, err, st); break;      \
    case 7: FN<D, 7>(g, grid, jobs, err, st); break;      \
    default: FN<D, 8>(g, grid, jobs, err, st); break;     \
  }

// Register-FWHT kernels work on 128-row passes: enough blocks per workgroup to fill one.
void set_valu_bpw(Geo* g) {
  const int rpb = g->S * g->H;
  g->bpw = rpb >= kRows ? 1 : (kRows + rpb - 1) / rpb;
}

}  // namespace
}  // namespace kvmi

extern "C" int kvmi_kstats_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream) {
  using namespace kvmi;
  Geo g;
  int rc = check_geo(geom, num_jobs, max_blocks, &g);
  if (rc) return rc;
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Geo v;
  if (paired_view(g, &v)) {  // the keys have the same layout in both views: finalize with g
    rc = mfma_kstats(v, jobs, num_jobs, max_blocks, err, st);
    if (rc) return rc;
  } else if (mfma_eligible(g)) {
    rc = mfma_kstats(g, jobs, num_jobs, max_blocks, err, st);
    if (rc) return rc;
  } else if (!quad_eligible(g)) {
    return rows_kstats(g, jobs, num_jobs, max_blocks, err, st);  // statistics of both parts + their finalize
  } else {
    // Statistics need only K: give each workgroup enough blocks that a job has at
    // most ~16 workgroups, which keeps the global atomics per channel small.
    set_valu_bpw(&g);
    const int bpw = (max_blocks + 15) / 16;
    if (bpw > g.bpw) g.bpw = bpw;
    dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
    if (g.D == 64)
      hipLaunchKernelGGL((kstats_kernel<64>), grid, dim3(kWG), 0, st, g, jobs, err);
    else
      hipLaunchKernelGGL((kstats_kernel<128>), grid, dim3(kWG), 0, st, g, jobs, err);
    if (hipGetLastError() != hipSuccess) return KVMI_ELAUNCH;
  }
  hipLaunchKernelGGL(kstats_finalize_kernel, dim3((unsigned)num_jobs), dim3(kWG), 0, st, g, jobs);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_encode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream) {
  using namespace kvmi;
  Geo g;
  int rc = check_geo(geom, num_jobs, max_blocks, &g);
  if (rc) return rc;
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Geo v;
  if (paired_view(g, &v)) return mfma_encode(v, jobs, num_jobs, max_blocks, err, st);
  if (mfma_eligible(g)) return mfma_encode(g, jobs, num_jobs, max_blocks, err, st);
  if (!quad_eligible(g)) return rows_encode(g, jobs, num_jobs, max_blocks, err, st);
  set_valu_bpw(&g);
  dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  if (g.D == 64) {
    KVMI_DISPATCH_BITS(launch_encode_db, 64, g, grid, jobs, err, st)
  } else {
    KVMI_DISPATCH_BITS(launch_encode_db, 128, g, grid, jobs, err, st)
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_decode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream) {
  using namespace kvmi;
  Geo g;
  int rc = check_geo(geom, num_jobs, max_blocks, &g);
  if (rc) return rc;
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Geo v;
  if (paired_view(g, &v)) return mfma_decode(v, jobs, num_jobs, max_blocks, err, st);
  if (mfma_eligible(g)) return mfma_decode(g, jobs, num_jobs, max_blocks, err, st);
  if (!quad_eligible(g)) return rows_decode(g, jobs, num_jobs, max_blocks, err, st);
  set_valu_bpw(&g);
  dim3 grid((unsigned)((max_blocks + g.bpw - 1) / g.bpw), (unsigned)num_jobs);
  if (g.D == 64) {
    KVMI_DISPATCH_BITS(launch_decode_db, 64, g, grid, jobs, err, st)
  } else {
    KVMI_DISPATCH_BITS(launch_decode_db, 128, g, grid, jobs, err, st)
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}
