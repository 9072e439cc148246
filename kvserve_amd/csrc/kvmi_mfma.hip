// Two-pass paged compress (K statistics, then encode) and the paged decompress
// with the Hadamard transform on MFMA (gfx950); the tile layout and the shared
// device helpers are described in kvmi_mfma_tiles.hpp.
#include <mutex>
#include <unordered_map>

#include "kvmi_mfma_tiles.hpp"


namespace kvmi {
namespace {

// ============================================================== K statistics (orientation N)
template <int NC, bool PAIRED>
__device__ __forceinline__ void kstats_body(const Geo& g, const kvmi_layer_job* __restrict__ jobs) {
  constexpr int D = 32 * NC;
  // jobs in reverse order: the statistics pass starts on the layers the previous kernel
  // (a decode, or the attention that wrote the cache) touched last, whose lines the
  // memory-side cache still holds, and ends on the first layers, where encode begins
  const kvmi_layer_job job = jobs[gridDim.y - 1 - blockIdx.y];
  const int S = g.S, H = g.H;
  const Run run = wg_run(job, g);
  if ((int)blockIdx.x >= run.nwg) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
  const int hme = r % H;

  __shared__ Tables T;
  __shared__ uint32_t lkey[2 * kMH * 128];
  // per-wave buffer that turns a coalesced tile into the lanes' half-rows
  __shared__ uint4 tbuf[kWaves * tile_buf_q<NC>()];
  fill_signs(T, job.signs, H, D);
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
  // running min / max per (output register % 4, chunk): see kstats_tile
  float mn[4][NC], mx[4][NC];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      mn[a][c] = __builtin_inff();
      mx[a][c] = -__builtin_inff();
    }
  const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool);
  uint4* wbuf = tbuf + wave * tile_buf_q<NC>();
  constexpr bool paired = PAIRED;
  auto accumulate = [&](uint4 (&x)[2 * NC]) {
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) pin(x[u]);
    tile_to_half_rows<NC>(wbuf, x);
    sign_half_row<NC>(T, hme, hl, x);
    kstats_tile<NC>(x, hp, hn, mn, mx, paired);
  };
  auto fetch = [&](int t, uint4 (&x)[2 * NC]) {
    load_tile<NC>(pool, tile_row0(job, S, H, tile_tok(run.tok0, H, t)), x);
  };
  // Two buffers: the loads of tile t + 4 are in flight while tile t is reduced.  The
  // prefetch is unconditional (past the end it re-reads the current tile, a cache
  // hit): loads issued on one path only make the compiler's wait counts conservative.
  const int last_tile = run.tiles - 1;
  uint4 xa[2 * NC], xb[2 * NC];
  if (wave < run.tiles) fetch(wave, xa);
  for (int t = wave; t < run.tiles; t += 2 * kWaves) {
    fetch(min(t + kWaves, last_tile), xb);
    accumulate(xa);
    if (t + kWaves >= run.tiles) break;
    fetch(min(t + 2 * kWaves, last_tile), xa);
    accumulate(xb);
  }
  const int HD = H * D;
  if (wave < run.tiles) push_lkeys<NC>(lkey, mn, mx, H, g.scale);
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kMW) {
    if (lkey[i] != 0xffffffffu) atomicMin(&job.kstats[i], lkey[i]);
    if (lkey[HD + i] != 0u) atomicMax(&job.kstats[HD + i], lkey[HD + i]);
  }
}

template <int NC>
__global__ __launch_bounds__(kMW) void kstats_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                          int32_t* __restrict__ err) {
  kstats_body<NC, false>(g, jobs);
}
// head_dim 256 as paired virtual heads of 128 (kPairedHeads), up to 4 real heads
__global__ __launch_bounds__(kMW) void kstats_mfma_pair_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                               int32_t* __restrict__ err) {
  kstats_body<4, true>(g, jobs);
}

// ============================================================== K statistics, 16 or 32 heads
// With 16 or 32 heads a token-major tile holds 16 heads per lane's registers in
// orientation N, too many running min / max to keep.  Here a tile is 32 consecutive
// tokens of ONE head instead (rows 2*H*D bytes apart in the pool, each row read by
// PR = 4NC lanes in 16-byte pieces; a run's last tile repeats its last token, which
// min / max ignore), so every output register of a lane is the same (head, channel):
// one running pair per chunk.  Wave w owns heads w, w + 4, ... of the workgroup's run
// and writes their keys into the workgroup's LDS keys without atomics.
struct SignTable {
  uint32_t smask[kWideH][64 + 4];
};
template <int NC, bool PAIRED>
__device__ __forceinline__ void kstats_wide_body(const Geo& g, const kvmi_layer_job* __restrict__ jobs) {
  constexpr int D = 32 * NC, HALF = 16 * NC, PR = 4 * NC;
  // jobs in reverse order: the statistics pass starts on the layers the previous kernel
  // (a decode, or the attention that wrote the cache) touched last, whose lines the
  // memory-side cache still holds, and ends on the first layers, where encode begins
  const kvmi_layer_job job = jobs[gridDim.y - 1 - blockIdx.y];
  const int S = g.S, H = g.H, HD = H * D;
  const Run run = wg_run(job, g);
  if ((int)blockIdx.x >= run.nwg) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;

  __shared__ SignTable T;
  __shared__ uint32_t lkey[2 * kWideH * 128];
  __shared__ uint4 tbuf[kWaves * tile_buf_q<NC>()];
  fill_signs(T, job.signs, H, D);
  for (int i = threadIdx.x; i < HD; i += kMW) {
    lkey[i] = 0xffffffffu;
    lkey[HD + i] = 0u;
  }
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, true, false);
  hp[1] = hadamard_tile(1, true, false);
  hn[0] = hadamard_tile(0, true, true);
  hn[1] = hadamard_tile(1, true, true);
  const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool);
  const int sh = __builtin_ctz((unsigned)S);  // S is a power of two (mfma_eligible)
  const int last_tok = run.tok_end - 1;
  // Paired virtual heads (head_dim 256): a tile is 16 tokens x both halves of one real
  // head (rows 2i, 2i + 1 = the halves of token i), so the butterfly stays in a lane.
  constexpr bool paired = PAIRED;
  const int HU = paired ? H / 2 : H;                   // heads a wave walks
  const int TPT = paired ? kTok / 2 : kTok;            // tokens per tile
  const int nk = (run.tok_end - run.tok0 + TPT - 1) / TPT;  // tiles per head
  const int nhw = (HU - wave + kWaves - 1) / kWaves;   // heads of this wave
  const int ntw = nhw * nk;
  uint4* wbuf = tbuf + wave * tile_buf_q<NC>();
  // tile n of this wave: head wave + 4 (n / nk), tokens tok0 + TPT (n % nk) + ...;
  // instruction v of a lane reads piece l % PR of row (64 / PR) v + l / PR
  auto fetch = [&](int n, uint4 (&x)[2 * NC]) {
    const int hu = wave + kWaves * (n / nk), t0 = run.tok0 + TPT * (n % nk);
#pragma unroll
    for (int v = 0; v < 2 * NC; ++v) {
      const int rho = (64 / PR) * v + l / PR;
      const int t = min(t0 + (paired ? rho >> 1 : rho), last_tok);
      const int vh = paired ? 2 * hu + (rho & 1) : hu;
      const int64_t row = ((int64_t)gld(job.block_ids + (t >> sh)) * S + (t & (S - 1))) * H + vh;
      x[v] = gld(reinterpret_cast<const uint4*>(pool + row * D) + l % PR);
    }
  };
  float mn[4][NC], mx[4][NC];
  auto reset = [&]() {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        mn[a][c] = __builtin_inff();
        mx[a][c] = -__builtin_inff();
      }
  };
  auto accumulate = [&](int n, uint4 (&x)[2 * NC]) {
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) pin(x[u]);
    const int hu = wave + kWaves * (n / nk);
    tile_to_half_rows<NC>(wbuf, x);
    // the lane's row r is half r & 1 of a token when paired: that virtual head's signs
    sign_half_row<NC>(T, paired ? 2 * hu + (r & 1) : hu, hl, x);
    kstats_tile<NC>(x, hp, hn, mn, mx, paired);
    if (n % nk == nk - 1) {
      // the head's last tile: its keys (channel HALF (r >> 4) + 16 c + (r & 15) of
      // chunk c; lanes r and r + 32 hold other rows of the same channel).  Register
      // i % 4 = a holds rows with m & 1 = a & 1: the half of a paired head.
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          if (!paired && half) break;
          float a = paired ? fminf(mn[half][c], mn[half + 2][c])
                           : fminf(fminf(mn[0][c], mn[1][c]), fminf(mn[2][c], mn[3][c]));
          float b = paired ? fmaxf(mx[half][c], mx[half + 2][c])
                           : fmaxf(fmaxf(mx[0][c], mx[1][c]), fmaxf(mx[2][c], mx[3][c]));
          a = halves_min(a);
          b = halves_max(b);
          if (hl == 0) {
            const int vh = paired ? 2 * hu + half : hu;
            const int f = HALF * (r >> 4) + 16 * c + (r & 15);
            lkey[vh * D + f] = f2key(a * g.scale);
            lkey[HD + vh * D + f] = f2key(b * g.scale);
          }
        }
      }
      reset();
    }
  };
  reset();
  uint4 xa[2 * NC], xb[2 * NC];
  if (ntw > 0) fetch(0, xa);
  for (int n = 0; n < ntw; n += 2) {
    fetch(min(n + 1, ntw - 1), xb);
    accumulate(n, xa);
    if (n + 1 >= ntw) break;
    fetch(min(n + 2, ntw - 1), xa);
    accumulate(n + 1, xb);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HD; i += kMW) {
    if (lkey[i] != 0xffffffffu) atomicMin(&job.kstats[i], lkey[i]);
    if (lkey[HD + i] != 0u) atomicMax(&job.kstats[HD + i], lkey[HD + i]);
  }
}

template <int NC>
__global__ __launch_bounds__(kMW) void kstats_wide_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                          int32_t* __restrict__ err) {
  kstats_wide_body<NC, false>(g, jobs);
}
// head_dim 256 as 16 or 32 paired virtual heads (8 or 16 real heads)
__global__ __launch_bounds__(kMW) void kstats_wide_pair_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                               int32_t* __restrict__ err) {
  kstats_wide_body<4, true>(g, jobs);
}

// ============================================================== encode (orientation T)
// HM: head capacity of the tables (kMH, or kWideH for 16 and 32 heads).
// PAIRED: head_dim 256 as paired virtual heads of 128 (kPairedHeads).
template <int NC, int BITS, bool CLAMP, int HM, bool PAIRED, int W = kWaves>
__device__ __forceinline__ void encode_body(const Geo& g, const kvmi_layer_job* __restrict__ jobs,
                                            int32_t* __restrict__ err) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int ntok = job.num_blocks * S;
  const Run run = wg_run(job, g);
  if ((int)blockIdx.x >= run.nwg) {
    // a job without blocks still heads its chunk (the stream of N = 0 symbols)
    if (run.nwg == 0 && blockIdx.x == 0 && threadIdx.x == 0 && job.write_header && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
    return;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;

  __shared__ TablesT<HM> T;
  // Per-wave LDS buffer with three uses in turn: it rearranges each loaded tile into the
  // lanes' half-rows, parks a V tile's rounded outputs between its statistics and its
  // quantization (2*NC uint4 per lane), and stages a section's packed symbols as the
  // byte image of the stream runs the tile covers -- H runs of 32/H tokens (permuted
  // order) or one run of 32 rows (native order) -- which are then written lane-linear,
  // 16 bytes a lane.  A wave's LDS operations execute in order, so the uses follow one
  // another without waits.
  constexpr int RB = D * BITS / 8;            // bytes of one packed row
  constexpr int TQ = kTok * RB / 16;          // uint4 per tile
  static_assert(tile_buf_q<NC>() >= 2 * NC * 64 && tile_buf_q<NC>() >= TQ, "a wave buffer holds each use");
  __shared__ uint4 ypark[W * tile_buf_q<NC>()];
  const bool native = g.flags & KVMI_F_NATIVE_LAYOUT;
  constexpr bool paired = PAIRED;
  stage_profile(T, job.profile, H, paired);
  fill_signs(T, job.signs, H, D);
  if (threadIdx.x == 0 && job.write_header && blockIdx.x == 0 && !(g.flags & KVMI_F_NO_HEADER))
    write_stream_header(job.stream, BITS, job.chunk_symbols);
  __syncthreads();
  fill_positions(T, H);
  fill_kconst<true>(T, job.kmeta, H, D);
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, false, false);
  hp[1] = hadamard_tile(1, false, false);
  hn[0] = hadamard_tile(0, false, true);
  hn[1] = hadamard_tile(1, false, true);
  const uint16_t* poolK = reinterpret_cast<const uint16_t*>(job.pool);
  const uint16_t* poolV = poolK + job.pool_part_stride;
  uint32_t over = 0;

  // this lane's head, its output positions and V statistic group
  const int hme = r % H;
  const LaneProfile lp = lane_profile(T, hme, hl);
  const float s = g.scale;

  uint4* ostage = ypark + wave * tile_buf_q<NC>();
  uint8_t* ost = reinterpret_cast<uint8_t*>(ostage);
  const int tpt = kTok / H;  // tokens per tile
#ifndef KVMI_COOP_FLUSH
#define KVMI_COOP_FLUSH 1
#endif
  // In the permuted order, flushed by the whole workgroup, each head's run in the staged
  // image is followed by 16 bytes: the lanes of one LDS store pass (two tokens of every
  // head) then fall 4 banks apart per head, instead of all on the same 4 banks (a run is
  // a multiple of the 256-byte bank row at 8 heads): 8-way conflicts become 2-way.
  constexpr int kRunPad = KVMI_COOP_FLUSH ? 1 : 0;  // uint4 after each head's run
  static_assert(tile_buf_q<NC>() >= TQ + HM * kRunPad, "the padded image fits a wave buffer");
  // byte offset of this lane's half-row in the staged image, by output position; a
  // permuted run of paired virtual heads is a real head's tokens, both halves each
  auto stage_off = [&](int j) {
    if (native) return (r / H) * (H * RB) + j * RB + hl * (RB / 2);
    if (paired) return (j >> 1) * (2 * tpt * RB) + (r / H) * (2 * RB) + (j & 1) * RB + hl * (RB / 2);
    return j * (tpt * RB + 16 * kRunPad) + (r / H) * RB + hl * (RB / 2);
  };
  const int offk = stage_off(lp.jk), offv = stage_off(lp.jv);
  // write the staged image of (part, tile starting at token ta) to the stream
  auto flush = [&](int part, int ta) {
    const int rq = native ? TQ : (paired ? 2 : 1) * tpt * RB / 16;  // uint4 per run
#pragma unroll
    for (int u = 0; u < (TQ + 63) / 64; ++u) {
      const int q = 64 * u + l;
      if (TQ % 64 == 0 || q < TQ) {
        const int run_j = q / rq;
        const int j0 = native ? 0 : (paired ? 2 * run_j : run_j);
        uint8_t* dst = seg_addr<BITS, PAIRED>(job, g, part, j0, ta, 0) + 16 * (q - run_j * rq);
        gst(reinterpret_cast<uint4*>(dst), ostage[q]);
      }
    }
  };
  // The wave's parking buffer also turns each coalesced tile into the lanes' half-rows
  // (the V tile is rearranged before its rounded outputs are parked there).
  uint4* wbuf = ypark + wave * tile_buf_q<NC>();
  // Permuted order: the workgroup's W waves take consecutive tiles t0 .. t0 + W - 1, so
  // head j's runs of the W tiles are consecutive in the stream; after a barrier the
  // workgroup writes them as one run per head (W times longer runs than a wave's own
  // flush), each thread a fixed set of 16-byte pieces, with streaming stores (the packed
  // stream is not read again by this pass).  Entry e of a thread: piece q = tid + 64 W e
  // of the W tiles' image, from wave w's buffer, to byte `dst` of head j's run.
  const bool coop = KVMI_COOP_FLUSH && !native && !paired;
  constexpr int QE = (W * TQ + 64 * W - 1) / (64 * W);  // pieces per thread
  int qsrc[QE], qw[QE];
  int64_t qdst[QE];
  {
    const int rq = tpt * RB / 16;  // uint4 per tile run
    const int64_t hs_bytes = (int64_t)ntok * RB;
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      const int q = (int)threadIdx.x + 64 * W * e;
      const int j = q / (W * rq), rem = q - j * (W * rq), w = rem / rq;
      qw[e] = q < W * TQ ? w : W;  // W: no piece
      qsrc[e] = w * tile_buf_q<NC>() + j * (rq + kRunPad) + (rem - w * rq);
      qdst[e] = j * hs_bytes + 16 * rem;
    }
  }
  auto flush_wg = [&](int part, int t0) {
    const int na = min(W, run.tiles - t0);
    uint8_t* base = seg_addr<BITS, PAIRED>(job, g, part, 0, tile_tok(run.tok0, H, t0), 0);
#pragma unroll
    for (int e = 0; e < QE; ++e)
      if (qw[e] < na) gst_stream(reinterpret_cast<uint4*>(base + qdst[e]), ypark[qsrc[e]]);
  };

  uint4 xk[2 * NC], xv[2 * NC];
  const int last_tile = run.tiles - 1;
  load_tile<NC>(poolK, tile_row0(job, S, H, tile_tok(run.tok0, H, min(wave, last_tile))), xk);
  const int niter = (run.tiles + W - 1) / W;  // the same for every wave (barriers)
  for (int it = 0; it < niter; ++it) {
    const int t = it * W + wave;
    const bool act = t < run.tiles;  // wave-uniform
#pragma unroll
    for (int u = 0; u < 2 * NC; ++u) pin(xk[u]);
    const int ta = tile_tok(run.tok0, H, act ? t : last_tile);
    const int64_t row0 = tile_row0(job, S, H, ta);
    const int tok = ta + r / H;
    load_tile<NC>(poolV, row0, xv);
    // ---------------- K: per-channel statistics from the kstats pass
    if (act) {
      tile_to_half_rows<NC>(wbuf, xk);
      sign_half_row<NC>(T, hme, hl, xk);
      LanePack<HALF, BITS> pkd;
      quant_k_tile<NC, BITS, CLAMP>(xk, hp, hn, &T.kc[0][0] + opaque(hme * (128 + 4) + HALF * hl), s, lp.lvk, pkd,
                                    over, paired);
      pkd.store_lds(ost + offk);
      if (!coop) flush(0, ta);
    }
    if (coop) {
      __syncthreads();
      flush_wg(0, it * W);
      __syncthreads();
    }
    // next tile's K (unconditional: past the end it re-reads the last tile, a cache hit)
    const int tn = min(t + W, last_tile);
    load_tile<NC>(poolK, tile_row0(job, S, H, tile_tok(run.tok0, H, tn)), xk);
    // ---------------- V: per-token statistics over the heads of a group
    if (act) {
      tile_to_half_rows<NC>(wbuf, xv);
      sign_half_row<NC>(T, hme, hl, xv);
      LanePack<HALF, BITS> pkd;
      quant_v_tile_lds<NC, BITS, CLAMP>(xv, hp, hn, lp, job, ntok, tok, G, H, s, wbuf + l, pkd, over, paired);
      pkd.store_lds(ost + offv);
      if (!coop) flush(1, ta);
    }
    if (coop) {
      __syncthreads();
      flush_wg(1, it * W);
      __syncthreads();
    }
  }
  if (over & overflow_mask<BITS>()) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
}

// Waves per workgroup of encode_mfma_kernel: 8 at D = 64, so that the workgroup-wide flush
// of the permuted order joins 8 tiles per head run (8 x 96 bytes at 3 bits) instead of 4;
// at D = 64 two such workgroups per CU hold the same 16 waves as four of 4.
template <int NC>
constexpr int kEncWaves = NC == 2 ? 8 : kWaves;
template <int NC, int BITS, bool CLAMP>
__global__ __launch_bounds__(64 * kEncWaves<NC>) void encode_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                                          int32_t* __restrict__ err) {
  encode_body<NC, BITS, CLAMP, kMH, false, kEncWaves<NC>>(g, jobs, err);
}
// 16 or 32 KV heads: a tile holds 2 tokens or 1 (32 rows), with tables for 32 heads.
template <int NC, int BITS, bool CLAMP>
__global__ __launch_bounds__(kMW) void encode_mfma_wide_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                               int32_t* __restrict__ err) {
  encode_body<NC, BITS, CLAMP, kWideH, false>(g, jobs, err);
}
// head_dim 256 as paired virtual heads of 128, with tables for HM virtual heads
template <int BITS, bool CLAMP, int HM>
__global__ __launch_bounds__(kMW) void encode_mfma_pair_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                               int32_t* __restrict__ err) {
  encode_body<4, BITS, CLAMP, HM, true>(g, jobs, err);
}

// ============================================================== decode (orientation T)
// NW waves per workgroup share one set of tables (and one header check).
template <int NC, int BITS, int NW, int HM, bool PAIRED>
__device__ __forceinline__ void decode_body(const Geo& g, const kvmi_layer_job* __restrict__ jobs,
                                            int32_t* __restrict__ err) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H, G = g.G;
  const int ntok = job.num_blocks * S;
  const Run run = wg_run(job, g);
  if ((int)blockIdx.x >= run.nwg) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;

  __shared__ TablesT<HM> T;
  __shared__ int ok;
  // Per-wave staging of an output tile (32 rows, row pitch RP uint4 with one of
  // padding): rows are written as the MFMA leaves them and stored lane-linear, so
  // each store instruction writes 1 KB of consecutive bytes of the tile.
  constexpr int RQ = 4 * NC, RP = RQ + 1;  // uint4 per row, pitch
  __shared__ uint4 stage[NW * kTok * RP];
  static_assert(!kVTable<BITS> || vtab_bytes<BITS>() <= kTok * RP * 16, "V table fits a wave's staging space");
  static_assert(vtab_bytes<3>() <= kTok * 9 * 16, "the 3-bit V table fits a wave's staging space");
  // At D = 64 and widths up to 4 (and up to 8 heads), K is dequantized by lookups in
  // a table of every (source head, channel, symbol) value too (9 KiB at 3 bits).
  constexpr bool kKTab = NC == 2 && BITS <= 4 && HM == kMH;
  __shared__ __attribute__((aligned(16))) uint8_t ktab[kKTab ? D * ktab_row<BITS>() : 16];
  if (threadIdx.x == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  constexpr bool paired = PAIRED;
  stage_profile(T, job.profile, H, paired);
  fill_signs(T, job.signs, H, D);
  __syncthreads();
  if (!ok) return;
  fill_positions(T, H);
  if constexpr (kKTab)
    fill_k_table_w<BITS>(ktab, T, job.kmeta, H, D);
  else
    fill_kconst<false>(T, job.kmeta, H, D);
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile(0, false, false);
  hp[1] = hadamard_tile(1, false, false);
  hn[0] = hadamard_tile(0, false, true);
  hn[1] = hadamard_tile(1, false, true);
  uint16_t* poolK = reinterpret_cast<uint16_t*>(job.pool);
  const int hme = r % H;
  const int jk = T.posk[hme], jv = T.posv[hme];
  const int gv = T.prof[1][2][jv];
  const float s = g.scale;
  const uint32_t kbase = lds_addr(ktab) + (uint32_t)(2 * hme + HALF * hl * ktab_row<kKTab ? BITS : 1>());

  // section q = part * tiles + t: K tiles, then V tiles.  A section's inputs are its
  // packed symbols and, for V, the row's (min, scale).
  struct In {
    LanePack<HALF, BITS> pk;
    uint32_t mn, sc;  // bf16 bits of the V row's (min, scale); unused for K
  };
  // Loads of every section have the same shape (the V metadata of the token is read
  // for K sections too), so no load is issued on one path only.
  auto fetch = [&](int q, In& in) {
    const int part = q >= run.tiles, t = q - part * run.tiles;
    const int tok = tile_tok(run.tok0, H, t) + r / H;
    in.pk.load(seg_addr<BITS, PAIRED>(job, g, part, part ? jv : jk, tok, HALF * hl));
    in.mn = gld(job.vmeta + (int64_t)gv * ntok + tok);
    in.sc = gld(job.vmeta + (int64_t)(G + gv) * ntok + tok);
  };
  auto section = [&](int q, In& in) {
#pragma unroll
    for (int i = 0; i < LanePack<HALF, BITS>::kWords; ++i) pin(in.pk.w[i]);
    pin(in.mn);
    pin(in.sc);
    const int part = q >= run.tiles, t = q - part * run.tiles;
    const int64_t row0 = tile_row0(job, S, H, tile_tok(run.tok0, H, t));
    // dequantize into bf16 MFMA operands: x~ = bf16(bf16(q * scale) + min)
    uint4 x[2 * NC];
    uint4* stg = stage + wave * (kTok * RP);
    if (part) {
      // V: the row table lives in the wave's staging space (free until the transform)
      if constexpr (kVTable<BITS>)
        dequant_v_table<NC, BITS>(in.pk, bf16_to_f32(in.mn), bf16_to_f32(in.sc), stg, x);
      else if constexpr (BITS == 3)
        dequant_v_table_bfe<NC, BITS>(in.pk, bf16_to_f32(in.mn), bf16_to_f32(in.sc), stg, x);
      else
        dequant_half_row<NC, BITS, false>(in.pk, nullptr, bf16_to_f32(in.mn), bf16_to_f32(in.sc), x);
    } else if constexpr (kKTab) {
      dequant_k_table_w<NC, BITS>(in.pk, opaque(kbase), x);
    } else
      dequant_half_row<NC, BITS, true>(in.pk, &T.kc[0][0] + opaque(hme * (128 + 4) + HALF * hl), 0.f, 0.f, x);
    chunk_fence();
    const uint4* sm = reinterpret_cast<const uint4*>(&T.smask[0][0] + opaque(hme * (64 + 4) + (HALF / 2) * hl));
#pragma unroll
    for (int cp = 0; cp < NC; ++cp) {
      f32x16 acc = transform_T<NC>(x, hp, hn, cp);
      if (paired) pair_butterfly_T(acc);
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = pack_bf16x2(acc[2 * i] * s, acc[2 * i + 1] * s);
      stg[r * RP + 2 * NC * hl + 2 * cp] = xor4(make_uint4(w[0], w[1], w[2], w[3]), sm[2 * cp]);
      stg[r * RP + 2 * NC * hl + 2 * cp + 1] = xor4(make_uint4(w[4], w[5], w[6], w[7]), sm[2 * cp + 1]);
      chunk_fence();
    }
    // the tile's 32 rows are contiguous in the pool
    uint4* dst = reinterpret_cast<uint4*>(poolK + part * job.pool_part_stride + row0 * D);
#pragma unroll
    for (int u = 0; u < RQ * kTok / 64; ++u) {
      const int qq = 64 * u + l;
      gst_stream(dst + qq, stg[(qq / RQ) * RP + qq % RQ]);
    }
  };
  const int nsec = 2 * run.tiles, last_sec = nsec - 1;
  if constexpr (NC == 2) {
    // Three input buffers: sections q + NW and q + 2 NW are loading while section q is
    // computed.  At D = 64 a section's loads are several small pieces (a 3-bit half-row
    // is 12 bytes) and its compute is short, so one section of look-ahead left them
    // exposed; a buffer is 5 VGPRs here.
    In a, b, c;
    if (wave < nsec) {
      fetch(wave, a);
      fetch(min(wave + NW, last_sec), b);
    }
    for (int q = wave; q < nsec; q += 3 * NW) {
      fetch(min(q + 2 * NW, last_sec), c);
      section(q, a);
      if (q + NW >= nsec) break;
      fetch(min(q + 3 * NW, last_sec), a);
      section(q + NW, b);
      if (q + 2 * NW >= nsec) break;
      fetch(min(q + 4 * NW, last_sec), b);
      section(q + 2 * NW, c);
    }
  } else {
    // Two input buffers: section q + NW is loading while section q is computed (past
    // the end the prefetch re-reads the current section, a cache hit).
    In a, b;
    if (wave < nsec) fetch(wave, a);
    for (int q = wave; q < nsec; q += 2 * NW) {
      fetch(min(q + NW, last_sec), b);
      section(q, a);
      if (q + NW >= nsec) break;
      fetch(min(q + 2 * NW, last_sec), a);
      section(q + NW, b);
    }
  }
}

template <int NC, int BITS, int NW>
__global__ __launch_bounds__(64 * NW) void decode_mfma_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                              int32_t* __restrict__ err) {
  decode_body<NC, BITS, NW, kMH, false>(g, jobs, err);
}
template <int NC, int BITS, int NW>
__global__ __launch_bounds__(64 * NW) void decode_mfma_wide_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                                   int32_t* __restrict__ err) {
  decode_body<NC, BITS, NW, kWideH, false>(g, jobs, err);
}
template <int BITS, int NW, int HM>
__global__ __launch_bounds__(64 * NW) void decode_mfma_pair_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                                   int32_t* __restrict__ err) {
  decode_body<4, BITS, NW, HM, true>(g, jobs, err);
}

// ============================================================== decode, K by table (D = 128, 4 bits)
// decode_mfma_kernel<4, 4, NW> with K dequantized by LDS lookups too.  A K element has
// per-channel constants, so its table covers every (source head, channel): 34 KiB per
// workgroup, made room for by staging half a row at a time.  That needs the element
// split of hadamard_tile_d, where a lane's outputs of chunks 0-1 (2-3) are the row's
// first (second) 128 bytes: the lane's inputs are then elements 16 s + 8 hl + (0..7),
// which the lane pair (r, r + 32) trades from their loaded half-rows with one
// v_permlane32_swap per two words.
template <int NW>
__global__ __launch_bounds__(64 * NW) void decode_kt_kernel(Geo g, const kvmi_layer_job* __restrict__ jobs,
                                                            int32_t* __restrict__ err) {
  constexpr int NC = 4, BITS = 4, D = 128, HALF = 64;
  const kvmi_layer_job job = jobs[blockIdx.y];
  const int S = g.S, H = g.H, G = g.G;
  const int ntok = job.num_blocks * S;
  const Run run = wg_run(job, g);
  if ((int)blockIdx.x >= run.nwg) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;

  __shared__ __attribute__((aligned(16))) DecTables T;
  __shared__ int ok;
  // Per-wave staging of half an output tile (32 rows x 128 bytes, pitch RP uint4 with
  // one of padding), stored lane-linear: every store instruction writes eight full
  // 128-byte lines.  The V row table lives in the same space until the transform.
  constexpr int RH = 8, RP = RH + 1;
  __shared__ uint4 stage[NW * kTok * RP];
  __shared__ __attribute__((aligned(16))) uint8_t ktab[D * kKtabRow];
  static_assert(vtab_bytes<BITS>() <= kTok * RP * 16, "V table fits a wave's staging space");
  if (threadIdx.x == 0) {
    int good = 1;
    if (!(g.flags & KVMI_F_NO_HEADER)) {
      good = header_matches(job.stream, BITS, job.chunk_symbols);
      if (!good && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    }
    ok = good;
  }
  stage_profile(T, job.profile, H);
  fill_signs(T, job.signs, H, D);
  __syncthreads();
  if (!ok) return;
  fill_positions(T, H);
  fill_k_table(ktab, T, job.kmeta, H, D);
  __syncthreads();

  uint4 hp[2], hn[2];
  hp[0] = hadamard_tile_d(0, false);
  hp[1] = hadamard_tile_d(1, false);
  hn[0] = hadamard_tile_d(0, true);
  hn[1] = hadamard_tile_d(1, true);
  uint16_t* poolK = reinterpret_cast<uint16_t*>(job.pool);
  const int hme = r % H;
  const int jk = T.posk[hme], jv = T.posv[hme];
  const int gv = T.prof[1][2][jv];
  const float s = g.scale;
  const uint32_t kbase = lds_addr(ktab) + (uint32_t)(8 * hl * kKtabRow + 2 * hme);

  struct In {
    LanePack<HALF, BITS> pk;
    uint32_t mn, sc;  // bf16 bits of the V row's (min, scale); unused for K
  };
  auto fetch = [&](int q, In& in) {
    const int part = q >= run.tiles, t = q - part * run.tiles;
    const int tok = tile_tok(run.tok0, H, t) + r / H;
    in.pk.load(seg_addr<BITS>(job, g, part, part ? jv : jk, tok, HALF * hl));
    in.mn = gld(job.vmeta + (int64_t)gv * ntok + tok);
    in.sc = gld(job.vmeta + (int64_t)(G + gv) * ntok + tok);
  };
  auto section = [&](int q, In& in) {
#pragma unroll
    for (int i = 0; i < LanePack<HALF, BITS>::kWords; ++i) pin(in.pk.w[i]);
    pin(in.mn);
    pin(in.sc);
    const int part = q >= run.tiles, t = q - part * run.tiles;
    const int64_t row0 = tile_row0(job, S, H, tile_tok(run.tok0, H, t));
    // word s: the symbols of elements 16 s + 8 hl + (0..7).  Lane half 0 holds words
    // (2u, 2u + 1) = elements 16u + (0..15) of its row, half 1 the same of 64 + 16u:
    // the swap leaves half 0 with (its 2u, the partner's 2u) and half 1 with (the
    // partner's 2u + 1, its 2u + 1).
    LanePack<HALF, BITS> W;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const auto pr = __builtin_amdgcn_permlane32_swap(in.pk.w[2 * u], in.pk.w[2 * u + 1], false, false);
      W.w[u] = pr[0];
      W.w[u + 4] = pr[1];
    }
    uint4 x[2 * NC];
    uint4* stg = stage + wave * (kTok * RP);
    if (part)
      dequant_v_table<NC, BITS>(W, bf16_to_f32(in.mn), bf16_to_f32(in.sc), stg, x);
    else
      dequant_k_table(W.w, kbase, x);
    chunk_fence();
    // output signs of (head, element pair 16 c' + 8 hl + (0..7)): uint4 4 c' and 4 c' + 1
    const uint4* sm = reinterpret_cast<const uint4*>(&T.smask[0][0] + opaque(hme * (64 + 4) + 8 * hl));
    // the tile's 32 rows are contiguous in the pool; half h of a row is its bytes
    // [128 h, 128 h + 128) = uint4 8 h .. 8 h + 7
    uint4* dst = reinterpret_cast<uint4*>(poolK + part * job.pool_part_stride + row0 * D);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const int cp = 2 * h + c2;
        const f32x16 acc = transform_T<NC>(x, hp, hn, cp);
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = pack_bf16x2(acc[2 * i] * s, acc[2 * i + 1] * s);
        stg[r * RP + 4 * c2 + 2 * hl] = xor4(make_uint4(w[0], w[1], w[2], w[3]), sm[4 * cp]);
        stg[r * RP + 4 * c2 + 2 * hl + 1] = xor4(make_uint4(w[4], w[5], w[6], w[7]), sm[4 * cp + 1]);
        chunk_fence();
      }
#pragma unroll
      for (int u = 0; u < RH * kTok / 64; ++u) {
        const int qq = 64 * u + l, row = qq / RH, j = qq % RH;
        gst_stream(dst + row * (4 * NC) + RH * h + j, stg[row * RP + j]);
      }
    }
  };
  const int nsec = 2 * run.tiles, last_sec = nsec - 1;
  In a, b;
  if (wave < nsec) fetch(wave, a);
  for (int q = wave; q < nsec; q += 2 * NW) {
    fetch(min(q + NW, last_sec), b);
    section(q, a);
    if (q + NW >= nsec) break;
    fetch(min(q + 2 * NW, last_sec), a);
    section(q + NW, b);
  }
}

// ============================================================== launch
// Workgroups that fit on the device at once for `kernel` (CUs x resident
// workgroups per CU), per (device, kernel), computed on first use.
constexpr int kMaxDevices = 64;
std::mutex g_resident_mu;
std::unordered_map<const void*, int> g_resident[kMaxDevices];
template <class K>
int resident_wgs(K kernel, int threads = kMW) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 1024;
  const void* key = reinterpret_cast<const void*>(kernel);
  std::lock_guard<std::mutex> lock(g_resident_mu);
  auto it = g_resident[dev].find(key);
  if (it != g_resident[dev].end()) return it->second;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, key, threads, 0) != hipSuccess) per = 2;
  const int v = (cus > 0 ? cus : 1) * (per > 0 ? per : 1);
  g_resident[dev].emplace(key, v);
  return v;
}

// Blocks per workgroup: whole multiples of the blocks that make up a 32-row tile
// (S*H % 32 == 0), sized so that the launch is about `target` workgroups.
int run_blocks(const Geo& g, int32_t max_blocks, int32_t num_jobs, int target) {
  const int unit = (kTok / g.H + g.S - 1) / g.S;  // blocks per tile (1 when S >= 32/H)
  const int64_t total = (int64_t)max_blocks * (num_jobs > 0 ? num_jobs : 1);
  int64_t want = (total + target - 1) / (target > 0 ? target : 1);
  if (want > max_blocks) want = max_blocks;
  int bpw = (int)((want + unit - 1) / unit) * unit;
  return bpw < unit ? unit : bpw;
}

// Workgroups per resident slot: more, shorter runs balance the end of a launch
// better; each run also pays its table set-up once.  A slot is a resident workgroup of
// the statistics kernel of the geometry's head_dim (slot_wgs), for every kernel: the
// launch shapes these counts were measured with (config 2: 768 slots, so 768, 2304 and
// 2304 workgroups; decode's own occupancy, 2 per CU, would give 1536 at 3 rounds,
// 2.4 % slower).
constexpr int kRoundsKstats = 1, kRoundsEncode = 3, kRoundsDecode = 3;
constexpr int kLongRunTiles = 128;

int slot_wgs(const Geo& g) {
  return g.D == 64 ? resident_wgs(kstats_mfma_kernel<2>) : resident_wgs(kstats_mfma_kernel<4>);
}

template <class K>
int launch(K kernel, Geo g, int32_t num_jobs, int32_t max_blocks, const kvmi_layer_job* jobs, int32_t* err,
           hipStream_t st, int rounds, int threads = kMW) {
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  g.bpw = run_blocks(g, max_blocks, num_jobs, slot_wgs(g) * rounds);
  // Long runs (more than kLongRunTiles tiles a workgroup: long requests, or batches sized
  // as if every request were as long as the longest) end the launch unbalanced: there the
  // rounds double, up to three times, while runs stay long and the longest job still splits
  // into at least four runs (config 3: compress -6.7 %, decompress -5.5 %; config 4 -5.5 %
  // and -5.8 %).  Config 2's runs of 32 tiles keep theirs (twice the rounds: +1 %), and so
  // do short jobs: splitting a 16-block job in two uneven runs made config 5 14 % slower.
  for (int k = 0; k < 3 && rounds > 1 && (int64_t)g.bpw * g.S * g.H > (int64_t)kLongRunTiles * kTok; ++k) {
    rounds *= 2;
    const int bpw2 = run_blocks(g, max_blocks, num_jobs, slot_wgs(g) * rounds);
    if (max_blocks < 4 * bpw2) break;
    g.bpw = bpw2;
  }

  const int per_job = (max_blocks + g.bpw - 1) / g.bpw;
  hipLaunchKernelGGL(kernel, dim3((unsigned)per_job, (unsigned)num_jobs), dim3(threads), 0, st, g, jobs, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

template <int NC, int BITS>
int launch_enc(const Geo& g, int32_t nj, int32_t mb, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  const bool clamp = g.flags & KVMI_F_CLAMP_LEVELS;
  if constexpr (NC == 4)
    if (g.flags & kPairedHeads) {
      if (g.H > kMH)
        return clamp ? launch(encode_mfma_pair_kernel<BITS, true, kWideH>, g, nj, mb, jobs, err, st, kRoundsEncode)
                     : launch(encode_mfma_pair_kernel<BITS, false, kWideH>, g, nj, mb, jobs, err, st, kRoundsEncode);
      return clamp ? launch(encode_mfma_pair_kernel<BITS, true, kMH>, g, nj, mb, jobs, err, st, kRoundsEncode)
                   : launch(encode_mfma_pair_kernel<BITS, false, kMH>, g, nj, mb, jobs, err, st, kRoundsEncode);
    }
  if (g.H > kMH)
    return clamp ? launch(encode_mfma_wide_kernel<NC, BITS, true>, g, nj, mb, jobs, err, st, kRoundsEncode)
                 : launch(encode_mfma_wide_kernel<NC, BITS, false>, g, nj, mb, jobs, err, st, kRoundsEncode);
  return clamp ? launch(encode_mfma_kernel<NC, BITS, true>, g, nj, mb, jobs, err, st, kRoundsEncode, 64 * kEncWaves<NC>)
               : launch(encode_mfma_kernel<NC, BITS, false>, g, nj, mb, jobs, err, st, kRoundsEncode,
                        64 * kEncWaves<NC>);
}
constexpr int kDecodeWaves = 8;  // waves per decode workgroup (two workgroups per CU)
template <int NC, int BITS>
int launch_dec(const Geo& g, int32_t nj, int32_t mb, const kvmi_layer_job* jobs, int32_t* err, hipStream_t st) {
  if constexpr (NC == 4)
    if (g.flags & kPairedHeads) {
      if (g.H > kMH)
        return launch(decode_mfma_pair_kernel<BITS, kDecodeWaves, kWideH>, g, nj, mb, jobs, err, st, kRoundsDecode,
                      64 * kDecodeWaves);
      return launch(decode_mfma_pair_kernel<BITS, kDecodeWaves, kMH>, g, nj, mb, jobs, err, st, kRoundsDecode,
                    64 * kDecodeWaves);
    }
  if (g.H > kMH)
    return launch(decode_mfma_wide_kernel<NC, BITS, kDecodeWaves>, g, nj, mb, jobs, err, st, kRoundsDecode,
                  64 * kDecodeWaves);
  if constexpr (NC == 4 && BITS == 4)
    return launch(decode_kt_kernel<kDecodeWaves>, g, nj, mb, jobs, err, st, kRoundsDecode, 64 * kDecodeWaves);
  else
    return launch(decode_mfma_kernel<NC, BITS, kDecodeWaves>, g, nj, mb, jobs, err, st, kRoundsDecode,
                  64 * kDecodeWaves);
}

#define KVMI_MFMA_BITS(FN, NC)                                 \
  switch (g.bits) {                                            \
    case 1: return FN<NC, 1>(g, nj, mb, jobs, err, st);        \
    case 2: return FN<NC, 2>(g, nj, mb, jobs, err, st);        \
    case 3: return FN<NC, 3>(g, nj, mb, jobs, err, st);        \
    case 4: return FN<NC, 4>(g, nj, mb, jobs, err, st);        \
    case 5: return FN<NC, 5>(g, nj, mb, jobs, err, st);        \
    case 6: return FN<NC, 6>(g, nj, mb, jobs, err, st);        \
    case 7: return FN<NC, 7>(g, nj, mb, jobs, err, st);        \
    default: return FN<NC, 8>(g, nj, mb, jobs, err, st);       \
  }

}  // namespace

int mfma_kstats(const Geo& g, const kvmi_layer_job* jobs, int32_t nj, int32_t mb, int32_t* err, hipStream_t st) {
  if (g.flags & kPairedHeads)
    return g.H > kMH ? launch(kstats_wide_pair_kernel, g, nj, mb, jobs, err, st, kRoundsKstats)
                     : launch(kstats_mfma_pair_kernel, g, nj, mb, jobs, err, st, kRoundsKstats);
  if (g.H > kMH)
    return g.D == 64 ? launch(kstats_wide_kernel<2>, g, nj, mb, jobs, err, st, kRoundsKstats)
                     : launch(kstats_wide_kernel<4>, g, nj, mb, jobs, err, st, kRoundsKstats);
  if (g.D == 64) return launch(kstats_mfma_kernel<2>, g, nj, mb, jobs, err, st, kRoundsKstats);
  return launch(kstats_mfma_kernel<4>, g, nj, mb, jobs, err, st, kRoundsKstats);
}

int mfma_encode(const Geo& g, const kvmi_layer_job* jobs, int32_t nj, int32_t mb, int32_t* err, hipStream_t st) {
  if (g.D == 64) {
    KVMI_MFMA_BITS(launch_enc, 2)
  }
  KVMI_MFMA_BITS(launch_enc, 4)
}

int mfma_decode(const Geo& g, const kvmi_layer_job* jobs, int32_t nj, int32_t mb, int32_t* err, hipStream_t st) {
  if (g.D == 64) {
    KVMI_MFMA_BITS(launch_dec, 2)
  }
  KVMI_MFMA_BITS(launch_dec, 4)
}

}  // namespace kvmi
