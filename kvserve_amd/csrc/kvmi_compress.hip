// One-pass paged compress on gfx950: every K and V value of a (request, layer) job is
// read from HBM once.
//
// K is quantized with per-channel statistics over all tokens of the job
// (quantizer_func.py:41-56, axis "channel"), so no K symbol can be written before the
// whole job's K of that channel has been seen.  The two-pass path (kvmi_mfma.hip) reads
// K twice.  Here a cooperative, persistent grid (one workgroup of 8 waves per CU) walks
// a host-built schedule of steps, and every wave keeps its K tile in registers from the
// statistics in one step to the quantization in the next:
//
//   * K work is split by (job, head): a "group" is the K of one head of one job, cut
//     into head-tiles of 32 consecutive tokens (rows H*D*2 bytes apart in the pool).
//     The per-channel statistics of a head depend on that head's tokens only, so a
//     group's barrier spans just the workgroups that hold its tiles (8 per workgroup,
//     one per wave): 32 workgroups for an 8192-token job, one for a 256-token job,
//     which then needs no device barrier at all.
//   * V work is token-major tiles (32 rows = 32/H tokens x H heads, as the cache stores
//     them), 8 per workgroup and step; per-token statistics need no other workgroup.
//   * Step s of a workgroup (all waves do the same kinds of work):
//       P1  statistics of its K head-tile of step s (MFMA orientation N, per-channel
//           min / max in registers, then LDS atomics); the last wave of the workgroup to
//           finish pushes the workgroup's keys to the group's device keys and stores the
//           call's epoch into the workgroup's arrival flag;
//       P3  quantization of its K head-tile of step s - 1 (orientation T), held in
//           registers since then: the first wave there waits for that group's flags,
//           turns the keys into per-channel constants for the whole workgroup and
//           writes the K metadata (the group's first workgroup);
//       P2  encode of its V tile of step s.
//     A group's arrival (P1 of step s) and its first use (P3 of step s + 1) are a V
//     encode and a statistics pass apart, which hides the barrier.  The loads of the
//     next K tile are issued after P3 into the registers of the tile it quantized, and
//     those of the next V tile after P2.
//   * Keys and flags need no clearing between calls: a key is a 64-bit (epoch << 32 |
//     order-preserving key) maximum, a flag holds the epoch of its workgroup's last
//     arrival.  The epoch lives in the workspace and a one-thread kernel enqueued just
//     before the pass advances it, so a captured graph advances it on every replay.
//   * Every wait is bounded: on timeout the kernel sets KVMI_ERR_SYNC, later device
//     waits give up at once, and every wave reaches the end of the kernel.
#include <algorithm>
#include <climits>
#include <cstring>
#include <vector>

#include "kvmi_mfma_tiles.hpp"

namespace kvmi {
namespace {

constexpr int kOW = 8;        // waves per workgroup (two per SIMD: three do not fit the registers at D = 128)
constexpr int kOT = 64 * kOW; // threads per workgroup
constexpr int kTPW = kOW;     // K head-tiles and V tiles per workgroup and step (one per wave)
constexpr uint32_t kOpMagic = 0x5350314Bu;  // "K1PS"
constexpr uint32_t kMaxPolls = 1u << 18;    // ~0.3 s of polling before KVMI_ERR_SYNC
constexpr int64_t kMinWorkspace = 16 * 1024;  // the idle waves' dummy loads read 8 KiB at its start

// One workgroup's work in one step.
struct OpRec {
  int32_t kjob;    // job of the K head-tiles (-1: none)
  int32_t khead;   // head | tiles << 8 (1..8)
  int32_t ktile0;  // first head-tile of the group this workgroup takes (rank * 8)
  int32_t kgroup;  // first workgroup of the group in the step | workgroups in the group << 16
  int32_t kslot;   // device key slot of a group of several workgroups (-1: one workgroup)
  int32_t vjob;    // job of the V tiles (-1: none)
  int32_t vtile0;  // first token-major V tile of the job
  int32_t vn;      // V tiles (1..8)
};
static_assert(sizeof(OpRec) == 32, "schedule records are 32 bytes");

// Header of a schedule image (first bytes of the workspace as well).
struct OpHeader {
  uint32_t magic;
  int32_t grid, steps, num_jobs;
  int32_t S, H, D, bits;
  uint32_t flags;
  int32_t nslots;
  int64_t rec_off, flag_off, key_off, epoch_off, total;
  int64_t image_bytes;
  int64_t blk_off;  // int32 [num_jobs]: the blocks of each job the schedule was built for
};
constexpr int64_t kHeaderBytes = 256;
static_assert(sizeof(OpHeader) <= kHeaderBytes, "header fits its slot");

int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

struct OpArgs {
  Geo g;
  const kvmi_layer_job* jobs;
  int32_t* err;
  const OpRec* recs;         // [steps][grid]
  uint32_t* flags;           // [steps][grid]
  unsigned long long* keys;  // [nslots][2][D]
  const uint32_t* epoch;     // advanced by onepass_epoch_kernel
  const uint16_t* dummy;     // 8 KiB of readable memory for the loads of idle waves
  const int32_t* sched_blocks;  // [num_jobs] blocks per job in the schedule
  int steps, grid, num_jobs;
};

// A job descriptor through the constant address space (scalar loads: the table is
// read-only for the whole launch).
__device__ __forceinline__ kvmi_layer_job load_job(const kvmi_layer_job* jobs, int i) {
  const kvmi_layer_job* q = jobs + i;
  kvmi_layer_job j;
  j.pool = cld(&q->pool);
  j.block_ids = cld(&q->block_ids);
  j.stream = cld(&q->stream);
  j.kmeta = cld(&q->kmeta);
  j.vmeta = cld(&q->vmeta);
  j.signs = cld(&q->signs);
  j.profile = cld(&q->profile);
  j.kstats = nullptr;
  j.pool_blocks = 0;
  j.pool_part_stride = cld(&q->pool_part_stride);
  j.symbol_offset = cld(&q->symbol_offset);
  j.chunk_symbols = cld(&q->chunk_symbols);
  j.num_blocks = cld(&q->num_blocks);
  j.write_header = cld(&q->write_header);
  return j;
}

__device__ __forceinline__ OpRec load_rec(const OpRec* recs, int64_t i) {
  const OpRec* q = recs + i;
  OpRec r;
  r.kjob = cld(&q->kjob);
  r.khead = cld(&q->khead);
  r.ktile0 = cld(&q->ktile0);
  r.kgroup = cld(&q->kgroup);
  r.kslot = cld(&q->kslot);
  r.vjob = cld(&q->vjob);
  r.vtile0 = cld(&q->vtile0);
  r.vn = cld(&q->vn);
  return r;
}
__device__ __forceinline__ OpRec no_rec() {
  OpRec r;
  r.kjob = r.vjob = r.kslot = -1;
  r.khead = r.ktile0 = r.kgroup = r.vtile0 = r.vn = 0;
  return r;
}

// Everything a workgroup needs of one step, staged into LDS two steps ahead by one wave
// (so that no other wave waits on the scalar loads of records, job descriptors and block
// ids: on gfx950 LDS and scalar loads share one wait counter, so an outstanding scalar
// load holds up the next LDS access of its wave).
struct StepTables {
  uint32_t smask[kMH][64 + 4];  // V: sign-flip masks per (head, element pair)
  uint32_t kmask[64 + 4];       // K statistics: the masks of the group's head
  uint8_t prof[2][3][kMH];      // the V job's profile
  int posk[kMH], posv[kMH], gfirst[kMH];
  OpRec rec;                    // this workgroup's record of the step
  int kjk, kjlv;                // K job: output position and levels of the group's head
  kvmi_layer_job kj, vj;        // the K and V jobs
  int32_t krow[kOW][8];         // K: pool row of each wave's load instruction v (-1 - row past the
                                // job's last token, INT32_MIN without a tile)
  int64_t vrow[kOW];            // V: first pool row of each wave's tile (-1 without one)
};

// Wave-uniform copies of LDS values (v_readfirstlane: the compiler cannot see that every
// lane reads the same address).
__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
template <class T>
__device__ __forceinline__ T* uni(T* p) { return reinterpret_cast<T*>(uni((int64_t)reinterpret_cast<uintptr_t>(p))); }
__device__ __forceinline__ OpRec uni(const OpRec& r) {
  OpRec u;
  u.kjob = uni(r.kjob);
  u.khead = uni(r.khead);
  u.ktile0 = uni(r.ktile0);
  u.kgroup = uni(r.kgroup);
  u.kslot = uni(r.kslot);
  u.vjob = uni(r.vjob);
  u.vtile0 = uni(r.vtile0);
  u.vn = uni(r.vn);
  return u;
}
__device__ __forceinline__ kvmi_layer_job uni(const kvmi_layer_job& j) {
  kvmi_layer_job u;
  u.pool = uni(j.pool);
  u.block_ids = uni(j.block_ids);
  u.stream = uni(j.stream);
  u.kmeta = uni(j.kmeta);
  u.vmeta = uni(j.vmeta);
  u.signs = uni(j.signs);
  u.profile = uni(j.profile);
  u.kstats = nullptr;
  u.pool_blocks = 0;
  u.pool_part_stride = uni(j.pool_part_stride);
  u.symbol_offset = uni(j.symbol_offset);
  u.chunk_symbols = uni(j.chunk_symbols);
  u.num_blocks = uni(j.num_blocks);
  u.write_header = uni(j.write_header);
  return u;
}

// ---------------------------------------------------------------- pipelined tile work
// Within a wave the products of output chunk cp + 1 are issued while chunk cp's results
// are reduced or quantized: the MFMA chain of one chunk and the VALU work of the other
// are independent, so the matrix cores and the VALU work at the same time (two
// accumulators live instead of one).  A fence closes each chunk so that no further
// chunk is hoisted.

// Orientation N product of output chunk cp (A = rows, B = Hadamard tile): column n of
// the result is channel HALF n2 + 16 cp + 8 n4 + 4 n3 + 2 n1 + n0 with the orientation-T
// operand tiles (the Sylvester matrix is symmetric).
template <int NC>
__device__ __forceinline__ f32x16 transform_N(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                              int cp) {
  f32x16 acc = {};
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = cp ^ k;
    const bool neg = __builtin_popcount(c & cp) & 1;
    acc = mfma(x[2 * c], neg ? hn[0] : hp[0], acc);
    acc = mfma(x[2 * c + 1], neg ? hn[1] : hp[1], acc);
  }
  return acc;
}

// K statistics of one signed head-tile into the workgroup's LDS keys [2][D] (unscaled).
template <int NC>
__device__ __forceinline__ void kstats_head_tile(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                                 uint32_t* lkey) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31;
  f32x16 a0 = transform_N<NC>(x, hp, hn, 0);
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 a1 = a0;
    if (cp + 1 < NC) a1 = transform_N<NC>(x, hp, hn, cp + 1);
    float mn = fminf(fminf(a0[0], a0[1]), fminf(a0[2], a0[3]));
    float mx = fmaxf(fmaxf(a0[0], a0[1]), fmaxf(a0[2], a0[3]));
#pragma unroll
    for (int i = 4; i < 16; i += 4) {
      mn = fminf(fminf(mn, a0[i]), fminf(a0[i + 1], fminf(a0[i + 2], a0[i + 3])));
      mx = fmaxf(fmaxf(mx, a0[i]), fmaxf(a0[i + 1], fmaxf(a0[i + 2], a0[i + 3])));
    }
    mn = halves_min(mn);
    mx = halves_max(mx);
    if (hl == 0) {
      const int f = HALF * ((r >> 2) & 1) + 16 * cp + 8 * ((r >> 4) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
      atomicMin(&lkey[f], f2key(mn));  // unscaled: 1/sqrt(D) > 0 commutes with min / max
      atomicMax(&lkey[D + f], f2key(mx));
    }
    chunk_fence();
    a0 = a1;
  }
}

// quant_k_tile with the next chunk's products in flight during each quantization.
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_k_tile_pipe(const uint4 (&xk)[2 * NC], const uint4 (&hp)[2],
                                                  const uint4 (&hn)[2], const float2* kq, float s, float lvk,
                                                  LanePack<16 * NC, BITS>& pkd, uint32_t& over) {
  pkd.clear();
  f32x16 a0 = transform_T<NC>(xk, hp, hn, 0);
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 a1 = a0;
    if (cp + 1 < NC) a1 = transform_T<NC>(xk, hp, hn, cp + 1);
    quant_chunk_k<16 * NC, BITS, CLAMP>(a0, cp, s, kq + 16 * cp, lvk, pkd, over);
    chunk_fence();
    a0 = a1;
  }
}

// quant_v_tile_lds with the next chunk's products in flight during each chunk's
// statistics and rounding.
template <int NC, int BITS, bool CLAMP>
__device__ __forceinline__ void quant_v_tile_pipe(const uint4 (&xv)[2 * NC], const uint4 (&hp)[2],
                                                  const uint4 (&hn)[2], const LaneProfile& lp,
                                                  const kvmi_layer_job& job, int ntok, int tok, int G, int H,
                                                  float s, uint4* ylane, LanePack<16 * NC, BITS>& pkd,
                                                  uint32_t& over) {
  constexpr int HALF = 16 * NC;
  float amn = __builtin_inff(), amx = -__builtin_inff();
  f32x16 a0 = transform_T<NC>(xv, hp, hn, 0);
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 a1 = a0;
    if (cp + 1 < NC) a1 = transform_T<NC>(xv, hp, hn, cp + 1);
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      amn = fminf(fminf(amn, a0[i]), fminf(a0[i + 1], fminf(a0[i + 2], a0[i + 3])));
      amx = fmaxf(fmaxf(amx, a0[i]), fmaxf(a0[i + 1], fmaxf(a0[i + 2], a0[i + 3])));
    }
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) w[i / 2] = pack_bf16x2(a0[i] * s, a0[i + 1] * s);
    ylane[(2 * cp) * 64] = make_uint4(w[0], w[1], w[2], w[3]);
    ylane[(2 * cp + 1) * 64] = make_uint4(w[4], w[5], w[6], w[7]);
    chunk_fence();
    a0 = a1;
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


// Advances the workspace epoch (one thread); the pass reads it at its start.  Tags are
// 32-bit: from 2^31 calls on one workspace on, a tag could come back while keys or flags
// of an earlier call still hold it, so the call is flagged instead.
__global__ void onepass_epoch_kernel(uint32_t* epoch, int32_t* err) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const uint32_t e = *epoch + 1;
    *epoch = e;
    if (e >= 0x80000000u) atomicOr(err, KVMI_ERR_SYNC);
  }
}

template <int NC, int BITS, bool CLAMP>
__global__ __launch_bounds__(kOT) void onepass_kernel(OpArgs a) {
  constexpr int D = 32 * NC, HALF = 16 * NC, U = 2 * NC, PR = 4 * NC;  // PR: 16-byte pieces per row
  constexpr int RPI = 64 / PR;         // rows per coalesced load instruction
  constexpr int RB = D * BITS / 8;     // bytes of one packed row
  constexpr int TQ = kTok * RB / 16;   // uint4 per packed tile
  constexpr int NSET = 8;              // table sets (a power of two: indices are masks)
  static_assert(tile_buf_q<NC>() >= 2 * NC * 64 && tile_buf_q<NC>() * 16 >= kTok * RB, "wave buffer uses");
  const Geo g = a.g;
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int wg = blockIdx.x, grid = a.grid, steps = a.steps;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // H and S are powers of two here (mfma_eligible, onepass_geometry): shifts, not divisions
  const int lgH = __builtin_ctz((unsigned)H), lgS = __builtin_ctz((unsigned)S);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31, hme = r & (H - 1), rtok = r >> lgH;
  const float sc_d = g.scale;
  const bool native = g.flags & KVMI_F_NATIVE_LAYOUT;
  const int tpt = kTok / H;  // tokens per V tile
  const uint32_t epoch = __builtin_amdgcn_readfirstlane(gld(a.epoch));

  // Waves are ordered by LDS flags and counters, not workgroup barriers, so that they
  // can be in different phases and steps.  Every wave starts step s only once every wave
  // has finished step s - 3 (`fin` counts finished steps: 8 per step), so at most three
  // steps are in flight, and each piece of per-step LDS state is buffered deeper than
  // that: table sets by s % 8 (staged two steps ahead by wave s % 8, and read up to the
  // next step), the workgroup keys and their arrival counters by s % 4, the K constants by
  // the step that uses them % 4.  A buffer's flag holds the step (+ 1) it was last
  // filled for, so no flag is ever cleared and every wait is "flag >= value".
  __shared__ StepTables tab[NSET];
  __shared__ uint32_t lkey[4][2 * D];     // the workgroup's min / max keys of a step's K group
  __shared__ float2 kc[4][D + 4];         // (min, -1/scale) per channel of the group quantized in step q
  __shared__ uint4 wbuf[kOW * tile_buf_q<NC>()];
  __shared__ uint32_t tready[NSET];       // step + 1 of the tables in each set
  __shared__ uint32_t karr[4], kfin[4];   // K waves arrived in step s; step + 1 once its keys are final
  __shared__ uint32_t kown[4], kready[4]; // claim and readiness of the constants used in step q
  __shared__ uint32_t fin;

  uint4* wb = wbuf + wave * tile_buf_q<NC>();
  uint8_t* ost = reinterpret_cast<uint8_t*>(wb);
  bool broken = false;  // a device wait of this wave timed out: later ones give up at once

  // ---------------------------------------------------------------- staging
  // Step k's tables into set e, by one wave: its record, the K and V job descriptors,
  // the pool rows every wave will load, sign masks and profile positions.
  auto stage = [&](int k, int e) {
    StepTables& T = tab[e];
    const OpRec rc = load_rec(a.recs, (int64_t)k * grid + wg);
    if (l == 0) T.rec = rc;
    int64_t vr = -1;
    if (rc.vjob >= 0) {
      const kvmi_layer_job jv = load_job(a.jobs, rc.vjob);
      if (l == 0) T.vj = jv;
      constexpr int W = D / 32;  // sign words per head
      const uint32_t sw = l < H * W ? gld(jv.signs + l) : 0u;
      const uint32_t pb = l < 6 * H ? (uint32_t)gld(jv.profile + l) : 0u;
      if (l < kOW && l < rc.vn) {  // lane w: first pool row of wave w's V tile
        const int vt = rc.vtile0 + l;
        if (vt * kTok < jv.num_blocks * S * H) {
          const int ta = vt * tpt;
          vr = ((int64_t)gld(jv.block_ids + (ta >> lgS)) * S + (ta & (S - 1))) * H;
        }
      }
      for (int i = l; i < H * (D / 2); i += 64) {
        const int h = i / (D / 2), q = i % (D / 2);
        const uint32_t sb = (uint32_t)__shfl((int)sw, h * W + (2 * q) / 32) >> ((2 * q) & 31);
        T.smask[h][q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
      }
      if (l < 6 * H) T.prof[l / (3 * H)][(l / H) % 3][l % H] = (uint8_t)pb;
      // lane h < H: output positions of source head h (K, V) and the source head of
      // the first output position of V group h (shuffles outside branches: every lane
      // takes part)
      int pk = 0, pv = 0, gf = -1;
      for (int q = 0; q < H; ++q) {
        const int ok = __shfl((int)pb, q), ov = __shfl((int)pb, 3 * H + q);
        if (ok == l) pk = q;
        if (ov == l) pv = q;
      }
      for (int q = H - 1; q >= 0; --q) {
        const int gq = __shfl((int)pb, 5 * H + q), oq = __shfl((int)pb, 3 * H + q);
        if (gq == l) gf = oq;
      }
      if (l < H) {
        T.posk[l] = pk;
        T.posv[l] = pv;
        T.gfirst[l] = gf;
      }
    }
    if (rc.kjob >= 0) {
      const kvmi_layer_job jk = load_job(a.jobs, rc.kjob);
      const int h = rc.khead & 0xff, kn = rc.khead >> 8, T_ = jk.num_blocks * S;
      if (l == 0) T.kj = jk;
      for (int q = l; q < D / 2; q += 64) {
        const uint32_t sb = gld(jk.signs + h * (D / 32) + (2 * q) / 32) >> ((2 * q) & 31);
        T.kmask[q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
      }
      const int pb = l < 2 * H ? (int)gld(jk.profile + l) : 0;  // K order and levels
      int jk_ = 0;
      for (int q = 0; q < H; ++q)
        if (__shfl(pb, q) == h) jk_ = q;
      const int lv = __shfl(pb, H + jk_);
      if (l == 0) {
        T.kjk = jk_;
        T.kjlv = lv;
      }
      // entry (w, v): row of wave w's load instruction v
      for (int i = l; i < kOW * U; i += 64) {
        const int w = i / U, v = i % U, tt = rc.ktile0 + w;
        int32_t kr = INT32_MIN;
        if (w < kn && 32 * tt < T_) {
          const int tv = 32 * tt + RPI * v;
          const bool past = tv >= T_;
          const int tb = past ? T_ - 1 : tv;
          const int row = (gld(jk.block_ids + (tb >> lgS)) * S + (tb & (S - 1))) * H + h;
          kr = past ? -1 - row : row;
        }
        T.krow[w][v] = kr;
      }
    } else {
      for (int i = l; i < kOW * U; i += 64) T.krow[i / U][i % U] = INT32_MIN;
    }
    if (l < kOW) T.vrow[l] = vr;
    lds_order();
    if (l == 0) __hip_atomic_store(&tready[e], (uint32_t)(k + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  auto wait_tables = [&](int k) {
    if (k < steps && !lds_wait(&tready[k & (NSET - 1)], (uint32_t)(k + 1)) && l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
  };

  // ---------------------------------------------------------------- loads
  // Every wave issues the same loads on every path (idle waves read `dummy`): a load
  // issued on one path only makes the compiler wait for every load in flight where the
  // paths join.  K head-tile t of (job, head): tokens 32t .. 32t + 31, instruction v reads
  // rows RPI v .. RPI v + RPI - 1 (PR lanes per row, 16 bytes each); S is a power of two
  // >= RPI, so the rows of one instruction lie in one block; rows past the job's last
  // token repeat that token (min / max ignore repeats, and the quantization does not
  // write them).
  // (`valid` false: no such step, every load reads `dummy`)
  auto k_fire = [&](const StepTables& T, bool valid, uint4 (&x)[U]) {
    const int32_t* kr = &T.krow[wave][0];
    const int32_t r0 = valid ? uni(kr[0]) : INT32_MIN;
    const uint16_t* base = r0 == INT32_MIN ? a.dummy : reinterpret_cast<const uint16_t*>(uni(T.kj.pool));
    const int lo = (l / PR) * H;
#pragma unroll
    for (int v = 0; v < U; ++v) {
      const int32_t rb = r0 == INT32_MIN ? INT32_MIN : uni(kr[v]);
      const int64_t row = rb == INT32_MIN ? 0 : rb < 0 ? (int64_t)(-1 - rb) : (int64_t)rb + lo;
      x[v] = gld(reinterpret_cast<const uint4*>(base + row * D) + l % PR);
    }
  };
  // V tile: 32 consecutive pool rows (one block), loaded 1 KiB per instruction
  auto v_fire = [&](const StepTables& T, bool valid, uint4 (&x)[U]) {
    const int64_t row0 = valid ? uni(T.vrow[wave]) : (int64_t)-1;
    const uint16_t* base = a.dummy;
    if (row0 >= 0) {
      const kvmi_layer_job* vj = &T.vj;
      base = reinterpret_cast<const uint16_t*>(uni(vj->pool)) + uni(vj->pool_part_stride);
    }
    load_tile<NC>(base, row0 >= 0 ? row0 : 0, x);
  };

  // ---------------------------------------------------------------- K constants
  // The constants of step s's K group (used in step s + 1), by the first wave to finish
  // step s: once the group's keys are final (this workgroup's arrivals, or every
  // workgroup's flag), per-channel (min, -1/scale) into kc[(s + 1) % 4] and the K metadata
  // (the group's first workgroup).
  auto claim = [&](int s, const OpRec& rc, const StepTables& T) {
    const int q = s + 1, e = q & 3, pk3 = s & 3;
    uint32_t old = 0;
    if (l == 0) old = __hip_atomic_fetch_max(&kown[e], (uint32_t)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old >= (uint32_t)q) return;  // another wave has it
    const int gw0 = rc.kgroup & 0xffff, gws = rc.kgroup >> 16;
    if (gws > 1) {
      const uint32_t* fl = a.flags + (int64_t)s * grid + gw0;
      bool done = false;
      for (uint32_t polls = 0; !broken && polls < kMaxPolls; ++polls) {
        bool ok = true;
        for (int w = l; w < gws; w += 64)
          ok &= __hip_atomic_load(fl + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
        if (__all(ok)) {
          done = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!done) {
        broken = true;
        if (l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
      }
    } else if (!lds_wait(&kfin[pk3], (uint32_t)(s + 1)) && l == 0) {  // this workgroup's keys are final
      atomicOr(a.err, KVMI_ERR_SYNC);
    }
    const int jk = uni(T.kjk), lv = uni(T.kjlv);
    uint16_t* kmeta = uni(T.kj.kmeta);
    const int T_ = uni(T.kj.num_blocks) * S;
    const unsigned long long* kk = a.keys + (int64_t)rc.kslot * 2 * D;
    bool stale = false;
    for (int c = l; c < D; c += 64) {
      uint32_t kmn, kmx;
      if (gws > 1) {
        const unsigned long long vmn = __hip_atomic_load(kk + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long vmx = __hip_atomic_load(kk + D + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stale |= (uint32_t)(vmn >> 32) != epoch || (uint32_t)(vmx >> 32) != epoch;
        kmn = ~(uint32_t)vmn;
        kmx = (uint32_t)vmx;
      } else {
        kmn = lkey[pk3][c];
        kmx = lkey[pk3][D + c];
        lkey[pk3][c] = 0xffffffffu;
        lkey[pk3][D + c] = 0u;
      }
      const float mn = round_bf16(key2f(kmn) * sc_d);  // keys are unscaled
      const float mx = round_bf16(key2f(kmx) * sc_d);
      const float scl = quant_scale(mn, mx, lv);
      kc[e][c] = make_float2(mn, -1.0f / scl);
      if (rc.ktile0 == 0 && T_ > 0) {  // the group's first workgroup writes the K metadata
        gst(kmeta + jk * D + c, (uint16_t)f32_to_bf16_bits(mn));
        gst(kmeta + HD + jk * D + c, (uint16_t)f32_to_bf16_bits(scl));
      }
    }
    if (stale && !broken) atomicOr(a.err, KVMI_ERR_SYNC);
    lds_order();
    if (l == 0) __hip_atomic_store(&kready[e], (uint32_t)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };

  // ---------------------------------------------------------------- set-up
  // The Sylvester matrix is symmetric, so the orientation-T operand tiles serve the
  // statistics (orientation N) too: column n of the product is then channel
  // HALF n2 + 16 c + 8 n4 + 4 n3 + 2 n1 + n0 instead of the T layout's row.
  uint4 hpT[2], hnT[2];
  hpT[0] = hadamard_tile(0, false, false);
  hpT[1] = hadamard_tile(1, false, false);
  hnT[0] = hadamard_tile(0, false, true);
  hnT[1] = hadamard_tile(1, false, true);
  uint32_t over = 0;

  for (int i = threadIdx.x; i < 2 * D; i += kOT) {
    const uint32_t init = i < D ? 0xffffffffu : 0u;
    lkey[0][i] = init;
    lkey[1][i] = init;
    lkey[2][i] = init;
    lkey[3][i] = init;
  }
  if (threadIdx.x < NSET) tready[threadIdx.x] = 0;
  if (threadIdx.x < 4) karr[threadIdx.x] = kfin[threadIdx.x] = 0;
  if (threadIdx.x < 4) kown[threadIdx.x] = kready[threadIdx.x] = 0;
  if (threadIdx.x == 0) fin = 0;
  // a job with more blocks than the schedule holds would be compressed in part: flagged
  for (int j = wg * kOT + (int)threadIdx.x; j < a.num_jobs; j += grid * kOT)
    if (gld(&a.jobs[j].num_blocks) > gld(a.sched_blocks + j)) atomicOr(a.err, KVMI_ERR_SCHEDULE);
  // chunks of jobs without blocks still get their header (the stream of N = 0 symbols)
  if (wg == 0 && !(g.flags & KVMI_F_NO_HEADER)) {
    for (int j = threadIdx.x; j < a.num_jobs; j += kOT) {
      const kvmi_layer_job* q = a.jobs + j;
      if (gld(&q->num_blocks) == 0 && gld(&q->write_header))
        write_stream_header(gld(&q->stream), BITS, gld(&q->chunk_symbols));
    }
  }
  __syncthreads();
  if (wave < 2 && wave < steps) stage(wave, wave);  // steps 0 and 1

  uint4 kb0[U], kb1[U], vb[U];
  wait_tables(0);
  k_fire(tab[0], steps > 0, kb0);
  v_fire(tab[0], steps > 0, vb);

  // ---------------------------------------------------------------- one step
  auto step = [&](int s, uint4 (&cur)[U], uint4 (&prev)[U]) {
    const int p3 = s & 3;
    if (s >= 3 && !lds_wait(&fin, (uint32_t)(kOW * (s - 2))) && l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
    if (s + 2 < steps && wave == s % kOW) stage(s + 2, (s + 2) & (NSET - 1));  // set last used in step s - 6
    wait_tables(s);
    const StepTables& T = tab[s & (NSET - 1)];
    const StepTables& TP = tab[(s - 1) & (NSET - 1)];
    const OpRec rc = s < steps ? uni(T.rec) : no_rec();
    const OpRec rp = s > 0 ? uni(TP.rec) : no_rec();

    // ------------------------------------------------ P1: K statistics of step s
    const int kn = rc.kjob >= 0 ? (rc.khead >> 8) : 0;
    if (wave < kn) {
      const int T_ = uni(T.kj.num_blocks) * S;
      if (32 * (rc.ktile0 + wave) < T_) {
        tile_to_half_rows<NC>(wb, cur);
        const uint4* sm = reinterpret_cast<const uint4*>(&T.kmask[0] + opaque((HALF / 2) * hl));
#pragma unroll
        for (int u = 0; u < U; ++u) cur[u] = xor4(cur[u], sm[u]);
        kstats_head_tile<NC>(cur, hpT, hnT, &lkey[p3][0]);
      }
      if (wave == 0 && rc.ktile0 == 0 && (rc.khead & 0xff) == 0 && !(g.flags & KVMI_F_NO_HEADER)) {
        const kvmi_layer_job jb = uni(T.kj);
        if (jb.write_header && l == 0) write_stream_header(jb.stream, BITS, jb.chunk_symbols);
      }
      // arrival: the last of the workgroup's K waves publishes its keys
      lds_order();
      uint32_t v = 0;
      if (l == 0) v = __hip_atomic_fetch_add(&karr[p3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      v = __builtin_amdgcn_readfirstlane(v);
      if (v == (uint32_t)(kn - 1)) {
        if (l == 0) karr[p3] = 0;
        if ((rc.kgroup >> 16) > 1) {
          unsigned long long* kk = a.keys + (int64_t)rc.kslot * 2 * D;
          const unsigned long long tag = (unsigned long long)epoch << 32;
          for (int e = l; e < 2 * D; e += 64) {
            const uint32_t k = lkey[p3][e];
            atomicMax(kk + e, tag | (unsigned long long)(e < D ? ~k : k));
            lkey[p3][e] = e < D ? 0xffffffffu : 0u;
          }
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the key pushes are performed
          if (l == 0)
            __hip_atomic_store(a.flags + (int64_t)s * grid + wg, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // a group of one workgroup keeps its final keys in lkey[p3] for the claim
        lds_order();
        if (l == 0) __hip_atomic_store(&kfin[p3], (uint32_t)(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }

    // ------------------------------------------------ P3: K quantization of step s - 1
    const int knp = rp.kjob >= 0 ? (rp.khead >> 8) : 0;
    if (wave < knp) {
      const int e = s & 3;
      if (!lds_wait(&kready[e], (uint32_t)s) && l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
      const kvmi_layer_job jb = uni(TP.kj);
      const int T_ = jb.num_blocks * S, tt = rp.ktile0 + wave;
      if (32 * tt < T_) {
        const int jk = uni(TP.kjk);
        const float lvk = (float)uni(TP.kjlv);
        LanePack<HALF, BITS> pkd;
        quant_k_tile_pipe<NC, BITS, CLAMP>(prev, hpT, hnT, &kc[e][0] + opaque(HALF * hl), sc_d, lvk, pkd, over);
        pkd.store_lds(ost + r * RB + hl * (RB / 2));
        // rows 0 .. nv - 1 of the head-tile exist (nv a multiple of S, or 32)
        const int nv = min(32, T_ - 32 * tt), t0 = 32 * tt;
        if (!native) {  // one run of nv rows of the head's stream
          uint4* dst = reinterpret_cast<uint4*>(seg_addr<BITS>(jb, g, 0, jk, t0, 0));
          const int nq = nv * RB / 16;
          for (int q = l; q < nq; q += 64) gst(dst + q, wb[q]);
        } else {  // row (token, position jk) at stride H * RB: 8-byte pieces
          constexpr int P8 = RB / 8;
          const uint2* src = reinterpret_cast<const uint2*>(ost);
          for (int q = l; q < nv * P8; q += 64) {
            const int row = q / P8, pc = q % P8;
            gst(reinterpret_cast<uint2*>(seg_addr<BITS>(jb, g, 0, jk, t0 + row, 0)) + pc, src[q]);
          }
        }
      }
    }
    // next step's K tile, into the registers of the tile just quantized
    wait_tables(s + 1);
    const StepTables& TN = tab[(s + 1) & (NSET - 1)];
    k_fire(TN, s + 1 < steps, prev);

    // ------------------------------------------------ P2: V encode of step s
    if (rc.vjob >= 0 && wave < rc.vn) {
      const int64_t row0 = uni(T.vrow[wave]);
      if (row0 >= 0) {
        const kvmi_layer_job jv = uni(T.vj);
        const int ntok = jv.num_blocks * S, ta = (rc.vtile0 + wave) * tpt;
        tile_to_half_rows<NC>(wb, vb);
        sign_half_row<NC>(T, hme, hl, vb);
        const LaneProfile lp = lane_profile(T, hme, hl);
        LanePack<HALF, BITS> pkd;
        quant_v_tile_pipe<NC, BITS, CLAMP>(vb, hpT, hnT, lp, jv, ntok, ta + rtok, G, H, sc_d, wb + l, pkd, over);
        const int off = native ? rtok * (H * RB) + lp.jv * RB + hl * (RB / 2)
                               : ((lp.jv * kTok * RB) >> lgH) + rtok * RB + hl * (RB / 2);
        pkd.store_lds(ost + off);
        // staged image: one run of the tile's tokens per output position (permuted,
        // 32 RB / H bytes each, run j at stream offset j * ntok * RB) or the tile's rows
        // in order (native); 16-byte pieces, lane-linear
        uint8_t* vbase = seg_addr<BITS>(jv, g, 1, 0, ta, 0);
        const int64_t jstride = (int64_t)ntok * RB;
#pragma unroll
        for (int u = 0; u < (TQ + 63) / 64; ++u) {
          const int q = 64 * u + l;
          if (TQ % 64 == 0 || q < TQ) {
            int64_t o = 16 * q;
            if (!native) {
              const int run_j = (q << (lgH + 4)) / (kTok * RB);  // byte 16 q of runs of 32 RB / H bytes
              o += run_j * (jstride - ((kTok * RB) >> lgH));
            }
            gst(reinterpret_cast<uint4*>(vbase + o), wb[q]);
          }
        }
      }
    }
    v_fire(TN, s + 1 < steps, vb);
    if (rc.kjob >= 0) claim(s, rc, T);
    lds_signal(&fin);
  };

  for (int s0 = 0; s0 <= steps; s0 += 2) {
    step(s0, kb0, kb1);
    if (s0 + 1 > steps) break;
    step(s0 + 1, kb1, kb0);
  }
  if (over & overflow_mask<BITS>()) atomicOr(a.err, KVMI_ERR_SYMBOL_RANGE);
}

// ------------------------------------------------------------------ host side
constexpr int kMaxDev = 64;

struct DeviceInfo {
  int cus = 0;
  bool coop = false;
};
DeviceInfo device_info() {
  static std::atomic<int> cus[kMaxDev], coop[kMaxDev];
  DeviceInfo d;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return d;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int v = 0, cp = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) v = -1;
    if (hipDeviceGetAttribute(&cp, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) cp = 0;
    coop[dev].store(cp ? 1 : -1, std::memory_order_relaxed);
    cus[dev].store(v > 0 ? v : -1, std::memory_order_relaxed);
    c = v > 0 ? v : -1;
  }
  d.cus = c > 0 ? c : 0;
  d.coop = coop[dev].load(std::memory_order_relaxed) > 0;
  return d;
}

template <class K>
int per_cu(K kernel) {
  int per = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel), kOT, 0) != hipSuccess)
    return 0;
  return per;
}

// The kernel instance of a geometry, as a function pointer (nullptr: none).
using OpKernel = void (*)(OpArgs);
template <int NC, int BITS>
OpKernel pick_bits(bool clamp) {
  return clamp ? onepass_kernel<NC, BITS, true> : onepass_kernel<NC, BITS, false>;
}
template <int NC>
OpKernel pick_nc(int bits, bool clamp) {
  switch (bits) {
    case 1: return pick_bits<NC, 1>(clamp);
    case 2: return pick_bits<NC, 2>(clamp);
    case 3: return pick_bits<NC, 3>(clamp);
    case 4: return pick_bits<NC, 4>(clamp);
    case 5: return pick_bits<NC, 5>(clamp);
    case 6: return pick_bits<NC, 6>(clamp);
    case 7: return pick_bits<NC, 7>(clamp);
    default: return pick_bits<NC, 8>(clamp);
  }
}
OpKernel pick(const Geo& g) {
  const bool clamp = g.flags & KVMI_F_CLAMP_LEVELS;
  return g.D == 64 ? pick_nc<2>(g.bits, clamp) : pick_nc<4>(g.bits, clamp);
}

// Geometries the one-pass kernel serves: the MFMA token-major tiles (H dividing 8),
// head-tiles whose load instructions stay inside one block (S a power of two, at least
// the rows of one instruction), and whole-byte rows in 8-byte pieces (native layout).
bool onepass_geometry(const Geo& g) {
  if (!mfma_eligible(g) || g.H > kMH || (g.flags & KVMI_F_TWO_PASS)) return false;
  if ((g.S & (g.S - 1)) != 0 || g.S < 64 / (g.D / 8)) return false;
  return ((g.D * g.bits / 8) % 8) == 0;
}

}  // namespace
}  // namespace kvmi

extern "C" int64_t kvmi_compress_schedule(const kvmi_geometry* geom, const int32_t* num_blocks, int32_t num_jobs,
                                          void* image, int64_t image_bytes) {
  using namespace kvmi;
  Geo g;
  const int rc = check_geo(geom, num_jobs, 0, &g);
  if (rc) return rc;
  if (num_jobs > 0 && !num_blocks) return KVMI_EINVAL;
  if (image_bytes < 0) return KVMI_EINVAL;
  if (!onepass_geometry(g)) return 0;
  const DeviceInfo d = device_info();
  if (!d.coop || d.cus == 0) return 0;
  const int per = per_cu(pick(g));
  if (per < 1) return 0;
  const int grid = d.cus * per;
  if (grid > 0xffff) return 0;
  const int S = g.S, H = g.H;
  // K groups (job, head), packed into steps without splitting a group
  std::vector<OpRec> recs;
  OpRec none{};
  none.kjob = none.vjob = none.kslot = -1;
  int steps = 0, cur = grid, nslots = 0;
  for (int j = 0; j < num_jobs; ++j) {
    if (num_blocks[j] < 0) return KVMI_EINVAL;
    const int64_t T = (int64_t)num_blocks[j] * S;
    if (T == 0) continue;
    const int64_t nkt = (T + 31) / 32, nwg = (nkt + kTPW - 1) / kTPW;
    if (nwg > grid) return 0;  // this job's K of one head exceeds the grid
    for (int h = 0; h < H; ++h) {
      if (cur + nwg > grid) {
        recs.resize((size_t)(steps + 1) * grid, none);
        ++steps;
        cur = 0;
      }
      const int slot = nwg > 1 ? nslots++ : -1;
      for (int k = 0; k < nwg; ++k) {
        OpRec& r = recs[(size_t)(steps - 1) * grid + cur + k];
        r.kjob = j;
        r.khead = h | (int)std::min<int64_t>(kTPW, nkt - (int64_t)kTPW * k) << 8;
        r.ktile0 = kTPW * k;
        r.kgroup = cur | (int)nwg << 16;
        r.kslot = slot;
      }
      cur += (int)nwg;
    }
  }
  // V groups of 8 token-major tiles, spread evenly over the steps from the last
  // workgroup down (the K groups fill each step from the first up)
  int64_t nvg = 0;
  for (int j = 0; j < num_jobs; ++j) nvg += ((int64_t)num_blocks[j] * S * H / kTok + kTPW - 1) / kTPW;
  const int64_t need = (nvg + grid - 1) / grid;
  if (need > steps) {
    recs.resize((size_t)need * grid, none);
    steps = (int)need;
  }
  int64_t k = 0;
  for (int j = 0; j < num_jobs; ++j) {
    const int64_t nvt = (int64_t)num_blocks[j] * S * H / kTok;
    for (int64_t t0 = 0; t0 < nvt; t0 += kTPW, ++k) {
      const int s = (int)(k * steps / nvg);
      const int64_t first = (s * nvg + steps - 1) / steps;  // first V group of step s
      OpRec& r = recs[(size_t)s * grid + (grid - 1 - (int)(k - first))];
      r.vjob = j;
      r.vtile0 = (int)t0;
      r.vn = (int)std::min<int64_t>(kTPW, nvt - t0);
    }
  }
  OpHeader h{};
  h.magic = kOpMagic;
  h.grid = grid;
  h.steps = steps;
  h.num_jobs = num_jobs;
  h.S = S;
  h.H = H;
  h.D = g.D;
  h.bits = g.bits;
  h.flags = g.flags;
  h.nslots = nslots;
  h.rec_off = kHeaderBytes;
  h.blk_off = h.rec_off + (int64_t)recs.size() * (int64_t)sizeof(OpRec);
  h.image_bytes = h.blk_off + 4 * (int64_t)num_jobs;
  h.flag_off = round256(h.image_bytes);
  h.key_off = round256(h.flag_off + (int64_t)steps * grid * 4);
  h.epoch_off = round256(h.key_off + (int64_t)nslots * 2 * g.D * 8);
  h.total = std::max<int64_t>(h.epoch_off + 256, kMinWorkspace);
  if (image) {
    if (image_bytes < h.image_bytes) return KVMI_EINVAL;
    std::memset(image, 0, (size_t)kHeaderBytes);
    std::memcpy(image, &h, sizeof h);
    if (!recs.empty()) std::memcpy(static_cast<uint8_t*>(image) + h.rec_off, recs.data(), recs.size() * sizeof(OpRec));
    if (num_jobs > 0) std::memcpy(static_cast<uint8_t*>(image) + h.blk_off, num_blocks, 4 * (size_t)num_jobs);
  }
  return h.image_bytes;
}

extern "C" int64_t kvmi_compress_workspace_bytes(const void* schedule) {
  using namespace kvmi;
  if (!schedule) return KVMI_EINVAL;
  OpHeader h;
  std::memcpy(&h, schedule, sizeof h);
  if (h.magic != kOpMagic) return KVMI_EINVAL;
  return h.total;
}

extern "C" int kvmi_kstats_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream);
extern "C" int kvmi_encode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream);

extern "C" int kvmi_compress_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                   int32_t max_blocks, const void* schedule, void* workspace, int32_t* err,
                                   kvmi_stream_t stream) {
  using namespace kvmi;
  Geo g;
  int rc = check_geo(geom, num_jobs, max_blocks, &g);
  if (rc) return rc;
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (schedule && workspace && !(g.flags & KVMI_F_TWO_PASS)) {
    OpHeader h;
    std::memcpy(&h, schedule, sizeof h);
    if (h.magic != kOpMagic || h.num_jobs != num_jobs || h.S != g.S || h.H != g.H || h.D != g.D ||
        h.bits != g.bits || h.flags != g.flags || ((uintptr_t)workspace & 255))
      return KVMI_EINVAL;
    if (h.steps > 0 && onepass_geometry(g)) {
      const DeviceInfo d = device_info();
      OpKernel kernel = pick(g);
      if (!d.coop || h.grid > d.cus * per_cu(kernel)) return KVMI_EINVAL;  // built for another device
      uint8_t* ws = static_cast<uint8_t*>(workspace);
      OpArgs a{};
      a.g = g;
      a.jobs = jobs;
      a.err = err;
      a.recs = reinterpret_cast<const OpRec*>(ws + h.rec_off);
      a.flags = reinterpret_cast<uint32_t*>(ws + h.flag_off);
      a.keys = reinterpret_cast<unsigned long long*>(ws + h.key_off);
      a.epoch = reinterpret_cast<const uint32_t*>(ws + h.epoch_off);
      a.dummy = reinterpret_cast<const uint16_t*>(ws);
      a.sched_blocks = reinterpret_cast<const int32_t*>(ws + h.blk_off);
      a.steps = h.steps;
      a.grid = h.grid;
      a.num_jobs = num_jobs;
      hipLaunchKernelGGL(onepass_epoch_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<uint32_t*>(ws + h.epoch_off),
                         err);
      if (hipGetLastError() != hipSuccess) return KVMI_ELAUNCH;
      void* args[] = {&a};
#ifdef KVMI_ORDINARY_LAUNCH
      // profiling build (python -m kvserve_amd.build --ordinary-launch): the same grid of
      // resident workgroups as an ordinary launch, which rocprofv3 can follow; every wait
      // of the kernel is bounded, so a workgroup that would not be resident ends in
      // KVMI_ERR_SYNC, never in a hang
      const hipError_t e =
          hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3((unsigned)h.grid), dim3(kOT), args, 0, st);
#else
      const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3((unsigned)h.grid),
                                                      dim3(kOT), args, 0, st);
#endif
      return e == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
    }
  }
  rc = kvmi_kstats_paged(geom, jobs, num_jobs, max_blocks, err, stream);
  if (rc) return rc;
  return kvmi_encode_paged(geom, jobs, num_jobs, max_blocks, err, stream);
}
