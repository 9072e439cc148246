// One-pass paged compress on gfx950: every K and V value of a (request, layer) job is
// read from HBM once.
//
// K is quantized with per-channel statistics over all tokens of the job
// (quantizer_func.py:41-56, axis "channel"), so no K symbol can be written before the
// whole job's K has been seen.  The two-pass path (kvmi_mfma.hip) reads K twice; here a
// cooperative, persistent grid keeps each workgroup's share of a job's K in LDS from
// the statistics to the quantization.
//
//   * The grid (one workgroup per CU) is split into groups of `gsize` workgroups; job j
//     belongs to group j % ngroups, and a group runs its jobs in order.  Workgroup
//     `rank` of a group owns tiles [rank*CAP, (rank+1)*CAP) of every job (CAP tiles are
//     64 KiB of bf16 K); a tile is the 32 pool rows of the MFMA kernels.
//   * A workgroup runs three kinds of waves, the stages of a pipeline over its jobs:
//       S-waves  load a job's K tiles into registers, flip their signs, take the
//                per-channel min / max (MFMA, orientation N), push the workgroup's keys
//                to the job's device keys and arrive at the job's barrier; then, once
//                slot i % 2 is handed back (i: the job's place in the group's order),
//                store the tiles there, issue the next job's loads and stage its
//                tables (sign masks, profile) into a ring of kRing.
//       Q-waves  wait for job i's barrier, turn its device keys into per-channel
//                constants, quantize the K tiles out of slot i % 2 (MFMA, orientation
//                T) and hand the slot back.
//       V-waves  encode V: per-token statistics need no other workgroup.
//     With a job in registers and two in the slots, the S-waves arrive at a job's
//     barrier up to three jobs before the Q-waves need it, so its latency is hidden
//     behind the quantization of the jobs before, and the V-waves keep HBM busy
//     throughout.  The S-waves wait only for a free slot, the Q-waves for the barrier,
//     the V-waves for tables.
//   * Keys and barrier flags need no clearing between calls: a key is a 64-bit
//     (epoch << 32 | order-preserving key) maximum, and a workgroup arrives at a job's
//     barrier by storing the call's epoch into its own flag of the job; the barrier is
//     crossed when every flag of the group holds the epoch (the host advances it).
//   * Every wait is bounded: on timeout the kernel sets KVMI_ERR_SYNC, later device
//     waits give up at once, and every wave reaches the end of the kernel.
#include "kvmi_mfma_tiles.hpp"

namespace kvmi {
namespace {

constexpr int kSW = 4;                  // S-waves per workgroup
constexpr int kQW = 4;                  // Q-waves per workgroup
constexpr int kSlotBytes = 64 * 1024;   // a workgroup's share of one job's K
constexpr int kRing = 3;                // job table sets in LDS
constexpr int kLdsBytes = 160 * 1024;   // LDS of a CU
constexpr int kCounterWords = 256;      // per job: one arrival flag per workgroup of its group
constexpr int kPrioS = 0, kPrioQ = 0, kPrioV = 0;  // wave priorities (s_setprio) of the three kinds
constexpr uint32_t kMaxPolls = 1u << 18;  // ~0.3 s of polling before KVMI_ERR_SYNC

// K tiles per workgroup per job at D = 32 NC (a tile: 32 rows of D bf16).
template <int NC>
constexpr int cap_tiles() {
  return kSlotBytes / (kTok * 64 * NC);
}

// One job's tables, staged by the S-waves and read by every kind of wave.
struct JobTables {
  uint32_t smask[kMH][64 + 4];  // sign-flip masks per (head, element pair), padded rows
  uint8_t prof[2][3][kMH];      // [part][order, levels, group][position]
  int8_t posk[kMH], posv[kMH], gfirst[kMH];
};

// LDS bytes of the kernel with `vw` V-waves: two slots, the V-waves' packed-tile
// stages, the workgroup keys, the K constants, the table ring and the counters.
template <int NC, int BITS>
constexpr int lds_bytes(int vw) {
  return 2 * kSlotBytes + vw * kTok * (32 * NC * BITS / 8) + 2 * kMH * 32 * NC * 4 + kMH * (32 * NC + 4) * 8 +
         kRing * (int)sizeof(JobTables) + 64;
}
// V-waves per workgroup: four where the LDS allows, else two (wide symbols at
// D = 128), else none (no one-pass kernel for that width).
template <int NC, int BITS>
constexpr int v_waves() {
  return lds_bytes<NC, BITS>(4) <= kLdsBytes ? 4 : lds_bytes<NC, BITS>(2) <= kLdsBytes ? 2 : 0;
}

struct PassArgs {
  Geo g;
  const kvmi_layer_job* jobs;
  int32_t* err;
  uint32_t* counters;                  // [num_jobs][kCounterWords]
  unsigned long long* keys;            // [num_jobs][2][H][D]: max of (epoch << 32 | key)
  int num_jobs, gsize, ngroups;
  uint32_t epoch;
};

// A job descriptor through the constant address space: scalar loads into SGPRs (the
// descriptor array is read-only for the whole launch), instead of vector loads, which
// the compiler would otherwise use for data read after the kernel's first stores.
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

// Barrier among the `n` waves of one kind: a monotone LDS counter, one arrival per
// wave; `gen` counts the barriers this wave has passed (the same on all n waves).
__device__ __forceinline__ void kind_sync(uint32_t* ctr, uint32_t& gen, int n, int32_t* err) {
  gen += 1;
  lds_signal(ctr);
  if (!lds_wait(ctr, gen * (uint32_t)n) && (threadIdx.x & 63) == 0) atomicOr(err, KVMI_ERR_SYNC);
}

// Sign flips of a lane's half-row (as sign_half_row) in two halves, with a scheduling
// barrier between them, so that at most half of the mask registers are live at once.
template <int NC>
__device__ __forceinline__ void sign_half_row_lean(const uint32_t (*smask)[64 + 4], int h, int hl,
                                                   uint4 (&x)[2 * NC]) {
  constexpr int HALF = 16 * NC;
  const uint4* sm = reinterpret_cast<const uint4*>(&smask[0][0] + opaque(h * (64 + 4) + (HALF / 2) * hl));
#pragma unroll
  for (int u = 0; u < NC; ++u) x[u] = xor4(x[u], sm[u]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = NC; u < 2 * NC; ++u) x[u] = xor4(x[u], sm[u]);
}

// K statistics of one signed tile (orientation N, see kstats_tile) pushed straight
// into the workgroup's LDS keys [2][H][D], unscaled: the device keys are scaled by
// 1/sqrt(D) when they are finalised, the same fp32 product as scaling before the
// reduction (a positive factor commutes with min / max).  off[a]: LDS index of (head
// of output registers a, a+4, a+8, a+12; channel (16 NC)(r >> 4) + (r & 15)).
template <int NC>
__device__ __forceinline__ void kstats_tile_keys(const uint4 (&x)[2 * NC], const uint4 (&hp)[2], const uint4 (&hn)[2],
                                                 uint32_t* lkey, const int (&off)[4], int HD) {
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) {
    f32x16 acc = {};
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c = cp ^ k;
      const bool neg = __builtin_popcount(c & cp) & 1;
      acc = mfma(x[2 * c], neg ? hn[0] : hp[0], acc);
      acc = mfma(x[2 * c + 1], neg ? hn[1] : hp[1], acc);
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float mn = fminf(fminf(acc[a], acc[a + 4]), fminf(acc[a + 8], acc[a + 12]));
      const float mx = fmaxf(fmaxf(acc[a], acc[a + 4]), fmaxf(acc[a + 8], acc[a + 12]));
      atomicMin(&lkey[off[a] + 16 * cp], f2key(mn));
      atomicMax(&lkey[HD + off[a] + 16 * cp], f2key(mx));
    }
    chunk_fence();
  }
}

template <int NC, int BITS, bool CLAMP, int VW>
__global__ __launch_bounds__(64 * (kSW + kQW + VW)) void compress_pass_kernel(PassArgs a) {
  constexpr int D = 32 * NC, HALF = 16 * NC, U = 2 * NC;  // U: uint4 of a lane's half-row
  constexpr int CAP = cap_tiles<NC>();
  constexpr int NTS = CAP / kSW, NTQ = CAP / kQW, NTV = CAP / VW;  // tiles per wave per job
  constexpr int RB = D * BITS / 8;    // bytes of one packed row
  constexpr int TQ = kTok * RB / 16;  // uint4 per packed tile
  static_assert(NTS % 2 == 0 && NTV % 2 == 0 && NTQ >= 1, "S- and V-waves alternate two load buffers");
  static_assert(TQ <= U * 64, "a packed tile fits in the slot tile it was quantized from");
  const Geo g = a.g;
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int grp = blockIdx.x / a.gsize, rank = blockIdx.x % a.gsize;
  if (grp >= a.ngroups) return;  // not part of any group (no barrier counts on it)
  const int nj = grp < a.num_jobs ? (a.num_jobs - 1 - grp) / a.ngroups + 1 : 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float s = g.scale;
  const bool native = g.flags & KVMI_F_NATIVE_LAYOUT;
  const int tpt = kTok / H;  // tokens per tile

  __shared__ uint4 slot[2][CAP][U][64];  // signed K tiles, operand-major: [.][.][u][lane]
  __shared__ uint4 vstage[VW][TQ];        // per V-wave: a packed tile on its way out
  __shared__ uint32_t lkey[2 * kMH * D];  // the workgroup's min / max keys of a job
  __shared__ float2 kc[kMH][D + 4];       // per-channel (min, 1/scale) by source head
  __shared__ JobTables ring[kRing];       // tables of job i in ring[i % kRing]
  __shared__ uint32_t sctr, qctr;         // S-wave and Q-wave barriers
  // staged: 1 + S-wave jobs done (job i in its slot, job i + 1's tables staged);
  // vdone / qdone: V- / Q-wave jobs done, one count per wave
  __shared__ uint32_t staged, vdone, qdone;

  auto job_index = [&](int i) { return grp + i * a.ngroups; };
  auto job_tiles = [&](const kvmi_layer_job& job) { return job.num_blocks * S * H / kTok; };
  // byte offset of lane (r, hl)'s half-row in a staged packed tile, by output position
  auto stage_off = [&](int j, int r, int hl) {
    return native ? (r / H) * (H * RB) + j * RB + hl * (RB / 2) : j * (tpt * RB) + (r / H) * RB + hl * (RB / 2);
  };
  // write a staged packed tile (part, first token ta) of `job` to its stream
  auto flush = [&](const uint4* st, const kvmi_layer_job& job, int part, int ta, int l) {
    const int rq = native ? TQ : tpt * RB / 16;  // uint4 per run
#pragma unroll
    for (int u = 0; u < (TQ + 63) / 64; ++u) {
      const int q = 64 * u + l;
      if (TQ % 64 == 0 || q < TQ) {
        const int run_j = q / rq;
        uint8_t* dst = seg_addr<BITS>(job, g, part, native ? 0 : run_j, ta, 0) + 16 * (q - run_j * rq);
        gst(reinterpret_cast<uint4*>(dst), st[q]);
      }
    }
  };
  // Tables of `job` into ring[e] by the S-waves (t: S-thread id); the chunk header.
  auto stage_tables = [&](const kvmi_layer_job& job, int e, int t) {
    JobTables& tb = ring[e];
    for (int i = t; i < H * (D / 2); i += 64 * kSW) {
      const int h = i / (D / 2), q = i % (D / 2);
      const uint32_t sb = gld(job.signs + h * (D / 32) + (2 * q) / 32) >> ((2 * q) & 31);
      tb.smask[h][q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
    }
    if (t < 6 * H) {
      const int part = t / (3 * H), f = (t / H) % 3, k = t % H;
      tb.prof[part][f][k] = gld(job.profile + t);
    }
    if (t < H) {
      int pk = 0, pv = 0, gf = -1;
      for (int k = 0; k < H; ++k) {
        if (gld(job.profile + k) == t) pk = k;
        if (gld(job.profile + 3 * H + k) == t) pv = k;
      }
      for (int k = H - 1; k >= 0; --k)  // first output position of V group t
        if (gld(job.profile + 5 * H + k) == t) gf = gld(job.profile + 3 * H + k);
      tb.posk[t] = (int8_t)pk;
      tb.posv[t] = (int8_t)pv;
      tb.gfirst[t] = (int8_t)gf;
    }
    if (t == 0 && rank == 0 && job.write_header && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
  };
  // A position without a tile re-reads the last tile its wave loaded (at first: the
  // workspace), so that every position issues the same loads: a load issued on one
  // path only makes the compiler wait for every load in flight where paths join.
  const uint16_t* const fallback = reinterpret_cast<const uint16_t*>(a.keys);

  if (threadIdx.x == 0) {
    sctr = qctr = vdone = qdone = 0;
    staged = 1;  // job 0's tables are staged right below
  }
  for (int e = threadIdx.x; e < HD; e += (int)blockDim.x) {
    lkey[e] = 0xffffffffu;
    lkey[HD + e] = 0u;
  }
  if (threadIdx.x < 64 * kSW && nj > 0) stage_tables(load_job(a.jobs, job_index(0)), 0, threadIdx.x);
  __syncthreads();  // the only barrier of all waves

  if (wave < kSW) {
    // ================================================================ S-waves
    // Job i: statistics of its K tiles (held in registers since job i - 1), key push
    // and arrival; then, once the Q-waves are done with job i - 2, the tiles go into
    // slot i % 2, the loads of job i + 1 are issued and its tables staged.  The arrival
    // waits for no other kind of wave.
    if (kPrioS) __builtin_amdgcn_s_setprio(kPrioS);
    const int t = threadIdx.x, l = t & 63, hl = l >> 5, r = l & 31, hme = r % H;
    uint32_t gen = 0;
    uint4 hp[2], hn[2];
    hp[0] = hadamard_tile(0, true, false);
    hp[1] = hadamard_tile(1, true, false);
    hn[0] = hadamard_tile(0, true, true);
    hn[1] = hadamard_tile(1, true, true);
    const uint16_t* lpool = fallback;
    int64_t lrow = 0;
    uint4 xs[NTS][U];  // the job in hand: position n = tile wave + kSW * n of the workgroup's range
    auto issue = [&](int i, int n) {
      if (i < nj) {
        const kvmi_layer_job jb = load_job(a.jobs, job_index(i));
        const int tt = rank * CAP + wave + kSW * n;
        if (tt < job_tiles(jb)) {
          lpool = reinterpret_cast<const uint16_t*>(jb.pool);
          lrow = tile_row0(jb, S, H, tt * tpt) + r;
        }
      }
      load_half_row<NC>(lpool, lrow, hl, xs[n]);
    };
    // LDS key index of (head of output registers a, channel (16 NC)(r >> 4) + (r & 15))
    int koff[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) koff[q] = ((4 * hl + q) % H) * D + (16 * NC) * (r >> 4) + (r & 15);
#pragma unroll
    for (int n = 0; n < NTS; ++n) issue(0, n);
    for (int i = 0; i < nj; ++i) {
      const int ji = job_index(i);
      const int T = job_tiles(load_job(a.jobs, ji)), p = i & 1, e = i % kRing;
      // statistics of the job's tiles into the LDS keys (signs flipped in place)
#pragma unroll
      for (int n = 0; n < NTS; ++n) {
        if (rank * CAP + wave + kSW * n < T) {
#pragma unroll
          for (int u = 0; u < U; ++u) pin(xs[n][u]);
          sign_half_row_lean<NC>(ring[e].smask, hme, hl, xs[n]);
          kstats_tile_keys<NC>(xs[n], hp, hn, lkey, koff, HD);
        }
      }
      if (T > 0) {
        kind_sync(&sctr, gen, kSW, a.err);  // the workgroup's keys of job i are complete
        // each workgroup starts at its own offset, so that the workgroups' atomics on
        // one key do not all arrive at once
        unsigned long long* kk = a.keys + (size_t)ji * 2 * HD;
        const unsigned long long tag = (unsigned long long)a.epoch << 32;
        const int rot = (rank * 64) % HD;
        for (int e0 = t; e0 < HD; e0 += 64 * kSW) {
          const int ee = (e0 + rot) % HD;
          const uint32_t kmn = lkey[ee], kmx = lkey[HD + ee];
          if (kmn != 0xffffffffu) atomicMax(kk + ee, tag | (unsigned long long)(~kmn));
          if (kmx != 0u) atomicMax(kk + HD + ee, tag | (unsigned long long)kmx);
          lkey[ee] = 0xffffffffu;
          lkey[HD + ee] = 0u;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the key pushes are performed
        kind_sync(&sctr, gen, kSW, a.err);
        if (t == 0)  // arrival: this workgroup's flag of the job holds the call's epoch
          __hip_atomic_store(a.counters + (size_t)ji * kCounterWords + rank, a.epoch, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
      // slot p is free once every Q-wave is done with job i - 2 (and so are the tables
      // of job i - 2, which those of job i + 1 replace)
      if (i >= 2 && !lds_wait(&qdone, (uint32_t)(kQW * (i - 1))) && t == 0) atomicOr(a.err, KVMI_ERR_SYNC);
#pragma unroll
      for (int n = 0; n < NTS; ++n) {
        const int c = wave + kSW * n;
        if (rank * CAP + c < T) {
#pragma unroll
          for (int u = 0; u < U; ++u) slot[p][c][u][l] = xs[n][u];
        }
        issue(i + 1, n);
      }
      if (i + 1 < nj) {
        if (i >= 2 && !lds_wait(&vdone, (uint32_t)(VW * (i - 1))) && t == 0) atomicOr(a.err, KVMI_ERR_SYNC);
        stage_tables(load_job(a.jobs, job_index(i + 1)), (i + 1) % kRing, t);
      }
      kind_sync(&sctr, gen, kSW, a.err);  // job i is in its slot, job i + 1's tables are staged
      if (t == 0) __hip_atomic_fetch_add(&staged, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return;
  }

  uint32_t over = 0;
  if (wave < kSW + kQW) {
    // ================================================================ Q-waves
    if (kPrioQ) __builtin_amdgcn_s_setprio(kPrioQ);
    const int qw = wave - kSW, t = (int)threadIdx.x - 64 * kSW;
    uint32_t gen = 0;
    bool broken = false;  // (the polling wave) a barrier timed out: later waits give up at once
    uint4 hp[2], hn[2];
    hp[0] = hadamard_tile(0, false, false);
    hp[1] = hadamard_tile(1, false, false);
    hn[0] = hadamard_tile(0, false, true);
    hn[1] = hadamard_tile(1, false, true);
    for (int i = 0; i < nj; ++i) {
      const int ji = job_index(i);
      const kvmi_layer_job jc = load_job(a.jobs, ji);
      const int T = job_tiles(jc), p = i & 1;
      const JobTables& tb = ring[i % kRing];
      if (rank * CAP < T) {  // the workgroup holds K tiles of job i
        if (qw == 0) {  // every workgroup's flag of the job holds this call's epoch
          const int l = threadIdx.x & 63;
          const uint32_t* fl = a.counters + (size_t)ji * kCounterWords;
          bool done = false;
          for (uint32_t polls = 0; !broken && polls < kMaxPolls; ++polls) {
            bool mine = true;
            for (int w = l; w < a.gsize; w += 64)
              mine &= __hip_atomic_load(fl + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
            if (__all(mine)) {
              done = true;
              break;
            }
            __builtin_amdgcn_s_sleep(1);
          }
          if (!done) {
            broken = true;
            if (l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
          }
        }
        kind_sync(&qctr, gen, kQW, a.err);  // job i's barrier is crossed; kc is free
        // job i's tiles are in slot p (the S-waves arrive before they store them)
        if (!lds_wait(&staged, (uint32_t)(i + 2)) && (threadIdx.x & 63) == 0) atomicOr(a.err, KVMI_ERR_SYNC);
        const unsigned long long* kk = a.keys + (size_t)ji * 2 * HD;
        bool stale = false;
        for (int ee = t; ee < HD; ee += 64 * kQW) {
          const int hs = ee / D, f = ee % D, j = tb.posk[hs];
          const unsigned long long vmn = __hip_atomic_load(kk + ee, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const unsigned long long vmx = __hip_atomic_load(kk + HD + ee, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          stale |= (uint32_t)(vmn >> 32) != a.epoch || (uint32_t)(vmx >> 32) != a.epoch;
          const float kmn = round_bf16(key2f(~(uint32_t)vmn) * s);  // keys are unscaled
          const float kmx = round_bf16(key2f((uint32_t)vmx) * s);
          const float sc = quant_scale(kmn, kmx, tb.prof[0][1][j]);
          kc[hs][f] = make_float2(kmn, 1.0f / sc);
          if (rank == 0) {
            gst(jc.kmeta + j * D + f, (uint16_t)f32_to_bf16_bits(kmn));
            gst(jc.kmeta + HD + j * D + f, (uint16_t)f32_to_bf16_bits(sc));
          }
        }
        if (stale) atomicOr(a.err, KVMI_ERR_SYNC);
        kind_sync(&qctr, gen, kQW, a.err);  // job i's constants are in kc
        // Per-lane values from an opaque lane id: left to itself the compiler hoists
        // the constant reads out of the tile loop and keeps them all live.
        const int l = opaque((int)threadIdx.x & 63), hl = l >> 5, r = l & 31, hme = r % H;
        const int jk = tb.posk[hme];
        const float lvk = (float)tb.prof[0][1][jk];
        const float2* kq = &kc[0][0] + opaque(hme * (D + 4) + HALF * hl);
#pragma unroll
        for (int n = 0; n < NTQ; ++n) {
          const int c = qw + kQW * n, tt = rank * CAP + c;
          if (tt >= T) break;
          uint4 x[U];
#pragma unroll
          for (int u = 0; u < U; ++u) x[u] = slot[p][c][u][l];
          LanePack<HALF, BITS> pkd;
          quant_k_tile<NC, BITS, CLAMP>(x, hp, hn, kq, s, lvk, pkd, over);
          // the tile is in registers: its slot space is this wave's stage
          uint4* st = &slot[p][c][0][0];
          pkd.store_lds(reinterpret_cast<uint8_t*>(st) + stage_off(jk, r, hl));
          flush(st, jc, 0, tt * tpt, l);
        }
      }
      lds_signal(&qdone);  // this Q-wave is done with job i's slot and tables
    }
  } else {
    // ================================================================ V-waves
    // Tiles v, v + VW, ... of the workgroup's range of every job, two load buffers
    // in turn (the loads of the next tile are in flight while a tile is encoded).
    if (kPrioV) __builtin_amdgcn_s_setprio(kPrioV);
    const int v = wave - kSW - kQW;
    const int r0 = threadIdx.x & 31, hl0 = (threadIdx.x >> 5) & 1;
    uint4* wst = &vstage[v][0];
    uint4 hp[2], hn[2];
    hp[0] = hadamard_tile(0, false, false);
    hp[1] = hadamard_tile(1, false, false);
    hn[0] = hadamard_tile(0, false, true);
    hn[1] = hadamard_tile(1, false, true);
    const uint16_t* lpool = fallback;
    int64_t lrow = 0;
    auto issue = [&](int i, int n, uint4 (&x)[U]) {
      if (i < nj) {
        const kvmi_layer_job jb = load_job(a.jobs, job_index(i));
        const int tt = rank * CAP + v + VW * n;
        if (tt < job_tiles(jb)) {
          lpool = reinterpret_cast<const uint16_t*>(jb.pool) + jb.pool_part_stride;
          lrow = tile_row0(jb, S, H, tt * tpt) + r0;
        }
      }
      load_half_row<NC>(lpool, lrow, hl0, x);
    };
    auto encode = [&](int i, int n, const kvmi_layer_job& jc, uint4 (&x)[U]) {
      const int tt = rank * CAP + v + VW * n;
      if (tt >= job_tiles(jc)) return;
      const JobTables& tb = ring[i % kRing];
      const int l = opaque((int)threadIdx.x & 63), hl = l >> 5, r = l & 31, hme = r % H;
      LaneProfile lp;
      lp.jv = tb.posv[hme];
      lp.gv = tb.prof[1][2][lp.jv];
      lp.lvv = (float)tb.prof[1][1][lp.jv];
      lp.rep_lane = hl == 0 && tb.gfirst[lp.gv] == hme;
      lp.jk = 0;
      lp.lvk = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) pin(x[u]);
      sign_half_row_lean<NC>(tb.smask, hme, hl, x);
      LanePack<HALF, BITS> pkd;
      // up to 4 bits the tile is transformed once and its rounded values kept as bf16
      // pairs (one MFMA pass fewer); wider packers need those registers themselves
      if constexpr (BITS <= 4)
        quant_v_tile<NC, BITS, CLAMP>(x, hp, hn, lp, jc, jc.num_blocks * S, tt * tpt + r / H, G, H, s, pkd, over);
      else
        quant_v_tile_twice<NC, BITS, CLAMP>(x, hp, hn, lp, jc, jc.num_blocks * S, tt * tpt + r / H, G, H, s, pkd,
                                            over);
      pkd.store_lds(reinterpret_cast<uint8_t*>(wst) + stage_off(lp.jv, r, hl));
      flush(wst, jc, 1, tt * tpt, l);
    };
    uint4 xa[U], xb[U];
    issue(0, 0, xa);
    for (int i = 0; i < nj; ++i) {
      if (!lds_wait(&staged, (uint32_t)(i + 1)) && (threadIdx.x & 63) == 0)  // tables of job i are in LDS
        atomicOr(a.err, KVMI_ERR_SYNC);
      const kvmi_layer_job jc = load_job(a.jobs, job_index(i));
#pragma unroll
      for (int n = 0; n < NTV; n += 2) {
        issue(i, n + 1, xb);
        encode(i, n, jc, xa);
        if (n + 2 < NTV)
          issue(i, n + 2, xa);
        else
          issue(i + 1, 0, xa);
        encode(i, n + 1, jc, xb);
      }
      lds_signal(&vdone);  // this V-wave is done with job i's tables
    }
  }
  if (over & overflow_mask<BITS>()) atomicOr(a.err, KVMI_ERR_SYMBOL_RANGE);
}

// ------------------------------------------------------------------ launch
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
int per_cu(K kernel, int threads) {
  int per = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel), threads, 0) !=
      hipSuccess)
    return 0;
  return per;
}

// Groups for these jobs, or false if the one-pass kernel cannot take them (a job's K
// exceeds the LDS of every workgroup of the grid, or no cooperative launch).  `cap`:
// K tiles a workgroup holds per job.
template <class K>
bool plan_groups(K kernel, int threads, int cap, const Geo& g, int32_t nj, int32_t mb, int* gsize, int* ngroups) {
  const DeviceInfo d = device_info();
  if (!d.coop || d.cus == 0) return false;
  const int per = per_cu(kernel, threads);
  if (per < 1) return false;
  const int grid = d.cus * per;
  const int64_t tiles = (int64_t)mb * g.S * g.H / kTok;
  const int64_t gs = (tiles + cap - 1) / cap;
  if (gs < 1 || gs > grid || gs > kCounterWords) return false;
  int ng = grid / (int)gs;
  if (ng > nj) ng = nj;
  *gsize = (int)gs;
  *ngroups = ng;
  return true;
}

template <int NC, int BITS, bool CLAMP>
int launch_pass(const PassArgs& in, int32_t mb, hipStream_t st, bool* taken) {
  constexpr int VW = v_waves<NC, BITS>();
  if constexpr (VW == 0) {
    *taken = false;  // the LDS cannot hold this width's stages: two passes
    return KVMI_OK;
  } else {
    auto kernel = compress_pass_kernel<NC, BITS, CLAMP, VW>;
    constexpr int threads = 64 * (kSW + kQW + VW);
    PassArgs a = in;
    if (!plan_groups(kernel, threads, cap_tiles<NC>(), a.g, a.num_jobs, mb, &a.gsize, &a.ngroups)) {
      *taken = false;
      return KVMI_OK;
    }
    *taken = true;
    void* args[] = {&a};
#ifdef KVMI_ORDINARY_LAUNCH
    // profiling build (python -m kvserve_amd.build --ordinary-launch): the same grid of
    // resident workgroups as an ordinary launch, which rocprofv3 can follow; every wait
    // of the kernel is bounded, so a workgroup that would not be resident ends in
    // KVMI_ERR_SYNC, never in a hang
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                         dim3((unsigned)(a.gsize * a.ngroups)), dim3(threads), args, 0, st);
#else
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel),
                                                    dim3((unsigned)(a.gsize * a.ngroups)), dim3(threads), args, 0, st);
#endif
    return e == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
  }
}

template <int NC, int BITS>
int launch_bits(const PassArgs& a, int32_t mb, hipStream_t st, bool* taken) {
  if (a.g.flags & KVMI_F_CLAMP_LEVELS) return launch_pass<NC, BITS, true>(a, mb, st, taken);
  return launch_pass<NC, BITS, false>(a, mb, st, taken);
}

template <int NC>
int launch_nc(const PassArgs& a, int32_t mb, hipStream_t st, bool* taken) {
  switch (a.g.bits) {
    case 1: return launch_bits<NC, 1>(a, mb, st, taken);
    case 2: return launch_bits<NC, 2>(a, mb, st, taken);
    case 3: return launch_bits<NC, 3>(a, mb, st, taken);
    case 4: return launch_bits<NC, 4>(a, mb, st, taken);
    case 5: return launch_bits<NC, 5>(a, mb, st, taken);
    case 6: return launch_bits<NC, 6>(a, mb, st, taken);
    case 7: return launch_bits<NC, 7>(a, mb, st, taken);
    default: return launch_bits<NC, 8>(a, mb, st, taken);
  }
}

int64_t counter_bytes(int32_t num_jobs) { return ((int64_t)num_jobs * kCounterWords * 4 + 255) / 256 * 256; }

}  // namespace
}  // namespace kvmi

extern "C" int64_t kvmi_compress_workspace_bytes(const kvmi_geometry* geom, int32_t num_jobs) {
  using namespace kvmi;
  Geo g;
  if (check_geo(geom, num_jobs, 0, &g)) return -1;
  return counter_bytes(num_jobs) + (int64_t)num_jobs * 2 * g.H * g.D * 8;
}

extern "C" int kvmi_kstats_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream);
extern "C" int kvmi_encode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                 int32_t max_blocks, int32_t* err, kvmi_stream_t stream);

extern "C" int kvmi_compress_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                                   int32_t max_blocks, void* workspace, uint32_t* epoch, int32_t* err,
                                   kvmi_stream_t stream) {
  using namespace kvmi;
  Geo g;
  int rc = check_geo(geom, num_jobs, max_blocks, &g);
  if (rc) return rc;
  if (num_jobs == 0 || max_blocks == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (mfma_eligible(g) && g.H <= kMH && !(g.flags & KVMI_F_TWO_PASS) && workspace) {
    if (!epoch || ((uintptr_t)workspace & 255)) return KVMI_EINVAL;
    // tags are 32-bit: past 2^31 calls a tag could come back while keys or flags of an
    // earlier call still hold it, so the caller must start the workspace afresh
    if (*epoch >= 0x80000000u) return KVMI_ERANGE;
    PassArgs a{};
    a.g = g;
    a.jobs = jobs;
    a.err = err;
    a.counters = static_cast<uint32_t*>(workspace);
    a.keys = reinterpret_cast<unsigned long long*>(static_cast<uint8_t*>(workspace) + counter_bytes(num_jobs));
    a.num_jobs = num_jobs;
    a.epoch = *epoch + 1;
    if (a.epoch == 0) a.epoch = 1;  // 0 is the value of keys never written
    bool taken = false;
    rc = g.D == 64 ? launch_nc<2>(a, max_blocks, st, &taken) : launch_nc<4>(a, max_blocks, st, &taken);
    if (taken) {
      if (rc == KVMI_OK) *epoch = a.epoch;
      return rc;
    }
  }
  rc = kvmi_kstats_paged(geom, jobs, num_jobs, max_blocks, err, stream);
  if (rc) return rc;
  return kvmi_encode_paged(geom, jobs, num_jobs, max_blocks, err, stream);
}
