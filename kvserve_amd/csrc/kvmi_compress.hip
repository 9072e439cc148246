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
//     `rank` of a group owns tiles [rank*CAP, (rank+1)*CAP) of every job (CAP = 64 KiB
//     of bf16 K); a tile is the 32 pool rows of the MFMA kernels.
//   * A workgroup has two kinds of waves.  The 8 K-waves own one LDS slot of K tiles
//     each and move through the group's jobs in lockstep (LDS-counter barriers among
//     themselves).  For job J (P = the job before):
//       A  per tile: read P's K tile out of the slot, sign J's K tile (loaded during
//          the previous job), reduce its per-channel min / max (MFMA, orientation N)
//          into LDS keys and store it into the slot; quantize P's tile with P's
//          per-channel constants and write its symbols;
//       B  push the workgroup's keys of J to the job's device keys, arrive at J's
//          barrier, start loading J+1's K tiles;
//       C  wait until every workgroup of the group has arrived for J; turn J's device
//          keys into per-channel constants (workgroup rank 0 also writes J's K
//          metadata); stage J+1's K tables.
//     The 4 V-waves encode the workgroup's V tiles of every job (per-token statistics
//     need no other workgroup), each with its own copy of the job's sign masks: they
//     never wait, and keep HBM busy while the K-waves sit in a barrier.
//   * Keys and barrier counters need no clearing between calls: a key is a 64-bit
//     (epoch << 32 | order-preserving key) maximum, and each call adds exactly
//     kArrivals to a job's counters; the kernel waits for epoch * kArrivals.
//   * Every wait is bounded: on timeout the kernel sets KVMI_ERR_SYNC, later waits give
//     up at once, and every wave reaches the end of the kernel.
#include "kvmi_mfma_tiles.hpp"

namespace kvmi {
namespace {

constexpr int kKW = 8;                 // K-waves per workgroup
constexpr int kVW = 4;                 // V-waves per workgroup
constexpr int kPW = 64 * (kKW + kVW);  // threads per workgroup
constexpr int kKT = 64 * kKW;          // threads of the K-waves
constexpr int kArrivals = 1024;        // barrier weight one call adds per job (grid <= kArrivals)
constexpr int kSubs = 8;               // counters per job, one per 128-byte line
constexpr int kSubStride = 32;         // uint32 between a job's counters
constexpr int kCounterWords = kSubs * kSubStride;
constexpr uint32_t kMaxPolls = 1u << 18;  // ~0.3 s of polling before KVMI_ERR_SYNC

struct PassArgs {
  Geo g;
  const kvmi_layer_job* jobs;
  int32_t* err;
  uint32_t* counters;                  // [num_jobs][kCounterWords]
  unsigned long long* keys;            // [num_jobs][2][H][D]: max of (epoch << 32 | key)
  int num_jobs, gsize, ngroups;
  uint32_t epoch;
};

// Barrier weight of workgroup `rank` of a group of `gsize`: the number of s in
// [0, kArrivals) with s % gsize == rank, so that a group always adds kArrivals.
__device__ __forceinline__ uint32_t arrival_weight(int rank, int gsize) {
  return (uint32_t)((kArrivals - 1 - rank) / gsize + 1);
}

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
  j.counter = nullptr;
  j.pool_part_stride = cld(&q->pool_part_stride);
  j.symbol_offset = cld(&q->symbol_offset);
  j.chunk_symbols = cld(&q->chunk_symbols);
  j.num_blocks = cld(&q->num_blocks);
  j.write_header = cld(&q->write_header);
  return j;
}

// K statistics of one signed tile (orientation N, see kstats_tile), pushed into the
// workgroup's LDS keys chunk by chunk, so that no running min / max stays live.
template <int NC>
__device__ __forceinline__ void kstats_tile_push(const uint4 (&x)[2 * NC], const uint4 (&hp)[2],
                                                 const uint4 (&hn)[2], uint32_t* lkey, int H, float scale, int l) {
  constexpr int D = 32 * NC;
  const int hl = l >> 5, r = l & 31, HD = H * D;
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
    const int f = (16 * NC) * (r >> 4) + 16 * cp + (r & 15);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float mn = fminf(fminf(acc[q], acc[q + 4]), fminf(acc[q + 8], acc[q + 12]));
      const float mx = fmaxf(fmaxf(acc[q], acc[q + 4]), fmaxf(acc[q + 8], acc[q + 12]));
      const int h = (4 * hl + q) % H;
      atomicMin(&lkey[h * D + f], f2key(mn * scale));
      atomicMax(&lkey[HD + h * D + f], f2key(mx * scale));
    }
    chunk_fence();
  }
}

// Barrier of the K-waves of a workgroup: a monotone LDS counter, one arrival per wave.
// `gen` counts the barriers this wave has passed (the same on every K-wave).
__device__ __forceinline__ bool kwave_sync(uint32_t* ctr, uint32_t& gen) {
  gen += 1;
  lds_signal(ctr);
  return lds_wait(ctr, gen * kKW);
}

template <int NC, int BITS, bool CLAMP>
__global__ __launch_bounds__(kPW) void compress_pass_kernel(PassArgs a) {
  constexpr int D = 32 * NC, HALF = 16 * NC;
  constexpr int NT = 128 / D;                 // K tiles per K-wave per job
  constexpr int CAP = kKW * NT;               // tiles per workgroup per job
  constexpr int NV = CAP / kVW;               // V tiles per V-wave per job (even)
  constexpr int RP = D / 8 + 1;               // uint4 per slot row (one of padding)
  constexpr int TS = kTok * RP;               // uint4 per slot tile
  constexpr int RB = D * BITS / 8;            // bytes of one packed row
  constexpr int TQ = kTok * RB / 16;          // uint4 per packed tile
  static_assert(NV % 2 == 0, "V-waves alternate two load buffers");
  const Geo g = a.g;
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int grp = blockIdx.x / a.gsize, rank = blockIdx.x % a.gsize;
  if (grp >= a.ngroups) return;  // not part of any group (no barrier counts on it)
  const int nj = grp < a.num_jobs ? (a.num_jobs - 1 - grp) / a.ngroups + 1 : 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float s = g.scale;
  const bool native = g.flags & KVMI_F_NATIVE_LAYOUT;
  const int tpt = kTok / H;  // tokens per tile
  const uint4 kNeg = make_uint4(0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u);

  __shared__ uint4 slot[CAP * TS];                   // K tiles between statistics and quantization
  __shared__ uint4 stage[(kKW + kVW) * TQ];          // per wave: a packed tile on its way out
  __shared__ uint32_t lkey[2 * kMH * 128];           // K-waves: the workgroup's min / max keys
  __shared__ uint32_t smask[2][kMH][64 + 4];         // [job parity] sign masks
  __shared__ float2 kc[kMH][128 + 4];                // per-channel (min, 1/scale) by source head
  __shared__ uint8_t prof[2][2][3][kMH];             // [job parity][part][order, levels, group][position]
  __shared__ int8_t posk[2][kMH], posv[2][kMH], gfirst[2][kMH];
  __shared__ uint32_t kctr, staged, vdone;           // K-wave barrier; tables staged; V jobs done

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
  auto load_tile = [&](const kvmi_layer_job& job, int part, int t, int l, uint4 (&x)[2 * NC]) {
    const uint16_t* pool = reinterpret_cast<const uint16_t*>(job.pool) + part * job.pool_part_stride;
    load_half_row<NC>(pool, tile_row0(job, S, H, t * tpt) + (l & 31), l >> 5, x);
  };
  // Tables of `job` into parity p by the K-waves (t: K-thread id): sign masks, profile,
  // positions; the chunk header.
  auto stage_tables = [&](const kvmi_layer_job& job, int p, int t) {
    for (int i = t; i < H * (D / 2); i += kKT) {
      const int h = i / (D / 2), q = i % (D / 2);
      const uint32_t sb = gld(job.signs + h * (D / 32) + (2 * q) / 32) >> ((2 * q) & 31);
      smask[p][h][q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
    }
    if (t < 6 * H) {
      const int part = t / (3 * H), f = (t / H) % 3, k = t % H;
      prof[p][part][f][k] = gld(job.profile + t);
    }
    if (t < H) {
      int pk = 0, pv = 0, gf = -1;
      for (int k = 0; k < H; ++k) {
        if (gld(job.profile + k) == t) pk = k;
        if (gld(job.profile + 3 * H + k) == t) pv = k;
      }
      for (int k = H - 1; k >= 0; --k)  // first output position of V group t
        if (gld(job.profile + 5 * H + k) == t) gf = gld(job.profile + 3 * H + k);
      posk[p][t] = (int8_t)pk;
      posv[p][t] = (int8_t)pv;
      gfirst[p][t] = (int8_t)gf;
    }
    if (t == 0 && rank == 0 && job.write_header && !(g.flags & KVMI_F_NO_HEADER))
      write_stream_header(job.stream, BITS, job.chunk_symbols);
  };
  uint32_t over = 0;
  // staged counts the jobs whose tables are in LDS: job 0's are staged right below
  if (threadIdx.x == 0) {
    kctr = vdone = 0;
    staged = 1;
  }
  for (int e = threadIdx.x; e < HD; e += kPW) {
    lkey[e] = 0xffffffffu;
    lkey[HD + e] = 0u;
  }
  if (threadIdx.x < kKT && nj > 0) stage_tables(load_job(a.jobs, job_index(0)), 0, threadIdx.x);
  __syncthreads();  // the only barrier of all waves: job 0's tables are staged

  if (wave >= kKW) {
    // ================================================================ V-waves
    // Tiles v, v + kVW, ... of the workgroup's range of every job, two load buffers
    // in turn (the loads of the next tile are in flight while a tile is encoded).
    const int v = wave - kKW;
    uint4* wst = stage + wave * TQ;
    auto vtile = [&](int T, int n) {
      const int t = rank * CAP + v + kVW * n;
      return t < T ? t : -1;
    };
    uint4 xa[2 * NC], xb[2 * NC];
    auto issue = [&](int i, int n, uint4 (&x)[2 * NC]) {  // loads of tile n of job i (if any)
      if (i < nj) {
        const kvmi_layer_job jb = load_job(a.jobs, job_index(i));
        const int t = vtile(job_tiles(jb), n);
        if (t >= 0) load_tile(jb, 1, t, threadIdx.x & 63, x);
      }
    };
    auto encode = [&](int i, int n, uint4 (&x)[2 * NC]) {
      const kvmi_layer_job jc = load_job(a.jobs, job_index(i));
      const int t = vtile(job_tiles(jc), n);
      if (t < 0) return;
      const int p = i & 1;
      const int l = opaque(threadIdx.x & 63), hl = l >> 5, r = l & 31, hme = r % H;
      LaneProfile lp;
      lp.jv = posv[p][hme];
      lp.gv = prof[p][1][2][lp.jv];
      lp.lvv = (float)prof[p][1][1][lp.jv];
      lp.rep_lane = hl == 0 && gfirst[p][lp.gv] == hme;
      lp.jk = 0;
      lp.lvk = 0.f;
#pragma unroll
      for (int u = 0; u < 2 * NC; ++u) pin(x[u]);
      sign_half_row<NC>(smask[p], hme, hl, x);
      uint4 hp[2], hn[2];
      hp[0] = hadamard_tile(l, 0, false, false);
      hp[1] = hadamard_tile(l, 1, false, false);
      hn[0] = xor4(hp[0], kNeg);
      hn[1] = xor4(hp[1], kNeg);
      LanePack<HALF, BITS> pkd;
      quant_v_tile_twice<NC, BITS, CLAMP>(x, hp, hn, lp, jc, jc.num_blocks * S, t * tpt + r / H, G, H, s, pkd, over);
      pkd.store_lds(reinterpret_cast<uint8_t*>(wst) + stage_off(lp.jv, r, hl));
      flush(wst, jc, 1, t * tpt, l);
    };
    issue(0, 0, xa);
    for (int i = 0; i < nj; ++i) {
      if (!lds_wait(&staged, (uint32_t)(i + 1)) && (threadIdx.x & 63) == 0)  // tables of job i are in LDS
        atomicOr(a.err, KVMI_ERR_SYNC);
#pragma unroll
      for (int n = 0; n < NV; n += 2) {
        issue(i, n + 1, xb);
        encode(i, n, xa);
        if (n + 2 < NV)
          issue(i, n + 2, xa);
        else
          issue(i + 1, 0, xa);
        encode(i, n + 1, xb);
      }
      lds_signal(&vdone);  // this wave is done with job i's tables
    }
    if (over & overflow_mask<BITS>()) atomicOr(a.err, KVMI_ERR_SYMBOL_RANGE);
    return;
  }

  // ================================================================== K-waves
  // The K-waves carry the chain every workgroup of the group waits for: they issue
  // ahead of the V-waves on their SIMD.
  __builtin_amdgcn_s_setprio(2);
  const int ktid = threadIdx.x;  // 0 .. kKT-1
  uint32_t gen = 0;
  bool broken = false;  // (thread 0) a barrier timed out: later waits give up at once
  auto ksync = [&](int t) {
    if (!kwave_sync(&kctr, gen) && t == 0) atomicOr(a.err, KVMI_ERR_SYNC);
  };
  // tile c of this K-wave in a job of T tiles (-1: none)
  auto ktile = [&](int T, int c) {
    const int t = rank * CAP + wave + kKW * c;
    return t < T ? t : -1;
  };
  uint4 xk[NT][2 * NC];
  // Statistics of job i's K tiles (in xk) into the LDS keys, then their push to the
  // job's device keys (issued, not waited for).
  auto stats_and_push = [&](int i, const kvmi_layer_job& job, int t) {
    const int l = t & 63, hl = l >> 5, r = l & 31, hme = r % H;
    const int T = job_tiles(job), p = i & 1;
    uint4 hp[2], hn[2];
    hp[0] = hadamard_tile(l, 0, true, false);
    hp[1] = hadamard_tile(l, 1, true, false);
    hn[0] = xor4(hp[0], kNeg);
    hn[1] = xor4(hp[1], kNeg);
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if (ktile(T, c) < 0) continue;
#pragma unroll
      for (int u = 0; u < 2 * NC; ++u) pin(xk[c][u]);
      sign_half_row<NC>(smask[p], hme, hl, xk[c]);
      kstats_tile_push<NC>(xk[c], hp, hn, lkey, H, s, l);
    }
    ksync(t);
    // each workgroup starts at its own offset, so that the workgroups' atomics on one
    // key do not all arrive at once
    unsigned long long* kk = a.keys + (size_t)job_index(i) * 2 * HD;
    const unsigned long long tag = (unsigned long long)a.epoch << 32;
    const int rot = (rank * 64) % HD;
    for (int e0 = t; e0 < HD; e0 += kKT) {
      const int e = (e0 + rot) % HD;
      const uint32_t kmn = lkey[e], kmx = lkey[HD + e];
      if (kmn != 0xffffffffu) atomicMax(kk + e, tag | (unsigned long long)(~kmn));
      if (kmx != 0u) atomicMax(kk + HD + e, tag | (unsigned long long)kmx);
      lkey[e] = 0xffffffffu;
      lkey[HD + e] = 0u;
    }
  };
  // The pushed keys are performed, then the arrival at job i's barrier.
  auto arrive = [&](int i, int t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ksync(t);
    if (t == 0)
      __hip_atomic_fetch_add(a.counters + (size_t)job_index(i) * kCounterWords + (rank % kSubs) * kSubStride,
                             arrival_weight(rank, a.gsize), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (nj > 0) {
    const kvmi_layer_job j0 = load_job(a.jobs, job_index(0));
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int t = ktile(job_tiles(j0), c);
      if (t >= 0) load_tile(j0, 0, t, ktid & 63, xk[c]);
    }
    if (j0.num_blocks > 0) {
      stats_and_push(0, j0, ktid);
      arrive(0, ktid);
    }
  }
  // Job i: (1) K(i-1) quantized out of the slot, K(i) into it; (2) K(i+1) loads; (3)
  // tables of job i+1 (over those of job i-1); (4) statistics and key push of job i+1;
  // (5) wait for job i's barrier (its arrival was a whole phase ago); (6) per-channel
  // constants of job i; (7) arrival of job i+1.
  for (int i = 0; i <= nj; ++i) {
    // Per-lane values are re-derived every phase from an opaque thread id: left to
    // itself the compiler hoists every per-lane address and table tile out of the job
    // loop, which keeps them all live and spills.
    const int t = opaque(ktid), l = t & 63, hl = l >> 5, r = l & 31, hme = r % H;
    uint4* wst = stage + wave * TQ;
    const int p = i & 1;
    const bool cur = i < nj, nxt = i + 1 < nj;
    const int jci = cur ? job_index(i) : 0;
    kvmi_layer_job jc, jn;
    if (cur) jc = load_job(a.jobs, jci);
    if (nxt) jn = load_job(a.jobs, job_index(i + 1));
    const bool live = cur && jc.num_blocks > 0, live_n = nxt && jn.num_blocks > 0;
    const int Tc = cur ? job_tiles(jc) : 0;
    // ---------------- (1)
    {
      kvmi_layer_job jp;
      int jk = 0, Tp = 0;
      float lvk = 0.f;
      if (i > 0) {
        jp = load_job(a.jobs, job_index(i - 1));
        Tp = job_tiles(jp);
        jk = posk[p ^ 1][hme];
        lvk = (float)prof[p ^ 1][0][1][jk];
      }
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        const int tp = ktile(Tp, c), tc = ktile(Tc, c);
        uint4* sl = slot + (wave + kKW * c) * TS + r * RP + 2 * NC * hl;
        if (tp >= 0) {
          uint4 xq[2 * NC];
#pragma unroll
          for (int u = 0; u < 2 * NC; ++u) xq[u] = sl[u];
#pragma unroll
          for (int u = 0; u < 2 * NC; ++u) pin(xq[u]);
          uint4 hp[2], hn[2];
          hp[0] = hadamard_tile(l, 0, false, false);
          hp[1] = hadamard_tile(l, 1, false, false);
          hn[0] = xor4(hp[0], kNeg);
          hn[1] = xor4(hp[1], kNeg);
          const float2* kq = &kc[0][0] + opaque(hme * (128 + 4) + HALF * hl);
          LanePack<HALF, BITS> pkd;
          quant_k_tile<NC, BITS, CLAMP>(xq, hp, hn, kq, s, lvk, pkd, over);
          pkd.store_lds(reinterpret_cast<uint8_t*>(wst) + stage_off(jk, r, hl));
          flush(wst, jp, 0, tp * tpt, l);
        }
        if (tc >= 0) {
#pragma unroll
          for (int u = 0; u < 2 * NC; ++u) sl[u] = xk[c][u];
        }
      }
    }
    if (!cur) break;
    // ---------------- (2)
    if (nxt) {
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        const int tt = ktile(job_tiles(jn), c);
        if (tt >= 0) load_tile(jn, 0, tt, l, xk[c]);
      }
    }
    ksync(t);  // every K-wave is done with job i-1's tables and constants
    // ---------------- (3)
    if (nxt) {
      if (!lds_wait(&vdone, (uint32_t)(kVW * i)) && t == 0) atomicOr(a.err, KVMI_ERR_SYNC);
      stage_tables(jn, p ^ 1, t);
      ksync(t);
      if (t == 0) __hip_atomic_fetch_add(&staged, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // ---------------- (4)
    if (live_n) stats_and_push(i + 1, jn, t);
    // ---------------- (5), (6)
    if (live) {
      if (t == 0) {
        const uint32_t* cb = a.counters + (size_t)jci * kCounterWords;
        const uint32_t target = a.epoch * (uint32_t)kArrivals;
        bool done = false;
        for (uint32_t polls = 0; !broken && polls < kMaxPolls; ++polls) {
          uint32_t sum = 0;
#pragma unroll
          for (int k = 0; k < kSubs; ++k)
            sum += __hip_atomic_load(cb + k * kSubStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if ((int32_t)(sum - target) >= 0) {
            done = true;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (!done) {
          broken = true;
          atomicOr(a.err, KVMI_ERR_SYNC);
        }
      }
      ksync(t);
      const unsigned long long* kk = a.keys + (size_t)jci * 2 * HD;
      bool stale = false;
      for (int e = t; e < HD; e += kKT) {
        const int hs = e / D, f = e % D, j = posk[p][hs];
        const unsigned long long vmn = __hip_atomic_load(kk + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long vmx = __hip_atomic_load(kk + HD + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stale |= (uint32_t)(vmn >> 32) != a.epoch || (uint32_t)(vmx >> 32) != a.epoch;
        const float kmn = round_bf16(key2f(~(uint32_t)vmn));
        const float kmx = round_bf16(key2f((uint32_t)vmx));
        const float sc = quant_scale(kmn, kmx, prof[p][0][1][j]);
        kc[hs][f] = make_float2(kmn, 1.0f / sc);
        if (rank == 0) {
          gst(jc.kmeta + j * D + f, (uint16_t)f32_to_bf16_bits(kmn));
          gst(jc.kmeta + HD + j * D + f, (uint16_t)f32_to_bf16_bits(sc));
        }
      }
      if (stale) atomicOr(a.err, KVMI_ERR_SYNC);
    }
    // ---------------- (7) (its barrier also publishes the constants to every K-wave)
    if (live_n)
      arrive(i + 1, t);
    else
      ksync(t);
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
int per_cu(K kernel) {
  int per = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel), kPW, 0) !=
      hipSuccess)
    return 0;
  return per;
}

// Groups for these jobs, or false if the one-pass kernel cannot take them (a job's K
// exceeds the LDS of every workgroup of the grid, or no cooperative launch).
template <class K>
bool plan_groups(K kernel, const Geo& g, int32_t nj, int32_t mb, int* gsize, int* ngroups) {
  const DeviceInfo d = device_info();
  if (!d.coop || d.cus == 0) return false;
  const int per = per_cu(kernel);
  if (per < 1) return false;
  int grid = d.cus * per;
  if (grid > kArrivals) grid = kArrivals;
  const int cap = kKW * (128 / g.D);
  const int64_t tiles = (int64_t)mb * g.S * g.H / kTok;
  const int64_t gs = (tiles + cap - 1) / cap;
  if (gs < 1 || gs > grid) return false;
  int ng = grid / (int)gs;
  if (ng > nj) ng = nj;
  *gsize = (int)gs;
  *ngroups = ng;
  return true;
}

template <int NC, int BITS, bool CLAMP>
int launch_pass(const PassArgs& in, int32_t mb, hipStream_t st, bool* taken) {
  auto kernel = compress_pass_kernel<NC, BITS, CLAMP>;
  PassArgs a = in;
  if (!plan_groups(kernel, a.g, a.num_jobs, mb, &a.gsize, &a.ngroups)) {
    *taken = false;
    return KVMI_OK;
  }
  *taken = true;
  void* args[] = {&a};
#ifdef KVMI_ORDINARY_LAUNCH
  // profiling build (python -m kvserve_amd.build --ordinary-launch): the same grid of
  // resident workgroups as an ordinary launch, which rocprofv3 can follow; every wait of
  // the kernel is bounded, so a workgroup that would not be resident ends in
  // KVMI_ERR_SYNC, never in a hang
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3((unsigned)(a.gsize * a.ngroups)),
                                       dim3(kPW), args, 0, st);
#else
  const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel),
                                                  dim3((unsigned)(a.gsize * a.ngroups)), dim3(kPW), args, 0, st);
#endif
  return e == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
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
  if (mfma_eligible(g) && !(g.flags & KVMI_F_TWO_PASS) && workspace) {
    if (!epoch || ((uintptr_t)workspace & 255)) return KVMI_EINVAL;
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
