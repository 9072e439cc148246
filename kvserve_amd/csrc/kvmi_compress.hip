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
#include <cstring>
#include <vector>

#include "kvmi_mfma_tiles.hpp"

namespace kvmi {
namespace {

constexpr int kOW = 8;        // waves per workgroup
constexpr int kOT = 512;      // threads per workgroup
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

// Tables of one step's V job (signs of every head, profile) and K-statistics head.
struct StepTables {
  uint32_t smask[kMH][64 + 4];  // V: sign-flip masks per (head, element pair)
  uint32_t kmask[64 + 4];       // K statistics: the masks of the group's head
  uint8_t prof[2][3][kMH];
  int posk[kMH], posv[kMH], gfirst[kMH];
};

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
  static_assert(tile_buf_q<NC>() >= 2 * NC * 64 && tile_buf_q<NC>() * 16 >= kTok * RB, "wave buffer uses");
  const Geo g = a.g;
  const int S = g.S, H = g.H, G = g.G, HD = H * D;
  const int wg = blockIdx.x, grid = a.grid, steps = a.steps;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, hl = l >> 5, r = l & 31, hme = r % H;
  const float sc_d = g.scale;
  const bool native = g.flags & KVMI_F_NATIVE_LAYOUT;
  const int tpt = kTok / H;  // tokens per V tile
  const uint32_t epoch = __builtin_amdgcn_readfirstlane(gld(a.epoch));

  __shared__ StepTables tab[3];           // by step % 3
  __shared__ uint32_t lkey[3][2 * D];     // the workgroup's min / max keys of a step's group, by step % 3
  __shared__ float2 kc[2][D + 4];         // (min, 1/scale) per channel of the group being quantized
  __shared__ int kinfo[2][2];             // its output position and levels
  __shared__ uint4 wbuf[kOW * tile_buf_q<NC>()];
  // Waves are ordered by monotone LDS counters, not workgroup barriers, so they may be up
  // to two steps apart: `staged` is the number of steps whose tables are staged (wave
  // s % 8 stages step s + 1's at the start of step s), `fin` counts the steps the waves
  // finished (every wave is past step s at 8 (s + 1)); a set is restaged only once every
  // wave is past its last step, and per-step LDS state is buffered deep enough for that.
  __shared__ uint32_t karr[2], kclaim, kready, kfinal, staged, fin;

  uint4* wb = wbuf + wave * tile_buf_q<NC>();
  uint8_t* ost = reinterpret_cast<uint8_t*>(wb);

  // ---------------------------------------------------------------- tables
  // Tables of a step into set e, by one wave: the job's sign words and profile bytes are
  // loaded once (one load per lane, all in flight together) and spread by lane shuffles.
  auto stage = [&](const OpRec& rc, int e) {
    StepTables& T = tab[e];
    if (rc.vjob >= 0) {
      const kvmi_layer_job jv = load_job(a.jobs, rc.vjob);
      constexpr int W = D / 32;  // sign words per head
      const uint32_t sw = l < H * W ? gld(jv.signs + l) : 0u;
      const uint32_t pb = l < 6 * H ? (uint32_t)gld(jv.profile + l) : 0u;
      for (int i = l; i < H * (D / 2); i += 64) {
        const int h = i / (D / 2), q = i % (D / 2);
        const uint32_t sb = (uint32_t)__shfl((int)sw, h * W + (2 * q) / 32) >> ((2 * q) & 31);
        T.smask[h][q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
      }
      if (l < 6 * H) T.prof[l / (3 * H)][(l / H) % 3][l % H] = (uint8_t)pb;
      // lane h < H: output positions of source head h (K, V) and the source head of
      // the first output position of V group h
      int pk = 0, pv = 0, gf = -1;
      for (int k = 0; k < H; ++k) {
        const int ok = __shfl((int)pb, k), ov = __shfl((int)pb, 3 * H + k);
        if (ok == l) pk = k;
        if (ov == l) pv = k;
      }
      for (int k = H - 1; k >= 0; --k) {  // (shuffles outside the branch: every lane takes part)
        const int gk = __shfl((int)pb, 5 * H + k), ok = __shfl((int)pb, 3 * H + k);
        if (gk == l) gf = ok;
      }
      if (l < H) {
        T.posk[l] = pk;
        T.posv[l] = pv;
        T.gfirst[l] = gf;
      }
    }
    if (rc.kjob >= 0) {
      const kvmi_layer_job jk = load_job(a.jobs, rc.kjob);
      const int h = rc.khead & 0xff;
      for (int q = l; q < D / 2; q += 64) {
        const uint32_t sb = gld(jk.signs + h * (D / 32) + (2 * q) / 32) >> ((2 * q) & 31);
        T.kmask[q] = ((sb & 1u) << 15) | ((sb & 2u) << 30);
      }
    }
  };

  // ---------------------------------------------------------------- loads
  // Every wave issues the same loads on every path (idle waves read `dummy`): a load
  // issued on one path only makes the compiler wait for every load in flight where the
  // paths join.
  //
  // K head-tile t of (job, head): tokens 32t .. 32t + 31, instruction v reads rows
  // RPI v .. RPI v + RPI - 1 (PR lanes per row, 16 bytes each).  S is a power of two
  // >= RPI, so the rows of one instruction lie in one block (block id by a scalar load);
  // rows past the job's last token repeat that token (min / max ignore repeats, and the
  // quantization does not write them).
  auto issue_k = [&](const OpRec& rc, uint4 (&x)[U]) {
    const uint16_t* base = a.dummy;
    int64_t rowoff[U];
#pragma unroll
    for (int v = 0; v < U; ++v) rowoff[v] = 0;
    const int kn = rc.kjob >= 0 ? (rc.khead >> 8) : 0;
    if (wave < kn) {
      const kvmi_layer_job jb = load_job(a.jobs, rc.kjob);
      const int T = jb.num_blocks * S, tt = rc.ktile0 + wave, h = rc.khead & 0xff;
      if (32 * tt < T) {
        base = reinterpret_cast<const uint16_t*>(jb.pool);
#pragma unroll
        for (int v = 0; v < U; ++v) {
          const int tv = 32 * tt + RPI * v;                // first token of the instruction
          const int tb = tv < T ? tv : T - 1;              // (uniform) token naming the block
          const int64_t blk = cld(jb.block_ids + tb / S);
          const int tok = tv < T ? tv + l / PR : T - 1;    // this lane's token
          rowoff[v] = ((blk * S + (tok & (S - 1))) * H + h) * D;
        }
      }
    }
#pragma unroll
    for (int v = 0; v < U; ++v) x[v] = gld(reinterpret_cast<const uint4*>(base + rowoff[v]) + l % PR);
  };
  // V tile vt of a job: rows 32 vt .. 32 vt + 31 of the job's token-major rows, within
  // one block (S*H % 32 == 0), loaded 1 KiB per instruction.
  auto issue_v = [&](const OpRec& rc, uint4 (&x)[U]) {
    const uint16_t* base = a.dummy;
    int64_t row0 = 0;
    if (rc.vjob >= 0 && wave < rc.vn) {
      const kvmi_layer_job jb = load_job(a.jobs, rc.vjob);
      const int vt = rc.vtile0 + wave;
      if (vt * kTok < jb.num_blocks * S * H) {
        base = reinterpret_cast<const uint16_t*>(jb.pool) + jb.pool_part_stride;
        row0 = tile_row0(jb, S, H, vt * tpt);
      }
    }
    load_tile<NC>(base, row0, x);
  };

  // ---------------------------------------------------------------- set-up
  uint4 hpN[2], hnN[2], hpT[2], hnT[2];
  hpN[0] = hadamard_tile(0, true, false);
  hpN[1] = hadamard_tile(1, true, false);
  hnN[0] = hadamard_tile(0, true, true);
  hnN[1] = hadamard_tile(1, true, true);
  hpT[0] = hadamard_tile(0, false, false);
  hpT[1] = hadamard_tile(1, false, false);
  hnT[0] = hadamard_tile(0, false, true);
  hnT[1] = hadamard_tile(1, false, true);
  uint32_t over = 0;
  bool broken = false;  // a device wait of this wave timed out: later ones give up at once

  for (int i = threadIdx.x; i < 2 * D; i += kOT) {
    const uint32_t init = i < D ? 0xffffffffu : 0u;
    lkey[0][i] = init;
    lkey[1][i] = init;
    lkey[2][i] = init;
  }
  if (threadIdx.x == 0) {
    karr[0] = karr[1] = 0;
    kclaim = kready = kfinal = fin = 0;
    staged = 1;  // step 0's tables, staged below
  }
  // chunks of jobs without blocks still get their header (the stream of N = 0 symbols)
  if (wg == 0 && !(g.flags & KVMI_F_NO_HEADER)) {
    for (int j = threadIdx.x; j < a.num_jobs; j += kOT) {
      const kvmi_layer_job* q = a.jobs + j;
      if (gld(&q->num_blocks) == 0 && gld(&q->write_header))
        write_stream_header(gld(&q->stream), BITS, gld(&q->chunk_symbols));
    }
  }
  if (steps > 0 && wave == 0) stage(load_rec(a.recs, wg), 0);
  __syncthreads();

  uint4 kb0[U], kb1[U], vb[U];
  {
    const OpRec r0 = steps > 0 ? load_rec(a.recs, wg) : no_rec();
    issue_k(r0, kb0);
    issue_v(r0, vb);
  }

  // ---------------------------------------------------------------- one step
  auto step = [&](int s, uint4 (&cur)[U], uint4 (&prev)[U]) {
    const int p = s & 1, p3 = s % 3;
    // step s's tables are staged (step 0's before the loop)
    if (s > 0 && s < steps && !lds_wait(&staged, (uint32_t)(s + 1)) && l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
    const OpRec rc = s < steps ? load_rec(a.recs, (int64_t)s * grid + wg) : no_rec();
    const OpRec rp = s > 0 ? load_rec(a.recs, (int64_t)(s - 1) * grid + wg) : no_rec();
    const OpRec rn = s + 1 < steps ? load_rec(a.recs, (int64_t)(s + 1) * grid + wg) : no_rec();
    if (s + 1 < steps && wave == s % kOW) {
      // step s + 1's tables into set (s + 1) % 3, last used in step s - 2
      if (s >= 2 && !lds_wait(&fin, (uint32_t)(kOW * (s - 1))) && l == 0) atomicOr(a.err, KVMI_ERR_SYNC);
      stage(rn, (s + 1) % 3);
      lds_order();
      if (l == 0) __hip_atomic_store(&staged, (uint32_t)(s + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // ------------------------------------------------ P1: K statistics of step s
    const int kn = rc.kjob >= 0 ? (rc.khead >> 8) : 0;
    if (wave < kn) {
      const kvmi_layer_job jb = load_job(a.jobs, rc.kjob);
      const bool mine = 32 * (rc.ktile0 + wave) < jb.num_blocks * S;
      if (mine) {
#pragma unroll
        for (int u = 0; u < U; ++u) pin(cur[u]);
        tile_to_half_rows<NC>(wb, cur);
        const uint4* sm = reinterpret_cast<const uint4*>(&tab[p3].kmask[0] + opaque((HALF / 2) * hl));
#pragma unroll
        for (int u = 0; u < U; ++u) cur[u] = xor4(cur[u], sm[u]);
        // orientation N: register i of chunk cp holds row 8(i/4) + 4hl + i%4, channel
        // HALF (r >> 4) + 16 cp + (r & 15); every row is the group's head
#pragma unroll
        for (int cp = 0; cp < NC; ++cp) {
          f32x16 acc = {};
#pragma unroll
          for (int k = 0; k < NC; ++k) {
            const int c = cp ^ k;
            const bool neg = __builtin_popcount(c & cp) & 1;
            acc = mfma(cur[2 * c], neg ? hnN[0] : hpN[0], acc);
            acc = mfma(cur[2 * c + 1], neg ? hnN[1] : hpN[1], acc);
          }
          float mn = fminf(fminf(acc[0], acc[1]), fminf(acc[2], acc[3]));
          float mx = fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3]));
#pragma unroll
          for (int i = 4; i < 16; i += 4) {
            mn = fminf(fminf(mn, acc[i]), fminf(acc[i + 1], fminf(acc[i + 2], acc[i + 3])));
            mx = fmaxf(fmaxf(mx, acc[i]), fmaxf(acc[i + 1], fmaxf(acc[i + 2], acc[i + 3])));
          }
          mn = halves_min(mn);
          mx = halves_max(mx);
          if (hl == 0) {
            const int f = HALF * (r >> 4) + 16 * cp + (r & 15);
            atomicMin(&lkey[p3][f], f2key(mn));  // unscaled: 1/sqrt(D) > 0 commutes with min / max
            atomicMax(&lkey[p3][D + f], f2key(mx));
          }
          chunk_fence();
        }
      }
      if (wave == 0 && rc.ktile0 == 0 && (rc.khead & 0xff) == 0 && jb.write_header &&
          !(g.flags & KVMI_F_NO_HEADER) && l == 0)
        write_stream_header(jb.stream, BITS, jb.chunk_symbols);
      // arrival: the last of the workgroup's K waves publishes its keys
      lds_order();
      uint32_t v = 0;
      if (l == 0) v = __hip_atomic_fetch_add(&karr[p], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      v = __builtin_amdgcn_readfirstlane(v);
      if (v == (uint32_t)(kn - 1)) {
        if (l == 0) karr[p] = 0;
        const int gws = rc.kgroup >> 16;
        if (gws > 1) {
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
        // a group of one workgroup keeps its final keys in lkey[p3] for P3 of step s + 1
        lds_order();
        if (l == 0) __hip_atomic_store(&kfinal, (uint32_t)(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }

    // ------------------------------------------------ P3: K quantization of step s - 1
    const int knp = rp.kjob >= 0 ? (rp.khead >> 8) : 0;
    if (wave < knp) {
      const kvmi_layer_job jb = load_job(a.jobs, rp.kjob);
      const int pp = (s - 1) % 3, hk = rp.khead & 0xff, T = jb.num_blocks * S;
      uint32_t old = 0;
      if (l == 0) old = __hip_atomic_fetch_max(&kclaim, (uint32_t)s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      old = __builtin_amdgcn_readfirstlane(old);
      if (old < (uint32_t)s) {
        // the first wave here: wait for the group, then the constants of its channels
        const int gw0 = rp.kgroup & 0xffff, gws = rp.kgroup >> 16;
        if (gws > 1) {
          const uint32_t* fl = a.flags + (int64_t)(s - 1) * grid + gw0;
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
        } else if (!lds_wait(&kfinal, (uint32_t)s) && l == 0) {  // step s - 1's keys are final (kfinal = s)
          atomicOr(a.err, KVMI_ERR_SYNC);
        }
        int jk = 0;
        for (int k = 0; k < H; ++k)
          if (cld(jb.profile + k) == hk) jk = k;
        const int lv = cld(jb.profile + H + jk);
        const unsigned long long* kk = a.keys + (int64_t)rp.kslot * 2 * D;
        bool stale = false;
        for (int e = l; e < D; e += 64) {
          uint32_t kmn, kmx;
          if (gws > 1) {
            const unsigned long long vmn = __hip_atomic_load(kk + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned long long vmx = __hip_atomic_load(kk + D + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            stale |= (uint32_t)(vmn >> 32) != epoch || (uint32_t)(vmx >> 32) != epoch;
            kmn = ~(uint32_t)vmn;
            kmx = (uint32_t)vmx;
          } else {
            kmn = lkey[pp][e];
            kmx = lkey[pp][D + e];
            lkey[pp][e] = 0xffffffffu;
            lkey[pp][D + e] = 0u;
          }
          const float mn = round_bf16(key2f(kmn) * sc_d);
          const float mx = round_bf16(key2f(kmx) * sc_d);
          const float scl = quant_scale(mn, mx, lv);
          kc[p][e] = make_float2(mn, 1.0f / scl);
          if (rp.ktile0 == 0 && T > 0) {  // the group's first workgroup writes the K metadata
            gst(jb.kmeta + jk * D + e, (uint16_t)f32_to_bf16_bits(mn));
            gst(jb.kmeta + HD + jk * D + e, (uint16_t)f32_to_bf16_bits(scl));
          }
        }
        if (stale && !broken) atomicOr(a.err, KVMI_ERR_SYNC);
        if (l == 0) {
          kinfo[p][0] = jk;
          kinfo[p][1] = lv;
        }
        lds_order();
        if (l == 0) __hip_atomic_store(&kready, (uint32_t)s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else if (!lds_wait(&kready, (uint32_t)s) && l == 0) {
        atomicOr(a.err, KVMI_ERR_SYNC);
      }
      const int tt = rp.ktile0 + wave;
      if (32 * tt < T) {
        const int jk = kinfo[p][0];
        const float lvk = (float)kinfo[p][1];
#pragma unroll
        for (int u = 0; u < U; ++u) pin(prev[u]);
        LanePack<HALF, BITS> pkd;
        quant_k_tile<NC, BITS, CLAMP>(prev, hpT, hnT, &kc[p][0] + opaque(HALF * hl), sc_d, lvk, pkd, over);
        pkd.store_lds(ost + r * RB + hl * (RB / 2));
        // rows 0 .. nv - 1 of the head-tile exist (nv a multiple of S, or 32)
        const int nv = min(32, T - 32 * tt), t0 = 32 * tt;
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
    issue_k(rn, prev);

    // ------------------------------------------------ P2: V encode of step s
    if (rc.vjob >= 0 && wave < rc.vn) {
      const kvmi_layer_job jv = load_job(a.jobs, rc.vjob);
      const int ntok = jv.num_blocks * S, vt = rc.vtile0 + wave;
      if (vt * kTok < ntok * H) {
        const StepTables& T = tab[p3];
        const int ta = vt * tpt;
#pragma unroll
        for (int u = 0; u < U; ++u) pin(vb[u]);
        tile_to_half_rows<NC>(wb, vb);
        sign_half_row<NC>(T, hme, hl, vb);
        const LaneProfile lp = lane_profile(T, hme, hl);
        LanePack<HALF, BITS> pkd;
        quant_v_tile_lds<NC, BITS, CLAMP>(vb, hpT, hnT, lp, jv, ntok, ta + r / H, G, H, sc_d, wb + l, pkd, over);
        const int off = native ? (r / H) * (H * RB) + lp.jv * RB + hl * (RB / 2)
                               : lp.jv * (tpt * RB) + (r / H) * RB + hl * (RB / 2);
        pkd.store_lds(ost + off);
        const int rq = native ? TQ : tpt * RB / 16;  // uint4 per run
#pragma unroll
        for (int u = 0; u < (TQ + 63) / 64; ++u) {
          const int q = 64 * u + l;
          if (TQ % 64 == 0 || q < TQ) {
            const int run_j = q / rq;
            uint8_t* dst = seg_addr<BITS>(jv, g, 1, native ? 0 : run_j, ta, 0) + 16 * (q - run_j * rq);
            gst(reinterpret_cast<uint4*>(dst), wb[q]);
          }
        }
      }
    }
    issue_v(rn, vb);
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
  h.image_bytes = h.rec_off + (int64_t)recs.size() * (int64_t)sizeof(OpRec);
  h.flag_off = round256(h.image_bytes);
  h.key_off = round256(h.flag_off + (int64_t)steps * grid * 4);
  h.epoch_off = round256(h.key_off + (int64_t)nslots * 2 * g.D * 8);
  h.total = std::max<int64_t>(h.epoch_off + 256, kMinWorkspace);
  if (image) {
    if (image_bytes < h.image_bytes) return KVMI_EINVAL;
    std::memset(image, 0, (size_t)kHeaderBytes);
    std::memcpy(image, &h, sizeof h);
    if (!recs.empty()) std::memcpy(static_cast<uint8_t*>(image) + h.rec_off, recs.data(), recs.size() * sizeof(OpRec));
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
