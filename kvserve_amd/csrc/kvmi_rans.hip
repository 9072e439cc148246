// rANS entropy codec for the codec stage (the place KVServe fills with nvCOMP ANS,
// kvserve_v1/compression/codec/kvserve_codec.py:57-64).  nvCOMP's stream format is
// closed, so this codec has its own; oracle/rans.c states it byte for byte and the
// parity tests compare the two.
//
// Input: n symbols of W bits packed LSB-first (the bitpack body).  The stream is a
// 32-byte header, a u64 offset per block, then the blocks.  A block covers 65536
// symbols in 4 sub-blocks of 16384 that share the block's 12-bit frequency table
// (K and V, layers and heads have different statistics).  A sub-block is coded by
// one wave: 64 interleaved 32-bit rANS states, lane i taking sub-block symbol
// (t/32)*2048 + i*32 + t%32 at step t (t < 256).  Blocks renormalise in 16-bit words
// and are stored raw when coding would not make them smaller.  Four waves per block
// keep the serial chain of a state at 256 steps, so a stream of a few hundred blocks
// still spreads over the chip.
//
// Kernels (one 256-thread workgroup per block, wave j on sub-block j):
//   rans_encode_kernel   histogram -> table -> encode (steps 255..0) into a
//                        per-block slot of a scratch buffer, block size out
//   rans_scan_kernel     one workgroup per stream: header and exclusive offsets
//   rans_compact_kernel  copies each block from its slot (or the raw input) to its
//                        offset in the stream
//   rans_decode_kernel   table -> decode (steps 0..255) -> packed symbols
// Division x / f by the 12-bit frequency uses a multiplier and two shifts per symbol
// (T. Granlund, P. Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, fig. 4.1).
#include "kvmi_device.hpp"
#include "../../include/kvserve_amd.h"

namespace kvmi {
namespace {

constexpr uint32_t kRansMagic = 0x5352564Bu;  // "KVRS"
constexpr uint32_t kPB = 12;
constexpr uint32_t kM = 1u << kPB;
constexpr uint32_t kLanes = 64;
constexpr uint32_t kRun = 32;
constexpr uint32_t kSubs = 4;                       // sub-blocks (waves) per block
constexpr uint32_t kSubSteps = 256;
constexpr uint32_t kSubRuns = kSubSteps / kRun;     // runs of 32 steps per sub-block
constexpr uint32_t kSub = kLanes * kSubSteps;       // 16384 symbols
constexpr uint32_t kBlock = kSub * kSubs;           // 65536 symbols
constexpr uint32_t kBlockThreads = kLanes * kSubs;  // workgroup of the block kernels
constexpr uint32_t kStateL = 1u << 16;
constexpr int kScanThreads = 1024;
constexpr int kCopyThreads = 256;

__host__ __device__ constexpr uint64_t pad4(uint64_t b) { return (b + 3u) & ~(uint64_t)3u; }

template <int W>
struct RansGeo {
  static constexpr uint32_t A = 1u << W;
  static constexpr uint32_t kTab = (uint32_t)pad4(2u * A);                 // u16 frequency table
  static constexpr uint32_t kCounts = 4u + kTab;                           // u32 count[3] of sub-blocks 1..3
  static constexpr uint32_t kStates = kCounts + 4u * (kSubs - 1u);         // u32 state[4][64]
  static constexpr uint32_t kHead = kStates + 4u * kLanes * kSubs;         // tag, table, counts, states
  static constexpr uint32_t kSubCap = kSub * W / 8;                        // packed bytes of a sub-block
  static constexpr uint32_t kGuard = 2u * kLanes * kRun;                   // one run of words past the capacity
  static constexpr uint32_t kRegion = kGuard + kSubCap;                    // word region of a sub-block
  static constexpr uint32_t kSlot = kHead + kSubs * kRegion;               // scratch bytes per block
};

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t rank_in(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o, 64));
  return v;
}

// Sum / max over the block's workgroup (every thread calls; red holds kSubs values).
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* red) {
  v = wave_sum(v);
  if (lane_id() == 0) red[threadIdx.x / kLanes] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (uint32_t j = 0; j < kSubs; ++j) r += red[j];
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* red) {
  v = wave_max(v);
  if (lane_id() == 0) red[threadIdx.x / kLanes] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (uint32_t j = 0; j < kSubs; ++j) r = max(r, red[j]);
  __syncthreads();
  return r;
}

// Exclusive prefix sum over the workgroup's threads (every thread calls; red holds
// kSubs values): in-wave shuffle scan, then the totals of the lower waves.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* red) {
  const uint32_t lane = lane_id(), wave = threadIdx.x / kLanes;
  uint32_t incl = v;
#pragma unroll
  for (int o = 1; o < (int)kLanes; o <<= 1) {
    const uint32_t u = __shfl_up(incl, o, 64);
    if ((int)lane >= o) incl += u;
  }
  if (lane == kLanes - 1) red[wave] = incl;
  __syncthreads();
  uint32_t below = 0;
#pragma unroll
  for (uint32_t j = 0; j < kSubs; ++j)
    if (j < wave) below += red[j];
  __syncthreads();
  return below + incl - v;
}

// Orders this wave's LDS accesses around a write-then-read by other lanes of the
// same wave (the wave's LDS instructions execute in issue order).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The W dwords of run r of `lane` (32 symbols) of a block whose packed bytes start at
// `blk` and of which `avail` bytes exist; bytes past the end read as zero.
template <int W>
__device__ __forceinline__ void load_run(const uint8_t* blk, uint64_t avail, uint32_t r, uint32_t lane,
                                         uint32_t (&d)[W]) {
  const uint64_t off = ((uint64_t)r * kLanes + lane) * (4u * W);
  if (off + 4u * W <= avail) {
#pragma unroll
    for (int k = 0; k < W; ++k) d[k] = gld(reinterpret_cast<const uint32_t*>(blk + off) + k);
  } else {
#pragma unroll
    for (int k = 0; k < W; ++k) {
      uint32_t v = 0;
      for (int byte = 0; byte < 4; ++byte) {
        const uint64_t o = off + 4u * k + byte;
        if (o < avail) v |= (uint32_t)gld(blk + o) << (8 * byte);
      }
      d[k] = v;
    }
  }
}

template <int W>
__device__ __forceinline__ uint32_t sym_at(const uint32_t (&d)[W], int j) {
  const int bit = j * W, k = bit >> 5, sh = bit & 31;
  uint32_t v = d[k] >> sh;
  if (sh + W > 32) v |= d[k + 1] << (32 - sh);
  return v & ((1u << W) - 1u);
}

__device__ __forceinline__ void gst16(uint16_t* p, uint32_t v) { gst(p, (uint16_t)v); }

// ------------------------------------------------------------------ batches
// Up to kMaxJobs streams per launch, passed by value: one grid covers the blocks of
// every stream of a request (the streams of an 8-layer-chunked request are coded by
// one launch per kernel), so small streams still fill the chip.
constexpr int kMaxJobs = 16;

struct EncBatch {
  const uint8_t* packed[kMaxJobs];
  uint8_t* out[kMaxJobs];
  uint8_t* slots[kMaxJobs];
  uint32_t* sizes[kMaxJobs];
  uint64_t* out_len[kMaxJobs];
  uint64_t n[kMaxJobs];
  uint32_t first[kMaxJobs + 1];  // first grid block of each job; first[count] = total
  int32_t count;
};

struct DecBatch {
  const uint8_t* in[kMaxJobs];
  uint8_t* out[kMaxJobs];
  uint64_t in_bytes[kMaxJobs];
  uint64_t n[kMaxJobs];
  uint32_t first[kMaxJobs + 1];
  int32_t count;
};

// job of grid block `g` (wave-uniform: kernel arguments live in scalar registers)
template <class Batch>
__device__ __forceinline__ int job_of(const Batch& bt, uint32_t g) {
  int j = 0;
  while (j + 1 < bt.count && g >= bt.first[j + 1]) ++j;
  return j;
}

// ------------------------------------------------------------------ encode
constexpr uint32_t kEncGroup = 8;  // steps whose table reads are issued together

// Steps 255..0 of one sub-block whose runs are block runs run0 .. run0 + 7 (FULL:
// every lane has a symbol at every step).  Leaves pos < 0 when the words outgrow the
// capacity (the block is then stored raw).
template <int W, bool FULL>
__device__ __forceinline__ void encode_runs(const uint8_t* blk, uint64_t avail, uint32_t run0, uint32_t lane,
                                            uint32_t nb, const uint2* tab, uint16_t* words, int32_t& pos,
                                            uint32_t& x) {
  uint32_t d[W], dn[W];
  load_run<W>(blk, avail, run0 + kSubRuns - 1, lane, d);
  for (int r = (int)kSubRuns - 1; r >= 0; --r) {
    if (r > 0) load_run<W>(blk, avail, run0 + (uint32_t)r - 1, lane, dn);  // next run in flight
    const uint32_t base = (run0 + (uint32_t)r) * (kLanes * kRun) + lane * kRun;
#pragma unroll
    for (int g = (int)kRun / kEncGroup - 1; g >= 0; --g) {
    // a group's table entries depend on its symbols only: their reads are in flight
    // before its first step, off the state's dependency chain
    uint2 ent[kEncGroup];
#pragma unroll
    for (int jj = 0; jj < (int)kEncGroup; ++jj) ent[jj] = tab[sym_at<W>(d, g * (int)kEncGroup + jj)];
#pragma unroll
    for (int jj = (int)kEncGroup - 1; jj >= 0; --jj) {
      const int j = g * (int)kEncGroup + jj;
      const bool valid = FULL || base + (uint32_t)j < nb;
      const uint2 e = ent[jj];
      const uint32_t fs = e.x & 0x1fffu;
      const bool emit = valid && (x >> 20) >= fs;
      const uint64_t mask = __ballot(emit);
      pos -= (int32_t)__popcll(mask);
      if (emit) {
        gst16(words + pos + (int32_t)rank_in(mask), x & 0xffffu);
        x >>= 16;
      }
      if (valid) {
        const uint32_t t1 = __umulhi(e.y, x);
        const uint32_t q = (t1 + ((x - t1) >> ((e.x >> 25) & 1u))) >> (e.x >> 26);
        x = (q << kPB) + (x - q * fs) + ((e.x >> 13) & 0xfffu);
      }
    }
    }
    if (pos < 0) return;
#pragma unroll
    for (int k = 0; k < W; ++k) d[k] = dn[k];
  }
}

template <int W>
__global__ __launch_bounds__(kBlockThreads) void rans_encode_kernel(const EncBatch bt) {
  using G = RansGeo<W>;
  constexpr bool kPrivate = W <= 5;  // lane-private histogram columns (no LDS contention)
  constexpr uint32_t kHist = kPrivate ? G::A * kLanes : G::A;  // per wave
  __shared__ __align__(16) uint32_t hist[kSubs * kHist];
  __shared__ uint2 tab[G::A];
  __shared__ uint32_t red[kSubs];
  __shared__ int32_t cnt[kSubs];

  const uint32_t lane = lane_id(), wave = threadIdx.x / kLanes, t = threadIdx.x;
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint64_t b = blockIdx.x - bt.first[jb];
  const uint64_t first = b * kBlock;
  const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
  const uint64_t in_bytes = (n * W + 7) / 8;
  const uint8_t* blk = bt.packed[jb] + first * W / 8;
  const uint64_t avail = in_bytes - first * W / 8;
  uint8_t* slot = bt.slots[jb] + b * G::kSlot;
  const uint32_t run0 = wave * kSubRuns;                    // this wave's sub-block
  const bool full = (wave + 1) * kSub <= nb;

  for (uint32_t i = t; i < kSubs * kHist; i += kBlockThreads) hist[i] = 0;
  __syncthreads();
  {
    uint32_t* h = hist + wave * kHist;
    uint32_t d[W], dn[W];
    load_run<W>(blk, avail, run0, lane, d);
    for (uint32_t r = 0; r < kSubRuns; ++r) {
      if (r + 1 < kSubRuns) load_run<W>(blk, avail, run0 + r + 1, lane, dn);  // next run in flight
      const uint32_t base = (run0 + r) * (kLanes * kRun) + lane * kRun;
#pragma unroll
      for (int j = 0; j < (int)kRun; ++j) {
        const uint32_t s = sym_at<W>(d, j);
        if (full || base + (uint32_t)j < nb) atomicAdd(&h[kPrivate ? s * kLanes + lane : s], 1u);
      }
#pragma unroll
      for (int k = 0; k < W; ++k) d[k] = dn[k];
    }
  }
  __syncthreads();

  // thread v < A: count of symbol v over the block
  uint32_t c = 0;
  if (t < G::A) {
    for (uint32_t j = 0; j < kSubs; ++j) {
      if (kPrivate) {
        const uint4* row = reinterpret_cast<const uint4*>(&hist[j * kHist + t * kLanes]);
        for (int q = 0; q < (int)kLanes / 4; ++q) {
          const uint4 hv = row[q];
          c += hv.x + hv.y + hv.z + hv.w;
        }
      } else {
        c += hist[j * kHist + t];
      }
    }
  }
  const uint32_t K = block_sum(c ? 1u : 0u, red);
  // most frequent, lowest value on ties
  const uint32_t top = 255u - (block_max(t < G::A ? (c << 8) | (255u - t) : 0u, red) & 255u);
  uint32_t f = c ? 1u + c * (kM - K) / nb : 0u;
  const uint32_t fsum = block_sum(f, red);
  if (t == top) f += kM - fsum;
  if (t < G::A) gst16(reinterpret_cast<uint16_t*>(slot + 4) + t, f);
  const uint32_t cum = block_exclusive_scan(f, red);  // f = 0 for threads >= A
  if (t < G::A) {
    const uint32_t l = f <= 1u ? 0u : 32u - __clz(f - 1u);
    const uint32_t mul = f ? (uint32_t)((((uint64_t)((1u << l) - f)) << 32) / f + 1u) : 0u;
    const uint32_t sh1 = l ? 1u : 0u, sh2 = l ? l - 1u : 0u;
    tab[t] = make_uint2(f | (cum << 13) | (sh1 << 25) | (sh2 << 26), mul);
  }
  __syncthreads();

  // encode, steps 255..0; words fill the sub-block's word region from its end.  The
  // capacity is checked once per run: a run emits at most 64 * 32 words, which the
  // guard region in front of the word region absorbs.
  uint16_t* words = reinterpret_cast<uint16_t*>(slot + G::kHead + wave * G::kRegion + G::kGuard);
  int32_t pos = (int32_t)(G::kSubCap / 2);
  uint32_t x = kStateL;
  if (full) encode_runs<W, true>(blk, avail, run0, lane, nb, tab, words, pos, x);
  else encode_runs<W, false>(blk, avail, run0, lane, nb, tab, words, pos, x);
  const uint32_t count = G::kSubCap / 2 - (uint32_t)pos;  // meaningful when pos >= 0
  gst(reinterpret_cast<uint32_t*>(slot + G::kStates) + wave * kLanes + lane, x);
  if (lane == 0) {
    cnt[wave] = pos < 0 ? -1 : (int32_t)count;
    if (pos >= 0 && (count & 1u)) gst16(words + pos - 1, 0u);
  }
  __syncthreads();
  if (t == 0) {
    bool over = false;
    uint64_t size = G::kHead;
    for (uint32_t j = 0; j < kSubs; ++j) {
      over |= cnt[j] < 0;
      size += pad4(2ull * (uint32_t)max(cnt[j], 0));
    }
    const uint64_t raw = 4u + pad4(((uint64_t)nb * W + 7) / 8);
    uint32_t* sizes = bt.sizes[jb];
    if (over || size >= raw) {
      gst(reinterpret_cast<uint32_t*>(slot), 1u);
      gst(sizes + b, (uint32_t)raw);
    } else {
      gst(reinterpret_cast<uint32_t*>(slot), (uint32_t)cnt[0] << 1);
      for (uint32_t j = 1; j < kSubs; ++j) gst(reinterpret_cast<uint32_t*>(slot + G::kCounts) + (j - 1), (uint32_t)cnt[j]);
      gst(sizes + b, (uint32_t)size);
    }
  }
}

// ------------------------------------------------------------------ scan + header
// One workgroup per stream: exclusive block offsets, header, stream length.
template <int W>
__global__ __launch_bounds__(kScanThreads) void rans_scan_kernel(const EncBatch bt) {
  __shared__ uint64_t part[kScanThreads];
  const int jb = blockIdx.x;
  const uint64_t n = bt.n[jb];
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  const uint32_t* sizes = bt.sizes[jb];
  uint8_t* out = bt.out[jb];
  const uint32_t t = threadIdx.x;
  const uint32_t per = (nblk + kScanThreads - 1) / kScanThreads;
  const uint32_t lo = min(nblk, t * per), hi = min(nblk, lo + per);
  uint64_t s = 0;
  for (uint32_t i = lo; i < hi; ++i) s += gld(sizes + i);
  part[t] = s;
  __syncthreads();
  for (int o = 1; o < kScanThreads; o <<= 1) {
    const uint64_t v = t >= (uint32_t)o ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  uint64_t off = part[t] - s;  // exclusive
  uint64_t* offs = reinterpret_cast<uint64_t*>(out + 32);
  for (uint32_t i = lo; i < hi; ++i) {
    gst(offs + i, off);
    off += gld(sizes + i);
  }
  if (t == kScanThreads - 1) {
    const uint64_t payload = part[t];
    uint32_t* h = reinterpret_cast<uint32_t*>(out);
    gst(h + 0, kRansMagic);
    gst(h + 1, 2u | ((uint32_t)W << 8) | (kPB << 16) | (8u << 24));
    gst(h + 2, kBlock);
    gst(h + 3, nblk);
    gst(reinterpret_cast<uint64_t*>(out + 16), n);
    gst(reinterpret_cast<uint64_t*>(out + 24), payload);
    gst(bt.out_len[jb], (uint64_t)(32u + 8ull * nblk + payload));
  }
}

// ------------------------------------------------------------------ compaction
// SCAN: the workgroup sums the sizes of the blocks in front of its own (streams of
// at most kFusedScanBlocks blocks), writes its offset, and the last block's
// workgroup writes the header and the length; otherwise rans_scan_kernel ran first.
constexpr uint32_t kFusedScanBlocks = 512;
static_assert(kCopyThreads == kBlockThreads, "block_sum covers the compaction workgroup");

template <int W, bool SCAN>
__global__ __launch_bounds__(kCopyThreads) void rans_compact_kernel(const EncBatch bt) {
  using G = RansGeo<W>;
  __shared__ uint32_t red[kSubs];
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  const uint64_t b = blockIdx.x - bt.first[jb];
  uint8_t* out = bt.out[jb];
  uint64_t off;
  if (SCAN) {
    const uint32_t* sizes = bt.sizes[jb];
    uint32_t part = 0;  // block sizes are < 2^17 and b < kFusedScanBlocks: no overflow
    for (uint32_t i = threadIdx.x; i < (uint32_t)b; i += kCopyThreads) part += gld(sizes + i);
    off = block_sum(part, red);
    if (threadIdx.x == 0) {
      gst(reinterpret_cast<uint64_t*>(out + 32) + b, off);
      if (b + 1 == nblk) {
        const uint64_t payload = off + gld(sizes + b);
        uint32_t* h = reinterpret_cast<uint32_t*>(out);
        gst(h + 0, kRansMagic);
        gst(h + 1, 2u | ((uint32_t)W << 8) | (kPB << 16) | (8u << 24));
        gst(h + 2, kBlock);
        gst(h + 3, nblk);
        gst(reinterpret_cast<uint64_t*>(out + 16), n);
        gst(reinterpret_cast<uint64_t*>(out + 24), payload);
        gst(bt.out_len[jb], (uint64_t)(32u + 8ull * nblk + payload));
      }
    }
  } else {
    off = gld(reinterpret_cast<const uint64_t*>(out + 32) + b);
  }
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + 32 + 8ull * nblk + off);
  const uint8_t* slot = bt.slots[jb] + b * G::kSlot;
  const uint32_t tag = gld(reinterpret_cast<const uint32_t*>(slot));
  const uint32_t t = threadIdx.x;
  if (tag & 1u) {
    const uint64_t first = b * kBlock;
    const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
    const uint64_t rb = ((uint64_t)nb * W + 7) / 8;
    const uint8_t* src = bt.packed[jb] + first * W / 8;
    const uint64_t avail = (n * W + 7) / 8 - first * W / 8;
    if (t == 0) gst(dst, 1u);
    for (uint64_t i = t; i < pad4(rb) / 4; i += kCopyThreads) {
      uint32_t v;
      if (4 * i + 4 <= avail) {
        v = gld(reinterpret_cast<const uint32_t*>(src) + i);
      } else {
        v = 0;
        for (int k = 0; k < 4; ++k)
          if (4 * i + k < rb) v |= (uint32_t)gld(src + 4 * i + k) << (8 * k);
      }
      gst(dst + 1 + i, v);
    }
    return;
  }
  const uint32_t* head = reinterpret_cast<const uint32_t*>(slot);
  for (uint32_t i = t; i < G::kHead / 4; i += kCopyThreads) gst(dst + i, gld(head + i));
  uint32_t at = G::kHead / 4;
  for (uint32_t j = 0; j < kSubs; ++j) {
    const uint32_t count = j ? gld(reinterpret_cast<const uint32_t*>(slot + G::kCounts) + (j - 1)) : tag >> 1;
    const uint32_t wbytes = (uint32_t)pad4(2ull * count);
    const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(slot + G::kHead + (j + 1) * G::kRegion - wbytes);
    for (uint32_t i = t; i < wbytes / 4; i += kCopyThreads) gst(dst + at + i, gld(wsrc + i));
    at += wbytes / 4;
  }
}

// ------------------------------------------------------------------ decode
// A sub-block's words are staged through its wave's LDS ring of kRing 16-bit units,
// refilled 256 units at a time (two coalesced dword loads per lane) so that a step
// reads its words from LDS instead of waiting on a dependent global load.
constexpr uint32_t kRing = 512;
constexpr uint32_t kRefill = 256;

// Stage units [filled, ...) of the word region into the ring until `want` units
// (or all) are staged; each pass stages 256 units, two dwords per lane.
__device__ __forceinline__ void ring_fill(uint16_t* ring, const uint32_t* region, uint32_t units, uint32_t& filled,
                                          uint32_t want, uint32_t lane) {
  if (filled >= want || filled >= units) return;
  do {
    const uint32_t u = filled + 4u * lane;
    uint32_t w0 = 0, w1 = 0;
    if (u < units) w0 = gld(region + u / 2);
    if (u + 2 < units) w1 = gld(region + u / 2 + 1);
    uint32_t* rp = reinterpret_cast<uint32_t*>(ring + (u & (kRing - 1)));
    rp[0] = w0;
    rp[1] = w1;
    filled += kRefill;
  } while (filled < want && filled < units);
  wave_lds_fence();
}

// Steps 0..255 of one sub-block (block runs run0 .. run0 + 7); returns the final
// state.  Before each group of kGroup steps (at most 64 * kGroup words) the ring
// holds at least that many unread units.  A refill pass starts only while fewer
// than 64 * kGroup units are staged past q, and kRing >= 64 * kGroup + kRefill, so
// it overwrites only units below q.
constexpr uint32_t kGroup = 4;
static_assert(kRing >= kGroup * kLanes + kRefill, "ring too small for the refill policy");

// Decode table: slot -> symbol (bits 0..7), frequency - 1 (8..19) and the slot's
// offset in its symbol's range (20..31); a step is one LDS read off the state.
template <int W, bool FULL>
__device__ __forceinline__ uint32_t decode_runs(const uint32_t* region, uint32_t units, uint32_t& q,
                                                const uint32_t* slot_tab, uint16_t* ring, uint8_t* dst, uint64_t room,
                                                uint32_t nb, uint32_t run0, uint32_t lane, uint32_t x) {
  uint32_t filled = 0;
  for (uint32_t r = run0; r < run0 + kSubRuns; ++r) {
    uint32_t acc[W];
#pragma unroll
    for (int k = 0; k < W; ++k) acc[k] = 0;
    const uint32_t base = r * (kLanes * kRun) + lane * kRun;
#pragma unroll
    for (int g = 0; g < (int)(kRun / kGroup); ++g) {
      ring_fill(ring, region, units, filled, q + kGroup * kLanes, lane);
#pragma unroll
      for (int jj = 0; jj < (int)kGroup; ++jj) {
        const int j = g * (int)kGroup + jj;
        const bool valid = FULL || base + (uint32_t)j < nb;
        const uint32_t ent = slot_tab[x & (kM - 1u)];
        const uint32_t s = ent & 0xffu;
        uint32_t y = (((ent >> 8) & 0xfffu) + 1u) * (x >> kPB) + (ent >> 20);
        const bool need = valid && y < kStateL;
        const uint64_t mask = __ballot(need);
        if (need) y = (y << 16) | (uint32_t)ring[(q + rank_in(mask)) & (kRing - 1)];
        q += (uint32_t)__popcll(mask);
        if (valid) {
          x = y;
          const int bit = j * W, kk = bit >> 5, sh = bit & 31;
          acc[kk] |= s << sh;
          if (sh + W > 32) acc[kk + 1] |= s >> (32 - sh);
        }
      }
    }
    const uint64_t off = ((uint64_t)r * kLanes + lane) * (4u * W);
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint64_t at = off + 4u * k;
      if (at + 4 <= room) {
        gst(reinterpret_cast<uint32_t*>(dst + at), acc[k]);
      } else {
        for (int qq = 0; qq < 4; ++qq)
          if (at + qq < room) gst(dst + at + qq, (uint8_t)(acc[k] >> (8 * qq)));
      }
    }
  }
  return x;
}

template <int W>
__global__ __launch_bounds__(kBlockThreads) void rans_decode_kernel(const DecBatch bt, int32_t* __restrict__ err) {
  using G = RansGeo<W>;
  __shared__ uint32_t slot_tab[kM];
  __shared__ uint32_t sym_fc[G::A];
  __shared__ uint32_t red[kSubs];
  __shared__ __align__(16) uint16_t rings[kSubs][kRing];

  const uint32_t lane = lane_id(), wave = threadIdx.x / kLanes, t = threadIdx.x;
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint64_t b = blockIdx.x - bt.first[jb];
  const uint8_t* in = bt.in[jb];
  const uint64_t in_bytes = bt.in_bytes[jb];
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  const uint32_t* h = reinterpret_cast<const uint32_t*>(in);
  const uint64_t head = 32u + 8ull * nblk;
  // Every check below is uniform over the workgroup (it reads the same bytes).  The
  // buffer must hold the header and offset table before any of it is read, and the
  // stated payload is compared with what is left of the buffer (never head + payload,
  // which a payload near 2^64 would wrap).
  if (in_bytes < head || gld(h) != kRansMagic ||
      gld(h + 1) != (2u | ((uint32_t)W << 8) | (kPB << 16) | (8u << 24)) || gld(h + 2) != kBlock ||
      gld(h + 3) != nblk || gld(reinterpret_cast<const uint64_t*>(in + 16)) != n ||
      gld(reinterpret_cast<const uint64_t*>(in + 24)) > in_bytes - head) {
    if (t == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    return;
  }
  const uint64_t payload = gld(reinterpret_cast<const uint64_t*>(in + 24));
  const uint64_t* offs = reinterpret_cast<const uint64_t*>(in + 32);
  const uint64_t o = gld(offs + b);
  const uint64_t e = b + 1 == nblk ? payload : gld(offs + b + 1);
  if (o > e || e > payload || e - o < 4 || (o & 3u)) {
    if (t == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    return;
  }
  const uint8_t* blk = in + head + o;
  const uint32_t tag = gld(reinterpret_cast<const uint32_t*>(blk));
  const uint64_t first = b * kBlock;
  const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
  const uint64_t out_bytes = (n * W + 7) / 8;
  uint8_t* dst = bt.out[jb] + first * W / 8;
  const uint64_t room = out_bytes - first * W / 8;

  if (tag & 1u) {
    const uint64_t rb = ((uint64_t)nb * W + 7) / 8;
    if (e - o != 4u + pad4(rb)) {
      if (t == 0) atomicOr(err, KVMI_ERR_CORRUPT);
      return;
    }
    const uint32_t* src = reinterpret_cast<const uint32_t*>(blk + 4);
    for (uint64_t i = t; i < pad4(rb) / 4; i += kBlockThreads) {
      const uint32_t v = gld(src + i);
      if (4 * i + 4 <= room) {
        gst(reinterpret_cast<uint32_t*>(dst) + i, v);
      } else {
        for (int k = 0; k < 4; ++k)
          if (4 * i + k < room) gst(dst + 4 * i + k, (uint8_t)(v >> (8 * k)));
      }
    }
    return;
  }
  uint32_t count[kSubs];
  uint64_t size = G::kHead;
#pragma unroll
  for (uint32_t j = 0; j < kSubs; ++j) {
    count[j] = j ? gld(reinterpret_cast<const uint32_t*>(blk + G::kCounts) + (j - 1)) : tag >> 1;
    size += pad4(2ull * count[j]);
  }
  if (e - o != size) {
    if (t == 0) atomicOr(err, KVMI_ERR_CORRUPT);
    return;
  }
  const uint16_t* ftab = reinterpret_cast<const uint16_t*>(blk + 4);
  const uint32_t fv = t < G::A ? gld(ftab + t) : 0u;
  if (block_sum(fv, red) != kM) {
    if (t == 0) atomicOr(err, KVMI_ERR_CORRUPT);
    return;
  }
  const uint32_t cum = block_exclusive_scan(fv, red);
  if (t < G::A) sym_fc[t] = fv | (cum << 13);
  __syncthreads();
  // slot -> (symbol, frequency, offset): thread i fills slots [16 i, 16 i + 16),
  // walking the cumulative table
  {
    constexpr uint32_t kPer = kM / kBlockThreads;
    const uint32_t s0 = t * kPer;
    // the symbol of slot s is the last v with cum_v <= s (cum is non-decreasing, and
    // an absent symbol shares its cum with the next one, so it is never the last)
    uint32_t lo = 0, hi = G::A - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) / 2;
      if ((sym_fc[mid] >> 13) <= s0) lo = mid;
      else hi = mid - 1;
    }
    uint32_t v = lo;
    uint32_t end = (sym_fc[v] >> 13) + (sym_fc[v] & 0x1fffu);
    for (uint32_t s = s0; s < s0 + kPer; ++s) {
      while (s >= end) {
        ++v;
        end = (sym_fc[v] >> 13) + (sym_fc[v] & 0x1fffu);
      }
      const uint32_t fv = sym_fc[v] & 0x1fffu, cum = sym_fc[v] >> 13;
      slot_tab[s] = v | ((fv - 1u) << 8) | ((s - cum) << 20);
    }
  }
  __syncthreads();

  // sub-block `wave`: its states, and its word region (pad4(2 count) bytes, the words
  // at its end; q counts 16-bit units from the region start)
  uint32_t x = gld(reinterpret_cast<const uint32_t*>(blk + G::kStates) + wave * kLanes + lane);
  uint64_t region_off = G::kHead;
#pragma unroll
  for (uint32_t j = 0; j < kSubs; ++j)
    if (j < wave) region_off += pad4(2ull * count[j]);
  const uint32_t cw = count[0] * (wave == 0) + count[1] * (wave == 1) + count[2] * (wave == 2) + count[3] * (wave == 3);
  const uint32_t* region = reinterpret_cast<const uint32_t*>(blk + region_off);
  const uint32_t units = (uint32_t)(pad4(2ull * cw) / 2);
  uint32_t q = units - cw;
  const uint32_t run0 = wave * kSubRuns;
  uint16_t* ring = rings[wave];
  if ((wave + 1) * kSub <= nb) x = decode_runs<W, true>(region, units, q, slot_tab, ring, dst, room, nb, run0, lane, x);
  else x = decode_runs<W, false>(region, units, q, slot_tab, ring, dst, room, nb, run0, lane, x);
  // a stream that is not this block's own encoding ends off its start state or
  // off the end of its words (ring reads are masked, so none leaves the ring)
  const bool ok = q == units && x == kStateL;
  if (__ballot(!ok) && lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
}

template <int W>
int rans_encode_w(const EncBatch& bt, hipStream_t stream) {
  const uint32_t total = bt.first[bt.count];
  // streams with no block (n = 0) get their header from the scan kernel
  bool fused = true;
  for (int i = 0; i < bt.count; ++i) {
    const uint32_t nblk = bt.first[i + 1] - bt.first[i];
    fused = fused && nblk >= 1 && nblk <= kFusedScanBlocks;
  }
  if (total) hipLaunchKernelGGL(rans_encode_kernel<W>, dim3(total), dim3(kBlockThreads), 0, stream, bt);
  if (fused) {
    hipLaunchKernelGGL((rans_compact_kernel<W, true>), dim3(total), dim3(kCopyThreads), 0, stream, bt);
  } else {
    hipLaunchKernelGGL(rans_scan_kernel<W>, dim3(bt.count), dim3(kScanThreads), 0, stream, bt);
    if (total) hipLaunchKernelGGL((rans_compact_kernel<W, false>), dim3(total), dim3(kCopyThreads), 0, stream, bt);
  }
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

template <int W>
int rans_decode_w(const DecBatch& bt, int32_t* err, hipStream_t stream) {
  const uint32_t total = bt.first[bt.count];
  if (total) hipLaunchKernelGGL(rans_decode_kernel<W>, dim3(total), dim3(kBlockThreads), 0, stream, bt, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

uint64_t slot_bytes(int w) {
  const uint64_t head = 4u + pad4(2u << w) + 4u * (kSubs - 1u) + 4u * kLanes * kSubs;
  return head + kSubs * (2u * kLanes * kRun + (uint64_t)kSub * w / 8);
}

}  // namespace
}  // namespace kvmi

using namespace kvmi;

extern "C" int64_t kvmi_rans_max_bytes(int64_t n, int32_t bits) {
  if (n < 0 || bits < 1 || bits > 8) return KVMI_EINVAL;
  const uint64_t nblk = ((uint64_t)n + kBlock - 1) / kBlock;
  uint64_t total = 32u + 8u * nblk;
  if (nblk) total += (nblk - 1) * (4u + (uint64_t)kBlock * bits / 8);
  if (nblk) total += 4u + pad4((((uint64_t)n - (nblk - 1) * kBlock) * bits + 7) / 8);
  return (int64_t)total;
}

extern "C" int64_t kvmi_rans_scratch_bytes(int64_t n, int32_t bits) {
  if (n < 0 || bits < 1 || bits > 8) return KVMI_EINVAL;
  const uint64_t nblk = ((uint64_t)n + kBlock - 1) / kBlock;
  return (int64_t)(nblk * slot_bytes(bits) + 4u * nblk);
}

static bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) != 0; }

extern "C" int kvmi_rans_encode_batch(const kvmi_rans_enc_job* jobs, int32_t num_jobs, int32_t bits,
                                      kvmi_stream_t stream) {
  if (num_jobs < 0 || bits < 1 || bits > 8 || (num_jobs > 0 && !jobs)) return KVMI_EINVAL;
  for (int32_t i = 0; i < num_jobs; ++i) {
    const kvmi_rans_enc_job& j = jobs[i];
    if (j.n < 0 || !j.out || !j.out_len || (j.n > 0 && (!j.packed || !j.scratch))) return KVMI_EINVAL;
    if (j.out_capacity < kvmi_rans_max_bytes(j.n, bits) || j.scratch_bytes < kvmi_rans_scratch_bytes(j.n, bits))
      return KVMI_EINVAL;
    if (misaligned(j.packed) || misaligned(j.out) || misaligned(j.scratch) || misaligned(j.out_len))
      return KVMI_EINVAL;
    if ((uint64_t)j.n > (uint64_t)kBlock * 0x7fffffffull) return KVMI_EINVAL;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int32_t base = 0; base < num_jobs; base += kMaxJobs) {
    EncBatch bt{};
    bt.count = min(kMaxJobs, num_jobs - base);
    uint64_t total = 0;
    for (int i = 0; i < bt.count; ++i) {
      const kvmi_rans_enc_job& j = jobs[base + i];
      const uint64_t nblk = ((uint64_t)j.n + kBlock - 1) / kBlock;
      bt.packed[i] = j.packed;
      bt.out[i] = j.out;
      bt.slots[i] = static_cast<uint8_t*>(j.scratch);
      bt.sizes[i] = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(j.scratch) + nblk * slot_bytes(bits));
      bt.out_len[i] = j.out_len;
      bt.n[i] = (uint64_t)j.n;
      bt.first[i] = (uint32_t)total;
      total += nblk;
    }
    if (total > 0x7fffffffull) return KVMI_EINVAL;
    bt.first[bt.count] = (uint32_t)total;
    int rc;
    switch (bits) {
      case 1: rc = rans_encode_w<1>(bt, s); break;
      case 2: rc = rans_encode_w<2>(bt, s); break;
      case 3: rc = rans_encode_w<3>(bt, s); break;
      case 4: rc = rans_encode_w<4>(bt, s); break;
      case 5: rc = rans_encode_w<5>(bt, s); break;
      case 6: rc = rans_encode_w<6>(bt, s); break;
      case 7: rc = rans_encode_w<7>(bt, s); break;
      default: rc = rans_encode_w<8>(bt, s); break;
    }
    if (rc != KVMI_OK) return rc;
  }
  return KVMI_OK;
}

extern "C" int kvmi_rans_decode_batch(const kvmi_rans_dec_job* jobs, int32_t num_jobs, int32_t bits, int32_t* err,
                                      kvmi_stream_t stream) {
  if (num_jobs < 0 || bits < 1 || bits > 8 || !err || (num_jobs > 0 && !jobs)) return KVMI_EINVAL;
  for (int32_t i = 0; i < num_jobs; ++i) {
    const kvmi_rans_dec_job& j = jobs[i];
    if (j.n < 0 || !j.stream || (j.n > 0 && !j.packed_out) || j.in_bytes < 32) return KVMI_EINVAL;
    if (misaligned(j.stream) || misaligned(j.packed_out)) return KVMI_EINVAL;
    if ((uint64_t)j.n > (uint64_t)kBlock * 0x7fffffffull) return KVMI_EINVAL;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int32_t base = 0; base < num_jobs; base += kMaxJobs) {
    DecBatch bt{};
    bt.count = min(kMaxJobs, num_jobs - base);
    uint64_t total = 0;
    for (int i = 0; i < bt.count; ++i) {
      const kvmi_rans_dec_job& j = jobs[base + i];
      bt.in[i] = j.stream;
      bt.out[i] = j.packed_out;
      bt.in_bytes[i] = (uint64_t)j.in_bytes;
      bt.n[i] = (uint64_t)j.n;
      bt.first[i] = (uint32_t)total;
      total += ((uint64_t)j.n + kBlock - 1) / kBlock;
    }
    if (total > 0x7fffffffull) return KVMI_EINVAL;
    bt.first[bt.count] = (uint32_t)total;
    int rc;
    switch (bits) {
      case 1: rc = rans_decode_w<1>(bt, err, s); break;
      case 2: rc = rans_decode_w<2>(bt, err, s); break;
      case 3: rc = rans_decode_w<3>(bt, err, s); break;
      case 4: rc = rans_decode_w<4>(bt, err, s); break;
      case 5: rc = rans_decode_w<5>(bt, err, s); break;
      case 6: rc = rans_decode_w<6>(bt, err, s); break;
      case 7: rc = rans_decode_w<7>(bt, err, s); break;
      default: rc = rans_decode_w<8>(bt, err, s); break;
    }
    if (rc != KVMI_OK) return rc;
  }
  return KVMI_OK;
}

extern "C" int kvmi_rans_encode(const uint8_t* packed, int64_t n, int32_t bits, uint8_t* out, int64_t out_capacity,
                                void* scratch, int64_t scratch_bytes, uint64_t* out_len, kvmi_stream_t stream) {
  const kvmi_rans_enc_job j{packed, n, out, out_capacity, scratch, scratch_bytes, out_len};
  return kvmi_rans_encode_batch(&j, 1, bits, stream);
}

extern "C" int kvmi_rans_decode(const uint8_t* stream_in, int64_t in_bytes, int64_t n, int32_t bits,
                                uint8_t* packed_out, int32_t* err, kvmi_stream_t stream) {
  const kvmi_rans_dec_job j{stream_in, in_bytes, n, packed_out};
  return kvmi_rans_decode_batch(&j, 1, bits, err, stream);
}
