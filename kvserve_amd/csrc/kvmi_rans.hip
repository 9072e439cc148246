// rANS entropy codec for the codec stage (the place KVServe fills with nvCOMP ANS,
// kvserve_v1/compression/codec/kvserve_codec.py:57-64).  nvCOMP's stream format is
// closed, so this codec has its own; oracle/rans.c states it byte for byte and the
// parity tests compare the two.
//
// Input: n symbols of W bits packed LSB-first (the bitpack body).  The stream is a
// 32-byte header, a u64 offset per block, then the blocks.  A block covers 65536
// symbols: 64 interleaved 32-bit rANS states, one per lane of the wave that codes
// it, lane i taking block symbol (t/32)*2048 + i*32 + t%32 at step t (t < 1024).
// Each block carries its own 12-bit frequency table (K and V, layers and heads have
// different statistics), renormalises in 16-bit words and is stored raw when coding
// would not make it smaller.
//
// Kernels (one wave per block):
//   rans_encode_kernel   histogram -> table -> encode (steps 1023..0) into a
//                        per-block slot of a scratch buffer, block size out
//   rans_scan_kernel     one workgroup: header and exclusive offsets of the blocks
//   rans_compact_kernel  copies each block from its slot (or the raw input) to its
//                        offset in the stream
//   rans_decode_kernel   table -> decode (steps 0..1023) -> packed symbols
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
constexpr uint32_t kSteps = 1024;
constexpr uint32_t kRuns = kSteps / kRun;
constexpr uint32_t kBlock = kLanes * kSteps;
constexpr uint32_t kStateL = 1u << 16;
constexpr int kScanThreads = 1024;
constexpr int kCopyThreads = 256;

__host__ __device__ constexpr uint64_t pad4(uint64_t b) { return (b + 3u) & ~(uint64_t)3u; }

template <int W>
struct RansGeo {
  static constexpr uint32_t A = 1u << W;
  static constexpr uint32_t kTab = (uint32_t)pad4(2u * A);       // u16 frequency table
  static constexpr uint32_t kHead = 4u + kTab + 4u * kLanes;     // tag, table, states
  static constexpr uint32_t kRawCap = kBlock * W / 8;            // packed bytes of a full block
  static constexpr uint32_t kGuard = 2u * kLanes * kRun;         // one run of words past the capacity
  static constexpr uint32_t kSlot = kHead + kGuard + kRawCap;    // scratch bytes per block
  static constexpr uint32_t kPerLane = A > kLanes ? A / kLanes : 1;
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
// Steps 1023..0 of one block (FULL: every lane has a symbol at every step).  Leaves
// pos < 0 when the words outgrow the capacity (the block is then stored raw).
template <int W, bool FULL>
__device__ __forceinline__ void encode_runs(const uint8_t* blk, uint64_t avail, uint32_t lane, uint32_t nb,
                                            const uint2* tab, uint16_t* words, int32_t& pos, uint32_t& x) {
  uint32_t d[W], dn[W];
  load_run<W>(blk, avail, kRuns - 1, lane, d);
  for (int r = (int)kRuns - 1; r >= 0; --r) {
    if (r > 0) load_run<W>(blk, avail, (uint32_t)r - 1, lane, dn);  // next run in flight
#pragma unroll
    for (int j = (int)kRun - 1; j >= 0; --j) {
      const uint32_t s = sym_at<W>(d, j);
      const bool valid = FULL || (uint32_t)r * (kLanes * kRun) + lane * kRun + (uint32_t)j < nb;
      const uint2 e = tab[s];
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
    if (pos < 0) return;
#pragma unroll
    for (int k = 0; k < W; ++k) d[k] = dn[k];
  }
}

template <int W>
__global__ __launch_bounds__(64) void rans_encode_kernel(const EncBatch bt) {
  using G = RansGeo<W>;
  constexpr bool kPrivate = W <= 5;  // lane-private histogram columns (no LDS contention)
  __shared__ __align__(16) uint32_t hist[kPrivate ? G::A * kLanes : G::A];
  __shared__ uint32_t fq[G::A];
  __shared__ uint2 tab[G::A];

  const uint32_t lane = lane_id();
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint64_t b = blockIdx.x - bt.first[jb];
  const uint64_t first = b * kBlock;
  const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
  const bool full = nb == kBlock;
  const uint64_t in_bytes = (n * W + 7) / 8;
  const uint8_t* blk = bt.packed[jb] + first * W / 8;
  const uint64_t avail = in_bytes - first * W / 8;
  uint8_t* slot = bt.slots[jb] + b * G::kSlot;

  for (uint32_t i = lane; i < (kPrivate ? G::A * kLanes : G::A); i += kLanes) hist[i] = 0;
  __syncthreads();
  {
    uint32_t d[W], dn[W];
    load_run<W>(blk, avail, 0, lane, d);
    for (uint32_t r = 0; r < kRuns; ++r) {
      if (r + 1 < kRuns) load_run<W>(blk, avail, r + 1, lane, dn);  // next run in flight
#pragma unroll
      for (int j = 0; j < (int)kRun; ++j) {
        const uint32_t s = sym_at<W>(d, j);
        if (full || r * (kLanes * kRun) + lane * kRun + j < nb)
          atomicAdd(&hist[kPrivate ? s * kLanes + lane : s], 1u);
      }
#pragma unroll
      for (int k = 0; k < W; ++k) d[k] = dn[k];
    }
  }
  __syncthreads();

  // counts c[v] for v = lane + 64 m
  uint32_t c[G::kPerLane];
#pragma unroll
  for (uint32_t m = 0; m < G::kPerLane; ++m) {
    const uint32_t v = lane + kLanes * m;
    uint32_t sum = 0;
    if (v < G::A) {
      if (kPrivate) {
        const uint4* row = reinterpret_cast<const uint4*>(&hist[v * kLanes]);
        for (int q = 0; q < (int)kLanes / 4; ++q) {
          const uint4 h = row[q];
          sum += h.x + h.y + h.z + h.w;
        }
      } else {
        sum = hist[v];
      }
    }
    c[m] = sum;
  }
  uint32_t present = 0, key = 0;
#pragma unroll
  for (uint32_t m = 0; m < G::kPerLane; ++m) {
    const uint32_t v = lane + kLanes * m;
    present += c[m] ? 1u : 0u;
    if (v < G::A) key = max(key, (c[m] << 8) | (255u - v));  // most frequent, lowest value on ties
  }
  const uint32_t K = wave_sum(present);
  const uint32_t top = 255u - (wave_max(key) & 255u);
  uint32_t f[G::kPerLane], fsum = 0;
#pragma unroll
  for (uint32_t m = 0; m < G::kPerLane; ++m) {
    f[m] = c[m] ? 1u + c[m] * (kM - K) / nb : 0u;
    fsum += f[m];
  }
  fsum = wave_sum(fsum);
#pragma unroll
  for (uint32_t m = 0; m < G::kPerLane; ++m) {
    const uint32_t v = lane + kLanes * m;
    if (v == top) f[m] += kM - fsum;
    if (v < G::A) {
      fq[v] = f[m];
      gst16(reinterpret_cast<uint16_t*>(slot + 4) + v, f[m]);
    }
  }
  __syncthreads();
#pragma unroll
  for (uint32_t m = 0; m < G::kPerLane; ++m) {
    const uint32_t v = lane + kLanes * m;
    if (v < G::A) {
      uint32_t cum = 0;
      for (uint32_t u = 0; u < v; ++u) cum += fq[u];
      const uint32_t fv = f[m];
      const uint32_t l = fv <= 1u ? 0u : 32u - __clz(fv - 1u);
      const uint32_t mul = fv ? (uint32_t)((((uint64_t)((1u << l) - fv)) << 32) / fv + 1u) : 0u;
      const uint32_t sh1 = l ? 1u : 0u, sh2 = l ? l - 1u : 0u;
      tab[v] = make_uint2(fv | (cum << 13) | (sh1 << 25) | (sh2 << 26), mul);
    }
  }
  __syncthreads();

  // encode, steps 1023..0; words fill the slot's word region from its end.  The
  // capacity is checked once per run: a run emits at most 64 * 32 words, which the
  // guard region in front of the word region absorbs.
  uint16_t* words = reinterpret_cast<uint16_t*>(slot + G::kHead + G::kGuard);
  int32_t pos = (int32_t)(G::kRawCap / 2);
  uint32_t x = kStateL;
  if (full) encode_runs<W, true>(blk, avail, lane, nb, tab, words, pos, x);
  else encode_runs<W, false>(blk, avail, lane, nb, tab, words, pos, x);
  const bool over = pos < 0;
  const uint32_t count = G::kRawCap / 2 - (uint32_t)pos;
  const uint64_t raw = 4u + pad4(((uint64_t)nb * W + 7) / 8);
  const uint64_t size = G::kHead + pad4(2ull * count);
  uint32_t* sizes = bt.sizes[jb];
  if (over || size >= raw) {
    if (lane == 0) {
      gst(reinterpret_cast<uint32_t*>(slot), 1u);
      gst(sizes + b, (uint32_t)raw);
    }
    return;
  }
  gst(reinterpret_cast<uint32_t*>(slot + 4 + G::kTab) + lane, x);
  if (lane == 0) {
    gst(reinterpret_cast<uint32_t*>(slot), count << 1);
    if (count & 1u) gst16(words + pos - 1, 0u);
    gst(sizes + b, (uint32_t)size);
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
    gst(h + 1, 1u | ((uint32_t)W << 8) | (kPB << 16) | (6u << 24));
    gst(h + 2, kBlock);
    gst(h + 3, nblk);
    gst(reinterpret_cast<uint64_t*>(out + 16), n);
    gst(reinterpret_cast<uint64_t*>(out + 24), payload);
    gst(bt.out_len[jb], (uint64_t)(32u + 8ull * nblk + payload));
  }
}

// ------------------------------------------------------------------ compaction
template <int W>
__global__ __launch_bounds__(kCopyThreads) void rans_compact_kernel(const EncBatch bt) {
  using G = RansGeo<W>;
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  const uint64_t b = blockIdx.x - bt.first[jb];
  uint8_t* out = bt.out[jb];
  const uint64_t off = gld(reinterpret_cast<const uint64_t*>(out + 32) + b);
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
  const uint32_t count = tag >> 1;
  const uint32_t wbytes = (uint32_t)pad4(2ull * count);
  const uint32_t* head = reinterpret_cast<const uint32_t*>(slot);
  for (uint32_t i = t; i < G::kHead / 4; i += kCopyThreads) gst(dst + i, gld(head + i));
  const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(slot + G::kSlot - wbytes);
  for (uint32_t i = t; i < wbytes / 4; i += kCopyThreads) gst(dst + G::kHead / 4 + i, gld(wsrc + i));
}

// ------------------------------------------------------------------ decode
// The block's words are staged through a per-wave LDS ring of kRing 16-bit units,
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
  __syncthreads();
}

// Steps 0..1023 of one block; returns the final state.  Before each group of
// kGroup steps (at most 64 * kGroup words) the ring holds at least that many
// unread units.  A refill pass starts only while fewer than 64 * kGroup units are
// staged past q, and kRing >= 64 * kGroup + kRefill, so it overwrites only units
// below q.
constexpr uint32_t kGroup = 4;
static_assert(kRing >= kGroup * kLanes + kRefill, "ring too small for the refill policy");

template <int W, bool FULL>
__device__ __forceinline__ uint32_t decode_runs(const uint32_t* region, uint32_t units, uint32_t& q,
                                                const uint8_t* slot_sym, const uint32_t* sym_fc, uint16_t* ring,
                                                uint8_t* dst, uint64_t room, uint32_t nb, uint32_t lane, uint32_t x) {
  uint32_t filled = 0;
  for (uint32_t r = 0; r < kRuns; ++r) {
    uint32_t acc[W];
#pragma unroll
    for (int k = 0; k < W; ++k) acc[k] = 0;
#pragma unroll
    for (int g = 0; g < (int)(kRun / kGroup); ++g) {
      ring_fill(ring, region, units, filled, q + kGroup * kLanes, lane);
#pragma unroll
      for (int jj = 0; jj < (int)kGroup; ++jj) {
        const int j = g * (int)kGroup + jj;
        const bool valid = FULL || r * (kLanes * kRun) + lane * kRun + (uint32_t)j < nb;
        const uint32_t slot = x & (kM - 1u);
        const uint32_t s = slot_sym[slot];
        const uint32_t fc = sym_fc[s];
        uint32_t y = (fc & 0x1fffu) * (x >> kPB) + slot - (fc >> 13);
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
__global__ __launch_bounds__(64) void rans_decode_kernel(const DecBatch bt, int32_t* __restrict__ err) {
  using G = RansGeo<W>;
  __shared__ uint8_t slot_sym[kM];
  __shared__ uint32_t sym_fc[G::A];
  __shared__ uint32_t fq[G::A];
  __shared__ __align__(16) uint16_t ring[kRing];

  const uint32_t lane = lane_id();
  const int jb = job_of(bt, blockIdx.x);
  const uint64_t n = bt.n[jb];
  const uint64_t b = blockIdx.x - bt.first[jb];
  const uint8_t* in = bt.in[jb];
  const uint64_t in_bytes = bt.in_bytes[jb];
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  const uint32_t* h = reinterpret_cast<const uint32_t*>(in);
  const uint64_t payload = gld(reinterpret_cast<const uint64_t*>(in + 24));
  const uint64_t head = 32u + 8ull * nblk;
  if (gld(h) != kRansMagic || gld(h + 1) != (1u | ((uint32_t)W << 8) | (kPB << 16) | (6u << 24)) ||
      gld(h + 2) != kBlock || gld(h + 3) != nblk || gld(reinterpret_cast<const uint64_t*>(in + 16)) != n ||
      in_bytes != head + payload) {
    if (lane == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
    return;
  }
  const uint64_t* offs = reinterpret_cast<const uint64_t*>(in + 32);
  const uint64_t o = gld(offs + b);
  const uint64_t e = b + 1 == nblk ? payload : gld(offs + b + 1);
  if (o > e || e > payload || e - o < 4 || (o & 3u)) {
    if (lane == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
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
      if (lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
      return;
    }
    const uint32_t* src = reinterpret_cast<const uint32_t*>(blk + 4);
    for (uint64_t i = lane; i < pad4(rb) / 4; i += kLanes) {
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
  const uint32_t count = tag >> 1;
  if (e - o != G::kHead + pad4(2ull * count)) {
    if (lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
    return;
  }
  const uint16_t* ftab = reinterpret_cast<const uint16_t*>(blk + 4);
  uint32_t fsum = 0;
  for (uint32_t v = lane; v < G::A; v += kLanes) {
    const uint32_t fv = gld(ftab + v);
    fq[v] = fv;
    fsum += fv;
  }
  if (wave_sum(fsum) != kM) {
    if (lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
    return;
  }
  __syncthreads();
  for (uint32_t v = lane; v < G::A; v += kLanes) {
    uint32_t cum = 0;
    for (uint32_t u = 0; u < v; ++u) cum += fq[u];
    sym_fc[v] = fq[v] | (cum << 13);
  }
  __syncthreads();
  // slot -> symbol: lane i fills slots [64 i, 64 i + 64), walking the cumulative table
  {
    const uint32_t s0 = lane * (kM / kLanes);
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
    for (uint32_t s = s0; s < s0 + kM / kLanes; ++s) {
      while (s >= end) {
        ++v;
        end = (sym_fc[v] >> 13) + (sym_fc[v] & 0x1fffu);
      }
      slot_sym[s] = (uint8_t)v;
    }
  }

  uint32_t x = gld(reinterpret_cast<const uint32_t*>(blk + 4 + G::kTab) + lane);
  // word region: pad4(2 count) bytes, the words at its end; q counts 16-bit units
  // from the region start, word p of the block is unit q = lead + p
  const uint32_t* region = reinterpret_cast<const uint32_t*>(blk + G::kHead);
  const uint32_t units = (uint32_t)(pad4(2ull * count) / 2);
  uint32_t q = units - count;
  __syncthreads();
  if (nb == kBlock) x = decode_runs<W, true>(region, units, q, slot_sym, sym_fc, ring, dst, room, nb, lane, x);
  else x = decode_runs<W, false>(region, units, q, slot_sym, sym_fc, ring, dst, room, nb, lane, x);
  // a stream that is not this block's own encoding ends off its start state or
  // off the end of its words (ring reads are masked, so none leaves the ring)
  const bool ok = q == units && x == kStateL;
  if (__ballot(!ok) && lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
}

template <int W>
int rans_encode_w(const EncBatch& bt, hipStream_t stream) {
  const uint32_t total = bt.first[bt.count];
  if (total) hipLaunchKernelGGL(rans_encode_kernel<W>, dim3(total), dim3(64), 0, stream, bt);
  hipLaunchKernelGGL(rans_scan_kernel<W>, dim3(bt.count), dim3(kScanThreads), 0, stream, bt);
  if (total) hipLaunchKernelGGL(rans_compact_kernel<W>, dim3(total), dim3(kCopyThreads), 0, stream, bt);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

template <int W>
int rans_decode_w(const DecBatch& bt, int32_t* err, hipStream_t stream) {
  const uint32_t total = bt.first[bt.count];
  if (total) hipLaunchKernelGGL(rans_decode_kernel<W>, dim3(total), dim3(64), 0, stream, bt, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

uint64_t slot_bytes(int w) {
  return 4u + pad4(2u << w) + 4u * kLanes + 2u * kLanes * kRun + (uint64_t)kBlock * w / 8;
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
