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
  static constexpr uint32_t kSlot = kHead + kRawCap;             // scratch bytes per block
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

// ------------------------------------------------------------------ encode
template <int W>
__global__ __launch_bounds__(64) void rans_encode_kernel(const uint8_t* __restrict__ in, uint64_t n,
                                                         uint8_t* __restrict__ slots,
                                                         uint32_t* __restrict__ sizes) {
  using G = RansGeo<W>;
  constexpr bool kPrivate = W <= 5;  // lane-private histogram columns (no LDS contention)
  __shared__ __align__(16) uint32_t hist[kPrivate ? G::A * kLanes : G::A];
  __shared__ uint32_t fq[G::A];
  __shared__ uint2 tab[G::A];

  const uint32_t lane = lane_id();
  const uint64_t b = blockIdx.x;
  const uint64_t first = b * kBlock;
  const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
  const bool full = nb == kBlock;
  const uint64_t in_bytes = (n * W + 7) / 8;
  const uint8_t* blk = in + first * W / 8;
  const uint64_t avail = in_bytes - first * W / 8;
  uint8_t* slot = slots + b * G::kSlot;

  for (uint32_t i = lane; i < (kPrivate ? G::A * kLanes : G::A); i += kLanes) hist[i] = 0;
  __syncthreads();
  for (uint32_t r = 0; r < kRuns; ++r) {
    uint32_t d[W];
    load_run<W>(blk, avail, r, lane, d);
#pragma unroll
    for (int j = 0; j < (int)kRun; ++j) {
      const uint32_t s = sym_at<W>(d, j);
      if (full || r * (kLanes * kRun) + lane * kRun + j < nb) atomicAdd(&hist[kPrivate ? s * kLanes + lane : s], 1u);
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

  // encode, steps 1023..0; words fill the slot's word region from its end
  uint16_t* words = reinterpret_cast<uint16_t*>(slot + G::kHead);
  int32_t pos = (int32_t)(G::kRawCap / 2);
  uint32_t x = kStateL;
  bool over = false;
  for (int r = (int)kRuns - 1; r >= 0 && !over; --r) {
    uint32_t d[W];
    load_run<W>(blk, avail, (uint32_t)r, lane, d);
#pragma unroll
    for (int j = (int)kRun - 1; j >= 0; --j) {
      const uint32_t s = sym_at<W>(d, j);
      const bool valid = full || (uint32_t)r * (kLanes * kRun) + lane * kRun + (uint32_t)j < nb;
      const uint2 e = tab[s];
      const uint32_t fs = e.x & 0x1fffu;
      const bool emit = valid && (x >> 20) >= fs;
      const uint64_t mask = __ballot(emit);
      pos -= (int32_t)__popcll(mask);
      if (pos < 0) {
        over = true;
        break;
      }
      if (emit) {
        gst16(words + pos + rank_in(mask), x & 0xffffu);
        x >>= 16;
      }
      if (valid) {
        const uint32_t t1 = __umulhi(e.y, x);
        const uint32_t q = (t1 + ((x - t1) >> ((e.x >> 25) & 1u))) >> (e.x >> 26);
        x = (q << kPB) + (x - q * fs) + ((e.x >> 13) & 0xfffu);
      }
    }
  }
  const uint32_t count = G::kRawCap / 2 - (uint32_t)pos;
  const uint64_t raw = 4u + pad4(((uint64_t)nb * W + 7) / 8);
  const uint64_t size = G::kHead + pad4(2ull * count);
  if (over || size >= raw) {
    if (lane == 0) {
      gst(reinterpret_cast<uint32_t*>(slot), 1u);
      sizes[b] = (uint32_t)raw;
    }
    return;
  }
  gst(reinterpret_cast<uint32_t*>(slot + 4 + G::kTab) + lane, x);
  if (lane == 0) {
    gst(reinterpret_cast<uint32_t*>(slot), count << 1);
    if (count & 1u) gst16(words + pos - 1, 0u);
    sizes[b] = (uint32_t)size;
  }
}

// ------------------------------------------------------------------ scan + header
__global__ __launch_bounds__(kScanThreads) void rans_scan_kernel(const uint32_t* __restrict__ sizes,
                                                                 uint32_t nblk, uint64_t n, int w,
                                                                 uint8_t* __restrict__ out,
                                                                 uint64_t* __restrict__ out_len) {
  __shared__ uint64_t part[kScanThreads];
  const uint32_t t = threadIdx.x;
  const uint32_t per = (nblk + kScanThreads - 1) / kScanThreads;
  const uint32_t lo = min(nblk, t * per), hi = min(nblk, lo + per);
  uint64_t s = 0;
  for (uint32_t i = lo; i < hi; ++i) s += sizes[i];
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
    off += sizes[i];
  }
  if (t == kScanThreads - 1) {
    const uint64_t payload = part[t];
    uint32_t* h = reinterpret_cast<uint32_t*>(out);
    gst(h + 0, kRansMagic);
    gst(h + 1, 1u | ((uint32_t)w << 8) | (kPB << 16) | (6u << 24));
    gst(h + 2, kBlock);
    gst(h + 3, nblk);
    gst(reinterpret_cast<uint64_t*>(out + 16), n);
    gst(reinterpret_cast<uint64_t*>(out + 24), payload);
    gst(out_len, (uint64_t)(32u + 8ull * nblk + payload));
  }
}

// ------------------------------------------------------------------ compaction
template <int W>
__global__ __launch_bounds__(kCopyThreads) void rans_compact_kernel(const uint8_t* __restrict__ in, uint64_t n,
                                                                    const uint8_t* __restrict__ slots,
                                                                    uint32_t nblk, uint8_t* __restrict__ out) {
  using G = RansGeo<W>;
  const uint64_t b = blockIdx.x;
  const uint64_t off = gld(reinterpret_cast<const uint64_t*>(out + 32) + b);
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + 32 + 8ull * nblk + off);
  const uint8_t* slot = slots + b * G::kSlot;
  const uint32_t tag = gld(reinterpret_cast<const uint32_t*>(slot));
  const uint32_t t = threadIdx.x;
  if (tag & 1u) {
    const uint64_t first = b * kBlock;
    const uint32_t nb = (uint32_t)min((uint64_t)kBlock, n - first);
    const uint64_t rb = ((uint64_t)nb * W + 7) / 8;
    const uint8_t* src = in + first * W / 8;
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
template <int W>
__global__ __launch_bounds__(64) void rans_decode_kernel(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                                         uint64_t n, uint8_t* __restrict__ out,
                                                         int32_t* __restrict__ err) {
  using G = RansGeo<W>;
  __shared__ uint8_t slot_sym[kM];
  __shared__ uint32_t sym_fc[G::A];
  __shared__ uint32_t fq[G::A];

  const uint32_t lane = lane_id();
  const uint64_t b = blockIdx.x;
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
  uint8_t* dst = out + first * W / 8;
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
  __syncthreads();

  uint32_t x = gld(reinterpret_cast<const uint32_t*>(blk + 4 + G::kTab) + lane);
  const uint16_t* words = reinterpret_cast<const uint16_t*>(blk + G::kHead + (pad4(2ull * count) - 2ull * count));
  uint32_t p = 0;
  bool bad = false;
  const bool full = nb == kBlock;
  for (uint32_t r = 0; r < kRuns; ++r) {
    uint32_t acc[W];
#pragma unroll
    for (int k = 0; k < W; ++k) acc[k] = 0;
#pragma unroll
    for (int j = 0; j < (int)kRun; ++j) {
      const bool valid = full || r * (kLanes * kRun) + lane * kRun + (uint32_t)j < nb;
      const uint32_t slot = x & (kM - 1u);
      const uint32_t s = slot_sym[slot];
      const uint32_t fc = sym_fc[s];
      uint32_t y = (fc & 0x1fffu) * (x >> kPB) + slot - (fc >> 13);
      const bool need = valid && y < kStateL;
      const uint64_t mask = __ballot(need);
      const uint32_t k = (uint32_t)__popcll(mask);
      if (p + k > count) {
        bad = true;
        break;
      }
      if (need) y = (y << 16) | (uint32_t)gld(words + p + rank_in(mask));
      p += k;
      if (valid) {
        x = y;
        const int bit = j * W, kk = bit >> 5, sh = bit & 31;
        acc[kk] |= s << sh;
        if (sh + W > 32) acc[kk + 1] |= s >> (32 - sh);
      }
    }
    if (bad) break;
    const uint64_t off = ((uint64_t)r * kLanes + lane) * (4u * W);
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint64_t at = off + 4u * k;
      if (at + 4 <= room) {
        gst(reinterpret_cast<uint32_t*>(dst + at), acc[k]);
      } else {
        for (int q = 0; q < 4; ++q)
          if (at + q < room) gst(dst + at + q, (uint8_t)(acc[k] >> (8 * q)));
      }
    }
  }
  const bool ok = !bad && p == count && x == kStateL;
  if (__ballot(!ok) && lane == 0) atomicOr(err, KVMI_ERR_CORRUPT);
}

template <int W>
int rans_encode_w(const uint8_t* in, int64_t n, uint8_t* out, void* scratch, uint64_t* out_len,
                  hipStream_t stream) {
  using G = RansGeo<W>;
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  uint8_t* slots = static_cast<uint8_t*>(scratch);
  uint32_t* sizes = reinterpret_cast<uint32_t*>(slots + (uint64_t)nblk * G::kSlot);
  if (nblk) hipLaunchKernelGGL(rans_encode_kernel<W>, dim3(nblk), dim3(64), 0, stream, in, (uint64_t)n, slots, sizes);
  hipLaunchKernelGGL(rans_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, sizes, nblk, (uint64_t)n, W, out,
                     out_len);
  if (nblk)
    hipLaunchKernelGGL(rans_compact_kernel<W>, dim3(nblk), dim3(kCopyThreads), 0, stream, in, (uint64_t)n, slots,
                       nblk, out);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

template <int W>
int rans_decode_w(const uint8_t* in, int64_t in_bytes, int64_t n, uint8_t* out, int32_t* err, hipStream_t stream) {
  const uint32_t nblk = (uint32_t)((n + kBlock - 1) / kBlock);
  if (nblk)
    hipLaunchKernelGGL(rans_decode_kernel<W>, dim3(nblk), dim3(64), 0, stream, in, (uint64_t)in_bytes, (uint64_t)n,
                       out, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

uint64_t slot_bytes(int w) { return 4u + pad4(2u << w) + 4u * kLanes + (uint64_t)kBlock * w / 8; }

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

extern "C" int kvmi_rans_encode(const uint8_t* packed, int64_t n, int32_t bits, uint8_t* out, int64_t out_capacity,
                                void* scratch, int64_t scratch_bytes, uint64_t* out_len, kvmi_stream_t stream) {
  if (n < 0 || bits < 1 || bits > 8 || !out || !out_len || (n > 0 && (!packed || !scratch))) return KVMI_EINVAL;
  if (out_capacity < kvmi_rans_max_bytes(n, bits) || scratch_bytes < kvmi_rans_scratch_bytes(n, bits))
    return KVMI_EINVAL;
  if ((reinterpret_cast<uintptr_t>(packed) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(scratch) | reinterpret_cast<uintptr_t>(out_len)) & 7u)
    return KVMI_EINVAL;
  if ((uint64_t)n > (uint64_t)kBlock * 0xffffffffull) return KVMI_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (bits) {
    case 1: return rans_encode_w<1>(packed, n, out, scratch, out_len, s);
    case 2: return rans_encode_w<2>(packed, n, out, scratch, out_len, s);
    case 3: return rans_encode_w<3>(packed, n, out, scratch, out_len, s);
    case 4: return rans_encode_w<4>(packed, n, out, scratch, out_len, s);
    case 5: return rans_encode_w<5>(packed, n, out, scratch, out_len, s);
    case 6: return rans_encode_w<6>(packed, n, out, scratch, out_len, s);
    case 7: return rans_encode_w<7>(packed, n, out, scratch, out_len, s);
    default: return rans_encode_w<8>(packed, n, out, scratch, out_len, s);
  }
}

extern "C" int kvmi_rans_decode(const uint8_t* stream_in, int64_t in_bytes, int64_t n, int32_t bits,
                                uint8_t* packed_out, int32_t* err, kvmi_stream_t stream) {
  if (n < 0 || bits < 1 || bits > 8 || !stream_in || !err || (n > 0 && !packed_out)) return KVMI_EINVAL;
  if ((reinterpret_cast<uintptr_t>(stream_in) | reinterpret_cast<uintptr_t>(packed_out)) & 7u) return KVMI_EINVAL;
  if (in_bytes < 32) return KVMI_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (bits) {
    case 1: return rans_decode_w<1>(stream_in, in_bytes, n, packed_out, err, s);
    case 2: return rans_decode_w<2>(stream_in, in_bytes, n, packed_out, err, s);
    case 3: return rans_decode_w<3>(stream_in, in_bytes, n, packed_out, err, s);
    case 4: return rans_decode_w<4>(stream_in, in_bytes, n, packed_out, err, s);
    case 5: return rans_decode_w<5>(stream_in, in_bytes, n, packed_out, err, s);
    case 6: return rans_decode_w<6>(stream_in, in_bytes, n, packed_out, err, s);
    case 7: return rans_decode_w<7>(stream_in, in_bytes, n, packed_out, err, s);
    default: return rans_decode_w<8>(stream_in, in_bytes, n, packed_out, err, s);
  }
}
