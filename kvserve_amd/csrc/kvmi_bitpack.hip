// Fixed-width LSB-first bit packing of uint8 symbols with KVServe's 16-byte header.
//
// Format (kvserve_v1/compression/codec/bitpack_codec.py:20-47):
//   bytes 0..3  magic 0x0150424B little-endian ("KBP", version 1)
//   byte  4     bits
//   bytes 5..7  zero
//   bytes 8..15 symbol count n, little-endian u64
//   payload     ceil(n*bits/8) bytes; bit b of symbol i is stream bit i*bits + b,
//               bytes filled LSB first; pad bits are zero.
//
// Work split: one thread owns 32 consecutive symbols, i.e. exactly 4*bits payload
// bytes, so no two threads share a byte; a workgroup's bytes are contiguous.
#include "kvmi_device.hpp"
#include "../../include/kvserve_amd.h"

namespace kvmi {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void write_header(uint8_t* out, int bits, uint64_t n) {
  uint32_t* o = reinterpret_cast<uint32_t*>(out);
  o[0] = KVMI_MAGIC;
  o[1] = (uint32_t)bits;
  o[2] = (uint32_t)(n & 0xffffffffu);
  o[3] = (uint32_t)(n >> 32);
}

__device__ __forceinline__ bool header_ok(const uint8_t* in, int bits, uint64_t n) {
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    h[i] = (uint32_t)in[4 * i] | ((uint32_t)in[4 * i + 1] << 8) | ((uint32_t)in[4 * i + 2] << 16) |
           ((uint32_t)in[4 * i + 3] << 24);
  return h[0] == KVMI_MAGIC && h[1] == (uint32_t)bits && h[2] == (uint32_t)(n & 0xffffffffu) &&
         h[3] == (uint32_t)(n >> 32);
}

// A workgroup's payload: kThreads chunks of 32 symbols, 4*BITS bytes each, contiguous
// in the stream.  On the encoder's VEC path (symbols and stream 16-byte aligned, the
// usual case for torch allocations) it passes through LDS, so that the stream is
// written lane-linear in 16-byte pieces (each store instruction writes 1 KiB of
// consecutive bytes) rather than as BITS dwords per lane at a 4*BITS-byte stride;
// otherwise bytes move one at a time.  The decoder reads its 4*BITS bytes per lane
// directly (reads do not depend on the lane stride here).
template <int BITS>
constexpr int wg_dwords() {
  return kThreads * BITS;
}

template <int BITS, bool VEC>
__global__ __launch_bounds__(kThreads) void bitpack_encode_kernel(const uint8_t* __restrict__ sym, int64_t n,
                                                                  uint8_t* __restrict__ out,
                                                                  int32_t* __restrict__ err) {
  __shared__ uint4 stage[wg_dwords<BITS>() / 4];
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // chunk of 32 symbols
  if (c == 0) write_header(out, BITS, (uint64_t)n);
  const int64_t s0 = c * 32;
  if (!VEC && s0 >= n) return;
  uint32_t s[32];
  if (VEC && s0 + 32 <= n) {
    const uint4* p = reinterpret_cast<const uint4*>(sym + s0);
    uint4 a = p[0], b = p[1];
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 32; ++j) s[j] = (w[j >> 2] >> ((j & 3) * 8)) & 0xffu;
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) s[j] = (s0 + j < n) ? (uint32_t)sym[s0 + j] : 0u;
  }
  uint32_t ov = 0;
#pragma unroll
  for (int j = 0; j < 32; ++j) ov |= s[j];
  if (ov >> BITS) atomicOr(err, KVMI_ERR_SYMBOL_RANGE);
  Packed<32, BITS> pk;
  pack_syms<32, BITS>(s, pk);
  const int64_t payload = (n * BITS + 7) / 8;
  if constexpr (VEC) {
    uint32_t* sw = reinterpret_cast<uint32_t*>(stage);
#pragma unroll
    for (int i = 0; i < BITS; ++i) sw[threadIdx.x * BITS + i] = pk.w[i];
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * (4 * wg_dwords<BITS>());  // payload bytes before this workgroup
    const int64_t rem = payload - base;                                   // bytes this workgroup writes
    uint8_t* dst = out + KVMI_HEADER_BYTES + base;
    for (int q = threadIdx.x; q < wg_dwords<BITS>() / 4; q += kThreads) {
      const int64_t off = 16 * (int64_t)q;
      if (off + 16 <= rem) {
        reinterpret_cast<uint4*>(dst)[q] = stage[q];
      } else if (off < rem) {  // the stream's last, partial 16 bytes
        const uint8_t* sb = reinterpret_cast<const uint8_t*>(stage);
        for (int64_t b = off; b < rem; ++b) dst[b] = sb[b];
      }
    }
  } else {
    uint8_t* dst = out + KVMI_HEADER_BYTES + c * (4 * BITS);
    const int64_t rem = payload - c * (4 * BITS);  // bytes this thread may write
    const int nb = rem < 4 * BITS ? (int)rem : 4 * BITS;
    for (int i = 0; i < nb; ++i) dst[i] = (uint8_t)(pk.w[i >> 2] >> ((i & 3) * 8));
  }
}

template <int BITS, bool VEC>
__global__ __launch_bounds__(kThreads) void bitpack_decode_kernel(const uint8_t* __restrict__ in, int64_t n,
                                                                  uint8_t* __restrict__ sym,
                                                                  int32_t* __restrict__ err) {
  __shared__ int ok;
  if (threadIdx.x == 0) {
    ok = header_ok(in, BITS, (uint64_t)n) ? 1 : 0;
    if (!ok && blockIdx.x == 0) atomicOr(err, KVMI_ERR_BAD_HEADER);
  }
  __syncthreads();
  if (!ok) return;
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t s0 = c * 32;
  if (s0 >= n) return;
  const uint8_t* src = in + KVMI_HEADER_BYTES + c * (4 * BITS);
  const int64_t payload = (n * BITS + 7) / 8;
  const int64_t rem = payload - c * (4 * BITS);
  Packed<32, BITS> pk;
  if (VEC && rem >= 4 * BITS) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
    for (int i = 0; i < BITS; ++i) pk.w[i] = p[i];
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) pk.w[i] = 0;
    const int nb = rem < 4 * BITS ? (int)rem : 4 * BITS;
    for (int i = 0; i < nb; ++i) pk.w[i >> 2] |= (uint32_t)src[i] << ((i & 3) * 8);
  }
  uint32_t s[32];
  unpack_syms<32, BITS>(pk, s);
  if (VEC && s0 + 32 <= n) {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = s[4 * i] | (s[4 * i + 1] << 8) | (s[4 * i + 2] << 16) | (s[4 * i + 3] << 24);
    uint4* d = reinterpret_cast<uint4*>(sym + s0);
    d[0] = make_uint4(w[0], w[1], w[2], w[3]);
    d[1] = make_uint4(w[4], w[5], w[6], w[7]);
  } else {
    for (int j = 0; j < 32; ++j)
      if (s0 + j < n) sym[s0 + j] = (uint8_t)s[j];
  }
}

template <int BITS>
int launch_encode(const uint8_t* sym, int64_t n, uint8_t* out, int32_t* err, hipStream_t st) {
  const int64_t chunks = (n + 31) / 32;
  const int64_t grid = chunks > 0 ? (chunks + kThreads - 1) / kThreads : 1;
  const bool vec = ((uintptr_t)sym % 16 == 0) && ((uintptr_t)out % 16 == 0);
  if (vec)
    hipLaunchKernelGGL((bitpack_encode_kernel<BITS, true>), dim3((unsigned)grid), dim3(kThreads), 0, st, sym, n, out, err);
  else
    hipLaunchKernelGGL((bitpack_encode_kernel<BITS, false>), dim3((unsigned)grid), dim3(kThreads), 0, st, sym, n, out, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

template <int BITS>
int launch_decode(const uint8_t* in, int64_t n, uint8_t* sym, int32_t* err, hipStream_t st) {
  const int64_t chunks = (n + 31) / 32;
  const int64_t grid = chunks > 0 ? (chunks + kThreads - 1) / kThreads : 1;
  const bool vec = ((uintptr_t)in % 4 == 0) && ((uintptr_t)sym % 16 == 0);
  if (vec)
    hipLaunchKernelGGL((bitpack_decode_kernel<BITS, true>), dim3((unsigned)grid), dim3(kThreads), 0, st, in, n, sym, err);
  else
    hipLaunchKernelGGL((bitpack_decode_kernel<BITS, false>), dim3((unsigned)grid), dim3(kThreads), 0, st, in, n, sym, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

}  // namespace
}  // namespace kvmi

extern "C" int kvmi_bitpack_encode(const uint8_t* sym, int64_t n, int32_t bits, uint8_t* out, int32_t* err,
                                   kvmi_stream_t stream) {
  using namespace kvmi;
  if (bits < 1 || bits > 8 || n < 0 || out == nullptr || err == nullptr || (n > 0 && sym == nullptr))
    return KVMI_EINVAL;
  if ((n + 31) / 32 > (int64_t)kThreads * 0x7fffffffLL) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (bits) {
    case 1: return launch_encode<1>(sym, n, out, err, st);
    case 2: return launch_encode<2>(sym, n, out, err, st);
    case 3: return launch_encode<3>(sym, n, out, err, st);
    case 4: return launch_encode<4>(sym, n, out, err, st);
    case 5: return launch_encode<5>(sym, n, out, err, st);
    case 6: return launch_encode<6>(sym, n, out, err, st);
    case 7: return launch_encode<7>(sym, n, out, err, st);
    default: return launch_encode<8>(sym, n, out, err, st);
  }
}

extern "C" int kvmi_bitpack_decode(const uint8_t* in, int64_t in_bytes, int64_t n, int32_t bits, uint8_t* sym,
                                   int32_t* err, kvmi_stream_t stream) {
  using namespace kvmi;
  if (bits < 1 || bits > 8 || n < 0 || in == nullptr || err == nullptr || (n > 0 && sym == nullptr))
    return KVMI_EINVAL;
  if (in_bytes != KVMI_HEADER_BYTES + (n * bits + 7) / 8) return KVMI_EINVAL;
  if ((n + 31) / 32 > (int64_t)kThreads * 0x7fffffffLL) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (bits) {
    case 1: return launch_decode<1>(in, n, sym, err, st);
    case 2: return launch_decode<2>(in, n, sym, err, st);
    case 3: return launch_decode<3>(in, n, sym, err, st);
    case 4: return launch_decode<4>(in, n, sym, err, st);
    case 5: return launch_decode<5>(in, n, sym, err, st);
    case 6: return launch_decode<6>(in, n, sym, err, st);
    case 7: return launch_decode<7>(in, n, sym, err, st);
    default: return launch_decode<8>(in, n, sym, err, st);
  }
}

extern "C" int kvmi_abi_version(void) { return KVMI_ABI_VERSION; }
