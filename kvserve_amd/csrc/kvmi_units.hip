// Unit kernels: paged block gather / scatter and the standalone random-sign
// Hadamard transform.  They serve the operator-level API (one stage at a time,
// as KVServe's CompressionManager calls its operators) and stage-by-stage parity
// checks; the fused path in kvmi_codec.hip does not use them.
#include "kvmi_common.hpp"

namespace kvmi {
namespace {

constexpr int kCopyThreads = 256;

// One workgroup copies one block of one part (both parts of a block at once for the
// [P, 2, ...] layout) in 16-byte vectors; the entry points require block sizes that
// are multiples of 16 bytes.
__global__ __launch_bounds__(kCopyThreads) void gather_kernel(const uint4* __restrict__ pool, int64_t part_stride16,
                                                              const int32_t* __restrict__ ids, int64_t blk16,
                                                              int32_t nblocks, uint4* __restrict__ out) {
  const int i = blockIdx.x, p = blockIdx.y;
  const uint4* src = pool + p * part_stride16 + (int64_t)ids[i] * blk16;
  uint4* dst = out + ((int64_t)p * nblocks + i) * blk16;
  for (int64_t k = threadIdx.x; k < blk16; k += kCopyThreads) dst[k] = src[k];
}

__global__ __launch_bounds__(kCopyThreads) void scatter_kernel(uint4* __restrict__ pool, int64_t part_stride16,
                                                               const int32_t* __restrict__ ids, int64_t blk16,
                                                               int32_t nblocks, const uint4* __restrict__ src) {
  const int i = blockIdx.x, p = blockIdx.y;
  uint4* dst = pool + p * part_stride16 + (int64_t)ids[i] * blk16;
  const uint4* s = src + ((int64_t)p * nblocks + i) * blk16;
  for (int64_t k = threadIdx.x; k < blk16; k += kCopyThreads) dst[k] = s[k];
}

// One workgroup per job: if any block id of the job lies outside [0, pool_blocks),
// flag it and clear num_blocks of every job, so that the kernels enqueued after this
// one on the stream run with nothing to do and touch no pool memory.
__global__ __launch_bounds__(kCopyThreads) void check_blocks_kernel(kvmi_layer_job* __restrict__ jobs,
                                                                    int32_t num_jobs, int32_t* __restrict__ err) {
  const int32_t* ids = jobs[blockIdx.x].block_ids;
  const int n = jobs[blockIdx.x].num_blocks;
  const int64_t P = jobs[blockIdx.x].pool_blocks;
  int mine = 0;
  for (int i = threadIdx.x; i < n; i += kCopyThreads) {
    const int32_t b = ids[i];
    mine |= b < 0 || b >= P;
  }
  if (!__syncthreads_or(mine)) return;
  if (threadIdx.x == 0) atomicOr(err, KVMI_ERR_BLOCK_ID);
  for (int k = threadIdx.x; k < num_jobs; k += kCopyThreads) jobs[k].num_blocks = 0;
}

constexpr int kHadWG = 512;

template <int D>
__global__ __launch_bounds__(kHadWG) void hadamard_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                          int64_t rows, int H, const uint32_t* __restrict__ signs,
                                                          int inverse, float scale) {
  constexpr int E = D / 4;
  const int tid = threadIdx.x, q = tid & 3;
  const int64_t r = (int64_t)blockIdx.x * (kHadWG / 4) + (tid >> 2);
  if (r >= rows) return;  // the 4 lanes of a quad share r
  const int h = (int)(r % H);
  const uint32_t* sg = signs + h * (D / 32);
  const uint32_t sb = (E == 32) ? sg[q] : ((sg[q >> 1] >> ((q & 1) * 16)) & 0xffffu);
  uint32_t w[E / 2];
  load_bf16_seg<E>(in + r * D + q * E, w);
  if (!inverse) apply_sign_bf16<E>(w, sb);
  float v[E];
  unpack_bf16<E>(w, v);
  fwht_row<E>(v, q);
#pragma unroll
  for (int i = 0; i < E / 2; ++i) w[i] = pack_bf16x2(v[2 * i] * scale, v[2 * i + 1] * scale);
  if (inverse) apply_sign_bf16<E>(w, sb);
  store_bf16_seg<E>(out + r * D + q * E, w);
}

}  // namespace
}  // namespace kvmi

extern "C" int kvmi_gather_blocks(const void* pool, int64_t pool_part_stride, const int32_t* block_ids,
                                  int32_t num_blocks, int64_t block_elems, void* out, kvmi_stream_t stream) {
  using namespace kvmi;
  if (num_blocks < 0 || block_elems <= 0 || pool_part_stride < 0) return KVMI_EINVAL;
  if (num_blocks == 0) return KVMI_OK;
  if (!pool || !block_ids || !out) return KVMI_EINVAL;
  if ((block_elems * 2) % 16 || (pool_part_stride * 2) % 16 || (uintptr_t)pool % 16 || (uintptr_t)out % 16)
    return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)num_blocks, 2), dim3(kCopyThreads), 0, st,
                     static_cast<const uint4*>(pool), pool_part_stride * 2 / 16, block_ids, block_elems * 2 / 16,
                     num_blocks, static_cast<uint4*>(out));
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_scatter_blocks(void* pool, int64_t pool_part_stride, const int32_t* block_ids,
                                   int32_t num_blocks, int64_t block_elems, const void* src, kvmi_stream_t stream) {
  using namespace kvmi;
  if (num_blocks < 0 || block_elems <= 0 || pool_part_stride < 0) return KVMI_EINVAL;
  if (num_blocks == 0) return KVMI_OK;
  if (!pool || !block_ids || !src) return KVMI_EINVAL;
  if ((block_elems * 2) % 16 || (pool_part_stride * 2) % 16 || (uintptr_t)pool % 16 || (uintptr_t)src % 16)
    return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)num_blocks, 2), dim3(kCopyThreads), 0, st,
                     static_cast<uint4*>(pool), pool_part_stride * 2 / 16, block_ids, block_elems * 2 / 16,
                     num_blocks, static_cast<const uint4*>(src));
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

// The MLA / FlashInfer cache layout [P, 2, S, H, D]: a block's K and V are adjacent,
// so a block is one unit of 2*block_elems elements (one part per workgroup column).
extern "C" int kvmi_gather_blocks_kv_adjacent(const void* pool, const int32_t* block_ids, int32_t num_blocks,
                                              int64_t block_elems, void* out, kvmi_stream_t stream) {
  using namespace kvmi;
  if (num_blocks < 0 || block_elems <= 0) return KVMI_EINVAL;
  if (num_blocks == 0) return KVMI_OK;
  if (!pool || !block_ids || !out) return KVMI_EINVAL;
  if ((block_elems * 2) % 16 || (uintptr_t)pool % 16 || (uintptr_t)out % 16) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)num_blocks, 1), dim3(kCopyThreads), 0, st,
                     static_cast<const uint4*>(pool), (int64_t)0, block_ids, block_elems * 4 / 16, num_blocks,
                     static_cast<uint4*>(out));
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_scatter_blocks_kv_adjacent(void* pool, const int32_t* block_ids, int32_t num_blocks,
                                               int64_t block_elems, const void* src, kvmi_stream_t stream) {
  using namespace kvmi;
  if (num_blocks < 0 || block_elems <= 0) return KVMI_EINVAL;
  if (num_blocks == 0) return KVMI_OK;
  if (!pool || !block_ids || !src) return KVMI_EINVAL;
  if ((block_elems * 2) % 16 || (uintptr_t)pool % 16 || (uintptr_t)src % 16) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)num_blocks, 1), dim3(kCopyThreads), 0, st,
                     static_cast<uint4*>(pool), (int64_t)0, block_ids, block_elems * 4 / 16, num_blocks,
                     static_cast<const uint4*>(src));
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_check_block_ids(kvmi_layer_job* jobs, int32_t num_jobs, int32_t* err, kvmi_stream_t stream) {
  using namespace kvmi;
  if (num_jobs < 0) return KVMI_EINVAL;
  if (num_jobs == 0) return KVMI_OK;
  if (!jobs || !err) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(check_blocks_kernel, dim3((unsigned)num_jobs), dim3(kCopyThreads), 0, st, jobs, num_jobs, err);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}

extern "C" int kvmi_hadamard(const void* in, void* out, int64_t rows, int32_t num_heads, int32_t head_dim,
                             const uint32_t* signs, int32_t inverse, kvmi_stream_t stream) {
  using namespace kvmi;
  if (rows < 0 || num_heads < 1 || head_dim < 2 || head_dim > 256 || head_dim % 2) return KVMI_EINVAL;
  if (rows == 0) return KVMI_OK;
  if (!in || !out || !signs) return KVMI_EINVAL;
  if ((uintptr_t)in % 16 || (uintptr_t)out % 16) return KVMI_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (head_dim != 64 && head_dim != 128)  // power-of-two chunks, one row per 16-channel lane group
    return rows_hadamard(in, out, rows, num_heads, head_dim, signs, inverse, st);
  const int64_t grid = (rows + kHadWG / 4 - 1) / (kHadWG / 4);
  if (grid > 0x7fffffffLL) return KVMI_EINVAL;
  const float scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  if (head_dim == 64)
    hipLaunchKernelGGL((hadamard_kernel<64>), dim3((unsigned)grid), dim3(kHadWG), 0, st,
                       static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, num_heads, signs, inverse,
                       scale);
  else
    hipLaunchKernelGGL((hadamard_kernel<128>), dim3((unsigned)grid), dim3(kHadWG), 0, st,
                       static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, num_heads, signs, inverse,
                       scale);
  return hipGetLastError() == hipSuccess ? KVMI_OK : KVMI_ELAUNCH;
}
