/*
 * kvserve_amd.h -- C ABI of the MI355X (gfx950) KV-cache compression engine.
 *
 * The library replaces KVServe's compression hot path:
 *   compress:   paged-KV block gather -> random-sign Hadamard (FWHT) -> min-max
 *               quantizer (K per channel, V per token) -> bitpack (16-byte header)
 *   decompress: unpack -> dequantize -> inverse FWHT -> sign -> paged scatter
 *
 * Conventions of every entry point:
 *   - all data pointers are device addresses owned by the caller, who keeps them
 *     alive until the stream has finished the work;
 *   - work is enqueued on `stream`; no entry point allocates, frees or
 *     synchronizes, and none uses the null stream unless `stream` is null;
 *   - the return value is 0 or a negative errno-style code for errors the host can
 *     see (bad sizes, bad bit width, launch failure).  Data errors found by the
 *     kernels (a symbol that does not fit the bit width, a stream header that does
 *     not match) are OR-ed into the caller's device word `err`
 *     (KVMI_ERR_* bits below); the caller reads it after the stream completes.
 *
 * Reference interfaces replaced (paths relative to the KVServe source tree):
 *   kvmi_bitpack_encode / kvmi_bitpack_decode
 *       kvserve_v1/compression/codec/bitpack_codec.py:100-135 (BitPackCodec.encode /
 *       .decode and the Triton _pack / _unpack kernels at :24-69)
 *   kvmi_gather_blocks
 *       kvserve_v1/utils/kv_utils.py:59-80 (extract_kv_from_layer_by_blocks)
 *   kvmi_scatter_blocks
 *       kvserve_v1/utils/kv_utils.py:83-119 (inject_kv_into_layer_by_blocks)
 *   kvmi_gather_blocks_kv_adjacent / kvmi_scatter_blocks_kv_adjacent
 *       kvserve_v1/utils/kv_utils.py:76-79 and :108-114 (the [num_blocks, 2, ...]
 *       branches of the same two functions)
 *   kvmi_hadamard
 *       kvserve_v1/compression/transformer/hadamard_func.py:161-231
 *       (HadamardTransform.transform / .inverse)
 *   kvmi_encode_paged (with kvmi_kstats_paged before it)
 *       kvserve_v1/compression/compression_manager.py:200-537 (compress_all_layers and
 *       its chunked variant: transform -> KVServeQuantizer.quantize
 *       (quantizer/kvserve_quantizer.py:171-233) -> codec-buffer permute (:155-164)
 *       -> KVServeCodec.encode (codec/kvserve_codec.py:154-178)), fused with the
 *       gather of kv_utils.py:59-80
 *   kvmi_decode_paged
 *       kvserve_v1/compression/compression_manager.py:539-757 (decompress_all_layers
 *       and its chunked variant), fused with the scatter of kv_utils.py:83-119
 */
#ifndef KVSERVE_AMD_H
#define KVSERVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* kvmi_stream_t;

#define KVMI_ABI_VERSION 2

/* Bits OR-ed into the caller's device error word. */
#define KVMI_ERR_SYMBOL_RANGE 1 /* a symbol >= 2^bits reached the packer */
#define KVMI_ERR_BAD_HEADER 2   /* stream header does not match the decode contract */
#define KVMI_ERR_CORRUPT 4      /* an entropy-coded block does not decode consistently */
#define KVMI_ERR_SYNC 8         /* a one-pass compress barrier timed out or met another call's keys */
#define KVMI_ERR_BLOCK_ID 16    /* a block id outside its pool (kvmi_check_block_ids) */
#define KVMI_ERR_SCHEDULE 32    /* a job has more blocks than its one-pass schedule */

/* Host-visible return codes. */
#define KVMI_OK 0
#define KVMI_EINVAL (-22)
#define KVMI_ELAUNCH (-5)
#define KVMI_ENOSPC (-28) /* the call needs more than a fixed scratch array holds */

/* Stream format constants (bitpack_codec.py:20-21). */
#define KVMI_HEADER_BYTES 16
#define KVMI_MAGIC 0x0150424Bu

/* Flags of kvmi_geometry.flags */
#define KVMI_F_NO_TRANSFORM 1u /* skip signs + FWHT (pipeline without "transformer") */
#define KVMI_F_NATIVE_LAYOUT 2u /* symbol order [l,2,B,S,H',D] instead of [l,2,H',B,S,D] */
#define KVMI_F_NO_HEADER 4u     /* raw symbol buffer: no 16-byte header (bits must be 8) */
#define KVMI_F_VALU_FWHT 8u     /* force the register (VALU) FWHT kernels instead of MFMA */
#define KVMI_F_CLAMP_LEVELS 16u /* some level count exceeds 128: clamp symbols to the level */
#define KVMI_F_TWO_PASS 32u     /* kvmi_compress_paged: statistics pass + encode pass (K read twice) */
/* Quantization axes (quantizer_func.py:41-49; KVServeQuantizer axis_key / axis_value,
 * kvserve_quantizer.py:136-139).  Default (no flag): K per channel, V per token.  At most
 * one flag per part; any of them selects the generic row kernels. */
#define KVMI_F_K_TOKEN 64u    /* K statistics per token over the heads of a K group */
#define KVMI_F_K_TENSOR 128u  /* one K statistic pair per K group */
#define KVMI_F_V_CHANNEL 256u /* V statistics per channel of each head */
#define KVMI_F_V_TENSOR 512u  /* one V statistic pair per V group */
/* Force the generic row kernels (register FWHT with DPP exchanges over next_pow2(D)/16
 * lanes of a row) instead of MFMA or the quad-per-row kernels. */
#define KVMI_F_ROW_FWHT 1024u

/* Launch-wide geometry shared by every job of one call. */
typedef struct kvmi_geometry {
  int32_t block_size; /* S: tokens per paged block (vLLM block_size) */
  int32_t num_heads;  /* H: KV heads of this worker's shard, 1..64 */
  int32_t head_dim;   /* D: even in [2, 256], with H * next_pow2(D) <= 8192 and D * bits a
                         multiple of 8 (whole-byte packed rows); a D that is not a power of
                         two is transformed in descending power-of-two chunks, down to
                         chunks of 1 channel (hadamard_func.py:50-103: 100 = 64 + 32 + 4) */
  int32_t bits;       /* bitpack width in [1, 8] */
  uint32_t flags;     /* KVMI_F_* */
  int32_t max_groups; /* G: V statistic groups per layer (<= H) */
  int32_t reserved[2];
} kvmi_geometry;

/*
 * One (request, layer) unit of work.  An array of these lives in device memory.
 *
 * profile: uint8 [2 parts][3][H]
 *   [p][0][j] source head that is stored at output position j (low heads first,
 *             ascending, then high heads: kvserve_quantizer.py:216-220)
 *   [p][1][j] quantization levels (max_value) of output position j, in [2, 255]
 *   [p][2][j] statistic group of output position j; groups are contiguous runs of
 *             positions sharing one level count.  A part on the token or tensor axis
 *             shares its statistics over the heads of a group (quantizer_func.py:44-53);
 *             on the channel axis groups only label the sections.
 * kmeta / vmeta: bf16 metadata of the K / V part, [0] = min, [1] = scale, laid out by
 *   the part's axis: channel [2][H][D] by output position (K's default), token
 *   [2][G][num_blocks*S] by group (V's default), tensor [2][G] by group.
 * kstats: uint32 [2][H][D] order-preserving keys of the running K min / max; with
 *   KVMI_F_V_CHANNEL or KVMI_F_V_TENSOR, [2 parts][2][H][D] (V's keys after K's);
 *   initialised to {0xFFFFFFFF, 0}; kvmi_kstats_paged leaves it initialised.
 * pool_blocks: P, the blocks of `pool`; read only by kvmi_check_block_ids.
 */
typedef struct kvmi_layer_job {
  void* pool;                /* bf16 [2, P, S, H, D] paged KV of this layer (NHD) */
  const int32_t* block_ids;  /* [num_blocks] pool block of each logical block */
  uint8_t* stream;           /* packed chunk stream this layer belongs to (16-byte aligned) */
  uint16_t* kmeta;
  uint16_t* vmeta;
  const uint32_t* signs;     /* [H][ceil(D/32)] Rademacher sign bits per source head (1 = -1) */
  const uint8_t* profile;
  uint32_t* kstats;
  int64_t pool_blocks;       /* P: block ids must lie in [0, P) */
  int64_t pool_part_stride;  /* elements between the K and V halves of `pool` */
  int64_t symbol_offset;     /* index of this layer's first symbol in the chunk */
  int64_t chunk_symbols;     /* symbol count N of the chunk (header bytes 8..15) */
  int32_t num_blocks;        /* B */
  int32_t write_header;      /* 1 for exactly one job of each chunk */
} kvmi_layer_job;

/* ABI version of the loaded library (KVMI_ABI_VERSION). */
int kvmi_abi_version(void);

/*
 * Bitpack codec.  Replaces BitPackCodec.encode (bitpack_codec.py:100-110):
 * out[0..15] = header {4B 42 50 01, bits, 0,0,0, n as u64 LE}; out[16 + ...] =
 * symbols packed LSB-first, symbol i at stream bit i*bits.  `out` holds
 * 16 + ceil(n*bits/8) bytes.  Symbols >= 2^bits set KVMI_ERR_SYMBOL_RANGE.
 */
int kvmi_bitpack_encode(const uint8_t* sym, int64_t n, int32_t bits, uint8_t* out,
                        int32_t* err, kvmi_stream_t stream);

/*
 * Replaces BitPackCodec.decode (bitpack_codec.py:112-135).  `in_bytes` must equal
 * 16 + ceil(n*bits/8) (else KVMI_EINVAL, the reference's length ValueError).  A
 * header that does not name (bits, n) sets KVMI_ERR_BAD_HEADER and leaves `sym`
 * unwritten.
 */
int kvmi_bitpack_decode(const uint8_t* in, int64_t in_bytes, int64_t n, int32_t bits,
                        uint8_t* sym, int32_t* err, kvmi_stream_t stream);

/*
 * Paged gather of whole blocks (kv_utils.py:59-80, FlashAttention NHD layout):
 * out[p, i] = pool[p, block_ids[i]] for p in {K, V}; `block_elems` = S*H*D.
 * out is contiguous [2, num_blocks, S, H, D]; element size 2 bytes.
 */
int kvmi_gather_blocks(const void* pool, int64_t pool_part_stride, const int32_t* block_ids,
                       int32_t num_blocks, int64_t block_elems, void* out,
                       kvmi_stream_t stream);

/*
 * Paged scatter (kv_utils.py:83-119): pool[p, block_ids[i]] = src[p, i] for
 * i < num_blocks (the caller passes min(len(block_ids), payload blocks)).
 */
int kvmi_scatter_blocks(void* pool, int64_t pool_part_stride, const int32_t* block_ids,
                        int32_t num_blocks, int64_t block_elems, const void* src,
                        kvmi_stream_t stream);

/*
 * The MLA / FlashInfer branch of the same two functions (kv_utils.py:76-79 and
 * :108-114), cache layout [P, 2, S, H, D] with a block's K and V adjacent:
 * gather out[i] = pool[block_ids[i]] into a contiguous [num_blocks, 2, S, H, D];
 * scatter pool[block_ids[i]] = src[i] for i < num_blocks.  `block_elems` = S*H*D
 * (one part of a block); element size 2 bytes.
 */
int kvmi_gather_blocks_kv_adjacent(const void* pool, const int32_t* block_ids, int32_t num_blocks,
                                   int64_t block_elems, void* out, kvmi_stream_t stream);
int kvmi_scatter_blocks_kv_adjacent(void* pool, const int32_t* block_ids, int32_t num_blocks,
                                    int64_t block_elems, const void* src, kvmi_stream_t stream);

/*
 * Device-side check of the block tables of a job table, for callers whose block ids
 * are a device tensor and who must not synchronize to check them on the host.  No
 * counterpart in the reference (its torch indexing faults or raises on a bad id).  If
 * any job holds an id outside [0, pool_blocks), sets KVMI_ERR_BLOCK_ID and sets
 * num_blocks of every job to 0, so that the kernels enqueued after it on the stream
 * (kvmi_kstats_paged, kvmi_encode_paged, kvmi_decode_paged) touch no pool memory.
 * One workgroup per job; `jobs` is written, so it is the job table of one call.
 */
int kvmi_check_block_ids(kvmi_layer_job* jobs, int32_t num_jobs, int32_t* err, kvmi_stream_t stream);

/*
 * Random-sign Hadamard transform of contiguous bf16 rows [rows, D], row r
 * belonging to head r % num_heads (hadamard_func.py:161-231), D even in [2, 256].  Each power-of-two chunk c of D (descending, hadamard_func.py:50-103) is
 * transformed on its own:
 *   forward: out = bf16( FWHT_fp32(x * s) * (1/sqrt(c)) )
 *   inverse: out = bf16( FWHT_fp32(x) * (1/sqrt(c)) ) * s
 * signs: [num_heads][ceil(D/32)] bits (1 = -1).  in and out may alias.
 */
int kvmi_hadamard(const void* in, void* out, int64_t rows, int32_t num_heads,
                  int32_t head_dim, const uint32_t* signs, int32_t inverse,
                  kvmi_stream_t stream);

/*
 * Pass 1 of compress: per-channel K statistics over all tokens of each job
 * (quantizer_func.py:41-53, axis "channel" reduces blocks and tokens).  Fills
 * each job's kmeta (min and scale of every K channel) and leaves kstats
 * re-initialised (two kernel launches).  `max_blocks` = max num_blocks over jobs
 * (grid sizing).  Jobs with num_blocks == 0 keep their kmeta.
 */
int kvmi_kstats_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                      int32_t max_blocks, int32_t* err, kvmi_stream_t stream);

/*
 * Pass 2 of compress: gather, transform, quantize K with the kmeta of pass 1 and V
 * with per-token group statistics, and bitpack every job into its chunk stream
 * (plus the 16-byte header of jobs with write_header = 1) and vmeta.
 */
int kvmi_encode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                      int32_t max_blocks, int32_t* err, kvmi_stream_t stream);

/*
 * Compress in one call: the gather, transform, quantization and bitpack of
 * kvmi_kstats_paged + kvmi_encode_paged (same outputs, bit for bit), reading every
 * K value from HBM once.  Replaces the same reference path as those two
 * (compression_manager.py:200-537 with kv_utils.py:59-80).  No counterpart of its own
 * in the reference.
 *
 * kvmi_compress_schedule (host only) cuts the jobs' K into (job, head) groups of
 * 32-token head-tiles and V into token-major tiles and lays them out as the steps of a
 * persistent grid of the current device (one workgroup of 8 waves per CU).  It writes
 * the schedule image into `image` (when not NULL and image_bytes suffices) and returns
 * its size in bytes; 0 when the one-pass kernel does not serve the geometry (MFMA
 * geometry with H dividing 8, S a power of two >= 4 (>= 8 at D = 64), default axes, no
 * KVMI_F_TWO_PASS), the device has no cooperative launch, or one head of a job has more
 * K than the grid holds (8 head-tiles of 32 tokens per workgroup: 65,536 tokens on 256
 * CUs); a negative KVMI_* code on bad arguments.  num_blocks: host array, B of each job.
 * The image's int32 at byte offset 36 counts the K groups that span several workgroups
 * (each needs a device barrier); 0 means every group fits one workgroup.
 *
 * kvmi_compress_workspace_bytes: device bytes the workspace of a schedule needs.
 *
 * kvmi_compress_paged: schedule = the host image (NULL selects the two passes, as does
 *   KVMI_F_TWO_PASS); workspace = 256-byte aligned device memory of
 *   kvmi_compress_workspace_bytes(schedule) bytes whose first bytes hold a copy of the
 *   image and the rest zero before the first call, then passed unchanged to every call
 *   for the same jobs (barrier flags and 64-bit min / max keys tagged with the call's
 *   epoch, so nothing is cleared between calls; the epoch lives in the workspace and a
 *   one-thread kernel enqueued before the pass advances it, so the call can be captured
 *   in a graph).  Calls sharing a workspace must be ordered on one stream.  From 2^31
 *   calls on one workspace on, KVMI_ERR_SYNC is set: initialise the workspace again.
 *   A schedule built for other jobs or another device returns KVMI_EINVAL (the jobs'
 *   num_blocks may be lower than the schedule's: the kernel skips missing tiles; a job
 *   with more blocks than the schedule's sets KVMI_ERR_SCHEDULE, and the blocks past
 *   the schedule's are not compressed).
 * A barrier that does not complete within about 0.3 s sets KVMI_ERR_SYNC (the
 * kernel still ends; later barriers of the launch then no longer wait).
 */
int64_t kvmi_compress_schedule(const kvmi_geometry* geom, const int32_t* num_blocks, int32_t num_jobs,
                               void* image, int64_t image_bytes);
int64_t kvmi_compress_workspace_bytes(const void* schedule);
int kvmi_compress_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                        int32_t max_blocks, const void* schedule, void* workspace, int32_t* err,
                        kvmi_stream_t stream);

/*
 * Decompress: check each chunk header, unpack, dequantize
 * (quantizer_func.py:77-113: bf16(bf16(q*scale)+min)), inverse transform and
 * scatter every job's blocks into its pool.  Blocks of a chunk whose header does
 * not match are left unwritten and KVMI_ERR_BAD_HEADER is set.
 */
int kvmi_decode_paged(const kvmi_geometry* geom, const kvmi_layer_job* jobs, int32_t num_jobs,
                      int32_t max_blocks, int32_t* err, kvmi_stream_t stream);

/*
 * Fused Hadamard quantizer with fp32 statistics: quantizer_config.impl
 * "tilelang_fused", replacing KVHadamardQuantOp.compress_v3 / decompress_v3
 * (kvserve_v1/tilelang_ops/kv_hadamard_quant.py:1519-1599, :1645-1750) behind
 * TileLangFusedQuantizer.quantize / .dequantize
 * (kvserve_v1/compression/quantizer/tilelang_quantizer.py:142-181).
 * One dense layer x = bf16 [2][rows][H][D] (rows = blocks * block_size, D in
 * {64, 128}, H dividing 64): y = FWHT_fp32(x * s) / sqrt(D) in the reference's
 * butterfly order; K per-(head, channel) and V per-(row, head) min / max of the fp32
 * y (V reduced over the heads of each group), scale = max(max - min, 1e-5) / (L - 1),
 * q = clamp(roundf((bf16(y) - min) / scale), 0, L) as uint8 [2][rows][H][D] (natural
 * head order).  levels: fp32 [2][H] (K then V), vgroup: int32 [H] group of each head
 * (heads with equal V levels).  Outputs fp32 kmeta [2][H][D] and vmeta [2][rows][H]
 * (min, scale).  `scratch` holds kvmi_v3_scratch_bytes(rows, H, D) bytes.  x, q, kmeta
 * and, below, out and kmeta16 are 16-byte aligned.
 */
int kvmi_v3_compress(const void* x, int64_t rows, int32_t num_heads, int32_t head_dim, const uint32_t* signs,
                     const float* levels, const int32_t* vgroup, uint8_t* q, float* kmeta, float* vmeta,
                     void* scratch, kvmi_stream_t stream);
/* Scratch bytes of kvmi_v3_compress: up to 256 per-workgroup K partials of 2*H*D*4
 * bytes, not depending on rows (-1 for an unsupported shape). */
int64_t kvmi_v3_scratch_bytes(int64_t rows, int32_t num_heads, int32_t head_dim);
/*
 * kvmi_v3_compress without the `scratch` argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops and harnesses that
 * forbid allocation).  No counterpart in the reference.  It allocates nothing: the K
 * partials live in a fixed device array of KVMI_V3_NOALLOC_SCRATCH_BYTES per GPU,
 * held from the library's first use on that GPU until the process ends.  A call needs
 * min(ceil(rows*H/64), 256) * 8*H*D bytes of it (every H*D <= 2048 fits); larger
 * calls return KVMI_ENOSPC before enqueueing anything.  Every call on one GPU shares
 * that GPU's array, so the library puts the calls on one GPU in one order: each call's
 * launches wait for the previous call's on that GPU (an event the library records after
 * them, created with the array's address on the GPU's first call), whichever stream or
 * host thread made it.  Calls enqueued under graph capture take no part in that order:
 * a replayed graph that runs at the same time as another call on the same GPU races
 * with it.  Results are identical to kvmi_v3_compress.
 */
#define KVMI_V3_NOALLOC_SCRATCH_BYTES (4 * 1024 * 1024)
int kvmi_v3_compress_noalloc(const void* x, int64_t rows, int32_t num_heads, int32_t head_dim,
                             const uint32_t* signs, const float* levels, const int32_t* vgroup, uint8_t* q,
                             float* kmeta, float* vmeta, kvmi_stream_t stream);
/* Inverse: x = fma(q, scale, min) with float16 metadata (the wire form: kmeta16
 * [2][H][D], vmeta16 [2][rows][H]), FWHT_fp32, bf16((y / sqrt(D)) * s) -> out
 * bf16 [2][rows][H][D]. */
int kvmi_v3_decompress(const uint8_t* q, int64_t rows, int32_t num_heads, int32_t head_dim, const uint32_t* signs,
                       const uint16_t* kmeta16, const uint16_t* vmeta16, void* out, kvmi_stream_t stream);

/*
 * Entropy codec (rANS) for the codec stage -- replaces the nvCOMP ANS codec that
 * KVServe's codec stage calls (kvserve_v1/compression/codec/kvserve_codec.py:57-64,
 * nvcomp_func.py:54-143: a uint8 view in, compressed bytes out, and back).  The
 * stream format is this engine's own (nvCOMP's is closed); oracle/rans.c
 * states it.  Input: n symbols of `bits` (1..8) bits packed LSB-first, i.e. a
 * bitpack body.  All pointers 8-byte aligned.
 *
 * kvmi_rans_max_bytes: capacity the encoder's `out` must have.
 * kvmi_rans_scratch_bytes: device scratch the encoder needs.
 * kvmi_rans_encode: three launches (encode blocks, scan, compact); the stream length
 *   is written to the device u64
 *   *out_len (read it after the stream completes).
 * kvmi_rans_decode: one launch; writes ceil(n*bits/8) packed bytes.  `in_bytes` is
 *   the size of the buffer holding the stream (at least the stream's length, which
 *   its header states; more is allowed).  A header that does not name (bits, n) or a
 *   stream longer than in_bytes sets KVMI_ERR_BAD_HEADER; a block that does not
 *   decode to its own end state sets KVMI_ERR_CORRUPT.
 */
typedef struct kvmi_rans_enc_job {
  const uint8_t* packed; /* n symbols of `bits` bits, LSB-first */
  int64_t n;
  uint8_t* out;          /* >= kvmi_rans_max_bytes(n, bits) */
  int64_t out_capacity;
  void* scratch;         /* >= kvmi_rans_scratch_bytes(n, bits) */
  int64_t scratch_bytes;
  uint64_t* out_len;     /* device u64: stream length */
} kvmi_rans_enc_job;     /* 56 bytes */

typedef struct kvmi_rans_dec_job {
  const uint8_t* stream;
  int64_t in_bytes;
  int64_t n;
  uint8_t* packed_out;   /* ceil(n*bits/8) bytes */
} kvmi_rans_dec_job;     /* 32 bytes */

int64_t kvmi_rans_max_bytes(int64_t n, int32_t bits);
int64_t kvmi_rans_scratch_bytes(int64_t n, int32_t bits);
int kvmi_rans_encode(const uint8_t* packed, int64_t n, int32_t bits, uint8_t* out, int64_t out_capacity,
                     void* scratch, int64_t scratch_bytes, uint64_t* out_len, kvmi_stream_t stream);
int kvmi_rans_decode(const uint8_t* stream_in, int64_t in_bytes, int64_t n, int32_t bits, uint8_t* packed_out,
                     int32_t* err, kvmi_stream_t stream);
/*
 * Batched forms: every stream of a request (e.g. the 8-layer chunks of a large
 * request) coded by one launch per kernel, so that small streams still fill the
 * GPU.  `jobs` is host memory; all jobs share `bits`.  The single-stream entry
 * points above are one-job batches.
 */
int kvmi_rans_encode_batch(const kvmi_rans_enc_job* jobs, int32_t num_jobs, int32_t bits, kvmi_stream_t stream);
int kvmi_rans_decode_batch(const kvmi_rans_dec_job* jobs, int32_t num_jobs, int32_t bits, int32_t* err,
                           kvmi_stream_t stream);

/*
 * Fixed-profile runtime numerics (kvserve_v1/compression/runtime/pipeline.py:264-804,
 * runtime/csrc/kvs_compress.cu), the second numerics mode:
 *   y = rn(FWHT(x * s) * D^-1/2) with every butterfly stage rounded to bf16;
 *   per section (axis channel / token / tensor) min, max,
 *   scale = rn(rn(max(rn(max - min), 1e-5)) / (L - 1)), inverse = rn(1 / scale);
 *   q = clamp(rint(rn(rn(y - min) * inverse)), 0, L - 1);  y~ = rn(rn(q * scale) + min).
 * Caches are HND views [blocks, heads, kernel_tokens, channels]; a KV part is the
 * channel window [channel_offset, channel_offset + head_dim).  Canonical rows are
 * (block, token) x [H, D] in output-head order (head_order[h] = cache head).
 */
#define KVMI_RT_TRANSFORM 1u /* signs + FWHT (pipeline stage "transformer") */
#define KVMI_RT_QUANTIZE 2u  /* min-max quantizer (stage "quantizer") */
/* every layer's cache pointer, strides and channel offset are multiples of 8
 * elements: cache rows move as 16-byte vectors */
#define KVMI_RT_ALIGNED 4u
/* take the multi-kernel path (transformed rows through the scratch) even where
 * the row kernels apply; the results are identical */
#define KVMI_RT_GENERIC 8u

typedef struct kvmi_rt_geometry {
  int32_t num_heads;
  int32_t head_dim;       /* power of two, <= 2048 */
  int32_t kernel_tokens;  /* tokens per physical block */
  uint32_t flags;         /* KVMI_RT_* */
  uint32_t axes;          /* axes present: 1 channel, 2 token, 4 tensor */
  int32_t reserved[3];
} kvmi_rt_geometry;       /* 32 bytes */

typedef struct kvmi_rt_section {
  int32_t head_start, head_count, levels, axis; /* axis 0 channel, 1 token, 2 tensor */
  int64_t aux_min_offset, aux_scale_offset;     /* bytes into the aux arena */
} kvmi_rt_section;                              /* 32 bytes */

typedef struct kvmi_rt_layer {
  void* cache;                 /* bf16 HND cache of the layer */
  int64_t block_stride, head_stride, token_stride, channel_offset; /* elements */
  const void* signs;           /* bf16 [H, D] by output head, or NULL */
  const int32_t* head_order;   /* [H] */
  int64_t u8_offset;           /* element offset of this layer-part in the payload */
  kvmi_rt_section sections[2];
  int32_t num_sections, reserved;
} kvmi_rt_layer;               /* 136 bytes; an array of them in device memory */

/*
 * Encode the body of one chunk for one KV part (runtime pipeline.py:557-669): rows of
 * `num_blocks` physical blocks (block_ids, device int64) of every layer.  Quantized:
 * aux receives the section minima / scales (and, at +aux_half_bytes, maxima /
 * inverses), the payload the u8 symbols at each layer's u8_offset; `canon` is device
 * scratch of kvmi_rt_scratch_bytes() (transformed rows, or per-workgroup column
 * statistics).  Not quantized: the payload gets the (transformed) bf16 rows.
 */
int kvmi_rt_encode(const kvmi_rt_geometry* geom, const kvmi_rt_layer* layers, int32_t num_layers,
                   const int64_t* block_ids, int64_t num_blocks, void* canon, uint8_t* packed, uint8_t* aux,
                   int64_t aux_half_bytes, kvmi_stream_t stream);
/* Scratch bytes kvmi_rt_encode needs for `rows` rows of `num_layers` layers of H x D. */
int64_t kvmi_rt_scratch_bytes(int32_t num_layers, int64_t rows, int32_t num_heads, int32_t head_dim);
/* Inverse (pipeline.py:720-804): payload (+ aux) -> the caches at block_ids. */
int kvmi_rt_decode(const kvmi_rt_geometry* geom, const kvmi_rt_layer* layers, int32_t num_layers,
                   const int64_t* block_ids, int64_t num_blocks, const uint8_t* packed, const uint8_t* aux,
                   kvmi_stream_t stream);
/* The runtime's normalized bf16-per-stage FWHT of rows [rows, head_dim]
 * (runtime cpp_backend.hadamard_transform); in and out may be equal, not overlap. */
int kvmi_rt_hadamard(const void* in, void* out, int64_t rows, int32_t head_dim, kvmi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVSERVE_AMD_H */
