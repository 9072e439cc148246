/*
 * CPU restatement of this engine's rANS entropy codec -- TEST INFRASTRUCTURE ONLY
 * (the checker of the HIP kernels; nothing in the product links it).
 *
 * Role in the reference: the lossless codec stage that KVServe fills with nvCOMP
 * ANS (codec_type "nvcomp", kvserve_v1/compression/codec/kvserve_codec.py:57-64;
 * nvcomp_func.py:54-143: encode a uint8 view to bytes, decode back to the
 * original dtype and shape) or LC (lc_codec.py).  nvCOMP is closed NVIDIA code
 * with an unpublished stream format, so this codec defines its own format; the
 * algorithm is range ANS (J. Duda, "Asymmetric numeral systems", 2013) with
 * interleaved states (F. Giesen, "Interleaved entropy coders", 2014) and, on the
 * GPU, division by invariant integers (Granlund & Montgomery, PLDI 1994).  This
 * file uses plain C division so that it checks the GPU's reciprocal path.
 *
 * Symbols: n symbols of w bits (1..8), packed LSB-first (symbol i at bits
 * [i*w, i*w + w) of a little-endian byte string) -- the bitpack body layout.
 *
 * Stream (little-endian):
 *   [0]  u32 magic 0x5352564B ("KVRS")   [4] u8 version 2, u8 w, u8 prob_bits 12, u8 log2(states) 8
 *   [8]  u32 block_symbols (65536)      [12] u32 num_blocks = ceil(n / block_symbols)
 *   [16] u64 n                          [24] u64 payload_bytes
 *   [32] u64 offset[num_blocks]  (block b starts at payload + offset[b]; payload = 32 + 8*num_blocks)
 *   blocks, each a multiple of 4 bytes:
 *     u32 tag = mode | count0 << 1      mode 0 = rANS, 1 = raw
 *     rANS: u16 freq[2^w] (padded to 4 bytes), u32 count[3] (sub-blocks 1..3),
 *           u32 state[4][64], then for each sub-block j = 0..3 a word region of
 *           pad4(2*count_j) bytes whose last 2*count_j are its words u16[count_j]
 *           (a zero u16 in front when count_j is odd)
 *     raw:  the block's packed symbols, ceil(nb*w/8) bytes, zero-padded to 4
 *
 * Block b holds symbols [b*65536, b*65536 + nb) in 4 sub-blocks of 16384 symbols
 * that share the block's frequency table and are coded independently (one GPU wave
 * each).  In sub-block j, lane i (0..63) owns, at step t (0..255), block symbol
 * j*16384 + (t/32)*2048 + i*32 + t%32 when it is < nb.  Encoding runs t = 255..0;
 * at each step every lane with a symbol s first renormalises (x >= freq[s] << 20:
 * emit x & 0xffff, x >>= 16), the step's emitted words are placed, in lane order,
 * in front of the words of later steps, then x = (x / f) << 12 | (x % f) + cum[s].
 * States start at 2^16; decoding runs t = 0..255 and ends with every state back at
 * 2^16.
 * Frequencies (prob_bits 12, M = 4096): with c[v] the block's counts and K the
 * number of symbols present, f[v] = c[v] ? 1 + c[v] * (M - K) / nb : 0, and the
 * remainder M - sum(f) goes to the most frequent symbol (lowest value on ties).
 * A block is stored raw when a sub-block's words exceed 16384*w/16 (its raw size)
 * or when its rANS form is not smaller than its raw form.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KVRS_MAGIC 0x5352564Bu
#define PB 12u
#define M (1u << PB)
#define LANES 64u
#define RUN 32u
#define SUBS 4u
#define SUB_STEPS 256u
#define SUB (LANES * SUB_STEPS)
#define BLOCK (SUB * SUBS)
#define RANS_L (1u << 16)

static uint64_t pad4(uint64_t b) { return (b + 3u) & ~(uint64_t)3u; }

static unsigned get_sym(const uint8_t* in, uint64_t i, int w) {
    uint64_t bit = i * (uint64_t)w;
    unsigned v = in[bit >> 3] >> (bit & 7u);
    if ((bit & 7u) + (unsigned)w > 8u) v |= (unsigned)in[(bit >> 3) + 1] << (8u - (bit & 7u));
    return v & ((1u << w) - 1u);
}

static void put_sym(uint8_t* out, uint64_t i, int w, unsigned s) {
    uint64_t bit = i * (uint64_t)w;
    unsigned sh = (unsigned)(bit & 7u);
    out[bit >> 3] |= (uint8_t)(s << sh);
    if (sh + (unsigned)w > 8u) out[(bit >> 3) + 1] |= (uint8_t)(s >> (8u - sh));
}

static void wr32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }
static void wr64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }
static uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

static uint64_t block_idx(unsigned j, unsigned t, unsigned lane) {
    return (uint64_t)j * SUB + (uint64_t)(t / RUN) * (LANES * RUN) + (uint64_t)lane * RUN + t % RUN;
}

static uint64_t raw_block_bytes(uint64_t nb, int w) { return 4u + pad4((nb * (uint64_t)w + 7u) / 8u); }
static uint64_t table_bytes(int w) { return pad4(2u << w); }
static uint64_t head_bytes(int w) { return 4u + table_bytes(w) + 4u * (SUBS - 1u) + 4u * LANES * SUBS; }

/* Upper bound of the stream size for n symbols of w bits. */
int64_t oracle_rans_max_bytes(uint64_t n, int w) {
    if (w < 1 || w > 8) return -1;
    uint64_t nblk = (n + BLOCK - 1) / BLOCK, total = 32u + 8u * nblk;
    for (uint64_t b = 0; b < nblk; ++b) {
        uint64_t nb = (b + 1 == nblk) ? n - b * BLOCK : BLOCK;
        total += raw_block_bytes(nb, w);
    }
    return (int64_t)total;
}

/* The block's frequency table; returns the number of distinct symbols. */
static void block_freqs(const uint8_t* in, uint64_t first, uint64_t nb, int w, uint32_t* f) {
    uint64_t c[256] = {0};
    unsigned A = 1u << w, K = 0, top = 0;
    for (uint64_t i = 0; i < nb; ++i) c[get_sym(in, first + i, w)]++;
    for (unsigned v = 0; v < A; ++v) {
        if (c[v]) ++K;
        if (c[v] > c[top]) top = v;
    }
    uint32_t sum = 0;
    for (unsigned v = 0; v < A; ++v) {
        f[v] = c[v] ? 1u + (uint32_t)(c[v] * (uint64_t)(M - K) / nb) : 0u;
        sum += f[v];
    }
    f[top] += M - sum;
}

/* Codes sub-block j of a block: words into words[*pos, cap) (front-filled), final
 * states into x; returns the word count. */
static uint64_t encode_sub(const uint8_t* in, uint64_t first, uint64_t nb, int w, unsigned j, const uint32_t* f,
                           const uint32_t* cum, uint16_t* words, uint64_t cap, uint32_t* x) {
    uint64_t pos = cap;
    for (unsigned i = 0; i < LANES; ++i) x[i] = RANS_L;
    for (int t = (int)SUB_STEPS - 1; t >= 0; --t) {
        unsigned s_of[LANES];
        int valid[LANES];
        unsigned emit = 0;
        for (unsigned i = 0; i < LANES; ++i) {
            uint64_t k = block_idx(j, (unsigned)t, i);
            valid[i] = k < nb;
            if (!valid[i]) continue;
            s_of[i] = get_sym(in, first + k, w);
            if ((x[i] >> 20) >= f[s_of[i]]) ++emit;
        }
        pos -= emit;
        uint64_t p = pos;
        for (unsigned i = 0; i < LANES; ++i) {
            if (!valid[i]) continue;
            uint32_t fs = f[s_of[i]];
            if ((x[i] >> 20) >= fs) {
                words[p++] = (uint16_t)(x[i] & 0xffffu);
                x[i] >>= 16;
            }
            x[i] = ((x[i] / fs) << PB) + (x[i] % fs) + cum[s_of[i]];
        }
    }
    return cap - pos;
}

/* Encodes one block into dst (capacity raw_block_bytes); returns its size. */
static uint64_t encode_block(const uint8_t* in, uint64_t first, uint64_t nb, int w, uint8_t* dst) {
    unsigned A = 1u << w;
    uint32_t f[256], cum[256];
    block_freqs(in, first, nb, w, f);
    cum[0] = 0;
    for (unsigned v = 1; v < A; ++v) cum[v] = cum[v - 1] + f[v - 1];

    uint64_t raw = raw_block_bytes(nb, w);
    uint64_t cap = LANES * SUB_STEPS; /* at most one word per symbol */
    uint64_t sub_cap = (uint64_t)SUB * (uint64_t)w / 16u;
    uint16_t* words = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(cap * SUBS));
    uint32_t x[SUBS][LANES];
    uint64_t count[SUBS], size = head_bytes(w);
    int over = 0;
    for (unsigned j = 0; j < SUBS; ++j) {
        count[j] = encode_sub(in, first, nb, w, j, f, cum, words + (uint64_t)j * cap, cap, x[j]);
        if (count[j] > sub_cap) over = 1;
        size += pad4(2u * count[j]);
    }
    if (over || size >= raw) {
        free(words);
        memset(dst, 0, raw);
        wr32(dst, 1u);
        uint64_t rb = (nb * (uint64_t)w + 7u) / 8u;
        memcpy(dst + 4, in + first * (uint64_t)w / 8u, rb);
        return raw;
    }
    memset(dst, 0, size);
    wr32(dst, (uint32_t)(count[0] << 1));
    uint8_t* q = dst + 4;
    for (unsigned v = 0; v < A; ++v) { uint16_t fv = (uint16_t)f[v]; memcpy(q + 2u * v, &fv, 2); }
    q += table_bytes(w);
    for (unsigned j = 1; j < SUBS; ++j) wr32(q + 4u * (j - 1u), (uint32_t)count[j]);
    q += 4u * (SUBS - 1u);
    for (unsigned j = 0; j < SUBS; ++j)
        for (unsigned i = 0; i < LANES; ++i) wr32(q + 4u * (LANES * j + i), x[j][i]);
    q += 4u * LANES * SUBS;
    for (unsigned j = 0; j < SUBS; ++j) {
        uint64_t region = pad4(2u * count[j]);
        memcpy(q + (region - 2u * count[j]), words + (uint64_t)j * cap + (cap - count[j]), 2u * count[j]);
        q += region;
    }
    free(words);
    return size;
}

/* Returns the stream size, or -1 for a bad width, -2 when cap is too small. */
int64_t oracle_rans_encode(const uint8_t* in, uint64_t n, int w, uint8_t* out, int64_t cap) {
    int64_t need = oracle_rans_max_bytes(n, w);
    if (need < 0) return -1;
    if (cap < need) return -2;
    uint32_t nblk = (uint32_t)((n + BLOCK - 1) / BLOCK);
    memset(out, 0, 32u + 8u * (uint64_t)nblk);
    wr32(out, KVRS_MAGIC);
    out[4] = 2; out[5] = (uint8_t)w; out[6] = (uint8_t)PB; out[7] = 8;
    wr32(out + 8, BLOCK);
    wr32(out + 12, nblk);
    wr64(out + 16, n);
    uint8_t* payload = out + 32u + 8u * (uint64_t)nblk;
    uint64_t off = 0;
    for (uint32_t b = 0; b < nblk; ++b) {
        uint64_t nb = (b + 1 == nblk) ? n - (uint64_t)b * BLOCK : BLOCK;
        wr64(out + 32u + 8u * b, off);
        off += encode_block(in, (uint64_t)b * BLOCK, nb, w, payload + off);
    }
    wr64(out + 24, off);
    return (int64_t)(32u + 8u * (uint64_t)nblk + off);
}

/* 0 = ok; -1 bad header / size; -2 corrupt block.  out holds ceil(n*w/8) bytes. */
int oracle_rans_decode(const uint8_t* in, int64_t in_bytes, uint64_t n, int w, uint8_t* out) {
    if (in_bytes < 32 || rd32(in) != KVRS_MAGIC || in[4] != 2 || in[5] != w || in[6] != PB || in[7] != 8)
        return -1;
    uint32_t nblk = rd32(in + 12);
    if (rd32(in + 8) != BLOCK || rd64(in + 16) != n || nblk != (n + BLOCK - 1) / BLOCK) return -1;
    uint64_t head = 32u + 8u * (uint64_t)nblk, pay = rd64(in + 24);
    /* the stream may sit in a larger buffer; compare without forming head + pay (wraps) */
    if ((uint64_t)in_bytes < head || pay > (uint64_t)in_bytes - head) return -1;
    const uint8_t* payload = in + head;
    unsigned A = 1u << w;
    memset(out, 0, (size_t)((n * (uint64_t)w + 7u) / 8u));
    for (uint32_t b = 0; b < nblk; ++b) {
        uint64_t nb = (b + 1 == nblk) ? n - (uint64_t)b * BLOCK : BLOCK;
        uint64_t o = rd64(in + 32u + 8u * b), e = (b + 1 == nblk) ? pay : rd64(in + 32u + 8u * (b + 1));
        if (o > e || e > pay || e - o < 4 || (o & 3u)) return -1;
        const uint8_t* blk = payload + o;
        uint32_t tag = rd32(blk);
        if (tag & 1u) {
            uint64_t rb = (nb * (uint64_t)w + 7u) / 8u;
            if (e - o != 4u + pad4(rb)) return -2;
            memcpy(out + (uint64_t)b * BLOCK * (uint64_t)w / 8u, blk + 4, rb);
            continue;
        }
        uint64_t count[SUBS], size = head_bytes(w);
        count[0] = tag >> 1;
        for (unsigned j = 1; j < SUBS; ++j) count[j] = rd32(blk + 4 + table_bytes(w) + 4u * (j - 1u));
        for (unsigned j = 0; j < SUBS; ++j) size += pad4(2u * count[j]);
        if (e - o != size) return -2;
        uint32_t f[256], cum[256], tot = 0;
        for (unsigned v = 0; v < A; ++v) { uint16_t fv; memcpy(&fv, blk + 4 + 2u * v, 2); f[v] = fv; cum[v] = tot; tot += fv; }
        if (tot != M) return -2;
        uint8_t slot_sym[M];
        for (unsigned v = 0; v < A; ++v)
            for (uint32_t k = 0; k < f[v]; ++k) slot_sym[cum[v] + k] = (uint8_t)v;
        const uint8_t* st = blk + 4 + table_bytes(w) + 4u * (SUBS - 1u);
        const uint8_t* region = st + 4u * LANES * SUBS;
        for (unsigned j = 0; j < SUBS; ++j) {
            uint32_t x[LANES];
            for (unsigned i = 0; i < LANES; ++i) x[i] = rd32(st + 4u * (LANES * j + i));
            const uint8_t* wp = region + (pad4(2u * count[j]) - 2u * count[j]);
            uint64_t p = 0;
            for (unsigned t = 0; t < SUB_STEPS; ++t) {
                for (unsigned i = 0; i < LANES; ++i) {
                    uint64_t k = block_idx(j, t, i);
                    if (k >= nb) continue;
                    uint32_t slot = x[i] & (M - 1u);
                    unsigned s = slot_sym[slot];
                    x[i] = f[s] * (x[i] >> PB) + slot - cum[s];
                    if (x[i] < RANS_L) {
                        if (p >= count[j]) return -2;
                        uint16_t wv; memcpy(&wv, wp + 2u * p, 2); ++p;
                        x[i] = (x[i] << 16) | wv;
                    }
                    put_sym(out, (uint64_t)b * BLOCK + k, w, s);
                }
            }
            if (p != count[j]) return -2;
            for (unsigned i = 0; i < LANES; ++i)
                if (x[i] != RANS_L) return -2;
            region += pad4(2u * count[j]);
        }
    }
    return 0;
}
