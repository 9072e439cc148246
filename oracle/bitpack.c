/*
 * C restatement of KVServe's bitpack codec -- TEST INFRASTRUCTURE ONLY.
 *
 * Follows kvserve_v1/compression/codec/bitpack_codec.py:20-69 (format and the
 * _pack / _unpack kernels): a 16-byte header {magic 0x0150424B LE, bits, 0,0,0,
 * n as u64 LE} followed by ceil(n*bits/8) bytes in which bit b of symbol i is
 * stream bit i*bits + b, bytes filled least-significant bit first.
 * Used by the tests to check full-size GPU streams quickly; never linked into the
 * product library.
 */
#include <stdint.h>
#include <string.h>

/* Returns 0, or -1 if a symbol does not fit in `bits` (the reference asserts). */
int oracle_bitpack_encode(const uint8_t* sym, int64_t n, int bits, uint8_t* out) {
  uint64_t un = (uint64_t)n;
  uint32_t magic = 0x0150424Bu;
  memset(out, 0, 16);
  for (int i = 0; i < 4; ++i) out[i] = (uint8_t)(magic >> (8 * i));
  out[4] = (uint8_t)bits;
  for (int i = 0; i < 8; ++i) out[8 + i] = (uint8_t)(un >> (8 * i));
  int64_t nbytes = (n * bits + 7) / 8;
  uint8_t* p = out + 16;
  memset(p, 0, (size_t)nbytes);
  int bad = 0;
  uint64_t acc = 0;
  int have = 0;
  int64_t o = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (sym[i] >> bits) bad = 1;
    acc |= (uint64_t)(sym[i] & ((1u << bits) - 1u)) << have;
    have += bits;
    while (have >= 8) {
      p[o++] = (uint8_t)acc;
      acc >>= 8;
      have -= 8;
    }
  }
  if (have > 0) p[o++] = (uint8_t)acc;
  return bad ? -1 : 0;
}

/* Returns 0, -1 on a length mismatch, -2 on a header mismatch. */
int oracle_bitpack_decode(const uint8_t* in, int64_t in_bytes, int64_t n, int bits, uint8_t* sym) {
  if (in_bytes != 16 + (n * bits + 7) / 8) return -1;
  uint8_t hdr[16];
  uint64_t un = (uint64_t)n;
  uint32_t magic = 0x0150424Bu;
  memset(hdr, 0, 16);
  for (int i = 0; i < 4; ++i) hdr[i] = (uint8_t)(magic >> (8 * i));
  hdr[4] = (uint8_t)bits;
  for (int i = 0; i < 8; ++i) hdr[8 + i] = (uint8_t)(un >> (8 * i));
  if (memcmp(hdr, in, 16) != 0) return -2;
  const uint8_t* p = in + 16;
  uint64_t acc = 0;
  int have = 0;
  int64_t o = 0;
  for (int64_t i = 0; i < n; ++i) {
    while (have < bits) {
      acc |= (uint64_t)p[o++] << have;
      have += 8;
    }
    sym[i] = (uint8_t)(acc & ((1u << bits) - 1u));
    acc >>= bits;
    have -= bits;
  }
  return 0;
}
