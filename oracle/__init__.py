"""CPU oracle of KVServe's compression hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (plus torch's CPU random generator for the sign
recipe), the reference's modular pipeline so that tests, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` can check the HIP engine against it.
Nothing in ``kvserve_amd`` imports it; the product path fails loudly when the HIP
library is missing instead of falling back here.

Modules
  kvpipe   bf16 arithmetic, signs, FWHT, min-max quantizer, head/layer masks,
           codec layout and chunking, bitpack, paged gather/scatter, and the whole
           compress / decompress of a request (each function cites the reference
           file:line it follows).
  cbitpack ctypes wrapper of ``bitpack.c``, a C restatement of the bitpack codec
           used for full-size streams.
  fused_v3 the arithmetic of quantizer impl "tilelang_fused" (compress_v3 /
           decompress_v3: fp32 statistics, grouped V, roundf, float16 metadata).

Pins (what fixes each function independently of this restatement):
  signs           torch CPU Generator recipe + committed fixture (tests/golden)
  fwht            Sylvester matrix (scipy.linalg.hadamard), H.H = D.I, {-1,0,1} inputs
  quantize/dequant golden vectors written by the reference's own quantizer_func /
                  KVServeQuantizer (tests/golden/make_golden.py) + exhaustive bf16
                  identities + fp32 min-max reference within +-1 level
  masks           brute force from the score tables
  layout/chunking golden vectors from the reference's CompressionManager
  bitpack         np.packbits closed form + hand-derived known answers
  gather/scatter  closed form on integer-valued pools
  fused_v3        float64 derivation on exactly representable inputs, half-step
                  reconstruction bound, planted bf16-statistics mistake
Parity unpinned: the summation order inside the third-party fast_hadamard_transform
(not vendored); this oracle uses the natural radix-2 order, lowest bit first.  In
fused_v3, the tie rule of T.round (taken as roundf) and the FMA contraction of the
dequant (taken as one fma) are TileLang / nvcc lowering choices.
"""
