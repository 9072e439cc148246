"""Codecs on gfx950: bitpack (the reference's format) and the rANS entropy codec
that serves codec_type "rans", "nvcomp" (ANS) and "lc"."""
from .bitpack_codec import BitPackCodec
from .kvserve_codec import ENTROPY_CODECS, KVServeCodec, is_entropy_codec
from .rans_codec import RANSCodec

__all__ = ["BitPackCodec", "KVServeCodec", "RANSCodec", "ENTROPY_CODECS", "is_entropy_codec"]
