"""Codecs: the bitpack codec on gfx950 (codec_type="bitpack")."""
from .bitpack_codec import BitPackCodec
from .kvserve_codec import KVServeCodec

__all__ = ["BitPackCodec", "KVServeCodec"]
