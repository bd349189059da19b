"""viktor_amd: the rollout-and-scoring path of the Viktor basecaller's decoder on MI355X (gfx950).

Public surface of the reference package this path needs (viktor/__init__.py): Decoder, DecoderConfig,
KVCache, DecodeEngine, Basecaller, BOS, EOS, PAD, KmerTokenizer, get_tokenizer. The compute runs on
libviktor_hip.so (hand-written HIP kernels behind a C ABI, include/viktor_hip.h); the encoder that
produces the frames is outside this package.
"""

from .decoder import Decoder, DecoderConfig, KVCache
from .engine import DecodeEngine
from .model import Basecaller
from .tokenizer import BOS, EOS, PAD, KmerTokenizer, get_tokenizer

__all__ = ["Decoder", "DecoderConfig", "KVCache", "DecodeEngine", "Basecaller", "BOS", "EOS", "PAD",
           "KmerTokenizer", "get_tokenizer"]
