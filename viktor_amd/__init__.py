"""viktor_amd: the rollout-and-scoring path of the Viktor basecaller on MI355X (gfx950).

Public surface of the reference package (viktor/__init__.py): Decoder, DecoderConfig, KVCache,
DoradoEncoder, load_dorado_encoder, DecodeEngine, Basecaller, BOS, EOS, PAD, KmerTokenizer, get_tokenizer.
The compute runs on libviktor_hip.so (hand-written HIP kernels behind a C ABI, include/viktor_hip.h).
"""

from .decoder import Decoder, DecoderConfig, KVCache
from .encoder import DoradoEncoder, load_dorado_encoder
from .engine import DecodeEngine
from .model import Basecaller
from .tokenizer import BOS, EOS, PAD, KmerTokenizer, get_tokenizer

__all__ = ["Decoder", "DecoderConfig", "KVCache", "DoradoEncoder", "load_dorado_encoder", "DecodeEngine",
           "Basecaller", "BOS", "EOS", "PAD", "KmerTokenizer", "get_tokenizer"]
