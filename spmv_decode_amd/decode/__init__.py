"""Decode-step caller of the sparse GEMV: a compact Llama-3.1 / Qwen3 decoder,
a hipGraph-captured greedy decode runner and the dense-vs-sparse benchmark."""
from .model import CONFIGS, Decoder, DecoderConfig, init_weights_
from .runner import GraphDecoder

__all__ = ["CONFIGS", "Decoder", "DecoderConfig", "GraphDecoder", "init_weights_"]
