"""gguf2bin_amd - MI355X (gfx950) decode-attention path for gguf2bin2.

The product is the C ABI of include/g2b_attn.h, built into
gguf2bin_amd/libg2b_attn.so.  This package holds its sources (csrc/, host/)
and a ctypes mirror (attn.py) used by tests and the benchmark.
"""
from .attn import (ARCH_LLAMA, ARCH_QWEN2, ARCH_QWEN3, Context, G2BError, Shape,  # noqa: F401
                   kv_bytes, kv_offset, kv_row_bytes, rope_table, stream_seed)

__all__ = ["ARCH_LLAMA", "ARCH_QWEN2", "ARCH_QWEN3", "Context", "G2BError", "Shape",
           "kv_bytes", "kv_offset", "kv_row_bytes", "rope_table", "stream_seed"]
