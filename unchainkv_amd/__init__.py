"""MI355X-native (gfx950) splitzip bf16 KV-cache codec.

A from-scratch HIP implementation of UnchainKV's Top-16 palette codec (and its
fixed6 fallback) behind the reference's C ABI and ``splitzip_cuda`` Python API.
"""

from . import codec_format  # noqa: F401

__all__ = ["codec_format", "splitzip_cuda"]
