"""MI355X (gfx950) Qwen3 decode megakernel with the qwen_megakernel Python API.

Exports the reference's names (qwen_megakernel/__init__.py:7-9).  The HIP
library is built by ``qwen_megakernel_amd.build.build()`` (or on first use by
``Decoder``); importing the package does not compile anything.
"""

from .model import BatchDecoder, Decoder, generate, load_weights  # noqa: F401

__all__ = ["load_weights", "Decoder", "generate", "BatchDecoder"]
