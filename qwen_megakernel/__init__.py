"""MI355X (gfx950) Qwen3 decode megakernel with the qwen_megakernel Python API.

Same import name and exports as the reference package
(qwen_megakernel/__init__.py:1-9): importing it makes
``torch.ops.qwen_megakernel_C`` available, building the HIP library in-tree
first if it is missing or older than its sources, so that callers written
against the reference (``from qwen_megakernel.model import Decoder``,
``torch.ops.qwen_megakernel_C.decode``) run unchanged.

Set ``QMK_NO_IMPORT_LOAD=1`` to import the Python modules without touching the
HIP library (the build step itself does this).
"""

import os as _os

if _os.environ.get("QMK_NO_IMPORT_LOAD", "0") != "1":
    from qwen_megakernel.build import get_extension as _get_ext

    _get_ext()

from qwen_megakernel.model import BatchDecoder, Decoder, generate, load_weights  # noqa: E402,F401

__all__ = ["load_weights", "Decoder", "generate", "BatchDecoder"]
