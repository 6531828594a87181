"""pocketlm_amd: MI355X (gfx950) backend for PocketLM's quantized-decode hot path.

``pocketlm_amd.native`` mirrors the hot-path functions of the reference's
``pcketlm.native`` module (FP8 block-scaled dequant / GEMV / SwiGLU MLP /
weighted MoE, Q4 dequant / GEMV / MoE, row8 GEMV, DeepSeek MoE session and
routers) on top of the C ABI of ``libpocketlm_hip.so``
(``include/pocketlm_hip.h``).  Build the library with
``python -m pocketlm_amd.build``.
"""

__version__ = "0.1.0"

__all__ = ["__version__"]
