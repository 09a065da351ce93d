"""MI355X (gfx950) attention hot path of the inference engine.

``engine.attention.flash_attention`` and ``engine.cache`` keep the reference
engine's call signatures; ``engine.attention.paged_attention`` is the added
paged decode / speculative-verify entry. All compute runs in the HIP library
``libcie_attn.so`` (see ``engine._lib``).
"""

from engine.attention import flash_attention, paged_attention  # noqa: F401
