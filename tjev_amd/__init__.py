"""tjev_amd: tjev's Gated DeltaNet megakernel (mega2) on MI355X (gfx950).

``gdn_megakernel`` / ``gdn_core_mega`` keep the reference's operator signature; the work runs
in hand-written HIP kernels behind the C ABI of ``libtjev_gdn.so`` (include/tjev_gdn.h).
``gated_rmsnorm`` is the GDN output norm (``gdn_megakernel_normed``: the core with that norm in its
output kernel); ``GatedDeltaNetBlock`` composes them with the
merged-LoRA projections (hipBLASLt GEMMs) into the reference's GDN layer.
"""

from .gdn import (GdnPlan, gdn_core_mega, gdn_megakernel, gdn_megakernel_normed, heads_per_block,  # noqa: F401
                  kernel_inverse)
from .norm import GatedRMSNorm, gated_rmsnorm  # noqa: F401
from .block import GatedDeltaNetBlock, LoRALinear, grouped  # noqa: F401

__all__ = ["GdnPlan", "gdn_core_mega", "gdn_megakernel", "gdn_megakernel_normed", "heads_per_block", "kernel_inverse", "GatedRMSNorm",
           "gated_rmsnorm", "GatedDeltaNetBlock", "LoRALinear", "grouped"]
