"""CPU oracle for the GDN megakernel path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU in torch (float64 for truth, float32 for the reference's own
numerics), the algorithm of tjev's XLA Gated DeltaNet path that the megakernel replaces.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it,
and only as the checker or the timed CPU baseline: the product path (``tjev_amd``) never
calls it and fails loudly when its HIP library is missing.

The reference is 100% Python (JAX 0.11 / Pallas TPU); nothing of it builds or imports here
(no jax, Python 3.10), so there is no ``oracle/_ref``. Every function cites the reference
file:line it follows.
"""

from .gdn_oracle import (  # noqa: F401
    PRECISIONS,
    chunk_gated_delta_rule,
    fp64_truth,
    gated_rmsnorm,
    heads_per_block,
    l2norm,
    masks,
    recurrent_gated_delta_rule,
    reference_core,
    reference_with_grads,
    segmented_causal_conv1d,
    tap_masks,
    unit_lower_inverse,
)
