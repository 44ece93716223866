"""Writes the golden fixtures of the GDN megakernel's parity tests (tests/golden/*.npz).

The reference commits no GDN arrays (its tests are differential on jax.random inputs), so the
fixtures come from this repository's oracle in float64 (the chunked form, equal to the token
recurrence to ~1e-12 as tests/test_oracle.py pins): inputs, the fixed upstream gradient, and
the expected output and gradients of qkv, a, b, A_log, dt_bias and the conv weight. Shapes
mirror the reference's tests (tests/kernels/test_gdn_mega.py:96-111) and the tiny fp32 benchmark config.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

# name: (B, T, Hk, H, D), chunk, cuts, mega2?, dtype, precision the GPU test runs, input style
CASES = {
    "ref_c16_mega2": ((1, 120, 2, 4, 16), 16, [16, 33, 50, 67, 95], True, "float32", "highest", "reference"),
    "ref_c16_mega1_gqa1": ((1, 120, 2, 2, 16), 16, [16, 33, 50, 67, 95], False, "float32", "highest", "reference"),
    "tiny_config1": ((1, 512, 4, 4, 64), 64, None, True, "float32", "highest", "baseline"),
    "bf16_d128_c128": ((1, 160, 2, 4, 128), 128, [64, 129], True, "bfloat16", "high", "baseline"),
}


def make(name: str) -> dict:
    from gdn_cases import case_inputs
    from oracle.gdn_oracle import reference_with_grads
    from tjev_amd.testing import cotangent, gdn_inputs

    (b, t, hk, h, d), chunk, cuts, conv, dtype, precision, style = CASES[name]
    dt = getattr(torch, dtype)
    if cuts is None:
        inputs = gdn_inputs(batch=b, length=t, key_heads=hk, value_heads=h, dim=d, dtype=dt, style=style)
        cot = cotangent(b, t, h, d)
    else:
        inputs, cot = case_inputs(b, t, hk, h, d, cuts=cuts, dtype=dt, style=style)
    want = reference_with_grads(inputs, cot, key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=conv,
                                dtype=torch.float64)
    qkv, a, bb, a_log, dt_bias, w, seg = inputs
    f32 = lambda x: x.float().numpy()  # noqa: E731  (bf16 values are exact in fp32)
    out = {
        "shape": np.array([b, t, hk, h, d, chunk, int(conv)]),
        "dtype": np.array(dtype), "precision": np.array(precision),
        "qkv": f32(qkv), "a": f32(a), "b": f32(bb), "a_log": f32(a_log), "dt_bias": f32(dt_bias),
        "w": f32(w), "seg": seg.numpy().astype(np.int32), "cot": f32(cot),
    }
    for k, v in want.items():
        out["want_" + k] = v.float().numpy()
    return out


def load(name: str) -> dict:
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def main() -> int:
    for name in CASES:
        np.savez_compressed(HERE / f"{name}.npz", **make(name))
        print("wrote", name)
    return 0


if __name__ == "__main__":
    sys.exit(main())
