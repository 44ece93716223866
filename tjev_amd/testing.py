"""Seeded synthetic inputs of the GDN megakernel: the benchmark configurations and the
reference tests' shapes (tests/kernels/test_gdn_mega.py:25-41).

numpy PCG64 streams (jax.random's threefry streams cannot be regenerated without jax): seed 0
for the inputs, seed 9 for the upstream gradient (test_gdn_mega.py:77).
"""

from __future__ import annotations

import math

import numpy as np
import torch

# name: (B, T, Hk, H, D, chunk, activation dtype, precision, segments)
CONFIGS = {
    "tiny": dict(batch=1, length=512, key_heads=4, value_heads=4, dim=64, chunk=64, dtype=torch.float32,
                 precision="highest", segments="one"),
    "0.8B": dict(batch=4, length=4096, key_heads=16, value_heads=16, dim=128, chunk=128, dtype=torch.bfloat16,
                 precision="high", segments="one"),
    "9B": dict(batch=2, length=8192, key_heads=16, value_heads=32, dim=128, chunk=128, dtype=torch.bfloat16,
               precision="high", segments="one"),
    "varlen": dict(batch=1, length=16384, key_heads=16, value_heads=16, dim=128, chunk=128,
                   dtype=torch.bfloat16, precision="high", segments="geometric"),
}


def geometric_segments(length: int, rng: np.random.Generator, mean: int = 300, lo: int = 16,
                       hi: int = 4096) -> np.ndarray:
    """Segment ids 1..n for one packed row: lengths ~ Geometric(p = 1/mean) clipped to
    [lo, hi], drawn until they cover ``length``; the last one is truncated."""
    ids = np.zeros(length, np.int32)
    pos, sid = 0, 1
    while pos < length:
        n = int(np.clip(rng.geometric(1.0 / mean), lo, hi))
        ids[pos: pos + n] = sid
        pos += n
        sid += 1
    return ids


def cut_segments(length: int, cuts, trailing_pad: int = 0) -> np.ndarray:
    """ids 1.. split at ``cuts``, then ``trailing_pad`` tokens of segment 0
    (test_gdn_mega.py:36-40)."""
    row = np.searchsorted(np.asarray(cuts), np.arange(length), side="right") + 1
    if trailing_pad:
        row[length - trailing_pad:] = 0
    return row.astype(np.int32)


def gdn_inputs(*, batch: int, length: int, key_heads: int, value_heads: int, dim: int, taps: int = 4,
               seed: int = 0, dtype=torch.float32, segments="one", cuts=None, trailing_pad: int = 0,
               style: str = "baseline", device="cpu", key_dim: int | None = None, value_dim: int | None = None):
    """(qkv, a, b, a_log, dt_bias, conv_w, segment_ids) as torch tensors.

    style "baseline" (the benchmark configurations): qkv, a, b, dt_bias ~ N(0,1), A_log ~ U(0, ln 16),
    conv w ~ N(0, 0.5). style "reference" (test_gdn_mega.py:25-41): A_log, dt_bias ~ 0.5 N(0,1).
    ``segments``: "one" (id 1 everywhere), "geometric" (varlen packing), "cuts" (``cuts``,
    plus ``trailing_pad`` segment-0 tokens) or "random4" (4 random cuts per row, as the
    reference tests draw them). qkv, a and b are cast to ``dtype``; the rest stay fp32.
    ``key_dim`` / ``value_dim`` (default ``dim``) give the heads' widths in qkv."""
    rng = np.random.default_rng(seed)
    width = 2 * key_heads * (key_dim or dim) + value_heads * (value_dim or dim)
    qkv = rng.standard_normal((batch, length, width), dtype=np.float32)
    a = rng.standard_normal((batch, length, value_heads), dtype=np.float32)
    b = rng.standard_normal((batch, length, value_heads), dtype=np.float32)
    if style == "baseline":
        a_log = rng.uniform(0.0, math.log(16.0), value_heads).astype(np.float32)
        dt_bias = rng.standard_normal(value_heads, dtype=np.float32)
    else:
        a_log = 0.5 * rng.standard_normal(value_heads, dtype=np.float32)
        dt_bias = 0.5 * rng.standard_normal(value_heads, dtype=np.float32)
    w = 0.5 * rng.standard_normal((taps, width), dtype=np.float32)
    rows = []
    for _ in range(batch):
        if segments == "one":
            row = np.ones(length, np.int32)
        elif segments == "geometric":
            row = geometric_segments(length, rng)
        elif segments == "cuts":
            row = cut_segments(length, cuts, trailing_pad)
        elif segments == "random4":
            c = np.sort(rng.choice(np.arange(1, length), 4, replace=False))
            row = cut_segments(length, c, trailing_pad)
        else:
            raise ValueError(f"segments={segments!r}")
        rows.append(row)
    seg = np.stack(rows)
    t = lambda x, dt=torch.float32: torch.from_numpy(x).to(dt).to(device)  # noqa: E731
    return (t(qkv, dtype), t(a, dtype), t(b, dtype), t(a_log), t(dt_bias), t(w),
            torch.from_numpy(seg).to(device))


def cotangent(batch: int, length: int, value_heads: int, dim: int, seed: int = 9, device="cpu") -> torch.Tensor:
    """The fixed random upstream gradient [B, T, H, Dv] (fp32)."""
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal((batch, length, value_heads, dim), dtype=np.float32)).to(device)
