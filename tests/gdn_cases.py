"""Shared helpers of the parity tests: run the HIP operator and the CPU oracle on the same
inputs, and the reference's error metrics (tests/kernels/test_gdn_mega.py:71-86,
tests/kernels/test_gdn_long.py:116-128)."""

from __future__ import annotations

import torch

from tjev_amd.testing import cotangent, gdn_inputs

NAMES = ("qkv", "a", "b", "A_log", "dt_bias", "w")


def rel(p: torch.Tensor, q: torch.Tensor) -> float:
    """max|p - q| / max|q| (test_gdn_mega.py:71-72)."""
    p, q = p.detach().double(), q.detach().double()
    return float((p - q).abs().max() / (q.abs().max() + 1e-30))


def rel_l2(p, q) -> float:
    p, q = p.double().ravel(), q.double().ravel()
    return float((p - q).norm() / (q.norm() + 1e-30))


def cosine(p, q) -> float:
    p, q = p.double().ravel(), q.double().ravel()
    return float(p @ q / (p.norm() * q.norm() + 1e-30))


def hip_outputs(inputs, cot, *, key_heads, key_dim, value_heads, value_dim, conv=True, want_w=True, **kw):
    """out and the gradients of sum(out * cot) from the HIP operator, as float64 CPU tensors."""
    from tjev_amd import gdn_megakernel

    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda() for x in inputs)
    leaves = [x.detach().clone().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
    wl = w.detach().clone().requires_grad_(want_w and conv) if conv else None
    out = gdn_megakernel(*leaves, wl, seg, key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                         value_dim=value_dim, **kw)
    loss = (out.float() * cot.cuda()).sum()
    targets = leaves + ([wl] if (wl is not None and wl.requires_grad) else [])
    grads = torch.autograd.grad(loss, targets)
    torch.cuda.synchronize()
    result = {"out": out.detach().double().cpu()}
    result.update({n: g.detach().double().cpu() for n, g in zip(NAMES, grads)})
    return result


def oracle_outputs(inputs, cot, *, key_heads, key_dim, value_heads, value_dim, conv=True, dtype=torch.float32,
                   rule="chunked"):
    from oracle.gdn_oracle import reference_with_grads

    return reference_with_grads(inputs, cot, key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                                value_dim=value_dim, conv=conv, rule=rule, dtype=dtype)


def case_inputs(batch, length, hk, h, d, *, cuts=None, seed=0, dtype=torch.float32, style="reference",
                trailing_pad=5, segments=None, taps=4, dk=None, dv=None):
    """test_gdn_mega._inputs: 4 random cuts (or ``cuts``) and 5 trailing padding tokens; head
    widths d, or dk (q, k) and dv (v)."""
    if segments is None:
        segments = "cuts" if cuts is not None else "random4"
    inputs = gdn_inputs(batch=batch, length=length, key_heads=hk, value_heads=h, dim=d, seed=seed, dtype=dtype,
                        segments=segments, cuts=cuts, trailing_pad=trailing_pad, style=style, taps=taps,
                        key_dim=dk, value_dim=dv)
    cot = cotangent(batch, length, h, dv or d)
    return inputs, cot
