"""The reference's tests of its v2 kernel (tests/kernels/test_pallas_tpu.py:114-232) on this
build's v2 operator (tjev_amd.v2.chunk_gated_delta_rule_v2), at their head dim (128), their
inputs (g = -softplus(N(0,1) - 1), beta = sigmoid(N(0,1) + 1), 4 segment boundaries anywhere
in each row) and their bars, against the oracle's chunked rule in fp64 (the reference compares
with its fp32 XLA rule): out and the gradients of q, k, v, g and beta.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import cosine, rel

pytestmark = pytest.mark.gpu


def _gdn_inputs(batch, length, heads, seed=0, dim=128):
    rng = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s))  # noqa: E731
    q = f(batch, length, heads, dim)
    q = q / q.norm(dim=-1, keepdim=True) * dim ** -0.5
    k = f(batch, length, heads, dim)
    k = k / k.norm(dim=-1, keepdim=True)
    v = f(batch, length, heads, dim)
    g = -torch.nn.functional.softplus(f(batch, length, heads) - 1.0)
    beta = torch.sigmoid(f(batch, length, heads) + 1.0)
    rows = []
    for _ in range(batch):  # boundaries anywhere, not only on chunk edges
        cuts = np.sort(rng.choice(np.arange(1, length), size=4, replace=False))
        rows.append(np.searchsorted(cuts, np.arange(length), side="right") + 1)
    return q, k, v, g, beta, torch.from_numpy(np.stack(rows).astype(np.int32))


def _run(inputs, cot, *, chunk, precision="highest", **kw):
    """(out, [dq, dk, dv, dg, dbeta]) of the HIP v2 operator, float64 on the CPU."""
    from tjev_amd.v2 import chunk_gated_delta_rule_v2

    q, k, v, g, beta, seg = inputs
    leaves = [x.float().cuda().requires_grad_(True) for x in (q, k, v, g, beta)]
    out = chunk_gated_delta_rule_v2(*leaves, seg.cuda(), chunk=chunk, precision=precision, **kw)
    grads = torch.autograd.grad((out.float() * cot.cuda()).sum(), leaves)
    return out.detach().double().cpu(), [x.double().cpu() for x in grads]


def _reference(inputs, cot):
    """The oracle's chunked rule in fp64, q and k repeated over each group of value heads."""
    from oracle.gdn_oracle import chunk_gated_delta_rule

    q, k, v, g, beta, seg = inputs
    leaves = [x.double().requires_grad_(True) for x in (q, k, v, g, beta)]
    ratio = v.shape[2] // q.shape[2]
    qq, kk = (x.repeat_interleave(ratio, dim=2) for x in leaves[:2])
    out, _ = chunk_gated_delta_rule(qq, kk, *leaves[2:], seg.long(), chunk=64)
    grads = torch.autograd.grad((out * cot.double()).sum(), leaves)
    return out.detach(), list(grads)


def _check(inputs, tol, grad_tol, **kw):
    cot = torch.from_numpy(np.random.default_rng(9).standard_normal(inputs[2].shape))
    got, got_g = _run(inputs, cot.float(), **kw)
    want, want_g = _reference(inputs, cot)
    errors = {"out": rel(got, want)} | {n: rel(a, b) for n, a, b in zip("qkvgb", got_g, want_g)}
    print(kw, {k: f"{v:.1e}" for k, v in errors.items()}, flush=True)
    assert errors["out"] < tol, errors
    for name in "qkvgb":
        assert errors[name] < grad_tol, (name, errors)
    return got_g, want_g


@pytest.mark.parametrize(("shape", "chunk"), [((1, 128, 2), 64), ((2, 200, 4), 64), ((1, 256, 8), 128)],
                         ids=["1x128x2-C64", "2x200x4-C64", "1x256x8-C128"])
def test_v2_matches_reference(shape, chunk):
    """test_pallas_tpu.py:114-127: fp32, out and every gradient within 1e-5."""
    _check(_gdn_inputs(*shape), 1e-5, 1e-5, chunk=chunk)


@pytest.mark.parametrize("inverse", ["doubling", "blocked"])
def test_v2_inverse_options_match_reference(inverse):
    """test_pallas_tpu.py:130-143 and :211-229: both in-kernel inverse forms, fp32, 1e-5."""
    _check(_gdn_inputs(2, 200, 4), 1e-5, 1e-5, chunk=64, inverse=inverse)


def test_v2_mixed_precision():
    """test_pallas_tpu.py:154-169: "mixed" (one bf16 pass on the state path): out within 3e-2,
    gradients within 6e-2, and the gate gradient summed per head (what A_log and dt_bias
    see) at cosine > 0.9999."""
    got_g, want_g = _check(_gdn_inputs(2, 256, 4), 3e-2, 6e-2, chunk=64, precision="mixed")
    assert cosine(got_g[3].sum((0, 1)), want_g[3].sum((0, 1))) > 0.9999


@pytest.mark.parametrize("precision", ["highest", "mixed"])
def test_v2_gqa_reads_key_heads(precision):
    """test_pallas_tpu.py:172-192: 2 value heads per key head against the rule on repeated q
    and k; dq and dk summed over each group; 1e-5 (fp32) or 3e-2 (mixed), gradients 2x."""
    q, k, v, g, beta, seg = _gdn_inputs(2, 200, 4)
    tol = 1e-5 if precision == "highest" else 3e-2
    _check((q[:, :, :2], k[:, :, :2], v, g, beta, seg), tol, 2 * tol, chunk=64, precision=precision)


@pytest.mark.parametrize(("shape", "chunk", "kw"), [
    ((2, 200, 4), 64, {"inverse": "blocked"}), ((1, 256, 4), 128, {"inverse": "blocked"}),
    ((1, 100, 4), 16, {"inverse": "blocked"}), ((2, 200, 8), 64, {"heads_per_step": 4}),
    ((2, 200, 8), 64, {"heads_per_step": 16, "inverse": "blocked"}),
], ids=["2x200x4-C64-blocked", "1x256x4-C128-blocked", "1x100x4-C16-blocked", "2x200x8-C64-hb4",
        "2x200x8-C64-hb16-blocked"])
def test_v2_options_match_reference(shape, chunk, kw):
    """test_pallas_tpu.py:211-229: the inverse and heads-per-step options give the same
    function, fp32, 1e-5."""
    _check(_gdn_inputs(*shape), 1e-5, 1e-5, chunk=chunk, **kw)
