"""GPU parity of the v2 operator (tjev's chunk_gated_delta_rule_v2, pallas_tpu_v2.py:541-582)
against the oracle's chunked rule (xla.py:170-262, the XLA path the v2 kernel is tested
against, test_pallas_tpu_v2.py) with torch autograd, GQA by repeating q and k as the
reference's dispatcher does for the XLA rules (__init__.py:78-80).

- fp32 ("highest"): out and d q, d k, d v, d g, d beta within max relative error 1e-5 of the
  fp64 oracle (packed segments, a segment-0 stretch, T not a multiple of the chunk);
- the model's mix, fp32 q/k with bf16 v ("high"): the bf16 bar against the oracle on the same
  values (max abs error <= 2e-2 RMS beyond the output's own rounding, gradient cosine >= 0.9999);
- the megakernel equals the v2 operator fed the megakernel's own q, k, v, g, beta (the
  oracle's preprocessing of the same raw inputs), fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import cosine, rel

pytestmark = pytest.mark.gpu


def _inputs(batch, length, hk, h, d, seed):
    rng = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32))  # noqa: E731
    q, k = f(batch, length, hk, d), f(batch, length, hk, d)
    q = q / q.norm(dim=-1, keepdim=True) * d ** -0.5
    k = k / k.norm(dim=-1, keepdim=True)
    v = f(batch, length, h, d)
    g = -torch.from_numpy(rng.uniform(0.01, 1.0, (batch, length, h)).astype(np.float32))
    beta = torch.sigmoid(f(batch, length, h))
    seg = np.ones((batch, length), np.int32)
    seg[:, length // 3:] = 2
    seg[:, length // 2: length // 2 + 9] = 0
    seg[:, 2 * length // 3:] = 3
    return q, k, v, g, beta, torch.from_numpy(seg)


def _oracle(q, k, v, g, beta, seg, chunk, dtype):
    from oracle.gdn_oracle import chunk_gated_delta_rule

    ratio = v.shape[2] // q.shape[2]
    leaves = [x.detach().to(dtype).requires_grad_(True) for x in (q, k, v, g, beta)]
    qq, kk = (x.repeat_interleave(ratio, dim=2) for x in leaves[:2])
    out, _ = chunk_gated_delta_rule(qq, kk, leaves[2], leaves[3], leaves[4], seg, chunk=chunk)
    return out, leaves


def _hip(q, k, v, g, beta, seg, chunk, precision, cot):
    from tjev_amd.v2 import chunk_gated_delta_rule_v2

    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta)]
    out = chunk_gated_delta_rule_v2(*leaves, seg.cuda(), chunk=chunk, precision=precision)
    grads = torch.autograd.grad((out.float() * cot.cuda()).sum(), leaves)
    torch.cuda.synchronize()
    return out.detach().double().cpu(), [x.double().cpu() for x in grads]


def test_v2_fp32_matches_fp64_oracle():
    q, k, v, g, beta, seg = _inputs(2, 200, 2, 4, 64, 1)
    cot = torch.randn(v.shape, generator=torch.Generator().manual_seed(2))
    out, grads = _hip(q, k, v, g, beta, seg, 64, "highest", cot)
    want, leaves = _oracle(q, k, v, g, beta, seg, 64, torch.float64)
    want_grads = torch.autograd.grad((want * cot.double()).sum(), leaves)
    print("v2 fp32: out", f"{rel(out, want.detach()):.1e}", "grads",
          [f"{rel(a, b):.1e}" for a, b in zip(grads, want_grads)], flush=True)
    assert rel(out, want.detach()) <= 1e-5
    for a, b in zip(grads, want_grads):
        assert rel(a, b) <= 1e-5 and cosine(a, b) >= 0.999999


def test_v2_mixed_dtypes_bf16_bar():
    q, k, v, g, beta, seg = _inputs(2, 256, 2, 4, 128, 3)
    vb = v.to(torch.bfloat16)
    cot = torch.randn(v.shape, generator=torch.Generator().manual_seed(4))
    out, grads = _hip(q, k, vb, g, beta, seg, 128, "high", cot)
    want, leaves = _oracle(q, k, vb.float(), g, beta, seg, 128, torch.float32)
    want_grads = torch.autograd.grad((want * cot).sum(), leaves)
    want = want.detach().double()
    rms = float(want.pow(2).mean().sqrt())
    err = float((out - want).abs().max()) / rms
    floor = float((want.to(torch.bfloat16).double() - want).abs().max()) / rms
    cos = [cosine(a, b.double()) for a, b in zip(grads, want_grads)]
    print(f"v2 mixed: out err {err:.2e} (floor {floor:.2e}), cosines {[f'{c:.6f}' for c in cos]}", flush=True)
    assert err - floor <= 2e-2 and all(c >= 0.9999 for c in cos)


def test_megakernel_equals_v2_on_its_own_inputs():
    from oracle.gdn_oracle import core_inputs
    from tjev_amd import gdn_megakernel
    from tjev_amd.testing import gdn_inputs
    from tjev_amd.v2 import chunk_gated_delta_rule_v2

    raw = gdn_inputs(batch=2, length=160, key_heads=2, value_heads=4, dim=64, seed=5, segments="random4",
                     trailing_pad=4)
    shape = dict(key_heads=2, key_dim=64, value_heads=4, value_dim=64)
    q, k, v, g, beta, seg = core_inputs(*raw, **shape)
    hk = 2
    q, k = q[:, :, ::2].contiguous(), k[:, :, ::2].contiguous()  # one copy per key head (they were repeated)
    assert q.shape[2] == hk
    mega = gdn_megakernel(*(x.cuda() for x in raw), chunk=64, precision="highest", **shape)
    v2 = chunk_gated_delta_rule_v2(q.cuda(), k.cuda(), v.cuda(), g.cuda(), beta.cuda(), seg.cuda(), chunk=64,
                                   precision="highest")
    torch.cuda.synchronize()
    assert rel(mega.double().cpu(), v2.double().cpu()) <= 1e-5
