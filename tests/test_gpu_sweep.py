"""A seeded random sweep of the operator against the fp64 oracle (GPU), at the fp32 bar of
precision "highest": batch, length (ragged and shorter than a chunk included), key/value heads
(GQA), head dims (the compiled 16 .. 128 and padded ones: Dk != Dv, 48, 96), chunk (16 .. 128),
conv taps (mega1 with none, mega2 with 2 .. 5), segment cuts with padding, the inverse form, the
residual policy, and a continued sequence (initial state in, final state out, gradients through
both). Each case prints its parameters before it runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import case_inputs, rel

pytestmark = pytest.mark.gpu

DIMS = [(16, 16), (32, 32), (64, 64), (128, 128), (64, 128), (128, 64), (48, 48), (32, 96), (16, 32)]


def _cases(n=24, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dk, dv = DIMS[rng.integers(len(DIMS))]
        hk = int(rng.choice([1, 2]))
        out.append(dict(
            batch=int(rng.choice([1, 2])), length=int(rng.integers(1, 300)), hk=hk, h=hk * int(rng.choice([1, 2])),
            dk=dk, dv=dv, chunk=int(rng.choice([16, 32, 64, 128])), taps=int(rng.choice([0, 2, 3, 4, 5])),
            cuts=int(rng.integers(0, 4)), inverse=str(rng.choice(["doubling", "blocked"])),
            residuals=str(rng.choice(["states", "tinv", "all"])), state=bool(rng.integers(2)), seed=i))
    return out


CASES = _cases()


def _label(c):
    return (f"B{c['batch']}T{c['length']}Hk{c['hk']}H{c['h']}Dk{c['dk']}Dv{c['dv']}C{c['chunk']}K{c['taps']}"
            f"-cuts{c['cuts']}-{c['inverse']}-{c['residuals']}" + ("-state" if c["state"] else ""))


@pytest.mark.parametrize("case", CASES, ids=[_label(c) for c in CASES])
def test_sweep_fp32(case):
    from oracle.gdn_oracle import chunk_gated_delta_rule, core_inputs
    from tjev_amd import gdn_megakernel

    c = case
    B, T, hk, h, dk, dv = c["batch"], c["length"], c["hk"], c["h"], c["dk"], c["dv"]
    rng = np.random.default_rng(c["seed"])
    cuts = sorted(set(int(x) for x in rng.integers(1, max(T, 2), c["cuts"]))) if T > 1 and c["cuts"] else []
    taps = c["taps"]
    print(f"sweep case {_label(c)} cuts={cuts}", flush=True)
    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(B, T, hk, h, 0, dk=dk, dv=dv, cuts=cuts, segments="cuts",
                                                           trailing_pad=int(rng.integers(0, 4)) if T > 8 else 0,
                                                           seed=c["seed"], taps=max(taps, 1))
    conv = taps > 0
    gen = torch.Generator().manual_seed(c["seed"])
    init = (0.3 * torch.randn((B, h, dk, dv), generator=gen)) if c["state"] else None
    hist = torch.randn((B, taps - 1, qkv.shape[-1]), generator=gen) if c["state"] and taps > 1 else None
    d_fin = torch.randn((B, h, dk, dv), generator=gen) if c["state"] else None
    # the HIP operator
    leaves = [x.cuda().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
    wl = w.cuda().requires_grad_(True) if conv else None
    extra = [x.cuda().requires_grad_(True) for x in (init, hist) if x is not None]
    kw = dict(key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv, chunk=c["chunk"], precision="highest",
              inverse=c["inverse"], residuals=c["residuals"])
    if c["state"]:
        out, fin, _ = gdn_megakernel(*leaves, wl, seg.cuda(), initial_state=extra[0],
                                     initial_conv=extra[1] if hist is not None else None, output_final_state=True, **kw)
        loss = (out * cot.cuda()).sum() + (fin * d_fin.cuda()).sum()
    else:
        out = gdn_megakernel(*leaves, wl, seg.cuda(), **kw)
        loss = (out * cot.cuda()).sum()
    targets = leaves + ([wl] if conv else []) + extra
    got = [out.detach()] + ([fin.detach()] if c["state"] else []) + list(torch.autograd.grad(loss, targets))
    # the oracle in fp64: the composition, then the chunked rule (from the initial state)
    ref = [x.double().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
    rw = w.double().requires_grad_(True) if conv else None
    rextra = [x.double().requires_grad_(True) for x in (init, hist) if x is not None]
    r_qkv = ref[0]
    if hist is not None:  # the history rows go in front of the row, read by token 0's segment
        r_in = torch.cat([rextra[1], r_qkv], dim=1)
        r_seg = torch.cat([seg[:, :1].expand(B, taps - 1), seg], dim=1)
    else:
        r_in, r_seg = r_qkv, seg
    q, k, v, g, beta, _ = core_inputs(r_in, torch.cat([ref[1][:, :1].expand(B, r_in.shape[1] - T, h), ref[1]], 1),
                                      torch.cat([ref[2][:, :1].expand(B, r_in.shape[1] - T, h), ref[2]], 1),
                                      ref[3], ref[4], rw, r_seg, key_heads=hk, key_dim=dk, value_heads=h,
                                      value_dim=dv, conv=conv, dtype=torch.float64)
    cut = r_in.shape[1] - T  # drop the history rows again
    q, k, v, g, beta = (x[:, cut:] for x in (q, k, v, g, beta))
    r_out, r_fin = chunk_gated_delta_rule(q, k, v, g, beta, seg, initial_state=rextra[0] if c["state"] else None,
                                          chunk=c["chunk"])
    r_loss = (r_out * cot.double()).sum() + ((r_fin * d_fin.double()).sum() if c["state"] else 0.0)
    r_targets = ref + ([rw] if conv else []) + rextra
    want = [r_out.detach()] + ([r_fin.detach()] if c["state"] else []) + list(
        torch.autograd.grad(r_loss, r_targets, allow_unused=True))
    names = ["out"] + (["final"] if c["state"] else []) + ["qkv", "a", "b", "A_log", "dt_bias"] + (
        ["w"] if conv else []) + (["init"] if c["state"] else []) + (["hist"] if hist is not None else [])
    errs = {}
    for n, x, y in zip(names, got, want):
        y = torch.zeros_like(x, dtype=torch.float64) if y is None else y
        assert bool(torch.isfinite(x).all()), n
        y = y.detach()
        # relative to the oracle's largest value; absolute where it is all zero (a final state of
        # a padding segment, a gradient no output reads)
        errs[n] = rel(x.double().cpu(), y) if float(y.abs().max()) > 0 else float(x.abs().max())
    print("   errors:", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (5e-5 if n in ("A_log", "dt_bias") else 1e-5), (n, e)
