"""GPU parity of the gated RMSNorm (tjev's GatedRMSNorm, norms.py:36-62, and the padding select of
gdn.py:163) through the C ABI against the oracle's ``gated_rmsnorm`` with torch autograd (the
oracle is pinned against HF ``Qwen3_5RMSNormGated``, forward and backward, in test_oracle.py).

fp32: y and every gradient within max relative error 1e-5 of the fp64 oracle. bf16: against the
oracle run at bf16 semantics on the CPU (the reference's roundings), at least 99% of y
bit-identical, within one bf16 ulp everywhere, max abs error <= 2e-2 * RMS, gradient cosine
>= 0.99999; against fp64 truth, no worse than those roundings and gradient cosine >= 0.9999.
Padding tokens: y, d_x and d_gate exactly 0."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import cosine, rel

pytestmark = pytest.mark.gpu


def _inputs(tokens, heads, dim, *, seed=0, pad=0, scale=1.0):
    rng = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32))  # noqa: E731
    x = f(tokens, heads, dim) * scale
    z = f(tokens, heads, dim)
    w = 1 + 0.1 * f(dim)
    dy = f(tokens, heads, dim)
    seg = torch.ones(tokens, dtype=torch.int32)
    if pad:
        seg[-pad:] = 0
        seg[: min(pad, tokens)] = 2
    return x, z, w, dy, seg


def _hip(x, z, w, dy, seg, dtype, *, flat=False, use_seg=True):
    from tjev_amd.norm import gated_rmsnorm

    t, h, d = x.shape
    shape = (t, h * d) if flat else (t, h, d)
    xs = x.to(dtype).reshape(shape).cuda().requires_grad_(True)
    zs = z.to(dtype).reshape(shape).cuda().requires_grad_(True)
    ws = w.cuda().requires_grad_(True)
    y = gated_rmsnorm(xs, zs, ws, 1e-6, heads=h if flat else None,
                      segment_ids=seg.cuda() if use_seg else None)
    grads = torch.autograd.grad(y, (xs, zs, ws), dy.to(dtype).reshape(shape).cuda())
    torch.cuda.synchronize()
    return [v.detach().cpu().reshape(x.shape) if v.dim() > 1 else v.detach().cpu() for v in (y, *grads)]


def _oracle(x, z, w, dy, seg, dtype):
    from oracle.gdn_oracle import gated_rmsnorm

    xs = x.to(dtype).requires_grad_(True)
    zs = z.to(dtype).requires_grad_(True)
    ws = w.to(torch.float64 if dtype == torch.float64 else torch.float32).requires_grad_(True)
    y = gated_rmsnorm(xs, zs, ws, 1e-6)
    y = torch.where((seg > 0)[:, None, None], y, torch.zeros_like(y))
    grads = torch.autograd.grad(y, (xs, zs, ws), dy.to(dtype))
    return [v.detach() for v in (y, *grads)]


SHAPES = [(37, 3, 16), (64, 4, 32), (100, 2, 64), (257, 16, 128), (50, 2, 256), (1, 1, 128)]


@pytest.mark.parametrize("shape", SHAPES)
def test_norm_fp32_matches_fp64_oracle(shape):
    x, z, w, dy, seg = _inputs(*shape, seed=sum(shape), pad=min(5, shape[0] // 4))
    got = _hip(x, z, w, dy, seg, torch.float32)
    want = _oracle(x.double(), z.double(), w.double(), dy.double(), seg, torch.float64)
    for name, g, h in zip(("y", "d_x", "d_gate", "d_weight"), got, want):
        assert rel(g, h) <= 1e-5, (name, rel(g, h))


@pytest.mark.parametrize("shape", SHAPES)
def test_norm_bf16_matches_oracle_roundings(shape):
    x, z, w, dy, seg = _inputs(*shape, seed=1 + sum(shape), pad=min(5, shape[0] // 4))
    y, dx, dz, dw = _hip(x, z, w, dy, seg, torch.bfloat16)
    oy, odx, odz, odw = _oracle(x, z, w, dy, seg, torch.bfloat16)
    assert y.dtype == dx.dtype == dz.dtype == torch.bfloat16
    same = float((y.view(torch.int16) == oy.view(torch.int16)).double().mean())
    assert same >= 0.99, same
    ulp = oy.float().abs() * 2.0 ** -7 + 1e-30
    assert bool(((y.float() - oy.float()).abs() <= ulp).all())
    for name, g, h in (("d_x", dx, odx), ("d_gate", dz, odz), ("d_weight", dw, odw)):
        assert cosine(g, h) >= 0.99999, (name, cosine(g, h))
    # the benchmark's bf16 bar against the reference's semantics (the oracle at bf16)
    assert float((y.double() - oy.double()).abs().max()) <= 2e-2 * float(oy.double().pow(2).mean().sqrt())
    # against fp64 truth of the same bf16 inputs: no worse than the reference's own roundings
    # (its intermediate cast of the normalized value to bf16 costs up to a bf16 ulp before the
    # output rounding), and gradient cosine >= 0.9999
    ty, tdx, tdz, tdw = _oracle(x.to(torch.bfloat16).double(), z.to(torch.bfloat16).double(), w.double(),
                                dy.to(torch.bfloat16).double(), seg, torch.float64)
    own = float((oy.double() - ty).abs().max())
    assert float((y.double() - ty).abs().max()) <= own + 2.0 ** -8 * float(ty.abs().max())
    for name, g, h in (("d_x", dx, tdx), ("d_gate", dz, tdz), ("d_weight", dw, tdw)):
        assert cosine(g, h) >= 0.9999, (name, cosine(g, h))


def test_norm_padding_tokens_are_exact_zeros():
    x, z, w, dy, seg = _inputs(40, 4, 64, seed=3, pad=7)
    for dtype in (torch.float32, torch.bfloat16):
        y, dx, dz, _ = _hip(x, z, w, dy, seg, dtype)
        pad = seg <= 0
        assert int(pad.sum()) == 7
        for v in (y, dx, dz):
            assert bool((v[pad] == 0).all())
            assert bool((v[~pad] != 0).any())


def test_norm_flat_layout_equals_per_head():
    x, z, w, dy, seg = _inputs(66, 4, 128, seed=4)
    for dtype in (torch.float32, torch.bfloat16):
        a = _hip(x, z, w, dy, seg, dtype)
        b = _hip(x, z, w, dy, seg, dtype, flat=True)
        for u, v in zip(a, b):
            assert torch.equal(u, v)


def test_norm_without_segments_and_small_scale():
    """No segment ids (no select), and inputs small enough that eps matters."""
    x, z, w, dy, seg = _inputs(80, 2, 128, seed=5, scale=1e-4)
    got = _hip(x, z, w, dy, seg, torch.float32, use_seg=False)
    want = _oracle(x.double(), z.double(), w.double(), dy.double(), torch.ones_like(seg), torch.float64)
    for name, g, h in zip(("y", "d_x", "d_gate", "d_weight"), got, want):
        assert rel(g, h) <= 1e-5, (name, rel(g, h))


def test_norm_model_shape_bf16():
    """The 0.8B layer's output norm: B*T = 16384 tokens, 16 heads of 128 (many backward
    workgroups per partial, the fixed-grid stride loop)."""
    x, z, w, dy, seg = _inputs(4 * 4096, 16, 128, seed=6, scale=0.05)
    y, dx, dz, dw = _hip(x, z, w, dy, seg, torch.bfloat16)
    oy, odx, odz, odw = _oracle(x, z, w, dy, seg, torch.bfloat16)
    same = float((y.view(torch.int16) == oy.view(torch.int16)).double().mean())
    assert same >= 0.99, same
    for name, g, h in (("d_x", dx, odx), ("d_gate", dz, odz), ("d_weight", dw, odw)):
        assert cosine(g, h) >= 0.99999, (name, cosine(g, h))
    assert rel(dw, odw) <= 1e-4


def test_norm_zero_tokens():
    from tjev_amd.norm import gated_rmsnorm

    x = torch.zeros(0, 2, 64, device="cuda", requires_grad=True)
    w = torch.ones(64, device="cuda", requires_grad=True)
    y = gated_rmsnorm(x, x.detach(), w)
    (dw,) = torch.autograd.grad(y.sum(), (w,), allow_unused=True)
    torch.cuda.synchronize()
    assert y.shape == (0, 2, 64)
    assert dw is not None and bool((dw == 0).all())


FUSED_CASES = [
    # (B, T, Hk, H, D, chunk, dtype): the model's head shape in bf16, and small fp32 shapes
    (2, 300, 2, 4, 128, 128, torch.bfloat16),
    (1, 150, 2, 4, 16, 32, torch.float32),
    (1, 200, 2, 4, 64, 64, torch.float32),
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[f"D{c[4]}C{c[5]}-{str(c[6])[6:]}" for c in FUSED_CASES])
def test_norm_in_the_output_kernel_equals_the_separate_norm(case):
    """gdn_megakernel_normed (the gated RMSNorm's forward in the core's output kernel) against
    gdn_megakernel followed by gated_rmsnorm, on inputs with segment cuts and trailing padding:
    y equals the separate norm's up to the order of its sum of squares (fp32: 1e-6 relative;
    bf16: at least 99.9% bit-identical, the rest one bf16 ulp apart); padding tokens exactly 0;
    every gradient (the core's inputs, the gate, the norm weight) bitwise the same: the backward
    is the same norm backward on the same saved out, so out is bitwise the same too."""
    from gdn_cases import case_inputs
    from tjev_amd import gdn_megakernel, gdn_megakernel_normed
    from tjev_amd.norm import gated_rmsnorm

    batch, length, hk, h, d, chunk, dtype = case
    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(batch, length, hk, h, d, dtype=dtype,
                                                            cuts=[chunk - 1, chunk + 2])
    gen = torch.Generator().manual_seed(3)
    z = torch.randn((batch, length, h, d), generator=gen).to(dtype)
    nw = 1 + 0.1 * torch.randn(d, generator=gen)
    kw = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, chunk=chunk,
              precision="high" if dtype == torch.bfloat16 else "highest")
    print(f"fused norm case {case}", flush=True)

    def leaves():
        return [t.detach().clone().cuda().requires_grad_(t.is_floating_point())
                for t in (qkv, a, b, a_log, dt_bias, w, z, nw)]

    segc, dy = seg.cuda(), cot.to(dtype).cuda()
    l1 = leaves()
    y1 = gdn_megakernel_normed(*l1[:6], segc, l1[6], l1[7], 1e-6, **kw)
    g1 = torch.autograd.grad(y1, l1, dy)
    l2 = leaves()
    out2 = gdn_megakernel(*l2[:6], segc, **kw)
    y2 = gated_rmsnorm(out2, l2[6], l2[7], 1e-6, segment_ids=segc)
    g2 = torch.autograd.grad(y2, l2, dy)
    torch.cuda.synchronize()
    y1, y2 = y1.detach(), y2.detach()
    pad = seg.cuda() <= 0
    assert bool((y1[pad] == 0).all())
    if dtype == torch.float32:
        assert rel(y1.cpu(), y2.cpu()) <= 1e-6
    else:
        same = (y1 == y2).float().mean().item()
        ulp = (y2.float().abs().clamp_min(1e-30).log2().floor() - 7).exp2()
        worst = float(((y1.float() - y2.float()).abs() / ulp).max())
        print(f"bit-identical {same:.5f}, worst {worst:.2f} ulp")
        assert same >= 0.999 and worst <= 1.0
    names = ["qkv", "a", "b", "A_log", "dt_bias", "w", "gate", "norm_weight"]
    for n, x1, x2 in zip(names, g1, g2):
        assert torch.equal(x1, x2), n
