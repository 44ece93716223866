"""GPU parity of the GDN block (``GatedDeltaNet.__call__``, src/tjev/model/gdn.py:126-164, flat
norm, merged LoRA on every projection) against the oracle's ``gdn_block`` with torch autograd.

- The merged-LoRA custom backward (lora.py:320-366: dx = sum dy W'^T, dA = s x^T (dy B^T),
  dB = s (x A)^T dy) against torch autograd of the same fp32 projections on the GPU.
- fp32 (precision "highest"): the block's output and the gradients of x and of every adapter
  within max relative error 1e-5 of the fp64 oracle (the adapter gradients, sums over all
  tokens, within 1e-4), packed segments and padding included.
- bf16 (precision "high"): against the oracle on the same bf16 values with the activations
  stored in bf16 between the stages as the reference's bf16 layer stores them (the core in
  fp32), the output's max abs error beyond its own bf16 rounding <= 2e-2 RMS and gradient
  cosine >= 0.9999; at the 4B block benchmark shape (hidden 2560, 16/32 heads of 128, r64) the
  output's error beyond one bf16 spacing of each element <= 2e-2 RMS.
"""

from __future__ import annotations

import pytest
import torch

from gdn_cases import cosine, rel

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=64, key_heads=2, key_dim=16, value_heads=4, value_dim=16)


def _block(dtype, precision, chunk, rank, seed=0, **shape):
    from tjev_amd.block import GatedDeltaNetBlock

    return GatedDeltaNetBlock(**shape, rank=rank, dtype=dtype, chunk=chunk, precision=precision, seed=seed,
                              b_std=0.05)


def _oracle_params(blk, dtype):
    f = lambda t: t.detach().cpu().to(dtype).requires_grad_(t.requires_grad)  # noqa: E731
    names = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj")
    p = {n: (f(getattr(blk, n).weight), f(getattr(blk, n).lora_a), f(getattr(blk, n).lora_b), getattr(blk, n).scale)
         for n in names}
    p.update(conv=blk.conv.cpu().to(dtype), a_log=blk.a_log.cpu().to(dtype), dt_bias=blk.dt_bias.cpu().to(dtype),
             norm=blk.norm_weight.cpu().to(dtype))
    return p


def _inputs(batch, length, hidden, seed, dtype):
    from tjev_amd.testing import cut_segments

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((batch, length, hidden), generator=gen).to(dtype)
    seg = torch.stack([torch.from_numpy(cut_segments(length, [length // 3, length // 2 + 7], 5)) for _ in range(batch)])
    dy = torch.randn((batch, length, hidden), generator=gen)
    return x, seg.to(torch.int32), dy


def _bf16_excess(got, want):
    """The output's error beyond one bf16 spacing of each element, relative to the output RMS:
    both outputs are bf16 values (the reference's bf16 layer rounds its last projection), so
    one rounding apart is a spacing; past it, the error is the kernels' own."""
    spacing = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(2.0 ** -126))) - 7)
    rms = float(want.pow(2).mean().sqrt())
    return float(((got - want).abs() - spacing).clamp_min(0).max()) / rms


def _run_hip(blk, x, seg, dy):
    xs = x.cuda().requires_grad_(True)
    out = blk(xs, seg.cuda())
    params = blk.parameters()
    grads = torch.autograd.grad((out.float() * dy.cuda()).sum(), [xs, *params])
    torch.cuda.synchronize()
    return out.detach().double().cpu(), [g.double().cpu() for g in grads]


def _run_oracle(blk, x, seg, dy, dtype, shape, io_dtype=None):
    from oracle.gdn_oracle import gdn_block

    p = _oracle_params(blk, dtype)
    xs = x.to(dtype).requires_grad_(True)
    out = gdn_block(xs, seg, p, key_heads=shape["key_heads"], key_dim=shape["key_dim"],
                    value_heads=shape["value_heads"], value_dim=shape["value_dim"], dtype=dtype, chunk=blk.chunk,
                    io_dtype=io_dtype)
    leaves = [xs] + [t for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj") for t in p[n][1:3]]
    grads = torch.autograd.grad((out.to(dtype) * dy.to(dtype)).sum(), leaves)
    return out.detach().double(), [g.double() for g in grads]


def test_merged_lora_backward_matches_autograd():
    from tjev_amd.block import LoRALinear, grouped

    gen = torch.Generator().manual_seed(1)
    x = torch.randn(300, 96, generator=gen).cuda()
    lins, ref_leaves = [], []
    for out in (128, 40, 4):
        w = (torch.randn(96, out, generator=gen) * 0.1).cuda()
        a = (torch.randn(96, 8, generator=gen) * 0.3).cuda().requires_grad_(True)
        b = (torch.randn(8, out, generator=gen) * 0.3).cuda().requires_grad_(True)
        lins.append(LoRALinear(w, a, b, 2.5))
        ref_leaves.append((w, a.detach().clone().requires_grad_(True), b.detach().clone().requires_grad_(True)))
    dys = [torch.randn(300, l.weight.shape[1], generator=gen).cuda() for l in lins]
    xg = x.clone().requires_grad_(True)
    ys = grouped(xg, *lins)
    got = torch.autograd.grad(sum((y * d).sum() for y, d in zip(ys, dys)), [xg] + [t for l in lins for t in (l.lora_a, l.lora_b)])
    xr = x.clone().requires_grad_(True)
    ys_ref = [xr @ (w + 2.5 * (a @ b)) for w, a, b in ref_leaves]
    want = torch.autograd.grad(sum((y * d).sum() for y, d in zip(ys_ref, dys)), [xr] + [t for _, a, b in ref_leaves for t in (a, b)])
    for y, yr in zip(ys, ys_ref):
        assert rel(y.detach().double().cpu(), yr.detach().double().cpu()) <= 1e-5
    for g, h in zip(got, want):
        assert rel(g.double().cpu(), h.double().cpu()) <= 1e-5


@pytest.mark.parametrize("k", [16384, 8192 + 4096, 1000])
def test_split_k_adapter_products(k):
    """The adapters' token-contracted products (a^T b over K tokens, fp32 accumulation) cut into
    K parts at long K: equal to one fp32-accumulated product to fp32 rounding, for a contiguous a
    and for a column slice of a wider a (the split of x A); K = 12288 cuts in 4, 1000 not at all."""
    from tjev_amd.block import _mm32, _mm32_tn

    gen = torch.Generator().manual_seed(2)
    wide = torch.randn(k, 256, generator=gen).to(torch.bfloat16).cuda()
    b = torch.randn(k, 640, generator=gen).to(torch.bfloat16).cuda()
    exact = (wide.double().t() @ b.double())
    for a, want in ((wide, exact), (wide[:, 64:128], exact[64:128])):
        got = _mm32_tn(a, b)
        plain = _mm32(a.t(), b)
        assert got.dtype == torch.float32 and got.shape == want.shape
        err, err_plain = rel(got.double(), want), rel(plain.double(), want)
        print(f"K={k} {tuple(a.shape)}: split {err:.1e}, plain {err_plain:.1e}", flush=True)
        assert err <= 1e-5 and err_plain <= 1e-5


def test_block_fp32_matches_fp64_oracle():
    blk = _block(torch.float32, "highest", 16, 8, **SMALL)
    x, seg, dy = _inputs(2, 150, SMALL["hidden"], 3, torch.float32)
    out, grads = _run_hip(blk, x, seg, dy)
    want_out, want = _run_oracle(blk, x.double(), seg, dy, torch.float64, SMALL)
    print("fp32 block: out", rel(out, want_out), "grads", [f"{rel(g, h):.1e}" for g, h in zip(grads, want)], flush=True)
    assert rel(out, want_out) <= 1e-5
    assert rel(grads[0], want[0]) <= 1e-5
    for g, h in zip(grads[1:], want[1:]):
        assert rel(g, h) <= 1e-4 and cosine(g, h) >= 0.999999


def test_block_bf16_matches_oracle():
    shape = dict(hidden=256, key_heads=2, key_dim=64, value_heads=4, value_dim=64)
    blk = _block(torch.bfloat16, "high", 64, 16, seed=2, **shape)
    x, seg, dy = _inputs(2, 256, shape["hidden"], 5, torch.bfloat16)
    out, grads = _run_hip(blk, x, seg, dy)
    want_out, want = _run_oracle(blk, x.float(), seg, dy, torch.float32, shape, io_dtype=torch.bfloat16)
    rms = float(want_out.pow(2).mean().sqrt())
    err = float((out - want_out).abs().max()) / rms
    floor = float((want_out.to(torch.bfloat16).double() - want_out).abs().max()) / rms
    cos = [cosine(g, h) for g, h in zip(grads, want)]
    print(f"bf16 block: out err {err:.2e} (rounding floor {floor:.2e}), cosines {[f'{c:.6f}' for c in cos]}", flush=True)
    assert err - floor <= 2e-2
    assert all(c >= 0.9999 for c in cos), cos


def test_block_bf16_config5_shape():
    """The 4B block benchmark config at its own shape (src/tjev/model/gdn.py:126-164 with the LoRA
    layouts of campaign/bench.py:383-390): hidden 2560, Hk/H 16/32, Dk = Dv = C = 128, merged
    LoRA r64 on all five projections (A ~ N(0, 1/r), B ~ N(0, 0.01)), precision "high", one row
    of 512 tokens with packed segments and padding, against the oracle block on the same bf16
    values with the activations stored in bf16 between the stages: the output within the bf16
    bar, dx and all ten adapter gradients at cosine >= 0.9999."""
    shape = dict(hidden=2560, key_heads=16, key_dim=128, value_heads=32, value_dim=128)
    from tjev_amd.block import GatedDeltaNetBlock

    blk = GatedDeltaNetBlock(**shape, rank=64, dtype=torch.bfloat16, chunk=128, precision="high", seed=4)
    x, seg, dy = _inputs(1, 512, shape["hidden"], 6, torch.bfloat16)
    print("config-5 block: B=1 T=512 hidden 2560 16/32 heads D=C=128 r64", flush=True)
    out, grads = _run_hip(blk, x, seg, dy)
    want_out, want = _run_oracle(blk, x.float(), seg, dy, torch.float32, shape, io_dtype=torch.bfloat16)
    rms = float(want_out.pow(2).mean().sqrt())
    err = float((out - want_out).abs().max()) / rms
    excess = _bf16_excess(out, want_out)
    cos = [cosine(g, h) for g, h in zip(grads, want)]
    print(f"config-5 block: out max err {err:.2e} RMS, beyond one bf16 spacing {excess:.2e} RMS, rel-l2 "
          f"{float((out - want_out).norm() / want_out.norm()):.2e}, cosines {[f'{c:.6f}' for c in cos]}", flush=True)
    assert excess <= 2e-2
    assert len(cos) == 11 and all(c >= 0.9999 for c in cos), cos
