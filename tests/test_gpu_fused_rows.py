"""The forward building q and v from the raw qkv rows (bf16 I/O, a conv of 1 to 4 taps, chunk =
head dim = 128: v in the chunk kernel, and q in the output kernel when each key head has one
value head; k_prep then skips those rows and the forward's workspace has none) against the
same kernels reading q and v from k_prep's rows (the LDS-poison debug library, which keeps those
rows, with TJEV_GDN_UNFUSED=1), bit for bit (the fused run under TJEV_GDN_POISON=1: NaN wherever
the kernels read memory they did not write; the unfused one with NaN in every LDS array before
its kernels run): outputs,
final state, conv state and every gradient (both routes end in the same backward, whose k_prep
writes the rows). The cases are those where the conv's halo crosses a chunk edge: segments
starting 1, 2 and 3 tokens before a chunk and 1-token segments there, rows continued from an
initial state and conv history, a padded tail, every conv width, each precision, the blocked
inverse with T kept, the 0.8B heads, and GQA (2 value heads per key head: v only) with the 9B
heads.
"""

from __future__ import annotations

import os

import pytest
import torch

pytestmark = pytest.mark.gpu

D = 128
CUTS = (1, 2, 125, 126, 127, 128, 129, 253, 254, 256, 257, 384, 511)


def _inputs(seed, batch, length, hk, h, taps, cont):
    gen = torch.Generator().manual_seed(seed)
    width = (2 * hk + h) * D
    qkv = torch.randn((batch, length, width), generator=gen).bfloat16()
    a = torch.randn((batch, length, h), generator=gen).bfloat16()
    b = torch.randn((batch, length, h), generator=gen).bfloat16()
    a_log = torch.rand(h, generator=gen)
    dt_bias = torch.randn(h, generator=gen)
    w = 0.5 * torch.randn((taps, width), generator=gen)
    seg = torch.ones((batch, length), dtype=torch.int32)
    for c in CUTS:
        if c < length:
            seg[:, c:] += 1
    seg[0, length - 7:] = 0  # a padded tail
    if batch > 1:
        seg[1, length - 140:] = 0  # a padded chunk and more
    cot = torch.randn((batch, length, h, D), generator=gen).bfloat16()
    extra = {}
    if cont:
        extra["initial_state"] = 0.1 * torch.randn((batch, h, D, D), generator=gen)
        if taps > 1:
            extra["initial_conv"] = torch.randn((batch, taps - 1, width), generator=gen).bfloat16()
        extra["output_final_state"] = True
    dev = torch.device("cuda")
    return ([x.to(dev) for x in (qkv, a, b, a_log, dt_bias, w, seg)], cot.to(dev),
            {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in extra.items()})


def _call(inputs, cot, extra, **kw):
    from tjev_amd import gdn_megakernel

    leaves = [x.clone().requires_grad_(True) for x in inputs[:6]]
    res = gdn_megakernel(*leaves[:5], leaves[5], inputs[6], chunk=128, **kw, **extra)
    out, more = (res[0], [x for x in res[1:] if x is not None]) if isinstance(res, tuple) else (res, [])
    grads = torch.autograd.grad((out.float() * cot.float()).sum(), leaves)
    torch.cuda.synchronize()
    return [out.detach()] + [x.detach() for x in more] + list(grads)


def _run(inputs, cot, extra, unfused, **kw):
    from tjev_amd import _lib

    if unfused:  # the debug library: k_prep's rows kept, and read with TJEV_GDN_UNFUSED=1
        os.environ["TJEV_GDN_UNFUSED"] = "1"
        try:
            with _lib.library(_lib.LDS_POISON_PATH) as lib:
                assert lib.tjev_gdn_lds_poison() == 1
                return _call(inputs, cot, extra, **kw)
        finally:
            os.environ.pop("TJEV_GDN_UNFUSED", None)
    os.environ["TJEV_GDN_POISON"] = "1"  # NaN in the workspace: a read of rows no kernel wrote shows
    try:
        return _call(inputs, cot, extra, **kw)
    finally:
        os.environ.pop("TJEV_GDN_POISON", None)


CASES = [(taps, cont, "high", {}, (2, 2)) for taps in (1, 2, 3, 4) for cont in (False, True)]
CASES += [(4, True, p, {}, (2, 2)) for p in ("highest", "mixed", "bf16")]
CASES += [(4, True, "high", {"inverse": "blocked", "residuals": "tinv"}, (2, 2)),
          (3, False, "high", {"residuals": "all"}, (2, 2)), (4, True, "high", {}, (16, 16)),
          (4, True, "high", {}, (2, 4)), (2, False, "mixed", {}, (2, 4)), (4, True, "high", {}, (16, 32))]


@pytest.mark.parametrize(("taps", "cont", "precision", "kw", "heads"), CASES,
                         ids=[f"K{t}-{'cont' if c else 'fresh'}-{p}{'-' + '-'.join(k.values()) if k else ''}-{h[0]}x{h[1]}"
                              for t, c, p, k, h in CASES])
def test_fused_rows_equal_k_prep_rows(taps, cont, precision, kw, heads):
    hk, h = heads
    length = 700 if hk == 2 else 400
    inputs, cot, extra = _inputs(taps + 10 * cont, 2, length, hk, h, taps, cont)
    shape = dict(key_heads=hk, key_dim=D, value_heads=h, value_dim=D, precision=precision, **kw)
    print(f"fused rows: taps={taps} cont={cont} {precision} {kw} heads={heads} T={length}", flush=True)
    fused = _run(inputs, cot, extra, False, **shape)
    plain = _run(inputs, cot, extra, True, **shape)
    names = ["out"] + (["final_state"] + (["conv_state"] if taps > 1 else []) if cont else []) + \
        ["qkv", "a", "b", "A_log", "dt_bias", "w"]
    assert len(names) == len(fused) == len(plain)
    for name, x, y in zip(names, fused, plain):
        assert bool(torch.isfinite(x.float()).all()), name
        assert torch.equal(x, y), (name, float((x.float() - y.float()).abs().max()))


def _random_case(rng):
    """A row layout drawn at random: length 1 to 600, 1 to 3 rows, 1 to 4 key heads with 1 or 2
    value heads each, 1 to 4 conv taps, cuts anywhere (chunk edges included) and trailing padding,
    fresh or continued rows, any precision and residual policy."""
    batch, length = int(rng.integers(1, 4)), int(rng.integers(1, 601))
    hk = int(rng.choice([1, 2, 4]))
    h = hk * int(rng.choice([1, 2]))
    taps = int(rng.integers(1, 5))
    cont = bool(rng.integers(0, 2))
    gen = torch.Generator().manual_seed(int(rng.integers(0, 2**31)))
    width = (2 * hk + h) * D
    qkv = torch.randn((batch, length, width), generator=gen).bfloat16()
    a, b = (torch.randn((batch, length, h), generator=gen).bfloat16() for _ in range(2))
    a_log, dt_bias = torch.rand(h, generator=gen), torch.randn(h, generator=gen)
    w = 0.5 * torch.randn((taps, width), generator=gen)
    seg = torch.ones((batch, length), dtype=torch.int32)
    for row in range(batch):
        edges = [c for c in (126, 127, 128, 129, 255, 256, 384) if c < length]
        cuts = sorted(set(rng.choice(range(1, length), size=min(length - 1, 4), replace=False).tolist() if length > 1
                          else []) | set(rng.choice(edges, size=min(len(edges), 2), replace=False).tolist() if edges else []))
        for c in cuts:
            seg[row, c:] += 1
        pad = int(rng.integers(0, min(length, 140)))
        if pad:
            seg[row, length - pad:] = 0
    cot = torch.randn((batch, length, h, D), generator=gen).bfloat16()
    extra = {}
    if cont:
        extra["initial_state"] = 0.1 * torch.randn((batch, h, D, D), generator=gen)
        if taps > 1:
            extra["initial_conv"] = torch.randn((batch, taps - 1, width), generator=gen).bfloat16()
        extra["output_final_state"] = True
    dev = torch.device("cuda")
    kw = dict(key_heads=hk, key_dim=D, value_heads=h, value_dim=D,
              precision=str(rng.choice(["high", "highest", "mixed", "bf16"])),
              residuals=str(rng.choice(["states", "tinv", "all"])), inverse=str(rng.choice(["doubling", "blocked"])))
    return ([x.to(dev) for x in (qkv, a, b, a_log, dt_bias, w, seg)], cot.to(dev),
            {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in extra.items()}, kw, taps, cont)


@pytest.mark.parametrize("index", range(12))
def test_fused_rows_random_layouts(index):
    """12 layouts drawn with seed 2027: fused and unfused runs bit-identical."""
    import numpy as np

    rng = np.random.default_rng([2027, index])
    inputs, cot, extra, kw, taps, cont = _random_case(rng)
    print(f"fused rows random {index}: B={inputs[0].shape[0]} T={inputs[0].shape[1]} taps={taps} cont={cont} {kw}",
          flush=True)
    fused = _run(inputs, cot, extra, False, **kw)
    plain = _run(inputs, cot, extra, True, **kw)
    assert len(fused) == len(plain)
    for i, (x, y) in enumerate(zip(fused, plain)):
        assert bool(torch.isfinite(x.float()).all()), i
        assert torch.equal(x, y), (i, float((x.float() - y.float()).abs().max()))


def test_fused_rows_at_the_08b_shape():
    """The 0.8B layer shape (4 rows of 4096 tokens, 16 key and value heads) with packed segments
    and a continued first row's history: fused and unfused bit for bit."""
    inputs, cot, extra = _inputs(42, 4, 4096, 16, 16, 4, True)
    kw = dict(key_heads=16, key_dim=D, value_heads=16, value_dim=D, precision="high")
    print("fused rows at the 0.8B shape", flush=True)
    fused = _run(inputs, cot, extra, False, **kw)
    plain = _run(inputs, cot, extra, True, **kw)
    for i, (x, y) in enumerate(zip(fused, plain)):
        assert bool(torch.isfinite(x.float()).all()), i
        assert torch.equal(x, y), (i, float((x.float() - y.float()).abs().max()))
