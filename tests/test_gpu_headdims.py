"""Head dims the kernels do not hold as they are (GPU): Dk != Dv, which the reference accepts
(pallas_tpu_mega.py:597-615, pallas_tpu_v2.py:528-538), widths other than 16, 32, 64, 128 (up
to 128), and value heads wider than 128 (the reference's TPU kernels take multiples of 128:
Dv = 256 with Dk = 128). The Python operators run the first two zero-padded to the next
compiled dim (run_dim in tjev_amd/gdn.py) and the wide value heads as groups of value columns
(value_groups), and cut or join the outputs; every output and gradient is held to the fp32 bar
against the oracle, which computes at the given widths.
"""

from __future__ import annotations

import pytest
import torch

from gdn_cases import NAMES, case_inputs, hip_outputs, oracle_outputs, rel

pytestmark = pytest.mark.gpu

SHAPES = [  # (Hk, Dk, H, Dv)
    (2, 64, 4, 128),
    (2, 128, 4, 64),
    (1, 48, 2, 48),
    (2, 32, 2, 96),
    (2, 128, 4, 256),  # two groups of 128 value columns
    (1, 32, 2, 300),   # groups of 128, 128 and 44 (padded)
]


@pytest.mark.parametrize("conv", [True, False], ids=["mega2", "mega1"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"Dk{s[1]}-Dv{s[3]}" for s in SHAPES])
def test_padded_head_dims_fp32(shape, conv):
    hk, dk, h, dv = shape
    inputs, cot = case_inputs(1, 200, hk, h, 0, dk=dk, dv=dv, cuts=[63, 65, 130], seed=3)
    kw = dict(key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv, conv=conv)
    got = hip_outputs(inputs, cot, chunk=64, precision="highest", **kw)
    want = oracle_outputs(inputs, cot, dtype=torch.float64, **kw)
    errs = {k: rel(got[k], want[k]) for k in got}
    print(f"Dk={dk} Dv={dv} conv={conv}:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    for k in ("out",) + NAMES:
        if k in errs:
            assert errs[k] <= (5e-5 if k in ("A_log", "dt_bias") else 1e-5), (k, errs[k])


@pytest.mark.parametrize("shape", [(2, 64, 4, 128), (2, 128, 4, 96), (2, 64, 4, 256), (1, 128, 2, 192)],
                         ids=["Dk64-Dv128", "Dk128-Dv96", "Dk64-Dv256", "Dk128-Dv192"])
def test_padded_head_dims_state_and_norm(shape):
    """The continued sequence (initial state and conv history in, final ones out, gradients
    through all of them) and the normed operator at padded head dims, fp32, against the oracle
    (the state's run: the fp64 chunked rule with the initial state; the norm: gated_rmsnorm)."""
    from oracle.gdn_oracle import chunk_gated_delta_rule, core_inputs, gated_rmsnorm
    from tjev_amd import gdn_megakernel, gdn_megakernel_normed

    hk, dk, h, dv = shape
    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(1, 150, hk, h, 0, dk=dk, dv=dv, segments="one", seed=5)
    gen = torch.Generator().manual_seed(7)
    init = 0.3 * torch.randn((1, h, dk, dv), generator=gen)
    kw = dict(key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv, chunk=64, precision="highest")
    leaves = [x.cuda().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias, w, init)]
    out, final, cs = gdn_megakernel(*leaves[:6], seg.cuda(), initial_state=leaves[6], output_final_state=True, **kw)
    assert final.shape == (1, h, dk, dv) and cs.shape == (1, 3, qkv.shape[-1])
    d_fin = torch.randn(final.shape, generator=gen)
    grads = torch.autograd.grad((out * cot.cuda()).sum() + (final * d_fin.cuda()).sum(), leaves)
    # the oracle: conv, gates and norms in fp64, then the chunked rule from the initial state
    ref = [x.double().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias, w, init)]
    q, k, v, g, beta, sg = core_inputs(*ref[:6], seg, key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv,
                                       dtype=torch.float64)
    r_out, r_fin = chunk_gated_delta_rule(q, k, v, g, beta, sg, initial_state=ref[6], chunk=64)
    r_grads = torch.autograd.grad((r_out * cot.double()).sum() + (r_fin * d_fin.double()).sum(), ref)
    errs = {"out": rel(out.cpu(), r_out), "final": rel(final.cpu(), r_fin)}
    errs.update({f"d{i}": rel(x.cpu(), y) for i, (x, y) in enumerate(zip(grads, r_grads))})
    # the conv history: the raw rows T-3 .. T-1 (one segment)
    errs["conv_state"] = rel(cs.cpu(), qkv[:, -3:])
    print(f"state Dk={dk} Dv={dv}:", {k_: f"{v_:.1e}" for k_, v_ in errs.items()}, flush=True)
    for k_, v_ in errs.items():
        assert v_ <= (5e-5 if k_ in ("d3", "d4") else 1e-5), (k_, v_)
    # the normed operator: the padded core, then the norm over the Dv lanes
    z = torch.randn((1, 150, h, dv), generator=gen)
    nw = 1 + 0.1 * torch.randn(dv, generator=gen)
    y = gdn_megakernel_normed(*(x.cuda() for x in (qkv, a, b, a_log, dt_bias, w)), seg.cuda(), z.cuda(), nw.cuda(),
                              **kw)
    fresh, _ = chunk_gated_delta_rule(q.detach(), k.detach(), v.detach(), g.detach(), beta.detach(), sg, chunk=64)
    want = gated_rmsnorm(fresh.float(), z, nw, 1e-6)  # (the normed call starts from a zero state)
    want = torch.where((seg > 0)[..., None, None], want, torch.zeros(()))
    err = rel(y.cpu(), want)
    print(f"normed Dk={dk} Dv={dv}: {err:.1e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("dv", [96, 200])
def test_padded_head_dims_v2(dv):
    """The v2 operator at Dk != Dv with a state (Dv = 200: two groups of value columns, the
    second padded): against the fp64 chunked rule."""
    from oracle.gdn_oracle import chunk_gated_delta_rule
    from tjev_amd.v2 import chunk_gated_delta_rule as v2_rule

    gen = torch.Generator().manual_seed(9)
    B, T, hk, dk, h = 1, 141, 2, 64, 4
    q, k = (torch.nn.functional.normalize(torch.randn((B, T, hk, dk), generator=gen), dim=-1) for _ in range(2))
    q = q * dk ** -0.5
    v = torch.randn((B, T, h, dv), generator=gen)
    g = -torch.rand((B, T, h), generator=gen)
    beta = torch.rand((B, T, h), generator=gen)
    s0 = 0.3 * torch.randn((B, h, dk, dv), generator=gen)
    seg = torch.ones((B, T), dtype=torch.int32)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    out, fin = v2_rule(*leaves[:5], seg.cuda(), initial_state=leaves[5], chunk=64)
    cot = torch.randn(out.shape, generator=gen)
    d_fin = torch.randn(fin.shape, generator=gen)
    grads = torch.autograd.grad((out * cot.cuda()).sum() + (fin * d_fin.cuda()).sum(), leaves)
    ref = [x.double().requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    rep = lambda x: x.repeat_interleave(h // hk, dim=2)  # noqa: E731
    r_out, r_fin = chunk_gated_delta_rule(rep(ref[0]), rep(ref[1]), *ref[2:5], seg, initial_state=ref[5], chunk=64)
    r_grads = torch.autograd.grad((r_out * cot.double()).sum() + (r_fin * d_fin.double()).sum(), ref)
    errs = {"out": rel(out.cpu(), r_out), "final": rel(fin.cpu(), r_fin)}
    errs.update({n: rel(x.cpu(), y) for n, x, y in zip(("q", "k", "v", "g", "beta", "s0"), grads, r_grads)})
    print(f"v2 Dk=64 Dv={dv}:", {k_: f"{v_:.1e}" for k_, v_ in errs.items()}, flush=True)
    for k_, v_ in errs.items():
        assert v_ <= 1e-5, (k_, v_)


@pytest.mark.parametrize("shape,inplace", [((2, 64, 4, 128), False), ((1, 48, 2, 48), True),
                                           ((2, 64, 4, 256), True), ((1, 32, 2, 160), False)],
                         ids=["Dk64-Dv128", "Dk48-Dv48-inplace", "Dk64-Dv256-inplace", "Dk32-Dv160"])
def test_padded_head_dims_prefill_then_decode(shape, inplace):
    """Serving at padded head dims: a prefill of T tokens then three decode steps equal the
    megakernel over T + 3 tokens (fp32), the state updated in place when asked."""
    from tjev_amd import gdn_megakernel
    from tjev_amd.serve import gdn_decode_step, gdn_prefill

    hk, dk, h, dv = shape
    length, extra = 150, 3
    (qkv, a, b, a_log, dt_bias, w, seg), _ = case_inputs(2, length + extra, hk, h, 0, dk=dk, dv=dv,
                                                         segments="one", seed=11)
    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda() for x in (qkv, a, b, a_log, dt_bias, w, seg))
    kw = dict(key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv)
    full = gdn_megakernel(qkv, a, b, a_log, dt_bias, w, seg, chunk=64, precision="highest", **kw)
    _, state, hist = gdn_prefill(qkv[:, :length], a[:, :length], b[:, :length], a_log, dt_bias, w, seg[:, :length],
                                 chunk=64, precision="highest", **kw)
    assert state.shape == (2, h, dk, dv) and hist.shape == (2, 3, qkv.shape[-1])
    outs = []
    for t in range(length, length + extra):
        o, hist, st = gdn_decode_step(qkv[:, t], a[:, t], b[:, t], a_log, dt_bias, w, hist, state, inplace=inplace,
                                      **kw)
        assert (st.data_ptr() == state.data_ptr()) == inplace
        state = st
        outs.append(o)
    torch.cuda.synchronize()
    err = rel(torch.stack(outs, 1).double().cpu(), full[:, length:].double().cpu())
    print(f"prefill + decode Dk={dk} Dv={dv}: {err:.1e}", flush=True)
    assert err <= 1e-5


def test_key_dims_above_128_raise():
    """Dk above 128 has no padded or split form: every operator refuses it before any launch."""
    from tjev_amd import gdn_megakernel
    from tjev_amd.serve import gdn_prefill
    from tjev_amd.v2 import chunk_gated_delta_rule_v2

    hk, dk, h, dv, T = 1, 256, 1, 256, 16
    qkv = torch.zeros((1, T, 2 * hk * dk + h * dv), device="cuda")
    a = b = torch.zeros((1, T, h), device="cuda")
    a_log = dt_bias = torch.zeros(h, device="cuda")
    seg = torch.ones((1, T), dtype=torch.int32, device="cuda")
    kw = dict(key_heads=hk, key_dim=dk, value_heads=h, value_dim=dv)
    with pytest.raises(ValueError, match="key dims up to 128"):
        gdn_megakernel(qkv, a, b, a_log, dt_bias, None, seg, **kw)
    with pytest.raises(ValueError, match="key dims up to 128"):
        gdn_prefill(qkv, a, b, a_log, dt_bias, None, seg, **kw)
    q = torch.zeros((1, T, hk, dk), device="cuda")
    with pytest.raises(ValueError, match="key dims up to 128"):
        chunk_gated_delta_rule_v2(q, q, torch.zeros((1, T, h, dv), device="cuda"), a, b, seg)
