"""The model head dimension (Dk = Dv = 128, chunk 128) at every precision (GPU): the chunk
kernels and the forward scan at this shape (its own kernel, k_scan_fwd_split) under fp32
("highest") against the fp64 oracle at the fp32 bar, with packed segments (the scans' chunk
ranges split at resets) and trailing padding; "mixed" and one-pass "bf16" at the bars of the
small-head precision test; a row run in two calls (initial state and conv history) equal to
the row run at once.
"""

import pytest
import torch

from gdn_cases import case_inputs, cosine, hip_outputs, oracle_outputs, rel, rel_l2

pytestmark = pytest.mark.gpu

# test_gdn_mega.py:89-91 (as in test_gpu_parity.py)
TOL = {"out": 1e-5, "qkv": 1e-5, "a": 1e-5, "b": 1e-5, "A_log": 5e-5, "dt_bias": 5e-5, "w": 1e-5}
SHAPE = dict(key_heads=2, key_dim=128, value_heads=4, value_dim=128)


@pytest.mark.parametrize("cuts", [None, [100, 177, 300, 301]], ids=["one-segment", "cuts"])
def test_d128_fp32_matches_oracle(cuts):
    inputs, cot = case_inputs(1, 520, 2, 4, 128, cuts=cuts, segments="cuts" if cuts else "one")
    print(f"D=128 C=128 fp32 cuts={cuts}", flush=True)
    got = hip_outputs(inputs, cot, chunk=128, precision="highest", **SHAPE)
    want = oracle_outputs(inputs, cot, dtype=torch.float64, **SHAPE)
    errors = {k: rel(got[k], want[k]) for k in got}
    print("D=128 fp32 vs fp64:", {k: f"{v:.1e}" for k, v in errors.items()})
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


@pytest.mark.parametrize("precision", ["mixed", "bf16"])
def test_d128_precision_modes(precision):
    inputs, cot = case_inputs(1, 384, 2, 4, 128, cuts=[100, 177])
    print(f"D=128 C=128 {precision}", flush=True)
    got = hip_outputs(inputs, cot, chunk=128, precision=precision, **SHAPE)
    want = oracle_outputs(inputs, cot, **SHAPE)
    l2 = {k: rel_l2(got[k], want[k]) for k in got}
    cos = {k: cosine(got[k], want[k]) for k in got}
    print(precision, {k: f"{l2[k]:.1e}/{cos[k]:.6f}" for k in got})
    per_token = ("out", "qkv", "b", "w")
    if precision == "mixed":
        assert all(l2[k] < 2e-3 for k in per_token), l2
        assert l2["a"] < 1e-2 and all(cos[k] > 0.999 for k in got), (l2, cos)
    else:
        assert all(l2[k] < 1e-2 for k in per_token), l2
        assert l2["a"] < 1e-1 and cos["a"] > 0.995, (l2, cos)


def test_d128_two_pieces_equal_one_run_fp32():
    """The second piece's forward scan starts from the first piece's final state (and its conv
    rows); outputs and every gradient equal those of the row run at once."""
    from tjev_amd import gdn_megakernel

    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(2, 400, 2, 4, 128, cuts=[60, 200, 330], trailing_pad=5,
                                                           segments="cuts")
    kw = dict(SHAPE, chunk=128, precision="highest")
    t1 = 256  # whole chunks
    leaves = lambda: [x.detach().clone().cuda().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias, w)]  # noqa: E731
    lv = leaves()
    segc, cotc = seg.cuda(), cot.cuda()
    full = gdn_megakernel(*lv[:5], lv[5], segc, **kw)
    g_full = torch.autograd.grad((full.float() * cotc).sum(), lv)
    lp = leaves()
    out1, state, hist = gdn_megakernel(*[x[:, :t1] for x in lp[:3]], lp[3], lp[4], lp[5], segc[:, :t1],
                                       output_final_state=True, **kw)
    out2 = gdn_megakernel(*[x[:, t1:] for x in lp[:3]], lp[3], lp[4], lp[5], segc[:, t1:], initial_state=state,
                          initial_conv=hist, **kw)
    pieces = torch.cat([out1, out2], 1)
    g_pieces = torch.autograd.grad((pieces.float() * cotc).sum(), lp)
    torch.cuda.synchronize()
    errs = {"out": rel(pieces.cpu(), full.cpu())}
    errs.update({n: rel(p.cpu(), f.cpu()) for n, p, f in zip(("qkv", "a", "b", "A_log", "dt_bias", "w"), g_pieces,
                                                              g_full)})
    print("D=128 pieces vs one run:", {k: f"{v:.1e}" for k, v in errs.items()})
    for n, e in errs.items():
        assert e <= TOL[n], (n, errs)
