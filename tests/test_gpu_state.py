"""A sequence continued from a given state (GPU): the chunked rule's ``initial_state`` and final
state (xla.py:170-262; test_gated_delta_rule.py:61-73's continuation) on the megakernel and the
v2 operator, through the C ABI's _cont entry points.

- pieces: a row run in two calls, the second from the first's final state and conv history,
  equals the row run at once -- outputs and the gradients of every input, the gradient crossing
  between the pieces through the state and the conv rows;
- the oracle: the v2 operator with an initial state against the fp64 chunked rule with that
  state, out, final state and every gradient (the initial state's included), at the fp32 bar;
- serving: a prefill in pieces equals the prefill of the whole prompt (bf16, model heads).
"""

import pytest
import torch

from gdn_cases import case_inputs, cosine, rel

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _leaves(*xs):
    return [x.detach().clone().cuda().requires_grad_(x.is_floating_point()) for x in xs]


@pytest.mark.parametrize("t1", [96, 77], ids=["whole-chunks", "ragged"])
@pytest.mark.parametrize("cuts", [None, [30, 110, 130]], ids=["one-segment", "cuts"])
@pytest.mark.parametrize("conv", [True, False], ids=["mega2", "mega1"])
def test_megakernel_in_two_pieces_equals_one_run(conv, cuts, t1):
    """The first piece ends after whole chunks (96) or inside a chunk (77 = 4 * 16 + 13: the
    kernels' padded tail carries its final state, and the final state's gradient enters there)."""
    from tjev_amd import gdn_megakernel

    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(2, 141, 2, 4, 16, cuts=cuts, trailing_pad=3 if cuts else 0,
                                                           segments="cuts" if cuts else "one")
    kw = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16, chunk=16, precision="highest")
    print(f"pieces conv={conv} cuts={cuts} t1={t1}", flush=True)
    lv = _leaves(qkv, a, b, a_log, dt_bias, w)
    wl = lv[5] if conv else None
    segc, cotc = seg.cuda(), cot.cuda()
    full = gdn_megakernel(*lv[:5], wl, segc, **kw)
    g_full = torch.autograd.grad((full.float() * cotc).sum(), lv[:5] + ([wl] if conv else []))
    lp = _leaves(qkv, a, b, a_log, dt_bias, w)
    wp = lp[5] if conv else None
    first = [x[:, :t1] for x in lp[:3]]
    second = [x[:, t1:] for x in lp[:3]]
    out1, state, hist = gdn_megakernel(*first, lp[3], lp[4], wp, segc[:, :t1], output_final_state=True, **kw)
    out2 = gdn_megakernel(*second, lp[3], lp[4], wp, segc[:, t1:], initial_state=state, initial_conv=hist, **kw)
    pieces = torch.cat([out1, out2], 1)
    g_pieces = torch.autograd.grad((pieces.float() * cotc).sum(), lp[:5] + ([wp] if conv else []))
    torch.cuda.synchronize()
    assert rel(pieces.cpu(), full.cpu()) <= TOL
    names = ["qkv", "a", "b", "A_log", "dt_bias", "w"]
    errs = {n: rel(p.cpu(), f.cpu()) for n, p, f in zip(names, g_pieces, g_full)}
    print("pieces vs one run:", {k: f"{v:.1e}" for k, v in errs.items()})
    for n, e in errs.items():
        assert e <= (5e-5 if n in ("A_log", "dt_bias") else TOL), (n, errs)


@pytest.mark.parametrize("T", [128, 141], ids=["whole-chunks", "ragged"])
def test_v2_initial_state_matches_the_oracle(T):
    """chunk_gated_delta_rule(q, k, v, g, beta, seg, initial_state) -> (out, final_state) against
    the fp64 chunked rule with the same state (xla.py:170-262), with segment cuts (the state is
    read by token 0's segment only) and GQA; every gradient, the initial state's and the one
    through the final state included, also at a length inside a chunk (141 = 8 * 16 + 13)."""
    import numpy as np

    from oracle.gdn_oracle import chunk_gated_delta_rule as ref_rule
    from oracle.gdn_oracle import l2norm
    from tjev_amd.v2 import chunk_gated_delta_rule

    print(f"v2 with an initial state, T={T}", flush=True)
    rng = np.random.default_rng(5)
    B, H, D = 2, 4, 16
    f = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32))  # noqa: E731
    q, k = l2norm(f(B, T, H, D)) * D ** -0.5, l2norm(f(B, T, H, D))
    v = f(B, T, H, D)
    g = -torch.nn.functional.softplus(f(B, T, H))
    beta = torch.sigmoid(f(B, T, H))
    s0 = 0.5 * f(B, H, D, D)
    seg = torch.ones((B, T), dtype=torch.int32)
    seg[1, 40:] = 2
    cot, cot_s = f(B, T, H, D), f(B, H, D, D)
    leaves = _leaves(q, k, v, g, beta, s0)
    out, fin = chunk_gated_delta_rule(*leaves[:5], seg.cuda(), initial_state=leaves[5], chunk=16)
    grads = torch.autograd.grad((out * cot.cuda()).sum() + (fin * cot_s.cuda()).sum(), leaves)
    torch.cuda.synchronize()
    ref_leaves = [x.double().requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    rout, rfin = ref_rule(*ref_leaves[:5], seg.long(), initial_state=ref_leaves[5], chunk=16)
    rgrads = torch.autograd.grad((rout * cot.double()).sum() + (rfin * cot_s.double()).sum(), ref_leaves)
    errs = {"out": rel(out.cpu(), rout), "final": rel(fin.cpu(), rfin)}
    errs.update({n: rel(x.cpu(), y) for n, x, y in zip(("q", "k", "v", "g", "beta", "initial_state"), grads, rgrads)})
    print("v2 with an initial state vs fp64:", {k: f"{v:.1e}" for k, v in errs.items()})
    for n, e in errs.items():
        assert e <= TOL, (n, errs)
    for x, y in zip(grads, rgrads):
        assert cosine(x.cpu(), y) >= 0.999999


def test_prefill_in_pieces_equals_the_whole_prompt():
    """Serving: gdn_prefill of a prompt in two pieces (the second from the first's state and conv
    history) leaves the same output, state and conv history as one prefill (bf16, D = C = 128)."""
    from tjev_amd.serve import gdn_prefill

    (qkv, a, b, a_log, dt_bias, w, seg), _ = case_inputs(2, 456, 2, 4, 128, dtype=torch.bfloat16, style="baseline",
                                                         segments="one")
    kw = dict(key_heads=2, key_dim=128, value_heads=4, value_dim=128, chunk=128, precision="high")
    x = [t.cuda() for t in (qkv, a, b, a_log, dt_bias, w, seg)]
    out, state, hist = gdn_prefill(*x, **kw)
    t1 = 256
    o1, s1, h1 = gdn_prefill(x[0][:, :t1], x[1][:, :t1], x[2][:, :t1], *x[3:6], x[6][:, :t1], **kw)
    o2, s2, h2 = gdn_prefill(x[0][:, t1:], x[1][:, t1:], x[2][:, t1:], *x[3:6], x[6][:, t1:], initial_state=s1,
                             initial_conv=h1, **kw)
    torch.cuda.synchronize()
    pieces = torch.cat([o1, o2], 1).float()
    rms = float(out.float().pow(2).mean().sqrt())
    err = float((pieces - out.float()).abs().max()) / rms
    print(f"prefill in pieces: out max|diff|/rms {err:.2e}, state {rel(s2.cpu(), state.cpu()):.1e}")
    # the same chunks and states; only the state carried through the final-state kernel is
    # rounded apart from the scan's (fp32), then the outputs' bf16 rounding
    assert err <= 1e-2
    assert rel(s2.cpu(), state.cpu()) <= 1e-5
    assert torch.equal(h2, hist)
