"""Debug checks of the kernels (GPU), the counterparts of the reference's interpret-mode run with
uninitialised scratch read as NaN (tests/kernels/test_gdn_mega.py:161-178):

- poisoned buffers: with TJEV_GDN_POISON=1 every forward fills its workspace and residual buffer,
  and every backward its workspace, with NaN before its kernels run; outputs and gradients are
  then bit for bit those of an ordinary run (and finite), so no kernel reads memory that no
  kernel wrote -- over segment cuts at chunk offsets, padding, GQA, every residual policy, the
  conv weight's gradient, a continued sequence with its state gradients, the gated RMSNorm
  path and the v2 operator;
- poisoned LDS: the same cases through the LDS-poison debug library (libtjev_gdn_lds_poison.so,
  every kernel fills its LDS arrays with NaN bytes before its own code runs; both forms of the
  inverse), bit for bit the ordinary library's results: no kernel reads LDS it did not write;
- NaN inputs: a NaN in one value head's input returns normally (status 0) and stays where the
  recurrence carries it: the other row, the chunks before it and the other heads' outputs are
  finite.
"""

import os

import pytest
import torch

from gdn_cases import case_inputs, hip_outputs

pytestmark = pytest.mark.gpu


POISONS = ["buffers", "lds"]


def _both(fn, kind="buffers"):
    """fn() plainly and under a poison: "buffers" (TJEV_GDN_POISON=1: the workspace and residual
    buffers filled with NaN before the kernels run) or "lds" (the calls go through the LDS-poison
    debug library, whose kernels fill their LDS with NaN before their own code runs)."""
    from tjev_amd import _lib

    os.environ.pop("TJEV_GDN_POISON", None)
    plain = fn()
    if kind == "lds":
        with _lib.library(_lib.LDS_POISON_PATH) as lib:
            assert lib.tjev_gdn_lds_poison() == 1
            poisoned = fn()
        return plain, poisoned
    os.environ["TJEV_GDN_POISON"] = "1"
    try:
        poisoned = fn()
    finally:
        os.environ.pop("TJEV_GDN_POISON", None)
    return plain, poisoned


def _same(plain, poisoned, label):
    for k in plain:
        assert bool(torch.isfinite(poisoned[k]).all()), (label, k)
        assert torch.equal(plain[k], poisoned[k]), (label, k, float((plain[k] - poisoned[k]).abs().max()))


CASES = [
    # (B, T, Hk, H, D), chunk, cuts, dtype, precision, residuals
    ((1, 120, 2, 4, 16), 16, [16, 33, 50, 67, 95], torch.float32, "highest", "states"),
    ((2, 200, 2, 4, 16), 64, None, torch.float32, "high", "tinv"),
    ((1, 300, 2, 2, 64), 64, [63, 65, 130], torch.float32, "mixed", "all"),
    ((1, 400, 2, 4, 128), 128, [100, 177], torch.bfloat16, "high", "states"),
    ((1, 400, 2, 2, 128), 128, [127, 128, 255], torch.bfloat16, "high", "tinv"),  # q and v from the raw rows
]


@pytest.mark.parametrize("kind", POISONS)
@pytest.mark.parametrize("case", CASES, ids=[f"D{c[0][4]}-C{c[1]}-{c[4]}-{c[5]}" for c in CASES])
@pytest.mark.parametrize("conv", [True, False], ids=["mega2", "mega1"])
def test_poisoned_buffers_change_nothing(case, conv, kind):
    (b, t, hk, h, d), chunk, cuts, dtype, precision, residuals = case
    inputs, cot = case_inputs(b, t, hk, h, d, cuts=cuts, dtype=dtype, style="baseline" if d == 128 else "reference")
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=conv)
    print(f"poison {kind} {case} conv={conv}", flush=True)
    for inverse in ("doubling", "blocked") if kind == "lds" else ("doubling",):
        plain, poisoned = _both(lambda: hip_outputs(inputs, cot, chunk=chunk, precision=precision,
                                                    residuals=residuals, inverse=inverse, **shape), kind)
        _same(plain, poisoned, (case, inverse))


@pytest.mark.parametrize("kind", POISONS)
def test_poisoned_buffers_continued_sequence_and_v2(kind):
    """The _cont entry points (an initial state and conv history, the final state's gradient)
    and the v2 operator under the poison modes."""
    from tjev_amd import gdn_megakernel
    from tjev_amd.v2 import chunk_gated_delta_rule

    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(2, 128, 2, 4, 16)
    gen = torch.Generator().manual_seed(3)
    init = (0.3 * torch.randn((2, 4, 16, 16), generator=gen)).cuda()
    hist = torch.randn((2, 3, qkv.shape[-1]), generator=gen).cuda()
    d_final = torch.randn((2, 4, 16, 16), generator=gen).cuda()

    def mega():
        leaves = [x.cuda().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias, w, init, hist)]
        out, fin, cs = gdn_megakernel(*leaves[:6], seg.cuda(), key_heads=2, key_dim=16, value_heads=4, value_dim=16,
                                      chunk=16, precision="highest", initial_state=leaves[6], initial_conv=leaves[7],
                                      output_final_state=True)
        loss = (out * cot.cuda()).sum() + (fin * d_final).sum() + cs.sum()
        grads = torch.autograd.grad(loss, leaves)
        return {"out": out.detach(), "final": fin.detach(), "conv": cs.detach(),
                **{f"d{i}": g for i, g in enumerate(grads)}}

    _same(*_both(mega, kind), "megakernel continued")

    def v2():
        g = torch.Generator().manual_seed(4)
        q, k, v = (torch.randn((2, 128, 4, 16), generator=g).cuda().requires_grad_(True) for _ in range(3))
        gg = (-torch.rand((2, 128, 4), generator=g)).cuda().requires_grad_(True)
        be = torch.rand((2, 128, 4), generator=g).cuda().requires_grad_(True)
        s0 = init.clone().requires_grad_(True)
        out, fin = chunk_gated_delta_rule(q, k, v, gg, be, seg.cuda(), initial_state=s0, chunk=16)
        grads = torch.autograd.grad((out * cot.cuda()).sum() + (fin * d_final).sum(), [q, k, v, gg, be, s0])
        return {"out": out.detach(), "final": fin.detach(), **{f"d{i}": x for i, x in enumerate(grads)}}

    _same(*_both(v2, kind), "v2 with a state")


def test_nan_input_stays_where_the_recurrence_carries_it():
    from tjev_amd import gdn_megakernel

    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(2, 256, 2, 4, 16, segments="one")
    d, hk, h = 16, 2, 4
    qkv = qkv.clone()
    v0 = 2 * hk * d  # value channels start here; value head 1 at v0 + d
    qkv[0, 70, v0 + d: v0 + 2 * d] = float("nan")
    leaves = [x.cuda().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
    out = gdn_megakernel(*leaves, w.cuda(), seg.cuda(), key_heads=hk, key_dim=d, value_heads=h, value_dim=d, chunk=64,
                         precision="highest")
    grads = torch.autograd.grad((out * cot.cuda()).sum(), leaves)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isnan(out[0, 70:, 1]).any()                  # the head that read it, from its chunk on
    assert torch.isfinite(out[0, :64]).all()                  # the chunk before it
    assert torch.isfinite(out[1]).all()                       # the other row
    for hh in (0, 2, 3):
        assert torch.isfinite(out[0, :, hh]).all(), hh        # the other value heads
    for g in grads[:3]:
        assert torch.isfinite(g[1].cpu()).all()               # the other row's gradients


@pytest.mark.parametrize("kind", POISONS)
@pytest.mark.parametrize("weight_grad", [False, True], ids=["frozen-weight", "weight-grad"])
def test_poisoned_buffers_normed_path(weight_grad, kind):
    """The core with its gated RMSNorm (tjev_gdn_mega2_fwd_normed / _bwd_normed, the bench's and
    the block's path) under the poison mode: the backward's whole workspace is poisoned, the
    norm's d out and weight partials after the megakernel's part included."""
    from tjev_amd import gdn_megakernel_normed

    (qkv, a, b, a_log, dt_bias, w, seg), cot = case_inputs(1, 400, 2, 4, 128, cuts=[100, 177], dtype=torch.bfloat16,
                                                           style="baseline")
    gen = torch.Generator().manual_seed(6)
    z = torch.randn((1, 400, 4, 128), generator=gen).to(torch.bfloat16)
    nw = 1 + 0.1 * torch.randn(128, generator=gen)
    print(f"poison {kind} normed weight_grad={weight_grad}", flush=True)

    def run():
        leaves = [x.cuda().requires_grad_(x.is_floating_point()) for x in (qkv, a, b, a_log, dt_bias, z)]
        wt = nw.cuda().requires_grad_(weight_grad)
        y = gdn_megakernel_normed(*leaves[:5], w.cuda(), seg.cuda(), leaves[5], wt, key_heads=2, key_dim=128,
                                  value_heads=4, value_dim=128, chunk=128, precision="high")
        grads = torch.autograd.grad((y.float() * cot.cuda()).sum(), leaves + ([wt] if weight_grad else []))
        return {"y": y.detach(), **{f"d{i}": g for i, g in enumerate(grads)}}

    _same(*_both(run, kind), f"normed weight_grad={weight_grad}")
