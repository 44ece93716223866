"""GPU parity of the serving path (tjev_amd/serve.py) against the oracle: the prefill's final
state and conv history, the decode step, and the two chained, which must continue exactly the
megakernel's own output (test_gated_delta_rule.py:61-73's continuation, on the megakernel's
inputs).

- final state vs the oracle's token recurrence run to the last token (segment resets, T not a
  multiple of the chunk, a padding tail), fp32: max relative error 1e-5;
- conv history: the raw rows T-K+1 .. T-1, zero outside the last token's segment, bit exact;
- decode step vs the oracle's ``decode_step`` (fp32 1e-5; bf16 activations: within one bf16
  rounding of the output's scale);
- prefill of T tokens then three decode steps vs the megakernel over T+3 tokens at those
  positions (fp32 1e-5; bf16 high: the bf16 bar, max abs error <= 2e-2 RMS).
"""

from __future__ import annotations

import pytest
import torch

from gdn_cases import rel

pytestmark = pytest.mark.gpu

SHAPE = dict(key_heads=2, key_dim=64, value_heads=4, value_dim=64)


def _inputs(batch, length, dtype, seed, segments="one", cuts=None, trailing_pad=0):
    from tjev_amd.testing import gdn_inputs

    return list(gdn_inputs(batch=batch, length=length, key_heads=2, value_heads=4, dim=64, dtype=dtype, seed=seed,
                           segments=segments, cuts=cuts, trailing_pad=trailing_pad))


def _oracle_final(inputs):
    from oracle.gdn_oracle import core_inputs, recurrent_gated_delta_rule

    f64 = [x.double() if x.is_floating_point() else x for x in inputs]
    q, k, v, g, beta, seg = core_inputs(*f64, dtype=torch.float64, **SHAPE)
    return recurrent_gated_delta_rule(q, k, v, g, beta, seg)[1]


@pytest.mark.parametrize("length,cuts,pad", [(200, [70, 150], 0), (256, [100], 0), (190, [60], 6)])
def test_prefill_final_state_and_history(length, cuts, pad):
    from tjev_amd.serve import gdn_prefill

    inputs = _inputs(2, length, torch.float32, 7, segments="cuts", cuts=cuts, trailing_pad=pad)
    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda() for x in inputs)
    out, state, hist = gdn_prefill(qkv, a, b, a_log, dt_bias, w, seg, chunk=64, precision="highest", **SHAPE)
    torch.cuda.synchronize()
    want = _oracle_final(inputs)
    err = rel(state.double().cpu(), want)
    print(f"T={length} cuts={cuts} pad={pad}: final state rel {err:.2e}", flush=True)
    assert err <= 1e-5
    k1 = w.shape[0] - 1
    s = inputs[6]
    for r in range(2):
        for i in range(k1):
            t = length - k1 + i
            keep = t >= 0 and int(s[r, t]) == int(s[r, -1])
            expect = inputs[0][r, t] if keep else torch.zeros_like(inputs[0][r, 0])
            assert torch.equal(hist[r, i].cpu(), expect), (r, i)


@pytest.mark.parametrize("dim,taps", [(64, 4), (128, 4), (128, 2), (16, 5)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_step_matches_oracle(dtype, dim, taps):
    """One decode step against the oracle's, at head dims of 1 to 4 state tiles and conv
    kernels of 2 to 5 taps (histories of 1 to 4 rows)."""
    from oracle.gdn_oracle import decode_step
    from tjev_amd.serve import gdn_decode_step
    from tjev_amd.testing import gdn_inputs

    shape = dict(key_heads=2, key_dim=dim, value_heads=4, value_dim=dim)
    gen = torch.Generator().manual_seed(3)
    t = 5
    qkv, a, b, a_log, dt_bias, w, _ = gdn_inputs(batch=3, length=t + 1, key_heads=2, value_heads=4, dim=dim,
                                                 dtype=dtype, seed=9, taps=taps)
    hist = qkv[:, t - (taps - 1):t]
    state = torch.randn((3, 4, dim, dim), generator=gen) * 0.1
    out, hist2, state2 = gdn_decode_step(qkv[:, t].cuda(), a[:, t].cuda(), b[:, t].cuda(), a_log.cuda(),
                                         dt_bias.cuda(), w.cuda(), hist.cuda(), state.cuda(), **shape)
    torch.cuda.synchronize()
    f = lambda x: x.double()  # noqa: E731
    want_out, want_hist, want_state = decode_step(f(qkv[:, t]), f(a[:, t]), f(b[:, t]), f(a_log), f(dt_bias), f(w),
                                                  f(hist), state.double(), dtype=torch.float64, **shape)
    assert torch.equal(hist2.cpu(), torch.cat([hist[:, 1:], qkv[:, t:t + 1]], 1))
    e_out, e_state = rel(out.double().cpu(), want_out), rel(state2.double().cpu(), want_state)
    print(f"{dtype} D={dim} taps={taps}: decode out rel {e_out:.2e}, state rel {e_state:.2e}", flush=True)
    if dtype == torch.float32:
        assert e_out <= 1e-5 and e_state <= 1e-5
    else:  # bf16 activations: the output's own rounding (2^-8 relative) dominates
        assert e_out <= 1e-2 and e_state <= 1e-3


@pytest.mark.parametrize("dtype,precision", [(torch.float32, "highest"), (torch.bfloat16, "high")])
def test_prefill_then_decode_continues_the_megakernel(dtype, precision):
    from tjev_amd import gdn_megakernel
    from tjev_amd.serve import gdn_decode_step, gdn_prefill

    length, extra = 250, 3
    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda() for x in _inputs(2, length + extra, dtype, 11))
    full = gdn_megakernel(qkv, a, b, a_log, dt_bias, w, seg, chunk=64, precision=precision, **SHAPE)
    _, state, hist = gdn_prefill(qkv[:, :length], a[:, :length], b[:, :length], a_log, dt_bias, w, seg[:, :length],
                                 chunk=64, precision=precision, **SHAPE)
    outs = []
    for t in range(length, length + extra):
        o, hist, state = gdn_decode_step(qkv[:, t], a[:, t], b[:, t], a_log, dt_bias, w, hist, state, **SHAPE)
        outs.append(o)
    torch.cuda.synchronize()
    got = torch.stack(outs, 1).double().cpu()
    want = full[:, length:].double().cpu()
    if dtype == torch.float32:
        assert rel(got, want) <= 1e-5, rel(got, want)
    else:
        rms = float(want.pow(2).mean().sqrt())
        err = float((got - want).abs().max()) / rms
        print(f"bf16 prefill+decode vs megakernel: max abs err / RMS {err:.2e}", flush=True)
        assert err <= 2e-2
