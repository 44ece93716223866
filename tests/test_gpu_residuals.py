"""The residual contract on the GPU (the forward's gdn_tinv and gdn_states,
pallas_tpu_mega.py:444-449, 543-548): what the forward keeps changes no result beyond rounding.

- "tinv" and "states" give the same output and gradients bit for bit: the forward's T comes
  from the same code as the backward's rebuilt one, and v_new from it by the same code;
- "all" (v_new from the forward's scan) matches "states" to rounding;
- the kept T is each chunk's (I + L)^-1: the oracle's ``chunk_tinv`` on the same inputs, under
  either form of the inverse; the pure doubling's diagonal blocks follow the oracle's doubling
  at the products' precision, the blocked form's are exact.
"""

from __future__ import annotations


import pytest
import torch

from gdn_cases import NAMES, case_inputs, cosine, hip_outputs, rel

pytestmark = pytest.mark.gpu

SHAPE = dict(key_heads=2, key_dim=64, value_heads=4, value_dim=64)


@pytest.mark.parametrize("precision,dtype", [("high", torch.bfloat16), ("highest", torch.float32)])
def test_residual_policies_agree(precision, dtype):
    inputs, cot = case_inputs(2, 300, 2, 4, 64, dtype=dtype, seed=3)
    runs = {mode: hip_outputs(inputs, cot, chunk=64, precision=precision, residuals=mode, **SHAPE)
            for mode in ("states", "tinv", "all")}
    print(f"{precision}: all vs states", {k: f"{rel(runs['all'][k], runs['states'][k]):.1e}" for k in runs["all"]},
          flush=True)
    for k in runs["states"]:
        assert torch.equal(runs["tinv"][k], runs["states"][k]), k
    assert torch.equal(runs["all"]["out"], runs["states"]["out"])
    for k in NAMES:
        if k in runs["all"]:
            assert cosine(runs["all"][k], runs["states"][k]) >= 0.999999, k
            if dtype == torch.float32 and k not in ("A_log", "dt_bias"):
                assert rel(runs["all"][k], runs["states"][k]) <= 1e-5, k


def _kept_tinv(inputs, C, precision, inverse):
    """The forward's kept T [B, H, N, C, C] (residuals "tinv") at the SHAPE heads, as stored."""
    from tjev_amd.gdn import GdnPlan

    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda().contiguous() for x in inputs)
    B, T, _ = qkv.shape
    plan = GdnPlan(batch=B, length=T, key_heads=2, key_dim=64, value_heads=4, value_dim=64, taps=w.shape[0],
                   chunk=C, io_dtype=torch.float32, gate_dtype=torch.float32, precision=precision,
                   inverse=inverse, residuals="tinv")
    res = plan.residuals("cuda")
    out = torch.empty((B, T, 4, 64), device="cuda")
    plan.forward(qkv, a, b, a_log, dt_bias, w, seg, out, res, plan.workspace(False, "cuda"))
    torch.cuda.synchronize()
    return plan.tinv_of(res).cpu()


def _chunk_lower(inputs, C):
    """L of every chunk [B, H, N, C, C] in fp64 from the oracle."""
    from oracle.gdn_oracle import _chunk_terms, core_inputs

    _, k, _, g, beta, sg = core_inputs(*(x.double() if x.is_floating_point() else x for x in inputs),
                                       key_heads=2, key_dim=64, value_heads=4, value_dim=64, dtype=torch.float64)
    z = torch.zeros_like(k)
    return k, g, beta, sg, _chunk_terms(z, k, z, g, beta, sg, None, C)["lower"]


@pytest.mark.parametrize("inverse", ["doubling", "blocked"])
def test_kept_tinv_is_the_chunk_inverse(inverse):
    from oracle.gdn_oracle import chunk_tinv

    inputs, _ = case_inputs(1, 200, 2, 4, 64, dtype=torch.float32, seed=4)
    C = 64
    got = _kept_tinv(inputs, C, "highest", inverse).double()
    k, g, beta, sg, _ = _chunk_lower(inputs, C)
    want = chunk_tinv(k, g, beta, sg, chunk=C)
    err = float((got - want).abs().max()) / float(want.abs().max())
    print(f"kept T ({inverse}) vs oracle: max rel {err:.2e}", flush=True)
    assert err <= 1e-5
    assert torch.all(got.triu(1) == 0) and torch.all(got.diagonal(dim1=-2, dim2=-1) == 1)


@pytest.mark.parametrize("C", [64, 128])
def test_doubling_inverse_runs_products_on_the_diagonal_blocks(C):
    """inverse="doubling" is the reference's pure doubling from T = I (pallas_tpu_v2.py:168-193
    with no diagonal blocks; xla.py:82-100). With one-pass bf16 products (precision "bf16", L
    itself then from bf16 k, T kept in bf16 as the reference's t_dtype) the 16 x 16 diagonal
    blocks of its T are the bf16 rounding of the oracle's doubling with bf16 operands on that L,
    and not of the exact inverse (the products' rounding moves many entries to another bf16
    value), where the blocked form's diagonal blocks (substitution in fp32) are the bf16 rounding
    of the exact inverse. Compared as the fraction of equal entries over the blocks' strictly
    lower entries that are not decayed away; only the diagonal blocks are compared with the
    emulation: above 16 the kernels associate each level's product as T_BR (L_LL T_TL), the
    reference as (T_BR L_LL) T_TL, another bf16 rounding."""
    from oracle.gdn_oracle import _chunk_terms, core_inputs, unit_lower_inverse

    inputs, _ = case_inputs(1, 2 * C, 2, 4, 64, dtype=torch.float32, seed=6)
    _, k, _, g, beta, sg = core_inputs(*(x.double() if x.is_floating_point() else x for x in inputs),
                                       key_heads=2, key_dim=64, value_heads=4, value_dim=64, dtype=torch.float64)
    z = torch.zeros_like(k)
    t = _chunk_terms(z, k, z, g, beta, sg, None, C)
    kb = t["k"].to(torch.bfloat16).double()
    lower = torch.tril(t["beta"][..., None] * (kb @ kb.transpose(-1, -2)) * t["decay"], -1)  # L from bf16 k
    exact = torch.linalg.inv(torch.eye(C, dtype=torch.float64) + lower)
    emulated = unit_lower_inverse(lower.float(), 0, bf16_operands=True)
    strict = torch.tril(torch.ones(16, 16, dtype=torch.bool), -1)

    def entries(x):  # the strictly lower entries of every 16 x 16 diagonal block
        return torch.cat([x[..., 16 * i:16 * i + 16, 16 * i:16 * i + 16][..., strict].reshape(-1)
                          for i in range(C // 16)])

    bf = lambda x: x.float().to(torch.bfloat16)  # noqa: E731
    want_exact, want_emu = bf(entries(exact)), bf(entries(emulated))
    live = entries(exact).abs() > 1e-6 * float(entries(exact).abs().max())
    dbl, blk = (entries(_kept_tinv(inputs, C, "bf16", inv)) for inv in ("doubling", "blocked"))
    assert dbl.dtype == torch.bfloat16 and blk.dtype == torch.bfloat16
    frac = lambda a, b: float((a == b)[live].double().mean())  # noqa: E731
    f_emu, f_dbl, f_blk = frac(dbl, want_emu), frac(dbl, want_exact), frac(blk, want_exact)
    print(f"C={C} diagonal blocks, equal entries: doubling vs bf16(bf16 doubling) {f_emu:.4f}, doubling vs "
          f"bf16(exact) {f_dbl:.4f}, blocked vs bf16(exact) {f_blk:.4f} ({int(live.sum())} entries)", flush=True)
    assert f_emu >= 0.99 and f_blk >= 0.99
    assert f_dbl <= 0.95


@pytest.mark.parametrize("precision", ["mixed", "bf16"])
@pytest.mark.parametrize("dim", [64, 128])
def test_states_are_bf16_when_the_state_products_are_one_pass(precision, dim):
    """Under "mixed" and "bf16" the kept states are bf16 (the reference's _state_dtypes,
    pallas_tpu_mega.py:425-426): each is the fp64 oracle's state at its chunk boundary to the
    mode's accuracy, and the state before the last chunk of a row is the bf16 rounding of the
    final state a run one chunk shorter returns. That final state is built from an fp32 copy of
    its last chunk's state (built from the bf16 residual instead, about half of its elements
    would round to another bf16 value). That holds bit for bit under "mixed", whose scan updates
    the state with bf16x3 products (k_final_state: fp32); under "bf16" the scan's one-pass
    update itself is that far from the final state's fp32 one (measured: 57% of the elements
    equal), so there the two only agree to the mode's accuracy. dim 128 runs the two-wave
    forward scan, dim 64 the generic one."""
    import ctypes

    from oracle.gdn_oracle import chunk_gated_delta_rule, core_inputs
    from tjev_amd.gdn import GdnPlan

    C, n, hk, h = dim, 4, 2, 4
    inputs, _ = case_inputs(1, n * C, hk, h, dim, dtype=torch.float32, seed=8, segments="one")

    def run(length):
        qkv, a, b, a_log, dt_bias, w, seg = (x.cuda().contiguous() for x in inputs)
        qkv, a, b, seg = (x[:, :length].contiguous() for x in (qkv, a, b, seg))  # the token-major inputs
        plan = GdnPlan(batch=1, length=length, key_heads=hk, key_dim=dim, value_heads=h, value_dim=dim,
                       taps=w.shape[0], chunk=C, io_dtype=torch.float32, gate_dtype=torch.float32,
                       precision=precision)
        res, ws = plan.residuals("cuda"), plan.workspace(False, "cuda")
        out = torch.empty((1, length, h, dim), device="cuda")
        final = torch.empty((1, h, dim, dim), device="cuda")
        conv = torch.empty((1, w.shape[0] - 1, qkv.shape[-1]), device="cuda")
        status = plan.lib.tjev_gdn_mega2_fwd_cont(
            ctypes.byref(plan.params), plan._stream(qkv.device), qkv.data_ptr(), a.data_ptr(), b.data_ptr(),
            a_log.data_ptr(), dt_bias.data_ptr(), w.data_ptr(), seg.data_ptr(), None, None, out.data_ptr(),
            res.data_ptr(), final.data_ptr(), conv.data_ptr(), ws.data_ptr(), ws.numel())
        assert status == 0
        torch.cuda.synchronize()
        states = plan.states_of(res)
        assert states.dtype == torch.bfloat16 and plan.states_bytes == states.numel() * 2
        return states.double().cpu(), final.cpu()

    states, _ = run(n * C)
    _, final_short = run((n - 1) * C)
    same = float((final_short.to(torch.bfloat16).double() == states[0, :, n - 1]).double().mean())
    q, k, v, g, beta, sg = core_inputs(*(x.double() if x.is_floating_point() else x for x in inputs), key_heads=hk,
                                       key_dim=dim, value_heads=h, value_dim=dim, dtype=torch.float64)
    errs = []
    for c in range(1, n):
        t = c * C
        _, want = chunk_gated_delta_rule(q[:, :t], k[:, :t], v[:, :t], g[:, :t], beta[:, :t], sg[:, :t], chunk=C)
        errs.append(float((states[0, :, c] - want[0]).norm() / want[0].norm()))
    print(f"{precision} D={dim}: states vs fp64 (relative L2 per chunk) {[f'{e:.1e}' for e in errs]}, "
          f"bf16(final state one chunk shorter) == last kept state for {same:.4f} of the elements", flush=True)
    assert torch.all(states[0, :, 0] == 0)
    assert max(errs) < 2e-2
    last = states[0, :, n - 1]
    assert float((final_short.double() - last).norm() / last.norm()) < 1e-2
    if precision == "mixed":  # measured 0.998
        assert same >= 0.99
