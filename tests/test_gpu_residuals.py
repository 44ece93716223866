"""The residual contract on the GPU (the forward's gdn_tinv and gdn_states,
pallas_tpu_mega.py:444-449, 543-548): what the forward keeps changes no result beyond rounding.

- "tinv" and "states" give the same output and gradients bit for bit: the forward's T comes
  from the same code as the backward's rebuilt one, and v_new from it by the same code;
- "all" (v_new from the forward's scan) matches "states" to rounding;
- the kept T is each chunk's (I + L)^-1: the oracle's ``chunk_tinv`` on the same inputs.
"""

from __future__ import annotations

import math

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


def test_kept_tinv_is_the_chunk_inverse():
    from oracle.gdn_oracle import chunk_tinv, core_inputs
    from tjev_amd.gdn import GdnPlan

    inputs, _ = case_inputs(1, 200, 2, 4, 64, dtype=torch.float32, seed=4)
    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda().contiguous() for x in inputs)
    B, T, _ = qkv.shape
    C = 64
    plan = GdnPlan(batch=B, length=T, key_heads=2, key_dim=64, value_heads=4, value_dim=64, taps=w.shape[0],
                   chunk=C, io_dtype=torch.float32, gate_dtype=torch.float32, precision="highest", residuals="tinv")
    res = plan.residuals("cuda")
    out = torch.empty((B, T, 4, 64), device="cuda")
    plan.forward(qkv, a, b, a_log, dt_bias, w, seg, out, res, plan.workspace(False, "cuda"))
    torch.cuda.synchronize()
    n = math.ceil(T / C)
    start = (math.prod(plan.states_shape) + 63) // 64 * 64  # the states part, 256-byte aligned
    got = res[start:start + B * 4 * n * C * C].view(B, 4, n, C, C).double().cpu()
    _, k, _, g, beta, sg = core_inputs(*(x.double() if x.is_floating_point() else x for x in inputs),
                                       key_heads=2, key_dim=64, value_heads=4, value_dim=64, dtype=torch.float64)
    want = chunk_tinv(k, g, beta, sg, chunk=C)
    err = float((got - want).abs().max()) / float(want.abs().max())
    print(f"kept T vs oracle: max rel {err:.2e}", flush=True)
    assert err <= 1e-5
    assert torch.all(got.triu(1) == 0) and torch.all(got.diagonal(dim1=-2, dim2=-1) == 1)
