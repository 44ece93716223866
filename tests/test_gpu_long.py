"""The reference's long-sequence tests (tests/kernels/test_gdn_long.py), on the GPU: the GDN core
at the long buckets' lengths (T = 8192, 16384) with ~T/1024 + 3 packed segments whose
boundaries fall inside chunks, at tiny heads (4 key / 8 value heads of 32) and the gates at the
trained 0.8B's spread (per-head A_log and dt_bias from its layers' minimum to maximum: decays
from ~-5 to ~-1e-5 per token, memories of ~10^5 tokens). The kernels run ``high`` (bf16x3),
as on the reference's TPU, where its CPU run emulates it.

- Every output and input gradient against the fp32 oracle on the same projection values, fp32
  and bf16 projections, within the reference's relative-L2 tolerances: the megakernel (chunk
  128, blocked inverse: the reference campaign's mega2) and the path it replaces (the glue
  around the v2 operator, chunk 64).
- The gate gradients' error against the fp64 oracle grows from T = 1024 to 16384 at most 4x as
  fast as the fp32 oracle's own (the sums over T of d A_log and d dt_bias accumulate fp32
  rounding in both), and their cosine stays >= 0.9999.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import case_inputs, cosine, hip_outputs, oracle_outputs, rel, rel_l2

pytestmark = pytest.mark.gpu

HK, H, D = 4, 8, 32
# test_gdn_long.py:32-35: per value head, the trained Qwen3.5-0.8B's A_log / dt_bias spread
A_LOG = (-6.5, -4.0, -2.2, -1.3, -1.3, -0.5, 0.3, 2.3)
DT_BIAS = (-13.0, -8.0, -5.2, -1.7, 0.0, 1.9, -3.0, -10.0)
CHUNKS = {"mega2": 128, "v2": 64}
# test_gdn_long.py:179-187: relative L2 against the fp32 reference at precision high
TOL = {
    "float32": {"out": 5e-5, "qkv": 5e-5, "a": 1.5e-4, "b": 5e-5, "A_log": 2e-3, "dt_bias": 2e-3, "w": 5e-5},
    "bfloat16": dict.fromkeys(("out", "qkv", "a", "b", "A_log", "dt_bias", "w"), 2e-2),
}
SHAPE = dict(key_heads=HK, key_dim=D, value_heads=H, value_dim=D)


def long_inputs(length: int, seed: int = 0):
    """test_gdn_long.long_inputs: ~length/1024 + 3 cuts at random offsets, 5 trailing padding
    tokens, the gates above."""
    rng = np.random.default_rng(seed + length)
    cuts = sorted(rng.choice(np.arange(1, length - 8), length // 1024 + 3, replace=False).tolist())
    (qkv, a, b, _, _, w, seg), cot = case_inputs(1, length, HK, H, D, seed=seed, cuts=cuts)
    return (qkv, a, b, torch.tensor(A_LOG), torch.tensor(DT_BIAS), w, seg), cot


def _path_outputs(path, xs, cot):
    if path == "mega2":
        return hip_outputs(xs, cot, chunk=CHUNKS[path], precision="high", inverse="blocked", **SHAPE)
    from test_gpu_model_heads import _v2_path_outputs

    return _v2_path_outputs(xs, cot, hk=HK, h=H, d=D, conv=True, chunk=CHUNKS[path])


def _report(got, want):
    return {k: {"max": rel(got[k], want[k]), "l2": rel_l2(got[k], want[k]), "cos": cosine(got[k], want[k]),
                "finite": bool(torch.isfinite(got[k]).all())} for k in got}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["float32", "bfloat16"])
@pytest.mark.parametrize("path", ["mega2", "v2"])
@pytest.mark.parametrize("length", [8192, 16384])
def test_long_high_matches_fp32_reference(length, path, dtype):
    (qkv, a, b, a_log, dt_bias, w, seg), cot = long_inputs(length)
    xs = (qkv.to(dtype), a.to(dtype), b.to(dtype), a_log, dt_bias, w, seg)
    xs_ref = tuple(x.float() if i < 3 else x for i, x in enumerate(xs))
    print(f"T={length} {path} {dtype} high", flush=True)
    want = oracle_outputs(xs_ref, cot, **SHAPE)
    errors = _report(_path_outputs(path, xs, cot), want)
    print("  rel-L2 / cos:", {k: f"{e['l2']:.1e} {e['cos']:.6f}" for k, e in errors.items()}, flush=True)
    assert all(e["finite"] for e in errors.values())
    tol = TOL["float32" if dtype == torch.float32 else "bfloat16"]
    bad = {k: e["l2"] for k, e in errors.items() if e["l2"] > tol[k]}
    assert not bad, errors


@pytest.mark.parametrize("path", ["mega2", "v2"])
def test_long_gate_gradients_do_not_degrade_with_length(path):
    rows = {}
    for length in (1024, 16384):
        xs, cot = long_inputs(length)
        truth = oracle_outputs(xs, cot, dtype=torch.float64, **SHAPE)
        ref = _report(oracle_outputs(xs, cot, **SHAPE), truth)
        got = _report(_path_outputs(path, xs, cot), truth)
        rows[length] = (got, ref)
        print(f"T={length} {path}: gate gradients vs fp64 (got / fp32 oracle) rel-L2",
              {k: f"{got[k]['l2']:.1e} / {ref[k]['l2']:.1e}" for k in ("a", "A_log", "dt_bias")}, flush=True)
    (short, short_ref), (long, long_ref) = rows[1024], rows[16384]
    for name in ("a", "A_log", "dt_bias"):
        assert long[name]["cos"] > 0.9999, (name, long[name])
        growth = long[name]["l2"] / max(short[name]["l2"], 1e-12)
        ref_growth = long_ref[name]["l2"] / max(short_ref[name]["l2"], 1e-12)
        assert growth < 4 * max(ref_growth, 1.0), (name, growth, ref_growth)
