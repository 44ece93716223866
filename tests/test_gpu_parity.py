"""The HIP megakernel against the CPU oracle on the same seeded inputs (GPU).

Mirrors tests/kernels/test_gdn_mega.py:94-122 (shapes, chunks, segment cuts at chunk offsets
0..3 and C-1, trailing padding, GQA, head grouping, blocked inverse, mega1 and mega2): the
output and the gradient of every input (qkv, a, b, A_log, dt_bias, the conv weight) under a
fixed random cotangent, at the reference's fp32 tolerance for precision "highest".
"""

import pytest
import torch

from gdn_cases import NAMES, case_inputs, cosine, hip_outputs, oracle_outputs, rel, rel_l2

pytestmark = pytest.mark.gpu

# test_gdn_mega.py:89-91: per-token terms at the fp32 level; A_log, dt_bias and the conv
# weight are sums over every token.
TOL = {"out": 1e-5, "qkv": 1e-5, "a": 1e-5, "b": 1e-5, "A_log": 5e-5, "dt_bias": 5e-5, "w": 1e-5}

CASES = [
    # (B, T, Hk, H), chunk, cuts, options -- test_gdn_mega.py:96-111
    ((1, 120, 2, 4), 16, [16, 33, 50, 67, 95], {}),
    ((1, 120, 2, 2), 16, [16, 33, 50, 67, 95], {}),
    ((1, 1100, 2, 4), 64, [510, 513, 1024, 1027], {}),
    ((1, 150, 2, 4), 32, [31, 64, 65, 98], {}),  # one doubling level (the level-16 product cleared at the end)
    ((2, 200, 2, 4), 64, None, {"inverse": "blocked"}),
    ((1, 256, 2, 4), 128, None, {"inverse": "blocked"}),
    ((1, 200, 4, 8), 64, None, {"heads_per_step": 4}),
    ((1, 256, 16, 32), 128, [100, 177], {"heads_per_step": 16, "inverse": "blocked"}),
    ((1, 256, 16, 32), 128, [100, 177], {"heads_per_step": 32, "inverse": "blocked"}),  # one head group
    ((1, 256, 8, 16), 128, [100, 177], {"heads_per_step": 16, "inverse": "blocked"}),
]


def _label(case):
    (b, t, hk, h), c, cuts, kw = case
    return f"B{b}T{t}Hk{hk}H{h}C{c}" + ("".join(f"-{k}={v}" for k, v in kw.items()))


@pytest.mark.parametrize("conv", [True, False], ids=["mega2", "mega1"])
@pytest.mark.parametrize("case", CASES, ids=[_label(c) for c in CASES])
def test_hip_matches_oracle_fp32(case, conv):
    (batch, length, hk, h), chunk, cuts, kw = case
    d = 16
    inputs, cot = case_inputs(batch, length, hk, h, d, cuts=cuts)
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=conv)
    print(f"case {_label(case)} conv={conv}", flush=True)
    got = hip_outputs(inputs, cot, chunk=chunk, precision="highest", **kw, **shape)
    want = oracle_outputs(inputs, cot, **shape)
    errors = {k: rel(got[k], want[k]) for k in got}
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


@pytest.mark.parametrize("taps", [1, 2, 5])
def test_hip_conv_widths_fp32(taps):
    """Conv kernels of 1, 2 and 5 taps (the model's is 4): the halo and look-ahead rows are sized
    to taps - 1, with segment cuts right after a chunk start and before a chunk end."""
    d, hk, h = 16, 2, 4
    inputs, cot = case_inputs(1, 150, hk, h, d, cuts=[31, 64, 65, 98], taps=taps)
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    print(f"taps {taps}", flush=True)
    got = hip_outputs(inputs, cot, chunk=32, precision="highest", **shape)
    want = oracle_outputs(inputs, cot, **shape)
    errors = {k: rel(got[k], want[k]) for k in got}
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


# every (chunk, head dim) pair with kernels beyond the d = 16 cases above: chunks below the head
# dim (16 and 32 at 128), chunk 128 over head dim 64, and the small pairs
SHAPE_GRID = [(16, 32), (32, 32), (64, 32), (16, 64), (32, 64), (128, 64), (16, 128), (32, 128), (64, 128)]


@pytest.mark.parametrize("chunk,d", SHAPE_GRID, ids=[f"C{c}D{d}" for c, d in SHAPE_GRID])
def test_hip_shape_grid_fp32(chunk, d):
    """The chunk and head-dim pairs the reference accepts (pallas_tpu_mega.py:597-615: any
    power-of-two chunk; Dk = Dv here), each against the oracle at the fp32 bar, with segment
    cuts inside the first chunks and a ragged tail."""
    hk, h = 2, 4
    length = 3 * chunk + 5
    inputs, cot = case_inputs(1, length, hk, h, d, cuts=[chunk - 1, chunk + 2, 2 * chunk + 1])
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    print(f"shape grid chunk={chunk} d={d}", flush=True)
    got = hip_outputs(inputs, cot, chunk=chunk, precision="highest", **shape)
    want = oracle_outputs(inputs, cot, **shape)
    errors = {k: rel(got[k], want[k]) for k in got}
    print({k: f"{v:.1e}" for k, v in errors.items()})
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


@pytest.mark.parametrize("chunk,d", [(256, 16), (512, 64)], ids=["C256D16", "C512D64"])
def test_hip_chunks_above_128_fp32(chunk, d):
    """Chunks above 128 (the reference accepts any power of two) run the chunk-128 kernels: the
    chunked form is exact for any chunk, so the result is the oracle's at the fp32 bar."""
    hk, h = 2, 4
    inputs, cot = case_inputs(1, 700, hk, h, d, cuts=[127, 300, 513])
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    print(f"chunk {chunk} d={d}", flush=True)
    got = hip_outputs(inputs, cot, chunk=chunk, precision="highest", **shape)
    want = oracle_outputs(inputs, cot, **shape)
    errors = {k: rel(got[k], want[k]) for k in got}
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


@pytest.mark.parametrize("d,chunk,taps", [(16, 32, 4), (16, 128, 4), (64, 64, 4), (16, 32, 5)])
def test_hip_frozen_conv_weight_fp32(d, chunk, taps):
    """The conv weight not differentiated (pallas_tpu_mega.py:548-571 emits no dz then), as in
    the benchmark's step: the backward's own conv path without the d(conv w) partials (with
    the 3-row halo of the model's conv of 4 taps, and the 4-row one of 5 taps)."""
    hk, h = 2, 4
    inputs, cot = case_inputs(1, 300, hk, h, d, cuts=[chunk - 1, chunk + 1, 2 * chunk + 2], taps=taps)
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    print(f"frozen conv d={d} chunk={chunk} taps={taps}", flush=True)
    got = hip_outputs(inputs, cot, chunk=chunk, precision="highest", want_w=False, **shape)
    want = oracle_outputs(inputs, cot, **shape)
    assert "w" not in got
    errors = {k: rel(got[k], want[k]) for k in got}
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


def test_hip_tiny_config_fp32():
    """The tiny benchmark config (B=1, T=512, Hk=H=4, D=64, chunk 64, fp32 "highest", one segment).
    Output and every gradient: max relative error <= 1e-5 against the fp32 reference path, and
    <= 5e-5 on the sums over every token (A_log, dt_bias: test_gdn_mega.py:89-91); gradient
    cosine >= 0.999999. The sums are also held to the fp32 reference path's own error against
    the fp64 truth: the kernels form dg without the terms that cancel in the reference's
    reverse cumsum of d gamma, whose fp32 noise the sums amplify (3.1e-5 on d A_log in the fp32
    path at this config)."""
    from tjev_amd.testing import cotangent, gdn_inputs

    inputs = gdn_inputs(batch=1, length=512, key_heads=4, value_heads=4, dim=64)
    cot = cotangent(1, 512, 4, 64)
    shape = dict(key_heads=4, key_dim=64, value_heads=4, value_dim=64)
    got = hip_outputs(inputs, cot, chunk=64, precision="highest", **shape)
    ref32 = oracle_outputs(inputs, cot, **shape)
    truth = oracle_outputs(inputs, cot, dtype=torch.float64, **shape)
    report = {k: (rel(got[k], ref32[k]), rel(got[k], truth[k]), rel(ref32[k], truth[k]), cosine(got[k], ref32[k]))
              for k in got}
    print("tiny fp32 (vs fp32 ref / vs fp64 / fp32 ref vs fp64 / cos):",
          {k: "/".join(f"{x:.1e}" for x in v[:3]) + f"/{v[3]:.8f}" for k, v in report.items()})
    for name, (r32, r64, own, c) in report.items():
        assert r32 <= TOL[name], (name, report)
        if name in ("A_log", "dt_bias"):
            assert r64 <= own, (name, report)
        if name != "out":
            assert c >= 0.999999, (name, report)


def test_hip_reference_high_case():
    """The reference's precision="high" case ((2, 200, 2, 4), chunk 64, test_gdn_mega.py:111).
    On its CPU run the reference's dots are fp32 whatever the precision (test_gdn_long.py's
    emulated_high: "CPU dots are fp32 whatever the precision"), so that case checks fp32
    arithmetic at the fp32 tolerance: here at "highest" against TOL. Its bf16x3 arithmetic
    ("high" here, as on the TPU) is held to the reference's emulated-bf16x3 bar
    (test_gdn_long.py:183-187, relative L2)."""
    inputs, cot = case_inputs(2, 200, 2, 4, 16)
    shape = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16)
    want = oracle_outputs(inputs, cot, **shape)
    got = hip_outputs(inputs, cot, chunk=64, precision="highest", **shape)
    errors = {k: rel(got[k], want[k]) for k in got}
    high = hip_outputs(inputs, cot, chunk=64, precision="high", **shape)
    l2 = {k: rel_l2(high[k], want[k]) for k in high}
    print("reference high case: highest max-rel", {k: f"{v:.1e}" for k, v in errors.items()},
          "high rel-L2", {k: f"{v:.1e}" for k, v in l2.items()})
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)
    for name, err in l2.items():
        assert err < HIGH_TOL[name], (name, l2)


HIGH_TOL = {"out": 5e-5, "qkv": 5e-5, "a": 1.5e-4, "b": 5e-5, "A_log": 2e-3, "dt_bias": 2e-3, "w": 5e-5}


@pytest.mark.parametrize("precision", ["high", "mixed", "bf16"])
def test_hip_precision_modes(precision):
    """bf16x3 ("high"): relative L2 within the reference's long-T fp32-input tolerances
    (test_gdn_long.py:183-187). "mixed" (one bf16 pass on the state path) and one-pass "bf16":
    bf16-level errors on the output and the per-token gradients; the gate-parameter sums
    d A_log / d dt_bias are only loosely bounded, as in the reference, whose one-pass bf16
    gate gradients are 10-30% off (docs/training.md:276) -- the reason "high" is production."""
    inputs, cot = case_inputs(2, 256, 2, 4, 16)
    shape = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16)
    got = hip_outputs(inputs, cot, chunk=64, precision=precision, **shape)
    want = oracle_outputs(inputs, cot, **shape)
    l2 = {k: rel_l2(got[k], want[k]) for k in got}
    cos = {k: cosine(got[k], want[k]) for k in got}
    print(precision, {k: f"{l2[k]:.1e}/{cos[k]:.6f}" for k in got})
    per_token = ("out", "qkv", "b", "w")
    if precision == "high":
        for k in got:
            assert l2[k] < HIGH_TOL[k], (k, l2)
    elif precision == "mixed":
        assert all(l2[k] < 2e-3 for k in per_token), l2
        assert l2["a"] < 1e-2 and all(cos[k] > 0.999 for k in got), (l2, cos)
    else:
        assert all(l2[k] < 1e-2 for k in per_token), l2
        assert l2["a"] < 1e-1 and cos["a"] > 0.995, (l2, cos)


def _bf16_bar(got, want):
    """The bf16 parity bar. Output: the max abs error beyond the bf16 rounding of the output
    itself, relative to the output RMS, <= 2e-2 (the rounding floor alone reaches 5e-2 when
    max|o|/RMS ~ 27, as at these shapes), and relative L2 <= 2e-2 (test_gdn_long.py:186);
    gradients: cosine >= 0.9999."""
    o = want["out"]
    rms = float(o.pow(2).mean().sqrt())
    err = float((got["out"] - o).abs().max()) / rms
    floor = float((o.to(torch.bfloat16).double() - o).abs().max()) / rms
    cos = {k: cosine(got[k], want[k]) for k in got if k != "out"}
    return err, floor, rel_l2(got["out"], o), cos


@pytest.mark.parametrize("hk,h", [(16, 16), (16, 32)], ids=["0.8B-heads", "9B-heads"])
def test_hip_bf16_model_heads(hk, h):
    """The 0.8B / 9B head shapes (Dk = Dv = 128, chunk 128, bf16 activations, precision high) at
    T = 1024 with packed segments and padding, against the fp32 oracle on the same values."""
    inputs, cot = case_inputs(1, 1024, hk, h, 128, cuts=[64, 129, 510, 513, 1000], dtype=torch.bfloat16,
                              style="baseline")
    shape = dict(key_heads=hk, key_dim=128, value_heads=h, value_dim=128)
    got = hip_outputs(inputs, cot, chunk=128, precision="high", **shape)
    want = oracle_outputs(inputs, cot, **shape)
    err, floor, l2, cos = _bf16_bar(got, want)
    print(f"bf16 {hk}/{h}: out maxabs/rms {err:.2e} (bf16 floor {floor:.2e}) rel-l2 {l2:.2e}",
          {k: f"{c:.7f}" for k, c in cos.items()})
    assert err - floor <= 2e-2 and l2 <= 2e-2
    for k, c in cos.items():
        assert c >= 0.9999, (k, cos)


@pytest.mark.parametrize("length", [1, 5, 63, 65])
def test_hip_rows_shorter_than_a_chunk_fp32(length):
    """Rows shorter than one chunk (and one token past it): the padded tail of the only chunk
    reads and writes nothing, at the fp32 bar against the fp64 oracle (the fp32 oracle is itself
    4.5e-5 from fp64 on d A_log at T = 65)."""
    d, hk, h = 16, 2, 4
    inputs, cot = case_inputs(2, length, hk, h, d, trailing_pad=0, segments="one")
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    print(f"short row T={length}", flush=True)
    got = hip_outputs(inputs, cot, chunk=64, precision="highest", **shape)
    want = oracle_outputs(inputs, cot, dtype=torch.float64, **shape)
    assert all(bool(torch.isfinite(v).all()) for v in got.values())
    for name in got:
        if not bool(want[name].any()):  # one token: no decay reaches anything, d a = 0 exactly
            assert not bool(got[name].any()), name
        else:
            assert rel(got[name], want[name]) < TOL[name], (name, rel(got[name], want[name]))


def test_hip_all_padding_row_fp32():
    """A batch row that is padding throughout (segment ids all 0) beside a packed row: the padded
    row's output and every gradient of its inputs are exact zeros, and the other row's match the
    fp64 oracle at the fp32 bar."""
    d, hk, h = 16, 2, 4
    inputs, cot = case_inputs(2, 150, hk, h, d, cuts=[31, 64, 65, 98])
    qkv, a, b, a_log, dt_bias, w, seg = inputs
    seg = seg.clone()
    seg[0] = 0
    inputs = (qkv, a, b, a_log, dt_bias, w, seg)
    shape = dict(key_heads=hk, key_dim=d, value_heads=h, value_dim=d, conv=True)
    got = hip_outputs(inputs, cot, chunk=32, precision="highest", **shape)
    want = oracle_outputs(inputs, cot, dtype=torch.float64, **shape)
    for name in ("out", "qkv", "a", "b"):
        assert bool((got[name][0] == 0).all()), name
    errors = {k: rel(got[k], want[k]) for k in got}
    for name, err in errors.items():
        assert err < TOL[name], (name, errors)


@pytest.mark.parametrize("conv", [True, False], ids=["mega2", "mega1"])
def test_hip_packed_rows_equal_segments_alone(conv):
    """test_gdn_mega.py:135-147: a packed row (segments at [0, 16), [16, 33), [33, 71), [71, 96):
    boundaries at chunk offsets 0 and 1 and mid-chunk, chunk 16) computes what each segment
    computes alone (conv taps and the state never cross a boundary). Beyond the reference's
    forward check: under one cotangent the packed row's gradients of each segment's qkv, a and
    b equal those of the segment alone, and its A_log, dt_bias and conv-weight gradients the
    sums over the segments."""
    (qkv, a, b, a_log, dt_bias, w, _), cot = case_inputs(1, 96, 2, 4, 16, segments="one")
    cuts = [0, 16, 33, 71, 96]
    spans = list(zip(cuts[:-1], cuts[1:]))
    seg = torch.cat([torch.full((e - s,), i + 1, dtype=torch.int32) for i, (s, e) in enumerate(spans)])[None]
    kw = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16, chunk=16, precision="highest", conv=conv)
    packed = hip_outputs((qkv, a, b, a_log, dt_bias, w, seg), cot, **kw)
    sums = {k: torch.zeros_like(packed[k]) for k in ("A_log", "dt_bias", "w") if k in packed}
    for s, e in spans:
        alone = hip_outputs((qkv[:, s:e], a[:, s:e], b[:, s:e], a_log, dt_bias, w,
                             torch.ones((1, e - s), dtype=torch.int32)), cot[:, s:e], **kw)
        errs = {k: rel(packed[k][:, s:e], alone[k]) for k in ("out", "qkv", "a", "b")}
        print(f"span [{s}, {e}) conv={conv}:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
        assert all(v < 1e-5 for v in errs.values()), (s, e, errs)
        for k in sums:
            sums[k] += alone[k]
    for k, total in sums.items():
        assert rel(packed[k], total) < 1e-5, (k, rel(packed[k], total))
