"""Pinning the CPU oracle (CPU only).

The reference ships no GDN golden arrays, so the oracle is pinned by what the mathematics and
the reference's own tests fix: the token recurrence (chunked == recurrent for any chunk, with
segments and states), packed rows == segments alone, state continuation, gradients, the
triangular inverse against a dense inverse, the l2norm known answer, the conv against a
textbook padded conv and torch's F.conv1d, HF transformers' independent GDN implementation
(transformers 5.15.0, single segment), and the known answers of heads_per_block. Each check
is chosen so that a plausible slip (a dropped reset, a wrong sign or index, a transposed
operand) fails it; the planted-mistake tests at the end show that they do.
"""

import itertools

import numpy as np
import pytest
import torch

import oracle.gdn_oracle as O

F64 = torch.float64


def _qkvgb(seed, batch=2, length=45, heads=3, dk=8, dv=6, dtype=F64):
    """tests/kernels/test_gated_delta_rule.py:18-25 (numpy streams)."""
    rng = np.random.default_rng(seed)
    t = lambda *s: torch.from_numpy(rng.standard_normal(s)).to(dtype)  # noqa: E731
    q = O.l2norm(t(batch, length, heads, dk)) * dk ** -0.5
    k = O.l2norm(t(batch, length, heads, dk))
    v = t(batch, length, heads, dv)
    g = -torch.nn.functional.softplus(t(batch, length, heads))
    beta = torch.sigmoid(t(batch, length, heads))
    return q, k, v, g, beta


def _segments(batch, length, seed):
    """test_gated_delta_rule.py:28-35: 4 random cuts per row."""
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(batch):
        cuts = np.sort(rng.choice(np.arange(1, length), size=4, replace=False))
        rows.append(np.searchsorted(cuts, np.arange(length), side="right") + 1)
    return torch.from_numpy(np.stack(rows)).to(torch.int64)


# ------------------------------------------------------------------ delta rule
@pytest.mark.parametrize("chunk", [4, 8, 16, 64])
def test_chunked_matches_recurrence(chunk):
    q, k, v, g, beta = _qkvgb(0)
    seg = _segments(2, 45, 0)
    ref, ref_state = O.recurrent_gated_delta_rule(q, k, v, g, beta, seg)
    out, state = O.chunk_gated_delta_rule(q, k, v, g, beta, seg, chunk=chunk)
    assert torch.allclose(out, ref, atol=1e-12, rtol=1e-10)
    assert torch.allclose(state, ref_state, atol=1e-12, rtol=1e-10)


def test_packed_segments_equal_runs_alone():
    """test_gated_delta_rule.py:47-58: each segment of a packed row alone."""
    q, k, v, g, beta = _qkvgb(1)
    seg = _segments(2, 45, 1)
    out, _ = O.chunk_gated_delta_rule(q, k, v, g, beta, seg, chunk=16)
    for b in range(2):
        for s in torch.unique(seg[b]):
            idx = torch.nonzero(seg[b] == s).ravel()
            alone, _ = O.recurrent_gated_delta_rule(*(x[b: b + 1, idx] for x in (q, k, v, g, beta)))
            assert torch.allclose(out[b, idx], alone[0], atol=1e-12)


def test_initial_state_continuation():
    """test_gated_delta_rule.py:61-73."""
    q, k, v, g, beta = _qkvgb(2, length=40)
    full, full_state = O.chunk_gated_delta_rule(q, k, v, g, beta, chunk=8)
    first, state = O.chunk_gated_delta_rule(*(x[:, :24] for x in (q, k, v, g, beta)), chunk=8)
    second, end = O.chunk_gated_delta_rule(*(x[:, 24:] for x in (q, k, v, g, beta)), initial_state=state,
                                           chunk=8)
    assert torch.allclose(torch.cat([first, second], 1), full, atol=1e-12)
    assert torch.allclose(end, full_state, atol=1e-12)
    step, _ = O.recurrent_gated_delta_rule(*(x[:, 24:25] for x in (q, k, v, g, beta)), initial_state=state)
    assert torch.allclose(step[:, 0], full[:, 24], atol=1e-12)


def test_gradients_chunked_match_recurrence():
    """test_gated_delta_rule.py:76-92, in float64."""
    xs = [x.requires_grad_(True) for x in _qkvgb(3, length=33)]
    seg = _segments(2, 33, 3)
    w = torch.from_numpy(np.random.default_rng(9).standard_normal((2, 33, 3, 6)))
    gc = torch.autograd.grad((O.chunk_gated_delta_rule(*xs, seg, chunk=8)[0] * w).sum(), xs)
    gr = torch.autograd.grad((O.recurrent_gated_delta_rule(*xs, seg)[0] * w).sum(), xs)
    for a, b in zip(gc, gr):
        assert torch.allclose(a, b, atol=1e-11, rtol=1e-9)


def test_hf_transformers_single_segment():
    """HF ``torch_chunk_gated_delta_rule`` / ``torch_recurrent_gated_delta_rule`` (the functions
    the reference's xla.py follows) on one segment, including their in-kernel l2norm and
    q scale: an implementation independent of this repository."""
    hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    rng = np.random.default_rng(4)
    B, T, H, D = 1, 100, 2, 16
    q, k, v = (torch.from_numpy(rng.standard_normal((B, T, H, D))) for _ in range(3))
    g = -torch.nn.functional.softplus(torch.from_numpy(rng.standard_normal((B, T, H))))
    beta = torch.sigmoid(torch.from_numpy(rng.standard_normal((B, T, H))))
    want_c, _ = hf.torch_chunk_gated_delta_rule(q, k, v, g, beta, chunk_size=32, use_qk_l2norm_in_kernel=True)
    want_r, _ = hf.torch_recurrent_gated_delta_rule(q, k, v, g, beta, None, False, use_qk_l2norm_in_kernel=True)
    qn, kn = O.l2norm(q) * D ** -0.5, O.l2norm(k)
    got, _ = O.chunk_gated_delta_rule(qn, kn, v, g, beta, chunk=32)
    # HF computes in float32 (its inputs are cast) and its l2norm has no zero-row guard (the
    # rows here are nonzero): agreement to fp32 rounding
    scale = float(got.abs().max())
    assert float((got - want_r.double()).abs().max()) < 2e-6 * scale
    assert float((got - want_c.double()).abs().max()) < 2e-6 * scale


# ------------------------------------------------------------------ inverse
@pytest.mark.parametrize("size", [16, 64, 128])
@pytest.mark.parametrize("block", [0, 16])
def test_inverse_matches_dense_inverse_correlated_keys(size, block):
    """test_pallas_tpu.py:194-207 / test_gated_delta_rule.py:137-147: correlated keys (L ~ beta
    on the whole strict lower triangle), doubling and blocked, against an fp64 dense inverse."""
    rng = np.random.default_rng(size)
    kk = torch.from_numpy(rng.standard_normal((3, size, 32))) + 2.0
    kk = kk / kk.norm(dim=-1, keepdim=True)
    lower = torch.tril(0.9 * kk @ kk.transpose(-1, -2), -1)
    exact = torch.linalg.inv(torch.eye(size, dtype=F64) + lower)
    got = O.unit_lower_inverse(lower, block)
    assert float((got - exact).abs().max()) < 1e-9 * float(exact.abs().max())


def test_inverse_bf16_operands_round_each_product():
    """The doubling with bf16 product operands (mode "bf16"): on a lower triangle whose every
    intermediate is a short dyadic (exact in bf16) it is the exact inverse; on correlated keys
    it leaves the fp32 doubling by about the bf16 rounding (2^-9 relative), not by 0 and not by
    more than a few times that."""
    size = 16
    lower = torch.zeros((size, size), dtype=torch.float32)
    for i in range(1, size):
        lower[i, i - 1] = 0.5  # T[i][j] = (-1/2)^(i-j): one significant bit each
    exact = torch.linalg.inv(torch.eye(size) + lower)
    assert torch.equal(O.unit_lower_inverse(lower, 0, bf16_operands=True), exact)
    rng = np.random.default_rng(5)
    kk = torch.from_numpy(rng.standard_normal((4, size, 32)).astype(np.float32)) + 2.0
    kk = kk / kk.norm(dim=-1, keepdim=True)
    lower = torch.tril(0.9 * kk @ kk.transpose(-1, -2), -1)
    plain = O.unit_lower_inverse(lower, 0)
    rounded = O.unit_lower_inverse(lower, 0, bf16_operands=True)
    err = float((rounded - plain).abs().max()) / float(plain.abs().max())
    assert 2.0 ** -12 < err < 2.0 ** -5, err
    blocked = O.unit_lower_inverse(lower, 16, bf16_operands=True)  # one block: substitution only
    assert float((blocked - plain).abs().max()) < 1e-5 * float(plain.abs().max())


# ------------------------------------------------------------------ l2norm, conv, norms
def test_l2norm_known_answer():
    """test_gated_delta_rule.py:172-183: a zero row maps to 0 with zero gradient; elsewhere the
    plain formula."""
    x = torch.tensor([[0.0, 0.0, 0.0, 0.0], [3.0, 0.0, 4.0, 0.0]], dtype=F64, requires_grad=True)
    cot = torch.tensor([[1.0, -2.0, 0.5, 3.0], [1.0, 2.0, -1.0, 0.5]], dtype=F64)
    out = O.l2norm(x)
    (grad,) = torch.autograd.grad((out * cot).sum(), x)
    assert torch.all(out[0] == 0) and torch.all(grad[0] == 0)
    row = torch.tensor([3.0, 0.0, 4.0, 0.0], dtype=F64, requires_grad=True)
    plain = row * torch.rsqrt((row * row).sum() + 1e-6)
    (pg,) = torch.autograd.grad((plain * cot[1]).sum(), row)
    assert torch.allclose(out[1], plain.detach(), rtol=1e-12)
    assert torch.allclose(grad[1], pg, rtol=1e-12)
    assert torch.allclose(out[1], torch.tensor([0.6, 0.0, 0.8, 0.0], dtype=F64), atol=1e-7)


def _conv_textbook(x, w, seg):
    """test_causal_conv1d.py:34-44: zero-padded causal conv with per-tap segment masks."""
    taps, length = w.shape[0], x.shape[1]
    xp = torch.nn.functional.pad(x, (0, 0, taps - 1, 0))
    sp = torch.nn.functional.pad(seg, (taps - 1, 0), value=-1)
    out = torch.zeros_like(x)
    for i in range(taps):
        keep = (sp[:, i: i + length] == seg)[..., None]
        out = out + torch.where(keep, xp[:, i: i + length], 0.0) * w[i]
    return out


def test_conv_matches_textbook_and_never_mixes_segments():
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((2, 30, 7)))
    w = torch.from_numpy(rng.standard_normal((4, 7)))
    seg = _segments(2, 30, 3)
    got = O.segmented_causal_conv1d(x, w, seg)
    assert torch.allclose(got, _conv_textbook(x, w, seg), atol=1e-12)
    for b in range(2):
        for s in torch.unique(seg[b]):
            idx = torch.nonzero(seg[b] == s).ravel()
            alone = O.segmented_causal_conv1d(x[b: b + 1, idx], w, torch.ones((1, len(idx)), dtype=torch.int64))
            assert torch.allclose(got[b, idx], alone[0], atol=1e-12)


def test_conv_single_segment_is_torch_conv1d():
    """HF's causal_conv1d_fn: F.conv1d with padding K-1, depthwise, weight [C, 1, K] (w[K-1]
    multiplies the current token)."""
    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((1, 25, 5)))
    w = torch.from_numpy(rng.standard_normal((4, 5)))
    want = torch.nn.functional.conv1d(x.transpose(1, 2), w.T[:, None, :], padding=3, groups=5)[..., :25]
    got = O.segmented_causal_conv1d(x, w, torch.ones((1, 25), dtype=torch.int64))
    assert torch.allclose(got, want.transpose(1, 2), atol=1e-12)


def test_gated_rmsnorm_matches_hf():
    hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((2, 7, 3, 16)).astype(np.float32)).to(torch.bfloat16)
    z = torch.from_numpy(rng.standard_normal((2, 7, 3, 16)).astype(np.float32)).to(torch.bfloat16)
    w = torch.from_numpy(rng.standard_normal(16).astype(np.float32))
    norm = hf.Qwen3_5RMSNormGated(16, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w)
        want = norm(x, z)
    got = O.gated_rmsnorm(x, z, w)
    assert got.dtype == torch.bfloat16
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_rmsnorm_backward_matches_hf(dtype):
    """The oracle's autograd through the norm (the cotangent of the bf16 rounding cast rounded
    to bf16, as JAX's convert_element_type transposes) equals HF's module autograd."""
    hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    rng = np.random.default_rng(6)
    shape = (2, 9, 3, 32)
    x0, z0, dy = (torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dtype) for _ in range(3))
    w0 = torch.from_numpy(1 + 0.1 * rng.standard_normal(32).astype(np.float32))
    norm = hf.Qwen3_5RMSNormGated(32, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w0)
    x, z = x0.clone().requires_grad_(True), z0.clone().requires_grad_(True)
    want = torch.autograd.grad((norm(x, z).float() * dy.float()).sum(), (x, z, norm.weight))
    x, z, w = x0.clone().requires_grad_(True), z0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    got = torch.autograd.grad((O.gated_rmsnorm(x, z, w).float() * dy.float()).sum(), (x, z, w))
    for g, h in zip(got, want):
        assert g.dtype == h.dtype
        scale = float(h.double().abs().max())
        # silu's autograd formula differs from F.silu's in the last bits: a bf16 ulp at most
        tol = 1e-6 if dtype == torch.float32 else 8e-3
        assert float((g.double() - h.double()).abs().max()) <= tol * scale


# ------------------------------------------------------------------ gates and the core's inputs
# (a, dt_bias, A_log, b) points: ordinary values, the end of the benchmark configs' A_log range (ln 16), large
# |a + dt_bias| where a naive log(1 + e^x) overflows or loses everything, and saturated b
GATE_POINTS = [(0.3, -0.5, 0.4, 0.1), (-2.0, 1.5, 2.772588722239781, -3.0), (25.0, 0.0, 0.0, 40.0),
               (-30.0, -5.0, 1.0, -40.0), (0.0, 0.0, -1.5, 0.0), (700.0, 10.0, 0.5, 5.0)]


def _gates_by_hand(a, dt_bias, a_log, b):
    """g = -e^{A_log} softplus(a + dt_bias), beta = 1 / (1 + e^{-b}) in Python's math, softplus
    as max(x, 0) + log1p(e^{-|x|}) (test_gdn_mega.py:52-53 with jax.nn.softplus)."""
    import math

    x = a + dt_bias
    softplus = max(x, 0.0) + math.log1p(math.exp(-abs(x)))
    beta = 1.0 / (1.0 + math.exp(-b)) if b >= 0 else math.exp(b) / (1.0 + math.exp(b))
    return -math.exp(a_log) * softplus, beta


def test_gates_closed_forms():
    """The oracle's gates at hand-picked points against the formulas evaluated in Python's math
    (pallas_tpu_mega.py:106-145; test_gdn_mega.py:52-53), both as ``gates`` and through
    ``core_inputs`` (per value head, zero qkv: the gates do not depend on it)."""
    a = torch.tensor([[[p[0] for p in GATE_POINTS]]], dtype=F64)
    dt = torch.tensor([p[1] for p in GATE_POINTS], dtype=F64)
    a_log = torch.tensor([p[2] for p in GATE_POINTS], dtype=F64)
    b = torch.tensor([[[p[3] for p in GATE_POINTS]]], dtype=F64)
    want = [_gates_by_hand(*p) for p in GATE_POINTS]
    g, beta = O.gates(a, b, a_log, dt)
    h = len(GATE_POINTS)
    _, _, _, g2, beta2, _ = O.core_inputs(torch.zeros((1, 1, 2 * 1 * 2 + h * 2), dtype=F64), a, b, a_log, dt,
                                          torch.ones((4, 2 * 1 * 2 + h * 2), dtype=F64),
                                          torch.ones((1, 1), dtype=torch.int64), key_heads=1, key_dim=2,
                                          value_heads=h, value_dim=2, dtype=F64)
    for got_g, got_b in ((g, beta), (g2, beta2)):
        for i, (wg, wb) in enumerate(want):
            assert abs(float(got_g[0, 0, i]) - wg) <= 1e-14 * max(1.0, abs(wg)), (i, float(got_g[0, 0, i]), wg)
            assert abs(float(got_b[0, 0, i]) - wb) <= 1e-15, (i, float(got_b[0, 0, i]), wb)


def _hf_core(inputs, cot, *, key_heads, key_dim, value_heads, value_dim, monkeypatch):
    """HF transformers' Qwen3_5GatedDeltaNet.forward (modeling_qwen3_5.py:432-530, an
    implementation independent of this repository) in float64 on given projections: the
    in_proj modules return qkv, a, b as given, conv1d / A_log / dt_bias hold the oracle's
    parameters, the delta rule is replaced by the float64 token recurrence (HF's own rule
    casts to float32) after HF's in-kernel l2norm and q scale, and the core output is read at
    the norm's input. Returns the rule's inputs as HF composed them (q, k after its l2norm and
    scale, v, g, beta), the core output [B,T,H,Dv] and the gradients of sum(out * cot) w.r.t.
    qkv, a, b, A_log, dt_bias and the conv weight (as [K, W])."""
    hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    qkv, a, b, a_log, dt_bias, w, _ = inputs
    batch, length, _ = qkv.shape
    cfg = Qwen3_5TextConfig(hidden_size=8, linear_num_key_heads=key_heads, linear_num_value_heads=value_heads,
                            linear_key_head_dim=key_dim, linear_value_head_dim=value_dim,
                            linear_conv_kernel_dim=w.shape[0], num_hidden_layers=1,
                            layer_types=["linear_attention"], hidden_act="silu", rms_norm_eps=1e-6)
    torch.manual_seed(0)
    m = hf.Qwen3_5GatedDeltaNet(cfg, 0).double()
    leaves = {n: x.detach().to(F64).clone().requires_grad_(True) for n, x in (("qkv", qkv), ("a", a), ("b", b))}

    class Given(torch.nn.Module):
        def __init__(self, t):
            super().__init__()
            self.t = t

        def forward(self, _x):
            return self.t

    m.in_proj_qkv, m.in_proj_a, m.in_proj_b = Given(leaves["qkv"]), Given(leaves["a"]), Given(leaves["b"])
    m.in_proj_z = Given(torch.zeros((batch, length, value_heads * value_dim), dtype=F64))
    with torch.no_grad():
        m.conv1d.weight.copy_(w.to(F64).T[:, None, :])
        m.A_log.copy_(a_log.to(F64))
        m.dt_bias.copy_(dt_bias.to(F64))
    seen = {}

    def rule64(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=False,
               use_qk_l2norm_in_kernel=False, **kw):
        if use_qk_l2norm_in_kernel:  # modeling_qwen3_5.py torch_chunk_gated_delta_rule's preamble
            query, key = hf.l2norm(query, dim=-1, eps=1e-6), hf.l2norm(key, dim=-1, eps=1e-6)
        query = query * query.shape[-1] ** -0.5
        seen.update(q=query, k=key, v=value, g=g, beta=beta)
        out, state = O.recurrent_gated_delta_rule(query, key, value, g, beta)
        return out, (state if output_final_state else None)

    monkeypatch.setattr(hf, "torch_chunk_gated_delta_rule", rule64)
    core = {}

    def grab(_mod, args):  # returns None: the norm's arguments stay as they are
        core["out"] = args[0]

    m.norm.register_forward_pre_hook(grab)
    m(torch.zeros((batch, length, 8), dtype=F64))
    out = core["out"].reshape(batch, length, value_heads, value_dim)
    params = [m.A_log, m.dt_bias, m.conv1d.weight]
    grads = torch.autograd.grad((out * cot.to(F64)).sum(), [leaves["qkv"], leaves["a"], leaves["b"], *params])
    names = ["qkv", "a", "b", "A_log", "dt_bias", "w"]
    result = {"out": out.detach()}
    result.update({n: g.detach() for n, g in zip(names, grads)})
    result["w"] = result["w"][:, 0, :].T
    return {k: v.detach() for k, v in seen.items()}, result


def _hf_vs_oracle(monkeypatch, seed=21):
    """Relative max errors of the oracle's composed core against HF's Qwen3_5GatedDeltaNet on
    one segment (T = 45, not a multiple of the chunk 16; GQA 2 -> 4 heads; the benchmark configs' gate
    spreads, A_log ~ U(0, ln 16)): the rule's inputs, the output and every gradient."""
    from tjev_amd.testing import cotangent, gdn_inputs

    shape = dict(key_heads=2, key_dim=8, value_heads=4, value_dim=8)
    qkv, a, b, a_log, dt_bias, w, seg = gdn_inputs(batch=2, length=45, key_heads=2, value_heads=4, dim=8,
                                                   seed=seed, style="baseline")
    cot = cotangent(2, 45, 4, 8, seed=seed + 1)
    # HF evaluates e^{A_log} in float32 (A_log.float().exp()); the oracle is given the A_log
    # whose float64 exponential is that float32 value, so both decay by the same rates
    a_log_hf = torch.log(a_log.to(F64).float().exp().to(F64))
    inputs = (qkv.to(F64), a.to(F64), b.to(F64), a_log.to(F64), dt_bias.to(F64), w.to(F64), seg)
    seen, hf = _hf_core(inputs, cot, monkeypatch=monkeypatch, **shape)
    ours_in = O.core_inputs(*inputs[:3], a_log_hf, *inputs[4:], dtype=F64, **shape)
    ours = O.reference_with_grads((*inputs[:3], a_log_hf, *inputs[4:]), cot, dtype=F64, chunk=16, **shape)
    err = {}
    for name, x in zip(("q", "k", "v", "g", "beta"), ours_in[:5]):
        err["in:" + name] = float((x - seen[name]).abs().max() / seen[name].abs().max())
    for name in hf:
        err[name] = float((ours[name] - hf[name]).abs().max() / hf[name].abs().max())
    return err


def test_core_inputs_match_hf_gated_deltanet(monkeypatch):
    """The oracle's composition conv -> SiLU -> split -> l2norm(q, k) -> q Dk^-1/2 -> gates ->
    GQA repeat (``core_inputs``, test_gdn_mega.py:44-58) against HF's GatedDeltaNet layer in
    float64: the delta rule's inputs and the core output agree to float64 rounding, and so
    does every gradient but those of a and A_log, which HF takes through float32 casts
    (``a.float()``, ``A_log.float().exp()``): those agree to float32 rounding."""
    err = _hf_vs_oracle(monkeypatch)
    for name, e in err.items():
        assert e <= (2e-7 if name in ("a", "A_log") else 1e-10), (name, err)


def test_padding_tokens_read_nothing_and_write_zeros():
    """valid = seg > 0 (pallas_tpu_mega.py:195-201, test_gdn_mega.py:47-48): padding tokens have
    zero q, k and v after the conv, their outputs are exactly 0, and the other tokens equal a
    run without them."""
    from tjev_amd.testing import gdn_inputs

    shape = dict(key_heads=2, key_dim=8, value_heads=4, value_dim=8)
    qkv, a, b, a_log, dt_bias, w, _ = gdn_inputs(batch=1, length=40, key_heads=2, value_heads=4, dim=8, seed=3,
                                                 dtype=F64)
    seg = torch.ones((1, 40), dtype=torch.int64)
    seg[0, 33:] = 0
    q, k, v, _, _, _ = O.core_inputs(qkv, a, b, a_log, dt_bias, w, seg, dtype=F64, **shape)
    assert torch.all(q[0, 33:] == 0) and torch.all(k[0, 33:] == 0) and torch.all(v[0, 33:] == 0)
    out = O.reference_core(qkv, a, b, a_log, dt_bias, w, seg, chunk=16, dtype=F64, **shape)
    assert torch.all(out[0, 33:] == 0)
    alone = O.reference_core(qkv[:, :33], a[:, :33], b[:, :33], a_log, dt_bias, w, seg[:, :33], chunk=16, dtype=F64,
                             **shape)
    assert float((out[:, :33] - alone).abs().max()) < 1e-12


def _slipped_gates(kind):
    def gates(a, b, a_log, dt_bias):
        sp = lambda x: torch.logaddexp(x, torch.zeros_like(x))  # noqa: E731
        if kind == "softplus(a) + dt_bias":
            return -torch.exp(a_log) * (sp(a) + dt_bias), torch.sigmoid(b)
        if kind == "A_log without exp":
            return -a_log * sp(a + dt_bias), torch.sigmoid(b)
        if kind == "beta = sigmoid(a)":
            return -torch.exp(a_log) * sp(a + dt_bias), torch.sigmoid(a)
        raise AssertionError(kind)
    return gates


@pytest.mark.parametrize("kind", ["softplus(a) + dt_bias", "A_log without exp", "beta = sigmoid(a)",
                                  "key heads tiled, not interleaved", "scale on k"])
def test_planted_composition_slips_are_caught(monkeypatch, kind):
    """A slip planted in the oracle's gates or composition fails the HF layer comparison and
    (for the gates) the closed forms."""
    if kind in ("softplus(a) + dt_bias", "A_log without exp", "beta = sigmoid(a)"):
        monkeypatch.setattr(O, "gates", _slipped_gates(kind))
        with pytest.raises(AssertionError):
            test_gates_closed_forms()
    else:
        orig = O.core_inputs

        def slipped(*args, **kw):
            q, k, v, g, beta, seg = orig(*args, **kw)
            ratio = kw["value_heads"] // kw["key_heads"]
            if kind == "key heads tiled, not interleaved":
                q, k = (x[:, :, ::ratio].repeat(1, 1, ratio, 1) for x in (q, k))
            else:
                q, k = q * kw["key_dim"] ** 0.5, k * kw["key_dim"] ** -0.5
            return q, k, v, g, beta, seg

        monkeypatch.setattr(O, "core_inputs", slipped)
    err = _hf_vs_oracle(monkeypatch)
    assert max(err.values()) > 1e-3, (kind, err)


# ------------------------------------------------------------------ masks
def test_masks_brute_force():
    """The integer masks against their per-token definitions on random rows with repeated,
    zero and negative ids (pallas_tpu_mega.py:349-361, pallas_tpu_v2.py:505-515)."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        chunk, taps = [8, 16][trial % 2], 1 + trial % 5
        n = 1 + trial % 4
        seg = rng.integers(-1, 4, size=(2, n * chunk))
        m = O.masks(seg, chunk, taps)
        for b in range(2):
            for t in range(n * chunk):
                c0 = (t // chunk) * chunk
                before = -2 if c0 == 0 else seg[b, c0 - 1]
                assert m["cont"][b, t] == int(seg[b, t] == before)
                assert m["in_last"][b, t] == int(seg[b, t] == seg[b, c0 + chunk - 1])
                assert m["valid"][b, t] == int(seg[b, t] > 0)
                for lag in range(1, taps):
                    # ids are padded with -1 in front (causal_conv1d.py:12): an id of -1 "keeps"
                    # the taps before the row start, which read the conv's zero padding
                    prev = seg[b, t - lag] if t - lag >= 0 else -1
                    assert m[f"keep_{lag}"][b, t] == int(prev == seg[b, t])


def test_masks_known_answer():
    seg = np.array([[1, 1, 1, 2, 2, 2, 0, 0]])
    m = O.masks(seg, 4, 3)
    assert m["cont"].tolist() == [[0, 0, 0, 0, 1, 1, 0, 0]]
    assert m["in_last"].tolist() == [[0, 0, 0, 1, 0, 0, 1, 1]]
    assert m["keep_1"].tolist() == [[0, 1, 1, 0, 1, 1, 0, 1]]
    assert m["keep_2"].tolist() == [[0, 0, 1, 0, 0, 1, 0, 0]]
    assert m["valid"].tolist() == [[1, 1, 1, 1, 1, 1, 0, 0]]
    m = O.masks(np.array([[3, 3, 3, 3, 3, 3, 3, 3]]), 4, 2)
    assert m["cont"].tolist() == [[0, 0, 0, 0, 1, 1, 1, 1]]


def test_heads_per_block_known_answers():
    """test_pallas_tpu.py:276-282."""
    got = [O.heads_per_block(h, r) for h, r in ((16, 1), (32, 2), (4, 2), (3, 1), (48, 3))]
    assert got == [8, 8, 4, 3, 6]
    with pytest.raises(ValueError):
        O.heads_per_block(5, 2)


# ------------------------------------------------------------------ the core
def test_reference_core_packed_rows_equal_segments_alone():
    """test_gdn_mega.py:135-147: conv taps and the state never cross a boundary."""
    from tjev_amd.testing import gdn_inputs

    qkv, a, b, a_log, dt_bias, w, _ = gdn_inputs(batch=1, length=96, key_heads=2, value_heads=4, dim=16,
                                                 style="reference", dtype=F64)
    spans = list(itertools.pairwise([0, 16, 33, 71, 96]))
    seg = torch.cat([torch.full((e - s,), i + 1) for i, (s, e) in enumerate(spans)])[None]
    kw = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16, chunk=16, dtype=F64)
    packed = O.reference_core(qkv, a, b, a_log, dt_bias, w, seg, **kw)
    for s, e in spans:
        alone = O.reference_core(qkv[:, s:e], a[:, s:e], b[:, s:e], a_log, dt_bias, w,
                                 torch.ones((1, e - s), dtype=torch.int64), **kw)
        assert torch.allclose(packed[:, s:e], alone, atol=1e-12)


def test_reference_core_chunked_equals_recurrent_with_grads():
    """The whole core (conv, norms, gates, rule) chunked vs token-recurrent in float64, forward
    and every input gradient, with packed segments and trailing padding."""
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).parent))
    from gdn_cases import case_inputs

    inputs, cot = case_inputs(1, 120, 2, 4, 16, cuts=[16, 33, 50, 67, 95])
    kw = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16)
    a = O.reference_with_grads(inputs, cot, rule="chunked", dtype=F64, **kw)
    b = O.reference_with_grads(inputs, cot, rule="recurrent", dtype=F64, **kw)
    for k in a:
        assert torch.allclose(a[k], b[k], atol=1e-10, rtol=1e-9), k


# ------------------------------------------------------------------ planted mistakes
def test_planted_mistakes_are_caught(monkeypatch):
    """Each check above has teeth: a broken oracle (no reset across a chunk boundary, a wrong
    decay sign, reversed conv taps, no zero-row guard) fails the corresponding check."""
    q, k, v, g, beta = _qkvgb(0)
    seg = _segments(2, 45, 0)
    ref, _ = O.recurrent_gated_delta_rule(q, k, v, g, beta, seg)

    # 1. the carried state never resets (cont forced true): chunked != recurrence
    orig_cat = torch.cat

    def no_reset(q_, k_, v_, g_, b_, s_, chunk):
        return O.chunk_gated_delta_rule(q_, k_, v_, g_, b_, torch.ones_like(s_), chunk=chunk)[0]
    assert not torch.allclose(no_reset(q, k, v, g, beta, seg, 16), ref, atol=1e-6)

    # 2. a sign slip in the decay (e^{+g}): chunked != recurrence
    bad, _ = O.chunk_gated_delta_rule(q, k, v, -g, beta, seg, chunk=16)
    assert not torch.allclose(bad, ref, atol=1e-6)

    # 3. reversed conv taps: textbook conv disagrees
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((1, 20, 3)))
    w = torch.from_numpy(rng.standard_normal((4, 3)))
    s1 = torch.ones((1, 20), dtype=torch.int64)
    assert not torch.allclose(O.segmented_causal_conv1d(x, w.flip(0), s1), _conv_textbook(x, w, s1), atol=1e-6)

    # 4. l2norm without the zero-row guard: the known answer's zero gradient fails
    monkeypatch.setattr(O, "l2norm", lambda x, eps=1e-6: x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps))
    xx = torch.zeros((1, 4), dtype=F64, requires_grad=True)
    (gr,) = torch.autograd.grad((O.l2norm(xx) * torch.ones(1, 4, dtype=F64)).sum(), xx)
    assert not torch.all(gr == 0)
    assert orig_cat is torch.cat


# ------------------------------------------------------------------ the gdn_tinv residual
def test_chunk_tinv_inverts_each_chunk_brute_force():
    """chunk_tinv against L built element by element from its definition (beta_i k_i.k_j
    e^(gamma_i - gamma_j) for i > j in one segment, gamma the in-chunk cumsum of g) and a dense
    fp64 inverse per chunk; a segment reset inside a chunk, padding, and T not a multiple of C."""
    rng = np.random.default_rng(7)
    b, t, h, d, c = 1, 40, 2, 8, 16
    k = torch.from_numpy(rng.standard_normal((b, t, h, d)))
    k = k / k.norm(dim=-1, keepdim=True)
    g = torch.from_numpy(-rng.uniform(0.01, 0.5, (b, t, h)))
    beta = torch.from_numpy(rng.uniform(0.1, 0.9, (b, t, h)))
    seg = torch.ones((b, t), dtype=torch.int64)
    seg[0, 21:] = 2
    seg[0, 37:] = 0
    got = O.chunk_tinv(k, g, beta, seg, chunk=c)
    n = (t + c - 1) // c
    assert got.shape == (b, h, n, c, c)
    for hh in range(h):
        for ch in range(n):
            lower = np.zeros((c, c))
            gam = np.zeros(c)
            run = 0.0
            for i in range(c):
                tok = ch * c + i
                run += float(g[0, tok, hh]) if tok < t else 0.0
                gam[i] = run
            for i in range(c):
                for j in range(i):
                    ti, tj = ch * c + i, ch * c + j
                    if ti >= t:  # padding: zero k and beta, the edge segment id
                        continue
                    if int(seg[0, ti]) != int(seg[0, tj]):
                        continue
                    lower[i, j] = float(beta[0, ti, hh]) * float(k[0, ti, hh] @ k[0, tj, hh]) * np.exp(gam[i] - gam[j])
            want = np.linalg.inv(np.eye(c) + lower)
            assert np.abs(got[0, hh, ch].numpy() - want).max() < 1e-12 * max(1.0, np.abs(want).max())
    # and the doubling restatement agrees with the solve on the same chunks
    lower = torch.linalg.inv(got) - torch.eye(c, dtype=got.dtype)
    assert float((O.unit_lower_inverse(lower) - got).abs().max()) < 1e-10


# ------------------------------------------------------------------ the GDN block
def test_merged_projection_equals_unmerged_fp64():
    """lora.py's two forms of one adapted projection, x (W + s A B) and x W + s (x A) B, agree
    in fp64, values and the gradients of x, A and B (the merged form's autograd gives the
    low-rank formulas dA = s x^T (dy B^T), dB = s (x A)^T dy)."""
    rng = np.random.default_rng(11)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s))  # noqa: E731
    x, w, a, b, dy = f(7, 12), f(12, 9), f(12, 3), f(3, 9), f(7, 9)
    leaves = [t.clone().requires_grad_(True) for t in (x, a, b)]
    ym = O.merged_projection(leaves[0], w, leaves[1], leaves[2], 1.7, F64)
    gm = torch.autograd.grad((ym * dy).sum(), leaves)
    leaves2 = [t.clone().requires_grad_(True) for t in (x, a, b)]
    yu = O.unmerged_projection(leaves2[0], w, leaves2[1], leaves2[2], 1.7, F64)
    gu = torch.autograd.grad((yu * dy).sum(), leaves2)
    assert float((ym - yu).detach().abs().max()) < 1e-12
    for p, q in zip(gm, gu):
        assert float((p - q).abs().max()) < 1e-12
    assert torch.allclose(gm[1], 1.7 * x.T @ (dy @ b.T)) and torch.allclose(gm[2], 1.7 * (x @ a).T @ dy)


def test_merged_projection_rounds_the_merged_kernel_once():
    """W' = W + s bf16(A) bf16(B) summed in the accumulation dtype and rounded once to the
    compute dtype (lora.py:284-295); x = [1] reads W' row 0."""
    w = torch.tensor([[1.0, 0.5]])
    a = torch.tensor([[2.0 ** -5]])
    b = torch.tensor([[2.0 ** -5, 3 * 2.0 ** -5]])
    x = torch.tensor([[1.0]])
    y = O.merged_projection(x, w, a, b, 0.5, torch.bfloat16)
    # W' = [1 + 2^-11, 0.5 + 3 * 2^-11]: both deltas are below half a bf16 ulp (2^-8 at 1,
    # 2^-9 at 0.5), so the merged kernel is W itself; in fp32 it is not
    assert y.dtype == torch.bfloat16 and y.tolist() == [[1.0, 0.5]]
    y32 = O.merged_projection(x, w, a, b, 0.5, torch.float32)
    assert y32.tolist() == [[1.0 + 2.0 ** -11, 0.5 + 3 * 2.0 ** -11]]


def test_gdn_block_zero_adapters_reduce_to_the_base_layer():
    """With B = 0 the block is the unadapted layer: base projections, the reference core, the
    gated norm, the padding select and out_proj, composed by hand here in fp64."""
    rng = np.random.default_rng(12)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s))  # noqa: E731
    hidden, hk, h, d = 8, 1, 2, 4
    width = 2 * hk * d + h * d
    names = {"in_proj_qkv": width, "in_proj_z": h * d, "in_proj_b": h, "in_proj_a": h}
    p = {n: (f(hidden, o) * 0.3, f(hidden, 2), torch.zeros(2, o, dtype=F64), 2.0) for n, o in names.items()}
    p["out_proj"] = (f(h * d, hidden) * 0.3, f(h * d, 2), torch.zeros(2, hidden, dtype=F64), 2.0)
    p.update(conv=f(4, width) * 0.5, a_log=torch.rand(h, dtype=F64), dt_bias=f(h), norm=1 + 0.1 * f(d))
    x = f(2, 11, hidden)
    seg = torch.tensor([[1] * 6 + [2] * 3 + [0] * 2, [1] * 11], dtype=torch.int32)
    got = O.gdn_block(x, seg, p, key_heads=hk, key_dim=d, value_heads=h, value_dim=d, dtype=F64, chunk=4)
    xm = torch.where((seg > 0)[..., None], x, 0.0)
    qkv, z, b, a = (xm @ p[n][0] for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"))
    core = O.reference_core(qkv, a, b, p["a_log"], p["dt_bias"], p["conv"], seg, key_heads=hk, key_dim=d,
                            value_heads=h, value_dim=d, chunk=4, dtype=F64)
    normed = O.gated_rmsnorm(core, z.reshape(2, 11, h, d), p["norm"]).reshape(2, 11, -1)
    want = torch.where((seg > 0)[..., None], normed, 0.0) @ p["out_proj"][0]
    assert float((got - want).abs().max()) < 1e-12
    assert torch.all(got[0, 9:] == 0)


def _block_case(seed=31):
    """A small GDN block in fp64 (hidden 8 = H * Dv, so a norm after out_proj is expressible as
    a slip; GQA 1 -> 2 heads of 4; nonzero adapters on all five projections, rsLoRA-sized
    scale), an input x [2, 23, 8], a cotangent, and per-row valid lengths (row 1 starts with
    three padding tokens). A_log is chosen so that its float32 exponential, as HF evaluates it,
    is exact in float64."""
    rng = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s))  # noqa: E731
    hidden, hk, h, d, r = 8, 1, 2, 4, 2
    width = 2 * hk * d + h * d
    names = {"in_proj_qkv": width, "in_proj_z": h * d, "in_proj_b": h, "in_proj_a": h}
    p = {n: (f(hidden, o) * 0.4, f(hidden, r) / r ** 0.5, f(r, o) * 0.1, 1.5) for n, o in names.items()}
    p["out_proj"] = (f(h * d, hidden) * 0.4, f(h * d, r) / r ** 0.5, f(r, hidden) * 0.1, 1.5)
    a_log = torch.log(torch.from_numpy(rng.uniform(1.0, 16.0, h)).float().to(F64))
    p.update(conv=f(4, width) * 0.5, a_log=a_log, dt_bias=f(h), norm=1 + 0.2 * f(d))
    x = f(2, 23, hidden)
    seg = torch.ones((2, 23), dtype=torch.int32)
    seg[1, :3] = 0
    return dict(hidden=hidden, key_heads=hk, key_dim=d, value_heads=h, value_dim=d), p, x, seg, f(2, 23, hidden)


def _hf_block(shape, p, x, seg, cot, monkeypatch):
    """HF transformers' whole Qwen3_5GatedDeltaNet layer (modeling_qwen3_5.py:432-545: input
    mask, in_proj_qkv/z/b/a, conv + SiLU, split, gates, l2norm and q scale, the delta rule,
    the gated RMSNorm per head with gate z, out_proj) in float64 with its Linear weights set to
    the block's merged kernels W + s A B and its conv, A_log, dt_bias and norm weight to the
    block's; the padding rows go in as HF's attention mask. Its delta rule is replaced by the
    float64 token recurrence (HF's own casts to float32). HF still evaluates the norm and
    e^{A_log} in float32. Returns the output and dx of sum(out * cot)."""
    hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    cfg = Qwen3_5TextConfig(hidden_size=shape["hidden"], linear_num_key_heads=shape["key_heads"],
                            linear_num_value_heads=shape["value_heads"], linear_key_head_dim=shape["key_dim"],
                            linear_value_head_dim=shape["value_dim"], linear_conv_kernel_dim=4, num_hidden_layers=1,
                            layer_types=["linear_attention"], hidden_act="silu", rms_norm_eps=1e-6)
    torch.manual_seed(0)
    m = hf.Qwen3_5GatedDeltaNet(cfg, 0).double()
    with torch.no_grad():
        for name in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
            w, la, lb, s = p[name]
            getattr(m, name).weight.copy_((w + s * (la @ lb)).T)
        m.conv1d.weight.copy_(p["conv"].T[:, None, :])
        m.A_log.copy_(p["a_log"])
        m.dt_bias.copy_(p["dt_bias"])
        m.norm.weight.copy_(p["norm"])

    def rule64(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=False,
               use_qk_l2norm_in_kernel=False, **kw):
        if use_qk_l2norm_in_kernel:
            query, key = hf.l2norm(query, dim=-1, eps=1e-6), hf.l2norm(key, dim=-1, eps=1e-6)
        query = query * query.shape[-1] ** -0.5
        out, state = O.recurrent_gated_delta_rule(query, key, value, g, beta)
        return out, (state if output_final_state else None)

    monkeypatch.setattr(hf, "torch_chunk_gated_delta_rule", rule64)
    xl = x.clone().requires_grad_(True)
    out = m(xl, attention_mask=(seg > 0).to(F64))
    (dx,) = torch.autograd.grad((out * cot).sum(), [xl])
    return out.detach(), dx


def _oracle_block(shape, p, x, seg, cot, block=None):
    kw = {k: v for k, v in shape.items() if k != "hidden"}
    xl = x.clone().requires_grad_(True)
    out = (block or O.gdn_block)(xl, seg, p, dtype=F64, chunk=8, **kw)
    (dx,) = torch.autograd.grad((out * cot).sum(), [xl])
    return out.detach(), dx


def _block_slip(kind):
    """gdn_block with one plausible slip in its composition (model/gdn.py:126-164 is the order
    being pinned): the norm's gate taken from the value part of in_proj_qkv instead of
    in_proj_z; the norm applied after out_proj; the RMS taken over all heads at once (one flat
    row) instead of per head; the input's padding mask dropped."""
    def block(x, segment_ids, params, *, key_heads, key_dim, value_heads, value_dim, dtype, chunk):
        batch, length, _ = x.shape
        valid = (segment_ids > 0)[..., None]
        if kind != "input mask dropped":
            x = torch.where(valid, x, torch.zeros((), dtype=x.dtype))
        proj = lambda t, n: O.merged_projection(t, *params[n], dtype)  # noqa: E731
        qkv, z, b, a = (proj(x, n) for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"))
        if kind == "gate from in_proj_qkv":
            z = qkv[..., 2 * key_heads * key_dim:]
        core = O.reference_core(qkv, a, b, params["a_log"], params["dt_bias"], params["conv"], segment_ids,
                                key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                                value_dim=value_dim, chunk=chunk, dtype=dtype)
        zh = z.reshape(batch, length, value_heads, value_dim)
        if kind == "norm after out_proj":
            y = proj(core.reshape(batch, length, -1), "out_proj").reshape(batch, length, value_heads, value_dim)
            y = O.gated_rmsnorm(y, zh, params["norm"]).reshape(batch, length, -1)
            return torch.where(valid, y, torch.zeros((), dtype=y.dtype))
        if kind == "one RMS over all heads":
            flat = core.reshape(batch, length, 1, -1)
            normed = O.gated_rmsnorm(flat, z.reshape(batch, length, 1, -1), params["norm"].repeat(value_heads))
        else:
            normed = O.gated_rmsnorm(core, zh, params["norm"])
        y = torch.where(valid, normed.reshape(batch, length, -1), torch.zeros((), dtype=dtype))
        return proj(y, "out_proj")
    return block


def _max_rel(a, b):
    return float((a - b).abs().max() / b.abs().max())


def test_gdn_block_matches_hf_layer(monkeypatch):
    """The oracle's whole block (``gdn_block``: input mask, merged-LoRA projections, core,
    per-head gated RMSNorm with gate z, padding select, out_proj; model/gdn.py:126-164) against
    HF's Qwen3_5GatedDeltaNet layer (an independent implementation of the same layer order)
    in float64 with the same parameters: output and dx agree to float32 rounding (HF evaluates
    the norm and e^{A_log} in float32: 1e-7), on a row without padding and on a row whose
    first three tokens are padding (HF's attention mask)."""
    shape, p, x, seg, cot = _block_case()
    hf_out, hf_dx = _hf_block(shape, p, x, seg, cot, monkeypatch)
    out, dx = _oracle_block(shape, p, x, seg, cot)
    err = {"out": _max_rel(out, hf_out), "dx": _max_rel(dx, hf_dx)}
    assert max(err.values()) < 2e-6, err
    assert torch.all(out[1, :3] == 0) and torch.all(dx[1, :3] == 0)


@pytest.mark.parametrize("kind", ["gate from in_proj_qkv", "norm after out_proj", "one RMS over all heads"])
def test_gdn_block_slips_fail_the_hf_layer(monkeypatch, kind):
    """Each composition slip, planted in a copy of the block, moves out or dx far beyond the
    float32 rounding at which the oracle agrees with HF."""
    shape, p, x, seg, cot = _block_case()
    hf_out, hf_dx = _hf_block(shape, p, x, seg, cot, monkeypatch)
    out, dx = _oracle_block(shape, p, x, seg, cot, block=_block_slip(kind))
    assert max(_max_rel(out, hf_out), _max_rel(dx, hf_dx)) > 1e-2, kind


def test_gdn_block_input_mask_is_redundant():
    """Dropping the block's input mask (gdn.py:126-164 masks x before the projections) changes
    neither out nor dx: every path from a padding token's x is masked downstream (its conv
    output by valid, its own output by the padding select, its gates cancel in the decay
    differences of the segment after it). So that mask cannot be pinned by any comparison of
    outputs; the HF comparison above pins the rest of the order."""
    shape, p, x, seg, cot = _block_case()
    out, dx = _oracle_block(shape, p, x, seg, cot)
    out2, dx2 = _oracle_block(shape, p, x, seg, cot, block=_block_slip("input mask dropped"))
    assert _max_rel(out2, out) < 1e-13 and _max_rel(dx2, dx) < 1e-13
    # the slips' copy of the block without a slip is the oracle's block itself
    out0, dx0 = _oracle_block(shape, p, x, seg, cot, block=_block_slip("none"))
    assert torch.equal(out0, out) and torch.equal(dx0, dx)


# ------------------------------------------------------------------ decode
def test_decode_step_continues_the_recurrence():
    """test_gated_delta_rule.py:61-73's continuation on the megakernel's inputs: the token
    recurrence over T+3 tokens equals a prefill of T (its final state and last K-1 raw rows)
    followed by three decode steps, output and state, in fp64 (mega2 and mega1)."""
    from tjev_amd.testing import gdn_inputs

    for conv in (True, False):
        qkv, a, b, a_log, dt_bias, w, _ = gdn_inputs(batch=2, length=23, key_heads=1, value_heads=2, dim=8,
                                                     dtype=F64, seed=13)
        w = w.to(F64) if conv else None
        kw = dict(key_heads=1, key_dim=8, value_heads=2, value_dim=8)
        seg = torch.ones((2, 23), dtype=torch.int64)
        full = O.reference_core(qkv, a, b, a_log, dt_bias, w, seg, conv=conv, rule="recurrent", dtype=F64, **kw)
        q, k, v, g, beta, _ = O.core_inputs(qkv[:, :20], a[:, :20], b[:, :20], a_log, dt_bias, w, seg[:, :20],
                                            conv=conv, dtype=F64, **kw)
        _, state = O.recurrent_gated_delta_rule(q, k, v, g, beta, seg[:, :20])
        hist = qkv[:, 17:20] if conv else None
        for t in range(20, 23):
            out, hist, state = O.decode_step(qkv[:, t], a[:, t], b[:, t], a_log, dt_bias, w, hist, state,
                                             dtype=F64, **kw)
            assert float((out - full[:, t]).abs().max()) < 1e-12
        _, end = O.recurrent_gated_delta_rule(*O.core_inputs(qkv, a, b, a_log, dt_bias, w, seg, conv=conv,
                                                               dtype=F64, **kw)[:5], seg)
        assert float((state - end).abs().max()) < 1e-12
