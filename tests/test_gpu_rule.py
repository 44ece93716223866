"""The reference's tests of the chunked delta rule's precision and inverse variants
(tests/kernels/test_gated_delta_rule.py:110-160), run on this build's kernels through
tjev_amd.v2.chunk_gated_delta_rule (the rule with its state I/O, xla.py:170-262, on the v2
operator; "solve" runs the blocked inverse): output and final state against the fp64 token
recurrence at the reference's tolerances, on its shapes (2 rows of 130 tokens, 3 heads, Dk 8,
Dv 6: zero-padded to the compiled dim 16, chunk 16, packed segments) and on correlated keys
with slow decays, the hard case for the inverse; the latter also at the model's head dim and
chunk (128), under both inverse forms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _l2norm(x):
    return x / x.norm(dim=-1, keepdim=True)


def _inputs(seed, batch=2, length=45, heads=3, dk=8, dv=6):
    """test_gated_delta_rule._inputs: q, k l2-normalized (q scaled by Dk^-1/2), g =
    -softplus(N(0, 1)), beta = sigmoid(N(0, 1))."""
    rng = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(rng.standard_normal(s))  # noqa: E731
    q = _l2norm(f(batch, length, heads, dk)) * dk ** -0.5
    k = _l2norm(f(batch, length, heads, dk))
    v = f(batch, length, heads, dv)
    g = -torch.nn.functional.softplus(f(batch, length, heads))
    beta = torch.sigmoid(f(batch, length, heads))
    return q, k, v, g, beta


def _segments(batch, length, seed):
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(batch):
        cuts = np.sort(rng.choice(np.arange(1, length), size=4, replace=False))
        rows.append(np.searchsorted(cuts, np.arange(length), side="right") + 1)
    return torch.from_numpy(np.stack(rows).astype(np.int32))


def _hip_rule(q, k, v, g, beta, seg, **kw):
    from tjev_amd.v2 import chunk_gated_delta_rule

    args = [x.float().cuda() for x in (q, k, v, g, beta)]
    out, state = chunk_gated_delta_rule(*args, None if seg is None else seg.cuda(), **kw)
    torch.cuda.synchronize()
    return out.double().cpu(), state.double().cpu()


def _max_rel(p, q):
    return float((p - q).abs().max() / q.abs().max())


@pytest.mark.parametrize(("precision", "inverse", "tol"), [
    ("highest", "doubling", 5e-5), ("highest", "blocked", 5e-5), ("high", "blocked", 3e-3), ("high", "solve", 3e-3),
    ("bf16", "solve", 3e-2), ("bf16", "doubling", 3e-2), ("mixed", "solve", 3e-2),
])
def test_fast_variants_match_recurrence(precision, inverse, tol):
    from oracle.gdn_oracle import recurrent_gated_delta_rule

    q, k, v, g, beta = _inputs(5, length=130)
    seg = _segments(q.shape[0], q.shape[1], 5)
    ref, ref_state = recurrent_gated_delta_rule(q, k, v, g, beta, seg.long())
    out, state = _hip_rule(q, k, v, g, beta, seg, chunk=16, precision=precision, inverse=inverse)
    errs = (_max_rel(out, ref), _max_rel(state, ref_state))
    print(f"{precision} {inverse}: out {errs[0]:.1e} state {errs[1]:.1e}", flush=True)
    assert errs[0] < tol and errs[1] < tol, errs


@pytest.mark.parametrize(("dim", "chunk", "inverse"), [(8, 16, "doubling"), (128, 128, "doubling"),
                                                       (128, 128, "blocked")])
def test_inverse_on_correlated_keys_matches_recurrence(dim, chunk, inverse):
    """test_gated_delta_rule.py:150-159 (Dk 8, chunk 16, doubling), and the model's Dk = Dv =
    128 at chunk 128: keys all close to one direction (L ~ beta on the whole strict lower
    triangle), beta in [0.9, 1], decays 100x slower than the other tests'."""
    from oracle.gdn_oracle import recurrent_gated_delta_rule

    rng = np.random.default_rng(13)
    base = torch.from_numpy(rng.standard_normal((1, 1, 1, dim)))
    k = _l2norm(base + 0.05 * torch.from_numpy(rng.standard_normal((2, 2 * chunk if dim > 8 else 64, 3, dim))))
    q, _, v, g, beta = _inputs(15, length=k.shape[1], dk=dim, dv=dim if dim > 8 else 6)
    g = g * 0.01
    beta = beta.clamp(0.9, 1.0)
    ref, ref_state = recurrent_gated_delta_rule(q, k, v, g, beta)
    out, state = _hip_rule(q, k, v, g, beta, None, chunk=chunk, inverse=inverse)
    err = float((out - ref).abs().max())
    print(f"correlated keys Dk={dim} C={chunk} {inverse}: max abs {err:.1e}, state {_max_rel(state, ref_state):.1e}",
          flush=True)
    torch.testing.assert_close(out, ref, atol=2e-4, rtol=2e-4)
    assert _max_rel(state, ref_state) < 2e-4
