"""CPU restatement of tjev's XLA Gated DeltaNet path (the megakernel's parity oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` (as the
checker) and ``bench.py``'s CPU-baseline leg, never by the product path.

Each function follows a reference file (paths relative to the tjev repository root):

- ``tap_masks`` / ``segmented_causal_conv1d``  src/tjev/kernels/causal_conv1d.py:10-46
- ``l2norm``                                   src/tjev/kernels/gated_delta_rule/xla.py:42-53
- ``unit_lower_inverse``                       xla.py:66-100 (doubling) and
                                               pallas_tpu_v2.py:144-193 (16x16 diagonal
                                               blocks by substitution, then doubling)
- ``recurrent_gated_delta_rule``               xla.py:141-167
- ``chunk_gated_delta_rule``                   xla.py:170-262 (precision "highest",
                                               inverse "solve")
- ``chunk_tinv``                               the forward's gdn_tinv residual
                                               (pallas_tpu_mega.py:444-449, 546): (I + L)^-1
                                               of each chunk, L as in xla.py:205-240
- ``masks``                                    pallas_tpu_mega.py:349-361 with
                                               pallas_tpu_v2.py:505-515 (integer logic)
- ``heads_per_block``                          pallas_tpu_v2.py:518-525
- ``gates``                                  pallas_tpu_mega.py:106-145, test_gdn_mega.py:52-53
- ``reference_core`` / ``core_inputs``        tests/kernels/test_gdn_mega.py:44-58
                                               (``_reference``), the recurrent variant
                                               tests/kernels/test_gdn_long.py:131-176
- ``gated_rmsnorm``                            src/tjev/model/norms.py:13-15, 36-40
- ``merged_projection`` / ``unmerged_projection``  src/tjev/model/lora.py:284-301 / 132-150
- ``gdn_block``                                src/tjev/model/gdn.py:126-164 (flat norm,
                                               every projection adapted)
- ``decode_step``                              xla.py:141-167 at T = 1 with an initial state,
                                               the conv as HF causal_conv1d_update

Gradients come from torch autograd through these functions, as the reference takes
``jax.grad`` of the same XLA program (test_gdn_mega.py:75-86). Arithmetic runs in the dtype
of the floating inputs: float32 reproduces the reference's fp32 ("highest") numerics up to
operation order, float64 is the truth the float32 path and the GPU kernels are judged by.
"""

from __future__ import annotations

import numpy as np
import torch

PRECISIONS = ("highest", "high", "bf16", "mixed")  # xla.py:23


# --------------------------------------------------------------------------- conv
def tap_masks(segment_ids: torch.Tensor, taps: int) -> list[torch.Tensor]:
    """keep[L] [B,T] bool: token t may read token t-L (same segment id, t-L >= 0), L = 0..K-1.
    causal_conv1d.py:10-17 (the front is padded with id -1)."""
    length = segment_ids.shape[1]
    sp = torch.nn.functional.pad(segment_ids, (taps - 1, 0), value=-1)
    return [sp[:, taps - 1 - lag : taps - 1 - lag + length] == segment_ids for lag in range(taps)]


def _shift(x: torch.Tensor, lag: int) -> torch.Tensor:
    """y[t] = x[t-lag], zeros before the start (causal_conv1d.py:20-23)."""
    if lag == 0:
        return x
    return torch.nn.functional.pad(x, (0, 0, lag, 0))[:, : x.shape[1]]


def segmented_causal_conv1d(x: torch.Tensor, weight: torch.Tensor,
                            segment_ids: torch.Tensor) -> torch.Tensor:
    """Depthwise causal conv that never mixes segments (causal_conv1d.py:32-46).

    x [B,T,W], weight [K,W] (weight[K-1] multiplies the current token). Accumulates in
    float32 (float64 when x is float64) lag 0 first, then lags 1..K-1; output in x.dtype."""
    taps = weight.shape[0]
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    keeps = tap_masks(segment_ids, taps)
    out = torch.zeros(x.shape, dtype=acc)
    for lag in range(taps):
        w = weight[taps - 1 - lag].to(acc)
        out = out + torch.where(keeps[lag][..., None], _shift(x, lag).to(acc), 0.0) * w
    return out.to(x.dtype)


# --------------------------------------------------------------------------- norms
def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(||x||^2 + eps) over the last axis; all-zero rows map to 0 with a zero
    gradient (the double select of xla.py:49-53)."""
    sq = torch.sum(x * x, dim=-1, keepdim=True)
    zero = sq == 0
    safe = torch.where(zero, torch.ones_like(x), x)
    out = safe * torch.rsqrt(torch.where(zero, torch.ones_like(sq), sq) + eps)
    return torch.where(zero, torch.zeros_like(x), out)


def gated_rmsnorm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor,
                  eps: float = 1e-6) -> torch.Tensor:
    """GDN output norm (norms.py:13-15, 36-40): w * (x*rsqrt(mean x^2 + eps)) rounded to
    x.dtype and back, times silu(gate), in float32, cast to x.dtype. x, gate [..., H, D]."""
    dtype = x.dtype
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    xf = x.to(acc)
    normed = (xf * torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps))
    normed = normed.to(dtype).to(acc)
    g = gate.to(acc)
    return (weight.to(acc) * normed * (g * torch.sigmoid(g))).to(dtype)


# --------------------------------------------------------------------------- inverse
def doubling_masks(size: int) -> list[np.ndarray]:
    """xla.py:66-79: per level s = 1, 2, 4, ...: the lower-left s x s block of every
    2s x 2s diagonal block."""
    row = np.arange(size)[:, None]
    col = np.arange(size)[None, :]
    out, s = [], 1
    while s < size:
        out.append((row // (2 * s) == col // (2 * s)) & (row // s == 2 * (row // (2 * s)) + 1)
                   & (col // s == 2 * (col // (2 * s))))
        s *= 2
    return out


def unit_lower_inverse(lower: torch.Tensor, block: int = 0, bf16_operands: bool = False) -> torch.Tensor:
    """(I + L)^-1 for strictly lower-triangular L [..., C, C] (C a power of two).

    ``block`` 0: recursive doubling from T = I (xla.py:82-100). ``block`` > 1: the exact
    block x block diagonal inverse by forward substitution first, then the remaining
    doubling levels (pallas_tpu_v2.py:144-193, ``inverse="blocked"``). ``bf16_operands``: each
    doubling product's operands rounded to bf16 first, the product accumulated in the input
    dtype (``mm`` / ``_dot`` at mode "bf16", xla.py:55-62, pallas_tpu_v2.py:88-93)."""

    def mm(a, b):
        if bf16_operands:
            a, b = a.to(torch.bfloat16).to(a.dtype), b.to(torch.bfloat16).to(b.dtype)
        return a @ b

    c = lower.shape[-1]
    row = torch.arange(c)[:, None]
    col = torch.arange(c)[None, :]
    eye = (row == col).to(lower.dtype)
    block = min(block, c)
    if block > 1:
        same = (row // block) == (col // block)
        ld = torch.where(same, lower, 0.0)
        x = eye.expand(lower.shape).clone()
        for r in range(block - 1):
            l_col = torch.sum(torch.where(col == (row // block) * block + r, ld, 0.0), -1,
                              keepdim=True)
            x_row = torch.sum(torch.where(row == (col // block) * block + r, x, 0.0), -2,
                              keepdim=True)
            x = x - torch.where(same, l_col * x_row, 0.0)
        tinv, s = x, block
    else:
        tinv, s = eye.expand(lower.shape).clone(), 1
    while s < c:
        mask = ((row // (2 * s)) == (col // (2 * s))) & ((row // s) % 2 == 1) & ((col // s) % 2 == 0)
        off = torch.where(mask, lower, 0.0)
        tinv = tinv - mm(mm(tinv, off), tinv)
        s *= 2
    return tinv


# --------------------------------------------------------------------------- delta rule
def recurrent_gated_delta_rule(q, k, v, g, beta, segment_ids=None, initial_state=None):
    """Token-by-token reference (xla.py:141-167). q,k [B,T,H,Dk]; v [B,T,H,Dv]; g, beta
    [B,T,H]. The state restarts where the segment id changes. Returns (out, final_state)."""
    batch, length, heads, dk = k.shape
    dv = v.shape[-1]
    dt = q.dtype
    if segment_ids is None:
        segment_ids = torch.ones((batch, length), dtype=torch.int64)
    previous = torch.cat([segment_ids[:, :1], segment_ids[:, :-1]], dim=1)
    restart = segment_ids != previous
    restart[:, 0] = initial_state is None
    s = (torch.zeros((batch, heads, dk, dv), dtype=dt) if initial_state is None
         else initial_state.to(dt))
    outs = []
    for t in range(length):
        s = torch.where(restart[:, t, None, None, None], torch.zeros_like(s), s)
        s = s * torch.exp(g[:, t])[..., None, None]
        memory = torch.einsum("bhkv,bhk->bhv", s, k[:, t])
        delta = (v[:, t] - memory) * beta[:, t][..., None]
        s = s + k[:, t][..., :, None] * delta[..., None, :]
        outs.append(torch.einsum("bhkv,bhk->bhv", s, q[:, t]))
    return torch.stack(outs, dim=1), s


def _chunk_terms(q, k, v, g, beta, segment_ids, initial_state, chunk: int) -> dict:
    """The chunk-local terms of the chunked form (xla.py:198-240): T padded to a multiple of
    ``chunk`` with zero q/k/v/beta, g = 0 and the edge segment id (xla.py:198-204), inputs as
    [B,H,N,C,...], the segment masks, the in-chunk decay and L = strict((k beta) k^T . decay)."""
    batch, length, heads, dk = k.shape
    if segment_ids is None:
        segment_ids = torch.ones((batch, length), dtype=torch.int64)
    segment_ids = segment_ids.to(torch.int64)
    pad = (-length) % chunk
    if pad:
        q, k, v = (torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad)) for x in (q, k, v))
        g, beta = (torch.nn.functional.pad(x, (0, 0, 0, pad)) for x in (g, beta))
        segment_ids = torch.cat([segment_ids, segment_ids[:, -1:].expand(batch, pad)], dim=1)
    n = (length + pad) // chunk

    def chunked(x):  # [B,T,H,...] -> [B,H,N,C,...]
        x = x.reshape(batch, n, chunk, heads, *x.shape[3:])
        return torch.movedim(x, 3, 1)

    q, k, v, g, beta = (chunked(x) for x in (q, k, v, g, beta))
    seg = segment_ids.reshape(batch, n, chunk)
    first = (seg[:, :1, 0] if initial_state is not None
             else torch.full((batch, 1), -2, dtype=seg.dtype))
    before = torch.cat([first, seg[:, :-1, -1]], dim=1)
    continues = (seg == before[..., None])[:, None]  # [B,1,N,C]
    in_last = (seg == seg[..., -1:])[:, None]
    causal = torch.tril(torch.ones((chunk, chunk), dtype=torch.bool))
    same = ((seg[..., :, None] == seg[..., None, :]) & causal)[:, None]  # [B,1,N,C,C]

    cum = torch.cumsum(g, dim=-1)  # [B,H,N,C]
    diff = cum[..., :, None] - cum[..., None, :]
    decay = torch.exp(torch.where(same, diff, torch.full_like(diff, -torch.inf)))
    k_beta = k * beta[..., None]
    strict = torch.tril(torch.ones((chunk, chunk), dtype=torch.bool), -1)
    lower = torch.where(strict, (k_beta @ k.transpose(-1, -2)) * decay, 0.0)
    return dict(q=q, k=k, v=v, beta=beta, n=n, length=length, continues=continues, in_last=in_last,
                cum=cum, decay=decay, k_beta=k_beta, lower=lower)


def chunk_tinv(k, g, beta, segment_ids=None, chunk: int = 64) -> torch.Tensor:
    """(I + L)^-1 of every chunk [B,H,N,C,C] by triangular solve: the forward's ``gdn_tinv``
    residual (pallas_tpu_mega.py:444-449, 546), L as in ``chunk_gated_delta_rule``."""
    z = torch.zeros_like(k)
    lower = _chunk_terms(z, k, z, g, beta, segment_ids, None, chunk)["lower"]
    eye = torch.eye(chunk, dtype=k.dtype).expand(lower.shape)
    return torch.linalg.solve_triangular(lower + eye, eye, upper=False, unitriangular=True)


def chunk_gated_delta_rule(q, k, v, g, beta, segment_ids=None, initial_state=None,
                           chunk: int = 64):
    """Chunked WY/UT form with segment resets (xla.py:170-262) at precision "highest"
    (the matmuls in the inputs' float dtype) with the triangular solve (``inverse="solve"``).

    Pads T to a multiple of ``chunk`` with zero q/k/v/beta, g = 0 and the edge segment id
    (xla.py:198-204). Returns (out [B,T,H,Dv], final state [B,H,Dk,Dv])."""
    batch, length, heads, dk = k.shape
    dv = v.shape[-1]
    dt = q.dtype
    t = _chunk_terms(q, k, v, g, beta, segment_ids, initial_state, chunk)
    q, k, v, beta, n = t["q"], t["k"], t["v"], t["beta"], t["n"]
    continues, in_last, cum, decay, k_beta, lower = (t[x] for x in ("continues", "in_last", "cum", "decay",
                                                                   "k_beta", "lower"))
    carry_keep = continues[..., -1]
    v_beta = v * beta[..., None]
    grow = torch.exp(cum) * continues
    rhs = torch.cat([v_beta, k_beta * grow[..., None]], dim=-1)
    eye = torch.eye(chunk, dtype=dt)
    solved = torch.linalg.solve_triangular(lower + eye, rhs, upper=False, unitriangular=True)
    u, w = solved[..., :dv], solved[..., dv:]
    intra = (q @ k.transpose(-1, -2)) * decay
    q_read = q * grow[..., None]
    k_write = k * (torch.exp(cum[..., -1:] - cum) * in_last)[..., None]
    carry = torch.exp(cum[..., -1]) * carry_keep  # [B,H,N]

    s = (torch.zeros((batch, heads, dk, dv), dtype=dt) if initial_state is None
         else initial_state.to(dt))
    outs = []
    for i in range(n):
        v_new = u[:, :, i] - w[:, :, i] @ s
        outs.append(q_read[:, :, i] @ s + intra[:, :, i] @ v_new)
        s = s * carry[:, :, i, None, None] + k_write[:, :, i].transpose(-1, -2) @ v_new
    out = torch.stack(outs, dim=2).reshape(batch, heads, n * chunk, dv)
    return out.transpose(1, 2)[:, :length], s


# --------------------------------------------------------------------------- masks
def masks(segment_ids, chunk: int, taps: int) -> dict[str, np.ndarray]:
    """The megakernel's per-token integer masks (pallas_tpu_mega.py:349-361,
    pallas_tpu_v2.py:505-515) on ids [B,T] with T a multiple of ``chunk``:

    cont[t]    token t reads the incoming state: seg[t] == id of the previous chunk's last
               token (-2 before chunk 0)
    in_last[t] token t writes the outgoing state: seg[t] == id of its chunk's last token
    keep_L[t]  (L = 1..K-1) token t's conv reads t-L: t-L >= 0 and seg[t-L] == seg[t]
    valid[t]   seg[t] > 0
    The reference carries them as float32 (exact for |id| < 2**24); here they are ints."""
    seg = np.asarray(segment_ids, dtype=np.int64)
    batch, length = seg.shape
    if length % chunk:
        raise ValueError("masks: T must be a multiple of chunk (the megakernel pads first)")
    n = length // chunk
    s = seg.reshape(batch, n, chunk)
    before = np.concatenate([np.full((batch, 1), -2, np.int64), s[:, :-1, -1]], axis=1)
    out = {
        "seg": seg.copy(),
        "cont": (s == before[..., None]).reshape(batch, length).astype(np.int32),
        "in_last": (s == s[..., -1:]).reshape(batch, length).astype(np.int32),
        "valid": (seg > 0).astype(np.int32),
    }
    padded = np.pad(seg, ((0, 0), (taps - 1, 0)), constant_values=-1)
    for lag in range(1, taps):
        out[f"keep_{lag}"] = (padded[:, taps - 1 - lag: taps - 1 - lag + length] == seg
                              ).astype(np.int32)
    return out


def heads_per_block(heads: int, ratio: int, preferred: int = 8) -> int:
    """Value heads per program (pallas_tpu_v2.py:518-525): the largest multiple of the GQA
    ratio dividing H, up to ``preferred``."""
    if heads % ratio:
        raise ValueError(f"{heads} value heads are not groups of {ratio}")
    sizes = range(ratio, max(preferred, ratio) + 1, ratio)
    return max(size for size in sizes if heads % size == 0)


# --------------------------------------------------------------------------- the core
def reference_core(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads: int,
                   key_dim: int, value_heads: int, value_dim: int, conv: bool = True,
                   rule: str = "chunked", chunk: int = 64, dtype=torch.float32):
    """The XLA path the megakernel replaces (test_gdn_mega.py:44-58, ``_reference``):
    segmented causal conv -> SiLU -> padding mask (``conv``), l2norm(q) * Dk^-1/2, l2norm(k),
    beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias), key heads repeated for GQA,
    then the chunked delta rule at fp32 ("highest", triangular solve) or, with
    ``rule="recurrent"``, the token recurrence (the fp64 truth of test_gdn_long.py:131-176).

    Every floating input is cast to ``dtype`` first (bf16 projections are judged against
    the reference on the same values in fp32, test_gdn_mega.py:281-297). Returns
    [B,T,H,Dv] in ``dtype``; differentiable by autograd."""
    q, k, v, g, beta, seg = core_inputs(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, key_heads=key_heads,
                                        key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, conv=conv,
                                        dtype=dtype)
    if rule == "chunked":
        return chunk_gated_delta_rule(q, k, v, g, beta, seg, chunk=chunk)[0]
    if rule == "recurrent":
        return recurrent_gated_delta_rule(q, k, v, g, beta, seg)[0]
    raise ValueError(f"rule in (chunked, recurrent), not {rule!r}")


def core_inputs(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads: int, key_dim: int,
                value_heads: int, value_dim: int, conv: bool = True, dtype=torch.float32):
    """q, k (repeated to the value heads), v, g, beta and the int64 segment ids that
    ``reference_core`` feeds the delta rule (test_gdn_mega.py:44-58)."""
    qkv, a, b, a_log, dt_bias = (x.to(dtype) for x in (qkv, a, b, a_log, dt_bias))
    seg = segment_ids.to(torch.int64)
    batch, length, _ = qkv.shape
    hk, h, dk, dv = key_heads, value_heads, key_dim, value_dim
    if conv:
        x = segmented_causal_conv1d(qkv, conv_weight.to(dtype), seg)
        x = torch.where((seg > 0)[..., None], x * torch.sigmoid(x), 0.0)
    else:
        x = qkv
    q, k, v = torch.split(x, [hk * dk, hk * dk, h * dv], dim=-1)
    q = l2norm(q.reshape(batch, length, hk, dk)) * dk ** -0.5
    k = l2norm(k.reshape(batch, length, hk, dk))
    v = v.reshape(batch, length, h, dv)
    g, beta = gates(a, b, a_log, dt_bias)
    ratio = h // hk
    q, k = q.repeat_interleave(ratio, dim=2), k.repeat_interleave(ratio, dim=2)
    return q, k, v, g, beta, seg


def gates(a, b, a_log, dt_bias):
    """(g, beta) from the raw gate projections a, b [..., H] (pallas_tpu_mega.py:106-145,
    test_gdn_mega.py:52-53): g = -e^{A_log} softplus(a + dt_bias) with jax.nn.softplus =
    logaddexp(x, 0), beta = sigmoid(b)."""
    xg = a + dt_bias
    g = -torch.exp(a_log) * torch.logaddexp(xg, torch.zeros_like(xg))
    return g, torch.sigmoid(b)


def reference_with_grads(inputs, cotangent, *, key_heads, key_dim, value_heads, value_dim,
                         conv=True, rule="chunked", chunk=64, dtype=torch.float32,
                         want_conv_grad=True):
    """out and the gradients of sum(out * cotangent) w.r.t. qkv, a, b, A_log, dt_bias and the
    conv weight (test_gdn_mega.py:75-86), all as ``dtype`` tensors.
    ``inputs`` = (qkv, a, b, a_log, dt_bias, conv_weight, segment_ids)."""
    qkv, a, b, a_log, dt_bias, w, seg = inputs
    leaves = [x.detach().to(dtype).requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
    wl = w.detach().to(dtype).requires_grad_(want_conv_grad and conv) if w is not None else None
    out = reference_core(*leaves, wl, seg, key_heads=key_heads, key_dim=key_dim,
                         value_heads=value_heads, value_dim=value_dim, conv=conv, rule=rule,
                         chunk=chunk, dtype=dtype)
    loss = torch.sum(out * cotangent.to(dtype))
    targets = leaves + ([wl] if (wl is not None and wl.requires_grad) else [])
    grads = torch.autograd.grad(loss, targets, allow_unused=True)  # (an input the loss ignores: zeros)
    grads = [torch.zeros_like(t) if g is None else g for g, t in zip(grads, targets)]
    names = ["qkv", "a", "b", "A_log", "dt_bias", "w"]
    result = {"out": out.detach()}
    result.update({n: g.detach() for n, g in zip(names, grads)})
    return result


def fp64_truth(inputs, cotangent, **kw):
    """The same math in float64, token by token (test_gdn_long.py:131-176)."""
    kw = dict(kw)
    kw.update(rule="recurrent", dtype=torch.float64)
    return reference_with_grads(inputs, cotangent, **kw)


# --------------------------------------------------------------------------- the GDN block
def merged_projection(x: torch.Tensor, weight: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor,
                      scale: float, dtype) -> torch.Tensor:
    """x W' with W' = W + s A B (lora.py:284-301, ``_merge`` and ``_base_matmul``): A and B
    cast to ``dtype`` first, their product and the sum in the accumulation dtype, W' rounded
    once to ``dtype``. x [..., in], W [in, out], A [in, r], B [r, out]."""
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    delta = lora_a.to(dtype).to(acc) @ lora_b.to(dtype).to(acc)
    merged = (weight.to(acc) + scale * delta).to(dtype)
    return (x.to(dtype).to(acc) @ merged.to(acc)).to(dtype)


def unmerged_projection(x, weight, lora_a, lora_b, scale: float, dtype):
    """x W + s (x A) B, the unmerged form of the same projection (lora.py:132-150, 236-250)."""
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    xa = x.to(dtype).to(acc) @ lora_a.to(dtype).to(acc)
    base = x.to(dtype).to(acc) @ weight.to(dtype).to(acc)
    return (base + scale * (xa @ lora_b.to(dtype).to(acc))).to(dtype)


def gdn_block(x, segment_ids, params: dict, *, key_heads: int, key_dim: int, value_heads: int, value_dim: int,
              dtype=torch.float32, eps: float = 1e-6, chunk: int = 64, merged: bool = True, io_dtype=None):
    """``GatedDeltaNet.__call__`` (gdn.py:126-164) with ``gdn_norm=flat`` and every projection
    adapted: x with padding rows zeroed -> in_proj_qkv, in_proj_z, in_proj_b, in_proj_a ->
    ``reference_core`` (conv, gates, l2norm, chunked delta rule) -> the gated RMSNorm of each
    head (norms.py:42-62: the flat form is the same arithmetic) -> padding select -> out_proj.
    ``params``: {name: (W, A, B, scale)} for the five projections, and "conv", "a_log",
    "dt_bias", "norm" tensors. Differentiable by autograd (the adapters' gradients are the
    low-rank formulas of lora.py:320-366). ``io_dtype`` (bf16): the activations between the
    stages are stored in it, as the reference's bf16 layer stores them (projection outputs,
    the core's output, the norm's output), the core computing in ``dtype``."""
    io = io_dtype or dtype
    proj = merged_projection if merged else unmerged_projection
    batch, length, _ = x.shape
    valid = (segment_ids > 0)[..., None]
    x = torch.where(valid, x, torch.zeros((), dtype=x.dtype)).to(io)
    qkv, z, b, a = (proj(x, *params[n], io) for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"))
    out = reference_core(qkv, a, b, params["a_log"], params["dt_bias"], params["conv"], segment_ids,
                         key_heads=key_heads, key_dim=key_dim, value_heads=value_heads, value_dim=value_dim,
                         chunk=chunk, dtype=dtype)
    zh = z.reshape(batch, length, value_heads, value_dim)
    out = gated_rmsnorm(out.to(io), zh, params["norm"], eps).reshape(batch, length, -1)
    out = torch.where(valid, out, torch.zeros((), dtype=out.dtype))
    return proj(out, *params["out_proj"], io)


# --------------------------------------------------------------------------- decode
def decode_step(qkv, a, b, a_log, dt_bias, conv_weight, conv_state, state, *, key_heads: int, key_dim: int,
                value_heads: int, value_dim: int, dtype=torch.float32):
    """One token per row after a prefill (xla.py:141-167 with T = 1 and ``initial_state``; the
    conv over the kept rows as HF ``causal_conv1d_update``): qkv [B, W], a, b [B, H],
    conv_state [B, K-1, W] (oldest first), state [B, H, Dk, Dv]. Returns (out [B, H, Dv],
    conv_state', state'). The window [conv_state; qkv] is one segment, so the last row's conv
    reads exactly the kept rows."""
    conv = conv_weight is not None
    rows = qkv[:, None] if not conv or conv_state is None else torch.cat([conv_state.to(qkv.dtype), qkv[:, None]], 1)
    batch, window, _ = rows.shape
    pad = lambda x: torch.cat([torch.zeros((batch, window - 1, x.shape[-1]), dtype=x.dtype), x[:, None]], 1)  # noqa: E731
    seg = torch.ones((batch, window), dtype=torch.int64)
    q, k, v, g, beta, _ = core_inputs(rows, pad(a), pad(b), a_log, dt_bias, conv_weight, seg, key_heads=key_heads,
                                      key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, conv=conv,
                                      dtype=dtype)
    last = slice(window - 1, window)
    out, new_state = recurrent_gated_delta_rule(q[:, last], k[:, last], v[:, last], g[:, last], beta[:, last],
                                                initial_state=state.to(dtype))
    new_conv = None if not conv or conv_state is None else rows[:, 1:]
    return out[:, 0], new_conv, new_state
