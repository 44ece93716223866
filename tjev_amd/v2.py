"""tjev's v2 operator on MI355X: ``chunk_gated_delta_rule_v2`` (src/tjev/kernels/gated_delta_rule/
pallas_tpu_v2.py:541-582), the chunked gated delta rule on given q, k, v, g, beta -- what the
model calls with ``gdn_impl=pallas_tpu_v2`` after its own conv, l2norm and gates (gdn.py:47-97)
-- computed by the HIP library's chunk, scan and output kernels through its C ABI.

Same arguments, defaults and ValueErrors as the reference; out [B, T, H, Dv] in v's dtype; q
and k keep their dtype (fp32 or bf16), g and beta theirs. GQA: value head h reads key head
h // (H / Hk). The custom VJP gives d q, d k, d v, d g and d beta. ``vmem_fraction`` is
TPU-only and ignored; ``heads_per_step`` is checked as the reference does. ``residuals`` as
for ``gdn_megakernel`` (this build's choice of what the forward keeps). No fallback: without
the HIP library, or on a CPU tensor, the operator raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .gdn import INVERSE_BLOCKS, LANES, PRECISIONS, GdnPlan, _ptr, heads_per_block, run_dim, value_groups

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


class _V2(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan: GdnPlan, q, k, v, g, beta, seg):
        out = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        res = plan.residuals(v.device)
        ws = plan.workspace(False, v.device)
        _lib.check_status(plan.lib.tjev_gdn_v2_fwd(
            ctypes.byref(plan.params), plan._stream(v.device), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
            _ptr(seg), _ptr(out), _ptr(res), _ptr(ws), ws.numel()))
        ctx.plan = plan
        ctx.save_for_backward(q, k, v, g, beta, seg, res)
        return out

    @staticmethod
    def backward(ctx, d_out):
        plan: GdnPlan = ctx.plan
        q, k, v, g, beta, seg, res = ctx.saved_tensors
        d_out = d_out.to(v.dtype).contiguous()
        d_q, d_k, d_v = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        d_g, d_beta = torch.empty_like(g), torch.empty_like(beta)
        ws = plan.workspace(True, v.device)
        _lib.check_status(plan.lib.tjev_gdn_v2_bwd(
            ctypes.byref(plan.params), plan._stream(v.device), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
            _ptr(seg), _ptr(res), _ptr(d_out), _ptr(d_q), _ptr(d_k), _ptr(d_v), _ptr(d_g), _ptr(d_beta), _ptr(ws),
            ws.numel()))
        return None, d_q, d_k, d_v, d_g, d_beta, None


class _V2Cont(torch.autograd.Function):
    """``_V2`` with a state in and out (tjev_gdn_v2_fwd_cont / _bwd_cont)."""

    @staticmethod
    def forward(ctx, plan: GdnPlan, q, k, v, g, beta, seg, init_state, want_state):
        ctx.set_materialize_grads(False)
        p = plan.params
        out = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        res = plan.residuals(v.device)
        ws = plan.workspace(False, v.device)
        final = None
        if want_state:
            final = torch.empty((p.batch, p.value_heads, p.key_dim, p.value_dim), dtype=torch.float32, device=v.device)
        _lib.check_status(plan.lib.tjev_gdn_v2_fwd_cont(
            ctypes.byref(p), plan._stream(v.device), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(seg),
            _ptr(init_state), _ptr(out), _ptr(res), _ptr(final), _ptr(ws), ws.numel()))
        ctx.plan = plan
        ctx.save_for_backward(q, k, v, g, beta, seg, res, init_state)
        return out, final

    @staticmethod
    def backward(ctx, d_out, d_final):
        plan: GdnPlan = ctx.plan
        q, k, v, g, beta, seg, res, init_state = ctx.saved_tensors
        d_out = torch.zeros_like(v) if d_out is None else d_out.to(v.dtype).contiguous()
        d_final = None if d_final is None else d_final.to(torch.float32).contiguous()
        d_q, d_k, d_v = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        d_g, d_beta = torch.empty_like(g), torch.empty_like(beta)
        d_init = torch.empty_like(init_state) if init_state is not None and ctx.needs_input_grad[7] else None
        ws = plan.workspace(True, v.device)
        _lib.check_status(plan.lib.tjev_gdn_v2_bwd_cont(
            ctypes.byref(plan.params), plan._stream(v.device), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
            _ptr(seg), _ptr(init_state), _ptr(res), _ptr(d_out), _ptr(d_final), _ptr(d_q), _ptr(d_k), _ptr(d_v),
            _ptr(d_g), _ptr(d_beta), _ptr(d_init), _ptr(ws), ws.numel()))
        return None, d_q, d_k, d_v, d_g, d_beta, None, d_init, None


def chunk_gated_delta_rule_v2(q, k, v, g, beta, segment_ids=None, *, chunk: int = 64, precision: str = "high",
                              inverse: str = "doubling", heads_per_step: int = 0, vmem_fraction: float = 0.0,
                              residuals: str = "states", initial_state: torch.Tensor | None = None,
                              output_final_state: bool = False):
    """q, k [B,T,Hk,Dk] (Hk divides H), v [B,T,H,Dv], g, beta [B,T,H] -> out [B,T,H,Dv] in v's
    dtype (pallas_tpu_v2.py:541-582). T is padded to whole chunks with zero inputs and the last
    token's segment id. Head dims the kernels do not hold as they are (Dk != Dv, or not 16, 32,
    64 or 128; up to 128) run zero-padded to the next compiled dim (q and k are taken as given,
    so zero lanes change nothing), the outputs cut back; value heads wider than 128 (Dk <= 128)
    run as groups of value columns, each column of v, the state and the output being
    independent of the others.

    Beyond the reference's v2 kernel: ``initial_state`` [B, H, Dk, Dv] fp32 continues a sequence
    (xla.py:170-262's ``initial_state``: token 0's segment reads it), and ``output_final_state``
    returns (out, final_state [B, H, Dk, Dv] fp32), the state after token T-1; gradients flow
    through both, for any T."""
    if precision not in PRECISIONS:
        raise ValueError(f"precision in {PRECISIONS}")
    if inverse not in INVERSE_BLOCKS:
        raise ValueError(f"gdn_impl=pallas_tpu_v2 inverse in {tuple(INVERSE_BLOCKS)}")
    batch, length, kheads, dk = k.shape
    heads, dv = v.shape[2], v.shape[-1]
    if heads % kheads:
        raise ValueError(f"{heads} value heads are not groups of {kheads} key heads")
    if chunk & (chunk - 1):
        raise ValueError("gdn_impl=pallas_tpu_v2 needs a power-of-two chunk")
    if 3 * heads_per_block(heads, heads // kheads, heads_per_step or 8) > LANES:
        raise ValueError("at most 42 heads per step")
    if q.shape != k.shape or v.shape[:2] != q.shape[:2] or g.shape != (batch, length, heads) or g.shape != beta.shape:
        raise ValueError(f"shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}, g {tuple(g.shape)}, "
                         f"beta {tuple(beta.shape)} do not agree")
    if not v.is_cuda:
        raise RuntimeError("chunk_gated_delta_rule_v2 runs on the GPU (HIP); got a CPU tensor")
    groups = value_groups(dk, dv)
    if groups is not None:  # value heads wider than 128: groups of value columns (value_groups)
        if initial_state is not None and initial_state.shape != (batch, heads, dk, dv):
            raise ValueError(f"initial_state must be [{batch}, {heads}, {dk}, {dv}], not {tuple(initial_state.shape)}")
        res = [chunk_gated_delta_rule_v2(q, k, v[..., c:c + w], g, beta, segment_ids, chunk=chunk, precision=precision,
                                         inverse=inverse, heads_per_step=heads_per_step, residuals=residuals,
                                         initial_state=None if initial_state is None else initial_state[..., c:c + w],
                                         output_final_state=output_final_state)
               for c, w in groups]
        if not output_final_state:
            return torch.cat(res, dim=-1)
        return torch.cat([r[0] for r in res], dim=-1), torch.cat([r[1] for r in res], dim=-1)
    run = run_dim(dk, dv)
    if run is None:
        raise ValueError(f"key dims up to 128: this build's kernels cannot hold Dk={dk}, Dv={dv}")
    if run != dk or run != dv:
        if initial_state is not None and initial_state.shape != (batch, heads, dk, dv):
            raise ValueError(f"initial_state must be [{batch}, {heads}, {dk}, {dv}], not {tuple(initial_state.shape)}")
        padk = lambda x: torch.nn.functional.pad(x, (0, run - dk))  # noqa: E731
        init = None if initial_state is None else torch.nn.functional.pad(
            initial_state.to(torch.float32), (0, run - dv, 0, run - dk))
        res = chunk_gated_delta_rule_v2(padk(q), padk(k), torch.nn.functional.pad(v, (0, run - dv)), g, beta,
                                        segment_ids, chunk=chunk, precision=precision, inverse=inverse,
                                        heads_per_step=heads_per_step, residuals=residuals, initial_state=init,
                                        output_final_state=output_final_state)
        if not output_final_state:
            return res[..., :dv]
        return res[0][..., :dv], res[1][:, :, :dk, :dv]
    if segment_ids is None:
        segment_ids = torch.ones((batch, length), dtype=torch.int32, device=v.device)
    qk_dtype = q.dtype if q.dtype in _DTYPES else torch.float32
    plan = GdnPlan(batch=batch, length=length, key_heads=kheads, key_dim=dk, value_heads=heads, value_dim=dv, taps=0,
                   chunk=chunk, io_dtype=v.dtype, gate_dtype=g.dtype if g.dtype in _DTYPES else torch.float32,
                   precision=precision, inverse=inverse, heads_per_step=heads_per_step, residuals=residuals)
    plan.params.qk_dtype = _DTYPES[qk_dtype]
    gd = torch.bfloat16 if plan.params.gate_dtype == _lib.BF16 else torch.float32
    args = (q.to(qk_dtype).contiguous(), k.to(qk_dtype).contiguous(), v.contiguous(), g.to(gd).contiguous(),
            beta.to(gd).contiguous(), segment_ids.to(torch.int32).contiguous())
    if initial_state is None and not output_final_state:
        return _V2.apply(plan, *args)
    if initial_state is not None and initial_state.shape != (batch, heads, dk, dv):
        raise ValueError(f"initial_state must be [{batch}, {heads}, {dk}, {dv}], not {tuple(initial_state.shape)}")
    init = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    out, final = _V2Cont.apply(plan, *args, init, output_final_state)
    return (out, final) if output_final_state else out


def chunk_gated_delta_rule(q, k, v, g, beta, segment_ids=None, initial_state=None, chunk: int = 64,
                           precision: str = "highest", inverse: str = "solve"):
    """The reference's chunked rule with its state I/O (src/tjev/kernels/gated_delta_rule/
    xla.py:170-262): (out [B,T,H,Dv], final_state [B,H,Dk,Dv]) from q, k [B,T,H or Hk,Dk], v,
    g, beta and an optional initial_state, on the v2 operator's kernels. ``inverse`` (xla.py:190-195
    lists the same three): "doubling" the pure doubling from T = I at the products' precision,
    "blocked" exact 16 x 16 diagonal blocks then doubling levels, and "solve" (the reference's
    triangular solve) runs the blocked form, the kernels' closest to an exact solve. Unlike
    xla.py, v keeps its dtype in the output (fp32 inputs give fp32, as there)."""
    if inverse not in ("solve", "doubling", "blocked"):
        raise ValueError(f"precision in {PRECISIONS}, inverse in ('solve', 'doubling', 'blocked')")
    if precision not in PRECISIONS:
        raise ValueError(f"precision in {PRECISIONS}, inverse in ('solve', 'doubling', 'blocked')")
    return chunk_gated_delta_rule_v2(q, k, v, g, beta, segment_ids, chunk=chunk, precision=precision,
                                     inverse="blocked" if inverse == "solve" else inverse,
                                     initial_state=initial_state, output_final_state=True)
