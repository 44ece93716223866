"""The gated RMSNorm of the GDN output on MI355X, computed by the HIP library.

Mirrors tjev's ``GatedRMSNorm`` (src/tjev/model/norms.py:28-62; HF ``Qwen3_5RMSNormGated``):

    y = w * (x * rsqrt(mean_D(x^2) + eps)).astype(dtype).astype(f32) * silu(gate), cast to dtype

per head over the last axis of x, gate [..., H, D] (``__call__``) or, for ``flat``, the heads
side by side [..., H*D] (the same arithmetic on the same memory). ``segment_ids`` adds the
padding select that follows the norm in the reference block (src/tjev/model/gdn.py:163):
y = 0 on tokens whose segment id is <= 0. The backward is the reference's autodiff of those
casts (the cotangent of the intermediate rounding is itself rounded to dtype). The weight's
gradient is computed only when it requires grad (the reference's weight is frozen). There is
no fallback: without the HIP library, or on a CPU tensor, the operator raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _params(tokens: int, heads: int, dim: int, dtype: torch.dtype, eps: float) -> _lib.NormParams:
    if dtype not in _DTYPES:
        raise ValueError(f"the gated RMSNorm takes float32 or bfloat16 activations, not {dtype}")
    return _lib.NormParams(tokens=tokens, heads=heads, dim=dim, dtype=_DTYPES[dtype], eps=eps)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def norm_forward(p: _lib.NormParams, x, gate, weight, seg, y) -> None:
    """Raw launch on the current stream: y from x, gate (contiguous, [tokens, heads, dim])."""
    lib = _lib.load()
    _lib.check_status(lib.tjev_gdn_gated_rmsnorm_fwd(
        ctypes.byref(p), _stream(x.device), x.data_ptr(), gate.data_ptr(), weight.data_ptr(),
        None if seg is None else seg.data_ptr(), y.data_ptr()))


def norm_backward(p: _lib.NormParams, x, gate, weight, seg, d_y, d_x, d_gate, d_weight, workspace) -> None:
    """Raw launch on the current stream: d_x, d_gate (and d_weight when given)."""
    lib = _lib.load()
    _lib.check_status(lib.tjev_gdn_gated_rmsnorm_bwd(
        ctypes.byref(p), _stream(x.device), x.data_ptr(), gate.data_ptr(), weight.data_ptr(),
        None if seg is None else seg.data_ptr(), d_y.data_ptr(), d_x.data_ptr(), d_gate.data_ptr(),
        None if d_weight is None else d_weight.data_ptr(),
        None if workspace is None else workspace.data_ptr(), 0 if workspace is None else workspace.numel()))


def workspace_bytes(p: _lib.NormParams, weight_grad: bool) -> int:
    return int(_lib.load().tjev_gdn_norm_workspace_bytes(ctypes.byref(p), int(weight_grad)))


class _GatedRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate, weight, seg, heads: int, dim: int, eps: float):
        tokens = x.numel() // (heads * dim)
        p = _params(tokens, heads, dim, x.dtype, eps)
        y = torch.empty_like(x)
        norm_forward(p, x, gate, weight, seg, y)
        ctx.p = p
        ctx.save_for_backward(x, gate, weight, seg)
        return y

    @staticmethod
    def backward(ctx, d_y):
        x, gate, weight, seg = ctx.saved_tensors
        p = ctx.p
        d_y = d_y.to(x.dtype).contiguous()
        d_x, d_gate = torch.empty_like(x), torch.empty_like(gate)
        want_dw = ctx.needs_input_grad[2]
        d_w = torch.empty_like(weight) if want_dw else None
        ws = None
        if want_dw:
            ws = torch.empty(workspace_bytes(p, True), dtype=torch.uint8, device=x.device)
        norm_backward(p, x, gate, weight, seg, d_y, d_x, d_gate, d_w, ws)
        return d_x, d_gate, d_w, None, None, None, None


def gated_rmsnorm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, *,
                  heads: int | None = None, segment_ids: torch.Tensor | None = None) -> torch.Tensor:
    """The norm over the last axis of x, gate [..., H, D] (``heads`` None), or over each of the
    ``heads`` groups of D lanes of x, gate [..., H*D]. ``weight`` [D]. ``segment_ids`` [B, T]
    (x [B, T, ...]) zeroes padding tokens. Returns y in x's dtype."""
    if x.shape != gate.shape:
        raise ValueError(f"x {tuple(x.shape)} and gate {tuple(gate.shape)} differ")
    if heads is None:
        heads, dim = (x.shape[-2], x.shape[-1]) if x.dim() >= 2 else (1, x.shape[-1])
    else:
        if x.shape[-1] % heads:
            raise ValueError(f"{x.shape[-1]} lanes are not {heads} heads")
        dim = x.shape[-1] // heads
    if weight.shape != (dim,):
        raise ValueError(f"weight {tuple(weight.shape)} is not [{dim}]")
    if not x.is_cuda:
        raise RuntimeError("gated_rmsnorm runs on the GPU (HIP); got a CPU tensor")
    seg = None
    if segment_ids is not None:
        seg = segment_ids.to(torch.int32).contiguous()
        if seg.numel() * heads * dim != x.numel():
            raise ValueError(f"segment_ids {tuple(segment_ids.shape)} do not index the tokens of x")
    return _GatedRMSNorm.apply(x.contiguous(), gate.to(x.dtype).contiguous(), weight.to(torch.float32).contiguous(),
                               seg, heads, dim, float(eps))


class GatedRMSNorm:
    """tjev's ``GatedRMSNorm`` (norms.py:28-62): ``norm(x, gate)`` on [..., H, D] and
    ``norm.flat(x, gate, heads)`` on [..., H*D]."""

    def __init__(self, weight: torch.Tensor, eps: float):
        self.weight = weight
        self.eps = eps

    def __call__(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return gated_rmsnorm(x, gate, self.weight, self.eps)

    def flat(self, x: torch.Tensor, gate: torch.Tensor, heads: int) -> torch.Tensor:
        return gated_rmsnorm(x, gate, self.weight, self.eps, heads=heads)
