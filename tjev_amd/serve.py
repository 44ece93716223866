"""Serving with the GDN megakernel on MI355X: a prefill that leaves the decode state, and the
decode step (one token per row), both inference-only (no autograd) through the HIP library.

The reference keeps state I/O in its XLA rules: ``chunk_gated_delta_rule`` and
``recurrent_gated_delta_rule`` take ``initial_state`` and return the final state
(src/tjev/kernels/gated_delta_rule/xla.py:141-262); its T=1 recurrence is the decode step.
Here the state is the megakernel's: the prefill returns the recurrent state after each row's
last token (fp32 [B, H, Dk, Dv]) and the conv history (the last K-1 raw rows [B, K-1, W] in
qkv's dtype, zero outside the last token's segment), and ``gdn_decode_step`` continues both
(HF ``causal_conv1d_update`` for the conv). A decode step continues the segment the state
belongs to; a new request starts from a fresh prefill.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .gdn import GdnPlan, _check, _ptr, merge_value_cols, pad_qkv, run_dim, unpad_qkv, value_cols, value_groups

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def gdn_prefill(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads: int, key_dim: int,
                value_heads: int, value_dim: int, chunk: int = 64, precision: str = "high",
                inverse: str = "doubling", heads_per_step: int = 0, initial_state=None, initial_conv=None):
    """The megakernel forward (``gdn_megakernel``'s arguments) and the decode state it leaves:
    (out [B, T, H, Dv], state [B, H, Dk, Dv] fp32, conv_state [B, K-1, W] or None). With
    ``initial_state`` / ``initial_conv`` (a previous prefill's state and conv_state) it
    continues that prefill: a long prompt in pieces."""
    batch, length, width = qkv.shape
    taps = _check(precision, inverse, chunk, width, key_heads, key_dim, value_heads, value_dim, heads_per_step,
                  conv_weight)
    if not qkv.is_cuda:
        raise RuntimeError("gdn_prefill runs on the GPU (HIP); got a CPU tensor")
    groups = value_groups(key_dim, value_dim)
    if groups is not None:  # value heads wider than 128: groups of value columns (gdn_megakernel's split)
        if initial_state is not None and initial_state.shape != (batch, value_heads, key_dim, value_dim):
            raise ValueError(f"initial_state must be [{batch}, {value_heads}, {key_dim}, {value_dim}], "
                             f"not {tuple(initial_state.shape)}")
        cut = lambda x, c, w: None if x is None else value_cols(  # noqa: E731
            x, key_heads, key_dim, value_heads, value_dim, c, w)
        res = [gdn_prefill(cut(qkv, c, w), a, b, a_log, dt_bias, cut(conv_weight, c, w), segment_ids,
                           key_heads=key_heads, key_dim=key_dim, value_heads=value_heads, value_dim=w, chunk=chunk,
                           precision=precision, inverse=inverse, heads_per_step=heads_per_step,
                           initial_state=None if initial_state is None else initial_state[..., c:c + w],
                           initial_conv=cut(initial_conv, c, w))
               for c, w in groups]
        conv_state = None if res[0][2] is None else merge_value_cols([r[2] for r in res], key_heads, key_dim,
                                                                       value_heads)
        return torch.cat([r[0] for r in res], dim=-1), torch.cat([r[1] for r in res], dim=-1), conv_state
    run = run_dim(key_dim, value_dim)
    if run is None:
        raise ValueError(f"key dims up to 128: this build's kernels cannot hold Dk={key_dim}, Dv={value_dim}")
    if run != key_dim or run != value_dim:  # zero-padded heads (gdn_megakernel's padded route)
        pad = lambda x: None if x is None else pad_qkv(x, key_heads, key_dim, value_heads, value_dim, run)  # noqa: E731
        init = None if initial_state is None else torch.nn.functional.pad(
            initial_state.to(torch.float32), (0, run - value_dim, 0, run - key_dim))
        out, state, conv_state = gdn_prefill(
            pad(qkv), a, b, a_log, dt_bias, pad(conv_weight), segment_ids, key_heads=key_heads, key_dim=run,
            value_heads=value_heads, value_dim=run, chunk=chunk, precision=precision, inverse=inverse,
            heads_per_step=heads_per_step, initial_state=init, initial_conv=pad(initial_conv))
        out = out[..., :value_dim] * math.sqrt(run / key_dim) if run != key_dim else out[..., :value_dim]
        if conv_state is not None:
            conv_state = unpad_qkv(conv_state, key_heads, key_dim, value_heads, value_dim, run)
        return out.contiguous(), state[:, :, :key_dim, :value_dim].contiguous(), conv_state
    plan = GdnPlan(batch=batch, length=length, key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                   value_dim=value_dim, taps=0 if conv_weight is None else taps, chunk=chunk, io_dtype=qkv.dtype,
                   gate_dtype=a.dtype, precision=precision, inverse=inverse, heads_per_step=heads_per_step)
    dev = qkv.device
    qkv, a, seg = qkv.contiguous(), a.contiguous(), segment_ids.to(torch.int32).contiguous()
    b = b.to(a.dtype).contiguous()
    a_log, dt_bias = a_log.to(torch.float32).contiguous(), dt_bias.to(torch.float32).contiguous()
    conv_w = None if conv_weight is None else conv_weight.to(torch.float32).contiguous()
    out = torch.empty((batch, length, value_heads, value_dim), dtype=qkv.dtype, device=dev)
    res = plan.residuals(dev)
    ws = plan.workspace(False, dev)
    state = torch.empty((batch, value_heads, key_dim, value_dim), dtype=torch.float32, device=dev)
    conv_state = None
    if conv_weight is not None and taps > 1:
        conv_state = torch.empty((batch, taps - 1, width), dtype=qkv.dtype, device=dev)
    init = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    hist = None if initial_conv is None or conv_state is None else initial_conv.to(qkv.dtype).contiguous()
    if init is not None and init.shape != state.shape:
        raise ValueError(f"initial_state must be {list(state.shape)}, not {list(init.shape)}")
    if hist is not None and hist.shape != conv_state.shape:
        raise ValueError(f"initial_conv must be {list(conv_state.shape)}, not {list(hist.shape)}")
    status = plan.lib.tjev_gdn_mega2_fwd_cont(
        ctypes.byref(plan.params), plan._stream(dev), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias),
        _ptr(conv_w), _ptr(seg), _ptr(init), _ptr(hist), _ptr(out), _ptr(res), _ptr(state), _ptr(conv_state),
        _ptr(ws), ws.numel())
    _lib.check_status(status)
    return out, state, conv_state


def gdn_decode_step(qkv, a, b, a_log, dt_bias, conv_weight, conv_state, state, *, key_heads: int, key_dim: int,
                    value_heads: int, value_dim: int, inplace: bool = False):
    """One token per row: qkv [B, W] (raw; post-conv for ``conv_weight`` None), a, b [B, H],
    conv_state [B, K-1, W], state [B, H, Dk, Dv] fp32. Returns (out [B, H, Dv],
    conv_state', state'); with ``inplace`` the state is updated in place (the conv history
    always goes to a new buffer)."""
    if qkv.dim() != 2:
        raise ValueError(f"qkv of one token per row is [B, W], not {tuple(qkv.shape)}")
    batch, width = qkv.shape
    taps = _check("high", "doubling", 64, width, key_heads, key_dim, value_heads, value_dim, 0, conv_weight)
    taps = 0 if conv_weight is None else taps
    if not qkv.is_cuda:
        raise RuntimeError("gdn_decode_step runs on the GPU (HIP); got a CPU tensor")
    if qkv.dtype not in _DTYPES or a.dtype not in _DTYPES:
        raise ValueError(f"the decode step takes float32 or bfloat16 tensors, not {qkv.dtype}/{a.dtype}")
    if state.shape != (batch, value_heads, key_dim, value_dim) or state.dtype != torch.float32:
        raise ValueError(f"state must be fp32 [{batch}, {value_heads}, {key_dim}, {value_dim}]")
    if taps > 1 and (conv_state is None or conv_state.shape != (batch, taps - 1, width)):
        raise ValueError(f"conv_state must be [{batch}, {taps - 1}, {width}]")
    groups = value_groups(key_dim, value_dim)
    if groups is not None:  # value heads wider than 128: groups of value columns (gdn_megakernel's split)
        cut = lambda x, c, w: None if x is None else value_cols(  # noqa: E731
            x, key_heads, key_dim, value_heads, value_dim, c, w)
        res = [gdn_decode_step(cut(qkv, c, w), a, b, a_log, dt_bias, cut(conv_weight, c, w), cut(conv_state, c, w),
                               state[..., c:c + w], key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                               value_dim=w)
               for c, w in groups]
        out = torch.cat([r[0] for r in res], dim=-1)
        hist_out = None if res[0][1] is None else merge_value_cols([r[1] for r in res], key_heads, key_dim,
                                                                     value_heads)
        st = torch.cat([r[2] for r in res], dim=-1)
        if inplace:
            state.copy_(st)
            st = state
        return out, hist_out, st
    run = run_dim(key_dim, value_dim)
    if run is None:
        raise ValueError(f"key dims up to 128: this build's kernels cannot hold Dk={key_dim}, Dv={value_dim}")
    if run != key_dim or run != value_dim:  # zero-padded heads (gdn_megakernel's padded route)
        pad = lambda x: None if x is None else pad_qkv(x, key_heads, key_dim, value_heads, value_dim, run)  # noqa: E731
        out, hist_out, st = gdn_decode_step(
            pad(qkv), a, b, a_log, dt_bias, pad(conv_weight), pad(conv_state),
            torch.nn.functional.pad(state, (0, run - value_dim, 0, run - key_dim)), key_heads=key_heads,
            key_dim=run, value_heads=value_heads, value_dim=run)
        out = out[..., :value_dim] * math.sqrt(run / key_dim) if run != key_dim else out[..., :value_dim]
        st = st[:, :, :key_dim, :value_dim]
        if inplace:
            state.copy_(st)
            st = state
        hist_out = None if hist_out is None else unpad_qkv(hist_out, key_heads, key_dim, value_heads, value_dim, run)
        return out.contiguous(), hist_out, st.contiguous() if not inplace else st
    lib = _lib.load()
    p = _lib.Params(batch, 1, key_heads, key_dim, value_heads, value_dim, taps, 64, _DTYPES[qkv.dtype],
                    _DTYPES[a.dtype], 1, 0, 0, 0)
    dev = qkv.device
    qkv, a = qkv.contiguous(), a.contiguous()
    b = b.to(a.dtype).contiguous()
    a_log, dt_bias = a_log.to(torch.float32).contiguous(), dt_bias.to(torch.float32).contiguous()
    conv_w = None if conv_weight is None else conv_weight.to(torch.float32).contiguous()
    hist = None if taps <= 1 else conv_state.to(qkv.dtype).contiguous()
    hist_out = None if taps <= 1 else torch.empty_like(hist)
    if inplace and (not state.is_contiguous() or state.data_ptr() % 16):
        raise ValueError("inplace: the state must be a contiguous, 16-byte aligned fp32 tensor (a copy would "
                         "leave the caller's cache unchanged)")
    state = state.contiguous()
    state_out = state if inplace else torch.empty_like(state)
    out = torch.empty((batch, value_heads, value_dim), dtype=qkv.dtype, device=dev)
    status = lib.tjev_gdn_decode_step(
        ctypes.byref(p), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream), _ptr(qkv), _ptr(a), _ptr(b),
        _ptr(a_log), _ptr(dt_bias), _ptr(conv_w), _ptr(hist), _ptr(state), _ptr(out), _ptr(hist_out),
        _ptr(state_out))
    _lib.check_status(status)
    return out, hist_out, state_out
