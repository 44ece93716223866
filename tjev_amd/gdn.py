"""The GDN megakernel operator on MI355X: tjev's ``gdn_megakernel`` signature and semantics,
computed by the HIP library through its C ABI.

Mirrors ``gdn_megakernel`` (src/tjev/kernels/gated_delta_rule/pallas_tpu_mega.py:585-639) and
its dispatcher form ``gdn_core_mega`` (src/tjev/kernels/gated_delta_rule/__init__.py:112-149):
same arguments, same ValueErrors before any launch, same segment-packing semantics, output
[B, T, H, Dv] in qkv's dtype. The custom VJP of ``_core`` (pallas_tpu_mega.py:538-575) is a
torch.autograd.Function whose residuals besides the inputs are, by ``residuals``: "states" (the
default) the fp32 state before each chunk alone (``gdn_states``), the backward recomputing every
intra-chunk quantity (T and v_new included); "tinv" the reference's pair
(pallas_tpu_mega.py:543-548), the states and each chunk's (I + L)^-1 (``gdn_tinv``), the
backward rebuilding v_new from T; "all" those and v_new, so that the backward rebuilds neither
(each of T and v_new costs 512 bytes per token and head in fp32 at C = Dv = 128). The conv
weight's gradient is computed only when the weight requires grad (the reference's
``gdn_mega2_bwd_dw`` variant, :549-551). There is no fallback: without the HIP library, or on a
CPU tensor, the operator raises.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

PRECISIONS = ("highest", "high", "bf16", "mixed")  # xla.py:23
INVERSE_BLOCKS = {"doubling": 0, "blocked": 16}    # pallas_tpu_v2.py:141
HALO = 8                                           # pallas_tpu_mega.py:71
LANES = 128                                        # pallas_tpu_mega.py:72


def heads_per_block(heads: int, ratio: int, preferred: int = 8) -> int:
    """Value heads per grid step of the reference kernels (pallas_tpu_v2.py:518-525): the
    largest multiple of the GQA ratio dividing H, up to ``preferred``. The HIP kernels run one
    value head per work item; this is kept for the reference's argument checks."""
    if heads % ratio:
        raise ValueError(f"{heads} value heads are not groups of {ratio}")
    sizes = range(ratio, max(preferred, ratio) + 1, ratio)
    return max(size for size in sizes if heads % size == 0)


def kernel_inverse(inverse: str) -> str:
    """``compute.gdn_inverse`` -> the in-kernel inverse (__init__.py:38-45)."""
    if inverse in ("default", "doubling"):
        return "doubling"
    if inverse == "blocked":
        return "blocked"
    raise ValueError(f"gdn_inverse={inverse} has no in-kernel form: default, doubling, blocked")


_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
RUN_DIMS = (16, 32, 64, 128)  # the head dims with compiled kernels (csrc/gdn_shapes.def), Dk = Dv
NORM_DIMS = (16, 32, 64, 128, 256)  # the gated RMSNorm's kernels


def run_dim(key_dim: int, value_dim: int) -> int | None:
    """The head dim the kernels run a (key_dim, value_dim) problem at: the two equal and compiled
    run as they are; otherwise both are zero-padded to the smallest compiled dim that holds the
    larger (None above 128). Zero q/k lanes change no dot product or l2 norm, and zero v lanes
    only add zero output and state columns, so the padded problem holds the original one."""
    if key_dim == value_dim and key_dim in RUN_DIMS:
        return key_dim
    return next((d for d in RUN_DIMS if d >= max(key_dim, value_dim)), None)


def pad_heads(x: torch.Tensor, heads: int, dim: int, run: int) -> torch.Tensor:
    """[..., heads * dim] -> [..., heads * run]: each head's lanes zero-padded at its end."""
    if dim == run:
        return x
    lead = x.shape[:-1]
    return torch.nn.functional.pad(x.reshape(*lead, heads, dim), (0, run - dim)).reshape(*lead, heads * run)


def pad_qkv(x: torch.Tensor, key_heads: int, key_dim: int, value_heads: int, value_dim: int, run: int):
    """The q | k | v lanes of x [..., 2 Hk Dk + H Dv] (qkv, the conv weight, conv history) with
    every head padded to ``run`` lanes."""
    q, k, v = torch.split(x, [key_heads * key_dim, key_heads * key_dim, value_heads * value_dim], dim=-1)
    return torch.cat([pad_heads(q, key_heads, key_dim, run), pad_heads(k, key_heads, key_dim, run),
                      pad_heads(v, value_heads, value_dim, run)], dim=-1)


def unpad_qkv(x: torch.Tensor, key_heads: int, key_dim: int, value_heads: int, value_dim: int, run: int):
    """The inverse of pad_qkv: each head's first lanes."""
    lead = x.shape[:-1]
    q, k, v = torch.split(x, [key_heads * run, key_heads * run, value_heads * run], dim=-1)

    def cut(t, heads, dim):
        return t.reshape(*lead, heads, run)[..., :dim].reshape(*lead, heads * dim)

    return torch.cat([cut(q, key_heads, key_dim), cut(k, key_heads, key_dim), cut(v, value_heads, value_dim)], dim=-1)


def value_groups(key_dim: int, value_dim: int) -> list[tuple[int, int]] | None:
    """Value heads wider than the kernels hold (Dv > 128, with Dk <= 128): the value columns cut
    into groups of at most 128, as (first column, width), each run as a problem of its own
    (which may in turn be padded, ``run_dim``). In the delta rule every value column of v, of the
    state and of the output evolves on its own (v_new = v - S^T k, S += beta k v_new^T and
    o = S^T q act column by column; q, k and the gates are shared), so the groups' outputs and
    states are the whole problem's columns and its gradients their sums. None when no split is
    needed, or when Dk itself exceeds 128 (no split holds that)."""
    top = RUN_DIMS[-1]
    if key_dim > top or value_dim <= top:
        return None
    return [(c, min(top, value_dim - c)) for c in range(0, value_dim, top)]


def value_cols(x: torch.Tensor, key_heads: int, key_dim: int, value_heads: int, value_dim: int, first: int,
               width: int) -> torch.Tensor:
    """x [..., 2 Hk Dk + H Dv] (qkv's lanes: qkv, the conv weight, the conv history) with each
    value head cut to its columns first .. first + width - 1; the q and k lanes as they are."""
    kq = 2 * key_heads * key_dim
    lead = x.shape[:-1]
    v = x[..., kq:].reshape(*lead, value_heads, value_dim)[..., first:first + width]
    return torch.cat([x[..., :kq], v.reshape(*lead, value_heads * width)], dim=-1)


def merge_value_cols(parts: list[torch.Tensor], key_heads: int, key_dim: int, value_heads: int) -> torch.Tensor:
    """The inverse of value_cols over a split's groups for a tensor whose q and k lanes are the
    same in every group (the conv history): those lanes from the first group, then each value
    head's columns from the groups in order."""
    kq = 2 * key_heads * key_dim
    lead = parts[0].shape[:-1]
    vs = [p[..., kq:].reshape(*lead, value_heads, -1) for p in parts]
    return torch.cat([parts[0][..., :kq], torch.cat(vs, dim=-1).reshape(*lead, -1)], dim=-1)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class GdnPlan:
    """The library's view of one problem shape: parameters, residual and workspace sizes,
    and raw forward / backward launches on the current stream (no autograd)."""

    def __init__(self, *, batch: int, length: int, key_heads: int, key_dim: int, value_heads: int,
                 value_dim: int, taps: int, chunk: int, io_dtype: torch.dtype,
                 gate_dtype: torch.dtype, precision: str = "high", inverse: str = "doubling",
                 heads_per_step: int = 0, residuals: str = "states"):
        self.lib = _lib.load()
        if io_dtype not in _DTYPES or gate_dtype not in _DTYPES:
            raise ValueError(f"the GDN megakernel takes float32 or bfloat16 tensors, not {io_dtype}/{gate_dtype}")
        if residuals not in _lib.RESIDUALS:
            raise ValueError(f"residuals in {tuple(_lib.RESIDUALS)}, not {residuals!r}")
        self.params = _lib.Params(batch, length, key_heads, key_dim, value_heads, value_dim, taps, chunk,
                                  _DTYPES[io_dtype], _DTYPES[gate_dtype], _lib.PRECISION[precision],
                                  _lib.INVERSE[inverse], heads_per_step, _lib.RESIDUALS[residuals])
        status = self.lib.tjev_gdn_check(ctypes.byref(self.params))
        if status == 1:
            raise ValueError(self.lib.tjev_gdn_last_error().decode())
        _lib.check_status(status)
        self.chunk_run = min(max(chunk, 16), 128)  # the kernels' chunk (tjev_gdn_params.chunk clamped)
        self.n_chunks = math.ceil(length / self.chunk_run)
        self.states_shape = (batch, value_heads, self.n_chunks, key_dim, value_dim)
        # the states' storage: bf16 when the state-path products are one bf16 pass, as the
        # reference's _state_dtypes (pallas_tpu_mega.py:425-426)
        self.states_dtype = torch.bfloat16 if precision in ("mixed", "bf16") else torch.float32
        self.tinv_dtype = torch.bfloat16 if precision == "bf16" else torch.float32  # the reference's t_dtype
        self.states_bytes = self.lib.tjev_gdn_states_bytes(ctypes.byref(self.params))
        self.residual_bytes = self.lib.tjev_gdn_residual_bytes(ctypes.byref(self.params))
        self.fwd_bytes = self.lib.tjev_gdn_workspace_bytes(ctypes.byref(self.params), 0)
        self.bwd_bytes = self.lib.tjev_gdn_workspace_bytes(ctypes.byref(self.params), 1)

    @staticmethod
    def _stream(device: torch.device) -> int:
        return torch.cuda.current_stream(device).cuda_stream

    def workspace(self, backward: bool, device) -> torch.Tensor:
        return torch.empty(self.bwd_bytes if backward else self.fwd_bytes, dtype=torch.uint8, device=device)

    def residuals(self, device) -> torch.Tensor:
        """The forward's residual buffer (4-byte words): the states first, then what ``residuals``
        keeps, each part 256-byte aligned."""
        return torch.empty(self.residual_bytes // 4, dtype=torch.float32, device=device)

    def states_of(self, residuals: torch.Tensor) -> torch.Tensor:
        """The states [B, H, N, Dk, Dv] part of a residual buffer (a view, ``states_dtype``)."""
        return residuals.view(torch.uint8)[: self.states_bytes].view(self.states_dtype).view(self.states_shape)

    def tinv_of(self, residuals: torch.Tensor) -> torch.Tensor:
        """The kept T [B, H, N, C, C] part of a residual buffer ("tinv" and "all"; ``tinv_dtype``)."""
        if self.params.residuals == _lib.RESIDUALS["states"]:
            raise ValueError("residuals='states' keeps no T")
        start = (self.states_bytes + 255) // 256 * 256
        b, h, n = self.states_shape[:3]
        size = b * h * n * self.chunk_run * self.chunk_run * self.tinv_dtype.itemsize
        return residuals.view(torch.uint8)[start:start + size].view(self.tinv_dtype).view(
            b, h, n, self.chunk_run, self.chunk_run)

    def forward(self, qkv, a, b, a_log, dt_bias, conv_w, seg, out, residuals, workspace) -> None:
        status = self.lib.tjev_gdn_mega2_fwd(
            ctypes.byref(self.params), self._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log),
            _ptr(dt_bias), _ptr(conv_w), _ptr(seg), _ptr(out), _ptr(residuals), _ptr(workspace),
            workspace.numel())
        _lib.check_status(status)

    def forward_normed(self, qkv, a, b, a_log, dt_bias, conv_w, seg, gate, norm_weight, eps: float, out, y,
                       residuals, workspace) -> None:
        """forward() with the gated RMSNorm of out into y in the output kernel
        (tjev_gdn_mega2_fwd_normed)."""
        status = self.lib.tjev_gdn_mega2_fwd_normed(
            ctypes.byref(self.params), self._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log),
            _ptr(dt_bias), _ptr(conv_w), _ptr(seg), None, None, _ptr(gate), _ptr(norm_weight),
            ctypes.c_float(eps), _ptr(out), _ptr(y), _ptr(residuals), None, None, _ptr(workspace),
            workspace.numel())
        _lib.check_status(status)

    def normed_bwd_bytes(self, norm_weight_grad: bool) -> int:
        return int(self.lib.tjev_gdn_workspace_bytes_normed(ctypes.byref(self.params), int(norm_weight_grad)))

    def backward_normed(self, qkv, a, b, a_log, dt_bias, conv_w, seg, residuals, out, gate, norm_weight,
                        eps: float, d_y, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_conv_w, d_gate, d_norm_weight,
                        workspace) -> None:
        """The backward of forward_normed: the norm's backward and the megakernel's in one call
        (tjev_gdn_mega2_bwd_normed)."""
        status = self.lib.tjev_gdn_mega2_bwd_normed(
            ctypes.byref(self.params), self._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log),
            _ptr(dt_bias), _ptr(conv_w), _ptr(seg), None, None, _ptr(residuals), _ptr(out), _ptr(gate),
            _ptr(norm_weight), ctypes.c_float(eps), _ptr(d_y), None, _ptr(d_qkv), _ptr(d_a), _ptr(d_b),
            _ptr(d_a_log), _ptr(d_dt_bias), _ptr(d_conv_w), None, None, _ptr(d_gate), _ptr(d_norm_weight),
            _ptr(workspace), workspace.numel())
        _lib.check_status(status)

    def backward(self, qkv, a, b, a_log, dt_bias, conv_w, seg, residuals, d_out, d_qkv, d_a, d_b, d_a_log,
                 d_dt_bias, d_conv_w, workspace) -> None:
        status = self.lib.tjev_gdn_mega2_bwd(
            ctypes.byref(self.params), self._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log),
            _ptr(dt_bias), _ptr(conv_w), _ptr(seg), _ptr(residuals), _ptr(d_out), _ptr(d_qkv), _ptr(d_a),
            _ptr(d_b), _ptr(d_a_log), _ptr(d_dt_bias), _ptr(d_conv_w), _ptr(workspace), workspace.numel())
        _lib.check_status(status)


class _Core(torch.autograd.Function):
    """The custom VJP of the reference's ``_core`` (pallas_tpu_mega.py:538-575)."""

    @staticmethod
    def forward(ctx, plan: GdnPlan, qkv, a, b, a_log, dt_bias, conv_w, seg, out_shape):
        out = torch.empty(out_shape, dtype=qkv.dtype, device=qkv.device)
        res = plan.residuals(qkv.device)
        ws = plan.workspace(False, qkv.device)
        plan.forward(qkv, a, b, a_log, dt_bias, conv_w, seg, out, res, ws)
        ctx.plan = plan
        ctx.save_for_backward(qkv, a, b, a_log, dt_bias, conv_w, seg, res)
        ctx.mark_non_differentiable(res)
        return out, res

    @staticmethod
    def backward(ctx, d_out, _d_res):
        plan: GdnPlan = ctx.plan
        qkv, a, b, a_log, dt_bias, conv_w, seg, res = ctx.saved_tensors
        if d_out is None:
            d_out = torch.zeros((qkv.shape[0], qkv.shape[1], plan.params.value_heads, plan.params.value_dim),
                                dtype=qkv.dtype, device=qkv.device)
        d_out = d_out.to(qkv.dtype).contiguous()
        d_qkv = torch.empty_like(qkv)
        d_a = torch.empty_like(a)
        d_b = torch.empty_like(b)
        d_a_log = torch.empty_like(a_log)
        d_dt_bias = torch.empty_like(dt_bias)
        want_dw = conv_w is not None and ctx.needs_input_grad[6]
        d_w = torch.empty_like(conv_w) if want_dw else None
        ws = plan.workspace(True, qkv.device)
        plan.backward(qkv, a, b, a_log, dt_bias, conv_w, seg, res, d_out, d_qkv, d_a, d_b, d_a_log, d_dt_bias,
                      d_w, ws)
        return None, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_w, None, None


class _CoreNormed(torch.autograd.Function):
    """``_Core`` followed by the gated RMSNorm of its output (GatedDeltaNet.__call__,
    model/gdn.py:157-160), the norm's forward in the output kernel; the backward is the norm's
    backward on the saved out, then the core's (one library call)."""

    @staticmethod
    def forward(ctx, plan: GdnPlan, qkv, a, b, a_log, dt_bias, conv_w, seg, gate, norm_weight, eps: float,
                out_shape):
        out = torch.empty(out_shape, dtype=qkv.dtype, device=qkv.device)
        y = torch.empty(out_shape, dtype=qkv.dtype, device=qkv.device)
        res = plan.residuals(qkv.device)
        ws = plan.workspace(False, qkv.device)
        plan.forward_normed(qkv, a, b, a_log, dt_bias, conv_w, seg, gate, norm_weight, eps, out, y, res, ws)
        ctx.plan = plan
        ctx.eps = eps
        ctx.save_for_backward(qkv, a, b, a_log, dt_bias, conv_w, seg, res, out, gate, norm_weight)
        return y

    @staticmethod
    def backward(ctx, d_y):
        plan: GdnPlan = ctx.plan
        qkv, a, b, a_log, dt_bias, conv_w, seg, res, out, gate, norm_weight = ctx.saved_tensors
        d_y = d_y.to(qkv.dtype).contiguous()
        d_gate = torch.empty_like(gate)
        want_nw = ctx.needs_input_grad[9]
        d_nw = torch.empty_like(norm_weight) if want_nw else None
        d_qkv = torch.empty_like(qkv)
        d_a = torch.empty_like(a)
        d_b = torch.empty_like(b)
        d_a_log = torch.empty_like(a_log)
        d_dt_bias = torch.empty_like(dt_bias)
        want_dw = conv_w is not None and ctx.needs_input_grad[6]
        d_w = torch.empty_like(conv_w) if want_dw else None
        ws = torch.empty(plan.normed_bwd_bytes(want_nw), dtype=torch.uint8, device=qkv.device)
        plan.backward_normed(qkv, a, b, a_log, dt_bias, conv_w, seg, res, out, gate, norm_weight, ctx.eps, d_y,
                             d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_w, d_gate, d_nw, ws)
        return None, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_w, None, d_gate, d_nw, None, None


def _conv_state_grad(d_cs, seg, d_qkv, d_init_conv, length: int):
    """Adds the gradient of the forward's conv_state (the raw rows T-K+1 .. T-1, zero outside
    token T-1's segment; rows before the row from the conv history) to those rows' gradients."""
    k1 = d_cs.shape[1]
    last = seg[:, length - 1]
    for r in range(k1):
        t = length - k1 + r
        if t >= 0:
            keep = (seg[:, t] == last)[:, None]
            d_qkv[:, t] += torch.where(keep, d_cs[:, r].to(d_qkv.dtype), torch.zeros((), dtype=d_qkv.dtype,
                                                                                     device=d_qkv.device))
        elif d_init_conv is not None:
            keep = (seg[:, 0] == last)[:, None]
            d_init_conv[:, k1 + t] += torch.where(keep, d_cs[:, r].to(d_init_conv.dtype),
                                                  torch.zeros((), dtype=d_init_conv.dtype, device=d_qkv.device))


class _CoreCont(torch.autograd.Function):
    """``_Core`` for a sequence continued from a given state: the initial recurrent state and
    conv history in, the final ones out, gradients through all four (tjev_gdn_mega2_fwd_cont /
    _bwd_cont)."""

    @staticmethod
    def forward(ctx, plan: GdnPlan, qkv, a, b, a_log, dt_bias, conv_w, seg, init_state, init_conv, out_shape,
                want_state):
        ctx.set_materialize_grads(False)
        dev = qkv.device
        p = plan.params
        out = torch.empty(out_shape, dtype=qkv.dtype, device=dev)
        res = plan.residuals(dev)
        ws = plan.workspace(False, dev)
        final = conv_state = None
        if want_state:
            final = torch.empty((p.batch, p.value_heads, p.key_dim, p.value_dim), dtype=torch.float32, device=dev)
            if p.taps > 1:
                conv_state = torch.empty((p.batch, p.taps - 1, qkv.shape[-1]), dtype=qkv.dtype, device=dev)
        _lib.check_status(plan.lib.tjev_gdn_mega2_fwd_cont(
            ctypes.byref(p), plan._stream(dev), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias),
            _ptr(conv_w), _ptr(seg), _ptr(init_state), _ptr(init_conv), _ptr(out), _ptr(res), _ptr(final),
            _ptr(conv_state), _ptr(ws), ws.numel()))
        ctx.plan = plan
        ctx.save_for_backward(qkv, a, b, a_log, dt_bias, conv_w, seg, res, init_state, init_conv)
        return out, final, conv_state

    @staticmethod
    def backward(ctx, d_out, d_final, d_cs):
        plan: GdnPlan = ctx.plan
        p = plan.params
        qkv, a, b, a_log, dt_bias, conv_w, seg, res, init_state, init_conv = ctx.saved_tensors
        if d_out is None:
            d_out = torch.zeros((qkv.shape[0], qkv.shape[1], p.value_heads, p.value_dim), dtype=qkv.dtype,
                                device=qkv.device)
        d_out = d_out.to(qkv.dtype).contiguous()
        d_final = None if d_final is None else d_final.to(torch.float32).contiguous()
        d_qkv, d_a, d_b = torch.empty_like(qkv), torch.empty_like(a), torch.empty_like(b)
        d_a_log, d_dt_bias = torch.empty_like(a_log), torch.empty_like(dt_bias)
        want_dw = conv_w is not None and ctx.needs_input_grad[6]
        d_w = torch.empty_like(conv_w) if want_dw else None
        d_init = torch.empty_like(init_state) if init_state is not None and ctx.needs_input_grad[8] else None
        want_hist = init_conv is not None and (ctx.needs_input_grad[9] or d_cs is not None)
        d_hist = torch.empty_like(init_conv) if want_hist else None
        ws = plan.workspace(True, qkv.device)
        _lib.check_status(plan.lib.tjev_gdn_mega2_bwd_cont(
            ctypes.byref(p), plan._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias),
            _ptr(conv_w), _ptr(seg), _ptr(init_state), _ptr(init_conv), _ptr(res), _ptr(d_out), _ptr(d_final),
            _ptr(d_qkv), _ptr(d_a), _ptr(d_b), _ptr(d_a_log), _ptr(d_dt_bias), _ptr(d_w), _ptr(d_init), _ptr(d_hist),
            _ptr(ws), ws.numel()))
        if d_cs is not None:
            _conv_state_grad(d_cs, seg, d_qkv, d_hist, qkv.shape[1])
        return (None, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_w, None, d_init,
                d_hist if init_conv is not None and ctx.needs_input_grad[9] else None, None, None)


def _check(precision, inverse, chunk, width, key_heads, key_dim, value_heads, value_dim, heads_per_step,
           conv_weight):
    """gdn_megakernel's checks, in its order and wording (pallas_tpu_mega.py:597-615)."""
    if precision not in PRECISIONS:
        raise ValueError(f"precision in {PRECISIONS}")
    if inverse not in INVERSE_BLOCKS:
        raise ValueError(f"the GDN megakernel's inverse in {tuple(INVERSE_BLOCKS)}")
    if chunk & (chunk - 1) or chunk < HALO:
        raise ValueError(f"the GDN megakernel needs a power-of-two chunk ≥ {HALO}, not {chunk}")
    if width != 2 * key_heads * key_dim + value_heads * value_dim:
        raise ValueError(f"qkv width {width} is not 2·{key_heads}·{key_dim} + {value_heads}·{value_dim}")
    ratio = value_heads // key_heads
    if ratio < 1 or value_heads % key_heads:
        raise ValueError(f"{value_heads} value heads are not groups of {key_heads} key heads")
    hb = heads_per_block(value_heads, ratio, heads_per_step or 8)
    if 3 * hb > LANES:
        raise ValueError(f"at most 42 heads per step, not {hb}")
    taps = 1 if conv_weight is None else conv_weight.shape[0]
    if not 1 <= taps <= 5:
        raise ValueError(f"conv kernel of {taps} taps: the megakernel supports 1..5")
    return taps


def gdn_megakernel(qkv: torch.Tensor, a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
                   dt_bias: torch.Tensor, conv_weight: torch.Tensor | None, segment_ids: torch.Tensor, *,
                   key_heads: int, key_dim: int, value_heads: int, value_dim: int, chunk: int = 64,
                   precision: str = "high", inverse: str = "doubling", heads_per_step: int = 0,
                   vmem_fraction: float = 0.0, residuals: str = "states", initial_state: torch.Tensor | None = None,
                   initial_conv: torch.Tensor | None = None, output_final_state: bool = False):
    """The GDN core from the projection outputs (pallas_tpu_mega.py:585-596).

    qkv [B, T, 2·Hk·Dk + H·Dv]: with ``conv_weight`` [K, 2·Hk·Dk + H·Dv] (mega2) the raw
    in_proj_qkv output, the conv + SiLU + padding mask in the kernel; with ``conv_weight``
    None (mega1) the post-conv, post-SiLU, masked activations. a, b [B, T, H] raw gate
    projections, a_log, dt_bias [H]; segment_ids [B, T] (0 = padding). Returns the delta
    rule's output [B, T, H, Dv] in qkv's dtype. ``vmem_fraction`` is TPU-only and ignored;
    ``heads_per_step`` is checked as the reference does and otherwise ignored. ``residuals``
    (this build's, not the reference's) picks what the forward keeps for the backward: "states"
    (chunk-boundary states only), "tinv" (the reference's gdn_states + gdn_tinv) or "all" (and
    v_new); every choice gives the same gradients up to rounding ("tinv" and "states" bit for
    bit).

    Beyond the reference's megakernel, which starts every row fresh: ``initial_state``
    [B, H, Dk, Dv] (fp32) and ``initial_conv`` [B, K-1, W] (qkv's dtype) continue a sequence
    from an earlier call (the chunked rule's ``initial_state``, xla.py:170-262: token 0's segment
    reads them), and ``output_final_state`` returns (out, final_state [B, H, Dk, Dv] fp32,
    conv_state [B, K-1, W] or None), the state after token T-1 and the last K-1 raw rows of its
    segment, which the next piece takes as its initial state and history. Gradients flow through
    all of them, for any T.

    Head dims: Dk = Dv in (16, 32, 64, 128) run as they are; other widths up to 128, Dk != Dv
    included, run zero-padded to the next of those (``run_dim``, ``_padded_megakernel``); value
    heads wider than 128 (with Dk <= 128) run as groups of value columns (``value_groups``,
    ``_split_megakernel``). Dk above 128 is refused."""
    batch, length, width = qkv.shape
    taps = _check(precision, inverse, chunk, width, key_heads, key_dim, value_heads, value_dim, heads_per_step,
                  conv_weight)
    if not qkv.is_cuda:
        raise RuntimeError("gdn_megakernel runs on the GPU (HIP); got a CPU tensor")
    groups = value_groups(key_dim, value_dim)
    if groups is not None:
        return _split_megakernel(groups, qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, key_heads=key_heads,
                                 key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, chunk=chunk,
                                 precision=precision, inverse=inverse, heads_per_step=heads_per_step,
                                 residuals=residuals, initial_state=initial_state, initial_conv=initial_conv,
                                 output_final_state=output_final_state)
    run = run_dim(key_dim, value_dim)
    if run is None:
        raise ValueError(f"key dims up to 128: this build's kernels cannot hold Dk={key_dim}, Dv={value_dim}")
    if run != key_dim or run != value_dim:
        return _padded_megakernel(run, qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, key_heads=key_heads,
                                  key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, chunk=chunk,
                                  precision=precision, inverse=inverse, heads_per_step=heads_per_step,
                                  residuals=residuals, initial_state=initial_state, initial_conv=initial_conv,
                                  output_final_state=output_final_state)
    plan = GdnPlan(batch=batch, length=length, key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                   value_dim=value_dim, taps=0 if conv_weight is None else taps, chunk=chunk,
                   io_dtype=qkv.dtype, gate_dtype=a.dtype, precision=precision, inverse=inverse,
                   heads_per_step=heads_per_step, residuals=residuals)
    b = b.to(a.dtype)
    conv_w = None if conv_weight is None else conv_weight.to(torch.float32).contiguous()
    args = (qkv.contiguous(), a.contiguous(), b.contiguous(), a_log.to(torch.float32).contiguous(),
            dt_bias.to(torch.float32).contiguous(), conv_w, segment_ids.to(torch.int32).contiguous())
    if initial_state is None and initial_conv is None and not output_final_state:
        out, _ = _Core.apply(plan, *args, (batch, length, value_heads, value_dim))
        return out
    if initial_state is not None and initial_state.shape != (batch, value_heads, key_dim, value_dim):
        raise ValueError(f"initial_state must be [{batch}, {value_heads}, {key_dim}, {value_dim}], "
                         f"not {tuple(initial_state.shape)}")
    if initial_conv is not None and (conv_weight is None or initial_conv.shape != (batch, taps - 1, width)):
        raise ValueError(f"initial_conv must be [{batch}, {taps - 1}, {width}] (a conv of 2 or more taps)")
    init = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    hist = None if initial_conv is None else initial_conv.to(qkv.dtype).contiguous()
    out, final, conv_state = _CoreCont.apply(plan, *args, init, hist, (batch, length, value_heads, value_dim),
                                             output_final_state)
    return (out, final, conv_state) if output_final_state else out


def gdn_megakernel_normed(qkv: torch.Tensor, a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
                          dt_bias: torch.Tensor, conv_weight: torch.Tensor | None, segment_ids: torch.Tensor,
                          gate: torch.Tensor, norm_weight: torch.Tensor, eps: float = 1e-6, *, key_heads: int,
                          key_dim: int, value_heads: int, value_dim: int, chunk: int = 64, precision: str = "high",
                          inverse: str = "doubling", heads_per_step: int = 0, residuals: str = "states"):
    """gdn_megakernel followed by the gated RMSNorm of its output, as GatedDeltaNet.__call__
    applies it (model/gdn.py:157-160, norms.py:36-62): gate [B, T, H, Dv] (the z projection,
    qkv's dtype), norm_weight [Dv]. Returns y [B, T, H, Dv] in qkv's dtype, the values of
    gated_rmsnorm(gdn_megakernel(...), gate, norm_weight, eps, segment_ids=segment_ids) up to the
    summation order of the norm's mean square (rare last-bit differences); the norm's forward
    runs in the megakernel's output kernel. Gradients flow to the megakernel's inputs, gate and
    norm_weight."""
    batch, length, width = qkv.shape
    taps = _check(precision, inverse, chunk, width, key_heads, key_dim, value_heads, value_dim, heads_per_step,
                  conv_weight)
    if not qkv.is_cuda:
        raise RuntimeError("gdn_megakernel_normed runs on the GPU (HIP); got a CPU tensor")
    shape = (batch, length, value_heads, value_dim)
    if tuple(gate.shape) != shape:
        raise ValueError(f"gate must be [{batch}, {length}, {value_heads}, {value_dim}], not {tuple(gate.shape)}")
    if tuple(norm_weight.shape) != (value_dim,):
        raise ValueError(f"norm_weight must be [{value_dim}], not {tuple(norm_weight.shape)}")
    if not (key_dim == value_dim and key_dim in RUN_DIMS):
        # padded or split head dims: the core (padded or by value columns), then the norm over
        # the Dv lanes on its own
        if value_dim > NORM_DIMS[-1]:
            raise ValueError(f"the gated RMSNorm's kernels hold Dv up to {NORM_DIMS[-1]}, not {value_dim}")
        out = gdn_megakernel(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, key_heads=key_heads,
                             key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, chunk=chunk,
                             precision=precision, inverse=inverse, heads_per_step=heads_per_step, residuals=residuals)
        return _norm_any_dim(out, gate, norm_weight, eps, segment_ids)
    plan = GdnPlan(batch=batch, length=length, key_heads=key_heads, key_dim=key_dim, value_heads=value_heads,
                   value_dim=value_dim, taps=0 if conv_weight is None else taps, chunk=chunk,
                   io_dtype=qkv.dtype, gate_dtype=a.dtype, precision=precision, inverse=inverse,
                   heads_per_step=heads_per_step, residuals=residuals)
    b = b.to(a.dtype)
    conv_w = None if conv_weight is None else conv_weight.to(torch.float32).contiguous()
    return _CoreNormed.apply(plan, qkv.contiguous(), a.contiguous(), b.contiguous(),
                             a_log.to(torch.float32).contiguous(), dt_bias.to(torch.float32).contiguous(), conv_w,
                             segment_ids.to(torch.int32).contiguous(), gate.to(qkv.dtype).contiguous(),
                             norm_weight.to(torch.float32).contiguous(), float(eps), shape)


def _padded_megakernel(run, qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads, key_dim,
                       value_heads, value_dim, initial_state, initial_conv, output_final_state, **kw):
    """gdn_megakernel on head dims the kernels do not hold as they are (Dk != Dv, or not a
    compiled dim): every q, k and v head zero-padded to ``run`` lanes (qkv, the conv weight and
    history, the initial state) around the kernels at Dk = Dv = run, the outputs cut back. The
    kernels scale q by run^-1/2; out is linear in q, so it is scaled by (run / Dk)^1/2 to the
    reference's Dk^-1/2. Gradients flow through the padding (torch's autograd)."""
    pad = lambda x: pad_qkv(x, key_heads, key_dim, value_heads, value_dim, run)  # noqa: E731
    init = None
    if initial_state is not None:
        if initial_state.shape != (qkv.shape[0], value_heads, key_dim, value_dim):
            raise ValueError(f"initial_state must be [{qkv.shape[0]}, {value_heads}, {key_dim}, {value_dim}], "
                             f"not {tuple(initial_state.shape)}")
        init = torch.nn.functional.pad(initial_state.to(torch.float32), (0, run - value_dim, 0, run - key_dim))
    if initial_conv is not None and (initial_conv.dim() != 3 or initial_conv.shape[-1] != qkv.shape[-1]):
        raise ValueError(f"initial_conv must be [B, K-1, {qkv.shape[-1]}], not {tuple(initial_conv.shape)}")
    res = gdn_megakernel(pad(qkv), a, b, a_log, dt_bias, None if conv_weight is None else pad(conv_weight),
                         segment_ids, key_heads=key_heads, key_dim=run, value_heads=value_heads, value_dim=run,
                         initial_state=init, initial_conv=None if initial_conv is None else pad(initial_conv),
                         output_final_state=output_final_state, **kw)
    out = res[0] if output_final_state else res
    out = out[..., :value_dim]
    if run != key_dim:
        out = out * math.sqrt(run / key_dim)
    if not output_final_state:
        return out
    _, final, conv_state = res
    final = final[:, :, :key_dim, :value_dim]
    if conv_state is not None:
        conv_state = unpad_qkv(conv_state, key_heads, key_dim, value_heads, value_dim, run)
    return out, final, conv_state


def _split_megakernel(groups, qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads, key_dim,
                      value_heads, value_dim, initial_state, initial_conv, output_final_state, **kw):
    """gdn_megakernel on value heads wider than the kernels hold: one call per group of value
    columns (``value_groups``), each on qkv with every value head cut to the group's columns
    (the conv weight and history alike, the initial state by its columns); outputs and final
    states are joined by columns, the conv history takes the q and k lanes from the first group.
    Gradients of the shared inputs (q and k lanes, gates, A_log, dt_bias, conv weight) sum over
    the groups through torch's autograd."""
    if initial_state is not None and initial_state.shape != (qkv.shape[0], value_heads, key_dim, value_dim):
        raise ValueError(f"initial_state must be [{qkv.shape[0]}, {value_heads}, {key_dim}, {value_dim}], "
                         f"not {tuple(initial_state.shape)}")
    if initial_conv is not None and (initial_conv.dim() != 3 or initial_conv.shape[-1] != qkv.shape[-1]):
        raise ValueError(f"initial_conv must be [B, K-1, {qkv.shape[-1]}], not {tuple(initial_conv.shape)}")
    cut = lambda x, c, w: None if x is None else value_cols(x, key_heads, key_dim, value_heads, value_dim, c, w)  # noqa: E731
    res = [gdn_megakernel(cut(qkv, c, w), a, b, a_log, dt_bias, cut(conv_weight, c, w), segment_ids,
                          key_heads=key_heads, key_dim=key_dim, value_heads=value_heads, value_dim=w,
                          initial_state=None if initial_state is None else initial_state[..., c:c + w],
                          initial_conv=cut(initial_conv, c, w), output_final_state=output_final_state, **kw)
           for c, w in groups]
    if not output_final_state:
        return torch.cat(res, dim=-1)
    out = torch.cat([r[0] for r in res], dim=-1)
    final = torch.cat([r[1] for r in res], dim=-1)
    conv_state = None if res[0][2] is None else merge_value_cols([r[2] for r in res], key_heads, key_dim, value_heads)
    return out, final, conv_state


def _norm_any_dim(out, gate, norm_weight, eps, segment_ids):
    """gated_rmsnorm(out, gate, norm_weight, eps, segment_ids) for any Dv: a dim without norm
    kernels runs zero-padded to the next one with eps and the weight rescaled so that the mean
    square over the padded lanes gives the Dv one: mean_P(x^2) + eps Dv/P = (Dv/P)(mean_Dv(x^2)
    + eps), whose rsqrt carries a factor (P/Dv)^1/2 that the weight takes back."""
    from .norm import gated_rmsnorm

    dv = out.shape[-1]
    if dv in NORM_DIMS:
        return gated_rmsnorm(out, gate, norm_weight, eps, segment_ids=segment_ids)
    pdim = next(d for d in NORM_DIMS if d >= dv)
    padding = (0, pdim - dv)
    w = torch.nn.functional.pad(norm_weight.to(torch.float32) * math.sqrt(dv / pdim), padding)
    y = gated_rmsnorm(torch.nn.functional.pad(out, padding), torch.nn.functional.pad(gate.to(out.dtype), padding),
                      w, eps * dv / pdim, segment_ids=segment_ids)
    return y[..., :dv]


def gdn_core_mega(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, *, key_heads: int, key_dim: int,
                  value_heads: int, value_dim: int, chunk: int = 64, precision: str = "high",
                  inverse: str = "default", heads_per_step: int = 0, vmem_fraction: float = 0.0,
                  residuals: str = "states", **state):
    """The dispatcher form (__init__.py:112-149): ``inverse`` "default" -> doubling. The
    reference shards rows over devices here (``batch_parallel_with``); this build runs one GPU,
    where that split is the identity."""
    return gdn_megakernel(qkv, a, b, a_log, dt_bias, conv_weight, segment_ids, key_heads=key_heads,
                          key_dim=key_dim, value_heads=value_heads, value_dim=value_dim, chunk=chunk,
                          precision=precision, inverse=kernel_inverse(inverse),
                          heads_per_step=heads_per_step, vmem_fraction=vmem_fraction, residuals=residuals, **state)
