"""tjev's Gated DeltaNet block on MI355X: ``GatedDeltaNet.__call__`` (src/tjev/model/gdn.py:126-164)
with merged-LoRA projections (src/tjev/model/lora.py:191-223 ``grouped``, :262-369
``_merged_matmuls``) and the flat gated RMSNorm (src/tjev/model/norms.py:42-62).

    x (padding rows zeroed) -> in_proj_qkv, in_proj_z, in_proj_b, in_proj_a (one input; each
    adapter merged per call, W' = W + s*A*B rounded once to the compute dtype) -> the GDN
    megakernel core (HIP) with the gated RMSNorm of its output and the padding select in its
    output kernel -> out_proj (merged LoRA)

The projections are plain GEMMs on hipBLASLt (torch.mm). Their backward is the reference's
custom VJP (lora.py:320-366): dx = sum_i dy_i W'_i^T, dA_i = s_i x^T (dy_i B_i^T),
dB_i = s_i (x A_i)^T dy_i, with fp32 accumulation and results, never the full dW. The frozen
kernels, the conv weight, A_log, dt_bias and the norm weight take no gradient; the adapters
(fp32, cast to the compute dtype for the products) train. LoRA scale: rsLoRA, alpha/sqrt(rank)
(src/tjev/config/schema.py:44-45, 79-81).
"""

from __future__ import annotations

import math

import torch

from .gdn import gdn_megakernel_normed


def _mm32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b accumulated and returned in fp32 (the reference's preferred_element_type=f32).
    Transposed views are read in place (the GEMM's transpose flags), never copied."""
    if a.dtype == torch.float32:
        return a @ b.to(torch.float32)
    return torch.mm(a, b, out_dtype=torch.float32)


def _addmm32_(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """c += a @ b in place (c fp32), the product accumulated in fp32: one GEMM with c as its
    addend and output (an out-of-place addmm first copies c, 168 MB at the 4B block's dx)."""
    if a.dtype == torch.float32:
        return c.addmm_(a, b.to(torch.float32))
    if a.is_cuda:
        return torch.addmm(c, a, b, out_dtype=torch.float32, out=c)
    return c.add_(_mm32(a, b))


def _mm32_tn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T @ b in fp32 for token-major a [K, M] and b [K, N] (K the tokens; a may be a column
    slice). With K long against a small output (the adapters' gradients: 64 x 2560 .. 2560 x 256
    from K = 16384), one product leaves most CUs idle; the K range cut into 4 or 8 parts of at
    least 2048 runs as one batched product whose partials are then summed (measured at the 4B
    block's shapes: 2-3.6x faster; the fp32 sums differ by rounding only)."""
    k = a.shape[0]
    parts = next((p for p in (8, 4) if k % p == 0 and k // p >= 2048), 1)
    if parts == 1 or not a.is_cuda:
        return _mm32(a.t(), b)
    at = a.view(parts, k // parts, a.shape[1]).transpose(1, 2)  # [p, M, K/p], read transposed in place
    bt = b.contiguous().view(parts, k // parts, b.shape[1])     # the right operand contiguous
    return torch.bmm(at, bt, out_dtype=torch.float32).sum(0)


def _merge(w: torch.Tensor, a: torch.Tensor, b: torch.Tensor, s: float, dtype) -> torch.Tensor:
    """W' = (W + s A B) rounded once to ``dtype``, A and B rounded to it first and their product
    accumulated in fp32 (lora.py:284-295, ``_merge``): one GEMM whose epilogue adds W in fp32
    and rounds once (W in ``dtype`` is exact in fp32)."""
    w, a, b = w.to(dtype), a.to(dtype), b.to(dtype)
    if dtype == torch.float32 or w.is_cuda:
        return torch.addmm(w, a, b, alpha=s)
    return (w.to(torch.float32) + s * _mm32(a, b)).to(dtype)


class _MergedLoRA(torch.autograd.Function):
    """``_merged_matmuls`` (lora.py:303-369) for projections sharing the input x [N, in]:
    y_i = x W'_i, W'_i = (W_i + s_i A_i B_i) in the compute dtype, A_i and B_i rounded to it
    first and their product accumulated in fp32 (``_merge``, :284-295)."""

    @staticmethod
    def forward(ctx, x, scales, *params):
        n = len(scales)
        ws, a_s, b_s = params[:n], params[n:2 * n], params[2 * n:]
        dtype = x.dtype
        merged = [_merge(w, a, b, s, dtype) for w, a, b, s in zip(ws, a_s, b_s, scales)]
        ys = tuple(x @ m for m in merged)
        ctx.scales = scales
        ctx.save_for_backward(x, *merged, *a_s, *b_s)
        return ys

    @staticmethod
    def backward(ctx, *dys):
        scales = ctx.scales
        n = len(scales)
        x, *rest = ctx.saved_tensors
        merged, a_s, b_s = rest[:n], rest[n:2 * n], rest[2 * n:]
        dtype = x.dtype
        dys = [torch.zeros((x.shape[0], m.shape[1]), dtype=dtype, device=x.device) if dy is None
               else dy.to(dtype).contiguous() for dy, m in zip(dys, merged)]
        # dx = sum_i dy_i W'_i^T, each product and the sum in fp32, rounded once (lora.py:333-338);
        # W'^T read in place. The narrow projections (b, a) as one product over their joined
        # outputs (a small copy), the wide ones each added onto the running sum in place. One
        # projection alone: its product rounded once by the GEMM itself.
        if n == 1:
            dx = dys[0] @ merged[0].t()
        else:
            wide = [i for i in range(n) if merged[i].shape[1] >= 256]
            narrow = [i for i in range(n) if merged[i].shape[1] < 256]
            dx = None
            if narrow:
                dyn = dys[narrow[0]] if len(narrow) == 1 else torch.cat([dys[i] for i in narrow], dim=1)
                mn = merged[narrow[0]] if len(narrow) == 1 else torch.cat([merged[i] for i in narrow], dim=1)
                dx = _mm32(dyn, mn.t())
            for i in wide:
                dx = _mm32(dys[i], merged[i].t()) if dx is None else _addmm32_(dx, dys[i], merged[i].t())
            dx = dx.to(dtype)
        # the adapters: one pass over x for every A, x^T [s_1 t_1 | s_2 t_2 | ...]
        ranks = [a.shape[1] for a in a_s]
        a_cat = a_s[0].to(dtype) if n == 1 else torch.cat([a.to(dtype) for a in a_s], dim=1)
        xa = x @ a_cat
        ts = [torch.mul(_mm32(dy, b.to(dtype).t()), s, out=torch.empty((x.shape[0], b.shape[0]), dtype=dtype,
                                                                         device=x.device))
              for dy, b, s in zip(dys, b_s, scales)]  # s t_i, rounded once to dtype
        t = ts[0] if n == 1 else torch.cat(ts, dim=1)
        da = torch.split(_mm32_tn(x, t), ranks, dim=1)
        xas = torch.split(xa, ranks, dim=1)
        db = [s * _mm32_tn(xai, dy) for xai, dy, s in zip(xas, dys, scales)]
        return (dx, None, *([None] * n), *[d.to(a.dtype) for d, a in zip(da, a_s)],
                *[d.to(b.dtype) for d, b in zip(db, b_s)])


class LoRALinear:
    """A frozen projection W [in, out] (compute dtype) with a trainable adapter A [in, r],
    B [r, out] (fp32) and scale s (``Linear``, lora.py:69-188, merged form)."""

    def __init__(self, weight: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scale: float):
        self.weight = weight
        self.lora_a = lora_a
        self.lora_b = lora_b
        self.scale = float(scale)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        (y,) = grouped(x, self)
        return y


def grouped(x: torch.Tensor, *linears: LoRALinear) -> list[torch.Tensor]:
    """``[l(x) for l in linears]`` for projections sharing x (lora.py:191-223), merged."""
    dtype = linears[0].weight.dtype
    lead = x.shape[:-1]
    x2 = x.to(dtype).reshape(-1, x.shape[-1]).contiguous()
    ys = _MergedLoRA.apply(x2, tuple(l.scale for l in linears), *(l.weight for l in linears),
                           *(l.lora_a for l in linears), *(l.lora_b for l in linears))
    return [y.reshape(*lead, y.shape[-1]) for y in ys]


class GatedDeltaNetBlock:
    """The block with every projection adapted (rank ``rank``, merged) and the flat norm
    (``compute.gdn_norm=flat``, ``compute.lora_impl=merged``), random weights of the given
    shape (no checkpoint is loaded). ``init``: the adapters as the 4B block benchmark config draws
    them (A ~ N(0, 1/r), B ~ N(0, 0.01)), base kernels ~ N(0, 1/fan_in), conv ~ N(0, 0.5),
    A_log ~ U(0, ln 16), dt_bias ~ N(0, 1), norm weight 1."""

    def __init__(self, *, hidden: int, key_heads: int, key_dim: int, value_heads: int, value_dim: int,
                 taps: int = 4, rank: int = 64, alpha: float = 32.0, dtype=torch.bfloat16, device="cuda",
                 seed: int = 0, chunk: int = 64, precision: str = "high", inverse: str = "doubling",
                 residuals: str = "states", eps: float = 1e-6, b_std: float = 0.1):
        self.hidden, self.hk, self.dk, self.h, self.dv = hidden, key_heads, key_dim, value_heads, value_dim
        self.dtype, self.chunk, self.precision, self.inverse = dtype, chunk, precision, inverse
        self.residuals, self.eps = residuals, eps
        gen = torch.Generator().manual_seed(seed)

        def normal(*shape, std=1.0):
            return (torch.randn(shape, generator=gen) * std).to(device)

        scale = alpha / math.sqrt(rank)
        width = 2 * key_heads * key_dim + value_heads * value_dim

        def proj(fan_in, fan_out):
            w = normal(fan_in, fan_out, std=fan_in ** -0.5).to(dtype)
            a = normal(fan_in, rank, std=rank ** -0.5).requires_grad_(True)
            b = normal(rank, fan_out, std=b_std).requires_grad_(True)
            return LoRALinear(w, a, b, scale)

        self.in_proj_qkv = proj(hidden, width)
        self.in_proj_z = proj(hidden, value_heads * value_dim)
        self.in_proj_b = proj(hidden, value_heads)
        self.in_proj_a = proj(hidden, value_heads)
        self.out_proj = proj(value_heads * value_dim, hidden)
        self.conv = normal(taps, width, std=0.5)
        self.a_log = (torch.rand(value_heads, generator=gen) * math.log(16.0)).to(device)
        self.dt_bias = normal(value_heads)
        self.norm_weight = torch.ones(value_dim, device=device)

    def projections(self) -> list[LoRALinear]:
        return [self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a, self.out_proj]

    def parameters(self) -> list[torch.Tensor]:
        """The trainable adapters: (A, B) of every projection."""
        return [t for p in self.projections() for t in (p.lora_a, p.lora_b)]

    def __call__(self, x: torch.Tensor, segment_ids: torch.Tensor) -> torch.Tensor:
        """x [B, T, hidden] -> [B, T, hidden] (gdn.py:126-164, gdn_input_mask on)."""
        batch, length, _ = x.shape
        valid = (segment_ids > 0)[..., None]
        x = torch.where(valid, x, torch.zeros((), dtype=x.dtype, device=x.device)).to(self.dtype)
        qkv, z, b, a = grouped(x, self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a)
        # the core and its gated RMSNorm (gdn.py:157-160), the norm in the core's output kernel
        out = gdn_megakernel_normed(qkv, a, b, self.a_log, self.dt_bias, self.conv, segment_ids,
                                    z.reshape(batch, length, self.h, self.dv), self.norm_weight, self.eps,
                                    key_heads=self.hk, key_dim=self.dk, value_heads=self.h, value_dim=self.dv,
                                    chunk=self.chunk, precision=self.precision, inverse=self.inverse,
                                    residuals=self.residuals)
        return self.out_proj(out.reshape(batch, length, self.h * self.dv))
