"""Algorithmic work of the GDN megakernel: FLOPs of the dense chunk contractions and minimal
HBM bytes, per kernel launch and for the whole operator, against MI355X's published peaks.

Per value head and chunk (C tokens, Dk = Dv = D), counting 2*m*n*k per product as in the
reference's cost model (pallas_tpu_v2.py:126-138):
  forward:  6 C^2 D + C^3/3 + 6 C D^2       (k k^T, the inverse, T [v beta | kbe], q k^T,
                                             intra v_new, [w; q_read] S, k_write^T v_new)
  backward: recompute k k^T, the inverse, kbe S_before and T (v beta - kbe S_before), then the
            products of the reverse chunk step (intra^T do, T^T(.), T^T k_write, Kt G, q_read^T do,
            kbe^T X, the m1 / m2 products and the state-gradient products).
Elementwise work (conv, gates, l2norm, exps) is not counted in FLOPs.
"""

from __future__ import annotations

# MI355X published peaks (dense): bf16 MFMA 2.5 PFLOP/s, fp32 MFMA 157.3 TFLOP/s, HBM 8 TB/s
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def fuses_v(*, io_bytes: int, chunk: int, dim: int, taps: int) -> bool:
    """Whether the forward's chunk kernel builds v from the raw rows (k_prep then skips them):
    bf16 I/O through a conv of 1 to 4 taps at chunk = head dim = 128, as the library's launch
    sequence decides."""
    return io_bytes == 2 and min(max(chunk, 16), 128) == 128 and dim == 128 and 1 <= taps <= 4


def fuses_q(*, io_bytes: int, chunk: int, dim: int, taps: int, key_heads: int, value_heads: int) -> bool:
    """Whether the forward's output kernel builds q from the raw rows (k_prep then skips them):
    where v is built from them (``fuses_v``) and each key head has one value head."""
    return fuses_v(io_bytes=io_bytes, chunk=chunk, dim=dim, taps=taps) and key_heads == value_heads


def kernel_work(*, batch: int, length: int, key_heads: int, value_heads: int, dim: int, chunk: int,
                io_bytes: int, residuals: str = "states", fused_norm: bool = False,
                fused_v: bool = False, fused_q: bool = False) -> dict[str, dict]:
    """Per-launch algorithmic work of each kernel: {"bytes": B, "flops": F}. Bytes are the
    minimal HBM traffic of the kernel's own inputs and outputs (each tensor read or written
    once); FLOPs count the dense chunk contractions once (zero for the elementwise kernels).
    ``residuals`` (states | tinv | all) sets what the forward's chunk kernel writes and what
    the backward's reads, as the library's residual policy does; ``fused_norm``: the output
    kernel also reads the norm's gate and writes its y; ``fused_v`` (``fuses_v``): the forward's
    chunk kernel reads v's raw rows (io dtype) instead of the fp32 v rows, which the forward's
    k_prep neither reads nor writes; ``fused_q`` (``fuses_q``): the same for q and the output
    kernel."""
    C, D = chunk, dim
    n = -(-length // C)
    tp = n * C
    units = batch * value_heads * n            # (row, value head, chunk) work items
    tok_h = batch * value_heads * tp           # token-heads
    tok_k = batch * key_heads * tp
    tokens = batch * length
    width = 2 * key_heads * D + value_heads * D
    sq = 2 * C * C * D                         # one C x C x D product
    sd = 2 * C * D * D                         # one C x D x D product
    inv = C ** 3 / 3
    f32 = 4
    act_k = tok_k * D * f32                    # q or k (key heads), fp32
    act_v = tok_h * D * f32                    # v, w, u, v_new, X, Kt, dq / dk per value head, fp32
    mats = units * D * D * f32                 # chunk-boundary states S or their gradients G
    tinv = units * C * (C - 1) // 2 * f32      # T per chunk: its strictly lower triangle (unit lower triangular)
    io = tok_h * D * io_bytes                  # out or d out
    ctx = batch * tp * 4 + 3 * tok_h * f32     # segment ids, gamma (hi, lo), beta
    prep = tokens * (width + 2 * value_heads) * io_bytes + (2 * tok_k + tok_h) * D * f32 + 3 * tok_h * f32
    raw_v = tokens * value_heads * D * io_bytes  # v's raw rows
    raw_q = tokens * key_heads * D * io_bytes    # q's raw rows
    prep_fwd = prep - (raw_v + tok_h * D * f32 if fused_v else 0) - (raw_q + act_k if fused_q else 0)
    v_in = raw_v if fused_v else act_v
    q_in = raw_q if fused_q else act_k
    w = {
        # conv + gates + l2norm: read qkv, a, b; write q, k (key heads), v, gamma (hi, lo), beta
        "gdn_prep_fwd": {"bytes": prep_fwd, "flops": 0},
        # k, v -> w, u (and T kept for the backward unless only the states are)
        "gdn_chunk_fwd": {"bytes": act_k + v_in + ctx + 2 * act_v + (tinv if residuals != "states" else 0),
                          "flops": units * (3 * sq + inv)},
        # w, u, k -> v_new, S before each chunk
        "gdn_scan_fwd": {"bytes": tok_h * D * f32 * 4 + units * D * D * f32, "flops": 0},
        # q, k, v_new, S -> out
        "gdn_out": {"bytes": q_in + act_k + act_v + mats + ctx + io * (3 if fused_norm else 1),
                    "flops": units * (2 * sq + sd)},
        "gdn_prep_bwd": {"bytes": prep, "flops": 0},
        # k, v, S (and T under tinv) -> v_new = T (v beta - kbe S) (and T under states)
        "gdn_chunk_bwd": {"bytes": act_k + 2 * act_v + mats + tinv + ctx,
                          "flops": units * ((2 * sq + inv + sd) if residuals == "states" else (sq + sd))},
        # q, k, d out, T -> X_loc, Kt
        "gdn_bwd_local": {"bytes": 2 * act_k + io + tinv + ctx + 2 * act_v, "flops": units * 4 * sq},
        "gdn_scan_bwd": {"bytes": tok_h * D * f32 * 5 + units * D * D * f32 * 2, "flops": 0},
        # q, k, X, v_new, S, G, d out -> dq, dk per value head, d gamma, d beta
        "gdn_bwd_grads": {"bytes": 2 * act_k + 4 * act_v + 2 * mats + io + ctx + 2 * tok_h * f32,
                          "flops": units * (6 * sq + 3 * sd)},
        # GQA sums, l2norm / SiLU / conv backward: read qkv, dq, dk, X, beta; write d_qkv, da, db
        "gdn_post": {"bytes": tokens * width * io_bytes * 2 + 3 * tok_h * D * f32
                     + 2 * tokens * value_heads * io_bytes, "flops": 0},
        "gdn_reduce": {"bytes": batch * n * value_heads * 16, "flops": 0},
        # gated RMSNorm: read x, z, write y; backward read x, z, dy, write dx, dz
        "gdn_norm_fwd": {"bytes": 3 * tokens * value_heads * D * io_bytes, "flops": 0},
        "gdn_norm_bwd": {"bytes": 5 * tokens * value_heads * D * io_bytes, "flops": 0},
        "gdn_norm_reduce": {"bytes": 2048 * D * f32, "flops": 0},
    }
    return w


def kernel_roofline(work: dict, seconds: float, peak_tflops: float) -> dict:
    """One launch of ``seconds`` against its roofline: the bound is the resource whose ideal
    time (algorithmic bytes at the HBM peak, algorithmic FLOPs at ``peak_tflops``) is longer,
    and ``achieved`` / ``frac`` are taken on that bound; ``mfma_frac`` / ``hbm_frac`` give
    both."""
    t_hbm = work["bytes"] / (PEAK_HBM_GBS * 1e9)
    t_mfma = work["flops"] / (peak_tflops * 1e12)
    gbs = work["bytes"] / seconds / 1e9
    tfs = work["flops"] / seconds / 1e12
    r = {"hbm_frac": gbs / PEAK_HBM_GBS, "mfma_frac": tfs / peak_tflops,
         "algorithmic_bytes": work["bytes"], "algorithmic_flops": work["flops"]}
    if t_mfma > t_hbm:
        r.update(bound="mfma", achieved=tfs, unit="TFLOP/s", peak=peak_tflops, frac=tfs / peak_tflops)
    else:
        r.update(bound="hbm", achieved=gbs, unit="GB/s", peak=PEAK_HBM_GBS, frac=gbs / PEAK_HBM_GBS)
    return r


def operator_work(*, batch: int, length: int, key_heads: int, value_heads: int, dim: int, chunk: int,
                  io_bytes: int, norm: bool = False) -> dict:
    """Whole fwd+bwd: algorithmic FLOPs (per token-head 18 C Dk + 14 C Dv + 2/3 C^2 + 20 Dk Dv)
    and minimal HBM bytes at the operator boundary (inputs, output, fp32 chunk states, the
    gradients), and the roofline time max(t_mfma, t_hbm) at the bf16 / HBM peaks. With the
    gated RMSNorm epilogue (``norm``) also its gate z and output y forward, and z, out and
    d z backward (out stays the saved residual; elementwise, no FLOPs counted)."""
    C, D = chunk, dim
    tokens = batch * length
    th = tokens * value_heads
    flops = th * (18 * C * D + 14 * C * D + (2 / 3) * C * C + 20 * D * D)
    width = 2 * key_heads * D + value_heads * D
    s = io_bytes
    state = value_heads * D * D * 4 / C
    fwd = tokens * (width * s + 2 * value_heads * s + value_heads * D * s + state)
    bwd = tokens * (2 * width * s + 2 * value_heads * s + state + value_heads * D * s + 2 * value_heads * 4)
    if norm:
        fwd += tokens * 2 * value_heads * D * s
        bwd += tokens * 3 * value_heads * D * s
    t_mfma = flops / (PEAK_BF16_TFLOPS * 1e12)
    t_hbm = (fwd + bwd) / (PEAK_HBM_GBS * 1e9)
    return {"flops": flops, "bytes": fwd + bwd, "t_mfma_s": t_mfma, "t_hbm_s": t_hbm,
            "ceiling_tokens_per_s": tokens / max(t_mfma, t_hbm)}
