#!/usr/bin/env python3
"""GDN megakernel fwd+bwd throughput on one MI355X (tjev's mega2: fwd+bwd tokens/s of the GDN layer).

A step is one forward and one backward pass of the GDN layer core over one batch of synthetic
inputs already resident in HBM (the HIP library called through its C ABI, no autograd): the
megakernel's out and chunk states, the gated RMSNorm y of out with gate z (in the megakernel's
output kernel, its backward in the same call as the megakernel's; ``--unfused-norm``: as their
own calls), then under a fixed upstream gradient of y
the norm's backward (d out, d z) and the megakernel's d(qkv), d(a), d(b), d(A_log),
d(dt_bias). ``--no-norm`` times the megakernel alone. W untimed warm-up steps, then K timed
steps between device synchronizations;
``value`` = B*T / (seconds per step). A second, event-profiled pass of K steps gives every
kernel's average duration (HIP events on the launch stream) for the dominant kernel's
roofline. The CPU baseline is the oracle (a CPU restatement of tjev's XLA chunked path, fp32,
torch autograd) on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 0.8B|9B|varlen|tiny|4B-block|decode|v2]

``--config 4B-block`` times the 4B block config instead: the 4B-shaped GDN block with merged
LoRA r64 (projections on hipBLASLt, core and norm in the HIP library), with peak activation
bytes; ``--config decode`` the serving path's one-token decode step (64 rows, 0.8B head shape);
``--config v2`` the v2 operator (pre-gated q, k, v, g, beta) fwd+bwd at the 0.8B layer shape.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

METRIC = "GDN layer fwd+bwd tokens/sec at 0.8B/9B shapes; MFMA util % and HBM GB/s"


def _args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="0.8B")
    ap.add_argument("--precision", default=None, help="override the config's precision")
    ap.add_argument("--no-norm", action="store_true", help="time the GDN core alone, without the gated RMSNorm")
    ap.add_argument("--unfused-norm", action="store_true",
                    help="the norm as its own forward and backward calls instead of in the megakernel's "
                         "(tjev_gdn_mega2_fwd_normed / _bwd_normed: the forward in the output kernel)")
    ap.add_argument("--residuals", default="states", choices=("states", "tinv", "all"),
                    help="what the forward keeps for the backward (default: the chunk-boundary states only)")
    ap.add_argument("--inverse", default="doubling", choices=("doubling", "blocked"),
                    help="the in-chunk inverse (the reference's default: pure doubling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=0, help="rows of the workload in the CPU baseline (0: all)")
    ap.add_argument("--details", default=None, help="also write the full report to this JSON file")
    ap.add_argument("--no-9b", action="store_true",
                    help="with the default 0.8B config, time it alone: skip the 9B, varlen and 4B-block configs "
                         "timed after it in the same run")
    return ap.parse_args(argv)


def _cpu_cores() -> tuple[int, int, str]:
    """(os.cpu_count(), the cores this process may run on, the lscpu model name)."""
    import subprocess

    total = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = total
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return total, usable, model


def _cpu_median(one_pass, reps: int = 3) -> tuple[float, list[float]]:
    """One warm-up pass, then the median of ``reps`` timed passes (the CPU baseline's timing rule)."""
    one_pass()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def _cpu_baseline(cfg, precision_dtype, rows: int, norm: bool) -> dict:
    """The oracle's fwd+bwd on the CPU over ``rows`` rows of the workload (all of them by
    default), with the gated RMSNorm epilogue when the GPU step has it, on every core the
    process may use: one warm-up pass, then the median of 3 passes (tokens/s)."""
    import torch

    from oracle.gdn_oracle import gated_rmsnorm, reference_core
    from tjev_amd.testing import cotangent, gdn_inputs

    total, usable, model = _cpu_cores()
    torch.set_num_threads(usable)
    threads = torch.get_num_threads()
    T, H, D = cfg["length"], cfg["value_heads"], cfg["dim"]
    inputs = gdn_inputs(batch=rows, length=T, key_heads=cfg["key_heads"], value_heads=H, dim=D,
                        dtype=precision_dtype, segments=cfg["segments"])
    cot = cotangent(rows, T, H, D).float()
    z = torch.randn((rows, T, H, D), generator=torch.Generator().manual_seed(11))
    norm_w = torch.ones(D)
    kw = dict(key_heads=cfg["key_heads"], key_dim=D, value_heads=H, value_dim=D, chunk=cfg["chunk"],
              dtype=torch.float32)

    def one_pass():
        qkv, a, b, a_log, dt_bias, w, seg = inputs
        leaves = [x.detach().float().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]
        out = reference_core(*leaves, w.detach().float(), seg, **kw)
        if norm:
            out = gated_rmsnorm(out, z, norm_w)
        torch.autograd.grad(torch.sum(out * cot), leaves)

    med, times = _cpu_median(one_pass)
    what = "GDN core + gated RMSNorm" if norm else "GDN core"
    return {"value": rows * T / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_count": total, "usable_cores": usable, "threads": threads, "cpu_model": model,
            "sample": (f"CPU restatement of tjev's XLA chunked path (the oracle, fp32, torch autograd) {what} "
                       f"fwd+bwd on B={rows} T={T} of the same workload (its heads, dims, chunk, segments): "
                       f"1 warm-up, median of 3 passes ({', '.join(f'{t:.2f}' for t in times)} s), "
                       f"{threads} threads on {model} (os.cpu_count() {total}, {usable} usable)")}


def _traffic(config: str, precision: str, kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed FETCH_SIZE / WRITE_SIZE summary of
    this workload (profiles/hbm_traffic_<config>_<precision>.json), or None without one."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"hbm_traffic_{config}_{precision}.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["bytes"]
    except (OSError, KeyError, ValueError):
        return None


BLOCK = dict(batch=2, length=8192, hidden=2560, key_heads=16, key_dim=128, value_heads=32, value_dim=128, rank=64,
             chunk=128, precision="high")


def _block_bench(args) -> dict:
    """The 4B block config: the 4B-shaped GDN block (src/tjev/model/gdn.py:126-164) fwd+bwd
    with merged LoRA r64 on every projection (tjev_amd/block.py), bf16, one segment per row.
    A step is the block's forward and the backward of sum(out * dy) to x and every adapter.
    Peak activation bytes: the step's allocator peak above what is resident before it
    (weights, adapters, inputs)."""
    import torch

    from oracle.gdn_oracle import gdn_block
    from tjev_amd import _lib
    from tjev_amd.block import GatedDeltaNetBlock

    c = BLOCK
    B, T, hid = c["batch"], c["length"], c["hidden"]
    blk = GatedDeltaNetBlock(hidden=hid, key_heads=c["key_heads"], key_dim=c["key_dim"],
                             value_heads=c["value_heads"], value_dim=c["value_dim"], rank=c["rank"],
                             dtype=torch.bfloat16, chunk=c["chunk"], precision=c["precision"],
                             inverse=args.inverse, residuals=args.residuals)
    gen = torch.Generator().manual_seed(21)
    x = torch.randn((B, T, hid), generator=gen).to(torch.bfloat16).cuda().requires_grad_(True)
    seg = torch.ones((B, T), dtype=torch.int32, device="cuda")
    dy = torch.randn((B, T, hid), generator=gen).to(torch.bfloat16).cuda()
    leaves = [x, *blk.parameters()]
    outs = {}

    def step():
        out = blk(x, seg)
        outs["grads"] = torch.autograd.grad(out, leaves, dy)
        outs["out"] = out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    resident = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - resident
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    with _lib.KernelTimer() as kt:
        for _ in range(args.steps):
            step()
    hip_ms = sum(kt.ms.values()) / args.steps
    finite = bool(torch.isfinite(outs["out"].float()).all()) and all(bool(torch.isfinite(g).all()) for g in outs["grads"])
    # projection GEMMs: forward x W' (4 in-projections + out_proj), backward dx and the adapter
    # products; the merge W + s A B per projection and call
    Hk, Dk, H, Dv, r = c["key_heads"], c["key_dim"], c["value_heads"], c["value_dim"], c["rank"]
    outs_in = [2 * Hk * Dk + H * Dv, H * Dv, H, H]
    n = B * T
    fwd = sum(2 * n * hid * o for o in outs_in) + 2 * n * H * Dv * hid
    bwd = fwd + sum(2 * n * hid * r + 2 * n * o * r * 2 + 2 * n * hid * r for o in outs_in) \
        + 2 * n * H * Dv * r + 2 * n * hid * r * 2 + 2 * n * H * Dv * r
    merge = sum(2 * hid * r * o for o in outs_in) + 2 * H * Dv * r * hid
    gemm_flops = fwd + bwd + merge
    gemm_ms = ms - hip_ms
    ach = gemm_flops / (gemm_ms * 1e-3) / 1e12
    report = {
        "metric": METRIC, "value": n / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "4B-shaped GDN block fwd+bwd (merged LoRA r64, flat gated RMSNorm)", "batch": B,
                   "seq_len": T, "hidden": hid, "key_heads": Hk, "value_heads": H, "head_dim": Dk, "lora_rank": r,
                   "chunk": c["chunk"], "precision": c["precision"], "segments": "one",
                   "inverse": args.inverse, "residuals": args.residuals},
        "peak_activation_bytes": peak,
        "roofline": {"kernel": "projections (hipBLASLt GEMMs, merge and glue: the step less the HIP library's kernels)",
                     "bound": "mfma", "achieved": ach, "peak": 2500.0, "unit": "TFLOP/s", "frac": ach / 2500.0,
                     "traffic": None},
        "split_ms": {"hip_kernels": hip_ms, "projections_and_glue": gemm_ms},
        "gemm_gflop": gemm_flops / 1e9,
        "finite": finite,
    }
    if not args.no_cpu_baseline:  # the oracle block on one row of 1024 tokens, fp32
        sample_t = 1024
        blk_cpu = {nm: (getattr(blk, nm).weight.float().cpu(), getattr(blk, nm).lora_a.detach().cpu(),
                        getattr(blk, nm).lora_b.detach().cpu(), getattr(blk, nm).scale)
                   for nm in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj")}
        blk_cpu.update(conv=blk.conv.cpu(), a_log=blk.a_log.cpu(), dt_bias=blk.dt_bias.cpu(), norm=blk.norm_weight.cpu())
        xc = x.detach()[:1, :sample_t].float().cpu()
        sc = seg[:1, :sample_t].cpu()
        dyc = dy[:1, :sample_t].float().cpu()

        def one_pass():
            xl = xc.clone().requires_grad_(True)
            ps = {k: ((v[0], v[1].clone().requires_grad_(True), v[2].clone().requires_grad_(True), v[3])
                      if isinstance(v, tuple) else v) for k, v in blk_cpu.items()}
            out = gdn_block(xl, sc, ps, key_heads=Hk, key_dim=Dk, value_heads=H, value_dim=Dv, chunk=c["chunk"])
            torch.autograd.grad((out * dyc).sum(), [xl] + [t for v in ps.values() if isinstance(v, tuple) for t in v[1:3]])

        total_cores, usable, model = _cpu_cores()
        torch.set_num_threads(usable)
        threads = torch.get_num_threads()
        med, times = _cpu_median(one_pass)
        report["cpu_baseline"] = {
            "value": sample_t / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_count": total_cores, "usable_cores": usable, "threads": threads, "cpu_model": model,
            "sample": (f"oracle gdn_block (CPU restatement of tjev's GatedDeltaNet with merged LoRA, fp32, torch "
                       f"autograd) fwd+bwd on B=1 T={sample_t} of the same block: 1 warm-up, median of 3 passes "
                       f"({', '.join(f'{t:.2f}' for t in times)} s), {threads} threads on {model}")}
    return report


def _decode_bench(args) -> dict:
    """One-token decode steps at the 0.8B layer shape (Hk = H = 16, D = 128, conv 4) for a
    batch of 64 rows, bf16 activations, fp32 state updated in place: the serving path's step
    (tjev_amd/serve.py). HBM-bound on the state: 2 x 64 KB per (row, head) per step."""
    import torch

    from tjev_amd import _lib
    from tjev_amd.serve import gdn_decode_step
    from tjev_amd.testing import gdn_inputs

    B, Hk, H, D = 64, 16, 16, 128
    qkv, a, b, a_log, dt_bias, w, _ = (x.cuda() for x in gdn_inputs(batch=B, length=4, key_heads=Hk, value_heads=H,
                                                                       dim=D, dtype=torch.bfloat16))
    state = (torch.randn((B, H, D, D), generator=torch.Generator().manual_seed(5)) * 0.05).cuda()
    hist = qkv[:, :3].contiguous()
    # the new token's rows as a serving loop receives them from the projections: contiguous
    # [B, W] and [B, H] tensors (strided slices would add a copy kernel each per step)
    x_t, a_t, b_t = qkv[:, 3].contiguous(), a[:, 3].contiguous(), b[:, 3].contiguous()
    kw = dict(key_heads=Hk, key_dim=D, value_heads=H, value_dim=D)

    def step():
        gdn_decode_step(x_t, a_t, b_t, a_log, dt_bias, w, hist, state, inplace=True, **kw)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    with _lib.KernelTimer() as kt:
        for _ in range(args.steps):
            step()
    k_ms = kt.ms["gdn_decode"] / kt.launches["gdn_decode"]
    state_bytes = 2 * B * H * D * D * 4
    ach = state_bytes / (k_ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "0.8B GDN layer core decode step (one token per row, state in place)", "batch": B,
                   "key_heads": Hk, "value_heads": H, "head_dim": D, "conv_taps": 4},
        "roofline": {"kernel": "gdn_decode", "bound": "hbm", "achieved": ach, "peak": 8000.0, "unit": "GB/s",
                     "frac": ach / 8000.0, "traffic": None},
        "kernel_ms": k_ms,
    }


def _v2_bench(args) -> dict:
    """The v2 operator (``chunk_gated_delta_rule_v2``, pallas_tpu_v2.py:541-582, the kernels behind
    ``gdn_impl=pallas_tpu_v2``) fwd+bwd at the 0.8B layer shape (B=4, T=4096, Hk=H=16, D=128,
    chunk 128, precision high, one segment per row): q and k l2-normalised with q scaled by
    Dk^-1/2 (as gdn.py:90-92 passes them), v ~ N(0, 1) in bf16; g = -exp(A_log) softplus(a +
    dt_bias) and beta = sigmoid(b) in fp32 from the benchmark's input distributions. A step is the forward
    and the backward of sum(out * dy) to q, k, v, g and beta. The chunk, scan and gradient kernels
    are the megakernel's (the roofline object is the dominant one's); the ends are v2's own."""
    import math

    import torch

    from tjev_amd import _lib
    from tjev_amd.roofline import PEAK_BF16_TFLOPS, kernel_roofline, kernel_work
    from tjev_amd.v2 import chunk_gated_delta_rule_v2

    B, T, Hk, H, D, C = 4, 4096, 16, 16, 128, 128
    gen = torch.Generator().manual_seed(13)

    def rn(*shape):
        return torch.randn(shape, generator=gen)

    q = torch.nn.functional.normalize(rn(B, T, Hk, D), dim=-1) * D ** -0.5
    k = torch.nn.functional.normalize(rn(B, T, Hk, D), dim=-1)
    a_log = torch.rand(H, generator=gen) * math.log(16.0)
    g = -torch.exp(a_log) * torch.nn.functional.softplus(rn(B, T, H) + rn(H))
    beta = torch.sigmoid(rn(B, T, H))
    leaves = [x.to(torch.bfloat16).cuda().requires_grad_(True) for x in (q, k, rn(B, T, H, D))]
    leaves += [x.cuda().requires_grad_(True) for x in (g, beta)]
    seg = torch.ones((B, T), dtype=torch.int32, device="cuda")
    dy = rn(B, T, H, D).to(torch.bfloat16).cuda()

    def step():
        out = chunk_gated_delta_rule_v2(*leaves, seg, chunk=C, precision="high", inverse=args.inverse,
                                        residuals=args.residuals)
        return torch.autograd.grad(out, leaves, dy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        grads = step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    finite = all(bool(torch.isfinite(x.float()).all()) for x in grads)
    with _lib.KernelTimer() as kt:
        for _ in range(args.steps):
            step()
    per_kernel = {n: kt.ms[n] / kt.launches[n] for n in kt.ms if kt.launches[n]}
    work = kernel_work(batch=B, length=T, key_heads=Hk, value_heads=H, dim=D, chunk=C, io_bytes=2,
                       residuals=args.residuals)
    ends = ("gdn_prep_fwd", "gdn_prep_bwd", "gdn_post")  # v2's own ends: their work differs from mega2's
    kernels = {n: ({"ms": t} if n in ends else {"ms": t, **kernel_roofline(work[n], t * 1e-3, PEAK_BF16_TFLOPS)})
               for n, t in per_kernel.items()}
    dominant = max((n for n in kernels if n not in ends), key=lambda n: kernels[n]["ms"])
    dk = kernels[dominant]
    return {
        "metric": METRIC, "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "0.8B GDN layer core, v2 operator (pre-gated q, k, v, g, beta) fwd+bwd", "batch": B,
                   "seq_len": T, "key_heads": Hk, "value_heads": H, "head_dim": D, "chunk": C, "precision": "high",
                   "segments": "one", "inverse": args.inverse, "residuals": args.residuals},
        "roofline": {"kernel": dominant, "bound": dk["bound"], "achieved": dk["achieved"], "peak": dk["peak"],
                     "unit": dk["unit"], "frac": dk["frac"], "traffic": None, "hbm_frac": dk["hbm_frac"],
                     "mfma_frac": dk["mfma_frac"]},
        "kernels": {n: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for n, v in kernels.items()},
        "finite": finite,
    }


def main(argv=None) -> int:
    args = _args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the operator would shard by batch rows, one process per GPU, with no exchange", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import torch

    if args.config in ("4B-block", "decode", "v2"):
        report = {"4B-block": _block_bench, "decode": _decode_bench, "v2": _v2_bench}[args.config](args)
        if args.details:
            with open(args.details, "w") as f:
                json.dump(report, f, indent=1)
        print(json.dumps(report), flush=True)
        return 0
    report = _layer_bench(args, args.config)
    if args.config == "0.8B" and not args.no_9b:
        # the metric names both layer shapes (campaign/bench.py:359-380 times (16,16) and (16,32)):
        # the 9B config in the same process, after the 0.8B buffers are released
        torch.cuda.empty_cache()
        nine = _layer_bench(args, "9B", cpu=False)
        report["config_9B"] = {
            "workload": nine["config"]["workload"], "value": nine["value"], "unit": "tokens/s",
            "ms_per_step": nine["ms_per_step"], "batch": nine["config"]["batch"], "seq_len": nine["config"]["seq_len"],
            "key_heads": nine["config"]["key_heads"], "value_heads": nine["config"]["value_heads"],
            "operator_roofline_frac": nine["operator_roofline"]["frac"],
            "operator_ceiling_tokens_per_s": nine["operator_roofline"]["ceiling_tokens_per_s"],
            "roofline": {k: nine["roofline"][k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac")},
            "kernels_ms": {k: v["ms"] for k, v in nine["kernels"].items()},
            "finite": nine["finite"], "wall_s_timed": nine["wall_s_timed"],
        }
        # the other BASELINE configs on one GPU: the packed varlen row and the 4B block
        del nine
        torch.cuda.empty_cache()
        var = _layer_bench(args, "varlen", cpu=False)
        report["config_varlen"] = {
            "workload": var["config"]["workload"], "value": var["value"], "unit": "tokens/s",
            "ms_per_step": var["ms_per_step"], "batch": var["config"]["batch"], "seq_len": var["config"]["seq_len"],
            "segments": var["config"]["segments"], "operator_roofline_frac": var["operator_roofline"]["frac"],
            "roofline": {k: var["roofline"][k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac")},
            "kernels_ms": {k: v["ms"] for k, v in var["kernels"].items()},
            "finite": var["finite"], "wall_s_timed": var["wall_s_timed"],
        }
        del var
        torch.cuda.empty_cache()
        blk = _block_bench(argparse.Namespace(**{**vars(args), "no_cpu_baseline": True}))
        report["config_4B_block"] = {
            "workload": blk["config"]["workload"], "value": blk["value"], "unit": "tokens/s",
            "ms_per_step": blk["ms_per_step"], "batch": blk["config"]["batch"], "seq_len": blk["config"]["seq_len"],
            "hidden": blk["config"]["hidden"], "lora_rank": blk["config"]["lora_rank"],
            "peak_activation_bytes": blk["peak_activation_bytes"], "split_ms": blk["split_ms"],
            "roofline": {k: blk["roofline"][k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac")},
            "finite": blk["finite"],
        }
    if args.details:
        with open(args.details, "w") as f:
            json.dump(report, f, indent=1)
    print(json.dumps(report), flush=True)
    return 0


def _layer_bench(args, config: str, cpu: bool = True) -> dict:
    """One layer config (0.8B, 9B, varlen, tiny): the report of its timed steps, per-kernel
    rooflines and (with ``cpu``) the CPU baseline."""
    import torch

    from tjev_amd import _lib
    from tjev_amd.gdn import GdnPlan
    from tjev_amd.norm import _params as _norm_params
    from tjev_amd.norm import norm_backward, norm_forward
    from tjev_amd.roofline import (PEAK_BF16_TFLOPS, PEAK_FP32_TFLOPS, fuses_q, fuses_v, kernel_roofline,
                                   kernel_work, operator_work)
    from tjev_amd.testing import CONFIGS, cotangent, gdn_inputs

    cfg = dict(CONFIGS[config])
    precision = args.precision or cfg["precision"]
    dtype = cfg["dtype"]
    dev = torch.device("cuda", 0)
    B, T, Hk, H, D, C = (cfg[k] for k in ("batch", "length", "key_heads", "value_heads", "dim", "chunk"))
    qkv, a, b, a_log, dt_bias, w, seg = gdn_inputs(batch=B, length=T, key_heads=Hk, value_heads=H, dim=D,
                                                  dtype=dtype, segments=cfg["segments"], device=dev)
    d_y = cotangent(B, T, H, D).to(dtype).to(dev)
    norm = not args.no_norm
    if norm:  # the output norm's gate z ~ N(0, 1) and weight (ones, as initialised)
        gen = torch.Generator().manual_seed(11)
        z = torch.randn((B, T, H, D), generator=gen).to(dtype).to(dev)
        norm_w = torch.ones(D, dtype=torch.float32, device=dev)
        norm_p = _norm_params(B * T, H, D, dtype, 1e-6)
        y = torch.empty((B, T, H, D), dtype=dtype, device=dev)
        d_out, d_z = torch.empty_like(y), torch.empty_like(y)
    else:
        d_out = d_y
    plan = GdnPlan(batch=B, length=T, key_heads=Hk, key_dim=D, value_heads=H, value_dim=D, taps=w.shape[0],
                   chunk=C, io_dtype=dtype, gate_dtype=dtype, precision=precision, inverse=args.inverse,
                   residuals=args.residuals)
    ws = torch.empty(max(plan.fwd_bytes, plan.bwd_bytes), dtype=torch.uint8, device=dev)
    out = torch.empty((B, T, H, D), dtype=dtype, device=dev)
    states = plan.residuals(dev)
    d_qkv, d_a, d_b = torch.empty_like(qkv), torch.empty_like(a), torch.empty_like(b)
    d_alog, d_dtb = torch.empty_like(a_log), torch.empty_like(dt_bias)

    fused = norm and not args.unfused_norm
    if fused:
        ws = torch.empty(max(plan.fwd_bytes, plan.normed_bwd_bytes(False)), dtype=torch.uint8, device=dev)

    def step():
        if fused:  # the norm's forward in the core's output kernel, its backward in the core's call
            plan.forward_normed(qkv, a, b, a_log, dt_bias, w, seg, z, norm_w, 1e-6, out, y, states, ws)
            plan.backward_normed(qkv, a, b, a_log, dt_bias, w, seg, states, out, z, norm_w, 1e-6, d_y, d_qkv, d_a,
                                 d_b, d_alog, d_dtb, None, d_z, None, ws)
            return
        plan.forward(qkv, a, b, a_log, dt_bias, w, seg, out, states, ws)
        if norm:
            norm_forward(norm_p, out, z, norm_w, seg, y)
            norm_backward(norm_p, out, z, norm_w, seg, d_y, d_out, d_z, None, None)
        plan.backward(qkv, a, b, a_log, dt_bias, w, seg, states, d_out, d_qkv, d_a, d_b, d_alog, d_dtb, None, ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    ms = start.elapsed_time(end) / args.steps
    finite = bool(torch.isfinite((y if norm else out).float()).all()) and bool(torch.isfinite(d_qkv.float()).all())

    with _lib.KernelTimer() as kt:  # the same steps again, each kernel between HIP events
        for _ in range(args.steps):
            step()
    per_kernel = {k: kt.ms[k] / kt.launches[k] for k in kt.ms if kt.launches[k]}
    io_bytes = 2 if dtype == torch.bfloat16 else 4
    shape = dict(batch=B, length=T, key_heads=Hk, value_heads=H, dim=D, chunk=C, io_bytes=io_bytes)
    taps = int(w.shape[0])
    work = kernel_work(**shape, residuals=args.residuals, fused_norm=fused,
                       fused_v=fuses_v(io_bytes=io_bytes, chunk=C, dim=D, taps=taps),
                       fused_q=fuses_q(io_bytes=io_bytes, chunk=C, dim=D, taps=taps, key_heads=Hk, value_heads=H))
    shape["norm"] = norm
    peak_mfma = PEAK_FP32_TFLOPS if precision == "highest" else PEAK_BF16_TFLOPS
    kernels = {name: {"ms": avg_ms, **kernel_roofline(work[name], avg_ms * 1e-3, peak_mfma)}
               for name, avg_ms in per_kernel.items()}
    dominant = max(kernels, key=lambda k: kernels[k]["ms"])
    dk = kernels[dominant]
    traffic = _traffic(config, precision, dominant)
    op = operator_work(**shape)
    value = B * T / (ms * 1e-3)
    report = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "f32",
        "data": "synthetic",
        "config": {"workload": f"{config} GDN layer core (mega2) fwd+bwd", "batch": B, "seq_len": T,
                   "key_heads": Hk, "value_heads": H, "head_dim": D, "chunk": C, "conv_taps": int(w.shape[0]),
                   "precision": precision, "segments": cfg["segments"],
                   "epilogue": ("gated_rmsnorm (forward in the output kernel)" if fused else "gated_rmsnorm")
                   if norm else None, "inverse": args.inverse, "residuals": args.residuals},
        "roofline": {"kernel": dominant, "bound": dk["bound"], "achieved": dk["achieved"], "peak": dk["peak"],
                     "unit": dk["unit"], "frac": dk["frac"], "traffic": traffic,
                     "hbm_frac": dk["hbm_frac"], "mfma_frac": dk["mfma_frac"]},
        "operator_roofline": {"algorithmic_gflop": op["flops"] / 1e9, "algorithmic_mb": op["bytes"] / 1e6,
                              "ceiling_tokens_per_s": op["ceiling_tokens_per_s"],
                              "frac": value / op["ceiling_tokens_per_s"],
                              "achieved_tflops": op["flops"] / (ms * 1e-3) / 1e12},
        "kernels": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "finite": finite,
        "wall_s_timed": t_wall,
    }
    if cpu and not args.no_cpu_baseline:
        report["cpu_baseline"] = _cpu_baseline(cfg, dtype, min(args.cpu_rows, B) if args.cpu_rows > 0 else B, norm)
    return report


if __name__ == "__main__":
    sys.exit(main())
