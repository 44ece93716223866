"""The library under HIP graph capture, and its determinism (GPU): the C ABI allocates nothing,
synchronizes nothing and launches only kernels on the caller's stream (no memset nodes), so a
caller can capture it; it uses no atomics, so runs repeat bit for bit.

- A training step (the megakernel's forward and its backward through torch autograd, bf16, the
  0.8B heads) captured once in a torch CUDA graph and replayed three times, with eager work of
  the program on other inputs and synchronizations between the replays: every replay's output
  and gradients equal the eager step's bit for bit.
- The allocation-free prefill (tjev_gdn_mega2_fwd_cont_noalloc, the entry point for callers that
  cannot allocate), captured and replayed the same way, with an eager call of the same entry
  point on another problem between the replays (it shares the static scratch array): every
  replay equals the eager call on the captured inputs bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from gdn_cases import case_inputs

pytestmark = pytest.mark.gpu

SHAPE = dict(key_heads=16, key_dim=128, value_heads=16, value_dim=128)


def _inputs(batch, length, seed):
    raw, cot = case_inputs(batch, length, 16, 16, 128, dtype=torch.bfloat16, style="baseline", segments="cuts",
                           cuts=[length // 3, length // 2 + 5], trailing_pad=7, seed=seed)
    return [x.cuda() for x in raw], cot.cuda()


def test_training_step_replays_in_a_graph():
    from tjev_amd import gdn_megakernel

    (qkv, a, b, a_log, dt_bias, w, seg), cot = _inputs(1, 512, seed=1)
    leaves = [x.clone().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias)]

    def step(xs, seg_, cot_):
        out = gdn_megakernel(*xs, w, seg_, chunk=128, precision="high", **SHAPE)
        return (out, *torch.autograd.grad((out.float() * cot_).sum(), xs))

    want = [x.detach().clone() for x in step(leaves, seg, cot)]
    other_xs, other_cot = _inputs(1, 512, seed=2)
    other = [x.clone().requires_grad_(True) for x in other_xs[:5]]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as torch's capture asks
        for _ in range(2):
            step(leaves, seg, cot)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step(leaves, seg, cot)
    for replay in range(3):
        print(f"training-step graph replay {replay}", flush=True)
        eager = step(other, other_xs[6], other_cot)  # the program's own work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("out", "qkv", "a", "b", "A_log", "dt_bias"), static, want):
            assert torch.equal(x, y), (replay, name, float((x.float() - y.float()).abs().max()))
        assert all(bool(torch.isfinite(t).all()) for t in eager)


def test_noalloc_prefill_replays_in_a_graph():
    from tjev_amd import _lib
    from tjev_amd.gdn import GdnPlan, _ptr

    lib = _lib.load()

    def buffers(plan, inputs):
        p = plan.params
        dev = inputs[0].device
        return (torch.full((p.batch, p.length, 16, 128), float("nan"), dtype=torch.bfloat16, device=dev),
                torch.full((plan.residual_bytes // 4,), float("nan"), device=dev),
                torch.full((p.batch, 16, 128, 128), float("nan"), device=dev),
                torch.full((p.batch, 3, inputs[0].shape[-1]), float("nan"), dtype=torch.bfloat16, device=dev))

    def call(plan, inputs, init, hist, outs):
        qkv, a, b, a_log, dt_bias, w, seg = inputs
        status = lib.tjev_gdn_mega2_fwd_cont_noalloc(
            ctypes.byref(plan.params), plan._stream(qkv.device), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log),
            _ptr(dt_bias), _ptr(w), _ptr(seg), _ptr(init), _ptr(hist), *(_ptr(x) for x in outs))
        assert status == 0, lib.tjev_gdn_last_error().decode()

    problems = []
    for batch, length, seed in ((2, 700, 3), (1, 300, 4)):
        inputs, _ = _inputs(batch, length, seed)
        inputs[6] = inputs[6].to(torch.int32)
        gen = torch.Generator().manual_seed(seed)
        init = (0.1 * torch.randn((batch, 16, 128, 128), generator=gen)).cuda()
        hist = torch.randn((batch, 3, inputs[0].shape[-1]), generator=gen).to(torch.bfloat16).cuda()
        plan = GdnPlan(batch=batch, length=length, taps=4, chunk=128, io_dtype=torch.bfloat16,
                       gate_dtype=torch.bfloat16, precision="high", **SHAPE)
        assert plan.fwd_bytes <= _lib.SCRATCH_BYTES
        problems.append((plan, inputs, init, hist))
    plan, inputs, init, hist = problems[0]
    want = buffers(plan, inputs)
    call(plan, inputs, init, hist, want)  # eager (also resolves the scratch array's address)
    torch.cuda.synchronize()
    n_states = plan.params.batch * 16 * plan.n_chunks * 128 * 128
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    static = buffers(plan, inputs)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(plan, inputs, init, hist, static)
    torch.cuda.synchronize()
    oplan, oinputs, oinit, ohist = problems[1]
    for replay in range(3):
        print(f"no-alloc prefill graph replay {replay}", flush=True)
        for x in static:
            x.fill_(float("nan"))
        call(oplan, oinputs, oinit, ohist, buffers(oplan, oinputs))  # eager, same scratch array
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("out", "residuals", "final_state", "conv_state"), static, want):
            if name == "residuals":
                x, y = x[:n_states], y[:n_states]
            assert torch.equal(x, y), (replay, name)


@pytest.mark.parametrize("hk,h", [(16, 16), (16, 32)], ids=["0.8B-heads", "9B-heads"])
def test_fwd_bwd_is_deterministic(hk, h):
    """No atomics and fixed-order reductions (the gate sums and the conv weight's gradient in
    fp64 over chunks in order): the same inputs give bit-identical outputs and gradients run
    after run, the conv weight's gradient included, with other work between the runs."""
    from tjev_amd import gdn_megakernel

    raw, cot = case_inputs(2, 1000, hk, h, 128, dtype=torch.bfloat16, style="baseline", segments="cuts",
                           cuts=[300, 301, 640], trailing_pad=3, seed=7)
    qkv, a, b, a_log, dt_bias, w, seg = (x.cuda() for x in raw)
    kw = dict(key_heads=hk, key_dim=128, value_heads=h, value_dim=128, chunk=128, precision="high")

    def run():
        xs = [x.clone().requires_grad_(True) for x in (qkv, a, b, a_log, dt_bias, w)]
        out = gdn_megakernel(*xs[:5], xs[5], seg, **kw)
        return [out.detach()] + list(torch.autograd.grad((out.float() * cot.cuda()).sum(), xs))

    first = run()
    for r in range(2):
        gdn_megakernel(qkv.flip(1), a, b, a_log, dt_bias, w, seg, **kw)  # other work in between
        again = run()
        for name, x, y in zip(("out", "qkv", "a", "b", "A_log", "dt_bias", "w"), again, first):
            assert torch.equal(x, y), (r, name)
