"""The allocation-free prefill entry point (tjev_gdn_mega2_fwd_cont_noalloc, GPU): its workspace is
the library's static per-GPU scratch array. Two calls in a row, the second on a smaller problem
(so it runs over what the first left in the array), against tjev_gdn_mega2_fwd_cont with a
workspace of its own: out, the states residual, the final state and the conv history equal bit
for bit (the same kernels on the same inputs). A problem whose workspace exceeds the array is
refused before any launch (CPU: that check passes made-up device addresses)."""

import ctypes

import pytest
import torch

from gdn_cases import case_inputs


def _call(plan, fn, inputs, init, hist, workspace):
    from tjev_amd.gdn import _ptr

    qkv, a, b, a_log, dt_bias, w, seg = inputs
    p = plan.params
    dev = qkv.device
    out = torch.full((p.batch, p.length, p.value_heads, p.value_dim), float("nan"), dtype=qkv.dtype, device=dev)
    res = torch.full((plan.residual_bytes // 4,), float("nan"), device=dev)
    final = torch.full((p.batch, p.value_heads, p.key_dim, p.value_dim), float("nan"), device=dev)
    conv = torch.full((p.batch, p.taps - 1, qkv.shape[-1]), float("nan"), dtype=qkv.dtype, device=dev)
    args = [ctypes.byref(p), plan._stream(dev), _ptr(qkv), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias), _ptr(w),
            _ptr(seg), _ptr(init), _ptr(hist), _ptr(out), _ptr(res), _ptr(final), _ptr(conv)]
    if workspace is not None:
        args += [_ptr(workspace), workspace.numel()]
    status = fn(*args)
    return status, (out, res, final, conv)


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [((2, 1024), (1, 300))])
def test_noalloc_prefill_equals_the_workspace_entry_point(first, second):
    from tjev_amd import _lib
    from tjev_amd.gdn import GdnPlan

    lib = _lib.load()
    for call, (batch, length) in enumerate((first, second)):
        print(f"no-alloc prefill call {call}: B={batch} T={length}, 16/16 heads of 128, bf16, C=128", flush=True)
        raw, _ = case_inputs(batch, length, 16, 16, 128, dtype=torch.bfloat16, style="baseline", segments="cuts",
                             cuts=[length // 3, length // 2 + 5], trailing_pad=7, seed=call)
        inputs = [x.cuda() for x in raw]
        inputs[6] = inputs[6].to(torch.int32)
        gen = torch.Generator().manual_seed(10 + call)
        init = (0.1 * torch.randn((batch, 16, 128, 128), generator=gen)).cuda()
        hist = torch.randn((batch, 3, inputs[0].shape[-1]), generator=gen).to(torch.bfloat16).cuda()
        plan = GdnPlan(batch=batch, length=length, key_heads=16, key_dim=128, value_heads=16, value_dim=128, taps=4,
                       chunk=128, io_dtype=torch.bfloat16, gate_dtype=torch.bfloat16, precision="high")
        assert plan.fwd_bytes <= _lib.SCRATCH_BYTES
        ws = plan.workspace(False, inputs[0].device)
        s1, want = _call(plan, lib.tjev_gdn_mega2_fwd_cont, inputs, init, hist, ws)
        s2, got = _call(plan, lib.tjev_gdn_mega2_fwd_cont_noalloc, inputs, init, hist, None)
        torch.cuda.synchronize()
        assert s1 == 0 and s2 == 0, (s1, s2, lib.tjev_gdn_last_error().decode())
        states = slice(0, batch * 16 * plan.n_chunks * 128 * 128)
        for name, x, y in zip(("out", "residuals", "final_state", "conv_state"), got, want):
            if name == "residuals":
                x, y = x[states], y[states]
            assert bool(torch.isfinite(x).all()), name
            assert torch.equal(x, y), (call, name, float((x.float() - y.float()).abs().max()))


def test_noalloc_prefill_refuses_a_problem_beyond_the_scratch():
    """The size check comes before any launch; the buffers are made-up addresses, so the case
    runs only where no GPU is visible (a regressed check could otherwise launch on them)."""
    if torch.cuda.is_available():
        pytest.skip("host-side refusal with made-up device addresses: CPU only")
    from tjev_amd import _lib
    from tjev_amd.gdn import GdnPlan

    lib = _lib.load()
    plan = GdnPlan(batch=4, length=4096, key_heads=16, key_dim=128, value_heads=16, value_dim=128, taps=4, chunk=128,
                   io_dtype=torch.bfloat16, gate_dtype=torch.bfloat16, precision="high")
    assert plan.fwd_bytes > _lib.SCRATCH_BYTES
    vp = [ctypes.c_void_p(4096 * (i + 1)) for i in range(13)]
    status = lib.tjev_gdn_mega2_fwd_cont_noalloc(ctypes.byref(plan.params), None, *vp)
    assert status == 3 and "static scratch" in lib.tjev_gdn_last_error().decode()
