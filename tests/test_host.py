"""Host-side checks of the drop-in boundary (CPU only, no kernel launches): the library loads and
exports every entry point its header declares; argument validation follows the reference's
ValueError conventions (pallas_tpu_mega.py:597-615) before anything is launched; the operator
never falls back to a CPU path."""

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "tjev_gdn.h").read_text()
    return sorted(set(re.findall(r"\b(tjev_gdn_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from tjev_amd import _lib

    lib = _lib.load()
    declared = _declared()
    assert set(declared) == set(_lib.EXPORTS), (declared, _lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.tjev_gdn_version() >> 16 == 0
    assert lib.tjev_gdn_lds_poison() == 0
    assert lib.tjev_gdn_kernel_name(0) == b"gdn_prep_fwd"
    text = (ROOT / "include" / "tjev_gdn.h").read_text()
    m = re.search(r"#define TJEV_GDN_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.SCRATCH_BYTES


def test_lds_poison_library_exports_the_same_symbols():
    """The LDS-poison debug build: the same ABI, and it says what it is."""
    from tjev_amd import _lib

    lib = _lib.open_library(_lib.LDS_POISON_PATH)
    for name in _lib.EXPORTS:
        assert hasattr(lib, name), name
    assert lib.tjev_gdn_lds_poison() == 1


def _params(**kw):
    from tjev_amd import _lib

    base = dict(batch=1, length=100, key_heads=2, key_dim=16, value_heads=4, value_dim=16, taps=4, chunk=16,
                io_dtype=0, gate_dtype=0, precision=1, inverse=0, heads_per_step=0)
    base.update(kw)
    return _lib.Params(**base)


@pytest.mark.parametrize("bad,status,msg", [
    (dict(precision=7), 1, "precision"),
    (dict(inverse=2), 1, "inverse"),
    (dict(chunk=96), 1, "power-of-two chunk"),
    (dict(chunk=4), 1, "power-of-two chunk"),
    (dict(value_heads=5), 1, "groups of"),
    (dict(taps=6), 1, "taps"),
    (dict(key_dim=48, value_dim=48), 2, "no kernels"),
    (dict(value_dim=32), 2, "key_dim == value_dim"),
    (dict(residuals=3), 1, "residuals"),
    # B*T*W = 2^27 * 48 passes the size bound, but the flat prep grid would hold 2^23 * 3
    # workgroups of 256 work-items: more than one launch takes
    (dict(length=1 << 27, key_heads=1, value_heads=1), 2, "too large for one launch"),
])
def test_c_abi_validation(bad, status, msg):
    from tjev_amd import _lib

    lib = _lib.load()
    p = _params(**bad)
    assert lib.tjev_gdn_check(ctypes.byref(p)) == status
    assert msg in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_workspace_bytes(ctypes.byref(p), 0) == 0


def test_c_abi_sizes():
    from tjev_amd import _lib

    lib = _lib.load()
    p = _params(batch=4, length=4096, key_heads=16, key_dim=128, value_heads=16, value_dim=128, chunk=128, io_dtype=1,
                gate_dtype=1)
    assert lib.tjev_gdn_check(ctypes.byref(p)) == 0
    assert lib.tjev_gdn_states_bytes(ctypes.byref(p)) == 4 * 16 * 32 * 128 * 128 * 4
    fwd, bwd = (lib.tjev_gdn_workspace_bytes(ctypes.byref(p), k) for k in (0, 1))
    assert 0 < fwd < bwd < (2 << 30)
    # the residuals: states, then T (B*H*N*C*C fp32) and v_new (B*H*N*C*Dv fp32) as kept; what
    # is kept leaves the workspaces
    part = 4 * 16 * 32 * 128 * 128 * 4
    assert lib.tjev_gdn_residual_bytes(ctypes.byref(p)) == part
    for mode, total in ((1, 2 * part), (2, 3 * part)):
        p.residuals = mode
        assert lib.tjev_gdn_residual_bytes(ctypes.byref(p)) == total
        assert lib.tjev_gdn_states_bytes(ctypes.byref(p)) == part
    assert lib.tjev_gdn_workspace_bytes(ctypes.byref(p), 0) == fwd - part
    assert lib.tjev_gdn_workspace_bytes(ctypes.byref(p), 1) == bwd - 2 * part
    # "mixed" and "bf16" keep the states in bf16 (the reference's _state_dtypes) and the forward
    # workspace an fp32 copy of each row's state before its last chunk (the final state's source)
    for precision in (2, 3):
        q = _params(batch=4, length=4096, key_heads=16, key_dim=128, value_heads=16, value_dim=128, chunk=128,
                    io_dtype=1, gate_dtype=1, precision=precision)
        assert lib.tjev_gdn_states_bytes(ctypes.byref(q)) == part // 2
        assert lib.tjev_gdn_residual_bytes(ctypes.byref(q)) == part // 2
        assert lib.tjev_gdn_workspace_bytes(ctypes.byref(q), 0) == fwd + 4 * 16 * 128 * 128 * 4
        # under "bf16" T between the backward's first two kernels is bf16 too (the reference's t_dtype)
        t_part = 4 * 16 * 32 * 128 * 128 * 2
        assert lib.tjev_gdn_workspace_bytes(ctypes.byref(q), 1) == bwd - (t_part if precision == 2 else 0)
        q.residuals = 1  # T after the bf16 states (256-byte aligned): bf16 under "bf16" only
        assert lib.tjev_gdn_residual_bytes(ctypes.byref(q)) == part // 2 + (part // 2 if precision == 2 else part)
    # a forward that builds v (bf16 I/O, 1 to 4 taps, chunk and head dim 128) and, with one value
    # head per key head, q from the raw rows has no fp32 rows of them in its workspace; the
    # backward's are unchanged
    rows = 4 * 16 * 4096 * 128 * 4
    for hv in (16, 32):
        f32, b16 = (_params(batch=4, length=4096, key_heads=16, key_dim=128, value_heads=hv, value_dim=128, chunk=128,
                            io_dtype=io, gate_dtype=io) for io in (0, 1))
        gap = lib.tjev_gdn_workspace_bytes(ctypes.byref(f32), 0) - lib.tjev_gdn_workspace_bytes(ctypes.byref(b16), 0)
        assert gap == 2 * rows, (hv, gap)  # 16 value heads: q and v rows; 32 (GQA): v rows of 32 heads
        assert lib.tjev_gdn_workspace_bytes(ctypes.byref(f32), 1) == lib.tjev_gdn_workspace_bytes(ctypes.byref(b16), 1)
    for kw in (dict(taps=5), dict(taps=0), dict(chunk=64), dict(key_dim=64, value_dim=64)):
        f32, b16 = (_params(batch=4, length=4096, key_heads=16, key_dim=128, value_heads=16, value_dim=128, chunk=128,
                            io_dtype=io, gate_dtype=io) for io in (0, 1))
        for x in (f32, b16):
            for k, v in kw.items():
                setattr(x, k, v)
        assert lib.tjev_gdn_workspace_bytes(ctypes.byref(f32), 0) == lib.tjev_gdn_workspace_bytes(ctypes.byref(b16), 0), kw
    # a ragged T is padded to whole chunks (the last segment's id carried over, as the reference pads)
    p = _params(length=100, chunk=16)
    assert lib.tjev_gdn_states_bytes(ctypes.byref(p)) == 1 * 4 * 7 * 16 * 16 * 4


def test_null_pointers_are_rejected_before_launch():
    from tjev_amd import _lib

    lib = _lib.load()
    p = _params()
    status = lib.tjev_gdn_mega2_fwd(ctypes.byref(p), None, *([None] * 10), 0)
    assert status == 1 and "null" in lib.tjev_gdn_last_error().decode()


def _args(**kw):
    base = dict(key_heads=2, key_dim=16, value_heads=4, value_dim=16, chunk=16)
    base.update(kw)
    return base


@pytest.mark.parametrize("kw,match", [
    (dict(precision="fp8"), "precision in"),
    (dict(inverse="solve"), "inverse in"),
    (dict(chunk=24), "power-of-two chunk"),
    (dict(chunk=4), "power-of-two chunk"),
    (dict(key_heads=3), "qkv width"),
])
def test_operator_raises_value_errors_like_the_reference(kw, match):
    from tjev_amd import gdn_megakernel

    qkv = torch.zeros((1, 64, 2 * 2 * 16 + 4 * 16))
    g = torch.zeros((1, 64, 4))
    h = torch.zeros(4)
    w = torch.zeros((4, qkv.shape[-1]))
    seg = torch.ones((1, 64), dtype=torch.int32)
    with pytest.raises(ValueError, match=match):
        gdn_megakernel(qkv, g, g, h, h, w, seg, **_args(**kw))


def test_operator_rejects_taps_and_head_groups():
    from tjev_amd import gdn_megakernel

    qkv = torch.zeros((1, 64, 2 * 2 * 16 + 4 * 16))
    g = torch.zeros((1, 64, 4))
    h = torch.zeros(4)
    seg = torch.ones((1, 64), dtype=torch.int32)
    with pytest.raises(ValueError, match="taps"):
        gdn_megakernel(qkv, g, g, h, h, torch.zeros((6, qkv.shape[-1])), seg, **_args())
    with pytest.raises(ValueError, match="42 heads"):
        big = torch.zeros((1, 64, 2 * 1 * 16 + 48 * 16))
        gdn_megakernel(big, torch.zeros((1, 64, 48)), torch.zeros((1, 64, 48)), torch.zeros(48), torch.zeros(48),
                       None, seg, key_heads=1, key_dim=16, value_heads=48, value_dim=16, chunk=16, heads_per_step=48)


def test_operator_has_no_cpu_fallback():
    from tjev_amd import gdn_megakernel

    qkv = torch.zeros((1, 64, 2 * 2 * 16 + 4 * 16))
    g = torch.zeros((1, 64, 4))
    h = torch.zeros(4)
    with pytest.raises(RuntimeError, match="GPU"):
        gdn_megakernel(qkv, g, g, h, h, None, torch.ones((1, 64), dtype=torch.int32), **_args())


def test_kernel_inverse_and_heads_per_block():
    from tjev_amd import heads_per_block, kernel_inverse

    assert [kernel_inverse(x) for x in ("default", "doubling", "blocked")] == ["doubling", "doubling", "blocked"]
    with pytest.raises(ValueError):
        kernel_inverse("solve")
    assert [heads_per_block(h, r) for h, r in ((16, 1), (32, 2), (4, 2), (3, 1), (48, 3))] == [8, 8, 4, 3, 6]


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert proc.returncode == 2 and "one GPU" in proc.stderr


def test_varlen_segments_follow_the_config():
    import numpy as np

    from tjev_amd.testing import geometric_segments

    ids = geometric_segments(16384, np.random.default_rng(0))
    assert ids.shape == (16384,) and ids[0] == 1 and np.all(np.diff(ids) >= 0)
    lengths = np.bincount(ids)[1:]
    assert np.all(lengths[:-1] >= 16) and np.all(lengths <= 4096)
    assert 30 <= len(lengths) <= 90  # mean 300 over 16384 tokens


def _norm_params(**kw):
    from tjev_amd import _lib

    base = dict(tokens=10, heads=2, dim=128, dtype=1, eps=1e-6)
    base.update(kw)
    return _lib.NormParams(**base)


@pytest.mark.parametrize("bad,status,msg", [
    (dict(dim=48), 2, "dim 16, 32, 64, 128 and 256"),
    (dict(dtype=3), 1, "dtype"),
    (dict(heads=0), 1, "heads"),
    (dict(tokens=-1), 1, "tokens"),
    (dict(eps=-1.0), 1, "eps"),
])
def test_norm_c_abi_validation(bad, status, msg):
    from tjev_amd import _lib

    lib = _lib.load()
    p = _norm_params(**bad)
    got = lib.tjev_gdn_gated_rmsnorm_fwd(ctypes.byref(p), None, *([None] * 5))
    assert got == status and msg in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_norm_workspace_bytes(ctypes.byref(p), 1) == 0


def test_norm_c_abi_nulls_and_workspace():
    from tjev_amd import _lib

    lib = _lib.load()
    p = _norm_params(tokens=4 * 4096, heads=16, dim=128)
    assert lib.tjev_gdn_gated_rmsnorm_fwd(ctypes.byref(p), None, *([None] * 5)) == 1
    assert "null" in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_norm_workspace_bytes(ctypes.byref(p), 0) == 0
    # one fp32 partial row of D per backward workgroup, at most 2048 of them
    assert lib.tjev_gdn_norm_workspace_bytes(ctypes.byref(p), 1) == 2048 * 128 * 4
    small = _norm_params(tokens=3, heads=2, dim=16)  # 6 rows fit one workgroup
    assert lib.tjev_gdn_norm_workspace_bytes(ctypes.byref(small), 1) == 16 * 4


def test_norm_operator_checks_and_no_cpu_fallback():
    from tjev_amd.norm import gated_rmsnorm

    x = torch.zeros(2, 3, 4, 16)
    with pytest.raises(ValueError, match="differ"):
        gated_rmsnorm(x, torch.zeros(2, 3, 4, 8), torch.ones(16))
    with pytest.raises(ValueError, match="weight"):
        gated_rmsnorm(x, x, torch.ones(8))
    with pytest.raises(ValueError, match="heads"):
        gated_rmsnorm(x.reshape(2, 3, 64), x.reshape(2, 3, 64), torch.ones(16), heads=5)
    with pytest.raises(RuntimeError, match="GPU"):
        gated_rmsnorm(x, x, torch.ones(16))


def _mir(before, after):
    head = "# *** IR Dump {} SI Load Store Optimizer (si-load-store-opt) ***:\n# Machine code for function k: x\nname: k\n"
    return head.format("Before") + before + head.format("After") + after


def test_ds_check_flags_the_miscompiled_merge_only():
    from tjev_amd.ds_check import bad_merges

    before = ("DS_WRITE_B32_gfx9 %5:vgpr_32, %7:vgpr_32, 272, 0, implicit $exec :: (store (s32) into %ir.p1, addrspace 3)\n"
              "DS_WRITE_B32_gfx9 %5:vgpr_32, %8:vgpr_32, 336, 0, implicit $exec :: (store (s32) into %ir.p2, addrspace 3)\n")
    # the miscompile seen with ROCm 7.2: 272 and 336 bytes merged as dword offsets 17 and 84
    wrong = ("DS_WRITE2_B32_gfx9 %5:vgpr_32, %7:vgpr_32, %8:vgpr_32, 17, 84, 0, implicit $exec :: "
             "(store (s32) into %ir.p1, addrspace 3), (store (s32) into %ir.p2, addrspace 3)\n")
    right = wrong.replace(" 17, 84,", " 68, 84,")
    assert len(bad_merges(_mir(before, wrong))) == 1
    assert bad_merges(_mir(before, right)) == []
    # accesses off two base registers carry no offsets to compare
    other = before.replace("DS_WRITE_B32_gfx9 %5:vgpr_32, %8", "DS_WRITE_B32_gfx9 %6:vgpr_32, %8").replace("336", "0")
    merged = wrong.replace(" 17, 84,", " 0, 4,").replace("DS_WRITE2_B32", "DS_WRITE2ST64_B32")
    assert bad_merges(_mir(other.replace("272", "0"), merged)) == []


def test_decode_step_validation():
    """The decode step's checks, before any launch: one token per row, grouped heads, a
    history buffer distinct from the one it reads, non-null and 16-byte aligned tensors. The
    buffers are made-up addresses (the calls must fail validation): not run where a GPU is
    visible, so that a regressed check cannot launch on them."""
    if torch.cuda.is_available():
        pytest.skip("host-side validation with made-up device addresses: CPU only")
    from tjev_amd import _lib

    lib = _lib.load()
    p = _params(length=1)
    bufs = [ctypes.c_void_p(256 * (i + 1)) for i in range(11)]
    assert lib.tjev_gdn_decode_step(ctypes.byref(_params(length=2)), None, *bufs) == 1
    assert "one token per row" in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_decode_step(ctypes.byref(_params(length=1, value_heads=5)), None, *bufs) == 1
    assert "groups of" in lib.tjev_gdn_last_error().decode()
    alias = list(bufs)
    alias[9] = alias[6]  # conv_state_out == conv_state
    assert lib.tjev_gdn_decode_step(ctypes.byref(p), None, *alias) == 1
    assert "alias" in lib.tjev_gdn_last_error().decode()
    nulls = list(bufs)
    nulls[7] = None  # state
    assert lib.tjev_gdn_decode_step(ctypes.byref(p), None, *nulls) == 1
    assert "null" in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_decode_step(ctypes.byref(_params(length=1, key_dim=48, value_dim=48)), None, *bufs) == 2
    for i in (0, 6, 7, 9, 10):  # qkv, conv_state, state, conv_state_out, state_out: 16-byte pieces
        odd = list(bufs)
        odd[i] = ctypes.c_void_p(256 * 20 + 8)
        assert lib.tjev_gdn_decode_step(ctypes.byref(p), None, *odd) == 1
        assert "16-byte aligned" in lib.tjev_gdn_last_error().decode()


def test_serving_rejects_cpu_tensors():
    import torch

    from tjev_amd.serve import gdn_decode_step, gdn_prefill

    x = torch.zeros(1, 16, 2 * 16 + 2 * 16)
    with pytest.raises(RuntimeError, match="GPU"):
        gdn_prefill(x, torch.zeros(1, 16, 2), torch.zeros(1, 16, 2), torch.zeros(2), torch.zeros(2),
                    torch.zeros(4, 64), torch.ones(1, 16, dtype=torch.int32), key_heads=1, key_dim=16,
                    value_heads=2, value_dim=16)
    with pytest.raises(RuntimeError, match="GPU"):
        gdn_decode_step(x[:, 0], torch.zeros(1, 2), torch.zeros(1, 2), torch.zeros(2), torch.zeros(2),
                        torch.zeros(4, 64), torch.zeros(1, 3, 64), torch.zeros(1, 2, 16, 16), key_heads=1,
                        key_dim=16, value_heads=2, value_dim=16)


def test_kernel_roofline_takes_the_longer_ideal_time():
    """The bound is the resource whose ideal time is longer: the 0.8B chunk kernels are HBM-bound
    against the bf16 peak and MFMA-bound against the fp32 one; bytes of every kernel are the sum
    of its operand tensors (bwd grads: q, k, X, v_new, dq, dk, S, G, d out and the context; T,
    unit lower triangular, counts as its strictly lower triangle)."""
    from tjev_amd.roofline import PEAK_BF16_TFLOPS, PEAK_FP32_TFLOPS, kernel_roofline, kernel_work

    w = kernel_work(batch=4, length=4096, key_heads=16, value_heads=16, dim=128, chunk=128, io_bytes=2)
    act, mat, io = 4 * 16 * 4096 * 128 * 4, 4 * 16 * 32 * 128 * 128 * 4, 4 * 16 * 4096 * 128 * 2
    ctx = 4 * 4096 * 4 + 3 * 4 * 16 * 4096 * 4
    assert w["gdn_bwd_grads"]["bytes"] == 6 * act + 2 * mat + io + ctx + 2 * 4 * 16 * 4096 * 4
    assert w["gdn_chunk_fwd"]["bytes"] == 4 * act + ctx
    tri = 4 * 16 * 32 * (128 * 127 // 2) * 4  # T: its strictly lower triangle per chunk
    assert kernel_work(batch=4, length=4096, key_heads=16, value_heads=16, dim=128, chunk=128, io_bytes=2,
                       residuals="tinv")["gdn_chunk_fwd"]["bytes"] == 4 * act + ctx + tri
    # v from the raw rows in the forward's chunk kernel: it reads bf16 raw v for the fp32 v rows,
    # which the forward's k_prep no longer reads (raw) or writes (fp32)
    fv = kernel_work(batch=4, length=4096, key_heads=16, value_heads=16, dim=128, chunk=128, io_bytes=2, fused_v=True)
    assert fv["gdn_chunk_fwd"]["bytes"] == 3 * act + io + ctx
    assert fv["gdn_prep_fwd"]["bytes"] == w["gdn_prep_fwd"]["bytes"] - io - act
    assert fv["gdn_prep_bwd"] == w["gdn_prep_bwd"] and fv["gdn_chunk_bwd"] == w["gdn_chunk_bwd"]
    # and q in the output kernel: bf16 raw q for the fp32 q rows k_prep no longer reads or writes
    fq = kernel_work(batch=4, length=4096, key_heads=16, value_heads=16, dim=128, chunk=128, io_bytes=2, fused_v=True,
                     fused_q=True)
    assert fq["gdn_out"]["bytes"] == w["gdn_out"]["bytes"] - act + io
    assert fq["gdn_prep_fwd"]["bytes"] == w["gdn_prep_fwd"]["bytes"] - 2 * (io + act)
    r = kernel_roofline(w["gdn_bwd_grads"], 338e-6, PEAK_BF16_TFLOPS)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and abs(r["frac"] - r["hbm_frac"]) < 1e-12
    assert abs(r["achieved"] - w["gdn_bwd_grads"]["bytes"] / 338e-6 / 1e9) < 1e-6
    r = kernel_roofline(w["gdn_bwd_grads"], 338e-6, PEAK_FP32_TFLOPS)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["frac"] == r["mfma_frac"]
    assert kernel_roofline(w["gdn_post"], 270e-6, PEAK_FP32_TFLOPS)["bound"] == "hbm"


def test_fuses_v_follows_the_launch_rule():
    """The forward's chunk kernel builds v from the raw rows for bf16 I/O through a conv of 1 to 4
    taps at chunk = head dim = 128 (chunks above 128 run the 128-token kernels), else not; its
    output kernel q where, besides, each key head has one value head."""
    from tjev_amd.roofline import fuses_q, fuses_v

    assert fuses_q(io_bytes=2, chunk=128, dim=128, taps=4, key_heads=16, value_heads=16)
    assert not fuses_q(io_bytes=2, chunk=128, dim=128, taps=4, key_heads=16, value_heads=32)
    assert not fuses_q(io_bytes=4, chunk=128, dim=128, taps=4, key_heads=16, value_heads=16)

    assert fuses_v(io_bytes=2, chunk=128, dim=128, taps=4) and fuses_v(io_bytes=2, chunk=256, dim=128, taps=1)
    assert not fuses_v(io_bytes=4, chunk=128, dim=128, taps=4)
    assert not fuses_v(io_bytes=2, chunk=64, dim=128, taps=4) and not fuses_v(io_bytes=2, chunk=128, dim=64, taps=4)
    assert not fuses_v(io_bytes=2, chunk=128, dim=128, taps=0) and not fuses_v(io_bytes=2, chunk=128, dim=128, taps=5)


def test_state_entry_points_validate_before_launch():
    """The continued-sequence entry points (an initial state and conv history in, the final
    ones out): their checks come before the workspace's, and every call here passes no
    workspace, so none can launch: a conv history needs a conv of 2+ taps, a gradient needs its
    input (the final state's gradient any length), state tensors are 16-byte aligned."""
    from tjev_amd import _lib

    lib = _lib.load()
    vp = lambda i: ctypes.c_void_p(4096 * (i + 1))  # noqa: E731  (256-byte aligned, never dereferenced)
    ws = ctypes.c_void_p(4096 * 64)

    def fwd(p, init=None, hist=None, final=None, cs=None):
        return lib.tjev_gdn_mega2_fwd_cont(ctypes.byref(p), None, *[vp(i) for i in range(7)], init, hist, vp(8),
                                           vp(9), final, cs, ws, 0)

    def bwd(p, init=None, hist=None, d_final=None, d_init=None, d_hist=None):
        return lib.tjev_gdn_mega2_bwd_cont(ctypes.byref(p), None, *[vp(i) for i in range(7)], init, hist, vp(9),
                                           vp(10), d_final, *[vp(11 + i) for i in range(6)], d_init, d_hist, ws, 0)

    p = _params(length=96, chunk=16)
    assert fwd(p) == 3 and "workspace" in lib.tjev_gdn_last_error().decode()  # all checks passed
    assert fwd(p, init=vp(20), hist=vp(21), final=vp(22), cs=vp(23)) == 3
    assert fwd(_params(taps=1), hist=vp(21)) == 1 and "2 or more taps" in lib.tjev_gdn_last_error().decode()
    assert fwd(_params(taps=0), cs=vp(23)) == 1
    assert fwd(p, init=ctypes.c_void_p(4096 * 20 + 8)) == 1
    assert "16-byte aligned" in lib.tjev_gdn_last_error().decode()
    assert bwd(p, init=vp(20), hist=vp(21), d_final=vp(22), d_init=vp(23), d_hist=vp(24)) == 3
    assert bwd(p, d_init=vp(23)) == 1 and "needs the initial state" in lib.tjev_gdn_last_error().decode()
    assert bwd(p, init=vp(20), d_hist=vp(24)) == 1 and "needs the conv history" in lib.tjev_gdn_last_error().decode()
    # a length inside a chunk: the final state's gradient is accepted (the padded tail carries it)
    assert bwd(_params(length=100, chunk=16), d_final=vp(22)) == 3
    assert "workspace" in lib.tjev_gdn_last_error().decode()
    # the v2 forms
    p0 = _params(taps=0, length=96, chunk=16)
    assert lib.tjev_gdn_v2_fwd_cont(ctypes.byref(p0), None, *[vp(i) for i in range(6)], vp(20), vp(7), vp(8),
                                    vp(9), ws, 0) == 3
    assert lib.tjev_gdn_v2_bwd_cont(ctypes.byref(p0), None, *[vp(i) for i in range(6)], None, vp(8), vp(9),
                                    None, *[vp(10 + i) for i in range(5)], vp(16), ws, 0) == 1
    assert "needs the initial state" in lib.tjev_gdn_last_error().decode()
    assert lib.tjev_gdn_v2_bwd_cont(ctypes.byref(_params(taps=0, length=90, chunk=16)), None,
                                    *[vp(i) for i in range(6)], vp(20), vp(8), vp(9), vp(21),
                                    *[vp(10 + i) for i in range(5)], vp(16), ws, 0) == 3


def test_state_operators_reject_cpu_tensors_and_bad_shapes():
    from tjev_amd import gdn_megakernel
    from tjev_amd.v2 import chunk_gated_delta_rule

    x = torch.zeros(1, 16, 2 * 16 + 2 * 16)
    with pytest.raises(RuntimeError, match="GPU"):
        gdn_megakernel(x, torch.zeros(1, 16, 2), torch.zeros(1, 16, 2), torch.zeros(2), torch.zeros(2),
                       torch.zeros(4, 64), torch.ones(1, 16, dtype=torch.int32), key_heads=1, key_dim=16,
                       value_heads=2, value_dim=16, initial_state=torch.zeros(1, 2, 16, 16))
    q = torch.zeros(1, 16, 2, 16)
    with pytest.raises(ValueError, match="inverse in"):
        chunk_gated_delta_rule(q, q, q, torch.zeros(1, 16, 2), torch.zeros(1, 16, 2), inverse="lu")
    with pytest.raises(RuntimeError, match="GPU"):
        chunk_gated_delta_rule(q, q, q, torch.zeros(1, 16, 2), torch.zeros(1, 16, 2))


def test_normed_forward_validates_before_launch():
    """tjev_gdn_mega2_fwd_normed (the core with the gated RMSNorm in its output kernel): y,
    gate and the norm weight are required, gate and y 16-byte aligned, eps >= 0; with every
    check passed and no workspace it stops at the workspace check, so nothing launches."""
    from tjev_amd import _lib

    lib = _lib.load()
    vp = lambda i: ctypes.c_void_p(4096 * (i + 1))  # noqa: E731  (never dereferenced)
    ws = ctypes.c_void_p(4096 * 64)

    def fwd(gate=vp(12), nw=vp(13), eps=1e-6, y=vp(15)):
        return lib.tjev_gdn_mega2_fwd_normed(ctypes.byref(_params(length=96, chunk=16)), None,
                                             *[vp(i) for i in range(7)], None, None, gate, nw, ctypes.c_float(eps),
                                             vp(14), y, vp(16), None, None, ws, 0)

    assert fwd() == 3 and "workspace" in lib.tjev_gdn_last_error().decode()
    assert fwd(y=None) == 1 and "null" in lib.tjev_gdn_last_error().decode()
    assert fwd(gate=None) == 1 and "null" in lib.tjev_gdn_last_error().decode()
    assert fwd(nw=None) == 1
    assert fwd(gate=ctypes.c_void_p(4096 * 12 + 8)) == 1 and "16-byte" in lib.tjev_gdn_last_error().decode()
    assert fwd(eps=-1.0) == 1 and "eps" in lib.tjev_gdn_last_error().decode()


def test_normed_operator_checks_shapes_and_has_no_cpu_fallback():
    from tjev_amd import gdn_megakernel_normed

    x = torch.zeros(1, 16, 2 * 16 + 2 * 16)
    g2 = torch.zeros(1, 16, 2)
    args = (x, g2, g2, torch.zeros(2), torch.zeros(2), torch.zeros(4, 64), torch.ones(1, 16, dtype=torch.int32))
    kw = dict(key_heads=1, key_dim=16, value_heads=2, value_dim=16)
    with pytest.raises(RuntimeError, match="GPU"):
        gdn_megakernel_normed(*args, torch.zeros(1, 16, 2, 16), torch.ones(16), **kw)
    with pytest.raises(ValueError, match="inverse"):
        gdn_megakernel_normed(*args, torch.zeros(1, 16, 2, 16), torch.ones(16), inverse="lu", **kw)


def test_normed_backward_validates_before_launch():
    """tjev_gdn_mega2_bwd_normed: out, gate, d_y and d_gate are required and 16-byte aligned,
    eps >= 0, and its workspace (tjev_gdn_workspace_bytes_normed) holds the megakernel
    backward's, d out and the norm's weight-gradient partials; with no workspace every valid
    call stops at the workspace check, before the norm's backward is launched."""
    from tjev_amd import _lib

    lib = _lib.load()
    vp = lambda i: ctypes.c_void_p(4096 * (i + 1))  # noqa: E731  (never dereferenced)
    ws = ctypes.c_void_p(4096 * 64)
    p = _params(length=96, chunk=16)
    base = lib.tjev_gdn_workspace_bytes(ctypes.byref(p), 1)
    dout = 1 * 96 * p.value_heads * p.value_dim * 4
    assert lib.tjev_gdn_workspace_bytes_normed(ctypes.byref(p), 0) == base + dout
    assert lib.tjev_gdn_workspace_bytes_normed(ctypes.byref(p), 1) > base + dout
    assert lib.tjev_gdn_workspace_bytes_normed(ctypes.byref(_params(chunk=24)), 0) == 0

    def bwd(out=vp(12), gate=vp(13), eps=1e-6, d_y=vp(15), d_gate=vp(26), d_nw=None):
        return lib.tjev_gdn_mega2_bwd_normed(ctypes.byref(p), None, *[vp(i) for i in range(7)], None, None, vp(9),
                                             out, gate, vp(14), ctypes.c_float(eps), d_y, None,
                                             *[vp(16 + i) for i in range(5)], None, None, None, d_gate, d_nw, ws, 0)

    assert bwd() == 3 and "workspace" in lib.tjev_gdn_last_error().decode()
    assert bwd(d_nw=vp(27)) == 3
    assert bwd(out=None) == 1 and "null" in lib.tjev_gdn_last_error().decode()
    assert bwd(d_gate=None) == 1
    assert bwd(d_y=ctypes.c_void_p(4096 * 15 + 4)) == 1 and "16-byte" in lib.tjev_gdn_last_error().decode()
    assert bwd(eps=float("nan")) == 1 and "eps" in lib.tjev_gdn_last_error().decode()


def test_chunks_above_128_run_the_128_kernels():
    """Every power-of-two chunk >= 8 is accepted (pallas_tpu_mega.py:597-615): chunks above 128 run
    the chunk-128 kernels, so their residual and workspace sizes are chunk 128's."""
    from tjev_amd import _lib

    lib = _lib.load()
    for c in (256, 512, 1024):
        p = _params(chunk=c, length=600)
        assert lib.tjev_gdn_check(ctypes.byref(p)) == 0
        q = _params(chunk=128, length=600)
        assert lib.tjev_gdn_residual_bytes(ctypes.byref(p)) == lib.tjev_gdn_residual_bytes(ctypes.byref(q))
        assert lib.tjev_gdn_workspace_bytes(ctypes.byref(p), 1) == lib.tjev_gdn_workspace_bytes(ctypes.byref(q), 1)


def test_head_dims_run_padded_to_a_compiled_dim():
    """Head dims the kernels do not hold as they are run zero-padded to the next compiled dim
    (Dk != Dv, or widths other than 16 .. 128 powers of two, up to 128); the lane layout of
    qkv round-trips through the padding."""
    from tjev_amd.gdn import pad_qkv, run_dim, unpad_qkv

    assert [run_dim(d, d) for d in (16, 32, 64, 128)] == [16, 32, 64, 128]
    assert run_dim(64, 128) == run_dim(128, 64) == 128 and run_dim(48, 48) == 64 and run_dim(32, 96) == 128
    assert run_dim(8, 8) == 16 and run_dim(256, 256) is None and run_dim(64, 192) is None
    hk, dk, h, dv = 2, 48, 3, 40
    x = torch.arange(5 * (2 * hk * dk + h * dv), dtype=torch.float32).reshape(5, -1)
    padded = pad_qkv(x, hk, dk, h, dv, 64)
    assert padded.shape == (5, 2 * hk * 64 + h * 64)
    heads = padded.reshape(5, 2 * hk + h, 64)
    assert torch.all(heads[..., :dk][:, :2 * hk] == x[:, :2 * hk * dk].reshape(5, 2 * hk, dk))
    assert torch.all(heads[:, :2 * hk, dk:] == 0) and torch.all(heads[:, 2 * hk:, dv:] == 0)
    assert torch.equal(unpad_qkv(padded, hk, dk, h, dv, 64), x)


def test_wide_value_heads_run_as_column_groups():
    """Value heads wider than 128 (Dk <= 128) run as groups of at most 128 value columns; the
    lanes of qkv cut into each group's and the conv history joined back round-trip; Dk above 128
    has no split."""
    from tjev_amd.gdn import merge_value_cols, value_cols, value_groups

    assert value_groups(128, 128) is None and value_groups(64, 96) is None and value_groups(256, 256) is None
    assert value_groups(128, 256) == [(0, 128), (128, 128)]
    assert value_groups(32, 300) == [(0, 128), (128, 128), (256, 44)]
    hk, dk, h, dv = 2, 16, 3, 300
    x = torch.arange(4 * (2 * hk * dk + h * dv), dtype=torch.float32).reshape(4, -1)
    parts = [value_cols(x, hk, dk, h, dv, c, w) for c, w in value_groups(dk, dv)]
    for (c, w), p in zip(value_groups(dk, dv), parts):
        assert p.shape == (4, 2 * hk * dk + h * w)
        assert torch.equal(p[:, :2 * hk * dk], x[:, :2 * hk * dk])
        assert torch.equal(p[:, 2 * hk * dk:].reshape(4, h, w), x[:, 2 * hk * dk:].reshape(4, h, dv)[..., c:c + w])
    assert torch.equal(merge_value_cols(parts, hk, dk, h), x)


def test_head_layout_round_trips_property():
    """For any head counts and widths (hypothesis): padding every head of qkv's lanes to a wider
    dim and cutting it back is the identity, the padded lanes are zero, and cutting qkv's lanes
    into value-column groups and joining them back is the identity; the groups tile Dv."""
    from hypothesis import given, settings
    from hypothesis import strategies as st

    from tjev_amd.gdn import merge_value_cols, pad_qkv, run_dim, unpad_qkv, value_cols, value_groups

    @settings(max_examples=60, deadline=None)
    @given(hk=st.integers(1, 4), ratio=st.integers(1, 3), dk=st.integers(1, 128), dv=st.integers(1, 400),
           rows=st.integers(1, 3))
    def check(hk, ratio, dk, dv, rows):
        h = hk * ratio
        x = torch.randn(rows, 2 * hk * dk + h * dv)
        groups = value_groups(dk, dv)
        if groups is None:
            run = run_dim(dk, dv)
            assert run is not None and run >= max(dk, dv)
            padded = pad_qkv(x, hk, dk, h, dv, run)
            assert padded.shape == (rows, (2 * hk + h) * run)
            assert torch.equal(unpad_qkv(padded, hk, dk, h, dv, run), x)
            lanes = padded.reshape(rows, 2 * hk + h, run)
            assert torch.all(lanes[:, :2 * hk, dk:] == 0) and torch.all(lanes[:, 2 * hk:, dv:] == 0)
        else:
            assert dv > 128 and sum(w for _, w in groups) == dv
            assert all(0 < w <= 128 for _, w in groups) and [c for c, _ in groups] == list(range(0, dv, 128))
            parts = [value_cols(x, hk, dk, h, dv, c, w) for c, w in groups]
            assert torch.equal(merge_value_cols(parts, hk, dk, h), x)

    check()


def test_integration_python_samples_compile():
    """The Python bindings INTEGRATION.md shows a maintainer parse as Python (they are compiled,
    not run: jax is not in this image)."""
    import re
    from pathlib import Path

    text = (Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    assert len(blocks) >= 2
    for i, src in enumerate(blocks):
        compile(src, f"INTEGRATION.md python block {i}", "exec")
