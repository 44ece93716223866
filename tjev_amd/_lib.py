"""ctypes binding of libtjev_gdn.so (include/tjev_gdn.h).

The library is built in-tree by ``python -m tjev_amd.build``. Loading never falls back to
anything: a missing or broken library raises, so no GDN call can silently run elsewhere.
torch is imported first so that the library shares torch's HIP runtime (same soname).
"""

from __future__ import annotations

import contextlib
import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "libtjev_gdn.so"
# the debug build whose kernels first fill their LDS with NaN (python -m tjev_amd.build --lds-poison)
LDS_POISON_PATH = Path(__file__).resolve().parent / "libtjev_gdn_lds_poison.so"

F32, BF16 = 0, 1
PRECISION = {"highest": 0, "high": 1, "bf16": 2, "mixed": 3}
INVERSE = {"doubling": 0, "blocked": 1}
RESIDUALS = {"states": 0, "tinv": 1, "all": 2}  # tjev_gdn_residuals
STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "workspace", 4: "HIP error"}

EXPORTS = (
    "tjev_gdn_check",
    "tjev_gdn_states_bytes",
    "tjev_gdn_residual_bytes",
    "tjev_gdn_workspace_bytes",
    "tjev_gdn_mega2_fwd",
    "tjev_gdn_mega2_fwd_state",
    "tjev_gdn_mega2_fwd_cont",
    "tjev_gdn_mega2_fwd_normed",
    "tjev_gdn_mega2_bwd_normed",
    "tjev_gdn_workspace_bytes_normed",
    "tjev_gdn_mega2_bwd_cont",
    "tjev_gdn_mega2_fwd_cont_noalloc",
    "tjev_gdn_decode_step",
    "tjev_gdn_v2_fwd",
    "tjev_gdn_v2_bwd",
    "tjev_gdn_v2_fwd_cont",
    "tjev_gdn_v2_bwd_cont",
    "tjev_gdn_mega2_bwd",
    "tjev_gdn_norm_workspace_bytes",
    "tjev_gdn_gated_rmsnorm_fwd",
    "tjev_gdn_gated_rmsnorm_bwd",
    "tjev_gdn_profile_begin",
    "tjev_gdn_profile_end",
    "tjev_gdn_kernel_name",
    "tjev_gdn_last_error",
    "tjev_gdn_version",
    "tjev_gdn_lds_poison",
)
N_KERNELS = 16  # TJEV_GDN_KERNELS
SCRATCH_BYTES = 128 << 20  # TJEV_GDN_SCRATCH_BYTES


class Params(ctypes.Structure):
    """tjev_gdn_params"""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "batch", "length", "key_heads", "key_dim", "value_heads", "value_dim", "taps", "chunk",
        "io_dtype", "gate_dtype", "precision", "inverse", "heads_per_step", "residuals", "qk_dtype",
    )]


class NormParams(ctypes.Structure):
    """tjev_gdn_norm_params"""

    _fields_ = [("tokens", ctypes.c_int64), ("heads", ctypes.c_int32), ("dim", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("eps", ctypes.c_float)]


class GdnLibraryError(RuntimeError):
    """A nonzero status from the library (the message is tjev_gdn_last_error())."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status}: {STATUS.get(status, '?')})")
        self.status = status


_LIB: ctypes.CDLL | None = None


_OPENED: dict[str, ctypes.CDLL] = {}


def load() -> ctypes.CDLL:
    """The loaded library (raises if it is not built)."""
    global _LIB
    if _LIB is None:
        _LIB = open_library(LIB_PATH)
    return _LIB


@contextlib.contextmanager
def library(path: Path):
    """Every call made inside the block (plans built inside it) goes through the library at
    ``path``: the LDS-poison debug build in its tests. The default library comes back after."""
    global _LIB
    saved = _LIB
    _LIB = open_library(path)
    try:
        yield _LIB
    finally:
        _LIB = saved


def open_library(path: Path) -> ctypes.CDLL:
    """The library at ``path`` with the ABI's argument types bound (opened once per path)."""
    key = str(path)
    if key in _OPENED:
        return _OPENED[key]
    if not Path(path).exists():
        raise RuntimeError(f"{path} is not built: run `python -m tjev_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(key)
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    pp = ctypes.POINTER(Params)
    lib.tjev_gdn_check.argtypes = [pp]
    lib.tjev_gdn_check.restype = i32
    lib.tjev_gdn_states_bytes.argtypes = [pp]
    lib.tjev_gdn_states_bytes.restype = sz
    lib.tjev_gdn_residual_bytes.argtypes = [pp]
    lib.tjev_gdn_residual_bytes.restype = sz
    lib.tjev_gdn_workspace_bytes.argtypes = [pp, i32]
    lib.tjev_gdn_workspace_bytes.restype = sz
    lib.tjev_gdn_mega2_fwd.argtypes = [pp, vp] + [vp] * 10 + [sz]
    lib.tjev_gdn_mega2_fwd.restype = i32
    lib.tjev_gdn_mega2_fwd_state.argtypes = [pp, vp] + [vp] * 12 + [sz]
    lib.tjev_gdn_mega2_fwd_state.restype = i32
    lib.tjev_gdn_mega2_fwd_cont.argtypes = [pp, vp] + [vp] * 14 + [sz]
    lib.tjev_gdn_mega2_fwd_cont.restype = i32
    lib.tjev_gdn_mega2_fwd_normed.argtypes = [pp, vp] + [vp] * 11 + [ctypes.c_float] + [vp] * 6 + [sz]
    lib.tjev_gdn_mega2_fwd_normed.restype = i32
    lib.tjev_gdn_mega2_bwd_normed.argtypes = [pp, vp] + [vp] * 13 + [ctypes.c_float] + [vp] * 13 + [sz]
    lib.tjev_gdn_mega2_bwd_normed.restype = i32
    lib.tjev_gdn_workspace_bytes_normed.argtypes = [pp, i32]
    lib.tjev_gdn_workspace_bytes_normed.restype = sz
    lib.tjev_gdn_mega2_bwd_cont.argtypes = [pp, vp] + [vp] * 21 + [sz]
    lib.tjev_gdn_mega2_bwd_cont.restype = i32
    lib.tjev_gdn_mega2_fwd_cont_noalloc.argtypes = [pp, vp] + [vp] * 13
    lib.tjev_gdn_mega2_fwd_cont_noalloc.restype = i32
    lib.tjev_gdn_v2_fwd_cont.argtypes = [pp, vp] + [vp] * 11 + [sz]
    lib.tjev_gdn_v2_fwd_cont.restype = i32
    lib.tjev_gdn_v2_bwd_cont.argtypes = [pp, vp] + [vp] * 17 + [sz]
    lib.tjev_gdn_v2_bwd_cont.restype = i32
    lib.tjev_gdn_decode_step.argtypes = [pp, vp] + [vp] * 11
    lib.tjev_gdn_decode_step.restype = i32
    lib.tjev_gdn_v2_fwd.argtypes = [pp, vp] + [vp] * 9 + [sz]
    lib.tjev_gdn_v2_fwd.restype = i32
    lib.tjev_gdn_v2_bwd.argtypes = [pp, vp] + [vp] * 14 + [sz]
    lib.tjev_gdn_v2_bwd.restype = i32
    lib.tjev_gdn_mega2_bwd.argtypes = [pp, vp] + [vp] * 16 + [sz]
    lib.tjev_gdn_mega2_bwd.restype = i32
    npp = ctypes.POINTER(NormParams)
    lib.tjev_gdn_norm_workspace_bytes.argtypes = [npp, i32]
    lib.tjev_gdn_norm_workspace_bytes.restype = sz
    lib.tjev_gdn_gated_rmsnorm_fwd.argtypes = [npp, vp] + [vp] * 5
    lib.tjev_gdn_gated_rmsnorm_fwd.restype = i32
    lib.tjev_gdn_gated_rmsnorm_bwd.argtypes = [npp, vp] + [vp] * 9 + [sz]
    lib.tjev_gdn_gated_rmsnorm_bwd.restype = i32
    lib.tjev_gdn_profile_begin.argtypes = []
    lib.tjev_gdn_profile_begin.restype = i32
    lib.tjev_gdn_profile_end.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int), i32]
    lib.tjev_gdn_profile_end.restype = i32
    lib.tjev_gdn_kernel_name.argtypes = [i32]
    lib.tjev_gdn_kernel_name.restype = ctypes.c_char_p
    lib.tjev_gdn_last_error.argtypes = []
    lib.tjev_gdn_last_error.restype = ctypes.c_char_p
    lib.tjev_gdn_version.argtypes = []
    lib.tjev_gdn_version.restype = i32
    lib.tjev_gdn_lds_poison.argtypes = []
    lib.tjev_gdn_lds_poison.restype = i32
    _OPENED[key] = lib
    return lib


def check_status(status: int) -> None:
    if status != 0:
        raise GdnLibraryError(status, load().tjev_gdn_last_error().decode())


class KernelTimer:
    """Per-kernel HIP-event timing of the library's launches (tjev_gdn_profile_*):
    ``with KernelTimer() as kt: ...`` then ``kt.ms`` / ``kt.launches`` keyed by kernel name."""

    def __enter__(self):
        check_status(load().tjev_gdn_profile_begin())
        return self

    def __exit__(self, *exc):
        lib = load()
        ms = (ctypes.c_float * N_KERNELS)()
        launches = (ctypes.c_int * N_KERNELS)()
        status = lib.tjev_gdn_profile_end(ms, launches, N_KERNELS)
        names = [lib.tjev_gdn_kernel_name(k).decode() for k in range(N_KERNELS)]
        self.ms = {n: float(ms[k]) for k, n in enumerate(names)}
        self.launches = {n: int(launches[k]) for k, n in enumerate(names)}
        if exc[0] is None:
            check_status(status)
        return False
