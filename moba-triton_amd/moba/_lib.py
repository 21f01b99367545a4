"""Loader and thin caller of the C ABI library `libmoba_hip.so`.

Every stage of the hot path calls into the HIP library through here. There
is no fallback: if the library is missing or the tensors are not on a GPU,
the call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_PATH = Path(os.environ.get("MOBA_HIP_LIB", _LIB_DIR / "libmoba_hip.so"))

MOBA_OK = 0
MOBA_ERR_INVALID = 1
MOBA_ERR_UNSUPPORTED = 2
MOBA_ERR_LAUNCH = 3
MOBA_ERR_WORKSPACE = 4

DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

# Every symbol declared in include/moba_hip.h, with its ctypes signature.
_P, _I, _L, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
SIGNATURES = {
    "moba_abi_version": (_I, []),
    "moba_last_error": (ctypes.c_char_p, []),
    "moba_status_string": (ctypes.c_char_p, [_I]),
    "moba_pool": (_I, [_P, _P, _P, _L, _L, _L, _L, _L, _L, _L, _I, _P]),
    "moba_gate_workspace_size": (_Z, [_L, _L, _L]),
    "moba_gate": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L,
                       _I, _I, _P, _Z, _P]),
    "moba_gate_refine": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L,
                              _I, _I, _P]),
    "moba_gate_noalloc": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L,
                               _I, _I, _P]),
    "moba_csc_workspace_size": (_Z, [_L, _L, _L, _L, _L, _L]),
    "moba_csc_build": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L,
                            _L, _L, _L, _P, _P, _P, _L, _L, _L, _P, _Z, _P]),
    "moba_attend": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                         _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _P, _P, _P, _L,
                         _I, _I, _I, _P]),
    "moba_combine": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _P]),
    "moba_bwd_delta": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _I, _P]),
    "moba_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                      _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _P, _P, _P, _L, _P, _L,
                      _I, _I, _I, _I, _P]),
    "moba_dq_reduce": (_I, [_P, _P, _L, _P, _L, _L, _L, _L, _L, _I, _I, _P]),
}

_lib = None


class LibraryMissing(RuntimeError):
    """The HIP library has not been built (or cannot be loaded)."""


# Version of include/moba_hip.h these bindings follow.
ABI_VERSION = 6


def load() -> ctypes.CDLL:
    """Loads the library once and binds every declared signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} not found; build it with `python -c 'import "
            f"__graft_entry__ as g; g.build()'` or `make -C moba-triton_amd/csrc`")
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise LibraryMissing(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.moba_abi_version() != ABI_VERSION:
        raise LibraryMissing(
            f"{LIB_PATH} has ABI version {lib.moba_abi_version()}, these bindings expect "
            f"{ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def available() -> tuple[bool, str]:
    """(True, '') when the library loads; never raises."""
    try:
        load()
        return True, ""
    except Exception as exc:  # noqa: BLE001 - must never raise
        return False, str(exc)


def ptr(t: torch.Tensor | None):
    """Device address of a tensor (None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device):
    """The current torch stream on `device`, as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name: str, *args) -> None:
    """Calls a library entry point and maps its status to an exception:
    invalid / unsupported configurations raise ValueError (as the
    reference's `_validate` does), launch and workspace failures raise
    RuntimeError."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc == MOBA_OK:
        return
    msg = lib.moba_last_error().decode(errors="replace")
    if rc in (MOBA_ERR_INVALID, MOBA_ERR_UNSUPPORTED):
        raise ValueError(f"{name}: {msg}")
    raise RuntimeError(f"{name} failed ({lib.moba_status_string(rc).decode()}): {msg}")


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU device; returns it. Raises otherwise -- there is
    no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"moba HIP kernels need GPU tensors, got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def aligned_contiguous(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels use 16-byte vector loads)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t
