"""Loading of the native libraries.

``libkernel_lab.so`` holds the gfx950 kernels behind the C-ABI of
``include/kernel_lab.h``; ``_C.so`` registers ``torch.ops.kernel_lab.*`` on top
of it. Both are built in-tree by ``kernel-lab_amd/build.py``.

PyTorch is imported first on purpose: it loads its own HIP runtime, and the
libraries here bind to that same copy (they name it only by soname), so a
process never holds two HIP runtimes.

There is no fallback. If the libraries are missing, ``available()`` is False,
``why_unavailable()`` says why, and every operator call raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path
from typing import Iterator

import torch

LIB_DIR = Path(__file__).resolve().parent
CORE_PATH = LIB_DIR / "libkernel_lab.so"
TORCH_EXT_PATH = LIB_DIR / "_C.so"

# C-ABI: name -> (restype, argtypes). Mirrors include/kernel_lab.h.
_i32, _i64, _f32, _vp, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "kl_status_string": (ctypes.c_char_p, [_i32]),
    "kl_last_error": (ctypes.c_char_p, []),
    "kl_version": (_i32, []),
    "kl_rms_norm": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _vp]),
    "kl_paged_decode_plan": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_sz)],
    ),
    "kl_paged_decode_attention": (
        _i32,
        [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _i32, _vp, _sz, _vp],
    ),
    "kl_cascade_decode_plan": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_sz)]),
    "kl_cascade_decode_attention": (
        _i32,
        [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _vp, _sz, _vp],
    ),
    "kl_paged_decode_last_merge": (_i32, []),
    "kl_paged_decode_reload_options": (_i32, []),
    "kl_paged_decode_attention_noalloc": (
        _i32,
        [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _i32, _vp],
    ),
    "kl_paged_decode_attention_fp8": (
        _i32,
        [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _i32, _vp, _sz, _vp],
    ),
}

# kl_dtype / kl_status values from include/kernel_lab.h.
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
KL_OK = 0

_core: ctypes.CDLL | None = None
_ops_registered = False
_error = ""


def _load() -> None:
    global _core, _ops_registered, _error
    try:
        core = ctypes.CDLL(str(CORE_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(core, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _core = core
    except OSError as exc:
        _error = f"{CORE_PATH.name} not loadable ({exc}); run kernel-lab_amd/build.py"
        return
    try:
        torch.ops.load_library(str(TORCH_EXT_PATH))
        _ops_registered = True
    except (OSError, RuntimeError) as exc:
        _error = f"{TORCH_EXT_PATH.name} not loadable ({exc}); run kernel-lab_amd/build.py"


_load()


def loaded() -> bool:
    """True when both native libraries loaded (no GPU needed)."""
    return _core is not None and _ops_registered


def available() -> bool:
    """True when the operators can run: libraries loaded and a GPU present."""
    return loaded() and torch.cuda.is_available()


def why_unavailable() -> str:
    if not loaded():
        return _error or "native libraries not loaded"
    return "no GPU device"


def core() -> ctypes.CDLL:
    """The C-ABI library; raises if it is not built."""
    if _core is None:
        raise RuntimeError(f"kernel_lab native library unavailable: {why_unavailable()}")
    return _core


def require_ops() -> None:
    if not _ops_registered:
        raise RuntimeError(f"kernel_lab operators unavailable: {why_unavailable()}")


def last_error() -> str:
    return core().kl_last_error().decode()


def status_string(status: int) -> str:
    return core().kl_status_string(status).decode()


@contextlib.contextmanager
def decode_switches(**values: str) -> Iterator[None]:
    """Sets the library's decode switches for the block: each keyword names one
    ``KL_DECODE_<NAME>`` environment variable (``paired="0"``,
    ``force_valu="1"``, ``fused_merge="0"``, ``balance_always="1"``). The
    library reads them once per process, so it is told to re-read them on entry
    and again on exit, after the previous values are restored."""
    names = {f"KL_DECODE_{key.upper()}": value for key, value in values.items()}
    saved = {name: os.environ.get(name) for name in names}
    lib = core()
    try:
        os.environ.update(names)
        lib.kl_paged_decode_reload_options()
        yield
    finally:
        for name, value in saved.items():
            if value is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = value
        lib.kl_paged_decode_reload_options()
