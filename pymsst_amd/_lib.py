"""ctypes binding of ``libpymsst_amd.so`` (the C ABI declared in ``include/pymsst_amd.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already mapped; HIP streams and
device pointers from torch are then valid inside the library.  Argument types
are derived from the header's prototypes, so the binding cannot drift from it.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library is loaded)

PKG_DIR = Path(__file__).resolve().parent
HEADER = PKG_DIR.parent / "include" / "pymsst_amd.h"
LIB_PATH = Path(os.environ.get("PYMSST_AMD_LIB", PKG_DIR / "libpymsst_amd.so"))

PMSST_F32, PMSST_F16, PMSST_BF16 = 0, 1, 2
_CTYPES = {
    "int": ctypes.c_int,
    "int64_t": ctypes.c_int64,
    "size_t": ctypes.c_size_t,
    "void": None,
}


class FusedKernelUnavailable(RuntimeError):
    """Raised when the HIP extension cannot be used (no library, no GPU, no HIP torch)."""


class PmsstError(RuntimeError):
    """A C-ABI call returned a nonzero status."""


def _ctype(decl: str):
    decl = decl.strip()
    if "*" in decl:
        if decl.replace(" ", "").startswith("constchar*"):
            return ctypes.c_char_p
        return ctypes.c_void_p
    base = decl.replace("const", "").split()[0]
    return _CTYPES[base]


def parse_header(path: Path = HEADER) -> dict[str, tuple[object, list[object]]]:
    """``{name: (restype, argtypes)}`` for every ``pmsst_*`` prototype in the header."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"^\s*((?:const\s+)?\w+\s*\*?)\s*(pmsst_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        argtypes = []
        if args.strip() not in ("", "void"):
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name
                a = re.sub(r"\b\w+$", "", a).strip()
                argtypes.append(_ctype(a))
        protos[name] = (_ctype(ret), argtypes)
    return protos


_lock = threading.Lock()
_lib = None


def load_library(path: Path | None = None):
    """Load and bind the library once; raises :class:`FusedKernelUnavailable` if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path or LIB_PATH)
        if not p.is_file():
            raise FusedKernelUnavailable(
                f"{p} is missing: build it with `python -m pymsst_amd.build` (or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
        except OSError as exc:
            raise FusedKernelUnavailable(f"failed to load {p}: {exc}") from exc
        for name, (restype, argtypes) in parse_header().items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    lib = load_library()
    msg = lib.pmsst_last_error()
    return msg.decode() if msg else ""


def check(rc: int, op: str) -> None:
    if rc != 0:
        raise PmsstError(f"{op}: {last_error()} (status {rc})")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return PMSST_F32
    if dtype == torch.float16:
        return PMSST_F16
    if dtype == torch.bfloat16:
        return PMSST_BF16
    raise PmsstError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16")
