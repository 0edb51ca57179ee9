"""ctypes binding of libek_hip.so, the C ABI declared in include/ek_hip.h.

torch is imported before the library is loaded: the library's
libamdhip64.so.7 dependency then resolves to the HIP runtime torch already
loaded (same soname), so kernels launched here run on torch's streams and
are recorded by torch.cuda.graph captures.

There is no fallback: if the library is missing or cannot load, every
kernel call raises HipUnavailable.
"""

from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (must precede the library load, see above)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EK_HIP_LIB") or os.path.join(HERE, "libek_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "ek_hip.h")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# argument types per entry point, in include/ek_hip.h order
SIGNATURES = {
    "ek_rms_norm": [_P, _P, _P, _I64, _I64, _I64, _I64, _F, _P],
    "ek_add_rms_norm": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "ek_add_rms_norm_parts": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "ek_silu_mul": [_P, _P, _I64, _I64, _I64, _I64, _P],
    "ek_qk_norm_rope_kv": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                           _I64, _I64, _I64, _I64, _I64, _F, _P],
    "ek_gemv": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "ek_gemv_parts": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "ek_gemv_swiglu": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "ek_norm_gemv": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _I,
                     _I64, _I64, _P],
    "ek_parts_norm_gemv": [_P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                           _I, _I64, _I64, _P],
    "ek_embed_norm_gemv": [_P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                           _P, _P, _I64, _I64, _P],
    "ek_attn_decode": [_P, _I64, _I64, _I, _P, _P, _P, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64,
                       _I64, _P, _P, _P, _I64, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
                       _I64, _I64, _I64, _I64, _F, _F, _P, _I64, _P, _P, _P],
    "ek_attn_prefill": [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "ek_attn_verify": [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                       _P, _I64, _I64, _P],
    "ek_ngram_draft": [_P, _P, _P, _I64, _I64, _I64, _P],
    "ek_spec_accept": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "ek_lm_head_argmax": [_P, _P, _I64, _P, _P, _F, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                          _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "ek_decode_step_plan": [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "ek_decode_step": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _F,
                       _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                       _P, _P, _P, _P, _P, _P, _P, _I64, _P,
                       _P, _P, _I64, _P, _P, _P],
    "ek_decode_step_noalloc": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _F,
                               _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                               _P, _P, _P, _P, _P, _P, _P, _I64, _P,
                               _P, _P, _P],
}


class HipUnavailable(RuntimeError):
    """The HIP kernel library is missing, failed to load, or no GPU is present."""


class HipKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero hipError_t."""

    def __init__(self, name: str, code: int, msg: str):
        super().__init__(f"{name} failed with hipError {code}" + (f": {msg}" if msg else ""))
        self.code = code


_lib = None
_load_error: str | None = None


def declared_symbols(header: str = HEADER) -> list[str]:
    """Every ek_* function name declared in include/ek_hip.h."""
    with open(header) as f:
        text = f.read()
    return re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(ek_\w+)\s*\(", text, flags=re.M)


def load(path: str | None = None):
    """Load (once) and return the ctypes library. Raises HipUnavailable."""
    global _lib, _load_error
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        _load_error = f"{p} is missing: run `python -m enginekernel_amd.build`"
        raise HipUnavailable(_load_error)
    try:
        lib = ctypes.CDLL(p)
    except OSError as e:
        _load_error = f"cannot load {p}: {e}"
        raise HipUnavailable(_load_error) from e
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.ek_version.restype = ctypes.c_char_p
    lib.ek_last_error.restype = ctypes.c_char_p
    lib.ek_device_info.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, ctypes.c_int]
    lib.ek_device_info.restype = ctypes.c_int
    lib.ek_set_wait_limit.argtypes = [ctypes.c_int64]
    lib.ek_set_wait_limit.restype = ctypes.c_int64
    if path is None:
        _lib = lib
    return lib


def available() -> bool:
    try:
        load()
    except HipUnavailable:
        return False
    return torch.cuda.is_available()


def call(name: str, *args) -> None:
    """Invoke one entry point; raise HipKernelError on a non-zero return."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ek_last_error().decode(errors="replace")
        raise HipKernelError(name, rc, msg)


def ptr(t) -> int | None:
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream() -> int:
    """The current torch stream as a hipStream_t value (captured by graphs)."""
    return torch.cuda.current_stream().cuda_stream


def set_wait_limit(polls: int) -> int:
    """Bound the device-side waits of later launches to `polls` polls (<= 0:
    the kernels' defaults); returns the previous setting."""
    return int(load().ek_set_wait_limit(int(polls)))


def device_info() -> tuple[int, str]:
    lib = load()
    n = ctypes.c_int(0)
    buf = ctypes.create_string_buffer(64)
    rc = lib.ek_device_info(ctypes.byref(n), buf, 64)
    if rc != 0:
        raise HipKernelError("ek_device_info", rc, "")
    return n.value, buf.value.decode()
