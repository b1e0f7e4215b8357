"""ctypes binding of `libomnia_hip.so`, the C ABI declared in `include/omnia_hip.h`.

The library is loaded once per process from the package directory. Nothing here falls
back to another implementation: a missing library raises `LibraryMissing`, a rejected
argument raises `ValueError` and a failed launch `RuntimeError`, each carrying the text
of `omnia_last_error()`.
"""

from __future__ import annotations

import ctypes
import errno
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent.parent / "libomnia_hip.so"
ABI_VERSION = 15

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

# name -> (restype, argtypes); must match include/omnia_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "omnia_abi_version": (_I32, []),
    "omnia_last_error": (ctypes.c_char_p, []),
    "omnia_add_rms_norm": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "omnia_rope_angle_atlas": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _P]),
    "omnia_rope_angle_atlas_fp32": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _P]),
    "omnia_stream_copy": (_I32, [_P, _P, _I64, _I32, _P]),
    "omnia_qk_norm_rope": (
        _I32,
        [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64,
         _I64, _I64, _F32, _F32, _P],
    ),
    "omnia_rope_epilogue": (
        _I32, [_P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _F32, _F32, _P]
    ),
    "omnia_swiglu": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _P]),
    "omnia_gate_softplus": (_I32, [_P, _I64, _P, _P, _P, _I64, _I64, _P]),
    "omnia_gated_activations": (
        _I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _P]
    ),
    "omnia_softmax_topk": (_I32, [_P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "omnia_softmax_topk_slots": (_I32, [_P, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P, _P]),
    "omnia_router_pack_bytes": (_I64, [_I64, _I64]),
    "omnia_pack_router_weight": (_I32, [_P, _I64, _I64, _P, _P]),
    "omnia_residual_rms_router": (
        _I32,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _P, _P, _P, _P],
    ),
    "omnia_sigmoid_topk": (_I32, [_P, _I64, _I32, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "omnia_residual_rms_router_sigmoid": (
        _I32,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _P, _P, _P, _P, _P],
    ),
    "omnia_moe_gate_up": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "omnia_moe_down_combine": (
        _I32, [_P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P]
    ),
    "omnia_moe_gate_up_affine": (
        _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _F32, _P, _P, _P, _I64,
               _I64, _P, _P]
    ),
    "omnia_moe_down_combine_affine": (
        _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64,
               _I64, _P, _P]
    ),
    "omnia_moe_gate_up_mxfp4": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _F32, _P, _P]),
    "omnia_moe_down_combine_mxfp4": (
        _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P]
    ),
    "omnia_moe_gate_up_nvfp4": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "omnia_moe_down_combine_nvfp4": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "omnia_attention_sink_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "omnia_attention_sink_decode": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _F32, _P, _I64,
                                           _P, _P]),
    "omnia_moe_down_combine_nvfp4_shared": (_I32, [_P, _P, _P, _I64, _P, _P, _I64, _I64, _P, _P, _I64, _I64, _P,
                                                   _P, _P]),
    "omnia_moe_gate_up_nvfp4_ordinal": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "omnia_dense_gate_up_swiglu": (_I32, [_P, _P, _I64, _I64, _P, _P]),
    "omnia_dense_down_residual": (_I32, [_P, _P, _P, _I64, _I64, _P, _P]),
    "omnia_attention_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "omnia_attention_decode": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P, _P, _I64,
                                      _I64, _P, _I64, _I64, _I64, _I64, _F32, _F32, _P, _I64,
                                      _P, _P]),
    "omnia_attention_decode_noalloc": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P, _P,
                                              _I64, _I64, _P, _I64, _I64, _I64, _I64, _F32, _F32,
                                              _P, _P]),
    "omnia_embed_atlas": (
        _I32,
        [_P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
    ),
}


class LibraryMissing(RuntimeError):
    """`libomnia_hip.so` is not built (or not loadable) in this tree."""


_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded library, with every declared signature bound."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.exists():
            raise LibraryMissing(
                f"{LIBRARY_PATH} is not built; run `python __graft_entry__.py` or "
                "`python mlx-omnia_amd/build.py` first"
            )
        # torch ships its own libamdhip64.so.7; importing it first makes this library's
        # libamdhip64.so.7 dependency bind to that same runtime instance, so torch's
        # stream handles are valid in our launches (one HIP runtime per process).
        import torch  # noqa: F401

        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            raise LibraryMissing(f"cannot load {LIBRARY_PATH}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.omnia_abi_version()
        if version != ABI_VERSION:
            raise LibraryMissing(f"ABI version {version}, expected {ABI_VERSION}")
        _library = lib
        return lib


def available() -> bool:
    try:
        library()
    except LibraryMissing:
        return False
    return True


def last_error() -> str:
    raw = library().omnia_last_error()
    return raw.decode() if raw else ""


def call(name: str, *args: object) -> None:
    """Invoke one entry point and turn a non-zero return code into an exception."""
    rc = getattr(library(), name)(*args)
    if rc == 0:
        return
    message = f"{name}: {last_error()} (code {rc})"
    if rc == -errno.EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)
