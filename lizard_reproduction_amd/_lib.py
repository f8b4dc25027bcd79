"""ctypes binding of liblizard_hip.so (declared in include/lizard_hip.h).

The library is built in-tree by ``lizard_reproduction_amd.build``.  Loading
never falls back to anything: a missing library raises ``RuntimeError``.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "liblizard_hip.so")
ABI_VERSION = 15

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t

# name -> (restype, argtypes); must match include/lizard_hip.h
SIGNATURES = {
    "lz_abi_version": (_I, []),
    "lz_init": (_I, []),
    "lz_last_error": (ctypes.c_char_p, []),
    "lz_gla_fwd_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I, _I]),
    "lz_gla_fwd": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _S, _P]),
    "lz_gla_fwd_noalloc": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lz_gla_prefill": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _S,
                            _P]),
    "lz_gla_fwd_phi": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _S,
                            _P]),
    "lz_gla_decode_step": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "lz_gla_bwd_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I, _I]),
    "lz_gla_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                        _I, _I, _I, _I, _I, _I, _I, _I, _P, _S, _P, _S, _P]),
    "lz_swa_fwd": (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "lz_swa_decode_step": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "lz_swa_bwd_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "lz_swa_bwd": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I,
                        _I, _I, _I, _I, _I, _I, _F, _P, _S, _P]),
    "lz_layer_prologue_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I,
                                   _I, _I, _I, _I, _I, _I, _P]),
    "lz_layer_prologue_bwd_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I]),
    "lz_layer_prologue_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _S, _P]),
    "lz_layer_combine_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "lz_layer_combine_bwd_workspace_bytes": (_S, []),
    "lz_layer_combine_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _S, _P]),
}

_lib = None


def load(path=LIB_PATH):
    """Load the library once and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m lizard_reproduction_amd.build` "
            "(the HIP kernels have no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.lz_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(rc, what):
    """Raise RuntimeError with the library's message for a non-zero status."""
    if rc != 0:
        msg = _lib.lz_last_error().decode(errors="replace") if _lib is not None else ""
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")
