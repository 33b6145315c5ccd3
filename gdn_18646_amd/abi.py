"""ctypes view of libgdn_amd.so's C ABI (include/gdn_amd.h).

This is how a non-torch host (or a test) binds the library directly: every
entry point gets its argtypes/restype from the header's declarations.
``call(name, *args)`` raises ``GdnError`` with the library's message on a
non-zero status.  Device pointers are plain integers (e.g.
``tensor.data_ptr()``), streams are ``hipStream_t`` handles as integers.
"""

import ctypes

from . import LIB_PATH, ExtensionMissing

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes), in declaration order of include/gdn_amd.h
SIGNATURES = {
    "gdn_abi_version": (_I, []),
    "gdn_status_string": (ctypes.c_char_p, [_I]),
    "gdn_last_error": (ctypes.c_char_p, []),
    "gdn_decode_hip": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _I, _P]),
    "gdn_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "gdn_prefill_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _F, _P, _P,
                             _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_prefill_tm_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _F, _P, _P,
                                _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_prefill_noalloc_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _F, _P, _P,
                                     _I, _I, _I, _I, _I, _P]),
    "gdn_prefill_intra_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _F, _P, _P,
                                   _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_prefill_state_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _F, _P, _P,
                                   _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_prefill_varlen_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "gdn_prefill_varlen_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _I, _I, _P, _F, _P, _P,
                                    _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_prefill_varlen_tm_hip": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, _P, _I, _I, _P, _F, _P, _P,
                                       _I, _I, _I, _I, _P, _SZ, _P]),
    "gdn_rmsnorm_hip": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "gdn_proj_conv_silu_hip": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "gdn_in_proj_hip": (_I, [_P] * 14 + [_I] * 7 + [_P]),
    "gdn_in_proj_varlen_hip": (_I, [_P, _P, _P, _P, _I] + [_P] * 11 + [_I] * 6 + [_P]),
    "gdn_decode_conv_step_hip": (_I, [_P] * 12 + [_I] * 6 + [_P]),
    "gdn_decode_in_proj_hip": (_I, [_P, _P, _F] + [_P] * 11 + [_I] * 6 + [_P]),
    "gdn_decode_out_proj_hip": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "gdn_layer_decode_step_hip": (_I, [_P, _P, _F] + [_P] * 10 + [_F] + [_P] * 8 + [_I] * 6 + [_P]),
}

STATUS = {0: "GDN_OK", 1: "GDN_ERR_INVALID_ARGUMENT", 2: "GDN_ERR_UNSUPPORTED",
          3: "GDN_ERR_WORKSPACE", 4: "GDN_ERR_HIP"}


class GdnError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None


def load(path=LIB_PATH):
    """Open the library (once) and attach the header's signatures."""
    global _lib
    if _lib is not None:
        return _lib
    try:
        lib = ctypes.CDLL(path)
    except OSError as exc:
        raise ExtensionMissing(f"cannot load {path}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    """Call an int-returning entry point; raise GdnError on failure."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        raise GdnError(st, lib.gdn_last_error().decode())
    return st
