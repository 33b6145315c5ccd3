"""gdn_18646_amd — Gated DeltaNet hot paths for AMD Instinct MI355X (gfx950).

Native pieces (built in-tree by ``gdn_18646_amd._build``):

* ``libgdn_amd.so`` — hand-written HIP kernels behind the C ABI declared in
  ``include/gdn_amd.h`` (decode, chunked prefill, varlen prefill, RMSNorm,
  projection + conv + SiLU);
* ``_gdn_ext`` — a thin torch binding that re-exports the reference project's
  module API over that ABI.

``compile_kernels()`` returns the same ``dict(rmsnorm, proj, prefill,
decode)`` of modules that the reference's ``bench_gdn.compile_kernels()``
returns (``bench_gdn.py:25-45``), so callers written against the reference
work unchanged.  There is no fallback: if the native code is missing, these
functions raise.
"""

import os

__all__ = ["compile_kernels", "native_extension", "ExtensionMissing", "LIB_PATH", "EXT_DIR"]

EXT_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(EXT_DIR, "libgdn_amd.so")


class ExtensionMissing(ImportError):
    """The HIP library or its binding has not been built."""


def native_extension():
    """Import and return the ``_gdn_ext`` binding module (raises if unbuilt)."""
    import torch  # noqa: F401  -- torch's HIP runtime must be loaded first

    try:
        from . import _gdn_ext
    except ImportError as exc:  # pragma: no cover - exercised only when unbuilt
        raise ExtensionMissing(
            "gdn_18646_amd native code is not built: run `python -m gdn_18646_amd._build` "
            f"(or __graft_entry__.build()) first ({exc})") from exc
    return _gdn_ext


def compile_kernels():
    """The four kernel modules keyed as the reference's ``compile_kernels()``.

    Nothing is compiled at call time (the reference JIT-built here); the
    prebuilt in-tree extension is imported.
    """
    ext = native_extension()
    return dict(rmsnorm=ext.rmsnorm, proj=ext.proj, prefill=ext.prefill, decode=ext.decode)
