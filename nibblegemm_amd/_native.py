"""Loader for the compiled library (``lib/libnibblegemm_amd.so``) and its
CPython binding (``_binding``).

There is no fallback: if the native extension is missing, every kernel entry
point raises ``RuntimeError`` naming the build command.
"""
from __future__ import annotations

import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "lib", "libnibblegemm_amd.so")
ABI_VERSION = 14

_binding = None


def binding():
    """The CPython binding module; raises RuntimeError if it is not built."""
    global _binding
    if _binding is None:
        try:
            from . import _binding as b  # noqa: PLC0415
        except ImportError as exc:
            raise RuntimeError(
                "nibblegemm_amd native extension is not built "
                f"(expected {LIBRARY_PATH}); run `python -m nibblegemm_amd.build`"
            ) from exc
        if b.abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"nibblegemm_amd ABI mismatch: library {b.abi_version()}, package {ABI_VERSION}"
            )
        _binding = b
    return _binding


def is_built() -> bool:
    try:
        binding()
        return True
    except RuntimeError:
        return False
