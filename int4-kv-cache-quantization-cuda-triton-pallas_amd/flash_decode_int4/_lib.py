"""Loading of the native parts: the torch binding ``_C`` and ``libfdi4.so``.

There is no fallback. ``load_binding()`` raises ``RuntimeError`` with the
reason when the built extension is missing or does not import, and the ops
that need the GPU raise when no GPU is visible. Build with
``python -m flash_decode_int4._build``.
"""

import importlib
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libfdi4.so")

_binding = None
_binding_error = None


def load_binding():
    """Import and return the compiled torch binding (``flash_decode_int4._C``)."""
    global _binding, _binding_error
    if _binding is not None:
        return _binding
    if _binding_error is not None:
        raise RuntimeError(_binding_error)
    # A missing build is not remembered: a build in the same process (the
    # package is imported before it compiles) must be able to load it after.
    if not os.path.exists(os.path.join(PKG_DIR, "_C.so")) or not os.path.exists(LIB_PATH):
        raise RuntimeError("the HIP extension is not built (missing _C.so / libfdi4.so in "
                           f"{PKG_DIR}); run `python -m flash_decode_int4._build`")
    try:
        import torch  # noqa: F401  (the binding links against torch's libraries)
        _binding = importlib.import_module(__package__ + "._C")
    except Exception as exc:  # pragma: no cover - depends on the install
        _binding_error = f"the HIP extension failed to import: {exc!r}"
        raise RuntimeError(_binding_error) from exc
    return _binding


def binding_available() -> bool:
    try:
        load_binding()
        return True
    except RuntimeError:
        return False


def gpu_available() -> bool:
    try:
        import torch
        return bool(torch.cuda.is_available())
    except Exception:
        return False
