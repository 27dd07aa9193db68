"""flash_decode_int4 -- INT4 key-cache quantization and fused INT4 flash decoding
for AMD Instinct MI355X (gfx950).

Drop-in for the reference package (src/__init__.py, installed as
``flash_decode_int4``): ``ops`` (quantize_int4, flash_decode, prepare_*),
``int4_pack`` (pack_int4, unpack_int4, packed_nbytes) and
``vllm_integration.INT4PagedKVCache``. The computation runs in hand-written
HIP kernels (libfdi4.so, C ABI in include/fdi4.h) reached through the thin
torch binding ``_C``; there is no CPU implementation in this package.
"""

__version__ = "0.1.0"

from .int4_pack import pack_int4, unpack_int4, packed_nbytes  # noqa: F401
from ._lib import binding_available, gpu_available  # noqa: F401

HAS_EXTENSION = binding_available()
HAS_HIP = HAS_EXTENSION and gpu_available()
HAS_CUDA = HAS_HIP

__all__ = [
    "pack_int4",
    "unpack_int4",
    "packed_nbytes",
    "HAS_EXTENSION",
    "HAS_HIP",
    "HAS_CUDA",
    "backend_info",
]


def backend_info():
    """Print what is available. reference: src/__init__.py:79-84."""
    print(f"HIP extension built: {'yes' if HAS_EXTENSION else 'no'}")
    print(f"GPU visible:         {'yes' if gpu_available() else 'no'}")
