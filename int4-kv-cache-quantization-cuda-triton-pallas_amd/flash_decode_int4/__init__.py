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
# The reference's availability flags (src/__init__.py:22-49). This package
# ships no NumPy reference implementations (quantize_int4_ref,
# dequantize_int4_ref, flash_decode_ref, online_softmax_ref are not part of
# it) and no Pallas/JAX backend, so the three are False; the device
# counterparts are ops.quantize_int4, dequantize_int4 and ops.flash_decode.
HAS_QUANT_REF = False
HAS_DECODE_REF = False
HAS_PALLAS = False


def dequantize_int4(q, scale, zp, target_shape=None, per_channel=True, packed=False,
                    num_channels=None):
    """INT4 values back to float32 on the GPU, bit-exact with the reference's
    dequantize_int4_ref (src/quantize_int4_ref.py:87-136); see
    ops.dequantize_int4."""
    from .ops import dequantize_int4 as _dequantize
    return _dequantize(q, scale, zp, target_shape=target_shape, per_channel=per_channel,
                       packed=packed, num_channels=num_channels)


__all__ = [
    "pack_int4",
    "unpack_int4",
    "packed_nbytes",
    "dequantize_int4",
    "HAS_EXTENSION",
    "HAS_HIP",
    "HAS_CUDA",
    "HAS_QUANT_REF",
    "HAS_DECODE_REF",
    "HAS_PALLAS",
    "backend_info",
]


def backend_info():
    """Print what is available. reference: src/__init__.py:79-84."""
    print(f"Quantization reference: {'yes' if HAS_QUANT_REF else 'no'} (not shipped)")
    print(f"Flash decode reference: {'yes' if HAS_DECODE_REF else 'no'} (not shipped)")
    print(f"HIP extension built:    {'yes' if HAS_EXTENSION else 'no'}")
    print(f"GPU visible:            {'yes' if gpu_available() else 'no'}")
    print(f"Pallas / JAX:           {'yes' if HAS_PALLAS else 'no'}")
