"""CPU oracle for the INT4 key quantizer and the fused INT4 flash-decode path.

TEST INFRASTRUCTURE ONLY. This package restates, in this project's own NumPy
and C code, the reference's CPU algorithm so that the HIP kernels can be
checked against it. Nothing in the product package
(``flash_decode_int4``) imports it. The only permitted callers are ``tests/``,
``__graft_entry__.smoke()`` (to verify the GPU result) and the ``cpu_baseline`` leg of
``bench.py`` (as the timed CPU baseline). It is never the thing measured on
the GPU and never a fallback.

Modules
-------
quantize   per-channel asymmetric INT4 quantizer, dequantizer, nibble packing
           (reference src/quantize_int4_ref.py:23-136, src/int4_pack.py:14-56)
attention  page-loop online softmax (reference src/flash_decode_ref.py:30-223),
           the float64 arbiter (reference tests/test_pallas_flash_decode.py:53-78)
           and the per-(sequence, kv-head) paged construction
fakequant  quantize-dequantize of key tensors in blocks (reference
           scripts/validate_llama.py:126-154; half-even form per block of
           src/quantize_int4_ref.py:139-158) and the bfloat16 rounding
pool       the paged oracle and the key re-quantization over every stream of a
           workload, spread over the host cores (results identical to the
           one-process functions)
cref       ctypes loader for the C restatement in ``oracle/c`` (quantizer,
           packing and a float64 attention arbiter), built by ``oracle/Makefile``

How each function is pinned (known answers, closed forms, invariants, brute
force) is recorded in the docstring of that function and exercised by
``tests/test_oracle_*.py``.
"""

from .quantize import (  # noqa: F401
    quantize_int4_ref,
    dequantize_int4_ref,
    quantize_and_dequantize_ref,
    pack_int4,
    unpack_int4,
    packed_nbytes,
    quantize_groups_ref,
)
from .attention import (  # noqa: F401
    online_softmax_ref,
    flash_decode_ref,
    online_softmax_fp32_ref,
    f64_attention,
    float32_floor,
    paged_decode_ref,
    paged_decode_f64,
)
from .fakequant import (  # noqa: F401
    fake_quantize_keys_ref,
    bf16_bits,
    bf16_bits_to_f32,
)
