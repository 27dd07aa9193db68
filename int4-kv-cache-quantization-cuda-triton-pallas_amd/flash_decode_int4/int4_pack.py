"""INT4 nibble-packing storage format (host helpers).

Drop-in for the reference's src/int4_pack.py:14-56: two 4-bit values per byte
along the last axis, the even index in the low nibble and the odd index in
the high nibble; an odd-length last axis is zero-padded. This is exactly the
byte layout the device quantizer writes into key pages and the decode kernel
reads, so host-packed and device-packed bytes are interchangeable.

The device form of pack_int4 is ``flash_decode_int4.ops.pack_int4_device``.
"""

import numpy as np


def pack_int4(q: np.ndarray) -> np.ndarray:
    """Pack uint8 values in [0, 15] into nibbles along the last axis.

    reference: src/int4_pack.py:14-29 (asserts on dtype and range are kept).
    """
    q = np.asarray(q)
    assert q.dtype == np.uint8, f"expected uint8, got {q.dtype}"
    assert q.max(initial=0) <= 15, "values must fit in 4 bits"
    n = q.shape[-1]
    out = np.zeros(q.shape[:-1] + ((n + 1) // 2,), dtype=np.uint8)
    out[...] = q[..., 0::2]
    out[..., : n // 2] |= q[..., 1::2] << 4
    return out


def unpack_int4(packed: np.ndarray, last_dim: int) -> np.ndarray:
    """Recover one value per byte; keep the first ``last_dim`` values.

    reference: src/int4_pack.py:32-47.
    """
    packed = np.asarray(packed)
    assert packed.dtype == np.uint8
    out = np.empty(packed.shape[:-1] + (2 * packed.shape[-1],), dtype=np.uint8)
    np.bitwise_and(packed, 0x0F, out=out[..., 0::2])
    np.right_shift(packed, 4, out=out[..., 1::2])
    return out[..., :last_dim]


def packed_nbytes(shape: tuple) -> int:
    """Storage bytes of the packed form of ``shape``. reference: src/int4_pack.py:50-56."""
    total = (int(shape[-1]) + 1) // 2
    for d in shape[:-1]:
        total *= int(d)
    return total
