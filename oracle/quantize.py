"""Oracle: per-channel asymmetric INT4 quantization and nibble packing.

Test infrastructure only (see ``oracle/__init__.py``).

Restates, op for op in float32, the reference quantizer
``src/quantize_int4_ref.py:46-84``:

    mn, mx  = min / max over every axis but the last           (:54-56)
    range   = maximum(mx - mn, float32(1e-8))                   (:65-66)
    scale   = range / 15                                        (:67)
    zp      = -mn / scale                                       (:70)
    q       = clip(round_half_even((x - mn) / scale), 0, 15)    (:74-75)

and the storage format ``src/int4_pack.py:14-56`` (even channel in the low
nibble, odd channel in the high nibble, odd widths zero-padded).

Pinned by (tests/test_oracle_quantize.py): the reference's known-answer test
(scales 10/15, tests/test_quantization.py:46-66), a constructed half-way tie
that separates round-half-even from round-half-up, the uniform-input case
(tests/test_quantization.py:89-103), the round-trip bound |x - dq(q(x))| <=
scale/2 (tests/test_quantization.py:21-44), the packing KAT [0,15,15,0,7,8]
and shapes (tests/test_int4_pack.py:12-61), exact agreement with the
independent C restatement in oracle/c, and the partial-group rule (a partial
group reduces over its own rows only, tests/test_perplexity_harness.py:122-131).
"""

import numpy as np

#: The floor on the per-channel range. NumPy casts the Python scalar 1e-8 to
#: the array's float32 dtype (NEP 50 under NumPy 2; value-based casting keeps
#: float32 under NumPy 1.x), so the floor is float32(1e-8).
RANGE_FLOOR = np.float32(1e-8)
LEVELS = np.float32(15.0)


def quantize_int4_ref(kv, per_channel=True):
    """One scale group over all leading axes; returns (q u8, scale, zp).

    reference: src/quantize_int4_ref.py:23-84. ``per_channel=False`` reduces
    over the last axis instead (reference :57-61).
    """
    kv = np.asarray(kv)
    if kv.ndim < 2:
        raise AssertionError(f"KV must be at least 2D, got {kv.ndim}D")
    if kv.dtype not in (np.float32, np.float16):
        raise AssertionError(f"Expected FP32/FP16, got {kv.dtype}")
    x = kv.astype(np.float32)

    if per_channel:
        axes = tuple(range(x.ndim - 1))
    else:
        axes = (x.ndim - 1,)
    lo = x.min(axis=axes, keepdims=True)
    hi = x.max(axis=axes, keepdims=True)

    span = np.maximum(hi - lo, RANGE_FLOOR)          # float32 throughout
    scale = span / LEVELS
    zp = (-lo) / scale
    bins = np.round((x - lo) / scale)                # half to even
    q = np.clip(bins, 0, 15).astype(np.uint8)

    scale = np.squeeze(scale, axis=axes)
    zp = np.squeeze(zp, axis=axes)
    return q, scale, zp


def dequantize_int4_ref(q, scale, zp, target_shape=None, per_channel=True):
    """k = q*scale - zp*scale in float32: two rounded products, then a subtract.

    reference: src/quantize_int4_ref.py:87-136 (the expression is :131; the
    attention oracle uses the same one at src/flash_decode_ref.py:92).
    """
    qf = np.asarray(q).astype(np.float32)
    s = np.asarray(scale).astype(np.float32)
    z = np.asarray(zp).astype(np.float32)
    if per_channel:
        while s.ndim < qf.ndim:
            s = s[np.newaxis]
            z = z[np.newaxis]
    else:
        while s.ndim < qf.ndim:
            s = s[..., np.newaxis]
            z = z[..., np.newaxis]
    out = qf * s - z * s
    if target_shape is not None:
        out = out.reshape(target_shape)
    return out


def quantize_and_dequantize_ref(kv, per_channel=True):
    """reference: src/quantize_int4_ref.py:139-158."""
    q, s, z = quantize_int4_ref(kv, per_channel=per_channel)
    return q, s, z, dequantize_int4_ref(q, s, z, target_shape=np.shape(kv),
                                        per_channel=per_channel)


def pack_int4(q):
    """Two nibbles per byte along the last axis; odd widths zero-padded.

    reference: src/int4_pack.py:14-29.
    """
    q = np.asarray(q)
    if q.dtype != np.uint8:
        raise AssertionError(f"expected uint8, got {q.dtype}")
    if q.size and int(q.max()) > 15:
        raise AssertionError("values must fit in 4 bits")
    if q.shape[-1] % 2:
        q = np.concatenate([q, np.zeros(q.shape[:-1] + (1,), np.uint8)], axis=-1)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed, last_dim):
    """Inverse of pack_int4, keeping ``last_dim`` values. reference: src/int4_pack.py:32-47."""
    p = np.asarray(packed)
    if p.dtype != np.uint8:
        raise AssertionError("expected uint8")
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out[..., :last_dim]


def packed_nbytes(shape):
    """Bytes of the packed form of an unpacked shape. reference: src/int4_pack.py:50-56."""
    n = (int(shape[-1]) + 1) // 2
    for d in shape[:-1]:
        n *= int(d)
    return n


def quantize_groups_ref(k, seq_lens, group_size=128):
    """Grouped quantization of a batch of key streams.

    ``k`` is float32 [B, H, T, D]; ``seq_lens`` int [B]. For every
    (b, h, g) the rows ``k[b, h, g*group : min((g+1)*group, seq_lens[b])]``
    are quantized as one group by :func:`quantize_int4_ref` -- a partial last
    group uses only its own valid rows (reference
    tests/test_perplexity_harness.py:122-131). Rows at or past seq_lens[b]
    are left as 0 in ``q``; groups with no valid rows leave scale = zp = 0.

    Returns q u8 [B, H, T, D] (unpacked), scale f32 [B, H, G, D],
    zp f32 [B, H, G, D] with G = ceil(T / group_size).
    """
    k = np.asarray(k, dtype=np.float32)
    B, H, T, D = k.shape
    G = (T + group_size - 1) // group_size
    q = np.zeros((B, H, T, D), np.uint8)
    scale = np.zeros((B, H, G, D), np.float32)
    zp = np.zeros((B, H, G, D), np.float32)
    for b in range(B):
        n = int(seq_lens[b])
        for g in range((n + group_size - 1) // group_size):
            r0, r1 = g * group_size, min((g + 1) * group_size, n)
            # Batched over heads: min/max and the elementwise steps are exact
            # per element, so reducing [H, rows, D] over the row axis gives
            # the same bits as H separate calls.
            blk = k[b, :, r0:r1, :]
            lo = blk.min(axis=1, keepdims=True)
            hi = blk.max(axis=1, keepdims=True)
            span = np.maximum(hi - lo, RANGE_FLOOR)
            s = span / LEVELS
            z = (-lo) / s
            q[b, :, r0:r1, :] = np.clip(np.round((blk - lo) / s), 0, 15).astype(np.uint8)
            scale[b, :, g, :] = s[:, 0, :]
            zp[b, :, g, :] = z[:, 0, :]
    return q, scale, zp
