"""Oracle: INT4 quantize-dequantize ("fake quantization") of key tensors.

Test infrastructure only (see ``oracle/__init__.py``).

Restates, op for op in float32, fake_quantize_keys of the reference's
perplexity harness (``scripts/validate_llama.py:126-154``) for keys
[batch, heads, seq, head_dim] and blocks of ``block_size`` positions:

    x       = k.float()                                          (:141)
    (a partial last block is padded with its last row, :145-147 -- the
     extremes of the block's valid rows are unchanged by it)
    mn, mx  = min / max over the block's rows                    (:150-151)
    scale   = maximum(mx - mn, float32(1e-8)) / 15               (:152)
    q       = clip(floor((x - mn) / scale + 0.5), 0, 15)         (:153)
    dq      = q * scale + mn, cast back to k's dtype             (:154-155)

With ``scale_op="reciprocal"`` the scale is instead
maximum(mx - mn, 1e-8) * float32(1/15): eager torch on a GPU evaluates the
harness's ``/ 15.0`` (a tensor divided by a Python scalar) as a multiplication
by the float32 reciprocal, so a reference run on a GPU uses these scales.

And, with ``rounding="half_even"``, the stored scheme of the kernels:
``quantize_and_dequantize_ref`` (``src/quantize_int4_ref.py:139-158``) applied
per block, i.e. q = clip(round_half_even((x - mn)/scale), 0, 15),
zp = -mn/scale and dq = q*scale - zp*scale.

Pinned by (tests/test_oracle_fakequant.py): hand-derived known answers on a
scale-1 channel (0.5 ties: half-up 2.5 -> 3, half-even 2.5 -> 2); block size 1
is the identity under half-up (one row: mn = x, q = 0, dq = mn); the
half-even form equals per-block calls of the pinned quantize_int4_ref /
dequantize_int4_ref; bit-for-bit agreement with the independent C
restatement (``oracle/c``: ``oracle_fake_quantize``); |x - dq| <= scale/2 up to
the float32 rounding of the dequantization; and the dtype casts agree with
torch's float16 / bfloat16 conversions and the C bfloat16 rounding. The
reciprocal scale: float32(1/15) is the correctly rounded reciprocal (checked
against exact rational arithmetic), and the scales equal torch's CPU
evaluation of ``span * (1/15)`` with the factor as a float32 tensor.
"""

import numpy as np

from .quantize import LEVELS, RANGE_FLOOR

ROUNDINGS = ("half_up", "half_even")
SCALE_OPS = ("divide", "reciprocal")
#: float32(1/15), correctly rounded (float32 division of exact operands).
RECIP_15 = np.float32(1.0) / LEVELS


def fake_quantize_keys_ref(k, block_size=256, rounding="half_up", scale_op="divide"):
    """float32 result of the quantize-dequantize of k [B, H, S, D] (any float dtype).

    reference: scripts/validate_llama.py:126-154 (half_up);
    src/quantize_int4_ref.py:139-158 per block (half_even).
    """
    if rounding not in ROUNDINGS:
        raise ValueError(f"rounding must be one of {ROUNDINGS}, got {rounding!r}")
    if scale_op not in SCALE_OPS:
        raise ValueError(f"scale_op must be one of {SCALE_OPS}, got {scale_op!r}")
    x = np.asarray(k).astype(np.float32)
    if x.ndim != 4:
        raise ValueError("k must be [batch, heads, seq, head_dim]")
    if block_size < 1:
        raise ValueError("block_size must be >= 1")
    out = np.empty_like(x)
    s = x.shape[2]
    for start in range(0, s, block_size):
        xb = x[:, :, start:start + block_size]
        mn = xb.min(axis=2, keepdims=True)
        mx = xb.max(axis=2, keepdims=True)
        span = np.maximum(mx - mn, RANGE_FLOOR)
        scale = span / LEVELS if scale_op == "divide" else span * RECIP_15
        t = (xb - mn) / scale
        if rounding == "half_up":
            q = np.clip(np.floor(t + np.float32(0.5)), 0, 15)
            dq = q * scale + mn
        else:
            zp = (-mn) / scale
            q = np.clip(np.round(t), 0, 15)
            dq = q * scale - zp * scale
        out[:, :, start:start + block_size] = dq
    return out


def bf16_bits(x):
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16).

    NaN becomes the quiet NaN 0x7FC0. Ties go to the even upper half: the
    rounding adds 0x7FFF plus the low bit of the upper half, then truncates.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    r = r.astype(np.uint16)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r[nan] = np.uint16(0x7FC0)
    return r


def bf16_bits_to_f32(bits):
    """Exact widening of bfloat16 bit patterns to float32."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)
