"""On-device INT4 fake quantization of keys, for quality studies.

Device form of the key quantize-dequantize of the reference's quality study
(``fake_quantize_keys``, scripts/validate_llama.py:126-154, with its block
size ``BLOCK_SIZE`` of :52). The quantize-dequantize runs in one HIP kernel
(``fdi4_fake_quantize``: one read and one write of the keys) instead of the
reference's chain of torch operations (pad, amin, amax, divide, floor,
clamp, multiply, add, cast), with the same float32 arithmetic. The study's
model driver (cache hook, sliding-window perplexity, weight and dataset
loading) is not part of this package.

Options beyond the reference's signature:

``rounding``  "half_up" is the study's rule (floor(t + 0.5), dq = q*scale +
              mn); "half_even" is the scheme the INT4 cache stores and the
              attention kernels dequantize (round half to even, dq = q*scale -
              zp*scale; reference src/quantize_int4_ref.py:139-158 per block),
              so a perplexity run can measure exactly what the kernels compute.
``scale_op``  "divide": scale = span / 15 with IEEE division, the reference's
              formula as NumPy and torch on the CPU evaluate it (its own tests
              run there); "reciprocal": scale = span * float32(1/15), what
              eager torch on a GPU computes for the same expression (a tensor
              divided by a Python scalar is multiplied by the reciprocal), for
              numbers identical to a reference run on a GPU. The two differ by
              one ulp in some scales, enough to move a value to the next bin.

Keys must be finite GPU tensors of float32, float16 or bfloat16; there is no
CPU path (the call raises without the HIP extension or a GPU).
"""

from typing import Optional

from ._lib import gpu_available, load_binding

#: Paged KV block size of the harness; scales are per (block, channel).
#: reference: scripts/validate_llama.py:52.
BLOCK_SIZE = 256

ROUNDING_MODES = {"half_up": 0, "half_even": 1}
SCALE_OPS = {"divide": 0, "reciprocal": 1}

_MAX_HEAD_DIM = 512


def _require_gpu_tensor(k) -> None:
    import torch
    if not isinstance(k, torch.Tensor):
        raise TypeError(f"k must be a torch tensor, got {type(k).__name__}")
    load_binding()  # raises with the reason when the extension is missing
    if not gpu_available():
        raise RuntimeError("fake_quantize_keys needs a visible GPU (torch.cuda.is_available() "
                           "is False); this package has no CPU path")
    if not k.is_cuda:
        raise RuntimeError("k must be a GPU (cuda device) tensor; this package has no CPU path")


def _byte_range(t):
    """[first, last) bytes a tensor's elements span."""
    if t.numel() == 0:
        return t.data_ptr(), t.data_ptr()
    span = sum((n - 1) * abs(st) for n, st in zip(t.shape, t.stride())) + 1
    return t.data_ptr(), t.data_ptr() + span * t.element_size()


def _aligned_rows(k):
    """k itself when its rows can be read as 16-byte vectors, else a contiguous copy."""
    esz = k.element_size()
    ok = (k.stride(-1) == 1 and k.data_ptr() % 16 == 0
          and all((k.stride(i) * esz) % 16 == 0 for i in range(3)))
    if ok:
        return k
    return k.contiguous() if not k.is_contiguous() else k.clone()


def fake_quantize_keys(k, block_size: int = BLOCK_SIZE, rounding: str = "half_up",
                       scale_op: str = "divide", out: Optional[object] = None):
    """INT4 quantize-dequantize of keys, matching the kernels' scheme.

    Args:
        k: torch tensor [batch, kv_heads, seq, head_dim] on the GPU -- the
           post-RoPE keys handed to Cache.update() -- float32, float16 or
           bfloat16, any strides with contiguous rows.
        block_size: positions per scale block (a partial last block uses its
           valid rows).
        rounding: "half_up" (the harness) or "half_even" (the stored scheme).
        scale_op: "divide" (IEEE span / 15) or "reciprocal" (span * (1/15),
           eager torch on a GPU).
        out: optional preallocated result (same shape and dtype, contiguous
           rows, not overlapping k).
    Returns:
        Tensor of k's shape and dtype holding the dequantized INT4 keys.
    reference: scripts/validate_llama.py:126-154.
    """
    import torch
    _require_gpu_tensor(k)
    if rounding not in ROUNDING_MODES:
        raise ValueError(f"rounding must be one of {tuple(ROUNDING_MODES)}, got {rounding!r}")
    if scale_op not in SCALE_OPS:
        raise ValueError(f"scale_op must be one of {tuple(SCALE_OPS)}, got {scale_op!r}")
    if k.dim() != 4:
        raise ValueError(f"k must be [batch, kv_heads, seq, head_dim], got shape {tuple(k.shape)}")
    if k.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError(f"k must be float32, float16 or bfloat16, got {k.dtype}")
    block_size = int(block_size)
    if block_size < 1:
        raise ValueError(f"block_size must be >= 1, got {block_size}")
    d = k.shape[-1]
    if d > _MAX_HEAD_DIM or (d * k.element_size()) % 16:
        raise ValueError(f"head_dim {d} is unsupported: rows of {d} x {k.element_size()} bytes "
                         f"must be a multiple of 16 bytes and head_dim <= {_MAX_HEAD_DIM}")
    if out is None:
        out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    elif out.shape != k.shape or out.dtype != k.dtype:
        raise ValueError("out must have k's shape and dtype")
    else:
        (k0, k1), (o0, o1) = _byte_range(k), _byte_range(out)
        if k0 < o1 and o0 < k1:
            raise ValueError("out must not overlap k")
    if k.numel() == 0:
        return out
    load_binding().fake_quantize(_aligned_rows(k), out, block_size, ROUNDING_MODES[rounding],
                                 SCALE_OPS[scale_op])
    return out
