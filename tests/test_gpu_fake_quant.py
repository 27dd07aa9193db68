"""Device quantize-dequantize of keys for quality studies (reference
scripts/validate_llama.py:126-154).

* bit-exact with the oracle for float32, float16 and bfloat16 keys, both
  roundings, both scale forms, partial blocks, head sizes whose 16-byte
  vectors do not divide the workgroup, blocks held in registers and blocks
  read twice, block size 1, strided and misaligned views;
* each scale form equals the study's formula as eager torch operations on
  the GPU (a Python-scalar divisor there is a reciprocal multiply);
* the C ABI entry point gives the binding's bytes and rejects misaligned rows;
* at full size (8 x 32 x 2048 x 128 float32 keys): block size 1 is the
  identity under half-up, and sampled streams match the oracle.
"""

import ctypes

import numpy as np
import pytest

from oracle import bf16_bits, fake_quantize_keys_ref

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float16", "bfloat16"]
ROUNDINGS = ["half_up", "half_even"]


def _torch_dtype(name):
    import torch
    return getattr(torch, name)


def _keys(shape, dtype, seed, ties=False):
    import torch
    g = torch.Generator().manual_seed(seed)
    if ties:
        # Channels spanning exactly 15 with half-integer values: every
        # quotient is an integer or a tie.
        x = torch.randint(0, 31, shape, generator=g).float() / 2
        x[:, :, 0::5] = 0.0
        x[:, :, 2::5] = 15.0
    else:
        x = torch.randn(shape, generator=g) * torch.rand(shape[-1], generator=g).mul(3).add(0.2)
    return x.to(_torch_dtype(dtype)).cuda()


def _bits(t):
    import torch
    t = t.contiguous().cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def _expected_bits(k, block, rounding, scale_op="divide"):
    """Oracle float32 result cast to k's dtype, as bit patterns."""
    import torch
    dq = fake_quantize_keys_ref(k.float().cpu().numpy(), block, rounding, scale_op)
    if k.dtype == torch.float32:
        return dq.view(np.uint32)
    if k.dtype == torch.float16:
        return dq.astype(np.float16).view(np.uint16)
    return bf16_bits(dq)


def _fq(*a, **kw):
    from flash_decode_int4.quality import fake_quantize_keys
    return fake_quantize_keys(*a, **kw)


SHAPES = [
    # (B, H, S, D, block, ties)
    ((1, 2, 300, 64), 128, False),       # partial last block
    ((2, 4, 513, 128), 256, False),
    ((1, 1, 1, 128), 256, False),        # one row
    ((2, 3, 1000, 80), 256, False),      # 20 / 10 vectors per row: idle threads
    ((1, 2, 2048, 256), 256, False),     # float32: 64 sweeps, half read twice
    ((1, 2, 700, 128), 1000, False),     # one block longer than the register cache
    ((2, 2, 64, 128), 1, False),         # block size 1
    ((1, 1, 40, 512), 16, False),        # widest head
    ((2, 2, 384, 128), 128, True),       # ties everywhere
    ((1, 3, 257, 64), 256, True),
]


@pytest.mark.parametrize("scale_op", ["divide", "reciprocal"])
@pytest.mark.parametrize("rounding", ROUNDINGS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,block,ties", SHAPES)
def test_bit_exact_with_oracle(shape, block, ties, dtype, rounding, scale_op):
    import torch
    k = _keys(shape, dtype, seed=sum(shape) + block, ties=ties)
    out = _fq(k, block, rounding, scale_op)
    assert out.shape == k.shape and out.dtype == k.dtype
    np.testing.assert_array_equal(_bits(out), _expected_bits(k, block, rounding, scale_op))
    if ties:
        # The two roundings must differ on tie-rich input.
        other = _fq(k, block, "half_even" if rounding == "half_up" else "half_up", scale_op)
        assert not torch.equal(other, out)


def _eager_chain(k, block, divisor):
    """The harness's formula as eager torch operations on the GPU (pad the
    last block with its last row, block extremes, bins, dequantize, cast)."""
    import torch
    b, h, s, d = k.shape
    nb = -(-s // block)
    x = k.float()
    if nb * block != s:
        x = torch.cat([x, x[:, :, -1:].expand(b, h, nb * block - s, d)], dim=2)
    x = x.reshape(b, h, nb, block, d)
    lo = x.amin(dim=3, keepdim=True)
    step = (x.amax(dim=3, keepdim=True) - lo).clamp_min(1e-8) / divisor
    q = torch.floor((x - lo) / step + 0.5).clamp_(0.0, 15.0)
    return (q * step + lo).reshape(b, h, nb * block, d)[:, :, :s].to(k.dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_scale_ops_match_eager_torch_on_the_gpu(dtype):
    """Eager torch on the GPU divides by a Python scalar through its float32
    reciprocal (scale_op='reciprocal'); by a tensor it divides (scale_op=
    'divide'). Each kernel mode reproduces its eager form bit for bit, and the
    two forms differ on this input."""
    import torch
    k = _keys((2, 8, 700, 128), dtype, seed=21)
    recip = _fq(k, 256, "half_up", "reciprocal")
    div = _fq(k, 256, "half_up", "divide")
    assert torch.equal(recip, _eager_chain(k, 256, 15.0))
    assert torch.equal(div, _eager_chain(k, 256, torch.tensor(15.0, device="cuda")))
    assert not torch.equal(recip, div)


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_view(dtype):
    """Keys as attention holds them before the transpose: [B, S, H, D] viewed as
    [B, H, S, D] (row stride H*D)."""
    base = _keys((2, 300, 4, 64), dtype, seed=11)
    k = base.transpose(1, 2)
    assert not k.is_contiguous()
    out = _fq(k, 128)
    np.testing.assert_array_equal(_bits(out), _expected_bits(k, 128, "half_up"))


def test_misaligned_view_is_copied():
    import torch
    flat = torch.randn(1 + 2 * 3 * 50 * 64, device="cuda")
    k = flat[1:].view(2, 3, 50, 64)            # 4 bytes past a 16-byte boundary
    assert k.data_ptr() % 16 != 0
    out = _fq(k, 32, "half_even")
    np.testing.assert_array_equal(_bits(out), _expected_bits(k, 32, "half_even"))


def test_preallocated_out_and_empty():
    import torch
    k = _keys((1, 2, 100, 64), "float16", seed=12)
    out = torch.empty_like(k)
    assert _fq(k, 64, out=out) is out
    np.testing.assert_array_equal(_bits(out), _expected_bits(k, 64, "half_up"))
    e = torch.empty(1, 2, 0, 64, device="cuda")
    assert _fq(e).shape == e.shape


def test_overlapping_out_is_rejected():
    import torch
    flat = torch.zeros(2 * 2 * 64 * 64, device="cuda")
    k = flat[:2 * 64 * 64].view(1, 2, 64, 64)
    with pytest.raises(ValueError, match="overlap"):
        _fq(k, 64, out=k)
    with pytest.raises(ValueError, match="overlap"):
        _fq(k, 64, out=flat[64 * 64:3 * 64 * 64].view(1, 2, 64, 64))
    out = flat[2 * 64 * 64:].view(1, 2, 64, 64)          # adjacent, not overlapping
    assert _fq(k, 64, out=out) is out


def test_argument_errors():
    import torch
    k = torch.zeros(1, 1, 8, 64, device="cuda")
    with pytest.raises(ValueError):
        _fq(k, 8, "nearest")
    with pytest.raises(ValueError):
        _fq(k, 0)
    with pytest.raises(ValueError):
        _fq(k, 8, "half_up", "multiply")
    with pytest.raises(ValueError):
        _fq(torch.zeros(1, 8, 64, device="cuda"))
    with pytest.raises(ValueError):
        _fq(torch.zeros(1, 1, 8, 100, dtype=torch.float16, device="cuda"))  # 200-byte rows
    with pytest.raises(TypeError):
        _fq(k.double())
    with pytest.raises(RuntimeError):
        _fq(k.cpu())


def test_c_abi_matches_binding_and_rejects_misaligned_rows():
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    k = _keys((2, 3, 200, 128), "bfloat16", seed=13)
    want = _fq(k, 64, "half_even")
    out = torch.empty_like(k)
    s = torch.cuda.current_stream().cuda_stream
    rc = lib.fdi4_fake_quantize(k.data_ptr(), capi.K_BF16, 2, 3, 200, 128, k.stride(0),
                                k.stride(1), k.stride(2), out.data_ptr(), out.stride(0),
                                out.stride(1), out.stride(2), 64, capi.ROUND_HALF_EVEN,
                                capi.SCALE_DIVIDE, ctypes.c_void_p(s))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    # Rows that are not 16-byte multiples are refused before any launch.
    rc = lib.fdi4_fake_quantize(k.data_ptr(), capi.K_BF16, 2, 3, 200, 100, k.stride(0),
                                k.stride(1), k.stride(2), out.data_ptr(), out.stride(0),
                                out.stride(1), out.stride(2), 64, capi.ROUND_HALF_UP,
                                capi.SCALE_DIVIDE, ctypes.c_void_p(s))
    assert rc == 1
    rc = lib.fdi4_fake_quantize(k.data_ptr() + 2, capi.K_BF16, 2, 3, 200, 128, k.stride(0),
                                k.stride(1), k.stride(2), out.data_ptr(), out.stride(0),
                                out.stride(1), out.stride(2), 64, capi.ROUND_HALF_UP,
                                capi.SCALE_DIVIDE, ctypes.c_void_p(s))
    assert rc == 1


def test_full_size_identity_and_sampled_streams():
    """8 x 32 x 2048 x 128 float32 keys (268 MB)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(5)
    k = torch.randn(8, 32, 2048, 128, device="cuda", generator=g)
    assert torch.equal(_fq(k, 1, "half_up"), k)
    out = _fq(k, 256, "half_up")
    rng = np.random.RandomState(3)
    for _ in range(4):
        b, h = int(rng.randint(8)), int(rng.randint(32))
        kk = k[b:b + 1, h:h + 1]
        np.testing.assert_array_equal(_bits(out[b:b + 1, h:h + 1]),
                                      _expected_bits(kk, 256, "half_up"))
    del k, out
    torch.cuda.empty_cache()
