"""Device dequantization (fdi4_dequantize_int4, flash_decode_int4.dequantize_int4)
bit for bit against the oracle's dequantize_int4_ref (reference
src/quantize_int4_ref.py:87-136): per-channel and per-row scales, one value
per byte and nibble-packed rows (odd channel counts), NumPy and torch inputs,
target_shape, the C ABI through ctypes. The data are chosen so that the
contracted form fma(q, s, -(zp*s)) differs from the reference's two rounded
products on some elements, so a fused evaluation would fail the tests."""

import ctypes

import numpy as np
import pytest

from oracle import dequantize_int4_ref, pack_int4, quantize_int4_ref

pytestmark = pytest.mark.gpu


def _fused_differs(q, s, z):
    """True when fma(q, s, -(z*s)), rounded once, differs from the oracle's
    q*s - z*s on at least one element (q*s and the difference formed exactly
    in float64, which holds both without rounding at these magnitudes)."""
    qf = q.astype(np.float64)
    zs = (z.astype(np.float32) * s.astype(np.float32)).astype(np.float64)
    fused = (qf * s.astype(np.float64) - zs).astype(np.float32)
    return bool((fused != dequantize_int4_ref(q, s, z)).any())


@pytest.mark.parametrize("shape", [(1, 1), (7, 5), (512, 128), (4, 33, 64), (3, 2, 16, 128)])
def test_per_channel_matches_oracle(shape):
    from flash_decode_int4 import dequantize_int4
    kv = np.random.RandomState(sum(shape)).randn(*shape).astype(np.float32) * 3.7
    q, s, z = quantize_int4_ref(kv)
    want = dequantize_int4_ref(q, s, z, target_shape=shape)
    got = dequantize_int4(q, s, z, target_shape=shape)
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, want)


def test_contracted_form_would_be_caught():
    rng = np.random.RandomState(5)
    kv = rng.randn(512, 128).astype(np.float32) * 3.7
    q, s, z = quantize_int4_ref(kv)
    assert _fused_differs(q, s, z)


def test_per_row_scales_match_oracle():
    from flash_decode_int4 import dequantize_int4
    rng = np.random.RandomState(11)
    q = rng.randint(0, 16, size=(6, 40, 96)).astype(np.uint8)
    s = rng.uniform(0.01, 2.0, size=(6, 40)).astype(np.float32)
    z = rng.uniform(0.0, 15.0, size=(6, 40)).astype(np.float32)
    assert _fused_differs(q, s[..., None], z[..., None])
    want = dequantize_int4_ref(q, s, z, per_channel=False)
    np.testing.assert_array_equal(dequantize_int4(q, s, z, per_channel=False), want)


def test_full_and_grouped_scale_shapes():
    """Scales of the output's own shape, and grouped [G, 1, D] scales that
    broadcast over rows within a group."""
    from flash_decode_int4 import dequantize_int4
    rng = np.random.RandomState(12)
    q = rng.randint(0, 16, size=(4, 32, 64)).astype(np.uint8)
    s = rng.uniform(0.01, 2.0, size=q.shape).astype(np.float32)
    z = rng.uniform(0.0, 15.0, size=q.shape).astype(np.float32)
    np.testing.assert_array_equal(dequantize_int4(q, s, z), dequantize_int4_ref(q, s, z))
    s3, z3 = s[:, :1], z[:, :1]
    np.testing.assert_array_equal(dequantize_int4(q, s3, z3), dequantize_int4_ref(q, s3, z3))


@pytest.mark.parametrize("C", [1, 7, 64, 127, 128])
def test_packed_rows_match_oracle(C):
    from flash_decode_int4 import dequantize_int4
    rng = np.random.RandomState(C)
    kv = rng.randn(300, C).astype(np.float32)
    q, s, z = quantize_int4_ref(kv)
    want = dequantize_int4_ref(q, s, z)
    got = dequantize_int4(pack_int4(q), s, z, packed=True, num_channels=C)
    np.testing.assert_array_equal(got, want)


def test_full_byte_values_like_astype():
    """One value per byte: the whole byte is the value (the reference's
    astype(float32)), not its low nibble."""
    from flash_decode_int4 import dequantize_int4
    q = np.arange(256, dtype=np.uint8).reshape(4, 64)
    s = np.full(64, 0.5, np.float32)
    z = np.full(64, 2.0, np.float32)
    np.testing.assert_array_equal(dequantize_int4(q, s, z), dequantize_int4_ref(q, s, z))


def test_torch_tensors_stay_on_the_gpu():
    import torch
    from flash_decode_int4 import dequantize_int4
    rng = np.random.RandomState(13)
    kv = rng.randn(1000, 128).astype(np.float32)
    q, s, z = quantize_int4_ref(kv)
    got = dequantize_int4(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(),
                          torch.from_numpy(z).cuda())
    assert isinstance(got, torch.Tensor) and got.is_cuda and got.dtype == torch.float32
    np.testing.assert_array_equal(got.cpu().numpy(), dequantize_int4_ref(q, s, z))


def test_device_quantizer_round_trip():
    """ops.quantize_int4 then dequantize_int4 on the GPU equals the oracle's
    quantize_and_dequantize (src/quantize_int4_ref.py:139-158) and stays
    within half a scale step of the input."""
    import torch
    from flash_decode_int4 import dequantize_int4, ops
    from oracle import quantize_and_dequantize_ref
    kv = np.random.RandomState(14).randn(2048, 128).astype(np.float32)
    q, s, z = ops.quantize_int4(torch.from_numpy(kv).cuda())
    got = dequantize_int4(q, s, z).cpu().numpy()
    np.testing.assert_array_equal(got, quantize_and_dequantize_ref(kv)[3])
    assert (np.abs(got - kv) <= s.cpu().numpy() / 2 + 1e-6).all()


def test_c_abi_through_ctypes_with_strides():
    """fdi4_dequantize_int4 with padded row strides (q and out) and
    per-channel scales given as strides (0, 1)."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    rng = np.random.RandomState(15)
    rows, C = 333, 96
    q_np = rng.randint(0, 16, size=(rows, C)).astype(np.uint8)
    s_np = rng.uniform(0.01, 2.0, size=C).astype(np.float32)
    z_np = rng.uniform(0.0, 15.0, size=C).astype(np.float32)
    qbuf = torch.zeros(rows, C + 32, dtype=torch.uint8, device="cuda")
    qbuf[:, :C] = torch.from_numpy(q_np).cuda()
    s, z = torch.from_numpy(s_np).cuda(), torch.from_numpy(z_np).cuda()
    out = torch.full((rows, C + 8), -1.0, device="cuda")
    rc = lib.fdi4_dequantize_int4(ctypes.c_void_p(qbuf.data_ptr()), rows, C, qbuf.stride(0), 0,
                                  ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(z.data_ptr()),
                                  0, 1, ctypes.c_void_p(out.data_ptr()), out.stride(0),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    capi.check(rc, "dequantize_int4")
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    np.testing.assert_array_equal(o[:, :C], dequantize_int4_ref(q_np, s_np, z_np))
    assert (o[:, C:] == -1.0).all()                     # row padding untouched
