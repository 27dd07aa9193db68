"""Pins of the oracle quantizer and packing (CPU).

Each test fails for a plausible mistake in the restatement: a wrong rounding
mode, a dropped range floor, a transposed reduction axis, swapped nibbles, a
partial group that borrows rows of its neighbour.
"""

import numpy as np
import pytest

from oracle import (dequantize_int4_ref, pack_int4, packed_nbytes, quantize_and_dequantize_ref,
                    quantize_groups_ref, quantize_int4_ref, unpack_int4)
from oracle import cref


class TestKnownAnswers:

    def test_per_channel_scales_known_answer(self):
        """reference tests/test_quantization.py:46-66: scales (11-1)/15 and (12-2)/15."""
        kv = np.array([[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]],
                       [[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]]], dtype=np.float32)
        q, scale, zp = quantize_int4_ref(kv)
        np.testing.assert_allclose(scale, [10.0 / 15.0, 10.0 / 15.0], rtol=1e-6)
        # Each channel is an arithmetic progression of 6 values spanning the range:
        # bins 0, 3, 6, 9, 12, 15.
        np.testing.assert_array_equal(q[..., 0].reshape(-1), [0, 3, 6, 9, 12, 15])
        np.testing.assert_array_equal(q[..., 1].reshape(-1), [0, 3, 6, 9, 12, 15])
        np.testing.assert_allclose(zp, [-1.0 / (10 / 15), -2.0 / (10 / 15)], rtol=1e-6)

    def test_round_half_to_even(self):
        """min 0, max 15 -> scale exactly 1: x.5 rounds to the even bin (NumPy),
        not up (the reference CUDA/Triton kernels' (int)(x+0.5))."""
        col = np.array([0.0, 15.0, 0.5, 1.5, 2.5, 3.5, 14.5, 7.5, 8.5], dtype=np.float32)
        q, scale, zp = quantize_int4_ref(col[:, None])
        assert scale[0] == np.float32(1.0)
        np.testing.assert_array_equal(q[:, 0], [0, 15, 0, 2, 2, 4, 14, 8, 8])
        assert zp[0] == 0.0

    def test_uniform_input_floor(self):
        """reference tests/test_quantization.py:89-103: a constant channel takes the
        1e-8 range floor (float32), so scale = f32(1e-8)/15 and every bin is 0."""
        kv = np.full((2, 4, 16), 5.0, dtype=np.float32)
        q, scale, zp = quantize_int4_ref(kv)
        assert np.all(scale == np.float32(np.float32(1e-8) / np.float32(15.0)))
        assert np.all(q == 0)
        np.testing.assert_array_equal(zp, np.float32(-5.0) / scale)

    def test_reduction_is_over_leading_axes(self):
        """Each channel has its own scale: scaling one channel scales only its scale."""
        rng = np.random.RandomState(5)
        kv = rng.randn(64, 8).astype(np.float32)
        kv2 = kv.copy()
        kv2[:, 3] *= 4.0
        _, s1, _ = quantize_int4_ref(kv)
        _, s2, _ = quantize_int4_ref(kv2)
        np.testing.assert_allclose(s2[3], 4 * s1[3], rtol=1e-6)
        np.testing.assert_array_equal(np.delete(s2, 3), np.delete(s1, 3))


class TestRoundTrip:

    @pytest.mark.parametrize("shape", [(4, 8, 64), (256, 128), (1, 7), (129, 33)])
    def test_error_within_half_step(self, shape):
        """reference tests/test_quantization.py:21-44: |x - dq(q(x))| <= scale/2
        (plus float32 rounding of the dequant expression)."""
        kv = np.random.RandomState(sum(shape)).randn(*shape).astype(np.float32)
        q, scale, zp, dq = quantize_and_dequantize_ref(kv)
        err = np.abs(kv - dq)
        bound = scale / 2 + 4 * np.finfo(np.float32).eps * (np.abs(kv).max(axis=tuple(
            range(kv.ndim - 1))) + scale * 15)
        assert np.all(err <= bound)

    def test_dequant_sign_and_offset(self):
        """Bin 0 dequantizes to the channel minimum and bin 15 to (about) the maximum."""
        kv = np.random.RandomState(9).randn(200, 16).astype(np.float32)
        q, s, z = quantize_int4_ref(kv)
        deq0 = dequantize_int4_ref(np.zeros((1, 16), np.uint8), s, z)[0]
        deq15 = dequantize_int4_ref(np.full((1, 16), 15, np.uint8), s, z)[0]
        np.testing.assert_allclose(deq0, kv.min(axis=0), atol=1e-6)
        np.testing.assert_allclose(deq15, kv.max(axis=0), atol=1e-5)


class TestPacking:

    def test_known_answer_bytes(self):
        """reference tests/test_int4_pack.py:33-35 values; the bytes are pinned by hand:
        low nibble = even index."""
        q = np.array([[0, 15, 15, 0, 7, 8]], dtype=np.uint8)
        p = pack_int4(q)
        np.testing.assert_array_equal(p, [[0xF0, 0x0F, 0x87]])
        np.testing.assert_array_equal(unpack_int4(p, 6), q)

    @pytest.mark.parametrize("shape,packed", [((256, 64), (256, 32)), ((10, 7), (10, 4)),
                                              ((4, 128, 32), (4, 128, 16))])
    def test_shapes_and_round_trip(self, shape, packed):
        """reference tests/test_int4_pack.py:12-31."""
        q = np.random.RandomState(shape[0]).randint(0, 16, shape).astype(np.uint8)
        p = pack_int4(q)
        assert p.shape == packed
        assert p.nbytes == packed_nbytes(shape)
        np.testing.assert_array_equal(unpack_int4(p, shape[-1]), q)

    def test_rejects_out_of_range(self):
        with pytest.raises(AssertionError):
            pack_int4(np.array([[16]], dtype=np.uint8))


class TestAgainstCRestatement:
    """The NumPy and C restatements are independent implementations of the same
    float32 operations; they must agree bit for bit."""

    @pytest.mark.parametrize("shape", [(1, 1), (1, 64), (255, 3), (256, 3), (257, 3),
                                       (1030, 8), (4096, 128), (128, 128)])
    def test_quantizer_bits(self, shape):
        kv = np.random.RandomState(shape[0]).randn(*shape).astype(np.float32)
        q, s, z = quantize_int4_ref(kv)
        qc, sc, zc = cref.quantize_group(kv)
        np.testing.assert_array_equal(q, qc)
        assert s.tobytes() == sc.tobytes()
        np.testing.assert_array_equal(z, zc)

    def test_quantizer_bits_outlier_channels(self):
        rng = np.random.RandomState(77)
        kv = rng.randn(128, 128).astype(np.float32)
        kv[:, [3, 40, 77, 100]] *= 20.0
        q, s, z = quantize_int4_ref(kv)
        qc, sc, zc = cref.quantize_group(kv)
        np.testing.assert_array_equal(q, qc)
        np.testing.assert_array_equal(s, sc)

    def test_pack_bits(self):
        q = np.random.RandomState(3).randint(0, 16, (33, 17)).astype(np.uint8)
        np.testing.assert_array_equal(pack_int4(q), cref.pack(q))


class TestGroupedQuantizer:

    def test_groups_equal_per_group_calls(self):
        rng = np.random.RandomState(11)
        k = rng.randn(2, 3, 300, 16).astype(np.float32)
        lens = np.array([300, 129])
        q, s, z = quantize_groups_ref(k, lens, group_size=128)
        for b in range(2):
            for h in range(3):
                for g in range((lens[b] + 127) // 128):
                    rows = k[b, h, g * 128:min((g + 1) * 128, lens[b])]
                    qq, ss, zz = quantize_int4_ref(rows)
                    np.testing.assert_array_equal(q[b, h, g * 128:g * 128 + len(rows)], qq)
                    np.testing.assert_array_equal(s[b, h, g], ss)
                    np.testing.assert_array_equal(z[b, h, g], zz)

    def test_partial_group_uses_only_its_rows(self):
        """reference tests/test_perplexity_harness.py:122-131: rows past the sequence
        end must not widen the last group's range."""
        rng = np.random.RandomState(1)
        k = rng.randn(1, 1, 300, 16).astype(np.float32)
        k[0, 0, 290:] = 1000.0  # past the end: must be ignored
        q, s, z = quantize_groups_ref(k, np.array([290]), group_size=128)
        tail = k[0, 0, 256:290]
        _, st, _ = quantize_int4_ref(tail)
        np.testing.assert_array_equal(s[0, 0, 2], st)
        assert np.all(q[0, 0, 290:] == 0)
