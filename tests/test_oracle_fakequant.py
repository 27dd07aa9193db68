"""Pins of the oracle's quantize-dequantize of key tensors (CPU).

Each test fails for a plausible mistake in the restatement: half-even where
the harness rounds half up (or the reverse), an exact t + 0.5 where the
harness adds in float32, the zero-point form of the dequantization where the
harness adds the minimum, a divided scale where the reciprocal form is asked
for (or the reverse), a block that borrows rows of its neighbour, a
reduction over the wrong axis, a bfloat16 cast that truncates.
"""

import numpy as np
import pytest

from oracle import (bf16_bits, bf16_bits_to_f32, fake_quantize_keys_ref,
                    quantize_and_dequantize_ref)
from oracle import cref


def _keys(shape, seed, ties=False):
    rng = np.random.RandomState(seed)
    x = (rng.standard_normal(shape) * rng.uniform(0.3, 3.0, shape[-1])).astype(np.float32)
    if ties:
        # Integer channels spanning exactly 15 (scale 1) with half-integer
        # values in between: every quotient is a tie or an integer.
        x = rng.randint(0, 31, size=shape).astype(np.float32) / np.float32(2.0)
        x[:, :, 0::7] = 0.0
        x[:, :, 3::7] = 15.0
    return x


class TestKnownAnswers:

    COL = np.array([0.0, 15.0, 0.5, 1.5, 2.5, 3.5, 14.5, 7.5, 8.5], np.float32)

    @staticmethod
    def _one(col, rounding, block=256):
        return fake_quantize_keys_ref(col[None, None, :, None], block, rounding)[0, 0, :, 0]

    def test_half_up_on_a_scale_one_channel(self):
        """min 0, max 15: scale exactly 1, t = x, dq = floor(x + 0.5)."""
        np.testing.assert_array_equal(self._one(self.COL, "half_up"),
                                      [0, 15, 1, 2, 3, 4, 15, 8, 9])

    def test_half_even_on_a_scale_one_channel(self):
        np.testing.assert_array_equal(self._one(self.COL, "half_even"),
                                      [0, 15, 0, 2, 2, 4, 14, 8, 8])

    def test_shifted_minimum_uses_each_dequantization(self):
        """min 2, max 17, x = 4.5: t = 2.5; half-up q = 3, dq = 3*1 + 2 = 5;
        half-even q = 2, zp = -2, dq = 2*1 - (-2)*1 = 4."""
        col = np.array([2.0, 17.0, 4.5], np.float32)
        assert self._one(col, "half_up")[2] == 5.0
        assert self._one(col, "half_even")[2] == 4.0

    def test_float32_add_of_one_half(self):
        """t = 0.5 - 2^-25 (the float below 0.5): exact t + 0.5 = 1 - 2^-25 is a
        tie between 1 - 2^-24 and 1 and rounds to 1.0 in float32, so floor
        gives bin 1 (the harness adds in float32); exact arithmetic gives 0."""
        t = np.nextafter(np.float32(0.5), np.float32(0.0))
        col = np.array([0.0, 15.0, t], np.float32)
        assert self._one(col, "half_up")[2] == 1.0
        assert self._one(col, "half_even")[2] == 0.0

    def test_reciprocal_scale_known_answer(self):
        """Channel [0, span, x], span = 1.5488135 (bits 1069956997), x =
        0.05162711 (bits 1028880115). IEEE span/15 = 0.10325423 (bits
        1037268724) and t = x/scale = 0.49999996... rounds to 0.49999997,
        + 0.5 ties to 1.0: bin 1, dq = scale. span * float32(1/15) =
        0.10325424 (one ulp up): t rounds to 0.49999994, + 0.5 = 0.99999994:
        bin 0, dq = 0. (Values derived with exact rational arithmetic.)"""
        span = np.uint32(1069956997).view(np.float32)
        x = np.uint32(1028880115).view(np.float32)
        col = np.array([0.0, span, x], np.float32)
        got = fake_quantize_keys_ref(col[None, None, :, None], 256, "half_up", "divide")[0, 0, :, 0]
        assert got[2].view(np.uint32) == 1037268724
        got = fake_quantize_keys_ref(col[None, None, :, None], 256, "half_up",
                                     "reciprocal")[0, 0, :, 0]
        assert got[2] == 0.0

    def test_reciprocal_of_fifteen_is_correctly_rounded(self):
        from fractions import Fraction
        from oracle.fakequant import RECIP_15
        err = abs(Fraction(float(RECIP_15)) - Fraction(1, 15))
        for nb in (np.nextafter(RECIP_15, np.float32(0)), np.nextafter(RECIP_15, np.float32(1))):
            assert err < abs(Fraction(float(nb)) - Fraction(1, 15))

    def test_block_size_one_is_the_identity_under_half_up(self):
        """One row per block: mn = x, q = floor(0 + 0.5) = 0, dq = 0*s + mn = x."""
        x = _keys((2, 3, 37, 16), seed=3)
        np.testing.assert_array_equal(fake_quantize_keys_ref(x, 1, "half_up"), x)

    def test_constant_block_floor(self):
        """A constant channel: span floored to 1e-8, every bin 0, dq = the constant."""
        x = np.full((1, 1, 10, 4), 3.25, np.float32)
        np.testing.assert_array_equal(fake_quantize_keys_ref(x, 256, "half_up"), x)

    def test_rejects_bad_arguments(self):
        with pytest.raises(ValueError):
            fake_quantize_keys_ref(np.zeros((1, 1, 4, 4), np.float32), 4, "nearest")
        with pytest.raises(ValueError):
            fake_quantize_keys_ref(np.zeros((1, 4, 4), np.float32), 4)
        with pytest.raises(ValueError):
            fake_quantize_keys_ref(np.zeros((1, 1, 4, 4), np.float32), 0)
        with pytest.raises(ValueError):
            fake_quantize_keys_ref(np.zeros((1, 1, 4, 4), np.float32), 4, "half_up", "mul")


class TestStructure:

    @pytest.mark.parametrize("block", [1, 5, 128, 256, 1000])
    def test_half_even_is_the_stored_scheme_per_block(self, block):
        """Per (sequence, head, block): quantize_and_dequantize_ref of the
        block's rows (reference src/quantize_int4_ref.py:139-158)."""
        x = _keys((2, 2, 300, 8), seed=block)
        got = fake_quantize_keys_ref(x, block, "half_even")
        for b in range(2):
            for h in range(2):
                for s0 in range(0, 300, block):
                    blk = x[b, h, s0:s0 + block]
                    _, _, _, dq = quantize_and_dequantize_ref(blk)
                    np.testing.assert_array_equal(got[b, h, s0:s0 + block], dq)

    def test_partial_block_equals_padding_with_the_last_row(self):
        """The harness pads a partial block with copies of its last row
        (scripts/validate_llama.py:145-147); the padded rows change no result."""
        x = _keys((1, 3, 200, 16), seed=4)
        pad = np.concatenate([x, np.repeat(x[:, :, -1:], 56, axis=2)], axis=2)
        for r in ("half_up", "half_even"):
            np.testing.assert_array_equal(fake_quantize_keys_ref(pad, 128, r)[:, :, :200],
                                          fake_quantize_keys_ref(x, 128, r))

    def test_blocks_and_channels_are_independent(self):
        """Changing one block's rows of one channel changes nothing elsewhere."""
        x = _keys((1, 2, 384, 8), seed=5)
        y = x.copy()
        y[0, 1, 128:256, 3] *= 7.0
        a = fake_quantize_keys_ref(x, 128, "half_up")
        b = fake_quantize_keys_ref(y, 128, "half_up")
        diff = np.argwhere(a != b)
        assert diff.size
        assert (diff[:, 0] == 0).all() and (diff[:, 1] == 1).all() and (diff[:, 3] == 3).all()
        assert ((diff[:, 2] >= 128) & (diff[:, 2] < 256)).all()

    @pytest.mark.parametrize("rounding", ["half_up", "half_even"])
    def test_round_trip_bound(self, rounding):
        """|x - dq| <= scale/2 plus the float32 rounding of q*scale (+ mn)."""
        x = _keys((2, 2, 512, 32), seed=6)
        dq = fake_quantize_keys_ref(x, 128, rounding)
        for s0 in range(0, 512, 128):
            blk = x[:, :, s0:s0 + 128]
            span = blk.max(axis=2, keepdims=True) - blk.min(axis=2, keepdims=True)
            bound = span / 30.0 + 4 * np.spacing(np.abs(blk).max(axis=2, keepdims=True))
            assert (np.abs(blk - dq[:, :, s0:s0 + 128]) <= bound).all()


class TestCRestatement:

    @pytest.mark.parametrize("scale_op", ["divide", "reciprocal"])
    @pytest.mark.parametrize("rounding", ["half_up", "half_even"])
    @pytest.mark.parametrize("shape,block,ties", [
        ((1, 1, 1, 4), 256, False),
        ((2, 3, 300, 16), 128, False),
        ((2, 2, 513, 64), 256, False),
        ((1, 4, 257, 8), 256, True),
        ((3, 2, 100, 12), 7, True),
        ((1, 2, 64, 128), 1, False),
    ])
    def test_bit_exact_with_c(self, shape, block, ties, rounding, scale_op):
        x = _keys(shape, seed=sum(shape) + block, ties=ties)
        want = fake_quantize_keys_ref(x, block, rounding, scale_op)
        code = 0 if rounding == "half_up" else 1
        recip = 1 if scale_op == "reciprocal" else 0
        for b in range(shape[0]):
            for h in range(shape[1]):
                got = cref.fake_quantize(x[b, h], block, code, recip)
                np.testing.assert_array_equal(got.view(np.uint32), want[b, h].view(np.uint32))


class TestCasts:

    @staticmethod
    def _values():
        rng = np.random.RandomState(8)
        x = rng.standard_normal(20000).astype(np.float32) * 100
        # Exact ties: a finite bfloat16 value plus half of its last place, both
        # parities and signs (NaN conversions differ between torch's code paths;
        # keys are finite).
        upper = rng.randint(0, 0x7F80, 4000).astype(np.uint32) | (rng.randint(0, 2, 4000) << 15)
        ties = ((upper << 16) | 0x8000).astype(np.uint32).view(np.float32)
        return np.concatenate([x, ties, np.float32([0.0, -0.0, 1e-40, -1e-40, 3.4e38, np.inf,
                                                    -np.inf])])

    def test_bf16_rounding_matches_torch(self):
        import torch
        x = self._values()
        want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(bf16_bits(x), want)
        np.testing.assert_array_equal(cref.f32_to_bf16_bits(x), want)

    def test_bf16_nan_and_widening(self):
        x = np.float32([np.nan, 1.0, -2.5])
        bits = bf16_bits(x)
        assert bits[0] == 0x7FC0
        np.testing.assert_array_equal(bf16_bits_to_f32(bits[1:]), [1.0, -2.5])

    def test_fp16_cast_matches_torch(self):
        import torch
        x = self._values()
        x = x[np.abs(x) < 65504]
        np.testing.assert_array_equal(x.astype(np.float16),
                                      torch.from_numpy(x).half().numpy())
