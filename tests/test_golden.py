"""The oracle reproduces the committed golden fixtures (CPU), and the HIP path
matches them (GPU).

Inputs are regenerated from the seeds in tests/golden/make_golden.py and
identified by SHA-256; quantizer outputs must match bit for bit. The float32
attention fixtures depend on the BLAS kernels of the host that wrote them, so
the oracle is held to 1e-6 of them and the float64 arbiter to 1e-12.
"""

import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN, load_golden

sys.path.insert(0, GOLDEN)
import make_golden as mg  # noqa: E402

from oracle import (f64_attention, online_softmax_ref, paged_decode_f64,  # noqa: E402
                    paged_decode_ref, quantize_int4_ref)

ROWS = load_golden("quantize_rows.npz")
PAGED = load_golden("paged.npz")
DROPIN = load_golden("dropin.npz")


def _rows_tag(shape):
    return f"rows_{shape[0]}x{shape[1]}"


class TestOracleReproducesGolden:

    @pytest.mark.parametrize("shape", mg.ROWS_CASES)
    def test_quantize_rows(self, shape):
        x = mg.rows_input(shape)
        tag = _rows_tag(shape)
        assert mg.sha(x) == str(ROWS[tag + "_sha"])
        q, s, z = quantize_int4_ref(x)
        np.testing.assert_array_equal(q, ROWS[tag + "_q"])
        assert s.tobytes() == ROWS[tag + "_scale"].tobytes()
        np.testing.assert_array_equal(z, ROWS[tag + "_zp"])

    def test_ties(self):
        q, _, _ = quantize_int4_ref(ROWS["ties_input"][:, None])
        np.testing.assert_array_equal(q[:, 0], ROWS["ties_expect"])

    @pytest.mark.parametrize("tag", list(mg.PAGED_CASES))
    def test_paged(self, tag):
        w, kp, s, z = mg.paged_case(mg.PAGED_CASES[tag])
        assert mg.sha(w["q"], w["k"], w["v_pages"], w["page_table"], w["seq_lens"]) == \
            str(PAGED[tag + "_sha"])
        np.testing.assert_array_equal(kp, PAGED[tag + "_pages"])
        np.testing.assert_array_equal(s, PAGED[tag + "_scale"])
        np.testing.assert_array_equal(z, PAGED[tag + "_zp"])
        args = (w["q"], kp, w["v_pages"], s, z, w["page_table"], w["seq_lens"])
        np.testing.assert_allclose(paged_decode_ref(*args), PAGED[tag + "_out32"], rtol=0,
                                   atol=1e-6)
        np.testing.assert_allclose(paged_decode_f64(*args), PAGED[tag + "_out64"], rtol=1e-12,
                                   atol=1e-13)

    @pytest.mark.parametrize("tag", list(mg.DROPIN_CASES))
    def test_dropin(self, tag):
        case = mg.dropin_case(mg.DROPIN_CASES[tag])
        query, k_q, k_s, k_z, vals, lens = case
        assert mg.sha(query, *k_q, *k_s, *k_z, *vals, lens) == str(DROPIN[tag + "_sha"])
        out = online_softmax_ref(query, list(zip(k_q, k_s, k_z)), vals, lens)[0]
        np.testing.assert_allclose(out, DROPIN[tag + "_out32"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(f64_attention(*case), DROPIN[tag + "_out64"], rtol=1e-12,
                                   atol=1e-13)


@pytest.mark.gpu
class TestHipMatchesGolden:

    @pytest.mark.parametrize("shape", mg.ROWS_CASES)
    def test_quantize_rows(self, shape):
        from flash_decode_int4 import ops
        tag = _rows_tag(shape)
        q, s, z = ops.quantize_int4(mg.rows_input(shape), backend="hip")
        np.testing.assert_array_equal(q, ROWS[tag + "_q"])
        assert s.tobytes() == ROWS[tag + "_scale"].tobytes()
        np.testing.assert_array_equal(z, ROWS[tag + "_zp"])

    @pytest.mark.parametrize("tag", list(mg.PAGED_CASES))
    def test_paged(self, tag):
        import torch
        from flash_decode_int4 import ops
        from flash_decode_int4.workloads import make_workload
        w = make_workload(**mg.PAGED_CASES[tag])
        dev = torch.device("cuda")
        B, H, D = w["batch"], w["heads"], w["head_dim"]
        G = (w["max_tokens"] + 127) // 128
        kp = torch.zeros(w["num_pages"], H, 16, D // 2, dtype=torch.uint8, device=dev)
        s = torch.zeros(B, H, G, D, device=dev)
        z = torch.zeros(B, H, G, D, device=dev)
        sl = torch.from_numpy(w["seq_lens"]).to(dev)
        pt = torch.from_numpy(w["page_table"]).to(dev)
        ops.quantize_int4_paged(torch.from_numpy(w["k"]).to(dev), sl, pt, kp, s, z, 128)
        out = ops.flash_decode_paged(torch.from_numpy(w["q"]).to(dev), kp,
                                     torch.from_numpy(w["v_pages"]).to(dev), s, z, pt, sl)
        np.testing.assert_array_equal(kp.cpu().numpy(), PAGED[tag + "_pages"])
        np.testing.assert_array_equal(s.cpu().numpy(), PAGED[tag + "_scale"])
        np.testing.assert_array_equal(z.cpu().numpy(), PAGED[tag + "_zp"])
        got = out.cpu().numpy()
        o32, o64 = PAGED[tag + "_out32"], PAGED[tag + "_out64"]
        assert np.abs(got - o32).max() <= max(1e-5, 1.25 * np.abs(o32 - o64).max())
        assert np.abs(got - o64).max() <= np.abs(o32 - o64).max() + 1e-6

    @pytest.mark.parametrize("tag", list(mg.DROPIN_CASES))
    def test_dropin(self, tag):
        from flash_decode_int4 import ops
        case = mg.dropin_case(mg.DROPIN_CASES[tag])
        got = ops.flash_decode(*case, backend="hip")
        assert np.abs(got - DROPIN[tag + "_out32"]).max() < 1e-5
        assert np.abs(got - DROPIN[tag + "_out64"]).max() < 1e-5
