#!/usr/bin/env python3
"""Write the golden fixtures in tests/golden/ from the oracle.

The oracle (oracle/) is pinned by known answers, closed forms, invariants and
a float64 arbiter (tests/test_oracle_*.py); these fixtures freeze its outputs
on small seeded problems so the GPU tests and later oracle edits are checked
against fixed vectors. Inputs are not stored: they are regenerated from the
seeds below (np.random.RandomState, whose stream is stable across NumPy
versions) and identified by the SHA-256 of their bytes.

    python tests/golden/make_golden.py
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "int4-kv-cache-quantization-cuda-triton-pallas_amd"))

from oracle import (f64_attention, online_softmax_ref, pack_int4, paged_decode_f64,  # noqa: E402
                    paged_decode_ref, quantize_groups_ref, quantize_int4_ref)
from flash_decode_int4.workloads import make_workload  # noqa: E402

ROWS_CASES = [(1, 1), (1, 64), (255, 3), (257, 3), (1030, 8), (512, 128)]
TIES_INPUT = np.array([0.0, 15.0, 0.5, 1.5, 2.5, 3.5, 14.5, 7.5, 8.5], dtype=np.float32)
TIES_EXPECT = np.array([0, 15, 0, 2, 2, 4, 14, 8, 8], dtype=np.uint8)  # by hand: half to even

PAGED_CASES = {
    "cpu": dict(name="cpu"),
    "ragged_mini": dict(batch=3, heads=2, head_dim=128, seq_lens=[0, 37, 300], seed=31),
    "wide_mini": dict(batch=2, heads=2, head_dim=256, seq_lens=[129, 400], seed=32),
}

# Shared-stream cases of the reference's own tests (lens of
# tests/test_ops_dispatch.py:245-251 and tests/test_pallas_flash_decode.py:97-148).
DROPIN_CASES = {
    "ops_ragged": dict(batch=2, heads=3, dim=32, n_blocks=3, rows=64, seed=0, lens=[64, 0, 17],
                       scaled=True),
    "var_lens": dict(batch=2, heads=4, dim=64, n_blocks=4, rows=128, seed=3,
                     lens=[128, 73, 5, 128], scaled=False),
    "empty_mid": dict(batch=2, heads=4, dim=64, n_blocks=4, rows=128, seed=4,
                      lens=[128, 0, 64, 128], scaled=False),
    "first_empty": dict(batch=1, heads=2, dim=64, n_blocks=3, rows=64, seed=6, lens=[0, 64, 64],
                        scaled=False),
    "d128": dict(batch=1, heads=4, dim=128, n_blocks=4, rows=256, seed=2,
                 lens=[256, 256, 256, 256], scaled=False),
}


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def rows_input(shape):
    return np.random.RandomState(shape[0] * 1000 + shape[1]).randn(*shape).astype(np.float32)


def paged_case(spec):
    """Workload of a paged case and its oracle-quantized pages."""
    w = make_workload(**spec)
    q, s, z = quantize_groups_ref(w["k"], w["seq_lens"])
    H, D = w["heads"], w["head_dim"]
    kp = np.zeros((w["num_pages"], H, 16, D // 2), np.uint8)
    for b in range(w["batch"]):
        n = int(w["seq_lens"][b])
        for lp in range((n + 15) // 16):
            rows = min(16, n - lp * 16)
            kp[w["page_table"][b, lp], :, :rows] = pack_int4(q[b, :, lp * 16:lp * 16 + rows])
    return w, kp, s, z


def dropin_case(spec):
    """reference tests/test_pallas_flash_decode.py:37-50 / test_ops_dispatch.py:159-169."""
    rng = np.random.RandomState(spec["seed"])
    b, h, d = spec["batch"], spec["heads"], spec["dim"]
    query = rng.randn(b, h, d).astype(np.float32)
    if spec["scaled"]:
        query = (query / np.sqrt(d)).astype(np.float32)
    k_q, k_s, k_z, vals = [], [], [], []
    for _ in range(spec["n_blocks"]):
        k = rng.randn(spec["rows"], d).astype(np.float32)
        v = rng.randn(spec["rows"], d).astype(np.float32)
        q_, s_, z_ = quantize_int4_ref(k)
        k_q.append(q_); k_s.append(s_); k_z.append(z_); vals.append(v)
    return query, k_q, k_s, k_z, vals, np.asarray(spec["lens"], np.int32)


def main():
    out = {}
    for shape in ROWS_CASES:
        x = rows_input(shape)
        q, s, z = quantize_int4_ref(x)
        tag = f"rows_{shape[0]}x{shape[1]}"
        out[tag + "_sha"] = np.array(sha(x))
        out[tag + "_q"], out[tag + "_scale"], out[tag + "_zp"] = q, s, z
    out["ties_input"] = TIES_INPUT
    out["ties_expect"] = TIES_EXPECT
    np.savez_compressed(os.path.join(HERE, "quantize_rows.npz"), **out)

    out = {}
    for tag, spec in PAGED_CASES.items():
        w, kp, s, z = paged_case(spec)
        args = (w["q"], kp, w["v_pages"], s, z, w["page_table"], w["seq_lens"])
        out[tag + "_sha"] = np.array(sha(w["q"], w["k"], w["v_pages"], w["page_table"],
                                         w["seq_lens"]))
        out[tag + "_pages"], out[tag + "_scale"], out[tag + "_zp"] = kp, s, z
        out[tag + "_out32"] = paged_decode_ref(*args)
        out[tag + "_out64"] = paged_decode_f64(*args)
    np.savez_compressed(os.path.join(HERE, "paged.npz"), **out)

    out = {}
    for tag, spec in DROPIN_CASES.items():
        case = dropin_case(spec)
        query, k_q, k_s, k_z, vals, lens = case
        out[tag + "_sha"] = np.array(sha(query, *k_q, *k_s, *k_z, *vals, lens))
        out[tag + "_out32"] = online_softmax_ref(query, list(zip(k_q, k_s, k_z)), vals, lens)[0]
        out[tag + "_out64"] = f64_attention(*case)
    np.savez_compressed(os.path.join(HERE, "dropin.npz"), **out)
    for f in ("quantize_rows.npz", "paged.npz", "dropin.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
