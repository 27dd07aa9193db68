"""Pins of the oracle attention (CPU).

The page-loop oracle is checked against mathematics it must satisfy and
against a float64 evaluation that shares no accumulation strategy with it;
the float64 arbiter itself is checked against scipy's softmax and textbook
special cases.
"""

import numpy as np
import pytest
from scipy.special import softmax

from oracle import (f64_attention, float32_floor, online_softmax_fp32_ref, online_softmax_ref,
                    paged_decode_f64, paged_decode_ref, pack_int4, quantize_groups_ref,
                    quantize_int4_ref)
from oracle import cref


def make_case(batch=2, heads=4, dim=64, n_blocks=4, block_size=128, seed=0, lens=None):
    """reference tests/test_pallas_flash_decode.py:37-50 (same construction)."""
    rng = np.random.RandomState(seed)
    query = rng.randn(batch, heads, dim).astype(np.float32)
    k_q, k_s, k_z, vals = [], [], [], []
    for _ in range(n_blocks):
        k = rng.randn(block_size, dim).astype(np.float32)
        v = rng.randn(block_size, dim).astype(np.float32)
        q_, s_, z_ = quantize_int4_ref(k)
        k_q.append(q_); k_s.append(s_); k_z.append(z_); vals.append(v)
    if lens is None:
        lens = np.full(n_blocks, block_size, dtype=np.int32)
    return query, k_q, k_s, k_z, vals, np.asarray(lens, dtype=np.int32)


def run_ref(case):
    query, k_q, k_s, k_z, vals, lens = case
    return online_softmax_ref(query, list(zip(k_q, k_s, k_z)), vals, lens)[0]


class TestArbiter:

    def test_arbiter_matches_scipy_softmax(self):
        case = make_case(batch=1, heads=2, dim=32, n_blocks=3, block_size=40, seed=3,
                         lens=[40, 7, 0])
        query, k_q, k_s, k_z, vals, lens = case
        keys, values = [], []
        for i in range(3):
            n = lens[i]
            keys.append(k_q[i][:n].astype(np.float64) * k_s[i].astype(np.float64)
                        - k_z[i].astype(np.float64) * k_s[i].astype(np.float64))
            values.append(vals[i][:n].astype(np.float64))
        K, V = np.concatenate(keys), np.concatenate(values)
        w = softmax(query.astype(np.float64) @ K.T, axis=-1)
        np.testing.assert_allclose(f64_attention(*case), w @ V, rtol=1e-12, atol=1e-13)

    def test_zero_query_gives_mean_of_valid_values(self):
        case = list(make_case(batch=1, heads=3, dim=16, n_blocks=3, block_size=20, seed=4,
                              lens=[20, 5, 11]))
        case[0] = np.zeros_like(case[0])
        vals, lens = case[4], case[5]
        expect = np.concatenate([vals[i][:lens[i]] for i in range(3)]).astype(np.float64).mean(0)
        np.testing.assert_allclose(f64_attention(*case)[0, 0], expect, rtol=1e-13)
        np.testing.assert_allclose(run_ref(case)[0, 0], expect, rtol=2e-6, atol=2e-7)


class TestPageLoopOracle:

    @pytest.mark.parametrize("dim", [64, 128])
    def test_within_float32_noise_floor(self, dim):
        """reference tests/test_pallas_flash_decode.py:181-217 (3x the floor)."""
        case = make_case(batch=1, heads=4, dim=dim, n_blocks=4, block_size=256, seed=2)
        truth = f64_attention(*case)
        err = np.abs(run_ref(case) - truth).mean()
        assert err <= 3.0 * float32_floor(truth, dim)

    @pytest.mark.parametrize("lens", [[128, 73, 5, 128], [128, 0, 64, 128], [0, 64, 64, 64]])
    def test_ragged_and_empty_pages(self, lens):
        case = make_case(batch=2, heads=4, dim=64, n_blocks=4, block_size=128, seed=3, lens=lens)
        got = run_ref(case)
        assert np.isfinite(got).all()
        np.testing.assert_allclose(got, f64_attention(*case), atol=1e-5)

    def test_all_pages_empty_is_exact_zero(self):
        case = make_case(batch=1, heads=2, dim=64, n_blocks=3, block_size=64, seed=5,
                         lens=[0, 0, 0])
        np.testing.assert_array_equal(run_ref(case), 0.0)

    def test_single_live_token_returns_its_value_row(self):
        case = make_case(batch=1, heads=2, dim=32, n_blocks=2, block_size=16, seed=8,
                         lens=[0, 1])
        np.testing.assert_array_equal(run_ref(case)[0, 0], case[4][1][0])

    def test_page_decomposition_invariance(self):
        """reference tests/test_pallas_flash_decode.py:220-252 and
        tests/test_flash_decode.py:276-304."""
        rng = np.random.RandomState(11)
        dim, total = 64, 512
        query = rng.randn(1, 2, dim).astype(np.float32)
        keys = rng.randn(total, dim).astype(np.float32)
        vals = rng.randn(total, dim).astype(np.float32)
        q_, s_, z_ = quantize_int4_ref(keys)
        outs = []
        for n_blocks in (1, 2, 4, 8):
            bs = total // n_blocks
            pages = [(q_[i * bs:(i + 1) * bs], s_, z_) for i in range(n_blocks)]
            vl = [vals[i * bs:(i + 1) * bs] for i in range(n_blocks)]
            outs.append(online_softmax_ref(query, pages, vl, np.full(n_blocks, bs))[0])
        for o in outs[1:]:
            assert np.abs(o - outs[0]).max() < 1e-5

    def test_fp32_multi_block_equals_concat(self):
        """reference tests/test_correctness.py:37-63."""
        rng = np.random.RandomState(6)
        query = rng.randn(2, 4, 32).astype(np.float32)
        ks = [rng.randn(256, 32).astype(np.float32) for _ in range(4)]
        vs = [rng.randn(256, 32).astype(np.float32) for _ in range(4)]
        a = online_softmax_fp32_ref(query, ks, vs, np.full(4, 256))
        b = online_softmax_fp32_ref(query, [np.concatenate(ks)], [np.concatenate(vs)],
                                    np.array([1024]))
        assert np.abs(a - b).max() < 1e-5


def _paged_problem(B, H, D, lens, seed, Hq=None):
    rng = np.random.RandomState(seed)
    Hq = Hq or H
    T = max(max(lens), 1)
    q = rng.randn(B, Hq, D).astype(np.float32)
    k = rng.randn(B, H, T, D).astype(np.float32)
    n_pages = [(t + 15) // 16 for t in lens]
    P = max(sum(n_pages), 1)
    v = rng.randn(P, H, 16, D).astype(np.float32)
    perm = rng.permutation(P)
    table = np.zeros((B, max(max(n_pages), 1)), np.int32)
    off = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[off:off + n]
        off += n
    kq, s, z = quantize_groups_ref(k, np.array(lens))
    kp = np.zeros((P, H, 16, D // 2), np.uint8)
    for b in range(B):
        for lp in range(n_pages[b]):
            rows = kq[b, :, lp * 16:(lp + 1) * 16]
            kp[table[b, lp], :, :rows.shape[1]] = pack_int4(rows)
    return q, kp, v, s, z, table, np.array(lens, np.int32)


class TestPagedOracle:

    def test_paged_matches_f64_and_c_arbiter(self):
        args = _paged_problem(3, 2, 64, [0, 37, 300], seed=21)
        o32 = paged_decode_ref(*args)
        o64 = paged_decode_f64(*args)
        oc = cref.paged_attention_f64(*args)
        np.testing.assert_allclose(oc, o64, rtol=1e-11, atol=1e-12)
        np.testing.assert_array_equal(o32[0], 0.0)
        assert np.abs(o32 - o64).max() < 1e-5

    def test_grouped_query_heads_read_their_kv_head(self):
        q, kp, v, s, z, table, lens = _paged_problem(2, 2, 64, [50, 129], seed=5, Hq=4)
        out = paged_decode_f64(q, kp, v, s, z, table, lens)
        # q-heads 0,1 read kv-head 0 and 2,3 read kv-head 1: duplicating kv-head 0
        # into both kv slots must leave q-heads 0,1 unchanged and change 2,3.
        kp2, v2, s2, z2 = kp.copy(), v.copy(), s.copy(), z.copy()
        kp2[:, 1], v2[:, 1], s2[:, 1], z2[:, 1] = kp[:, 0], v[:, 0], s[:, 0], z[:, 0]
        out2 = paged_decode_f64(q, kp2, v2, s2, z2, table, lens)
        np.testing.assert_array_equal(out2[:, :2], out[:, :2])
        assert np.abs(out2[:, 2:] - out[:, 2:]).max() > 1e-3
