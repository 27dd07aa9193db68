"""INT4PagedKVCache over the device page pool (reference
tests/test_vllm_integration.py:12-101), plus exactness against the oracle."""

import numpy as np
import pytest

from oracle import f64_attention, online_softmax_fp32_ref, online_softmax_ref, quantize_int4_ref

pytestmark = pytest.mark.gpu


def _cache(*a):
    from flash_decode_int4.vllm_integration import INT4PagedKVCache
    return INT4PagedKVCache(*a)


class TestINT4PagedKVCache:

    def test_write_and_decode(self):
        np.random.seed(0)
        cache = _cache(16, 128, 64)
        for b in range(4):
            cache.write_block(b, np.random.randn(128, 64).astype(np.float32),
                              np.random.randn(128, 64).astype(np.float32))
        out = cache.decode_attention(np.random.randn(2, 4, 64).astype(np.float32), [0, 1, 2, 3])
        assert out.shape == (2, 4, 64) and np.isfinite(out).all()

    def test_int4_decode_close_to_fp32(self):
        np.random.seed(1)
        head_dim = 64
        cache = _cache(8, 256, head_dim)
        keys, values = [], []
        for b in range(3):
            k = np.random.randn(256, head_dim).astype(np.float32)
            v = np.random.randn(256, head_dim).astype(np.float32)
            cache.write_block(b, k, v)
            keys.append(k)
            values.append(v)
        query = (np.random.randn(1, 2, head_dim) / np.sqrt(head_dim)).astype(np.float32)
        out = cache.decode_attention(query, [0, 1, 2])
        ref = online_softmax_fp32_ref(query, keys, values, np.full(3, 256, dtype=np.int32))
        assert np.abs(out - ref).mean() < 0.05

    def test_matches_reference_cache_semantics(self):
        """The reference cache quantizes each block as one group, stores V as fp16
        and attends every query over the block table; the oracle on the same
        (fp16-rounded) values is the exact expectation."""
        rng = np.random.RandomState(5)
        cache = _cache(8, 96, 48)
        blocks = {}
        for b, rows in [(2, 96), (5, 40), (0, 96), (7, 1)]:
            k = rng.randn(rows, 48).astype(np.float32)
            v = rng.randn(rows, 48).astype(np.float32)
            cache.write_block(b, k, v)
            blocks[b] = (k, v)
        table = [5, 0, 7, 2]
        query = rng.randn(2, 3, 48).astype(np.float32)
        got = cache.decode_attention(query, table)
        pages, vals, lens = [], [], []
        for b in table:
            k, v = blocks[b]
            q_, s_, z_ = quantize_int4_ref(k)
            pages.append((q_, s_, z_))
            vals.append(v.astype(np.float16).astype(np.float32))
            lens.append(len(k))
        ref = online_softmax_ref(query, pages, vals, np.array(lens))[0]
        f64 = f64_attention(query, [p[0] for p in pages], [p[1] for p in pages],
                            [p[2] for p in pages], vals, lens)
        assert np.abs(got - ref).max() < 1e-5
        assert np.abs(got - f64).max() < 1e-5
        np.testing.assert_array_equal(cache.k_scale[5], pages[0][1])

    def test_free_block(self):
        cache = _cache(4, 64, 32)
        k = np.random.randn(64, 32).astype(np.float32)
        cache.write_block(0, k, k)
        cache.free_block(0)
        assert 0 not in cache.k_packed
        assert cache.memory_stats()["blocks"] == 0

    def test_memory_compression_ratio(self):
        cache = _cache(16, 256, 128)
        for b in range(8):
            k = np.random.randn(256, 128).astype(np.float32)
            cache.write_block(b, k, k)
        stats = cache.memory_stats()
        assert stats["ratio"] > 1.5, stats

    def test_memory_stats_count_the_stored_arrays(self):
        """As the reference counts them (src/vllm_integration.py:80-102): the
        bytes of the packed key rows, scales, zero-points and fp16 value rows
        that the mapping views return; the pool's whole slots separately."""
        rng = np.random.RandomState(4)
        cache = _cache(4, 32, 48)
        for b, rows in [(0, 32), (3, 7), (9, 70)]:
            k = rng.randn(rows, 48).astype(np.float32)
            cache.write_block(b, k, k)
        stats = cache.memory_stats()
        stored = sum(cache.k_packed[b].nbytes + cache.k_scale[b].nbytes + cache.k_zp[b].nbytes
                     + cache.v[b].nbytes for b in cache.k_packed)
        fp16 = sum(cache.lens[b] * 48 * 2 * 2 for b in cache.lens)
        assert stats["stored_mb"] == round(stored / 1048576, 3)
        assert stats["fp16_equiv_mb"] == round(fp16 / 1048576, 3)
        assert stats["ratio"] == round(fp16 / stored, 2)
        # 1 + 1 + 3 slots of 32 rows at the padded head_dim 64
        slot = 32 * 32 + 32 * 64 * 2 + 2 * 64 * 4
        assert stats["pool_mb"] == round(5 * slot / 1048576, 3)

    def test_packed_storage_is_real(self):
        from oracle import pack_int4
        np.random.seed(7)
        cache = _cache(4, 128, 64)
        k = np.random.randn(128, 64).astype(np.float32)
        v = np.random.randn(128, 64).astype(np.float32)
        cache.write_block(0, k, v)
        assert cache.k_packed[0].nbytes == 128 * 64 // 2
        np.testing.assert_array_equal(cache.k_packed[0], pack_int4(quantize_int4_ref(k)[0]))
        out = cache.decode_attention((np.random.randn(1, 2, 64) / 8.0).astype(np.float32), [0])
        assert np.isfinite(out).all()

    def test_variable_block_lengths(self):
        np.random.seed(2)
        cache = _cache(4, 128, 32)
        cache.write_block(0, np.random.randn(128, 32).astype(np.float32),
                          np.random.randn(128, 32).astype(np.float32))
        cache.write_block(1, np.random.randn(40, 32).astype(np.float32),
                          np.random.randn(40, 32).astype(np.float32))
        out = cache.decode_attention(np.random.randn(1, 1, 32).astype(np.float32), [0, 1])
        assert np.isfinite(out).all()

    def test_unknown_block_raises_keyerror(self):
        cache = _cache(4, 16, 64)
        with pytest.raises(KeyError):
            cache.decode_attention(np.zeros((1, 1, 64), np.float32), [3])

    def test_malformed_blocks_rejected_before_the_cache_changes(self):
        cache = _cache(4, 16, 64)
        k = np.random.randn(20, 64).astype(np.float32)
        cache.write_block(0, k, k)
        with pytest.raises(ValueError):
            cache.write_block(0, np.zeros((17, 63), np.float32), np.zeros((17, 63), np.float32))
        with pytest.raises(ValueError):
            cache.write_block(0, np.zeros((0, 64), np.float32), np.zeros((0, 64), np.float32))
        with pytest.raises(AssertionError):
            cache.write_block(0, np.zeros((17, 64), np.float32), np.zeros((16, 64), np.float32))
        assert cache.lens[0] == 20
        np.testing.assert_array_equal(cache.k_scale[0], quantize_int4_ref(k)[1])

    def test_blocks_of_any_size_and_id(self):
        """The reference's dictionaries take any block id and any row count
        (src/vllm_integration.py:48-56): blocks longer than block_size take
        several pool slots (the pool grows past num_blocks), each with the
        block's one scale group, and decode as one page of the reference."""
        from oracle import pack_int4
        rng = np.random.RandomState(9)
        cache = _cache(4, 16, 64)
        blocks = {}
        for b, rows in [(0, 40), (1000, 16), (2, 100), (-3, 1), (5, 17)]:
            k = rng.randn(rows, 64).astype(np.float32)
            v = rng.randn(rows, 64).astype(np.float32)
            cache.write_block(b, k, v)
            blocks[b] = (k, v)
        # Rewriting a block with another length frees or takes slots.
        k = rng.randn(33, 64).astype(np.float32)
        v = rng.randn(33, 64).astype(np.float32)
        cache.write_block(2, k, v)
        blocks[2] = (k, v)
        cache.free_block(5)
        del blocks[5]
        assert cache.memory_stats()["blocks"] == 4
        table = [2, 1000, -3, 0, 2]
        query = rng.randn(2, 3, 64).astype(np.float32)
        got = cache.decode_attention(query, table)
        pages, vals, lens = [], [], []
        for b in table:
            k, v = blocks[b]
            q_, s_, z_ = quantize_int4_ref(k)
            pages.append((q_, s_, z_))
            vals.append(v.astype(np.float16).astype(np.float32))
            lens.append(len(k))
            np.testing.assert_array_equal(cache.k_packed[b], pack_int4(q_))
            np.testing.assert_array_equal(cache.k_scale[b], s_)
            np.testing.assert_array_equal(cache.k_zp[b], z_)
            np.testing.assert_array_equal(cache.v[b], v.astype(np.float16))
        ref = online_softmax_ref(query, pages, vals, np.array(lens))[0]
        f64 = f64_attention(query, [p[0] for p in pages], [p[1] for p in pages],
                            [p[2] for p in pages], vals, lens)
        assert np.abs(got - ref).max() < 1e-5
        assert np.abs(got - f64).max() < 1e-5
        with pytest.raises(KeyError):
            cache.decode_attention(query, [5])
