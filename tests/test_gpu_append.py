"""Decode-time append (one token per sequence per step) into the batched INT4
cache: after any mix of prefill and appends the packed pages, group scales
and values must equal the grouped quantizer applied to each whole sequence
(a partial group is quantized over its valid rows, reference
tests/test_perplexity_harness.py:122-131), bit for bit, and the decode over
the result must match the page-loop oracle."""

import numpy as np
import pytest

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _cache(**kw):
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    return INT4PagedSequenceCache(**kw)


def _stored(v, vdtype):
    """float32 values as the cache stores them (rounded to vdtype), widened back."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(v)).to(getattr(torch, vdtype)).float().numpy()


def _check_against_oracle(cache, streams, lens, group, vdtype):
    """streams[b] = (K [H, n, D] float32, V [H, n, D]) of sequence b's tokens."""
    B = len(streams)
    H, _, D = streams[0][0].shape
    T = max(max(lens), 1)
    k = np.zeros((B, H, T, D), np.float32)
    for b, (kb, _) in enumerate(streams):
        k[b, :, :lens[b]] = kb[:, :lens[b]]
    qr, sr, zr = quantize_groups_ref(k, np.array(lens), group_size=group)
    kp = cache.k_pages.cpu().numpy()
    vp = cache.v_pages.float().cpu().numpy()
    sc = cache.k_scale.cpu().numpy()
    zc = cache.k_zp.cpu().numpy()
    table = cache.page_table.cpu().numpy()
    assert list(cache.seq_lens[:B].cpu().numpy()) == list(lens)
    for b in range(B):
        ng = (lens[b] + group - 1) // group
        np.testing.assert_array_equal(sc[b, :, :ng], sr[b, :, :ng])
        np.testing.assert_array_equal(zc[b, :, :ng], zr[b, :, :ng])
        vb = streams[b][1]
        for lp in range((lens[b] + 15) // 16):
            n = min(16, lens[b] - lp * 16)
            np.testing.assert_array_equal(kp[table[b, lp], :, :n],
                                          pack_int4(qr[b, :, lp * 16:lp * 16 + n]))
            np.testing.assert_array_equal(vp[table[b, lp], :, :n],
                                          _stored(vb[:, lp * 16:lp * 16 + n], vdtype))
    return table


@pytest.mark.parametrize("D,group,vdtype,H", [(128, 128, "float32", 2), (64, 64, "float16", 3),
                                              (256, 256, "float32", 1),
                                              (128, 128, "bfloat16", 2)])
def test_append_equals_whole_sequence_quantization(D, group, vdtype, H):
    import torch
    rng = np.random.RandomState(D + group)
    B, steps = 3, 150
    lens0 = [0, group - 1, 2 * group - 56]  # empty, one short of a group, mid-group
    total = [n + steps for n in lens0]
    streams = [(rng.randn(H, n, D).astype(np.float32), rng.randn(H, n, D).astype(np.float32))
               for n in total]
    cache = _cache(num_pages=128, num_kv_heads=H, head_dim=D, max_seqs=4,
                   max_seq_len=max(total) + 16, group_rows=group, value_dtype=vdtype)
    T0 = max(lens0)
    k0 = np.zeros((B, H, T0, D), np.float32)
    v0 = np.zeros((B, H, T0, D), np.float32)
    for b in range(B):
        k0[b, :, :lens0[b]] = streams[b][0][:, :lens0[b]]
        v0[b, :, :lens0[b]] = streams[b][1][:, :lens0[b]]
    vt = getattr(torch, vdtype)
    cache.prefill(torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda().to(vt), lens0)
    for s in range(steps):
        kn = np.stack([streams[b][0][:, lens0[b] + s] for b in range(B)])
        vn = np.stack([streams[b][1][:, lens0[b] + s] for b in range(B)])
        cache.append(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda().to(vt))
        if s in (0, 1, 57):  # partial states are exact too
            _check_against_oracle(cache, streams, [n + s + 1 for n in lens0], group, vdtype)
    table = _check_against_oracle(cache, streams, total, group, vdtype)

    # The decode over the appended cache matches the page-loop oracle (q-heads
    # grouped two per kv-head).
    q = rng.randn(B, 2 * H, D).astype(np.float32)
    got = cache.decode(torch.from_numpy(q).cuda()).cpu().numpy()
    args = (q, cache.k_pages.cpu().numpy(), cache.v_pages.float().cpu().numpy(),
            cache.k_scale[:B].cpu().numpy(), cache.k_zp[:B].cpu().numpy(), table[:B],
            np.array(total), 16, group)
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    assert np.abs(got - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())


def test_append_matches_prefill_of_the_same_tokens():
    """Prefill of T tokens and prefill of T-40 plus 40 appends store the same
    bytes (pages may differ; compare through the page tables)."""
    import torch
    rng = np.random.RandomState(3)
    B, H, D, T = 2, 4, 128, 300
    k = rng.randn(B, H, T, D).astype(np.float32)
    v = rng.randn(B, H, T, D).astype(np.float32)
    a = _cache(num_pages=64, num_kv_heads=H, head_dim=D, max_seqs=B, max_seq_len=T)
    b_ = _cache(num_pages=64, num_kv_heads=H, head_dim=D, max_seqs=B, max_seq_len=T)
    a.prefill(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), [T, T])
    b_.prefill(torch.from_numpy(k[:, :, :T - 40]).cuda(), torch.from_numpy(v[:, :, :T - 40]).cuda(),
               [T - 40, T - 40])
    for t in range(T - 40, T):
        b_.append(torch.from_numpy(np.ascontiguousarray(k[:, :, t])).cuda(),
                  torch.from_numpy(np.ascontiguousarray(v[:, :, t])).cuda())
    for c in (a, b_):
        c.kp, c.vp, c.tb = (c.k_pages.cpu().numpy(), c.v_pages.cpu().numpy(),
                            c.page_table.cpu().numpy())
    for bi in range(B):
        for lp in range((T + 15) // 16):
            n = min(16, T - lp * 16)
            np.testing.assert_array_equal(a.kp[a.tb[bi, lp], :, :n], b_.kp[b_.tb[bi, lp], :, :n])
            np.testing.assert_array_equal(a.vp[a.tb[bi, lp], :, :n], b_.vp[b_.tb[bi, lp], :, :n])
    np.testing.assert_array_equal(a.k_scale.cpu().numpy(), b_.k_scale.cpu().numpy())
    q = torch.from_numpy(rng.randn(B, H, D).astype(np.float32)).cuda()
    assert torch.equal(a.decode(q), b_.decode(q))


def test_capacity_and_shapes_are_checked():
    import torch
    c = _cache(num_pages=4, num_kv_heads=1, head_dim=64, max_seqs=1, max_seq_len=32)
    k = torch.zeros(1, 1, 32, 64, device="cuda")
    c.prefill(k, k.clone(), [32])
    with pytest.raises(ValueError, match="holds"):
        c.append(torch.zeros(1, 1, 64, device="cuda"), torch.zeros(1, 1, 64, device="cuda"))
    with pytest.raises(ValueError):
        c.append(torch.zeros(1, 2, 64, device="cuda"), torch.zeros(1, 2, 64, device="cuda"))
    c.free(0)
    assert c.lengths()[0] == 0 and c.memory_stats()["pages"] == 0


def test_append_after_unsynced_steps():
    """step() advances the lengths on the device only; an append() right after
    (no sync_lengths()) must map pages from the device lengths. The lengths
    after the steps end exactly on page (and group) boundaries, so the append
    needs a page that the reservation did not map."""
    import torch
    B, H, D, group = 3, 2, 128, 128
    lens0 = [13, 125, 301]
    rng = np.random.RandomState(11)
    cache = _cache(num_pages=64, num_kv_heads=H, head_dim=D, max_seqs=B, max_seq_len=400)
    k0 = rng.randn(B, H, 320, D).astype(np.float32)
    v0 = rng.randn(B, H, 320, D).astype(np.float32)
    cache.prefill(torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda(), lens0)
    cache.reserve(B, 3)
    new = [(rng.randn(B, H, D).astype(np.float32), rng.randn(B, H, D).astype(np.float32))
           for _ in range(6)]
    q = torch.from_numpy(rng.randn(B, H, D).astype(np.float32)).cuda()
    for kn, vn in new[:3]:
        cache.step(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(), q)
    for kn, vn in new[3:]:
        cache.append(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda())
    lens = [n + 6 for n in lens0]
    assert list(cache.lengths()[:B]) == lens
    streams = []
    for b in range(B):
        kb = np.concatenate([k0[b, :, :lens0[b]]] + [kn[b][:, None] for kn, _ in new], axis=1)
        vb = np.concatenate([v0[b, :, :lens0[b]]] + [vn[b][:, None] for _, vn in new], axis=1)
        streams.append((kb, vb))
    _check_against_oracle(cache, streams, lens, group, "float32")


def test_append_at_the_anchor_size():
    """B8 H32 D128, float32 values, prefill lengths around 2048 (on and next to
    page and group edges), then two appends: every page and scale equals the
    grouped quantizer over the whole sequences."""
    import torch
    B, H, D, group = 8, 32, 128, 128
    lens0 = [2047, 2046, 2048, 2032, 1919, 1920, 2045, 1]
    rng = np.random.RandomState(21)
    k0 = rng.randn(B, H, 2048, D).astype(np.float32)
    v0 = rng.randn(B, H, 2048, D).astype(np.float32)
    cache = _cache(num_pages=B * 130, num_kv_heads=H, head_dim=D, max_seqs=B, max_seq_len=2064)
    cache.prefill(torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda(), lens0)
    new = [(rng.randn(B, H, D).astype(np.float32), rng.randn(B, H, D).astype(np.float32))
           for _ in range(2)]
    for kn, vn in new:
        cache.append(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda())
    streams = []
    for b in range(B):
        kb = np.concatenate([k0[b, :, :lens0[b]]] + [kn[b][:, None] for kn, _ in new], axis=1)
        vb = np.concatenate([v0[b, :, :lens0[b]]] + [vn[b][:, None] for _, vn in new], axis=1)
        streams.append((kb, vb))
    _check_against_oracle(cache, streams, [n + 2 for n in lens0], group, "float32")


def test_out_of_pages_keeps_the_page_table_consistent():
    """An append that runs out of pages after mapping a page for an earlier
    sequence must still write that page to the device table: the next append
    of that sequence uses it without mapping it again."""
    import torch
    rng = np.random.RandomState(3)
    c = _cache(num_pages=3, num_kv_heads=1, head_dim=64, max_seqs=2, max_seq_len=64,
               group_rows=64)
    k0 = rng.randn(2, 1, 16, 64).astype(np.float32)
    v0 = rng.randn(2, 1, 16, 64).astype(np.float32)
    c.prefill(torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda(), [16, 16])
    kn = [rng.randn(2, 1, 64).astype(np.float32) for _ in range(2)]
    vn = [rng.randn(2, 1, 64).astype(np.float32) for _ in range(2)]
    with pytest.raises(RuntimeError, match="out of pages"):
        c.append(torch.from_numpy(kn[0]).cuda(), torch.from_numpy(vn[0]).cuda())
    c.free(1)
    c.append(torch.from_numpy(kn[1]).cuda(), torch.from_numpy(vn[1]).cuda())
    streams = [(np.concatenate([k0[0], kn[1][0][:, None]], axis=1),
                np.concatenate([v0[0], vn[1][0][:, None]], axis=1)),
               (kn[1][1][:, None], vn[1][1][:, None])]
    _check_against_oracle(c, streams, [17, 1], 64, "float32")


def test_step_past_the_reservation_raises():
    import torch
    c = _cache(num_pages=4, num_kv_heads=1, head_dim=64, max_seqs=1, max_seq_len=64)
    k = torch.zeros(1, 1, 16, 64, device="cuda")
    c.prefill(k, k.clone(), [16])                # exactly one page mapped
    kn = torch.zeros(1, 1, 64, device="cuda")
    q = torch.zeros(1, 1, 64, device="cuda")
    with pytest.raises(RuntimeError, match="reserve"):
        c.step(kn, kn.clone(), q)
    assert int(c.seq_lens[0]) == 16              # nothing was launched
    c.reserve(1, 1)                              # maps the second page: 32 tokens
    for _ in range(16):
        c.step(kn, kn.clone(), q)
    with pytest.raises(RuntimeError, match="reserve"):
        c.step(kn, kn.clone(), q)                # both pages are full
    c.sync_lengths()
    assert c.lengths()[0] == 32 and int(c.seq_lens[0]) == 32


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill_and_appends(seed):
    """Seeded random caches (head dims, page sizes 8-32, scale groups 64-256,
    1-3 kv-heads, value dtypes, prefill lengths on and next to page and group
    edges, 1-40 appended tokens): pages, scales and values equal the grouped
    quantizer applied to each whole sequence, bit for bit."""
    import torch
    rng = np.random.RandomState(500 + seed)
    D = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 3]))
    B = int(rng.randint(1, 4))
    page_rows = int(rng.choice([8, 16, 32]))
    group = int(rng.choice([64, 128, 256]))
    vdtype = str(rng.choice(["float32", "float16", "bfloat16"]))
    steps = int(rng.randint(1, 41))
    edges = [0, 1, page_rows - 1, page_rows, group - 1, group, group + 1, 2 * group - 3]
    lens0 = [int(rng.choice(edges)) if rng.rand() < 0.7 else int(rng.randint(0, 400))
             for _ in range(B)]
    total = [n + steps for n in lens0]
    streams = [(rng.randn(H, n, D).astype(np.float32), rng.randn(H, n, D).astype(np.float32))
               for n in total]
    cap = max(total) + page_rows
    cache = _cache(num_pages=sum((n + page_rows) // page_rows + 1 for n in total) + 4,
                   num_kv_heads=H, head_dim=D, max_seqs=B, max_seq_len=cap,
                   page_rows=page_rows, group_rows=group, value_dtype=vdtype)
    vt = getattr(torch, vdtype)
    T0 = max(max(lens0), 1)
    k0 = np.zeros((B, H, T0, D), np.float32)
    v0 = np.zeros((B, H, T0, D), np.float32)
    for b in range(B):
        k0[b, :, :lens0[b]] = streams[b][0][:, :lens0[b]]
        v0[b, :, :lens0[b]] = streams[b][1][:, :lens0[b]]
    cache.prefill(torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda().to(vt), lens0)
    for s in range(steps):
        kn = np.stack([streams[b][0][:, lens0[b] + s] for b in range(B)])
        vn = np.stack([streams[b][1][:, lens0[b] + s] for b in range(B)])
        cache.append(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda().to(vt))
    # Compare through the cache's own page table, at its page size.
    kk = np.zeros((B, H, max(total), D), np.float32)
    for b in range(B):
        kk[b, :, :total[b]] = streams[b][0]
    qr, sr, zr = quantize_groups_ref(kk, np.array(total), group_size=group)
    kp = cache.k_pages.cpu().numpy()
    vp = cache.v_pages.float().cpu().numpy()
    sc, zc = cache.k_scale.cpu().numpy(), cache.k_zp.cpu().numpy()
    table = cache.page_table.cpu().numpy()
    assert list(cache.seq_lens[:B].cpu().numpy()) == total
    for b in range(B):
        ng = (total[b] + group - 1) // group
        np.testing.assert_array_equal(sc[b, :, :ng], sr[b, :, :ng])
        np.testing.assert_array_equal(zc[b, :, :ng], zr[b, :, :ng])
        for lp in range((total[b] + page_rows - 1) // page_rows):
            n = min(page_rows, total[b] - lp * page_rows)
            np.testing.assert_array_equal(kp[table[b, lp], :, :n],
                                          pack_int4(qr[b, :, lp * page_rows:lp * page_rows + n]))
            np.testing.assert_array_equal(
                vp[table[b, lp], :, :n],
                _stored(streams[b][1][:, lp * page_rows:lp * page_rows + n], vdtype))
