"""Oracle: online-softmax flash decoding over INT4 paged keys.

Test infrastructure only (see ``oracle/__init__.py``).

``online_softmax_ref`` restates the reference page loop
``src/flash_decode_ref.py:30-139`` op for op in float32: skip a page whose
length is 0 (:78-82), truncate to the valid rows (:85-86), dequantize
``q*s - zp*s`` (:92), unscaled logits ``q @ k.T`` (:97), running max (:106),
rescale ``exp(m_old - m_new)`` (:109), ``p = exp(logits - m_new)`` (:113),
``l = l*c + sum(p)`` (:119), ``o = o*c + p @ v`` (:124-126), and finally
``o / max(l, 1e-10)`` (:136-137).

``f64_attention`` is the float64 arbiter of the reference's own tests
(tests/test_pallas_flash_decode.py:53-78): it concatenates every live page
and evaluates one full softmax, so it shares no accumulation strategy with
the page loop. ``float32_floor`` is the reference's sqrt(D)*eps*mean|o|
round-off estimate (same file :151-157).

The paged functions apply these per (sequence, kv-head) stream -- the
construction the reference prescribes for distinct KV per head ("one call per
(sequence, head) stream", src/ops.py:189-192) -- to the device layout:
packed keys [P, Hkv, page, ceil(D/2)], values [P, Hkv, page, D], group
scales [B, Hkv, G, D], page table [B, max_pages], sequence lengths [B].

Pinned by (tests/test_oracle_attention.py): the float64 arbiter within 3x
the float32 floor; the arbiter against scipy.special.softmax; the textbook
special cases (q = 0 gives the mean of the valid value rows; one live token
gives that token's value row exactly); page-decomposition invariance;
empty pages skipped; all-empty sequences give exact zeros.
"""

import numpy as np

from .quantize import unpack_int4

L_FLOOR = 1e-10


def online_softmax_ref(query, key_scale_zp_list, value_list, block_lens=None):
    """Page-loop online softmax; returns (output [B,H,D], log_partition [B,H]).

    reference: src/flash_decode_ref.py:30-139.
    """
    if query.ndim != 3:
        raise AssertionError(f"Query must be 3D (batch, heads, dim), got {query.ndim}D")
    nb_, nh, _ = query.shape
    n = len(key_scale_zp_list)
    if len(value_list) != n:
        raise AssertionError("Number of blocks must match")
    if block_lens is None:
        block_lens = np.array([key_scale_zp_list[i][0].shape[0] for i in range(n)])

    m = np.full((nb_, nh), -np.inf, dtype=np.float32)
    l = np.zeros((nb_, nh), dtype=np.float32)
    o = np.zeros(query.shape, dtype=np.float32)

    for i in range(n):
        kq, s, z = key_scale_zp_list[i]
        rows = int(block_lens[i])
        if rows == 0:
            continue
        kq = kq[:rows]
        v = value_list[i][:rows]
        k = kq.astype(np.float32) * s[np.newaxis, :] - z[np.newaxis, :] * s[np.newaxis, :]
        logits = np.matmul(query, k.T)
        m_new = np.maximum(m, np.max(logits, axis=-1))
        c = np.exp(m - m_new)
        p = np.exp(logits - m_new[:, :, np.newaxis])
        l = l * c + np.sum(p, axis=-1)
        o = o * c[:, :, np.newaxis] + np.einsum('bhs,sd->bhd', p, v)
        m = m_new

    lp = np.log(np.maximum(l, L_FLOOR))
    o = o / np.maximum(l, L_FLOOR)[:, :, np.newaxis]
    return o, lp


def online_softmax_fp32_ref(query, key_list, value_list, block_lens=None):
    """Unquantized page loop. reference: src/flash_decode_ref.py:177-223."""
    nb_, nh, _ = query.shape
    n = len(key_list)
    if block_lens is None:
        block_lens = np.array([key_list[i].shape[0] for i in range(n)])
    m = np.full((nb_, nh), -np.inf, dtype=np.float32)
    l = np.zeros((nb_, nh), dtype=np.float32)
    o = np.zeros(query.shape, dtype=np.float32)
    for i in range(n):
        rows = int(block_lens[i])
        if rows == 0:
            continue
        k = key_list[i].astype(np.float32)[:rows]
        v = value_list[i].astype(np.float32)[:rows]
        logits = np.matmul(query, k.T)
        m_new = np.maximum(m, np.max(logits, axis=-1))
        c = np.exp(m - m_new)
        p = np.exp(logits - m_new[:, :, np.newaxis])
        l = l * c + np.sum(p, axis=-1)
        o = o * c[:, :, np.newaxis] + np.einsum('bhs,sd->bhd', p, v)
        m = m_new
    return o / np.maximum(l, L_FLOOR)[:, :, np.newaxis]


def flash_decode_ref(query, key_list, value_list, scale_list=None, zp_list=None,
                     block_lens=None, use_quantization=False):
    """reference: src/flash_decode_ref.py:142-174."""
    if use_quantization:
        if scale_list is None or zp_list is None:
            raise AssertionError("scales and zero-points are required")
        ksz = [(key_list[i], scale_list[i], zp_list[i]) for i in range(len(key_list))]
        return online_softmax_ref(query, ksz, value_list, block_lens)[0]
    return online_softmax_fp32_ref(query, key_list, value_list, block_lens)


def f64_attention(query, k_q, k_s, k_z, vals, lens):
    """Float64 full-softmax evaluation of the same mathematics (the arbiter).

    Dequantization is exact in float64 (4-bit x 24-bit and 24-bit x 24-bit
    products fit in 53 bits). reference: tests/test_pallas_flash_decode.py:53-78.
    """
    nb_, nh, d = query.shape
    q64 = np.asarray(query, np.float64)
    logits, values = [], []
    for i in range(len(k_q)):
        rows = int(lens[i])
        if rows == 0:
            continue
        s64 = np.asarray(k_s[i], np.float64)
        z64 = np.asarray(k_z[i], np.float64)
        k64 = np.asarray(k_q[i][:rows], np.float64) * s64 - z64 * s64
        logits.append(q64 @ k64.T)
        values.append(np.asarray(vals[i][:rows], np.float64))
    if not logits:
        return np.zeros((nb_, nh, d), np.float64)
    lg = np.concatenate(logits, axis=-1)
    vv = np.concatenate(values, axis=0)
    m = lg.max(axis=-1, keepdims=True)
    p = np.exp(lg - m)
    return np.einsum('bhs,sd->bhd', p, vv) / p.sum(axis=-1, keepdims=True)


def float32_floor(truth, dim):
    """sqrt(D) * eps32 * mean|o|. reference: tests/test_pallas_flash_decode.py:151-157."""
    return float(np.sqrt(dim) * np.finfo(np.float32).eps * np.abs(truth).mean())


def _stream_pages(k_cache, v_cache, k_scale, k_zp, page_table, seq_lens, b, hk,
                  head_dim, page_size, pages_per_group):
    """The logical pages of stream (b, hk) in the list form the page loop takes."""
    n = int(seq_lens[b])
    n_pages = (n + page_size - 1) // page_size
    kqs, ss, zs, vs, lens = [], [], [], [], []
    for lp in range(n_pages):
        phys = int(page_table[b, lp])
        kqs.append(unpack_int4(k_cache[phys, hk], head_dim))
        vs.append(np.asarray(v_cache[phys, hk], np.float32))
        g = lp // pages_per_group
        ss.append(k_scale[b, hk, g])
        zs.append(k_zp[b, hk, g])
        lens.append(min(page_size, n - lp * page_size))
    return kqs, ss, zs, vs, np.asarray(lens, np.int32)


def paged_decode_ref(query, k_cache, v_cache, k_scale, k_zp, page_table, seq_lens,
                     page_size=16, group_size=128):
    """Float32 page-loop oracle, one call per (sequence, kv-head) stream.

    query [B, Hq, D]; q-head h reads kv-head h // (Hq // Hkv).
    """
    B, Hq, D = query.shape
    Hkv = k_cache.shape[1]
    rep = Hq // Hkv
    ppg = group_size // page_size
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        for hk in range(Hkv):
            kqs, ss, zs, vs, lens = _stream_pages(k_cache, v_cache, k_scale, k_zp,
                                                  page_table, seq_lens, b, hk, D,
                                                  page_size, ppg)
            for h in range(hk * rep, (hk + 1) * rep):
                out[b, h] = online_softmax_ref(query[b:b + 1, h:h + 1],
                                               list(zip(kqs, ss, zs)), vs, lens)[0][0, 0]
    return out


def paged_decode_f64(query, k_cache, v_cache, k_scale, k_zp, page_table, seq_lens,
                     page_size=16, group_size=128):
    """Float64 arbiter over the paged layout, one stream at a time."""
    B, Hq, D = query.shape
    Hkv = k_cache.shape[1]
    rep = Hq // Hkv
    ppg = group_size // page_size
    out = np.zeros((B, Hq, D), np.float64)
    for b in range(B):
        for hk in range(Hkv):
            kqs, ss, zs, vs, lens = _stream_pages(k_cache, v_cache, k_scale, k_zp,
                                                  page_table, seq_lens, b, hk, D,
                                                  page_size, ppg)
            qh = query[b:b + 1, hk * rep:(hk + 1) * rep]
            out[b, hk * rep:(hk + 1) * rep] = f64_attention(qh, kqs, ss, zs, vs, lens)[0]
    return out
