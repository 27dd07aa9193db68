"""Host-side input contract of the paged attention entry points.

Same contract and message substrings as the reference's
src/_validate.py:11-64 ("query must be", "same length", "key page",
"value page", "scale/zero-point", "entries", "outside"), so malformed input
raises the same ValueError here as on the reference. The decode
kernel additionally clamps every page length to [0, page_rows] and every
page-table entry to the pool, so a malformed call that bypasses this check
cannot read outside its buffers.
"""

import numpy as np


def normalize_attention_inputs(query, k_q_blocks, k_scales, k_zps, v_blocks, block_lens):
    """Validate list-of-pages attention inputs; return (query, block_lens int32)."""
    query = np.asarray(query)
    if query.ndim != 3:
        raise ValueError(f"query must be [batch, heads, head_dim], got shape {query.shape}")
    head_dim = query.shape[2]

    n = len(k_q_blocks)
    counts = (len(k_scales), len(k_zps), len(v_blocks))
    if any(c != n for c in counts):
        raise ValueError(
            "k_q_blocks, k_scales, k_zps and v_blocks must have the same length, "
            f"got {n}, {counts[0]}, {counts[1]}, {counts[2]}")

    rows = np.zeros(n, dtype=np.int64)
    for i in range(n):
        ks, vs = np.shape(k_q_blocks[i]), np.shape(v_blocks[i])
        if len(ks) != 2 or ks[1] != head_dim:
            raise ValueError(f"key page {i} must be [rows, {head_dim}], got shape {ks}")
        if vs != ks:
            raise ValueError(
                f"value page {i} has shape {vs}, expected {ks} to match its key page")
        ss, zs = np.shape(k_scales[i]), np.shape(k_zps[i])
        if ss != (head_dim,) or zs != (head_dim,):
            raise ValueError(
                f"scale/zero-point for page {i} must have shape ({head_dim},), "
                f"got {ss} and {zs}")
        rows[i] = ks[0]

    if block_lens is None:
        return query, rows.astype(np.int32)
    lens = np.asarray(block_lens).astype(np.int64).reshape(-1)
    if lens.shape[0] != n:
        raise ValueError(f"block_lens has {lens.shape[0]} entries for {n} pages")
    bad = np.flatnonzero((lens < 0) | (lens > rows))
    if bad.size:
        i = int(bad[0])
        raise ValueError(
            f"block_lens[{i}] = {int(lens[i])} is outside [0, {int(rows[i])}], "
            "the number of rows actually present in that page")
    return query, lens.astype(np.int32)
