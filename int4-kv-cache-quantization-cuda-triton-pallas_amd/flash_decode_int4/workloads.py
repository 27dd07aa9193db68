"""Seeded synthetic inputs for the paged INT4 decode workloads.

Layout (one GPU's share, the device layout of flash_decode_int4):
  q          float32 [B, H, D]
  k          float32 [B, H, Tmax, D]   dense keys, quantized into pages
  v_pages    float32 [P, H, page_rows, D] (or float16) values, already paged
  page_table int32 [B, max_pages]      sequence b's logical page lp lives in
                                       physical page page_table[b, lp]
  seq_lens   int32 [B]

Pages are a seeded random permutation of the P = sum_b ceil(T_b/page_rows)
physical pages, dealt to the sequences in order (non-contiguous, shuffled);
unused table entries are 0. q, K and V are i.i.d. N(0, 1) and unscaled, as in
the reference benchmark's problem builder (benchmarks/bench_three_backend.py:113-129).

Named workloads (sizes of the reference's measurement plan):
  cpu         B1  H4  D64  T512, contiguous page table
  anchor      B8  H32 D128 T2048
  sweep_<T>   B8  H32 D128 T in {512, 2048, 8192, 32768}
  ragged      B32 H32 D128, T_b ~ U[1, 8192] with sequences 3, 17 forced to 0
              and partial last pages
  llama       B64 H32 D128 T4096, keys RoPE-rotated (base 10000, rotate-half
              pairing of channels d and d + D/2) at positions 0..T-1, then 4
              seeded channels per head scaled x20 (after rotation)
  gqa         B8 Hkv8 Hq32 D128 T8192 (four query heads per kv-head; the
              same key/value bytes as the anchor)

``backend="numpy"`` draws from ``np.random.RandomState(seed)`` (reproducible on
any host); ``backend="torch"`` draws on the GPU from a seeded
``torch.Generator`` (for the multi-GB workloads; different numbers, same
distribution).
"""

import numpy as np

PAGE_ROWS = 16
GROUP_ROWS = 128

WORKLOADS = {
    "cpu": dict(batch=1, heads=4, head_dim=64, tokens=512, contiguous=True),
    "anchor": dict(batch=8, heads=32, head_dim=128, tokens=2048),
    "sweep_512": dict(batch=8, heads=32, head_dim=128, tokens=512),
    "sweep_2048": dict(batch=8, heads=32, head_dim=128, tokens=2048),
    "sweep_8192": dict(batch=8, heads=32, head_dim=128, tokens=8192),
    "sweep_32768": dict(batch=8, heads=32, head_dim=128, tokens=32768),
    "ragged": dict(batch=32, heads=32, head_dim=128, tokens="ragged", max_tokens=8192),
    "llama": dict(batch=64, heads=32, head_dim=128, tokens=4096, rope=True, outliers=4),
    "gqa": dict(batch=8, heads=8, q_heads=32, head_dim=128, tokens=8192),
}


def ragged_lengths(batch, max_tokens, seed):
    """T_b ~ U[1, max_tokens]; sequences 3 and 17 (when present) are empty."""
    rng = np.random.RandomState(seed + 7)
    lens = rng.randint(1, max_tokens + 1, size=batch).astype(np.int32)
    for b in (3, 17):
        if b < batch:
            lens[b] = 0
    return lens


def page_layout(seq_lens, page_rows=PAGE_ROWS, seed=1234, contiguous=False):
    """(page_table int32 [B, max_pages], num_pages) for the given lengths."""
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    n_pages = (seq_lens + page_rows - 1) // page_rows
    P = int(n_pages.sum())
    max_pages = max(int(n_pages.max(initial=0)), 1)
    perm = np.arange(P) if contiguous else np.random.RandomState(seed + 1).permutation(P)
    table = np.zeros((len(seq_lens), max_pages), dtype=np.int32)
    off = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[off:off + n]
        off += n
    return table, max(P, 1)


def rope_rotate(k, base=10000.0):
    """Rotate-half RoPE of k[..., T, D] at positions 0..T-1 (float64 angles)."""
    T, D = k.shape[-2], k.shape[-1]
    half = D // 2
    inv = base ** (-np.arange(half, dtype=np.float64) / half)
    ang = np.arange(T, dtype=np.float64)[:, None] * inv[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x1, x2 = k[..., :half], k[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1).astype(np.float32)


def make_workload(name=None, *, batch=None, heads=None, head_dim=None, tokens=None,
                  seq_lens=None, max_tokens=None, contiguous=False, rope=False, outliers=0,
                  value_dtype="float32", seed=1234, backend="numpy", device="cuda",
                  q_heads=None):
    """Build a workload dict (see the module docstring for the layout); q has
    q_heads heads (default: heads), q-head h reading kv-head h // (q_heads // heads)."""
    if name is not None:
        spec = dict(WORKLOADS[name])
        batch, heads, head_dim = spec["batch"], spec["heads"], spec["head_dim"]
        q_heads = spec.get("q_heads", q_heads)
        tokens = spec["tokens"]
        max_tokens = spec.get("max_tokens", max_tokens)
        contiguous = spec.get("contiguous", contiguous)
        rope = spec.get("rope", rope)
        outliers = spec.get("outliers", outliers)
    if seq_lens is None:
        if tokens == "ragged":
            seq_lens = ragged_lengths(batch, max_tokens, seed)
        else:
            seq_lens = np.full(batch, int(tokens), dtype=np.int32)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    tmax = max(int(seq_lens.max(initial=0)), 1)
    table, P = page_layout(seq_lens, PAGE_ROWS, seed, contiguous)
    q_heads = heads if q_heads is None else int(q_heads)
    if q_heads % heads:
        raise ValueError("q_heads must be a multiple of heads")
    out = dict(name=name, batch=batch, heads=heads, q_heads=q_heads, head_dim=head_dim,
               seq_lens=seq_lens,
               page_table=table, num_pages=P, page_rows=PAGE_ROWS, group_rows=GROUP_ROWS,
               max_tokens=tmax)
    if backend == "numpy":
        rng = np.random.RandomState(seed)
        out["q"] = rng.randn(batch, q_heads, head_dim).astype(np.float32)
        k = rng.randn(batch, heads, tmax, head_dim).astype(np.float32)
        if value_dtype == "bfloat16":
            raise ValueError("bfloat16 values need backend='torch' (NumPy has no bfloat16)")
        out["v_pages"] = rng.randn(P, heads, PAGE_ROWS, head_dim).astype(value_dtype)
        if rope:
            k = rope_rotate(k)
        if outliers:
            orng = np.random.RandomState(seed + 3)
            for h in range(heads):
                ch = orng.choice(head_dim, outliers, replace=False)
                k[:, h, :, ch] *= np.float32(20.0)
        out["k"] = k
        return out
    import torch
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    out["q"] = torch.randn(batch, q_heads, head_dim, generator=g, device=dev)
    k = torch.randn(batch, heads, tmax, head_dim, generator=g, device=dev)
    vdt = getattr(torch, value_dtype)
    out["v_pages"] = torch.randn(P, heads, PAGE_ROWS, head_dim, generator=g, device=dev).to(vdt)
    if rope:
        half = head_dim // 2
        inv = 10000.0 ** (-torch.arange(half, dtype=torch.float64, device=dev) / half)
        ang = torch.arange(tmax, dtype=torch.float64, device=dev)[:, None] * inv[None, :]
        cos, sin = ang.cos().float(), ang.sin().float()
        x1, x2 = k[..., :half].clone(), k[..., half:].clone()
        k[..., :half] = x1 * cos - x2 * sin
        k[..., half:] = x2 * cos + x1 * sin
    if outliers:
        orng = np.random.RandomState(seed + 3)
        for h in range(heads):
            ch = torch.as_tensor(orng.choice(head_dim, outliers, replace=False), device=dev)
            k[:, h, :, ch] *= 20.0
    out["k"] = k
    return out


def decode_bytes(seq_lens, heads, head_dim, value_bytes=4, page_rows=PAGE_ROWS,
                 group_rows=GROUP_ROWS, q_heads=None):
    """Algorithmic HBM bytes of one decode over valid tokens only.

    Per (b, kv-head h): packed K T*D/2 + V T*D*value_bytes + scale and zp
    ceil(T/group)*D*8; per b: page table ceil(T/page_rows)*4 and seq_len 4;
    plus q and the output, B*Hq*D*4 each (Hq = q_heads, default heads).
    Split partials are excluded.
    """
    q_heads = heads if q_heads is None else q_heads
    total = 0
    for t in np.asarray(seq_lens, dtype=np.int64):
        t = int(t)
        g = (t + group_rows - 1) // group_rows
        total += heads * (t * head_dim // 2 + t * head_dim * value_bytes + g * head_dim * 8)
        total += ((t + page_rows - 1) // page_rows) * 4 + 4
    total += 2 * len(seq_lens) * q_heads * head_dim * 4
    return total


def quantize_bytes(seq_lens, heads, head_dim, page_rows=PAGE_ROWS, group_rows=GROUP_ROWS):
    """Algorithmic HBM bytes of one grouped quantization: read fp32 K, write packed K,
    scale and zp, read the page table (the B sequence lengths are not counted)."""
    total = 0
    for t in np.asarray(seq_lens, dtype=np.int64):
        t = int(t)
        g = (t + group_rows - 1) // group_rows
        total += heads * (t * head_dim * 4 + t * head_dim // 2 + g * head_dim * 8)
        total += ((t + page_rows - 1) // page_rows) * 4
    return total
