"""Paged INT4 key/value cache with the reference's page-table interface.

Drop-in for the reference's src/vllm_integration.py:29-102
(``INT4PagedKVCache(num_blocks, block_size, head_dim)`` with ``write_block``,
``free_block``, ``decode_attention(query, block_table)`` and
``memory_stats``), backed by a device page pool instead of host dicts:

  keys    uint8 [slots, block_size, Dp/2]  nibble-packed (Dp = head_dim
          padded to 64/128/256; padding channels hold nibble 0, scale 0)
  values  float16 [slots, block_size, Dp]  (the reference stores fp16 V)
  scales  float32 [slots, Dp] and zero-points, a block's group in each of
          its slots

``write_block`` quantizes the block on the GPU as ONE scale group over its
rows (reference :48-56, bit-exact with quantize_int4_ref) and writes the
packed rows into the block's slots (one per block_size rows; any block id). ``decode_attention`` runs the
packed-native split-K decode over the block table with no host unpack (the
reference unpacks every block on the host, :62-78). As in the reference all
queries attend the same block table.

``k_packed``, ``k_scale``, ``k_zp`` and ``v`` are read-only mappings
block_id -> NumPy copy of the stored data (``k_packed[i].nbytes`` is the
packed size of the rows written), so code written against the reference's
dicts keeps working.
"""

from typing import List

import numpy as np

from . import ops
from ._lib import load_binding


class _SlotView:
    """Read-only mapping block_id -> NumPy copy of one slot's stored data."""

    def __init__(self, cache, getter):
        self._cache = cache
        self._get = getter

    def __contains__(self, block_id):
        return block_id in self._cache.lens

    def __getitem__(self, block_id):
        if block_id not in self._cache.lens:
            raise KeyError(block_id)
        return self._get(block_id)

    def __len__(self):
        return len(self._cache.lens)

    def __iter__(self):
        return iter(list(self._cache.lens))

    def keys(self):
        return list(self._cache.lens)

    def values(self):
        return [self._get(b) for b in self._cache.lens]

    def items(self):
        return [(b, self._get(b)) for b in self._cache.lens]


class INT4PagedKVCache:
    """Paged KV cache: nibble-packed INT4 keys and fp16 values in HBM.

    The device pool is made of slots of block_size rows. A block -- any
    block id and any row count, as the reference's dictionaries allow --
    takes ceil(rows / block_size) slots; the pool starts with num_blocks
    slots and grows when the written blocks need more. Every slot of a block
    carries the block's scale and zero-point (one group over all its rows,
    as the reference quantizes a block), so the decode reads a long block
    as consecutive pages of one group, in row order.
    """

    def __init__(self, num_blocks: int, block_size: int, head_dim: int):
        import torch
        ops._require_device(None)
        if num_blocks < 1 or block_size < 1 or not 1 <= head_dim <= ops.HIP_MAX_HEAD_DIM:
            raise ValueError(
                f"need num_blocks >= 1, block_size >= 1 and 1 <= head_dim <= "
                f"{ops.HIP_MAX_HEAD_DIM}; got {num_blocks}, {block_size}, {head_dim}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.head_dim = head_dim
        self._dp = ops._padded_dim(head_dim)
        dev = torch.device("cuda")
        self._cap = num_blocks
        self._k = torch.zeros(num_blocks, block_size, self._dp // 2, dtype=torch.uint8, device=dev)
        self._v = torch.zeros(num_blocks, block_size, self._dp, dtype=torch.float16, device=dev)
        self._s = torch.zeros(num_blocks, self._dp, dtype=torch.float32, device=dev)
        self._z = torch.zeros(num_blocks, self._dp, dtype=torch.float32, device=dev)
        self._slots = {}                                  # block_id -> pool slots, in row order
        self._free = list(range(num_blocks - 1, -1, -1))  # pop() hands out slot 0 first
        self.lens = {}
        pk = (head_dim + 1) // 2
        self.k_packed = _SlotView(self, lambda b: self._rows(self._k, b)[:, :pk].cpu().numpy())
        self.k_scale = _SlotView(self, lambda b: self._s[self._slots[b][0], :head_dim].cpu().numpy())
        self.k_zp = _SlotView(self, lambda b: self._z[self._slots[b][0], :head_dim].cpu().numpy())
        self.v = _SlotView(self, lambda b: self._rows(self._v, b)[:, :head_dim].cpu().numpy())

    def _pieces(self, block_id):
        """(slot, rows) of each slot of a block, in row order."""
        n, bs = self.lens[block_id], self.block_size
        return [(s, min(bs, n - j * bs)) for j, s in enumerate(self._slots[block_id])]

    def _rows(self, pool, block_id):
        import torch
        return torch.cat([pool[s, :r] for s, r in self._pieces(block_id)])

    def _take(self, n):
        """n free slots; the pool grows (at least doubling) when too few are free."""
        import torch
        short = n - len(self._free)
        if short > 0:
            cap = max(self._cap + short, 2 * self._cap)
            for name in ("_k", "_v", "_s", "_z"):
                old = getattr(self, name)
                new = torch.zeros((cap,) + tuple(old.shape[1:]), dtype=old.dtype,
                                  device=old.device)
                new[:self._cap] = old
                setattr(self, name, new)
            self._free = list(range(cap - 1, self._cap - 1, -1)) + self._free
            self._cap = cap
        return [self._free.pop() for _ in range(n)]

    def write_block(self, block_id: int, k_block: np.ndarray, v_block: np.ndarray) -> None:
        """Quantize (one group over the block's rows), pack and store one block."""
        import torch
        # The reference asserts equal shapes (src/vllm_integration.py:50); the
        # same exception is raised explicitly so that it also holds under -O.
        if np.shape(k_block) != np.shape(v_block):
            raise AssertionError(f"k_block shape {np.shape(k_block)} != v_block shape "
                                 f"{np.shape(v_block)}")
        if np.ndim(k_block) != 2 or np.shape(k_block)[1] != self.head_dim:
            raise ValueError(f"block must be [rows, {self.head_dim}], got {np.shape(k_block)}")
        rows, d = np.shape(k_block)
        if rows < 1:
            raise ValueError("a block needs at least one row")
        dev = torch.device("cuda")
        # Everything that can fail happens before the cache changes.
        k_t = torch.from_numpy(np.ascontiguousarray(k_block, dtype=np.float32)).to(dev)
        kq = torch.zeros(rows, self._dp // 2, dtype=torch.uint8, device=dev)
        sc = torch.zeros(self._dp, dtype=torch.float32, device=dev)
        zp = torch.zeros(self._dp, dtype=torch.float32, device=dev)
        load_binding().quantize_rows_into(k_t, kq, sc, zp, True)
        v_t = torch.from_numpy(np.ascontiguousarray(np.asarray(v_block).astype(np.float16)))
        v_t = v_t.to(dev)
        old = self._slots.pop(block_id, None)
        if old:
            self._free.extend(reversed(old))
        self.lens.pop(block_id, None)
        slots = self._take(-(-rows // self.block_size))
        bs = self.block_size
        for j, s in enumerate(slots):
            r0, r1 = j * bs, min(rows, (j + 1) * bs)
            self._k[s, :r1 - r0] = kq[r0:r1]
            self._v[s, :r1 - r0, :d] = v_t[r0:r1]
            self._s[s] = sc
            self._z[s] = zp
        self._slots[block_id] = slots
        self.lens[block_id] = rows

    def free_block(self, block_id: int) -> None:
        slots = self._slots.pop(block_id, None)
        if slots:
            self._free.extend(reversed(slots))
        self.lens.pop(block_id, None)

    def decode_attention(self, query: np.ndarray, block_table: List[int]) -> np.ndarray:
        """Fused INT4 attention of every query over the blocks of ``block_table``."""
        import torch
        query = np.asarray(query, dtype=np.float32)
        if query.ndim != 3 or query.shape[2] != self.head_dim:
            raise ValueError(f"query must be [batch, heads, {self.head_dim}], got "
                             f"{query.shape}")
        pieces = [p for b in block_table for p in self._pieces(b)]  # KeyError for unknown
        B, H, D = query.shape
        if not pieces:
            return np.zeros(query.shape, dtype=np.float32)
        n = len(pieces)
        dev = torch.device("cuda")
        qp = np.zeros((B, H, self._dp), dtype=np.float32)
        qp[..., :D] = query
        q_t = torch.from_numpy(qp).to(dev)
        table = torch.tensor([s for s, _ in pieces], dtype=torch.int32,
                             device=dev).view(1, n).expand(B, n)
        lens_t = torch.tensor([r for _, r in pieces], dtype=torch.int32,
                              device=dev).view(1, n).expand(B, n)
        nb, bs, dp = self._cap, self.block_size, self._dp
        out = load_binding().decode_paged(
            q_t, self._k.view(nb, 1, bs, dp // 2), self._v.view(nb, 1, bs, dp), self._s,
            self._z, table, None, lens_t, 1, n, 0)
        return out[..., :D].cpu().numpy()

    def memory_stats(self) -> dict:
        """The stored data against fp16 K+V, counted as the reference counts its
        arrays (src/vllm_integration.py:80-102: packed key rows, fp16 value
        rows, a scale and a zero-point per block), plus ``pool_mb``, what the
        device pool holds for the written blocks (whole slots of block_size
        rows at the padded head_dim)."""
        n = len(self.lens)
        if n == 0:
            return {"blocks": 0, "stored_mb": 0.0, "fp16_equiv_mb": 0.0, "ratio": 0.0,
                    "pool_mb": 0.0}
        D = self.head_dim
        rows = sum(self.lens.values())
        stored = rows * ((D + 1) // 2) + rows * D * 2 + n * 2 * D * 4
        fp16_equiv = rows * D * 2 * 2
        slot = (self._k[0].numel() * self._k.element_size()
                + self._v[0].numel() * self._v.element_size()
                + 2 * self._s[0].numel() * self._s.element_size())
        pool = sum(len(s) for s in self._slots.values()) * slot
        return {
            "blocks": n,
            "stored_mb": round(stored / 1048576, 3),
            "fp16_equiv_mb": round(fp16_equiv / 1048576, 3),
            "ratio": round(fp16_equiv / max(stored, 1), 2),
            "pool_mb": round(pool / 1048576, 3),
        }


class INT4PagedSequenceCache:
    """Batched per-sequence INT4 cache in the decode kernel's native layout.

    The batched counterpart of the reference's page-table cache
    (src/vllm_integration.py:29-102): sequences, kv-heads and 128-token scale
    groups instead of one shared block stream, and a decode-time append that
    writes one token per sequence per step on the device.

      k_pages    uint8 [num_pages, kv_heads, page_rows, D/2]  nibble-packed keys
      v_pages    float32, float16 or bfloat16 [num_pages, kv_heads, page_rows, D]
      k_scale    float32 [max_seqs, kv_heads, max_groups, D]  (and k_zp)
      page_table int32 [max_seqs, max_pages_per_seq]
      seq_lens   int32 [max_seqs]
      k_stage    float32 [max_seqs, kv_heads, group_rows, D]  float keys of
                 each sequence's open (partial) scale group

    Sequences 0..B-1 of a call are the first B slots. Pages come from a host
    free list; the page table is updated on the device when a sequence enters
    a new page. A partial last group is quantized over its valid rows, so after
    any mix of prefill and append the pages and scales equal the grouped
    quantizer applied to each whole sequence (reference
    tests/test_perplexity_harness.py:122-131).
    """

    def __init__(self, num_pages: int, num_kv_heads: int, head_dim: int, max_seqs: int,
                 max_seq_len: int, page_rows: int = 16, group_rows: int = 128,
                 value_dtype: str = "float32"):
        import torch
        ops._require_device(None)
        if head_dim not in (64, 128, 256):
            raise ValueError(f"head_dim must be 64, 128 or 256, got {head_dim}")
        if group_rows not in (64, 128, 256) or group_rows % page_rows:
            raise ValueError("group_rows must be 64, 128 or 256 and a multiple of page_rows")
        if value_dtype not in ("float32", "float16", "bfloat16"):
            raise ValueError("value_dtype must be float32, float16 or bfloat16")
        if min(num_pages, num_kv_heads, max_seqs, max_seq_len, page_rows) < 1:
            raise ValueError("sizes must be positive")
        self.num_pages, self.num_kv_heads, self.head_dim = num_pages, num_kv_heads, head_dim
        self.max_seqs, self.page_rows, self.group_rows = max_seqs, page_rows, group_rows
        self.max_pages_per_seq = (max_seq_len + page_rows - 1) // page_rows
        groups = (self.max_pages_per_seq * page_rows + group_rows - 1) // group_rows
        dev = torch.device("cuda")
        vdt = getattr(torch, value_dtype)
        H, D = num_kv_heads, head_dim
        self.k_pages = torch.zeros(num_pages, H, page_rows, D // 2, dtype=torch.uint8, device=dev)
        self.v_pages = torch.zeros(num_pages, H, page_rows, D, dtype=vdt, device=dev)
        self.k_scale = torch.zeros(max_seqs, H, groups, D, dtype=torch.float32, device=dev)
        self.k_zp = torch.zeros_like(self.k_scale)
        self.page_table = torch.zeros(max_seqs, self.max_pages_per_seq, dtype=torch.int32,
                                      device=dev)
        self.seq_lens = torch.zeros(max_seqs, dtype=torch.int32, device=dev)
        # step(): per-sequence arrival counters of the one-launch step (zero
        # between steps) and the advanced lengths of the two-launch step.
        self._step_counters = torch.zeros(max_seqs, dtype=torch.int32, device=dev)
        self._lens_next = torch.zeros(max_seqs, dtype=torch.int32, device=dev)
        self.k_stage = torch.zeros(max_seqs, H, group_rows, D, dtype=torch.float32, device=dev)
        self._free = list(range(num_pages - 1, -1, -1))
        self._pages = [[] for _ in range(max_seqs)]
        self._lens = np.zeros(max_seqs, dtype=np.int64)
        self._mapped = np.zeros(max_seqs, dtype=np.int64)   # tokens the mapped pages hold
        # Eager step() calls since the host lengths were last read from the
        # device (replays of a captured step() are not counted).
        self._unsynced_steps = 0

    # ---- page bookkeeping (host) -------------------------------------------

    def _grow(self, b: int, n_tokens: int, updates: list) -> None:
        """Map the pages sequence b needs to hold n_tokens, taking them from
        the free list in one slice (the order successive pops would give)."""
        need = (n_tokens + self.page_rows - 1) // self.page_rows
        if need > self.max_pages_per_seq:
            raise ValueError(f"sequence {b} would hold {n_tokens} tokens; the cache holds "
                             f"{self.max_pages_per_seq * self.page_rows} per sequence")
        have = len(self._pages[b])
        take = min(need - have, len(self._free))
        if take > 0:
            new = self._free[len(self._free) - take:][::-1]
            del self._free[len(self._free) - take:]
            updates.append((b, have, np.asarray(new, dtype=np.int64)))
            self._pages[b].extend(new)
            self._mapped[b] = len(self._pages[b]) * self.page_rows
        if need > len(self._pages[b]):
            raise RuntimeError("out of pages")

    def _grow_all(self, targets) -> None:
        """Map pages so that sequence b holds n tokens, for (b, n) in targets.
        Pages taken before a failure (out of pages, too long) are written to
        the device page table too, so the host lists and the table agree."""
        updates = []
        try:
            for b, n in targets:
                self._grow(b, n, updates)
        finally:
            self._apply(updates)

    def _apply(self, updates: list) -> None:
        """Write (sequence, first logical page, physical pages) runs into the
        device page table with one scatter."""
        import torch
        if not updates:
            return
        seq = np.concatenate([np.full(len(p), b, np.int64) for b, _, p in updates])
        col = np.concatenate([np.arange(lp, lp + len(p), dtype=np.int64) for _, lp, p in updates])
        phys = np.concatenate([p for _, _, p in updates])
        u = torch.from_numpy(np.stack([seq, col, phys])).cuda()
        self.page_table[u[0], u[1]] = u[2].to(torch.int32)

    def _sync_if_stepped(self) -> None:
        # step() advances the lengths on the device only; host-side page
        # mapping must start from the device's lengths.
        if self._unsynced_steps:
            self.sync_lengths()

    def _release(self, b: int) -> None:
        """Host side of free(): sequence b's pages go back to the free list."""
        self._free.extend(reversed(self._pages[b]))
        self._pages[b] = []
        self._mapped[b] = 0
        self._lens[b] = 0

    def free(self, b: int) -> None:
        """Release sequence b's pages; its slot starts empty."""
        self._sync_if_stepped()
        self._release(b)
        self.seq_lens[b] = 0

    # ---- writes ------------------------------------------------------------

    def _check_prefill(self, k, v, lens) -> None:
        """Every condition prefill() and the quantizer need, checked before
        the cache is touched, so a rejected call leaves it as it was."""
        import torch
        if not isinstance(k, torch.Tensor) or not isinstance(v, torch.Tensor):
            raise TypeError("k and v must be torch tensors on the GPU")
        if k.dim() != 4 or tuple(v.shape) != tuple(k.shape):
            raise ValueError("k and v must be [batch, kv_heads, tokens, head_dim] of this cache")
        B, H, T, D = k.shape
        if (H, D) != (self.num_kv_heads, self.head_dim):
            raise ValueError("k and v must be [batch, kv_heads, tokens, head_dim] of this cache")
        if B > self.max_seqs or len(lens) != B or (lens < 0).any() or (lens > T).any():
            raise ValueError("bad batch size or sequence lengths")
        cap = self.max_pages_per_seq * self.page_rows
        if (lens > cap).any():
            raise ValueError(f"a sequence of {int(lens.max())} tokens exceeds the "
                             f"{cap} tokens per sequence this cache holds")
        if not (k.is_cuda and v.is_cuda):
            raise RuntimeError("k and v must be GPU (cuda device) tensors")
        if k.dtype != torch.float32:
            raise TypeError(f"k must be float32, got {k.dtype}")
        if (k.stride(3) != 1 or k.data_ptr() % 16
                or any((k.stride(i) * 4) % 16 for i in range(3))):
            raise ValueError("k needs contiguous rows starting on 16-byte boundaries")
        if v.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise TypeError(f"v must be float32, float16 or bfloat16, got {v.dtype}")
        need = int(((lens + self.page_rows - 1) // self.page_rows).sum())
        held = sum(len(self._pages[b]) for b in range(B))
        if need > len(self._free) + held:
            raise RuntimeError(f"out of pages: the batch needs {need}, "
                               f"{len(self._free) + held} are free or held by it")

    def prefill(self, k, v, seq_lens) -> None:
        """Start sequences 0..B-1 from k, v [B, kv_heads, T, D] (keys float32,
        values converted to the cache's dtype) with seq_lens[b] <= T valid
        tokens. Raises before changing the cache when an argument is
        unusable."""
        import torch
        lens = np.asarray(seq_lens.cpu() if hasattr(seq_lens, "cpu") else seq_lens, np.int64)
        lens = lens.reshape(-1)
        self._check_prefill(k, v, lens)
        B, _, T, _ = k.shape
        self._sync_if_stepped()
        for b in range(B):
            self._release(b)
        try:
            self._grow_all((b, int(lens[b])) for b in range(B))
        except Exception:
            self.seq_lens[:B] = 0  # the released slots are empty on the device too
            raise
        lens_t = torch.as_tensor(lens, dtype=torch.int32).cuda()
        self.seq_lens[:B] = lens_t
        self._lens[:B] = lens
        ops.quantize_int4_paged(k, self.seq_lens[:B], self.page_table[:B], self.k_pages,
                                self.k_scale[:B], self.k_zp[:B], self.group_rows)
        # Values: token t of sequence b -> row t % page_rows of physical page
        # page_table[b, t // page_rows], gathered and scattered on the device.
        if T and lens.any():
            dev = self.seq_lens.device
            t = torch.arange(T, device=dev)
            bi, ti = torch.nonzero(t[None, :] < lens_t[:, None], as_tuple=True)
            pages = self.page_table[bi, ti // self.page_rows].long()
            self.v_pages[pages, :, ti % self.page_rows, :] = v[bi, :, ti, :].to(self.v_pages.dtype)
        # Open groups: the float keys of each sequence's partial last group.
        for b in range(B):
            r = int(lens[b]) % self.group_rows
            if r:
                g0 = int(lens[b]) - r
                self.k_stage[b, :, :r] = k[b, :, g0:g0 + r]

    def append(self, k_new, v_new) -> None:
        """Append one token to each of sequences 0..B-1: k_new float32 and v_new
        (the cache's value dtype) [B, kv_heads, D]. One kernel launch."""
        B = k_new.shape[0]
        if B > self.max_seqs or tuple(k_new.shape) != (B, self.num_kv_heads, self.head_dim):
            raise ValueError("k_new must be [batch <= max_seqs, kv_heads, head_dim]")
        self._sync_if_stepped()
        self._grow_all((b, int(self._lens[b]) + 1) for b in range(B))
        load_binding().append_paged(k_new, v_new.to(self.v_pages.dtype), self.k_stage[:B],
                                    self.k_pages, self.v_pages, self.k_scale[:B],
                                    self.k_zp[:B], self.page_table[:B], self.seq_lens[:B],
                                    self.group_rows)
        self.seq_lens[:B] += 1
        self._lens[:B] += 1

    # ---- device-only decode steps (graph capture) ----------------------------

    def reserve(self, batch: int, n_tokens: int) -> None:
        """Map the pages sequences 0..batch-1 need to grow by n_tokens, so that
        step() does no host work until they have."""
        self._sync_if_stepped()
        self._grow_all((b, int(self._lens[b]) + n_tokens) for b in range(batch))

    def step(self, k_new, v_new, query, num_splits: int = 0):
        """One decode step on the device alone: append (k_new, v_new) [B,
        kv_heads, D] at each sequence's length, advance the lengths on the
        device, attend with query [B, Hq, D] (float32, float16 or bfloat16);
        returns [B, Hq, D] in the query's dtype.
        No host bookkeeping happens, so the call can be captured in a HIP
        graph and replayed. Each graph launch leaves the GPU idle for a few
        microseconds before the graph's first kernel (about 4.3-4.7 us on
        MI355X, measured: a graph holding one B8 H32 T2048 step replays in
        58.2 us against 53.9 us eager), so capture it together with the rest
        of the token step (the other layers' caches) or several steps per
        graph (53.6 us per step from a graph of eight). The pages must already
        be mapped (reserve), and
        lengths() reflects the steps only after sync_lengths(); append(),
        prefill(), reserve() and free() read the device lengths first.
        An eager call whose token would fall outside the reserved pages raises
        RuntimeError before anything is launched (the host knows the lengths up
        to the eager steps since the last sync; replays are the caller's to
        keep within the reservation)."""
        B = k_new.shape[0]
        if B > self.max_seqs or tuple(k_new.shape) != (B, self.num_kv_heads, self.head_dim):
            raise ValueError("k_new must be [batch <= max_seqs, kv_heads, head_dim]")
        short = np.nonzero(self._lens[:B] + self._unsynced_steps + 1 > self._mapped[:B])[0]
        if len(short):
            raise RuntimeError(f"step() would write past the pages reserved for sequence "
                               f"{int(short[0])}; call reserve() first")
        self._unsynced_steps += 1
        if num_splits:
            # An explicit split count: the two-launch form (the append writes
            # seq_lens + 1 to _lens_next, the decode attends over it with the
            # given splits and copies it back to seq_lens when it ends).
            C = load_binding()
            C.append_paged_advance(k_new, v_new, self.k_stage[:B], self.k_pages, self.v_pages,
                                   self.k_scale[:B], self.k_zp[:B], self.page_table[:B],
                                   self.seq_lens[:B], self.group_rows, self._lens_next[:B])
            return C.decode_paged_advance(query, self.k_pages, self.v_pages, self.k_scale[:B],
                                          self.k_zp[:B], self.page_table[:B],
                                          self._lens_next[:B],
                                          self.group_rows // self.page_rows,
                                          self.max_pages_per_seq, int(num_splits),
                                          self.seq_lens[:B])
        # One launch (plus the split merge) with one q-head per kv-head when
        # the splits hold whole scale groups, two otherwise (fdi4_decode_step
        # decides).
        return load_binding().decode_step(query, k_new, v_new, self.k_stage, self.k_pages,
                                          self.v_pages, self.k_scale, self.k_zp,
                                          self.page_table, self.seq_lens, self.group_rows,
                                          self._step_counters, self._lens_next)

    def sync_lengths(self) -> None:
        """Refresh the host copy of the lengths from the device (after step())."""
        self._lens[:] = self.seq_lens.cpu().numpy()
        self._unsynced_steps = 0

    # ---- reads -------------------------------------------------------------

    def decode(self, query, num_splits: int = 0):
        """Fused INT4 attention of query [B, Hq, D] (float32, float16 or bfloat16;
        Hq a multiple of kv_heads) over sequences 0..B-1; returns [B, Hq, D] in
        the query's dtype (float32 arithmetic, one rounding at the end)."""
        B = query.shape[0]
        return ops.flash_decode_paged(query, self.k_pages, self.v_pages, self.k_scale[:B],
                                      self.k_zp[:B], self.page_table[:B], self.seq_lens[:B],
                                      self.group_rows, num_splits,
                                      max_pages=self.max_pages_per_seq)

    def lengths(self) -> np.ndarray:
        return self._lens.copy()

    def memory_stats(self) -> dict:
        """Bytes of the pages in use (packed keys, values, their scale groups)
        against the same tokens as fp16 K + V."""
        used = sum(len(p) for p in self._pages)
        H, D, pr = self.num_kv_heads, self.head_dim, self.page_rows
        vb = self.v_pages.element_size()
        stored = used * H * pr * (D // 2 + D * vb) + int(
            sum((n + self.group_rows - 1) // self.group_rows for n in self._lens)) * H * D * 8
        tokens = int(self._lens.sum())
        fp16 = tokens * H * D * 2 * 2
        return {"pages": used, "tokens": tokens, "stored_mb": round(stored / 1048576, 3),
                "fp16_equiv_mb": round(fp16 / 1048576, 3),
                "ratio": round(fp16 / max(stored, 1), 2)}
