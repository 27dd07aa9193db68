"""Paged INT4 key/value cache with the reference's page-table interface.

Drop-in for the reference's src/vllm_integration.py:29-102
(``INT4PagedKVCache(num_blocks, block_size, head_dim)`` with ``write_block``,
``free_block``, ``decode_attention(query, block_table)`` and
``memory_stats``), backed by a device page pool instead of host dicts:

  keys    uint8 [num_blocks, block_size, Dp/2]  nibble-packed (Dp = head_dim
          padded to 64/128/256; padding channels hold nibble 0, scale 0)
  values  float16 [num_blocks, block_size, Dp]  (the reference stores fp16 V)
  scales  float32 [num_blocks, Dp] and zero-points, one group per block

``write_block`` quantizes the block on the GPU as ONE scale group over its
rows (reference :48-56, bit-exact with quantize_int4_ref) and writes the
packed rows straight into the block's slot. ``decode_attention`` runs the
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
    """Paged KV cache: nibble-packed INT4 keys and fp16 values in HBM."""

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
        self._k = torch.zeros(num_blocks, block_size, self._dp // 2, dtype=torch.uint8, device=dev)
        self._v = torch.zeros(num_blocks, block_size, self._dp, dtype=torch.float16, device=dev)
        self._s = torch.zeros(num_blocks, self._dp, dtype=torch.float32, device=dev)
        self._z = torch.zeros(num_blocks, self._dp, dtype=torch.float32, device=dev)
        self.lens = {}
        pk = (head_dim + 1) // 2
        self.k_packed = _SlotView(self, lambda b: self._k[b, :self.lens[b], :pk].cpu().numpy())
        self.k_scale = _SlotView(self, lambda b: self._s[b, :head_dim].cpu().numpy())
        self.k_zp = _SlotView(self, lambda b: self._z[b, :head_dim].cpu().numpy())
        self.v = _SlotView(self, lambda b: self._v[b, :self.lens[b], :head_dim].cpu().numpy())

    def write_block(self, block_id: int, k_block: np.ndarray, v_block: np.ndarray) -> None:
        """Quantize (one group over the block's rows), pack and store one block."""
        import torch
        assert np.shape(k_block) == np.shape(v_block)
        rows, d = np.shape(k_block)
        if d != self.head_dim:
            raise ValueError(f"block has head_dim {d}, cache has {self.head_dim}")
        if not 1 <= rows <= self.block_size:
            raise ValueError(f"block has {rows} rows; 1..{self.block_size} fit in a block")
        if not 0 <= block_id < self.num_blocks:
            raise ValueError(f"block_id {block_id} outside [0, {self.num_blocks})")
        k_t = torch.from_numpy(np.ascontiguousarray(k_block, dtype=np.float32)).cuda()
        load_binding().quantize_rows_into(k_t, self._k[block_id, :rows], self._s[block_id],
                                          self._z[block_id], True)
        v16 = np.ascontiguousarray(np.asarray(v_block).astype(np.float16))
        self._v[block_id, :rows, :d] = torch.from_numpy(v16).cuda()
        self.lens[block_id] = rows

    def free_block(self, block_id: int) -> None:
        self.lens.pop(block_id, None)

    def decode_attention(self, query: np.ndarray, block_table: List[int]) -> np.ndarray:
        """Fused INT4 attention of every query over the blocks of ``block_table``."""
        import torch
        query = np.asarray(query, dtype=np.float32)
        if query.ndim != 3 or query.shape[2] != self.head_dim:
            raise ValueError(f"query must be [batch, heads, {self.head_dim}], got "
                             f"{query.shape}")
        lens = [self.lens[b] for b in block_table]  # KeyError for unknown blocks
        n = len(block_table)
        B, H, D = query.shape
        if n == 0:
            return np.zeros(query.shape, dtype=np.float32)
        dev = torch.device("cuda")
        qp = np.zeros((B, H, self._dp), dtype=np.float32)
        qp[..., :D] = query
        q_t = torch.from_numpy(qp).to(dev)
        table = torch.tensor(block_table, dtype=torch.int32, device=dev).view(1, n).expand(B, n)
        lens_t = torch.tensor(lens, dtype=torch.int32, device=dev).view(1, n).expand(B, n)
        nb, bs, dp = self.num_blocks, self.block_size, self._dp
        out = load_binding().decode_paged(
            q_t, self._k.view(nb, 1, bs, dp // 2), self._v.view(nb, 1, bs, dp), self._s,
            self._z, table, None, lens_t, 1, n, 0)
        return out[..., :D].cpu().numpy()

    def memory_stats(self) -> dict:
        """Bytes held for the written blocks (their full pool slots) vs fp16 K+V."""
        n = len(self.lens)
        if n == 0:
            return {"blocks": 0, "stored_mb": 0.0, "fp16_equiv_mb": 0.0, "ratio": 0.0}
        slot = (self._k[0].numel() * self._k.element_size()
                + self._v[0].numel() * self._v.element_size()
                + 2 * self._s[0].numel() * self._s.element_size())
        stored = n * slot
        fp16_equiv = sum(r * self.head_dim * 2 * 2 for r in self.lens.values())
        return {
            "blocks": n,
            "stored_mb": round(stored / 1048576, 3),
            "fp16_equiv_mb": round(fp16_equiv / 1048576, 3),
            "ratio": round(fp16_equiv / max(stored, 1), 2),
        }
