"""The decode kernels' device-side clamps, for calls that reach the C ABI
without the host contract (reference clamp: csrc/flash_decode_int4.cu:155-157;
host contract: src/_validate.py:53-62):

  page-table entries   clamped to [0, num_pages)
  seq_lens             clamped to [0, max_pages * page_rows]
  page_lens            clamped to [0, page_rows]

Each case runs a decode on malformed metadata and the same decode on the
metadata clamped on the host; the two outputs must be equal bit for bit.
Every buffer a missing clamp could reach is allocated and filled with
poison: pages before and after the pool (num_pages is passed below the
allocation; keys 0xFF, values NaN), page-table columns past max_pages, a
scale group past the last one. So an unclamped entry, length or row count
reads poison inside the allocation (and shows up as a difference or a NaN),
never memory outside it. The one exception is seq_lens = INT32_MAX, which no
allocation could cover; its clamp is the same unconditional min/max as the
other lengths' (decode_common.hpp, seq_len_of), which the cap + 3 case shows
working."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

INT32_MAX = 2 ** 31 - 1


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Pool:
    """B sequences of max_pages pages (page_rows rows, D = 128, Hkv kv-heads)
    in a pool of P = B * max_pages real pages framed by E poison pages on
    each side, group-indexed scales with one poison group past the last, a
    page table with `extra` poison columns."""

    def __init__(self, B, hkv, max_pages, page_rows, group_rows, seed, E=8, extra=2):
        import torch
        rng = np.random.RandomState(seed)
        D = 128
        self.B, self.hkv, self.D, self.E = B, hkv, D, E
        self.max_pages, self.page_rows, self.extra = max_pages, page_rows, extra
        self.ppg = group_rows // page_rows
        self.P = P = B * max_pages
        cap = max_pages * page_rows
        self.cap = cap
        self.G = G = (cap + group_rows - 1) // group_rows
        kp = np.full((E + P + E, hkv, page_rows, D // 2), 0xFF, np.uint8)
        kp[E:E + P] = rng.randint(0, 256, size=(P, hkv, page_rows, D // 2))
        v = np.full((E + P + E, hkv, page_rows, D), np.nan, np.float32)
        v[E:E + P] = rng.randn(P, hkv, page_rows, D)
        s = np.full((B, hkv, G + 1, D), np.nan, np.float32)
        z = np.full((B, hkv, G + 1, D), np.nan, np.float32)
        s[:, :, :G] = rng.uniform(0.05, 0.3, size=(B, hkv, G, D))
        z[:, :, :G] = rng.uniform(0.0, 15.0, size=(B, hkv, G, D))
        pt = np.full((B, max_pages + extra), P + 1, np.int32)
        pt[:, :max_pages] = rng.permutation(P).reshape(B, max_pages)
        self.pt_clean = pt.copy()
        dev = torch.device("cuda")
        self.kp = torch.from_numpy(kp).to(dev)
        self.v = torch.from_numpy(v).to(dev)
        self.s = torch.from_numpy(s).to(dev)
        self.z = torch.from_numpy(z).to(dev)
        self.pt = torch.from_numpy(pt).to(dev)

    def desc(self, page_table, seq_lens=None, page_lens=None):
        from flash_decode_int4 import capi
        kp, v, s = self.kp, self.v, self.s
        return capi.PagedCache(
            k_pages=kp[self.E].data_ptr(), k_page_stride=kp.stride(0),
            k_head_stride=kp.stride(1), k_row_stride=kp.stride(2),
            v_pages=v[self.E].data_ptr(), v_dtype=capi.V_F32, v_page_stride=v.stride(0),
            v_head_stride=v.stride(1), v_row_stride=v.stride(2),
            k_scale=s.data_ptr(), k_zp=self.z.data_ptr(), s_batch_stride=s.stride(0),
            s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
            page_table=page_table.data_ptr(), pt_batch_stride=page_table.stride(0),
            seq_lens=None if seq_lens is None else seq_lens.data_ptr(),
            page_lens=None if page_lens is None else page_lens.data_ptr(),
            pl_batch_stride=0 if page_lens is None else page_lens.stride(0),
            num_kv_heads=self.hkv, head_dim=self.D, page_rows=self.page_rows,
            pages_per_group=self.ppg, max_pages=self.max_pages, num_pages=self.P)

    def decode(self, desc, hq, splits, seed):
        import torch
        from flash_decode_int4 import capi
        lib = capi.load()
        q = torch.from_numpy(
            np.random.RandomState(seed).randn(self.B, hq, self.D).astype(np.float32)).cuda()
        out = torch.full((self.B, hq, self.D), -3.0, device="cuda")
        nbytes = lib.fdi4_decode_workspace_bytes(self.B, hq, self.D, splits)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        capi.check(lib.fdi4_decode_paged(_ptr(q), self.B, hq, q.stride(0), q.stride(1), desc,
                                         _ptr(out), out.stride(0), out.stride(1), splits,
                                         _ptr(ws), nbytes, _stream()), "decode_paged")
        torch.cuda.synchronize()
        return out.cpu().numpy()


KERNELS = [
    # (q-heads per kv-head, tuning): per-head kernel, int8 matrix-core grouped
    # kernel, vector grouped kernel
    pytest.param(1, {}, id="per_head"),
    pytest.param(4, {}, id="grouped_mfma"),
    pytest.param(4, {"decode_vector_only": 1}, id="grouped_vector"),
]


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("rep,tune", KERNELS)
def test_page_table_entries_and_lengths_clamped(rep, tune, splits):
    import torch
    from flash_decode_int4 import capi
    pool = Pool(B=5, hkv=2, max_pages=12, page_rows=16, group_rows=128, seed=101)
    P, E, cap = pool.P, pool.E, pool.cap
    bad = pool.pt_clean.copy()
    # Entries at and past num_pages and below 0, every one inside the poison
    # frame, in columns the sequences read.
    bad[0, 2], bad[0, 11] = P, P + E - 1
    bad[2, 7] = P + 3
    bad[3, 1] = -5
    bad[4, 0], bad[4, 5] = -1, -E
    # Sequence 2's length is three rows past the capacity (unclamped, they
    # would come from the first poison column); sequence 1's negative length
    # reads no page at all.
    lens_bad = np.array([INT32_MAX, -7, cap + 3, 61, cap], np.int32)
    lens_ok = np.clip(lens_bad.astype(np.int64), 0, cap).astype(np.int32)
    pt_ok = pool.pt_clean.copy()
    pt_ok[:, :pool.max_pages] = np.clip(bad[:, :pool.max_pages], 0, P - 1)
    pt_bad = torch.from_numpy(bad).cuda()
    pt_ok_t = torch.from_numpy(pt_ok).cuda()
    sl_bad = torch.from_numpy(lens_bad).cuda()
    sl_ok = torch.from_numpy(lens_ok).cuda()
    hq = pool.hkv * rep
    with capi.tuning(**tune):
        got = pool.decode(pool.desc(pt_bad, seq_lens=sl_bad), hq, splits, seed=7)
        want = pool.decode(pool.desc(pt_ok_t, seq_lens=sl_ok), hq, splits, seed=7)
    assert np.isfinite(want).all()
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got[1], 0.0)          # a negative length has no rows


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("rep,tune", KERNELS)
def test_page_lens_clamped(rep, tune, splits):
    """seq_lens absent (every sequence spans max_pages pages), page_lens with
    values below 0 and above page_rows = 8 (half a 16-row chunk, so an
    unclamped count would read the rows after the page)."""
    import torch
    from flash_decode_int4 import capi
    pool = Pool(B=3, hkv=2, max_pages=16, page_rows=8, group_rows=64, seed=202)
    rng = np.random.RandomState(5)
    pl_bad = np.full((pool.B, pool.max_pages + pool.extra), 40, np.int32)
    pl_bad[:, :pool.max_pages] = rng.choice([-4, 0, 3, 8, 11, 40], size=(pool.B, pool.max_pages))
    pl_bad[:, -3] = 11                                   # every sequence's last pages too
    pl_ok = np.clip(pl_bad, 0, pool.page_rows).astype(np.int32)
    pt = torch.from_numpy(pool.pt_clean).cuda()
    hq = pool.hkv * rep
    with capi.tuning(**tune):
        got = pool.decode(pool.desc(pt, page_lens=torch.from_numpy(pl_bad).cuda()), hq, splits,
                          seed=9)
        want = pool.decode(pool.desc(pt, page_lens=torch.from_numpy(pl_ok).cuda()), hq, splits,
                           seed=9)
    assert np.isfinite(want).all()
    np.testing.assert_array_equal(got, want)


def test_reference_entry_point_block_lens_clamped():
    """fdi4_flash_decode_int4 (the reference's cu_flash_decode_int4 arguments)
    with block_lens outside [0, block_size]: the same output as with the
    lengths clamped, as the reference kernel's own clamp gives. The value
    array has a poison page after the last block, so rows read past a page
    stay inside it."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    rng = np.random.RandomState(303)
    B, H, D, nb, bs = 2, 4, 128, 6, 8
    q = torch.from_numpy(rng.randn(B, H, D).astype(np.float32)).cuda()
    kq = torch.from_numpy(rng.randint(0, 16, size=(nb, bs, D)).astype(np.uint8)).cuda()
    ks = torch.from_numpy(rng.uniform(0.05, 0.3, size=(nb, D)).astype(np.float32)).cuda()
    kz = torch.from_numpy(rng.uniform(0, 15, size=(nb, D)).astype(np.float32)).cuda()
    v_all = np.full((nb + 1, bs, D), np.nan, np.float32)
    v_all[:nb] = rng.randn(nb, bs, D)
    v = torch.from_numpy(v_all).cuda()
    lens_bad = np.array([300, -3, 5, 8, 9, 2 ** 20], np.int32)
    lens_ok = np.clip(lens_bad, 0, bs).astype(np.int32)
    outs = []
    for lens in (lens_bad, lens_ok):
        lt = torch.from_numpy(lens).cuda()
        out = torch.full((B, H, D), -3.0, device="cuda")
        capi.check(lib.fdi4_flash_decode_int4(_ptr(q), _ptr(kq), _ptr(ks), _ptr(kz), _ptr(v),
                                              _ptr(lt), B, H, D, nb, bs, _ptr(out), _stream()),
                   "flash_decode_int4")
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.isfinite(outs[1]).all()
    np.testing.assert_array_equal(outs[0], outs[1])
