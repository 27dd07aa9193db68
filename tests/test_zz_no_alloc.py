"""fdi4_decode_paged_noalloc (split partials in the library's static device
array) against fdi4_decode_paged (partials in a caller workspace), called
through the C ABI: identical outputs on two calls in a row, the second on a
smaller input, so the array holds the first call's partials when the second
starts."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _cache(hkv, seq_lens, seed):
    """A quantized paged cache of hkv kv-heads at D=128 (16-row pages,
    128-row scale groups) and its ctypes description."""
    import torch
    from flash_decode_int4 import capi, ops
    from flash_decode_int4.workloads import make_workload
    w = make_workload(batch=len(seq_lens), heads=hkv, head_dim=128, seq_lens=seq_lens,
                      seed=seed)
    dev = torch.device("cuda")
    B, D = len(seq_lens), 128
    G = (w["max_tokens"] + 127) // 128
    t = dict(kp=torch.zeros(w["num_pages"], hkv, 16, D // 2, dtype=torch.uint8, device=dev),
             s=torch.zeros(B, hkv, G, D, device=dev), z=torch.zeros(B, hkv, G, D, device=dev),
             sl=torch.from_numpy(w["seq_lens"]).to(dev),
             pt=torch.from_numpy(w["page_table"]).to(dev),
             v=torch.from_numpy(w["v_pages"]).to(dev))
    ops.quantize_int4_paged(torch.from_numpy(w["k"]).to(dev), t["sl"], t["pt"], t["kp"],
                            t["s"], t["z"], 128)
    kp, v, s = t["kp"], t["v"], t["s"]
    cache = capi.PagedCache(
        k_pages=kp.data_ptr(), k_page_stride=kp.stride(0), k_head_stride=kp.stride(1),
        k_row_stride=kp.stride(2), v_pages=v.data_ptr(), v_dtype=capi.V_F32,
        v_page_stride=v.stride(0), v_head_stride=v.stride(1), v_row_stride=v.stride(2),
        k_scale=s.data_ptr(), k_zp=t["z"].data_ptr(), s_batch_stride=s.stride(0),
        s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
        page_table=t["pt"].data_ptr(), pt_batch_stride=t["pt"].stride(0),
        seq_lens=t["sl"].data_ptr(), page_lens=None, pl_batch_stride=0, num_kv_heads=hkv,
        head_dim=D, page_rows=16, pages_per_group=8, max_pages=t["pt"].shape[1],
        num_pages=w["num_pages"])
    return cache, t


def _both(cache, B, hq, splits, seed):
    """Outputs of the no-allocation call and of the workspace call."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    dev = torch.device("cuda")
    q = torch.from_numpy(np.random.RandomState(seed).randn(B, hq, 128).astype(np.float32)).to(dev)
    out_na = torch.full((B, hq, 128), float("nan"), device=dev)
    out_ws = torch.full((B, hq, 128), float("nan"), device=dev)
    nbytes = lib.fdi4_decode_workspace_bytes(B, hq, 128, splits)
    assert 0 < nbytes <= capi.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    capi.check(lib.fdi4_decode_paged_noalloc(_ptr(q), B, hq, q.stride(0), q.stride(1), cache,
                                             _ptr(out_na), out_na.stride(0), out_na.stride(1),
                                             splits, _stream()), "decode_paged_noalloc")
    capi.check(lib.fdi4_decode_paged(_ptr(q), B, hq, q.stride(0), q.stride(1), cache,
                                     _ptr(out_ws), out_ws.stride(0), out_ws.stride(1), splits,
                                     _ptr(ws), nbytes, _stream()), "decode_paged")
    torch.cuda.synchronize()
    return out_na.cpu().numpy(), out_ws.cpu().numpy()


def test_noalloc_matches_workspace_call_twice_second_smaller():
    # First call: grouped query heads (4 q-heads per kv-head), 6 splits.
    cache1, keep1 = _cache(4, [2000, 1500, 37, 0], seed=11)
    na, ws = _both(cache1, 4, 16, 6, seed=12)
    assert np.isfinite(na).all()
    np.testing.assert_array_equal(na, ws)
    np.testing.assert_array_equal(na[3], 0.0)
    # Second call, smaller: one q-head per kv-head, 3 splits; the array still
    # holds the first call's partials.
    cache2, keep2 = _cache(8, [700, 129], seed=13)
    na2, ws2 = _both(cache2, 2, 8, 3, seed=14)
    assert np.isfinite(na2).all()
    np.testing.assert_array_equal(na2, ws2)


def test_noalloc_single_split_needs_no_scratch():
    cache, keep = _cache(2, [300, 64, 1], seed=21)
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    q = torch.from_numpy(np.random.RandomState(22).randn(3, 2, 128).astype(np.float32)).cuda()
    out_na = torch.full((3, 2, 128), float("nan"), device="cuda")
    out_ws = torch.full((3, 2, 128), float("nan"), device="cuda")
    capi.check(lib.fdi4_decode_paged_noalloc(_ptr(q), 3, 2, q.stride(0), q.stride(1), cache,
                                             _ptr(out_na), out_na.stride(0), out_na.stride(1),
                                             1, _stream()))
    capi.check(lib.fdi4_decode_paged(_ptr(q), 3, 2, q.stride(0), q.stride(1), cache,
                                     _ptr(out_ws), out_ws.stride(0), out_ws.stride(1), 1, None,
                                     0, _stream()))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out_na.cpu().numpy(), out_ws.cpu().numpy())


def test_noalloc_replayed_from_a_graph():
    """After one eager call on the device (the first call looks the array's
    address up, which is not a stream operation), the call is captured in a
    HIP graph; each replay, with new queries written between replays, equals
    the workspace call on the same queries bit for bit."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    cache, keep = _cache(4, [1200, 333, 0], seed=31)
    B, hq, D, splits = 3, 16, 128, 4
    rng = np.random.RandomState(32)
    q = torch.from_numpy(rng.randn(B, hq, D).astype(np.float32)).cuda()
    out_g = torch.full((B, hq, D), float("nan"), device="cuda")
    nbytes = lib.fdi4_decode_workspace_bytes(B, hq, D, splits)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ref = torch.empty(B, hq, D, device="cuda")

    def noalloc():
        return lib.fdi4_decode_paged_noalloc(_ptr(q), B, hq, q.stride(0), q.stride(1), cache,
                                             _ptr(out_g), out_g.stride(0), out_g.stride(1),
                                             splits, _stream())

    capi.check(noalloc(), "decode_paged_noalloc (eager)")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = noalloc()
    assert rc == 0
    for r in range(3):
        q.copy_(torch.from_numpy(rng.randn(B, hq, D).astype(np.float32)))
        out_g.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        capi.check(lib.fdi4_decode_paged(_ptr(q), B, hq, q.stride(0), q.stride(1), cache,
                                         _ptr(ref), ref.stride(0), ref.stride(1), splits,
                                         _ptr(ws), nbytes, _stream()), "decode_paged")
        torch.cuda.synchronize()
        assert torch.isfinite(out_g).all(), r
        assert torch.equal(out_g, ref), r
