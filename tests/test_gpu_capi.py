"""The C ABI called directly through ctypes with raw device pointers -- the
path a non-torch caller (cgo, JNI, N-API, ctypes) takes -- checked against the
oracle and against the torch binding."""

import ctypes

import numpy as np
import pytest

from oracle import paged_decode_f64, paged_decode_ref, quantize_int4_ref

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_quantize_int4_exact_reference_signature():
    """fdi4_quantize_int4: the reference's cu_quantize_int4 argument list."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    kv = np.random.RandomState(3).randn(1000, 96).astype(np.float32)
    x = torch.from_numpy(kv).cuda()
    q = torch.empty(1000, 96, dtype=torch.uint8, device="cuda")
    s = torch.empty(96, device="cuda")
    z = torch.empty(96, device="cuda")
    capi.check(lib.fdi4_quantize_int4(_ptr(x), 1000, 96, _ptr(q), _ptr(s), _ptr(z), _stream()))
    torch.cuda.synchronize()
    qr, sr, zr = quantize_int4_ref(kv)
    np.testing.assert_array_equal(q.cpu().numpy(), qr)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(z.cpu().numpy(), zr)


def _default_pool_release_threshold():
    """Release threshold of the current device's default memory pool, read
    through the HIP runtime (hipDeviceGetDefaultMemPool / hipMemPoolGetAttribute)."""
    import torch
    hip = ctypes.CDLL("libamdhip64.so")
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), torch.cuda.current_device()) == 0
    value = ctypes.c_uint64()
    release_threshold = 0x4  # hipMemPoolAttrReleaseThreshold
    assert hip.hipMemPoolGetAttribute(pool, release_threshold, ctypes.byref(value)) == 0
    return value.value


def test_reference_signatures_use_library_pool_on_any_stream():
    """The entry points without a workspace argument take their temporaries
    from the library's own pool: repeated calls on the default and on a side
    stream give the oracle's results, and the process's default pool keeps
    the release threshold it had."""
    import torch
    from flash_decode_int4 import capi
    lib = capi.load()
    before = _default_pool_release_threshold()
    kv = np.random.RandomState(5).randn(3000, 64).astype(np.float32)
    qr, sr, zr = quantize_int4_ref(kv)
    x = torch.from_numpy(kv).cuda()
    side = torch.cuda.Stream()
    for stream in (torch.cuda.current_stream(), side, side, torch.cuda.current_stream()):
        q = torch.zeros(3000, 64, dtype=torch.uint8, device="cuda")
        s = torch.zeros(64, device="cuda")
        z = torch.zeros(64, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            capi.check(lib.fdi4_quantize_int4(_ptr(x), 3000, 64, _ptr(q), _ptr(s), _ptr(z),
                                              ctypes.c_void_p(stream.cuda_stream)))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), qr)
        np.testing.assert_array_equal(s.cpu().numpy(), sr)
        np.testing.assert_array_equal(z.cpu().numpy(), zr)
    assert _default_pool_release_threshold() == before


def test_flash_decode_int4_exact_reference_signature():
    """fdi4_flash_decode_int4: the reference's cu_flash_decode_int4 argument list
    (unpacked keys, shared page stream)."""
    import torch
    from flash_decode_int4 import capi
    from oracle import online_softmax_ref
    lib = capi.load()
    rng = np.random.RandomState(4)
    B, H, D, nb, bs = 2, 3, 64, 3, 48
    query = rng.randn(B, H, D).astype(np.float32)
    kq, ss, zz, vv = [], [], [], []
    for _ in range(nb):
        q_, s_, z_ = quantize_int4_ref(rng.randn(bs, D).astype(np.float32))
        kq.append(q_); ss.append(s_); zz.append(z_); vv.append(rng.randn(bs, D).astype(np.float32))
    lens = np.array([48, 0, 31], np.int32)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in
           (query, np.stack(kq), np.stack(ss), np.stack(zz), np.stack(vv), lens)]
    out = torch.empty(B, H, D, device="cuda")
    capi.check(lib.fdi4_flash_decode_int4(*[_ptr(t) for t in dev], B, H, D, nb, bs, _ptr(out),
                                          _stream()))
    torch.cuda.synchronize()
    ref = online_softmax_ref(query, list(zip(kq, ss, zz)), vv, lens)[0]
    assert np.abs(out.cpu().numpy() - ref).max() < 1e-5


def test_decode_paged_through_ctypes_matches_oracle_and_binding():
    import torch
    from flash_decode_int4 import capi, ops
    from flash_decode_int4.workloads import make_workload
    lib = capi.load()
    w = make_workload(batch=3, heads=4, head_dim=128, seq_lens=[100, 1000, 0], seed=41)
    dev = torch.device("cuda")
    B, H, D = 3, 4, 128
    G = (w["max_tokens"] + 127) // 128
    kp = torch.zeros(w["num_pages"], H, 16, 64, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, H, G, D, device=dev)
    z = torch.zeros(B, H, G, D, device=dev)
    sl = torch.from_numpy(w["seq_lens"]).to(dev)
    pt = torch.from_numpy(w["page_table"]).to(dev)
    k = torch.from_numpy(w["k"]).to(dev)
    v = torch.from_numpy(w["v_pages"]).to(dev)
    q = torch.from_numpy(w["q"]).to(dev)
    cache = capi.PagedCache(
        k_pages=kp.data_ptr(), k_page_stride=kp.stride(0), k_head_stride=kp.stride(1),
        k_row_stride=kp.stride(2), v_pages=v.data_ptr(), v_dtype=capi.V_F32,
        v_page_stride=v.stride(0), v_head_stride=v.stride(1), v_row_stride=v.stride(2),
        k_scale=s.data_ptr(), k_zp=z.data_ptr(), s_batch_stride=s.stride(0),
        s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
        page_table=pt.data_ptr(), pt_batch_stride=pt.stride(0), seq_lens=sl.data_ptr(),
        page_lens=None, pl_batch_stride=0, num_kv_heads=H, head_dim=D, page_rows=16,
        pages_per_group=8, max_pages=pt.shape[1], num_pages=w["num_pages"])
    capi.check(lib.fdi4_quantize_paged(_ptr(k), B, k.shape[2], k.stride(0), k.stride(1),
                                       k.stride(2), 128, cache, _stream()), "quantize_paged")
    splits = lib.fdi4_decode_num_splits(B, H, cache)
    nbytes = lib.fdi4_decode_workspace_bytes(B, H, D, splits)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty(B, H, D, device=dev)
    capi.check(lib.fdi4_decode_paged(_ptr(q), B, H, q.stride(0), q.stride(1), cache, _ptr(out),
                                     out.stride(0), out.stride(1), splits, _ptr(ws), ws.numel(),
                                     _stream()), "decode_paged")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    args = (w["q"], kp.cpu().numpy(), w["v_pages"], s.cpu().numpy(), z.cpu().numpy(),
            w["page_table"], w["seq_lens"])
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    assert np.abs(got - o32).max() <= max(1e-5, 1.25 * np.abs(o32 - o64).max())
    np.testing.assert_array_equal(got[2], 0.0)
    via_binding = ops.flash_decode_paged(q, kp, v, s, z, pt, sl, num_splits=splits)
    assert bool((via_binding == out).all())


def test_partials_then_merge_equals_one_call():
    """fdi4_decode_paged_partials + fdi4_merge_splits == fdi4_decode_paged."""
    import torch
    from flash_decode_int4 import ops
    from flash_decode_int4.workloads import make_workload
    C = ops._C
    w = make_workload(batch=2, heads=4, head_dim=128, seq_lens=[2048, 333], seed=42)
    dev = torch.device("cuda")
    G = 16
    kp = torch.zeros(w["num_pages"], 4, 16, 64, dtype=torch.uint8, device=dev)
    s = torch.zeros(2, 4, G, 128, device=dev)
    z = torch.zeros(2, 4, G, 128, device=dev)
    sl = torch.from_numpy(w["seq_lens"]).to(dev)
    pt = torch.from_numpy(w["page_table"]).to(dev)
    ops.quantize_int4_paged(torch.from_numpy(w["k"]).to(dev), sl, pt, kp, s, z, 128)
    q = torch.from_numpy(w["q"]).to(dev)
    v = torch.from_numpy(w["v_pages"]).to(dev)
    for S in (1, 4, 9):
        parts = torch.empty(int(C.decode_partials_bytes(2, 4, 128, S)), dtype=torch.uint8,
                            device=dev)
        C.decode_paged_partials(q, kp, v, s, z, pt, sl, None, 8, pt.shape[1], S, parts)
        merged = C.merge_splits(parts, 2, 4, 128, S)
        one = ops.flash_decode_paged(q, kp, v, s, z, pt, sl, num_splits=S)
        assert (merged - one).abs().max().item() < 1e-6, S


def test_advance_pair_through_ctypes():
    """fdi4_append_paged_advance then fdi4_decode_paged_advance with raw device
    pointers: lens_next holds the advanced lengths after the append, the
    cache's lengths are unchanged until the decode copies them back, and the
    output equals the workspace decode over the advanced lengths."""
    import torch
    from flash_decode_int4 import capi
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    lib = capi.load()
    B, H, D = 2, 4, 128
    c = INT4PagedSequenceCache(num_pages=64, num_kv_heads=H, head_dim=D, max_seqs=B,
                               max_seq_len=512)
    g = torch.Generator(device="cuda").manual_seed(21)
    k = torch.randn(B, H, 300, D, device="cuda", generator=g)
    c.prefill(k, torch.randn_like(k), [300, 127])
    c.reserve(B, 1)
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, H, D, device="cuda", generator=g)
    nxt = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    kp, v, s = c.k_pages, c.v_pages, c.k_scale

    def cache_desc(lens):
        return capi.PagedCache(
            k_pages=kp.data_ptr(), k_page_stride=kp.stride(0), k_head_stride=kp.stride(1),
            k_row_stride=kp.stride(2), v_pages=v.data_ptr(), v_dtype=capi.V_F32,
            v_page_stride=v.stride(0), v_head_stride=v.stride(1), v_row_stride=v.stride(2),
            k_scale=s.data_ptr(), k_zp=c.k_zp.data_ptr(), s_batch_stride=s.stride(0),
            s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
            page_table=c.page_table.data_ptr(), pt_batch_stride=c.page_table.stride(0),
            seq_lens=lens.data_ptr(), page_lens=None, pl_batch_stride=0, num_kv_heads=H,
            head_dim=D, page_rows=16, pages_per_group=8, max_pages=c.page_table.shape[1],
            num_pages=kp.shape[0])

    st = c.k_stage
    capi.check(lib.fdi4_append_paged_advance(
        _ptr(kn), kn.stride(0), kn.stride(1), _ptr(vn), vn.stride(0), vn.stride(1), B, _ptr(st),
        st.stride(0), st.stride(1), st.stride(2), 128, cache_desc(c.seq_lens), _ptr(nxt),
        _stream()), "append_paged_advance")
    torch.cuda.synchronize()
    assert nxt.tolist() == [301, 128] and c.seq_lens[:B].tolist() == [300, 127]
    out = torch.empty(B, H, D, device="cuda")
    ref = torch.empty(B, H, D, device="cuda")
    capi.check(lib.fdi4_decode_paged_advance(
        _ptr(q), capi.K_F32, B, H, q.stride(0), q.stride(1), cache_desc(nxt), _ptr(out),
        capi.K_F32, out.stride(0), out.stride(1), 1, None, 0, _ptr(c.seq_lens), _stream()),
        "decode_paged_advance")
    torch.cuda.synchronize()
    assert c.seq_lens[:B].tolist() == [301, 128]
    capi.check(lib.fdi4_decode_paged_ex(
        _ptr(q), capi.K_F32, B, H, q.stride(0), q.stride(1), cache_desc(c.seq_lens), _ptr(ref),
        capi.K_F32, ref.stride(0), ref.stride(1), 1, None, 0, _stream()), "decode_paged_ex")
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_decode_step_rejects_a_bad_workspace_before_touching_the_cache():
    """fdi4_decode_step on its two-launch path (grouped query heads, several
    splits) with no workspace, a short one and a misaligned one: each call
    returns hipErrorInvalidValue and leaves pages, values, scales, staging
    rows, lengths and lens_next bitwise as they were; with the workspace the
    library asks for, the same call appends and advances."""
    import torch
    from flash_decode_int4 import capi
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    lib = capi.load()
    B, H, HQ, D = 2, 4, 16, 128
    c = INT4PagedSequenceCache(num_pages=2 * 128 + 8, num_kv_heads=H, head_dim=D, max_seqs=B,
                               max_seq_len=2048)
    g = torch.Generator(device="cuda").manual_seed(33)
    k = torch.randn(B, H, 1500, D, device="cuda", generator=g)
    c.prefill(k, torch.randn_like(k), [1500, 700])
    c.reserve(B, 1)
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, HQ, D, device="cuda", generator=g)
    out = torch.zeros(B, HQ, D, device="cuda")
    kp, v, s = c.k_pages, c.v_pages, c.k_scale
    desc = capi.PagedCache(
        k_pages=kp.data_ptr(), k_page_stride=kp.stride(0), k_head_stride=kp.stride(1),
        k_row_stride=kp.stride(2), v_pages=v.data_ptr(), v_dtype=capi.V_F32,
        v_page_stride=v.stride(0), v_head_stride=v.stride(1), v_row_stride=v.stride(2),
        k_scale=s.data_ptr(), k_zp=c.k_zp.data_ptr(), s_batch_stride=s.stride(0),
        s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
        page_table=c.page_table.data_ptr(), pt_batch_stride=c.page_table.stride(0),
        seq_lens=c.seq_lens.data_ptr(), page_lens=None, pl_batch_stride=0, num_kv_heads=H,
        head_dim=D, page_rows=16, pages_per_group=8, max_pages=c.page_table.shape[1],
        num_pages=kp.shape[0])
    splits = lib.fdi4_decode_num_splits(B, HQ, desc)
    assert splits > 1
    need = lib.fdi4_decode_workspace_bytes(B, HQ, D, splits)
    ws = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
    st = c.k_stage
    nxt, cnt = c._lens_next, c._step_counters

    def call(ptr, nbytes):
        return lib.fdi4_decode_step(
            _ptr(q), capi.K_F32, B, HQ, q.stride(0), q.stride(1), _ptr(kn), kn.stride(0),
            kn.stride(1), _ptr(vn), vn.stride(0), vn.stride(1), _ptr(st), st.stride(0),
            st.stride(1), st.stride(2), 128, desc, _ptr(out), capi.K_F32, out.stride(0),
            out.stride(1), _ptr(cnt), _ptr(nxt), ptr, nbytes, _stream())

    names = ("k_pages", "v_pages", "k_scale", "k_zp", "k_stage", "seq_lens", "_lens_next")
    before = {n: getattr(c, n).clone() for n in names}
    for ptr, nbytes in ((None, 0), (_ptr(ws), need - 256),
                        (ctypes.c_void_p(ws.data_ptr() + 4), need)):
        assert call(ptr, nbytes) == 1          # hipErrorInvalidValue
        torch.cuda.synchronize()
        for n in names:
            assert torch.equal(getattr(c, n), before[n]), n
    capi.check(call(_ptr(ws), need), "decode_step")
    torch.cuda.synchronize()
    assert c.seq_lens[:B].tolist() == [1501, 701]
    assert torch.isfinite(out).all()
