"""The one-call decode with several splits (fdi4_decode_paged: the split
kernel, then the merge kernel on the same stream) against the two-call form
(fdi4_decode_paged_partials, then fdi4_merge_splits) bit for bit, for every
kernel family, and against the oracle; through a caller-owned workspace that
starts as garbage and is reused across calls with other queries and split
counts; and through HIP graph replays that reuse the captured workspace.
"""

import numpy as np
import pytest

from oracle import paged_decode_f64, paged_decode_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _problem(batch, kv_heads, head_dim, seq_lens, q_heads=None, seed=0, value_dtype=None):
    import torch
    from flash_decode_int4 import ops
    from flash_decode_int4.workloads import make_workload
    w = make_workload(batch=batch, heads=kv_heads, head_dim=head_dim, seq_lens=seq_lens,
                      seed=seed, q_heads=q_heads)
    dev = torch.device("cuda")
    G = (w["max_tokens"] + 127) // 128
    kp = torch.zeros(w["num_pages"], kv_heads, 16, head_dim // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(batch, kv_heads, G, head_dim, device=dev)
    z = torch.zeros_like(s)
    k = torch.as_tensor(w["k"], device=dev)
    sl = torch.as_tensor(w["seq_lens"], device=dev)
    pt = torch.as_tensor(w["page_table"], device=dev)
    ops.quantize_int4_paged(k, sl, pt, kp, s, z, 128)
    v = torch.as_tensor(w["v_pages"], device=dev)
    if value_dtype is not None:
        v = v.to(value_dtype)
    q = torch.as_tensor(w["q"], device=dev)
    return w, (q, kp, v, s, z, pt, sl)


def _two_launch(C, args, splits):
    """Partials, then the merge kernel, as two calls."""
    import torch
    q, kp, v, s, z, pt, sl = args
    B, Hq, D = q.shape
    parts = torch.empty(int(C.decode_partials_bytes(B, Hq, D, splits)), dtype=torch.uint8,
                        device="cuda")
    C.decode_paged_partials(q, kp, v, s, z, pt, sl, None, 8, pt.shape[1], splits, parts)
    return C.merge_splits(parts, B, Hq, D, splits)


CASES = [
    # (batch, kv_heads, q_heads, head_dim, seq_lens, splits, value dtype)
    (2, 4, None, 128, [2048, 700], 4, None),          # per-head kernel
    (1, 2, None, 64, [4096], 16, None),
    (2, 2, None, 256, [1500, 0], 3, "float16"),       # an empty sequence
    (2, 2, 8, 128, [3000, 1024], 4, None),            # matrix-core grouped kernel
    (1, 2, 16, 64, [2500], 8, "float16"),
    (2, 2, 4, 256, [1024, 999], 5, None),             # vector grouped kernel (D = 256)
]


@pytest.mark.parametrize("batch,kv,hq,d,lens,splits,vdt", CASES)
def test_one_call_equals_two_calls(batch, kv, hq, d, lens, splits, vdt):
    import torch
    from flash_decode_int4 import ops
    from flash_decode_int4._lib import load_binding
    C = load_binding()
    w, args = _problem(batch, kv, d, lens, q_heads=hq, seed=splits + d,
                       value_dtype=getattr(torch, vdt) if vdt else None)
    one = ops.flash_decode_paged(*args, num_splits=splits)
    two = _two_launch(C, args, splits)
    assert torch.equal(one, two)
    # And against the oracle.
    q, kp, v, s, z, pt, sl = args
    oargs = (q.cpu().numpy(), kp.cpu().numpy(), v.float().cpu().numpy(), s.cpu().numpy(),
             z.cpu().numpy(), w["page_table"], w["seq_lens"])
    o32, o64 = paged_decode_ref(*oargs), paged_decode_f64(*oargs)
    got = one.cpu().numpy()
    assert np.abs(got - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())
    empty = np.asarray(w["seq_lens"]) == 0
    assert np.all(got[empty] == 0.0)


def test_dirty_workspace_through_the_c_abi():
    """One caller-owned workspace, filled with garbage and then reused across
    calls with different queries and split counts: every call's output equals
    the two-call form."""
    import ctypes
    import torch
    from flash_decode_int4 import capi
    from flash_decode_int4._lib import load_binding
    C = load_binding()
    lib = capi.load()
    w, args = _problem(2, 4, 128, [3000, 2047], seed=5)
    q, kp, v, s, z, pt, sl = args
    B, Hq, D = q.shape
    cache = capi.PagedCache(
        k_pages=kp.data_ptr(), k_page_stride=kp.stride(0), k_head_stride=kp.stride(1),
        k_row_stride=kp.stride(2), v_pages=v.data_ptr(), v_dtype=capi.V_F32,
        v_page_stride=v.stride(0), v_head_stride=v.stride(1), v_row_stride=v.stride(2),
        k_scale=s.data_ptr(), k_zp=z.data_ptr(), s_batch_stride=s.stride(0),
        s_head_stride=s.stride(1), s_group_stride=s.stride(2), s_page_stride=0,
        page_table=pt.data_ptr(), pt_batch_stride=pt.stride(0), seq_lens=sl.data_ptr(),
        page_lens=None, pl_batch_stride=0, num_kv_heads=4, head_dim=D, page_rows=16,
        pages_per_group=8, max_pages=pt.shape[1], num_pages=kp.shape[0])
    nbytes = max(lib.fdi4_decode_workspace_bytes(B, Hq, D, sp) for sp in (3, 7))
    ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")  # garbage
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda").manual_seed(9)
    for it, splits in enumerate((3, 7, 3, 7, 7)):
        qi = torch.randn(B, Hq, D, device="cuda", generator=g)
        out = torch.empty(B, Hq, D, device="cuda")
        rc = lib.fdi4_decode_paged(qi.data_ptr(), B, Hq, qi.stride(0), qi.stride(1),
                                   ctypes.byref(cache), out.data_ptr(), out.stride(0),
                                   out.stride(1), splits, ws.data_ptr(), nbytes, stream)
        assert rc == 0, (it, rc)
        want = _two_launch(C, (qi, kp, v, s, z, pt, sl), splits)
        torch.cuda.synchronize()
        assert torch.equal(out, want), (it, splits)


def test_graph_replays_reuse_the_captured_workspace():
    """A captured split decode (split kernel and merge kernel) replays with the
    captured workspace; each replay, with new query values copied in between,
    equals an eager call."""
    import torch
    from flash_decode_int4 import ops
    _, args = _problem(2, 2, 128, [4000, 3100], q_heads=8, seed=11)
    q, kp, v, s, z, pt, sl = args
    q_static = q.clone()
    ops.flash_decode_paged(q_static, kp, v, s, z, pt, sl, num_splits=4)  # warm up outside
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = ops.flash_decode_paged(q_static, kp, v, s, z, pt, sl, num_splits=4)
    gen = torch.Generator(device="cuda").manual_seed(2)
    for rep in range(4):
        q_new = torch.randn(q.shape, device="cuda", generator=gen)
        q_static.copy_(q_new)
        graph.replay()
        torch.cuda.synchronize()
        eager = ops.flash_decode_paged(q_new, kp, v, s, z, pt, sl, num_splits=4)
        torch.cuda.synchronize()
        assert torch.equal(out_static, eager), rep
