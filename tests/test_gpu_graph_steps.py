"""Decode steps captured in a HIP graph.

A serving loop appends one token per sequence and attends, every step. The
sequence cache's step() does both on the device alone (append kernel, length
advance, decode), so one step can be captured and replayed. Two identical
caches are driven side by side, one eagerly and one by graph replays with new
inputs copied in between; every replay's output and the final pages, scales,
values and lengths must equal the eager ones bit for bit, and the eager path
must match the oracle.
"""

import numpy as np
import pytest

from oracle import paged_decode_f64, paged_decode_ref, quantize_groups_ref, pack_int4

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _cache(value_dtype):
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    return INT4PagedSequenceCache(num_pages=256, num_kv_heads=4, head_dim=128, max_seqs=3,
                                  max_seq_len=1024, value_dtype=value_dtype)


@pytest.mark.parametrize("value_dtype,q_heads,steps,q_dtype", [
    ("float32", 4, 6, "float32"), ("float16", 16, 5, "float32"),
    ("bfloat16", 8, 4, "bfloat16"), ("float16", 4, 4, "float16")])
def test_graph_replayed_steps_equal_eager_steps(value_dtype, q_heads, steps, q_dtype):
    import torch
    vdt = getattr(torch, value_dtype)
    qdt = getattr(torch, q_dtype)
    B, H, D, T0 = 3, 4, 128, 400
    lens0 = [100, 127, 300]                      # 127: the first step closes a group
    g = torch.Generator(device="cuda").manual_seed(5)
    k = torch.randn(B, H, T0, D, device="cuda", generator=g)
    v = torch.randn(B, H, T0, D, device="cuda", generator=g).to(vdt)
    eager, graphed = _cache(value_dtype), _cache(value_dtype)
    for c in (eager, graphed):
        c.prefill(k, v, lens0)
        c.reserve(B, steps + 1)
    k_in = [torch.randn(B, H, D, device="cuda", generator=g) for _ in range(steps + 1)]
    v_in = [torch.randn(B, H, D, device="cuda", generator=g).to(vdt) for _ in range(steps + 1)]
    q_in = [torch.randn(B, q_heads, D, device="cuda", generator=g).to(qdt)
            for _ in range(steps + 1)]

    # Step 0 eagerly on both (warm-up outside the capture), then capture step 1.
    eager_out = [eager.step(k_in[0], v_in[0], q_in[0])]
    graphed.step(k_in[0], v_in[0], q_in[0])
    k_s, v_s, q_s = k_in[1].clone(), v_in[1].clone(), q_in[1].clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = graphed.step(k_s, v_s, q_s)
    # Capturing recorded the step without running it.
    for i in range(1, steps + 1):
        eager_out.append(eager.step(k_in[i], v_in[i], q_in[i]))
        torch.cuda.synchronize()
        k_s.copy_(k_in[i])
        v_s.copy_(v_in[i])
        q_s.copy_(q_in[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager_out[i]), i
    for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
        assert torch.equal(getattr(graphed, name), getattr(eager, name)), name
    graphed.sync_lengths()
    assert list(graphed.lengths()[:B]) == [n + steps + 1 for n in lens0]

    # The eager path against the oracle after the last step.
    n = [l0 + steps + 1 for l0 in lens0]
    kk = torch.zeros(B, H, max(n), D, device="cuda")
    vv = torch.zeros(B, H, max(n), D, device="cuda")
    for b in range(B):
        kk[b, :, :lens0[b]] = k[b, :, :lens0[b]]
        vv[b, :, :lens0[b]] = v[b, :, :lens0[b]].float()
        for i in range(steps + 1):
            kk[b, :, lens0[b] + i] = k_in[i][b]
            vv[b, :, lens0[b] + i] = v_in[i][b].float()
    qr, sr, zr = quantize_groups_ref(kk.cpu().numpy(), np.array(n))
    sc = eager.k_scale[:B].cpu().numpy()
    for b in range(B):
        ng = (n[b] + 127) // 128
        np.testing.assert_array_equal(sc[b, :, :ng], sr[b, :, :ng])
    table = eager.page_table[:B].cpu().numpy()
    kp = eager.k_pages.cpu().numpy()
    vp = eager.v_pages.float().cpu().numpy()
    for b in range(B):
        npg = (n[b] + 15) // 16
        got = kp[table[b, :npg]].transpose(1, 0, 2, 3).reshape(H, npg * 16, D // 2)[:, :n[b]]
        np.testing.assert_array_equal(got, pack_int4(qr[b, :, :n[b]]))
    args = (q_in[steps].float().cpu().numpy(), kp, vp, sc, eager.k_zp[:B].cpu().numpy(), table,
            np.array(n, np.int32))
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    # A 16-bit query's output is the float32 decode of the widened query,
    # rounded once; the float32 decode is what the oracle bounds.
    full = eager.decode(q_in[steps].float())
    assert torch.equal(eager_out[steps], full.to(qdt))
    got = full.cpu().numpy()
    assert np.abs(got - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())


@pytest.mark.parametrize("q_heads,num_splits", [(4, 0), (8, 3), (16, 1)])
def test_step_equals_append_increment_decode(q_heads, num_splits):
    """step() (two launches: the append writes the advanced lengths to a
    second array, the decode reads them and writes them back) against the
    three-launch form (append, a separate length increment, decode): the same
    outputs, pages, scales, staging rows and lengths, bit for bit, over steps
    that cross a page and a group boundary, with one and several splits and
    the per-head, grouped and matrix-core kernels."""
    import torch
    from flash_decode_int4._lib import load_binding
    C = load_binding()
    B, H, D = 3, 4, 128
    lens0 = [126, 15, 250]
    g = torch.Generator(device="cuda").manual_seed(11)
    k = torch.randn(B, H, 256, D, device="cuda", generator=g)
    v = torch.randn(B, H, 256, D, device="cuda", generator=g)
    new, old = _cache("float32"), _cache("float32")
    for c in (new, old):
        c.prefill(k, v, lens0)
        c.reserve(B, 8)
    for i in range(5):
        kn = torch.randn(B, H, D, device="cuda", generator=g)
        vn = torch.randn(B, H, D, device="cuda", generator=g)
        q = torch.randn(B, q_heads, D, device="cuda", generator=g)
        out_new = new.step(kn, vn, q, num_splits)
        C.append_paged(kn, vn, old.k_stage[:B], old.k_pages, old.v_pages, old.k_scale[:B],
                       old.k_zp[:B], old.page_table[:B], old.seq_lens[:B], old.group_rows)
        old.seq_lens[:B] += 1
        out_old = old.decode(q, num_splits)
        torch.cuda.synchronize()
        assert torch.equal(out_new, out_old), i
        for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
            assert torch.equal(getattr(new, name), getattr(old, name)), (i, name)
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + 5 for n in lens0]


def test_graph_of_several_steps_equals_eager_steps():
    """Four steps captured in one graph, replayed twice: the outputs of the
    last step of each replay and the final cache equal eight eager steps."""
    import torch
    B, H, D = 3, 4, 128
    lens0 = [60, 128, 9]
    g = torch.Generator(device="cuda").manual_seed(13)
    k = torch.randn(B, H, 200, D, device="cuda", generator=g)
    v = torch.randn(B, H, 200, D, device="cuda", generator=g)
    eager, graphed = _cache("float32"), _cache("float32")
    for c in (eager, graphed):
        c.prefill(k, v, lens0)
        c.reserve(B, 9)
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, 8, D, device="cuda", generator=g)
    eager.step(kn, vn, q)
    graphed.step(kn, vn, q)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(4):
            out_g = graphed.step(kn, vn, q)
    for r in range(2):
        for _ in range(4):
            out_e = eager.step(kn, vn, q)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), r
    for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
        assert torch.equal(getattr(graphed, name), getattr(eager, name)), name
    graphed.sync_lengths()
    assert list(graphed.lengths()[:B]) == [n + 9 for n in lens0]
