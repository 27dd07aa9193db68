"""The one-launch serving step (fdi4_decode_step with one decode workgroup per
(sequence, kv-head)): every workgroup appends its token, re-quantizes the
open scale group (four waves, a quarter of the channels each, with no
workgroup barrier, while the other waves decode), decodes over the advanced
length, and the last workgroup of a sequence advances its length. Checked bit for bit against the
three-launch form (append kernel, a length increment, decode) on twin
caches, over steps that cross page and group boundaries, for every value
type, head_dim 64/128/256, page sizes 2/8/16/32 and groups 64/128/256; replayed
from a captured HIP graph; at a sequence already at the cache's capacity;
and at the anchor size B8 H32 D128 from 2048 tokens."""

import pytest

pytestmark = pytest.mark.gpu


def _twins(B, H, D, lens0, page_rows, group_rows, value_dtype, max_seq_len, seed):
    import torch
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    pages = B * ((max_seq_len + page_rows - 1) // page_rows) + 4
    caches = [INT4PagedSequenceCache(num_pages=pages, num_kv_heads=H, head_dim=D, max_seqs=B,
                                     max_seq_len=max_seq_len, page_rows=page_rows,
                                     group_rows=group_rows, value_dtype=value_dtype)
              for _ in range(2)]
    g = torch.Generator(device="cuda").manual_seed(seed)
    T = max(max(lens0), 1)
    k = torch.randn(B, H, T, D, device="cuda", generator=g)
    v = torch.randn(B, H, T, D, device="cuda", generator=g).to(getattr(torch, value_dtype))
    for c in caches:
        c.prefill(k, v, lens0)
    return caches, g


def _old_step(c, kn, vn, q):
    """Append kernel, a separate length increment, decode."""
    from flash_decode_int4._lib import load_binding
    B = kn.shape[0]
    load_binding().append_paged(kn, vn, c.k_stage[:B], c.k_pages, c.v_pages, c.k_scale[:B],
                                c.k_zp[:B], c.page_table[:B], c.seq_lens[:B], c.group_rows)
    c.seq_lens[:B] += 1
    return c.decode(q)


def _same(a, b, what):
    import torch
    for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
        assert torch.equal(getattr(a, name), getattr(b, name)), (what, name)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("D,page_rows,group_rows,value_dtype,lens0", [
    (128, 16, 128, "float32", [126, 15, 250, 1]),
    (128, 16, 64, "float16", [62, 16, 0, 300]),
    (64, 32, 256, "bfloat16", [250, 31, 64, 5]),
    (256, 16, 128, "float32", [127, 200, 17, 40]),
    (128, 32, 256, "float16", [255, 1, 96, 130]),
    # long enough that each SIMD's last chunks form a range of their own,
    # which the step hands to the older wave of the SIMD (eight waves)
    (128, 16, 128, "float32", [1023, 700, 517, 2047]),
    (64, 16, 64, "bfloat16", [1500, 64, 900, 1279]),
    # pages of 8 rows; pages of 2 rows, so a 256-row group spans 128 pages
    (128, 8, 128, "bfloat16", [129, 7, 300, 64]),
    (64, 2, 256, "float32", [255, 140, 3, 0]),
])
def test_fused_step_equals_three_launches(D, page_rows, group_rows, value_dtype, lens0, waves):
    import torch
    from flash_decode_int4 import capi
    B, H, steps = len(lens0), 2, 6
    (new, old), g = _twins(B, H, D, lens0, page_rows, group_rows, value_dtype,
                           max(512, max(lens0) + 64), 31)
    vdt = getattr(torch, value_dtype)
    for c in (new, old):
        c.reserve(B, steps)
    # one split (the one-launch step), both workgroup sizes
    with capi.tuning(decode_target_waves=1, decode_waves=waves):
        for i in range(steps):
            kn = torch.randn(B, H, D, device="cuda", generator=g)
            vn = torch.randn(B, H, D, device="cuda", generator=g).to(vdt)
            q = torch.randn(B, H, D, device="cuda", generator=g)
            out_new = new.step(kn, vn, q)
            out_old = _old_step(old, kn, vn, q)
            torch.cuda.synchronize()
            assert torch.equal(out_new, out_old), i
            _same(new, old, i)
    assert int(new._step_counters.abs().sum()) == 0          # counters left at zero
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + steps for n in lens0]


def test_fused_steps_replayed_from_a_graph():
    """Three one-launch steps per captured graph, replayed with new inputs in
    between, against eager three-launch steps on a twin cache."""
    import torch
    from flash_decode_int4 import capi
    B, H, D = 3, 4, 128
    lens0 = [125, 16, 300]
    (new, old), g = _twins(B, H, D, lens0, 16, 128, "float32", 512, 41)
    for c in (new, old):
        c.reserve(B, 10)
    kn = torch.zeros(B, H, D, device="cuda")
    vn = torch.zeros(B, H, D, device="cuda")
    q = torch.zeros(B, H, D, device="cuda")
    with capi.tuning(decode_target_waves=1):
        new.step(kn, vn, q)                                # warm-up, outside the capture
        _old_step(old, kn, vn, q)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(3):
                out_g = new.step(kn, vn, q)
        for r in range(3):
            kn.copy_(torch.randn(B, H, D, device="cuda", generator=g))
            vn.copy_(torch.randn(B, H, D, device="cuda", generator=g))
            q.copy_(torch.randn(B, H, D, device="cuda", generator=g))
            torch.cuda.synchronize()
            graph.replay()
            for _ in range(3):
                out_o = _old_step(old, kn, vn, q)
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_o), r
            _same(new, old, r)
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + 10 for n in lens0]


def test_fused_step_at_capacity_appends_nothing():
    """A sequence already holding the cache's capacity keeps its length and
    attends over its rows, as the three-launch form does (its append kernel
    skips the position and the increment is not applied)."""
    import torch
    from flash_decode_int4 import capi
    B, H, D = 2, 2, 128
    (new, old), g = _twins(B, H, D, [128, 40], 16, 128, "float32", 128, 51)
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, H, D, device="cuda", generator=g)
    with capi.tuning(decode_target_waves=1):
        out_new = load_step(new, kn, vn, q)
    torch.cuda.synchronize()
    assert new.seq_lens[:B].tolist() == [128, 41]
    from flash_decode_int4._lib import load_binding
    load_binding().append_paged(kn, vn, old.k_stage[:B], old.k_pages, old.v_pages,
                                old.k_scale[:B], old.k_zp[:B], old.page_table[:B],
                                old.seq_lens[:B], old.group_rows)
    old.seq_lens[1] += 1
    out_old = old.decode(q)
    torch.cuda.synchronize()
    assert torch.equal(out_new, out_old)
    _same(new, old, "capacity")


def load_step(c, kn, vn, q):
    """fdi4_decode_step through the binding, without the cache's host-side
    reservation check (the full sequence has no page left to reserve)."""
    from flash_decode_int4._lib import load_binding
    return load_binding().decode_step(q, kn, vn, c.k_stage, c.k_pages, c.v_pages, c.k_scale,
                                      c.k_zp, c.page_table, c.seq_lens, c.group_rows,
                                      c._step_counters, c._lens_next)


def test_fused_step_at_the_anchor_size():
    """B8 H32 D128 from 2048 tokens: the library's own plan is one split, so
    step() takes the one-launch form; 20 steps against the three-launch form."""
    import torch
    from flash_decode_int4 import capi
    B, H, D = 8, 32, 128
    (new, old), g = _twins(B, H, D, [2048] * B, 16, 128, "float32", 2100, 61)
    lib = capi.load()
    cache = capi.PagedCache(max_pages=new.max_pages_per_seq, page_rows=16, num_kv_heads=H,
                            head_dim=D)
    assert lib.fdi4_decode_num_splits(B, H, cache) == 1
    for c in (new, old):
        c.reserve(B, 20)
    for i in range(20):
        kn = torch.randn(B, H, D, device="cuda", generator=g)
        vn = torch.randn(B, H, D, device="cuda", generator=g)
        q = torch.randn(B, H, D, device="cuda", generator=g)
        out_new = new.step(kn, vn, q)
        out_old = _old_step(old, kn, vn, q)
        torch.cuda.synchronize()
        assert torch.equal(out_new, out_old), i
    _same(new, old, "anchor")
    assert int(new._step_counters.abs().sum()) == 0


def _reference_step(c, kn, vn, q, after, splits):
    """Append kernel (which skips a position outside [0, capacity)), the
    lengths set to `after`, decode with `splits` splits."""
    import torch
    from flash_decode_int4._lib import load_binding
    B = kn.shape[0]
    load_binding().append_paged(kn, vn, c.k_stage[:B], c.k_pages, c.v_pages, c.k_scale[:B],
                                c.k_zp[:B], c.page_table[:B], c.seq_lens[:B], c.group_rows)
    c.seq_lens[:B] = torch.tensor(after, dtype=torch.int32, device="cuda")
    return c.decode(q, num_splits=splits)


@pytest.mark.parametrize("form", ["one_launch", "split_fused", "two_launch"])
def test_step_lengths_outside_the_cache(form):
    """Lengths below 0 and above the cache's capacity: no token is appended,
    the length is left as read, and the decode attends over it clamped to
    [0, capacity] -- in the one-launch step, in the fused step over two splits
    (then the merge), in the two-launch step (two q-heads per kv-head), and in
    the append kernel + decode form, bit for bit (outputs, pages, scales,
    values, staging rows, lengths)."""
    import torch
    from flash_decode_int4 import capi
    from flash_decode_int4._lib import load_binding
    B, H, D = 5, 2, 128
    HQ = 2 * H if form == "two_launch" else H
    lens0 = [100, 40, 200, 17, 511]
    (new, old), g = _twins(B, H, D, lens0, 16, 128, "float32", 512, 71)
    cap = new.max_pages_per_seq * new.page_rows
    assert cap == 512
    raw = [-5, 40, 2 ** 31 - 1, cap + 9, 511]
    after = [-5, 41, 2 ** 31 - 1, cap + 9, 512]
    for c in (new, old):
        c.seq_lens[:B] = torch.tensor(raw, dtype=torch.int32, device="cuda")
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, HQ, D, device="cuda", generator=g)
    # One split takes the one-launch step; four-wave workgroups and a high
    # wave target give two splits (32 chunks of 4 per wave, 16 per split:
    # two whole 128-row groups each), so the fused step and the merge; with
    # two q-heads per kv-head the step is the append kernel, then the decode.
    tune = {"decode_waves": 4,
            "decode_target_waves": 1 if form == "one_launch" else 4096}
    C = load_binding()
    with capi.tuning(**tune):
        splits = int(C.decode_num_splits(B, HQ, H, D, new.max_pages_per_seq, 16))
        assert (splits == 1) == (form == "one_launch")
        out_new = load_step(new, kn, vn, q)
        out_old = _reference_step(old, kn, vn, q, after, splits)
    torch.cuda.synchronize()
    assert new.seq_lens[:B].tolist() == after
    assert torch.isfinite(out_new).all()
    assert torch.equal(out_new[0], torch.zeros_like(out_new[0]))    # length -5: no rows
    assert torch.equal(out_new, out_old)
    _same(new, old, form)
    assert int(new._step_counters.abs().sum()) == 0
