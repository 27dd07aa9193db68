"""Pages of one row: every 16-row chunk of the decode holds one valid row,
and a 256-row scale group spans 256 pages, the most the serving step keeps
of a group's page-table entries. The grouped quantizer is bit-exact and the
decode within max(1e-5, 1.25 x the oracle's own distance from float64) of
the page-loop oracle over random page permutations (lengths 0, 1, on and
next to group edges); the serving step is bit for bit the three-launch form
(append kernel, a length increment, decode) over steps that cross a group
boundary, with one split at either workgroup size and with the library's
own plan."""

import numpy as np
import pytest

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.mark.parametrize("D,group,vdtype,splits", [
    (64, 64, "float32", 0),
    (128, 256, "float16", 3),
    (128, 128, "bfloat16", 0),
    (256, 256, "float32", 2),
])
def test_quantize_and_decode_with_one_row_pages(D, group, vdtype, splits):
    import torch
    from flash_decode_int4 import ops
    rng = np.random.RandomState(D + group)
    hkv, rep = 2, 2
    lens = np.array([0, 1, group - 1, group, group + 1, 2 * group + 45, 300], np.int32)
    B, hq = len(lens), hkv * rep
    P = int(lens.sum()) + 3
    perm = rng.permutation(P)
    table = np.zeros((B, int(lens.max())), np.int32)
    off = 0
    for b, n in enumerate(lens):
        table[b, :n] = perm[off:off + n]
        off += n
    T = int(lens.max())
    G = (T + group - 1) // group
    k = rng.randn(B, hkv, T, D).astype(np.float32)
    v = rng.randn(P, hkv, 1, D).astype(np.float32)
    q = rng.randn(B, hq, D).astype(np.float32)
    dev = torch.device("cuda")
    vt = torch.from_numpy(v).to(dev).to(getattr(torch, vdtype))
    kp = torch.zeros(P, hkv, 1, D // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, hkv, G, D, device=dev)
    z = torch.zeros(B, hkv, G, D, device=dev)
    pt = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(lens).to(dev)
    ops.quantize_int4_paged(torch.from_numpy(k).to(dev), sl, pt, kp, s, z, group)

    qr, sr, zr = quantize_groups_ref(k, lens, group_size=group)
    kpn, sn, zn = kp.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy()
    for b in range(B):
        n = int(lens[b])
        ng = (n + group - 1) // group
        np.testing.assert_array_equal(sn[b, :, :ng], sr[b, :, :ng])
        np.testing.assert_array_equal(zn[b, :, :ng], zr[b, :, :ng])
        for t in range(n):
            np.testing.assert_array_equal(kpn[table[b, t], :, 0], pack_int4(qr[b, :, t]))

    out = ops.flash_decode_paged(torch.from_numpy(q).to(dev), kp, vt, s, z, pt, sl, group,
                                 splits)
    args = (q, kpn, vt.float().cpu().numpy(), sn, zn, table, lens, 1, group)
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    got = out.cpu().numpy()
    e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
    print(f"[parity] one-row pages D{D} group {group} {vdtype}: |hip-oracle| {e32:.2e} "
          f"|oracle-f64| {eo:.2e}", flush=True)
    assert e32 <= max(TOL, 1.25 * eo), (e32, eo)
    assert np.all(got[lens == 0] == 0.0)


def _twins(B, H, D, lens0, group, value_dtype, max_seq_len, seed):
    import torch
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    caches = [INT4PagedSequenceCache(num_pages=B * max_seq_len + 4, num_kv_heads=H, head_dim=D,
                                     max_seqs=B, max_seq_len=max_seq_len, page_rows=1,
                                     group_rows=group, value_dtype=value_dtype)
              for _ in range(2)]
    g = torch.Generator(device="cuda").manual_seed(seed)
    T = max(lens0)
    k = torch.randn(B, H, T, D, device="cuda", generator=g)
    v = torch.randn(B, H, T, D, device="cuda", generator=g).to(getattr(torch, value_dtype))
    for c in caches:
        c.prefill(k, v, lens0)
    return caches, g


def _old_step(c, kn, vn, q):
    from flash_decode_int4._lib import load_binding
    B = kn.shape[0]
    load_binding().append_paged(kn, vn, c.k_stage[:B], c.k_pages, c.v_pages, c.k_scale[:B],
                                c.k_zp[:B], c.page_table[:B], c.seq_lens[:B], c.group_rows)
    c.seq_lens[:B] += 1
    return c.decode(q)


@pytest.mark.parametrize("waves", [4, 8, 0])
def test_serving_step_with_one_row_pages(waves):
    import contextlib
    import torch
    from flash_decode_int4 import capi
    B, H, D, steps = 3, 2, 128, 5
    lens0 = [254, 30, 509]
    (new, old), g = _twins(B, H, D, lens0, 256, "float32", 600, 71 + waves)
    for c in (new, old):
        c.reserve(B, steps)
    tune = (capi.tuning(decode_target_waves=1, decode_waves=waves) if waves
            else contextlib.nullcontext())
    with tune:
        for i in range(steps):
            kn = torch.randn(B, H, D, device="cuda", generator=g)
            vn = torch.randn(B, H, D, device="cuda", generator=g)
            q = torch.randn(B, H, D, device="cuda", generator=g)
            out_new = new.step(kn, vn, q)
            out_old = _old_step(old, kn, vn, q)
            torch.cuda.synchronize()
            assert torch.equal(out_new, out_old), i
    for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
        assert torch.equal(getattr(new, name), getattr(old, name)), name
    assert int(new._step_counters.abs().sum()) == 0
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + steps for n in lens0]
