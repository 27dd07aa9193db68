"""Page pools past 4 GiB, every page in use lying past the first 2^32 bytes
of the key pool (and 2^34 bytes of the value pool): with 2 kv-heads, 16-row
pages and head_dim 128 a key page is 2 KiB, so page 2^21 starts at byte
2^32 of the keys. Every kernel forms a page's address in 64 bits (the
grouped quantizer's page writes, the decode kernels' key, value and scale
loads, the append kernel's and the one-launch step's writes), so pages at
the top of a pool read and write like pages at the bottom.

Checked against the oracle on host copies of the used pages (the quantizer
bit-exact, the decode within max(1e-5, 1.25 x the oracle's own distance
from float64)), per q-head and grouped (four q-heads per kv-head), with the
library's split count and forced ones; and the serving step bit for bit
against the three-launch form (append kernel, a length increment, decode)
on a twin cache whose pages also come from the top of its pool."""

import numpy as np
import pytest

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5
HKV, PR, D, GROUP = 2, 16, 128, 128
P_LOW = (1 << 32) // (HKV * PR * D // 2)      # first page past 2^32 bytes of keys


def _free_gpu():
    import gc
    import torch
    gc.collect()
    torch.cuda.empty_cache()


def _compact(table, lens, pages_used):
    """The page table over a compact copy of the used pages (in the order of
    pages_used)."""
    where = {int(p): j for j, p in enumerate(pages_used)}
    ct = np.zeros_like(table)
    for b, n in enumerate(lens):
        for lp in range((int(n) + PR - 1) // PR):
            ct[b, lp] = where[int(table[b, lp])]
    return ct


def _check_decode(out, q, kpc, vc32, sn, zn, ctable, lens, what):
    args = (q, kpc, vc32, sn, zn, ctable, lens, PR, GROUP)
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    got = out.float().cpu().numpy()
    e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
    print(f"[parity] large pool {what}: |hip-oracle| {e32:.2e} |oracle-f64| {eo:.2e}",
          flush=True)
    assert e32 <= max(TOL, 1.25 * eo), (what, e32, eo)


def test_quantize_and_decode_past_4_gib():
    import torch
    from flash_decode_int4 import ops
    rng = np.random.RandomState(11)
    lens = np.array([300, 1000, 129], np.int32)
    B = len(lens)
    n_pages = (lens + PR - 1) // PR
    used = int(n_pages.sum())
    P = P_LOW + used + 7
    pages_used = P_LOW + rng.permutation(used + 7)[:used]
    table = np.zeros((B, int(n_pages.max())), np.int32)
    off = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = pages_used[off:off + n]
        off += n
    dev = torch.device("cuda")
    kp = torch.empty(P, HKV, PR, D // 2, dtype=torch.uint8, device=dev)
    vt = torch.empty(P, HKV, PR, D, dtype=torch.float16, device=dev)
    assert kp.numel() > (1 << 32) and vt.numel() * 2 > (1 << 34)
    idx = torch.from_numpy(pages_used.astype(np.int64)).to(dev)
    vc16 = rng.randn(used, HKV, PR, D).astype(np.float16)
    vt[idx] = torch.from_numpy(vc16).to(dev)
    T = int(lens.max())
    G = (T + GROUP - 1) // GROUP
    k = rng.randn(B, HKV, T, D).astype(np.float32)
    s = torch.zeros(B, HKV, G, D, device=dev)
    z = torch.zeros(B, HKV, G, D, device=dev)
    pt = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(lens).to(dev)
    ops.quantize_int4_paged(torch.from_numpy(k).to(dev), sl, pt, kp, s, z, GROUP)
    torch.cuda.synchronize()

    kpc = kp[idx].cpu().numpy()
    sn, zn = s.cpu().numpy(), z.cpu().numpy()
    ctable = _compact(table, lens, pages_used)
    qr, sr, zr = quantize_groups_ref(k, lens, group_size=GROUP)
    for b in range(B):
        n = int(lens[b])
        ng = (n + GROUP - 1) // GROUP
        np.testing.assert_array_equal(sn[b, :, :ng], sr[b, :, :ng])
        np.testing.assert_array_equal(zn[b, :, :ng], zr[b, :, :ng])
        for lp in range((n + PR - 1) // PR):
            rows = min(PR, n - lp * PR)
            np.testing.assert_array_equal(kpc[ctable[b, lp], :, :rows],
                                          pack_int4(qr[b, :, lp * PR:lp * PR + rows]))

    vc32 = vc16.astype(np.float32)
    for rep, splits in [(1, 0), (1, 3), (4, 0), (4, 2)]:
        q = rng.randn(B, HKV * rep, D).astype(np.float32)
        out = ops.flash_decode_paged(torch.from_numpy(q).to(dev), kp, vt, s, z, pt, sl, GROUP,
                                     splits)
        _check_decode(out, q, kpc, vc32, sn, zn, ctable, lens,
                      f"q-heads per kv-head {rep}, splits {splits}")
    del kp, vt, s, z, pt, sl, idx
    _free_gpu()


def _old_step(c, kn, vn, q):
    """Append kernel, a separate length increment, decode."""
    from flash_decode_int4._lib import load_binding
    B = kn.shape[0]
    load_binding().append_paged(kn, vn, c.k_stage[:B], c.k_pages, c.v_pages, c.k_scale[:B],
                                c.k_zp[:B], c.page_table[:B], c.seq_lens[:B], c.group_rows)
    c.seq_lens[:B] += 1
    return c.decode(q)


def test_serving_step_past_4_gib():
    import torch
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    B, steps = 2, 6
    lens0 = [125, 250]
    P = P_LOW + 64
    caches = [INT4PagedSequenceCache(num_pages=P, num_kv_heads=HKV, head_dim=D, max_seqs=B,
                                     max_seq_len=512, page_rows=PR, group_rows=GROUP,
                                     value_dtype="float16")
              for _ in range(2)]
    for c in caches:
        c._free = list(range(P))           # pages are taken from the top: P-1, P-2, ...
    g = torch.Generator(device="cuda").manual_seed(5)
    T = max(lens0)
    k = torch.randn(B, HKV, T, D, device="cuda", generator=g)
    v = torch.randn(B, HKV, T, D, device="cuda", generator=g).half()
    for c in caches:
        c.prefill(k, v, lens0)
        c.reserve(B, steps)
    new, old = caches
    mapped = [p for b in range(B) for p in new._pages[b]]
    assert min(mapped) >= P_LOW, min(mapped)
    assert torch.equal(new.page_table, old.page_table)
    for i in range(steps):
        kn = torch.randn(B, HKV, D, device="cuda", generator=g)
        vn = torch.randn(B, HKV, D, device="cuda", generator=g).half()
        q = torch.randn(B, HKV, D, device="cuda", generator=g)
        out_new = new.step(kn, vn, q)
        out_old = _old_step(old, kn, vn, q)
        assert torch.equal(out_new, out_old), i
    torch.cuda.synchronize()
    idx = torch.tensor(mapped, dtype=torch.int64, device="cuda")
    for name in ("k_pages", "v_pages"):
        assert torch.equal(getattr(new, name)[idx], getattr(old, name)[idx]), name
    for name in ("k_scale", "k_zp", "seq_lens", "k_stage"):
        assert torch.equal(getattr(new, name), getattr(old, name)), name
    lens = new.seq_lens.cpu().numpy().astype(np.int32)
    assert list(lens) == [n + steps for n in lens0]

    # The last step's output against the oracle on copies of the used pages.
    table = new.page_table.cpu().numpy()
    ctable = _compact(table, lens, np.asarray(mapped))
    kpc = new.k_pages[idx].cpu().numpy()
    vc32 = new.v_pages[idx].float().cpu().numpy()
    _check_decode(out_new, q.cpu().numpy(), kpc, vc32, new.k_scale.cpu().numpy(),
                  new.k_zp.cpu().numpy(), ctable, lens, "after the serving steps")
    del caches, new, old, idx
    _free_gpu()
