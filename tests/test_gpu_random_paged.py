"""Seeded random configurations of the paged path against the oracle: head
dims 64/128/256, page sizes 4..64 rows, scale groups of 64/128/256 tokens,
1-3 kv-heads with 1-8 q-heads each, lengths from 0 to ~700 (empty sequences,
lengths on and next to page and group edges), float32/float16/bfloat16 values
and queries, automatic and forced split counts, random page permutations.

Per case: the grouped quantizer's packed pages, scales and zero-points are
bit-exact with the oracle's grouped quantizer (read back through the page
table); the float32-query decode is within max(1e-5, 1.25 x the oracle's own
distance from float64) of the page-loop oracle fed the identical widened
values; a 16-bit query's output equals that float32 decode of the widened
query rounded to the query's type, bit for bit."""

import numpy as np
import pytest

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5
N_CASES = 100


def _case(seed):
    rng = np.random.RandomState(seed)
    D = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 3]))
    rep = int(rng.choice([1, 2, 3, 4, 8]))
    B = int(rng.randint(1, 5))
    page_rows = int(rng.choice([4, 8, 16, 32, 64]))
    group = int(rng.choice([g for g in (64, 128, 256) if g % page_rows == 0]))
    edges = [0, 1, page_rows - 1, page_rows, page_rows + 1, group - 1, group, group + 1,
             2 * group + page_rows, int(rng.randint(1, 700))]
    lens = [int(rng.choice(edges)) if rng.rand() < 0.6 else int(rng.randint(0, 700))
            for _ in range(B)]
    vdtype = str(rng.choice(["float32", "float16", "bfloat16"]))
    qdtype = str(rng.choice(["float32", "float16", "bfloat16"]))
    splits = int(rng.choice([0, 0, 1, 2, 5]))
    return dict(D=D, hkv=hkv, rep=rep, B=B, page_rows=page_rows, group=group, lens=lens,
                vdtype=vdtype, qdtype=qdtype, splits=splits)


def _layout(lens, page_rows, rng):
    n_pages = [(n + page_rows - 1) // page_rows for n in lens]
    P = max(sum(n_pages), 1)
    perm = rng.permutation(P)
    table = np.zeros((len(lens), max(max(n_pages), 1)), np.int32)
    off = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[off:off + n]
        off += n
    return table, P


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_paged_case(seed):
    import torch
    from flash_decode_int4 import ops
    c = _case(seed)
    D, hkv, B, pr, group = c["D"], c["hkv"], c["B"], c["page_rows"], c["group"]
    hq = hkv * c["rep"]
    lens = np.array(c["lens"], np.int32)
    rng = np.random.RandomState(1000 + seed)
    table, P = _layout(lens, pr, rng)
    T = max(int(lens.max()), 1)
    G = (T + group - 1) // group
    k = rng.randn(B, hkv, T, D).astype(np.float32)
    v = rng.randn(P, hkv, pr, D).astype(np.float32)
    q = rng.randn(B, hq, D).astype(np.float32)
    dev = torch.device("cuda")
    vt = torch.from_numpy(v).to(dev).to(getattr(torch, c["vdtype"]))
    qdt = getattr(torch, c["qdtype"])
    qt = torch.from_numpy(q).to(dev).to(qdt)
    kp = torch.zeros(P, hkv, pr, D // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, hkv, G, D, device=dev)
    z = torch.zeros(B, hkv, G, D, device=dev)
    pt = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(lens).to(dev)
    ops.quantize_int4_paged(torch.from_numpy(k).to(dev), sl, pt, kp, s, z, group)

    # Quantizer: bit-exact through the page table.
    qr, sr, zr = quantize_groups_ref(k, lens, group_size=group)
    kpn, sn, zn = kp.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy()
    for b in range(B):
        n = int(lens[b])
        ng = (n + group - 1) // group
        np.testing.assert_array_equal(sn[b, :, :ng], sr[b, :, :ng], err_msg=str(c))
        np.testing.assert_array_equal(zn[b, :, :ng], zr[b, :, :ng], err_msg=str(c))
        for lp in range((n + pr - 1) // pr):
            rows = min(pr, n - lp * pr)
            np.testing.assert_array_equal(kpn[table[b, lp], :, :rows],
                                          pack_int4(qr[b, :, lp * pr:lp * pr + rows]),
                                          err_msg=str(c))

    # Decode: float32 path against the oracle, 16-bit queries against it rounded.
    q32 = qt.float()
    out32 = ops.flash_decode_paged(q32, kp, vt, s, z, pt, sl, group, c["splits"])
    args = (q32.cpu().numpy(), kpn, vt.float().cpu().numpy(), sn, zn, table, lens, pr, group)
    o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
    got = out32.cpu().numpy()
    e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
    assert e32 <= max(TOL, 1.25 * eo), (c, e32, eo)
    assert np.all(got[lens == 0] == 0.0), c
    if c["qdtype"] != "float32":
        out16 = ops.flash_decode_paged(qt, kp, vt, s, z, pt, sl, group, c["splits"])
        assert out16.dtype == qdt
        assert torch.equal(out16.view(torch.int16), out32.to(qdt).view(torch.int16)), c
