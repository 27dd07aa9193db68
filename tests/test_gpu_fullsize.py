"""The path at the benchmark's full sizes (B8 H32 D128 T2048; the
context-length sweep B8 H32 D128 at T = 512, 8192 and 32768, the last a
4.3 GB value pool; B64 H32 D128 T4096, also a 4.3 GB pool whose byte offsets
pass 2^32; ragged B32 up to 8192 tokens), through properties that do not
depend on size plus sampled streams against the oracle (float32 value pages;
the anchor also with float16 and bfloat16 value pages; grouped query heads at
B8 Hkv8 Hq32 T8192):

* the grouped quantizer is bit-exact on sampled (sequence, head) streams;
* decoding is invariant, bit for bit, under a different physical page
  permutation of the same logical data (page-table and offset arithmetic);
* split counts agree (split-K merge);
* sampled streams of the full decode match the page-loop oracle.
"""

import numpy as np
import pytest

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _ops():
    from flash_decode_int4 import ops
    return ops


def _build(name, value_dtype="float32"):
    import torch
    from flash_decode_int4.workloads import make_workload
    w = make_workload(name, backend="torch", seed=2024, value_dtype=value_dtype)
    B, H, D = w["batch"], w["heads"], w["head_dim"]
    G = (w["max_tokens"] + 127) // 128
    dev = torch.device("cuda")
    st = dict(w=w, q=w["q"], k=w["k"], v=w["v_pages"],
              pt=torch.as_tensor(w["page_table"], device=dev),
              sl=torch.as_tensor(w["seq_lens"], device=dev),
              kp=torch.zeros(w["num_pages"], H, 16, D // 2, dtype=torch.uint8, device=dev),
              s=torch.zeros(B, H, G, D, device=dev), z=torch.zeros(B, H, G, D, device=dev))
    _ops().quantize_int4_paged(st["k"], st["sl"], st["pt"], st["kp"], st["s"], st["z"], 128)
    return st


def _streams(st, n, seed):
    """n (sequence, head) pairs with at least one token, chosen at random."""
    lens = np.asarray(st["w"]["seq_lens"])
    rng = np.random.RandomState(seed)
    live = np.nonzero(lens > 0)[0]
    return [(int(rng.choice(live)), int(rng.randint(st["w"]["heads"]))) for _ in range(n)]


def _stream_problem(st, b, h):
    """The stream's pages gathered into a one-sequence, one-head paged problem."""
    n = int(st["w"]["seq_lens"][b])
    npg = (n + 15) // 16
    phys = st["w"]["page_table"][b, :npg]
    kp = st["kp"][phys, h:h + 1].cpu().numpy()
    vp = st["v"][phys, h:h + 1].float().cpu().numpy()
    s = st["s"][b:b + 1, h:h + 1].cpu().numpy()
    z = st["z"][b:b + 1, h:h + 1].cpu().numpy()
    q = st["q"][b:b + 1, h:h + 1].cpu().numpy()
    table = np.arange(npg, dtype=np.int32)[None]
    return (q, kp, vp, s, z, table, np.array([n], np.int32), 16, 128)


def torch_index(mask):
    import torch
    return torch.as_tensor(np.nonzero(mask)[0], device="cuda")


@pytest.fixture(scope="module",
                params=["anchor", "sweep_512", "sweep_8192", "sweep_32768", "llama", "ragged"])
def built(request):
    import torch
    st = _build(request.param)
    yield request.param, st
    del st
    torch.cuda.empty_cache()


def test_quantizer_bit_exact_on_sampled_streams(built):
    name, st = built
    for b, h in _streams(st, 6, seed=1):
        n = int(st["w"]["seq_lens"][b])
        k = st["k"][b:b + 1, h:h + 1, :n].cpu().numpy()
        qr, sr, zr = quantize_groups_ref(k, np.array([n]))
        ng = (n + 127) // 128
        np.testing.assert_array_equal(st["s"][b, h, :ng].cpu().numpy(), sr[0, 0, :ng])
        np.testing.assert_array_equal(st["z"][b, h, :ng].cpu().numpy(), zr[0, 0, :ng])
        npg = (n + 15) // 16
        phys = st["w"]["page_table"][b, :npg]
        got = st["kp"][phys, h].cpu().numpy()                     # [npg, 16, D/2]
        want = pack_int4(qr[0, 0])                                 # [n, D/2]
        for lp in range(npg):
            r = min(16, n - lp * 16)
            np.testing.assert_array_equal(got[lp, :r], want[lp * 16:lp * 16 + r])


def test_decode_matches_oracle_on_sampled_streams(built):
    name, st = built
    out = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                    st["sl"])
    assert bool(out.isfinite().all())
    lens = np.asarray(st["w"]["seq_lens"])
    if (lens == 0).any():
        assert bool((out[torch_index(lens == 0)] == 0).all())
    for b, h in _streams(st, 6, seed=2):
        args = _stream_problem(st, b, h)
        o32, o64 = paged_decode_ref(*args)[0, 0], paged_decode_f64(*args)[0, 0]
        got = out[b, h].cpu().numpy()
        e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
        assert e32 <= max(TOL, 1.25 * eo), (name, b, h, e32, eo)


def test_page_permutation_invariance(built):
    """Same logical pages at other physical places: identical packed bytes
    (through the tables) and a bitwise identical decode."""
    import torch
    name, st = built
    w = st["w"]
    P = w["num_pages"]
    perm = torch.as_tensor(np.random.RandomState(9).permutation(P), device="cuda")
    pt2 = perm[st["pt"].long()].to(torch.int32)
    v2 = torch.empty_like(st["v"])
    v2[perm] = st["v"]
    kp2 = torch.zeros_like(st["kp"])
    s2, z2 = torch.zeros_like(st["s"]), torch.zeros_like(st["z"])
    _ops().quantize_int4_paged(st["k"], st["sl"], pt2, kp2, s2, z2, 128)
    used = torch.as_tensor(np.unique(np.concatenate(
        [w["page_table"][b, :(int(n) + 15) // 16] for b, n in enumerate(w["seq_lens"])])),
        device="cuda").long()
    # Every stored row of every used page moved with its page (rows past a
    # sequence's length are never written, in either pool).
    assert torch.equal(kp2[perm[used]], st["kp"][used])
    assert torch.equal(s2, st["s"]) and torch.equal(z2, st["z"])
    a = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"], st["sl"])
    b = _ops().flash_decode_paged(st["q"], kp2, v2, s2, z2, pt2, st["sl"])
    assert torch.equal(a, b)
    del v2, kp2


def test_split_counts_agree(built):
    """One split against 4 and 16: the same float64 logits, but value sums over
    up to 8192 rows accumulated in float32 in another order and merged with
    other weights, so a few ulps of the output's magnitude (~1) apart."""
    name, st = built
    base = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                     st["sl"], num_splits=1)
    for splits in (4, 16):
        got = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                        st["sl"], num_splits=splits)
        assert (got - base).abs().max().item() < 5e-6, (name, splits)


@pytest.mark.parametrize("value_dtype", ["float16", "bfloat16"])
def test_16bit_values_at_the_anchor(value_dtype):
    """B8 H32 D128 T2048 with 16-bit value pages: sampled streams of the full
    decode against the oracle fed the same (widened) values."""
    import torch
    st = _build("anchor", value_dtype)
    assert st["v"].dtype == getattr(torch, value_dtype)
    out = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                    st["sl"])
    assert out.dtype == torch.float32 and bool(out.isfinite().all())
    for b, h in _streams(st, 6, seed=3):
        args = _stream_problem(st, b, h)
        o32, o64 = paged_decode_ref(*args)[0, 0], paged_decode_f64(*args)[0, 0]
        got = out[b, h].cpu().numpy()
        e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
        assert e32 <= max(TOL, 1.25 * eo), (value_dtype, b, h, e32, eo)
    del st
    torch.cuda.empty_cache()


def test_grouped_query_heads_at_full_size():
    """B8 Hkv8 Hq32 D128 T8192 (four q-heads per kv-head: the int8 matrix-core
    kernel with splits and the merge): sampled (sequence, q-head) streams
    against the oracle over the kv-head the q-head reads."""
    import torch
    st = _build("gqa")
    w = st["w"]
    hq, hkv = w["q_heads"], w["heads"]
    assert st["q"].shape[1] == hq and hq == 4 * hkv
    out = _ops().flash_decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                    st["sl"])
    assert bool(out.isfinite().all())
    rng = np.random.RandomState(4)
    for _ in range(8):
        b, qh = int(rng.randint(w["batch"])), int(rng.randint(hq))
        q_, kp, vp, s_, z_, table, n, pr, grp = _stream_problem(st, b, qh // (hq // hkv))
        q_ = st["q"][b:b + 1, qh:qh + 1].cpu().numpy()
        args = (q_, kp, vp, s_, z_, table, n, pr, grp)
        o32, o64 = paged_decode_ref(*args)[0, 0], paged_decode_f64(*args)[0, 0]
        got = out[b, qh].cpu().numpy()
        e32, eo = np.abs(got - o32).max(), np.abs(o32 - o64).max()
        assert e32 <= max(TOL, 1.25 * eo), (b, qh, e32, eo)
    del st
    torch.cuda.empty_cache()
