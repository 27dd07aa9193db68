"""Strided views as the paged path's tensors: a query transposed from
[Hq, B, D] or sliced from wider rows, key and value pages that are the
leading columns of wider page rows, scales and zero-points that are a slice
of a larger group array, a page table with spare columns. The quantizer
writes into such views exactly what it writes into contiguous tensors, and
the decode over them gives the contiguous inputs' output bit for bit (the
kernels take every stride from the caller). Views whose rows break the
16-byte alignment of the kernels' loads and stores, and queries whose channels are not contiguous, are refused on the
host before anything is launched."""

import pytest

pytestmark = pytest.mark.gpu


def _inputs(D, hkv, rep, vdtype, seed):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, pr, group = 3, 16, 128
    lens = torch.tensor([300, 0, 129], dtype=torch.int32, device="cuda")
    maxp = 20
    P = B * maxp + 5
    table = torch.randperm(P, generator=g, device="cuda")[:B * maxp].to(torch.int32)
    table = table.view(B, maxp)
    T = int(lens.max())
    G = (maxp * pr + group - 1) // group
    k = torch.randn(B, hkv, T, D, device="cuda", generator=g)
    v = torch.randn(P, hkv, pr, D, device="cuda", generator=g).to(getattr(torch, vdtype))
    q = torch.randn(B, hkv * rep, D, device="cuda", generator=g)
    return dict(B=B, pr=pr, group=group, lens=lens, maxp=maxp, P=P, table=table, G=G, k=k,
                v=v, q=q, hkv=hkv, D=D)


def _contiguous_run(c, splits):
    import torch
    from flash_decode_int4 import ops
    kp = torch.zeros(c["P"], c["hkv"], c["pr"], c["D"] // 2, dtype=torch.uint8, device="cuda")
    s = torch.zeros(c["B"], c["hkv"], c["G"], c["D"], device="cuda")
    z = torch.zeros_like(s)
    ops.quantize_int4_paged(c["k"], c["lens"], c["table"], kp, s, z, c["group"])
    out = ops.flash_decode_paged(c["q"], kp, c["v"], s, z, c["table"], c["lens"], c["group"],
                                 splits)
    return kp, s, z, out


def _view_run(c, splits):
    """The same call with every tensor a strided view of a larger buffer."""
    import torch
    from flash_decode_int4 import ops
    B, hkv, D, P, pr, G = c["B"], c["hkv"], c["D"], c["P"], c["pr"], c["G"]
    # (the quantizer stores 16-byte pieces of packed rows: rows 16-byte aligned)
    kbig = torch.full((P, hkv, pr, D // 2 + 16), 0xAB, dtype=torch.uint8, device="cuda")
    kp = kbig[..., :D // 2]
    sbig = torch.full((B, hkv, G + 2, D), float("nan"), device="cuda")
    zbig = torch.full((B, hkv, G + 2, D), float("nan"), device="cuda")
    s, z = sbig[:, :, 1:G + 1], zbig[:, :, 1:G + 1]
    s.zero_()
    z.zero_()
    vbig = torch.full((P, hkv, pr, D + 8), float("nan"), dtype=c["v"].dtype, device="cuda")
    vbig[..., :D] = c["v"]
    v = vbig[..., :D]
    tbig = torch.full((B, c["maxp"] + 7), -5, dtype=torch.int32, device="cuda")
    tbig[:, :c["maxp"]] = c["table"]
    table = tbig[:, :c["maxp"]]
    kwide = torch.zeros(B, hkv, c["k"].shape[2], D + 4, device="cuda")
    kwide[..., :D] = c["k"]
    ops.quantize_int4_paged(kwide[..., :D], c["lens"], table, kp, s, z, c["group"])
    q_t = c["q"].transpose(0, 1).contiguous().transpose(0, 1)     # strides (D, B*D, 1)
    assert not q_t.is_contiguous()
    out_t = ops.flash_decode_paged(q_t, kp, v, s, z, table, c["lens"], c["group"], splits)
    qwide = torch.zeros(B, c["q"].shape[1], 2 * D, device="cuda")
    qwide[..., D:] = c["q"]
    out_w = ops.flash_decode_paged(qwide[..., D:], kp, v, s, z, table, c["lens"], c["group"],
                                   splits)
    return kbig, sbig, zbig, kp, s, z, out_t, out_w


@pytest.mark.parametrize("D,rep,vdtype,splits", [
    (128, 1, "float32", 0),
    (128, 4, "float16", 0),
    (64, 2, "bfloat16", 3),
    (256, 1, "float32", 2),
])
def test_views_match_contiguous_bitwise(D, rep, vdtype, splits):
    import torch
    c = _inputs(D, 2, rep, vdtype, 13 + D + rep)
    kp, s, z, out = _contiguous_run(c, splits)
    kbig, sbig, zbig, kpv, sv, zv, out_t, out_w = _view_run(c, splits)
    torch.cuda.synchronize()
    # The quantizer wrote the views' pages and groups only: same bytes, and
    # the padding columns and spare groups are untouched.
    full = c["table"][0, :18].long()        # sequence 0's 18 full pages (300 tokens)
    assert torch.equal(kpv[full], kp[full])
    assert torch.equal(sv, s) and torch.equal(zv, z)
    assert bool((kbig[..., D // 2:] == 0xAB).all())
    assert bool(torch.isnan(sbig[:, :, 0]).all()) and bool(torch.isnan(sbig[:, :, -1]).all())
    assert torch.equal(out_t, out) and torch.equal(out_w, out)
    assert bool(torch.isfinite(out).all())


def test_misaligned_views_are_refused():
    import torch
    from flash_decode_int4 import ops
    c = _inputs(128, 2, 1, "float32", 29)
    kp, s, z, out = _contiguous_run(c, 0)
    torch.cuda.synchronize()
    P, hkv, pr, D, B, G = c["P"], c["hkv"], c["pr"], c["D"], c["B"], c["G"]
    args = dict(page_table=c["table"], seq_lens=c["lens"], group_rows=c["group"])

    def call(q=c["q"], k_pages=kp, v_pages=c["v"], k_scale=s, k_zp=z):
        return ops.flash_decode_paged(q, k_pages, v_pages, k_scale, k_zp, **args)

    vbig = torch.zeros(P, hkv, pr, D + 8, device="cuda")
    with pytest.raises((RuntimeError, ValueError)):
        call(v_pages=vbig[..., 1:D + 1])                     # 4 bytes off 16
    kbig = torch.zeros(P, hkv, pr, D // 2 + 16, dtype=torch.uint8, device="cuda")
    with pytest.raises((RuntimeError, ValueError)):
        call(k_pages=kbig[..., 8:D // 2 + 8])                # 8 bytes off 16
    sbig = torch.zeros(B, hkv, G, D + 4, device="cuda")
    with pytest.raises((RuntimeError, ValueError)):
        call(k_scale=sbig[..., 1:D + 1], k_zp=sbig[..., 1:D + 1])
    qbig = torch.zeros(B, hkv, 2 * D, device="cuda")
    with pytest.raises((RuntimeError, ValueError)):
        call(q=qbig[..., ::2])                               # channel stride 2
    torch.cuda.synchronize()
    # The refused calls launched nothing that changed the cache.
    assert torch.equal(call(), out)
