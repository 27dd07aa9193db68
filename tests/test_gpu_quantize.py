"""GPU parity of the HIP quantizers against the oracle: bit-exact bins, packed
bytes, scales and zero-points (the bar this path is held to; the reference itself
held its CUDA/Triton quantizers only to "<= 1 bin on < 1%")."""

import numpy as np
import pytest

from oracle import pack_int4, quantize_groups_ref, quantize_int4_ref

pytestmark = pytest.mark.gpu


def _ops():
    from flash_decode_int4 import ops
    return ops


class TestRowsQuantizer:
    """The 2-D contract: one group over all rows (reference src/ops.py:111-161)."""

    # Shapes on both sides of each kernel choice: scalar kernels (C % 4 != 0),
    # the one-launch 16-byte kernel (rows <= 512, or <= 1024 for C <= 16;
    # every slice width and rows-per-thread instance, slice tails with
    # C % 32 != 0), the two-pass form (up to 64 tiles of 256 rows, or 128
    # for C <= 256: extremes, then finalize fused with the bins) and the
    # three-pass form (more rows; partial last tile, many tiles).
    @pytest.mark.parametrize("shape", [(1, 1), (1, 64), (255, 3), (256, 3), (257, 3),
                                       (1030, 8), (4096, 128), (512, 128), (32768, 128),
                                       (3, 1000), (5, 4), (64, 36), (65, 36), (129, 100),
                                       (300, 128), (777, 64), (2048, 128), (2049, 128),
                                       (2047, 4), (8191, 36), (70000, 100), (1024, 128),
                                       (1025, 128), (1024, 4), (8, 4096), (1000, 2048),
                                       (200, 512), (40, 256), (100, 1024), (16384, 64),
                                       (16385, 64), (512, 64), (513, 64), (1024, 16),
                                       (1025, 16), (300, 4096), (20000, 100), (32769, 128),
                                       (17000, 512)])
    def test_bit_exact(self, shape):
        kv = np.random.RandomState(shape[0]).randn(*shape).astype(np.float32)
        q, scale, zp = _ops().quantize_int4(kv, backend="hip")
        qr, sr, zr = quantize_int4_ref(kv)
        np.testing.assert_array_equal(q, qr)
        assert scale.tobytes() == sr.tobytes()
        np.testing.assert_array_equal(zp, zr)

    def test_ties_round_half_to_even(self):
        col = np.array([0.0, 15.0, 0.5, 1.5, 2.5, 3.5, 14.5, 7.5, 8.5], dtype=np.float32)
        q, s, z = _ops().quantize_int4(np.tile(col[:, None], (1, 5)), backend="hip")
        np.testing.assert_array_equal(q[:, 0], [0, 15, 0, 2, 2, 4, 14, 8, 8])

    def test_uniform_channel_floor(self):
        kv = np.full((64, 16), 5.0, dtype=np.float32)
        q, s, z = _ops().quantize_int4(kv, backend="cuda")
        qr, sr, zr = quantize_int4_ref(kv)
        np.testing.assert_array_equal(q, qr)
        np.testing.assert_array_equal(s, sr)

    def test_higher_rank_auto_backend(self):
        kv = np.random.RandomState(4).randn(4, 8, 64).astype(np.float32)
        q, s, z = _ops().quantize_int4(kv)
        qr, sr, zr = quantize_int4_ref(kv)
        np.testing.assert_array_equal(q, qr)
        np.testing.assert_array_equal(s, sr)

    def test_named_backend_rejects_3d(self):
        with pytest.raises(ValueError, match="2D"):
            _ops().quantize_int4(np.zeros((2, 3, 4), np.float32), backend="hip")

    def test_binding_rejects_bad_quantizer_input(self):
        """reference tests/test_ops_dispatch.py:321-328."""
        import torch
        C = _ops()._C
        with pytest.raises(RuntimeError, match="float32"):
            C.quantize_int4(torch.zeros(4, 4, dtype=torch.float64, device="cuda"))
        with pytest.raises(RuntimeError, match="non-empty"):
            C.quantize_int4(torch.zeros(0, 4, device="cuda"))
        with pytest.raises(RuntimeError, match="2D"):
            C.quantize_int4(torch.zeros(4, device="cuda"))

    @pytest.mark.parametrize("rows,cols,offset", [(300, 64, 0), (300, 64, 1), (3000, 128, 0),
                                                  (3000, 128, 1), (17, 8, 0)])
    def test_packed_rows_16_byte_path(self, rows, cols, offset):
        """C % 4 == 0: the 16-byte kernels, packed into a pool view whose rows
        are 2-byte aligned (offset 0: half-word stores) or not (byte stores)."""
        import torch
        kv = np.random.RandomState(rows + cols).randn(rows, cols).astype(np.float32)
        nb = cols // 2
        pool = torch.zeros(2, rows + 3, nb + 4, dtype=torch.uint8, device="cuda")
        view = pool[1, 1:rows + 1, offset:offset + nb]
        s = torch.zeros(cols, device="cuda")
        z = torch.zeros(cols, device="cuda")
        _ops()._C.quantize_rows_into(torch.from_numpy(kv).cuda(), view, s, z, True)
        qr, sr, zr = quantize_int4_ref(kv)
        got = pool.cpu().numpy()
        np.testing.assert_array_equal(got[1, 1:rows + 1, offset:offset + nb], pack_int4(qr))
        outside = got.copy()
        outside[1, 1:rows + 1, offset:offset + nb] = 0
        assert not outside.any()
        np.testing.assert_array_equal(s.cpu().numpy(), sr)
        np.testing.assert_array_equal(z.cpu().numpy(), zr)

    def test_unpacked_rows_unaligned_output(self):
        """Unpacked bins into a byte-offset view (4-byte stores not possible)."""
        import torch
        kv = np.random.RandomState(3).randn(500, 64).astype(np.float32)
        pool = torch.zeros(501, 70, dtype=torch.uint8, device="cuda")
        view = pool[1:, 3:67]
        s = torch.zeros(64, device="cuda")
        z = torch.zeros(64, device="cuda")
        _ops()._C.quantize_rows_into(torch.from_numpy(kv).cuda(), view, s, z, False)
        qr, _, _ = quantize_int4_ref(kv)
        got = pool.cpu().numpy()
        np.testing.assert_array_equal(got[1:, 3:67], qr)
        assert not got[0].any() and not got[:, :3].any() and not got[:, 67:].any()

    def test_packed_rows_into_strided_view(self):
        import torch
        kv = np.random.RandomState(8).randn(40, 33).astype(np.float32)
        pool = torch.zeros(3, 64, 24, dtype=torch.uint8, device="cuda")
        s = torch.zeros(33, device="cuda")
        z = torch.zeros(33, device="cuda")
        _ops()._C.quantize_rows_into(torch.from_numpy(kv).cuda(), pool[1, :40], s, z, True)
        qr, sr, zr = quantize_int4_ref(kv)
        got = pool.cpu().numpy()
        np.testing.assert_array_equal(got[1, :40, :17], pack_int4(qr))
        assert not got[0].any() and not got[2].any() and not got[1, 40:].any()
        assert not got[1, :, 17:].any()
        np.testing.assert_array_equal(s.cpu().numpy(), sr)


class TestDevicePack:

    @pytest.mark.parametrize("shape", [(10, 7), (256, 64), (3, 1), (1000, 128)])
    def test_matches_host_pack(self, shape):
        import torch
        q = np.random.RandomState(shape[1]).randint(0, 16, shape).astype(np.uint8)
        got = _ops().pack_int4_device(torch.from_numpy(q).cuda()).cpu().numpy()
        np.testing.assert_array_equal(got, pack_int4(q))


def _paged_keys(B, H, D, lens, seed, group=128):
    import torch
    from flash_decode_int4.workloads import page_layout
    rng = np.random.RandomState(seed)
    T = max(max(lens), 1)
    k = rng.randn(B, H, T, D).astype(np.float32)
    table, P = page_layout(lens, 16, seed)
    dev = torch.device("cuda")
    G = (T + group - 1) // group
    kp = torch.zeros(P, H, 16, D // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, H, G, D, device=dev)
    z = torch.zeros(B, H, G, D, device=dev)
    _ops().quantize_int4_paged(torch.from_numpy(k).to(dev),
                               torch.tensor(lens, dtype=torch.int32, device=dev),
                               torch.from_numpy(table).to(dev), kp, s, z, group)
    return k, table, kp.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy()


class TestPagedQuantizer:

    @pytest.mark.parametrize("B,H,D,lens,group", [
        (1, 4, 64, [512], 128),
        (3, 2, 128, [0, 37, 300], 128),
        (2, 3, 128, [2048, 1999], 128),
        (2, 2, 256, [129, 256], 128),
        (2, 2, 128, [100, 513], 64),
        (1, 2, 64, [700], 256),
    ])
    def test_bit_exact_pages_and_scales(self, B, H, D, lens, group):
        k, table, kp, s, z = _paged_keys(B, H, D, lens, seed=B * 100 + D, group=group)
        qr, sr, zr = quantize_groups_ref(k, np.array(lens), group_size=group)
        for b in range(B):
            ng = (lens[b] + group - 1) // group
            np.testing.assert_array_equal(s[b, :, :ng], sr[b, :, :ng])
            np.testing.assert_array_equal(z[b, :, :ng], zr[b, :, :ng])
            for lp in range((lens[b] + 15) // 16):
                n = min(16, lens[b] - lp * 16)
                want = pack_int4(qr[b, :, lp * 16:lp * 16 + n])
                np.testing.assert_array_equal(kp[table[b, lp], :, :n], want)

    def test_outlier_channels_bit_exact(self):
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=4, head_dim=128, tokens=300, rope=True, outliers=4,
                          seed=9)
        dev = torch.device("cuda")
        G = 3
        kp = torch.zeros(w["num_pages"], 4, 16, 64, dtype=torch.uint8, device=dev)
        s = torch.zeros(2, 4, G, 128, device=dev)
        z = torch.zeros(2, 4, G, 128, device=dev)
        _ops().quantize_int4_paged(torch.from_numpy(w["k"]).to(dev),
                                   torch.from_numpy(w["seq_lens"]).to(dev),
                                   torch.from_numpy(w["page_table"]).to(dev), kp, s, z, 128)
        qr, sr, zr = quantize_groups_ref(w["k"], w["seq_lens"])
        np.testing.assert_array_equal(s.cpu().numpy(), sr)
        kpn = kp.cpu().numpy()
        for b in range(2):
            for lp in range(19):
                n = min(16, 300 - lp * 16)
                np.testing.assert_array_equal(kpn[w["page_table"][b, lp], :, :n],
                                              pack_int4(qr[b, :, lp * 16:lp * 16 + n]))


def _tie_keys(B, H, T, D, seed):
    """Keys whose quotients (x - mn) / scale sit on or within a few ulps of
    half-integers, per 128-row group and channel: row 0 is the minimum, row 1
    the maximum, the other rows mn + (j + 1/2) * scale nudged by -3..3 ulps.
    A quarter of the channels have mn = 0 and span 15 * 2^e, so the scale is a
    power of two and the nudge-0 rows are exact ties (round half to even)."""
    rng = np.random.RandomState(seed)
    k = np.empty((B, H, T, D), np.float32)
    for b in range(B):
        for h in range(H):
            for g0 in range(0, T, 128):
                n = min(128, T - g0)
                for c in range(D):
                    if c % 4 == 0:
                        e = rng.randint(-20, 10)
                        mn = np.float32(0.0)
                        mx = np.float32(15.0 * 2.0 ** e)
                    else:
                        span = 10.0 ** rng.uniform(-6, 3)
                        mn = np.float32(rng.uniform(-2, 2) * span)
                        mx = np.float32(mn + np.float32(span))
                    s = np.float32(np.maximum(np.float32(mx - mn), np.float32(1e-8)) /
                                   np.float32(15.0))
                    col = np.empty(n, np.float32)
                    col[0], col[1 % n] = mn, mx
                    for r in range(2, n):
                        j = rng.randint(0, 15)
                        x = np.float32(np.float64(mn) + (j + 0.5) * np.float64(s))
                        d = rng.randint(-3, 4)
                        for _ in range(abs(d)):
                            x = np.nextafter(x, np.float32(np.inf if d > 0 else -np.inf))
                        col[r] = np.clip(x, mn, mx)
                    k[b, h, g0:g0 + n, c] = col
    return k


class TestQuantizerTies:
    """The grouped kernel divides through the reciprocal with an FMA correction;
    the bins must still equal IEEE division + round-half-even at and next to
    every tie (random data almost never lands there)."""

    def test_paged_bins_at_and_near_ties(self):
        import torch
        from flash_decode_int4.workloads import page_layout
        B, H, T, D = 2, 2, 300, 128
        k = _tie_keys(B, H, T, D, seed=5)
        lens = np.array([300, 173], np.int32)
        table, P = page_layout(lens, 16, 5)
        dev = torch.device("cuda")
        kp = torch.zeros(P, H, 16, D // 2, dtype=torch.uint8, device=dev)
        s = torch.zeros(B, H, 3, D, device=dev)
        z = torch.zeros(B, H, 3, D, device=dev)
        _ops().quantize_int4_paged(torch.from_numpy(k).to(dev), torch.from_numpy(lens).to(dev),
                                   torch.from_numpy(table).to(dev), kp, s, z, 128)
        qr, sr, zr = quantize_groups_ref(k, lens)
        # The construction does put values on exact ties.
        y = k[:, :, :128] - k[:, :, :1]
        assert np.any(np.float32(y / sr[:, :, :1]) % 1 == 0.5)
        kpn, sn = kp.cpu().numpy(), s.cpu().numpy()
        for b in range(B):
            ng = (lens[b] + 127) // 128
            np.testing.assert_array_equal(sn[b, :, :ng], sr[b, :, :ng])
            for lp in range((lens[b] + 15) // 16):
                n = min(16, lens[b] - lp * 16)
                np.testing.assert_array_equal(kpn[table[b, lp], :, :n],
                                              pack_int4(qr[b, :, lp * 16:lp * 16 + n]))


@pytest.mark.parametrize("seed", range(30))
def test_random_rows_contract(seed):
    """Seeded random 2-D inputs through quantize_rows_into: row counts 1 to
    ~40000 (every kernel form), channel counts 1 to 600, padded input row
    strides (which decide between the 16-byte and the scalar kernels), packed
    or unpacked bins into offset views of a larger pool; bins, scales and
    zero-points bit-exact with the oracle and nothing outside the view
    written."""
    import torch
    rng = np.random.RandomState(300 + seed)
    rows = int(np.exp(rng.uniform(0, np.log(40000))))
    C = int(rng.choice([int(rng.randint(1, 600)), 4 * int(rng.randint(1, 150))]))
    pad = int(rng.choice([0, 0, 1, 3, 4, 8]))
    packed = bool(rng.rand() < 0.5)
    off = int(rng.choice([0, 1, 2, 4]))
    kv = rng.randn(rows, C).astype(np.float32)
    if rng.rand() < 0.3:
        kv[:, rng.randint(C)] *= np.float32(20.0)          # an outlier channel
    src = torch.zeros(rows, C + pad, device="cuda")
    src[:, :C] = torch.from_numpy(kv).cuda()
    nb = (C + 1) // 2 if packed else C
    pool = torch.zeros(rows + 2, nb + off + 3, dtype=torch.uint8, device="cuda")
    view = pool[1:rows + 1, off:off + nb]
    s = torch.zeros(C, device="cuda")
    z = torch.zeros(C, device="cuda")
    _ops()._C.quantize_rows_into(src[:, :C], view, s, z, packed)
    qr, sr, zr = quantize_int4_ref(kv)
    got = pool.cpu().numpy()
    want = pack_int4(qr) if packed else qr
    np.testing.assert_array_equal(got[1:rows + 1, off:off + nb], want)
    outside = got.copy()
    outside[1:rows + 1, off:off + nb] = 0
    assert not outside.any()
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(z.cpu().numpy(), zr)
