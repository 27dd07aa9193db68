"""GPU parity of the fused INT4 decode against the oracle.

Tolerance: max |HIP - oracle| <= 1e-5 on identical seeded
inputs, where the oracle is the float32 page loop. The HIP kernel computes
logits in float64, so it sits closer to the float64 arbiter than the float32
oracle does; every test also checks the arbiter, and at sizes where the
oracle's own distance from the arbiter approaches 1e-5 the gate is stated as
max(1e-5, 1.25 * that distance) with both numbers in the message.
"""

import numpy as np
import pytest

from oracle import (f64_attention, float32_floor, online_softmax_ref, paged_decode_f64,
                    paged_decode_ref, pack_int4, quantize_groups_ref, quantize_int4_ref)

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _ops():
    from flash_decode_int4 import ops
    return ops


def _paged_problem(batch=2, heads=3, dim=32, n_blocks=3, rows=64, seed=0):
    """reference tests/test_ops_dispatch.py:159-169 (same construction)."""
    rng = np.random.RandomState(seed)
    query = (rng.randn(batch, heads, dim) / np.sqrt(dim)).astype(np.float32)
    k_q, k_s, k_z, vals = [], [], [], []
    for _ in range(n_blocks):
        k = rng.randn(rows, dim).astype(np.float32)
        v = rng.randn(rows, dim).astype(np.float32)
        q, s_, z = quantize_int4_ref(k)
        k_q.append(q); k_s.append(s_); k_z.append(z); vals.append(v)
    return query, k_q, k_s, k_z, vals


def make_case(batch=2, heads=4, dim=64, n_blocks=4, block_size=128, seed=0, lens=None):
    """reference tests/test_pallas_flash_decode.py:37-50 (same construction)."""
    rng = np.random.RandomState(seed)
    query = rng.randn(batch, heads, dim).astype(np.float32)
    k_q, k_s, k_z, vals = [], [], [], []
    for _ in range(n_blocks):
        k = rng.randn(block_size, dim).astype(np.float32)
        v = rng.randn(block_size, dim).astype(np.float32)
        q_, s_, z_ = quantize_int4_ref(k)
        k_q.append(q_); k_s.append(s_); k_z.append(z_); vals.append(v)
    if lens is None:
        lens = np.full(n_blocks, block_size, dtype=np.int32)
    return query, k_q, k_s, k_z, vals, np.asarray(lens, dtype=np.int32)


def ref_out(case):
    query, k_q, k_s, k_z, vals, lens = case
    return online_softmax_ref(query, list(zip(k_q, k_s, k_z)), vals, lens)[0]


class TestSharedStreamDropIn:
    """ops.flash_decode: every (b, h) query attends one page stream."""

    def test_valid_ragged_input_matches_reference(self):
        """reference tests/test_ops_dispatch.py:245-251."""
        query, k_q, k_s, k_z, vals = _paged_problem()
        lens = np.array([64, 0, 17], dtype=np.int32)
        got = _ops().flash_decode(query, k_q, k_s, k_z, vals, lens, backend="hip")
        ref = ref_out((query, k_q, k_s, k_z, vals, lens))
        assert np.isfinite(got).all()
        assert np.abs(got - ref).max() < TOL

    @pytest.mark.parametrize("lens", [[128, 73, 5, 128], [128, 0, 64, 128], [0, 64, 64, 64],
                                      [128, 128, 128, 128]])
    def test_ragged_and_empty_pages(self, lens):
        """reference tests/test_pallas_flash_decode.py:97-148."""
        case = make_case(batch=2, heads=4, dim=64, n_blocks=4, block_size=128, seed=3, lens=lens)
        got = _ops().flash_decode(*case, backend="cuda")
        assert not np.isnan(got).any()
        assert np.abs(got - ref_out(case)).max() < TOL
        assert np.abs(got - f64_attention(*case)).max() < TOL

    def test_all_pages_empty_is_exact_zero(self):
        case = make_case(batch=1, heads=2, dim=64, n_blocks=3, block_size=64, seed=5,
                         lens=[0, 0, 0])
        got = _ops().flash_decode(*case, backend="hip")
        np.testing.assert_array_equal(got, 0.0)

    def test_empty_cache_returns_exact_zeros(self):
        query, *_ = _paged_problem()
        out = _ops().flash_decode(query, [], [], [], [], backend="hip")
        np.testing.assert_array_equal(out, np.zeros_like(query))

    @pytest.mark.parametrize("dim", [1, 2, 31, 32, 33, 64, 127, 128, 129, 255, 256])
    def test_head_dim_boundaries(self, dim):
        """reference tests/test_ops_dispatch.py:263-270 (gate tightened 1e-4 -> 1e-5)."""
        query, k_q, k_s, k_z, vals = _paged_problem(dim=dim, rows=96, seed=dim)
        lens = np.array([96, 40, 96], dtype=np.int32)
        got = _ops().flash_decode(query, k_q, k_s, k_z, vals, lens, backend="hip")
        ref = ref_out((query, k_q, k_s, k_z, vals, lens))
        assert np.isfinite(got).all()
        assert np.abs(got - ref).max() < TOL, f"head_dim {dim}"

    @pytest.mark.parametrize("rows", [1, 3, 4, 5, 15, 16, 17, 127, 128, 129])
    def test_page_sizes(self, rows):
        """reference tests/test_ops_dispatch.py:284-291 (16-row chunks instead of 4 warps)."""
        query, k_q, k_s, k_z, vals = _paged_problem(dim=64, rows=rows, seed=rows)
        got = _ops().flash_decode(query, k_q, k_s, k_z, vals, backend="hip")
        ref = ref_out((query, k_q, k_s, k_z, vals, np.full(3, rows)))
        assert np.abs(got - ref).max() < TOL, f"rows {rows}"

    @pytest.mark.parametrize("dim", [64, 128])
    def test_within_float32_noise_floor(self, dim):
        """reference tests/test_pallas_flash_decode.py:181-201."""
        case = make_case(batch=1, heads=4, dim=dim, n_blocks=4, block_size=256, seed=2)
        truth = f64_attention(*case)
        err = np.abs(_ops().flash_decode(*case, backend="hip") - truth).mean()
        assert err <= 3.0 * float32_floor(truth, dim)

    def test_page_decomposition_invariance(self):
        rng = np.random.RandomState(11)
        dim, total = 64, 512
        query = rng.randn(1, 2, dim).astype(np.float32)
        keys = rng.randn(total, dim).astype(np.float32)
        vals = rng.randn(total, dim).astype(np.float32)
        q_, s_, z_ = quantize_int4_ref(keys)
        outs = []
        for n_blocks in (1, 2, 4, 8):
            bs = total // n_blocks
            outs.append(_ops().flash_decode(
                query, [q_[i * bs:(i + 1) * bs] for i in range(n_blocks)], [s_] * n_blocks,
                [z_] * n_blocks, [vals[i * bs:(i + 1) * bs] for i in range(n_blocks)],
                backend="hip"))
        for o in outs[1:]:
            assert np.abs(o - outs[0]).max() < 1e-6

    def test_block_lens_accepts_a_plain_list(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        a = _ops().flash_decode(query, k_q, k_s, k_z, vals, [64, 10, 0], backend="hip")
        b = _ops().flash_decode(query, k_q, k_s, k_z, vals, np.array([64, 10, 0]),
                                backend="hip")
        np.testing.assert_array_equal(a, b)

    def test_deterministic(self):
        case = make_case(batch=2, heads=8, dim=128, n_blocks=8, block_size=256, seed=1)
        a = _ops().flash_decode(*case, backend="hip")
        b = _ops().flash_decode(*case, backend="hip")
        assert a.tobytes() == b.tobytes()

    def test_wide_head_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem(dim=320, rows=32)
        with pytest.raises(ValueError, match="head_dim"):
            _ops().flash_decode(query, k_q, k_s, k_z, vals, backend="hip")

    def test_binding_rejects_mismatched_shapes(self):
        """reference tests/test_ops_dispatch.py:293-319."""
        import torch
        C = _ops()._C
        q = torch.zeros(1, 1, 64, device="cuda")
        k = torch.zeros(2, 16, 64, dtype=torch.uint8, device="cuda")
        v = torch.zeros(2, 16, 64, device="cuda")
        sc = torch.ones(2, 64, device="cuda")
        zp = torch.zeros(2, 64, device="cuda")
        lens = torch.full((2,), 16, dtype=torch.int32, device="cuda")
        out = C.flash_decode_int4(q, k, sc, zp, v, lens)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        with pytest.raises(RuntimeError, match="k_scale"):
            C.flash_decode_int4(q, k, sc[:1], zp, v, lens)
        with pytest.raises(RuntimeError, match="value"):
            C.flash_decode_int4(q, k, sc, zp, v[:, :8], lens)
        with pytest.raises(RuntimeError, match="block_lens"):
            C.flash_decode_int4(q, k, sc, zp, v, lens[:1])
        with pytest.raises(RuntimeError, match="int32"):
            C.flash_decode_int4(q, k, sc, zp, v, lens.long())
        with pytest.raises(RuntimeError, match="head_dim"):
            wide = torch.zeros(1, 1, 320, device="cuda")
            C.flash_decode_int4(
                wide, torch.zeros(1, 4, 320, dtype=torch.uint8, device="cuda"),
                torch.ones(1, 320, device="cuda"), torch.zeros(1, 320, device="cuda"),
                torch.zeros(1, 4, 320, device="cuda"),
                torch.full((1,), 4, dtype=torch.int32, device="cuda"))

    @pytest.mark.parametrize("dim,bs,lens", [(64, 16, [16, 3]), (33, 40, [40, 0, 17]),
                                             (128, 96, [96, 40, 96]), (256, 20, [1, 20])])
    def test_binding_unpacked_keys_match_reference(self, dim, bs, lens):
        """_C.flash_decode_int4 with the reference's unpacked [nb, bs, D] keys
        (packed on the device by fdi4_flash_decode_int4_ws)."""
        import torch
        query, k_q, k_s, k_z, vals = _paged_problem(batch=2, heads=3, dim=dim,
                                                    n_blocks=len(lens), rows=bs, seed=dim + bs)
        lens = np.array(lens, np.int32)
        dev = torch.device("cuda")
        out = _ops()._C.flash_decode_int4(
            torch.from_numpy(query).to(dev), torch.from_numpy(np.stack(k_q)).to(dev),
            torch.from_numpy(np.stack(k_s)).to(dev), torch.from_numpy(np.stack(k_z)).to(dev),
            torch.from_numpy(np.stack(vals)).to(dev), torch.from_numpy(lens).to(dev))
        ref = ref_out((query, k_q, k_s, k_z, vals, lens))
        assert np.abs(out.cpu().numpy() - ref).max() < TOL


def _paged_device(w, value_dtype=None):
    """Quantize a workload's keys on the device; return device tensors."""
    import torch
    dev = torch.device("cuda")
    B, H, D = w["batch"], w["heads"], w["head_dim"]
    G = (w["max_tokens"] + 127) // 128
    kp = torch.zeros(w["num_pages"], H, 16, D // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, H, G, D, device=dev)
    z = torch.zeros(B, H, G, D, device=dev)
    k_t = w["k"] if isinstance(w["k"], torch.Tensor) else torch.from_numpy(w["k"]).to(dev)
    sl = torch.as_tensor(w["seq_lens"], device=dev)
    pt = torch.as_tensor(w["page_table"], device=dev)
    _ops().quantize_int4_paged(k_t, sl, pt, kp, s, z, 128)
    v = w["v_pages"]
    v_t = v if isinstance(v, torch.Tensor) else torch.from_numpy(v).to(dev)
    if value_dtype is not None:
        v_t = v_t.to(value_dtype)
    q_t = w["q"] if isinstance(w["q"], torch.Tensor) else torch.from_numpy(w["q"]).to(dev)
    return q_t, kp, v_t, s, z, pt, sl


def _oracle_inputs(w, kp, s, z, v=None):
    return (w["q"], kp.cpu().numpy(), w["v_pages"] if v is None else v, s.cpu().numpy(),
            z.cpu().numpy(), w["page_table"], w["seq_lens"])


class TestPagedDecode:

    @pytest.mark.parametrize("name_or_spec", [
        "cpu",
        dict(batch=3, heads=2, head_dim=128, seq_lens=[0, 37, 300]),
        dict(batch=2, heads=4, head_dim=256, seq_lens=[129, 1000]),
        dict(batch=4, heads=2, head_dim=64, seq_lens=[1, 16, 17, 2049]),
        dict(batch=2, heads=8, head_dim=128, seq_lens=[2048, 2048]),
    ])
    def test_matches_oracle(self, name_or_spec):
        from flash_decode_int4.workloads import make_workload
        w = (make_workload(name_or_spec) if isinstance(name_or_spec, str)
             else make_workload(seed=31, **name_or_spec))
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        out = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl).cpu().numpy()
        args = _oracle_inputs(w, kp, s, z)
        o32 = paged_decode_ref(*args)
        o64 = paged_decode_f64(*args)
        e32, e64, eo = (np.abs(out - o32).max(), np.abs(out - o64).max(),
                        np.abs(o32 - o64).max())
        assert e32 <= max(TOL, 1.25 * eo), (e32, e64, eo)
        assert e64 <= eo + 1e-6, (e32, e64, eo)
        empty = np.asarray(w["seq_lens"]) == 0
        assert np.all(out[empty] == 0.0)

    @pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64])
    def test_split_count_invariance(self, splits):
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=4, head_dim=128, seq_lens=[2048, 700], seed=4)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        base = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl, num_splits=1)
        got = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl, num_splits=splits)
        assert (got - base).abs().max().item() < 2e-6

    def test_grouped_query_heads(self):
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=2, head_dim=128, seq_lens=[300, 129], seed=12)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        q4 = torch.randn(2, 8, 128, device="cuda", generator=torch.Generator("cuda").manual_seed(1))
        out = _ops().flash_decode_paged(q4, kp, v_t, s, z, pt, sl).cpu().numpy()
        args = list(_oracle_inputs(w, kp, s, z))
        args[0] = q4.cpu().numpy()
        o64 = paged_decode_f64(*args)
        o32 = paged_decode_ref(*args)
        assert np.abs(out - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())

    def test_fp16_values(self):
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=4, head_dim=128, seq_lens=[500, 1024], seed=13)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w, value_dtype=torch.float16)
        out = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl).cpu().numpy()
        v16 = v_t.float().cpu().numpy()  # the oracle gets the identical upcast values
        args = _oracle_inputs(w, kp, s, z, v=v16)
        o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
        assert np.abs(out - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())

    @pytest.mark.parametrize("D", [64, 128, 256])
    def test_bf16_values(self, D):
        """bfloat16 value pages: the oracle gets the identical widened values."""
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=3, heads=2, head_dim=D, seq_lens=[500, 0, 1031], seed=D + 1)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w, value_dtype=torch.bfloat16)
        out = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl).cpu().numpy()
        args = _oracle_inputs(w, kp, s, z, v=v_t.float().cpu().numpy())
        o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
        assert np.abs(out - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())
        assert np.all(out[1] == 0.0)

    @pytest.mark.parametrize("qdtype", ["float16", "bfloat16"])
    @pytest.mark.parametrize("vdtype,rep,splits", [("float32", 1, 1), ("float16", 1, 3),
                                                   ("bfloat16", 4, 1), ("float16", 4, 2),
                                                   ("bfloat16", 1, 5)])
    def test_16_bit_queries_and_outputs(self, qdtype, vdtype, rep, splits):
        """A float16 / bfloat16 query gives an output of its own type equal, bit
        for bit, to the float32 decode of the widened query rounded to that type
        (one rounding, to nearest even, in the final store or in the merge),
        for the per-head and the grouped kernels, with and without splits; and
        the float32 result is within the oracle's tolerance."""
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=3, heads=2, head_dim=128, seq_lens=[700, 0, 1500], seed=rep + 40)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w, value_dtype=getattr(torch, vdtype))
        dt = getattr(torch, qdtype)
        g = torch.Generator("cuda").manual_seed(rep + splits)
        q16 = torch.randn(3, 2 * rep, 128, device="cuda", generator=g).to(dt)
        out16 = _ops().flash_decode_paged(q16, kp, v_t, s, z, pt, sl, num_splits=splits)
        assert out16.dtype == dt
        out32 = _ops().flash_decode_paged(q16.float(), kp, v_t, s, z, pt, sl, num_splits=splits)
        assert torch.equal(out16, out32.to(dt))
        assert bool((out16[1] == 0).all())
        args = list(_oracle_inputs(w, kp, s, z, v=v_t.float().cpu().numpy()))
        args[0] = q16.float().cpu().numpy()
        o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
        got = out32.cpu().numpy()
        assert np.abs(got - o32).max() <= max(TOL, 1.25 * np.abs(o32 - o64).max())

    @pytest.mark.parametrize("qdtype", ["float16", "bfloat16"])
    def test_16_bit_output_rounding_at_the_range_ends(self, qdtype):
        """One live token: the output is that token's value row exactly, so
        the 16-bit output must be torch's rounding of the row itself, here
        values that overflow the 16-bit type, sit at its largest finite value,
        fall in its subnormal range or below it."""
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=1, heads=1, head_dim=64, seq_lens=[1], seed=3)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        row = torch.tensor([3.4e38, -3.4e38, 3.3895e38, 65504.0, 65520.0, -65520.0, 1e-40,
                            -1e-40, 6e-8, 3e-8, 1.0 + 2.0 ** -9, 1.0 + 2.0 ** -8, 0.0, 1.5],
                           device="cuda")
        v_t[pt[0, 0], 0, 0, :] = 0.0
        v_t[pt[0, 0], 0, 0, :row.numel()] = row
        dt = getattr(torch, qdtype)
        out = _ops().flash_decode_paged(q_t.to(dt), kp, v_t, s, z, pt, sl)
        want = v_t[pt[0, 0], 0, 0, :].to(dt)
        assert torch.equal(out[0, 0].view(torch.int16), want.view(torch.int16))

    def test_deterministic_bitwise(self):
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=4, head_dim=128, seq_lens=[2048, 999], seed=14)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        a = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl)
        b = _ops().flash_decode_paged(q_t, kp, v_t, s, z, pt, sl)
        assert bool((a == b).all())


class TestGroupedQueryHeads:
    """Several q-heads per kv-head: the grouped kernel serves 2, 4 or 8 heads
    per workgroup (one read of the kv-head's pages for all of them); head
    counts that no group size divides run the per-head kernel. Every case is
    held to the oracle, whose q-head h reads kv-head h // (Hq / Hkv)."""

    @pytest.mark.parametrize("D,rep,vdtype,lens,splits", [
        (128, 4, "float32", [0, 37, 300, 2048], 0),
        (128, 4, "float32", [700, 129], 3),
        (128, 2, "float16", [1, 513, 1000], 0),
        (64, 8, "float32", [16, 900], 0),
        (64, 4, "float16", [257, 0, 60], 2),
        (256, 4, "float32", [333, 1024], 0),
        (256, 2, "float16", [129, 700], 0),
        (128, 6, "float32", [400, 77], 0),   # groups of 2
        (128, 3, "float32", [400, 77], 0),   # per-head kernel
        (128, 8, "float32", [1200, 5], 0),   # eight heads per workgroup at D=128
        (128, 8, "float16", [1200, 5, 0], 0),
        (128, 16, "float16", [300, 2000], 0),  # two workgroups of 8 per kv-head
        (64, 8, "float16", [700, 33], 3),
        (128, 4, "bfloat16", [900, 17], 0),
        (64, 8, "bfloat16", [300, 1100], 2),
        (256, 4, "bfloat16", [129, 700], 0),
    ])
    def test_matches_oracle(self, D, rep, vdtype, lens, splits):
        import torch
        from flash_decode_int4.workloads import make_workload
        hkv = 2
        w = make_workload(batch=len(lens), heads=hkv, head_dim=D, seq_lens=lens, seed=D + rep)
        vt = None if vdtype == "float32" else getattr(torch, vdtype)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w, value_dtype=vt)
        g = torch.Generator("cuda").manual_seed(rep)
        q = torch.randn(len(lens), hkv * rep, D, device="cuda", generator=g)
        out = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=splits)
        out = out.cpu().numpy()
        args = list(_oracle_inputs(w, kp, s, z, v=v_t.float().cpu().numpy()))
        args[0] = q.cpu().numpy()
        o32, o64 = paged_decode_ref(*args), paged_decode_f64(*args)
        e32, eo = np.abs(out - o32).max(), np.abs(o32 - o64).max()
        assert e32 <= max(TOL, 1.25 * eo), (e32, eo)
        assert np.abs(out - o64).max() <= eo + 1e-6
        empty = np.asarray(lens) == 0
        assert np.all(out[empty] == 0.0)

    @pytest.mark.parametrize("D,rep,vdtype", [(128, 4, None), (64, 8, None), (128, 2, None),
                                              (128, 8, None), (128, 8, "float16"),
                                              (64, 4, "float16"), (128, 4, "bfloat16")])
    def test_matrix_core_equals_vector_kernel(self, D, rep, vdtype):
        """The int8 matrix-core kernel's logits are exact up to the 41-bit
        rounding of q*s; it agrees with the vector grouped kernel (fp64
        products) to float32 rounding."""
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=2, head_dim=D, seq_lens=[1500, 333], seed=D + rep)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(
            w, value_dtype=getattr(torch, vdtype) if vdtype else None)
        q = torch.randn(2, 2 * rep, D, device="cuda", generator=torch.Generator("cuda").manual_seed(7))
        from flash_decode_int4 import capi
        mfma = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=2)
        with capi.tuning(decode_vector_only=1):
            vec = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=2)
        assert (mfma - vec).abs().max().item() < 2e-6

    def test_grouped_equals_per_head_kernel(self):
        """The grouped and the per-head kernel compute the same logits up to
        fp64 rounding (other channel partitions per lane); the outputs agree to
        float32 rounding."""
        import torch
        from flash_decode_int4.workloads import make_workload
        w = make_workload(batch=2, heads=4, head_dim=128, seq_lens=[2048, 999], seed=21)
        q_t, kp, v_t, s, z, pt, sl = _paged_device(w)
        q = torch.randn(2, 16, 128, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
        from flash_decode_int4 import capi
        grouped = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=1)
        with capi.tuning(decode_heads_per_wg=1):
            per_head = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=1)
            again = _ops().flash_decode_paged(q, kp, v_t, s, z, pt, sl, num_splits=1)
        assert (grouped - per_head).abs().max().item() < 2e-6
        assert torch.equal(per_head, again)
