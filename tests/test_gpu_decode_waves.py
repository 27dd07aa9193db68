"""The per-head decode kernel at either wave count: the library picks four
waves per workgroup (one per SIMD) for float32 values at head_dim 128 on up
to 512 (sequence, head) streams and eight elsewhere, and the launch-shape
override forces either. Every case runs with both forced counts and the
automatic one, with one split and with several, over ragged lengths (empty
sequences, partial chunks, fewer chunks than waves), against the oracle, and
twice (bit-identical). The fused serving step takes the decode's wave count
(with four, plus four helper waves that re-quantize the open group): the
one-launch step against the append and the decode, bit for bit, at both
counts.
"""

import numpy as np
import pytest

from oracle import paged_decode_f64, paged_decode_ref

pytestmark = pytest.mark.gpu

TOL = 1e-5

CASES = [
    # (batch, heads, head_dim, seq_lens, value dtype)
    (6, 4, 128, [2048, 700, 0, 1, 17, 129], "float32"),
    (3, 8, 128, [5000, 31, 256], "float16"),
    (4, 2, 64, [1024, 3, 16, 2500], "float32"),
    (2, 4, 256, [1500, 47], "float32"),
    (3, 2, 256, [900, 0, 4096], "bfloat16"),
    (1, 32, 128, [8192], "float32"),
]


def _problem(batch, heads, head_dim, seq_lens, value_dtype, seed):
    import torch
    from flash_decode_int4 import ops
    from flash_decode_int4.workloads import make_workload
    w = make_workload(batch=batch, heads=heads, head_dim=head_dim, seq_lens=seq_lens, seed=seed)
    dev = torch.device("cuda")
    G = (w["max_tokens"] + 127) // 128
    kp = torch.zeros(w["num_pages"], heads, 16, head_dim // 2, dtype=torch.uint8, device=dev)
    s = torch.zeros(batch, heads, G, head_dim, device=dev)
    z = torch.zeros_like(s)
    k = torch.as_tensor(w["k"], device=dev)
    sl = torch.as_tensor(w["seq_lens"], device=dev)
    pt = torch.as_tensor(w["page_table"], device=dev)
    ops.quantize_int4_paged(k, sl, pt, kp, s, z, 128)
    v = torch.as_tensor(w["v_pages"], device=dev).to(getattr(torch, value_dtype))
    q = torch.as_tensor(w["q"], device=dev)
    return w, (q, kp, v, s, z, pt, sl)


@pytest.mark.parametrize("batch,heads,d,lens,vdt", CASES)
def test_either_wave_count_matches_the_oracle(batch, heads, d, lens, vdt):
    import torch
    from flash_decode_int4 import capi, ops
    w, args = _problem(batch, heads, d, lens, vdt, seed=d + len(lens))
    q, kp, v, s, z, pt, sl = args
    oargs = (q.cpu().numpy(), kp.cpu().numpy(), v.float().cpu().numpy(), s.cpu().numpy(),
             z.cpu().numpy(), w["page_table"], w["seq_lens"])
    o32, o64 = paged_decode_ref(*oargs), paged_decode_f64(*oargs)
    bound = max(TOL, 1.25 * np.abs(o32 - o64).max())
    for splits in (1, 3, 0):
        for waves in (4, 8, 0):
            with capi.tuning(decode_waves=waves):
                one = ops.flash_decode_paged(*args, num_splits=splits)
                two = ops.flash_decode_paged(*args, num_splits=splits)
            assert torch.equal(one, two), f"splits={splits} waves={waves}"
            got = one.cpu().numpy()
            assert np.isfinite(got).all()
            err = np.abs(got - o32).max()
            assert err <= bound, f"splits={splits} waves={waves}: {err} > {bound}"


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("vdt,d", [("float32", 128), ("float16", 128), ("float32", 64),
                                   ("bfloat16", 256)])
def test_fused_step_equals_append_and_decode_at_either_wave_count(waves, vdt, d):
    """B4 H8 from 600 tokens, one split (so the step is one launch), 12 steps
    across a scale-group boundary: the one-launch step against the append,
    the length increment and the decode of a twin cache. The step's
    workgroup: four decode waves plus four helpers; eight decode waves plus
    four helpers (16-bit values at D = 128, float32 at D = 64; the first
    helper counts the arrival with 16-bit values); eight decode waves whose
    younger four re-quantize (float32 at D = 128, D = 256)."""
    import torch
    from flash_decode_int4 import capi
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    B, H, D, T0 = 4, 8, d, 600
    g = torch.Generator(device="cuda")
    g.manual_seed(waves)
    k = torch.randn(B, H, T0, D, device="cuda", generator=g)
    v = torch.randn(B, H, T0, D, device="cuda", generator=g)
    caches = []
    for _ in range(2):
        c = INT4PagedSequenceCache(num_pages=B * (T0 // 16 + 4), num_kv_heads=H, head_dim=D,
                                   max_seqs=B, max_seq_len=T0 + 40, group_rows=128,
                                   value_dtype=vdt)
        c.prefill(k, v, [T0] * B)
        c.reserve(B, 12)
        caches.append(c)
    new, old = caches
    with capi.tuning(decode_waves=waves, decode_target_waves=1):
        for i in range(12):
            kn = torch.randn(B, H, D, device="cuda", generator=g)
            vn = torch.randn(B, H, D, device="cuda", generator=g).to(getattr(torch, vdt))
            q = torch.randn(B, H, D, device="cuda", generator=g)
            out_new = new.step(kn, vn, q)
            old.append(kn, vn)
            out_old = old.decode(q)
            torch.cuda.synchronize()
            assert torch.equal(out_new, out_old), f"step {i}"
            for name in ("k_pages", "v_pages", "k_scale", "k_zp", "seq_lens", "k_stage"):
                assert torch.equal(getattr(new, name), getattr(old, name)), (i, name)
    new.sync_lengths()
    assert list(new.lengths()[:B]) == list(old.lengths()[:B]) == [T0 + 12] * B
