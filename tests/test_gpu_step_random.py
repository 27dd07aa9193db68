"""Seeded random configurations of the one-launch serving step (one decode
workgroup per (sequence, kv-head): fdi4_decode_step fuses the append, the
re-quantization of the open scale group, the decode and the length advance)
against the three-launch form (append kernel, a length increment, decode):
head dims 64/128/256, pages of 2..64 rows, scale groups of 64/128/256
tokens, 1-3 kv-heads, 1-4 sequences with lengths on and next to page and
group edges (and 0), float32/float16/bfloat16 values, 4- and 8-wave
workgroups, 2-5 consecutive steps. Per step: the outputs, packed pages,
scales, zero-points, values, staging rows and lengths are equal bit for
bit, and the step's arrival counters are back at zero. Then the same for
shapes that take the two-launch form (several q-heads per kv-head, the
library's own split count)."""

import numpy as np
import pytest

from test_gpu_step_fused import _old_step, _same, _twins

pytestmark = pytest.mark.gpu

N_CASES = 40


def _case(seed):
    rng = np.random.RandomState(7000 + seed)
    D = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 3]))
    B = int(rng.randint(1, 5))
    page_rows = int(rng.choice([2, 4, 8, 16, 32, 64]))
    group = int(rng.choice([g for g in (64, 128, 256) if g % page_rows == 0]))
    edges = [0, 1, page_rows - 1, page_rows, page_rows + 1, group - 2, group - 1, group,
             group + 1, 2 * group - 1, int(rng.randint(1, 600))]
    lens = [int(rng.choice(edges)) if rng.rand() < 0.7 else int(rng.randint(0, 600))
            for _ in range(B)]
    return dict(D=D, H=H, B=B, page_rows=page_rows, group=group, lens=lens,
                vdtype=str(rng.choice(["float32", "float16", "bfloat16"])),
                waves=int(rng.choice([4, 8])), steps=int(rng.randint(2, 6)))


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_fused_step_case(seed):
    import torch
    from flash_decode_int4 import capi
    c = _case(seed)
    print("case", seed, c, flush=True)
    B, H, D = c["B"], c["H"], c["D"]
    max_seq_len = max(max(c["lens"]) + c["steps"] + 1, 64)
    (new, old), g = _twins(B, H, D, c["lens"], c["page_rows"], c["group"], c["vdtype"],
                           max_seq_len, 100 + seed)
    vdt = getattr(torch, c["vdtype"])
    for cache in (new, old):
        cache.reserve(B, c["steps"])
    with capi.tuning(decode_target_waves=1, decode_waves=c["waves"]):
        for i in range(c["steps"]):
            kn = torch.randn(B, H, D, device="cuda", generator=g)
            vn = torch.randn(B, H, D, device="cuda", generator=g).to(vdt)
            q = torch.randn(B, H, D, device="cuda", generator=g)
            out_new = new.step(kn, vn, q)
            out_old = _old_step(old, kn, vn, q)
            torch.cuda.synchronize()
            assert torch.equal(out_new, out_old), (seed, i)
            _same(new, old, (seed, i))
    assert int(new._step_counters.abs().sum()) == 0
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + c["steps"] for n in c["lens"]]


@pytest.mark.parametrize("seed", range(20))
def test_random_step_any_plan(seed):
    """The same comparison for shapes that take the two-launch form (the
    append writes the advanced lengths, the decode attends over them and
    hands them back): 2, 4 or 8 q-heads per kv-head (grouped and matrix-core
    kernels) or the library's automatic split count."""
    import torch
    c = _case(500 + seed)
    rng = np.random.RandomState(9000 + seed)
    rep = int(rng.choice([1, 2, 4, 8]))
    print("case", seed, c, "q-heads per kv-head", rep, flush=True)
    B, H, D = c["B"], c["H"], c["D"]
    max_seq_len = max(max(c["lens"]) + c["steps"] + 1, 64)
    (new, old), g = _twins(B, H, D, c["lens"], c["page_rows"], c["group"], c["vdtype"],
                           max_seq_len, 300 + seed)
    vdt = getattr(torch, c["vdtype"])
    for cache in (new, old):
        cache.reserve(B, c["steps"])
    for i in range(c["steps"]):
        kn = torch.randn(B, H, D, device="cuda", generator=g)
        vn = torch.randn(B, H, D, device="cuda", generator=g).to(vdt)
        q = torch.randn(B, H * rep, D, device="cuda", generator=g)
        out_new = new.step(kn, vn, q)
        out_old = _old_step(old, kn, vn, q)
        torch.cuda.synchronize()
        assert torch.equal(out_new, out_old), (seed, i)
        _same(new, old, (seed, i))
    new.sync_lengths()
    assert list(new.lengths()[:B]) == [n + c["steps"] for n in c["lens"]]
