#!/usr/bin/env python3
"""Benchmark of the INT4 paged decode path on one MI355X.

Metric: fused INT4 decode attention time (us) and its fraction of the HBM
roofline at B8 x H32 x D128 x 2048 tokens (16-token pages, 128-token scale
groups, fp32 values), plus the grouped quantizer's GB/s.

A step is one decode of the whole batch on inputs already resident in HBM:
the decode kernel (plus the split merge when the library splits the
sequences). Input sets are rotated so their total exceeds twice the 256 MB
Infinity Cache (nothing is served from the cache across steps). Bytes are
algorithmic (valid tokens only): packed K T*D/2, V T*D*4, scale and
zero-point ceil(T/128)*D*8 per (sequence, head), the page table, sequence
lengths, q and the output.

Clocks. `value` and `ms_per_step` come from the wall clock around exactly K
(--steps) back-to-back steps, synchronized on both sides (the step contract;
host launch cost included). `decode_us` and the roofline figure come from
HIP events on the launch stream around a steady-state window of at least 400
back-to-back launches (20 blocks, an event between blocks, no host
synchronization inside the window, whatever --steps is), which follows ~30
ms of untimed launches (a GPU that has been idle runs its first ~15 ms of
launches 1-7 % slower); `decode_us_median` is the median over the window's
blocks. `roofline.trace_*` are the decode
kernel's per-dispatch durations over the same window, from a rocprofv3
--kernel-trace child process (`--no-trace` skips it). The quantizers and the
other decode paths are timed over windows of the same shape.

hbm_probe reports what a plain torch elementwise kernel reading and writing
1 GiB reaches on the same box, beside the 8 TB/s specification used as the
roofline peak.

reference_config times the drop-in API (prepare_flash_decode_hip().run()) on
the reference's own benchmark semantics, beside the reference's published
CUDA time for it on other hardware (context, not vs_baseline).

reference_quantizer times the drop-in quantize_int4 (one scale group over all
rows of a [rows, 128] array, unpacked bins) at the two row counts the
reference publishes CUDA times for, beside those times; the CPU leg checks its
bins, scales and zero-points bit for bit against the oracle, and the PMC
children give the HBM traffic of its kernels.

other_paths times the decode with fp16 value pages at the anchor shape and with
grouped-query heads (B8, 8 kv-heads, 32 q-heads, 8192 tokens), and the serving
loop's step (append + decode + length advance, one launch at these shapes) on
the sequence cache, issued eagerly and replayed from HIP graphs of one and of
eight steps, interleaved so that the three forms see the same lengths.

fake_quant times the quality-study kernel (INT4 quantize-dequantize of a key
tensor in blocks) on a Llama-2-7B-sized perplexity window and on the decode
workload's keys, beside the same computation as eager torch operations.

append_us times the decode-time append kernel (one token per (sequence,
kv-head), open scale group re-quantized) on a cache of the workload's shape,
at the first and at the last row of a group.

The cpu_baseline leg times the NumPy oracle (the reference's page loop, one
call per (sequence, head) stream, one BLAS thread) on this host's cores over
the same workload and uses its output as the parity check of the GPU result.

The HBM traffic of the decode kernel (and of the grouped quantizer and the
fake-quantization kernel) comes from two rocprofv3 --pmc child runs (FETCH_SIZE, then WRITE_SIZE), each
calibrated by the same counter on a kernel that moves 256 MiB in that
direction only (a sum for reads, a fill for writes); --no-pmc skips them (and
must be given when this script itself runs under rocprofv3).

checks.seq_len_plus_1 re-runs the decode with every length + 1 (pages and
groups one row into fresh ones); its "interleaved" record times the workload
and the + 1 lengths in alternating blocks of back-to-back launches (no host
synchronization between blocks), so the two figures share clocks and memory
state.

Prints ONE JSON line on stdout (progress lines go to stderr). Options:
--workload (anchor, sweep_512 ... llama, ragged), --tokens (every sequence at
that length), --splits, --value-dtype float16|bfloat16, --no-cpu, --no-pmc,
--no-trace (both required when this script itself runs under rocprofv3),
--decode-only (the workload's decode and quantizer timings alone).
"""

import argparse
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(ROOT, "int4-kv-cache-quantization-cuda-triton-pallas_amd")
if PKG_ROOT not in sys.path:
    sys.path.insert(0, PKG_ROOT)

METRIC = ("fused INT4 decode attn µs + % HBM peak @B8×H32×D128×2048; "
          "quantizer GB/s")
HBM_PEAK_GBS = 8000.0
#: Decode kernel families (the planner picks one per shape).
DECODE_KERNELS = ("decode_kernel", "decode_gqa_kernel", "decode_mfma_kernel")
INFINITY_CACHE = 256 * 2 ** 20


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    # 200 anchor steps take ~10 ms of GPU time; the synchronize at each end of
    # the timed region is then ~0.5 % of the per-step figure.
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="anchor")
    p.add_argument("--tokens", type=int, default=-1,
                   help="every sequence's length (default: the workload's own lengths)")
    p.add_argument("--splits", type=int, default=0, help="0 = the library's choice")
    p.add_argument("--value-dtype", default="float32",
                   choices=["float32", "float16", "bfloat16"])
    p.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    p.add_argument("--cpu-runs", type=int, default=3)
    p.add_argument("--no-pmc", action="store_true",
                   help="skip the rocprofv3 --pmc traffic runs (required under rocprofv3)")
    p.add_argument("--decode-only", action="store_true",
                   help="time the decode and the grouped quantizer of the workload and "
                        "nothing else (no other paths, trace, PMC or CPU legs)")
    p.add_argument("--step-only", action="store_true",
                   help="time the serving step (B8 H32 D128 around 2048 tokens, eager steps "
                        "and the plain decode of the same cache) and nothing else, then run "
                        "the 256 MiB calibration kernels; prints other_paths.decode_step "
                        "without the graph figures (the command rocprofv3 --pmc passes over "
                        "the step kernel run)")
    p.add_argument("--no-trace", action="store_true",
                   help="skip the rocprofv3 --kernel-trace child of the headline window "
                        "(required under rocprofv3)")
    p.add_argument("--pmc-child", default="", help=argparse.SUPPRESS)
    p.add_argument("--trace-child", action="store_true", help=argparse.SUPPRESS)
    return p.parse_args()


def progress(msg):
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def workload_lens(args):
    """Every sequence at --tokens rows, or None for the workload's own lengths."""
    if args.tokens < 0:
        return None
    import numpy as np
    from flash_decode_int4 import workloads
    return np.full(workloads.WORKLOADS[args.workload]["batch"], args.tokens, np.int32)


def build_sets(name, value_dtype, n_sets_hint=0, seq_lens=None):
    """Independent input sets in HBM (different seeds), keys quantized into pages.
    seq_lens overrides the workload's lengths (same heads, head_dim and pages)."""
    import torch
    from flash_decode_int4 import ops, workloads
    sets = []
    first = workloads.make_workload(name, seq_lens=seq_lens, value_dtype=value_dtype,
                                    backend="torch", seed=1234)
    vbytes = 4 if value_dtype == "float32" else 2
    set_bytes = workloads.decode_bytes(first["seq_lens"], first["heads"], first["head_dim"],
                                       vbytes, q_heads=first["q_heads"])
    if n_sets_hint:
        n_sets = n_sets_hint
    else:
        n_sets = max(2, math.ceil(2 * INFINITY_CACHE / set_bytes) + 1)
    for i in range(n_sets):
        # Same lengths (and so the same bytes) in every set; different data.
        w = first if i == 0 else workloads.make_workload(
            name, seq_lens=first["seq_lens"], value_dtype=value_dtype, backend="torch",
            seed=1234 + 101 * i)
        dev = torch.device("cuda")
        B, H, D = w["batch"], w["heads"], w["head_dim"]
        G = (w["max_tokens"] + w["group_rows"] - 1) // w["group_rows"]
        s = dict(
            q=w["q"], k=w["k"], v=w["v_pages"],
            kp=torch.zeros(w["num_pages"], H, w["page_rows"], D // 2, dtype=torch.uint8,
                           device=dev),
            s=torch.zeros(B, H, G, D, device=dev),
            z=torch.zeros(B, H, G, D, device=dev),
            pt=torch.as_tensor(w["page_table"], device=dev),
            sl=torch.as_tensor(w["seq_lens"], device=dev),
            w=w)
        ops.quantize_int4_paged(s["k"], s["sl"], s["pt"], s["kp"], s["s"], s["z"],
                                w["group_rows"])
        sets.append(s)
    torch.cuda.synchronize()
    return sets, set_bytes


def time_reference_config(steps, warmup):
    """The reference's own benchmark semantics through the drop-in API: B8 H32
    D128 queries all attending one shared stream of 8 pages x 256 rows
    (2048 tokens), each page one scale group with unpacked INT4 keys and fp32
    values (reference benchmarks/bench_three_backend.py:113-129, src/ops.py
    :176-253). Keys are quantized with the package's quantize_int4; run() of
    prepare_flash_decode_hip is timed (inputs staged in HBM once)."""
    import numpy as np
    import torch
    from flash_decode_int4 import ops
    rng = np.random.RandomState(1234)
    B, H, D, nb, bs = 8, 32, 128, 8, 256
    query = rng.randn(B, H, D).astype(np.float32)
    kq, ks, kz, vv = [], [], [], []
    for _ in range(nb):
        k = rng.randn(bs, D).astype(np.float32)
        q, sc, zp = ops.quantize_int4(k, backend="hip")
        kq.append(q); ks.append(sc); kz.append(zp)
        vv.append(rng.randn(bs, D).astype(np.float32))
    call = ops.prepare_flash_decode_hip(query, kq, ks, kz, vv)
    for _ in range(warmup):
        call.run()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        out = call.run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    return {"workload": "reference semantics: B8 H32 D128, one shared stream of 8 pages x "
                        "256 rows (one scale group per page, unpacked INT4 keys, fp32 values)",
            "decode_us": round(us, 3), "finite": bool(torch.isfinite(out).all()),
            "reference_cuda_h100_us": 400.0,
            "note": "the reference's published CUDA time for this configuration on an "
                    "NVIDIA H100 (its README and results JSON); other hardware, context only"}


def time_reference_quantizer(steps, warmup, window=True):
    """The reference's own quantizer benchmark semantics through the drop-in
    API: ops.quantize_int4 of one [rows, 128] float32 array, one scale group
    over all rows, one unpacked INT4 value per output byte (reference
    benchmarks/bench_three_backend.py:141-159, src/ops.py:111-161), at the
    two row counts the reference publishes CUDA times for. run() of
    prepare_quantize_int4_hip is timed over input sets rotated past twice the
    Infinity Cache. Bytes: the input read once, the unpacked bins and the
    scale/zero-point rows written. Returns the record and, per row count, the
    first set's input and outputs on the host for the CPU leg's bit-for-bit
    check against the oracle."""
    import torch
    from flash_decode_int4 import ops
    out, host = {}, {}
    published_us = {2048: 15.4, 32768: 149.6}
    for rows, ref_us in published_us.items():
        C = 128
        in_bytes = rows * C * 4
        n_sets = max(2, math.ceil(2 * INFINITY_CACHE / in_bytes) + 1)
        g = torch.Generator(device="cuda")
        g.manual_seed(4321)
        sets = [torch.randn(rows, C, generator=g, device="cuda") for _ in range(n_sets)]
        calls = [ops.prepare_quantize_int4_hip(k) for k in sets]
        host[f"rows_{rows}x{C}"] = (sets[0].cpu().numpy(), calls[0]())
        for i in range(warmup):
            calls[i % n_sets].run()
        if not window:
            # A counter pass: K calls over the rotated inputs.
            for i in range(steps):
                calls[i % n_sets].run()
            torch.cuda.synchronize()
            del sets, calls
            torch.cuda.empty_cache()
            continue
        nb, blk = window_shape(steps)
        us, us_med, _ = window_us(lambda i: calls[i % n_sets].run(), nb, blk)
        # The same call on one input over and over (every read served by the
        # caches): against the rotated figure, what reading the input from
        # HBM costs the call.
        res_us, _, _ = window_us(lambda i: calls[0].run(), nb, blk)
        nbytes = in_bytes + rows * C + 2 * C * 4
        out[f"rows_{rows}x{C}"] = {
            "us": round(us, 3), "us_median": round(us_med, 3), "bytes": nbytes,
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "resident_us": round(res_us, 3),
            "input_sets": n_sets, "reference_cuda_h100_us": ref_us}
        del sets, calls
        torch.cuda.empty_cache()
    out["note"] = ("reference's published CUDA quantizer times on an NVIDIA H100 "
                   "(results/three_backend_quantize_h100.json); other hardware, context only")
    return out, host


def cpu_check_reference_quantizer(host):
    """CPU leg: the NumPy oracle on the first input set of each row count of
    time_reference_quantizer, compared bit for bit with the device's bins,
    scales and zero-points."""
    import numpy as np
    from oracle import quantize_int4_ref
    res = {}
    for name, (kv, (q, s, z)) in host.items():
        rq, rs, rz = quantize_int4_ref(kv)
        res[name] = bool(np.array_equal(q, rq) and np.array_equal(s, rs)
                         and np.array_equal(z, rz))
    return res


#: The steady-state window of the roofline figure: WINDOW_BLOCKS blocks of
#: back-to-back launches (at least WINDOW_MIN launches in all, more when
#: --steps asks for more), one HIP event between blocks and no host
#: synchronization inside the window.
WINDOW_BLOCKS = 20
WINDOW_MIN = 400


def window_shape(steps):
    """(blocks, launches per block) of the steady-state window."""
    per = max(WINDOW_MIN, steps)
    return WINDOW_BLOCKS, -(-per // WINDOW_BLOCKS)


#: GPU time spent in untimed launches before a window: a GPU that has been
#: idle runs its first ~15 ms of back-to-back launches 1-7 % slower (B8 H32
#: T2048 decode, blocks of 20 launches: 50-54 us, then a steady 49.0-49.3).
SETTLE_MS = 30.0


def settle(fn, start=0):
    """Untimed back-to-back launches for about SETTLE_MS of GPU time (ten to
    measure the launch, then as many as the rest needs); returns the next
    launch index."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(10):
        fn(start + i)
    e1.record()
    torch.cuda.synchronize()
    per_ms = max(e0.elapsed_time(e1) / 10, 1e-3)
    n = max(0, math.ceil((SETTLE_MS - 10 * per_ms) / per_ms))
    for i in range(n):
        fn(start + 10 + i)
    return start + 10 + n


def window_us(fn, blocks, block, start=0):
    """After settle(), back-to-back launches in `blocks` blocks of `block`,
    one event on the launch stream before the first block and after every
    block, one synchronize at the end (the GPU never idles inside the
    window). Returns (mean per launch over the window, median over the blocks
    of the per-launch time of a block, launches)."""
    import torch
    start = settle(fn, start)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(blocks + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    k = start
    for j in range(blocks):
        for _ in range(block):
            fn(k)
            k += 1
        ev[j + 1].record()
    torch.cuda.synchronize()
    per = [ev[j].elapsed_time(ev[j + 1]) * 1e3 / block for j in range(blocks)]
    return ev[0].elapsed_time(ev[blocks]) * 1e3 / (blocks * block), median(per), blocks * block


def blocked_median_us(fn, n, block=10):
    """Median over the blocks of a window of back-to-back launches (at least
    20 blocks of `block` launches, more when n asks for more), with no host
    synchronization between blocks."""
    return window_us(fn, max(20, -(-n // block)), block)[1]


def hbm_probes():
    """Achievable bandwidth on this box with a plain torch elementwise kernel
    that reads and writes 1 GiB."""
    import torch
    n = 2 ** 28
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)

    def rate(fn, nbytes, reps=5):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)

    res = {"elementwise_copy_gbs": rate(lambda: torch.mul(a, 1.0, out=b), 2 * 4 * n)}
    del a, b
    torch.cuda.empty_cache()
    return res


def decode_launchers(sets, splits):
    """(S, step, decode_only): the production decode of input set i % len(sets)
    (decode kernel, plus the merge with S > 1 splits) and the decode kernel
    alone."""
    import torch
    from flash_decode_int4._lib import load_binding
    C = load_binding()
    w0 = sets[0]["w"]
    B, H, D, Hq = w0["batch"], w0["heads"], w0["head_dim"], w0["q_heads"]
    ppg = w0["group_rows"] // w0["page_rows"]
    maxp = w0["page_table"].shape[1]
    S = splits or int(C.decode_num_splits(B, Hq, H, D, maxp, w0["page_rows"]))
    S = max(1, min(S, maxp * ((w0["page_rows"] + 15) // 16)))
    parts = torch.empty(int(C.decode_partials_bytes(B, Hq, D, S)), dtype=torch.uint8,
                        device="cuda")

    def step(i):
        # The production call: with one split it is the decode kernel alone
        # (writing the output); with several it is the decode kernel and the
        # merge -- issued here as the same two launches the one-call entry
        # point makes, so the decode kernel can also be timed alone.
        st = sets[i % len(sets)]
        if S == 1:
            return C.decode_paged(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                  st["sl"], None, ppg, maxp, 1)
        C.decode_paged_partials(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                st["sl"], None, ppg, maxp, S, parts)
        return C.merge_splits(parts, B, Hq, D, S)

    def decode_only(i):
        st = sets[i % len(sets)]
        C.decode_paged_partials(st["q"], st["kp"], st["v"], st["s"], st["z"], st["pt"],
                                st["sl"], None, ppg, maxp, S, parts)

    return S, step, decode_only


# Launches per block of the alternating check: each block starts on the other
# input sets, so a longer block leaves that switch a smaller share of it.
INTERLEAVE_BLOCK = 40


def interleaved_us(fa, fb, rounds=10, block=INTERLEAVE_BLOCK):
    """Per-launch time of two launch sequences measured in alternating blocks
    (A, B, A, B, ...) of `block` back-to-back launches after settle(), one
    event between blocks and one synchronize at the end, so both see the same
    clocks and memory state and the GPU never idles between blocks; returns
    the two medians over the rounds."""
    import torch
    settle(fa)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * rounds + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for r in range(rounds):
        for j, fn in enumerate((fa, fb)):
            for i in range(block):
                fn(r * block + i)
            ev[2 * r + j + 1].record()
    torch.cuda.synchronize()
    ta = [ev[2 * r].elapsed_time(ev[2 * r + 1]) * 1e3 / block for r in range(rounds)]
    tb = [ev[2 * r + 1].elapsed_time(ev[2 * r + 2]) * 1e3 / block for r in range(rounds)]
    return median(ta), median(tb)


def time_decode(sets, splits, steps, warmup, window=True):
    import torch
    S, step, decode_only = decode_launchers(sets, splits)

    def timed(fn, n):
        """n back-to-back launches; one event pair on the launch stream (per-launch
        event markers would add their own time to the GPU timeline) plus wall clock."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        out = None
        for i in range(n):
            out = fn(i)
        e1.record()
        torch.cuda.synchronize()
        return out, time.perf_counter() - t0, e0.elapsed_time(e1) * 1e3 / n

    for i in range(warmup):
        step(i)
    out, wall, step_us = timed(step, steps)
    if not window:
        # A check or a counter pass: the K steps only.
        return dict(splits=S, wall_s=wall, step_us=step_us, window_us=step_us,
                    step_median_us=step_us, window_launches=steps, window_blocks=1,
                    decode_us=step_us, decode_median_us=step_us, merge_us=0.0, last_out=out,
                    last_set=(steps - 1) % len(sets))
    nb, blk = window_shape(steps)
    win_us, win_median, win_n = window_us(step, nb, blk, start=steps)
    if S == 1:
        dec_us, dec_median = win_us, win_median
    else:
        for i in range(warmup):
            decode_only(i)
        dec_us, dec_median, _ = window_us(decode_only, nb, blk)
    return dict(splits=S, wall_s=wall, step_us=step_us, window_us=win_us,
                step_median_us=win_median, window_launches=win_n, window_blocks=nb,
                decode_us=dec_us, decode_median_us=dec_median,
                merge_us=max(win_us - dec_us, 0.0), last_out=out,
                last_set=(steps - 1) % len(sets))


def time_quantizer(sets, steps, warmup, window=True):
    """Grouped quantizer over the rotated input sets: (mean per launch over a
    steady-state window, median over the window's blocks); window=False: K
    launches (a counter pass)."""
    from flash_decode_int4 import ops
    g = sets[0]["w"]["group_rows"]

    def q(i):
        st = sets[i % len(sets)]
        ops.quantize_int4_paged(st["k"], st["sl"], st["pt"], st["kp"], st["s"], st["z"], g)

    for i in range(warmup):
        q(i)
    if not window:
        for i in range(steps):
            q(i)
        return None, None
    nb, blk = window_shape(steps)
    mean, med, _ = window_us(q, nb, blk)
    return mean, med


def time_append(w, value_dtype, steps, warmup):
    """Decode-time append (one token per (sequence, kv-head)) on a cache of the
    workload's shape: the kernel re-quantizes the open scale group, so its cost
    runs from one row (first token of a group) to a full group (last token).
    Both ends are timed over back-to-back launches at a fixed position (the
    call is idempotent when the lengths are not advanced)."""
    import torch
    from flash_decode_int4._lib import load_binding
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    C = load_binding()
    B, H, D, G = w["batch"], w["heads"], w["head_dim"], w["group_rows"]
    T = int(max(w["seq_lens"]))
    T = max(T, G)
    out = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    vdt = getattr(torch, value_dtype)
    k = torch.randn(B, H, T, D, generator=g, device="cuda")
    v = torch.randn(B, H, T, D, generator=g, device="cuda").to(vdt)
    kn = torch.randn(B, H, D, generator=g, device="cuda")
    vn = torch.randn(B, H, D, generator=g, device="cuda").to(vdt)
    for name, t in (("first_row", T - G), ("full_group", T - 1)):
        cache = INT4PagedSequenceCache(num_pages=B * (T // 16 + 2), num_kv_heads=H, head_dim=D,
                                       max_seqs=B, max_seq_len=T, group_rows=G,
                                       value_dtype=value_dtype)
        cache.prefill(k, v, [t] * B)

        def call():
            C.append_paged(kn, vn, cache.k_stage, cache.k_pages, cache.v_pages, cache.k_scale,
                           cache.k_zp, cache.page_table, cache.seq_lens, G)

        for _ in range(warmup):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) * 1e3 / steps, 3)
        del cache
    return out


def _torch_chain_fake_quant(k, block):
    """The harness's fake quantization (scripts/validate_llama.py:126-154) as
    a chain of eager torch operations, timed as the unfused baseline: upcast,
    pad the last block with its last row, per-block extremes, bins, dequantize,
    cast back."""
    import torch
    b, h, s, d = k.shape
    nb = -(-s // block)
    x = k.float()
    if nb * block != s:
        x = torch.cat([x, x[:, :, -1:].expand(b, h, nb * block - s, d)], dim=2)
    x = x.view(b, h, nb, block, d)
    lo = x.amin(dim=3, keepdim=True)
    step = (x.amax(dim=3, keepdim=True) - lo).clamp_min(1e-8) / 15.0
    q = torch.floor((x - lo) / step + 0.5).clamp_(0.0, 15.0)
    return (q * step + lo).view(b, h, nb * block, d)[:, :, :s].to(k.dtype)


def time_fake_quant(steps, warmup):
    """Device fake quantization of keys (quality-study path) on two shapes:
    one perplexity window of a Llama-2-7B-sized model (32 kv-heads x 2048
    positions x 128, float16, 256-position blocks, the harness defaults) and
    the decode workload's key tensor (8 x 32 x 2048 x 128 float32, 128-position
    blocks). Inputs rotate over enough sets to exceed twice the Infinity Cache;
    bytes are one read and one write of the keys. The harness window is also
    timed as an eager chain of torch operations (the unfused formulation)."""
    import torch
    from flash_decode_int4.quality import fake_quantize_keys
    out = {}
    cases = (("harness_window_f16", (1, 32, 2048, 128), torch.float16, 256),
             ("decode_keys_f32", (8, 32, 2048, 128), torch.float32, 128))
    for name, shape, dt, block in cases:
        nbytes = 2 * math.prod(shape) * torch.empty(0, dtype=dt).element_size()
        n_sets = max(2, math.ceil(2 * INFINITY_CACHE / nbytes))
        g = torch.Generator(device="cuda")
        g.manual_seed(91)
        ks = [torch.randn(shape, generator=g, device="cuda").to(dt) for _ in range(n_sets)]
        outs = [torch.empty_like(k) for k in ks]
        # Eager torch divides by the Python scalar 15.0 through its float32
        # reciprocal: the kernel's reciprocal scale form reproduces it bit for bit.
        ok = bool(torch.equal(fake_quantize_keys(ks[0], block, scale_op="reciprocal"),
                              _torch_chain_fake_quant(ks[0], block)))

        def fq(i):
            fake_quantize_keys(ks[i % n_sets], block, out=outs[i % n_sets])

        for i in range(warmup):
            fq(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(steps):
            fq(i)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        rec = {"shape": list(shape), "dtype": str(dt).replace("torch.", ""), "block": block,
               "bytes": nbytes, "us": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "reciprocal_form_equals_torch_chain": ok}
        if name == "harness_window_f16":
            for i in range(warmup):
                _torch_chain_fake_quant(ks[i % n_sets], block)
            torch.cuda.synchronize()
            e0.record()
            for i in range(steps):
                _torch_chain_fake_quant(ks[i % n_sets], block)
            e1.record()
            torch.cuda.synchronize()
            rec["torch_chain_us"] = round(e0.elapsed_time(e1) * 1e3 / steps, 3)
        out[name] = rec
        del ks, outs
        torch.cuda.empty_cache()
    return out


def time_other_paths(args):
    """Decode timings of the paths beside the headline one, on their own
    workloads (inputs rotated past the Infinity Cache as for the headline):
    fp16 and bf16 value pages at the anchor shape, and grouped-query heads (B8,
    8 kv-heads, 32 q-heads, 8192 tokens). Skipped when the headline workload
    is already one of them."""
    import torch
    from flash_decode_int4 import workloads
    out = {}
    cases = (("fp16_values", "anchor", "float16"), ("bf16_values", "anchor", "bfloat16"),
             ("grouped_query", "gqa", "float32"))
    for key, name, vdt in cases:
        if name == args.workload and vdt == args.value_dtype:
            continue
        sets, nbytes = build_sets(name, vdt)
        r = time_decode(sets, 0, args.steps, args.warmup)
        w = sets[0]["w"]
        out[key] = {
            "workload": f"{name}: B{w['batch']} Hkv{w['heads']} Hq{w['q_heads']} D{w['head_dim']} "
                        f"T{int(max(w['seq_lens']))}, {vdt} values",
            "kernel": decode_kernel_label(w, vdt), "num_splits": r["splits"],
            "bytes": nbytes, "decode_us": round(r["window_us"], 3),
            "decode_us_median": round(r["step_median_us"], 3),
            "gbs": round(nbytes / (r["window_us"] * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (r["window_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "finite": bool(torch.isfinite(r["last_out"]).all())}
        del sets
        torch.cuda.empty_cache()
    return out


def time_decode_step(args, B=8, H=32, D=128, T=2048, graph_steps=8, graphs=True,
                     max_seq_len=None):
    """The serving loop's step on the sequence cache (fp32 values, B sequences
    of H heads around T tokens): append one token per (sequence, kv-head),
    decode over the advanced lengths, advance them -- one launch when each
    (sequence, kv-head) is one decode workgroup (fdi4_decode_step). Every
    timed segment is one scale group of steps (group_rows = 128) from the same
    state, T - 64 tokens, restored before it (the device lengths and the open
    group's staging rows), so a segment re-quantizes every row count of a
    group once and its mean length is T - 0.5: the steps issued eagerly from
    Python, one-step graph replays, and replays of a graph of `graph_steps`
    steps (the graph launch's own cost spread over them). Medians over the
    rounds, per step; `decode_us` is the plain decode of the same cache at T
    tokens (graphs=False: the eager steps and that decode only)."""
    import torch
    from flash_decode_int4.vllm_integration import INT4PagedSequenceCache
    G = 128
    T0 = T - G // 2
    rounds = 4
    cap = max_seq_len or T0 + G
    cache = INT4PagedSequenceCache(num_pages=B * ((T0 + G) // 16 + 2), num_kv_heads=H,
                                   head_dim=D, max_seqs=B, max_seq_len=cap, group_rows=G)
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    k = torch.randn(B, H, T0, D, device="cuda", generator=g)
    cache.prefill(k, torch.randn_like(k), [T0] * B)
    del k
    cache.reserve(B, G)
    stage0 = cache.k_stage.clone()
    kn = torch.randn(B, H, D, device="cuda", generator=g)
    vn = torch.randn(B, H, D, device="cuda", generator=g)
    q = torch.randn(B, H, D, device="cuda", generator=g)

    def restore(length=T0):
        torch.cuda.synchronize()
        cache.seq_lens[:B].fill_(length)
        cache.k_stage.copy_(stage0)
        torch.cuda.synchronize()
        cache.sync_lengths()

    def timed(fn, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3

    for _ in range(min(args.warmup, G)):
        cache.step(kn, vn, q)
    restore()
    graph_1 = graph_k = None
    if graphs:
        graph_1 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_1):
            out_1 = cache.step(kn, vn, q)
        graph_k = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_k):
            for _ in range(graph_steps):
                out_k = cache.step(kn, vn, q)
    eager, rep_1, rep_k = [], [], []
    for _ in range(rounds):
        restore()
        eager.append(timed(lambda: cache.step(kn, vn, q), G) / G)
        if graphs:
            restore()
            rep_1.append(timed(graph_1.replay, G) / G)
            restore()
            rep_k.append(timed(graph_k.replay, G // graph_steps) / G)
    cache.sync_lengths()
    end_len = int(cache.lengths()[0])
    if graphs:
        ok = bool(torch.isfinite(out_1).all()) and bool(torch.isfinite(out_k).all())
    else:
        restore()
        ok = bool(torch.isfinite(cache.step(kn, vn, q)).all())
    restore(T)
    dec = median([timed(lambda: cache.decode(q), 20) / 20 for _ in range(rounds)])
    res = {"workload": f"B{B} H{H} D{D}, fp32 values: append + decode + length advance per "
                       f"step, steps from {T0} to {T0 + G} tokens (one {G}-token scale group, "
                       f"mean {T - 0.5}), a cache of {cap} tokens per sequence",
           "eager_us": round(median(eager), 3),
           "graph_replay_us": round(median(rep_1), 3) if graphs else None,
           f"graph_{graph_steps}_steps_replay_us_per_step":
               round(median(rep_k), 3) if graphs else None,
           "decode_us": round(dec, 3), "rounds": rounds, "finite": ok,
           "final_length": end_len}
    del cache, graph_1, graph_k
    torch.cuda.empty_cache()
    return res


def median(x):
    s = sorted(x)
    n = len(s)
    return s[n // 2] if n % 2 else 0.5 * (s[n // 2 - 1] + s[n // 2])


def _oracle_streams(path, b, h0, h1):
    """Worker of the all-core CPU run (a fresh interpreter, no GPU): the oracle
    decode of sequence b, kv-heads h0..h1-1, from arrays memory-mapped at path."""
    import numpy as np
    from oracle import paged_decode_ref
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    a = {k: np.load(os.path.join(path, k + ".npy"), mmap_mode="r")
         for k in ("q", "kp", "v", "s", "z", "pt", "sl")}
    rep = a["q"].shape[1] // a["kp"].shape[1]
    args = (np.asarray(a["q"][b:b + 1, h0 * rep:h1 * rep]), a["kp"][:, h0:h1], a["v"][:, h0:h1],
            np.asarray(a["s"][b:b + 1, h0:h1]), np.asarray(a["z"][b:b + 1, h0:h1]),
            np.asarray(a["pt"][b:b + 1]), np.asarray(a["sl"][b:b + 1]))
    if threadpool_limits is None:
        return b, h0 * rep, paged_decode_ref(*args)[0]
    with threadpool_limits(limits=1):
        return b, h0 * rep, paged_decode_ref(*args)[0]


def cpu_all_cores(host, o32, runs=2):
    """The same oracle decode spread over this host's cores (one process per
    core, (sequence, kv-head-block) tasks); returns (seconds, workers, max |diff|
    from the one-core output)."""
    import multiprocessing
    import numpy as np
    from concurrent.futures import ProcessPoolExecutor
    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    B, Hkv = host["q"].shape[0], host["kp"].shape[1]
    per = max(1, (B * Hkv + 2 * workers - 1) // (2 * workers))
    tasks = [(b, h, min(h + per, Hkv)) for b in range(B) for h in range(0, Hkv, per)]
    with tempfile.TemporaryDirectory(prefix="fdi4_cpu_") as d:
        for k in ("q", "kp", "v", "s", "z", "pt", "sl"):
            np.save(os.path.join(d, k + ".npy"), np.ascontiguousarray(host[k]))
        ctx = multiprocessing.get_context("spawn")
        with ProcessPoolExecutor(max_workers=workers, mp_context=ctx) as pool:
            list(pool.map(_oracle_streams, [d] * workers, [0] * workers, [0] * workers,
                          [1] * workers))  # start and warm every worker
            times = []
            out = np.zeros_like(o32)
            for _ in range(max(1, runs)):
                t0 = time.perf_counter()
                futs = [pool.submit(_oracle_streams, d, *t) for t in tasks]
                for f in futs:
                    b, q0, rows = f.result()
                    out[b, q0:q0 + rows.shape[0]] = rows
                times.append(time.perf_counter() - t0)
    return median(times), workers, float(np.abs(out - o32).max())


def cpu_baseline(st, gpu_out, runs, vbytes):
    """Time the NumPy oracle on the host over the same workload; check the GPU output."""
    import numpy as np
    import torch
    from oracle import cref, paged_decode_ref, quantize_groups_ref, pack_int4
    from flash_decode_int4 import workloads
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    w = st["w"]
    host = dict(q=st["q"].cpu().numpy(), kp=st["kp"].cpu().numpy(),
                v=st["v"].float().cpu().numpy(), s=st["s"].cpu().numpy(),
                z=st["z"].cpu().numpy(), pt=w["page_table"], sl=w["seq_lens"])
    k_host = st["k"].cpu().numpy()
    args = (host["q"], host["kp"], host["v"], host["s"], host["z"], host["pt"], host["sl"])
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    times, qtimes = [], []
    try:
        if ctx is not None:
            ctx.__enter__()
        for _ in range(max(1, runs)):
            t0 = time.perf_counter()
            o32 = paged_decode_ref(*args)
            times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        qr, sr, zr = quantize_groups_ref(k_host, host["sl"])
        qtimes.append(time.perf_counter() - t0)
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    o64 = cref.paged_attention_f64(*args)
    got = gpu_out.cpu().numpy()
    # Quantizer parity: scales and every packed page of this set, bit for bit.
    scales_ok = bool(np.array_equal(host["s"], sr) and np.array_equal(host["z"], zr))
    pages_ok = True
    for b in range(len(host["sl"])):
        n = int(host["sl"][b])
        for lp in range((n + 15) // 16):
            rows = min(16, n - lp * 16)
            want = pack_int4(qr[b, :, lp * 16:lp * 16 + rows])
            if not np.array_equal(host["kp"][host["pt"][b, lp], :, :rows], want):
                pages_ok = False
                break
        if not pages_ok:
            break
    nbytes = workloads.decode_bytes(host["sl"], w["heads"], w["head_dim"], vbytes,
                                    q_heads=w["q_heads"])
    qbytes = workloads.quantize_bytes(host["sl"], w["heads"], w["head_dim"])
    t = median(times)
    base = {
        "value": round(nbytes / t / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"whole workload: NumPy oracle page loop, one call per (sequence, head) "
                   f"stream, {len(times)} runs, median {t * 1e3:.1f} ms per decode; "
                   f"quantizer oracle {qtimes[0] * 1e3:.1f} ms "
                   f"({qbytes / qtimes[0] / 1e9:.3f} GB/s); BLAS limited to 1 thread; "
                   f"host cores available {len(os.sched_getaffinity(0))}"),
        "decode_ms": round(t * 1e3, 3),
        "quantizer_ms": round(qtimes[0] * 1e3, 3),
    }
    try:
        ta, nw, dall = cpu_all_cores(host, o32)
        base["all_cores"] = {"value": round(nbytes / ta / 1e9, 4), "cores": nw,
                             "decode_ms": round(ta * 1e3, 3),
                             "max_abs_vs_one_core": dall}
    except Exception as exc:  # the one-core figure stands on its own
        base["all_cores"] = {"error": repr(exc)[:200]}
    parity = {
        "max_abs_vs_oracle_f32": float(np.abs(got - o32).max()),
        "max_abs_vs_f64": float(np.abs(got - o64).max()),
        "oracle_f32_vs_f64": float(np.abs(o32 - o64).max()),
        "tolerance": 1e-5,
        "quantizer_bit_exact": bool(scales_ok and pages_ok),
    }
    return base, parity


def pmc_child(args):
    """Run a few decode and quantizer launches on one set (for rocprofv3
    --pmc), the calibration kernels (256 MiB fill, sum and copy) whose
    counters give the bytes/counter factors, then the fake-quantization
    workloads."""
    import torch
    sets, _ = build_sets(args.workload, args.value_dtype, n_sets_hint=1,
                         seq_lens=workload_lens(args))
    r = time_decode(sets, args.splits, steps=3, warmup=1, window=False)
    time_quantizer(sets, steps=3, warmup=1, window=False)
    del sets
    torch.cuda.empty_cache()
    calibration_kernels()
    time_fake_quant(steps=2, warmup=1)
    time_reference_quantizer(steps=3, warmup=1, window=False)
    print(json.dumps({"splits": r["splits"]}))


def calibration_kernels():
    """Kernels over 256 MiB of float32 whose PMC readings give bytes per
    counter unit: a fill (writes only), a sum (reads only) and an elementwise
    copy (reads and writes), three launches each."""
    import torch
    a = torch.empty(64 * 2 ** 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        a.fill_(1.0)
    for _ in range(3):
        torch.sum(a)
    for _ in range(3):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    del a, b
    torch.cuda.empty_cache()


def pmc_traffic(args):
    """HBM bytes per decode-kernel launch from FETCH_SIZE and WRITE_SIZE passes,
    each scaled by the same counter's reading for a kernel that moves 256 MiB
    in that direction only; also the grouped quantizer's and the
    fake-quantization kernel's bytes."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    import csv
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="fdi4_pmc_")
        cmd = [exe, "--pmc", counter, "-d", d, "-o", "pmc", "--output-format", "csv", "--",
               sys.executable, os.path.abspath(__file__), "--workload", args.workload,
               "--tokens", str(args.tokens), "--splits", str(args.splits),
               "--value-dtype", args.value_dtype, "--pmc-child", counter]
        try:
            subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=180,
                           check=False)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 --pmc {counter} timed out"
        rows = []
        for dirpath, _, files in os.walk(d):
            for f in files:
                if f.endswith("counter_collection.csv"):
                    with open(os.path.join(dirpath, f)) as fh:
                        rows += list(csv.DictReader(fh))
        def values(pred):
            return [float(r["Counter_Value"]) for r in rows
                    if pred(r.get("Kernel_Name", "")) and r.get("Counter_Name") == counter]

        dec = values(lambda k: any(f"{n}<" in k for n in DECODE_KERNELS))
        # The calibration kernel for this counter: reads only for FETCH_SIZE
        # (the sum), writes only for WRITE_SIZE (the fill).
        cal = values(lambda k: ("sum_functor" in k) if counter == "FETCH_SIZE"
                     else ("FillFunctor" in k))
        cpy = values(lambda k: "MulFunctor" in k)
        qz = values(lambda k: "quantize_paged_kernel" in k)
        fq = {name: values(lambda k, t=tag: "fake_quant_kernel" in k and t in k)
              for name, tag in (("harness_window_f16", "F16Key"), ("decode_keys_f32", "F32Key"))}
        # The 2-D quantizer's kernels (fdi4::rows_*) by grid, then kernel: at
        # both row counts a call is two launches on the same (channel slices,
        # row tiles) grid, which grows with the rows.
        rq = {}
        for row in rows:
            k = row.get("Kernel_Name", "")
            if "fdi4::rows_" in k and row.get("Counter_Name") == counter:
                name = k.split("fdi4::", 1)[1].split("(")[0]
                rq.setdefault(int(row["Grid_Size"]), {}).setdefault(name, []).append(
                    float(row["Counter_Value"]))
        shutil.rmtree(d, ignore_errors=True)
        if not dec or not cal or not cpy:
            return None, f"no {counter} rows for the decode or calibration kernels"
        out[counter] = (median(dec), max(cal), {k: median(v) for k, v in fq.items() if v},
                        max(cpy), median(qz) if qz else None, rq)
    # Each calibration kernel moves 256 MiB in the counted direction: the
    # factor converts counter units to bytes. The copy's factors are reported
    # beside them (its reads can include line fills for its writes).
    cal_bytes = 256 * 2 ** 20
    ff = cal_bytes / out["FETCH_SIZE"][1]
    wf = cal_bytes / out["WRITE_SIZE"][1]
    fake = {name: {"fetch_bytes": out["FETCH_SIZE"][2][name] * ff,
                   "write_bytes": out["WRITE_SIZE"][2][name] * wf}
            for name in out["FETCH_SIZE"][2] if name in out["WRITE_SIZE"][2]}
    quant = None
    if out["FETCH_SIZE"][4] is not None and out["WRITE_SIZE"][4] is not None:
        quant = {"fetch_bytes": out["FETCH_SIZE"][4] * ff,
                 "write_bytes": out["WRITE_SIZE"][4] * wf}
    # Per row count of the reference quantizer (the smaller grid is the
    # 2048-row call), the medians of the call's kernels summed.
    ref_q = {}
    for counter, factor in (("FETCH_SIZE", ff), ("WRITE_SIZE", wf)):
        by_grid = out[counter][5]
        for i, g in enumerate(sorted(by_grid)[:2]):
            rec = ref_q.setdefault(f"rows_{(2048, 32768)[i]}x128", {})
            key = "fetch_bytes" if counter == "FETCH_SIZE" else "write_bytes"
            rec[key] = sum(median(v) for v in by_grid[g].values()) * factor
            rec["kernels"] = sorted(by_grid[g])
    return {"fetch_bytes": out["FETCH_SIZE"][0] * ff, "write_bytes": out["WRITE_SIZE"][0] * wf,
            "fetch_factor_bytes_per_unit": ff, "write_factor_bytes_per_unit": wf,
            "copy_fetch_factor_bytes_per_unit": cal_bytes / out["FETCH_SIZE"][3],
            "copy_write_factor_bytes_per_unit": cal_bytes / out["WRITE_SIZE"][3],
            "fake_quant": fake, "quantizer": quant, "reference_quantizer": ref_q}, None


def trace_child(args):
    """The headline's decode window alone, for a rocprofv3 --kernel-trace
    child: the same input sets, warmup, then (after settle()) the
    steady-state window of the decode kernel (window_shape(--steps)); prints
    its own event figures."""
    sets, _ = build_sets(args.workload, args.value_dtype, seq_lens=workload_lens(args))
    S, step, decode_only = decode_launchers(sets, args.splits)
    fn = step if S == 1 else decode_only
    for i in range(args.warmup):
        fn(i)
    nb, blk = window_shape(args.steps)
    mean, med, n = window_us(fn, nb, blk)
    print(json.dumps({"splits": S, "window_launches": n, "event_us": mean,
                      "event_median_us": med}), flush=True)


def trace_window(args):
    """Per-dispatch durations of the decode kernel over the steady-state
    window, from a rocprofv3 --kernel-trace run of trace_child: the last
    window_launches dispatches of the decode kernel (the warmup ones before
    them are dropped)."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    import csv
    d = tempfile.mkdtemp(prefix="fdi4_trace_")
    cmd = [exe, "--kernel-trace", "--stats", "-d", d, "-o", "trace", "--output-format", "csv",
           "--", sys.executable, os.path.abspath(__file__), "--workload", args.workload,
           "--tokens", str(args.tokens), "--splits", str(args.splits),
           "--value-dtype", args.value_dtype, "--steps", str(args.steps),
           "--warmup", str(args.warmup), "--trace-child"]
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                           timeout=240, check=False)
    except subprocess.TimeoutExpired:
        shutil.rmtree(d, ignore_errors=True)
        return None, "rocprofv3 --kernel-trace timed out"
    child = None
    for line in r.stdout.splitlines():
        if line.startswith("{"):
            child = json.loads(line)
    rows = []
    for dirpath, _, files in os.walk(d):
        for f in files:
            if f.endswith("kernel_trace.csv"):
                with open(os.path.join(dirpath, f)) as fh:
                    rows += list(csv.DictReader(fh))
    shutil.rmtree(d, ignore_errors=True)
    if child is None:
        return None, f"trace child printed no result (rc {r.returncode})"
    dec = sorted((int(x["Start_Timestamp"]), int(x["End_Timestamp"])) for x in rows
                 if any(f"{n}<" in x.get("Kernel_Name", "") for n in DECODE_KERNELS))
    n = int(child["window_launches"])
    if len(dec) < n:
        return None, f"{len(dec)} decode dispatches in the trace, {n} expected"
    durs = [(e - b) * 1e-3 for b, e in dec[-n:]]
    return {"trace_mean_us": sum(durs) / n, "trace_median_us": median(durs),
            "trace_dispatches": n, "child_event_us": child["event_us"]}, None


def decode_kernel_label(w, value_dtype):
    """The decode kernel the library's planner picks for this workload: the
    per-head kernel for one q-head per kv-head, the int8 matrix-core kernel
    for grouped heads at head_dim 64 / 128 (unless the decode_vector_only
    override is set), the vector grouped kernel otherwise."""
    from flash_decode_int4 import capi
    d, rep = w["head_dim"], w["q_heads"] // w["heads"]
    if rep == 1:
        return f"decode_kernel<D={d}, {value_dtype} values>"
    vector_only = capi.load().fdi4_get_tuning(capi.TUNE["decode_vector_only"]) == 1
    kind = ("decode_mfma_kernel" if d in (64, 128) and not vector_only
            else "decode_gqa_kernel")
    return f"{kind}<D={d}, {value_dtype} values, {rep} q-heads per kv-head>"


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU (the decode path shards by sequence "
              f"and head with no exchange); --gpus {args.gpus} / WORLD_SIZE {world} is not "
              f"supported", file=sys.stderr)
        sys.exit(2)
    if args.pmc_child:
        pmc_child(args)
        return
    if args.trace_child:
        trace_child(args)
        return
    import torch
    from flash_decode_int4 import ops, workloads
    if not ops.HAS_HIP:
        print("bench.py: the HIP extension or the GPU is unavailable: "
              f"{ops.backend_status()}", file=sys.stderr)
        sys.exit(1)
    if args.step_only:
        res = time_decode_step(args, graphs=False)
        calibration_kernels()
        print(json.dumps({"decode_step": res}))
        return

    progress(f"building the {args.workload} input sets")
    sets, set_bytes = build_sets(args.workload, args.value_dtype, seq_lens=workload_lens(args))
    w0 = sets[0]["w"]
    # The seq_len + 1 inputs are built now, so that the GPU does not sit idle
    # between the headline window and the check timed right after it (an
    # idle GPU starts the next launches at different clocks).
    odd_sets = odd_bytes = None
    if not args.decode_only:
        odd_sets, odd_bytes = build_sets(args.workload, args.value_dtype,
                                         seq_lens=w0["seq_lens"] + 1)
    vbytes = 4 if args.value_dtype == "float32" else 2
    qbytes = workloads.quantize_bytes(w0["seq_lens"], w0["heads"], w0["head_dim"])

    # Correctness before timing: the timed two-call path equals the one-call
    # path, and a different split count gives the same answer.
    st0 = sets[0]
    ref1 = ops.flash_decode_paged(st0["q"], st0["kp"], st0["v"], st0["s"], st0["z"], st0["pt"],
                                  st0["sl"], num_splits=1)
    r = time_decode([st0], args.splits, steps=1, warmup=0, window=False)
    gate = float((r["last_out"] - ref1).abs().max())
    if not (math.isfinite(gate) and gate < 2e-6 and bool(torch.isfinite(ref1).all())):
        print(f"bench.py: correctness gate failed (split vs single-split diff {gate})",
              file=sys.stderr)
        sys.exit(1)

    progress("timing the decode")
    res = time_decode(sets, args.splits, args.steps, args.warmup)
    dec_us, mrg_us, win_us = res["decode_us"], res["merge_us"], res["window_us"]
    ms_per_step = res["wall_s"] / args.steps * 1e3
    line = {
        "metric": METRIC,
        "value": round(set_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("f32 (f64 logit accumulation)" if vbytes == 4 else
                  f"f32 with {'f16' if args.value_dtype == 'float16' else 'bf16'} values"),
        "data": "synthetic N(0,1) q/K/V, seeded; keys quantized on the GPU; random page "
                "permutation",
        "config": {
            "workload": (f"{args.workload}: B{w0['batch']} "
                         + (f"H{w0['heads']} " if w0["q_heads"] == w0["heads"]
                            else f"Hkv{w0['heads']} Hq{w0['q_heads']} ")
                         + f"D{w0['head_dim']} "
                         f"T{int(max(w0['seq_lens']))}, {w0['page_rows']}-token pages, "
                         f"{w0['group_rows']}-token scale groups, {args.value_dtype} values"),
            "batch": w0["batch"], "heads": w0["heads"], "q_heads": w0["q_heads"],
            "head_dim": w0["head_dim"],
            "max_tokens": int(max(w0["seq_lens"])), "page_rows": w0["page_rows"],
            "group_rows": w0["group_rows"], "num_splits": res["splits"],
            "input_sets": len(sets), "bytes_per_step": set_bytes,
        },
        "clocks": {
            "value": f"wall clock around the {args.steps} timed steps (synchronize on both "
                     "sides; host launch cost included)",
            "decode_us": f"HIP events on the launch stream around a steady-state window of "
                         f"{res['window_launches']} back-to-back steps "
                         f"({res['window_blocks']} blocks, no host synchronization inside)",
            "decode_us_median": "median over the window's blocks of the per-step time",
            "decode_us_timed_loop": f"HIP events around the {args.steps} timed steps",
        },
        "decode_us": round(win_us, 3),
        "decode_us_median": round(res["step_median_us"], 3),
        "decode_us_timed_loop": round(res["step_us"], 3),
        "decode_kernel_us": round(dec_us, 3),
        "merge_us": round(mrg_us, 3),
        "hbm_frac": round(set_bytes / (win_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
    }
    roofline = {
        "bound": "hbm",
        "achieved": round(set_bytes / (dec_us * 1e-6) / 1e9, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(set_bytes / (dec_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": decode_kernel_label(w0, args.value_dtype),
        "clock": (f"HIP events on the launch stream, mean over a steady-state window of "
                  f"{res['window_launches']} back-to-back launches of the decode kernel"),
        "window_launches": res["window_launches"],
        "kernel_us": round(dec_us, 3),
        "kernel_us_median": round(res["decode_median_us"], 3),
    }
    if args.decode_only:
        qt, qt_median = time_quantizer(sets, args.steps, args.warmup)
        line.update({"quantizer_us": round(qt, 3), "quantizer_us_median": round(qt_median, 3),
                     "quantizer_hbm_frac": round(qbytes / (qt * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        line["roofline"] = roofline
        print(json.dumps(line), flush=True)
        return
    # No shape specialization (the reference bench re-runs at seq_len + 1): every
    # length + 1, so pages end one row into a fresh page and groups one row into
    # a fresh group; the output must be finite and the rate must hold. Timed
    # right after the headline (inputs built before it), then the two lengths
    # in alternating blocks (the same clocks and memory state for both).
    odd_lens = w0["seq_lens"] + 1
    progress("seq_len + 1 check")
    odd = time_decode(odd_sets, args.splits, max(args.steps // 2, 5), args.warmup)
    odd_ok = bool(torch.isfinite(odd["last_out"]).all())
    _, step_a, _ = decode_launchers(sets, args.splits)
    _, step_b, _ = decode_launchers(odd_sets, args.splits)
    base_us, odd_us = interleaved_us(step_a, step_b)
    del odd_sets, step_b
    torch.cuda.empty_cache()
    if not args.no_trace:
        progress("rocprofv3 --kernel-trace child of the decode window")
        tr, err = trace_window(args)
        if tr is not None:
            roofline.update({
                "trace_mean_us": round(tr["trace_mean_us"], 3),
                "trace_median_us": round(tr["trace_median_us"], 3),
                "trace_dispatches": tr["trace_dispatches"],
                "trace_frac": round(set_bytes / (tr["trace_mean_us"] * 1e-6) / 1e9
                                    / HBM_PEAK_GBS, 4),
                "trace_child_event_us": round(tr["child_event_us"], 3),
                "trace_note": "per-dispatch kernel durations (rocprofv3 --kernel-trace) of the "
                              "same window run in a child process; the event figure includes "
                              "the gaps between back-to-back dispatches, the trace figure "
                              "does not"})
        else:
            roofline["trace_error"] = err

    progress("timing the quantizer, append, reference semantics and fake quantization")
    qt, qt_median = time_quantizer(sets, args.steps, args.warmup)
    app = time_append(w0, args.value_dtype, args.steps, args.warmup)
    probe = hbm_probes()
    refcfg = time_reference_config(args.steps, args.warmup)
    refq, refq_host = time_reference_quantizer(args.steps, args.warmup)
    fq = time_fake_quant(args.steps, args.warmup)
    progress("timing the other decode paths and the serving step")
    other = time_other_paths(args)
    other["decode_step"] = time_decode_step(args)
    # One sequence in a 2048-token cache: four splits of whole scale groups,
    # so the step is one launch and the merge.
    other["decode_step_small"] = time_decode_step(args, B=1, H=8, D=128, T=1024,
                                                  max_seq_len=2048)

    q_us = qt

    line.update({
        "quantizer_us": round(q_us, 3),
        "quantizer_us_median": round(qt_median, 3),
        "quantizer_gbs": round(qbytes / (q_us * 1e-6) / 1e9, 2),
        "quantizer_hbm_frac": round(qbytes / (q_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "append_us": app,
        "hbm_probe": probe,
        "reference_config": refcfg,
        "reference_quantizer": refq,
        "fake_quant": fq,
        "other_paths": other,
        "checks": {
            "split_invariance_max_abs": gate,
            "seq_len_plus_1": {
                "pass": odd_ok, "max_tokens": int(odd_lens.max()),
                "decode_us": round(odd["window_us"], 3),
                "hbm_frac": round(odd_bytes / (odd["window_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                  4),
                "interleaved": {"anchor_us": round(base_us, 3), "plus_1_us": round(odd_us, 3),
                                "ratio": round(odd_us / base_us, 4), "rounds": 10,
                                "launches_per_block": INTERLEAVE_BLOCK,
                                "anchor_vs_headline": round(base_us / win_us, 4)}},
        },
        "roofline": roofline,
    })
    if not args.no_pmc:
        progress("rocprofv3 --pmc children (FETCH_SIZE, WRITE_SIZE)")
        traffic, err = pmc_traffic(args)
        if traffic is not None:
            fake = traffic.pop("fake_quant")
            quant = traffic.pop("quantizer")
            for name, t in traffic.pop("reference_quantizer").items():
                rec = line["reference_quantizer"].get(name)
                if rec is None or "fetch_bytes" not in t or "write_bytes" not in t:
                    continue
                rec["traffic"] = round(t["fetch_bytes"] + t["write_bytes"])
                rec["traffic_vs_algorithmic"] = round(rec["traffic"] / rec["bytes"], 4)
                rec["traffic_kernels"] = t["kernels"]
            if quant is not None:
                qt_bytes = round(quant["fetch_bytes"] + quant["write_bytes"])
                line["quantizer_traffic"] = qt_bytes
                line["quantizer_traffic_vs_algorithmic"] = round(qt_bytes / qbytes, 4)
            line["roofline"]["traffic"] = round(traffic["fetch_bytes"] + traffic["write_bytes"])
            line["roofline"]["traffic_detail"] = {k: round(v, 4) for k, v in traffic.items()}
            for name, t in fake.items():
                rec = line["fake_quant"][name]
                rec["traffic"] = round(t["fetch_bytes"] + t["write_bytes"])
                rec["traffic_vs_algorithmic"] = round(rec["traffic"] / rec["bytes"], 4)
        else:
            line["roofline"]["traffic_error"] = err
    if not args.no_cpu:
        progress("CPU baseline (NumPy oracle)")
        st = sets[res["last_set"]]
        base, parity = cpu_baseline(st, res["last_out"], args.cpu_runs, vbytes)
        line["cpu_baseline"] = base
        line["parity"] = parity
        for name, exact in cpu_check_reference_quantizer(refq_host).items():
            line["reference_quantizer"][name]["bit_exact_vs_oracle"] = exact
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
