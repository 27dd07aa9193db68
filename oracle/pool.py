"""The paged oracle over every stream of a workload, spread over host cores.

Test infrastructure only (see ``oracle/__init__.py``): the callers are the
GPU parity tests and the ``cpu_baseline`` leg of ``bench.py``.

``paged_oracle_all`` evaluates, for every (sequence, kv-head) stream of a
paged workload, the float32 page-loop oracle (``paged_decode_ref``, the
reference page loop src/flash_decode_ref.py:30-139 per stream) and the
float64 arbiter (``paged_decode_f64``, tests/test_pallas_flash_decode.py:53-78),
and, when the dense keys are given, re-quantizes every stream with
``quantize_groups_ref`` (src/quantize_int4_ref.py:23-84 per 128-token group,
src/int4_pack.py:14-29) and compares the result with the given scales,
zero-points and packed pages bit for bit. The arrays are saved once to a
temporary directory and memory-mapped by one spawned process per core (fresh
interpreters that never touch a GPU), each taking (sequence, kv-head block)
tasks with BLAS limited to one thread, so the results are those of the
one-process functions (the same calls on the same slices).
"""

import multiprocessing
import os
import tempfile
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np

_KEYS = ("q", "kp", "v", "s", "z", "pt", "sl")


def _one_thread():
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        return None
    return threadpool_limits(limits=1)


def _task(path, b, h0, h1, f64, keys, page_size, group_size):
    """Oracle outputs of sequence b, kv-heads h0..h1-1, and the number of
    those streams whose quantized keys differ from the stored ones."""
    from .attention import paged_decode_f64, paged_decode_ref
    from .quantize import pack_int4, quantize_groups_ref
    names = _KEYS + (("k",) if keys else ())
    a = {k: np.load(os.path.join(path, k + ".npy"), mmap_mode="r") for k in names}
    rep = a["q"].shape[1] // a["kp"].shape[1]
    n = int(a["sl"][b])
    args = (np.asarray(a["q"][b:b + 1, h0 * rep:h1 * rep]), a["kp"][:, h0:h1],
            a["v"][:, h0:h1], np.asarray(a["s"][b:b + 1, h0:h1]),
            np.asarray(a["z"][b:b + 1, h0:h1]), np.asarray(a["pt"][b:b + 1]),
            np.asarray(a["sl"][b:b + 1]), page_size, group_size)
    ctx = _one_thread()
    try:
        if ctx is not None:
            ctx.__enter__()
        o32 = paged_decode_ref(*args)[0]
        o64 = paged_decode_f64(*args)[0] if f64 else None
        bad = 0
        if keys and n > 0:
            qr, sr, zr = quantize_groups_ref(np.asarray(a["k"][b:b + 1, h0:h1, :n]),
                                             np.array([n], np.int32), group_size)
            ng = (n + group_size - 1) // group_size
            npg = (n + page_size - 1) // page_size
            want = pack_int4(qr[0])                                  # [Hs, n, D/2]
            got = np.asarray(a["kp"][np.asarray(a["pt"][b, :npg]), h0:h1])
            got = got.transpose(1, 0, 2, 3).reshape(h1 - h0, npg * page_size, -1)[:, :n]
            for i in range(h1 - h0):
                same = (np.array_equal(sr[0, i, :ng], a["s"][b, h0 + i, :ng]) and
                        np.array_equal(zr[0, i, :ng], a["z"][b, h0 + i, :ng]) and
                        np.array_equal(want[i], got[i]))
                bad += 0 if same else 1
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    return b, h0 * rep, o32, o64, bad


def default_workers():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def paged_oracle_all(arrays, workers=None, f64=True, page_size=16, group_size=128):
    """Oracle over every stream of a paged workload.

    arrays: dict of host arrays q [B, Hq, D] float32, kp [P, Hkv, page, D/2]
    uint8, v [P, Hkv, page, D] float32, s and z [B, Hkv, G, D] float32, pt
    [B, max_pages] int32, sl [B] int32 and, optionally, the dense keys k
    [B, Hkv, T, D] float32 that kp, s and z were quantized from.

    Returns a dict: o32 [B, Hq, D] float32, o64 [B, Hq, D] float64 (None
    when f64 is False), key_mismatch (streams whose re-quantized keys differ
    from kp/s/z; None without k), workers, seconds (wall time of the tasks).
    """
    workers = workers or default_workers()
    B, Hq, D = arrays["q"].shape
    Hkv = arrays["kp"].shape[1]
    keys = "k" in arrays
    per = max(1, (B * Hkv + 4 * workers - 1) // (4 * workers))
    tasks = [(b, h, min(h + per, Hkv)) for b in range(B) for h in range(0, Hkv, per)]
    o32 = np.zeros((B, Hq, D), np.float32)
    o64 = np.zeros((B, Hq, D), np.float64) if f64 else None
    bad = 0
    with tempfile.TemporaryDirectory(prefix="fdi4_oracle_") as d:
        for k in _KEYS + (("k",) if keys else ()):
            np.save(os.path.join(d, k + ".npy"), np.ascontiguousarray(arrays[k]))
        ctx = multiprocessing.get_context("spawn")
        with ProcessPoolExecutor(max_workers=workers, mp_context=ctx) as pool:
            t0 = time.perf_counter()
            futs = [pool.submit(_task, d, b, h0, h1, f64, keys, page_size, group_size)
                    for b, h0, h1 in tasks]
            for f in futs:
                b, q0, r32, r64, nbad = f.result()
                o32[b, q0:q0 + r32.shape[0]] = r32
                if f64:
                    o64[b, q0:q0 + r64.shape[0]] = r64
                bad += nbad
            seconds = time.perf_counter() - t0
    return dict(o32=o32, o64=o64, key_mismatch=bad if keys else None, workers=workers,
                seconds=seconds)
