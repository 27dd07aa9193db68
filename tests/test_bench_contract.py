"""bench.py's command-line contract, without a GPU: it measures one GPU and
says so for any other count, and without the HIP extension or a visible
device it fails with a message instead of timing a fallback."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(args, extra_env=None):
    env = dict(os.environ)
    env.update(extra_env or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, cwd=ROOT,
                          env=env, capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench(["--gpus", "2"])
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout.strip() == ""                 # no JSON line for an unsupported count


def test_a_distributed_launch_is_refused():
    r = _bench([], {"WORLD_SIZE": "4"})
    assert r.returncode == 2
    assert "WORLD_SIZE 4" in r.stderr


def test_no_visible_device_fails_loudly():
    # The device is hidden from the child, so this holds on a GPU host too.
    r = _bench(["--steps", "1", "--warmup", "0"],
               {"HIP_VISIBLE_DEVICES": "-1", "CUDA_VISIBLE_DEVICES": "-1"})
    assert r.returncode == 1
    assert "unavailable" in r.stderr
    assert r.stdout.strip() == ""


def test_headline_window_is_steady_state_whatever_the_steps():
    """The roofline figure is timed over at least 400 back-to-back launches in
    20 blocks (the median over blocks then has 20 samples) for any --steps,
    including the driver's short runs."""
    sys.path.insert(0, ROOT)
    import bench
    for steps in (1, 5, 20, 200, 400):
        blocks, per = bench.window_shape(steps)
        assert blocks == 20 and blocks * per >= 400
    blocks, per = bench.window_shape(1000)
    assert blocks == 20 and blocks * per >= 1000
    assert bench.median([3.0, 1.0, 2.0]) == 2.0 and bench.median([4.0, 1.0, 2.0, 3.0]) == 2.5
