"""The bench's command-line contract, checked on the CPU: it refuses more than
one GPU before touching any device, and its options include the driver's
(--gpus, --steps, --warmup)."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_is_refused_before_any_device_work():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_options_include_the_driver_contract():
    r = subprocess.run([sys.executable, BENCH, "--help"], capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--workload", "--dtype"):
        assert opt in r.stdout
