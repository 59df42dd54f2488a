"""bench.py's command line on a host without a GPU: more than one GPU is
refused with a message and exit status 2, and with no HIP device the run
fails loudly instead of printing a result line from some other path."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    r = _bench("--gpus", n)
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU" in r.stderr and f"--gpus {n}" in r.stderr


def _json_lines(text):
    out = []
    for line in text.splitlines():
        try:
            out.append(json.loads(line))
        except ValueError:
            pass
    return out


def test_no_device_fails_loudly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present on this host")
    r = _bench("--quick", "--no-cpu", "--steps", "1", "--warmup", "0")
    assert r.returncode != 0
    assert _json_lines(r.stdout) == []
    assert "no HIP device" in r.stderr
