"""bench.py's command line on the CPU: it measures one GPU, and a request for
more exits with status 2 and says so before touching the device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    for n in ("2", "8"):
        r = _bench("--gpus", n, "--steps", "1", "--warmup", "0")
        assert r.returncode == 2, (r.returncode, r.stderr)
        assert f"--gpus {n} is not supported" in r.stderr and "one GPU" in r.stderr
        assert r.stdout == ""  # no JSON line


def test_help_lists_the_contract_flags():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in r.stdout
