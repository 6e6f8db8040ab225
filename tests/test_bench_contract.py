"""bench.py's command-line contract, checked without a GPU: the one-GPU build
refuses --gpus N > 1 with a message (before touching torch or the device) and
documents its flags."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    p = _bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert p.returncode != 0
    assert "one GPU" in p.stderr and "--gpus 2" in p.stderr
    assert p.stdout.strip() == ""   # no JSON line for a refused run


def test_help_lists_the_driver_flags():
    p = _bench("--help")
    assert p.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in p.stdout
