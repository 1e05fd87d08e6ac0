"""bench.py's command-line contract, the parts that need no GPU: more than one GPU is refused with a
message and no JSON line before anything touches a device, and the defaults are one GPU with a
step / warm-up count the driver can run within minutes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""                       # no JSON line for a refused run


def test_default_arguments(monkeypatch):
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    a = bench.parse()
    assert (a.gpus, a.steps, a.warmup) == (1, 200, 20)
    assert (a.batch, a.ctx) == (32, 65536)      # the headline workload: bs32, 64K context
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "7", "--warmup", "3"])
    a = bench.parse()
    assert (a.steps, a.warmup) == (7, 3)
