"""bench.py's command line on the CPU: more than one GPU is refused with a
message and exit status 2 before anything touches a GPU, and the JSON
line's fixed fields are the ones the measurement contract names."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one MI355X" in r.stderr and "--gpus 2" in r.stderr


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 2
    assert "WORLD_SIZE 4" in r.stderr


def test_contract_fields_in_the_line():
    """The fixed keys of the one JSON line, as bench.py writes them."""
    src = open(os.path.join(ROOT, "bench.py")).read()
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert f'"{key}"' in src, key
    for key in ("bound", "achieved", "peak", "frac", "traffic"):
        assert f'"{key}"' in src, key
