"""bench.py's command-line contract on the CPU: one GPU only (N > 1 exits
non-zero with a JSON message), and the arguments the driver passes parse."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1",
                        "--warmup", "0"], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]


def test_arguments_parse():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
        argv = sys.argv
        sys.argv = ["bench.py", "--gpus", "1", "--steps", "7", "--warmup", "2", "--only",
                    "decode,oproj", "--cpu-seconds", "0"]
        try:
            a = bench.parse()
        finally:
            sys.argv = argv
        assert (a.gpus, a.steps, a.warmup, a.only, a.cpu_seconds) == (1, 7, 2, "decode,oproj", 0)
    finally:
        sys.path.remove(str(ROOT))
