"""bench.py's command-line contract on the host: more than one GPU is
refused with a message before anything touches a device."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    for argv, env_world in ((["--gpus", "2"], "1"), (["--gpus", "1"], "8")):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], cwd=ROOT,
                           capture_output=True, text=True, timeout=60,
                           env={"PATH": "/usr/bin:/bin", "WORLD_SIZE": env_world})
        assert r.returncode == 2, r.stderr
        assert "one GPU only" in r.stderr
        assert r.stdout == ""
