"""bench.py's command line on the CPU: a request for more than one GPU is
refused with a message before anything touches a device (this build measures
one GPU; how the path would shard is design only)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("argv,env", [
    (["--gpus", "2"], {}),
    (["--gpus", "8", "--steps", "3"], {}),
    ([], {"WORLD_SIZE": "4"}),
])
def test_bench_refuses_more_than_one_gpu(argv, env):
    e = dict(os.environ, **env)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv], cwd=ROOT, env=e,
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line
