"""bench.py's guards that need no GPU: a graph run under rocprofv3 (tracing or counters) is
refused before any device work, and more than one GPU is refused with a message."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(args, extra_env):
    env = {k: v for k, v in os.environ.items() if not k.startswith("ROCPROF_")}
    env.update(extra_env)
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], env=env, capture_output=True,
                          text=True, timeout=120)


def test_graph_run_under_the_tracer_is_refused():
    for var in ("ROCPROF_KERNEL_TRACE", "ROCPROF_HIP_RUNTIME_API_TRACE", "ROCPROF_COUNTER_COLLECTION"):
        proc = _bench(["--quick"], {var: "1"})
        assert proc.returncode == 3, (var, proc.stderr)
        assert "rocprofv3" in proc.stderr and var in proc.stderr


def test_more_than_one_gpu_is_refused():
    proc = _bench(["--gpus", "2"], {})
    assert proc.returncode == 2 and "one GPU" in proc.stderr
