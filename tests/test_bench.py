"""bench.py's contract on the CPU: one GPU only, the committed traffic figure it reports, the workloads' shapes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
  r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                     timeout=300, cwd=ROOT)
  assert r.returncode == 2
  assert "one GPU" in r.stderr and not r.stdout.strip()


def test_traffic_is_the_committed_counter_summary():
  import bench
  # the dominant GEMV's HBM bytes a launch (FETCH_SIZE + WRITE_SIZE, calibrated): within 1% of its algorithmic bytes,
  # K N 9/16 of bfp4 weight + x + the norm's weights + y
  t = bench.measured_traffic("gate_up", "c3", 1)
  algorithmic = 4096 * 28672 * 9 // 16 + 4096 * 4 + 4096 * 4 + 14336 * 4
  assert t is not None and abs(t - algorithmic) <= 0.01 * algorithmic, (t, algorithmic)
  assert bench.measured_traffic("gate_up", "c3", 7) is None


def test_config3_is_the_8b_shape():
  import bench
  c, mode, context = bench.config("c3")
  assert (c.dim, c.heads, c.kv, c.layers, c.ffn, c.vocab) == (4096, 32, 8, 32, 14336, 128256)
  assert mode == "experts" and context == 2048  # (attention and output layer bfp8, MLP bfp4)
  c8, mode8, _ = bench.config("c3-bfp8")
  assert mode8 == "bfp8" and c8.dim == c.dim
