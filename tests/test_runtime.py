"""The Runtime's wait and profile (ferrite/runtime.py:416-428, 473-484) on the host, with stand-in events: a launch that
never finishes raises TimeoutError naming it, launches that keep finishing do not, however long they take in all, and
profile sums each name's times. No GPU: every event here is a stand-in, and nothing is launched."""
import time
import pytest
from ferrite_amd.tensor import Runtime


class Event:
  """A stand-in for a torch.cuda.Event: done once `at` (a time.monotonic() value) has passed; ms of elapsed time."""
  def __init__(self, at=None, ms=0.0): self.at, self.ms = at, ms
  def query(self): return self.at is not None and time.monotonic() >= self.at
  def elapsed_time(self, end): return end.ms - self.ms


def runtime():
  rt = Runtime("cpu")  # (no stream: only the stand-in events are waited for)
  assert rt.stream is None
  return rt


def queue(rt, name, end, start=None, nbytes=None):
  rt.launches += 1
  rt.queued.append((rt.launches, name, end))
  rt.times[rt.launches % rt.TIMES] = (rt.launches, name, start or Event(0, 0.0), end, nbytes)


def test_wait_times_out_naming_the_launch():
  rt = runtime()
  queue(rt, "pack", Event(0))
  queue(rt, "matmul", Event(None))  # never finishes
  queue(rt, "map", Event(None))
  t0 = time.monotonic()
  with pytest.raises(TimeoutError, match=r"launch 2 \(matmul\), 1 queued behind it"):
    rt.wait(timeout=0.2)
  assert 0.2 <= time.monotonic() - t0 < 2


def test_wait_so_long_as_launches_keep_finishing():
  # five launches 0.1 s apart take 0.5 s in all, more than the timeout, but none is late: no error
  rt = runtime()
  now = time.monotonic()
  for i in range(5): queue(rt, f"k{i}", Event(now + 0.1 * (i + 1)))
  rt.wait(timeout=0.25)
  assert not rt.queued and time.monotonic() - now >= 0.5


def test_profile_by_name():
  rt = runtime()
  queue(rt, "matmul", Event(0, 5.0), Event(0, 2.0))     # 3 ms
  since = rt.launches
  queue(rt, "matmul", Event(0, 10.0), Event(0, 6.0))    # 4 ms
  queue(rt, "map", Event(0, 1.5), Event(0, 1.0))        # 0.5 ms
  queue(rt, "matmul", Event(0, 12.0), Event(0, 11.0))   # 1 ms
  got = rt.profile(since)
  assert [(n, k, round(us)) for n, k, us, b in got] == [("matmul", 2, 5000), ("map", 1, 500)] and all(b is None for *_, b in got)


def test_profile_bytes_by_name():
  # each launch's counted bytes summed by name (ferrite's profile reports bytes read a name); a name with a launch the
  # host did not count reports None
  rt = runtime()
  since = rt.launches
  queue(rt, "matmul", Event(0, 4.0), Event(0, 1.0), nbytes=1000)
  queue(rt, "matmul", Event(0, 8.0), Event(0, 6.0), nbytes=24)
  queue(rt, "map", Event(0, 1.5), Event(0, 1.0), nbytes=8)
  queue(rt, "map", Event(0, 2.5), Event(0, 2.0))
  got = {n: (k, b) for n, k, us, b in rt.profile(since)}
  assert got == {"matmul": (2, 1024), "map": (2, None)}


def test_queue_drains_without_wait():
  # launches already done leave the queue as new ones come: a loop of launches with no wait() keeps a bounded queue
  rt = runtime()
  for i in range(rt.TIMES + 50): queue(rt, "map", Event(0))
  assert len(rt.queued) == rt.TIMES + 50  # (queue() is the bookkeeping alone; run()'s drain is what is checked next)
  class Stream:
    def query(self): return True
  rt.stream = Stream()
  import torch
  real = torch.cuda.stream, torch.cuda.is_current_stream_capturing, torch.cuda.Event
  class Ev:
    def __init__(self, **k): pass
    def record(self, s): pass
    def query(self): return True
  try:
    torch.cuda.stream = lambda s: __import__("contextlib").nullcontext()
    torch.cuda.is_current_stream_capturing = lambda: False
    torch.cuda.Event = Ev
    rt.run(lambda: None, "map", 8)
  finally:
    torch.cuda.stream, torch.cuda.is_current_stream_capturing, torch.cuda.Event = real
  assert len(rt.queued) == rt.TIMES
