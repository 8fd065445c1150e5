"""ctypes loader of the oracle's C restatement of gpt2.bfp (oracle/bfp_c.c, built by oracle/build.py): the same values
as oracle/bfp.py's bfp, as float32, for weights too large for numpy in a test's time.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module; the product (ferrite_amd) never calls it."""
import ctypes
import numpy as np
from oracle import build as _build

_lib = None


def _load():
  global _lib
  if _lib is None:
    if not _build.LIB.exists(): raise RuntimeError(f"{_build.LIB} is not built: run python -m oracle.build")
    lib = ctypes.CDLL(str(_build.LIB))
    for name in ("oracle_bfp_bf16", "oracle_bfp_f32"):
      getattr(lib, name).argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
      getattr(lib, name).restype = None
    _lib = lib
  return _lib


def bfp(a, fmt="bfp8"):
  """gpt2.bfp(a, fmt) (models/gpt2.py:21-32) along the last axis, as float32 (exact): a is float32 values (rounded to
  bf16 first) or uint16 bf16 bits."""
  assert fmt in ("bfp8", "bfp4"), fmt
  a = np.ascontiguousarray(a)
  assert a.shape[-1] % 16 == 0, "runs of 16 along the last axis"
  out = np.empty(a.shape, np.float32)
  if a.dtype == np.uint16: fn = _load().oracle_bfp_bf16
  else:
    a = np.ascontiguousarray(a, np.float32)
    fn = _load().oracle_bfp_f32
  fn(a.ctypes.data, a.size, int(fmt == "bfp4"), out.ctypes.data)
  return out
