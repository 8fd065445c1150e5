"""The C-ABI library builds, loads and exports every entry point include/ferrite_hip.h declares, and the ctypes
binding knows each one (no GPU needed: nothing here computes)."""
import ctypes, pathlib, re
import pytest
from ferrite_amd import lib

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "ferrite_hip.h"


def declared():
  text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
  return sorted(set(re.findall(r"\b(fh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
  names = declared()
  assert "fh_gemv_bfp" in names and "fh_bfp_pack" in names and len(names) >= 10, names


def test_library_exports_every_declared_symbol():
  if not lib.PATH.exists(): pytest.skip("libferrite_hip.so not built")
  raw = ctypes.CDLL(str(lib.PATH))
  missing = [n for n in declared() if not hasattr(raw, n)]
  assert not missing, missing
  assert set(declared()) == set(lib.SIGNATURES), set(declared()) ^ set(lib.SIGNATURES)


def test_errors_without_gpu_work():
  # argument checks happen on the host before any launch: bad shapes come back as ValueError with the reason
  if not lib.PATH.exists(): pytest.skip("libferrite_hip.so not built")
  lib.load()
  assert lib.bfp_bytes(576, 1536, lib.BFP8) == (576 * 1536, 576 * 1536 // 16)
  assert lib.bfp_bytes(576, 1536, lib.BFP4) == (576 * 1536 // 2, 576 * 1536 // 16)
  with pytest.raises(ValueError, match="multiple of 16"):
    lib.bfp_bytes(576, 1530, lib.BFP8)
  with pytest.raises(ValueError, match="null pointer"):
    lib.call("fh_bfp_pack", None, lib.F32, 16, 16, 16, lib.BFP8, lib.AXIS_N, None, None, None)
  with pytest.raises(ValueError):
    lib.call("fh_gemv_bfp", None, lib.F32, 16, 1, 16, 16, None, None, lib.BFP8, None, None, lib.F32, 16, None)
  assert lib.load().fh_version().decode().endswith("gfx950")
  # a KV cache's bytes: fp32 / bf16 elements; a block float's magnitudes then a byte a run of 16 (2 kv heads, 10 rows)
  kb = lib.load().fh_kv_cache_bytes
  assert kb(lib.F32, 2, 10, 64) == 4 * 10 * 64 * 4 and kb(lib.BF16, 2, 10, 64) == 4 * 10 * 64 * 2
  assert kb(lib.BFP8, 2, 10, 128) == 4 * 10 * (128 + 8) and kb(lib.BFP4, 2, 10, 128) == 4 * 10 * (64 + 8)
  assert kb(lib.BFP8, 2, 10, 48) == 0 and kb(7, 2, 10, 64) == 0
