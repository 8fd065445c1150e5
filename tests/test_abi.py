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


def test_tile_layout_and_its_refusals():
  # FH_BF16_T16: the header's value is the binding's, ops' helpers follow the layout's formula (element (r, c) at
  # (r // 16) 16 ld + (c // 8) 128 + (r % 16) 8 + c % 8, whole tiles of 16 rows), and the entry points refuse on the
  # host, before any launch, what the layout does not cover
  import torch
  from ferrite_amd import ops
  assert re.search(r"#define FH_BF16_T16 (\d+)", HEADER.read_text()).group(1) == str(lib.BF16_T16)
  x = (torch.arange(37 * 24, dtype=torch.float32) % 251).view(37, 24)
  t = ops.to_tiles16(x, fill=-1.0)
  flat = t.data.float()
  assert flat.numel() == 48 * 24
  for r in range(37):
    for c in range(24):
      assert flat[(r // 16) * 16 * 24 + (c // 8) * 128 + (r % 16) * 8 + c % 8] == (r * 24 + c) % 251
  assert (flat[2 * 16 * 24:].view(3, 16, 8)[:, 5:, :] == -1).all()  # (rows 37..47 of the last tile: the fill)
  assert torch.equal(t.to_rows(), x.to(torch.bfloat16))
  with pytest.raises(ValueError):
    ops.tiles16(3, 12)  # (columns a multiple of 8)
  if not lib.PATH.exists(): pytest.skip("libferrite_hip.so not built")
  lib.load()
  buf = ctypes.create_string_buffer(1 << 16)
  p = ctypes.addressof(buf)
  # more than 64 rows: the tiled GEMM takes rows only
  with pytest.raises(NotImplementedError, match="FH_BF16_T16"):
    lib.call("fh_gemm_bfp", p, lib.BF16_T16, 64, 65, 64, 16, p, p, lib.BFP8, None, p, lib.F32, 16, None)
  with pytest.raises(NotImplementedError, match="FH_BF16_T16"):
    lib.call("fh_gemm_bfp", p, lib.BF16, 64, 65, 64, 16, p, p, lib.BFP8, None, p, lib.BF16_T16, 16, None)
  # the GEMV writes rows only; fh_rms_rows' tiles need whole groups of 8 columns; the read probe whole 16 bytes
  with pytest.raises(ValueError):
    lib.call("fh_gemv_bfp", p, lib.F32, 64, 1, 64, 16, p, p, lib.BFP8, None, p, lib.BF16_T16, 16, None)
  with pytest.raises(ValueError, match="multiple of 8"):
    lib.call("fh_rms_rows", p, 12, 2, 12, p, ctypes.c_float(1e-5), 0, p, lib.BF16_T16, 12, None)
  with pytest.raises(ValueError):
    lib.call("fh_read_probe", p, 10, p, 1, None)
