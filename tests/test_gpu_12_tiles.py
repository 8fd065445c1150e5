"""bf16 rows in tiles of 16 rows (FH_BF16_T16), the layout a decode step of many sequences passes between its
matrix-core matmuls, through the C-ABI: every entry point that takes or writes it gives the bits it gives with plain
bf16 rows (the same values, the same products and sums), rows past M in the last tile (filled with NaN here) are never
used, and a matmul on tiles is checked against the oracle as well (the north star's bar). No reference counterpart:
a device layout; parity rides on the row-major path's own tests and the oracle check here."""
import numpy as np
import pytest
import torch
from oracle import bfp as O

pytestmark = pytest.mark.gpu


def ops():
  from ferrite_amd import ops as m
  return m


def lib():
  from ferrite_amd import lib as m
  return m


def bits(t):
  return t.contiguous().view(torch.int16).cpu().numpy() if t.dtype == torch.bfloat16 else t.contiguous().cpu().numpy().view(np.int32)


def same(a, b, what):
  assert np.array_equal(bits(a), bits(b)), what


def test_tile_layout_helpers(cuda):
  # the layout's definition: element (r, c) at (r // 16) 16 cols + (c // 8) 128 + (r % 16) 8 + c % 8
  x = (torch.arange(37 * 24, dtype=torch.float32, device="cuda") % 251).view(37, 24)  # (integers bf16 holds)
  t = ops().to_tiles16(x)
  flat = t.data.float().cpu().numpy()
  for r in (0, 5, 15, 16, 31, 36):
    for c in (0, 7, 8, 23):
      assert flat[(r // 16) * 16 * 24 + (c // 8) * 128 + (r % 16) * 8 + c % 8] == (r * 24 + c) % 251
  assert t.data.numel() == 48 * 24
  same(t.to_rows(), x.to(torch.bfloat16), "to_rows inverts to_tiles16")


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_matmul_tiles_equal_rows(cuda, fmt):
  L = lib()
  rng = np.random.default_rng(41)
  for M, K, N in ((3, 256, 64), (16, 1024, 96), (37, 512, 160), (64, 2048, 128)):
    w = (rng.normal(0, 0.02, (K, N))).astype(np.float32)
    bw = ops().pack(torch.from_numpy(w).cuda(), fmt)
    x = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float32)).cuda().to(torch.bfloat16)
    xt = ops().to_tiles16(x, fill=float("nan"))
    print(f"tiles: {fmt} M={M} K={K} N={N}", flush=True)
    # STORE, fp32 out
    y_rows = ops().gemm(x, bw)
    y_tiles = ops().gemm(xt, bw)
    same(y_tiles, y_rows, ("STORE", M))
    # against the oracle: bf16 x, exact weight values, fp32 sums
    want = x.float().cpu().numpy().astype(np.float64) @ O.bfp(w, fmt).astype(np.float64)
    got = y_tiles.cpu().numpy().astype(np.float64)
    rel = np.abs(got - want).max() / np.abs(want).max()
    cos = (got * want).sum() / (np.linalg.norm(got) * np.linalg.norm(want))
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    # STORE into bf16 tiles
    yt = ops().tiles16(M, N, fill=float("nan"))
    ops().gemm(xt, bw, out=yt)
    same(yt.to_rows(), ops().gemm(x, bw, out_dtype=torch.bfloat16), ("STORE bf16 tiles", M))
    # SiLU * gate into bf16 tiles (down's x in a decode step)
    ep = lambda: ops().epilogue(L.EP_SILU_GATE, split=N // 2)
    ht = ops().tiles16(M, N // 2)
    ops().gemm(xt, bw, ep(), out=ht)
    same(ht.to_rows(), ops().gemm(x, bw, ep(), out_dtype=torch.bfloat16), ("SILU_GATE tiles", M))
    # the residual epilogue's bf16 copy (times the next norm's weight) in tiles
    res = torch.from_numpy(rng.normal(0, 1, (M, N)).astype(np.float32)).cuda()
    cw = torch.from_numpy(rng.normal(1, 0.1, N).astype(np.float32)).cuda()
    y1, y2 = res.clone(), res.clone()
    s1, s2 = torch.zeros(M, N // 16, device="cuda"), torch.zeros(M, N // 16, device="cuda")
    c_rows = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    c_tiles = ops().tiles16(M, N, fill=float("nan"))
    ops().gemm(x, bw, ops().epilogue(L.EP_RESIDUAL, residual=y1, ssq_out=s1, copy_bf16=c_rows, copy_w=cw), out=y1)
    ops().gemm(xt, bw, ops().epilogue(L.EP_RESIDUAL, residual=y2, ssq_out=s2, copy_bf16=c_tiles, copy_w=cw), out=y2)
    same(y2, y1, ("RESIDUAL y", M))
    same(s2, s1, ("RESIDUAL ssq", M))
    same(c_tiles.to_rows(), c_rows, ("RESIDUAL copy tiles", M))


def test_gemv_copy_tiles(cuda):
  # the GEMV's residual copy in tiles, 10 rows: two launches (8 rows, then 2), the second's rows at tile rows 8 and 9
  L = lib()
  rng = np.random.default_rng(42)
  M, K, N = 10, 512, 96
  w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
  bw = ops().pack(torch.from_numpy(w).cuda(), "bfp8")
  x = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float32)).cuda()
  res = torch.from_numpy(rng.normal(0, 1, (M, N)).astype(np.float32)).cuda()
  y1, y2 = res.clone(), res.clone()
  c_rows = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
  c_tiles = ops().tiles16(M, N, fill=float("nan"))
  ops().gemv(x, bw, ops().epilogue(L.EP_RESIDUAL, residual=y1, copy_bf16=c_rows), out=y1)
  ops().gemv(x, bw, ops().epilogue(L.EP_RESIDUAL, residual=y2, copy_bf16=c_tiles), out=y2)
  same(y2, y1, "GEMV y")
  same(c_tiles.to_rows(), c_rows, "GEMV copy tiles")


def test_attention_and_rms_tiles(cuda):
  rng = np.random.default_rng(43)
  B, heads, kv, hd, ctx = 5, 8, 2, 128, 300
  cache = torch.from_numpy(rng.normal(0, 1, (2 * kv, B * ctx, hd)).astype(np.float32)).cuda().to(torch.bfloat16)
  q = torch.from_numpy(rng.normal(0, 1, (B, heads * hd)).astype(np.float32)).cuda()
  places = torch.tensor([299, 0, 63, 64, 200], dtype=torch.int32, device="cuda")
  first = torch.arange(B, dtype=torch.int32, device="cuda") * ctx
  for context in (64, ctx):  # (one chunk: the attention kernel writes o; more: the combine does)
    pl = places.clamp(max=context - 1)
    ws = ops().attention_workspace(B, heads, hd, context)
    o_rows = torch.zeros(B, heads * hd, dtype=torch.bfloat16, device="cuda")
    o_tiles = ops().tiles16(B, heads * hd, fill=float("nan"))
    ops().attention_decode(q, cache, heads, kv, hd, pl, first, context, ws, o=o_rows)
    ops().attention_decode(q, cache, heads, kv, hd, pl, first, context, ws, o=o_tiles)
    same(o_tiles.to_rows(), o_rows, ("attention o tiles", context))
  x = torch.from_numpy(rng.normal(0, 1, (B, 4096)).astype(np.float32)).cuda()
  g = torch.from_numpy(rng.normal(1, 0.1, 4096).astype(np.float32)).cuda()
  r_rows = ops().rms_rows(x, g, 1e-5)
  r_tiles = ops().tiles16(B, 4096, fill=float("nan"))
  ops().rms_rows(x, g, 1e-5, out=r_tiles)
  same(r_tiles.to_rows(), r_rows, "rms_rows tiles")


def test_tiles_refused_past_64_rows(cuda):
  rng = np.random.default_rng(44)
  bw = ops().pack(torch.from_numpy(rng.normal(0, 0.02, (256, 64)).astype(np.float32)).cuda(), "bfp8")
  xt = ops().tiles16(65, 256)
  with pytest.raises(NotImplementedError, match="FH_BF16_T16"):
    ops().gemm(xt, bw)
  with pytest.raises(NotImplementedError, match="FH_BF16_T16"):
    ops().gemm(torch.zeros(65, 256, device="cuda"), bw, out=ops().tiles16(65, 64))
  with pytest.raises(ValueError):  # (the GEMV writes rows only)
    ops().gemv(torch.zeros(2, 256, device="cuda"), bw, out=ops().tiles16(2, 64))
