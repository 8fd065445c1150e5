"""Parity of the prefill GEMM (fh_gemm_bfp, matrix cores) with the oracle, through the C-ABI. Its arithmetic is the
chip's (ferrite/tensor.py:443-485: the unpacker hands the matrix unit bf16): x, times the RMSNorm weight, rounded to
bf16, the weight's values exact, fp32 sums. So each output is checked twice: against that restatement (numpy in
float64 on the bf16-rounded rows) within fp32 summation's error, and against the float64 oracle on unrounded x within
the north star's bar (max relative error 1e-2, cosine 0.9999). The reference's tests of the same products:
test_matmul_random (test/test_sim.py:325-335, a bf16 output's bound), test_matmul_exact (310-323)."""
import numpy as np
import pytest
import torch
from oracle import bfp as O
from oracle import llama as OL

pytestmark = pytest.mark.gpu


def ops():
  from ferrite_amd import ops as m
  return m


def lib():
  from ferrite_amd import lib as m
  return m


def to_gpu(a, dtype=torch.float32):
  return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def wide(rng, shape):
  return (rng.normal(0, 1, shape) * np.exp(rng.normal(0, 2, shape))).astype(np.float32)


def north_star(got, want, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)


def within(got, want, bound, what):
  err = np.abs(np.asarray(got, np.float64) - want)
  assert (err <= bound).all(), (what, float((err / np.maximum(bound, 1e-300)).max()))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_gemm_shapes(cuda, fmt):
  # row counts around the 128-row tile, N not a multiple of the 128-column tile, K not a multiple of the 64-row step
  rng = np.random.default_rng(11)
  # (up to 64 rows with K a multiple of 64 take the skinny kernel: K split among a workgroup's waves; 3 runs of 16
  # leave its last item one run)
  for M, K, N in ((1, 64, 16), (5, 576, 960), (33, 64, 48), (64, 1536, 576), (16, 4096, 1024), (128, 1536, 576),
                  (200, 96, 2064), (300, 4096, 256)):
    w = wide(rng, (K, N)) * 0.02
    bw = ops().pack(to_gpu(w), fmt)
    wv = O.bfp(w, fmt)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    xb = O.bf16(x).astype(np.float64)
    bound = 1e-5 * (np.abs(xb) @ np.abs(wv)) + 1e-30
    for dtype in (torch.float32, torch.bfloat16):
      y = ops().gemm(to_gpu(x, dtype), bw).cpu().numpy()
      within(y, xb @ wv, bound, (M, K, N, dtype))
      north_star(y, x.astype(np.float64) @ wv, (M, K, N, dtype))
    yb = ops().gemm(to_gpu(x), bw, out_dtype=torch.bfloat16).float().cpu().numpy()
    within(yb, xb @ wv, 2.0 ** -8 * np.abs(xb @ wv) + bound, (M, K, N, "bf16 out"))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_skinny_row_counts(cuda, fmt):
  # every row count around the skinny kernel's 16-row blocks (one, two or four a workgroup: 1-16, 17-32, 33-64), a
  # pass of 64 and a second pass past it (65), with one-run items (N of 3 runs: the last item alone) and pairs of runs
  rng = np.random.default_rng(21)
  K = 320
  for N in (48, 256):
    w = wide(rng, (K, N)) * 0.02
    bw = ops().pack(to_gpu(w), fmt)
    wv = O.bfp(w, fmt)
    for M in (1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 63, 64, 65):
      x = rng.normal(0, 1, (M, K)).astype(np.float32)
      xb = O.bf16(x).astype(np.float64)
      y = ops().gemm(to_gpu(x, torch.bfloat16), bw).cpu().numpy()
      within(y, xb @ wv, 1e-5 * (np.abs(xb) @ np.abs(wv)) + 1e-30, (fmt, N, M))


def test_gemm_exact_integers(cuda):
  # small integers (exact in bf16) times a power of 2 per run: every product and sum exact in fp32, so bit for bit;
  # and x @ I returns x's bf16 values
  rng = np.random.default_rng(12)
  M, K, N = 150, 256, 192
  w = (rng.integers(-7, 8, (K, N)) * 2.0 ** rng.integers(-3, 3, (K, 1))).astype(np.float32)
  x = rng.integers(-4, 5, (M, K)).astype(np.float32)
  for fmt in ("bfp8", "bfp4"):
    y = ops().gemm(to_gpu(x), ops().pack(to_gpu(w), fmt)).cpu().numpy()
    assert np.array_equal(y, (x.astype(np.float64) @ O.bfp(w, fmt)).astype(np.float32)), fmt
  eye = np.eye(128, dtype=np.float32)
  x = rng.normal(0, 1, (131, 128)).astype(np.float32)
  assert np.array_equal(ops().gemm(to_gpu(x), ops().pack(to_gpu(eye))).cpu().numpy(), O.bf16(x))


def test_gemm_rejects(cuda):
  w = ops().pack(to_gpu(np.ones((48, 32), np.float32)))
  with pytest.raises(ValueError, match="multiple of 32"):
    ops().gemm(to_gpu(np.ones((2, 48), np.float32)), w)


@pytest.mark.parametrize("M", [150, 37, 16])
def test_gemm_epilogues(cuda, M):
  # every epilogue over a prompt's rows (150: the tiled kernel), or a decode step of many sequences (37, 16: the
  # skinny one), each row its own place (models/llama.py's prefill, 498-504)
  L = lib()
  rng = np.random.default_rng(13)
  c = OL.model(dim=576, heads=9, kv=3, layers=1, eps=1e-5, theta=10000.0, ffn=1536, places=256)
  x = rng.normal(0, 1, (M, c.dim)).astype(np.float32)
  g = O.bf16(rng.normal(1, 0.1, (1, c.dim)))
  ssq = (x.reshape(M, -1, 16).astype(np.float32) ** 2).sum(-1)
  rs = 1 / np.sqrt(ssq.astype(np.float64).sum(1, keepdims=True) / c.dim + c.eps)
  hb = O.bf16(x * g).astype(np.float64)          # the rows the matrix cores take: bf16(x * w), then times 1/rms
  h = OL.rms(x.astype(np.float64), g, c)         # the oracle's
  # residual, and the sums of squares it leaves
  w = rng.normal(0, 0.02, (c.dim, c.dim)).astype(np.float32)
  wv = O.bfp(w)
  res = rng.normal(0, 1, (M, c.dim)).astype(np.float32)
  y, s = to_gpu(res.copy()), torch.zeros(M, c.dim // 16, device="cuda")
  xb = O.bf16(x).astype(np.float64)
  cp = torch.zeros(M, c.dim, dtype=torch.bfloat16, device="cuda")
  bw = ops().pack(to_gpu(w))
  ops().gemm(to_gpu(x), bw, ops().epilogue(L.EP_RESIDUAL, residual=y, ssq_out=s, copy_bf16=cp), out=y)
  want = res + xb @ wv
  within(y.cpu().numpy(), want, 1e-5 * (np.abs(xb) @ np.abs(wv)) + 1e-6, "residual")
  north_star(y.cpu().numpy(), res + x @ wv, "residual")
  assert np.allclose(s.cpu().numpy(), (y.cpu().numpy().astype(np.float64).reshape(M, -1, 16) ** 2).sum(-1), rtol=1e-5)
  # the rows again in bf16 (nearest even) for the next matmul; the GEMV's epilogue writes the same
  assert np.array_equal(cp.float().cpu().numpy(), O.bf16(y.cpu().numpy()))
  yv, cv = to_gpu(res.copy()), torch.zeros(M, c.dim, dtype=torch.bfloat16, device="cuda")
  ops().gemv(to_gpu(x), bw, ops().epilogue(L.EP_RESIDUAL, residual=yv, copy_bf16=cv), out=yv)
  assert np.array_equal(cv.float().cpu().numpy(), O.bf16(yv.cpu().numpy()))
  with pytest.raises(ValueError):  # a copy is the residual epilogue's
    ops().gemm(to_gpu(x), bw, ops().epilogue(L.EP_STORE, copy_bf16=cv))
  # the copy times the next RMSNorm's weight, and a matmul of those rows with 1/rms alone (ssq_in without norm_w):
  # the same products as the RMSNorm prologue on the fp32 rows, bf16(x w), so the same result
  gw = to_gpu(g.reshape(-1))
  yw, cw, sw = to_gpu(res.copy()), torch.zeros(M, c.dim, dtype=torch.bfloat16, device="cuda"), torch.zeros(M, c.dim // 16, device="cuda")
  ops().gemm(to_gpu(x), bw, ops().epilogue(L.EP_RESIDUAL, residual=yw, ssq_out=sw, copy_bf16=cw, copy_w=gw), out=yw)
  assert np.array_equal(cw.float().cpu().numpy(), O.bf16(yw.cpu().numpy() * g))
  w2 = ops().pack(to_gpu(rng.normal(0, 0.02, (c.dim, 256)).astype(np.float32)))
  a1 = ops().gemm(yw, w2, ops().epilogue(L.EP_STORE, norm_w=gw, ssq_in=sw, eps=c.eps))
  a2 = ops().gemm(cw, w2, ops().epilogue(L.EP_STORE, ssq_in=sw, eps=c.eps))
  assert torch.equal(a1, a2)
  # RMSNorm prologue, store with the argmax pairs
  parts = torch.zeros(M, c.dim // 16, dtype=torch.int64, device="cuda")
  ep = ops().epilogue(L.EP_STORE, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps, argmax_parts=parts)
  y = ops().gemm(to_gpu(x), ops().pack(to_gpu(w)), ep).cpu().numpy()
  within(y, hb @ wv * rs, 1e-5 * (np.abs(hb) @ np.abs(wv)) * rs + 1e-6, "norm")
  north_star(y, h @ wv, "norm")
  assert ops().argmax_parts(parts).cpu().numpy().tolist() == np.argmax(y, 1).tolist()
  # RMSNorm and SwiGLU
  w = rng.normal(0, 0.02, (c.dim, 2 * c.ffn)).astype(np.float32)
  wv = O.bfp(w)
  ep = ops().epilogue(L.EP_SILU_GATE, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps, split=c.ffn)
  y = ops().gemm(to_gpu(x), ops().pack(to_gpu(w)), ep).cpu().numpy()
  gu = hb @ wv * rs
  within(y, OL.glu(gu[:, :c.ffn], gu[:, c.ffn:]), 1e-5 * (np.abs(hb) @ np.abs(wv[:, :c.ffn])) * rs * (1 + np.abs(gu[:, c.ffn:])) + 1e-6, "silu")
  gu = h @ wv
  north_star(y, OL.glu(gu[:, :c.ffn], gu[:, c.ffn:]), "silu")
  # RMSNorm, RoPE on q's and k's heads, k and v into the cache at each row's cache row
  hd, nh = 64, c.heads + 2 * c.kv
  w = rng.normal(0, 0.02, (c.dim, nh * hd)).astype(np.float32)
  wv = O.bfp(w)
  places = rng.permutation(c.places)[:M].astype(np.int32)
  rows = places + 5
  full_cos, full_sin, t = OL.rotary(c, c.places)
  cos, sin = OL.rotary_head(c, c.places)
  for cache_dtype in (torch.float32, torch.bfloat16):
    cache = torch.zeros(2 * c.kv, c.places + 8, hd, dtype=cache_dtype, device="cuda")
    ep = ops().epilogue(L.EP_ROPE_KV, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps, heads=c.heads,
                        kv_heads=c.kv, head_dim=hd, cos_tab=to_gpu(cos), sin_tab=to_gpu(sin), rope_rows=len(cos), places=to_gpu(places, torch.int32),
                        cache_rows=to_gpu(rows, torch.int32), cache=cache,
                        cache_dtype=L.DTYPES["fp32" if cache_dtype == torch.float32 else "bf16"], cache_len=c.places + 8)
    q = ops().gemm(to_gpu(x), ops().pack(to_gpu(w)), ep).cpu().numpy()
    for rows_in, what in ((hb @ wv * rs, "chip"), (h @ wv, "oracle")):
      qkv = OL.merge(OL.rope(OL.split(rows_in, nh), OL.split(full_cos[places], nh), OL.split(full_sin[places], nh), t))
      kv = OL.split(qkv[:, c.heads * hd:], 2 * c.kv)
      got = cache.float().cpu().numpy()
      if what == "chip":
        bound = 1e-5 * (np.abs(hb) @ np.abs(wv)).max() * rs.max() + 1e-6
        within(q, qkv[:, :c.heads * hd], bound, "rope q")
        want = kv if cache_dtype == torch.float32 else O.bf16(kv)
        tol = bound if cache_dtype == torch.float32 else 2 ** -8 * np.abs(kv).max()
        assert np.abs(got[:, rows] - want).max() <= tol, cache_dtype
      else:
        north_star(q, qkv[:, :c.heads * hd], "rope q")
        north_star(got[:, rows], kv, "rope kv")
    mask = np.ones(c.places + 8, bool); mask[rows] = False
    assert not got[:, mask].any(), "only the rows' cache rows written"


@pytest.mark.parametrize("N,pairs", [(33600, False), (51200, False), (35200, True), (51200, True)])
def test_gemm_wide_tiles(cuda, N, pairs):
  # the two-group kernel's 192- and 256-column tiles: on an MI355X's 256 CUs, 200 rows by 2100 runs (33600) or 1100
  # SwiGLU pairs (35200) take 192-column tiles, 3200 runs or 1600 pairs (51200) 256-column ones (the narrower tiles
  # would need a second round they do not fill). bf16 rows against the same values as fp32 rows, which the 4-wave
  # kernel takes (the same products in the same order: bit for bit), and against the oracle on the first and last
  # 1024 columns (or pairs); K = 192, three steps (an odd count: a last step of zero weights)
  L = lib()
  rng = np.random.default_rng(16)
  M, K = 200, 192
  w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
  x = O.bf16(rng.normal(0, 1, (M, K)))
  bw = ops().pack(to_gpu(w))
  ep = (lambda: ops().epilogue(L.EP_SILU_GATE, split=N // 2)) if pairs else (lambda: None)
  a = ops().gemm(to_gpu(x, torch.bfloat16), bw, ep())
  b = ops().gemm(to_gpu(x), bw, ep())
  assert torch.equal(a, b), float((a - b).abs().max())
  y, xb = a.cpu().numpy(), x.astype(np.float64)
  cols = np.r_[0:1024, y.shape[1] - 1024:y.shape[1]]
  if pairs:
    h = N // 2
    g, u = xb @ O.bfp(w[:, cols]), xb @ O.bfp(w[:, h + cols])
    bound = 1e-5 * (np.abs(xb) @ np.abs(O.bfp(w[:, cols]))) * (1 + np.abs(u)) + 1e-6
    within(y[:, cols], OL.glu(g, u), bound, ("silu", N))
  else:
    wv = O.bfp(w[:, cols])
    within(y[:, cols], xb @ wv, 1e-5 * (np.abs(xb) @ np.abs(wv)) + 1e-30, ("store", N))


def test_gemm_agrees_with_gemv(cuda):
  # on rows already in bf16, the matrix cores and the exact-product GEMV differ by summation order only
  rng = np.random.default_rng(14)
  K, N = 4096, 1024
  w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
  bw = ops().pack(to_gpu(w))
  x = O.bf16(rng.normal(0, 1, (8, K)))
  a = ops().gemm(to_gpu(x), bw).cpu().numpy()
  b = ops().gemv(to_gpu(x), bw).cpu().numpy()
  wv = O.bfp(w)
  within(a, b, 2e-5 * (np.abs(x) @ np.abs(wv)), "gemm vs gemv")
