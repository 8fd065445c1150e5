"""Parity of the HIP kernels with the CPU oracle on the same seeded inputs, through the C-ABI (ferrite_amd.ops calls
libferrite_hip.so): packing and unpacking bit for bit, the GEMV and each epilogue within fp32 summation's error, decode
attention. Sizes are those the oracle finishes in seconds; the benchmark's shapes appear as properties where numpy would be
slow. The reference's own tests of the same path: test_bfp (test/test_sim.py:371-388), test_matmul_random (325-335),
test_matmul_exact (310-323), test_block_float_cache (2081-2107)."""
import math
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


def wide(rng, shape):  # values whose exponents spread wide within each run (test_sim.py:378)
  return (rng.normal(0, 1, shape) * np.exp(rng.normal(0, 2, shape))).astype(np.float32)


def to_gpu(a, dtype=torch.float32):
  return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def gpu_bytes(t):
  return t.cpu().numpy()


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("src", ["fp32", "bf16"])
def test_pack_bit_exact(cuda, fmt, src):
  rng = np.random.default_rng(5)
  for K, N in ((64, 96), (576, 1536), (100, 48), (1, 16)):
    w = wide(rng, (K, N))
    if src == "bf16": w = O.bf16(w)
    bw = ops().pack(to_gpu(w, torch.float32 if src == "fp32" else torch.bfloat16), fmt)
    q, top = O.bfp_parts(w, fmt)
    mant, exps = O.pack_layout(q, top, fmt)
    assert np.array_equal(gpu_bytes(bw.exps), exps.reshape(-1)), (K, N)
    assert np.array_equal(gpu_bytes(bw.mant), mant.reshape(-1)), (K, N)
    got = ops().dequant(bw).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, O.exact_bf16(q, top, fmt)), (K, N)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_pack_axis_k(cuda, fmt):
  # runs down the columns (FH_AXIS_K): gpt2.bfp(W.T).T, packed as W^T is along N
  rng = np.random.default_rng(6)
  w = wide(rng, (96, 80))
  bw = ops().pack(to_gpu(w), fmt, axis=lib().AXIS_K)
  q, top = O.bfp_parts(w.T, fmt)
  mant, exps = O.pack_layout(q, top, fmt)
  assert np.array_equal(gpu_bytes(bw.mant), mant.reshape(-1)) and np.array_equal(gpu_bytes(bw.exps), exps.reshape(-1))
  got = ops().dequant(bw).view(torch.int16).cpu().numpy().view(np.uint16)
  assert np.array_equal(O.bf16_floats(got).astype(np.float64), O.bfp(w, fmt, axis=0))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_pack_every_value_and_exponent(cuda, fmt):
  # every finite bf16 value under every block exponent at or above its own, 15 to a run behind a carrier that sets the
  # exponent: the GPU's bytes are the oracle's, all ~8.4 million of them
  vals = np.arange(65536, dtype=np.uint32)
  vals = vals[(vals >> 7 & 255) != 255].astype(np.uint16)
  e = vals >> 7 & 255
  rows = []
  for top in range(255):
    sel = vals[e <= top]
    sel = np.concatenate([sel, np.zeros((-sel.size) % 15, np.uint16)]).reshape(-1, 15)
    rows.append(np.concatenate([np.full((sel.shape[0], 1), top << 7, np.uint16), sel], 1))
  bits = np.concatenate(rows)
  w = O.bf16_floats(bits)
  bw = ops().pack(to_gpu(bits.view(np.int16), torch.int16).view(torch.bfloat16), fmt)
  q, top = O.bfp_parts(w, fmt)
  mant, exps = O.pack_layout(q, top, fmt)
  assert np.array_equal(gpu_bytes(bw.exps), exps.reshape(-1))
  assert np.array_equal(gpu_bytes(bw.mant), mant.reshape(-1))


def check_close(got, want, bound, what):
  """max relative error (to the largest |want|) at most 1e-2, cosine at least 0.9999 (the north star's bar), and each
  element within bound (fp32 summation's error)."""
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  err = np.abs(got - want)
  rel = err.max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)
  assert (err <= bound).all(), (what, float((err / np.maximum(bound, 1e-300)).max()))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_gemv_config1(cuda, fmt):
  # benchmark config 1: x[1,576] bf16 ~N(0,1), W[576,1536] ~N(0,0.02) fp32 packed (16 along N, ferrite's), y fp32
  rng = np.random.default_rng(0)
  x = O.bf16(rng.normal(0, 1, (1, 576)))
  w = rng.normal(0, 0.02, (576, 1536)).astype(np.float32)
  bw = ops().pack(to_gpu(w), fmt)
  wv = O.bfp(w, fmt)
  want = O.gemv(x, wv)
  bound = 2e-6 * (np.abs(x) @ np.abs(wv)) + 1e-30
  y = ops().gemv(to_gpu(x), bw).cpu().numpy()  # (x's bf16 values, held in fp32 as every activation is)
  check_close(y, want, bound, fmt)
  with pytest.raises(NotImplementedError):
    ops().gemv(to_gpu(x, torch.bfloat16), bw)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_gemv_shapes_and_batches(cuda, fmt):
  # batch 1..11 (past 8: several launches), K not a multiple of 64, and a K long enough for every wave of a workgroup
  rng = np.random.default_rng(1)
  for K, N in ((64, 16), (100, 48), (576, 960), (1536, 576), (4096, 256)):
    w = wide(rng, (K, N)) * 0.02
    bw = ops().pack(to_gpu(w), fmt)
    wv = O.bfp(w, fmt)
    for batch in (1, 2, 3, 5, 8, 11):
      x = rng.normal(0, 1, (batch, K)).astype(np.float32)
      y = ops().gemv(to_gpu(x), bw).cpu().numpy()
      check_close(y, O.gemv(x, wv), 2e-6 * (np.abs(x) @ np.abs(wv)) + 1e-30, (K, N, batch))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_gemv_config1_blocks_along_k(cuda, fmt):
  # benchmark config 1 as its text states it: W[576,1536] packed with its 16-element blocks along K (each run 16
  # consecutive rows of a column, gpt2.bfp(W.T).T), y = x @ W in fp32 by fh_gemv_bfp_k; against the oracle's
  # bfp(W, axis=0) in float64 within fp32 summation's error (2e-6 of sum |x w|) and the north star's bar; the
  # dequantised weight bit for bit the oracle's; batches up to 11 rows (past 8: two launches), an N off 64 and 16
  L = lib()
  rng = np.random.default_rng(9)
  x = O.bf16(rng.normal(0, 1, (1, 576)))
  w = rng.normal(0, 0.02, (576, 1536)).astype(np.float32)
  bw = ops().pack(to_gpu(w), fmt, axis=L.AXIS_K)
  wv = O.bfp(w, fmt, axis=0)
  assert not np.array_equal(wv, O.bfp(w, fmt))  # (a different block float from ferrite's own, N-blocked one)
  got = ops().dequant(bw).view(torch.int16).cpu().numpy().view(np.uint16)
  assert np.array_equal(O.bf16_floats(got), wv.astype(np.float32)), fmt
  y = ops().gemv(to_gpu(x), bw).cpu().numpy()
  check_close(y, O.gemv(x, wv), 2e-6 * (np.abs(x) @ np.abs(wv)) + 1e-30, ("config 1 along K", fmt))
  for K, N in ((16, 5), (64, 100), (1536, 576), (4096, 256)):
    w = wide(rng, (K, N)) * 0.02
    bw = ops().pack(to_gpu(w), fmt, axis=L.AXIS_K)
    wv = O.bfp(w, fmt, axis=0)
    for batch in (1, 3, 8, 11):
      x = rng.normal(0, 1, (batch, K)).astype(np.float32)
      y = ops().gemv(to_gpu(x), bw).cpu().numpy()
      check_close(y, O.gemv(x, wv), 2e-6 * (np.abs(x) @ np.abs(wv)) + 1e-30, ("along K", K, N, batch))


def test_gemv_along_k_exact_and_epilogues(cuda):
  # integers times a power of 2 per run down each column: every product and partial sum exact, so y is bit for bit;
  # x @ I picks out x exactly; then the residual epilogue (with its sums of squares by 16 columns and a bf16 copy), the
  # RMSNorm prologue and a program epilogue, against numpy on the same values
  L = lib()
  rng = np.random.default_rng(10)
  K, N = 256, 64
  w = (rng.integers(-7, 8, (K, N)) * 2.0 ** rng.integers(-3, 3, (1, N))).astype(np.float32)
  x = rng.integers(-4, 5, (3, K)).astype(np.float32)
  for fmt in ("bfp8", "bfp4"):
    wv = O.bfp(w, fmt, axis=0)
    y = ops().gemv(to_gpu(x), ops().pack(to_gpu(w), fmt, axis=L.AXIS_K)).cpu().numpy()
    assert np.array_equal(y, (x.astype(np.float64) @ wv).astype(np.float32)), fmt
  eye = np.eye(64, dtype=np.float32)
  xe = O.bf16(rng.normal(0, 1, (2, 64)))
  assert np.array_equal(ops().gemv(to_gpu(xe), ops().pack(to_gpu(eye), axis=L.AXIS_K)).cpu().numpy(), xe)
  K, N = 576, 1536
  w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
  bw = ops().pack(to_gpu(w), "bfp8", axis=L.AXIS_K)
  wv = O.bfp(w, "bfp8", axis=0)
  x = rng.normal(0, 1, (2, K)).astype(np.float32)
  res = rng.normal(0, 1, (2, N)).astype(np.float32)
  y, ssq = to_gpu(res.copy()), torch.zeros(2, N // 16, device="cuda")
  copy = torch.zeros(2, N, dtype=torch.bfloat16, device="cuda")
  ops().gemv(to_gpu(x), bw, ops().epilogue(L.EP_RESIDUAL, residual=y, ssq_out=ssq, copy_bf16=copy), out=y)
  want = res + O.gemv(x, wv)
  bound = 2e-6 * (np.abs(x) @ np.abs(wv) + np.abs(res)) + 1e-30
  check_close(y.cpu().numpy(), want, bound, "residual along K")
  g = y.cpu().numpy().astype(np.float64)
  assert np.allclose(ssq.cpu().numpy(), (g * g).reshape(2, -1, 16).sum(-1), rtol=1e-5)
  assert np.array_equal(copy.float().cpu().numpy(), O.bf16(y.cpu().numpy()))
  # the RMSNorm prologue: x * rsqrt(mean(x^2) + eps) * norm_w, from x's sums of squares by 16
  nw = rng.normal(1, 0.1, K).astype(np.float32)
  xs = to_gpu(x)
  ssq_in = to_gpu((x.astype(np.float64) ** 2).reshape(2, -1, 16).sum(-1).astype(np.float32))
  y = ops().gemv(xs, bw, ops().epilogue(L.EP_STORE, norm_w=to_gpu(nw), ssq_in=ssq_in, eps=1e-5)).cpu().numpy()
  c = OL.model(dim=K, eps=1e-5)
  xn = OL.rms(x.astype(np.float64), nw.astype(np.float64), c)
  check_close(y, xn @ wv, 4e-6 * (np.abs(xn) @ np.abs(wv)) + 1e-30, "RMSNorm prologue along K")


def test_gemv_exact_integers(cuda):
  # small integers times a power of 2 per run: every product and partial sum exact in fp32, so y is bit for bit
  # (test_matmul_exact's idea, test/test_sim.py:310-323); and x @ I picks out x's columns exactly
  rng = np.random.default_rng(2)
  K, N = 256, 64
  w = (rng.integers(-7, 8, (K, N)) * 2.0 ** rng.integers(-3, 3, (K, 1))).astype(np.float32)
  x = rng.integers(-4, 5, (3, K)).astype(np.float32)
  for fmt in ("bfp8", "bfp4"):
    wv = O.bfp(w, fmt)
    y = ops().gemv(to_gpu(x), ops().pack(to_gpu(w), fmt)).cpu().numpy()
    assert np.array_equal(y, (x.astype(np.float64) @ wv).astype(np.float32)), fmt
  eye = np.eye(64, dtype=np.float32)
  x = O.bf16(rng.normal(0, 1, (2, 64)))
  assert np.array_equal(ops().gemv(to_gpu(x), ops().pack(to_gpu(eye))).cpu().numpy(), x)


def test_epilogues(cuda):
  L = lib()
  rng = np.random.default_rng(3)
  c = OL.model(dim=576, heads=9, kv=3, layers=1, eps=1e-5, theta=10000.0, ffn=1536, places=64)
  for batch in (1, 2, 3, 4, 6):  # (paired runs take 4 rows a launch: 6 is two launches)
    x = rng.normal(0, 1, (batch, c.dim)).astype(np.float32)
    g = O.bf16(rng.normal(1, 0.1, (1, c.dim)))
    ssq = (x.reshape(batch, -1, 16).astype(np.float32) ** 2).sum(-1)
    # residual, and the sums of squares it leaves
    w = rng.normal(0, 0.02, (c.dim, c.dim)).astype(np.float32)
    wv = O.bfp(w)
    res = rng.normal(0, 1, (batch, c.dim)).astype(np.float32)
    y, s = to_gpu(res.copy()), torch.zeros(batch, c.dim // 16, device="cuda")
    ops().gemv(to_gpu(x), ops().pack(to_gpu(w)), ops().epilogue(L.EP_RESIDUAL, residual=y, ssq_out=s), out=y)
    want = res + O.gemv(x, wv)
    check_close(y.cpu().numpy(), want, 2e-6 * (np.abs(x) @ np.abs(wv)) + 1e-6, "residual")
    assert np.allclose(s.cpu().numpy(), (want.reshape(batch, -1, 16) ** 2).sum(-1), rtol=1e-5)
    # RMSNorm prologue and SwiGLU
    w = rng.normal(0, 0.02, (c.dim, 2 * c.ffn)).astype(np.float32)
    wv = O.bfp(w)
    ep = ops().epilogue(L.EP_SILU_GATE, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps, split=c.ffn)
    y = ops().gemv(to_gpu(x), ops().pack(to_gpu(w)), ep).cpu().numpy()
    h = OL.rms(x.astype(np.float64), g, c)
    gu = h @ wv
    want = OL.glu(gu[:, :c.ffn], gu[:, c.ffn:])
    check_close(y, want, 1e-5 * (np.abs(h) @ np.abs(wv[:, :c.ffn])) * (1 + np.abs(gu[:, c.ffn:])) + 1e-6, "silu")
    # RMSNorm, RoPE on q's and k's heads, k and v into the cache at each row's place
    hd, nh = 64, c.heads + 2 * c.kv
    w = rng.normal(0, 0.02, (c.dim, nh * hd)).astype(np.float32)
    wv = O.bfp(w)
    places = rng.permutation(60)[:batch].astype(np.int32)
    rows = places + 3
    for cache_dtype in (torch.float32, torch.bfloat16):
      cache = torch.zeros(2 * c.kv, 64, hd, dtype=cache_dtype, device="cuda")
      cos, sin = OL.rotary_head(c, c.places)
      ep = ops().epilogue(L.EP_ROPE_KV, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps, heads=c.heads,
                          kv_heads=c.kv, head_dim=hd, cos_tab=to_gpu(cos), sin_tab=to_gpu(sin), rope_rows=len(cos), places=to_gpu(places, torch.int32),
                          cache_rows=to_gpu(rows, torch.int32), cache=cache, cache_dtype=L.DTYPES["fp32" if cache_dtype == torch.float32 else "bf16"],
                          cache_len=64)
      q = ops().gemv(to_gpu(x), ops().pack(to_gpu(w)), ep).cpu().numpy()
      full_cos, full_sin, t = OL.rotary(c, c.places)
      qkv = OL.merge(OL.rope(OL.split(h @ wv, nh), OL.split(full_cos[places], nh), OL.split(full_sin[places], nh), t))
      bound = 1e-5 * np.abs(qkv).max() + 1e-6
      check_close(q, qkv[:, :c.heads * hd], np.full(q.shape, bound), "rope q")
      kv = OL.split(qkv[:, c.heads * hd:], 2 * c.kv)  # (2 kv, batch, hd)
      got = cache.float().cpu().numpy()
      want = kv if cache_dtype == torch.float32 else O.bf16(kv)
      tol = bound if cache_dtype == torch.float32 else 2 ** -8 * np.abs(kv).max()
      assert np.abs(got[:, rows] - want).max() <= tol, cache_dtype
      mask = np.ones(64, bool); mask[rows] = False
      assert not got[:, mask].any(), "only the rows' places written"


@pytest.mark.parametrize("hd,heads,kv", [(64, 9, 3), (128, 32, 8), (256, 16, 1)])
def test_attention_decode(cuda, hd, heads, kv):
  # rows of a batch at different places (one chunk, several, a chunk's edge), each over its own slot of the cache, a
  # key head shared by 3, 4 and 16 query heads, against numpy's softmax(q k^T / sqrt(hd) + mask) v (models/llama.py:141-142)
  rng = np.random.default_rng(4)
  part, batch = 300, 4
  places = np.array([0, 63, 64, 299], np.int32)
  first = np.arange(batch, dtype=np.int32) * part
  cache = rng.normal(0, 1, (2 * kv, batch * part, hd)).astype(np.float32)
  q = rng.normal(0, 1, (batch, heads * hd)).astype(np.float32)
  ws = ops().attention_workspace(batch, heads, hd, part)
  for cd in (torch.float32, torch.bfloat16):
    cv = cache if cd == torch.float32 else O.bf16(cache)
    o = ops().attention_decode(to_gpu(q), to_gpu(cache, cd), heads, kv, hd, to_gpu(places, torch.int32),
                               to_gpu(first, torch.int32), part, ws).cpu().numpy()
    # o in bf16 (the matrix cores' rows): the fp32 result rounded to nearest even, bit for bit (one chunk, combined)
    ob = torch.empty(q.shape, dtype=torch.bfloat16, device="cuda")
    ops().attention_decode(to_gpu(q), to_gpu(cache, cd), heads, kv, hd, to_gpu(places, torch.int32),
                           to_gpu(first, torch.int32), part, ws, o=ob)
    assert torch.equal(ob.cpu(), torch.from_numpy(o).to(torch.bfloat16)), cd
    for b in range(batch):
      n = places[b] + 1
      k = np.repeat(cv[:kv, first[b]:first[b] + n], heads // kv, 0)
      v = np.repeat(cv[kv:, first[b]:first[b] + n], heads // kv, 0)
      qq = q[b].reshape(heads, 1, hd).astype(np.float64)
      want = (OL.softmax(qq @ k.swapaxes(-1, -2) / math.sqrt(hd)) @ v).reshape(-1)
      assert np.abs(o[b] - want).max() <= 1e-5 * np.abs(want).max() + 1e-6, (cd, b)
  # the same call again gives the same result
  o2 = ops().attention_decode(to_gpu(q), to_gpu(cache, torch.bfloat16), heads, kv, hd, to_gpu(places, torch.int32),
                              to_gpu(first, torch.int32), part, ws).cpu().numpy()
  assert np.array_equal(o, o2)


@pytest.mark.parametrize("hd,heads,kv", [(64, 9, 3), (128, 32, 8), (128, 8, 2)])
def test_attention_decode_short_contexts(cuda, hd, heads, kv):
  # contexts of 2-4 chunks of 64 (a row in one workgroup, a group of waves a chunk, the parts combined in LDS: no
  # second kernel), rows ending in each chunk and on their edges, against numpy; fp32 and bf16 caches, and bf16 o
  # bit for bit the fp32 result rounded
  rng = np.random.default_rng(9 + hd + heads)
  for context in (65, 128, 129, 192, 256):
    batch = 5
    places = np.array([0, 63, 64, context - 2, context - 1], np.int32)
    first = np.arange(batch, dtype=np.int32) * context
    cache = rng.normal(0, 1, (2 * kv, batch * context, hd)).astype(np.float32)
    q = rng.normal(0, 1, (batch, heads * hd)).astype(np.float32)
    ws = ops().attention_workspace(batch, heads, hd, context)
    for cd in (torch.float32, torch.bfloat16):
      cv = cache if cd == torch.float32 else O.bf16(cache)
      args = (heads, kv, hd, to_gpu(places, torch.int32), to_gpu(first, torch.int32), context, ws)
      o = ops().attention_decode(to_gpu(q), to_gpu(cache, cd), *args).cpu().numpy()
      ob = ops().attention_decode(to_gpu(q), to_gpu(cache, cd), *args, o=torch.empty(q.shape, dtype=torch.bfloat16, device="cuda"))
      assert torch.equal(ob.cpu(), torch.from_numpy(o).to(torch.bfloat16)), (context, cd)
      for b in range(batch):
        n = places[b] + 1
        k = np.repeat(cv[:kv, first[b]:first[b] + n], heads // kv, 0)
        v = np.repeat(cv[kv:, first[b]:first[b] + n], heads // kv, 0)
        qq = q[b].reshape(heads, 1, hd).astype(np.float64)
        want = (OL.softmax(qq @ k.swapaxes(-1, -2) / math.sqrt(hd)) @ v).reshape(-1)
        assert np.abs(o[b] - want).max() <= 1e-5 * np.abs(want).max() + 1e-6, (context, cd, b)


@pytest.mark.parametrize("hd,heads,kv,batch,part", [(128, 32, 8, 16, 1000), (64, 9, 3, 64, 600)])
def test_attention_decode_many_rows(cuda, hd, heads, kv, batch, part):
  # many rows x key heads: few enough workgroups that each walks several chunks of its row (online softmax across
  # them; a bf16 or block-float cache takes the matrix cores, q and p in two bf16 terms each), rows shorter than the
  # workgroups sharing them, ending inside a chunk and at its edge; a block float's values read bit for bit as the
  # same values in a bf16 cache
  rng = np.random.default_rng(5 + hd)
  places = rng.integers(0, part, batch).astype(np.int32)
  places[:6] = [0, 1, 63, 64, part - 1, part - 2]
  first = (np.arange(batch, dtype=np.int32) * part)[::-1].copy()  # (slots in another order than the rows)
  cache = O.bf16(rng.normal(0, 1, (2 * kv, batch * part, hd)))
  q = rng.normal(0, 1, (batch, heads * hd)).astype(np.float32)
  ws = ops().attention_workspace(batch, heads, hd, part)
  args = (heads, kv, hd, to_gpu(places, torch.int32), to_gpu(first, torch.int32), part, ws)
  for cd in (torch.bfloat16, torch.float32):
    o = ops().attention_decode(to_gpu(q), to_gpu(cache, cd), *args).cpu().numpy()
    ob = ops().attention_decode(to_gpu(q), to_gpu(cache, cd), *args, o=torch.empty(q.shape, dtype=torch.bfloat16, device="cuda"))
    assert torch.equal(ob.cpu(), torch.from_numpy(o).to(torch.bfloat16)), cd  # (bf16 o: fp32's rounded to nearest even)
    for b in range(batch):
      n = places[b] + 1
      k = np.repeat(cache[:kv, first[b]:first[b] + n], heads // kv, 0)
      v = np.repeat(cache[kv:, first[b]:first[b] + n], heads // kv, 0)
      qq = q[b].reshape(heads, 1, hd).astype(np.float64)
      want = (OL.softmax(qq @ k.swapaxes(-1, -2) / math.sqrt(hd)) @ v).reshape(-1)
      assert np.abs(o[b] - want).max() <= 1e-5 * np.abs(want).max() + 1e-6, (cd, b, places[b])
  for fmt in ("bfp8", "bfp4"):
    same = O.bfp(cache, fmt).astype(np.float32)
    c = ops().kv_cache(2 * kv, batch * part, hd, fmt)
    qv, top = O.bfp_parts(cache, fmt)
    mant = qv.astype(np.int8).view(np.uint8).reshape(-1) if fmt == "bfp8" else \
        ((qv[..., 0::2] & 15) | ((qv[..., 1::2] & 15) << 4)).astype(np.uint8).reshape(-1)
    c.data.copy_(torch.from_numpy(np.concatenate([mant, top.astype(np.uint8).reshape(-1)])).cuda())
    got = ops().attention_decode(to_gpu(q), c, *args).cpu()
    want = ops().attention_decode(to_gpu(q), to_gpu(same, torch.bfloat16), *args).cpu()
    assert torch.equal(got, want), fmt


def test_embed_and_argmax(cuda):
  rng = np.random.default_rng(7)
  table = O.bf16(rng.normal(0, 1, (100, 64)))
  ids = np.array([5, 99, 0], np.int32)
  x, ssq = ops().embed_rows(to_gpu(table, torch.bfloat16), to_gpu(ids, torch.int32))
  assert np.array_equal(x.cpu().numpy(), table[ids])
  assert np.allclose(ssq.cpu().numpy(), (table[ids].reshape(3, -1, 16) ** 2).sum(-1), rtol=1e-6)
  v = rng.normal(0, 1, (3, 50000)).astype(np.float32)
  v[1, 7] = v[1, 70] = v[1].max() + 1  # a tie: the first
  v[2, :] = 0
  assert ops().argmax_rows(to_gpu(v)).cpu().numpy().tolist() == np.argmax(v, 1).tolist()
  # the same picks from a GEMV epilogue's per-run pairs: y = x @ I holds x, ties included
  from ferrite_amd import lib as L
  x = v[:, :4096].copy()
  x[0, 100] = x[0, 3000] = x[0].max() + 1
  eye = ops().pack(to_gpu(np.eye(4096, dtype=np.float32)))
  parts = torch.zeros(3, 4096 // 16, dtype=torch.int64, device="cuda")
  y = ops().gemv(to_gpu(x), eye, ops().epilogue(L.EP_STORE, argmax_parts=parts))
  assert np.array_equal(y.cpu().numpy(), x)
  assert ops().argmax_parts(parts).cpu().numpy().tolist() == np.argmax(x, 1).tolist()
