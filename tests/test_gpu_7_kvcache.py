"""A KV cache in a block float (bfp8 or bfp4; models/llama.py:127-128), the reference's test_block_float_cache
(test/test_sim.py:2081-2107) on the GPU, through the C-ABI. The qkv matmul's FH_EP_ROPE_KV epilogue puts each key and
value row's runs of 16 rounded from bf16 as numpy's bfp rounds them (oracle/bfp.py's bfp_parts, pinned against the
packer's golden vectors): bit for bit, on every matmul path (the GEMV, the skinny matrix-core kernel, the tiled GEMM).
Decode and prefill attention read the cache in place: bit for bit what they give over a bf16 cache holding the same
values (the reference's own bar). Then a whole decode and a prefill with a bfp8 and a bfp4 cache against the numpy
model, whose attention rounds its cache by the same bfp (oracle/llama.py, llama.py:127-128)."""
import numpy as np
import pytest
import torch
from oracle import bfp as O
from oracle import llama as OL

pytestmark = pytest.mark.gpu

FMTS = ("bfp8", "bfp4")


def ops():
  from ferrite_amd import ops as m
  return m


def lib():
  from ferrite_amd import lib as m
  return m


def to_gpu(a, dtype=torch.float32):
  return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def cache_bytes(values, fmt):
  """values [planes][rows][hd] as a block-float cache's bytes (fh_kv_cache_bytes' layout): numpy's bfp parts, the
  magnitudes of every row (bfp4: columns 2i, 2i + 1 in a byte's low, high nibble), then every row's exponents."""
  q, top = O.bfp_parts(values, fmt)
  if fmt == "bfp8":
    mant = q.astype(np.int8).view(np.uint8).reshape(-1)
  else:
    mant = ((q[..., 0::2] & 15) | ((q[..., 1::2] & 15) << 4)).astype(np.uint8).reshape(-1)
  return np.concatenate([mant, top.astype(np.uint8).reshape(-1)])


def cache_parts(cache):
  """A BfpCache's (q, top) read back from its bytes: q [planes][rows][hd], top [planes][rows][hd / 16]."""
  P, R, hd = cache.shape
  b = cache.data.cpu().numpy()
  nm = P * R * (hd if cache.fmt == "bfp8" else hd // 2)
  assert b.size == nm + P * R * hd // 16
  m = b[:nm]
  if cache.fmt == "bfp8":
    q = m.view(np.int8).astype(np.int32).reshape(P, R, hd)
  else:
    lo, hi = (m & 15).astype(np.int32), (m >> 4).astype(np.int32)
    q = np.stack([np.where(lo > 7, lo - 16, lo), np.where(hi > 7, hi - 16, hi)], -1).reshape(P, R, hd)
  return q, b[nm:].astype(np.int32).reshape(P, R, hd // 16)


def wide_rows(rng, shape):
  """bf16 rows spread over 5 decades a row (test_sim.py:2094), every run of 16 with values far below its largest."""
  return O.bf16(rng.normal(0, 2, shape) * 10.0 ** rng.integers(-3, 3, shape[:-1] + (1,)))


def test_cache_helpers_round_trip(cuda):
  # the tests' own layout helpers against the library's size, and each other
  rng = np.random.default_rng(70)
  for fmt in FMTS:
    v = wide_rows(rng, (4, 10, 64))
    c = ops().kv_cache(4, 10, 64, fmt)
    assert c.data.numel() == lib().load().fh_kv_cache_bytes(lib().DTYPES[fmt], 2, 10, 64) == cache_bytes(v, fmt).size
    c.data.copy_(to_gpu(cache_bytes(v, fmt), torch.uint8))
    q, top = cache_parts(c)
    wq, wt = O.bfp_parts(v, fmt)
    assert np.array_equal(q, wq) and np.array_equal(top, wt)


def qkv_case(rng, hd, heads, kv, M, dim=512):
  """x [M][dim], a qkv weight whose columns' scales spread over 4 decades (so k and v runs mix sizes), the rotary
  tables, M distinct places and cache rows."""
  c = OL.model(dim=dim, heads=heads, kv=kv, head_dim=hd, theta=10000.0, eps=1e-5, places=256)
  nh = heads + 2 * kv
  x = rng.normal(0, 1, (M, dim)).astype(np.float32)
  w = (rng.normal(0, 0.02, (dim, nh * hd)) * 10.0 ** rng.integers(-2, 2, (1, nh * hd))).astype(np.float32)
  cos, sin = OL.rotary_head(c, c.places)
  places = rng.permutation(c.places)[:M].astype(np.int32)
  return c, x, w, cos, sin, places, places + 3


@pytest.mark.parametrize("path,M", [("gemv", 1), ("gemv", 3), ("skinny", 37), ("gemm", 150)])
@pytest.mark.parametrize("hd,heads,kv", [(64, 9, 3), (128, 8, 2)])
def test_rope_kv_puts_block_floats(cuda, path, M, hd, heads, kv):
  # the same qkv matmul into a bf16 cache and into a block-float one: the block float's parts are numpy's bfp parts of
  # the bf16 cache's rows, bit for bit; q is the same; rows not put stay zero
  rng = np.random.default_rng(71 + M + hd)
  c, x, w, cos, sin, places, rows = qkv_case(rng, hd, heads, kv, M)
  bw = ops().pack(to_gpu(w), "bfp8")
  mm = ops().gemv if path == "gemv" else ops().gemm
  xin = to_gpu(x) if path == "gemv" else to_gpu(x, torch.bfloat16)  # (the matrix cores take bf16 rows)
  length = c.places + 8
  outs = {}
  for fmt in ("bf16",) + FMTS:
    cache = ops().kv_cache(2 * kv, length, hd, fmt)
    data, dtype, n = ops().cache_fields(cache)
    ep = ops().epilogue(lib().EP_ROPE_KV, heads=heads, kv_heads=kv, head_dim=hd, cos_tab=to_gpu(cos), sin_tab=to_gpu(sin), rope_rows=len(cos),
                        places=to_gpu(places, torch.int32), cache_rows=to_gpu(rows, torch.int32), cache=data,
                        cache_dtype=dtype, cache_len=n)
    outs[fmt] = (mm(xin, bw, ep).cpu().numpy(), cache)
  q16, c16 = outs["bf16"]
  vals = c16.float().cpu().numpy()
  assert np.abs(vals[:, rows]).max() > 0
  for fmt in FMTS:
    q, cache = outs[fmt]
    assert np.array_equal(q, q16), (fmt, "q")
    gq, gt = cache_parts(cache)
    wq, wt = O.bfp_parts(vals, fmt)
    assert np.array_equal(gt, wt), (fmt, "exponents")
    assert np.array_equal(gq, wq), (fmt, "magnitudes", np.argwhere(gq != wq)[:4])
    put = vals[:, rows].reshape(2 * kv, M, hd // 16, 16)
    e = (O.bf16_bits(put).astype(np.int32) >> 7) & 255
    assert np.where(put != 0, e.max(-1, keepdims=True) - e, 0).max() >= 9  # values past bfp8's 8 bits of shift
    unput = np.ones(length, bool)
    unput[rows] = False
    assert not gq[:, unput].any() and not gt[:, unput].any()


@pytest.mark.parametrize("hd,heads,kv", [(64, 9, 3), (128, 32, 8), (256, 16, 1)])
def test_attention_decode_reads_block_floats(cuda, hd, heads, kv):
  # rows at places inside one chunk, across several, at a chunk's edge: the block-float cache gives exactly what a
  # bf16 cache of its values gives (test_sim.py:2100-2101)
  rng = np.random.default_rng(72 + hd)
  part, batch = 300, 4
  places = np.array([5, 63, 64, 299], np.int32)
  first = np.arange(batch, dtype=np.int32) * part
  q = rng.normal(0, 1, (batch, heads * hd)).astype(np.float32)
  ws = ops().attention_workspace(batch, heads, hd, part)
  for fmt in FMTS:
    v = wide_rows(rng, (2 * kv, batch * part, hd))
    same = O.bfp(v, fmt).astype(np.float32)  # the block float's values, each a bf16
    assert np.array_equal(O.bf16(same), same)
    cache = ops().kv_cache(2 * kv, batch * part, hd, fmt)
    cache.data.copy_(to_gpu(cache_bytes(v, fmt), torch.uint8))
    args = (heads, kv, hd, to_gpu(places, torch.int32), to_gpu(first, torch.int32), part, ws)
    got = ops().attention_decode(to_gpu(q), cache, *args).cpu()
    want = ops().attention_decode(to_gpu(q), to_gpu(same, torch.bfloat16), *args).cpu()
    assert torch.equal(got, want), (fmt, (got - want).abs().max())
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("hd,heads,kv,T,p0", [(64, 9, 3, 150, 0), (128, 8, 2, 70, 100)])
def test_attention_prefill_reads_block_floats(cuda, hd, heads, kv, T, p0):
  rng = np.random.default_rng(73 + hd)
  slot, length = 20, 300
  q = rng.normal(0, 1, (T, heads * hd)).astype(np.float32)
  for fmt in FMTS:
    v = wide_rows(rng, (2 * kv, length, hd))
    same = O.bfp(v, fmt).astype(np.float32)
    cache = ops().kv_cache(2 * kv, length, hd, fmt)
    cache.data.copy_(to_gpu(cache_bytes(v, fmt), torch.uint8))
    got = ops().attention_prefill(to_gpu(q), cache, heads, kv, hd, p0, slot).cpu()
    want = ops().attention_prefill(to_gpu(q), to_gpu(same, torch.bfloat16), heads, kv, hd, p0, slot).cpu()
    assert torch.equal(got, want), fmt


def north_star(got, want, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)


@pytest.mark.parametrize("mode,kv", [("bfp8", "bfp8"), ("bfp4", "bfp4")])
def test_decode_with_block_float_cache(cuda, mode, kv):
  # two SmolLM-shape blocks: a prompt as a batch of rows, then greedy steps a token at a time (a graph replayed), the
  # cache a block float; numpy's model rounds its cache by the same bfp: its tokens, logits within fp32 summation
  from test_gpu_2_decode import greedy, smol
  rng = np.random.default_rng(74)
  c = smol(2, 512)
  w = OL.random_weights(c, rng)
  prompt = [int(i) for i in rng.integers(0, 512, 7)]
  want, got, wl, gl = greedy(c, w, mode, kv, prompt, 8, 64)
  for a, b in zip(wl, gl):
    assert np.abs(a - b).max() <= 1e-3 * np.abs(a).max(), np.abs(a - b).max() / np.abs(a).max()
  assert got == want, (got, want)


@pytest.mark.parametrize("kv", FMTS)
def test_prefill_with_block_float_cache(cuda, kv):
  # a prompt through the matrix cores into a block-float cache, then decode steps from it, against numpy's forward
  # with the same cache format (test_llama_precision's bfp8 KV, test_sim.py:1994-2029)
  from ferrite_amd import llama as G
  rng = np.random.default_rng(75)
  c = OL.smollm(layers=3, vocab=1024, places=256)
  w = OL.random_weights(c, rng)
  prec = OL.precision(c, "bfp8", kv)
  c.precision = prec
  arrays = OL.arrays(w, prec)
  prompt = [int(i) for i in rng.integers(0, 1024, 140)]
  np_kv = OL.kv_cache(c, 256)
  want = OL.forward(prompt, range(len(prompt)), arrays, c, np_kv)[0]
  gc = G.model(**{k: getattr(c, k) for k in ("dim", "heads", "kv", "layers", "eps", "theta", "vocab", "ffn", "places", "rope", "tied")})
  dec = G.Decoder(gc, G.numpy_weights(w), mode="bfp8", kv=kv, batch=1, context=256)
  logits, pick = dec.prefill(prompt, chunk=100)
  north_star(logits[0].cpu().numpy(), want, "prefill logits")
  # the cache's values against numpy's (itself bfp-rounded): the matrix cores' bf16 rows move a value across a rounding
  # boundary now and then, so each value lies within two steps of its run's block float (the larger run exponent's
  # step, 2^(top - 133) for bfp8, 2^(top - 129) for bfp4), and the whole cache points the same way
  for l in range(c.layers):
    q, top = cache_parts(dec.cache[l])
    got = O.bfp_values(q, top, kv)[:, :len(prompt)]
    want_kv = np_kv[l][:, :len(prompt)]
    big = np.maximum(top[:, :len(prompt)], O.bfp_parts(want_kv, kv)[1])
    step = np.repeat(np.ldexp(1.0, big - (133 if kv == "bfp8" else 129)), 16, -1)
    assert (np.abs(got - want_kv) <= 2 * step).all(), ("cache", l, (np.abs(got - want_kv) / step).max())
    # (a crossing costs bfp4 a step of 1/8 of its run's largest value: ~1e-4 off the cosine at bf16 rows' 2^-9)
    cos = (got * want_kv).sum() / np.linalg.norm(got) / np.linalg.norm(want_kv)
    assert cos >= (0.9999 if kv == "bfp8" else 0.999), ("cache", l, cos)
  nxt = int(np.argmax(want))
  for i in range(3):
    place = len(prompt) + i
    want = OL.forward([nxt], [place], arrays, c, np_kv)[0]
    got = dec.step([nxt], [place], replay=False)[0][0].cpu().numpy()
    north_star(got, want, ("decode", i))
    nxt = int(np.argmax(want))
