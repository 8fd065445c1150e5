"""Parity of the prompt path's kernels with the oracle, through the C-ABI: causal prefill attention on the matrix cores
(fh_attention_prefill) and the row RMSNorm (fh_rms_rows). The attention holds q, k, v and the softmax weights in bf16
(as ferrite's chip does), so it is checked against numpy's softmax(q k^T / sqrt(hd) + mask) v (models/llama.py:141-142)
on the bf16-rounded q, k, v within the weights' rounding (2^-8 of the largest |v|), and against the unrounded float64
oracle within the north star's bar. The reference's tests of the same: test_kv_cache (test/test_sim.py:1451-1469),
test_chunked_prefill's invariant (2016)."""
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


def to_gpu(a, dtype=torch.float32):
  return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def north_star(got, want, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)


def causal(q, cache, heads, kv, hd, p0, slot):
  """numpy: row t at place p0 + t over cache rows slot .. slot + p0 + t, grouped-query."""
  T = q.shape[0]
  out = np.zeros((T, heads * hd))
  rep = heads // kv
  for t in range(T):
    n = p0 + t + 1
    k = np.repeat(cache[:kv, slot:slot + n], rep, 0)
    v = np.repeat(cache[kv:, slot:slot + n], rep, 0)
    qq = q[t].reshape(heads, 1, hd).astype(np.float64)
    out[t] = (OL.softmax(qq @ k.swapaxes(-1, -2) / math.sqrt(hd)) @ v).reshape(-1)
  return out


@pytest.mark.parametrize("hd,heads,kv,T,p0", [(64, 9, 3, 150, 0), (128, 8, 2, 200, 37), (128, 4, 4, 1, 5), (64, 2, 1, 129, 64)])
def test_attention_prefill(cuda, hd, heads, kv, T, p0):
  rng = np.random.default_rng(31)
  slot, rows = 7, 7 + p0 + T + 3
  cache = rng.normal(0, 1, (2 * kv, rows, hd)).astype(np.float32)
  q = rng.normal(0, 1, (T, heads * hd)).astype(np.float32)
  for cd in (torch.float32, torch.bfloat16):
    for od in (torch.float32, torch.bfloat16):
      o = ops().attention_prefill(to_gpu(q), to_gpu(cache, cd), heads, kv, hd, p0, slot, out_dtype=od).float().cpu().numpy()
      want = causal(O.bf16(q), O.bf16(cache), heads, kv, hd, p0, slot)
      tol = 2.0 ** -8 * np.abs(cache).max() * (2 if od == torch.bfloat16 else 1)
      assert np.abs(o - want).max() <= tol, (cd, od, np.abs(o - want).max())
      north_star(o, causal(q, cache, heads, kv, hd, p0, slot), (cd, od))


def test_attention_prefill_in_chunks(cuda):
  # a prompt in chunks (each chunk's rows attend to the earlier chunks' keys) equals the prompt at once
  rng = np.random.default_rng(32)
  hd, heads, kv, T = 128, 8, 2, 300
  cache = to_gpu(rng.normal(0, 1, (2 * kv, T, hd)), torch.bfloat16)
  q = to_gpu(rng.normal(0, 1, (T, heads * hd)))
  whole = ops().attention_prefill(q, cache, heads, kv, hd, 0, 0)
  parts = [ops().attention_prefill(q[a:b], cache, heads, kv, hd, a, 0) for a, b in ((0, 100), (100, 228), (228, 300))]
  assert torch.equal(torch.cat(parts), whole)


def test_attention_prefill_rejects(cuda):
  cache = torch.zeros(2, 10, 64, device="cuda")
  with pytest.raises(ValueError, match="must lie in the cache"):
    ops().attention_prefill(torch.zeros(8, 64, device="cuda"), cache, 1, 1, 64, 5, 0)
  with pytest.raises(NotImplementedError):
    ops().attention_prefill(torch.zeros(8, 96, device="cuda"), torch.zeros(2, 10, 96, device="cuda"), 1, 1, 96, 0, 0)


@pytest.mark.parametrize("dim", [576, 4096, 578, 5000])
def test_rms_rows(cuda, dim):
  # a row of up to 4096 values held in registers, 4 a load where the row allows it (576: a partial last round of 1024;
  # 4096: all 4 rounds full), one a load otherwise (578: not a multiple of 4); past 4096 the row read twice (5000)
  rng = np.random.default_rng(33)
  c = OL.model(dim=dim, eps=1e-5)
  x = rng.normal(0, 3, (37, dim)).astype(np.float32)
  w = O.bf16(rng.normal(1, 0.1, (1, dim)))
  for centered in (False, True):
    c.centered = centered
    want = OL.rms(x.astype(np.float64), w, c)
    got = ops().rms_rows(to_gpu(x), to_gpu(w.reshape(-1)), c.eps, centered, out_dtype=torch.float32).cpu().numpy()
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max(), centered
    got = ops().rms_rows(to_gpu(x), to_gpu(w.reshape(-1)), c.eps, centered).float().cpu().numpy()
    assert np.array_equal(got, O.bf16(got)) and np.abs(got - want).max() <= 2.0 ** -8 * np.abs(want).max()


def test_decoder_prefill_then_decode(cuda):
  # a SmolLM-shape model: the prompt through the matrix cores (in two chunks), then greedy decode steps from the cache
  # it filled; against numpy's forward over the same prompt and its greedy continuation (models/llama.py:498-504,
  # 787-796). The prompt's rows are bf16 into the matrix cores, so its logits meet the north star's bar, not fp32's.
  from ferrite_amd import llama as G
  rng = np.random.default_rng(34)
  c = OL.smollm(layers=4, vocab=2048, places=256)
  w = OL.random_weights(c, rng)
  prec = OL.precision(c, "bfp8", "bf16")
  c.precision = prec  # (numpy's cache unrounded, as models/llama.py:127-128 keeps it: the bf16 cache's rounding is
  arrays = OL.arrays(w, prec)  # within the north star's bar)
  prompt = [int(i) for i in rng.integers(0, 2048, 150)]
  np_kv = OL.kv_cache(c, 256)
  want = OL.forward(prompt, range(len(prompt)), arrays, c, np_kv)[0]
  gc = G.model(**{k: getattr(c, k) for k in ("dim", "heads", "kv", "layers", "eps", "theta", "vocab", "ffn", "places", "rope", "tied")})
  dec = G.Decoder(gc, G.numpy_weights(w), mode="bfp8", kv="bf16", batch=1, context=256)
  logits, pick = dec.prefill(prompt, chunk=100)
  got = logits[0].cpu().numpy()
  north_star(got, want, "prefill logits")
  assert int(pick[0]) == int(np.argmax(got))
  # the cache rows it wrote: the numpy cache's within bf16 rounding and the rows' bf16 inputs
  for l in range(c.layers):
    k = dec.cache[l][:, :len(prompt)].float().cpu().numpy()
    north_star(k, np_kv[l][:, :len(prompt)], ("cache", l))
  # then decode: each step's logits within the north star's bar of numpy's, fed numpy's own tokens
  nxt = int(np.argmax(want))
  for i in range(4):
    place = len(prompt) + i
    want = OL.forward([nxt], [place], arrays, c, np_kv)[0]
    got = dec.step([nxt], [place], replay=False)[0][0].cpu().numpy()
    north_star(got, want, ("decode", i))
    nxt = int(np.argmax(want))
