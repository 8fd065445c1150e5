"""A Llama decode written with the lazy Tensor the way ferrite's models/llama.py writes its chip path (layer 95-109,
attention 111-146, rms 82-85, rope 92-93, mlp 266-275; fns' Tensor table, 41-47): the embedding's rows by gather,
RMSNorm from mean and rsqrt, the fused qkv matmul by a block float, RoPE as x cos + (x @ turn) sin over the heads
split as a batch, the keys and values put into the cache at the tokens' places, attend over each query head's
repeated key head, the heads merged back, o_proj and the SwiGLU MLP added back, the output layer. Two calls (a
three-token prompt, then a token) against the numpy oracle's forward over the same bfp8 weights: logits within the
north star's bar and the same picks."""
import math
import numpy as np
import pytest
from oracle import llama as OL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt(cuda):
  from ferrite_amd import tensor
  return tensor.Runtime(0)


def test_decode_written_with_tensors(rt):
  from ferrite_amd.tensor import Tensor
  c = OL.model(dim=256, heads=4, kv=2, layers=2, eps=1e-5, theta=10000.0, vocab=256, ffn=512, places=16)
  c.precision = OL.precision(c, "bfp8", "fp32")
  w = OL.random_weights(c, np.random.default_rng(151))
  hd, nh, rep, size = OL.head(c), c.heads + 2 * c.kv, c.heads // c.kv, 16
  T = lambda a, dtype="fp32": Tensor.of(rt, np.asarray(a, np.float32).tolist(), dtype)
  W = {k: (T(v).cast("bfp8") if k.endswith("_proj") or k == "embed.T" else T(v)) for k, v in w.items() if k not in ("cos", "sin", "turn")}
  cos, sin, turn = T(w["cos"]), T(w["sin"]), T(w["turn"])
  caches = [Tensor.of(rt, np.zeros((2 * c.kv, size, hd)).tolist(), "fp32") for _ in range(c.layers)]

  def rms(x, g): return x * ((x * x).mean(2) + c.eps).rsqrt() * g

  def step(ids, places):
    at = Tensor.of(rt, [list(places)], "int32")           # the places as a row (put, gather) and a column (attend)
    col = Tensor.of(rt, [[p] for p in places], "int32")
    return forward(Tensor.of(rt, [list(ids)], "int32"), at, col).numpy()[0]

  def forward(ids, at, col):  # (tensors only: jit replays it with new ids and places)
    n = ids.cols
    x = W["embed"].gather(ids)
    cs, sn = cos.gather(at).split(nh), sin.gather(at).split(nh)
    for l in range(c.layers):
      p = lambda name: W[f"layers.{l}.{name}"]
      h = rms(x, p("input_layernorm"))
      heads = h.matmul(p("qkv_proj"), "fp32").split(nh)
      heads = (heads * cs + heads.matmul(turn) * sn).merge().split(nh)
      caches[l].put(at, heads[c.heads:nh, :, :])
      q, k, v = heads[:c.heads, :, :], caches[l][:c.kv, :, :], caches[l][c.kv:, :, :]
      o = (q * (1 / math.sqrt(hd))).attend(k.repeat_interleave(rep), v.repeat_interleave(rep), col)
      x = (x + o.merge().matmul(p("o_proj"), "fp32")).realize()
      gu = rms(x, p("post_attention_layernorm")).matmul(p("gate_up_proj"), "fp32").realize()
      x = (x + (gu[:, :, :c.ffn].silu() * gu[:, :, c.ffn:]).matmul(p("down_proj"), "fp32")).realize()
    assert x.shape == (1, n, c.dim)
    return rms(x, W["norm"]).matmul(W["embed.T"], "fp32")

  def check(got, want, what):
    rel = np.abs(got - want).max() / np.abs(want).max()
    cosine = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    assert rel <= 1e-2 and cosine >= 0.9999, (what, rel, cosine)
    assert int(np.argmax(got)) == int(np.argmax(want)), what

  arrays, ocache = OL.arrays(w, c.precision), OL.kv_cache(c, size)
  for ids, places in (([5, 9, 200], [0, 1, 2]), ([77], [3])):
    check(step(ids, places)[-1], OL.forward(ids, places, arrays, c, ocache)[0], ids)
  # then greedy decoding with the step as ferrite's jit replays it (tensor.py:788-810): the first call runs, the second
  # is captured as a HIP graph, later calls copy the token and its place in and replay; each pick fed back
  from ferrite_amd import tensor
  f = tensor.jit(forward)
  token = 77
  for place in range(4, 9):
    want = OL.forward([token], [place], arrays, c, ocache)[0]
    got = f(Tensor.of(rt, [[token]], "int32"), Tensor.of(rt, [[place]], "int32"), Tensor.of(rt, [[place]], "int32")).numpy()[0][-1]
    check(got, want, ("jit", place))
    token = int(np.argmax(want))
