"""CPU restatement (numpy) of ferrite's Llama model path, the numpy branch of models/llama.py: the checker for the GPU
decode and prefill, and the CPU baseline bench.py times.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package; the product (ferrite_amd) never calls it.

It keeps the reference's dtype behaviour (models/llama.py:506-514, 783): weights are float32 arrays of the values the
GPU holds (bf16, or a block float's exact values), caches are np.zeros (float64), so activations are float32 until
the first attention and float64 after it; products are exact (mm = a @ b, llama.py:33). Each function cites the
line it follows. The model is a plain Llama (RMSNorm, RoPE, grouped-query attention, SwiGLU) with Llama 3's RoPE
scaling, and Mixtral's mixture of experts in the MLP's place; the reference's other families (Qwen3.5's DeltaNet,
gpt-oss's sinks, ...) are not on this path. The reference commits no golden vectors and its models/llama.py cannot be
imported here (Python 3.12 syntax on 3.10), so tests/test_oracle_llama.py pins this restatement against an independent
implementation of the same models (transformers' Llama and Mixtral blocks in float64) and the invariants the
reference's tests assert (cached decode = full recompute, chunked prefill = the whole prompt).
"""
import math
from types import SimpleNamespace
import numpy as np
from oracle.bfp import bf16, bf16_bits, bf16_floats, bfp

DEFAULTS = dict(head_dim=None, rope=None, k=0, experts=0, norm_topk=True, centered=False, tied=False, precision=None,
                places=4096, vocab=0, ffn=0, mtp=0)


def model(**c):
  """A config (models/llama.py:541-543): what it says, the rest a plain Llama's."""
  return SimpleNamespace(**(DEFAULTS | c))


def head(c):  # llama.py:87
  return c.head_dim or c.dim // c.heads


def precision(c, mode="bf16", kv=None):
  """Each matmul's weights' (format, phases) (models/llama.py:54-76): bf16, bfp8, bfp4 (the MLP's gate and up in
  bfp4), tt (bfp4's formats at one phase for a bfp4 B and two for a bfp8 one; Llama-3.1-8B's last gate_up in bfp8),
  experts (every MLP matrix in bfp4 at one phase, the rest bfp8 at two, and a draft head of the output layer in bfp4).
  The key ("kv", None) is the KV cache's format (tt's and experts' bfp8, else bf16). Phases are the chip's alone: the
  GPU's products are exact at any. Pinned by the reference's own answers (test_sim.py:1999-2008) in
  tests/test_precision.py."""
  four = {"bfp4": ("gate_up",), "tt": ("gate_up",), "experts": ("gate_up", "down")}.get(mode, ())
  fast = mode in ("tt", "experts")

  def entry(op):
    if mode in ("bf16", "bfp8"): return mode, 4
    f = "bfp4" if op in four else "bfp8"
    return f, ((1 if f == "bfp4" else 2) if fast else 4)
  p = {(op, l): entry(op) for l in range(c.layers + c.mtp) for op in ("qkv", "o", "gate_up", "down")}
  if mode == "tt" and (c.layers, c.dim) == (32, 4096): p["gate_up", 31] = ("bfp8", 2)
  p["head", None] = entry("head")
  if mode == "experts": p["draft head", None] = ("bfp4", 1)
  attention = {("attention", "decode"): (None, 2 if mode == "tt" else 4), ("attention", "prefill"): (None, 4)}
  return p | attention | {("kv", None): (kv or ("bfp8" if fast else "bf16"), None)}


def weight_format(name, prec):
  """A weight's format (models/llama.py:615-623): the matrices a matmul reads as its B in prec's, the rest bf16."""
  op = name.split(".")[-1].removesuffix("_proj")
  matrix = name.endswith(("_proj", "experts.gate_up", "experts.down"))
  key = {"embed.T": ("head", None), "embed.T draft": ("draft head", None)}.get(name) or ((op, int(name.split(".")[1])) if matrix else None)
  return prec[key][0] if prec and key in prec else "bf16"


def arrays(weights, prec=None):
  """The weights as numpy float32 values as the GPU holds them (models/llama.py:645-654): a block float's rounded by
  bfp along the last axis (a batch of experts' too)."""
  out = {}
  for name, v in weights.items():
    f = weight_format(name, prec)
    if f not in ("bfp8", "bfp4"):
      out[name] = v
      continue
    rows = v.reshape(-1, v.shape[-1])
    out[name] = bfp(rows, f).astype(np.float32).reshape(v.shape)
  return out


def rms(x, w, c):  # llama.py:82-85
  n = x * (1 / np.sqrt((x * x).mean(-1, keepdims=True) + c.eps))
  return n * w + n if c.centered else n * w


def frequencies(c):
  """RoPE's inverse frequencies in fp32, with Llama 3's scaling when c.rope says llama3 (models/llama.py:333-344)."""
  hd = head(c)
  inv = 1 / c.theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd)
  r = c.rope
  if r and r.get("rope_type") == "llama3":
    old, wavelen = r["original_max_position_embeddings"], 2 * math.pi / inv
    scaled = np.where(wavelen > old / r["low_freq_factor"], inv / r["factor"], inv)
    smooth = (old / wavelen - r["low_freq_factor"]) / (r["high_freq_factor"] - r["low_freq_factor"])
    between = (wavelen >= old / r["high_freq_factor"]) & (wavelen <= old / r["low_freq_factor"])
    inv = np.where(between, (1 - smooth) * scaled / r["factor"] + smooth * scaled, scaled).astype(np.float32)
  return inv


def rotary_head(c, n):
  """cos and sin for places 0..n-1, one head's (n, head_dim): fp32 angles, the tables rounded to bf16, the half
  turned twice over (models/llama.py:354-368, whose tables repeat this for every q and k head, 1 and 0 for v's)."""
  angles = np.arange(n, dtype=np.float32)[:, None] * frequencies(c)[None]
  cos = np.concatenate([np.cos(angles)] * 2, 1)
  sin = np.concatenate([np.sin(angles)] * 2, 1)
  return bf16(cos), bf16(sin)


def turn(hd):  # x @ turn is (-x2, x1) (models/llama.py:361-362)
  t, half = np.zeros((hd, hd), np.float32), np.arange(hd // 2)
  t[half + hd // 2, half], t[half, half + hd // 2] = -1, 1
  return t


def rotary(c, n):
  """The reference's full tables (models/llama.py:354-368): each head's cos and sin for q's and k's heads, 1 and 0
  for v's, side by side, and turn."""
  cos, sin = rotary_head(c, n)
  heads = lambda t, v: np.concatenate([t] * (c.heads + c.kv) + [np.full_like(t, v)] * c.kv, 1)
  return heads(cos, 1), heads(sin, 0), turn(head(c))


def rope(x, cos, sin, t):  # llama.py:92-93
  return x * cos + (x @ t) * sin


def split(a, n):  # gpt2.fns: the heads as a batch
  return a.reshape(a.shape[0], n, -1).transpose(1, 0, 2)


def merge(a):
  return a.transpose(1, 0, 2).reshape(a.shape[1], -1)


def softmax(a):  # models/gpt2.py:52
  e = np.exp(a - a.max(-1, keepdims=True))
  return e / e.sum(-1, keepdims=True)


def masked(places, size):  # models/gpt2.py:107-110: -1e9 where a key lies past the row's place
  k = np.arange(size)
  return np.where(k > np.asarray(places)[:, None], np.float32(-1e9), np.float32(0))


def attention(h, p, c, tables, mask, cache, rows):
  """A block's attention over its cache (models/llama.py:111-146, numpy, no slots): qkv, RoPE on q's and k's heads,
  this call's keys and values put at rows, softmax(q k^T / sqrt(hd) + mask) v over the cache, o_proj."""
  hd, rep, nh = head(c), c.heads // c.kv, c.heads + 2 * c.kv
  cos, sin, t = tables
  qkv = h @ p["qkv_proj"]
  qkv = merge(rope(split(qkv, nh), split(cos, nh), split(sin, nh), t))
  heads = split(qkv, nh)
  kv = heads[c.heads:]
  fmt = (c.precision or {}).get(("kv", None), ("bf16", None))[0]
  if fmt in ("bfp8", "bfp4"): kv = bfp(kv, fmt)  # (llama.py:127-128: numpy rounds a block-float cache as the chip does,
                                                 # and keeps a bf16 one's values unrounded)
  cache[:, list(rows)] = kv
  q, k, v = heads[:c.heads], cache[:c.kv], cache[c.kv:]
  m = mask.shape[-1]
  k, v = np.repeat(k[:, :m], rep, 0), np.repeat(v[:, :m], rep, 0)
  s = (q @ k.swapaxes(-1, -2)) * (1 / math.sqrt(hd))
  o = softmax(s + mask) @ v
  return merge(o) @ p["o_proj"]


def glu(gate, up):  # llama.py:271-273
  return gate / (1 + np.exp(-gate)) * up


def mlp(h, p):  # llama.py:266-269
  m = p["down_proj"].shape[-2]
  gu = h @ p["gate_up_proj"]
  return glu(gu[:, :m], gu[:, m:]) @ p["down_proj"]


def topk(a, k):  # llama.py:27: numpy's stable argsort, the first of equals first
  i = np.argsort(-a, -1, kind="stable")[..., :k]
  return np.take_along_axis(a, i, -1), i


def moe(h, p, c):
  """A mixture of experts (models/llama.py:277-300, numpy): router logits, the k best, softmax over those k
  (norm_topk), each chosen expert's SwiGLU weighted and summed."""
  logits = h @ p["router"]
  values, ids = topk(logits if c.norm_topk else softmax(logits), c.k)
  w = softmax(values) if c.norm_topk else values
  gate_up, down = p["experts.gate_up"], p["experts.down"]
  m = down.shape[-2]

  def expert(x, e):
    g = x @ gate_up[e]
    return glu(g[:m], g[m:]) @ down[e]
  return np.stack([sum(w[t, j] * expert(h[t], e) for j, e in enumerate(ids[t])) for t in range(len(h))]), ids, w


def layer(x, p, c, tables, mask, cache, rows):  # llama.py:95-109
  h = rms(x, p["input_layernorm"], c)
  x = x + attention(h, p, c, tables, mask, cache, rows)
  h = rms(x, p["post_attention_layernorm"], c)
  return x + (moe(h, p, c)[0] if "router" in p else mlp(h, p))


def block(w, pre):  # models/gpt2.py:70
  return {k[len(pre):]: w[k] for k in w if k.startswith(pre)}


def kv_cache(c, size, zeros=np.zeros):  # llama.py:506-514: keys' heads then values', a row each place
  return [zeros((2 * c.kv, size, head(c))) for _ in range(c.layers)]


def forward(ids, places, w, c, caches, every=False):
  """The logits for the token after ids (every: each token's), the tokens at places (models/llama.py:459-480): their
  keys and values into caches, each seeing the places up to its own."""
  x = w["embed"][list(ids)]
  size = caches[0].shape[-2]
  places = np.asarray(places)
  cos, sin, t = w["cos"][places], w["sin"][places], w["turn"]
  mask = masked(places, size)
  for l in range(c.layers):
    x = layer(x, block(w, f"layers.{l}."), c, (cos, sin, t), mask, caches[l], places)
  h = rms(x, w["norm"], c)
  return (h if every else h[-1:]) @ w["embed.T"]


def forward_slots(ids, places, w, c, caches):
  """Several sequences decoding together, one token each (models/llama.py:459-480 with slots, attention's slots branch
  at 133-137 and around's rows, 429-452): the matmuls take every row at once, each row's keys and values go to its own
  sequence's cache (caches[b], one kv_cache of its own rather than a part of a shared one: the same rows) at its place,
  and it attends over that sequence's places up to its own. Every row's logits. (The reference's convention for a free
  slot, a token on its part's last row seeing only the part's first, serves idle slots of a server and is not
  restated: every row here is live.)"""
  x = w["embed"][list(ids)]
  places = np.asarray(places)
  cos, sin, t = w["cos"][places], w["sin"][places], w["turn"]
  size = caches[0][0].shape[-2]
  hd, rep, nh = head(c), c.heads // c.kv, c.heads + 2 * c.kv
  for l in range(c.layers):
    p = block(w, f"layers.{l}.")
    h = rms(x, p["input_layernorm"], c)
    qkv = merge(rope(split(h @ p["qkv_proj"], nh), split(cos, nh), split(sin, nh), t))
    heads = split(qkv, nh)  # [heads][rows][hd]
    fmt = (c.precision or {}).get(("kv", None), ("bf16", None))[0]
    o = np.zeros((len(ids), c.heads * hd))
    for b, place in enumerate(places):
      kv = heads[c.heads:, b:b + 1]
      if fmt in ("bfp8", "bfp4"): kv = bfp(kv, fmt)
      cache = caches[b][l]
      cache[:, [place]] = kv
      k, v = np.repeat(cache[:c.kv], rep, 0), np.repeat(cache[c.kv:], rep, 0)
      s = (heads[:c.heads, b:b + 1] @ k.swapaxes(-1, -2)) * (1 / math.sqrt(hd)) + masked([place], size)
      o[b] = merge(softmax(s) @ v)[0]
    x = x + o @ p["o_proj"]
    h = rms(x, p["post_attention_layernorm"], c)
    x = x + (moe(h, p, c)[0] if "router" in p else mlp(h, p))
  return rms(x, w["norm"], c) @ w["embed.T"]


def prefill(ids, w, c, caches, tokens):  # llama.py:498-504: a prompt so many tokens at a time
  for i in range(0, len(ids), tokens):
    out = forward(ids[i:i + tokens], list(range(i, min(i + tokens, len(ids)))), w, c, caches)
  return out


def random_weights(c, rng, sd=0.02, norm_sd=0.1, embed_sd=1.0):
  """Random weights in c's shapes, named as models/llama.py's fuse leaves them (x @ w: q, k and v side by side, gate and
  up), bf16 values as float32: matrices N(0, sd), norms N(1, norm_sd), the embedding N(0, embed_sd) (test_sim.py's
  smol, 1319-1327), RoPE's tables for c.places places."""
  hd, qkv = head(c), (c.heads + 2 * c.kv) * head(c)
  w = {}
  for l in range(c.layers):
    pre = f"layers.{l}."
    w[pre + "input_layernorm"] = bf16(rng.normal(1, norm_sd, (1, c.dim)))
    w[pre + "post_attention_layernorm"] = bf16(rng.normal(1, norm_sd, (1, c.dim)))
    w[pre + "qkv_proj"] = bf16(rng.normal(0, sd, (c.dim, qkv)))
    w[pre + "o_proj"] = bf16(rng.normal(0, sd, (c.heads * hd, c.dim)))
    if c.experts:
      w[pre + "router"] = bf16(rng.normal(0, sd, (c.dim, c.experts)))
      w[pre + "experts.gate_up"] = bf16(rng.normal(0, sd, (c.experts, c.dim, 2 * c.ffn)))
      w[pre + "experts.down"] = bf16(rng.normal(0, sd, (c.experts, c.ffn, c.dim)))
    else:
      w[pre + "gate_up_proj"] = bf16(rng.normal(0, sd, (c.dim, 2 * c.ffn)))
      w[pre + "down_proj"] = bf16(rng.normal(0, sd, (c.ffn, c.dim)))
  w["norm"] = bf16(rng.normal(1, norm_sd, (1, c.dim)))
  w["embed"] = bf16(rng.normal(0, embed_sd, (c.vocab, c.dim)))
  w["embed.T"] = np.ascontiguousarray(w["embed"].T) if c.tied else bf16(rng.normal(0, sd, (c.dim, c.vocab)))
  w["cos"], w["sin"], w["turn"] = rotary(c, c.places)
  return w


def smollm(layers=30, vocab=49152, places=256):
  """SmolLM-135M's shape (benchmark config 2): 576 wide, 9 query heads sharing 3 key heads of 64, MLP 1536, RMSNorm eps
  1e-5, RoPE theta 10000, the output layer the embedding (tied)."""
  return model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536, places=places, tied=True)


def llama8b(layers=32, vocab=128256, places=2048, rope=True):
  """Llama-3.1-8B's shape (benchmark config 3): 4096 wide, 32 query heads sharing 8 key heads of 128, MLP 14336, vocab
  128256, theta 500000 with Llama 3's RoPE scaling (test_sim.py:1933-1934), its own output layer."""
  r = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
  return model(dim=4096, heads=32, kv=8, layers=layers, eps=1e-5, theta=500000.0, vocab=vocab, ffn=14336, places=places,
               rope=r if rope else None)
