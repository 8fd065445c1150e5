"""Parity at the benchmark configs' own widths (the reference's test_llama_8b_shapes, test/test_sim.py:1926-1949: blocks
in Llama-3.1-8B's shapes against numpy), through the C-ABI:
- config 3: two Llama-3.1-8B-shape blocks (4096 wide, 32 query heads sharing 8 key heads of 128, MLP 14336, vocab
  128256, Llama 3's RoPE) at precision "experts" (attention and output layer bfp8, MLP bfp4), a bf16 KV cache at
  context 2048: a batch-1 step at place 2047 (the GEMV path) and a batch-16 step of 16 sequences at places up to 2047
  (the skinny matrix-core path); a 64-token prompt then 32 greedy steps of batch 1, the same tokens as numpy's
  (models/llama.py:787-796); and the reference's own case at "tt" precision with a bfp8 cache (a 64-token prompt,
  two decode steps);
- config 4: a 2048-token prefill of two such blocks, all bfp8 (the tiled MFMA GEMM and the causal prefill attention),
  its keys and values and last logits, then a decode step from the cache it filled;
- config 5: a Mixtral-shape mixture of experts (4096 wide, 8 experts of MLP 14336 in bfp4, top 2) over 32 tokens.
Weights are drawn on the GPU (ferrite_amd.llama.random_weights: bf16 values, seeded by name) and copied to the host,
where the oracle rounds them to their block floats (oracle/cbfp.py: oracle/bfp.py's bfp in C, pinned bit for bit
against it) and runs models/llama.py's numpy restatement (oracle/llama.py) in float64 as ferrite's numpy does (float64
caches, unrounded). The bar is the north star's: max relative error 1e-2 of the largest value and cosine >= 0.9999, and
the same greedy pick. Config 3's caches hold seeded bf16 rows (the same values in both) rather than a 2047-token
prefill, which config 4 covers at this width."""
import numpy as np
import pytest
import torch
from oracle import bfp as O
from oracle import cbfp
from oracle import llama as OL

pytestmark = pytest.mark.gpu


def north_star(got, want, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  print(f"{what}: max relative error {rel:.2e}, cosine {cos:.8f}", flush=True)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)
  return rel


def host_bits(t):
  """A bf16 tensor on the GPU as its bits (uint16) on the host."""
  return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def gpu_model(c):
  from ferrite_amd import llama as G
  return G.model(**{k: getattr(c, k) for k in ("dim", "heads", "kv", "layers", "eps", "theta", "vocab", "ffn", "places", "rope", "tied")})


def oracle_arrays(c, draw, prec):
  """The oracle's weights (OL.arrays' values, models/llama.py:645-654) of the bf16 weights draw(name, shape) makes on
  the GPU: each block float's values by the C restatement of gpt2.bfp along the last axis, the rest as their bf16
  values; RoPE's tables for c.places places."""
  hd = OL.head(c)
  shapes = {"norm": (1, c.dim), "embed": (c.vocab, c.dim), "embed.T": (c.dim, c.vocab)}
  for l in range(c.layers):
    pre = f"layers.{l}."
    shapes |= {pre + "input_layernorm": (1, c.dim), pre + "post_attention_layernorm": (1, c.dim),
               pre + "qkv_proj": (c.dim, (c.heads + 2 * c.kv) * hd), pre + "o_proj": (c.heads * hd, c.dim),
               pre + "gate_up_proj": (c.dim, 2 * c.ffn), pre + "down_proj": (c.ffn, c.dim)}
  w = {}
  for name, shape in shapes.items():
    bits = host_bits(draw(name, shape))
    f = OL.weight_format(name, prec)
    w[name] = cbfp.bfp(bits, f) if f in ("bfp8", "bfp4") else O.bf16_floats(bits)
  w["cos"], w["sin"], w["turn"] = OL.rotary(c, c.places)
  return w


class Model:
  """Two Llama-3.1-8B-shape blocks drawn once on the GPU, with the oracle's arrays of them per precision mode."""
  def __init__(self):
    from ferrite_amd import llama as G
    self.c = OL.llama8b(layers=2, places=2048 + 64)
    self.gc = gpu_model(self.c)
    self.draw = G.random_weights(self.gc, seed=31)
    self.arrays = {}

  def oracle(self, mode):
    if mode not in self.arrays:
      self.arrays.clear()  # (one mode's arrays at a time on the host: about 8 GB)
      self.arrays[mode] = oracle_arrays(self.c, self.draw, OL.precision(self.c, mode, "bf16"))
    return self.arrays[mode]


@pytest.fixture(scope="module")
def m8b(cuda):
  return Model()


def seeded_rows(gen, shape):
  """bf16 N(0, 1) rows drawn on the GPU (a seeded generator), and their values as float64 on the host."""
  t = torch.randn(*shape, generator=gen, device="cuda").to(torch.bfloat16)
  return t, O.bf16_floats(host_bits(t)).astype(np.float64)


def test_config3_decode_batch1_and_16(m8b):
  from ferrite_amd import llama as G
  c, ctx = m8b.c, 2048
  c.precision = OL.precision(c, "experts", "bf16")
  w = m8b.oracle("experts")
  gen = torch.Generator(device="cuda")
  gen.manual_seed(33)
  # batch 1, the GEMV path: rows 0..2046 of each block's cache seeded, the token at place 2047
  dec = G.Decoder(m8b.gc, m8b.draw, mode="experts", kv="bf16", batch=1, context=ctx)
  caches = OL.kv_cache(c, ctx)
  for l in range(c.layers):
    t, v = seeded_rows(gen, (2 * c.kv, ctx - 1, 128))
    dec.cache[l][:, :ctx - 1].copy_(t)
    caches[l][:, :ctx - 1] = v
  tok = 91011
  logits, picks = dec.step([tok], [ctx - 1], replay=False)
  want = OL.forward([tok], [ctx - 1], w, c, caches)[0]
  got = logits[0].cpu().numpy()
  rel = north_star(got, want, "config 3 batch 1 logits")
  assert rel <= 1e-3  # (exact products, fp32 sums: far inside the bar)
  assert int(picks[0]) == int(np.argmax(want))
  # the key and value the step put at place 2047, bf16 of the oracle's
  for l in range(c.layers):
    put = dec.cache[l][:, ctx - 1].float().cpu().numpy()
    north_star(put, caches[l][:, ctx - 1], f"config 3 block {l} k/v put")
  # batch 16 on the matrix cores: 16 sequences, each its own slot and place
  B = 16
  places = [2047, 2000, 1500, 1024, 1023, 777, 512, 300, 129, 128, 64, 63, 17, 5, 1, 0]
  many = G.Decoder(m8b.gc, None, mode="experts", kv="bf16", batch=B, context=ctx, slots=B, share=dec)
  assert many.mm.__name__ == "gemm"
  seqs = [OL.kv_cache(c, ctx) for _ in range(B)]
  for l in range(c.layers):
    t, v = seeded_rows(gen, (2 * c.kv, B * ctx, 128))
    many.cache[l].copy_(t)
    for b in range(B): seqs[b][l][:] = v[:, b * ctx:(b + 1) * ctx]
  toks = [int(i) for i in np.random.default_rng(34).integers(0, c.vocab, B)]
  logits, picks = many.step(toks, places, slots=list(range(B)), replay=False)
  want = OL.forward_slots(toks, places, w, c, seqs)
  got = logits.cpu().numpy()
  for b in range(B):
    north_star(got[b], want[b], f"config 3 batch 16 row {b} (place {places[b]}) logits")
  assert [int(p) for p in picks.cpu()] == [int(i) for i in np.argmax(want, 1)]


def test_config4_prefill_2048_then_decode(m8b):
  from ferrite_amd import llama as G
  c, T, ctx = m8b.c, 2048, 2048 + 64
  c.precision = OL.precision(c, "bfp8", "bf16")
  w = m8b.oracle("bfp8")
  ids = [int(i) for i in np.random.default_rng(35).integers(0, c.vocab, T)]
  dec = G.Decoder(m8b.gc, m8b.draw, mode="bfp8", kv="bf16", batch=1, context=ctx)
  logits, pick = dec.prefill(ids)
  caches = OL.kv_cache(c, ctx)
  want = OL.forward(ids, range(T), w, c, caches)[0]
  north_star(logits[0].cpu().numpy(), want, "config 4 prefill last logits")
  assert int(pick[0]) == int(np.argmax(want))
  for l in range(c.layers):  # every row's key and value (block 1's come through block 0's attention)
    got = dec.cache[l][:, :T].float().cpu().numpy()
    north_star(got, caches[l][:, :T], f"config 4 block {l} keys and values, {T} rows")
  # then a decode step from the cache the prefill filled (the GEMV path at place 2048)
  nxt = int(np.argmax(want))
  logits, pick = dec.step([nxt], [T], replay=False)
  want = OL.forward([nxt], [T], w, c, caches)[0]
  north_star(logits[0].cpu().numpy(), want, "config 4 decode after prefill")
  assert int(pick[0]) == int(np.argmax(want))


def test_config5_moe_mixtral_width(cuda):
  from ferrite_amd import llama as G, ops
  T, dim, ffn, E, k = 32, 4096, 14336, 8, 2
  c = OL.model(dim=dim, k=k, experts=E, eps=1e-5)
  draw = G.random_weights(G.model(dim=dim, heads=32, kv=8, layers=1, eps=1e-5, theta=1e4, vocab=16, ffn=ffn), seed=36)
  gu, dn = draw("experts.gate_up", (E, dim, 2 * ffn)), draw("experts.down", (E, ffn, dim))
  router = draw("router", (dim, E))
  gen = torch.Generator(device="cuda")
  gen.manual_seed(37)
  x, xv = seeded_rows(gen, (T, dim))
  ex = ops.pack_experts(gu, dn, "bfp4")
  ids, wts, dense = ops.moe_route(x.float(), router, E, k)
  y = ops.moe_experts(x.float(), ex, dense)
  p = {"router": O.bf16_floats(host_bits(router)), "experts.gate_up": cbfp.bfp(host_bits(gu), "bfp4"),
       "experts.down": cbfp.bfp(host_bits(dn), "bfp4")}
  del gu, dn
  want, want_ids, want_w = OL.moe(xv, p, c)
  assert np.array_equal(ids.cpu().numpy(), want_ids)
  assert np.abs(wts.cpu().numpy() - want_w).max() <= 1e-5
  assert len(set(want_ids.reshape(-1).tolist())) == E  # (every expert read, as config 5 expects)
  got = y.cpu().numpy()
  north_star(got, want, "config 5 MoE, 32 tokens")
  for t in range(T): north_star(got[t], want[t], f"config 5 token {t}")


def greedy_8b(m8b, kv, forced):
  """A 64-token seeded prompt (one step of 64 rows, the exact-product GEMV), then 31 more steps of batch 1 (the
  benchmark's step, replayed as a graph) at precision "experts": numpy's model as written (float64, its cache
  unrounded) and the GPU each fed its own pick, or (forced) both fed numpy's pick, as models/llama.py's main does
  (787-796: "so that one near tie does not send the two down different paths"). Returns numpy's and the GPU's picks
  and logits, step by step."""
  from ferrite_amd import llama as G
  c, ctx, P, steps = m8b.c, 128, 64, 32
  c.precision = OL.precision(c, "experts", kv)
  w = m8b.oracle("experts")
  prompt = [int(i) for i in np.random.default_rng(38).integers(0, c.vocab, P)]
  np_kv = OL.kv_cache(c, ctx)
  first = G.Decoder(m8b.gc, m8b.draw, mode="experts", kv=kv, batch=P, context=ctx, mfma_from=None)
  one = G.Decoder(m8b.gc, None, mode="experts", kv=kv, batch=1, context=ctx, share=first)
  want, got, wl, gl = [], [], [], []
  new, places = prompt, list(range(P))
  for i in range(steps):
    a = OL.forward(new, places, w, c, np_kv)[0]
    if i == 0:
      logits, picks = first.step(prompt, places, replay=False)
      b = logits[-1].cpu().numpy().astype(np.float64)
      for l in range(c.layers): one.cache[l].copy_(first.cache[l])
    else:
      logits, picks = one.step([nxt], [P + i - 1])
      b = logits[0].cpu().numpy().astype(np.float64)
    want.append(int(np.argmax(a)))
    got.append(int(picks[-1]))
    wl.append(a)
    gl.append(b)
    nxt = want[-1] if forced else got[-1]
    new, places = [want[-1]] if forced else [got[-1]], [P + i]
  return want, got, wl, gl


def test_config3_prompt_then_32_greedy_tokens(m8b):
  # models/llama.py's main at config 3's width (its check of every step against numpy, models/llama.py:787-796), two
  # Llama-3.1-8B-shape blocks at precision "experts", 32 steps (the prompt's and 31 greedy ones). An fp32 cache: the
  # GPU's logits within fp32 summation of numpy's (1e-4 of the largest), and each fed its own pick, the 32 tokens the
  # same. The benchmark's bf16 cache rounds each key and value (2^-9 relative), which moves the logits by up to ~3e-3
  # of their largest: both fed numpy's pick, as the reference's main feeds them, each step within the north star's
  # bar, and the picks the same at every step whose top-1 / top-2 gap is more than twice that step's largest error
  # (a nearer tie goes either way; its count printed)
  want, got, wl, gl = greedy_8b(m8b, "fp32", forced=False)
  for i, (a, b) in enumerate(zip(wl, gl)):
    top = np.sort(a)[-2:]
    rel = float(np.abs(a - b).max() / np.abs(a).max())
    print(f"fp32 cache, step {i}: token {want[i]} (GPU {got[i]}), gap {top[1] - top[0]:.3e}, error {rel:.2e} of the largest", flush=True)
    assert rel <= 1e-4, (i, rel)
  assert got == want, (got, want)
  want, got, wl, gl = greedy_8b(m8b, "bf16", forced=True)
  ties = 0
  for i, (a, b) in enumerate(zip(wl, gl)):
    top = np.sort(a)[-2:]
    err = float(np.abs(a - b).max())
    print(f"bf16 cache, step {i}: token {want[i]} (GPU {got[i]}), gap {top[1] - top[0]:.3e}, error {err:.3e}", flush=True)
    north_star(b, a, f"config 3 bf16 cache, step {i} logits")
    if top[1] - top[0] > 2 * err: assert got[i] == want[i], (i, got[i], want[i])
    else: ties += 1
  print(f"bf16 cache: the same pick at {sum(g == w for g, w in zip(got, want))} of 32 steps, {ties} near ties")


def test_config3_tt_precision_bfp8_cache(m8b):
  # the reference's own 8B-shape case (test_llama_8b_shapes, test/test_sim.py:1926-1949): TT's performance precision
  # ("tt": gate_up bfp4, the rest bfp8) with its bfp8 KV cache, a 64-token prompt (here the prefill on the matrix
  # cores) and two decode steps (tokens 5 at place 64 and 9 at 65, the GEMV path); each time the pick the same as
  # numpy's and the logits within 2% of numpy's span (its bar, np.ptp)
  from ferrite_amd import llama as G
  c, ctx = m8b.c, 96
  c.precision = OL.precision(c, "tt", "bfp8")
  w = m8b.oracle("tt")
  dec = G.Decoder(m8b.gc, m8b.draw, mode="tt", kv="bfp8", batch=1, context=ctx)
  np_kv = OL.kv_cache(c, ctx)
  prompt = [int(i) for i in np.random.default_rng(8).integers(0, c.vocab, 64)]
  for new, places in ((prompt, list(range(64))), ([5], [64]), ([9], [65])):
    if len(new) > 1: got = dec.prefill(new)[0][0].cpu().numpy().astype(np.float64)
    else: got = dec.step(new, places, replay=False)[0][0].cpu().numpy().astype(np.float64)
    want = OL.forward(new, places, w, c, np_kv)[0]
    err, span = float(np.abs(got - want).max()), float(np.ptp(want))
    print(f"tt, bfp8 cache, places {places[0]}..{places[-1]}: logits' largest error {err:.3e}, numpy's span {span:.3e}",
          flush=True)
    assert int(np.argmax(got)) == int(np.argmax(want)) and err < 0.02 * span, (places[0], err, span)
