"""The CPU oracle's Llama path (oracle/llama.py) pinned by an independent implementation of the same models: Hugging
Face transformers' LlamaForCausalLM and MixtralSparseMoeBlock (transformers 5.15.0, installed in this image), run in
float64 on the same weights. ferrite's own models/llama.py cannot be imported here (ferrite/compiler.py uses Python
3.12's f-string syntax; this image has 3.10), so the composition is pinned against transformers, as the reference pins
its own numpy model (NOTES.md: "real blocks within 0.22% in numpy" of transformers) and its RoPE frequencies
(test/test_sim.py:1351-1361). Plus the invariants the reference's tests assert: a cached decode equals the full
recompute (test_sim.py:1469), and chunked prefill equals the whole prompt (test_sim.py:2016)."""
import numpy as np
import pytest
from oracle import bfp as O
from oracle import llama as OL

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")


def hf_llama(c, w):
  """transformers' Llama with w's weights (x @ w, fused as oracle.llama names them), float64, eager attention, its RoPE
  tables rounded to bf16 as ferrite's rotary rounds them (models/llama.py:360)."""
  hd = OL.head(c)
  cfg = transformers.LlamaConfig(hidden_size=c.dim, intermediate_size=c.ffn, num_attention_heads=c.heads,
                                 num_key_value_heads=c.kv, num_hidden_layers=c.layers, rms_norm_eps=c.eps, vocab_size=c.vocab,
                                 max_position_embeddings=c.places, tie_word_embeddings=c.tied, rope_theta=c.theta,
                                 rope_scaling=c.rope, attn_implementation="eager", head_dim=hd)
  m = transformers.LlamaForCausalLM(cfg).double().eval()
  t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float64))
  sd = {"model.embed_tokens.weight": t(w["embed"]), "model.norm.weight": t(w["norm"][0])}
  if not c.tied: sd["lm_head.weight"] = t(w["embed.T"].T)
  q, kv = c.heads * hd, c.kv * hd
  for l in range(c.layers):
    pre, p = f"model.layers.{l}.", f"layers.{l}."
    qkv = w[p + "qkv_proj"]
    sd[pre + "self_attn.q_proj.weight"] = t(qkv[:, :q].T)
    sd[pre + "self_attn.k_proj.weight"] = t(qkv[:, q:q + kv].T)
    sd[pre + "self_attn.v_proj.weight"] = t(qkv[:, q + kv:].T)
    sd[pre + "self_attn.o_proj.weight"] = t(w[p + "o_proj"].T)
    gu = w[p + "gate_up_proj"]
    sd[pre + "mlp.gate_proj.weight"] = t(gu[:, :c.ffn].T)
    sd[pre + "mlp.up_proj.weight"] = t(gu[:, c.ffn:].T)
    sd[pre + "mlp.down_proj.weight"] = t(w[p + "down_proj"].T)
    sd[pre + "input_layernorm.weight"] = t(w[p + "input_layernorm"][0])
    sd[pre + "post_attention_layernorm.weight"] = t(w[p + "post_attention_layernorm"][0])
  missing, unexpected = m.load_state_dict(sd, strict=False)
  assert not unexpected and all(k == "lm_head.weight" for k in missing), (missing, unexpected)
  rot = m.model.rotary_emb
  real = rot.forward
  def rounded(x, position_ids):
    cos, sin = real(x, position_ids)
    return cos.to(torch.bfloat16).to(cos.dtype), sin.to(torch.bfloat16).to(sin.dtype)
  rot.forward = rounded
  return m


def small(layers=2, rope=None):
  return OL.model(dim=128, heads=4, kv=2, layers=layers, eps=1e-5, theta=10000.0 if rope is None else 500000.0, vocab=96,
                  ffn=192, places=64, tied=True, rope=rope)


LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def test_frequencies_llama3():
  # Llama 3.1's RoPE scaling, as the reference's test_llama_frequencies checks models/llama.py (test_sim.py:1351-1361)
  m = pytest.importorskip("transformers.modeling_rope_utils")
  hf = transformers.LlamaConfig(hidden_size=4096, num_attention_heads=32, rope_theta=500000.0, rope_scaling=LLAMA3,
                                max_position_embeddings=131072)
  want = m.ROPE_INIT_FUNCTIONS["llama3"](hf, "cpu")[0].numpy()
  got = OL.frequencies(OL.model(dim=4096, heads=32, theta=500000.0, rope=LLAMA3))
  # numpy's float32 pow and torch's differ in the last bits for some exponents (this image: numpy 2.2, torch 2.10;
  # the blend's arithmetic carries one such difference to 2 ulps), so the bar is 4 ulps, about 2.4e-7 relative; a
  # wrong band, factor or blend is off by 10% or more
  ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
  assert got.dtype == np.float32 and ulps.max() <= 4, ulps.max()
  plain = OL.frequencies(OL.model(dim=4096, heads=32, theta=500000.0))
  assert plain[0] == got[0] and plain[-1] == 8 * got[-1]


@pytest.mark.parametrize("rope", [None, LLAMA3])
def test_forward_matches_transformers(rope):
  # a prompt's last logits, every place's logits, and 3 cached decode steps: the oracle against transformers
  rng = np.random.default_rng(21)
  c = small(rope=rope)
  w = OL.random_weights(c, rng, sd=0.05, norm_sd=0.3)
  m = hf_llama(c, w)
  ids = [int(i) for i in rng.integers(0, c.vocab, 9)]
  with torch.no_grad():
    want = m(torch.tensor([ids])).logits[0].numpy()
  got = OL.forward(ids, range(len(ids)), w, c, OL.kv_cache(c, 32), every=True)
  err = np.abs(got - want).max() / np.abs(want).max()
  assert err < 1e-5, err  # (transformers' RMSNorm computes in fp32)
  # decode a token at a time from the cache: the same logits as the whole sequence at once
  caches = OL.kv_cache(c, 32)
  OL.forward(ids[:6], range(6), w, c, caches)
  for p in range(6, 9):
    step = OL.forward([ids[p]], [p], w, c, caches)[0]
    assert np.abs(step - got[p]).max() <= 1e-6 * np.abs(got[p]).max(), p  # (float32 first-block products: BLAS order)


def test_prefill_in_chunks_is_the_whole_prompt():
  # llama.prefill's chunks (models/llama.py:498-504) against the prompt at once (test_chunked_prefill's invariant)
  rng = np.random.default_rng(22)
  c = small()
  w = OL.random_weights(c, rng, sd=0.05, norm_sd=0.3)
  ids = [int(i) for i in rng.integers(0, c.vocab, 21)]
  whole = OL.forward(ids, range(21), w, c, OL.kv_cache(c, 32))[0]
  chunks = OL.prefill(ids, w, c, OL.kv_cache(c, 32), 8)[0]
  assert np.allclose(whole, chunks, rtol=1e-9, atol=1e-9)


def test_moe_matches_mixtral():
  # the oracle's mixture of experts (models/llama.py:277-300) against transformers' Mixtral block: softmax over the
  # top-k logits is the renormalised top-k of the softmax over all
  pytest.importorskip("transformers.models.mixtral.modeling_mixtral")
  from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
  rng = np.random.default_rng(23)
  dim, ffn, E, k = 64, 96, 8, 2
  c = OL.model(dim=dim, k=k, experts=E)
  p = {"router": O.bf16(rng.normal(0, 0.5, (dim, E))), "experts.gate_up": O.bf16(rng.normal(0, 0.1, (E, dim, 2 * ffn))),
       "experts.down": O.bf16(rng.normal(0, 0.1, (E, ffn, dim)))}
  h = O.bf16(rng.normal(0, 1, (7, dim))).astype(np.float64)
  got, ids, wts = OL.moe(h, p, c)
  blk = MixtralSparseMoeBlock(transformers.MixtralConfig(hidden_size=dim, intermediate_size=ffn, num_local_experts=E,
                                                         num_experts_per_tok=k)).double().eval()
  t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float64))
  blk.load_state_dict({"gate.weight": t(p["router"].T), "experts.gate_up_proj": t(p["experts.gate_up"].transpose(0, 2, 1)),
                       "experts.down_proj": t(p["experts.down"].transpose(0, 2, 1))})
  with torch.no_grad():
    want = blk(t(h)[None])[0].numpy() if not isinstance(blk(t(h)[None]), tuple) else blk(t(h)[None])[0][0].numpy()
  assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max(), np.abs(got - want).max()
  # the picks: the oracle's ids, largest first, are the router's top-k indices, and its weights the router's
  # renormalised top-k probabilities (transformers' router computes them in float32)
  with torch.no_grad():
    _, scores, idx = blk.gate(t(h))
  assert np.array_equal(ids, idx.numpy()), (ids, idx.numpy())
  assert np.abs(wts - scores.numpy()).max() <= 1e-6 and np.allclose(wts.sum(1), 1)


def test_forward_slots_is_each_sequences_forward():
  # several sequences a step (forward_slots, models/llama.py's slots) against each sequence's own forward: the same
  # logits, row by row, and the same caches; a slip in a row's own cache or place would differ by far more
  rng = np.random.default_rng(24)
  c = small()
  w = OL.random_weights(c, rng, sd=0.05, norm_sd=0.3)
  S, size = 3, 16
  caches = [OL.kv_cache(c, size) for _ in range(S)]
  alone = [OL.kv_cache(c, size) for _ in range(S)]
  prompts = [[int(i) for i in rng.integers(0, c.vocab, n)] for n in (5, 9, 1)]
  for b, ids in enumerate(prompts):  # the sequences' prompts, each into both of its caches
    OL.forward(ids, range(len(ids)), w, c, caches[b])
    OL.forward(ids, range(len(ids)), w, c, alone[b])
  toks, places = [3, 17, 40], [len(p) for p in prompts]
  got = OL.forward_slots(toks, places, w, c, caches)
  for b in range(S):
    want = OL.forward([toks[b]], [places[b]], w, c, alone[b])[0]
    # (the first block's float32 products sum in BLAS's order for 3 rows or 1: within float32's rounding)
    assert np.abs(got[b] - want).max() <= 1e-6 * np.abs(want).max(), b
    assert all(np.abs(x - y).max() <= 1e-6 * np.abs(y).max() for x, y in zip(caches[b], alone[b]))
