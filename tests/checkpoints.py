"""Synthetic Hugging Face checkpoints for the loader's tests: safetensors files written from numpy (an 8-byte header
size, the JSON header, the data), Llama- and Mixtral-named as their checkpoints are, in one file or two with an index
(the layout test/test_sim.py:1363-1389 writes), and the same weights fused for x @ W as models/llama.py's load and
fuse give them (llama.py:376-427, 572-604)."""
import json
import struct
import numpy as np
from oracle import bfp as O


def write_safetensors(path, tensors):
  """{name: array} as a safetensors file: uint16 arrays are bf16 bits (BF16), float32 arrays F32."""
  header, blobs, off = {}, [], 0
  for name, a in tensors.items():
    a = np.ascontiguousarray(a)
    dtype = {np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32"}[a.dtype]
    header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
    blobs.append(a.tobytes())
    off += a.nbytes
  head = json.dumps(header).encode()
  path.write_bytes(struct.pack("<Q", len(head)) + head + b"".join(blobs))


def values(a):
  """A stored tensor's values as the loader reads them: bf16 bits as floats, fp32 rounded to bf16 (nearest even)."""
  return O.bf16_floats(a) if a.dtype == np.uint16 else O.bf16(a)


def llama(folder, rng, dim=256, heads=4, kv=2, layers=2, ffn=384, vocab=512, tied=False, experts=0, k=2, two_files=True,
          rope=None):
  """A checkpoint folder: config.json and the tensors (attention and output layer bf16, the MLP's gate and up and the
  norms fp32, so both are read). Returns the tensors by checkpoint name."""
  hd = dim // heads
  bits = lambda *shape: O.bf16_bits(rng.normal(0, 0.05, shape).astype(np.float32))
  f32 = lambda *shape: rng.normal(0, 0.05, shape).astype(np.float32)
  t = {"model.embed_tokens.weight": bits(vocab, dim), "model.norm.weight": 1 + f32(dim)}
  if not tied: t["lm_head.weight"] = bits(vocab, dim)
  for l in range(layers):
    p = f"model.layers.{l}."
    t |= {p + "input_layernorm.weight": 1 + f32(dim), p + "post_attention_layernorm.weight": 1 + f32(dim),
          p + "self_attn.q_proj.weight": bits(heads * hd, dim), p + "self_attn.k_proj.weight": bits(kv * hd, dim),
          p + "self_attn.v_proj.weight": bits(kv * hd, dim), p + "self_attn.o_proj.weight": bits(dim, heads * hd)}
    if experts:  # Mixtral's names: w1 gate, w2 down, w3 up; the router "gate"
      t[p + "block_sparse_moe.gate.weight"] = bits(experts, dim)
      for e in range(experts):
        q = f"{p}block_sparse_moe.experts.{e}."
        t |= {q + "w1.weight": f32(ffn, dim), q + "w2.weight": bits(dim, ffn), q + "w3.weight": f32(ffn, dim)}
    else:
      t |= {p + "mlp.gate_proj.weight": f32(ffn, dim), p + "mlp.up_proj.weight": f32(ffn, dim),
            p + "mlp.down_proj.weight": bits(dim, ffn)}
  names = list(t)
  if two_files:
    half = len(names) // 2
    files = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    for f, ns in files.items(): write_safetensors(folder / f, {n: t[n] for n in ns})
    (folder / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {n: f for f, ns in files.items() for n in ns}}))
  else:
    write_safetensors(folder / "model.safetensors", t)
  cfg = {"hidden_size": dim, "num_attention_heads": heads, "num_key_value_heads": kv, "num_hidden_layers": layers,
         "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "max_position_embeddings": 131072, "vocab_size": vocab,
         "intermediate_size": ffn, "tie_word_embeddings": tied}
  if rope: cfg["rope_scaling"] = rope
  if experts: cfg |= {"num_local_experts": experts, "num_experts_per_tok": k}
  (folder / "config.json").write_text(json.dumps(cfg))
  return t


def fused(t, layers, tied):
  """The same weights as x @ W takes them, fused (models/llama.py's load and fuse), values as float32:
  {layers.l.qkv_proj, o_proj, gate_up_proj, down_proj, norms, norm, embed, embed.T}."""
  v = lambda n: values(t[n])
  w = {"embed": v("model.embed_tokens.weight"), "norm": v("model.norm.weight")[None]}
  w["embed.T"] = np.ascontiguousarray((w["embed"] if tied else v("lm_head.weight")).T)
  for l in range(layers):
    p, q = f"model.layers.{l}.", f"layers.{l}."
    w[q + "input_layernorm"] = v(p + "input_layernorm.weight")[None]
    w[q + "post_attention_layernorm"] = v(p + "post_attention_layernorm.weight")[None]
    w[q + "qkv_proj"] = np.concatenate([v(p + f"self_attn.{n}_proj.weight").T for n in "qkv"], 1)
    w[q + "o_proj"] = np.ascontiguousarray(v(p + "self_attn.o_proj.weight").T)
    if p + "mlp.gate_proj.weight" in t:
      w[q + "gate_up_proj"] = np.concatenate([v(p + "mlp.gate_proj.weight").T, v(p + "mlp.up_proj.weight").T], 1)
      w[q + "down_proj"] = np.ascontiguousarray(v(p + "mlp.down_proj.weight").T)
  return w
