"""A Hugging Face checkpoint (config.json and safetensors) onto the GPU, for Decoder and the mixture-of-experts path:
models/llama.py's config, load, fuse and upload (llama.py:541-604, 376-427, 628-640), MI355X's way. The files are
memory-mapped and read a tensor at a time; each tensor's bytes go to the GPU as they are (bf16, or fp32, which the
packer rounds to bf16 to nearest even as gpt2.tensor_bits does); a linear layer is packed straight from its [out][in]
rows (ops.pack_rows_into: along its first axis, which is x @ W's layout of its transpose), q|k|v and gate|up into one
block float each, so neither the host nor the GPU forms a transposed or fused copy. At most one matrix's bytes are on
the GPU besides the packed model.

  c = checkpoint.config(folder, places=2048)
  dec = Decoder(c, checkpoint.Checkpoint(folder), mode="bfp4", kv="bfp8")
"""
import json
import os
import re
import struct
import warnings
import numpy as np
import torch
from ferrite_amd import llama as G, ops


def _json(path):
  with open(path, encoding="utf-8") as f:
    return json.load(f)


def config(folder, places=4096):
  """The model of a checkpoint's config.json (models/llama.py:541-570) for the blocks this path runs: Llama's, SmolLM's,
  Mistral's (where its sliding window covers every place the tables hold) and Mixtral's; RoPE plain or with Llama 3's
  scaling. places: the most places RoPE's tables need rows for (at most the model's). What it cannot run raises
  NotImplementedError rather than loading into wrong logits: a sliding window shorter than the places, Qwen3.5's
  gated and linear-attention blocks, a shared expert, dense blocks among a mixture's, gpt-oss's clamped GLU (and, in
  Checkpoint, the tensors of Qwen2's q/k/v biases, Qwen3's q/k norms, gpt-oss's sinks and o_proj bias)."""
  j = _json(os.path.join(folder, "config.json"))
  j = j.get("text_config", j)
  window = j.get("sliding_window") if j.get("use_sliding_window", True) else None
  if window and window < min(j["max_position_embeddings"], places):
    raise NotImplementedError(f"checkpoint: a sliding window of {window} places (attention here sees every place)")
  unsupported = [k for k in ("layer_types", "attn_output_gate", "linear_conv_kernel_dim", "shared_expert_intermediate_size",
                             "swiglu_limit", "mlp_only_layers") if j.get(k)]
  if j.get("decoder_sparse_step", 1) != 1: unsupported.append("decoder_sparse_step")
  if j.get("model_type", "").startswith(("qwen3_5", "qwen3_next", "gpt_oss")): unsupported.append(f"model_type {j['model_type']}")
  if unsupported: raise NotImplementedError(f"checkpoint: {', '.join(unsupported)} (not on this path)")
  rope = dict(j.get("rope_parameters") or (j.get("rope_scaling") or {}) | {"rope_theta": j["rope_theta"]})
  theta, kind = rope.pop("rope_theta"), rope.pop("type", None)
  rope.setdefault("rope_type", kind or "default")
  if rope["rope_type"] not in ("default", "llama3"):
    raise NotImplementedError(f"checkpoint: RoPE scaling {rope['rope_type']} (plain or llama3 on this path)")
  if rope.get("partial_rotary_factor", j.get("partial_rotary_factor")) not in (None, 1, 1.0):
    raise NotImplementedError("checkpoint: partial rotary embeddings")
  experts = j.get("num_experts") or j.get("num_local_experts") or 0
  return G.model(dim=j["hidden_size"], heads=j["num_attention_heads"], kv=j["num_key_value_heads"],
                 layers=j["num_hidden_layers"], eps=j["rms_norm_eps"], theta=theta,
                 places=min(j["max_position_embeddings"], places), vocab=j["vocab_size"],
                 ffn=j.get("moe_intermediate_size") if experts and j.get("moe_intermediate_size") else j.get("intermediate_size"),
                 head_dim=j.get("head_dim"), rope=rope if rope["rope_type"] != "default" else None,
                 tied=j.get("tie_word_embeddings", False), experts=experts, k=j.get("num_experts_per_tok") or 0,
                 norm_topk=j.get("norm_topk_prob", True))


def _safetensors(path):
  """A safetensors file: its header (each tensor's dtype, shape and byte range) and its data, memory-mapped
  (gpt2.safetensors, models/gpt2.py:34-38: 8 bytes of header size, the JSON header, the data)."""
  with open(path, "rb") as f:
    size = struct.unpack("<Q", f.read(8))[0]
    header = json.loads(f.read(size))
  header.pop("__metadata__", None)
  return header, np.memmap(path, np.uint8, "r", offset=8 + size)


def _name(full):
  """A tensor's name as models/llama.py:582-586 keys it: without "model." and ".weight", the attention's and MLP's
  scopes dropped, Mixtral's experts' w1/w2/w3 as gate/down/up."""
  name = full.removeprefix("model.").removeprefix("language_model.").removesuffix(".weight")
  for part in ("self_attn.", "mlp.", "block_sparse_moe."): name = name.replace(part, "")
  return re.sub(r"(experts\.\d+)\.w([123])$", lambda m: m[1] + (".gate_proj", ".down_proj", ".up_proj")[int(m[2]) - 1], name)


class Checkpoint:
  """The tensors of a checkpoint folder (model.safetensors, or the files model.safetensors.index.json names), read
  from the mapped files when asked. For Decoder: pack(name, fmt) gives the fused matrices the model reads
  (layers.l.qkv_proj, o_proj, gate_up_proj, down_proj; embed.T, the output layer: lm_head, or the embedding where the
  model has none), vector(name) the norms, table(name) the embedding; experts(l, fmt) and router(l) a mixture's."""

  def __init__(self, folder, device="cuda"):
    self.folder, self.device = folder, torch.device(device)
    index = os.path.join(folder, "model.safetensors.index.json")
    files = sorted(set(_json(index)["weight_map"].values())) if os.path.exists(index) else ["model.safetensors"]
    self.tensors = {}
    for file in files:
      header, data = _safetensors(os.path.join(folder, file))
      for full, t in header.items():
        if t["dtype"] not in ("BF16", "F32"): raise NotImplementedError(f"checkpoint: {full} is {t['dtype']} (BF16 or F32)")
        self.tensors[_name(full)] = (data, t)
    if "embed_tokens" not in self.tensors: raise ValueError("checkpoint: no embed_tokens")
    extra = sorted(n for n in self.tensors if n.endswith(("q_proj.bias", "k_proj.bias", "v_proj.bias", "o_proj.bias", "q_norm",
                                                          "k_norm", "sinks")))
    if extra: raise NotImplementedError(f"checkpoint: {extra[0]} and the like (biases, q/k norms, sinks) are not on this path")

  def shape(self, name):
    return tuple(self.tensors[name][1]["shape"])

  def host(self, name):
    """The tensor's values in the file, without a copy: bf16 bits as uint16, or float32."""
    data, t = self.tensors[name]
    raw = data[t["data_offsets"][0]:t["data_offsets"][1]]
    return (raw.view(np.uint16) if t["dtype"] == "BF16" else raw.view(np.float32)).reshape(t["shape"])

  def gpu(self, name):
    """The tensor on the GPU as the file holds it: bf16, or fp32."""
    a = self.host(name)
    with warnings.catch_warnings():  # (the mapped file is read-only; it is only read, by the copy to the GPU)
      warnings.filterwarnings("ignore", message="The given NumPy array is not writable")
      t = torch.from_numpy(np.ascontiguousarray(a))
    t = t.view(torch.bfloat16) if a.dtype == np.uint16 else t
    return t.to(self.device)

  def _parts(self, name):
    """The checkpoint rows a fused matrix is made of (models/llama.py:376-427, 602-603)."""
    if name == "embed.T": return ["lm_head"] if "lm_head" in self.tensors else ["embed_tokens"]
    pre, op = name.rsplit(".", 1)
    if op == "qkv_proj": return [f"{pre}.q_proj", f"{pre}.k_proj", f"{pre}.v_proj"]
    if op == "gate_up_proj": return [f"{pre}.gate_proj", f"{pre}.up_proj"]
    return [name]

  def pack(self, name, fmt, K=None):
    """Matrix `name` (x @ W's layout, W[K][N]) as a block float packed along N, from its parts' rows."""
    parts = self._parts(name)
    shapes = [self.shape(p) for p in parts]
    K = K or shapes[0][1]
    if any(len(s) != 2 or s[1] != K for s in shapes): raise ValueError(f"checkpoint: {name}'s parts {shapes} for K = {K}")
    bw = ops.bfp_empty(K, sum(s[0] for s in shapes), fmt, self.device)
    n0 = 0
    for p, s in zip(parts, shapes):
      ops.pack_rows_into(bw, self.gpu(p), n0)  # (one part's bytes at a time)
      n0 += s[0]
    return bw

  def vector(self, name):
    """A norm's weights in fp32 on the GPU, each a bf16 value (fp32 in the file rounded to nearest even, as
    gpt2.tensor_bits reads it)."""
    return self.gpu(name).to(torch.bfloat16).to(torch.float32).reshape(-1).contiguous()

  def table(self, name="embed_tokens"):
    """The embedding table [vocab][dim] in bf16 on the GPU (fp32 in the file rounded to nearest even)."""
    return self.gpu(name).to(torch.bfloat16).contiguous()

  def experts(self, layer, fmt="bfp4"):
    """Block `layer`'s experts as ops.Experts: each expert's gate|up (its [dim][2 ffn]) and its down ([ffn][dim]),
    packed one after another, straight from the checkpoint's rows (models/llama.py:418-422)."""
    pre = f"layers.{layer}.experts."
    E = sum(1 for k in self.tensors if k.startswith(pre) and k.endswith(".down_proj"))
    if not E: raise ValueError(f"checkpoint: block {layer} has no experts")
    ffn, dim = self.shape(f"{pre}0.gate_proj")
    gu = ops.bfp_empty(dim, 2 * ffn * E, fmt, self.device)   # (E blocks of [dim][2 ffn], one after another)
    dn = ops.bfp_empty(ffn, dim * E, fmt, self.device)       # (E blocks of [ffn][dim])
    one_gu, one_dn = [x // E for x in (gu.mant.numel(), gu.exps.numel())], [x // E for x in (dn.mant.numel(), dn.exps.numel())]
    for e in range(E):
      g = ops.BfpWeight(gu.mant[e * one_gu[0]:(e + 1) * one_gu[0]], gu.exps[e * one_gu[1]:(e + 1) * one_gu[1]], dim, 2 * ffn, fmt)
      ops.pack_rows_into(g, self.gpu(f"{pre}{e}.gate_proj"), 0)
      ops.pack_rows_into(g, self.gpu(f"{pre}{e}.up_proj"), ffn)
      d = ops.BfpWeight(dn.mant[e * one_dn[0]:(e + 1) * one_dn[0]], dn.exps[e * one_dn[1]:(e + 1) * one_dn[1]], ffn, dim, fmt)
      ops.pack_rows_into(d, self.gpu(f"{pre}{e}.down_proj"), 0)
    gu.N, dn.N = 2 * ffn, dim  # (each expert's own shape: fh_moe_experts steps through them)
    return ops.Experts(gu, dn, E, dim, ffn)

  def router(self, layer):
    """Block `layer`'s router as x @ router takes it, [dim][experts] (the checkpoint's rows transposed, llama.py:412),
    bf16 on the GPU."""
    name = f"layers.{layer}.router" if f"layers.{layer}.router" in self.tensors else f"layers.{layer}.gate"
    return self.gpu(name).to(torch.bfloat16).t().contiguous()


_DT = {torch.uint8: "U8", torch.float32: "F32", torch.bfloat16: "BF16"}
_NP = {"U8": np.uint8, "F32": np.float32, "BF16": np.uint16}


def save_packed(dec, path):
  """A Decoder's weights as it holds them, in one safetensors file (the packed-weights cache of models/llama.py's
  upload path, llama.py:628-640, for this layout): each block-float matrix's magnitudes and exponents as U8 (its format,
  K and N in the header's metadata), the norms as F32, the embedding as BF16. Packed(path) gives them back to a Decoder
  without a checkpoint or a repacking; the KV cache and the step's buffers are not saved."""
  tensors, meta = {}, {"format": "ferrite_amd packed", "mode": dec.mode}
  for l, L in enumerate(dec.layers):
    for op in ("qkv", "o", "gate_up", "down"):
      name, bw = f"layers.{l}.{op}_proj", getattr(L, op)
      tensors[name + ".mant"], tensors[name + ".exps"] = bw.mant, bw.exps
      meta[name] = f"{bw.fmt} {bw.K} {bw.N}"
    tensors[f"layers.{l}.input_layernorm"], tensors[f"layers.{l}.post_attention_layernorm"] = L.norm1, L.norm2
  tensors["norm"], tensors["embed_tokens"] = dec.norm, dec.embed
  tensors["embed.T.mant"], tensors["embed.T.exps"] = dec.head.mant, dec.head.exps
  meta["embed.T"] = f"{dec.head.fmt} {dec.head.K} {dec.head.N}"
  header, offset = {"__metadata__": meta}, 0
  for name, t in tensors.items():
    n = t.numel() * t.element_size()
    header[name] = {"dtype": _DT[t.dtype], "shape": list(t.shape), "data_offsets": [offset, offset + n]}
    offset += n
  raw = json.dumps(header).encode()
  raw += b" " * (-len(raw) % 8)
  with open(path, "wb") as f:
    f.write(struct.pack("<Q", len(raw)))
    f.write(raw)
    for t in tensors.values():  # (a tensor at a time through host memory)
      c = t.detach().contiguous().cpu()
      f.write((c.view(torch.int16) if c.dtype == torch.bfloat16 else c).numpy().tobytes())


class Packed:
  """A file save_packed wrote, for Decoder (as a Checkpoint): pack(name, fmt) gives the stored block float (which must
  be in fmt), vector(name) a norm, table() the embedding, each copied to the GPU as stored."""

  def __init__(self, path, device="cuda"):
    self.device = torch.device(device)
    with open(path, "rb") as f:
      size = struct.unpack("<Q", f.read(8))[0]
      header = json.loads(f.read(size))
    self.meta = header.pop("__metadata__", {})
    if self.meta.get("format") != "ferrite_amd packed": raise ValueError(f"{path}: not a file save_packed wrote")
    self.header, self.data = header, np.memmap(path, np.uint8, "r", offset=8 + size)

  def _gpu(self, name):
    t = self.header[name]
    raw = np.asarray(self.data[t["data_offsets"][0]:t["data_offsets"][1]]).view(_NP[t["dtype"]]).reshape(t["shape"])
    x = torch.from_numpy(raw.copy())
    return (x.view(torch.bfloat16) if t["dtype"] == "BF16" else x).to(self.device)

  def pack(self, name, fmt):
    if name not in self.meta: raise KeyError(f"packed file: no matrix {name}")
    stored, K, N = self.meta[name].split()
    if stored != fmt: raise ValueError(f"packed file: {name} is {stored}, the model's precision says {fmt}")
    return ops.BfpWeight(self._gpu(name + ".mant"), self._gpu(name + ".exps"), int(K), int(N), fmt)

  def vector(self, name):
    return self._gpu(name).reshape(-1).contiguous()

  def table(self, name="embed_tokens"):
    return self._gpu(name).contiguous()
