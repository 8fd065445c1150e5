"""The checkpoint reader's host side (no GPU): config.json as models/llama.py's config reads it, tensor names as
load keys them (Mixtral's w1/w2/w3 included), the mapped files' values, the index of two files (the reference's
test_llama_load, test/test_sim.py:1371-1396, on this loader)."""
import json
import numpy as np
import pytest
import checkpoints as C
from ferrite_amd import checkpoint as K


def test_config_and_names(tmp_path):
  rope = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
  t = C.llama(tmp_path, np.random.default_rng(40), layers=1, rope=rope)
  c = K.config(str(tmp_path), places=64)
  assert (c.dim, c.heads, c.kv, c.layers, c.ffn, c.vocab, c.places, c.tied) == (256, 4, 2, 1, 384, 512, 64, False)
  assert c.rope == rope and c.theta == 500000.0 and c.eps == 1e-5 and c.experts == 0
  ck = K.Checkpoint(str(tmp_path))
  assert set(ck.tensors) == {K._name(n) for n in t} and "layers.0.q_proj" in ck.tensors and "lm_head" in ck.tensors
  for name, a in t.items():
    got = ck.host(K._name(name))
    assert got.dtype == a.dtype and np.array_equal(got, a), name  # (the mapped bytes as they were written)
  assert ck._parts("layers.0.qkv_proj") == ["layers.0.q_proj", "layers.0.k_proj", "layers.0.v_proj"]
  assert ck._parts("embed.T") == ["lm_head"]


def test_mixtral_names_and_tied(tmp_path):
  C.llama(tmp_path, np.random.default_rng(41), layers=1, experts=4, k=2, tied=True, two_files=False)
  c = K.config(str(tmp_path))
  assert (c.experts, c.k, c.tied, c.norm_topk, c.places) == (4, 2, True, True, 4096)
  ck = K.Checkpoint(str(tmp_path))
  assert {"layers.0.gate", "layers.0.experts.3.gate_proj", "layers.0.experts.3.down_proj", "layers.0.experts.3.up_proj"} <= set(ck.tensors)
  assert ck._parts("embed.T") == ["embed_tokens"]  # no lm_head: the embedding's rows


def test_refuses_what_it_cannot_read(tmp_path):
  C.write_safetensors(tmp_path / "model.safetensors", {"model.embed_tokens.weight": np.zeros((4, 16), np.float32)})
  header, data = K._safetensors(str(tmp_path / "model.safetensors"))
  assert header["model.embed_tokens.weight"]["dtype"] == "F32" and data.size == 4 * 16 * 4
  cfg = {"hidden_size": 16, "num_attention_heads": 1, "num_key_value_heads": 1, "num_hidden_layers": 1, "rms_norm_eps": 1e-5,
         "rope_theta": 1e4, "max_position_embeddings": 32, "vocab_size": 4, "intermediate_size": 16,
         "rope_scaling": {"rope_type": "yarn", "factor": 4.0}}
  (tmp_path / "config.json").write_text(json.dumps(cfg))
  with pytest.raises(NotImplementedError, match="yarn"):
    K.config(str(tmp_path))


@pytest.mark.parametrize("extra,match", [({"sliding_window": 64}, "sliding window"), ({"layer_types": ["linear_attention"]}, "layer_types"),
                                         ({"model_type": "qwen3_5_moe"}, "qwen3_5"), ({"shared_expert_intermediate_size": 32}, "shared_expert")])
def test_refuses_blocks_it_cannot_run(tmp_path, extra, match):
  # a config whose blocks this path does not run raises rather than loading into wrong logits; a window that covers
  # every place the tables hold changes nothing and loads
  cfg = {"hidden_size": 16, "num_attention_heads": 1, "num_key_value_heads": 1, "num_hidden_layers": 1, "rms_norm_eps": 1e-5,
         "rope_theta": 1e4, "max_position_embeddings": 256, "vocab_size": 4, "intermediate_size": 16}
  (tmp_path / "config.json").write_text(json.dumps(cfg | extra))
  with pytest.raises(NotImplementedError, match=match):
    K.config(str(tmp_path), places=128)
  (tmp_path / "config.json").write_text(json.dumps(cfg | {"sliding_window": 4096}))
  assert K.config(str(tmp_path), places=128).places == 128


@pytest.mark.parametrize("name", ["model.layers.0.self_attn.q_proj.bias", "model.layers.0.self_attn.k_norm.weight"])
def test_refuses_tensors_it_cannot_apply(tmp_path, name):
  # Qwen2's q/k/v biases and Qwen3's q/k norms are refused at load, not silently dropped
  C.write_safetensors(tmp_path / "model.safetensors", {"model.embed_tokens.weight": np.zeros((4, 16), np.float32),
                                                       name: np.zeros((16,), np.float32)})
  with pytest.raises(NotImplementedError, match="not on this path"):
    K.Checkpoint(str(tmp_path), device="cpu")


def test_packed_file_round_trip(tmp_path):
  # save_packed's file read back by Packed (on the CPU: any torch tensors): the matrices' bytes with their format and
  # shape, the norms, the embedding; a file of another kind refused
  import torch
  from types import SimpleNamespace
  from ferrite_amd import ops
  rng = np.random.default_rng(46)
  u8 = lambda n: torch.from_numpy(rng.integers(0, 256, n).astype(np.uint8))
  mat = lambda K, N, fmt: ops.BfpWeight(u8(K * N // (1 if fmt == "bfp8" else 2)), u8(K * N // 16), K, N, fmt)
  f32 = lambda n: torch.from_numpy(rng.normal(0, 1, n).astype(np.float32))
  L = SimpleNamespace(qkv=mat(64, 96, "bfp8"), o=mat(32, 64, "bfp8"), gate_up=mat(64, 128, "bfp4"), down=mat(64, 64, "bfp4"),
                      norm1=f32(64), norm2=f32(64))
  dec = SimpleNamespace(mode="bfp4", layers=[L], norm=f32(64), embed=f32((10, 64)).to(torch.bfloat16), head=mat(64, 16, "bfp8"))
  path = str(tmp_path / "p.safetensors")
  K.save_packed(dec, path)
  p = K.Packed(path, device="cpu")
  for name, bw in (("layers.0.qkv_proj", L.qkv), ("layers.0.gate_up_proj", L.gate_up), ("embed.T", dec.head)):
    got = p.pack(name, bw.fmt)
    assert (got.K, got.N, got.fmt) == (bw.K, bw.N, bw.fmt) and torch.equal(got.mant, bw.mant) and torch.equal(got.exps, bw.exps)
  with pytest.raises(ValueError): p.pack("layers.0.qkv_proj", "bfp4")
  assert torch.equal(p.vector("layers.0.post_attention_layernorm"), L.norm2) and torch.equal(p.vector("norm"), dec.norm)
  assert torch.equal(p.table(), dec.embed)
  C.write_safetensors(tmp_path / "other.safetensors", {"x": np.zeros((2, 2), np.float32)})
  with pytest.raises(ValueError): K.Packed(str(tmp_path / "other.safetensors"), device="cpu")
