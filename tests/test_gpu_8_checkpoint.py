"""A checkpoint onto the GPU (ferrite_amd.checkpoint: models/llama.py's load, fuse and upload, llama.py:376-427,
572-604, 628-640): each fused matrix packed straight from the checkpoint's rows is byte for byte the packing of the
fused, transposed matrix (and its values numpy's bfp of it, bit for bit); a Decoder loaded from the files gives
exactly the logits of one built from the same weights fused in numpy; a mixture's experts and router likewise."""
import numpy as np
import pytest
import torch
import checkpoints as C
from oracle import bfp as O

pytestmark = pytest.mark.gpu


def test_fused_matrices_from_rows(cuda, tmp_path):
  from ferrite_amd import checkpoint as K, ops
  t = C.llama(tmp_path, np.random.default_rng(42), layers=1)
  ck = K.Checkpoint(str(tmp_path))
  w = C.fused(t, 1, tied=False)
  for name, fmt in (("layers.0.qkv_proj", "bfp8"), ("layers.0.gate_up_proj", "bfp4"), ("layers.0.o_proj", "bfp8"),
                    ("layers.0.down_proj", "bfp4"), ("embed.T", "bfp8")):
    got = ck.pack(name, fmt)
    want = ops.pack(torch.from_numpy(w[name]).cuda(), fmt)
    assert (got.K, got.N) == (want.K, want.N), name
    assert torch.equal(got.mant, want.mant) and torch.equal(got.exps, want.exps), name
    q, top = O.bfp_parts(w[name], fmt)
    bits = ops.dequant(got).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(bits, O.exact_bf16(q, top, fmt)), name
  assert torch.equal(ck.vector("layers.0.input_layernorm").cpu(), torch.from_numpy(w["layers.0.input_layernorm"][0]))


@pytest.mark.parametrize("tied", [False, True])
def test_decoder_from_checkpoint(cuda, tmp_path, tied):
  # the same model from the files and from numpy: identical packed weights, so identical logits, step by step
  from ferrite_amd import checkpoint as K, llama as G
  rope = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
  t = C.llama(tmp_path, np.random.default_rng(43), layers=2, tied=tied, rope=rope)
  c = K.config(str(tmp_path), places=64)
  a = G.Decoder(c, K.Checkpoint(str(tmp_path)), mode="bfp4", kv="bf16", context=64)
  b = G.Decoder(c, G.numpy_weights(C.fused(t, 2, tied)), mode="bfp4", kv="bf16", context=64)
  for L, M in zip(a.layers, b.layers):
    for n in ("qkv", "o", "gate_up", "down"):
      assert torch.equal(getattr(L, n).mant, getattr(M, n).mant) and torch.equal(getattr(L, n).exps, getattr(M, n).exps), n
    assert torch.equal(L.norm1, M.norm1) and torch.equal(L.norm2, M.norm2)
  assert torch.equal(a.head.mant, b.head.mant) and torch.equal(a.embed, b.embed)
  for i, tok in enumerate([5, 300, 17]):
    la = a.step([tok], [i], replay=False)[0].cpu()
    lb = b.step([tok], [i], replay=False)[0].cpu()
    assert torch.equal(la, lb) and torch.isfinite(la).all(), i


def test_packed_weights_file(cuda, tmp_path):
  # a Decoder's packed weights saved once (save_packed) and loaded back (Packed) without the checkpoint or a repacking:
  # the same bytes, so the same logits bit for bit; a precision that asks another format is refused
  from ferrite_amd import checkpoint as K, llama as G
  t = C.llama(tmp_path, np.random.default_rng(45), layers=2, tied=True)
  c = K.config(str(tmp_path), places=64)
  a = G.Decoder(c, K.Checkpoint(str(tmp_path)), mode="bfp4", kv="bf16", context=64)
  path = str(tmp_path / "packed.safetensors")
  K.save_packed(a, path)
  b = G.Decoder(c, K.Packed(path), mode="bfp4", kv="bf16", context=64)
  for L, M in zip(a.layers, b.layers):
    for n in ("qkv", "o", "gate_up", "down"):
      assert torch.equal(getattr(L, n).mant, getattr(M, n).mant) and torch.equal(getattr(L, n).exps, getattr(M, n).exps), n
  assert torch.equal(a.head.mant, b.head.mant) and torch.equal(a.embed, b.embed) and torch.equal(a.norm, b.norm)
  for i, tok in enumerate([5, 300, 17]):
    assert torch.equal(a.step([tok], [i], replay=False)[0].cpu(), b.step([tok], [i], replay=False)[0].cpu()), i
  with pytest.raises(ValueError): G.Decoder(c, K.Packed(path), mode="bfp8", kv="bf16", context=64)


def test_mixtral_experts_from_rows(cuda, tmp_path):
  from ferrite_amd import checkpoint as K, ops
  t = C.llama(tmp_path, np.random.default_rng(44), layers=1, experts=4, ffn=128)
  ck = K.Checkpoint(str(tmp_path))
  ex = ck.experts(0, "bfp4")
  v = lambda n: C.values(t[n])
  p = "model.layers.0.block_sparse_moe."
  gu = np.stack([np.concatenate([v(f"{p}experts.{e}.w1.weight").T, v(f"{p}experts.{e}.w3.weight").T], 1) for e in range(4)])
  dn = np.stack([v(f"{p}experts.{e}.w2.weight").T for e in range(4)])
  want = ops.pack_experts(torch.from_numpy(gu).cuda(), torch.from_numpy(np.ascontiguousarray(dn)).cuda(), "bfp4")
  assert (ex.experts, ex.dim, ex.ffn) == (want.experts, want.dim, want.ffn) == (4, 256, 128)
  assert (ex.gate_up.K, ex.gate_up.N, ex.down.K, ex.down.N) == (want.gate_up.K, want.gate_up.N, want.down.K, want.down.N)
  for a, b in ((ex.gate_up, want.gate_up), (ex.down, want.down)):
    assert torch.equal(a.mant, b.mant) and torch.equal(a.exps, b.exps)
  assert torch.equal(ck.router(0).float().cpu(), torch.from_numpy(np.ascontiguousarray(v(p + "gate.weight").T)))
