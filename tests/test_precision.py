"""The precision tables: which format each matmul's weights take in each mode (models/llama.py:54-76, 615-623), pinned by
the reference's own known answers (test_llama_precision, test/test_sim.py:1999-2008), and the GPU path's table
(ferrite_amd/llama.py:precision, which the Decoder packs by) giving the same format for every (op, block). No GPU."""
import pytest
from oracle import llama as OL
from ferrite_amd import llama as G


def test_reference_answers():
  # test_sim.py:1999-2008, the same assertions on the oracle's tables
  big = OL.model(layers=32, dim=4096)
  assert OL.precision(big, "tt")["gate_up", 31] == ("bfp8", 2) and OL.precision(big, "tt")["gate_up", 30] == ("bfp4", 1)
  assert OL.precision(big, "tt")["head", None] == ("bfp8", 2) and OL.precision(big, "bf16")["qkv", 0] == ("bf16", 4)
  tt = OL.precision(big, "tt")
  assert [tt[k] for k in (("attention", "decode"), ("attention", "prefill"), ("kv", None))] == [(None, 2), (None, 4), ("bfp8", None)]
  experts = OL.precision(big, "experts")
  keys = (("gate_up", 31), ("down", 0), ("qkv", 5), ("head", None), ("draft head", None), ("kv", None))
  assert [experts[k] for k in keys] == [("bfp4", 1), ("bfp4", 1), ("bfp8", 2), ("bfp8", 2), ("bfp4", 1), ("bfp8", None)]
  assert OL.weight_format("layers.3.shared_expert.down_proj", experts) == OL.weight_format("layers.3.experts.down", experts) == "bfp4"
  assert OL.weight_format("embed.T draft", experts) == "bfp4" and ("draft head", None) not in OL.precision(big, "tt")


def test_modes_by_op():
  # what each mode's docstring says (models/llama.py:54-66), op by op, and the cache's format
  c = OL.model(layers=3, dim=576)
  for mode, fmt in (("bf16", "bf16"), ("bfp8", "bfp8")):
    p = OL.precision(c, mode)
    assert all(p[op, l] == (fmt, 4) for l in range(3) for op in ("qkv", "o", "gate_up", "down")) and p["head", None] == (fmt, 4)
    assert p["kv", None] == ("bf16", None)
  p = OL.precision(c, "bfp4")
  assert [p[op, 1] for op in ("qkv", "o", "gate_up", "down")] == [("bfp8", 4), ("bfp8", 4), ("bfp4", 4), ("bfp8", 4)]
  p = OL.precision(c, "tt")  # (the last block's gate_up stays bfp4 away from Llama-3.1-8B's shape)
  assert p["gate_up", 2] == ("bfp4", 1) and p["down", 2] == ("bfp8", 2) and p["kv", None] == ("bfp8", None)
  assert OL.precision(c, "tt", kv="bf16")["kv", None] == ("bf16", None)
  assert OL.precision(OL.model(layers=32, dim=2048), "tt")["gate_up", 31] == ("bfp4", 1)
  assert OL.weight_format("layers.1.input_layernorm", p) == "bf16" and OL.weight_format("embed", p) == "bf16"
  assert OL.weight_format("layers.1.gate_up_proj", p) == "bfp4" and OL.weight_format("embed.T", p) == "bfp8"
  assert OL.weight_format("layers.1.o_proj", None) == "bf16"


@pytest.mark.parametrize("layers,dim", [(30, 576), (32, 4096), (2, 4096), (32, 2048)])
@pytest.mark.parametrize("mode", ["bfp8", "bfp4", "tt", "experts"])
def test_gpu_table_is_the_oracles(layers, dim, mode):
  # the Decoder's formats are the oracle's, for every matrix it packs
  c = OL.model(layers=layers, dim=dim)
  want = OL.precision(c, mode)
  got = G.precision(G.model(dim=dim, heads=1, kv=1, layers=layers, eps=1e-5, theta=1e4, vocab=16, ffn=16), mode)
  assert set(got) == {(op, l) for l in range(layers) for op in ("qkv", "o", "gate_up", "down")} | {("head", None)}
  assert all(got[k] == want[k][0] for k in got), [k for k in got if got[k] != want[k][0]]
