"""Contracts of the C-ABI that no parity test covers by itself, on the GPU:
- a workspace needs no clearing: fh_attention_decode, fh_moe_experts and fh_logit_heads give the same bits on a
  workspace filled with NaN bytes as on a zeroed one (include/ferrite_hip.h's workspace rule);
- an FH_EP_PROGRAM epilogue reads its per-row inputs at the call's row when the GEMV takes more rows than one launch
  does (rows 8 and up: several launches, each its own rows);
- the Decoder refuses, on the host, a slot outside its cache and a step past its context (so no kernel is ever handed
  a cache row outside the cache);
- fh_read_probe, the read floor bench.py measures the GEMVs against, reads every byte it is given."""
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


def nan_bytes(n):
  return torch.full((max(n, 256),), 0xFF, dtype=torch.uint8, device="cuda")


def test_attention_workspace_needs_no_clearing(cuda):
  rng = np.random.default_rng(91)
  hd, heads, kv, batch, part = 128, 32, 8, 4, 700
  places = np.array([0, 63, 450, 699], np.int32)
  first = np.arange(batch, dtype=np.int32) * part
  cache = to_gpu(O.bf16(rng.normal(0, 1, (2 * kv, batch * part, hd))), torch.bfloat16)
  q = to_gpu(rng.normal(0, 1, (batch, heads * hd)))
  n = ops().attention_workspace(batch, heads, hd, part).numel()
  args = (heads, kv, hd, to_gpu(places, torch.int32), to_gpu(first, torch.int32), part)
  zero = ops().attention_decode(q, cache, *args, torch.zeros(n, dtype=torch.uint8, device="cuda"))
  nan = ops().attention_decode(q, cache, *args, nan_bytes(n))
  assert torch.equal(zero, nan) and not torch.isnan(nan).any()


def test_moe_workspace_needs_no_clearing(cuda):
  rng = np.random.default_rng(92)
  T, dim, ffn, E, k = 40, 256, 512, 8, 2
  gu = to_gpu(O.bf16(rng.normal(0, 0.05, (E, dim, 2 * ffn))))
  dn = to_gpu(O.bf16(rng.normal(0, 0.05, (E, ffn, dim))))
  ex = ops().pack_experts(gu, dn, "bfp4")
  x = to_gpu(rng.normal(0, 1, (T, dim)))
  router = to_gpu(O.bf16(rng.normal(0, 0.5, (dim, E))), torch.bfloat16)
  _, _, dense = ops().moe_route(x, router, E, k)
  from ferrite_amd import lib
  n = lib.load().fh_moe_workspace_bytes(T, E, ffn, dim)
  zero = ops().moe_experts(x, ex, dense, ws=torch.zeros(n, dtype=torch.uint8, device="cuda"))
  nan = ops().moe_experts(x, ex, dense, ws=nan_bytes(n))
  assert torch.equal(zero, nan) and not torch.isnan(nan).any()


def test_heads_workspace_needs_no_clearing(cuda):
  rng = np.random.default_rng(93)
  logits = to_gpu(rng.normal(0, 3, (3, 50000)))
  from ferrite_amd import lib
  n = lib.load().fh_heads_workspace_bytes(3, 50000, 64)
  assert n > 0
  a = ops().logit_heads(logits, 64, ws=torch.zeros(n, dtype=torch.uint8, device="cuda"))
  b = ops().logit_heads(logits, 64, ws=nan_bytes(n))
  assert all(torch.equal(u, v) for u, v in zip(a, b))


@pytest.mark.parametrize("rows", [9, 20])
def test_program_epilogue_reads_each_rows_inputs(cuda, rows):
  # K = 48 is no multiple of 32: the lazy matmul takes the exact-product GEMV, which runs more than 8 rows as several
  # launches; a per-row input (Y, [rows][N]) must be read at each launch's own rows
  from ferrite_amd import tensor
  rt = tensor.Runtime(0)
  rng = np.random.default_rng(94)
  K, N = 48, 64
  x = rng.normal(0, 1, (rows, K)).astype(np.float32)
  w = rng.normal(0, 0.1, (K, N)).astype(np.float32)
  y = O.bf16(rng.normal(0, 1, (rows, N)))
  X, Y = tensor.Tensor.of(rt, x.tolist(), "fp32"), tensor.Tensor.of(rt, y.tolist(), "fp32")
  W = tensor.Tensor.of(rt, w.tolist(), "fp32").cast("bfp8")
  got = (X @ W + Y).relu().numpy()[0]
  want = np.maximum(x.astype(np.float64) @ O.bfp(w) + y, 0)
  bound = 1e-5 * (np.abs(x) @ np.abs(O.bfp(w)) + np.abs(y)) + 1e-30
  assert (np.abs(got - want) <= bound).all(), float((np.abs(got - want) / bound).max())


def test_decoder_refuses_rows_outside_its_cache(cuda):
  from ferrite_amd import llama as G
  c = G.model(dim=128, heads=2, kv=1, layers=1, eps=1e-5, theta=1e4, vocab=64, ffn=128, places=16)
  dec = G.Decoder(c, G.random_weights(c, seed=3), mode="bfp8", kv="bf16", batch=2, context=8, slots=2)
  with pytest.raises(ValueError, match="slot"):
    dec.set_rows([0, 1], [0, 2])
  with pytest.raises(ValueError, match="place"):
    dec.set_rows([0, 8], [0, 1])
  with pytest.raises(ValueError, match="slot"):
    dec.prefill([1, 2], slot=2)
  dec.step([1, 2], [5, 6], slots=[0, 1], replay=False)
  dec.advance()  # places 6 and 7: the last row of each slot
  with pytest.raises(ValueError, match="advance"):
    dec.advance()


def test_read_probe_reads_every_byte(cuda):
  # fh_read_probe (bench.py's read floor): the xor of the workgroups' sinks is the xor of every 32-bit word, so each
  # byte was read, once or an odd number of times; sizes with a ragged tail past the four-load steps
  from ferrite_amd import lib
  rng = np.random.default_rng(71)
  for words, blocks in ((4, 1), (4 * 1000 + 4, 7), (1 << 20, 2048), ((1 << 20) + 36, 2048)):
    data = rng.integers(0, 1 << 32, words, dtype=np.uint32)
    src = torch.from_numpy(data.view(np.int32)).cuda()
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    lib.call("fh_read_probe", src.data_ptr(), 4 * words, sink.data_ptr(), blocks, torch.cuda.current_stream().cuda_stream)
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(data), (words, blocks)
  with pytest.raises(ValueError):
    lib.call("fh_read_probe", src.data_ptr(), 10, sink.data_ptr(), blocks, None)
