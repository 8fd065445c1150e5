"""fh_attention_decode_noalloc (the decode attention that allocates nothing: its partial results in the library's own
per-GPU scratch array) against fh_attention_decode with a workspace, through the C-ABI: the same bits, on two calls in
a row, the second with a smaller input (the scratch keeps the first call's contents, which the second must not read),
then the first again; a call past the scratch's maximum is refused on the host. No counterpart in the reference."""
import ctypes
import numpy as np
import pytest
import torch
from oracle import bfp as O

pytestmark = pytest.mark.gpu


def call_both(lib, ops, q, cache, heads, kv, hd, places, first, ctx, o_dtype):
  data, dtype, length = ops.cache_fields(cache)
  batch = q.shape[0]
  ws = torch.full((max(lib.load().fh_attention_workspace_bytes(batch, heads, hd, ctx), 256),), 0xFF, dtype=torch.uint8, device="cuda")
  o_ws = torch.empty(q.shape, dtype=o_dtype, device="cuda")
  o_na = torch.full(q.shape, float("nan"), dtype=o_dtype, device="cuda")
  common = (ops._ptr(q), ops._ptr(data), dtype, length, batch, heads, kv, hd, ops._ptr(places), ops._ptr(first), ctx)
  lib.call("fh_attention_decode", *common, ops._ptr(o_ws), ops._TORCH[o_dtype], ops._ptr(ws), ws.numel(), ops._stream())
  lib.call("fh_attention_decode_noalloc", *common, ops._ptr(o_na), ops._TORCH[o_dtype], ops._stream())
  torch.cuda.synchronize()
  return o_ws, o_na


def case(rng, batch, heads, kv, hd, part, fmt):
  from ferrite_amd import ops
  places = rng.integers(0, part, batch).astype(np.int32)
  places[:2] = [part - 1, 0]
  first = (np.arange(batch, dtype=np.int32) * part)[::-1].copy()
  vals = O.bf16(rng.normal(0, 1, (2 * kv, batch * part, hd)))
  cache = torch.from_numpy(vals).to("cuda").to(torch.bfloat16) if fmt == "bf16" else torch.from_numpy(vals).to("cuda")
  q = torch.from_numpy(rng.normal(0, 1, (batch, heads * hd)).astype(np.float32)).to("cuda")
  to = lambda a: torch.from_numpy(a).to("cuda")
  return q, cache, to(places), to(first)


def test_noalloc_matches_the_workspace_entry_point(cuda):
  from ferrite_amd import lib, ops
  rng = np.random.default_rng(97)
  # first: an 8B model's batch 16 at context 2048 (the matrix-core attention, 32 chunks a row, 8.5 MB of partials),
  # then a smaller call (batch 3 of 9 heads sharing 3 at context 300, fp32 cache: the VALU attention, fewer parts) that
  # must not read what the first left, then the first's shape again
  shapes = [(16, 32, 8, 128, 2048, "bf16", torch.bfloat16), (3, 9, 3, 64, 300, "fp32", torch.float32),
            (16, 32, 8, 128, 2048, "bf16", torch.float32)]
  for batch, heads, kv, hd, ctx, fmt, od in shapes:
    q, cache, places, first = case(rng, batch, heads, kv, hd, ctx, fmt)
    print(f"noalloc: batch {batch}, heads {heads}/{kv}, head_dim {hd}, context {ctx}, {fmt} cache, o {od}", flush=True)
    a, b = call_both(lib, ops, q, cache, heads, kv, hd, places, first, ctx, od)
    assert torch.equal(a, b), (batch, ctx, float((a.float() - b.float()).abs().max()))
    assert not torch.isnan(b.float()).any()


def test_noalloc_refuses_past_its_scratch(cuda):
  from ferrite_amd import lib
  # batch 32 of 32 heads at context 2048 needs 17 MB of partials: refused with the reason, nothing launched
  n = lib.load().fh_attention_workspace_bytes(32, 32, 128, 2048)
  assert n > 16 << 20
  dummy = ctypes.c_void_p(16)  # (never dereferenced: the bound is checked before anything else runs)
  with pytest.raises(ValueError, match="FH_ATTENTION_SCRATCH_BYTES"):
    lib.call("fh_attention_decode_noalloc", dummy, dummy, lib.BF16, 32 * 2048, 32, 32, 8, 128, dummy, dummy, 2048, dummy,
             lib.F32, None)


def test_noalloc_under_graph_capture(cuda):
  # the callers it is for: code under HIP graph capture. One call captured (torch.cuda.graph, on its side stream) and
  # replayed three times, with eager work on the same scratch between the replays (a call of another shape), each
  # replay's bits those of the workspace entry point. (The device's scratch address is looked up by the first call on
  # that device, made here outside the capture, as a caller warming up before capture does.)
  from ferrite_amd import lib, ops
  rng = np.random.default_rng(98)
  batch, heads, kv, hd, ctx = 16, 32, 8, 128, 2048
  q, cache, places, first = case(rng, batch, heads, kv, hd, ctx, "bf16")
  want, warm = call_both(lib, ops, q, cache, heads, kv, hd, places, first, ctx, torch.float32)
  assert torch.equal(want, warm)
  data, dtype, length = ops.cache_fields(cache)
  o = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
  common = (ops._ptr(q), ops._ptr(data), dtype, length, batch, heads, kv, hd, ops._ptr(places), ops._ptr(first), ctx)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    lib.call("fh_attention_decode_noalloc", *common, ops._ptr(o), lib.F32, ops._stream())
  q2, cache2, places2, first2 = case(rng, 3, 9, 3, 64, 300, "fp32")
  for r in range(3):
    o.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    print(f"noalloc under capture: replay {r}", flush=True)
    assert torch.equal(o, want), (r, float((o - want).abs().max()))
    call_both(lib, ops, q2, cache2, 9, 3, 64, places2, first2, 300, torch.float32)  # (eager work on the scratch)
