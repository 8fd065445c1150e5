"""Parity of the mixture of experts (fh_moe_route, fh_moe_experts) with the oracle's moe (oracle/llama.py, pinned by
transformers' Mixtral block): the router's top k exactly (ids, the first of equals first) and its weights within fp32
rounding; the experts' weighted sum within the north star's bar (x and the SwiGLU outputs go to bf16 for the matrix
cores). The reference's test of the same: test_moe (test/test_sim.py:1511-1555)."""
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


def north_star(got, want, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
  cos = (got * want).sum() / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300)
  assert rel <= 1e-2 and cos >= 0.9999, (what, rel, cos)


@pytest.mark.parametrize("E,k,norm_topk", [(8, 2, True), (16, 4, False), (128, 8, True)])
def test_route(cuda, E, k, norm_topk):
  rng = np.random.default_rng(41)
  T, dim = 37, 256
  c = OL.model(dim=dim, eps=1e-5, k=k, experts=E, norm_topk=norm_topk)
  x = rng.normal(0, 1, (T, dim)).astype(np.float32)
  g = O.bf16(rng.normal(1, 0.1, (1, dim)))
  router = O.bf16(rng.normal(0, 0.5, (dim, E)))
  router[:, 3] = router[:, 1]  # equal logits: the first of equals first
  h = OL.rms(x.astype(np.float64), g, c)
  logits = h @ router
  values, want_ids = OL.topk(logits if norm_topk else OL.softmax(logits), k)
  want_w = OL.softmax(values) if norm_topk else values
  ids, w, dense = ops().moe_route(to_gpu(x), to_gpu(router, torch.bfloat16), E, k, norm_topk, norm_w=to_gpu(g.reshape(-1)), eps=c.eps)
  assert np.array_equal(ids.cpu().numpy(), want_ids)
  # the logits are fp32 sums of dim products: their error, about 2^-24 sqrt(dim) sum |h r|, moves a weight by at most
  # that much (a softmax's derivative is at most 1)
  bound = 2.0 ** -24 * np.sqrt(dim) * (np.abs(h) @ np.abs(router)).max() * 4
  got_w = w.cpu().numpy()
  assert np.abs(got_w - want_w).max() <= bound, (np.abs(got_w - want_w).max(), bound)
  d = np.zeros((T, E)); np.put_along_axis(d, want_ids, want_w, 1)
  assert np.abs(dense.cpu().numpy() - d).max() <= bound


@pytest.mark.parametrize("T,fmt", [(32, "bfp4"), (5, "bfp8"), (64, "bfp4"), (100, "bfp4"), (300, "bfp4"),
                                   (2200, "bfp8"), (2100, "bfp4")])
def test_experts(cuda, T, fmt):
  # benchmark config 5's shape at a smaller width: 8 experts, top 2, the tokens' SwiGLUs weighted and summed onto the
  # residual; up to 64 tokens one pass through the skinny kernel; past that (models/llama.py:314-329's group path)
  # passes of up to 2048 through the tiled GEMM (as many as the workspace budget allows: 2048 at this width), each
  # expert's gathered rows a layer of the grid: 100 and 300 in one pass, 2200 in a pass of 2048 and one of 152, 2100
  # in a pass of 2048 and one of 52 (through the skinny kernel)
  rng = np.random.default_rng(42)
  dim, ffn, E, k = 256, 512, 8, 2
  c = OL.model(dim=dim, eps=1e-5, k=k, experts=E)
  x = rng.normal(0, 1, (T, dim)).astype(np.float32)
  g = O.bf16(rng.normal(1, 0.1, (1, dim)))
  ssq = (x.reshape(T, -1, 16) ** 2).sum(-1).astype(np.float32)
  p = {"router": O.bf16(rng.normal(0, 0.5, (dim, E))), "experts.gate_up": rng.normal(0, 0.05, (E, dim, 2 * ffn)).astype(np.float32),
       "experts.down": rng.normal(0, 0.05, (E, ffn, dim)).astype(np.float32)}
  q = {"router": p["router"], "experts.gate_up": O.bfp(p["experts.gate_up"], fmt), "experts.down": O.bfp(p["experts.down"], fmt)}
  h = OL.rms(x.astype(np.float64), g, c)
  want, want_ids, want_w = OL.moe(h, q, c)
  res = rng.normal(0, 1, (T, dim)).astype(np.float32)
  ex = ops().pack_experts(to_gpu(p["experts.gate_up"]), to_gpu(p["experts.down"]), fmt)
  ids, w, dense = ops().moe_route(to_gpu(x), to_gpu(p["router"], torch.bfloat16), E, k, True, norm_w=to_gpu(g.reshape(-1)), eps=c.eps)
  assert np.array_equal(ids.cpu().numpy(), want_ids)
  y = torch.empty(T, dim, device="cuda")
  s = torch.zeros(T, dim // 16, device="cuda")
  ops().moe_experts(to_gpu(x), ex, dense, out=y, residual=to_gpu(res), ssq_out=s, norm_w=to_gpu(g.reshape(-1)),
                    ssq_in=to_gpu(ssq), eps=c.eps)
  got = y.cpu().numpy()
  north_star(got - res, want, ("moe", T, fmt))
  assert np.allclose(s.cpu().numpy(), (got.astype(np.float64).reshape(T, -1, 16) ** 2).sum(-1), rtol=1e-4)
  # without a residual: the sum alone; and an expert no row picked is skipped (its weights are never read)
  only = dense.clone()
  only[:, 1:] = 0
  y0 = ops().moe_experts(to_gpu(x), ex, only, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps).cpu().numpy()
  d0 = only.cpu().numpy()[:, 0:1]
  gu = h @ q["experts.gate_up"][0]
  want0 = d0 * (OL.glu(gu[:, :ffn], gu[:, ffn:]) @ q["experts.down"][0])
  if np.abs(want0).max() > 0: north_star(y0, want0, ("expert 0 alone", T))
  else: assert not y0.any()


@pytest.mark.parametrize("T", [17, 64])
def test_experts_every_row_on_two_experts(cuda, T):
  # every token picks the same two experts (positive rows, a router whose columns 3 and 5 dominate for all of them), so
  # those experts' gathered lists hold all T rows: 2 (17 tokens) and 4 (64 tokens) blocks of 16 rows through the
  # skinny kernel's third grid dimension, the last one partial at 17; the other six experts take no row
  rng = np.random.default_rng(7)
  dim, ffn, E, k = 256, 512, 8, 2
  c = OL.model(dim=dim, eps=1e-5, k=k, experts=E)
  x = np.abs(rng.normal(0, 1, (T, dim))).astype(np.float32) + 0.1
  g = O.bf16(rng.normal(1, 0.1, (1, dim)))
  ssq = (x.reshape(T, -1, 16) ** 2).sum(-1).astype(np.float32)
  router = rng.normal(0, 0.01, (dim, E))
  router[:, 3] += 0.05
  router[:, 5] += 0.04
  p = {"router": O.bf16(router), "experts.gate_up": rng.normal(0, 0.05, (E, dim, 2 * ffn)).astype(np.float32),
       "experts.down": rng.normal(0, 0.05, (E, ffn, dim)).astype(np.float32)}
  q = {"router": p["router"], "experts.gate_up": O.bfp(p["experts.gate_up"], "bfp4"), "experts.down": O.bfp(p["experts.down"], "bfp4")}
  h = OL.rms(x.astype(np.float64), g, c)
  want, want_ids, want_w = OL.moe(h, q, c)
  assert (np.sort(want_ids, axis=1) == [3, 5]).all()
  ex = ops().pack_experts(to_gpu(p["experts.gate_up"]), to_gpu(p["experts.down"]), "bfp4")
  ids, w, dense = ops().moe_route(to_gpu(x), to_gpu(p["router"], torch.bfloat16), E, k, True, norm_w=to_gpu(g.reshape(-1)), eps=c.eps)
  assert np.array_equal(ids.cpu().numpy(), want_ids)
  y = ops().moe_experts(to_gpu(x), ex, dense, norm_w=to_gpu(g.reshape(-1)), ssq_in=to_gpu(ssq), eps=c.eps)
  north_star(y.cpu().numpy(), want, ("two experts take every row", T))
