"""Matmul of plain operands (fh_matmul; Tensor.matmul with a bf16 or fp32 B, ferrite/tensor.py:443-485) against numpy,
after the reference's own checks (test/test_sim.py: test_matmul_exact 310-323, test_matmul_random 325-335,
test_matmul_blocks 337-354, test_fp32's fp32 matmul 870-880): small integers and x @ I bit for bit; x @ diag(d) with
full-mantissa d, each output one product, exact in fp32; random bf16 operands within a bf16 step of sum |a b| (bf16
out) or fp32 rounding of it (fp32 out); fp32 operands as bf16x3 within 2^-14 of sum |a b|, a bound bf16 operands
alone miss by far; batches and broadcasting; the elementwise chain on top fused into the same launch."""
import numpy as np
import pytest
import torch
from oracle import bfp as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt(cuda):
  from ferrite_amd import tensor
  return tensor.Runtime(0)


def Tn():
  from ferrite_amd import tensor
  return tensor.Tensor


def ops():
  from ferrite_amd import ops as o
  return o


def gpu(a, dtype):
  return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda").to(dtype)


def test_exact_integers_identity_and_diagonal(cuda):
  a = np.array([[float((r * 7 + c * 3) % 3 - 1) for c in range(64)] for r in range(32)], np.float32)
  b = np.array([[float((r * 5 + c) % 3 - 1) for c in range(32)] for r in range(64)], np.float32)
  want = a.astype(np.float64) @ b
  for da in (torch.bfloat16, torch.float32):
    for db in (torch.bfloat16, torch.float32):
      got = ops().matmul(gpu(a, da)[None], gpu(b, db)[None])[0].cpu().numpy()
      assert np.array_equal(got, want), (da, db)
  rng = np.random.default_rng(131)
  x = O.bf16(rng.uniform(-8, 8, (96, 64)))
  eye = np.eye(64, dtype=np.float32)
  assert np.array_equal(ops().matmul(gpu(x, torch.bfloat16)[None], gpu(eye, torch.bfloat16)[None])[0].cpu().numpy(), x)
  d = O.bf16(rng.uniform(1, 2, 64))
  got = ops().matmul(gpu(x, torch.bfloat16)[None], gpu(np.diag(d), torch.bfloat16)[None])[0].cpu().numpy()
  assert np.array_equal(got, (x.astype(np.float64) * d).astype(np.float32))  # one bf16 x bf16 product each: exact
  gb = ops().matmul(gpu(x, torch.bfloat16)[None], gpu(np.diag(d), torch.bfloat16)[None], out_dtype=torch.bfloat16)
  assert np.array_equal(gb[0].float().cpu().numpy(), O.bf16(x.astype(np.float64) * d))  # rounded once, to nearest even


def test_random_bf16_shapes(cuda):
  rng = np.random.default_rng(132)
  # (a 64 x 64 tile's edges: M, N and K not multiples of 64 or of the 32-k step; one row; one column of K)
  for M, K, N in ((64, 96, 128), (160, 96, 192), (1, 4096, 64), (45, 70, 33), (7, 1, 9), (130, 33, 65)):
    a, b = O.bf16(rng.uniform(-1, 1, (M, K))), O.bf16(rng.uniform(-1, 1, (K, N)))
    want = a.astype(np.float64) @ b
    mag = np.abs(a).astype(np.float64) @ np.abs(b)
    got = ops().matmul(gpu(a, torch.bfloat16)[None], gpu(b, torch.bfloat16)[None])[0].cpu().numpy()
    assert (np.abs(got - want) <= 2 ** -22 * mag + 1e-30).all(), (M, K, N)  # exact products, fp32 sums
    gb = ops().matmul(gpu(a, torch.bfloat16)[None], gpu(b, torch.bfloat16)[None], out_dtype=torch.bfloat16)[0].float().cpu().numpy()
    assert (np.abs(gb - want) <= 2 ** -8 * mag + 1e-30).all(), (M, K, N)


def test_fp32_operands_bf16x3(cuda):
  rng = np.random.default_rng(133)
  for M, K, N in ((45, 70, 33), (128, 512, 96)):
    a, b = rng.uniform(-2, 2, (M, K)).astype(np.float32), rng.uniform(-2, 2, (K, N)).astype(np.float32)
    want = a.astype(np.float64) @ b
    mag = np.abs(a).astype(np.float64) @ np.abs(b)
    got = ops().matmul(gpu(a, torch.float32)[None], gpu(b, torch.float32)[None])[0].cpu().numpy()
    err = np.abs(got - want) / mag
    assert err.max() <= 2 ** -14, err.max()
    # bf16 operands alone are far off that bound: the lo parts are in the sum
    bf = ops().matmul(gpu(a, torch.bfloat16)[None], gpu(b, torch.bfloat16)[None])[0].cpu().numpy()
    assert (np.abs(bf - want) / mag).max() > 2 ** -12
    # one fp32 operand: its lo part with the other's hi (hi@hi + hi@lo or lo@hi)
    ab = O.bf16(a)
    got = ops().matmul(gpu(ab, torch.bfloat16)[None], gpu(b, torch.float32)[None])[0].cpu().numpy()
    assert (np.abs(got - ab.astype(np.float64) @ b) / mag).max() <= 2 ** -14


def test_batches_and_broadcast(cuda):
  rng = np.random.default_rng(134)
  a3, b3 = O.bf16(rng.normal(0, 1, (3, 20, 48))), O.bf16(rng.normal(0, 1, (3, 48, 40)))
  a1, b1 = a3[:1], b3[:1]
  for a, b in ((a3, b3), (a3, b1), (a1, b3)):
    want = np.einsum("bmk,bkn->bmn", np.broadcast_to(a, (3,) + a.shape[1:]).astype(np.float64), np.broadcast_to(b, (3,) + b.shape[1:]))
    got = ops().matmul(gpu(a, torch.bfloat16), gpu(b, torch.bfloat16)).cpu().numpy()
    assert got.shape == (3, 20, 40)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_rejects(cuda):
  a = torch.zeros(1, 4, 8, device="cuda", dtype=torch.bfloat16)
  with pytest.raises(ValueError): ops().matmul(a, torch.zeros(1, 9, 4, device="cuda", dtype=torch.bfloat16))
  with pytest.raises(ValueError): ops().matmul(a, torch.zeros(1, 8, 4, device="cuda", dtype=torch.int32))
  with pytest.raises(ValueError): ops().matmul(torch.zeros(2, 4, 8, device="cuda"), torch.zeros(3, 8, 4, device="cuda"))


def test_tensor_matmul_plain_with_its_chain(rt):
  rng = np.random.default_rng(135)
  x, w = O.bf16(rng.normal(0, 1, (37, 80))), O.bf16(rng.normal(0, 0.1, (80, 50)))
  bias = O.bf16(rng.normal(0, 1, (1, 50)))
  X, W, Bv = Tn().of(rt, x.tolist()), Tn().of(rt, w.tolist()), Tn().of(rt, bias.tolist())
  y = (X @ W + Bv).relu() * 0.5
  assert y.dtype == "bf16"
  before = rt.launches
  got = np.array(y.tolist(), np.float64)
  assert rt.launches - before == 1, rt.launches - before  # the matmul and its chain: one launch
  want = np.maximum(x.astype(np.float64) @ w + bias, 0) * 0.5
  assert (np.abs(got - O.bf16(want)) <= 2 ** -8 * np.abs(want) + 2 ** -8 * (np.abs(x) @ np.abs(w)) * 2 ** -7 + 1e-6).all()
  # fp32 operands, a batch by one matrix, the result fp32 (ferrite's dtype rule), and a transposed operand's view
  a = rng.uniform(-1, 1, (2, 9, 30)).astype(np.float32)
  A, Wt = Tn().of(rt, a.tolist(), "fp32"), Tn().of(rt, w[:30, :20].T.tolist(), "fp32")
  z = A @ Wt.T
  assert z.dtype == "fp32" and z.shape == (2, 9, 20)
  want = a.astype(np.float64) @ w[:30, :20]
  assert np.abs(np.array(z.tolist()) - want).max() <= 2 ** -14 * (np.abs(a) @ np.abs(w[:30, :20])).max()
