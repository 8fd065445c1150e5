"""ferrite's lazy Tensor surface on the GPU (ferrite_amd.tensor) against numpy, the way the reference's test_sim.py
checks its Tensor on ttsim: values in and out (bf16 to nearest even), elementwise trees fused into one launch, the
reductions and what is built from them, matmul by a block float with its elementwise chain in the same kernel, casts to
block floats read back as the oracle decodes them. Programs compute in fp32 and round once, so a bf16 result is within
2^-8 of numpy's float64 value of the same expression on the same (bf16) inputs. Reference tests of the same:
test_elementwise / test_reduce / test_softmax / test_matmul_random (test/test_sim.py)."""
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


def close(got, want, rel, what):
  got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
  err = np.abs(got - want)
  bound = rel * np.maximum(np.abs(want), np.abs(want).max() * 1e-3) + 1e-30
  assert (err <= bound).all(), (what, float((err / bound).max()))


def test_values_in_and_out(rt):
  rng = np.random.default_rng(61)
  a = rng.normal(0, 3, (3, 5, 7)).astype(np.float32)
  t = Tn().of(rt, a.tolist(), "bf16")
  assert np.array_equal(np.array(t.tolist(), np.float32), O.bf16(a))
  f = Tn().of(rt, a[0].tolist(), "fp32")
  assert np.array_equal(np.array(f.tolist(), np.float32), a[0])
  i = Tn().frombytes(rt, 2, 3, np.arange(6, dtype=np.int32).tobytes(), dtype="int32")
  assert i.tolist() == [[0, 1, 2], [3, 4, 5]] and i.tobytes() == np.arange(6, dtype=np.int32).tobytes()


def test_elementwise_tree_is_one_launch(rt):
  rng = np.random.default_rng(62)
  x = O.bf16(rng.normal(0, 1, (1, 64, 96)))
  y = O.bf16(rng.normal(0, 1, (1, 1, 96)))        # a row, broadcast down the rows
  c = O.bf16(rng.normal(0, 1, (1, 64, 1)))        # a column, broadcast along the rows
  X, Y, C = (Tn().of(rt, a[0].tolist()) for a in (x, y, c))
  z = ((X * Y + C).sigmoid() * X - (X - 0.5).relu()).maximum(Y * 0.25)
  before = rt.launches
  got = z.numpy()
  assert rt.launches - before == 1, rt.launches - before
  s = 1 / (1 + np.exp(-(x.astype(np.float64) * y + c)))
  want = np.maximum(s * x - np.maximum(x - 0.5, 0), y * 0.25)
  close(got, O.bf16(want), 2 ** -8, "tree")


@pytest.mark.parametrize("name", ["exp", "log", "sqrt", "sin", "cos", "reciprocal", "silu", "gelu", "exp2", "log2"])
def test_unary(rt, name):
  rng = np.random.default_rng(63)
  a = O.bf16(np.abs(rng.normal(0, 2, (16, 48))) + 0.1)
  f = {"exp": np.exp, "log": np.log, "sqrt": np.sqrt, "sin": np.sin, "cos": np.cos, "reciprocal": lambda v: 1 / v,
       "silu": lambda v: v / (1 + np.exp(-v)), "exp2": np.exp2, "log2": np.log2,
       "gelu": lambda v: 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))}[name]
  got = getattr(Tn().of(rt, a.tolist(), "fp32"), name)().numpy()[0]
  close(got, f(a.astype(np.float64)), 1e-5, name)


def test_where_and_comparisons(rt):
  a = np.array([[1.0, -2.0, 3.0, 0.0]], np.float32)
  b = np.array([[1.0, 2.0, -3.0, 0.0]], np.float32)
  A, B = Tn().of(rt, a.tolist(), "fp32"), Tn().of(rt, b.tolist(), "fp32")
  assert (A < B).tolist() == [[0.0, 1.0, 0.0, 0.0]]
  assert (A >= B).tolist() == [[1.0, 0.0, 1.0, 1.0]]
  assert A.eq(B).tolist() == [[1.0, 0.0, 0.0, 1.0]]
  assert (A > 0).where(A, B * 10).tolist() == [[1.0, 20.0, 3.0, 0.0]]
  assert A.minimum(B).tolist() == [[1.0, -2.0, -3.0, 0.0]]


def test_int32(rt):
  a = Tn().of(rt, [[5, -7, 2**20]], "int32")
  b = Tn().of(rt, [[3, 3, 1]], "int32")
  assert (a + b).tolist() == [[8, -4, 2**20 + 1]] and (a - b).tolist() == [[2, -10, 2**20 - 1]]
  assert a.maximum(b).tolist() == [[5, 3, 2**20]] and (a + b).dtype == "int32"
  assert (a * 2).tolist() == [[10, -14, 2**21]]


@pytest.mark.parametrize("axis", [0, 1, 2, None])
def test_reductions(rt, axis):
  rng = np.random.default_rng(64)
  a = rng.normal(0, 1, (3, 40, 300)).astype(np.float32)
  t = Tn().of(rt, a.tolist(), "fp32")
  kw = dict(axis=axis, keepdims=True) if axis is not None else {}
  n = a.size if axis is None else a.shape[axis]
  absum = np.abs(a.astype(np.float64)).sum(**kw).reshape(-1)
  for f, ref in (("sum", np.sum), ("max", np.max), ("mean", np.mean)):
    got = getattr(t, f)(axis).numpy().reshape(-1)
    want = ref(a.astype(np.float64), **kw).reshape(-1)
    if f == "max":
      assert np.array_equal(got, want), (f, axis)  # (a largest is one of the values, exactly)
    else:  # fp32 sums in order: within n 2^-24 of the sum of magnitudes
      bound = n * 2.0 ** -24 * absum / (n if f == "mean" else 1) + 1e-30
      assert (np.abs(got - want) <= bound).all(), (f, axis, float((np.abs(got - want) / bound).max()))


def test_softmax_family(rt):
  rng = np.random.default_rng(65)
  a = rng.normal(0, 3, (1, 33, 1000)).astype(np.float32)
  t = Tn().of(rt, a[0].tolist(), "fp32")
  e = np.exp(a - a.max(-1, keepdims=True))
  close(t.softmax().numpy(), e / e.sum(-1, keepdims=True), 1e-5, "softmax")
  close(t.log_softmax().numpy(), np.log(e / e.sum(-1, keepdims=True)), 1e-5, "log_softmax")
  # along the last axis one launch, the elementwise tree under it in the same kernel; the composed form (another axis)
  # agrees; bf16 rows round their sum as the composed form's bf16 sum does
  before = rt.launches
  got = (t * 0.5 + 1.0).softmax().numpy()
  assert rt.launches - before == 1, rt.launches - before
  e2 = np.exp(a * 0.5 - (a * 0.5).max(-1, keepdims=True))
  close(got, e2 / e2.sum(-1, keepdims=True), 1e-5, "fused softmax")
  tt = Tn().of(rt, np.swapaxes(a, 1, 2)[0].tolist(), "fp32")
  close(tt.softmax(axis=1).numpy(), np.swapaxes(e / e.sum(-1, keepdims=True), 1, 2), 1e-5, "softmax down the rows")
  b = Tn().of(rt, a[0].tolist(), "bf16")
  ab = O.bf16(a).astype(np.float64)
  eb = np.exp(ab - ab.max(-1, keepdims=True))
  want = eb / O.bf16(eb.sum(-1, keepdims=True)).astype(np.float64)
  close(b.softmax().numpy(), O.bf16(want), 2 ** -7, "bf16 softmax")
  close(b.log_softmax().numpy(), O.bf16(np.log(want)), 2 ** -7, "bf16 log_softmax")
  c = a - a.mean(-1, keepdims=True)
  close(t.layernorm().numpy(), c / np.sqrt((c * c).mean(-1, keepdims=True) + 1e-5), 1e-4, "layernorm")


@pytest.mark.parametrize("rows", [1, 16, 200])
def test_matmul_and_its_chain(rt, rows):
  # bf16 rows @ a bfp8 weight, then bias, relu and a row softmax: the matmul and its elementwise chain one kernel,
  # the softmax one more
  rng = np.random.default_rng(66)
  K, N = 576, 1536
  x = O.bf16(rng.normal(0, 1, (rows, K)))
  w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
  bias = O.bf16(rng.normal(0, 0.1, (1, N)))
  W = Tn().of(rt, w.tolist(), "fp32").cast("bfp8")
  X, Bias = Tn().of(rt, x.tolist()), Tn().of(rt, bias.tolist())
  h = (X @ W + Bias).relu()
  before = rt.launches
  hv = h.float().realize()
  assert rt.launches - before == 1
  wv = O.bfp(w)
  want = np.maximum(x.astype(np.float64) @ wv + bias, 0)
  # (x is bf16 already: exact products on either path, fp32 sums): within fp32 summation's error, 1e-5 of sum |x w|
  bound = 1e-5 * (np.abs(x) @ np.abs(wv) + np.abs(bias)) + 1e-30
  err = np.abs(hv.numpy()[0] - want)
  assert (err <= bound).all(), ("matmul", rows, float((err / bound).max()))
  # the softmax of an fp32 matmul's chain: its two reductions realize the matmul apart (fp32, so nothing rounds to
  # bf16 between them); within exp's growth of the sums' fp32 error
  before = rt.launches
  s = (X.matmul(W, "fp32") + Bias).relu().softmax().numpy()[0]
  assert rt.launches - before == 2, rt.launches - before  # the matmul with its chain, then the softmax
  e = np.exp(want - want.max(-1, keepdims=True))
  close(s, e / e.sum(-1, keepdims=True), 1e-4, ("softmax", rows))
  # Runtime.profile (ferrite/runtime.py:416-428): each launch's time and the bytes it read, by name. The first matmul
  # read the packed weight (K N 17/16 bytes), x's bf16 rows and the bias row once; the second, under a softmax, the
  # weight and x only (its chain goes into the softmax's program, which reads the fp32 rows and the bias)
  since = rt.launches
  (X @ W + Bias).relu().float().realize()
  (X.matmul(W, "fp32") + Bias).relu().softmax().realize()
  got = {name: (n, us, b) for name, n, us, b in rt.profile(since)}
  assert got["matmul"][0] == 2 and got["matmul"][1] > 0 and got["softmax"][0] == 1
  assert got["matmul"][2] == 2 * (K * N * 17 // 16 + rows * K * 2) + N * 2, got["matmul"]
  assert got["softmax"][2] == rows * N * 4 + N * 2, got["softmax"]


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_cast_to_block_float(rt, fmt):
  # Tensor.cast("bfp8"/"bfp4") read back as bf16 (tensor._bf16s): the oracle's values, bit for bit
  rng = np.random.default_rng(67)
  a = O.bf16(rng.normal(0, 1, (64, 96)) * np.exp(rng.normal(0, 2, (64, 96))))
  t = Tn().of(rt, a.tolist()).cast(fmt)
  got = np.frombuffer(t.tobytes(), np.uint16).reshape(64, 96)
  q, top = O.bfp_parts(a, fmt)
  assert np.array_equal(got, O.exact_bf16(q, top, fmt))


def test_views(rt):
  rng = np.random.default_rng(68)
  a = rng.normal(0, 1, (2, 6, 8)).astype(np.float32)
  t = Tn().of(rt, a.tolist(), "fp32")
  assert np.array_equal(t.T.numpy(), a.transpose(0, 2, 1))
  assert np.array_equal(t[1].numpy(), a[1:2])
  assert np.array_equal(t[:, 1:5:2, ::3].numpy(), a[:, 1:5:2, ::3])
  assert np.array_equal(t[0][:, :, 0:1].expand(1, 6, 8).numpy(), np.broadcast_to(a[0:1, :, 0:1], (1, 6, 8)))
  assert np.array_equal(t.reshape(4, 24).numpy(), a.reshape(1, 4, 24))
  assert np.array_equal((t.T * 2).numpy(), a.transpose(0, 2, 1) * 2)


def test_long_tree_in_parts(rt):
  # more than MAX_OPS ops: realized in parts, the value the same
  rng = np.random.default_rng(69)
  a = rng.normal(0, 1, (4, 32)).astype(np.float32)
  t = Tn().of(rt, a.tolist(), "fp32")
  z, want = t, a.astype(np.float64)
  for i in range(20):
    z = (z * 0.9 + 0.1).relu() if i % 2 else z * 1.01 - 0.02
    want = np.maximum(want * 0.9 + 0.1, 0) if i % 2 else want * 1.01 - 0.02
  close(z.numpy()[0], want, 1e-5, "long")


def test_jit_replays_the_recording(rt):
  # ferrite's jit (tensor.py:788-810): the first call runs, the second is captured as a HIP graph and replayed, later
  # calls copy their inputs in and replay; each call's result equals the same expression run eagerly, bit for bit
  # (the same kernels), with eager work between the replays
  from ferrite_amd import tensor
  rng = np.random.default_rng(66)
  w = Tn().of(rt, rng.normal(0, 0.05, (64, 48)).tolist(), "fp32").cast("bfp8")
  b = Tn().of(rt, rng.normal(0, 1, (1, 48)).tolist(), "fp32")
  f = tensor.jit(lambda x: ((x @ w) + b).relu().softmax())
  out = None
  for i in range(5):
    x = Tn().of(rt, rng.normal(0, 1, (3, 64)).tolist(), "fp32")
    got = f(x)
    if i >= 2: assert got is out, "the recording's result, every call"
    out = got
    got = np.array(got.tolist(), np.float32)
    want = np.array((((x @ w) + b).relu().softmax()).tolist(), np.float32)
    assert np.array_equal(got, want), i
    assert np.allclose(got.sum(-1), 1, atol=1e-5)


def test_matmul_picked_by_index(rt):
  # matmul(index=) (tensor.py:443-460): each batch entry multiplies the block float its index names (a mixture's
  # experts), an index past the batch gives zeros; entries of one row each, and one shared row; fidelity is taken
  rng = np.random.default_rng(67)
  E, K, N = 3, 64, 48
  W = rng.normal(0, 0.05, (E, K, N)).astype(np.float32)
  wb = Tn().of(rt, W.tolist(), "fp32").cast("bfp8")
  assert wb.shape == (E, K, N)
  assert np.array_equal(np.array(wb.float().tolist(), np.float32), np.stack([O.bfp(W[e]) for e in range(E)]).astype(np.float32))
  idx = np.array([[0, 2], [1, 1], [2, 0], [3, 1]], np.int32)
  index = Tn().of(rt, idx.tolist(), "int32")
  X = rng.normal(0, 1, (8, 1, K)).astype(np.float32)
  y = Tn().of(rt, X.tolist(), "fp32").matmul(wb, "fp32", fidelity=2, index=index)
  assert y.shape == (8, 1, N)
  got = np.array(y.tolist(), np.float64)
  for b in range(8):
    e = idx[b // 2, b % 2]
    want = X[b] @ O.bfp(W[e]) if e < E else np.zeros((1, N))
    assert np.abs(got[b] - want).max() <= 2e-6 * (np.abs(X[b]) @ np.abs(W[min(e, E - 1)])).max() + 1e-6, b
  one = rng.normal(0, 1, (1, K)).astype(np.float32)
  y1 = np.array(Tn().of(rt, one.tolist(), "fp32").matmul(wb, "fp32", index=index).tolist(), np.float64)
  for b in range(8):
    e = idx[b // 2, b % 2]
    want = one @ O.bfp(W[e]) if e < E else np.zeros((1, N))
    assert np.abs(y1[b] - want).max() <= 1e-5 * np.abs(want).max() + 1e-6, b


def test_topk(rt):
  # Tensor.topk (tensor.py:373-388): largest first, the first column of equals first, bf16 and fp32, a batch of rows,
  # a width that is not a multiple of 4
  rng = np.random.default_rng(68)
  a = np.round(rng.normal(0, 2, (2, 5, 301)) * 2) / 2
  for dtype in ("bf16", "fp32"):
    t = Tn().of(rt, a.tolist(), dtype)
    v, i = t.topk(20)
    assert v.dtype == dtype and i.dtype == "int32" and v.shape == i.shape == (2, 5, 20)
    ids = np.array(i.tolist())
    want = np.argsort(-a, -1, kind="stable")[..., :20]
    assert np.array_equal(ids, want), dtype
    assert np.array_equal(np.array(v.tolist()), np.take_along_axis(a, want, -1))


def test_topk_parts_and_labels(rt):
  # ferrite's two-call form for rows wider than a worker's L1 (tensor.py:373-388): each part's k best side by side with
  # their columns in the whole row, then a topk over those given the columns as labels gives the whole row's k best
  # and their columns, ties in column order. Widths whose parts are not a multiple of 4 wide, and a batch.
  rng = np.random.default_rng(69)
  for parts, width in ((4, 1024), (3, 303), (5, 250)):
    a = np.round(rng.normal(0, 2, (2, 3, width)) * 2) / 2
    cols = width // parts
    for dtype in ("bf16", "fp32"):
      t = Tn().of(rt, a.tolist(), dtype)
      v, i = t.topk(8, parts=parts)
      assert v.dtype == dtype and i.dtype == "int32" and v.shape == i.shape == (2, 3, 8 * parts)
      ids = np.array(i.tolist())
      want = np.concatenate([np.argsort(-a[..., p * cols:(p + 1) * cols], -1, kind="stable")[..., :8] + p * cols for p in range(parts)], -1)
      assert np.array_equal(ids, want), (parts, width, dtype)
      assert np.array_equal(np.array(v.tolist()), np.take_along_axis(a, want, -1))
      v2, i2 = v.topk(8, labels=i)
      got = np.array(i2.tolist())
      whole = np.argsort(-a, -1, kind="stable")[..., :8]
      assert np.array_equal(got, whole), (parts, width, dtype)
      assert np.array_equal(np.array(v2.tolist()), np.take_along_axis(a, whole, -1))
  # the reference's own cases (test_sim.py:1492-1503): fp32 rows, k of 64 and 32, a tie across parts
  for rows, cols, parts, k in ((5, 2560, 4, 64), (40, 1024, 2, 32)):
    x = rng.normal(0, 3, (rows, cols)).astype(np.float32)
    x[0, 100] = x[0, cols // 2 + 3] = x[0].max() + 1
    values, ids = Tn().frombytes(rt, rows, cols, x.tobytes(), dtype="fp32").topk(k, parts)
    w = cols // parts
    want = np.concatenate([np.argsort(-x[:, p * w:(p + 1) * w], -1, kind="stable")[:, :k] + p * w for p in range(parts)], 1)
    assert np.array_equal(np.array(ids.tolist()), want) and np.array_equal(np.array(values.tolist()), np.take_along_axis(x, want, -1))
    values, ids = values.topk(k, labels=ids)
    want = np.argsort(-x, -1, kind="stable")[:, :k]
    assert np.array_equal(np.array(ids.tolist()), want) and np.array_equal(np.array(values.tolist()), np.take_along_axis(x, want, -1))
