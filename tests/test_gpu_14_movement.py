"""The lazy Tensor's data movement (ferrite/tensor.py:116-236, 273-283) against numpy: permute, split and merge,
pad, cat, repeat_interleave, assign into a view, gather and put by int32 rows read on the GPU, and put into a block
float (each put row's runs of 16 rounded as cast rounds them: the oracle's bfp of those rows, the other rows untouched).
The methods ferrite's model code builds its chip path from (models/llama.py:36-47, 116-146, 318-328)."""
import numpy as np
import pytest
from oracle import bfp as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt(cuda):
  from ferrite_amd import tensor
  return tensor.Runtime(0)


def Tn():
  from ferrite_amd import tensor
  return tensor.Tensor


def test_permute_split_merge(rt):
  rng = np.random.default_rng(141)
  a = O.bf16(rng.normal(0, 1, (3, 5, 8)))
  t = Tn().of(rt, a.tolist())
  for order in ((0, 1, 2), (0, 2, 1), (1, 0, 2), (1, 2, 0), (2, 0, 1), (2, 1, 0)):
    got = t.permute(*order)
    assert got.shape == tuple(a.shape[k] for k in order)
    assert np.array_equal(got.numpy(), np.transpose(a, order)), order
  m = O.bf16(rng.normal(0, 1, (6, 64)))
  x = Tn().of(rt, m.tolist())
  heads = x.split(4)  # columns: attention's heads as a batch
  assert heads.shape == (4, 6, 16) and np.array_equal(heads.numpy(), m.reshape(6, 4, 16).transpose(1, 0, 2))
  assert np.array_equal(heads.merge().numpy()[0], m)
  assert np.array_equal((heads * 2.0).merge().numpy()[0], m * 2)  # a tree computed straight into its columns
  rows = Tn().of(rt, a.tolist()).split(5, 1)  # rows: each matrix's parts one after another
  assert rows.shape == (15, 1, 8) and np.array_equal(rows.numpy(), a.reshape(15, 1, 8))


def test_pad_cat_repeat(rt):
  rng = np.random.default_rng(142)
  a = rng.normal(0, 1, (2, 3, 5)).astype(np.float32)
  t = Tn().of(rt, a.tolist(), "fp32")
  w = ((1, 0), (2, 3), (0, 4))
  assert np.array_equal(t.pad(w).numpy(), np.pad(a, w))
  assert np.array_equal(t.pad(((0, 2), (1, 1))).numpy(), np.pad(a, ((0, 0), (0, 2), (1, 1))))
  b = rng.normal(0, 1, (2, 3, 5)).astype(np.float32)
  u = Tn().of(rt, b.tolist(), "fp32")
  for axis in (0, 1, 2):
    assert np.array_equal(t.cat(u, t * 2.0, axis=axis).numpy(), np.concatenate([a, b, a * 2], axis)), axis
  assert np.array_equal(t.repeat_interleave(3).numpy(), np.repeat(a, 3, 0))
  i = Tn().of(rt, [[1, 2], [3, 4]], "int32")
  assert i.pad(((1, 1),)).tolist() == [[0, 1, 2, 0], [0, 3, 4, 0]]


def test_assign_into_a_view(rt):
  rng = np.random.default_rng(143)
  a = rng.normal(0, 1, (2, 6, 7)).astype(np.float32)
  y = rng.normal(0, 1, (2, 3, 7)).astype(np.float32)
  t, u = Tn().of(rt, a.tolist(), "fp32"), Tn().of(rt, y.tolist(), "fp32")
  t[:, 2:5, :].assign(u * 3.0 + 1.0)
  want = a.copy()
  want[:, 2:5, :] = y * np.float32(3.0) + np.float32(1.0)
  assert np.array_equal(t.numpy(), want)


def test_gather_and_put_rows(rt):
  rng = np.random.default_rng(144)
  for dtype, npt in (("bf16", O.bf16), ("fp32", lambda v: v.astype(np.float32))):
    table = npt(rng.normal(0, 1, (50, 96)))
    t = Tn().of(rt, table.tolist(), dtype)
    ids = [7, 0, 49, 7, 13]
    assert np.array_equal(t.gather(ids).numpy()[0], table[ids])
    by = Tn().of(rt, [ids], "int32")  # indices on the GPU: a computed row works the same
    assert np.array_equal(t.gather(by + 0).numpy()[0], table[ids])
    # put: rows of x at places in each matrix of a batch (a KV cache's put)
    cache = npt(rng.normal(0, 1, (3, 40, 96)))
    x = npt(rng.normal(0, 1, (3, 4, 96)))
    c, X = Tn().of(rt, cache.tolist(), dtype), Tn().of(rt, x.tolist(), dtype)
    places = [31, 2, 39, 0]
    c.put(Tn().of(rt, [places], "int32"), X)
    want = cache.copy()
    want[:, places] = x
    assert np.array_equal(c.numpy(), want), dtype
  # an index outside the rows: put writes nothing, gather reads the nearest row
  c.put(Tn().of(rt, [[-1, 40, 5, 1000]], "int32"), X)
  want[:, 5] = x[:, 2]
  assert np.array_equal(c.numpy(), want)
  assert np.array_equal(t.gather(Tn().of(rt, [[-3, 99]], "int32")).numpy()[0], table[[0, 49]])


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_put_into_block_float(rt, fmt):
  rng = np.random.default_rng(145)
  base = rng.normal(0, 1, (64, 128)).astype(np.float32)
  cache = Tn().of(rt, base.tolist(), "fp32").cast(fmt)
  x = O.bf16(rng.normal(0, 3, (5, 128)) * np.exp(rng.normal(0, 2, (5, 128))))
  places = [3, 60, 17, 0, 44]
  cache.put(Tn().of(rt, [places], "int32"), Tn().of(rt, x.tolist()))
  got = cache.numpy()[0]
  want = O.bfp(base, fmt)
  want[places] = O.bfp(x, fmt)
  assert np.array_equal(got, want.astype(np.float32))
  # its packed rows gathered back: the same values
  assert np.array_equal(cache.gather([60, 0]).numpy()[0], want[[60, 0]].astype(np.float32))
