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


def test_empty_then_filled(rt):
  # the model's `empty` (models/llama.py:47): a tensor made with no value, its memory taken when first used
  rng = np.random.default_rng(148)
  e = Tn()(rt, 3, 4, batch=2, dtype="fp32")
  y = rng.normal(0, 1, (2, 3, 4)).astype(np.float32)
  e.assign(Tn().of(rt, y.tolist(), "fp32"))
  assert np.array_equal(e.numpy(), y)
  c = Tn()(rt, 5, 4, batch=2, dtype="fp32")
  c.put(Tn().of(rt, [[4, 1, 0]], "int32"), Tn().of(rt, y.tolist(), "fp32"))
  assert np.array_equal(c.numpy()[:, [4, 1, 0]], y)


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


def _attend_np(q, k, v, places, window):
  B, T, hd = q.shape
  out = np.zeros((B, T, hd))
  for b in range(B):
    for t in range(T):
      p = places[b if places.shape[0] > 1 else 0, t, 0]
      hi, lo = min(p, k.shape[1] - 1), (max(p - window + 1, 0) if window else 0)
      if hi < lo: continue
      s = q[b, t].astype(np.float64) @ k[b, lo:hi + 1].T.astype(np.float64)
      e = np.exp(s - s.max())
      out[b, t] = e @ v[b, lo:hi + 1] / e.sum()
  return out


@pytest.mark.parametrize("hd", [64, 96, 128])
def test_attend(rt, hd):
  # Tensor.attend as models/llama.py:134-139 calls it: q scaled by 1/sqrt(hd), a batch of heads, each row's place, with
  # and without a window; keys and values bf16, fp32, or a block float (a KV cache's bfp8 values, read as those); grouped
  # query heads by repeat_interleave
  rng = np.random.default_rng(146 + hd)
  B, T, S = 4, 6, 70
  q = O.bf16(rng.normal(0, 1, (B, T, hd)))
  k, v = O.bf16(rng.normal(0, 1, (B, S, hd))), O.bf16(rng.normal(0, 1, (B, S, hd)))
  places = rng.integers(0, S + 5, (1, T, 1)).astype(np.int32)  # (some past the keys: clipped)
  scale = 1 / np.sqrt(hd)
  Q, K, V, Pl = Tn().of(rt, q.tolist()), Tn().of(rt, k.tolist()), Tn().of(rt, v.tolist()), Tn().of(rt, places[0].tolist(), "int32")
  for window in (0, 9):
    got = (Q * scale).attend(K, V, Pl, window).numpy()
    want = _attend_np(O.bf16(q * scale), k, v, places, window)
    assert np.abs(got - want).max() <= 2 ** -7 * np.abs(want).max(), (hd, window)
  # fp32 keys and values; places a column for each matrix
  pb = rng.integers(0, S, (B, T, 1)).astype(np.int32)
  got = (Q * scale).attend(K.float(), V.float(), Tn().of(rt, pb.tolist(), "int32")).numpy()
  assert np.abs(got - _attend_np(O.bf16(q * scale), k, v, pb, 0)).max() <= 2 ** -7 * 4
  # a bfp8 cache: the same as attending over its values in bf16
  Kc, Vc = Tn().of(rt, k.tolist()).cast("bfp8"), Tn().of(rt, v.tolist()).cast("bfp8")
  got = (Q * scale).attend(Kc, Vc, Pl).numpy()
  want = _attend_np(O.bf16(q * scale), np.stack([O.bfp(m) for m in k]), np.stack([O.bfp(m) for m in v]), places, 0)
  assert np.abs(got - want).max() <= 2 ** -7 * np.abs(want).max()
  # grouped-query: 2 key heads serving 4 query heads
  K2, V2 = Tn().of(rt, k[:2].tolist()), Tn().of(rt, v[:2].tolist())
  got = (Q * scale).attend(K2.repeat_interleave(2), V2.repeat_interleave(2), Pl).numpy()
  want = _attend_np(O.bf16(q * scale), np.repeat(k[:2], 2, 0), np.repeat(v[:2], 2, 0), places, 0)
  assert np.abs(got - want).max() <= 2 ** -7 * np.abs(want).max()


@pytest.mark.parametrize("dense", [True, False])
def test_experts_by_touched_and_group(rt, dense):
  # models/llama.py:302-329's chip_experts on this Tensor, both ways: each picked expert once with every token its rows
  # (touched; a decode step's), or each expert's tokens grouped into whole tiles of 32 (group; a prompt's), gathered
  # back and weighted; against numpy_experts (llama.py:294-300) over the same bf16 rows and block-float experts
  rng = np.random.default_rng(147)
  rows, dim, m, e, k = 40, 64, 96, 8, 2
  h = O.bf16(rng.normal(0, 1, (rows, dim)))
  ids = np.stack([rng.choice(e - 1, k, replace=False) for _ in range(rows)]).astype(np.int32)  # (a row's experts distinct,
                                                                                              # as topk's; expert 7 picked
                                                                                              # by none: an entry is none)
  w = O.bf16(rng.uniform(0.1, 1, (rows, k)))
  gu = rng.normal(0, 0.05, (e, dim, 2 * m)).astype(np.float32)
  dn = rng.normal(0, 0.05, (e, m, dim)).astype(np.float32)
  H, Ids, W = Tn().of(rt, h.tolist()), Tn().of(rt, ids.tolist(), "int32"), Tn().of(rt, w.tolist())
  GU, DN = Tn().of(rt, gu.tolist(), "fp32").cast("bfp8"), Tn().of(rt, dn.tolist(), "fp32").cast("bfp8")
  glu = lambda g: g[:, :, :m].silu() * g[:, :, m:]
  if dense:
    picks, weights = Ids.touched(e, W)
    assert picks.numpy().ravel().tolist() == sorted(set(ids.ravel().tolist())) + [e] * (min(rows * k, e) - len(set(ids.ravel().tolist())))
    got = (glu(H.matmul(GU, index=picks)) * weights).matmul(DN, index=picks).sum(0).numpy()[0]
  else:
    order, picks, places = Ids.group(e)
    x = H.gather(order).split(picks.rows, 1)
    y = glu(x.matmul(GU, index=picks)).matmul(DN, index=picks).reshape(order.cols, dim)
    run = places.cols // k
    terms = [y.gather(places[:, :, j * run:j * run + rows]) * W[:, :, j:j + 1] for j in range(k)]
    got = (terms[0] + terms[1]).numpy()[0]
    o = order.numpy().ravel()
    for t in range(rows):  # every choice has a slot holding its row, in its value's run
      for j in range(k):
        s = places.numpy().ravel()[j * run + t]
        assert o[s] == t and picks.numpy().ravel()[s // 32] == ids[t, j]
  gv, dv = np.stack([O.bfp(a) for a in gu]), np.stack([O.bfp(a) for a in dn])
  silu = lambda a: a / (1 + np.exp(-a))
  def expert(x, i):
    g = O.bf16(x.astype(np.float64) @ gv[i]).astype(np.float64)
    return O.bf16(O.bf16(silu(g[:m])) * g[m:]).astype(np.float64) @ dv[i]
  want = np.stack([sum(w[t, j] * expert(h[t], ids[t, j]) for j in range(k)) for t in range(rows)])
  assert np.abs(got - want).max() <= 2 ** -6 * np.abs(want).max(), np.abs(got - want).max() / np.abs(want).max()
