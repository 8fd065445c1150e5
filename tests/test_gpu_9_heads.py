"""Logit heads on the GPU (fh_logit_heads; models/serve.py:31-47) against the oracle's Head.of (oracle/serve.py,
serve.py:23-27): the k best values and their columns exactly (the first column of equal values first), the log of
the sum of exp(x t) within fp32's rounding of numpy's float64, for one part and many (a row wider than 4096 columns,
merged by the second kernel), rows full of ties and -inf, ragged widths, several temperatures a batch."""
import numpy as np
import pytest
import torch
from oracle.serve import head_of

pytestmark = pytest.mark.gpu


def ops():
  from ferrite_amd import ops as m
  return m


@pytest.mark.parametrize("vocab,k,rows", [(100, 64, 3), (4096, 5, 2), (4100, 64, 2), (49152, 64, 4), (128256, 64, 16),
                                          (128256, 1, 1), (262144, 64, 2), (151936, 17, 3)])
def test_heads(cuda, vocab, k, rows):
  rng = np.random.default_rng(vocab + k + rows)
  x = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
  x[0] = np.round(x[0] * 2) / 2                      # row 0: steps of 0.5, thousands of equal values
  if rows > 1: x[1, rng.integers(0, vocab, 50)] = -np.inf
  if rows > 2: x[2, :] = 1.25                        # a row all equal: the first k columns
  t = rng.choice([1.0, 0.5, 2.0, 1 / 0.7], rows).astype(np.float32)
  g = torch.from_numpy(x).cuda()
  values, ids, lse = ops().logit_heads(g, k, torch.from_numpy(t).cuda())
  values, ids, lse = values.cpu().numpy(), ids.cpu().numpy(), lse.cpu().numpy()
  for r in range(rows):
    wv, wi, wl = head_of(x[r], float(t[r]), k)
    assert np.array_equal(ids[r], wi), (r, ids[r][:8], wi[:8])
    assert np.array_equal(values[r], wv), r
    assert abs(lse[r] - wl) <= 2e-6 * abs(wl) + 2e-6, (r, lse[r], wl)
  v2, i2 = ops().logit_heads(g, k)  # without temperatures: the same picks
  assert torch.equal(i2.cpu(), torch.from_numpy(ids)) and torch.equal(v2.cpu(), torch.from_numpy(values))


def test_heads_of_the_decoders_logits(cuda):
  # a row of strided logits (a view of a wider buffer) and a Decoder-shaped batch: the same picks as argmax at k = 1
  rng = np.random.default_rng(51)
  buf = torch.from_numpy(rng.normal(0, 1, (4, 50000)).astype(np.float32)).cuda()
  view = buf[:, :49152]
  v, i = ops().logit_heads(view, 1)
  assert torch.equal(i[:, 0].long().cpu(), view.argmax(1).cpu())


def test_heads_reject(cuda):
  g = torch.zeros(2, 300000, device="cuda")
  with pytest.raises(NotImplementedError, match="too wide"):
    ops().logit_heads(g, 64)
  with pytest.raises(ValueError):
    ops().logit_heads(g[:, :1000], 65)


def test_decoder_heads(cuda):
  # a decode step's heads: the pick is the first of them, and they are numpy's Head.of of the step's logits
  from ferrite_amd import llama as G
  from oracle import llama as OL
  rng = np.random.default_rng(52)
  c = OL.smollm(layers=2, vocab=4096 + 512)
  w = OL.random_weights(c, rng)
  gc = G.model(**{k: getattr(c, k) for k in ("dim", "heads", "kv", "layers", "eps", "theta", "vocab", "ffn", "places", "rope", "tied")})
  dec = G.Decoder(gc, G.numpy_weights(w), mode="bfp8", kv="bf16", batch=2, context=64)
  logits, picks = dec.step([3, 9], [0, 0], replay=False)
  values, ids, lse = dec.heads(8, [1.0, 0.5])
  for r, t in enumerate((1.0, 0.5)):
    wv, wi, wl = head_of(logits[r].cpu().numpy(), t, 8)
    assert np.array_equal(ids[r].cpu().numpy(), wi) and int(ids[r, 0]) == int(picks[r])
    assert abs(float(lse[r]) - wl) <= 2e-6 * abs(wl) + 2e-6
