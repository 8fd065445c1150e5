"""CPU restatement (numpy) of ferrite's logit heads, models/serve.py's Head.of (serve.py:23-27), the checker for
fh_logit_heads.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package; the product (ferrite_amd) never calls it.
"""
import math
import numpy as np


def head_of(logits, t=1.0, k=64):
  """A row's head as Head.of makes it (serve.py:23-27): its k largest values, largest first, the first column of equal
  values first (numpy's stable argsort of -x), their columns, and log sum exp(x t) over the row in float64, as
  max t + log sum exp((x - max) t). Pinned in tests/test_oracle.py by a brute-force sort of (-value, column) and by
  scipy's logsumexp."""
  logits = np.asarray(logits)
  ids = np.argsort(-logits, kind="stable")[:k]
  m = float(logits.max())
  return logits[ids], ids, m * t + math.log(np.exp((np.float64(logits) - m) * t).sum())
