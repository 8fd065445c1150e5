"""The CPU oracle (oracle/bfp.py) pinned by what the mathematics fixes, independently of how the oracle computes:
exact rational rounding of bf16, the block-float rounding as "nearest multiple of the block's step, ties away from 0,
clamped" on every (bf16 value, block exponent) pair, and q 2^(e - 133) for every decoded value. The reference's
own test of the cast (test/test_sim.py:371-388, test_bfp) checks the chip against models/gpt2.py:21-32; these check
the restatement of that function against its definition."""
from fractions import Fraction
import math
import numpy as np
import pytest
from oracle import bfp as O


def all_bf16():
  bits = np.arange(65536, dtype=np.uint32)
  e = bits >> 7 & 255
  return bits[e != 255].astype(np.uint16)  # finite ones


def test_bf16_rne_exact():
  # each fp32 rounded to the nearest bf16, ties to the even one, by rational arithmetic (a sample with every
  # exponent, every tie and both neighbours of each tie)
  rng = np.random.default_rng(0)
  bits = np.concatenate([rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32),
                         (np.arange(0, 255, dtype=np.uint32) << 23) | 0x8000,  # exact ties at every exponent
                         (np.arange(0, 255, dtype=np.uint32) << 23) | 0x18000,
                         (np.arange(0, 255, dtype=np.uint32) << 23) | 0x7FFF,
                         np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x80000000, 0x00000001], np.uint32)])
  bits = bits[(bits >> 23 & 255) != 255]
  got = O.bf16_bits(bits.view(np.float32))
  for b, g in zip(bits, got):
    x = Fraction(float(np.uint32(b).view(np.float32)))
    cands = []
    for h in ((int(b) >> 16) - 1, int(b) >> 16, (int(b) >> 16) + 1):
      h &= 0xFFFF
      if (h >> 7 & 255) == 255:
        if (h & 127) == 0: cands.append((h, math.inf if h >> 15 == 0 else -math.inf))
        continue
      cands.append((h, Fraction(float(np.uint32(h << 16).view(np.float32)))))
    best = min(abs(v - x) for _, v in cands if not isinstance(v, float))
    ok = [h for h, v in cands if not isinstance(v, float) and abs(v - x) == best]
    want = [h for h in ok if h % 2 == 0] if len(ok) > 1 else ok
    if not want or int(g) != want[0]:
      # above the largest finite bf16's half-way point rounding gives infinity
      assert (int(g) >> 7 & 255) == 255 and (int(g) & 127) == 0, hex(b)
  assert O.bf16_bits(np.float32(1 + 2**-8)) == 0x3F80  # a tie, to even
  assert O.bf16_bits(np.float32(1 + 3 * 2**-8)) == 0x3F82  # a tie, to even (up)


@pytest.mark.parametrize("dtype", O.FORMATS)
def test_bfp_every_value_and_exponent(dtype):
  # every finite bf16 value v with every block exponent top >= its own: the block float keeps
  # q = min(floor(|v| / step + 1/2), qmax) steps of 2^(top - 133) (bfp8, qmax 127) or 2^(top - 129) (bfp4, qmax 7),
  # v's sign on a q above 0. For a subnormal v (exponent field 0) the reference's rounding reads its magnitude as
  # m 2^-134, half its value (models/gpt2.py:26): that is what the chip does, and what is checked here.
  vals = all_bf16()
  e = (vals >> 7 & 255).astype(np.int64)
  for top in range(0, 255):
    sel = vals[e <= top]
    if sel.size == 0: continue
    n = sel.size
    pad = (-n) % 15
    sel = np.concatenate([sel, np.zeros(pad, np.uint16)])
    blocks = sel.reshape(-1, 15)
    carrier = np.full((blocks.shape[0], 1), top << 7, np.uint16)  # 2^(top-127): sets the block's exponent to top
    x = O.bf16_floats(np.concatenate([carrier, blocks], 1))
    q, tops = O.bfp_parts(x, dtype)
    assert (tops == top).all()
    q = q[:, 1:].reshape(-1)[:n]
    v = sel[:n]
    ee = (v >> 7 & 255).astype(np.int64)
    mag = np.abs(O.bf16_floats(v).astype(np.float64))
    mag = np.where(ee == 0, mag / 2, mag)  # the reference's reading of a subnormal
    step = 2.0 ** (top - (133 if dtype == "bfp8" else 129))
    qmax = 127 if dtype == "bfp8" else 7
    want = np.minimum(np.floor(mag / step + 0.5), qmax)
    want = np.where(v >> 15 != 0, -want, want)
    assert np.array_equal(q, want.astype(np.int32)), (dtype, top)


def test_bfp_rational_sample():
  # the same rule on random blocks by Fractions: nearest multiple, ties away from 0, clamped
  rng = np.random.default_rng(1)
  x = O.bf16(rng.normal(0, 1, (40, 64)) * np.exp(rng.normal(0, 3, (40, 64))))
  for dtype, base, qmax in (("bfp8", 133, 127), ("bfp4", 129, 7)):
    q, top = O.bfp_parts(x, dtype)
    for i in range(x.shape[0]):
      for j in range(x.shape[1]):
        v = Fraction(float(x[i, j]))
        step = Fraction(2) ** (int(top[i, j // 16]) - base)
        n = min(math.floor(abs(v) / step + Fraction(1, 2)), qmax)
        assert q[i, j] == (-n if v < 0 else n), (dtype, i, j)
    vals = O.bfp(x, dtype)
    assert np.array_equal(vals, np.where(q == 0, 0.0, vals))  # no -0
    assert (np.signbit(vals) == (q < 0)).all()


def test_bfp_special_cases():
  # saturation without an exponent bump; zeros; a block of zeros; bfp4's shift of 4 and more; no -0; K-blocked axis
  top_val = np.float32(2.0 ** 0 * (1 + 127 / 128))  # m = 255 at the top exponent: rounds to 128 -> saturates at 127
  x = np.zeros(16, np.float32); x[0] = top_val
  q, top = O.bfp_parts(x, "bfp8")
  assert q[0] == 127 and top[0] == 127
  q, top = O.bfp_parts(x, "bfp4")
  assert q[0] == 7
  q, top = O.bfp_parts(np.zeros(16, np.float32), "bfp8")
  assert (q == 0).all() and top[0] == 0
  x = np.array([1.0, -2.0 ** -9] + [0.0] * 14, np.float32)  # -2^-9 is 9 binades below: 0, unsigned
  assert O.bfp_parts(x, "bfp8")[0][1] == 0 and not np.signbit(O.bfp(x)[1])
  x = np.array([1.0, -2.0 ** -4] + [0.0] * 14, np.float32)  # bfp4: a shift of 4 gives 0
  assert O.bfp_parts(x, "bfp4")[0][1] == 0
  w = O.bf16(np.random.default_rng(2).normal(0, 1, (32, 48)))
  assert np.array_equal(O.bfp(w, "bfp8", axis=0), O.bfp(w.T, "bfp8").T)


@pytest.mark.parametrize("dtype", O.FORMATS)
def test_decode_every_code(dtype):
  # every (q, top, sign): the unpacker's normalised bf16 (tensor._bf16s) is q 2^(top - 133) (bfp8) or q 2^(top - 129)
  # (bfp4) exactly wherever that is a normal bf16, and exact_bf16 is that value everywhere
  qmax = 127 if dtype == "bfp8" else 7
  qs = np.arange(-qmax, qmax + 1)
  tops = np.arange(0, 255)
  Q = np.repeat(qs, 16)[None, :].repeat(len(tops), 0)  # each row: every q 16 times... one block per q value
  Q = Q.reshape(len(tops), -1)
  T = np.repeat(tops[:, None], Q.shape[1] // 16, 1)
  want = O.bfp_values(Q, T, dtype)
  got = O.decode_bf16(Q, T, dtype)
  exact = O.exact_bf16(Q, T, dtype)
  assert np.array_equal(O.bf16_floats(exact).astype(np.float64), want)
  normal = np.abs(want) >= 2.0 ** -126
  assert np.array_equal(got[normal], exact[normal])
  assert (got[Q == 0] == 0).all()


def test_pack_layout_roundtrip():
  rng = np.random.default_rng(3)
  w = O.bf16(rng.normal(0, 0.02, (64, 96)))
  for dtype in O.FORMATS:
    q, top = O.bfp_parts(w, dtype)
    mant, exps = O.pack_layout(q, top, dtype)
    assert exps.shape == (6, 64)
    if dtype == "bfp8":
      back = mant.view(np.int8).reshape(6, 64, 16).transpose(1, 0, 2).reshape(64, 96)
    else:
      lo = (mant & 15).astype(np.int8); hi = (mant >> 4).astype(np.int8)
      lo = np.where(lo > 7, lo - 16, lo); hi = np.where(hi > 7, hi - 16, hi)
      back = np.stack([lo, hi], -1).reshape(6, 64, 16).transpose(1, 0, 2).reshape(64, 96)
    assert np.array_equal(back, q)


def test_head_of_pinned():
  # the heads' oracle (serve.py:23-27) against a brute-force sort by (-value, column) on rows full of ties, and its
  # log-sum-exp against scipy's, at several temperatures
  from scipy.special import logsumexp
  from oracle.serve import head_of
  rng = np.random.default_rng(50)
  for n, k in ((7, 7), (100, 1), (300, 64), (2000, 33)):
    x = (np.round(rng.normal(0, 2, n) * 2) / 2).astype(np.float32)  # steps of 0.5: many equal values
    x[rng.integers(0, n, 3)] = -np.inf
    for t in (1.0, 0.5, 2.0):
      v, i, lse = head_of(x, t, k)
      want = sorted(range(n), key=lambda c: (-x[c], c))[:k]
      assert list(i) == want and np.array_equal(v, x[want])
      assert abs(lse - logsumexp(np.float64(x) * t)) <= 1e-12 * abs(lse) + 1e-12


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_c_restatement_is_numpys(fmt):
  # oracle/bfp_c.c (the full-width tests' bfp) against oracle/bfp.py's bfp, bit for bit: every finite bf16 value in a
  # run with 15 others whose largest exponent is drawn from 0..254 (so every shift, subnormal scales included), as bf16
  # bits and as float32 values, and random float32 matrices (rounded to bf16 first)
  from oracle import cbfp
  rng = np.random.default_rng(7)
  allv = np.arange(65536, dtype=np.uint32)
  allv = allv[((allv >> 7) & 255) != 255].astype(np.uint16)  # finite values
  runs = np.empty((allv.size, 16), np.uint16)
  runs[:, 0] = allv
  tops = rng.integers(0, 255, allv.size)
  for j in range(1, 16):  # exponents at most the drawn top, one of them the top itself
    e = np.minimum(rng.integers(0, 255, allv.size), tops) if j > 1 else tops
    runs[:, j] = (rng.integers(0, 2, allv.size) << 15 | e << 7 | rng.integers(0, 128, allv.size)).astype(np.uint16)
  for a in (runs, O.bf16_floats(runs)):
    got = cbfp.bfp(a, fmt)
    want = O.bfp(O.bf16_floats(runs), fmt).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), fmt
  m = rng.normal(0, 0.02, (64, 4096)).astype(np.float32)
  m[3, :16] = 0
  assert np.array_equal(cbfp.bfp(m, fmt).view(np.uint32), O.bfp(m, fmt).astype(np.float32).view(np.uint32))
