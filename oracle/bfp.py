"""CPU restatement (numpy) of ferrite's bf16 rounding and block-float formats: the checker for the HIP kernels.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only to check or to time the CPU path; the product (ferrite_amd) never calls it.

Each function cites the reference file:line it follows (paths under alkinun/ferrite). How each is pinned, beyond
restating it: tests/test_oracle.py checks bf16_bits against exact rational rounding, bfp against an independent
rational-arithmetic rounding of every (bf16 value, block exponent) pair, and decode_bf16 against q * 2^(e - 133) over
every (q, e, sign). The reference commits no golden vectors for these functions and cannot be imported here, so no
vectors were written from it.
"""
import numpy as np

FORMATS = ("bfp8", "bfp4")


def bf16_bits(a, packer=False):
  """fp32 values as bf16 bits: to nearest even, or half up as the chip's packer rounds (models/gpt2.py:16-18)."""
  b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)  # (64-bit: no wrap where the reference's uint32 wraps)
  r = (b + (0x8000 if packer else 0x7FFF + (b >> 16 & 1))) >> 16
  return (r & 0xFFFF).astype(np.uint16)


def bf16_floats(bits):
  """bf16 bits as float32 values (models/gpt2.py:19)."""
  return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def bf16(a):
  """a rounded to bf16 (nearest even), as float32."""
  return bf16_floats(bf16_bits(a))


def _runs(x):
  return x.reshape(*x.shape[:-1], -1, 16)


def bfp_parts(a, dtype="bfp8"):
  """The block float of a along its last axis, as the chip casts it (models/gpt2.py:21-32): (q, top), q the signed
  magnitude of each value (-127..127 for bfp8, -7..7 for bfp4; no sign on a zero) in a's shape, top each run of 16's
  exponent (the largest bf16 biased exponent in it), shape a.shape[:-1] + (n/16,)."""
  assert dtype in FORMATS, dtype
  a = np.asarray(a)
  assert a.shape[-1] % 16 == 0, "runs of 16 along the last axis"
  bits = bf16_bits(a).astype(np.int64)
  s, e = bits >> 15, bits >> 7 & 255
  m = (bits & 127) | np.where(e != 0, 128, 0)
  top = _runs(e).max(-1, keepdims=True)
  shift = np.minimum(top - _runs(e), 8)
  if dtype == "bfp8":
    q = np.minimum((_runs(m) + (1 << shift)) >> (shift + 1), 127)
  else:
    q = np.where(shift < 4, np.minimum((_runs(m) + (16 << np.minimum(shift, 3))) >> (np.minimum(shift, 3) + 5), 7), 0)
  q = np.where(_runs(s) != 0, -q, q).reshape(a.shape)
  return q.astype(np.int32), top[..., 0].astype(np.int32)


def bfp_values(q, top, dtype="bfp8"):
  """The values of a block float's parts, float64 and exact: q 2^(top - 133) (bfp8), q 2^(top - 129) (bfp4)."""
  q = np.asarray(q, np.float64)
  scale = np.ldexp(1.0, np.asarray(top, np.int64) - (133 if dtype == "bfp8" else 129))
  return (_runs(q) * scale[..., None]).reshape(q.shape)


def bfp(a, dtype="bfp8", axis=-1):
  """numpy's model of a block float as the chip makes it, as float64 values (models/gpt2.py:21-32). axis: the axis
  the runs of 16 lie along; -1 is ferrite's (the last axis of a weight stored for x @ w); 0 on a matrix blocks down
  its columns, bfp(a.T).T."""
  a = np.asarray(a)
  if axis in (-1, a.ndim - 1):
    q, top = bfp_parts(a, dtype)
    return bfp_values(q, top, dtype)
  return np.moveaxis(bfp(np.moveaxis(a, axis, -1), dtype), -1, axis)


def decode_bf16(q, top, dtype="bfp8"):
  """A block float's values as bf16 bits the unpacker's way (ferrite/tensor.py:718-727): normalised, a magnitude of 0
  as 0 (the parts here never carry a sign on a zero). Wherever the result is a normal bf16 (top - shift >= 1) this is
  exactly bfp_values' value; below that the unpacker's exponent wraps modulo 256 and this returns what it does."""
  q = np.asarray(q, np.int64)
  x = np.abs(q) if dtype == "bfp8" else np.abs(q) << 4  # bfp4's 3 bits sit at the top of bfp8's 7
  sign = (q < 0).astype(np.int64)
  e = np.repeat(np.asarray(top, np.int64), 16, -1).reshape(q.shape)
  m = x << 1
  bl = np.zeros_like(m)
  for i in range(8):  # bit_length of m (at most 8 bits)
    bl = np.where(m >> i != 0, i + 1, bl)
  shift = 8 - bl
  out = sign << 15 | ((e - shift) % 256) << 7 | ((m << shift) & 0x7E)
  return np.where(x == 0, 0, out).astype(np.uint16)


def exact_bf16(q, top, dtype="bfp8"):
  """The bf16 bits of each value, exactly (every block-float value is a bf16 value; below 2^-126 a subnormal)."""
  v = bfp_values(q, top, dtype).astype(np.float32)  # exact: at most 7 significant bits, exponent >= -133
  return (v.view(np.uint32) >> 16).astype(np.uint16)


# ---- the packed layout the HIP kernels use (FH_AXIS_N: runs along a row of W[K][N]) -------------------------------

def pack_layout(q, top, dtype="bfp8"):
  """The bytes libferrite_hip keeps for W[K][N] packed along N: exps [N/16][K], mant [N/16][K][16] int8 (bfp8) or
  [N/16][K][8] (bfp4: value 2i in byte i's low nibble, 2i+1 in its high one, each a signed 4-bit number)."""
  K, N = q.shape
  exps = np.ascontiguousarray(top.T).astype(np.uint8)  # top is [K][N/16]
  qb = q.reshape(K, N // 16, 16).transpose(1, 0, 2)
  if dtype == "bfp8":
    return np.ascontiguousarray(qb).astype(np.int8).view(np.uint8), exps
  nib = (qb & 15).astype(np.uint8)
  return np.ascontiguousarray(nib[..., 0::2] | nib[..., 1::2] << 4), exps


def gemv(x, w_values):
  """y = x @ W in float64 with W's block-float values: numpy's mm (models/llama.py:33)."""
  return np.asarray(x, np.float64) @ np.asarray(w_values, np.float64)
