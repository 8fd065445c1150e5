"""The hot path's operations on torch tensors resident on the GPU: shape and dtype checks on the host, then one call
into libferrite_hip.so on torch's current stream. torch is the buffer and stream provider only; every computation is
a HIP kernel of the library, and a missing library raises (ferrite_amd.lib.load)."""
import ctypes
from dataclasses import dataclass
import torch
from ferrite_amd import lib

_TORCH = {torch.float32: lib.F32, torch.bfloat16: lib.BF16}


def _ptr(t):
  return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
  return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(*ts):
  for t in ts:
    if t is not None and not t.is_cuda: raise ValueError("ferrite_amd: tensors must be on the GPU")


@dataclass
class BfpWeight:
  """A weight W[K][N] (x @ W) as a block float on the GPU: mant and exps in libferrite_hip's packed layout."""
  mant: torch.Tensor
  exps: torch.Tensor
  K: int
  N: int
  fmt: str  # "bfp8" or "bfp4"
  axis: int = lib.AXIS_N

  @property
  def nbytes(self): return self.mant.numel() + self.exps.numel()


def pack(w, fmt="bfp8", axis=lib.AXIS_N):
  """w [K][N] (fp32 or bf16, on the GPU) as a block float (fh_bfp_pack)."""
  _dev(w)
  if w.dim() != 2: raise ValueError("pack: a matrix")
  if w.dtype not in _TORCH: raise ValueError("pack: fp32 or bf16")
  w = w if w.stride(1) == 1 else w.contiguous()
  K, N = w.shape
  mb, eb = lib.bfp_bytes(K, N, lib.DTYPES[fmt], axis)
  mant = torch.empty(mb, dtype=torch.uint8, device=w.device)
  exps = torch.empty(eb, dtype=torch.uint8, device=w.device)
  lib.call("fh_bfp_pack", _ptr(w), _TORCH[w.dtype], K, N, w.stride(0), lib.DTYPES[fmt], axis, _ptr(mant), _ptr(exps), _stream())
  return BfpWeight(mant, exps, K, N, fmt, axis)


def bfp_empty(K, N, fmt="bfp8", device="cuda"):
  """An unfilled block float W[K][N] packed along N, for pack_rows_into."""
  mb, eb = lib.bfp_bytes(K, N, lib.DTYPES[fmt], lib.AXIS_N)
  return BfpWeight(torch.empty(mb, dtype=torch.uint8, device=device), torch.empty(eb, dtype=torch.uint8, device=device),
                   K, N, fmt)


def pack_rows_into(bw, part, n0):
  """Columns n0 .. n0 + out of bw (a W[K][N] packed along N) from part [out][K] (fp32 or bf16 on the GPU): W's columns
  as a checkpoint stores a linear layer's rows (models/llama.py's load transposes them for x @ w, llama.py:572-604).
  The part is packed along its first axis (FH_AXIS_K, runs of 16 down its columns), whose layout is that of its
  transpose packed along N: run-blocks n0 / 16 .. of bw, byte for byte, with no transposed copy formed. n0 and out are
  multiples of 16."""
  _dev(part)
  if bw.axis != lib.AXIS_N: raise ValueError("pack_rows_into: a weight packed along N")
  if part.dim() != 2 or part.shape[1] != bw.K or part.dtype not in _TORCH or part.stride(1) != 1:
    raise ValueError(f"pack_rows_into: part [out][{bw.K}] fp32 or bf16 with contiguous rows, not {tuple(part.shape)} {part.dtype}")
  out = part.shape[0]
  if n0 % 16 or out % 16 or n0 + out > bw.N: raise ValueError(f"pack_rows_into: columns {n0}..{n0 + out} of {bw.N} (multiples of 16)")
  fmt = lib.DTYPES[bw.fmt]
  m0, e0 = lib.bfp_bytes(bw.K, n0, fmt, lib.AXIS_N) if n0 else (0, 0)
  mb, eb = lib.bfp_bytes(out, bw.K, fmt, lib.AXIS_K)
  assert m0 + mb <= bw.mant.numel() and e0 + eb <= bw.exps.numel()
  lib.call("fh_bfp_pack", _ptr(part), _TORCH[part.dtype], out, bw.K, part.stride(0), fmt, lib.AXIS_K,
           ctypes.c_void_p(bw.mant.data_ptr() + m0), ctypes.c_void_p(bw.exps.data_ptr() + e0), _stream())


def pack_parts(parts, fmt="bfp8"):
  """W = [P0ᵀ | P1ᵀ | ...] packed along N from parts in a checkpoint's layout, P_i [out_i][K]: a fused q|k|v or
  gate|up (models/llama.py:376-427) straight from the checkpoint's rows (pack_rows_into)."""
  K, N = parts[0].shape[1], sum(p.shape[0] for p in parts)
  bw = bfp_empty(K, N, fmt, parts[0].device)
  n0 = 0
  for p in parts:
    pack_rows_into(bw, p, n0)
    n0 += p.shape[0]
  return bw


def dequant(bw, out=None):
  """The weight's values as bf16 [K][N] (fh_bfp_dequant), bit for bit."""
  if out is None: out = torch.empty(bw.K, bw.N, dtype=torch.bfloat16, device=bw.mant.device)
  lib.call("fh_bfp_dequant", _ptr(bw.mant), _ptr(bw.exps), bw.K, bw.N, lib.DTYPES[bw.fmt], bw.axis, _ptr(out), out.stride(0), _stream())
  return out


@dataclass
class Tiles16:
  """bf16 rows [rows][cols] in tiles of 16 rows (FH_BF16_T16): element (r, c) at (r // 16) * 16 * cols + (c // 8) * 128
  + (r % 16) * 8 + c % 8 of `data`, which holds 16 * ceil(rows / 16) rows. The rows a decode step of many sequences
  passes between its matrix-core matmuls (each 16 rows' 8 columns one contiguous 256-byte piece)."""
  data: torch.Tensor
  rows: int
  cols: int

  @property
  def dtype(self): return "bf16_t16"

  def to_rows(self):
    """The rows as a [rows][cols] bf16 tensor (a copy)."""
    r16 = -(-self.rows // 16) * 16
    t = self.data.view(r16 // 16, self.cols // 8, 16, 8).permute(0, 2, 1, 3).reshape(r16, self.cols)
    return t[:self.rows].contiguous()


def tiles16(rows, cols, device="cuda", fill=0.0):
  """Zeros (or `fill`) as bf16 tiles of 16 rows: [rows][cols], cols a multiple of 8."""
  if cols % 8: raise ValueError("tiles16: cols a multiple of 8")
  r16 = -(-rows // 16) * 16
  return Tiles16(torch.full((r16 * cols,), fill, dtype=torch.bfloat16, device=device), rows, cols)


def to_tiles16(x, fill=0.0):
  """A [rows][cols] tensor's values as bf16 tiles of 16 rows (the rows past `rows` in the last tile hold `fill`)."""
  rows, cols = x.shape
  t = tiles16(rows, cols, x.device, fill)
  r16 = -(-rows // 16) * 16
  full = torch.full((r16, cols), fill, dtype=torch.bfloat16, device=x.device)
  full[:rows] = x.to(torch.bfloat16)
  t.data.copy_(full.view(r16 // 16, 16, cols // 8, 8).permute(0, 2, 1, 3).reshape(-1))
  return t


def epilogue(kind=lib.EP_STORE, **kw):
  """An fh_epilogue; tensors given are kept alive with it (the kernel reads them when it runs, after this returns). A
  Tiles16 copy_bf16 sets copy_tiles."""
  ep = lib.Epilogue()
  ep.kind = kind
  ep.keep = []
  for k, v in kw.items():
    if isinstance(v, Tiles16):
      if k != "copy_bf16": raise ValueError(f"epilogue: {k} cannot be bf16 tiles")
      _dev(v.data)
      ep.keep.append(v.data)
      ep.copy_tiles = 1
      v = v.data.data_ptr()
    if isinstance(v, torch.Tensor):
      _dev(v)
      ep.keep.append(v)
      v = v.data_ptr()
    setattr(ep, k, v)
  return ep


def _layout(t):
  """(pointer, dtype code, row stride, rows) of a matmul operand: a [rows][cols] tensor or bf16 tiles of 16 rows."""
  if isinstance(t, Tiles16):
    _dev(t.data)
    return t.data.data_ptr(), lib.BF16_T16, t.cols, t.rows
  _dev(t)
  return _ptr(t), _TORCH[t.dtype], t.stride(0), t.shape[0]


def _matmul(entry, x, bw, ep, out, out_dtype):
  if bw.axis != lib.AXIS_N:
    if entry != "fh_gemv_bfp": raise NotImplementedError(f"{entry}: weights packed along N (along K: the GEMV)")
    entry = "fh_gemv_bfp_k"
  if isinstance(x, Tiles16):
    if x.cols != bw.K: raise ValueError(f"{entry}: x tiles of {x.cols} columns for W {bw.K}x{bw.N}")
  elif x.dim() != 2 or x.shape[1] != bw.K or x.stride(1) != 1: raise ValueError(f"{entry}: x {tuple(x.shape)} for W {bw.K}x{bw.N}")
  xp, xdt, ldx, rows = _layout(x)
  if out is None:
    cols = bw.N
    if ep is not None and ep.kind == lib.EP_SILU_GATE: cols = ep.split
    if ep is not None and ep.kind == lib.EP_ROPE_KV: cols = ep.heads * ep.head_dim
    dev = x.data.device if isinstance(x, Tiles16) else x.device
    out = torch.empty(rows, cols, dtype=out_dtype, device=dev)
  yp, ydt, ldy, _ = _layout(out)
  lib.call(entry, xp, xdt, ldx, rows, bw.K, bw.N, _ptr(bw.mant), _ptr(bw.exps),
           lib.DTYPES[bw.fmt], ctypes.byref(ep) if ep is not None else None, yp, ydt, ldy, _stream())
  return out


def gemv(x, bw, ep=None, out=None, out_dtype=torch.float32):
  """y = x @ W with the epilogue ep: a few rows, fp32 x, exact products. W packed along N (fh_gemv_bfp), or along K
  (fh_gemv_bfp_k: the store, residual and program epilogues)."""
  return _matmul("fh_gemv_bfp", x, bw, ep, out, out_dtype)


def gemm(x, bw, ep=None, out=None, out_dtype=torch.float32):
  """y = x @ W with the epilogue ep (fh_gemm_bfp): many rows on the matrix cores, x (fp32 or bf16) rounded to bf16. x
  and out may be Tiles16 (up to 64 rows, K a multiple of 64)."""
  return _matmul("fh_gemm_bfp", x, bw, ep, out, out_dtype)


_DT_OUT = {torch.float32: lib.F32, torch.bfloat16: lib.BF16, torch.int32: lib.I32}


def matmul(a, b, program=None, out=None, out_dtype=torch.float32):
  """out[i] = program(a[i] @ b[i]) (fh_matmul) for plain operands: a [batch][M][K], b [batch][K][N] (fp32 or bf16,
  rows contiguous; a batch of 1 serves every entry), out [batch][M][N] (fp32, bf16 or int32, rows contiguous). An fp32
  operand goes in as ferrite's bf16x3. program: an fh_program over the sum (lib.OPND_ACC), or None to store it."""
  _dev(a, b)
  if a.dim() != 3 or b.dim() != 3 or a.shape[2] != b.shape[1]: raise ValueError(f"matmul: {tuple(a.shape)} @ {tuple(b.shape)}")
  if a.dtype not in _TORCH or b.dtype not in _TORCH: raise ValueError("matmul: fp32 or bf16 operands")
  if a.stride(2) != 1 or b.stride(2) != 1: raise ValueError("matmul: operands' rows contiguous")
  batch = max(a.shape[0], b.shape[0])
  if a.shape[0] not in (1, batch) or b.shape[0] not in (1, batch): raise ValueError(f"matmul: batches {a.shape[0]} and {b.shape[0]}")
  M, K, N = a.shape[1], a.shape[2], b.shape[2]
  if out is None: out = torch.empty(batch, M, N, dtype=out_dtype, device=a.device)
  if tuple(out.shape) != (batch, M, N) or out.stride(2) != 1 or out.dtype not in _DT_OUT: raise ValueError(f"matmul: out {tuple(out.shape)}")
  sa = a.stride(0) if a.shape[0] > 1 else 0
  sb = b.stride(0) if b.shape[0] > 1 else 0
  lib.call("fh_matmul", _ptr(a), _TORCH[a.dtype], sa, a.stride(1), _ptr(b), _TORCH[b.dtype], sb, b.stride(1), batch, M, K, N,
           ctypes.byref(program) if program is not None else None, _ptr(out), _DT_OUT[out.dtype], out.stride(0), out.stride(1), _stream())
  return out


def embed_rows(table, ids, x=None, ssq=None):
  """Rows ids of table into x (fp32), with their sums of squares by runs of 16 (fh_embed_rows)."""
  _dev(table, ids)
  vocab, dim = table.shape
  batch = ids.numel()
  if x is None: x = torch.empty(batch, dim, dtype=torch.float32, device=table.device)
  if ssq is None: ssq = torch.empty(batch, dim // 16, dtype=torch.float32, device=table.device)
  lib.call("fh_embed_rows", _ptr(table), _TORCH[table.dtype], vocab, dim, _ptr(ids), batch, _ptr(x), _ptr(ssq), _stream())
  return x, ssq


@dataclass
class BfpCache:
  """A KV cache [planes = 2 kv][length][head_dim] in a block float (bfp8 or bfp4; models/llama.py:127-128): one uint8
  buffer in fh_kv_cache_bytes' layout, every row's magnitudes then every row's exponents. Zero bytes: zeros."""
  data: torch.Tensor
  fmt: str
  planes: int
  length: int
  head_dim: int

  @property
  def shape(self): return (self.planes, self.length, self.head_dim)

  @property
  def dtype(self): return self.fmt

  def zero_(self):
    self.data.zero_()
    return self

  def copy_(self, other):
    if other.shape != self.shape or other.fmt != self.fmt: raise ValueError("BfpCache.copy_: another shape or format")
    self.data.copy_(other.data)
    return self


def kv_cache(planes, length, head_dim, fmt="bf16", device="cuda"):
  """A KV cache of zeros [planes][length][head_dim]: a torch tensor for fp32 and bf16, a BfpCache for bfp8 and bfp4."""
  if fmt in ("fp32", "bf16"):
    return torch.zeros(planes, length, head_dim, dtype=torch.float32 if fmt == "fp32" else torch.bfloat16, device=device)
  if planes % 2: raise ValueError("kv_cache: keys' planes then values', an even count")
  n = lib.load().fh_kv_cache_bytes(lib.DTYPES[fmt], planes // 2, length, head_dim)
  if not n: raise ValueError(f"kv_cache: no {fmt} cache of head_dim {head_dim}")
  return BfpCache(torch.zeros(n, dtype=torch.uint8, device=device), fmt, planes, length, head_dim)


def cache_fields(cache):
  """The fh_epilogue / attention arguments of a cache: (tensor, cache_dtype, cache_len)."""
  if isinstance(cache, BfpCache): return cache.data, lib.DTYPES[cache.fmt], cache.length
  if cache.dtype not in _TORCH or cache.dim() != 3: raise ValueError("a KV cache is [2 kv][len][hd], fp32 or bf16, or a BfpCache")
  return cache, _TORCH[cache.dtype], cache.shape[1]


def attention_workspace(batch, heads, head_dim, max_context, device="cuda"):
  """fh_attention_decode's workspace, uninitialised (a workspace needs no clearing)."""
  n = lib.load().fh_attention_workspace_bytes(batch, heads, head_dim, max_context)
  return torch.empty(max(n, 256), dtype=torch.uint8, device=device)


def attention_decode(q, cache, heads, kv_heads, head_dim, places, first_row, max_context, workspace, o=None):
  """softmax(q k^T / sqrt(hd)) v over each row's cache rows (fh_attention_decode). cache [2 kv][len][hd] (fp32, bf16 or
  a BfpCache); o fp32 (by default) or bf16, or bf16 Tiles16 of q's shape."""
  data, dtype, length = cache_fields(cache)
  _dev(q, data, places, first_row)
  batch = q.shape[0]
  if o is None: o = torch.empty_like(q)
  if isinstance(o, Tiles16):
    if (o.rows, o.cols) != tuple(q.shape): raise ValueError("attention_decode: o tiles of q's shape")
  elif o.dtype not in (torch.float32, torch.bfloat16) or o.shape != q.shape or not o.is_contiguous():
    raise ValueError("attention_decode: o is a contiguous fp32 or bf16 tensor of q's shape")
  op, odt, _, _ = _layout(o)
  lib.call("fh_attention_decode", _ptr(q), _ptr(data), dtype, length, batch, heads, kv_heads, head_dim, _ptr(places),
           _ptr(first_row), max_context, op, odt, _ptr(workspace), workspace.numel(), _stream())
  return o


def attention_prefill(q, cache, heads, kv_heads, head_dim, p0, slot_row, o=None, out_dtype=torch.float32):
  """A prompt's causal attention (fh_attention_prefill): q [T][heads*hd] at places p0 .. p0 + T - 1 of the sequence
  whose cache rows start at slot_row; cache [2 kv][len][hd]."""
  data, dtype, length = cache_fields(cache)
  _dev(q, data)
  T = q.shape[0]
  if o is None: o = torch.empty(T, heads * head_dim, dtype=out_dtype, device=q.device)
  _dev(o)
  lib.call("fh_attention_prefill", _ptr(q), q.stride(0), _ptr(data), dtype, length, T, heads,
           kv_heads, head_dim, p0, slot_row, _ptr(o), _TORCH[o.dtype], o.stride(0), _stream())
  return o


def rms_rows(x, w, eps, centered=False, out=None, out_dtype=torch.bfloat16):
  """x * rsqrt(mean(x^2) + eps) * w, a row at a time (fh_rms_rows); bf16 out by default (a prefill GEMM's input), or
  bf16 Tiles16."""
  _dev(x, w)
  if out is None: out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
  op, odt, ldo, _ = _layout(out)
  lib.call("fh_rms_rows", _ptr(x), x.stride(0), x.shape[0], x.shape[1], _ptr(w), eps, int(centered), op, odt, ldo,
           _stream())
  return out


def moe_route(x, router, experts, k, norm_topk=True, norm_w=None, eps=1e-5, centered=False):
  """Router logits, top k and their weights (fh_moe_route): (ids [rows][k] int32, weights [rows][k], dense [rows][E])."""
  _dev(x, router, norm_w)
  rows, dim = x.shape
  ids = torch.empty(rows, k, dtype=torch.int32, device=x.device)
  wts = torch.empty(rows, k, dtype=torch.float32, device=x.device)
  dense = torch.empty(rows, experts, dtype=torch.float32, device=x.device)
  lib.call("fh_moe_route", _ptr(x), x.stride(0), rows, dim, _ptr(norm_w), eps, int(centered), _ptr(router),
           _TORCH[router.dtype], experts, k, int(norm_topk), _ptr(ids), _ptr(wts), _ptr(dense), _stream())
  return ids, wts, dense


@dataclass
class Experts:
  """A mixture of experts' weights on the GPU: gate_up, the experts' [dim][2 ffn] packed one after another; down, the
  experts' [ffn][dim] packed one after another."""
  gate_up: BfpWeight
  down: BfpWeight
  experts: int
  dim: int
  ffn: int


def pack_experts(gate_up, down, fmt="bfp4"):
  """gate_up [E][dim][2 ffn] and down [E][ffn][dim] (fp32 or bf16, on the GPU) as block floats (fh_bfp_pack)."""
  E, dim, two = gate_up.shape
  ffn = two // 2
  parts = [pack(gate_up[e], fmt) for e in range(E)]
  gu = BfpWeight(torch.cat([p.mant for p in parts]), torch.cat([p.exps for p in parts]), dim, 2 * ffn, fmt)
  parts = [pack(down[e], fmt) for e in range(E)]
  dn = BfpWeight(torch.cat([p.mant for p in parts]), torch.cat([p.exps for p in parts]), ffn, dim, fmt)
  return Experts(gu, dn, E, dim, ffn)


def moe_experts(x, ex, dense, out=None, residual=None, ssq_out=None, norm_w=None, ssq_in=None, eps=1e-5, centered=False, ws=None):
  """The picked experts' SwiGLUs weighted by dense and summed, plus residual (fh_moe_experts). x [rows][dim] fp32."""
  _dev(x, dense, out, residual, ssq_out, norm_w, ssq_in)
  rows = x.shape[0]
  if out is None: out = torch.empty(rows, ex.dim, dtype=torch.float32, device=x.device)
  n = lib.load().fh_moe_workspace_bytes(rows, ex.experts, ex.ffn, ex.dim)
  if ws is None or ws.numel() < n: ws = torch.empty(max(n, 256), dtype=torch.uint8, device=x.device)
  lib.call("fh_moe_experts", _ptr(x), x.stride(0), rows, ex.dim, _ptr(norm_w), _ptr(ssq_in), eps, int(centered),
           ex.experts, ex.ffn, _ptr(ex.gate_up.mant), _ptr(ex.gate_up.exps), lib.DTYPES[ex.gate_up.fmt], _ptr(ex.down.mant),
           _ptr(ex.down.exps), lib.DTYPES[ex.down.fmt], _ptr(dense), _ptr(out), _ptr(residual), _ptr(ssq_out), _ptr(ws),
           ws.numel(), _stream())
  return out


def logit_heads(logits, k=64, inv_temp=None, ws=None):
  """Each row's head (fh_logit_heads; models/serve.py:31-47): its k largest logits, largest first and the first column
  of equals first, their columns, and given inv_temp (each row's 1/temperature, [rows] fp32) the log of the sum of
  exp(x t) over the row: (values [rows][k], ids [rows][k] int32[, lse [rows]])."""
  _dev(logits, inv_temp)
  if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1: raise ValueError("logit_heads: fp32 rows")
  rows, vocab = logits.shape
  values = torch.empty(rows, k, dtype=torch.float32, device=logits.device)
  ids = torch.empty(rows, k, dtype=torch.int32, device=logits.device)
  lse = torch.empty(rows, dtype=torch.float32, device=logits.device) if inv_temp is not None else None
  n = lib.load().fh_heads_workspace_bytes(rows, vocab, k)
  if n and (ws is None or ws.numel() < n): ws = torch.empty(n, dtype=torch.uint8, device=logits.device)
  lib.call("fh_logit_heads", _ptr(logits), logits.stride(0), rows, vocab, k, _ptr(inv_temp), _ptr(values), _ptr(ids),
           _ptr(lse), _ptr(ws) if n else None, ws.numel() if n else 0, _stream())
  return (values, ids) if lse is None else (values, ids, lse)


def argmax_rows(x, ids=None):
  _dev(x)
  if ids is None: ids = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
  lib.call("fh_argmax_rows", _ptr(x), x.shape[0], x.shape[1], _ptr(ids), _stream())
  return ids


def argmax_parts(parts, ids=None):
  """Each row's argmax from the (value, column) pairs a GEMV epilogue left (fh_argmax_parts). parts: int64 [rows][n]."""
  _dev(parts)
  if ids is None: ids = torch.empty(parts.shape[0], dtype=torch.int32, device=parts.device)
  lib.call("fh_argmax_parts", _ptr(parts), parts.shape[0], parts.shape[1], _ptr(ids), _stream())
  return ids
