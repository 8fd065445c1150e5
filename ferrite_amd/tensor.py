"""ferrite's lazy Tensor (ferrite/tensor.py) on an MI355X: the same surface for the block-float matmul path
(Tensor.of, frombytes, tobytes/tolist, @ by a bfp8/bfp4 weight, cast, the elementwise ops and reductions, softmax),
built lazily and resolved on read, every computation a kernel of libferrite_hip.so.

A tensor is batch x rows x cols of bf16, fp32 or int32 (a torch tensor on the device, which is only its memory), or a
block float (bfp8/bfp4: a matmul's B, packed by fh_bfp_pack). Ops build a tree; realize() (reading does it) compiles
the tree under the root into as few launches as its shape allows, as ferrite's realize/_fit/_tree do (tensor.py:247-272,
651-767):
  - elementwise ops (and views: T, slices, expand, reshape of a stored tensor, read in place by strides) become one
    fh_program, at most MAX_OPS (15) ops over at most 8 inputs, run by fh_map;
  - a matmul by a block float with elementwise ops on top runs as one matmul kernel whose epilogue is that program
    (FH_EP_PROGRAM): fh_gemv_bfp for a few rows (products exact), fh_gemm_bfp for many (x in bf16, as the chip's);
  - a reduction (sum, max along an axis) is fh_reduce over its operand's program;
  - what does not fit (a tree of more than 15 ops, a value read by two kernels, a matmul's operands) is realized first,
    the heaviest shared part first.
Programs compute in fp32 and round once, to the result's dtype (bf16 to nearest even); ferrite's SFPU rounds where its
Dst does. int32 goes through fp32, exact below 2^24, as ferrite's does for what int32 does not do itself."""
import collections, contextlib, ctypes, math, time
import numpy as np
import torch
from ferrite_amd import lib, ops

MAX_OPS = lib.MAX_OPS
BFP = ("bfp8", "bfp4")
TORCH = {"bf16": torch.bfloat16, "fp32": torch.float32, "int32": torch.int32}
DT = {"bf16": lib.BF16, "fp32": lib.F32, "int32": lib.I32}
ITEMSIZE = {"bf16": 2, "fp32": 4, "int32": 4}
UNARY = ("relu", "exp", "exp2", "log", "log2", "sin", "cos", "recip", "sqrt", "ftob", "itof", "ftoi", "cast")
BINARY = ("add", "sub", "mul", "max", "cmplt", "cmpne", "keep", "drop")
INT32_OPS = ("add", "sub", "max", "cmplt", "cmpne", "keep", "drop")
REDUCE = {f"{f}{ax}": (f, ax) for f in ("sum", "max") for ax in range(3)}
ROWWISE = ("softmax", "log_softmax")  # along each row, a launch of their own (fh_softmax_rows)


class Runtime:
  """The GPU in the place of ferrite's Runtime(chip) (ferrite/runtime.py:304-310): a device and the HIP stream every
  launch of this runtime's tensors goes on, in order. Every buffer its tensors own is allocated with that stream
  current (on()), so torch's caching allocator hands a freed block only to later work on the same stream: a kernel
  still queued never sees its memory reused under it. wait() waits for the launches (Runtime.wait), profile() times
  them by name (Runtime.profile)."""

  TIMES = 4096  # launches whose times profile() keeps (ferrite/runtime.py's TIMES ring)

  def __init__(self, device=0):
    lib.load()
    self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
    self.stream = torch.cuda.Stream(device=self.device) if self.device.type == "cuda" else None
    self.launches = 0  # kernels launched (how many a realize took)
    self.queued = collections.deque()  # (launch, name, end event) of the launches that may not be done
    self.times = {}  # launch % TIMES -> (launch, name, start event, end event, bytes read or None)

  def on(self):
    """A context with this runtime's stream current: torch allocations and copies inside it are ordered with its
    launches."""
    return torch.cuda.stream(self.stream) if self.stream is not None else contextlib.nullcontext()

  def run(self, fn, name="launch", nbytes=None):
    """fn() with this runtime's stream current (its library calls go on it), as launch number self.launches + 1 named
    `name`, reading `nbytes` bytes of device memory (the algorithmic bytes of its operands, each once; None if not
    counted); outside a graph capture it is bracketed by events, which wait() polls and profile() reads. The launches
    already done leave the queue here too (its head polled), so a loop of launches with no wait() keeps at most the
    unfinished ones and TIMES more."""
    self.launches += 1
    if self.stream is None: return fn()
    with torch.cuda.stream(self.stream):
      if torch.cuda.is_current_stream_capturing(): return fn()  # (a recording's launches carry no events)
      start = torch.cuda.Event(enable_timing=True)
      start.record(self.stream)
      out = fn()
      end = torch.cuda.Event(enable_timing=True)
      end.record(self.stream)
    self.times[self.launches % self.TIMES] = (self.launches, name, start, end, nbytes)
    self.queued.append((self.launches, name, end))
    while len(self.queued) > self.TIMES and self.queued[0][2].query(): self.queued.popleft()
    return out

  def wait(self, timeout=60):
    """Until every launch queued has finished (Runtime.wait, ferrite/runtime.py:473-484): polls each launch's end
    event, so long as launches keep finishing. None finishing in `timeout` seconds means the GPU hangs: TimeoutError,
    naming the launch it is on and how many wait behind it."""
    since, last = time.monotonic(), None
    while True:
      while self.queued and self.queued[0][2].query(): self.queued.popleft()
      if not self.queued and (self.stream is None or self.stream.query()): return
      head = self.queued[0][0] if self.queued else None
      if head != last: since, last = time.monotonic(), head  # progress: the deadline starts again
      elif time.monotonic() - since > timeout:
        n, name, _ = self.queued[0] if self.queued else (self.launches, "a recording's launches", None)
        raise TimeoutError(f"no launch finished in {timeout} s: the GPU is on launch {n} ({name}), "
                           f"{max(0, len(self.queued) - 1)} queued behind it")
      time.sleep(0.0002)

  def profile(self, since):
    """The launches after launch number `since` by name, once they are done: [(name, launches, microseconds, bytes)],
    the most time first (Runtime.profile, ferrite/runtime.py:416-428). A launch's time runs between events recorded on
    the stream before and after it; its bytes are what the host counted for it (run's nbytes: each operand read once,
    a block float's packed bytes), summed by name, None where a launch of that name was not counted. Only the last
    TIMES launches are kept, and those replayed from a recording carry no events."""
    self.wait()
    assert self.launches - since <= self.TIMES, f"{self.launches - since} launches to profile, the last {self.TIMES} kept"
    totals = {}
    for n in range(since + 1, self.launches + 1):
      rec = self.times.get(n % self.TIMES)
      if rec is None or rec[0] != n: continue
      _, name, start, end, nbytes = rec
      t = totals.setdefault(name, [0, 0.0, 0])
      t[0] += 1
      t[1] += start.elapsed_time(end) * 1000.0
      t[2] = None if t[2] is None or nbytes is None else t[2] + nbytes
    return sorted(((name, k, us, b) for name, (k, us, b) in totals.items()), key=lambda r: -r[2])


class Tensor:
  """batch x rows x cols (ferrite/tensor.py:14-35): a stored tensor (data) or an op on others, until realized."""

  def __init__(self, rt, rows, cols, op=None, srcs=(), batch=1, dtype="bf16", args=()):
    self.rt, self.rows, self.cols, self.batch, self.op, self.srcs, self.dtype, self.args = rt, rows, cols, batch, op, srcs, dtype, args
    self.data = None  # a torch tensor [batch][rows][cols] (its strides may be a view's), or a BfpWeight

  @property
  def shape(self): return (self.batch, self.rows, self.cols)

  def __repr__(self): return f"Tensor({self.shape}, {self.dtype}{', ' + self.op if self.op else ''})"

  # ---- making and reading (ferrite/tensor.py:51-114) ------------------------------------------------------------
  @classmethod
  def _stored(cls, rt, t, dtype):
    x = cls(rt, t.shape[1], t.shape[2], batch=t.shape[0], dtype=dtype)
    x.data = t
    return x

  @classmethod
  def full(cls, rt, rows, cols, value, dtype="bf16"): return cls.of(rt, [[value] * cols for _ in range(rows)], dtype)

  @classmethod
  def of(cls, rt, data, dtype="bf16"):
    """From a list of rows of numbers, or a list of those (a batch), rounded to dtype (bf16: to nearest even)."""
    assert dtype not in BFP, "a block float is made on the GPU, by cast"
    matrices = data if isinstance(data[0][0], (list, tuple)) else [data]
    a = torch.tensor(matrices, dtype=torch.int32 if dtype == "int32" else torch.float32)
    with rt.on():  # (its memory allocated and filled on the runtime's stream)
      return cls._stored(rt, a.to(TORCH[dtype]).to(rt.device), dtype)

  @classmethod
  def frombytes(cls, rt, rows, cols, data, batch=1, dtype="bf16"):
    """From dtype's values in row-major order (little-endian), matrix after matrix."""
    assert dtype not in BFP, "a block float is made on the GPU, by cast"
    n = ITEMSIZE[dtype]
    assert len(data) == n * batch * rows * cols, f"{len(data)} bytes for {batch} x {rows} x {cols} of {dtype}"
    raw = torch.frombuffer(bytearray(data), dtype={2: torch.int16, 4: torch.int32}[n]).reshape(batch, rows, cols)
    with rt.on():
      return cls._stored(rt, raw.view(TORCH[dtype]).to(rt.device), dtype)

  def tobytes(self):
    """dtype's values in row-major order, as frombytes takes them (a block float's as bf16: each of its values is one,
    tensor._bf16s's). Waits for the launches queued."""
    x = self.realize()
    if x.dtype in BFP:
      t = x.rt.run(lambda: torch.stack([ops.dequant(w) for w in _matrices(x)]), "dequant")
    else:
      if not x.data.is_contiguous(): x = (x + 0).realize()  # a view: copied by our kernel first
      t = x.data
    x.rt.wait()
    t = t.cpu()
    return (t.view(torch.int16) if t.dtype == torch.bfloat16 else t).numpy().tobytes()

  def tolist(self):
    """Rows of numbers, or a list of those if this is a batch."""
    raw = self.tobytes()
    if self.dtype in ("bf16", *BFP): v = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
    else: v = np.frombuffer(raw, np.int32 if self.dtype == "int32" else np.float32)
    m = v.reshape(self.batch, self.rows, self.cols).tolist()
    return m if self.batch > 1 else m[0]

  def numpy(self):
    return np.array(self.tolist(), np.int32 if self.dtype == "int32" else np.float32).reshape(self.shape)

  # ---- views: read in place by strides (ferrite/tensor.py:149-233's views and moves) ----------------------------
  def _view(self, shape, offset, strides):
    src = self.realize()
    assert src.dtype not in BFP, "a block float is read only as a matmul's B"
    t = Tensor(self.rt, shape[1], shape[2], "view", (src,), shape[0], self.dtype)
    t.data = torch.as_strided(src.data, shape, strides, src.data.storage_offset() + offset)
    t.op, t.srcs = None, ()
    return t

  @property
  def T(self):
    """The transpose of each matrix, read in place (a matmul's block-float B is transposed when packed)."""
    if self.dtype in BFP: raise NotImplementedError("T of a block float: pack the transpose instead")
    x = self.realize()
    b, r, c = x.data.stride()
    return x._view((self.batch, self.cols, self.rows), 0, (b, c, r))

  def __getitem__(self, key):
    """x[b], one matrix of a batch; x[rows, cols] or x[batch, rows, cols] with slices (any positive step): a view."""
    x = self.realize()
    if isinstance(key, int):
      b, r, c = x.data.stride()
      return x._view((1, self.rows, self.cols), key * b, (b, r, c))
    key = (slice(None),) * (3 - len(key)) + tuple(key)
    rng = [range(*k.indices(n)) for k, n in zip(key, self.shape)]
    assert all(g.step > 0 and len(g) for g in rng), "slices of positive steps, not empty"
    st = x.data.stride()
    return x._view(tuple(map(len, rng)), sum(g.start * s for g, s in zip(rng, st)), tuple(g.step * s for g, s in zip(rng, st)))

  def permute(self, *order):
    """The axes in a new order, read in place (ferrite/tensor.py:186-190: swapping rows and columns is the transpose)."""
    assert sorted(order) == [0, 1, 2]
    if tuple(order) == (0, 1, 2): return self
    x = self.realize()
    st = x.data.stride()
    return x._view(tuple(self.shape[k] for k in order), 0, tuple(st[k] for k in order))

  def split(self, n, axis=2):
    """The matrix cut into n equal parts along axis (2: columns, 1: rows) as a batch of n, read in place
    (ferrite/tensor.py:218-229: attention's heads; by rows, each matrix of a batch too, its parts one after another)."""
    assert axis in (1, 2)
    x = self.realize()
    if axis == 2:
      assert self.batch == 1 and self.cols % n == 0, "equal parts of one matrix"
      st = x.data.stride()
      return x._view((n, self.rows, self.cols // n), 0, (self.cols // n * st[2], st[1], st[2]))
    assert self.rows % n == 0, "equal parts"
    if not x.data.is_contiguous(): x = (x + 0).realize()
    return x._view((self.batch * n, self.rows // n, self.cols), 0, (self.rows // n * self.cols, self.cols, 1))

  def merge(self):
    """The batch side by side as one matrix, split's inverse (ferrite/tensor.py:231-236): x.split(n).merge() is x."""
    out = Tensor._empty(self.rt, 1, self.rows, self.batch * self.cols, self.dtype)
    view = out._view((self.batch, self.rows, self.cols), 0, (self.cols, self.batch * self.cols, 1))
    self.realize(into=view)
    return out

  def pad(self, widths):
    """Zeros around: (before, after) for each of the last len(widths) axes, as numpy's (ferrite/tensor.py:196-199)."""
    widths = ((0, 0),) * (3 - len(widths)) + tuple(widths)
    shape = tuple(n + w[0] + w[1] for n, w in zip(self.shape, widths))
    out = Tensor._empty(self.rt, *shape, self.dtype, zero=True)
    key = tuple(slice(w[0], w[0] + n) for w, n in zip(widths, self.shape))
    self.realize(into=out[key])
    return out

  def cat(self, *xs, axis=0):
    """Along axis, the other sizes the same (ferrite/tensor.py:201-208): each copied into its place in one tensor."""
    ts, axis = (self, *xs), axis % 3
    assert all(t.dtype == self.dtype and all(a == b for k, (a, b) in enumerate(zip(t.shape, self.shape)) if k != axis) for t in ts)
    shape = list(self.shape)
    shape[axis] = sum(t.shape[axis] for t in ts)
    out, at = Tensor._empty(self.rt, *shape, self.dtype), 0
    for t in ts:
      key = [slice(None)] * 3
      key[axis] = slice(at, at + t.shape[axis])
      t.realize(into=out[tuple(key)])
      at += t.shape[axis]
    return out

  def repeat_interleave(self, n):
    """Each matrix n times over, one after another along the batch (numpy's repeat; ferrite/tensor.py:210-216: grouped-
    query attention's keys and values, each head once for every query head it serves), as a copy."""
    out = Tensor._empty(self.rt, self.batch * n, self.rows, self.cols, self.dtype)
    for i in range(n): self.realize(into=out[i::n, :, :])
    return out

  def assign(self, x):
    """x's value in this tensor (a stored tensor or a view of one), in place (ferrite/tensor.py:273-283)."""
    if self.op is None: self.realize()  # (one made empty: its memory)
    assert self.data is not None and not isinstance(self.data, list) and self.dtype not in BFP, "a stored tensor or view"
    assert (x.shape, x.dtype) == (self.shape, self.dtype), f"{x.shape} {x.dtype} into {self.shape} {self.dtype}"
    x.realize(into=self)
    return self

  def gather(self, ids):
    """Rows ids of this matrix, as a tensor (ferrite/tensor.py:116-126: an embedding lookup): ids an int32 tensor of
    one row (read on the GPU, so it can be computed there) or a list. An index outside the rows reads the nearest. A
    block float's rows are gathered packed (its runs' magnitudes and exponents)."""
    if not isinstance(ids, Tensor):
      assert all(0 <= i < self.rows for i in ids)
      ids = Tensor.of(self.rt, [list(ids)], "int32")
    assert self.batch == 1 and ids.dtype == "int32" and ids.shape[:2] == (1, 1), "rows of a matrix, by a row of int32"
    idx, n = _ids(ids), ids.cols
    x = self.realize()
    if x.dtype in BFP:
      (w,) = _matrices(x)
      out = Tensor(self.rt, n, self.cols, dtype=self.dtype)
      with self.rt.on(): g = ops.bfp_empty(n, w.N, w.fmt, device=self.rt.device)
      rb, runs = (16 if w.fmt == "bfp8" else 8), w.N // 16
      self.rt.run(lambda: (lib.call("fh_gather_rows", ops._ptr(w.mant), w.K, rb, w.K * rb, ops._ptr(idx), n, rb, runs, ops._ptr(g.mant), rb, n * rb, ops._stream()),
                           lib.call("fh_gather_rows", ops._ptr(w.exps), w.K, 1, w.K, ops._ptr(idx), n, 1, runs, ops._ptr(g.exps), 1, n, ops._stream())), "gather")
      out.data = g
      return out
    if x.data.stride(2) != 1: x = (x + 0).realize()
    es, st = ITEMSIZE[self.dtype], x.data.stride()
    out = Tensor._empty(self.rt, 1, n, self.cols, self.dtype)
    self.rt.run(lambda: lib.call("fh_gather_rows", ops._ptr(x.data), self.rows, st[1] * es, 0, ops._ptr(idx), n, self.cols * es, 1,
                                 ops._ptr(out.data), self.cols * es, 0, ops._stream()), "gather")
    return out

  def put(self, ids, x):
    """x's rows into rows ids of each matrix of this tensor, in place, gather's inverse (ferrite/tensor.py:128-140: a KV
    cache takes a token's keys at its place): ids an int32 tensor of one row, read on the GPU. Into a block float, x is
    bf16, each of its runs of 16 rounded as cast rounds them (fh_bfp_pack), then its packed rows put in place. An index
    outside the rows writes nothing."""
    assert ids.dtype == "int32" and ids.shape[:2] == (1, 1) and ids.cols == x.rows, "rows of x, by a row of int32 places"
    assert (x.batch, x.cols) == (self.batch, self.cols) and x.dtype == ("bf16" if self.dtype in BFP else self.dtype), \
      f"{x.shape} {x.dtype} into {self.shape} {self.dtype}"
    self.realize()  # (one made empty: its memory)
    assert self.data is not None, "into a stored tensor"
    idx, n = _ids(ids), x.rows
    xr = x.realize()
    if not xr.data.is_contiguous(): xr = (xr + 0).realize()
    if self.dtype in BFP:
      for b, w in enumerate(_matrices(self)):
        rb, runs = (16 if w.fmt == "bfp8" else 8), w.N // 16
        p = self.rt.run(lambda b=b, w=w: ops.pack(xr.data[b], w.fmt), "pack")
        self.rt.run(lambda w=w, p=p: (lib.call("fh_put_rows", ops._ptr(w.mant), w.K, rb, w.K * rb, ops._ptr(idx), n, rb, runs, ops._ptr(p.mant), rb, n * rb, ops._stream()),
                                      lib.call("fh_put_rows", ops._ptr(w.exps), w.K, 1, w.K, ops._ptr(idx), n, 1, runs, ops._ptr(p.exps), 1, n, ops._stream())), "put")
      return self
    assert self.data.stride(2) == 1, "into rows of contiguous elements"
    es, st = ITEMSIZE[self.dtype], self.data.stride()
    self.rt.run(lambda: lib.call("fh_put_rows", ops._ptr(self.data), self.rows, st[1] * es, st[0] * es, ops._ptr(idx), n, self.cols * es,
                                 self.batch, ops._ptr(xr.data), self.cols * es, n * self.cols * es, ops._stream()), "put")
    return self

  def attend(self, k, v, places, window=0, fidelity=None, parts=None):
    """softmax(self @ k^T + mask) @ v (ferrite/tensor.py:487-516): self a batch of query rows (bf16 or fp32; scaled by
    the caller), k and v the keys and values for each matrix (bf16, fp32 or a block float: a KV cache's, whose values
    are bf16 values, read as those), places an int32 column (batch 1 or self's): row t sees keys up to places[t], and
    with a window, none window or more before it. Scores and sums in fp32; the result bf16 (fh_attend). fidelity and
    parts (ferrite's product phases and its workers' share of the keys) are taken and ignored: one kernel reads every
    key a row sees."""
    assert self.dtype in ("bf16", "fp32") and k.dtype == v.dtype and k.dtype != "int32" and self.batch == k.batch == v.batch
    assert self.cols == k.cols == v.cols and k.rows == v.rows and self.cols <= 256, f"{self.shape} by {k.shape}, {v.shape}"
    assert places.rows == self.rows and places.cols == 1 and places.batch in (1, self.batch) and places.dtype == "int32", \
      f"{self.shape} by {k.shape}, {places.shape}"
    def plain(t):  # a block float as its bf16 values (exact); rows of contiguous elements
      x = t.realize()
      if x.dtype in BFP:
        out = Tensor._empty(self.rt, x.batch, x.rows, x.cols, "bf16")
        for b, w in enumerate(_matrices(x)): self.rt.run(lambda b=b, w=w: ops.dequant(w, out.data[b]), "dequant")
        return out
      return x if x.data.stride(2) == 1 else (x + 0).realize()
    q, k, v = plain(self), plain(k), plain(v)
    if k.dtype != v.dtype: k, v = k.float().realize(), v.float().realize()
    pl = places.realize()
    if not pl.data.is_contiguous(): pl = (pl + 0).realize()
    out = Tensor._empty(self.rt, self.batch, self.rows, self.cols, "bf16")
    qs, ks, vs, os_ = (t.data.stride() for t in (q, k, v, out))
    self.rt.run(lambda: lib.call("fh_attend", ops._ptr(q.data), DT[q.dtype], qs[0], qs[1], ops._ptr(k.data), ops._ptr(v.data), DT[k.dtype],
                                 ks[0], ks[1], vs[0], vs[1], k.rows, self.batch, self.rows, self.cols, ops._ptr(pl.data),
                                 self.rows if pl.batch > 1 else 0, int(window), ops._ptr(out.data), lib.BF16, os_[0], os_[1],
                                 ops._stream()), "attention")
    return out

  def touched(self, n, weights):
    """A mixture of experts' choices (int32, rows x k, values below n) as the experts some row picks by a weight not 0,
    each once, and each such entry's weight from each row (ferrite/tensor.py:403-416): experts, a column of
    min(rows k, n), those picked in increasing order then n (none); weights (that many, rows, 1) bf16, 0 for a row that
    did not pick the entry's expert. A decode step's few tokens then go through each picked expert once (matmul by
    index=experts). By fh_moe_touched."""
    assert self.dtype == "int32" and weights.dtype == "bf16" and self.shape == weights.shape and self.batch == 1
    rows, k = self.rows, self.cols
    slots = min(rows * k, n)
    x, w = (t.realize() if t.realize().data.stride(2) == 1 else (t + 0).realize() for t in (self, weights))
    experts = Tensor._empty(self.rt, 1, slots, 1, "int32")
    out = Tensor._empty(self.rt, slots, rows, 1, "bf16")
    self.rt.run(lambda: lib.call("fh_moe_touched", ops._ptr(x.data), x.data.stride(1), ops._ptr(w.data), w.data.stride(1), rows, k, n,
                                 ops._ptr(experts.data), ops._ptr(out.data), ops._stream()), "touched")
    return experts, out

  def group(self, n):
    """A mixture of experts' tokens grouped by expert (ferrite/tensor.py:389-402), from int32 choices (rows x k, values
    below n): order, a row of 32 t slots in which each value's choices have a run of whole tiles of 32 (each slot the
    row it holds, 0 for none); tiles, a column of t, each tile's value (n past those used); places, a row of k runs of
    the rows rounded up to 32, run j holding the slot of each row's choice j. Each expert's tokens are then a batch entry
    of whole tiles for a matmul that picks its weights (index=tiles). By fh_moe_group."""
    assert self.dtype == "int32" and self.batch == 1, "a matrix of int32 choices"
    rows, k = self.rows, self.cols
    t, rp = -(-rows * k // 32) + min(n, rows * k), -(-rows // 32) * 32
    x = self.realize()
    if x.data.stride(2) != 1: x = (x + 0).realize()
    order, tiles, places = (Tensor._empty(self.rt, 1, r, c, "int32") for r, c in ((1, 32 * t), (t, 1), (1, k * rp)))
    with self.rt.on(): fill = torch.empty(n, dtype=torch.int32, device=self.rt.device)
    self.rt.run(lambda: lib.call("fh_moe_group", ops._ptr(x.data), x.data.stride(1), rows, k, n, ops._ptr(order.data), ops._ptr(tiles.data),
                                 ops._ptr(places.data), ops._ptr(fill), ops._stream()), "group")
    return order, tiles, places

  @classmethod
  def _empty(cls, rt, batch, rows, cols, dtype, zero=False):
    """A stored tensor of its own memory (zeros by our fill kernel if asked)."""
    with rt.on(): t = torch.empty(batch, rows, cols, dtype=TORCH[dtype], device=rt.device)
    out = cls._stored(rt, t, dtype)
    if zero:
      p = _cprogram([("copy", lib.OPND_IMM, lib.OPND_IMM, 0.0)], [])
      rt.run(lambda: lib.call("fh_map", ctypes.byref(p), ops._ptr(t), DT[dtype], batch, rows, cols, rows * cols, cols, ops._stream()), "map")
    return out

  def expand(self, *shape):  # dimensions of 1 repeated (a stride of 0), missing ones in front being 1
    shape = (1,) * (3 - len(shape)) + shape
    assert all(n in (m, 1) for n, m in zip(self.shape, shape)), f"cannot expand {self.shape} to {shape}"
    x = self.realize()
    return x._view(shape, 0, tuple(0 if n == 1 and m > 1 else s for n, m, s in zip(self.shape, shape, x.data.stride())))

  def reshape(self, *shape):  # up to three sizes, missing ones in front being 1
    shape = (1,) * (3 - len(shape)) + shape
    assert math.prod(shape) == math.prod(self.shape), f"cannot reshape {self.shape} to {shape}"
    x = self.realize()
    if not x.data.is_contiguous(): x = (x + 0).realize()  # a copy first
    return x._view(shape, 0, (shape[1] * shape[2], shape[2], 1))

  # ---- elementwise (ferrite/tensor.py:300-360) --------------------------------------------------------------------
  def _unary(self, op):
    if self.dtype == "int32" and op != "relu": return self.float()._unary(op)
    return Tensor(self.rt, self.rows, self.cols, op, (self,), self.batch, self.dtype)

  def _binop(self, op, x, reverse=False):
    """numpy's broadcasting; a number is the op's immediate; different dtypes meet in fp32, and so does int32 for what
    it does not do itself."""
    if not isinstance(x, Tensor):
      num = float(x)
      dtype = "fp32" if self.dtype == "int32" and isinstance(x, float) else self.dtype
      a = self if dtype == self.dtype else self.float()
      return Tensor(self.rt, self.rows, self.cols, op, (a,), self.batch, dtype, args=(num, reverse))
    a, b = (x, self) if reverse else (self, x)
    if a.dtype != b.dtype or (a.dtype == "int32" and op not in INT32_OPS): a, b = a.float(), b.float()
    assert all(n == m or 1 in (n, m) for n, m in zip(a.shape, b.shape)), f"cannot broadcast {a.shape} with {b.shape}"
    batch, rows, cols = map(max, a.shape, b.shape)
    return Tensor(self.rt, rows, cols, op, (a, b), batch, a.dtype)

  def cast(self, dtype):
    """To another dtype; to a block float, packed at once (fh_bfp_pack, Tensor.cast's bfp4_kernel / packer)."""
    if dtype == self.dtype: return self
    if dtype in BFP:  # (a batch: each matrix packed, a mixture's experts for matmul(index=))
      x = self.realize()
      if x.dtype == "int32" or not x.data.is_contiguous(): x = (x.float() if x.dtype == "int32" else x + 0).realize()
      out = Tensor(self.rt, self.rows, self.cols, batch=x.batch, dtype=dtype)
      packed = [x.rt.run(lambda b=b: ops.pack(x.data[b], dtype), "pack") for b in range(x.batch)]
      out.data = packed[0] if x.batch == 1 else packed
      return out
    if self.dtype in BFP:  # a block float's values (each a bf16 value)
      b = Tensor(self.rt, self.rows, self.cols, batch=self.batch, dtype="bf16")
      b.data = self.rt.run(lambda: torch.stack([ops.dequant(w) for w in _matrices(self)]), "dequant")
      return b.cast(dtype)
    return Tensor(self.rt, self.rows, self.cols, "cast", (self,), self.batch, dtype)

  def float(self): return self.cast("fp32")
  def bfloat16(self): return self.cast("bf16")
  def exp2(self): return self._unary("exp2")
  def log2(self): return self._unary("log2")
  def sin(self): return self._unary("sin")
  def sqrt(self): return self._unary("sqrt")
  def reciprocal(self): return self._unary("recip")
  def exp(self): return self._unary("exp")
  def log(self): return self._unary("log")
  def cos(self): return self._unary("cos")
  def relu(self): return self._unary("relu")
  def rsqrt(self): return self.sqrt().reciprocal()
  def maximum(self, x): return self._binop("max", x)
  def minimum(self, x): return -((-self).maximum(-x))
  def where(self, x, y):  # x where self is not 0, else y
    dtype = next((t.dtype for t in (x, y) if isinstance(t, Tensor)), self.dtype)
    c = self if self.dtype == dtype else self.ne(0).cast(dtype)
    return c._binop("keep", x) + c._binop("drop", y)
  def __add__(self, x): return self._binop("add", x)
  def __sub__(self, x): return self._binop("sub", x)
  def __mul__(self, x): return self._binop("mul", x)
  def __rsub__(self, x): return self._binop("sub", x, True)
  __radd__, __rmul__ = __add__, __mul__
  def __truediv__(self, x): return self * (1 / x if isinstance(x, (int, float)) else x.reciprocal())
  def __neg__(self): return 0 - self if self.dtype == "int32" else self * -1
  def __lt__(self, x): return self._binop("cmplt", x)
  def __gt__(self, x): return self._binop("cmplt", x, True)
  def __ge__(self, x): return 1 - (self < x)
  def __le__(self, x): return 1 - (self > x)
  def ne(self, x): return self._binop("cmpne", x)
  def eq(self, x): return 1 - self.ne(x)
  __ne__, __eq__ = ne, eq
  def __hash__(self): return id(self)
  def sigmoid(self): return (1 + (-self).exp()).reciprocal()
  def silu(self): return self * self.sigmoid()
  def gelu(self):
    k = 2 * math.sqrt(2 / math.pi)
    return self * (1 + (self * (self * self * (-0.044715 * k) - k)).exp()).reciprocal()

  # ---- reductions (ferrite/tensor.py:362-372, 430-440) -------------------------------------------------------------
  def sum(self, axis=None): return self._reduce("sum", axis)
  def max(self, axis=None): return self._reduce("max", axis)

  def _reduce(self, f, axis):
    if self.dtype == "int32": return self.float()._reduce(f, axis).cast("int32")
    if axis is None: return self._reduce(f, 0)._reduce(f, 1)._reduce(f, 2)
    shape = [1 if ax == axis % 3 else s for ax, s in enumerate(self.shape)]
    if shape == list(self.shape): return self
    return Tensor(self.rt, shape[1], shape[2], f"{f}{axis % 3}", (self,), shape[0], self.dtype)

  def mean(self, axis=None):
    s = self.sum(axis)
    return s * (math.prod(s.shape) / math.prod(self.shape))

  def softmax(self, axis=-1):  # the max first, so exp stays in range
    if axis % 3 == 2 and self.dtype != "int32": return self._rowwise("softmax")
    e = (self - self.max(axis)).exp()
    return e / e.sum(axis)

  def log_softmax(self, axis=-1):
    if axis % 3 == 2 and self.dtype != "int32": return self._rowwise("log_softmax")
    m = self - self.max(axis)
    return m - m.exp().sum(axis).log()

  def _rowwise(self, op):
    """softmax / log_softmax along each row as one node: the same arithmetic as the composed form above (the row's
    max, exp(x - max), its sum, the quotient or the difference of logs), one launch (fh_softmax_rows) that evaluates
    the elementwise tree under it three times instead of two reductions and a map over realized rows."""
    return Tensor(self.rt, self.rows, self.cols, op, (self,), self.batch, self.dtype)

  def layernorm(self, axis=-1, eps=1e-5):
    c = self - self.mean(axis)
    return c * ((c * c).mean(axis) + eps).rsqrt()

  def topk(self, k, parts=1, labels=None):
    """Each row's k (<= 64) largest values, largest first, and their columns (int32), the first column of equal values
    first (Tensor.topk, ferrite/tensor.py:373-388: numpy's stable order), by fh_logit_heads. parts: each row cut into
    so many parts of equal width, each part's k best side by side, (rows, parts k), each index its column in the whole
    row. labels: an int32 tensor of this one's shape (parts 1), each pick's label (labels at its column) instead of its
    column: a second topk over the parts' best given their indices picks the whole row's best with its columns. One call
    here takes a row of any width; parts and labels keep ferrite's two-call form working."""
    assert self.dtype in ("bf16", "fp32"), "bf16 or fp32"
    cols = self.cols // parts
    assert 1 <= k <= min(cols, 64) and parts * cols == self.cols, "k of at most 64 and the row's width, whole parts"
    assert labels is None or (labels.dtype == "int32" and labels.shape == self.shape and parts == 1), "labels: int32, x's shape"
    n = self.batch * self.rows
    R, ld = n * parts, (cols + 3) // 4 * 4  # each part a row of its own, rows 16-byte aligned for the kernel's loads
    with self.rt.on(): x = torch.empty(R, ld, dtype=torch.float32, device=self.rt.device)
    prog, inputs = _fit_program(self.float() if self.dtype != "fp32" else self, self.shape, allow_acc=False)
    p = _cprogram(prog, inputs)
    if ld == cols:  # the parts of a row are consecutive rows of width cols: the row as it is
      self.rt.run(lambda: lib.call("fh_map", ctypes.byref(p), ops._ptr(x), lib.F32, *self.shape, self.rows * self.cols,
                                   self.cols, ops._stream()), "map")
    else:  # the rows first, then each part into a row of its own, padded
      with self.rt.on(): x0 = torch.empty(n, self.cols, dtype=torch.float32, device=self.rt.device)
      self.rt.run(lambda: lib.call("fh_map", ctypes.byref(p), ops._ptr(x0), lib.F32, *self.shape, self.rows * self.cols,
                                   self.cols, ops._stream()), "map")
      q = lib.Program()
      q.n_ops, q.n_inputs = 1, 1
      q.op[0], q.a[0], q.b[0] = lib.OP["copy"], 16, lib.OPND_IMM
      q.input[0], q.in_dtype[0] = x0.data_ptr(), lib.F32
      q.in_stride[0][0], q.in_stride[0][1], q.in_stride[0][2] = 0, cols, 1
      self.rt.run(lambda: lib.call("fh_map", ctypes.byref(q), ops._ptr(x), lib.F32, 1, R, cols, R * ld, ld, ops._stream()), "map")
    values, ids = self.rt.run(lambda: ops.logit_heads(x[:, :cols], k), "topk")
    i = Tensor(self.rt, R, k, dtype="int32")
    i.data = ids.reshape(1, R, k)
    if parts > 1:  # each part's columns from its first in the whole row
      first = Tensor.of(self.rt, [[(r % parts) * cols] for r in range(R)], "int32")
      i = (i + first).realize()
    if labels is not None:
      lab = labels.realize()
      if not lab.data.is_contiguous(): lab = (lab + 0).realize()
      with self.rt.on(): got = torch.empty(n, k, dtype=torch.int32, device=self.rt.device)
      self.rt.run(lambda: lib.call("fh_gather_cols", ops._ptr(lab.data), self.cols, self.cols, ops._ptr(i.data), k, n, k,
                                   ops._ptr(got), k, ops._stream()), "labels")
      i = Tensor(self.rt, R, k, dtype="int32")
      i.data = got.reshape(1, R, k)
    v = Tensor(self.rt, self.rows, parts * k, batch=self.batch, dtype="fp32")
    v.data = values.reshape(self.batch, self.rows, parts * k)
    ids_out = Tensor(self.rt, self.rows, parts * k, batch=self.batch, dtype="int32")
    ids_out.data = i.data.reshape(self.batch, self.rows, parts * k)
    return (v if self.dtype == "fp32" else v.cast(self.dtype)), ids_out

  # ---- matmul (ferrite/tensor.py:443-485) ----------------------------------------------------------------------------
  def __matmul__(self, x): return self.matmul(x)

  def matmul(self, x, dtype=None, fidelity=None, index=None):
    """self (1 x rows x K) @ x (K x N, a block float: bfp8 or bfp4, cast once), written as dtype: bf16, or fp32 if
    self is, unless said. A plain x (bf16 or fp32, a batch of matrices or one; self's batch the same or 1): fh_matmul,
    bf16 products summed in fp32, an fp32 operand as ferrite's bf16x3 (hi@hi + hi@lo + lo@hi), written as dtype: fp32
    if either operand is, else bf16, unless said. fp32 rows, a few, by a block float go through the exact-product
    GEMV; otherwise the matrix cores take self's
    values in bf16, as ferrite's chip does (bf16 rows: exact products too); the elementwise ops on top of it run in
    the same kernel. fidelity: the chip's product phases (ferrite/tensor.py:443-452); taken and ignored, the products
    here being exact or bf16 x bf16 whatever it says. index: an int32 (rows, k) tensor choosing, for each batch entry b
    of the result, which of x's matrices (x a batch of block floats: a mixture's experts) multiplies self's entry b (or
    its only one), index's (b // k, b % k); an entry choosing none (x.batch or more) is zeros. It is resolved on the GPU
    (each matrix's product, then each entry's pick), so a recording replays it; ops.moe_experts is the path that reads
    only the chosen experts."""
    if x.dtype not in BFP:  # plain operands (fh_matmul): bf16 products summed in fp32, an fp32 operand as bf16x3
      assert index is None, "index= picks among a batch of block floats"
      assert "int32" not in (self.dtype, x.dtype), "the matrix cores multiply floats"
      assert self.cols == x.rows and (self.batch == x.batch or 1 in (self.batch, x.batch)), f"{self.shape} @ {x.shape}"
      dtype = dtype or ("fp32" if "fp32" in (self.dtype, x.dtype) else "bf16")
      return Tensor(self.rt, self.rows, x.cols, "matmul", (self, x), max(self.batch, x.batch), dtype)
    if index is not None:
      assert index.dtype == "int32" and self.cols == x.rows and self.batch in (1, index.rows * index.cols) and index.batch == 1, \
        f"{self.shape} @ {x.shape} picked by {index.shape} {index.dtype}"
      return Tensor(self.rt, self.rows, x.cols, "picked", (self, x.realize(), index), index.rows * index.cols,
                    dtype or ("fp32" if self.dtype == "fp32" else "bf16"))
    assert x.batch == 1, "a batch of block floats is read through index="
    assert self.batch == 1 and self.cols == x.rows and self.dtype != "int32", f"{self.shape} @ {x.shape}"
    return Tensor(self.rt, self.rows, x.cols, "matmul", (self, x.realize()), 1, dtype or ("fp32" if self.dtype == "fp32" else "bf16"))

  # ---- realizing ----------------------------------------------------------------------------------------------------
  def realize(self, into=None):
    """Compute it now (if it is an op), into memory of its own, or into `into`'s (a stored tensor of the same shape and
    dtype, rows contiguous: jit's copies of its inputs); returns it, realized."""
    if into is not None:
      assert into.data is not None and into.shape == self.shape and into.dtype == self.dtype and into.dtype not in BFP
      assert into.data.stride(2) == 1 or into.cols == 1, "realize(into=): rows contiguous"
      if self is into: return into
      prog, inputs = _fit_program(self, self.shape, allow_acc=False)  # (a stored tensor: one copy op)
      p = _cprogram(prog, inputs)
      out, ld = into.data, into.data.stride()
      self.rt.run(lambda: lib.call("fh_map", ctypes.byref(p), ops._ptr(out), DT[into.dtype], *into.shape, ld[0], ld[1], ops._stream()), "map",
                  _read_bytes(inputs, into.shape))
      return into
    if self.data is not None: return self
    if self.op is None:  # made empty (ferrite's Tensor(rt, rows, cols, batch, dtype), the model's `empty`): its memory now
      assert self.dtype not in BFP, "a block float is made by cast"
      with self.rt.on(): self.data = torch.empty(self.shape, dtype=TORCH[self.dtype], device=self.rt.device)
      return self
    if self.op == "picked":
      self._done(_picked(self).data)
      return self
    if self.op in ROWWISE:
      src = self.srcs[0]
      prog, inputs = _fit_program(src, src.shape, allow_acc=False)
      with self.rt.on(): out = torch.empty(self.shape, dtype=TORCH[self.dtype], device=self.rt.device)
      p = _cprogram(prog, inputs)
      self.rt.run(lambda: lib.call("fh_softmax_rows", ctypes.byref(p), int(self.op == "log_softmax"), *src.shape, ops._ptr(out),
                                   DT[self.dtype], ops._stream()), "softmax", _read_bytes(inputs, src.shape))
      self._done(out)
      return self
    if self.op in REDUCE:
      f, axis = REDUCE[self.op]
      src = self.srcs[0]
      prog, inputs = _fit_program(src, src.shape, allow_acc=False)
      with self.rt.on(): out = torch.empty(self.shape, dtype=TORCH[self.dtype], device=self.rt.device)
      p = _cprogram(prog, inputs)
      self.rt.run(lambda: lib.call("fh_reduce", ctypes.byref(p), lib.REDUCE_MAX if f == "max" else lib.REDUCE_SUM, axis,
                                   *src.shape, ops._ptr(out), DT[self.dtype], ops._stream()), "reduce", _read_bytes(inputs, src.shape))
      self._done(out)
      return self
    prog, inputs = _fit_program(self, self.shape, allow_acc=True)
    mm = next((t for t in _walk(self) if getattr(t, "_acc", False)), None)
    with self.rt.on(): out = torch.empty(self.shape, dtype=TORCH[self.dtype], device=self.rt.device)
    p = _cprogram(prog, inputs)
    if mm is not None and mm.srcs[1].dtype not in BFP:  # plain operands: every batch entry, rows contiguous
      mm._acc = False
      a, b = (u.realize() for u in mm.srcs)
      a, b = ((u if u.data.stride(2) == 1 else (u + 0).realize()) for u in (a, b))
      self.rt.run(lambda: ops.matmul(a.data, b.data, p, out=out), "matmul",
                  _tensor_bytes(a) + _tensor_bytes(b) + _read_bytes([i for i in inputs if i[0] is not mm], self.shape))
    elif mm is not None:
      mm._acc = False
      a, w = mm.srcs[0].realize(), mm.srcs[1].data
      if a.data.stride(2) != 1: a = (a + 0).realize()  # rows contiguous (our copy kernel)
      x = a.data[0]
      y = out[0]
      program = [p]
      ep = ops.epilogue(lib.EP_PROGRAM)
      ep.program = ctypes.pointer(p)
      ep.keep.append(program)
      nb = w.nbytes + _read_bytes([i for i in inputs if i[0] is not mm], self.shape)
      if w.K % 32 or (a.dtype == "fp32" and a.rows <= 8):  # fp32 rows, or a K the matrix cores do not take: the
        if x.dtype != torch.float32: x = a.float().realize().data[0]  # exact-product GEMV
        self.rt.run(lambda: ops.gemv(x, w, ep, out=y), "matmul", nb + x.numel() * x.element_size())
      else:  # the matrix cores (bf16 rows go in as they are: their products are exact too)
        self.rt.run(lambda: ops.gemm(x, w, ep, out=y), "matmul", nb + x.numel() * x.element_size())
    else:
      ld = out.stride()
      self.rt.run(lambda: lib.call("fh_map", ctypes.byref(p), ops._ptr(out), DT[self.dtype], *self.shape, ld[0], ld[1], ops._stream()), "map",
                  _read_bytes(inputs, self.shape))
    self._done(out)
    return self

  def _done(self, data):
    self.data, self.op, self.srcs, self.args = data, None, (), ()


def _ids(ids):
  """An int32 row tensor's values on the GPU, contiguous."""
  d = ids.realize().data
  return d if d.is_contiguous() else (ids + 0).realize().data


def _matrices(t):
  """A block-float tensor's matrices (BfpWeights)."""
  return t.data if isinstance(t.data, list) else [t.data]


def _picked(t):
  """matmul(index=): each of x's matrices times self's rows (all entries' rows at once), then each entry keeps the
  product of the matrix its index names (keep/drop: selected, never multiplied by 0)."""
  a, w, index = t.srcs
  mats = _matrices(w)
  n = t.batch
  rows = a.realize()
  flat = rows.reshape(1, rows.batch * rows.rows, rows.cols)  # every entry's rows, one matrix
  choice = index.realize().reshape(n, 1, 1)
  acc = None
  for e, m in enumerate(mats):
    we = Tensor(t.rt, w.rows, w.cols, batch=1, dtype=w.dtype)
    we.data = m
    y = flat.matmul(we, t.dtype).realize().reshape(rows.batch, rows.rows, w.cols)
    pick = choice.eq(e)
    acc = (pick.where(y, 0.0) if acc is None else pick.where(y, acc)).realize()
  return acc


class Recording:
  """A function's launches captured once as a HIP graph on its runtime's stream (ferrite's Recording, tensor.py:775-785:
  launches recorded once and sent again as one block); send() replays them."""

  def __init__(self, rt): self.rt, self.graph = rt, torch.cuda.CUDAGraph()

  def __enter__(self):
    self._ctx = torch.cuda.graph(self.graph, stream=self.rt.stream)
    self._ctx.__enter__()
    return self

  def __exit__(self, *exc): return self._ctx.__exit__(*exc)

  def send(self):
    with torch.cuda.stream(self.rt.stream):
      self.graph.replay()


def jit(f):
  """f, a function of tensors that returns one, run from a recording (ferrite's jit, tensor.py:788-810): its first call
  runs as any would (so every kernel and table is set up), its second is captured as a HIP graph (each launch, and the
  memory it writes, kept from then on) and replayed, and each later call copies its inputs into the second call's
  (a launch each) and replays the graph: one host call for the whole step. Its inputs keep their shapes and dtypes;
  nothing else it reads may change, and it may not read back. Its result is the same tensor every call, written again by
  the next."""
  calls, inputs, out, rec = 0, (), None, None

  def run(*xs):
    nonlocal calls, inputs, out, rec
    calls, rt = calls + 1, xs[0].rt
    if calls == 1: return f(*xs).realize()
    if calls == 2:
      inputs = [x.realize() if x.data is not None and x.data.is_contiguous() else (x + 0).realize() for x in xs]
      rt.wait()
      with Recording(rt) as rec:
        out = f(*inputs).realize()
      rec.send()
      return out
    for x, to in zip(xs, inputs):
      assert (x.shape, x.dtype) == (to.shape, to.dtype), f"{x.shape} {x.dtype} where the recording had {to.shape} {to.dtype}"
      if x is not to: x.realize(into=to)
    rec.send()
    return out
  return run


def _walk(t, seen=None):
  """The unrealized nodes under t (t first), each once."""
  seen = set() if seen is None else seen
  if t.data is not None or id(t) in seen: return
  seen.add(id(t))
  yield t
  for s in t.srcs: yield from _walk(s, seen)


def _ops(t, acc_ok):
  """How many program ops t's tree would take, counting each shared node once and stopping at what realizes apart."""
  n = 0
  for u in _walk(t):
    if u.op in REDUCE or u.op in ROWWISE or u.op == "picked" or (u.op == "matmul" and not acc_ok): continue
    if u.op == "matmul": n += 1; continue
    n += 1
  return n


def _fit_program(root, shape, allow_acc):
  """The program computing root's elementwise tree at each element of shape, its inputs; realizing first what does
  not fit: reductions, matmuls other than one (the epilogue's acc), and, while the tree holds more than MAX_OPS ops,
  the biggest subtree two ops read, else the heaviest operand (ferrite/tensor.py:651-669's _fit)."""
  while True:
    readers = {}
    for u in _walk(root):
      for s in u.srcs: readers[id(s)] = readers.get(id(s), 0) + 1
    for u in list(_walk(root)):  # reductions (a reduction's own operand too), picked matmuls, and every matmul but
      if u.op in REDUCE or u.op in ROWWISE or u.op == "picked": u.realize()  # the root's chain's first are realized apart
    accs = [u for u in _walk(root) if u.op == "matmul"]
    for i, u in enumerate(accs):
      if not allow_acc or i > 0 or readers.get(id(u), 0) > 1 or u.shape != tuple(shape): u.realize()
    n = _ops(root, allow_acc)
    if n <= MAX_OPS: break
    lazy = [u for u in _walk(root)][1:]
    shared = [u for u in lazy if readers.get(id(u), 0) > 1 and _ops(u, False) <= MAX_OPS]
    u = max(shared, key=lambda v: _ops(v, False)) if shared else root
    while _ops(u, False) > MAX_OPS: u = max((s for s in u.srcs if s.data is None), key=lambda v: _ops(v, False))
    u.realize()
  prog, inputs, regs = [], [], {"root": root}
  _emit(root, shape, prog, inputs, regs)
  if not prog: prog.append(("copy", _operand(root, shape, prog, inputs, regs), lib.OPND_IMM, 0.0))
  return prog, inputs


def _operand(t, shape, prog, inputs, regs):
  """t's operand code: an earlier op's register, an input (a stored tensor, broadcast by strides), or acc."""
  if t.data is not None:
    for k, (u, _) in enumerate(inputs):
      if u is t: return 16 + k
    assert len(inputs) < lib.MAX_INPUTS, "a program reads at most 8 inputs"
    st = [0 if n == 1 and m > 1 else s for n, m, s in zip(t.shape, shape, t.data.stride())]
    inputs.append((t, st))
    return 16 + len(inputs) - 1
  return _emit(t, shape, prog, inputs, regs)


def _emit(t, shape, prog, inputs, regs):
  """Emits t's ops (operands first) into prog; returns the code of t's value."""
  if id(t) in regs: return regs[id(t)]
  if t.op == "matmul":
    t._acc = True
    regs[id(t)] = lib.OPND_ACC
    return lib.OPND_ACC
  if t.data is None and t.op is None: t.realize()  # (made empty: its memory)
  if t.data is not None or t.op is None: return _operand(t, shape, prog, inputs, regs)
  op = t.op
  if op == "cast" and t is not regs["root"] and t.dtype != "fp32":  # a rounding below the root: realized first, as
    t.realize()                                                     # ferrite's casts below the root are
    return _operand(t, shape, prog, inputs, regs)
  if op == "cast":  # rounding happens at the result's store; a cast to int32 truncates toward 0 there
    a = _operand(t.srcs[0], shape, prog, inputs, regs)
    prog.append(("ftoi" if t.dtype == "int32" and t.srcs[0].dtype != "int32" else "copy", a, lib.OPND_IMM, 0.0))
  elif op in UNARY:
    a = _operand(t.srcs[0], shape, prog, inputs, regs)
    prog.append((op, a, lib.OPND_IMM, 0.0))
  elif op in BINARY and len(t.srcs) == 1:  # with a number
    num, reverse = t.args
    a = _operand(t.srcs[0], shape, prog, inputs, regs)
    prog.append((op, lib.OPND_IMM, a, num) if reverse else (op, a, lib.OPND_IMM, num))
  elif op in BINARY:
    a = _operand(t.srcs[0], shape, prog, inputs, regs)
    b = _operand(t.srcs[1], shape, prog, inputs, regs)
    prog.append((op, a, b, 0.0))
  else:
    raise NotImplementedError(f"op {op}")
  regs[id(t)] = len(prog) - 1
  return regs[id(t)]


def _cprogram(prog, inputs):
  """The fh_program of an emitted program."""
  assert 1 <= len(prog) <= MAX_OPS, f"{len(prog)} ops"
  p = lib.Program()
  p.n_ops, p.n_inputs = len(prog), len(inputs)
  for i, (op, a, b, imm) in enumerate(prog):
    p.op[i], p.a[i], p.b[i], p.imm[i] = lib.OP[op], a, b, imm
  for k, (t, st) in enumerate(inputs):
    p.input[k] = t.data.data_ptr()
    p.in_dtype[k] = DT[t.dtype]
    for j in range(3): p.in_stride[k][j] = st[j]
  p.keep = [t.data for t, _ in inputs]
  return p


def _read_bytes(inputs, shape):
  """The bytes a program over `shape` reads from its inputs, each element once: an input's elements along the axes it
  does not broadcast (a stride of 0 reads one element for all of that axis)."""
  n = 0
  for t, st in inputs:
    n += math.prod(d for d, s in zip(shape, st) if s != 0) * ITEMSIZE[t.dtype]
  return n


def _tensor_bytes(t):
  """A realized tensor's bytes (a block float's packed bytes)."""
  if isinstance(t.data, ops.BfpWeight): return t.data.nbytes
  return sum(w.nbytes for w in t.data) if isinstance(t.data, (list, tuple)) else t.data.numel() * t.data.element_size()
