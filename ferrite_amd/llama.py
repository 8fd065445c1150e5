"""A Llama decoder on MI355X: models/llama.py's layer structure (layer -> attention / mlp -> mm, models/llama.py:95-146,
266-269, 459-480) run as the library's fused kernels, a step replayable as one HIP graph (tensor.jit's place,
ferrite/tensor.py:775-810).

A decode step of `batch` rows (one token of each of `batch` sequences, or a prompt's tokens at consecutive places)
is, per block:
  qkv     fh_gemv_bfp  RMSNorm prologue, RoPE on q's and k's heads, k and v put into the cache at each row's place
  attend  fh_attention_decode over the rows each place reaches
  o       fh_gemv_bfp  + the residual (x += o), with x's sums of squares for the next norm
  gate_up fh_gemv_bfp  RMSNorm prologue, silu(gate) * up
  down    fh_gemv_bfp  + the residual
then the final norm and the output layer (fp32 logits) and each row's argmax. Activations stay fp32 between
kernels; weights are block floats (precision's formats); the KV cache is bf16 or fp32.

A prompt (prefill: T tokens at consecutive places of one sequence, models/llama.py:498-504) runs on the matrix cores,
the residual stream fp32 and each GEMM's input bf16 (as ferrite's chip feeds its matrix unit), per block:
  norm    fh_rms_rows  x -> bf16 rows
  qkv     fh_gemm_bfp  RoPE on q's and k's heads, k and v put into the cache at each row's place
  attend  fh_attention_prefill, causal over the sequence's rows (bf16 out)
  o       fh_gemm_bfp  + the residual
  norm    fh_rms_rows
  gate_up fh_gemm_bfp  silu(gate) * up (bf16 out)
  down    fh_gemm_bfp  + the residual, with x's sums of squares
then the final norm and the output layer for the last row only (fh_gemv_bfp), and its argmax.
"""
import math
from types import SimpleNamespace
import numpy as np
import torch
from ferrite_amd import lib, ops


def model(**c):
  """A config: dim, heads, kv, layers, eps, theta, vocab, ffn, places (RoPE rows), head_dim, rope (Llama 3's scaling),
  tied (output layer = embedding), centered (RMSNorm by 1 + w), as models/llama.py:541-543 keeps them."""
  d = dict(head_dim=None, rope=None, centered=False, tied=False, places=4096, k=0, experts=0, norm_topk=True)
  return SimpleNamespace(**(d | c))


def head(c): return c.head_dim or c.dim // c.heads


def precision(c, mode="bfp8"):
  """Each matrix's format (models/llama.py:54-76): bfp8 (all), bfp4 (the MLP's gate and up in bfp4), experts (every MLP
  matrix in bfp4), the rest bfp8. (Fidelity phases are the chip's: products here are exact.)"""
  four = {"bfp4": ("gate_up",), "tt": ("gate_up",), "experts": ("gate_up", "down")}.get(mode, ())
  if mode not in ("bfp8", "bfp4", "tt", "experts"): raise ValueError(f"precision: {mode} (the GPU path reads block floats)")
  p = {(op, l): ("bfp4" if op in four else "bfp8") for l in range(c.layers) for op in ("qkv", "o", "gate_up", "down")}
  if mode == "tt" and (c.layers, c.dim) == (32, 4096): p["gate_up", 31] = "bfp8"
  p["head", None] = "bfp8"
  return p


def frequencies(c):
  """RoPE's inverse frequencies in fp32, Llama 3's scaling if c.rope says llama3 (models/llama.py:333-344)."""
  hd = head(c)
  inv = 1 / c.theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd)
  r = c.rope
  if r and r.get("rope_type") == "llama3":
    old, wavelen = r["original_max_position_embeddings"], 2 * math.pi / inv
    scaled = np.where(wavelen > old / r["low_freq_factor"], inv / r["factor"], inv)
    smooth = (old / wavelen - r["low_freq_factor"]) / (r["high_freq_factor"] - r["low_freq_factor"])
    between = (wavelen >= old / r["high_freq_factor"]) & (wavelen <= old / r["low_freq_factor"])
    inv = np.where(between, (1 - smooth) * scaled / r["factor"] + smooth * scaled, scaled).astype(np.float32)
  return inv


def rotary_tables(c, n):
  """One head's cos and sin for places 0..n-1, (n, head_dim) fp32 holding bf16 values: fp32 angles rounded to bf16,
  each half the same (models/llama.py:354-368; the kernel applies them to every q and k head)."""
  angles = np.arange(n, dtype=np.float32)[:, None] * frequencies(c)[None]
  def bf16(a):
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + (b >> 16 & 1)) >> 16 & 0xFFFF).astype(np.uint32) << 16).view(np.float32)
  return bf16(np.concatenate([np.cos(angles)] * 2, 1)), bf16(np.concatenate([np.sin(angles)] * 2, 1))


class Decoder:
  """The model's weights on the GPU (block floats by precision), its KV cache, and the buffers of a step of `batch`
  rows. weights(name, shape) gives each weight as a torch fp32 (or bf16) tensor on the GPU, named as models/llama.py's
  fuse leaves them: layers.{l}.input_layernorm, .post_attention_layernorm, .qkv_proj, .o_proj, .gate_up_proj,
  .down_proj (x @ w), norm, embed, embed.T (the output layer; the embedding's transpose when tied)."""

  def __init__(self, c, weights, mode="bfp8", kv="bf16", batch=1, context=256, device="cuda", slots=1, mfma_from=3,
               share=None):
    """mfma_from: the batch from which a step's matmuls run on the matrix cores (fh_gemm_bfp, bf16 rows) rather than
    the exact-product GEMV (None: never); 3 by default, where the two meet on MI355X (an 8B step: 3.0 ms either way at
    3 rows, 3.06 against 3.42 at 4, 3.44 against 6.49 at 8). share: another Decoder of the same model whose weights this one uses."""
    self.c, self.mode, self.batch, self.context, self.device = c, mode, batch, context, torch.device(device)
    self.prec = precision(c, mode)
    hd = head(c)
    self.hd, self.qkv_cols = hd, (c.heads + 2 * c.kv) * hd
    self.mm = ops.gemm if mfma_from is not None and batch >= mfma_from else ops.gemv
    if share is not None:
      self.layers, self.norm, self.embed, self.head, self.cos, self.sin = share.layers, share.norm, share.embed, share.head, share.cos, share.sin
    else:
      self._load(weights)
    self._buffers(kv, batch, context, slots)

  def _load(self, weights):
    """weights: weights(name, shape) giving x @ W's layout (numpy_weights, random_weights), or a checkpoint.Checkpoint,
    whose matrices are packed straight from its rows (fused and transposed in the packing)."""
    c, hd = self.c, self.hd
    ck = weights if hasattr(weights, "pack") else None
    f32 = lambda t: t.to(self.device, torch.float32).contiguous()

    def mat(name, K, N, fmt):
      bw = ck.pack(name, fmt) if ck is not None else ops.pack(weights(name, (K, N)).to(self.device), fmt)
      if (bw.K, bw.N) != (K, N): raise ValueError(f"{name}: {bw.K}x{bw.N}, the model says {K}x{N}")
      return bw

    def vec(name):
      return ck.vector(name) if ck is not None else f32(weights(name, (1, c.dim))).reshape(-1)

    self.layers = []
    for l in range(c.layers):
      pre = f"layers.{l}."
      L = SimpleNamespace()
      L.norm1, L.norm2 = vec(pre + "input_layernorm"), vec(pre + "post_attention_layernorm")
      L.qkv = mat(pre + "qkv_proj", c.dim, self.qkv_cols, self.prec["qkv", l])
      L.o = mat(pre + "o_proj", c.heads * hd, c.dim, self.prec["o", l])
      L.gate_up = mat(pre + "gate_up_proj", c.dim, 2 * c.ffn, self.prec["gate_up", l])
      L.down = mat(pre + "down_proj", c.ffn, c.dim, self.prec["down", l])
      self.layers.append(L)
    self.norm = vec("norm")
    # the embedding in bf16 (a row read per token); the output layer its own matrix, or the embedding's rows packed
    # as its transpose (tied)
    self.embed = ck.table() if ck is not None else weights("embed", (c.vocab, c.dim)).to(self.device, torch.bfloat16).contiguous()
    if ck is not None: self.head = mat("embed.T", c.dim, c.vocab, self.prec["head", None])
    elif c.tied: self.head = ops.pack_parts([self.embed], self.prec["head", None])
    else: self.head = mat("embed.T", c.dim, c.vocab, self.prec["head", None])
    cos, sin = rotary_tables(c, c.places)
    self.cos, self.sin = torch.from_numpy(cos).to(self.device), torch.from_numpy(sin).to(self.device)

  def _buffers(self, kv, batch, context, slots):
    c, hd = self.c, self.hd
    # the KV cache: a block's keys' heads then values', `slots` sequences' rows side by side (models/llama.py:506-514)
    self.slots = slots or 1
    self.part = context  # rows a sequence
    # (bfp8 / bfp4: a block-float cache, each run of 16 of a row rounded as the qkv epilogue puts it; llama.py:127-128)
    if kv not in ("fp32", "bf16", "bfp8", "bfp4"): raise ValueError(f"kv cache: fp32, bf16, bfp8 or bfp4, not {kv}")
    self.kv = kv
    self.cache = [ops.kv_cache(2 * c.kv, self.slots * context, hd, kv, self.device) for _ in range(c.layers)]
    # a step's buffers, fixed so a step replays as a graph
    B = batch
    z = lambda *s: torch.zeros(*s, dtype=torch.float32, device=self.device)
    self.ids = torch.zeros(B, dtype=torch.int32, device=self.device)
    self.places = torch.zeros(B, dtype=torch.int32, device=self.device)
    self.rows = torch.zeros(B, dtype=torch.int32, device=self.device)       # cache row of each row's token
    self.first = torch.zeros(B, dtype=torch.int32, device=self.device)      # its sequence's first cache row
    self.x, self.ssq = z(B, c.dim), z(B, c.dim // 16)
    self.q, self.att = z(B, c.heads * hd), z(B, c.heads * hd)
    self.h = z(B, c.ffn)
    # the matrix cores' bf16 rows: each residual epilogue's copy, SwiGLU's output, attention's output for o; in tiles of
    # 16 rows (FH_BF16_T16) up to 64 rows, which the matrix-core kernel for a few rows loads a whole line at a time. That
    # kernel takes K a multiple of 64 only: a model with any matmul's K (dim, heads head_dim, ffn) off that keeps plain
    # bf16 rows, which the tiled GEMM takes at any K
    tiled = B <= 64 and all(k % 64 == 0 for k in (c.dim, c.heads * hd, c.ffn))
    rows16 = ops.tiles16 if tiled else (lambda r, n, d: torch.zeros(r, n, dtype=torch.bfloat16, device=d))
    self.xn = rows16(B, c.dim, self.device)
    self.hb = rows16(B, c.ffn, self.device)
    self.attb = rows16(B, c.heads * hd, self.device)
    self.logits = z(B, c.vocab)
    self.picks = torch.zeros(B, dtype=torch.int32, device=self.device)
    self.parts = torch.zeros(B, c.vocab // 16, dtype=torch.int64, device=self.device)  # each run of 16 logits' best
    self.ws = ops.attention_workspace(B, c.heads, hd, context, self.device)
    self.graph = None
    self.top = 0  # the largest place of the rows set (set_rows), which advance raises

  def weight_bytes(self):
    """Bytes of the weights one decode step reads: every matrix, a row of the embedding, the norms."""
    n = sum(w.nbytes for L in self.layers for w in (L.qkv, L.o, L.gate_up, L.down)) + self.head.nbytes
    return n + self.c.dim * 2 + (2 * self.c.layers + 1) * self.c.dim * 4

  def set_rows(self, places, slots=None):
    """Each row's place, and the cache rows: slot s's sequence keeps rows s * context .. (models/llama.py:429-452)."""
    places = torch.as_tensor(places, dtype=torch.int32)
    slots = torch.zeros_like(places) if slots is None else torch.as_tensor(slots, dtype=torch.int32)
    if places.shape != (self.batch,) or slots.shape != (self.batch,): raise ValueError(f"set_rows: {self.batch} places and slots")
    if (places < 0).any() or (places >= min(self.context, self.c.places)).any(): raise ValueError("a place past the cache or RoPE's tables")
    if (slots < 0).any() or (slots >= self.slots).any(): raise ValueError(f"a slot outside 0..{self.slots - 1}")
    self.top = int(places.max())  # (the largest place, kept on the host for advance's check)
    self.places.copy_(places)
    self.first.copy_(slots * self.part)
    self.rows.copy_(slots * self.part + places)

  def _cache(self, l):
    data, dtype, length = ops.cache_fields(self.cache[l])
    return dict(cache=data, cache_dtype=dtype, cache_len=length)

  def _step(self):
    if self.mm is ops.gemm: return self._step_rows()
    c, B, hd = self.c, self.batch, self.hd
    ops.embed_rows(self.embed, self.ids, self.x, self.ssq)
    for l, L in enumerate(self.layers):
      ep = ops.epilogue(lib.EP_ROPE_KV, norm_w=L.norm1, ssq_in=self.ssq, eps=c.eps, centered=int(c.centered),
                        heads=c.heads, kv_heads=c.kv, head_dim=hd, cos_tab=self.cos, sin_tab=self.sin, rope_rows=self.cos.shape[0],
                        places=self.places, cache_rows=self.rows, **self._cache(l))
      ops.gemv(self.x, L.qkv, ep, out=self.q)
      ops.attention_decode(self.q, self.cache[l], c.heads, c.kv, hd, self.places, self.first, self.context, self.ws, o=self.att)
      ep = ops.epilogue(lib.EP_RESIDUAL, residual=self.x, ssq_out=self.ssq)
      ops.gemv(self.att, L.o, ep, out=self.x)
      ep = ops.epilogue(lib.EP_SILU_GATE, norm_w=L.norm2, ssq_in=self.ssq, eps=c.eps, centered=int(c.centered), split=c.ffn)
      ops.gemv(self.x, L.gate_up, ep, out=self.h)
      ep = ops.epilogue(lib.EP_RESIDUAL, residual=self.x, ssq_out=self.ssq)
      ops.gemv(self.h, L.down, ep, out=self.x)
    ep = ops.epilogue(lib.EP_STORE, norm_w=self.norm, ssq_in=self.ssq, eps=c.eps, centered=int(c.centered), argmax_parts=self.parts)
    ops.gemv(self.x, self.head, ep, out=self.logits)
    ops.argmax_parts(self.parts, self.picks)

  def _norm_weights(self):
    """Each RMSNorm's multiplier (its weight, + 1 where centered) in the order a step meets them: block l's norm1,
    norm2, ..., then the final norm."""
    if getattr(self, "_nw", None) is None:
      c = self.c
      ws = [w for L in self.layers for w in (L.norm1, L.norm2)] + [self.norm]
      self._nw = [w + 1 if c.centered else w for w in ws]
    return self._nw

  def _step_rows(self):
    """A step of many rows on the matrix cores. The residual stream stays fp32; each residual epilogue also writes
    its rows times the next RMSNorm's weight in bf16 (copy_bf16, copy_w) with their sums of squares, and the next
    matmul takes those rows scaled by 1/rms (ssq_in alone): the products are its RMSNorm prologue's, bf16(x w), with
    no normalising pass (the first block's norm a kernel of its own). SwiGLU's output bf16."""
    c, B, hd = self.c, self.batch, self.hd
    nw = self._norm_weights()
    ops.embed_rows(self.embed, self.ids, self.x, self.ssq)
    rs = dict(ssq_in=self.ssq, eps=c.eps)  # rows that hold x w: 1/rms only
    for l, L in enumerate(self.layers):
      rope = dict(heads=c.heads, kv_heads=c.kv, head_dim=hd, cos_tab=self.cos, sin_tab=self.sin, rope_rows=self.cos.shape[0], places=self.places,
                  cache_rows=self.rows, **self._cache(l))
      if l == 0:
        ops.rms_rows(self.x, L.norm1, c.eps, c.centered, out=self.xn)
        ops.gemm(self.xn, L.qkv, ops.epilogue(lib.EP_ROPE_KV, **rope), out=self.q)
      else:
        ops.gemm(self.xn, L.qkv, ops.epilogue(lib.EP_ROPE_KV, **rs, **rope), out=self.q)
      ops.attention_decode(self.q, self.cache[l], c.heads, c.kv, hd, self.places, self.first, self.context, self.ws, o=self.attb)
      ops.gemm(self.attb, L.o, ops.epilogue(lib.EP_RESIDUAL, residual=self.x, ssq_out=self.ssq, copy_bf16=self.xn,
                                           copy_w=nw[2 * l + 1]), out=self.x)
      ops.gemm(self.xn, L.gate_up, ops.epilogue(lib.EP_SILU_GATE, split=c.ffn, **rs), out=self.hb)
      ops.gemm(self.hb, L.down, ops.epilogue(lib.EP_RESIDUAL, residual=self.x, ssq_out=self.ssq, copy_bf16=self.xn,
                                             copy_w=nw[2 * l + 2]), out=self.x)
    ops.gemm(self.xn, self.head, ops.epilogue(lib.EP_STORE, argmax_parts=self.parts, **rs), out=self.logits)
    ops.argmax_parts(self.parts, self.picks)

  def _prefill_buffers(self, T):
    c, hd, dev = self.c, self.hd, self.device
    P = getattr(self, "_pre", None)
    if P is None or P.T < T:
      z = lambda *s, dtype=torch.float32: torch.zeros(*s, dtype=dtype, device=dev)
      P = SimpleNamespace(T=T, ids=z(T, dtype=torch.int32), places=z(T, dtype=torch.int32), rows=z(T, dtype=torch.int32),
                          x=z(T, c.dim), ssq=z(T, c.dim // 16), xn=z(T, c.dim, dtype=torch.bfloat16), q=z(T, c.heads * hd),
                          att=z(T, c.heads * hd, dtype=torch.bfloat16), h=z(T, c.ffn, dtype=torch.bfloat16),
                          logits=z(1, c.vocab), parts=z(1, c.vocab // 16, dtype=torch.int64), pick=z(1, dtype=torch.int32))
      self._pre = P
    return P

  def prefill(self, ids, slot=0, p0=0, chunk=None):
    """A prompt's tokens at places p0 .. p0 + len(ids) - 1 of sequence `slot`, on the matrix cores (in chunks of
    `chunk` tokens, as models/llama.py:498-504 prefills): their keys and values go into the cache; returns the last
    token's logits ([1][vocab] fp32) and its greedy pick ([1] int32)."""
    ids = [int(i) for i in ids]
    T = len(ids)
    if T < 1 or p0 < 0 or p0 + T > min(self.context, self.c.places): raise ValueError("prefill: the prompt's places past the cache or RoPE's tables")
    if not 0 <= slot < self.slots: raise ValueError(f"prefill: slot {slot} outside 0..{self.slots - 1}")
    chunk = chunk or T
    for a in range(0, T, chunk):
      out = self._prefill_chunk(ids[a:a + chunk], slot, p0 + a)
    return out

  def _prefill_chunk(self, ids, slot, p0):
    c, hd = self.c, self.hd
    T = len(ids)
    P = self._prefill_buffers(T)
    ids_t, places, rows = P.ids[:T], P.places[:T], P.rows[:T]
    x, ssq, xn, q, att, h = P.x[:T], P.ssq[:T], P.xn[:T], P.q[:T], P.att[:T], P.h[:T]
    ids_t.copy_(torch.as_tensor(ids, dtype=torch.int32))
    places.copy_(torch.arange(p0, p0 + T, dtype=torch.int32))
    rows.copy_(places + slot * self.part)
    ops.embed_rows(self.embed, ids_t, x, ssq)
    # (each RMSNorm a pass of its own here: at 2048 rows the tiled kernel's per-tile sums of the rows' squares cost
    # more than fh_rms_rows; the batched decode takes the residual epilogues' scaled copies instead)
    for l, L in enumerate(self.layers):
      ops.rms_rows(x, L.norm1, c.eps, c.centered, out=xn)
      ep = ops.epilogue(lib.EP_ROPE_KV, heads=c.heads, kv_heads=c.kv, head_dim=hd, cos_tab=self.cos, sin_tab=self.sin, rope_rows=self.cos.shape[0],
                        places=places, cache_rows=rows, **self._cache(l))
      ops.gemm(xn, L.qkv, ep, out=q)
      ops.attention_prefill(q, self.cache[l], c.heads, c.kv, hd, p0, slot * self.part, o=att)
      ops.gemm(att, L.o, ops.epilogue(lib.EP_RESIDUAL, residual=x), out=x)
      ops.rms_rows(x, L.norm2, c.eps, c.centered, out=xn)
      ops.gemm(xn, L.gate_up, ops.epilogue(lib.EP_SILU_GATE, split=c.ffn), out=h)
      ops.gemm(h, L.down, ops.epilogue(lib.EP_RESIDUAL, residual=x, ssq_out=ssq), out=x)
    ep = ops.epilogue(lib.EP_STORE, norm_w=self.norm, ssq_in=ssq[T - 1:], eps=c.eps, centered=int(c.centered), argmax_parts=P.parts)
    ops.gemv(x[T - 1:], self.head, ep, out=P.logits)
    ops.argmax_parts(P.parts, P.pick)
    return P.logits, P.pick

  def step(self, ids=None, places=None, slots=None, replay=True):
    """One step: the logits (fp32, [batch][vocab]) and picks for tokens ids at places. With replay, the step runs as
    a HIP graph captured on the first call (every later step launches the same kernels: places are data)."""
    if ids is not None: self.ids.copy_(torch.as_tensor(ids, dtype=torch.int32))
    if places is not None: self.set_rows(places, slots)
    if not replay:
      self._step()
    else:
      if self.graph is None:
        self._step()  # warm: every kernel loaded before capture
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
          self._step()
        self.graph = g
      self.graph.replay()
    return self.logits, self.picks

  def advance(self):
    """Each row's next place and its pick as the next token, on the GPU (no host round trip): greedy decoding. Raises
    once a row's next place would pass the cache or RoPE's tables (the host keeps the largest place: set_rows', plus
    one a call)."""
    if self.top + 1 >= min(self.context, self.c.places): raise ValueError(f"advance: place {self.top + 1} past the cache or RoPE's tables")
    self.top += 1
    self.ids.copy_(self.picks)
    self.places.add_(1)
    self.rows.add_(1)

  def heads(self, k=64, inv_temp=None):
    """The last step's logit heads (models/serve.py:31-47): each row's k best logits and their tokens, and given each
    row's 1/temperature, the log of the sum of exp(x t) over its row (ops.logit_heads: fh_logit_heads)."""
    if inv_temp is not None and not isinstance(inv_temp, torch.Tensor):
      inv_temp = torch.as_tensor(inv_temp, dtype=torch.float32, device=self.device).reshape(-1)
    return ops.logit_heads(self.logits, k, inv_temp)


def numpy_weights(w):
  """weights(name, shape) over a dict of numpy arrays (bf16 values as float32), for Decoder."""
  def get(name, shape):
    a = np.asarray(w[name], np.float32).reshape(shape)
    return torch.from_numpy(np.ascontiguousarray(a))
  return get


def random_weights(c, seed=0, sd=0.02, norm_sd=0.1, embed_sd=1.0, device="cuda"):
  """weights(name, shape) drawn on the GPU: matrices N(0, sd), norms N(1, norm_sd), the embedding N(0, embed_sd), each
  rounded to bf16, from a generator seeded by seed and the weight's name (so each is the same whatever asks first)."""
  def get(name, shape):
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1000003 + sum(ord(ch) * 31 ** i for i, ch in enumerate(name)) % (2**31))
    if "norm" in name: t = torch.randn(*shape, generator=g, device=device) * norm_sd + 1
    elif name == "embed": t = torch.randn(*shape, generator=g, device=device) * embed_sd
    else: t = torch.randn(*shape, generator=g, device=device) * sd
    return t.to(torch.bfloat16)
  return get
