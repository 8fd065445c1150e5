"""The hot path's benchmark: ferrite's block-float decode on one MI355X, on the 8B decode workload (Llama-3.1-8B's shape,
attention and the output layer in bfp8, every MLP matrix in bfp4, a bf16 KV cache at context 2048, batch 1).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3|c3-bfp8|c2] [--batch B] [--no-cpu] [--no-prefill]
                [--only bs1|bs16|prefill|moe|floor|peaks|c1|c2]

Prints ONE JSON line: tokens/s of the whole decode step (every kernel of it replayed as one HIP graph, inputs resident
in HBM), the dominant GEMV's achieved HBM bandwidth against the 8 TB/s peak (timed live with HIP events on its own
stream), each GEMV's GB/s, and the CPU baseline: the numpy restatement (oracle/) of one block and the output layer
timed on this host's cores and scaled to a token; and config 4's prefill (a 2048-token prompt on the matrix cores) as
its own field, with the same step with every matrix bfp8 (`decode_bfp8`), batches 2-16, and config 5's MoE layer;
`configs` holds config 1's GEMV and config 2's SmolLM step on the GPU, and the numpy CPU baselines of configs 1, 2, 4
and 5 (bounded samples, each saying how it was scaled). Synthetic data: random-init weights, drawn on the GPU and
packed there. --only runs one part by itself and prints its fields as the JSON line (what a profiler run of one part
uses): the batch-1 step and its GEMVs, the batch-16 step, config 4's prefill, config 5's MoE layer, the read floor (read_floor), the matrix cores'
and LDS's own rates (core_peaks), config 1's GEMVs or config 2's SmolLM step."""
import argparse, json, os, statistics, sys, time
import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s (published)
MFMA_PEAK = 2.5e15  # MI355X dense bf16 matrix-core FLOP/s (published)


def config(name):
  from ferrite_amd import llama as G
  r = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
  if name in ("c3", "c3-bfp8"):
    c = G.model(dim=4096, heads=32, kv=8, layers=32, eps=1e-5, theta=500000.0, vocab=128256, ffn=14336, places=2048, rope=r)
    return c, ("experts" if name == "c3" else "bfp8"), 2048
  if name == "c2":
    c = G.model(dim=576, heads=9, kv=3, layers=30, eps=1e-5, theta=10000.0, vocab=49152, ffn=1536, places=256, tied=True)
    return c, "bfp8", 144
  raise SystemExit(f"unknown config {name}")


def timed_graph(fn, reps, stream):
  """Captures fn into a HIP graph, replays it reps times between two HIP events on `stream` (the stream the kernels
  are launched on), returns milliseconds per replay."""
  with torch.cuda.stream(stream):
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
      fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps): g.replay()
    b.record(stream)
    b.synchronize()
  return a.elapsed_time(b) / reps


def gemv_rates(dec, stream, reps=5):
  """Each GEMV of the step exactly as the step launches it (its epilogue and prologue included), back to back over
  every block's weight (32 distinct matrices, past the 256 MB Infinity Cache), in a graph timed by HIP events on the
  stream the kernels run on: {name: (fmt, K, N, bytes a launch, us a launch, GB/s)}. Bytes are the algorithmic ones:
  the packed weight, x and the norm's weights read once, y written once."""
  from ferrite_amd import lib, ops
  c, B = dec.c, dec.batch
  calls = {
    "qkv": [(dec.x, L.qkv, lambda L=L, l=l: ops.epilogue(lib.EP_ROPE_KV, norm_w=L.norm1, ssq_in=dec.ssq, eps=c.eps, heads=c.heads,
             kv_heads=c.kv, head_dim=dec.hd, cos_tab=dec.cos, sin_tab=dec.sin, rope_rows=dec.cos.shape[0], places=dec.places, cache_rows=dec.rows,
             **dec._cache(l)), dec.q, c.dim * 4)
            for l, L in enumerate(dec.layers)],
    "o": [(dec.att, L.o, lambda: ops.epilogue(lib.EP_RESIDUAL, residual=dec.x, ssq_out=dec.ssq), dec.x, 0) for L in dec.layers],
    "gate_up": [(dec.x, L.gate_up, lambda L=L: ops.epilogue(lib.EP_SILU_GATE, norm_w=L.norm2, ssq_in=dec.ssq, eps=c.eps, split=c.ffn),
                 dec.h, c.dim * 4) for L in dec.layers],
    "down": [(dec.h, L.down, lambda: ops.epilogue(lib.EP_RESIDUAL, residual=dec.x, ssq_out=dec.ssq), dec.x, 0) for L in dec.layers],
    "head": [(dec.x, dec.head, lambda: ops.epilogue(lib.EP_STORE, norm_w=dec.norm, ssq_in=dec.ssq, eps=c.eps, argmax_parts=dec.parts),
              dec.logits, c.dim * 4)] * 4,
  }
  out = {}
  for name, seq in calls.items():
    eps = [(x, w, make(), y, extra) for x, w, make, y, extra in seq]  # built once, outside the capture
    def run():
      for x, w, ep, y, extra in eps: ops.gemv(x, w, ep, out=y)
    ms = timed_graph(run, reps, stream)
    per = ms / len(eps) * 1e-3
    x, w, ep, y, extra = eps[0]
    nbytes = w.nbytes + B * w.K * 4 + B * y.shape[1] * 4 + extra  # W, x, y (and the norm's weights)
    out[name] = dict(fmt=w.fmt, K=w.K, N=w.N, bytes=nbytes, us=per * 1e6, gbs=nbytes / per / 1e9)
  return out


def step_rate(dec, context, steps, warmup, stream):
  """A batch-1 decoder's whole step at the last place of a full context of random keys and values, captured as one
  HIP graph and replayed `steps` times between two HIP events on `stream` (as main times config 3's step)."""
  c = dec.c
  for cache in dec.cache: cache.normal_(0, 1)
  with torch.cuda.stream(stream):
    dec.ids.copy_(torch.tensor([1], dtype=torch.int32))
    dec.set_rows([context - 1], [0])
    dec.step(replay=True)
    for _ in range(warmup): dec.graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps): dec.graph.replay()
    b.record(stream)
    b.synchronize()
  ms = a.elapsed_time(b) / steps
  nbytes = dec.weight_bytes() + c.layers * 2 * c.kv * dec.hd * context * 2
  mats = "every matrix bfp8" if dec.mode == "bfp8" else "attention and output layer bfp8, MLP bfp4"
  return {"workload": f"config 3 with {mats}: Llama-3.1-8B-shape decode, batch 1, context {context}, bf16 KV",
          "ms_per_step": round(ms, 4), "tokens_per_s": round(1000 / ms, 2), "step_bytes": nbytes,
          "step_gbs": round(nbytes / ms / 1e6, 1)}


def prefill_rate(T=2048, reps=3):
  """Config 4: a T-token prompt through the 8B shape with every matrix bfp8 (the matrix-core path: fh_rms_rows,
  fh_gemm_bfp, fh_attention_prefill; the output layer on the last token), timed by HIP events on its stream; and each
  GEMM shape and the attention alone. FLOPs are the algorithmic ones: 2 T K N a matmul, 4 hd heads T(T+1)/2 a
  block's causal attention, 2 dim vocab the last token's output layer."""
  from ferrite_amd import llama as G, ops
  c, _, _ = config("c3")
  dev = torch.device("cuda:0")
  dec = G.Decoder(c, G.random_weights(c, seed=2, device=dev), mode="bfp8", kv="bf16", batch=1, context=T)
  hd = dec.hd
  ids = [(7 * i + 3) % c.vocab for i in range(T)]
  stream = torch.cuda.Stream(device=dev)
  mats = {"qkv": (c.dim, dec.qkv_cols), "o": (c.heads * hd, c.dim), "gate_up": (c.dim, 2 * c.ffn), "down": (c.ffn, c.dim)}
  lin = sum(2 * T * k * n for k, n in mats.values()) * c.layers
  att = 4 * hd * c.heads * T * (T + 1) // 2 * c.layers
  flops = lin + att + 2 * c.dim * c.vocab
  def timed(fn, n):
    with torch.cuda.stream(stream):
      fn()
      torch.cuda.synchronize()
      a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
      a.record(stream)
      for _ in range(n): fn()
      b.record(stream)
      b.synchronize()
    return a.elapsed_time(b) / n
  ms = timed(lambda: dec.prefill(ids), reps)
  out = {"workload": f"config 4: Llama-3.1-8B-shape prefill of {T} tokens, all bfp8, bf16 KV", "ms": round(ms, 3),
         "tokens_per_s": round(T * 1000 / ms, 1), "tflops": round(flops / ms / 1e9, 1),
         "mfma_frac": round(flops / ms * 1e3 / MFMA_PEAK, 4), "flops": flops}
  L = dec.layers[0]
  xb = torch.randn(T, max(c.dim, c.ffn), device=dev).to(torch.bfloat16)
  P = dec._prefill_buffers(T)
  shapes = {"qkv": (L.qkv, xb[:, :c.dim], torch.empty(T, dec.qkv_cols, device=dev)),
            "o": (L.o, xb[:, :c.dim], torch.empty(T, c.dim, device=dev)),
            "gate_up": (L.gate_up, xb[:, :c.dim], torch.empty(T, 2 * c.ffn, device=dev)),
            "down": (L.down, xb[:, :c.ffn], torch.empty(T, c.dim, device=dev))}
  g = {}
  for name, (w, x, y) in shapes.items():
    x = x.contiguous()
    t = timed(lambda: ops.gemm(x, w, out=y), 5)
    g[name] = round(2 * T * w.K * w.N / t / 1e9, 1)
  t = timed(lambda: ops.attention_prefill(P.q[:T], dec.cache[0], c.heads, c.kv, hd, 0, 0, o=P.att[:T]), 5)
  out["gemm_tflops"] = g
  out["attention_tflops"] = round(4 * hd * c.heads * T * (T + 1) / 2 / t / 1e9, 1)
  del dec
  torch.cuda.empty_cache()
  return out


def decode_batch(dec, context, B=16, steps=20):
  """Config 3 at batch B (16 by default): B sequences a step, each at the last place of a full context of its own (a
  slot of the cache each), the matmuls on the matrix cores (the skinny kernel) from Decoder's mfma_from rows on, the
  step replayed as a HIP graph; the weights are the batch-1 decoder's."""
  from ferrite_amd import llama as G
  c = dec.c
  d = G.Decoder(c, None, mode=dec.mode, kv="bf16", batch=B, context=context, slots=B, share=dec)
  for cache in d.cache: cache.normal_(0, 1)
  stream = torch.cuda.Stream()
  with torch.cuda.stream(stream):
    d.ids.copy_(torch.arange(B, dtype=torch.int32) * 7 + 1)
    d.set_rows([context - 1] * B, list(range(B)))
    d.step(replay=True)
    for _ in range(3): d.graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps): d.graph.replay()
    b.record(stream)
    b.synchronize()
  ms = a.elapsed_time(b) / steps
  kv = c.layers * 2 * c.kv * d.hd * context * 2 * B
  nbytes = d.weight_bytes() + kv
  on = "the matrix cores" if d.mm.__name__ == "gemm" else "the GEMV"
  out = {"workload": f"config 3 at batch {B}: {B} sequences at context {context}, matmuls on {on}",
         "batch": B, "ms_per_step": round(ms, 4), "tokens_per_s": round(B * 1000 / ms, 1),
         "step_gbs": round(nbytes / ms / 1e6, 1)}
  del d
  torch.cuda.empty_cache()
  return out


def moe_rate(T=32, reps=20):
  """Config 5: a Mixtral-shape mixture-of-experts layer for T tokens: h [T][4096] ~N(0,1) bf16 values, router
  [4096][8] bf16 ~N(0, 0.02), 8 experts' gate_up [4096][28672] and down [14336][4096] ~N(0, 0.02) in bfp4, top 2
  (fh_moe_route, fh_moe_experts), timed as one HIP graph by events. Bytes: the experts some token picked, each read
  once, the router, h and the output."""
  from ferrite_amd import ops
  dev = torch.device("cuda:0")
  dim, ffn, E, k = 4096, 14336, 8, 2
  g = torch.Generator(device=dev)
  g.manual_seed(5)
  h = torch.randn(T, dim, generator=g, device=dev).to(torch.bfloat16).float()
  router = (torch.randn(dim, E, generator=g, device=dev) * 0.02).to(torch.bfloat16)
  gu = (torch.randn(E, dim, 2 * ffn, generator=g, device=dev) * 0.02).to(torch.bfloat16)
  dn = (torch.randn(E, ffn, dim, generator=g, device=dev) * 0.02).to(torch.bfloat16)
  ex = ops.pack_experts(gu, dn, "bfp4")
  del gu, dn
  torch.cuda.empty_cache()
  y = torch.empty(T, dim, device=dev)
  ws = torch.empty(max(ops.lib.load().fh_moe_workspace_bytes(T, E, ffn, dim), 256), dtype=torch.uint8, device=dev)
  state = {}
  def run():
    ids, w, dense = ops.moe_route(h, router, E, k)
    state["dense"] = dense
    ops.moe_experts(h, ex, dense, out=y, ws=ws)
  stream = torch.cuda.Stream(device=dev)
  ms = timed_graph(run, reps, stream)
  touched = int((state["dense"] != 0).any(0).sum())
  nbytes = touched * (ex.gate_up.nbytes + ex.down.nbytes) // E + dim * E * 2 + T * dim * 4 * 2
  flops = 2 * T * k * dim * 3 * ffn  # (each token's k experts: gate_up 2 ffn and down ffn columns of dim)
  return {"workload": f"config 5: Mixtral-shape MoE layer, {T} tokens, {E} experts bfp4, top {k}", "us": round(ms * 1e3, 2),
          "experts_touched": touched, "bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
          "frac": round(nbytes / ms * 1e3 / HBM_PEAK, 4), "tflops": round(flops / ms / 1e9, 1)}


def config1_rate(dev, copies=300, reps=10):
  """Config 1: the bfp8 GEMV x[1,576] @ W[576,1536] (fp32 out), its 16-element blocks along N (ferrite's own layout,
  fh_gemv_bfp) and, as config 1's text states it, along K (fh_gemv_bfp_k). Over `copies` distinct packed weights
  (940,032 bytes each: 282 MB, past the 256 MB Infinity Cache) launched back to back in a HIP graph, so each launch
  reads its weight from HBM; and the same weight replayed (cache-resident: the launch's latency). Bytes a launch: the
  packed weight, x (bf16 values held in fp32, 576 x 4) and y (1536 x 4): 947,328 algorithmic bytes as config 1 counts
  them with x in bf16 (x is 2,304 bytes here, read as fp32)."""
  from ferrite_amd import lib, ops
  K, N = 576, 1536
  nbytes = K * N * 17 // 16 + K * 2 + N * 4
  out = {"workload": "config 1: bfp8 GEMV x[1,576] @ W[576,1536], fp32 out", "bytes": nbytes, "copies": copies}
  for axis, key in ((lib.AXIS_N, ""), (lib.AXIS_K, "along_k_")):
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    ws = [ops.pack(torch.randn(K, N, generator=g, device=dev) * 0.02, "bfp8", axis=axis) for _ in range(copies)]
    x = torch.randn(1, K, generator=g, device=dev).to(torch.bfloat16).float()
    y = torch.empty(1, N, device=dev)
    stream = torch.cuda.Stream(device=dev)
    def many():
      for w in ws: ops.gemv(x, w, out=y)
    ms = timed_graph(many, reps, stream) / copies
    one = timed_graph(lambda: [ops.gemv(x, ws[0], out=y) for _ in range(copies)], reps, stream) / copies
    del ws
    torch.cuda.empty_cache()
    out |= {key + "us": round(ms * 1e3, 3), key + "gbs": round(nbytes / ms / 1e6, 1),
            key + "us_cache_resident": round(one * 1e3, 3)}
  return out


def config2_rate(dev, steps=50, warmup=5, place=143):
  """Config 2: SmolLM-135M's shape (30 blocks, 576 wide, 9/3 heads of 64, MLP 1536, vocab 49152 tied, bfp8), one
  token's decode step at place 143 of a bf16 KV cache (128 prompt rows and 16 decoded before it), the whole step one
  HIP graph replayed between HIP events."""
  from ferrite_amd import llama as G
  c, mode, context = config("c2")
  dec = G.Decoder(c, G.random_weights(c, seed=3, device=dev), mode=mode, kv="bf16", batch=1, context=256)
  for cache in dec.cache: cache.normal_(0, 1)
  stream = torch.cuda.Stream(device=dev)
  with torch.cuda.stream(stream):
    dec.ids.copy_(torch.tensor([7], dtype=torch.int32))
    dec.set_rows([place], [0])
    dec.step(replay=True)
    for _ in range(warmup): dec.graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps): dec.graph.replay()
    b.record(stream)
    b.synchronize()
  ms = a.elapsed_time(b) / steps
  nbytes = dec.weight_bytes() + c.layers * 2 * c.kv * dec.hd * (place + 1) * 2
  del dec
  torch.cuda.empty_cache()
  # the step's launches (embedding; qkv, attention, o, gate_up, down a block, the attention one launch at a context
  # of at most 4 chunks of 64 rows; output layer; pick), each replaced by a one-workgroup read of 4 KiB in a graph
  # of as many launches: what the launches alone cost
  from ferrite_amd import lib
  launches = 5 * c.layers + 3
  buf, sink = torch.ones(1024, device=dev), torch.empty(64, dtype=torch.int32, device=dev)
  floor = timed_graph(lambda: [lib.call("fh_read_probe", buf.data_ptr(), 4096, sink.data_ptr(), 1,
                                        torch.cuda.current_stream().cuda_stream) for _ in range(launches)], 5, stream)
  return {"workload": f"config 2: SmolLM-135M-shape decode, batch 1, place {place}, bfp8, bf16 KV", "ms_per_step": round(ms, 4),
          "tokens_per_s": round(1000 / ms, 1), "step_bytes": nbytes, "step_gbs": round(nbytes / ms / 1e6, 1),
          "launches": launches, "launch_floor_ms": round(floor, 4)}


def _median_time(fn, runs):
  fn()
  ts = []
  for _ in range(runs):
    t0 = time.perf_counter(); fn(); ts.append(time.perf_counter() - t0)
  return statistics.median(ts)


def cpu_configs():
  """The numpy restatement (oracle/) of configs 1, 2, 4 and 5 on this host's cores, every core BLAS gives, each a
  bounded sample of the workload timed as benchmark.timed does (median after a warm-up): float32 weights holding the
  block floats' values (the timing does not depend on the values, so they are drawn in float32 directly)."""
  from oracle import llama as OL
  rng = np.random.default_rng(0)
  f32 = lambda shape, sd=0.02: rng.standard_normal(shape, dtype=np.float32) * np.float32(sd)
  out = {}
  # config 1: x @ W (numpy's mm: float32 x float32), GB/s counted on the packed bytes as on the GPU
  x, w = f32((1, 576), 1.0), f32((576, 1536))
  t = _median_time(lambda: [x @ w for _ in range(1000)], 5) / 1000
  out["c1"] = {"us": round(t * 1e6, 3), "gbs": round(947328 / t / 1e9, 2), "unit": "us per GEMV",
               "sample": "1000 x @ W float32 (numpy sgemv) a run, median of 5"}
  # config 2: one token through the 30 blocks and the tied output layer at place 143, float64 caches (models/llama.py)
  c = OL.smollm(layers=30, vocab=49152, places=256)
  hd, qkv = OL.head(c), (c.heads + 2 * c.kv) * OL.head(c)
  wts = {"norm": np.ones((1, c.dim), np.float32), "embed": f32((c.vocab, c.dim), 1.0)}
  wts["embed.T"] = np.ascontiguousarray(wts["embed"].T)
  for l in range(c.layers):
    pre = f"layers.{l}."
    wts |= {pre + "input_layernorm": np.ones((1, c.dim), np.float32), pre + "post_attention_layernorm": np.ones((1, c.dim), np.float32),
            pre + "qkv_proj": f32((c.dim, qkv)), pre + "o_proj": f32((c.heads * hd, c.dim)),
            pre + "gate_up_proj": f32((c.dim, 2 * c.ffn)), pre + "down_proj": f32((c.ffn, c.dim))}
  wts["cos"], wts["sin"], wts["turn"] = OL.rotary(c, c.places)
  caches = OL.kv_cache(c, 256)
  for cache in caches: cache[:, :143] = rng.standard_normal(cache[:, :143].shape)
  t = _median_time(lambda: OL.forward([7], [143], wts, c, caches), 5)
  out["c2"] = {"tokens_per_s": round(1 / t, 2), "unit": "tokens/s", "sample": "one token at place 143, all 30 blocks, median of 5"}
  del wts, caches
  # config 4: one block of the 2048-token prefill (8B shape, float64 caches), scaled by 32 blocks, plus the output layer
  # for the last token
  c8 = OL.llama8b(layers=1, places=2048)
  hd, T = OL.head(c8), 2048
  p = {"input_layernorm": np.ones((1, c8.dim), np.float32), "post_attention_layernorm": np.ones((1, c8.dim), np.float32),
       "qkv_proj": f32((c8.dim, (c8.heads + 2 * c8.kv) * hd)), "o_proj": f32((c8.heads * hd, c8.dim)),
       "gate_up_proj": f32((c8.dim, 2 * c8.ffn)), "down_proj": f32((c8.ffn, c8.dim))}
  cos, sin, turn = OL.rotary(c8, T)
  mask = OL.masked(np.arange(T), T)
  xs = f32((T, c8.dim), 1.0)
  t = _median_time(lambda: OL.layer(xs, p, c8, (cos, sin, turn), mask, np.zeros((2 * c8.kv, T, hd)), np.arange(T)), 3)
  head = f32((c8.dim, 128256))
  th = _median_time(lambda: OL.rms(xs[-1:], p["norm"] if "norm" in p else p["input_layernorm"], c8) @ head, 3)
  out["c4"] = {"s": round(t * 32 + th, 2), "unit": "s per 2048-token prefill", "scaled": "one block's time x 32 + the output layer",
               "tokens_per_s": round(T / (t * 32 + th), 1), "sample": "one 8B-shape block over 2048 tokens, median of 3"}
  del p, head
  # config 5: the MoE layer for 32 tokens: each (token, chosen expert) pair's SwiGLU (numpy_experts, models/llama.py:294-300)
  # timed on 8 pairs of one expert's 4096 x 28672 and 14336 x 4096 float32 matrices and scaled to the 64 pairs of
  # 32 tokens x top 2, plus the router
  cm = OL.model(dim=4096, k=2, experts=8)
  gu, dn = f32((4096, 28672)), f32((14336, 4096))
  h = f32((32, 4096), 1.0)
  def pairs():
    for tkn in range(8):
      g = h[tkn] @ gu
      OL.glu(g[:14336], g[14336:]) @ dn
  tp = _median_time(pairs, 3) / 8
  router = f32((4096, 8))
  tr = _median_time(lambda: OL.topk(h @ router, 2), 5)
  out["c5"] = {"ms": round((tp * 64 + tr) * 1e3, 2), "unit": "ms per MoE layer (32 tokens)",
               "scaled": "8 (token, expert) SwiGLUs timed, x64 pairs, + the router", "sample": "one expert's matrices, median of 3"}
  return out


def measured_traffic(kernel, config, batch):
  """HBM bytes a launch of `kernel` moves, as the committed rocprofv3 counter summaries under profiles/ record them
  (lines `traffic: <kernel> <config> b<batch> <bytes>`: FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's
  reading for a copy kernel of known size in the same run), or None when no summary covers it."""
  import glob, re
  for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
    for m in re.finditer(r"^traffic: (\S+) (\S+) b(\d+) (\d+)$", open(f).read(), re.M):
      if (m[1], m[2], int(m[3])) == (kernel, config, batch): return int(m[4])
  return None


def core_peaks(dev, reps=5):
  """What the matrix cores and LDS reach on this GPU with nothing else to do (fh_mfma_probe, fh_lds_probe): MFMA loops
  of each form over 1024 and 2048 workgroups of 4 waves (16 and 32 waves a CU), 8 independent accumulators a wave;
  16-byte LDS reads over 2048 workgroups of 256 threads (8 a CU, 16 KiB of LDS each). Timed by HIP events on the
  current stream after a warm-up, the best of the grids; the LDS rate also per CU and clock at the 2.4 GHz peak engine
  clock."""
  from ferrite_amd import lib
  s = torch.cuda.current_stream().cuda_stream
  sink = torch.empty(2048, dtype=torch.float32, device=dev)
  def timed(fn):
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps): fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps * 1e-3
  out = {}
  for form, name, flops in ((0, "mfma_32x32x16_bf16_tflops", 32768), (1, "mfma_16x16x32_bf16_tflops", 16384)):
    iters = 200
    out[name] = round(max(blocks * 4 * iters * 8 * flops / timed(lambda: lib.call("fh_mfma_probe", form, iters, sink.data_ptr(), blocks, s))
                          for blocks in (1024, 2048)) / 1e12, 1)
  iters, blocks = 2000, 2048
  t = timed(lambda: lib.call("fh_lds_probe", iters, sink.data_ptr(), blocks, s))
  rate = blocks * 256 * iters * 4 * 16 / t
  cus = torch.cuda.get_device_properties(dev).multi_processor_count
  out["lds_read_tbs"] = round(rate / 1e12, 1)
  out["lds_read_bytes_per_clk_cu"] = round(rate / cus / 2.4e9, 1)
  return out


def read_floor(dev, reps=5):
  """What a plain read of each batch-1 GEMV's bytes takes, launched as the step launches a GEMV: a graph of 32 launches
  back to back over 32 distinct buffers (each read from HBM), each launch fh_read_probe (16-byte loads, four in flight
  a thread, the fastest of 1024-8192 workgroups of 256 threads: every byte read once, nothing else done), timed by HIP events on the
  stream: the floor a kernel of that many bytes meets before any arithmetic. Sizes: the 8B shapes' packed weights
  (magnitudes and exponents) of qkv and o (bfp8), gate_up and down (bfp4), and the all-bfp8 gate_up and down."""
  from ferrite_amd import lib
  sizes = {"qkv bfp8": 4096 * 6144 * 17 // 16, "o bfp8": 4096 * 4096 * 17 // 16, "down bfp4": 14336 * 4096 * 9 // 16,
           "gate_up bfp4": 4096 * 28672 * 9 // 16, "down bfp8": 14336 * 4096 * 17 // 16, "gate_up bfp8": 4096 * 28672 * 17 // 16}
  stream = torch.cuda.Stream(device=dev)
  sink = torch.empty(8192, dtype=torch.int32, device=dev)
  out = {}
  for name, nbytes in sizes.items():
    n = (nbytes + 15) // 16 * 16
    bufs = [torch.ones(n // 4, device=dev) for _ in range(32)]
    best = None
    for blocks in (1024, 2048, 4096, 8192):  # (the fastest grid of each size)
      def run():
        for t in bufs: lib.call("fh_read_probe", t.data_ptr(), n, sink.data_ptr(), blocks, torch.cuda.current_stream().cuda_stream)
      ms = timed_graph(run, reps, stream) / 32
      if best is None or ms < best[0]: best = (ms, blocks)
    ms, blocks = best
    out[name] = {"bytes": n, "us": round(ms * 1e3, 3), "gbs": round(n / ms / 1e6, 1), "blocks": blocks}
    del bufs
  torch.cuda.empty_cache()
  return out


def measured_peaks(dev, reps=10):
  """What this GPU reaches on plain library kernels, beside the published peaks: HBM read (torch.sum of 2 GiB of fp32
  by rows of 1024, every byte read once: the fastest of the reductions tried, ~6.4 TB/s) and copy (torch.neg, 2 GiB in and out), and a large bf16 GEMM on the matrix cores
  (torch.matmul, hipBLASLt, 8192^3), each timed by HIP events on the current stream after a warm-up."""
  def timed(fn):
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps): fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps * 1e-3
  n = 1 << 29
  src = torch.ones(n, device=dev)
  dst = torch.empty_like(src)
  rows = src.view(-1, 1024)
  acc = torch.empty(rows.shape[0], device=dev)
  read = 4 * n / timed(lambda: torch.sum(rows, 1, out=acc))
  copy = 8 * n / timed(lambda: torch.neg(src, out=dst))
  del src, dst
  m = 8192
  x = torch.randn(m, m, device=dev, dtype=torch.bfloat16)
  w = torch.randn(m, m, device=dev, dtype=torch.bfloat16)
  y = torch.empty(m, m, device=dev, dtype=torch.bfloat16)
  gemm = 2 * m ** 3 / timed(lambda: torch.matmul(x, w, out=y))
  del x, w, y
  torch.cuda.empty_cache()
  return {"hbm_read_gbs": round(read / 1e9, 1), "hbm_copy_gbs": round(copy / 1e9, 1),
          "bf16_gemm_tflops": round(gemm / 1e12, 1)}


def cpu_baseline(c, mode, context, runs=5):
  """The numpy restatement (oracle/llama.py) of one decode token on this host: one block at the step's context plus the
  output layer, each the median of `runs` timed runs after a warm-up, the block's time scaled by c.layers. The value:
  every core BLAS gives, float64 caches and activations as models/llama.py's main makes them (float32 weights promote);
  beside it (medians of 3) the same on one BLAS thread, and with float32 activations and caches."""
  from threadpoolctl import threadpool_limits, threadpool_info
  from oracle import llama as OL
  rng = np.random.default_rng(0)
  hd = c.dim // c.heads
  oc = OL.model(dim=c.dim, heads=c.heads, kv=c.kv, layers=1, eps=c.eps, theta=c.theta, vocab=c.vocab, ffn=c.ffn,
                places=context, rope=c.rope)
  p = {"input_layernorm": np.ones((1, c.dim), np.float32), "post_attention_layernorm": np.ones((1, c.dim), np.float32)}
  # block-float values as the GPU holds them; drawn already in float32 (the timing does not depend on the values)
  for name, shape in (("qkv_proj", (c.dim, (c.heads + 2 * c.kv) * hd)), ("o_proj", (c.heads * hd, c.dim)),
                      ("gate_up_proj", (c.dim, 2 * c.ffn)), ("down_proj", (c.ffn, c.dim))):
    p[name] = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)
  head_w = rng.standard_normal((c.dim, c.vocab), dtype=np.float32) * np.float32(0.02)
  cos, sin, t = OL.rotary(oc, context)
  place = context - 1
  mask = OL.masked([place], context)
  tables = (cos[[place]], sin[[place]], t)

  def per_token(dtype, runs=runs):
    cache = np.zeros((2 * c.kv, context, hd), dtype)
    x = rng.standard_normal((1, c.dim)).astype(dtype)
    fns = {"block": lambda: OL.layer(x, p, oc, tables, mask, cache, [place]),
           "head": lambda: OL.rms(x, p["input_layernorm"], oc) @ head_w}
    times = {}
    for name, fn in fns.items():
      fn()
      ts = []
      for _ in range(runs):
        t0 = time.perf_counter(); fn(); ts.append(time.perf_counter() - t0)
      times[name] = statistics.median(ts)
    return times["block"] * c.layers + times["head"], times

  all64, times = per_token(np.float64)
  all32, _ = per_token(np.float32, 3)
  with threadpool_limits(limits=1, user_api="blas"):
    one64, _ = per_token(np.float64, 3)
  blas = [f"{i['internal_api']} {i['version']} x{i['num_threads']}" for i in threadpool_info() if i["user_api"] == "blas"]
  return dict(value=1.0 / all64, unit="tokens/s", cores=len(os.sched_getaffinity(0)), kind="port",
              sample=f"numpy oracle: 1 of {c.layers} blocks at context {context} + output layer, median of {runs}, block "
                     f"x{c.layers}; float64 cache and activations (float32 weights), every core BLAS gives",
              block_s=times["block"], head_s=times["head"], blas=", ".join(blas),
              one_thread_tokens_per_s=1.0 / one64, float32_tokens_per_s=1.0 / all32)


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=50)
  ap.add_argument("--warmup", type=int, default=5)
  ap.add_argument("--config", default="c3")
  ap.add_argument("--batch", type=int, default=1)
  ap.add_argument("--no-cpu", action="store_true")
  ap.add_argument("--no-prefill", action="store_true", help="skip config 4's prefill measurement")
  ap.add_argument("--only", choices=("bs1", "bs16", "prefill", "moe", "floor", "peaks", "c1", "c2"), help="run one part alone (see above)")
  ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                  help="first run a plain copy kernel (torch.neg) over MIB MiB: the known-size kernel that calibrates "
                       "rocprofv3's FETCH_SIZE/WRITE_SIZE counters in the same run")
  args = ap.parse_args()
  if args.gpus != 1:
    print("bench.py measures one GPU: this build has no multi-GPU path (a decode would shard each weight by columns)",
          file=sys.stderr)
    raise SystemExit(2)
  from ferrite_amd import lib
  from ferrite_amd import llama as G
  lib.load()
  dev = torch.device("cuda:0")
  if args.copy_probe:
    src = torch.ones(args.copy_probe << 18, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2): torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
  c, mode, context = config(args.config)
  if args.only:
    if args.only == "bs1":  # the --config step at batch 1 and each of its GEMVs
      dec = G.Decoder(c, G.random_weights(c, seed=1, device=dev), mode=mode, kv="bf16", batch=1, context=context)
      stream = torch.cuda.Stream(device=dev)
      r = step_rate(dec, context, args.steps, args.warmup, stream)
      r["gemv"] = {k: {"us": round(v["us"], 2), "gbs": round(v["gbs"], 1)} for k, v in gemv_rates(dec, stream).items()}
    elif args.only == "bs16":
      dec = G.Decoder(c, G.random_weights(c, seed=1, device=dev), mode=mode, kv="bf16", batch=1, context=context)
      r = decode_batch(dec, context)
    elif args.only == "prefill": r = prefill_rate()
    elif args.only == "moe": r = {"moe": moe_rate(), "moe_prompt": moe_rate(2048, reps=5)}
    elif args.only == "peaks": r = core_peaks(dev)
    elif args.only == "c1": r = config1_rate(dev)
    elif args.only == "c2": r = config2_rate(dev)
    else: r = read_floor(dev)
    print(json.dumps({"only": args.only, **r}), flush=True)
    return
  t0 = time.time()
  dec = G.Decoder(c, G.random_weights(c, seed=1, device=dev), mode=mode, kv="bf16", batch=args.batch, context=context,
                  slots=args.batch)
  torch.cuda.synchronize()
  print(f"# weights packed on the GPU in {time.time() - t0:.1f}s: {dec.weight_bytes() / 1e9:.3f} GB", file=sys.stderr, flush=True)
  for cache in dec.cache: cache.normal_(0, 1)  # a full context of keys and values
  stream = torch.cuda.Stream(device=dev)
  B = args.batch
  place = context - 1
  with torch.cuda.stream(stream):
    dec.ids.copy_(torch.arange(B, dtype=torch.int32) * 7 + 1)
    dec.set_rows([place] * B, list(range(B)))
    dec.step(replay=True)  # captures the step's graph
    for _ in range(args.warmup): dec.graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(args.steps): dec.graph.replay()
    b.record(stream)
    b.synchronize()
  ms = a.elapsed_time(b) / args.steps
  tok_s = B * 1000.0 / ms
  kv_bytes = c.layers * 2 * c.kv * dec.hd * context * 2 * B
  step_bytes = dec.weight_bytes() + kv_bytes
  print(f"# step {ms:.3f} ms, {tok_s:.1f} tok/s, {step_bytes / 1e9:.3f} GB a step -> {step_bytes / ms / 1e6:.0f} GB/s", file=sys.stderr, flush=True)
  rates = gemv_rates(dec, stream)
  peaks = measured_peaks(dev)
  print(f"# measured on this GPU: HBM read {peaks['hbm_read_gbs']:.0f} GB/s, copy {peaks['hbm_copy_gbs']:.0f} GB/s (published "
        f"{HBM_PEAK / 1e9:.0f}); bf16 GEMM {peaks['bf16_gemm_tflops']:.0f} TFLOP/s (published dense {MFMA_PEAK / 1e12:.0f})",
        file=sys.stderr, flush=True)
  for k, r in rates.items():
    print(f"# gemv {k:8s} {r['fmt']} {r['K']}x{r['N']}: {r['us']:.2f} us, {r['gbs']:.0f} GB/s ({r['gbs'] * 1e9 / HBM_PEAK:.1%})", file=sys.stderr, flush=True)
  floor = read_floor(dev) if args.config == "c3" and B == 1 else None
  if floor: print("# read floor (32 distinct buffers a graph): " + ", ".join(f"{k} {v['us']:.2f} us" for k, v in floor.items()),
                  file=sys.stderr, flush=True)
  rates8 = None
  extra = {}
  if args.config == "c3" and B == 1:  # the target's own kernels: the 8B shapes with every matrix bfp8
    c8, mode8, _ = config("c3-bfp8")
    dec8 = G.Decoder(c8, G.random_weights(c8, seed=2, device=dev), mode=mode8, kv="bf16", batch=1, context=context)
    extra["decode_bfp8"] = step_rate(dec8, context, args.steps, args.warmup, stream)
    print(f"# {extra['decode_bfp8']['workload']}: {extra['decode_bfp8']['ms_per_step']:.3f} ms, "
          f"{extra['decode_bfp8']['tokens_per_s']:.1f} tok/s, {extra['decode_bfp8']['step_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    rates8 = gemv_rates(dec8, stream)
    for k, r8 in rates8.items():
      print(f"# gemv all-bfp8 {k:8s} {r8['fmt']} {r8['K']}x{r8['N']}: {r8['us']:.2f} us, {r8['gbs']:.0f} GB/s "
            f"({r8['gbs'] * 1e9 / HBM_PEAK:.1%})", file=sys.stderr, flush=True)
    del dec8
    torch.cuda.empty_cache()
  dom = max(rates, key=lambda k: rates[k]["us"] * (c.layers if k != "head" else 1))  # the most time in a step
  r = rates[dom]
  epi = {"qkv": "RMSNorm+RoPE+KV put", "o": "residual", "gate_up": "RMSNorm+SiLU*gate", "down": "residual", "head": "RMSNorm+argmax"}
  if args.config == "c3" and B == 1 and not args.no_prefill:
    extra["decode_bs16"] = decode_batch(dec, context)
    extra["decode_batches"] = {}
    for nb in (2, 4, 8):  # (2 on the GEMV, 4 and 8 on the matrix cores: Decoder's mfma_from)
      rb = decode_batch(dec, context, B=nb)
      extra["decode_batches"][str(nb)] = {"ms_per_step": rb["ms_per_step"], "tokens_per_s": rb["tokens_per_s"]}
    print("# decode at batch " + ", ".join(f"{nb}: {v['ms_per_step']:.3f} ms ({v['tokens_per_s']:.0f} tok/s)"
                                           for nb, v in extra["decode_batches"].items()), file=sys.stderr, flush=True)
    print(f"# {extra['decode_bs16']['workload']}: {extra['decode_bs16']['ms_per_step']:.3f} ms, "
          f"{extra['decode_bs16']['tokens_per_s']:.0f} tok/s, {extra['decode_bs16']['step_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    extra["moe"] = moe_rate()
    print(f"# {extra['moe']['workload']}: {extra['moe']['us']:.1f} us, {extra['moe']['gbs']:.0f} GB/s "
          f"({extra['moe']['frac']:.1%}), {extra['moe']['experts_touched']} experts touched", file=sys.stderr, flush=True)
    extra["moe_prompt"] = moe_rate(2048, reps=5)  # (a prompt's tokens: the group path, on the matrix cores)
    print(f"# {extra['moe_prompt']['workload']}: {extra['moe_prompt']['us']:.1f} us, {extra['moe_prompt']['tflops']:.0f} TFLOP/s "
          f"({extra['moe_prompt']['tflops'] * 1e12 / MFMA_PEAK:.1%} of {MFMA_PEAK / 1e15:.1f} PFLOP/s)", file=sys.stderr, flush=True)
  pre = None
  if not args.no_prefill and args.config == "c3":
    pre = prefill_rate()
    pre["mfma_frac_measured"] = round(pre["tflops"] / peaks["bf16_gemm_tflops"], 4)  # (of hipBLASLt's bf16 GEMM here)
    print(f"# prefill {pre['workload']}: {pre['ms']:.1f} ms, {pre['tokens_per_s']:.0f} tok/s, {pre['tflops']:.0f} TFLOP/s "
          f"({pre['mfma_frac']:.1%} of {MFMA_PEAK / 1e15:.1f} PFLOP/s); gemm {pre['gemm_tflops']}, attention {pre['attention_tflops']} TFLOP/s",
          file=sys.stderr, flush=True)
  configs = {}
  if args.config == "c3" and B == 1 and not args.no_prefill:  # configs 1 and 2 on the GPU, beside config 3
    configs["c1"] = config1_rate(dev)
    print(f"# {configs['c1']['workload']}: {configs['c1']['us']:.2f} us, {configs['c1']['gbs']:.0f} GB/s over "
          f"{configs['c1']['copies']} distinct weights ({configs['c1']['us_cache_resident']:.2f} us cache-resident)", file=sys.stderr, flush=True)
    configs["c2"] = config2_rate(dev)
    print(f"# {configs['c2']['workload']}: {configs['c2']['ms_per_step']:.3f} ms, {configs['c2']['tokens_per_s']:.0f} tok/s",
          file=sys.stderr, flush=True)
  cpu = None
  if not args.no_cpu:
    cpu = cpu_baseline(c, mode, context)
    print(f"# cpu baseline: {cpu['value']:.3f} tok/s on {cpu['cores']} cores (block {cpu['block_s']:.3f}s, head "
          f"{cpu['head_s']:.3f}s; {cpu['blas']}); one BLAS thread {cpu['one_thread_tokens_per_s']:.3f}, float32 "
          f"activations and cache {cpu['float32_tokens_per_s']:.3f} tok/s", file=sys.stderr)
    cpu = {k: (round(cpu[k], 4) if isinstance(cpu[k], float) else cpu[k])
           for k in ("value", "unit", "cores", "kind", "sample", "blas", "one_thread_tokens_per_s", "float32_tokens_per_s")}
    if args.config == "c3" and B == 1 and not args.no_prefill:
      for name, v in cpu_configs().items():
        configs.setdefault(name, {})["cpu"] = v | {"cores": cpu["cores"], "kind": "port"}
      print("# cpu baselines: " + "; ".join(f"{k} {v['cpu']}" for k, v in configs.items()), file=sys.stderr, flush=True)
  line = {
    "metric": "8B-shape bfp8 decode tok/s @bs1; GEMV HBM GB/s as % of peak",
    "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
    "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
    "dtype": "bfp8/bfp4 weights, fp32 math", "data": "synthetic (random-init weights, random bf16 KV cache)",
    "config": {"workload": f"config 3: Llama-3.1-8B-shape decode, batch {B}, context {context}, "
                           f"{'attention+head bfp8, MLP bfp4' if mode == 'experts' else 'all bfp8'}, bf16 KV",
               "global_batch": B, "seq_len": context, "parallelism": "none (1 GPU)"},
    "step_gbs": round(step_bytes / ms / 1e6, 1), "step_bytes": step_bytes,
    "roofline": {"bound": "hbm", "kernel": f"gemv {dom} + {epi[dom]} ({r['fmt']} {r['K']}x{r['N']})", "achieved": round(r["gbs"], 1),
                 "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(r["gbs"] * 1e9 / HBM_PEAK, 4),
                 "traffic": measured_traffic(dom, args.config, B),
                 "measured_peak": peaks["hbm_read_gbs"], "frac_measured": round(r["gbs"] / peaks["hbm_read_gbs"], 4)},
    "measured_peaks": peaks,
    "gemv_gbs": {k: round(v["gbs"], 1) for k, v in rates.items()},
    "gemv_us": {k: round(v["us"], 3) for k, v in rates.items()},
    "read_floor": floor,
    "gemv_of_floor": None if floor is None else {k: round(floor[f"{k} {rates[k]['fmt']}"]["us"] / rates[k]["us"], 3)
                                                 for k in ("qkv", "o", "gate_up", "down")},
    "gemv_bfp8_8b": None if rates8 is None else {k: {"us": round(v["us"], 3), "gbs": round(v["gbs"], 1),
                                                     "frac": round(v["gbs"] * 1e9 / HBM_PEAK, 4)} for k, v in rates8.items()},
    "cpu_baseline": cpu,
    "prefill": pre,
    "configs": configs,
    **extra,
  }
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
