// Decode GEMV by a block-float weight: y = epilogue(prologue(x) @ W), batch 1..8 rows per launch, W packed along N
// (FH_AXIS_N: 16 columns of a row share an exponent, the layout [N/16][K][16]).
//
// A workgroup takes one item (one run of 16 columns, or two paired runs: RoPE's halves of a head, SwiGLU's gate and up)
// and its W waves split the K rows into W slices. A lane takes one row k of a run at a time: one 16-byte load of the
// 16 magnitudes (8 bytes for bfp4), the exponent byte and the row's x values, then for each batch row x scaled by the
// block's 2^(e - 133) (exact) and 16 FMAs, each bfp8 magnitude converted by one sign-extending byte convert (bfp4's
// two a conversion through the fp8 converter, offset by 8: magnitudes_off8). A wave's 64
// lanes read 64 consecutive rows, 1 KiB contiguous (512 B for bfp4), and keep U such loads in flight. The lanes'
// partial sums are reduced across the wave by lane swaps and DPP moves (no LDS), across the waves through LDS in a
// fixed order (results do not depend on timing), and the epilogue runs on the workgroup's outputs. Few registers
// (about 60 a lane at batch 1) keep ~32 waves on every CU, each with its loads in flight: a decode GEMV is a
// latency-bound stream, and that is what hides the latency. Nothing crosses workgroups: no atomics, no fences.
#include <math.h>
#include <algorithm>
#include <type_traits>
#include "fh_epilogue.h"

namespace fh {

// rows a lane has in flight at once, by format and batch rows (about 4 KiB of weight a wave and run at batch 1)
__host__ __device__ constexpr int gemv_group(bool four, int b, int p) { return (b <= 2 ? 4 : b <= 4 ? 2 : 1) * (four ? 2 : 1) + 0 * p; }

// threads a workgroup at most: 16 waves for one row, 8 for more (whose partial sums need the registers)
__host__ __device__ constexpr int gemv_threads(int b) { return b == 1 ? 1024 : 512; }

// The first arguments are what the stream's first loads need, passed apart from MatArgs so that they arrive in
// SGPRs with the wave (kernel-argument preloading, -amdgpu-kernarg-preload-count): the loads go out without waiting
// for the argument buffer (~0.6 us a launch measured on MI355X, in graphs of back-to-back launches).
template <bool FOUR, int B, int P, bool NORM>
__global__ __launch_bounds__(gemv_threads(B)) void gemv_kernel(const uint8_t* __restrict__ mant, const uint8_t* __restrict__ exps,
                                                              const float* __restrict__ xf, const float* __restrict__ norm_w,
                                                              int K, int rows, int ldx, int pair_half, MatArgs a) {
  constexpr int V = B * P * 16;       // a lane's partial sums: [b][p][j]
  constexpr int G = B * P;
  constexpr int U = gemv_group(FOUR, B, P);
  constexpr int RB = FOUR ? 8 : 16;   // bytes of a run's row
  using Row = typename std::conditional<FOUR, uint2, uint4>::type;
  const int lane = threadIdx.x & 63;
  const int slice = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6, item = blockIdx.x;
  int64_t nb[P];
  if (P == 1) nb[0] = item;
  else { nb[0] = pair_first(item, pair_half); nb[P - 1] = nb[0] + pair_half; }
  const int r0 = slice * rows, r1 = min(K, r0 + rows);  // (the host keeps K below 2^27)

  const uint8_t* mb[P];
  const uint8_t* eb[P];
#pragma unroll
  for (int p = 0; p < P; ++p) { mb[p] = mant + nb[p] * K * RB; eb[p] = exps + nb[p] * K; }

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;

  // what wave 0's epilogue reads, loaded once the first weight loads are out (their addresses need only the preloaded
  // arguments, these the argument buffer) so that the loads overlap the stream: the sums of squares (up to 256 runs a
  // row, K <= 4096; a longer row is read at the end) and each row's place
  constexpr int PRE = 4;
  float ssq_pre[B][PRE];
  int place_pre[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    place_pre[b] = 0;
#pragma unroll
    for (int i = 0; i < PRE; ++i) ssq_pre[b][i] = 0.f;
  }
  auto prefetch = [&]() {
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
      for (int i = 0; i < PRE; ++i) {
        const int at = lane + 64 * i;
        ssq_pre[b][i] = (a.ssq_in && a.ssq_parts <= 64 * PRE && at < a.ssq_parts) ? a.ssq_in[(int64_t)b * a.ssq_parts + at] : 0.f;
      }
      place_pre[b] = a.places ? (int)rope_place(a, a.places[b]) : 0;
    }
  };

  // U rows of each run, 64 apart, a lane; rows past r1 are read at r1 - 1 (they exist) and count as 0. The first
  // group's loads go out before anything reads the argument buffer: their addresses need only the preloaded arguments
  Row m[U][P];
  int e[U][P];
  float xv[U][B], g[U];
  auto load_group = [&](int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(k0 + 64 * u + lane, r1 - 1);
#pragma unroll
      for (int p = 0; p < P; ++p) { m[u][p] = *(const Row*)(mb[p] + (uint32_t)k * RB); e[u][p] = eb[p][k]; }
      if (NORM) g[u] = norm_w[k];
#pragma unroll
      for (int b = 0; b < B; ++b) xv[u][b] = xf[b * ldx + k];
    }
  };
  // bfp4: each value as (q + 8) 2^-9 (magnitudes_off8), its row's scale x 2^(e - 120) so that the products are
  // x (q + 8) 2^(e - 129); the 8 comes back out at the end, the lane's sum of its rows' scales times 2^-6 off each of
  // the run's 16 sums (exact products either way, the sums' rounding of the same order)
  float off[B * P];
#pragma unroll
  for (int i = 0; i < B * P; ++i) off[i] = 0.f;
  auto compute = [&](int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = k0 + 64 * u + lane < r1;
      float gw = 1.f;
      if (NORM) gw = a.centered ? g[u] + 1.f : g[u];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float f[16];
        if constexpr (FOUR) magnitudes_off8(m[u][p], f);
        else magnitudes(m[u][p], f);
        float xs[B];
#pragma unroll
        for (int b = 0; b < B; ++b) xs[b] = ok ? ldexpf(xv[u][b] * gw, e[u][p] - (FOUR ? 120 : 133)) : 0.f;
        if constexpr (FOUR) {
#pragma unroll
          for (int b = 0; b < B; ++b) off[b * P + p] += xs[b];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
          for (int b = 0; b < B; ++b) acc[(b * P + p) * 16 + j] = fmaf(xs[b], f[j], acc[(b * P + p) * 16 + j]);
      }
    }
  };
  if (r0 < r1) {  // the first group apart: its loads, then wave 0's reads of the argument buffer, then its arithmetic
    load_group(r0);
    __builtin_amdgcn_sched_barrier(0);
    if (slice == 0) prefetch();
    __builtin_amdgcn_sched_barrier(0);
    compute(r0);
  } else if (slice == 0) {
    prefetch();
  }
  for (int k0 = r0 + 64 * U; k0 < r1; k0 += 64 * U) {
    load_group(k0);
    __builtin_amdgcn_sched_barrier(0);  // every load above in flight before any arithmetic
    compute(k0);
  }

  if constexpr (FOUR) {  // the offset's products out: 8 2^-9 times the scales' sum
#pragma unroll
    for (int i = 0; i < B * P; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[i * 16 + j] = fmaf(off[i], -0.015625f, acc[i * 16 + j]);
  }
  // each run of 16 across the wave: lane holds the sum of value reduce16_index(lane) of each group in sums[g]
  float sums[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float r16[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) r16[j] = acc[gi * 16 + j];
    wave_reduce16(r16);
    sums[gi] = r16[0];
  }
  const int j16 = reduce16_index(lane);
  __shared__ float red[gemv_threads(B) / 64][V];
  __shared__ float fin[V];
  if ((lane & 3) == 0) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) red[slice][gi * 16 + j16] = sums[gi];
  }
  __syncthreads();
  if (slice != 0) return;  // wave 0 adds the slices in order and runs the epilogue
  for (int i = lane; i < V; i += 64) {
    float t = red[0][i];
    for (int w = 1; w < W; ++w) t += red[w][i];
    fin[i] = t;
  }
  // each batch row's 1 / rms, from the sums of squares its maker left by runs of 16
  float rs[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    rs[b] = 1.f;
    if (a.ssq_in) {  // (NORM, or rows that already hold x * w)
      float s = 0.f;
      if (a.ssq_parts <= 64 * PRE) {
#pragma unroll
        for (int i = 0; i < PRE; ++i) s += ssq_pre[b][i];
      } else {
        for (int i = lane; i < a.ssq_parts; i += 64) s += a.ssq_in[(int64_t)b * a.ssq_parts + i];
      }
      s = wave_sum(s);
      rs[b] = 1.0f / sqrtf(s / (float)K + a.eps);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

  // the epilogue, a lane an output (or a pair of them)
  const int kind = a.kind;
  if (kind == FH_EP_PROGRAM) {  // (a loop of its own: the program's decoding, hoisted out of the loop, runs only here)
    for (int i = lane; i < V; i += 64) {
      const int b = i / (P * 16), p = (i / 16) % P, j = i % 16;
      const int64_t col = nb[p] * 16 + j;
      store_out(a.y, a.y_bf16, b * a.ldy + col, prog_eval(a.prog, fin[i] * rs[b], 0, a.row_base + b, col));
    }
  } else if (kind == FH_EP_STORE || kind == FH_EP_RESIDUAL) {
    for (int i = lane; i < V; i += 64) {  // (V is a multiple of 16: a run's 16 values are 16 neighbouring lanes)
      const int b = i / (P * 16), p = (i / 16) % P, j = i % 16;
      const int64_t col = nb[p] * 16 + j, at = b * a.ldy + col;
      float v = fin[i] * rs[b];
      if (kind == FH_EP_RESIDUAL) v += a.residual[at];
      store_out(a.y, a.y_bf16, at, v);
      if (kind == FH_EP_RESIDUAL && a.copy_bf16) put_copy(a, a.copy_tiles ? a.row_base + b : b, col, v);  // (tiles: rows from the call's first)
      if (kind == FH_EP_RESIDUAL && a.ssq_out) {
        float s = v * v;
        s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
        if (j == 0) a.ssq_out[(int64_t)b * (a.N / 16) + nb[p]] = s;
      }
      if (kind == FH_EP_STORE && a.argmax_parts) {  // the run's largest and its first column
        float bv = v;
        int bc = (int)col;
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) {
          const float ov = __shfl_xor(bv, m, 64);
          const int oc = __shfl_xor(bc, m, 64);
          if (ov > bv || (ov == bv && oc < bc)) { bv = ov; bc = oc; }
        }
        if (j == 0) a.argmax_parts[(int64_t)b * (a.N / 16) + nb[p]] = make_int2(__float_as_int(bv), bc);
      }
    }
  } else if (P == 2 && kind == FH_EP_SILU_GATE) {
    for (int i = lane; i < B * 16; i += 64) {
      const int b = i / 16, j = i % 16;
      const float r = rs[b];
      const float gv = fin[(b * P) * 16 + j] * r, uv = fin[(b * P + 1) * 16 + j] * r;
      store_out(a.y, a.y_bf16, b * a.ldy + nb[0] * 16 + j, silu(gv) * uv);
    }
  } else if (P == 2 && kind == FH_EP_ROPE_KV) {
    const int hd = a.head_dim;
    for (int i = lane; i < B * 16; i += 64) {
      const int b = i / 16, j = i % 16;
      const int64_t c0 = nb[0] * 16 + j;            // in the first half of its head
      const int h = (int)c0 / hd, d = (int)c0 % hd, d1 = d + hd / 2;  // (c0 < N < 2^31)
      const float r = rs[b];
      float x0 = fin[(b * P) * 16 + j] * r, x1 = fin[(b * P + 1) * 16 + j] * r;
      int place = place_pre[0];
#pragma unroll
      for (int q = 1; q < B; ++q) if (b == q) place = place_pre[q];
      if (h < a.heads + a.kv_heads) {  // q's and k's heads turn: x cos + (-x2, x1) sin (models/llama.py:92-93)
        const float* cs = a.cos_tab + (int64_t)place * hd;
        const float* sn = a.sin_tab + (int64_t)place * hd;
        const float t0 = x0 * cs[d] - x1 * sn[d], t1 = x1 * cs[d1] + x0 * sn[d1];
        x0 = t0; x1 = t1;
      }
      if (h < a.heads) {
        float* q = (float*)a.y + b * a.ldy + (int64_t)h * hd;
        q[d] = x0; q[d1] = x1;
      } else {  // keys' heads then values' heads, each at the row's cache row
        const int ch = h - a.heads;  // 0 .. 2 kv_heads - 1
        cache_put(a, ch, a.cache_rows[b], d, d1, j, x0, x1);
      }
    }
  }
}

template <bool FOUR, int B, int P>
static void launch(const MatArgs& a, int items, int W, hipStream_t s) {
  const dim3 g(items), t(64 * W);
  const float* x = (const float*)a.x;
  if (a.norm_w) hipLaunchKernelGGL((gemv_kernel<FOUR, B, P, true>), g, t, 0, s, a.mant, a.exps, x, a.norm_w, (int)a.K, a.rows, (int)a.ldx, a.pair_half, a);
  else hipLaunchKernelGGL((gemv_kernel<FOUR, B, P, false>), g, t, 0, s, a.mant, a.exps, x, a.norm_w, (int)a.K, a.rows, (int)a.ldx, a.pair_half, a);
}

template <bool FOUR, int P>
static int dispatch_batch(const MatArgs& a, int batch, int items, int W, hipStream_t s) {
  switch (batch) {
    case 1: launch<FOUR, 1, P>(a, items, W, s); break;
    case 2: launch<FOUR, 2, P>(a, items, W, s); break;
    case 3: launch<FOUR, 3, P>(a, items, W, s); break;
    case 4: launch<FOUR, 4, P>(a, items, W, s); break;
    default:
      if (P == 1) {
        switch (batch) {
          case 5: launch<FOUR, 5, 1>(a, items, W, s); break;
          case 6: launch<FOUR, 6, 1>(a, items, W, s); break;
          case 7: launch<FOUR, 7, 1>(a, items, W, s); break;
          case 8: launch<FOUR, 8, 1>(a, items, W, s); break;
          default: return fail(FH_EUNSUP, "gemv: more than 8 rows in one launch");
        }
      } else {
        return fail(FH_EUNSUP, "gemv: more than 4 rows in one paired launch");
      }
  }
  return FH_OK;
}

// The K slices: W waves a workgroup, the least power of 2 giving about 16384 waves in all (64 a CU on 256 CUs, in
// turns), at most one a group of U loads of 64 rows a lane, at most 8 for more than one row (their launch bound is 512
// threads, so that the rows' partial sums stay in registers: bound to 1024 threads they spilled, and batch 8 of an 8B
// step took 35.6 ms instead of 6.5), and at most 16 for bfp4 and 8 for bfp8 at one row: a bfp8 wave needs
// ~100 registers at two runs an item, so a 16-wave workgroup fills a CU alone and the grid runs in lock-step rounds
// (on MI355X: the 8B shapes' bfp8 gate_up 31.7 us at 16, 25.9 at 8; bfp4's down 11.0 at 16, 11.4 at 8).
struct Plan { int W, rows, P, most, items; };
static Plan plan(int64_t K, int64_t N, int fmt, int kind, int batch) {
  Plan p;
  p.P = (kind == FH_EP_SILU_GATE || kind == FH_EP_ROPE_KV) ? 2 : 1;  // as epilogue_args sets MatArgs::P
  p.most = p.P == 1 ? 8 : 4;
  p.items = (int)(N / 16 / p.P);
  const int b = batch < p.most ? batch : p.most;
  const int unit = 64 * gemv_group(fmt == FH_BFP4, b, p.P);
  const int64_t units = (K + unit - 1) / unit;
  const int64_t most = std::min<int64_t>(fmt == FH_BFP4 ? 16 : 8, gemv_threads(b) / 64);  // (measured: bfp8's 16-wave
                                                                                           // workgroups run in lock-step rounds)
  int64_t W = 1;
  while (W < most && W * p.items < 16384) W *= 2;
  while (W > 1 && W > units) W /= 2;
  int64_t rows = (K + W - 1) / W;
  rows = (rows + 63) / 64 * 64;
  p.W = (int)((K + rows - 1) / rows);
  p.rows = (int)rows;
  return p;
}

}  // namespace fh

using namespace fh;

extern "C" int fh_gemv_bfp(const void* x, int x_dtype, int64_t ldx, int batch, int64_t K, int64_t N, const void* w_mant,
                           const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy,
                           void* stream) {
  if (!x || !w_mant || !w_exps || !y) return fail(FH_EINVAL, "fh_gemv_bfp: null pointer");
  if (batch < 1 || K < 1 || N < 16 || N % 16) return fail(FH_EINVAL, "fh_gemv_bfp: need batch >= 1, K >= 1, N a multiple of 16");
  if (x_dtype != FH_F32) return fail(FH_EUNSUP, "fh_gemv_bfp: x is FH_F32 (activations stay fp32 between kernels)");
  if (y_dtype != FH_F32 && y_dtype != FH_BF16) return fail(FH_EINVAL, "fh_gemv_bfp: y is FH_F32 or FH_BF16");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_gemv_bfp: fmt is FH_BFP8 or FH_BFP4");
  if (ldx < K) return fail(FH_EINVAL, "fh_gemv_bfp: ldx < K");
  if (K >= (1LL << 27) || (int64_t)batch * ldx >= (1LL << 31)) return fail(FH_EUNSUP, "fh_gemv_bfp: K or x too large for 32-bit row offsets");
  MatArgs a = {};
  a.x = x; a.ldx = ldx;
  a.mant = (const uint8_t*)w_mant; a.exps = w_exps; a.K = K; a.N = N; a.M = batch;
  a.y = y; a.y_bf16 = y_dtype == FH_BF16; a.ldy = ldy;
  if (int rc = epilogue_args("fh_gemv_bfp", ep, K, N, y_dtype, ldy, a)) return rc;
  const Plan p = plan(K, N, fmt, a.kind, batch);
  a.rows = p.rows;
  hipStream_t s = as_stream(stream);
  const bool four = fmt == FH_BFP4;
  for (int b0 = 0; b0 < batch; b0 += p.most) {  // more rows than a launch takes: several launches, each reading W again
    const int n = batch - b0 < p.most ? batch - b0 : p.most;
    MatArgs c = a;
    c.row_base = b0;
    c.x = (const char*)x + (size_t)b0 * ldx * 4;
    c.y = (char*)y + (size_t)b0 * ldy * (a.y_bf16 ? 2 : 4);
    if (c.ssq_in) c.ssq_in += (int64_t)b0 * c.ssq_parts;
    if (c.residual) c.residual += (int64_t)b0 * ldy;
    if (c.copy_bf16 && !c.copy_tiles) c.copy_bf16 += (int64_t)b0 * N;
    if (c.ssq_out) c.ssq_out += (int64_t)b0 * (N / 16);
    if (c.places) { c.places += b0; c.cache_rows += b0; }
    if (c.argmax_parts) c.argmax_parts += (int64_t)b0 * (N / 16);
    int rc = p.P == 1 ? (four ? dispatch_batch<true, 1>(c, n, p.items, p.W, s) : dispatch_batch<false, 1>(c, n, p.items, p.W, s))
                      : (four ? dispatch_batch<true, 2>(c, n, p.items, p.W, s) : dispatch_batch<false, 2>(c, n, p.items, p.W, s));
    if (rc) return rc;
    if ((rc = check_launch("fh_gemv_bfp"))) return rc;
  }
  return FH_OK;
}
