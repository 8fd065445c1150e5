// A mixture of experts in the MLP's place (models/llama.py:277-300): the router and its top k, then the chosen
// experts' SwiGLUs weighted and summed.
//
// fh_moe_route: a workgroup a token row: RMSNorm of the row (if norm_w), the router's logits (fp32 sums of the row
// times the router's bf16 or fp32 columns, each thread a share of the router's rows), the k largest (the first of equals first,
// as numpy's stable argsort orders them, llama.py:27), and their weights (a softmax over the k, or the softmax over all
// taken at the k, as norm_topk says), written as ids and weights and as a dense [rows][experts] matrix of weights (0
// where a row did not pick an expert).
//
// fh_moe_experts: the experts of a decode step's few tokens (ferrite's dense path, Tensor.touched / chip_experts,
// llama.py:302-321, computes every picked expert for every row, weighted 0 where a row did not pick it; the sum is the
// same). Here each expert multiplies only its own rows: a first kernel writes the rows (normed when norm_w is given)
// as bf16 once and, from dense, each expert's list of the rows that picked it (in row order) with their weights;
// the skinny matrix-core kernel over (32 columns, expert) then takes gate_up for the expert's rows through the list,
// with the SiLU·gate epilogue scaled by the row's weight, into the expert's own bf16 rows, and down on those into the
// expert's own fp32 rows; a last kernel adds each row's experts in expert order (no atomics: the result does not
// depend on timing) onto the residual. An expert no row picked reads no weight.
#include <math.h>
#include "fh_epilogue.h"

namespace fh {

constexpr int RT_THREADS = 256;

// REG (dim a multiple of 16, at most 4096, x rows 16-byte aligned): a thread holds dimensions 16 t .. 16 t + 15 of the
// row in registers, each loaded once, and issues all its router rows of a group of 8 experts together; otherwise the
// row goes through LDS a dimension a thread at a time (a second pass of registers took every VGPR: the compiler hoists
// its loads over the first pass's arithmetic)
constexpr int RT_RUN = 16, RT_PASS = RT_THREADS * RT_RUN, RT_MAXP = 1;

template <bool RBF16, bool REG>
__global__ __launch_bounds__(RT_THREADS) void route_kernel(const float* x, int64_t ldx, int dim, const float* norm_w,
                                                           float eps, int centered, const void* router, int E, int k,
                                                           int norm_topk, int32_t* ids, float* wts, float* dense) {
  extern __shared__ float rt_smem[];   // [dim] the normed row (the generic path)
  __shared__ float logit_s[256];
  __shared__ float red_s[RT_THREADS / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  const int t = threadIdx.x;
  float* h = rt_smem;
  float hr[RT_MAXP][RT_RUN];  // (REG) this thread's dimensions, normed
  // the row, normed
  if constexpr (REG) {
    float s = 0.f;
#pragma unroll
    for (int p = 0; p < RT_MAXP; ++p) {
      const int c = p * RT_PASS + RT_RUN * t;
#pragma unroll
      for (int q = 0; q < RT_RUN / 4; ++q) {
        const float4 f = c < dim ? *(const float4*)(xr + c + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
        hr[p][4 * q] = f.x; hr[p][4 * q + 1] = f.y; hr[p][4 * q + 2] = f.z; hr[p][4 * q + 3] = f.w;
      }
#pragma unroll
      for (int j = 0; j < RT_RUN; ++j) s = fmaf(hr[p][j], hr[p][j], s);
    }
    if (norm_w) {
      s = wave_sum(s);
      if ((t & 63) == 0) red_s[t >> 6] = s;
      __syncthreads();
      float tot = 0.f;
      for (int w = 0; w < RT_THREADS / 64; ++w) tot += red_s[w];
      const float rs = 1.0f / sqrtf(tot / (float)dim + eps);
#pragma unroll
      for (int p = 0; p < RT_MAXP; ++p) {
        const int c = p * RT_PASS + RT_RUN * t;
        if (c >= dim) continue;
#pragma unroll
        for (int q = 0; q < RT_RUN / 4; ++q) {
          float4 g = *(const float4*)(norm_w + c + 4 * q);
          if (centered) { g.x += 1.f; g.y += 1.f; g.z += 1.f; g.w += 1.f; }
          hr[p][4 * q] *= rs * g.x; hr[p][4 * q + 1] *= rs * g.y; hr[p][4 * q + 2] *= rs * g.z; hr[p][4 * q + 3] *= rs * g.w;
        }
      }
    }
  } else {
    float rs = 1.f;
    if (norm_w) {
      float s = 0.f;
      for (int i = t; i < dim; i += RT_THREADS) s += xr[i] * xr[i];
      s = wave_sum(s);
      if ((t & 63) == 0) red_s[t >> 6] = s;
      __syncthreads();
      float tot = 0.f;
      for (int w = 0; w < RT_THREADS / 64; ++w) tot += red_s[w];
      rs = 1.0f / sqrtf(tot / (float)dim + eps);
    }
    for (int i = t; i < dim; i += RT_THREADS) {
      const float g = norm_w ? (centered ? norm_w[i] + 1.f : norm_w[i]) : 1.f;
      h[i] = norm_w ? xr[i] * rs * g : xr[i];
    }
    __syncthreads();
  }
  // logits, 8 experts at a time (a router row's 8 values one 16-byte load where the layout allows), then the
  // workgroup sums each expert's partials in a fixed order
  constexpr int EC = 8;
  __shared__ float part8[RT_THREADS / 64][EC];
  const bool wide = RBF16 && E % 8 == 0;
  auto weight = [&](int64_t d, int e) {
    return RBF16 ? bf16_to_f(((const uint16_t*)router)[d * E + e]) : ((const float*)router)[d * E + e];
  };
  for (int e0 = 0; e0 < E; e0 += EC) {
    float acc[EC];
#pragma unroll
    for (int j = 0; j < EC; ++j) acc[j] = 0.f;
    if constexpr (REG) {
      auto pass = [&](const float (&hv)[RT_RUN], int c) {  // a pass's 16 router rows in flight at once
        if (c >= dim) return;
        if (wide) {
          uint4 w[RT_RUN];
#pragma unroll
          for (int i = 0; i < RT_RUN; ++i) w[i] = *(const uint4*)((const uint16_t*)router + (int64_t)(c + i) * E + e0);
#pragma unroll
          for (int i = 0; i < RT_RUN; ++i) {
            const uint32_t ww[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc[2 * j] = fmaf(hv[i], __uint_as_float(ww[j] << 16), acc[2 * j]);
              acc[2 * j + 1] = fmaf(hv[i], __uint_as_float(ww[j] & 0xFFFF0000u), acc[2 * j + 1]);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < RT_RUN; ++i)
#pragma unroll
            for (int j = 0; j < EC; ++j) acc[j] = fmaf(hv[i], weight(c + i, min(e0 + j, E - 1)), acc[j]);
        }
      };
      static_assert(RT_MAXP == 1, "one pass");
      pass(hr[0], RT_RUN * t);
    } else {
#pragma unroll 4
      for (int i = t; i < dim; i += RT_THREADS) {
        const float hv = h[i];
        if (wide) {
          const uint4 w = *(const uint4*)((const uint16_t*)router + (int64_t)i * E + e0);
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[2 * j] = fmaf(hv, __uint_as_float(ww[j] << 16), acc[2 * j]);
            acc[2 * j + 1] = fmaf(hv, __uint_as_float(ww[j] & 0xFFFF0000u), acc[2 * j + 1]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < EC; ++j) acc[j] = fmaf(hv, weight(i, min(e0 + j, E - 1)), acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < EC; ++j) {
      const float v = wave_sum(acc[j]);
      if ((t & 63) == 0) part8[t >> 6][j] = v;
    }
    __syncthreads();
    if (t < EC && e0 + t < E) {
      float v = part8[0][t];
#pragma unroll
      for (int w = 1; w < RT_THREADS / 64; ++w) v += part8[w][t];
      logit_s[e0 + t] = v;
    }
    __syncthreads();
  }
  if (t == 0) {
    // softmax over all first when the k are not renormalised (their probabilities among all)
    if (!norm_topk) {
      float m = logit_s[0];
      for (int e = 1; e < E; ++e) m = fmaxf(m, logit_s[e]);
      float z = 0.f;
      for (int e = 0; e < E; ++e) z += expf(logit_s[e] - m);
      for (int e = 0; e < E; ++e) logit_s[e] = expf(logit_s[e] - m) / z;
    }
    // the k largest, the first of equals first
    float val[16];
    int idx[16];
    for (int j = 0; j < k; ++j) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        bool taken = false;
        for (int i = 0; i < j; ++i) taken |= idx[i] == e;
        if (!taken && (best < 0 || logit_s[e] > logit_s[best])) best = e;
      }
      idx[j] = best; val[j] = logit_s[best];
    }
    if (norm_topk) {  // softmax over the k (val[0] the largest)
      const float top = val[0];
      float z = 0.f;
      for (int j = 0; j < k; ++j) z += expf(val[j] - top);
      for (int j = 0; j < k; ++j) val[j] = expf(val[j] - top) / z;
    }
    for (int e = 0; e < E; ++e) dense[row * E + e] = 0.f;
    for (int j = 0; j < k; ++j) {
      ids[row * k + j] = idx[j];
      wts[row * k + j] = val[j];
      dense[row * E + idx[j]] = val[j];
    }
  }
}

// Blocks 0 .. n-1: row r of x as bf16 into xn (times 1 / rms from the sums of squares by runs of 16 and the RMSNorm
// weight, when norm_w is given). Block n: each expert's rows (thread e: the rows whose dense weight for e is not 0,
// in row order), their weights, the counts, and each row's slot in each expert's list (-1 where it did not pick it).
__global__ __launch_bounds__(256) void moe_prep_kernel(const float* x, int64_t ldx, int n, int dim, const float* norm_w,
                                                       const float* ssq_in, float eps, int centered, const float* dense,
                                                       int E, uint16_t* xn, int32_t* counts, int32_t* rows_of,
                                                       float* row_w, int32_t* slot) {
  __shared__ float red_s[4];
  __shared__ int wave_n[4];
  const int r = blockIdx.x, t = threadIdx.x;
  if (r == n) {  // each expert's rows in order: a thread a row, its place among the expert's by a workgroup count
    const int lane = t & 63, wave = t >> 6;
    for (int e = 0; e < E; ++e) {
      int base = 0;
      for (int i0 = 0; i0 < n; i0 += 256) {
        const int i = i0 + t;
        const float w = i < n ? dense[(int64_t)i * E + e] : 0.f;
        const uint64_t picked = __ballot(w != 0.f);
        const int before = __builtin_amdgcn_mbcnt_hi((uint32_t)(picked >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)picked, 0u));
        if (lane == 0) wave_n[wave] = __popcll(picked);
        __syncthreads();
        int off = base, total = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) { off += v < wave ? wave_n[v] : 0; total += wave_n[v]; }
        if (i < n) {
          const int c = off + before;
          if (w != 0.f) { rows_of[e * n + c] = i; row_w[e * n + c] = w; slot[i * E + e] = c; }
          else slot[i * E + e] = -1;
        }
        base += total;
        __syncthreads();  // (wave_n is rewritten next)
      }
      if (t == 0) counts[e] = base;
    }
    return;
  }
  float rs = 1.f;
  if (norm_w) {
    const int parts = dim / 16;
    float s = 0.f;
    for (int i = t; i < parts; i += 256) s += ssq_in[(int64_t)r * parts + i];
    s = wave_sum(s);
    if ((t & 63) == 0) red_s[t >> 6] = s;
    __syncthreads();
    rs = 1.0f / sqrtf((red_s[0] + red_s[1] + red_s[2] + red_s[3]) / (float)dim + eps);
  }
  for (int i = t; i < dim; i += 256) {
    float v = x[(int64_t)r * ldx + i];
    if (norm_w) v *= rs * (centered ? norm_w[i] + 1.f : norm_w[i]);
    xn[(int64_t)r * dim + i] = (uint16_t)bf16_rne_f(v);
  }
}

// y[row] = residual[row] + the row's experts' outputs (parts: each expert's own rows) in expert order, and y's sums of
// squares by 16 columns; a workgroup 256 columns of a row
__global__ __launch_bounds__(256) void moe_sum_kernel(const float* parts, const int32_t* slot, int experts, int n, int dim,
                                                      const float* residual, float* y, float* ssq_out) {
  const int64_t row = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  float v = 0.f;
  if (c < dim) {
    v = residual ? residual[row * dim + c] : 0.f;
    for (int e = 0; e < experts; ++e) {
      const int sl = slot[row * experts + e];
      if (sl >= 0) v += parts[((int64_t)e * n + sl) * dim + c];
    }
    y[row * dim + c] = v;
  }
  if (ssq_out) {  // (dim is a multiple of 64: a run of 16 is 16 neighbouring lanes, all in range)
    float s = v * v;
    s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
    if (c < dim && (c & 15) == 0) ssq_out[row * (dim / 16) + c / 16] = s;
  }
}

// A pass's workspace (n rows, E experts): counts [E], rows_of [E][n], row_w [E][n], slot [n][E], xn [n][dim] bf16,
// g [E][n][ffn] bf16, parts [E][n][dim] fp32, each region 256-byte aligned
struct MoeSpace { size_t counts, rows_of, row_w, slot, xn, g, parts, total; };
static MoeSpace moe_space(int64_t n, int64_t E, int64_t ffn, int64_t dim) {
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  MoeSpace m;
  m.counts = 0;
  m.rows_of = m.counts + up(E * 4);
  m.row_w = m.rows_of + up(E * n * 4);
  m.slot = m.row_w + up(E * n * 4);
  m.xn = m.slot + up(n * E * 4);
  m.g = m.xn + up(n * dim * 2);
  m.parts = m.g + up(E * n * ffn * 2);
  m.total = m.parts + up(E * n * dim * 4);
  return m;
}

}  // namespace fh

using namespace fh;

extern "C" int fh_moe_route(const float* x, int64_t ldx, int rows, int64_t dim, const float* norm_w, float eps,
                            int centered, const void* router, int router_dtype, int experts, int k, int norm_topk,
                            int32_t* ids, float* weights, float* dense, void* stream) {
  if (!x || !router || !ids || !weights || !dense) return fail(FH_EINVAL, "fh_moe_route: null pointer");
  if (rows < 1 || dim < 1 || ldx < dim) return fail(FH_EINVAL, "fh_moe_route: need rows, dim >= 1, ldx >= dim");
  if (experts < 1 || experts > 256 || k < 1 || k > 16 || k > experts) return fail(FH_EUNSUP, "fh_moe_route: 1 <= k <= 16, k <= experts <= 256");
  if (router_dtype != FH_F32 && router_dtype != FH_BF16) return fail(FH_EINVAL, "fh_moe_route: router is FH_F32 or FH_BF16");
  // (the register path for a decode step's rows, where each workgroup's latency is the time; many rows keep the lean
  // kernel, more of whose workgroups fit a CU)
  const bool reg = rows <= 512 && dim % RT_RUN == 0 && dim <= RT_MAXP * RT_PASS && ldx % 4 == 0 && !((uintptr_t)x & 15) &&
                   !((uintptr_t)norm_w & 15) && !((uintptr_t)router & 15);
  const size_t lds = reg ? 0 : (size_t)dim * sizeof(float);
  if (lds > 120 * 1024) return fail(FH_EUNSUP, "fh_moe_route: row too long");
  hipStream_t s = as_stream(stream);
  const dim3 g(rows), b(RT_THREADS);
  if (router_dtype == FH_BF16 && reg) hipLaunchKernelGGL((route_kernel<true, true>), g, b, lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  else if (router_dtype == FH_BF16) hipLaunchKernelGGL((route_kernel<true, false>), g, b, lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  else if (reg) hipLaunchKernelGGL((route_kernel<false, true>), g, b, lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  else hipLaunchKernelGGL((route_kernel<false, false>), g, b, lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  return check_launch("fh_moe_route");
}

// Rows a pass: up to 64 rows (a decode step's), one pass through the skinny kernel, each touched expert's weight read
// once; past 64 (a prompt's), passes through the tiled GEMM, an expert's weight read once for every 128 of its rows
// (models/llama.py:314-329: the touched path for a decode step, the group path past it; the reference turns at 128
// tokens, here the tiled GEMM is already faster from 65: 560 us against 680 for two skinny passes at the Mixtral
// shape). A pass's workspace holds each expert's whole pass of rows (a `dense` may pick every expert for a row), so a
// pass is the most rows, a power of 2 from 2048 down to 128, whose workspace fits MOE_BUDGET: 2048 at the Mixtral
// shape (~740 MB; 13% faster at 2048 tokens than passes of 1024), 128 for 256 experts of 2048 x 7168.
constexpr int64_t MOE_BUDGET = (int64_t)1 << 30;
static int64_t moe_pass(int64_t rows, int64_t experts, int64_t ffn, int64_t dim) {
  if (rows <= 64) return 64;
  int64_t p = 2048;
  while (p > 128 && (int64_t)moe_space(p, experts, ffn, dim).total > MOE_BUDGET) p /= 2;
  return p;
}

extern "C" size_t fh_moe_workspace_bytes(int rows, int experts, int64_t ffn, int64_t dim) {
  if (rows < 1 || experts < 1 || ffn < 1 || dim < 1) return 0;
  const int64_t pass = moe_pass(rows, experts, ffn, dim);
  const int64_t r = rows < pass ? rows : pass;  // a pass's rows
  if (r < 1 || experts < 1 || ffn < 1 || dim < 1) return 0;
  return moe_space(r, experts, ffn, dim).total;
}

extern "C" int fh_moe_experts(const float* x, int64_t ldx, int rows, int64_t dim, const float* norm_w, const float* ssq_in,
                              float eps, int centered, int experts, int64_t ffn, const void* gu_mant, const uint8_t* gu_exps,
                              int gu_fmt, const void* down_mant, const uint8_t* down_exps, int down_fmt, const float* dense,
                              float* y, const float* residual, float* ssq_out, void* workspace, size_t ws_bytes,
                              void* stream) {
  if (!x || !gu_mant || !gu_exps || !down_mant || !down_exps || !dense || !y || !workspace)
    return fail(FH_EINVAL, "fh_moe_experts: null pointer");
  if (rows < 1 || dim < 64 || dim % 64 || ffn < 64 || ffn % 64 || ldx < dim) return fail(FH_EINVAL, "fh_moe_experts: need dim and ffn multiples of 64");
  if (experts < 1 || experts > 256) return fail(FH_EUNSUP, "fh_moe_experts: at most 256 experts");
  if ((gu_fmt != FH_BFP8 && gu_fmt != FH_BFP4) || (down_fmt != FH_BFP8 && down_fmt != FH_BFP4)) return fail(FH_EINVAL, "fh_moe_experts: weights are FH_BFP8 or FH_BFP4");
  if (norm_w && !ssq_in) return fail(FH_EINVAL, "fh_moe_experts: the RMSNorm prologue needs ssq_in");
  if (ws_bytes < fh_moe_workspace_bytes(rows, experts, ffn, dim)) return fail(FH_EINVAL, "fh_moe_experts: workspace too small");
  hipStream_t s = as_stream(stream);
  const int64_t gu_n = 2 * ffn;
  size_t mb, eb;
  if (int rc = fh_bfp_bytes(dim, gu_n, gu_fmt, FH_AXIS_N, &mb, &eb)) return rc;
  size_t dmb, deb;
  if (int rc = fh_bfp_bytes(ffn, dim, down_fmt, FH_AXIS_N, &dmb, &deb)) return rc;
  const int pass = (int)moe_pass(rows, experts, ffn, dim);
  for (int r0 = 0; r0 < rows; r0 += pass) {
    const int n = rows - r0 < pass ? rows - r0 : pass;
    const MoeSpace m = moe_space(n, experts, ffn, dim);
    char* w = (char*)workspace;
    int32_t* counts = (int32_t*)(w + m.counts);
    int32_t* rows_of = (int32_t*)(w + m.rows_of);
    float* row_w = (float*)(w + m.row_w);
    int32_t* slot = (int32_t*)(w + m.slot);
    uint16_t* xn = (uint16_t*)(w + m.xn);
    uint16_t* g = (uint16_t*)(w + m.g);          // [experts][n][ffn]
    float* parts = (float*)(w + m.parts);        // [experts][n][dim]
    hipLaunchKernelGGL(moe_prep_kernel, dim3(n + 1), dim3(256), 0, s, x + (int64_t)r0 * ldx, ldx, n, (int)dim, norm_w,
                       ssq_in ? ssq_in + (int64_t)r0 * (dim / 16) : nullptr, eps, centered, dense + (int64_t)r0 * experts,
                       experts, xn, counts, rows_of, row_w, slot);
    // gate_up of each expert on its rows: silu(gate) * up * the row's weight
    MatArgs a = {};
    fh_epilogue ep = {};
    ep.kind = FH_EP_SILU_GATE; ep.split = (int)ffn;
    a.x = xn; a.ldx = dim; a.x_bf16 = 1;
    a.mant = (const uint8_t*)gu_mant; a.exps = gu_exps; a.K = dim; a.N = gu_n; a.M = n;
    a.y = g; a.y_bf16 = 1;
    if (int rc = epilogue_args("fh_moe_experts", &ep, dim, gu_n, FH_BF16, ffn, a)) return rc;
    a.ldy = ffn;
    SkinnyMoe moe = {};
    moe.expert_mant = (int64_t)mb; moe.expert_exps = (int64_t)eb; moe.experts = experts; moe.scale_rows = 1;
    moe.counts = counts; moe.x_rows = rows_of; moe.row_w = row_w;
    if (int rc = n > 64 ? gemm_tiles(a, moe, gu_fmt, experts, s) : skinny_matmul(a, moe, gu_fmt, experts, s)) return rc;
    // down, each expert on its own rows of g
    MatArgs d = {};
    fh_epilogue de = {};
    de.kind = FH_EP_STORE;
    d.x = g; d.ldx = ffn; d.x_bf16 = 1;
    d.mant = (const uint8_t*)down_mant; d.exps = down_exps; d.K = ffn; d.N = dim; d.M = n;
    d.y = parts; d.y_bf16 = 0;
    if (int rc = epilogue_args("fh_moe_experts", &de, ffn, dim, FH_F32, dim, d)) return rc;
    d.ldy = dim;
    SkinnyMoe dm = {};
    dm.expert_mant = (int64_t)dmb; dm.expert_exps = (int64_t)deb; dm.experts = experts; dm.scale_rows = 0;
    dm.counts = counts;
    if (int rc = n > 64 ? gemm_tiles(d, dm, down_fmt, experts, s) : skinny_matmul(d, dm, down_fmt, experts, s)) return rc;
    hipLaunchKernelGGL(moe_sum_kernel, dim3(n, (unsigned)((dim + 255) / 256)), dim3(256), 0, s, parts, slot, experts, n,
                       (int)dim, residual ? residual + (int64_t)r0 * dim : nullptr, y + (int64_t)r0 * dim,
                       ssq_out ? ssq_out + (int64_t)r0 * (dim / 16) : nullptr);
    if (int rc = check_launch("fh_moe_experts")) return rc;
  }
  return FH_OK;
}
