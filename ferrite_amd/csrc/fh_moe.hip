// A mixture of experts in the MLP's place (models/llama.py:277-300): the router and its top k, then the chosen
// experts' SwiGLUs weighted and summed.
//
// fh_moe_route: a workgroup a token row: RMSNorm of the row (if norm_w), the router's logits (fp32 sums of the row
// times the router's bf16 or fp32 columns, the threads splitting the row), the k largest (the first of equals first,
// as numpy's stable argsort orders them, llama.py:27), and their weights (a softmax over the k, or the softmax over all
// taken at the k, as norm_topk says), written as ids and weights and as a dense [rows][experts] matrix of weights (0
// where a row did not pick an expert).
//
// fh_moe_experts: ferrite's dense path for a decode step's few tokens (Tensor.touched, chip_experts: every expert some
// row picked takes every row, weighted by each row's weight, 0 where it did not pick it; llama.py:302-321): the skinny
// matrix-core kernel over (32 columns, expert) for gate_up with the SiLU·gate epilogue scaled by the row's weight into
// a [rows][experts * ffn] bf16 workspace, then for down into [rows][experts * dim] fp32, and a last kernel sums the
// experts in expert order (no atomics: the result does not depend on timing) onto the residual. An expert no row
// picked reads no weight and leaves zeros.
#include <math.h>
#include "fh_epilogue.h"

namespace fh {

constexpr int RT_THREADS = 256;

template <bool RBF16>
__global__ __launch_bounds__(RT_THREADS) void route_kernel(const float* x, int64_t ldx, int dim, const float* norm_w,
                                                           float eps, int centered, const void* router, int E, int k,
                                                           int norm_topk, int32_t* ids, float* wts, float* dense) {
  extern __shared__ float rt_smem[];   // [dim] the normed row, then [parts][E] partial logits
  __shared__ float logit_s[256];
  __shared__ float red_s[RT_THREADS / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  const int t = threadIdx.x;
  float* h = rt_smem;
  // the row, normed
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
  // logits: thread t takes expert t % E over part t / E of the row
  const int parts = RT_THREADS / E;
  float* partial = h + dim;
  if (t < parts * E) {
    const int e = t % E, p = t / E;
    const int per = (dim + parts - 1) / parts, k0 = p * per, k1 = min(dim, k0 + per);
    float s = 0.f;
    for (int i = k0; i < k1; ++i) {
      const float w = RBF16 ? bf16_to_f(((const uint16_t*)router)[(int64_t)i * E + e]) : ((const float*)router)[(int64_t)i * E + e];
      s += h[i] * w;
    }
    partial[p * E + e] = s;
  }
  __syncthreads();
  if (t < E) {
    float s = 0.f;
    for (int p = 0; p < parts; ++p) s += partial[p * E + t];
    logit_s[t] = s;
  }
  __syncthreads();
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

// y[row] = residual[row] + the experts' outputs summed in expert order, and y's sums of squares by 16 columns
__global__ __launch_bounds__(256) void moe_sum_kernel(const float* parts, int experts, int dim, const float* residual,
                                                      float* y, float* ssq_out) {
  const int64_t row = blockIdx.x;
  for (int n0 = 0; n0 < dim; n0 += 256) {
    const int n = n0 + threadIdx.x;
    float v = 0.f;
    if (n < dim) {
      v = residual ? residual[row * dim + n] : 0.f;
      for (int e = 0; e < experts; ++e) v += parts[(row * experts + e) * dim + n];
      y[row * dim + n] = v;
    }
    if (ssq_out) {  // (dim is a multiple of 64: a run of 16 is 16 neighbouring lanes, all in range)
      float s = v * v;
      s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
      if (n < dim && (n & 15) == 0) ssq_out[row * (dim / 16) + n / 16] = s;
    }
  }
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
  const int parts = RT_THREADS / experts;
  const size_t lds = ((size_t)dim + (size_t)parts * experts) * sizeof(float);
  if (lds > 120 * 1024) return fail(FH_EUNSUP, "fh_moe_route: row too long");
  hipStream_t s = as_stream(stream);
  if (router_dtype == FH_BF16)
    hipLaunchKernelGGL((route_kernel<true>), dim3(rows), dim3(RT_THREADS), lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  else
    hipLaunchKernelGGL((route_kernel<false>), dim3(rows), dim3(RT_THREADS), lds, s, x, ldx, (int)dim, norm_w, eps, centered, router, experts, k, norm_topk, ids, weights, dense);
  return check_launch("fh_moe_route");
}

extern "C" size_t fh_moe_workspace_bytes(int rows, int experts, int64_t ffn, int64_t dim) {
  const int64_t r = rows < 64 ? rows : 64;  // a pass: its gate_up outputs (bf16) and its experts' down outputs (fp32)
  return (size_t)(r > 0 ? r : 0) * experts * (ffn * 2 + dim * 4);
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
  for (int r0 = 0; r0 < rows; r0 += 64) {  // 64 rows a pass
    const int n = rows - r0 < 64 ? rows - r0 : 64;
    uint16_t* g = (uint16_t*)workspace;                                   // [n][experts * ffn] bf16
    float* parts = (float*)((char*)workspace + (size_t)n * experts * ffn * 2);  // [n][experts * dim]
    // gate_up of every picked expert: silu(gate) * up * the row's weight
    MatArgs a = {};
    fh_epilogue ep = {};
    ep.kind = FH_EP_SILU_GATE; ep.split = (int)ffn; ep.norm_w = norm_w; ep.ssq_in = ssq_in ? ssq_in + (int64_t)r0 * (dim / 16) : nullptr;
    ep.eps = eps; ep.centered = centered;
    a.x = x + (int64_t)r0 * ldx; a.ldx = ldx; a.x_bf16 = 0;
    a.mant = (const uint8_t*)gu_mant; a.exps = gu_exps; a.K = dim; a.N = gu_n; a.M = n;
    a.y = g; a.y_bf16 = 1;
    if (int rc = epilogue_args("fh_moe_experts", &ep, dim, gu_n, FH_BF16, ffn, a)) return rc;
    a.ldy = (int64_t)experts * ffn;
    SkinnyMoe moe = {};
    moe.expert_mant = (int64_t)mb; moe.expert_exps = (int64_t)eb; moe.expert_cols = ffn;
    moe.row_scale = dense + (int64_t)r0 * experts; moe.experts = experts; moe.scale_rows = 1;
    if (int rc = skinny_matmul(a, moe, gu_fmt, experts, s)) return rc;
    // down, each picked expert's own outputs
    MatArgs d = {};
    fh_epilogue de = {};
    de.kind = FH_EP_STORE;
    d.x = g; d.ldx = (int64_t)experts * ffn; d.x_bf16 = 1;
    d.mant = (const uint8_t*)down_mant; d.exps = down_exps; d.K = ffn; d.N = dim; d.M = n;
    d.y = parts; d.y_bf16 = 0;
    if (int rc = epilogue_args("fh_moe_experts", &de, ffn, dim, FH_F32, dim, d)) return rc;
    d.ldy = (int64_t)experts * dim;
    SkinnyMoe dm = {};
    dm.expert_mant = (int64_t)dmb; dm.expert_exps = (int64_t)deb; dm.expert_cols = dim; dm.expert_xcols = ffn;
    dm.row_scale = dense + (int64_t)r0 * experts; dm.experts = experts; dm.scale_rows = 0;
    if (int rc = skinny_matmul(d, dm, down_fmt, experts, s)) return rc;
    hipLaunchKernelGGL(moe_sum_kernel, dim3(n), dim3(256), 0, s, parts, experts, (int)dim,
                       residual ? residual + (int64_t)r0 * dim : nullptr, y + (int64_t)r0 * dim,
                       ssq_out ? ssq_out + (int64_t)r0 * (dim / 16) : nullptr);
    if (int rc = check_launch("fh_moe_experts")) return rc;
  }
  return FH_OK;
}
