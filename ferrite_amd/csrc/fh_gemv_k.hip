// Decode GEMV by a block-float weight packed along K (FH_AXIS_K: 16 consecutive rows of a column share an exponent,
// gpt2.bfp(W.T).T; the layout exps [K/16][N], mant [K/16][N][16] bytes for bfp8, [K/16][N][8] for bfp4):
// y = epilogue(prologue(x) @ W) for 1..8 rows a launch.
//
// A lane takes one column: a run of its 16 rows is one 16-byte load (8 for bfp4) and an exponent byte, and a wave's
// 64 lanes read 64 neighbouring columns' runs, 1 KiB (512 B) contiguous, U runs in flight. The run's 16 values of x
// are the same for every lane (scalar loads); the lane sums x_j q_j over the run (each magnitude converted by one
// sign-extending byte convert, FMAs in fp32), then adds that sum times the run's 2^(e - 133) (exact) to its column.
// A workgroup takes 64 columns, its W waves splitting the K/16 runs; their sums meet in LDS in a fixed order and the
// epilogue runs on the workgroup's outputs. Nothing crosses workgroups.
#include <math.h>
#include <type_traits>
#include "fh_epilogue.h"

namespace fh {

constexpr int GK_U = 4;  // runs of a column a lane has in flight

template <bool FOUR, int B, bool NORM>
__global__ __launch_bounds__(1024) void gemv_k_kernel(MatArgs a) {
  constexpr int RB = FOUR ? 8 : 16;  // bytes of a run
  using Run = typename std::conditional<FOUR, uint2, uint4>::type;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6;
  const int64_t N = a.N;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t cc = col < N ? col : N - 1;  // (lanes past N read the last column and store nothing)
  const int KB = (int)(a.K / 16);
  const int r0 = wave * a.rows, r1 = min(KB, r0 + a.rows);  // this wave's runs (a.rows of them)
  const float* xf = (const float*)a.x;
  const int64_t ldx = a.ldx;

  float acc[B];
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.f;

  for (int k0 = r0; k0 < r1; k0 += GK_U) {
    Run m[GK_U];
    int e[GK_U];
#pragma unroll
    for (int u = 0; u < GK_U; ++u) {
      const int64_t kb = min(k0 + u, r1 - 1);
      m[u] = *(const Run*)(a.mant + (kb * N + cc) * RB);
      e[u] = a.exps[kb * N + cc];
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above in flight before any arithmetic
#pragma unroll
    for (int u = 0; u < GK_U; ++u) {
      const bool live = k0 + u < r1;  // (uniform: runs past the wave's last add nothing)
      const int64_t k = (int64_t)min(k0 + u, r1 - 1) * 16;
      float f[16];
      magnitudes(m[u], f);
      float g[16];
      if (NORM) {
#pragma unroll
        for (int j = 0; j < 16; ++j) g[j] = a.centered ? a.norm_w[k + j] + 1.f : a.norm_w[k + j];
      }
      const float sc = live ? ldexpf(1.f, e[u] - 133) : 0.f;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) t = fmaf(NORM ? xf[b * ldx + k + j] * g[j] : xf[b * ldx + k + j], f[j], t);
        acc[b] = fmaf(t, sc, acc[b]);
      }
    }
  }

  // the waves' sums meet in LDS, in wave order; wave 0 runs the epilogue
  __shared__ float red[16][B][64];
#pragma unroll
  for (int b = 0; b < B; ++b) red[wave][b][lane] = acc[b];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int b = 0; b < B; ++b) {
    float t = red[0][b][lane];
    for (int w = 1; w < W; ++w) t += red[w][b][lane];
    red[0][b][lane] = t;  // (a lane rewrites only its own sums)
  }
  const bool ok = col < N;
  const int kind = a.kind;
  for (int b = 0; b < B; ++b) {  // (not unrolled: the epilogue's code once)
    const int64_t at = b * a.ldy + col;
    float o = red[0][b][lane];
    if (a.ssq_in) {  // the row's 1 / rms, from the sums of squares its maker left by runs of 16
      float s = 0.f;
      for (int i = lane; i < a.ssq_parts; i += 64) s += a.ssq_in[(int64_t)b * a.ssq_parts + i];
      s = wave_sum(s);
      o *= 1.0f / sqrtf(s / (float)a.K + a.eps);
    }
    if (kind == FH_EP_PROGRAM) {
      if (ok) store_out(a.y, a.y_bf16, at, prog_eval(a.prog, o, 0, a.row_base + b, col));
      continue;
    }
    if (kind == FH_EP_RESIDUAL && ok) o += a.residual[at];
    if (ok) store_out(a.y, a.y_bf16, at, o);
    if (kind == FH_EP_RESIDUAL && a.copy_bf16 && ok) put_copy(a, b, col, o);
    if (kind == FH_EP_RESIDUAL && a.ssq_out) {  // (N a multiple of 16: a run of 16 columns is 16 neighbouring lanes)
      float s = o * o;
      s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
      if (ok && (lane & 15) == 0) a.ssq_out[(int64_t)b * (N / 16) + col / 16] = s;
    }
    if (kind == FH_EP_STORE && a.argmax_parts) {  // each run of 16 columns' largest and its first column
      float bv = o;
      int bc = (int)col;
#pragma unroll
      for (int s = 8; s >= 1; s >>= 1) {
        const float ov = __shfl_xor(bv, s, 64);
        const int oc = __shfl_xor(bc, s, 64);
        if (ov > bv || (ov == bv && oc < bc)) { bv = ov; bc = oc; }
      }
      if (ok && (lane & 15) == 0) a.argmax_parts[(int64_t)b * (N / 16) + col / 16] = make_int2(__float_as_int(bv), bc);
    }
  }
}

template <bool FOUR, int B>
static void launch_k(const MatArgs& a, int items, int W, hipStream_t s) {
  if (a.norm_w) hipLaunchKernelGGL((gemv_k_kernel<FOUR, B, true>), dim3(items), dim3(64 * W), 0, s, a);
  else hipLaunchKernelGGL((gemv_k_kernel<FOUR, B, false>), dim3(items), dim3(64 * W), 0, s, a);
}

template <bool FOUR>
static void dispatch_k(const MatArgs& a, int batch, int items, int W, hipStream_t s) {
  switch (batch) {
    case 1: launch_k<FOUR, 1>(a, items, W, s); break;
    case 2: launch_k<FOUR, 2>(a, items, W, s); break;
    case 3: launch_k<FOUR, 3>(a, items, W, s); break;
    case 4: launch_k<FOUR, 4>(a, items, W, s); break;
    case 5: launch_k<FOUR, 5>(a, items, W, s); break;
    case 6: launch_k<FOUR, 6>(a, items, W, s); break;
    case 7: launch_k<FOUR, 7>(a, items, W, s); break;
    default: launch_k<FOUR, 8>(a, items, W, s); break;
  }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_gemv_bfp_k(const void* x, int x_dtype, int64_t ldx, int batch, int64_t K, int64_t N, const void* w_mant,
                             const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy,
                             void* stream) {
  if (!x || !w_mant || !w_exps || !y) return fail(FH_EINVAL, "fh_gemv_bfp_k: null pointer");
  if (batch < 1 || K < 16 || K % 16 || N < 1) return fail(FH_EINVAL, "fh_gemv_bfp_k: need batch >= 1, K a multiple of 16, N >= 1");
  if (x_dtype != FH_F32) return fail(FH_EUNSUP, "fh_gemv_bfp_k: x is FH_F32");
  if (y_dtype != FH_F32 && y_dtype != FH_BF16) return fail(FH_EINVAL, "fh_gemv_bfp_k: y is FH_F32 or FH_BF16");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_gemv_bfp_k: fmt is FH_BFP8 or FH_BFP4");
  if (ldx < K) return fail(FH_EINVAL, "fh_gemv_bfp_k: ldx < K");
  if (K >= (1LL << 27) || (int64_t)batch * ldx >= (1LL << 31) || N >= (1LL << 31) / 64)
    return fail(FH_EUNSUP, "fh_gemv_bfp_k: K, N or x too large");
  if (ep && (ep->kind == FH_EP_SILU_GATE || ep->kind == FH_EP_ROPE_KV))
    return fail(FH_EUNSUP, "fh_gemv_bfp_k: FH_EP_STORE, FH_EP_RESIDUAL or FH_EP_PROGRAM (the pairs are fh_gemv_bfp's)");
  if (ep && (ep->ssq_out || ep->argmax_parts) && N % 16)
    return fail(FH_EINVAL, "fh_gemv_bfp_k: ssq_out and argmax_parts need N a multiple of 16");
  if (ep && ep->copy_tiles) return fail(FH_EUNSUP, "fh_gemv_bfp_k: copy_bf16 as plain rows");
  MatArgs a = {};
  a.x = x; a.ldx = ldx;
  a.mant = (const uint8_t*)w_mant; a.exps = w_exps; a.K = K; a.N = N; a.M = batch;
  a.y = y; a.y_bf16 = y_dtype == FH_BF16; a.ldy = ldy;
  if (int rc = epilogue_args("fh_gemv_bfp_k", ep, K, N, y_dtype, ldy, a)) return rc;
  // W waves a workgroup of 64 columns: the least power of 2 giving ~4096 waves in all, at most 16, at most one a run
  const int items = (int)((N + 63) / 64);
  const int KB = (int)(K / 16);
  int W = 1;
  while (W < 16 && W * items < 4096 && W * 2 <= KB) W *= 2;
  const int rows = (KB + W - 1) / W;
  W = (KB + rows - 1) / rows;
  a.rows = rows;
  hipStream_t s = as_stream(stream);
  for (int b0 = 0; b0 < batch; b0 += 8) {  // more than 8 rows: several launches, each reading W again
    const int n = batch - b0 < 8 ? batch - b0 : 8;
    MatArgs c = a;
    c.row_base = b0;
    c.x = (const char*)x + (size_t)b0 * ldx * 4;
    c.y = (char*)y + (size_t)b0 * ldy * (a.y_bf16 ? 2 : 4);
    if (c.ssq_in) c.ssq_in += (int64_t)b0 * c.ssq_parts;
    if (c.residual) c.residual += (int64_t)b0 * ldy;
    if (c.copy_bf16) c.copy_bf16 += (int64_t)b0 * N;
    if (c.ssq_out) c.ssq_out += (int64_t)b0 * (N / 16);
    if (c.argmax_parts) c.argmax_parts += (int64_t)b0 * (N / 16);
    if (fmt == FH_BFP4) dispatch_k<true>(c, n, items, W, s);
    else dispatch_k<false>(c, n, items, W, s);
    if (int rc = check_launch("fh_gemv_bfp_k")) return rc;
  }
  return FH_OK;
}
