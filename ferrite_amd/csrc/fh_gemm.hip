// Prefill GEMM by a block-float weight on the matrix cores: y = epilogue(prologue(x) @ W) for M rows at once, W packed
// along N ([N/16][K][16] magnitudes, [N/16][K] exponents), the same epilogues as the decode GEMV.
//
// As on ferrite's chip (the unpacker feeds bf16 to the matrix unit; ferrite/tensor.py:443-485), the products are bf16 x
// bf16 with fp32 sums: x (times the RMSNorm weight) is rounded to bf16, and the weight's values q * 2^(e - 133) are
// exact in bf16 (at most 7 significant bits). A workgroup of 4 waves computes a 128 x 128 tile (8 runs of 16 columns,
// or 4 runs and their RoPE / SiLU·gate partners) in K steps of 64: its threads load the next step's x rows and weight
// rows from HBM into registers while the matrix cores work on the current step from LDS, then convert: x to bf16 rows,
// the weight's 16-byte runs to bf16 columns (K-contiguous, as v_mfma_f32_16x16x32_bf16 takes its operands). Each wave
// owns a 64 x 64 quarter: 4 x 4 blocks of 16 x 16, 32 MFMAs a step. The epilogue stages the tile in LDS as fp32 so
// that each output sees its row's 1/rms and its pair partner, whichever wave computed it.
//
// Tiles go to the XCDs in contiguous ranges (the hardware deals workgroups round-robin over the 8 XCDs) and within a
// range in groups of 8 row tiles, so that an XCD's L2 keeps both the weight columns and the x rows it re-reads.
#include "fh_epilogue.h"

namespace fh {

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64;
constexpr int GM_LD = GM_BK + 8;     // LDS row of a tile operand, bf16: 144 bytes (16-byte aligned, spreads banks)
constexpr int GM_LDC = GM_BN + 4;    // LDS row of the fp32 output tile
constexpr int GM_THREADS = 256;
constexpr int GM_GROUP = 8;          // row tiles a group (tile order)
constexpr int GM_LDS = GM_BM * GM_LDC * 4;  // 67,584 bytes: the output tile; the operand tiles (2 x 18,432) alias it

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;

__device__ inline uint32_t pack_bf16_exact(float lo, float hi) {  // both exact in bf16: the high halves
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}
__device__ inline uint32_t pack_bf16_rne(float lo, float hi) { return bf16_rne_f(lo) | (bf16_rne_f(hi) << 16); }

// the run a tile's local run lr (0..7) stands for, or -1 past the weight
__device__ inline int64_t tile_run(const MatArgs& a, int tn, int lr) {
  if (a.P == 1) {
    const int64_t nb = (int64_t)tn * 8 + lr;
    return nb < a.N / 16 ? nb : -1;
  }
  const int64_t it = (int64_t)tn * 4 + (lr & 3);
  if (it >= a.items) return -1;
  const int64_t nb0 = pair_first(it, a.pair_half);
  return lr < 4 ? nb0 : nb0 + a.pair_half;
}

template <bool FOUR, bool XBF16>
__global__ __launch_bounds__(GM_THREADS, 2) void gemm_kernel(MatArgs a, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(16))) char smem[GM_LDS];
  __shared__ float rs_s[GM_BM];
  uint16_t* As = (uint16_t*)smem;                      // [128 rows][72]: x, bf16
  uint16_t* Bs = (uint16_t*)(smem + GM_BM * GM_LD * 2); // [128 columns][72]: W, bf16, K-contiguous
  float* Cs = (float*)smem;                            // [128][132]: the output tile (after the K loop)

  // tile order
  const int T = tiles_m * tiles_n;
  int id = blockIdx.x;
  if (T % 8 == 0) id = (id % 8) * (T / 8) + id / 8;
  const int per_group = GM_GROUP * tiles_n;
  const int first_m = id / per_group * GM_GROUP;
  const int gm = min(tiles_m - first_m, GM_GROUP);
  const int tm = first_m + (id % per_group) % gm, tn = (id % per_group) / gm;
  const int64_t m0 = (int64_t)tm * GM_BM;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int K = (int)a.K;

  // this thread's loads: x row ar (of 128), k half ah (32 values); weight run lr (of 8), rows 2 rp and 2 rp + 1
  const int ar = t >> 1, ah = t & 1;
  const int64_t xrow = min(m0 + ar, a.M - 1);
  const bool xok = m0 + ar < a.M;
  const int lr = t >> 5, rp = t & 31;
  const int64_t nb = tile_run(a, tn, lr);
  constexpr int RB = FOUR ? 8 : 16;
  const uint8_t* mrun = a.mant + (nb < 0 ? 0 : nb) * a.K * RB;
  const uint8_t* erun = a.exps + (nb < 0 ? 0 : nb) * a.K;

  using Row = typename std::conditional<FOUR, uint2, uint4>::type;
  float4 xf[8];      // fp32 x: 32 values
  uint4 xb[4];       // bf16 x: 32 values
  Row wm[2];
  uint32_t we;

  auto load = [&](int k0) {
    const int kx = k0 + 32 * ah;
    if (XBF16) {
      const uint16_t* p = (const uint16_t*)a.x + xrow * a.ldx;
#pragma unroll
      for (int i = 0; i < 4; ++i) xb[i] = kx + 8 * i < K ? *(const uint4*)(p + kx + 8 * i) : make_uint4(0, 0, 0, 0);
    } else {
      const float* p = (const float*)a.x + xrow * a.ldx;
#pragma unroll
      for (int i = 0; i < 8; ++i) xf[i] = kx + 4 * i < K ? *(const float4*)(p + kx + 4 * i) : make_float4(0, 0, 0, 0);
    }
    const int k = min(k0 + 2 * rp, K - 2);  // (K is even; rows past K meet zero x)
    wm[0] = *(const Row*)(mrun + (int64_t)k * RB);
    wm[1] = *(const Row*)(mrun + (int64_t)(k + 1) * RB);
    we = *(const uint16_t*)(erun + k);
  };

  auto store = [&](int k0) {
    // x -> bf16 (times the RMSNorm weight), 4 x 16 bytes
    const int kx = k0 + 32 * ah;
    uint4 out[4];
    if (XBF16 && !a.norm_w) {
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = xb[i];
    } else {
      float v[32];
      if (XBF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w4[4] = {xb[i].x, xb[i].y, xb[i].z, xb[i].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) { v[8 * i + 2 * j] = __uint_as_float(w4[j] << 16); v[8 * i + 2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u); }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) { v[4 * i] = xf[i].x; v[4 * i + 1] = xf[i].y; v[4 * i + 2] = xf[i].z; v[4 * i + 3] = xf[i].w; }
      }
      if (a.norm_w) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float4 g = kx + 4 * i < K ? *(const float4*)(a.norm_w + kx + 4 * i) : make_float4(0, 0, 0, 0);
          if (a.centered) { g.x += 1.f; g.y += 1.f; g.z += 1.f; g.w += 1.f; }
          v[4 * i] *= g.x; v[4 * i + 1] *= g.y; v[4 * i + 2] *= g.z; v[4 * i + 3] *= g.w;
        }
      }
      if (!xok) {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        out[i] = make_uint4(pack_bf16_rne(v[8 * i], v[8 * i + 1]), pack_bf16_rne(v[8 * i + 2], v[8 * i + 3]),
                            pack_bf16_rne(v[8 * i + 4], v[8 * i + 5]), pack_bf16_rne(v[8 * i + 6], v[8 * i + 7]));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *(uint4*)(As + ar * GM_LD + 32 * ah + 8 * i) = out[i];

    // the weight's two rows -> 16 columns of 2 bf16 each; rows past K (clamped loads) are zero here too
    float f0[16], f1[16];
    magnitudes(wm[0], f0);
    magnitudes(wm[1], f1);
    const bool r0ok = k0 + 2 * rp < K;
    const float s0 = r0ok ? ldexpf(1.f, (int)(we & 255u) - 133) : 0.f;
    const float s1 = r0ok ? ldexpf(1.f, (int)(we >> 8) - 133) : 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c)
      *(uint32_t*)(Bs + (lr * 16 + c) * GM_LD + 2 * rp) = pack_bf16_exact(f0[c] * s0, f1[c] * s1);
  };

  load(0);

  // each row's 1 / rms from the sums of squares its maker left by runs of 16 (two threads a row)
  if (a.norm_w) {
    float s = 0.f;
    if (xok) {
      const float* q = a.ssq_in + xrow * a.ssq_parts;
      for (int i = ah; i < a.ssq_parts; i += 2) s += q[i];
    }
    s += __shfl_xor(s, 1, 64);
    if (ah == 0) rs_s[ar] = 1.0f / sqrtf(s / (float)K + a.eps);
  } else if (ah == 0) {
    rs_s[ar] = 1.f;
  }

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  for (int k0 = 0; k0 < K; k0 += GM_BK) {
    __syncthreads();            // the previous step's operands are read
    store(k0);
    __syncthreads();
    if (k0 + GM_BK < K) load(k0 + GM_BK);
#pragma unroll
    for (int kk = 0; kk < GM_BK; kk += 32) {
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *(const bf16x8*)(As + (wr + 16 * i + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = *(const bf16x8*)(Bs + (wc + 16 * j + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  }

  // the output tile, fp32, through LDS: block (i, j)'s value r of lane l is row 4 (l / 16) + r, column l % 16
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) Cs[(wr + 16 * i + 4 * (lane >> 4) + r) * GM_LDC + wc + 16 * j + (lane & 15)] = acc[i][j][r];
  __syncthreads();

  const int kind = a.kind;
  if (a.P == 1) {  // FH_EP_STORE, FH_EP_RESIDUAL: a thread a column, 2 rows a pass; a run is 16 neighbouring lanes
    const int c = t & 127, j = c & 15;
    const int64_t run = tile_run(a, tn, c >> 4);
    const int64_t col = run * 16 + j;
    for (int r = t >> 7; r < GM_BM; r += 2) {
      const int64_t m = m0 + r;
      const bool ok = m < a.M && run >= 0;
      const int64_t at = m * a.ldy + col;
      float v = Cs[r * GM_LDC + c] * rs_s[r];
      if (kind == FH_EP_RESIDUAL && ok) v += a.residual[at];
      if (ok) store_out(a.y, a.y_bf16, at, v);
      if (kind == FH_EP_RESIDUAL && a.ssq_out) {
        float s = v * v;
        s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
        if (ok && j == 0) a.ssq_out[m * (a.N / 16) + run] = s;
      }
      if (kind == FH_EP_STORE && a.argmax_parts) {
        float bv = v;
        int bc = (int)col;
#pragma unroll
        for (int s = 8; s >= 1; s >>= 1) {
          const float ov = __shfl_xor(bv, s, 64);
          const int oc = __shfl_xor(bc, s, 64);
          if (ov > bv || (ov == bv && oc < bc)) { bv = ov; bc = oc; }
        }
        if (ok && j == 0) a.argmax_parts[m * (a.N / 16) + run] = make_int2(__float_as_int(bv), bc);
      }
    }
  } else {  // the pairs: a thread a (first-half) column, 4 rows a pass
    const int c = t & 63, p = c >> 4, j = c & 15;
    const int64_t run = tile_run(a, tn, p);
    const int64_t c0 = run * 16 + j;
    for (int r = t >> 6; r < GM_BM; r += 4) {
      const int64_t m = m0 + r;
      if (m >= a.M || run < 0) continue;
      float x0 = Cs[r * GM_LDC + c] * rs_s[r], x1 = Cs[r * GM_LDC + c + 64] * rs_s[r];
      if (kind == FH_EP_SILU_GATE) {
        store_out(a.y, a.y_bf16, m * a.ldy + c0, silu(x0) * x1);
      } else {  // FH_EP_ROPE_KV
        const int hd = a.head_dim;
        const int h = (int)(c0 / hd), d = (int)(c0 % hd), d1 = d + hd / 2;
        if (h < a.heads + a.kv_heads) {  // q's and k's heads turn: x cos + (-x2, x1) sin (models/llama.py:92-93)
          const int64_t place = a.places[m];
          const float* cs = a.cos_tab + place * hd;
          const float* sn = a.sin_tab + place * hd;
          const float t0 = x0 * cs[d] - x1 * sn[d], t1 = x1 * cs[d1] + x0 * sn[d1];
          x0 = t0; x1 = t1;
        }
        if (h < a.heads) {
          float* q = (float*)a.y + m * a.ldy + (int64_t)h * hd;
          q[d] = x0; q[d1] = x1;
        } else {
          const int ch = h - a.heads;
          const int64_t at = ((int64_t)ch * a.cache_len + a.cache_rows[m]) * hd;
          store_out(a.cache, a.cache_bf16, at + d, x0);
          store_out(a.cache, a.cache_bf16, at + d1, x1);
        }
      }
    }
  }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_gemm_bfp(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t N, const void* w_mant,
                           const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy,
                           void* stream) {
  if (!x || !w_mant || !w_exps || !y) return fail(FH_EINVAL, "fh_gemm_bfp: null pointer");
  if (M < 1 || K < 32 || K % 32 || N < 16 || N % 16)
    return fail(FH_EINVAL, "fh_gemm_bfp: need M >= 1, K a multiple of 32, N a multiple of 16");
  if (x_dtype != FH_F32 && x_dtype != FH_BF16) return fail(FH_EINVAL, "fh_gemm_bfp: x is FH_F32 or FH_BF16");
  if (y_dtype != FH_F32 && y_dtype != FH_BF16) return fail(FH_EINVAL, "fh_gemm_bfp: y is FH_F32 or FH_BF16");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_gemm_bfp: fmt is FH_BFP8 or FH_BFP4");
  if (ldx < K || ldx % 8) return fail(FH_EINVAL, "fh_gemm_bfp: ldx < K or not a multiple of 8 (16-byte row loads)");
  MatArgs a = {};
  a.x = x; a.ldx = ldx; a.x_bf16 = x_dtype == FH_BF16;
  a.mant = (const uint8_t*)w_mant; a.exps = w_exps; a.K = K; a.N = N; a.M = M;
  a.y = y; a.y_bf16 = y_dtype == FH_BF16; a.ldy = ldy;
  if (int rc = epilogue_args("fh_gemm_bfp", ep, K, N, y_dtype, ldy, a)) return rc;
  const int64_t tiles_m = (M + GM_BM - 1) / GM_BM;
  const int64_t tiles_n = a.P == 1 ? (N / 16 + 7) / 8 : ((int64_t)a.items + 3) / 4;
  if (tiles_m * tiles_n >= (1LL << 31)) return fail(FH_EUNSUP, "fh_gemm_bfp: too many tiles");
  const dim3 g((unsigned)(tiles_m * tiles_n)), b(GM_THREADS);
  hipStream_t s = as_stream(stream);
  const bool four = fmt == FH_BFP4;
  if (four) {
    if (a.x_bf16) hipLaunchKernelGGL((gemm_kernel<true, true>), g, b, 0, s, a, (int)tiles_m, (int)tiles_n);
    else hipLaunchKernelGGL((gemm_kernel<true, false>), g, b, 0, s, a, (int)tiles_m, (int)tiles_n);
  } else {
    if (a.x_bf16) hipLaunchKernelGGL((gemm_kernel<false, true>), g, b, 0, s, a, (int)tiles_m, (int)tiles_n);
    else hipLaunchKernelGGL((gemm_kernel<false, false>), g, b, 0, s, a, (int)tiles_m, (int)tiles_n);
  }
  return check_launch("fh_gemm_bfp");
}
