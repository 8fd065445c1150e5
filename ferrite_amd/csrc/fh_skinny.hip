// Block-float matmul for a few rows on the matrix cores (up to 64 a pass): a decode step of many sequences (batch 16),
// and a mixture of experts' expert matmuls. y = epilogue(prologue(x) @ W), with fh_gemm_bfp's arithmetic (x times the
// RMSNorm weight rounded to bf16, the weight's values exact, fp32 sums).
//
// Built like the decode GEMV: a workgroup takes one item of 32 columns (two runs of 16, or a RoPE / SiLU·gate pair)
// and its W waves split K; nothing crosses workgroups. A wave walks its K slice 64 rows at a time: each lane loads 4
// rows x 8 columns of the weight (the same 1 KiB of a run's rows a wave as the GEMV), turns them into bf16 and writes
// them K-contiguous into the wave's own LDS (no workgroup barrier in the loop: a wave reads back only what it wrote),
// loads x's rows for the same 64 k, and issues v_mfma_f32_32x32x16_bf16: 32 rows x 32 columns x 16 k each. The waves'
// 32 x 32 (or 64 x 32) sums then meet in LDS in a fixed order and the epilogue runs on the item's outputs.
//
// For a mixture of experts the grid's second dimension is the expert: the weight is the expert's (`expert_mant` /
// `expert_exps` bytes apart), its outputs go `expert_cols` columns further on, and (scale_rows) each row's output is
// scaled by that row's weight for the expert (0 where the row did not pick it); an expert no row picked reads nothing.
//
// A wave keeps two steps' loads in flight: each step's loads go out right after the step two before it is done.
#include "fh_epilogue.h"

namespace fh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

constexpr int SK_BK = 64;              // K rows a wave's step
constexpr int SK_LD = SK_BK + 8;       // a column of the wave's bf16 weight tile in LDS
constexpr int SK_TILE = 32 * SK_LD;    // the wave's tile, bf16 values: 4,608 bytes


__device__ inline uint32_t sk_pack_exact(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// threads a workgroup at most: fewer where a lane holds more (fp32 x, 64 rows), so that registers do not spill
__host__ __device__ constexpr int skinny_threads(bool xbf16, int mb) { return xbf16 ? (mb == 1 ? 1024 : 512) : (mb == 1 ? 512 : 256); }

template <bool FOUR, bool XBF16, bool NORM, int MB>
__global__ __launch_bounds__(skinny_threads(XBF16, MB)) void skinny_kernel(MatArgs a, SkinnyMoe moe) {
  constexpr int RB = FOUR ? 8 : 16;
  constexpr int XW = XBF16 ? 1 : 2;  // 16-byte loads for 8 of x's values
  using Half = typename std::conditional<FOUR, uint32_t, uint2>::type;
  extern __shared__ __attribute__((aligned(16))) char sk_smem[];
  __shared__ float rs_s[32 * MB];
  __shared__ float scale_s[32 * MB];
  __shared__ int any_s;

  const int item = blockIdx.x, e = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), W = blockDim.x >> 6;
  const int M = (int)a.M, K = (int)a.K;

  // the rows' weights for this expert; an expert no row picked writes its zeros and reads nothing
  if (t == 0) any_s = moe.row_scale ? 0 : 1;
  __syncthreads();
  if (t < 32 * MB) {
    float sc = 1.f;
    if (moe.row_scale) {
      const float r = t < M ? moe.row_scale[(int64_t)t * moe.experts + e] : 0.f;
      if (r != 0.f) any_s = 1;
      if (moe.scale_rows) sc = r;
    }
    scale_s[t] = sc;
  }
  // each row's 1 / rms from the sums of squares its maker left by runs of 16: wave w the rows w, w + W, ..
  for (int row = wave; row < 32 * MB; row += W) {
    float r = 1.f;
    if (NORM && row < M) {
      const float* q = a.ssq_in + (int64_t)row * a.ssq_parts;
      float s = 0.f;
      for (int i = lane; i < a.ssq_parts; i += 64) s += q[i];
      s = wave_sum(s);
      r = 1.0f / sqrtf(s / (float)K + a.eps);
    }
    if (lane == 0) rs_s[row] = r;
  }
  __syncthreads();

  // the item's two runs
  int64_t nb[2];
  if (a.P == 1) { nb[0] = 2 * (int64_t)item; nb[1] = nb[0] + 1; }
  else { nb[0] = pair_first(item, a.pair_half); nb[1] = nb[0] + a.pair_half; }
  const bool run1_ok = nb[1] < a.N / 16;  // (P == 1 with an odd count of runs: the last item's second run is absent)
  const uint8_t* mant = a.mant + (int64_t)e * moe.expert_mant;
  const uint8_t* exps = a.exps + (int64_t)e * moe.expert_exps;

  floatx16 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  uint16_t* Bs = (uint16_t*)sk_smem + wave * SK_TILE;
  const int r0 = wave * a.rows, r1 = min(K, r0 + a.rows);
  if (any_s && r0 < r1) {
    // this lane's weight loads: run lr, rows 4 rq .. 4 rq + 3 of the step, columns 8 ch .. 8 ch + 7
    const int lr = lane >> 5, rq = (lane & 31) >> 1, ch = lane & 1;
    const int64_t run = (lr == 1 && !run1_ok) ? nb[0] : nb[lr];
    const uint8_t* mrun = mant + run * a.K * RB + ch * (RB / 2);
    const uint8_t* erun = exps + run * a.K;
    // x's loads: row (lane % 32) of each 32-row block, k 16 s + 8 (lane / 32) .. + 7
    const int xr = lane & 31, xh = lane >> 5;
    const char* xp[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b)
      xp[b] = (const char*)a.x + ((int64_t)min(xr + 32 * b, M - 1) * a.ldx + (int64_t)e * moe.expert_xcols) * (XBF16 ? 2 : 4);
    const int last = r1 - SK_BK;  // (r1 - r0 is a multiple of 64: K is)

    // a step's loads (unconditional, a step past the slice re-reads its last: the compiler can count them and wait
    // for the older set only), two sets in flight
    auto load = [&](int k0, Half (&wm)[4], uint32_t& we, uint4 (&xv)[MB][4][XW]) {
      __builtin_amdgcn_sched_barrier(0);  // the loads stay together, in this order, between the steps: a step waits
                                          // only for its own set, the older one
      k0 = min(k0, last);
      const int k = k0 + 4 * rq;
#pragma unroll
      for (int r = 0; r < 4; ++r) wm[r] = *(const Half*)(mrun + (int64_t)(k + r) * RB);
      we = *(const uint32_t*)(erun + k);
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4* p = (const uint4*)(xp[b] + (k0 + 16 * s + 8 * xh) * (XBF16 ? 2 : 4));
#pragma unroll
          for (int i = 0; i < XW; ++i) xv[b][s][i] = p[i];
        }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](int k0, bool valid, const Half (&wm)[4], uint32_t we, const uint4 (&xv)[MB][4][XW]) {
      // the weight tile, K-contiguous: 8 columns of 4 rows a lane
      float f[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) magnitudes8(wm[r], f[r]);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = valid ? ldexpf(1.f, (int)((we >> (8 * r)) & 255u) - 133) : 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *(uint2*)(Bs + (lr * 16 + ch * 8 + c) * SK_LD + 4 * rq) =
            make_uint2(sk_pack_exact(f[0][c] * sc[0], f[1][c] * sc[1]), sk_pack_exact(f[2][c] * sc[2], f[3][c] * sc[3]));
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 bf = *(const bf16x8*)(Bs + (lane & 31) * SK_LD + 16 * s + 8 * xh);
        float gw[8];
        if (NORM) {
          const int kg = min(k0, last) + 16 * s + 8 * xh;
          const float4 g0 = *(const float4*)(a.norm_w + kg), g1 = *(const float4*)(a.norm_w + kg + 4);
          const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) gw[i] = a.centered ? g[i] + 1.f : g[i];
        }
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          bf16x8 af;
          if (XBF16 && !NORM) {
            af = *(const bf16x8*)&xv[b][s][0];
          } else {
            float v[8];
            if (XBF16) {
              const uint32_t w4[4] = {xv[b][s][0].x, xv[b][s][0].y, xv[b][s][0].z, xv[b][s][0].w};
#pragma unroll
              for (int j = 0; j < 4; ++j) { v[2 * j] = __uint_as_float(w4[j] << 16); v[2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u); }
            } else {
              const uint4 u0 = xv[b][s][0], u1 = xv[b][s][XW - 1];
              const uint32_t w8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
              for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w8[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) af[j] = (__bf16)(NORM ? v[j] * gw[j] : v[j]);
          }
          acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc[b], 0, 0, 0);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // every lane's reads of the tile are done before the next step overwrites it
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    Half w0[4], w1[4];
    uint32_t e0, e1;
    uint4 x0[MB][4][XW], x1[MB][4][XW];
    load(r0, w0, e0, x0);
    load(r0 + SK_BK, w1, e1, x1);
    for (int k0 = r0; k0 < r1; k0 += 2 * SK_BK) {  // (an odd count of steps ends with a step of zero weights)
      step(k0, true, w0, e0, x0);
      load(k0 + 2 * SK_BK, w0, e0, x0);
      step(k0 + SK_BK, k0 + SK_BK < r1, w1, e1, x1);
      load(k0 + 3 * SK_BK, w1, e1, x1);
    }
  }

  // the waves' sums meet in LDS, in wave order: block b's value r of lane l is row 32 b + 8 (r / 4) + 4 (l / 32) +
  // r % 4, column l % 32
  __syncthreads();
  float* part = (float*)sk_smem;  // [W][32 MB][33]
  constexpr int PLD = 33;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      part[(wave * 32 * MB + 32 * b + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * PLD + (lane & 31)] = acc[b][r];
  __syncthreads();
  float* fin = part + W * 32 * MB * PLD;  // [32 MB][33]
  for (int i = t; i < 32 * MB * 32; i += blockDim.x) {
    const int row = i >> 5, col = i & 31;
    float s = 0.f;
    for (int w = 0; w < W; ++w) s += part[(w * 32 * MB + row) * PLD + col];
    fin[row * PLD + col] = s * rs_s[row];
  }
  __syncthreads();

  const int kind = a.kind;
  const int64_t col_off = (int64_t)e * moe.expert_cols;
  if (a.P == 1) {  // FH_EP_STORE / FH_EP_RESIDUAL: a thread a column of a row; a run is 16 neighbouring lanes
    for (int i = t; i < 32 * MB * 32; i += blockDim.x) {
      const int row = i >> 5, c = i & 31, j = c & 15;
      const int64_t run = nb[c >> 4];
      const bool ok = row < M && (c < 16 || run1_ok);
      const int64_t col = run * 16 + j;
      const int64_t at = (int64_t)row * a.ldy + col + col_off;
      float v = fin[row * PLD + c] * scale_s[row];
      if (kind == FH_EP_RESIDUAL && ok) v += a.residual[at];
      if (ok) store_out(a.y, a.y_bf16, at, v);
      if (kind == FH_EP_RESIDUAL && a.ssq_out) {
        float s = v * v;
        s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
        if (ok && j == 0) a.ssq_out[(int64_t)row * (a.N / 16) + run] = s;
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
        if (ok && j == 0) a.argmax_parts[(int64_t)row * (a.N / 16) + run] = make_int2(__float_as_int(bv), bc);
      }
    }
  } else {  // the pair: columns 0..15 the first run (gate, or a head's first half), 16..31 its partner
    for (int i = t; i < 32 * MB * 16; i += blockDim.x) {
      const int row = i >> 4, j = i & 15;
      if (row >= M) continue;
      float x0 = fin[row * PLD + j], x1 = fin[row * PLD + 16 + j];
      const int64_t c0 = nb[0] * 16 + j;
      if (kind == FH_EP_SILU_GATE) {
        store_out(a.y, a.y_bf16, (int64_t)row * a.ldy + c0 + col_off, silu(x0) * x1 * scale_s[row]);
      } else {  // FH_EP_ROPE_KV
        const int hd = a.head_dim;
        const int h = (int)(c0 / hd), d = (int)(c0 % hd), d1 = d + hd / 2;
        if (h < a.heads + a.kv_heads) {  // q's and k's heads turn: x cos + (-x2, x1) sin (models/llama.py:92-93)
          const int64_t place = a.places[row];
          const float* cs = a.cos_tab + place * hd;
          const float* sn = a.sin_tab + place * hd;
          const float t0 = x0 * cs[d] - x1 * sn[d], t1 = x1 * cs[d1] + x0 * sn[d1];
          x0 = t0; x1 = t1;
        }
        if (h < a.heads) {
          float* q = (float*)a.y + (int64_t)row * a.ldy + (int64_t)h * hd;
          q[d] = x0; q[d1] = x1;
        } else {
          const int ch = h - a.heads;
          const int64_t at = ((int64_t)ch * a.cache_len + a.cache_rows[row]) * hd;
          store_out(a.cache, a.cache_bf16, at + d, x0);
          store_out(a.cache, a.cache_bf16, at + d1, x1);
        }
      }
    }
  }
}

// W waves: the least power of 2 giving ~4096 waves in all (16 a CU), at most what skinny_threads allows (and the
// sums' tiles fit LDS), each at least one 64-row step
static void skinny_plan(int64_t K, int items, int experts, int most, int& W, int& rows) {
  int64_t w = 1;
  while (w < most && w * items * experts < 4096) w *= 2;
  const int64_t steps = (K + SK_BK - 1) / SK_BK;
  while (w > 1 && w > steps) w /= 2;
  int64_t r = (K + w - 1) / w;
  r = (r + SK_BK - 1) / SK_BK * SK_BK;
  W = (int)((K + r - 1) / r);
  rows = (int)r;
}

template <bool FOUR, bool XBF16, bool NORM>
static void skinny_launch(const MatArgs& a, const SkinnyMoe& moe, int items, int experts, int W, int mb, hipStream_t s) {
  const dim3 g(items, experts), b(64 * W);
  const size_t lds = (size_t)W * 32 * mb * 33 * 4 + 32 * mb * 33 * 4;  // the sums' tiles (they reuse the weight tiles)
  const size_t tiles = (size_t)W * SK_TILE * 2;
  const size_t bytes = lds > tiles ? lds : tiles;
  if (mb == 1) hipLaunchKernelGGL((skinny_kernel<FOUR, XBF16, NORM, 1>), g, b, bytes, s, a, moe);
  else hipLaunchKernelGGL((skinny_kernel<FOUR, XBF16, NORM, 2>), g, b, bytes, s, a, moe);
}

// M rows (at most 64 a pass) of a [grouped] skinny matmul; the caller checked the epilogue
int skinny_matmul(const MatArgs& a0, const SkinnyMoe& moe, int fmt, int experts, hipStream_t s) {
  if (a0.K % 64) return fail(FH_EUNSUP, "skinny matmul: K a multiple of 64");
  const int items = (int)(a0.P == 1 ? (a0.N / 16 + 1) / 2 : a0.items);
  if (experts > 256) return fail(FH_EUNSUP, "skinny matmul: at most 256 experts");
  int W, rows;
  skinny_plan(a0.K, items, experts, skinny_threads(a0.x_bf16, a0.M > 32 ? 2 : 1) / 64, W, rows);
  for (int64_t m0 = 0; m0 < a0.M; m0 += 64) {
    MatArgs a = a0;
    a.M = a0.M - m0 < 64 ? a0.M - m0 : 64;
    a.rows = rows;
    a.x = (const char*)a0.x + m0 * a0.ldx * (a0.x_bf16 ? 2 : 4);
    a.y = (char*)a0.y + m0 * a0.ldy * (a0.y_bf16 ? 2 : 4);
    if (a.ssq_in) a.ssq_in += m0 * a.ssq_parts;
    if (a.residual) a.residual += m0 * a0.ldy;
    if (a.ssq_out) a.ssq_out += m0 * (a0.N / 16);
    if (a.places) { a.places += m0; a.cache_rows += m0; }
    if (a.argmax_parts) a.argmax_parts += m0 * (a0.N / 16);
    SkinnyMoe mo = moe;
    if (mo.row_scale) mo.row_scale += m0 * mo.experts;
    const int mb = a.M > 32 ? 2 : 1;
    const int which = (fmt == FH_BFP4) * 4 + a.x_bf16 * 2 + (a.norm_w != nullptr);
    switch (which) {
      case 0: skinny_launch<false, false, false>(a, mo, items, experts, W, mb, s); break;
      case 1: skinny_launch<false, false, true>(a, mo, items, experts, W, mb, s); break;
      case 2: skinny_launch<false, true, false>(a, mo, items, experts, W, mb, s); break;
      case 3: skinny_launch<false, true, true>(a, mo, items, experts, W, mb, s); break;
      case 4: skinny_launch<true, false, false>(a, mo, items, experts, W, mb, s); break;
      case 5: skinny_launch<true, false, true>(a, mo, items, experts, W, mb, s); break;
      case 6: skinny_launch<true, true, false>(a, mo, items, experts, W, mb, s); break;
      default: skinny_launch<true, true, true>(a, mo, items, experts, W, mb, s); break;
    }
    if (int rc = check_launch("skinny matmul")) return rc;
  }
  return FH_OK;
}

}  // namespace fh
