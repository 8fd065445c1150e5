// The arguments a block-float matmul kernel takes (the decode GEMV and the MFMA GEMM alike) and the host-side check of
// an fh_epilogue: the RMSNorm prologue and the epilogue chains models/llama.py puts after its matmuls.
#pragma once
#include <type_traits>
#include "fh_program.h"

namespace fh {

struct MatArgs {
  const void* x; int64_t ldx; int x_bf16;
  const uint8_t* mant; const uint8_t* exps; int64_t K; int64_t N; int64_t M;
  int P;                    // runs an item: 1, or 2 for the SiLU·gate and RoPE pairs
  int pair_half;            // P == 2: the runs of a pair are nb0 and nb0 + pair_half
  int items;                // N / 16 / P
  int rows;                 // GEMV: K in slices of `rows` rows (a multiple of 64), one a wave
  // prologue
  const float* norm_w; const float* ssq_in; int ssq_parts; float eps; int centered;
  // epilogue
  int kind;
  void* y; int64_t ldy; int y_bf16;
  const float* residual; float* ssq_out; uint16_t* copy_bf16; const float* copy_w;
  int split;
  int heads, kv_heads, head_dim;
  const float* cos_tab; const float* sin_tab; const int32_t* places; const int32_t* cache_rows;
  void* cache; int cache_bf16; int64_t cache_len;
  int2* argmax_parts;
  fh_program prog;          // FH_EP_PROGRAM
};

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ inline void store_out(void* y, int bf16, int64_t at, float v) {
  if (bf16) ((uint16_t*)y)[at] = (uint16_t)bf16_rne_f(v);
  else ((float*)y)[at] = v;
}

// the 16 magnitudes of a run's row as floats: bfp8's 16 bytes are the signed q; bfp4's 8 bytes give 16 q (the 16 is
// folded into the scale: q * 2^(e - 129) = 16 q * 2^(e - 133))
__device__ inline void magnitudes(const uint4& m, float (&f)[16]) {
  const uint32_t w[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = (float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 255u);
}
__device__ inline void magnitudes(const uint2& m, float (&f)[16]) {
  const uint32_t w[2] = {m.x, m.y};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t hi = w[d] & 0xF0F0F0F0u, lo = (w[d] << 4) & 0xF0F0F0F0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[8 * d + 2 * i] = (float)(int8_t)((lo >> (8 * i)) & 255u);
      f[8 * d + 2 * i + 1] = (float)(int8_t)((hi >> (8 * i)) & 255u);
    }
  }
}

// 8 of a run's 16 magnitudes (columns 8h .. 8h + 7 of a row): bfp8's 8 bytes, bfp4's 4 bytes (16 q as above)
__device__ inline void magnitudes8(const uint2& m, float (&f)[8]) {
  const uint32_t w[2] = {m.x, m.y};
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = (float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 255u);
}
__device__ inline void magnitudes8(const uint32_t& m, float (&f)[8]) {
  const uint32_t hi = m & 0xF0F0F0F0u, lo = (m << 4) & 0xF0F0F0F0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = (float)(int8_t)((lo >> (8 * i)) & 255u);
    f[2 * i + 1] = (float)(int8_t)((hi >> (8 * i)) & 255u);
  }
}

// A pair item's first run: pairs are (nb0, nb0 + half) within each group of 2 half runs (a head's two halves for
// RoPE, where half = head_dim / 32; gate and up for SiLU·gate, where half = split / 16 and there is one group).
__host__ __device__ inline int64_t pair_first(int64_t item, int half) { return item / half * (2 * half) + item % half; }

// A grouped (mixture-of-experts) skinny matmul's extras (fh_skinny.hip): grid.y = expert, its weight `expert_mant` /
// `expert_exps` bytes on and its outputs `expert_cols` columns on; an expert whose row_scale[.][expert] are all 0 reads
// nothing; with scale_rows, each row's output is scaled by row_scale[row][expert]; expert e's x starts expert_xcols * e
// columns into x's rows. Or gathered: each expert multiplies only its own rows (below).
struct SkinnyMoe {
  int64_t expert_mant, expert_exps, expert_cols, expert_xcols;
  const float* row_scale; int experts;
  int scale_rows;
  // gathered (counts set): expert e takes counts[e] rows (at most M); its x row r is row x_rows[e M + r] of x (row
  // e M + r where x_rows is null), its output row r is y's row e M + r, and (scale_rows) its scale row_w[e M + r]
  const int32_t* counts; const int32_t* x_rows; const float* row_w;
};

// x @ W for up to 64 rows a pass on the matrix cores (fh_skinny.hip); a's epilogue already checked
int skinny_matmul(const MatArgs& a, const SkinnyMoe& moe, int fmt, int experts, hipStream_t s);

// Checks an fh_epilogue against the matmul's shape and fills a's prologue and epilogue fields (x, weight and y
// fields are the caller's). `who` names the entry point in messages.
inline int epilogue_args(const char* who, const fh_epilogue* ep, int64_t K, int64_t N, int y_dtype, int64_t ldy, MatArgs& a) {
  char msg[192];
  auto bad = [&](int code, const char* what) { snprintf(msg, sizeof msg, "%s: %s", who, what); return fail(code, msg); };
  a.kind = ep ? ep->kind : FH_EP_STORE;
  a.P = 1; a.pair_half = 1;
  int64_t out_cols = N;
  if (ep && ep->copy_bf16 && ep->kind != FH_EP_RESIDUAL) return bad(FH_EINVAL, "copy_bf16 is FH_EP_RESIDUAL's");
  if (ep && ep->copy_w && !ep->copy_bf16) return bad(FH_EINVAL, "copy_w scales copy_bf16");
  if (ep) {
    if (ep->norm_w || ep->ssq_in) {  // (ssq_in alone: rows that already hold x * w, scaled by 1/rms only)
      if (!ep->ssq_in || K % 16) return bad(FH_EINVAL, "RMSNorm prologue needs ssq_in and K a multiple of 16");
      a.norm_w = ep->norm_w; a.ssq_in = ep->ssq_in; a.ssq_parts = (int)(K / 16); a.eps = ep->eps; a.centered = ep->centered;
    }
    switch (ep->kind) {
      case FH_EP_STORE: a.argmax_parts = (int2*)ep->argmax_parts; break;
      case FH_EP_RESIDUAL:
        if (!ep->residual) return bad(FH_EINVAL, "FH_EP_RESIDUAL needs residual");
        a.residual = ep->residual; a.ssq_out = ep->ssq_out; a.copy_bf16 = (uint16_t*)ep->copy_bf16; a.copy_w = ep->copy_w;
        if (y_dtype != FH_F32) return bad(FH_EUNSUP, "FH_EP_RESIDUAL writes fp32");
        break;
      case FH_EP_SILU_GATE:
        if (ep->split * 2 != N || ep->split % 16) return bad(FH_EINVAL, "FH_EP_SILU_GATE needs N = 2 * split, split a multiple of 16");
        a.P = 2; a.pair_half = ep->split / 16; a.split = ep->split; out_cols = ep->split;
        break;
      case FH_EP_ROPE_KV: {
        const int hd = ep->head_dim;
        if (hd < 32 || hd % 32 || ep->heads < 1 || ep->kv_heads < 1 || (int64_t)(ep->heads + 2 * ep->kv_heads) * hd != N)
          return bad(FH_EINVAL, "FH_EP_ROPE_KV needs N = (heads + 2 kv_heads) * head_dim, head_dim a multiple of 32");
        if (!ep->cos_tab || !ep->sin_tab || !ep->places || !ep->cache_rows || !ep->cache || ep->cache_len < 1)
          return bad(FH_EINVAL, "FH_EP_ROPE_KV needs tables, places, cache rows and a cache");
        if (ep->cache_dtype != FH_F32 && ep->cache_dtype != FH_BF16) return bad(FH_EUNSUP, "cache is FH_F32 or FH_BF16");
        if (y_dtype != FH_F32) return bad(FH_EUNSUP, "FH_EP_ROPE_KV writes q in fp32");
        a.P = 2; a.pair_half = hd / 32; out_cols = (int64_t)ep->heads * hd;
        a.heads = ep->heads; a.kv_heads = ep->kv_heads; a.head_dim = hd;
        a.cos_tab = ep->cos_tab; a.sin_tab = ep->sin_tab; a.places = ep->places; a.cache_rows = ep->cache_rows;
        a.cache = ep->cache; a.cache_bf16 = ep->cache_dtype == FH_BF16; a.cache_len = ep->cache_len;
        break;
      }
      case FH_EP_PROGRAM:
        if (int rc = check_program(who, ep->program, true)) return rc;
        a.prog = *ep->program;
        break;
      default: return bad(FH_EINVAL, "unknown epilogue kind");
    }
  }
  if (ldy < out_cols) return bad(FH_EINVAL, "ldy smaller than the output's columns");
  a.items = (int)(N / 16 / a.P);
  return FH_OK;
}

}  // namespace fh
