// The arguments a block-float matmul kernel takes (the decode GEMV and the MFMA GEMM alike) and the host-side check of
// an fh_epilogue: the RMSNorm prologue and the epilogue chains models/llama.py puts after its matmuls.
#pragma once
#include <type_traits>
#include "fh_program.h"

namespace fh {

struct MatArgs {
  const void* x; int64_t ldx; int x_bf16; int x_tiles;  // (x_tiles: FH_BF16_T16 rows)
  const uint8_t* mant; const uint8_t* exps; int64_t K; int64_t N; int64_t M;
  int P;                    // runs an item: 1, or 2 for the SiLU·gate and RoPE pairs
  int pair_half;            // P == 2: the runs of a pair are nb0 and nb0 + pair_half
  int items;                // N / 16 / P
  int rows;                 // GEMV: K in slices of `rows` rows (a multiple of 64), one a wave
  int64_t row_base;         // the launch's first row among the call's (a call of many rows in several launches): the
                            // row an FH_EP_PROGRAM input is read at
  // prologue
  const float* norm_w; const float* ssq_in; int ssq_parts; float eps; int centered;
  // epilogue
  int kind;
  void* y; int64_t ldy; int y_bf16; int y_tiles;
  const float* residual; float* ssq_out; uint16_t* copy_bf16; const float* copy_w; int copy_tiles;
  int split;
  int heads, kv_heads, head_dim;
  const float* cos_tab; const float* sin_tab; int64_t rope_rows; const int32_t* places; const int32_t* cache_rows;
  void* cache; int cache_fmt; int64_t cache_len; uint8_t* cache_exps;  // (cache_exps: a block float's exponents)
  int2* argmax_parts;
  fh_program prog;          // FH_EP_PROGRAM
};

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ inline void store_out(void* y, int bf16, int64_t at, float v) {
  if (bf16) ((uint16_t*)y)[at] = (uint16_t)bf16_rne_f(v);
  else ((float*)y)[at] = v;
}

// where output (row, col) of a matmul goes in y, and in the residual epilogue's bf16 copy (row length N)
__device__ inline int64_t y_at(const MatArgs& a, int64_t row, int64_t col) {
  return a.y_tiles ? tile16_at(row, col, a.ldy) : row * a.ldy + col;
}
__device__ inline void put_copy(const MatArgs& a, int64_t row, int64_t col, float v) {
  const int64_t at = a.copy_tiles ? tile16_at(row, col, a.N) : row * a.N + col;
  a.copy_bf16[at] = (uint16_t)bf16_rne_f(a.copy_w ? v * a.copy_w[col] : v);
}

// A row's place as an index into the RoPE tables: a place outside them reads their nearest row (the host checks
// places; this keeps a bad one from reading past the tables)
__device__ inline int64_t rope_place(const MatArgs& a, int32_t place) {
  return place < 0 ? 0 : (place >= a.rope_rows ? a.rope_rows - 1 : place);
}

// A key or value pair into the cache: x0 at column d of row `crow` of plane ch (0 .. 2 kv_heads - 1: keys' heads
// then values'), x1 at d + head_dim / 2. A row outside 0 .. cache_len - 1 is not written (the host checks the rows;
// this keeps a bad one from writing past the cache). A block-float cache rounds bf16(x) (nearest even) run by run as
// fh_bfp_pack does (ferrite/compiler.py:1638-1714, put_kernel): the 16 lanes lane & ~15 .. (lane & ~15) + 15 hold a
// run's 16 columns, in order (j = lane & 15), and all of them must be here (they share the row, so they skip
// together); the run's exponent is their largest.
__device__ inline void cache_put(const MatArgs& a, int ch, int32_t crow, int d, int d1, int j, float x0, float x1) {
  if (crow < 0 || crow >= a.cache_len) return;
  const int64_t row = (int64_t)ch * a.cache_len + crow;
  const int hd = a.head_dim;
  if (a.cache_fmt == FH_F32 || a.cache_fmt == FH_BF16) {
    store_out(a.cache, a.cache_fmt == FH_BF16, row * hd + d, x0);
    store_out(a.cache, a.cache_fmt == FH_BF16, row * hd + d1, x1);
    return;
  }
  const bool four = a.cache_fmt == FH_BFP4;
  const uint32_t b0 = bf16_rne_f(x0), b1 = bf16_rne_f(x1);
  uint32_t t0 = (b0 >> 7) & 255u, t1 = (b1 >> 7) & 255u;
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) {
    t0 = max(t0, (uint32_t)__shfl_xor((int)t0, m, 64));
    t1 = max(t1, (uint32_t)__shfl_xor((int)t1, m, 64));
  }
  int q0 = (int)bfp_magnitude(b0, t0, four), q1 = (int)bfp_magnitude(b1, t1, four);
  if (b0 >> 15) q0 = -q0;
  if (b1 >> 15) q1 = -q1;
  uint8_t* mant = (uint8_t*)a.cache;
  if (four) {  // a byte holds columns 2i (low nibble) and 2i + 1
    const int o0 = __shfl_xor(q0, 1, 64), o1 = __shfl_xor(q1, 1, 64);
    if (!(j & 1)) {
      mant[row * (hd / 2) + d / 2] = (uint8_t)((q0 & 15) | ((o0 & 15) << 4));
      mant[row * (hd / 2) + d1 / 2] = (uint8_t)((q1 & 15) | ((o1 & 15) << 4));
    }
  } else {
    mant[row * hd + d] = (uint8_t)q0;
    mant[row * hd + d1] = (uint8_t)q1;
  }
  if (j == 0) {
    a.cache_exps[row * (hd / 16) + d / 16] = (uint8_t)t0;
    a.cache_exps[row * (hd / 16) + d1 / 16] = (uint8_t)t1;
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
  // e M + r where x_rows is null), its output row r is y's row e M + r, and (scale_rows) its scale row_w[e M + r];
  // a workgroup takes the expert's rows row0 + 16 MB z .. row0 + 16 MB z + 16 MB - 1 of those, z its layer of the
  // grid's third dimension
  const int32_t* counts; const int32_t* x_rows; const float* row_w;
  int row0;
};

// x @ W for up to 64 rows a pass on the matrix cores (fh_skinny.hip); a's epilogue already checked
int skinny_matmul(const MatArgs& a, const SkinnyMoe& moe, int fmt, int experts, hipStream_t s);
// x @ W in 128 x 128 tiles on the matrix cores (fh_gemm.hip), gathered per expert when moe.counts is set (STORE or
// SILU_GATE epilogues, no prologue); a's epilogue already checked
int gemm_tiles(const MatArgs& a, const SkinnyMoe& moe, int fmt, int experts, hipStream_t s);

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
        a.copy_tiles = ep->copy_bf16 && ep->copy_tiles;
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
        if (ep->rope_rows < 1) return bad(FH_EINVAL, "FH_EP_ROPE_KV needs rope_rows, the rows of cos_tab and sin_tab");
        if (ep->cache_dtype < FH_F32 || ep->cache_dtype > FH_BFP4) return bad(FH_EUNSUP, "cache is FH_F32, FH_BF16, FH_BFP8 or FH_BFP4");
        if (y_dtype != FH_F32) return bad(FH_EUNSUP, "FH_EP_ROPE_KV writes q in fp32");
        a.P = 2; a.pair_half = hd / 32; out_cols = (int64_t)ep->heads * hd;
        a.heads = ep->heads; a.kv_heads = ep->kv_heads; a.head_dim = hd;
        a.cos_tab = ep->cos_tab; a.sin_tab = ep->sin_tab; a.rope_rows = ep->rope_rows; a.places = ep->places; a.cache_rows = ep->cache_rows;
        a.cache = ep->cache; a.cache_fmt = ep->cache_dtype; a.cache_len = ep->cache_len;
        a.cache_exps = (uint8_t*)ep->cache + kv_exps_at(ep->cache_dtype, ep->kv_heads, ep->cache_len, hd);
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
