// Prefill GEMM by a block-float weight on the matrix cores: y = epilogue(prologue(x) @ W) for M rows at once, W packed
// along N ([N/16][K][16] magnitudes, [N/16][K] exponents), the same epilogues as the decode GEMV.
//
// As on ferrite's chip (the unpacker feeds bf16 to the matrix unit; ferrite/tensor.py:443-485), the products are bf16 x
// bf16 with fp32 sums: x (times the RMSNorm weight) is rounded to bf16, and the weight's values q * 2^(e - 133) are
// exact in bf16 (at most 7 significant bits). A workgroup of 4 waves computes a 128 x 128 tile (8 runs of 16 columns,
// or 4 runs and their RoPE / SiLU·gate partners) in K steps of 64, the operands in two LDS stages: while the matrix
// cores work on one stage, the threads' loads of the next step's x rows and weight rows are in flight, and once the
// step's products are issued they convert them into the other stage: x to bf16 rows, the weight's 16-byte runs to bf16
// columns (K-contiguous, as v_mfma_f32_32x32x16_bf16 takes its operands). One barrier a step. Each wave owns a 64 x 64
// quarter, 2 x 2 blocks of 32 x 32, 16 MFMAs a step. Where the grid would not give every CU a workgroup anyway, a
// workgroup of 8 waves takes 256 rows (4 x 2 waves of 64 x 64; the first 4 waves load and convert the weight, once for
// all 256 rows). The epilogue stages the tile in LDS as fp32 so that each output sees its row's 1/rms and its pair
// partner, whichever wave computed it.
//
// Tiles go to the XCDs in contiguous ranges (the hardware deals workgroups round-robin over the 8 XCDs) and within a
// range in groups of 8 row tiles, so that an XCD's L2 keeps both the weight columns and the x rows it re-reads.
//
// Gathered (a mixture of experts' many tokens, models/llama.py:314-329's group path): grid.y is the expert, whose
// weight lies expert_mant / expert_exps bytes on; its rows are the first counts[e] (at most M) of its list, x row
// x_rows[e M + r] (row e M + r where x_rows is null), output row e M + r, scaled by row_w[e M + r] (scale_rows); a
// row tile past the expert's count returns at once, so the grid is sized for the most rows an expert can have.
#include "fh_epilogue.h"

namespace fh {

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64;
constexpr int GM_LD = GM_BK + 8;     // LDS row of a tile operand, bf16: 144 bytes (16-byte aligned, spreads banks)
constexpr int GM_LDC = GM_BN + 4;    // LDS row of the fp32 output tile
constexpr int GM_THREADS = 256;
constexpr int GM_GROUP = 8;          // row tiles a group (tile order)

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

__device__ inline uint32_t pack_bf16_exact(float lo, float hi) {  // both exact in bf16: the high halves
  // (the high halves of two floats whose low halves are 0: one byte permute, v_perm_b32)
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
__device__ inline uint32_t pack_bf16_rne(float lo, float hi) { return bf16_rne_f(lo) | (bf16_rne_f(hi) << 16); }

// the run a tile's local run lr (0 .. RUNS - 1) stands for, or -1 past the weight: RUNS runs of 16 columns a tile, or
// RUNS / 2 pairs (the first runs, then their partners)
template <int RUNS = 8>
__device__ inline int64_t tile_run(const MatArgs& a, int tn, int lr) {
  if (a.P == 1) {
    const int64_t nb = (int64_t)tn * RUNS + lr;
    return nb < a.N / 16 ? nb : -1;
  }
  const int64_t it = (int64_t)tn * (RUNS / 2) + lr % (RUNS / 2);
  if (it >= a.items) return -1;
  const int64_t nb0 = pair_first(it, a.pair_half);
  return lr < RUNS / 2 ? nb0 : nb0 + a.pair_half;
}

// RoPE's per-row values for the epilogue, staged in LDS while the tile's first loads are in flight: row ar's place and
// cache row (m: the row, clamped into the matrix)
__device__ inline void stage_rope_rows(const MatArgs& a, int32_t* rows_s, int bm, int ar, int64_t m) {
  rows_s[ar] = a.places[m];
  rows_s[bm + ar] = a.cache_rows[m];
}

// The tile's epilogue: every output of the fp32 tile Cs [BM][BN + 4] (staged in LDS: each output sees its row's 1/rms
// and its pair partner, whichever wave computed it) through a's epilogue, NT threads (those of whole passes over the
// tile's columns: NT / BN of them a pass, the rest idle; a pass's threads start at a multiple of 64, so a run's 16
// columns are 16 lanes of one wave)
template <int BM, int NT, int BN = 128>
__device__ inline void gemm_epilogue(const MatArgs& a, const SkinnyMoe& g, const float* Cs, const float* rs_s, int tn,
                                     int64_t m0, int64_t M, int64_t ybase, int t, const int32_t* place_s,
                                     const int32_t* crow_s) {
  constexpr int LDC = BN + 4, RUNS = BN / 16, H = BN / 2;
  const int kind = a.kind;
  if (a.P == 1 && kind == FH_EP_PROGRAM) {  // (a loop of its own: the program's decoding, hoisted out of the loop,
                                            // runs only here)
    if (t >= NT / BN * BN) return;
    const int c = t % BN;
    const int64_t run = tile_run<RUNS>(a, tn, c >> 4);
    const int64_t col = run * 16 + (c & 15);
    for (int r = t / BN; r < BM; r += NT / BN) {
      const int64_t m = m0 + r;
      if (m < M && run >= 0)
        store_out(a.y, a.y_bf16, (ybase + m) * a.ldy + col, prog_eval(a.prog, Cs[r * LDC + c] * rs_s[r], 0, m, col));
    }
  } else if (a.P == 1) {  // FH_EP_STORE, FH_EP_RESIDUAL: a thread a column, NT / BN rows a pass; a run is 16 lanes
    if (t >= NT / BN * BN) return;
    const int c = t % BN, j = c & 15;
    const int64_t run = tile_run<RUNS>(a, tn, c >> 4);
    const int64_t col = run * 16 + j;
    // rows in batches of RB, the batch's residual loads issued together before its stores (one loop iteration a row
    // would wait for each load in turn: the stores may alias them, so nothing moves a load above the store before it)
    constexpr int S = NT / BN, RB = 8;
    for (int rb = t / BN; rb < BM; rb += RB * S) {
      float res[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int64_t m = min(m0 + rb + u * S, M - 1);
        res[u] = (kind == FH_EP_RESIDUAL && run >= 0) ? a.residual[(ybase + m) * a.ldy + col] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int r = rb + u * S;
        if (r >= BM) continue;  // (the same for a wave's lanes)
        const int64_t m = m0 + r;
        const bool ok = m < M && run >= 0;
        const int64_t at = (ybase + m) * a.ldy + col;
        float v = Cs[r * LDC + c] * rs_s[r];
        if (kind == FH_EP_RESIDUAL) v += res[u];
        if (ok) store_out(a.y, a.y_bf16, at, v);
        if (kind == FH_EP_RESIDUAL && a.copy_bf16 && ok) put_copy(a, m, col, v);
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
    }
  } else {  // the pairs: a thread a (first-half) column, NT / H rows a pass, in batches of RB rows (their loads first;
            // RoPE's places and cache rows staged in LDS by the kernel: place_s[r], crow_s[r] for the tile's row r)
    if (t >= NT / H * H) return;
    const int c = t % H, p = c >> 4, j = c & 15;
    const int64_t run = tile_run<RUNS>(a, tn, p);
    const int64_t c0 = run * 16 + j;
    const bool rope = kind == FH_EP_ROPE_KV;
    const int hd = rope ? a.head_dim : 1;
    const int h = (int)c0 / hd, d = (int)c0 % hd, d1 = d + hd / 2;  // (c0 < N < 2^31)
    const bool turn = rope && h < a.heads + a.kv_heads;  // q's and k's heads turn: x cos + (-x2, x1) sin (models/llama.py:92-93)
    constexpr int S = NT / H, RB = 8;
    for (int rb = t / H; rb < BM; rb += RB * S) {
      float cs0[RB], cs1[RB], sn0[RB], sn1[RB], sc[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {  // the batch's per-row loads: the row's weight, or its place's table rows
        const int r = min(rb + u * S, BM - 1);
        const int64_t m = min(m0 + r, M - 1);
        sc[u] = (!rope && g.scale_rows) ? g.row_w[ybase + m] : 1.f;
        cs0[u] = cs1[u] = 1.f;
        sn0[u] = sn1[u] = 0.f;
        if (turn) {
          const int64_t place = rope_place(a, place_s[r]);
          cs0[u] = a.cos_tab[place * hd + d]; cs1[u] = a.cos_tab[place * hd + d1];
          sn0[u] = a.sin_tab[place * hd + d]; sn1[u] = a.sin_tab[place * hd + d1];
        }
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int r = rb + u * S;
        const int64_t m = m0 + r;
        if (r >= BM || m >= M || run < 0) continue;
        float x0 = Cs[r * LDC + c] * rs_s[r], x1 = Cs[r * LDC + c + H] * rs_s[r];
        if (!rope) {  // FH_EP_SILU_GATE
          store_out(a.y, a.y_bf16, (ybase + m) * a.ldy + c0, silu(x0) * x1 * sc[u]);
        } else {
          if (turn) {
            const float t0 = x0 * cs0[u] - x1 * sn0[u], t1 = x1 * cs1[u] + x0 * sn1[u];
            x0 = t0; x1 = t1;
          }
          if (h < a.heads) {
            float* q = (float*)a.y + m * a.ldy + (int64_t)h * hd;
            q[d] = x0; q[d1] = x1;
          } else {
            cache_put(a, h - a.heads, crow_s[r], d, d1, j, x0, x1);
          }
        }
      }
    }
  }
}

template <bool FOUR, bool XBF16, bool NORM, int TM>  // TM: 128-row halves of the tile (1, or 2 with 8 waves)
__global__ __launch_bounds__(GM_THREADS * TM, 3 - TM) void gemm_kernel(MatArgs a, int tiles_m, int tiles_n, SkinnyMoe g) {
  constexpr int BM = GM_BM * TM, NT = GM_THREADS * TM;
  constexpr int STAGE = (BM + GM_BN) * GM_LD * 2;
  constexpr int LDS = 2 * STAGE > BM * GM_LDC * 4 ? 2 * STAGE : BM * GM_LDC * 4;
  __shared__ __attribute__((aligned(16))) char smem[LDS];
  __shared__ float rs_s[BM];
  __shared__ int32_t rows_s[2 * BM];  // (RoPE) the tile's rows' places, then their cache rows
  // stage s: x at smem + s * STAGE ([BM rows][72] bf16), W after it ([128 columns][72] bf16, K-contiguous); the fp32
  // output tile [BM][132] aliases them after the K loop
  float* Cs = (float*)smem;                            // [128][132]: the output tile (after the K loop)

  // the rows of this matmul, its first output row, its weight (gathered: expert blockIdx.y's; `a` itself is left as
  // it is: a kernel argument changed in place is copied to scratch memory)
  int64_t M = a.M, ybase = 0;
  const uint8_t* wmant = a.mant;
  const uint8_t* wexps = a.exps;
  int id = blockIdx.x;
  if (g.counts) {  // the tiles of the expert's own rows, dealt to the XCDs in 8 contiguous ranges; the rest return
    const int e = blockIdx.y;
    M = min((int64_t)g.counts[e], a.M);
    ybase = (int64_t)e * a.M;
    wmant += e * g.expert_mant;
    wexps += e * g.expert_exps;
    tiles_m = (int)((M + BM - 1) / BM);
    const int q = (tiles_m * tiles_n + 7) / 8;
    if (id >= 8 * q) return;
    id = (id % 8) * q + id / 8;
    if (id >= tiles_m * tiles_n) return;
  } else if ((tiles_m * tiles_n) % 8 == 0) {
    id = (id % 8) * (tiles_m * tiles_n / 8) + id / 8;
  }
  // tile order: within a range, groups of GM_GROUP row tiles, row tile fastest
  const int per_group = GM_GROUP * tiles_n;
  const int first_m = id / per_group * GM_GROUP;
  const int gm = min(tiles_m - first_m, GM_GROUP);
  const int tm = first_m + (id % per_group) % gm, tn = (id % per_group) / gm;
  const int64_t m0 = (int64_t)tm * BM;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int K = (int)a.K;

  // this thread's loads: x row ar (of 128), k half ah (32 values); weight run lr (of 8), rows 4 rq .. 4 rq + 3,
  // columns 8 ch .. 8 ch + 7
  const int ar = t >> 1, ah = t & 1;
  const int64_t xr0 = min(m0 + ar, M - 1);
  const int64_t xrow = g.counts ? (g.x_rows ? (int64_t)g.x_rows[ybase + xr0] : ybase + xr0) : xr0;
  const bool xok = m0 + ar < M;
  const int lr = (t >> 5) & 7, rq = (t & 31) >> 1, ch = t & 1;
  const bool wt = TM == 1 || t < GM_THREADS;  // (the weight's loads and conversion: the first 256 threads)
  const int64_t nb = tile_run(a, tn, lr);
  constexpr int RB = FOUR ? 8 : 16;
  const uint8_t* mrun = wmant + (nb < 0 ? 0 : nb) * a.K * RB + ch * (RB / 2);
  const uint8_t* erun = wexps + (nb < 0 ? 0 : nb) * a.K;

  // a K step's loads, in registers: two sets, so that each step's loads have two steps' compute to arrive
  using Half = typename std::conditional<FOUR, uint32_t, uint2>::type;  // 8 of a row's 16 magnitudes
  constexpr int XW = XBF16 ? 4 : 8;  // x's 32 values: 4 x 16 bytes (bf16) or 8 (fp32), as uint4

  // Loads are unconditional (addresses clamped into the tensors) so that the compiler can count them and wait only
  // for the older set: x's k past K reads the row's last 32 values, whose weight rows are zero; a step past the last
  // re-reads the last.
  const int last = (K - 1) / GM_BK * GM_BK;
  auto load = [&](int k0, uint4 (&xr)[XW], Half (&wm)[4], uint32_t& we) {
    __builtin_amdgcn_sched_barrier(0);  // (issued here, not sunk below the step's arithmetic)
    k0 = min(k0, last);
    const int kx = min(k0 + 32 * ah, K - 32);
    const uint4* p = (const uint4*)((const char*)a.x + (xrow * a.ldx + kx) * (XBF16 ? 2 : 4));
#pragma unroll
    for (int i = 0; i < XW; ++i) xr[i] = p[i];
    const int k = min(k0 + 4 * rq, K - 4);  // (K is a multiple of 32)
    if (wt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) wm[r] = *(const Half*)(mrun + (int64_t)(k + r) * RB);
      we = *(const uint32_t*)(erun + k);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  auto store = [&](int k0, int stage, const uint4 (&xr)[XW], const Half (&wm)[4], uint32_t we) {
    uint16_t* As = (uint16_t*)(smem + stage * STAGE);
    uint16_t* Bs = As + BM * GM_LD;
    // x -> bf16 (times the RMSNorm weight), 4 x 16 bytes
    const int kx = min(k0 + 32 * ah, K - 32);
    if (XBF16 && !NORM) {
#pragma unroll
      for (int i = 0; i < 4; ++i)  // (element by element: a whole-array copy became a memcpy through scratch)
        *(uint4*)(As + ar * GM_LD + 32 * ah + 8 * i) = make_uint4(xr[i].x, xr[i].y, xr[i].z, xr[i].w);
    } else {
      float v[32];
      if (XBF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w4[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) { v[8 * i + 2 * j] = __uint_as_float(w4[j] << 16); v[8 * i + 2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u); }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          v[4 * i] = __uint_as_float(xr[i].x); v[4 * i + 1] = __uint_as_float(xr[i].y);
          v[4 * i + 2] = __uint_as_float(xr[i].z); v[4 * i + 3] = __uint_as_float(xr[i].w);
        }
      }
      if (NORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float4 g = *(const float4*)(a.norm_w + kx + 4 * i);
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
        *(uint4*)(As + ar * GM_LD + 32 * ah + 8 * i) =
            make_uint4(pack_bf16_rne(v[8 * i], v[8 * i + 1]), pack_bf16_rne(v[8 * i + 2], v[8 * i + 3]),
                       pack_bf16_rne(v[8 * i + 4], v[8 * i + 5]), pack_bf16_rne(v[8 * i + 6], v[8 * i + 7]));
    }

    // the weight's 4 rows x 8 columns -> 8 columns of 4 bf16 (one 8-byte LDS write each); rows past K are zero
    if (!wt) return;
    float f[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r) magnitudes8(wm[r], f[r]);
    const bool ok = k0 + 4 * rq < K;
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = ok ? ldexpf(1.f, (int)((we >> (8 * r)) & 255u) - 133) : 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c)
      *(uint2*)(Bs + (lr * 16 + ch * 8 + c) * GM_LD + 4 * rq) =
          make_uint2(pack_bf16_exact(f[0][c] * sc[0], f[1][c] * sc[1]), pack_bf16_exact(f[2][c] * sc[2], f[3][c] * sc[3]));
  };

  uint4 x0[XW], x1[XW];
  Half w0[4], w1[4];
  uint32_t e0, e1;
  load(0, x0, w0, e0);
  load(GM_BK, x1, w1, e1);

  // each row's 1 / rms from the sums of squares its maker left by runs of 16 (two threads a row)
  if (a.ssq_in) {  // (NORM, or rows that already hold x * w)
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
  if (a.kind == FH_EP_ROPE_KV && ah == 1) stage_rope_rows(a, rows_s, BM, ar, xr0);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  auto compute = [&](int stage) {
    const uint16_t* As = (const uint16_t*)(smem + stage * STAGE);
    const uint16_t* Bs = As + BM * GM_LD;
#pragma unroll
    for (int kk = 0; kk < GM_BK; kk += 16) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const bf16x8*)(As + (wr + 32 * i + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int j = 0; j < 2; ++j) bfr[j] = *(const bf16x8*)(Bs + (wc + 32 * j + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  };
  // step i computes stage i % 2 from the LDS, issues step i + 2's loads into the registers step i's came in, and
  // stores step i + 1's (loaded during step i - 1) into the other stage
  store(0, 0, x0, w0, e0);
  for (int k0 = 0; k0 < K; k0 += 2 * GM_BK) {  // (an odd count of steps ends with a step of zero weights)
    __syncthreads();            // stage 0 is stored; stage 1's readers are done
    load(k0 + 2 * GM_BK, x0, w0, e0);
    compute(0);
    store(k0 + GM_BK, 1, x1, w1, e1);
    __syncthreads();
    load(k0 + 3 * GM_BK, x1, w1, e1);
    compute(1);
    store(k0 + 2 * GM_BK, 0, x0, w0, e0);  // (past the last step: a stage nobody reads)
  }

  // the output tile, fp32, through LDS: block (i, j)'s value r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4,
  // column l % 32
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        Cs[(wr + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * GM_LDC + wc + 32 * j + (lane & 31)] = acc[i][j][r];
  __syncthreads();

  gemm_epilogue<BM, NT>(a, g, Cs, rs_s, tn, m0, M, ybase, t, rows_s, rows_s + BM);
}

// The same GEMM in the two-group ("ping-pong") form, for bf16 rows with no RMSNorm prologue (a prompt's matmuls: their
// x rows come normalised, as bf16, from fh_rms_rows, attention or SwiGLU): a workgroup of 8 waves takes a 256 x BN
// tile (BN = 64 WN: 128, 192 or 256 columns, 4 WN runs of 16 or 2 WN pairs), each wave 64 rows x 32 WN columns; waves
// 0-3 (one a SIMD) load and convert the weight, waves 4-7 (the other one a SIMD) load and copy x's rows. A K step is
// two phases between workgroup barriers: in the first, waves 0-3 run their products on the step's LDS stage while
// waves 4-7 write the next step's x into the other stage; in the second, waves 4-7 run their products while waves 0-3
// write the next step's weight. So on each SIMD one wave keeps the matrix core busy while the other does the loads,
// the conversion and the LDS writes, and the products' wave has the higher issue priority (s_setprio). Global loads
// run two steps ahead, in two register sets. The products are gemm_kernel's in the same order, so the results are its
// bit for bit. Measured at 2048 rows of the 8B shapes against gemm_kernel in the same run (128 columns): o 739 -> 796,
// gate_up 803 -> 842, down 826 -> 922 TFLOP/s. A tile wider than 128 columns stages its fp32 output in two halves of
// 128 rows (its whole would not fit in LDS).
template <bool FOUR, int WN>
__global__ __launch_bounds__(2 * GM_THREADS, 1) void gemm_pp_kernel(MatArgs a, int tiles_m, int tiles_n, SkinnyMoe g) {
  constexpr int BM = 2 * GM_BM, NT = 2 * GM_THREADS, BN = 64 * WN, RUNS = 4 * WN, LDC = BN + 4;
  constexpr int STAGE = (BM + BN) * GM_LD * 2;
  constexpr bool ONE_PASS = BM * LDC * 4 <= 150 * 1024;  // the whole output tile in LDS at once
  constexpr int CROWS = ONE_PASS ? BM : BM / 2;           // rows of the output tile a pass
  constexpr int LDS = 2 * STAGE > CROWS * LDC * 4 ? 2 * STAGE : CROWS * LDC * 4;
  constexpr int UPT = (RUNS + 7) / 8;  // the weight's units (8 columns x 4 rows of a step) a thread: 32 RUNS in all
  __shared__ __attribute__((aligned(16))) char smem[LDS];
  __shared__ float rs_s[BM];
  __shared__ int32_t rows_s[2 * BM];  // (RoPE) the tile's rows' places, then their cache rows
  float* Cs = (float*)smem;  // [CROWS][BN + 4]: the output tile (after the K loop)

  const int64_t M = a.M, ybase = 0;
  int id = blockIdx.x;
  if ((tiles_m * tiles_n) % 8 == 0) id = (id % 8) * (tiles_m * tiles_n / 8) + id / 8;  // (contiguous ranges an XCD)
  const int per_group = GM_GROUP * tiles_n;
  const int first_m = id / per_group * GM_GROUP;
  const int gm = min(tiles_m - first_m, GM_GROUP);
  const int tm = first_m + (id % per_group) % gm, tn = (id % per_group) / gm;
  const int64_t m0 = (int64_t)tm * BM;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool wgrp = t < GM_THREADS;  // waves 0-3: the weight; 4-7: x
  const int K = (int)a.K;
  const int last = (K - 1) / GM_BK * GM_BK;
  constexpr int RB = FOUR ? 8 : 16;
  using Half = typename std::conditional<FOUR, uint32_t, uint2>::type;  // 8 of a row's 16 magnitudes

  // the weight's threads (0-255): unit t + 256 i is run lr_i = (t >> 5) + 8 i, rows 4 rq .. 4 rq + 3, columns
  // 8 ch .. 8 ch + 7 of the run (a wave's 32-lane halves write 8 columns apart: no LDS bank in common); a unit past the
  // tile's runs (12 runs: the second unit of threads 128-255) is skipped, a whole wave at a time
  const int rq = (t & 31) >> 1, ch = t & 1;
  int lr[UPT];
  bool uok[UPT];
  const uint8_t* mrun[UPT];
  const uint8_t* erun[UPT];
#pragma unroll
  for (int i = 0; i < UPT; ++i) {
    lr[i] = ((t >> 5) & 7) + 8 * i;
    uok[i] = lr[i] < RUNS;
    const int64_t nb = uok[i] ? tile_run<RUNS>(a, tn, lr[i]) : -1;
    mrun[i] = a.mant + (nb < 0 ? 0 : nb) * a.K * RB + ch * (RB / 2);
    erun[i] = a.exps + (nb < 0 ? 0 : nb) * a.K;
  }
  // x's threads (256-511): rows xa and xa + 128 of the tile, k half xh (32 values, 4 x 16 bytes each)
  // (a row's two halves in neighbouring lanes: 16 lanes over 16 rows of one half write LDS without bank conflicts
  // but load 16 lines where these load 8, and measured slower: o 796 -> 743, gate_up 842 -> 772 TFLOP/s)
  const int tb = t & (GM_THREADS - 1), xa = tb >> 1, xh = tb & 1;
  const char* xp[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) xp[r] = (const char*)a.x + min(m0 + xa + 128 * r, M - 1) * a.ldx * 2;

  Half wm[2][UPT][4];
  uint32_t we[2][UPT];
  uint4 xr[2][2][4];  // [set][row][16 bytes]
  auto load_w = [&](int k0, int set) {
    __builtin_amdgcn_sched_barrier(0);
    const int k = min(min(k0, last) + 4 * rq, K - 4);
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (!uok[i]) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) wm[set][i][r] = *(const Half*)(mrun[i] + (int64_t)(k + r) * RB);
      we[set][i] = *(const uint32_t*)(erun[i] + k);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto load_x = [&](int k0, int set) {
    __builtin_amdgcn_sched_barrier(0);
    const int kx = min(min(k0, last) + 32 * xh, K - 32);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) xr[set][r][i] = ((const uint4*)(xp[r] + (int64_t)kx * 2))[i];
    __builtin_amdgcn_sched_barrier(0);
  };
  auto store_w = [&](int k0, int stage, int set) {  // a unit's 4 rows x 8 columns -> 8 columns of 4 bf16; rows past K 0
    uint16_t* Bs = (uint16_t*)(smem + stage * STAGE) + BM * GM_LD;
    const bool ok = k0 + 4 * rq < K;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (!uok[i]) continue;
      float f[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) magnitudes8(wm[set][i][r], f[r]);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = ok ? ldexpf(1.f, (int)((we[set][i] >> (8 * r)) & 255u) - 133) : 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *(uint2*)(Bs + (lr[i] * 16 + ch * 8 + c) * GM_LD + 4 * rq) =
            make_uint2(pack_bf16_exact(f[0][c] * sc[0], f[1][c] * sc[1]), pack_bf16_exact(f[2][c] * sc[2], f[3][c] * sc[3]));
    }
  };
  auto store_x = [&](int stage, int set) {
    uint16_t* As = (uint16_t*)(smem + stage * STAGE);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(uint4*)(As + (xa + 128 * r) * GM_LD + 32 * xh + 8 * i) = make_uint4(xr[set][r][i].x, xr[set][r][i].y, xr[set][r][i].z, xr[set][r][i].w);
  };

  floatx16 acc[2][WN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 32 * WN;
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  auto compute = [&](int stage) {
    const uint16_t* As = (const uint16_t*)(smem + stage * STAGE);
    const uint16_t* Bs = As + BM * GM_LD;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kk = 0; kk < GM_BK; kk += 16) {
      bf16x8 af[2], bfr[WN];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const bf16x8*)(As + (wr + 32 * i + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int j = 0; j < WN; ++j) bfr[j] = *(const bf16x8*)(Bs + (wc + 32 * j + fr) * GM_LD + kk + fk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // each row's 1 / rms from the sums of squares its maker left by runs of 16 (two threads a row)
  auto row_scales = [&] {
    const int ar = t >> 1, ah = t & 1;
    const int64_t xrow = min(m0 + ar, M - 1);
    if (a.ssq_in) {
      float s = 0.f;
      if (m0 + ar < M) {
        const float* q = a.ssq_in + xrow * a.ssq_parts;
        for (int i = ah; i < a.ssq_parts; i += 2) s += q[i];
      }
      s += __shfl_xor(s, 1, 64);
      if (ah == 0) rs_s[ar] = 1.0f / sqrtf(s / (float)K + a.eps);
    } else if (ah == 0) {
      rs_s[ar] = 1.f;
    }
    if (a.kind == FH_EP_ROPE_KV && ah == 1) stage_rope_rows(a, rows_s, BM, ar, xrow);
  };
  // Each group runs a loop of its own (the same barriers, in the same order), so that the compiler sees one group's
  // loads alone and waits only for the set a store takes, not for the loads issued after it. Step s's operands are
  // in stage s % 2; a pair of steps is 4 phases: [A: products of stage 0 | B: x of step s + 1 into stage 1], [A: the
  // weight of step s + 1 into stage 1 | B: products of stage 0], then the same with the stages swapped; each store
  // takes the register set loaded two phases of its group before, which then takes the loads of 3 steps on.
  // (An odd count of steps ends with a step of zero weights.)
  if (wgrp) {
    load_w(0, 0); load_w(GM_BK, 1); store_w(0, 0, 0); load_w(2 * GM_BK, 0);
    row_scales();
    __syncthreads();
    for (int s = 0; s * GM_BK < K; s += 2) {
      compute(0);
      __syncthreads();
      store_w((s + 1) * GM_BK, 1, 1); load_w((s + 3) * GM_BK, 1);
      __syncthreads();
      compute(1);
      __syncthreads();
      store_w((s + 2) * GM_BK, 0, 0); load_w((s + 4) * GM_BK, 0);
      __syncthreads();
    }
  } else {
    load_x(0, 0); load_x(GM_BK, 1); store_x(0, 0); load_x(2 * GM_BK, 0);
    row_scales();
    __syncthreads();
    for (int s = 0; s * GM_BK < K; s += 2) {
      store_x(1, 1); load_x((s + 3) * GM_BK, 1);
      __syncthreads();
      compute(0);
      __syncthreads();
      store_x(0, 0); load_x((s + 4) * GM_BK, 0);
      __syncthreads();
      compute(1);
      __syncthreads();
    }
  }

  // the output tile, fp32, through LDS (the stages are free: the last barrier passed every wave's products), in one
  // pass or in two of 128 rows (waves 0-3's rows, then 4-7's)
  for (int h = 0; h < BM / CROWS; ++h) {
    if (ONE_PASS || (wave >> 2) == h) {
      const int r0 = wr - h * CROWS;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            Cs[(r0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LDC + wc + 32 * j + (lane & 31)] = acc[i][j][r];
    }
    __syncthreads();
    gemm_epilogue<CROWS, NT, BN>(a, g, Cs, rs_s + h * CROWS, tn, m0 + h * CROWS, M, ybase, t, rows_s + h * CROWS,
                                 rows_s + BM + h * CROWS);
    if (h + 1 < BM / CROWS) __syncthreads();  // (the next pass rewrites Cs)
  }
}

// The tiled kernel over a's M rows (per expert, gathered, when g.counts is set: grid.y = experts)
int gemm_tiles(const MatArgs& a, const SkinnyMoe& g, int fmt, int experts, hipStream_t s) {
  // 256-row tiles (8 waves, the weight's conversion shared by twice the rows) where they still give every CU a
  // workgroup or fewer (measured at 2048 rows of the 8B shapes: o 720 -> 765 TFLOP/s, down 780 -> 895; qkv and gate_up,
  // with more tiles than CUs, slower), 128-row tiles (4 waves, two workgroups a CU) otherwise
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    return n;
  }();
  const int64_t tiles_n0 = a.P == 1 ? (a.N / 16 + 7) / 8 : ((int64_t)a.items + 3) / 4;
  const int64_t tiles2 = (a.M + 2 * GM_BM - 1) / (2 * GM_BM) * tiles_n0;
  // gemm_pp_kernel for bf16 rows without the norm, its 256-row tiles 128, 192 or 256 columns wide: the widest whose
  // tiles fill the CUs' rounds (at most one round, or the last at least 7/8 full) and no narrower tile takes fewer
  // rounds of as much work; none filling them, the 4-wave kernel (qkv's 384 tiles of 2048 rows x 128 columns ran at
  // 656 TFLOP/s against 712-750 for 128-row tiles two a CU)
  int WNv = 0;
  if (!g.counts && a.x_bf16 && !a.x_tiles && !a.norm_w) {
    const int64_t mt = (a.M + 2 * GM_BM - 1) / (2 * GM_BM);
    int64_t best = 0;
    for (int wn = 2; wn <= 4; ++wn) {
      const int64_t tiles = mt * (a.P == 1 ? (a.N / 16 + 4 * wn - 1) / (4 * wn) : ((int64_t)a.items + 2 * wn - 1) / (2 * wn));
      const int64_t rounds = (tiles + cus - 1) / cus;
      const bool fills = tiles <= cus || tiles * 8 >= rounds * cus * 7;
      if (fills && (best == 0 || rounds * wn <= best)) { WNv = wn; best = rounds * wn; }
    }
  }
  const bool pp = WNv != 0;
  const int TMv = (pp || (!g.counts && tiles2 <= cus)) ? 2 : 1;
  const int64_t tiles_m = (a.M + GM_BM * TMv - 1) / (GM_BM * TMv);
  const int64_t tiles_n = tiles_n0;
  if (tiles_m * tiles_n >= (1LL << 31)) return fail(FH_EUNSUP, "fh_gemm_bfp: too many tiles");
  if (g.counts && (a.ssq_in || a.kind == FH_EP_ROPE_KV || a.kind == FH_EP_RESIDUAL)) return fail(FH_EUNSUP, "gathered GEMM: STORE or SILU_GATE, no prologue");
  // (gathered: a grid for the most rows an expert can have, in whole multiples of the 8 XCDs)
  const int64_t tiles = g.counts ? (tiles_m * tiles_n + 7) / 8 * 8 : tiles_m * tiles_n;
  const dim3 grid((unsigned)tiles, g.counts ? experts : 1), b(GM_THREADS * TMv);
  const int tm = (int)tiles_m, tn = (int)tiles_n;
  const int which = (fmt == FH_BFP4) * 4 + a.x_bf16 * 2 + (a.norm_w != nullptr);
  if (pp) {
    const int64_t tnw = a.P == 1 ? (a.N / 16 + 4 * WNv - 1) / (4 * WNv) : ((int64_t)a.items + 2 * WNv - 1) / (2 * WNv);
    const dim3 gridw((unsigned)(tiles_m * tnw));
    const int tnv = (int)tnw;
#define GM_PP(F) do { if (WNv == 2) hipLaunchKernelGGL((gemm_pp_kernel<F, 2>), gridw, b, 0, s, a, tm, tnv, g); \
                      else if (WNv == 3) hipLaunchKernelGGL((gemm_pp_kernel<F, 3>), gridw, b, 0, s, a, tm, tnv, g); \
                      else hipLaunchKernelGGL((gemm_pp_kernel<F, 4>), gridw, b, 0, s, a, tm, tnv, g); } while (0)
    if (fmt == FH_BFP4) GM_PP(true);
    else GM_PP(false);
#undef GM_PP
    return FH_OK;
  }
#define GM_LAUNCH(F, X, N) do { if (TMv == 2) hipLaunchKernelGGL((gemm_kernel<F, X, N, 2>), grid, b, 0, s, a, tm, tn, g); \
                                 else hipLaunchKernelGGL((gemm_kernel<F, X, N, 1>), grid, b, 0, s, a, tm, tn, g); } while (0)
  switch (which) {
    case 0: GM_LAUNCH(false, false, false); break;
    case 1: GM_LAUNCH(false, false, true); break;
    case 2: GM_LAUNCH(false, true, false); break;
    case 3: GM_LAUNCH(false, true, true); break;
    case 4: GM_LAUNCH(true, false, false); break;
    case 5: GM_LAUNCH(true, false, true); break;
    case 6: GM_LAUNCH(true, true, false); break;
    default: GM_LAUNCH(true, true, true); break;
  }
#undef GM_LAUNCH
  return FH_OK;
}

}  // namespace fh

using namespace fh;

extern "C" int fh_gemm_bfp(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t N, const void* w_mant,
                           const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy,
                           void* stream) {
  if (!x || !w_mant || !w_exps || !y) return fail(FH_EINVAL, "fh_gemm_bfp: null pointer");
  if (M < 1 || K < 32 || K % 32 || N < 16 || N % 16)
    return fail(FH_EINVAL, "fh_gemm_bfp: need M >= 1, K a multiple of 32, N a multiple of 16");
  if (x_dtype != FH_F32 && x_dtype != FH_BF16 && x_dtype != FH_BF16_T16)
    return fail(FH_EINVAL, "fh_gemm_bfp: x is FH_F32, FH_BF16 or FH_BF16_T16");
  if (y_dtype != FH_F32 && y_dtype != FH_BF16 && y_dtype != FH_BF16_T16)
    return fail(FH_EINVAL, "fh_gemm_bfp: y is FH_F32, FH_BF16 or FH_BF16_T16");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_gemm_bfp: fmt is FH_BFP8 or FH_BFP4");
  if (ldx < K || ldx % 8) return fail(FH_EINVAL, "fh_gemm_bfp: ldx < K or not a multiple of 8 (16-byte row loads)");
  MatArgs a = {};
  a.x = x; a.ldx = ldx; a.x_bf16 = x_dtype != FH_F32; a.x_tiles = x_dtype == FH_BF16_T16;
  a.mant = (const uint8_t*)w_mant; a.exps = w_exps; a.K = K; a.N = N; a.M = M;
  a.y = y; a.y_bf16 = y_dtype != FH_F32; a.y_tiles = y_dtype == FH_BF16_T16; a.ldy = ldy;
  if (int rc = epilogue_args("fh_gemm_bfp", ep, K, N, y_dtype, ldy, a)) return rc;
  if (a.y_tiles && ldy % 8) return fail(FH_EINVAL, "fh_gemm_bfp: FH_BF16_T16 y needs ldy a multiple of 8");
  hipStream_t s = as_stream(stream);
  if (M <= 64 && K % 64 == 0) {  // a few rows: the skinny kernel (K split among waves, as the GEMV splits it)
    const SkinnyMoe none = {};
    return skinny_matmul(a, none, fmt, 1, s);
  }
  if (a.x_tiles || a.y_tiles || a.copy_tiles)
    return fail(FH_EUNSUP, "fh_gemm_bfp: FH_BF16_T16 rows (and copy_tiles) are for up to 64 rows with K a multiple of 64");
  const SkinnyMoe none = {};
  if (int rc = gemm_tiles(a, none, fmt, 1, s)) return rc;
  return check_launch("fh_gemm_bfp");
}
