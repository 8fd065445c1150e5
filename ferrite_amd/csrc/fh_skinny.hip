// Block-float matmul for a few rows on the matrix cores (up to 64 a pass): a decode step of many sequences (batch 16),
// and a mixture of experts' expert matmuls. y = epilogue(prologue(x) @ W), with fh_gemm_bfp's arithmetic (x times the
// RMSNorm weight rounded to bf16, the weight's values exact, fp32 sums).
//
// Built like the decode GEMV: a workgroup takes one item of 32 columns (two runs of 16, or a RoPE / SiLU·gate pair;
// one run of 16 where items of two would leave CUs idle) and its W waves split K; nothing crosses workgroups. A wave walks its K slice 64 rows at a time and reads the
// weight as the GEMV does: a lane a row of a run (16 bytes of bfp8, 8 of bfp4, and its exponent byte), a wave's loads
// 1 KiB (512 B) contiguous, four steps of them in flight. A lane turns its row into 16 bf16 values and writes them
// row-major into the wave's own LDS tile (no workgroup barrier in the loop: a wave reads back only what it wrote);
// ds_read_b64_tr_b16 then reads the tile back K-contiguous, as v_mfma_f32_16x16x32_bf16 takes its operand (in each
// 16-lane group, lane 4m + q addresses row m, columns 4q .. 4q + 3; lane j receives column j of the four rows). x's
// rows (16 a block, up to 4 blocks) come straight from memory, 8 consecutive k a lane, a step ahead: a wave's load
// takes 16 rows' 64 bytes from rows, 1 KiB in one piece from bf16 tiles of 16 rows (FH_BF16_T16), which a decode step
// of many sequences passes between its kernels (down's 33 MB of bfp4 at batch 16: 21.5 us from rows, ~17 from tiles). The waves' sums
// then meet in LDS in a fixed order and the epilogue runs on the item's outputs.
//
// For a mixture of experts the grid's second dimension is the expert: the weight is the expert's (`expert_mant` /
// `expert_exps` bytes apart), its outputs go `expert_cols` columns further on (and its x `expert_xcols`), and
// (scale_rows) each row's output is scaled by that row's weight for the expert (0 where the row did not pick it); an
// expert no row picked reads nothing. Gathered (SkinnyMoe::counts), an expert takes only the rows that picked it,
// through a list of their indices, and writes its outputs to rows of its own: x's traffic is each expert's rows, not
// every row once an item.
#include "fh_epilogue.h"

namespace fh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short short4v;
#define FH_LDS __attribute__((address_space(3)))

constexpr int SK_BK = 64;              // K rows a wave's step (a lane a row)
constexpr int SK_RS = 40;              // a row of the wave's bf16 tile in LDS: 32 columns + 8 (80 bytes: banks spread)
constexpr int SK_TILE = SK_BK * SK_RS; // the wave's tile, bf16 values: 5,120 bytes
constexpr int SK_RING = 4;             // steps of weight loads in flight

__device__ inline uint32_t sk_pack_exact(float lo, float hi) {
  // (the high halves of two floats whose low halves are 0: one byte permute, v_perm_b32)
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// threads a workgroup at most: fewer where a lane holds more, so that registers do not spill
__host__ __device__ constexpr int skinny_threads(bool xbf16, int mb) { return (xbf16 && mb == 1) ? 1024 : 512; }

template <bool FOUR, bool XBF16, bool NORM, int MB, int R>  // MB: blocks of 16 rows; R: runs of 16 columns an item
__global__ __launch_bounds__(skinny_threads(XBF16, MB)) void skinny_kernel(MatArgs a, SkinnyMoe moe) {
  constexpr int RB = FOUR ? 8 : 16;
  constexpr int XW = XBF16 ? 1 : 2;    // 16-byte loads for 8 of x's values
  using Row = typename std::conditional<FOUR, uint2, uint4>::type;
  extern __shared__ __attribute__((aligned(16))) char sk_smem[];
  __shared__ float rs_s[16 * MB];
  __shared__ float scale_s[16 * MB];

  const int item = blockIdx.x, e = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), W = blockDim.x >> 6;
  const bool gathered = moe.counts != nullptr;
  // (gathered: this workgroup's rows of the expert, from row0 of its list: the launch's first, then 16 MB a layer of
  // the grid's third dimension)
  const int row0 = moe.row0 + 16 * MB * (int)blockIdx.z;
  const int M = gathered ? max(0, min(moe.counts[e], (int)a.M) - row0) : (int)a.M, K = (int)a.K;
  const int64_t list0 = gathered ? (int64_t)e * a.M + row0 : 0;
  // a row's place in x and in y (gathered: the expert's own rows)
  auto xrow = [&](int r) -> int64_t {
    return gathered ? (moe.x_rows ? moe.x_rows[list0 + r] : list0 + r) : r;
  };
  const int64_t yrow0 = list0;

  // the rows' weights for this expert (read by the epilogue, after the stream's barrier); an expert no row picked
  // writes its zeros and reads nothing. No workgroup barrier comes before the stream: a barrier waits for every load
  // issued before it, which would put a whole memory latency in front of the first weight loads. Each wave decides
  // for itself whether the expert has rows.
  bool any = true;
  if (gathered) any = M > 0;
  else if (moe.row_scale) {
    const float r = lane < min(M, 16 * MB) ? moe.row_scale[(int64_t)lane * moe.experts + e] : 0.f;
    any = __ballot(r != 0.f) != 0;
  }
  if (t < 16 * MB) {
    float sc = 1.f;
    if (gathered) {
      if (moe.scale_rows) sc = t < M ? moe.row_w[list0 + t] : 0.f;
    } else if (moe.row_scale && moe.scale_rows) {
      sc = t < M ? moe.row_scale[(int64_t)t * moe.experts + e] : 0.f;
    }
    scale_s[t] = sc;
  }
  // each row's sums of squares (its maker left them by runs of 16), spread over the workgroup's threads (tpr
  // consecutive lanes a row): loaded now, summed into 1 / rms after the stream, so that the loads overlap it
  int tpr = 1;  // (the largest power of 2 that the workgroup's threads give each row, at most 64: within a wave;
                // W need not be a power of 2, and threads past tpr 16 MB take no row)
  while (tpr < 64 && tpr * 2 * 16 * MB <= (int)blockDim.x) tpr *= 2;
  const int srow = t / tpr, sk = t % tpr;
  constexpr int SQ = 8;
  const bool has_ssq = a.ssq_in != nullptr && M > 0;
  const float* sqp = has_ssq ? a.ssq_in + xrow(min(srow, M - 1)) * a.ssq_parts : (const float*)a.x;
  const int sqn = has_ssq ? a.ssq_parts : 1;
  float sq[SQ];
#pragma unroll
  for (int i = 0; i < SQ; ++i) sq[i] = sqp[min(sk + tpr * i, sqn - 1)];

  // the item's two runs
  int64_t nb[2];
  if (R == 1) { nb[0] = item; nb[1] = item; }
  else if (a.P == 1) { nb[0] = 2 * (int64_t)item; nb[1] = nb[0] + 1; }
  else { nb[0] = pair_first(item, a.pair_half); nb[1] = nb[0] + a.pair_half; }
  // (P == 1 with an odd count of runs: the last item's second run is absent)
  const bool run1_ok = R == 2 && nb[1] < a.N / 16;
  const uint8_t* mant = a.mant + (int64_t)e * moe.expert_mant;
  const uint8_t* exps = a.exps + (int64_t)e * moe.expert_exps;

  floatx4 acc[MB][R];  // [16-row block][run]: lane l holds rows 4 (l / 16) + i, column l % 16 of the run
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int j = 0; j < R; ++j) acc[b][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  uint16_t* Bs = (uint16_t*)sk_smem + wave * SK_TILE;
  const int r0 = wave * a.rows, r1 = min(K, r0 + a.rows);
  if (any && r0 < r1) {
    const uint8_t* mrun[R];
    const uint8_t* erun[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int64_t run = (j == 1 && !run1_ok) ? nb[0] : nb[j];
      mrun[j] = mant + run * a.K * RB;
      erun[j] = exps + run * a.K;
    }
    // x: row 16 b + lane % 16, k 8 (lane / 16) .. + 7 of each 32 k. In rows, a wave's 16-byte loads take 16 rows'
    // 64 bytes each (rows past M read row M - 1); in tiles of 16 rows (FH_BF16_T16, bf16), 1 KiB in a piece
    const bool tiles = XBF16 && a.x_tiles;
    const char* xp[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b)
      xp[b] = tiles ? (const char*)a.x + ((int64_t)16 * b * a.ldx + 8 * lane) * 2
                    : (const char*)a.x + (xrow(min(16 * b + (lane & 15), M - 1)) * a.ldx + (int64_t)e * moe.expert_xcols + 8 * (lane >> 4)) * (XBF16 ? 2 : 4);
    const int xk = tiles ? 32 : XBF16 ? 2 : 4;  // bytes a column of k moves the loads on
    const int last = r1 - SK_BK;  // (r1 - r0 is a multiple of 64: K is)
    // the transposed reads' addresses in the tile: 16-lane group g reads k 8 (g / 2)... of the 32-k block; in the
    // group, lane 4 m + q points at row m, columns 4 q .. 4 q + 3 of the run
    const int g = lane >> 4, m4 = (lane & 15) >> 2, q4 = lane & 3;
    FH_LDS short4v* trp = (FH_LDS short4v*)(Bs + (8 * g + m4) * SK_RS + 4 * q4);

    Row wr[SK_RING][R];
    uint32_t we[SK_RING][R];
    auto load_w = [&](int k0, Row (&w)[R], uint32_t (&ex)[R]) {
      __builtin_amdgcn_sched_barrier(0);
      const int k = min(k0, last) + lane;
#pragma unroll
      for (int j = 0; j < R; ++j) { w[j] = *(const Row*)(mrun[j] + (uint32_t)k * RB); ex[j] = erun[j][(uint32_t)k]; }
      __builtin_amdgcn_sched_barrier(0);
    };
    uint4 xv[2][MB][2][XW];  // [set][block][k32 half][16 bytes]
    auto load_x = [&](int k0, uint4 (&xs)[MB][2][XW]) {
      __builtin_amdgcn_sched_barrier(0);
      k0 = min(k0, last);
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4* p = (const uint4*)(xp[b] + (int64_t)(k0 + 32 * h) * xk);
#pragma unroll
          for (int i = 0; i < XW; ++i) xs[b][h][i] = p[i];
        }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](int k0, bool valid, const Row (&w)[R], const uint32_t (&ex)[R], const uint4 (&xs)[MB][2][XW]) {
      // the lane's rows of the R runs -> 16 bf16 values each, row-major into the tile (rows past the slice: zero)
#pragma unroll
      for (int j = 0; j < R; ++j) {
        float f[16];
        magnitudes(w[j], f);
        const float sc = valid ? ldexpf(1.f, (int)ex[j] - 133) : 0.f;
        uint32_t p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = sk_pack_exact(f[2 * i] * sc, f[2 * i + 1] * sc);
        uint4* dst = (uint4*)(Bs + lane * SK_RS + 16 * j);
        dst[0] = make_uint4(p[0], p[1], p[2], p[3]);
        dst[1] = make_uint4(p[4], p[5], p[6], p[7]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // the step's two blocks of 32 k
        bf16x8 bfr[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
          const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(trp + (32 * h * SK_RS + 16 * j) / 4);
          const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(trp + (32 * h * SK_RS + 4 * SK_RS + 16 * j) / 4);
          const short v8[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          bfr[j] = *(const bf16x8*)v8;
        }
        float gw[8];
        if (NORM) {
          const int kg = min(k0, last) + 32 * h + 8 * (lane >> 4);
          const float4 g0 = *(const float4*)(a.norm_w + kg), g1 = *(const float4*)(a.norm_w + kg + 4);
          const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) gw[i] = a.centered ? gg[i] + 1.f : gg[i];
        }
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          bf16x8 af;
          if (XBF16 && !NORM) {
            af = *(const bf16x8*)&xs[b][h][0];
          } else {
            float v[8];
            if (XBF16) {
              const uint32_t w4[4] = {xs[b][h][0].x, xs[b][h][0].y, xs[b][h][0].z, xs[b][h][0].w};
#pragma unroll
              for (int j = 0; j < 4; ++j) { v[2 * j] = __uint_as_float(w4[j] << 16); v[2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u); }
            } else {
              const uint4 u0 = xs[b][h][0], u1 = xs[b][h][XW - 1];
              const uint32_t w8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
              for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w8[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) af[j] = (__bf16)(NORM ? v[j] * gw[j] : v[j]);
          }
#pragma unroll
          for (int j = 0; j < R; ++j) acc[b][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[j], acc[b][j], 0, 0, 0);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // every lane's reads of the tile are done before the next step overwrites it
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
#pragma unroll
    for (int i = 0; i < SK_RING; ++i) load_w(r0 + SK_BK * i, wr[i], we[i]);
    load_x(r0, xv[0]);
    for (int k0 = r0; k0 < r1; k0 += SK_RING * SK_BK) {  // (steps past the slice carry zero weights)
#pragma unroll
      for (int i = 0; i < SK_RING; ++i) {
        const int k = k0 + SK_BK * i;
        load_x(k + SK_BK, xv[(i + 1) & 1]);
        step(k, k < r1, wr[i], we[i], xv[i & 1]);
        load_w(k + SK_RING * SK_BK, wr[i], we[i]);
      }
    }
  }

  // each row's 1 / rms (1 past M or without ssq_in)
  {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < SQ; ++i) sum += sk + tpr * i < sqn ? sq[i] : 0.f;
    for (int i0 = SQ * tpr + sk; i0 < sqn; i0 += SQ * tpr) {  // (more runs than SQ tpr: SQ loads at a time, added in order)
      float v[SQ];
#pragma unroll
      for (int i = 0; i < SQ; ++i) v[i] = i0 + tpr * i < sqn ? sqp[i0 + tpr * i] : 0.f;
#pragma unroll
      for (int i = 0; i < SQ; ++i) sum += v[i];
    }
    for (int m = tpr >> 1; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    if (sk == 0 && srow < 16 * MB) rs_s[srow] = (has_ssq && srow < M) ? 1.0f / sqrtf(sum / (float)K + a.eps) : 1.f;
  }

  // the waves' sums meet in LDS, in wave order: block b, run j's value i of lane l is row 16 b + 4 (l / 16) + i,
  // column 16 j + l % 16
  __syncthreads();
  float* part = (float*)sk_smem;  // [W][16 MB][33]
  constexpr int PLD = 33;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j)  // (R == 1: the second run's columns are zeros, never stored)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part[(wave * 16 * MB + 16 * b + 4 * (lane >> 4) + i) * PLD + 16 * j + (lane & 15)] = j < R ? acc[b][j < R ? j : 0][i] : 0.f;
  __syncthreads();
  float* fin = part + W * 16 * MB * PLD;  // [16 MB][33]
  for (int i = t; i < 16 * MB * 32; i += blockDim.x) {
    const int row = i >> 5, col = i & 31;
    float s = 0.f;
    for (int w = 0; w < W; ++w) s += part[(w * 16 * MB + row) * PLD + col];
    fin[row * PLD + col] = s * rs_s[row];
  }
  __syncthreads();

  const int kind = a.kind;
  const int64_t col_off = (int64_t)e * moe.expert_cols;
  if (a.P == 1 && kind == FH_EP_PROGRAM) {  // (a loop of its own: the program's decoding, hoisted out of the loop,
                                            // runs only here)
    for (int i = t; i < 16 * MB * 32; i += blockDim.x) {
      const int row = i >> 5, c = i & 31;
      const int64_t col = nb[c >> 4] * 16 + (c & 15);
      if (row < M && (c < 16 || run1_ok))
        store_out(a.y, a.y_bf16, y_at(a, yrow0 + row, col + col_off),
                  prog_eval(a.prog, fin[row * PLD + c] * scale_s[row], 0, a.row_base + row, col));
    }
  } else if (a.P == 1) {  // FH_EP_STORE / FH_EP_RESIDUAL: a thread a column of a row; a run is 16 lanes
    for (int i = t; i < 16 * MB * 32; i += blockDim.x) {
      const int row = i >> 5, c = i & 31, j = c & 15;
      const int64_t run = nb[c >> 4];
      const bool ok = row < M && (c < 16 || run1_ok);
      const int64_t col = run * 16 + j;
      const int64_t at = (yrow0 + row) * a.ldy + col + col_off;
      float v = fin[row * PLD + c] * scale_s[row];
      if (kind == FH_EP_RESIDUAL && ok) v += a.residual[at];
      if (ok) store_out(a.y, a.y_bf16, y_at(a, yrow0 + row, col + col_off), v);  // (RESIDUAL's y is rows: at)
      if (kind == FH_EP_RESIDUAL && a.copy_bf16 && ok) put_copy(a, yrow0 + row, col, v);
      if (kind == FH_EP_RESIDUAL && a.ssq_out) {
        float s = v * v;
        s += __shfl_xor(s, 8, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 1, 64);
        if (ok && j == 0) a.ssq_out[(yrow0 + row) * (a.N / 16) + run] = s;
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
        if (ok && j == 0) a.argmax_parts[(yrow0 + row) * (a.N / 16) + run] = make_int2(__float_as_int(bv), bc);
      }
    }
  } else {  // the pair: columns 0..15 the first run (gate, or a head's first half), 16..31 its partner
    for (int i = t; i < 16 * MB * 16; i += blockDim.x) {
      const int row = i >> 4, j = i & 15;
      if (row >= M) continue;
      float x0 = fin[row * PLD + j], x1 = fin[row * PLD + 16 + j];
      const int64_t c0 = nb[0] * 16 + j;
      if (kind == FH_EP_SILU_GATE) {
        store_out(a.y, a.y_bf16, y_at(a, yrow0 + row, c0 + col_off), silu(x0) * x1 * scale_s[row]);
      } else {  // FH_EP_ROPE_KV
        const int hd = a.head_dim;
        const int h = (int)c0 / hd, d = (int)c0 % hd, d1 = d + hd / 2;  // (c0 < N < 2^31)
        if (h < a.heads + a.kv_heads) {  // q's and k's heads turn: x cos + (-x2, x1) sin (models/llama.py:92-93)
          const int64_t place = rope_place(a, a.places[row]);
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
          cache_put(a, ch, a.cache_rows[row], d, d1, j, x0, x1);
        }
      }
    }
  }
}

// W waves: the least power of 2 giving 1536 waves in all or more (6 a CU; 4096 for a mixture's experts), at most what
// skinny_threads allows (and the sums' tiles fit LDS), each at least one 64-row step. (Measured at batch 16 of the 8B
// shape, against a target of 4096: down 28.7 -> 25.3 us at 8 waves, o 17.0 -> 15.6, gate_up 31.3 -> 29.4 at 2, the
// step 4.25 -> 3.96 ms; the Mixtral-shape experts at 32 tokens stay a little faster at 4096.)
static void skinny_plan(int64_t K, int items, int experts, int most, int& W, int& rows) {
  const int64_t target = experts > 1 ? 4096 : 1536;
  int64_t w = 1;
  while (w < most && w * items * experts < target) w *= 2;
  const int64_t steps = (K + SK_BK - 1) / SK_BK;
  while (w > 1 && w > steps) w /= 2;
  int64_t r = (K + w - 1) / w;
  r = (r + SK_BK - 1) / SK_BK * SK_BK;
  W = (int)((K + r - 1) / r);
  rows = (int)r;
}

template <bool FOUR, bool XBF16, bool NORM, int R>
static void skinny_launch(const MatArgs& a, const SkinnyMoe& moe, int items, int experts, int W, int mb, int blocks,
                          hipStream_t s) {
  const dim3 g(items, experts, blocks), b(64 * W);
  const size_t lds = (size_t)(W + 1) * 16 * mb * 33 * 4;  // the sums' tiles (they reuse the weight tiles)
  const size_t tiles = (size_t)W * SK_TILE * 2;
  const size_t bytes = lds > tiles ? lds : tiles;
  if (mb == 1) hipLaunchKernelGGL((skinny_kernel<FOUR, XBF16, NORM, 1, R>), g, b, bytes, s, a, moe);
  else if (mb == 2) hipLaunchKernelGGL((skinny_kernel<FOUR, XBF16, NORM, 2, R>), g, b, bytes, s, a, moe);
  else hipLaunchKernelGGL((skinny_kernel<FOUR, XBF16, NORM, 4, R>), g, b, bytes, s, a, moe);
}

template <bool FOUR, bool XBF16, bool NORM>
static void skinny_runs(const MatArgs& a, const SkinnyMoe& moe, bool one, int items, int experts, int W, int mb,
                        int blocks, hipStream_t s) {
  if (one) skinny_launch<FOUR, XBF16, NORM, 1>(a, moe, items, experts, W, mb, blocks, s);
  else skinny_launch<FOUR, XBF16, NORM, 2>(a, moe, items, experts, W, mb, blocks, s);
}

// M rows (at most 64 a pass) of a [grouped] skinny matmul; the caller checked the epilogue
int skinny_matmul(const MatArgs& a0, const SkinnyMoe& moe, int fmt, int experts, hipStream_t s) {
  if (a0.K % 64) return fail(FH_EUNSUP, "skinny matmul: K a multiple of 64");
  // an item is two runs (32 columns), or one where two a workgroup would leave CUs idle (P == 1, under 256 items)
  const bool one = a0.P == 1 && (a0.N / 32) * (int64_t)experts < 256;
  const int items = (int)(one ? a0.N / 16 : a0.P == 1 ? (a0.N / 16 + 1) / 2 : a0.items);
  if (experts > 256) return fail(FH_EUNSUP, "skinny matmul: at most 256 experts");
  int W, rows;
  // gathered (an expert's rows through a list): one 16-row block a workgroup, the blocks a layer each of the grid's
  // third dimension: most experts have few rows, and an expert with none in a workgroup's block reads nothing (two
  // blocks a workgroup for 32 rows a pass took 158 registers a lane; a launch a block spent ~9-13 us a launch on grids
  // of workgroups that all exit at once)
  const bool gathered = moe.counts != nullptr;
  const int mb0 = gathered ? 1 : a0.M > 32 ? 4 : a0.M > 16 ? 2 : 1;
  skinny_plan(a0.K, items, experts, skinny_threads(a0.x_bf16, mb0) / 64, W, rows);
  auto launch = [&](const MatArgs& a, const SkinnyMoe& mo, int mb, int blocks) {
    const int which = (fmt == FH_BFP4) * 4 + a.x_bf16 * 2 + (a.norm_w != nullptr);
    switch (which) {
      case 0: skinny_runs<false, false, false>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 1: skinny_runs<false, false, true>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 2: skinny_runs<false, true, false>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 3: skinny_runs<false, true, true>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 4: skinny_runs<true, false, false>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 5: skinny_runs<true, false, true>(a, mo, one, items, experts, W, mb, blocks, s); break;
      case 6: skinny_runs<true, true, false>(a, mo, one, items, experts, W, mb, blocks, s); break;
      default: skinny_runs<true, true, true>(a, mo, one, items, experts, W, mb, blocks, s); break;
    }
    return check_launch("skinny matmul");
  };
  if (gathered) {
    if (a0.M > 64) return fail(FH_EUNSUP, "skinny matmul: at most 64 gathered rows an expert");
    MatArgs a = a0;
    a.rows = rows;
    SkinnyMoe mo = moe;
    mo.row0 = 0;
    return launch(a, mo, 1, (int)((a0.M + 15) / 16));
  }
  for (int64_t m0 = 0; m0 < a0.M; m0 += 64) {
    MatArgs a = a0;
    a.row_base = m0;
    a.M = a0.M - m0 < 64 ? a0.M - m0 : 64;
    a.rows = rows;
    a.x = (const char*)a0.x + m0 * a0.ldx * (a0.x_bf16 ? 2 : 4);
    a.y = (char*)a0.y + m0 * a0.ldy * (a0.y_bf16 ? 2 : 4);
    if (a.ssq_in) a.ssq_in += m0 * a.ssq_parts;
    if (a.residual) a.residual += m0 * a0.ldy;
    if (a.copy_bf16) a.copy_bf16 += m0 * a0.N;
    if (a.ssq_out) a.ssq_out += m0 * (a0.N / 16);
    if (a.places) { a.places += m0; a.cache_rows += m0; }
    if (a.argmax_parts) a.argmax_parts += m0 * (a0.N / 16);
    SkinnyMoe mo = moe;
    if (mo.row_scale) mo.row_scale += m0 * mo.experts;
    const int mb = a.M > 32 ? 4 : a.M > 16 ? 2 : 1;
    if (int rc = launch(a, mo, mb, 1)) return rc;
  }
  return FH_OK;
}

}  // namespace fh
