// A prompt's causal attention on the matrix cores, and the row RMSNorm that hands the prefill GEMMs bf16 rows.
//
// Attention (models/llama.py:129-142 for a chunk of T consecutive places p0 .. p0 + T - 1 of one sequence, whose
// keys and values are already in the cache: its own rows and every earlier place of the slot). A workgroup of 4 waves
// takes 128 query rows of one query head, a wave 32 of them, and walks the keys in tiles of 64 that its rows reach,
// each tile's loads in flight during the previous tile's arithmetic and the tile stored into the second of two LDS
// buffers after it, one barrier a tile (a 2048-token prompt's attention 250 -> ~450 TFLOP/s on MI355X with them).
// The scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_bf16, keys down, queries across), so that a lane
// holds one query's scores: its softmax statistics need no cross-lane work beyond the two halves of the wave. The
// online softmax (a running max and sum, rescaling the partial output) follows flash attention; the output is
// accumulated transposed too, O^T += V^T P^T, with P^T taken straight from the score registers: the order of the keys
// inside a 16-key step does not change the sum, so V^T is read from LDS in the order the score layout holds them.
// q, k, v go to bf16 for the matrix cores (as ferrite's chip holds them); scores, softmax and sums are fp32. Masked
// scores are -1e30 (the reference adds -1e9; either leaves exp() at 0). Query tiles are issued longest first (the second half of the heads shortest first). A
// block-float cache's runs are decoded exactly into the bf16 tiles (their values are bf16 values).
#include <math.h>
#include "fh_common.h"

namespace fh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

constexpr int PA_BQ = 128;      // query rows a workgroup (32 a wave)
constexpr int PA_BK = 64;       // keys a tile
constexpr float PA_MASKED = -1e30f;

struct PrefArgs {
  const float* q; int64_t ldq;
  const void* cache; int64_t cache_len; const uint8_t* cache_exps;
  int T, heads, kv_heads; float scale;
  int64_t p0, slot_row;
  void* o; int64_t ldo; int o_bf16;
};

__device__ inline uint32_t pack2_rne(float lo, float hi) { return bf16_rne_f(lo) | (bf16_rne_f(hi) << 16); }

// A cache piece of 8 values as loaded (bf16: 16 bytes; fp32: 32; a block float: its magnitudes and the run's
// exponent), converted to bf16 when it goes to LDS: a tile's loads are issued a tile ahead, before the arithmetic
struct CacheRaw { uint4 a, b; uint32_t e; };
template <int HD, int CF>
__device__ inline CacheRaw cache_raw(const PrefArgs& a, int64_t row, int c) {
  CacheRaw r;
  if constexpr (CF == FH_BF16) {
    r.a = *(const uint4*)((const uint16_t*)a.cache + row * HD + c);
  } else if constexpr (CF == FH_F32) {
    const uint4* p = (const uint4*)((const float*)a.cache + row * HD + c);
    r.a = p[0]; r.b = p[1];
  } else {
    if constexpr (CF == FH_BFP8) { const uint2 m = *(const uint2*)((const uint8_t*)a.cache + row * HD + c); r.a.x = m.x; r.a.y = m.y; }
    else r.a.x = *(const uint32_t*)((const uint8_t*)a.cache + row * (HD / 2) + c / 2);
    r.e = a.cache_exps[row * (HD / 16) + c / 16];
  }
  return r;
}
template <int CF>
__device__ inline uint4 raw_bf16x8(const CacheRaw& r) {
  if constexpr (CF == FH_BF16) {
    return r.a;
  } else if constexpr (CF == FH_F32) {
    return make_uint4(pack2_rne(__uint_as_float(r.a.x), __uint_as_float(r.a.y)), pack2_rne(__uint_as_float(r.a.z), __uint_as_float(r.a.w)),
                      pack2_rne(__uint_as_float(r.b.x), __uint_as_float(r.b.y)), pack2_rne(__uint_as_float(r.b.z), __uint_as_float(r.b.w)));
  } else {
    float f[8];
    uint32_t w[4];
    if constexpr (CF == FH_BFP8) magnitudes8(make_uint2(r.a.x, r.a.y), f);
    else magnitudes8(r.a.x, f);
    bfp_run_bf16<8>(f, r.e, w);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int HD, int CF>
__global__ __launch_bounds__(256, 2) void attention_prefill_kernel(PrefArgs a) {
  constexpr int KLD = HD + 8;        // K tile row in LDS (bf16): 16-byte aligned, banks spread
  constexpr int VLD = PA_BK + 8;     // V^T tile row (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t Ks2[2][PA_BK * KLD];  // two buffers: a tile's arithmetic reads
  __shared__ __attribute__((aligned(16))) uint16_t Vt2[2][HD * VLD];     // one while the next tile is stored in the other

  const int ntiles = (a.T + PA_BQ - 1) / PA_BQ;
  // the longest tiles first; the second half of the heads shortest first, so that the two workgroups a CU holds
  // (blocks b and b + half the grid) together walk about the same number of key tiles whatever b is
  const bool flip = (int)blockIdx.y >= ((int)gridDim.y + 1) / 2;
  const int qt = flip ? (int)blockIdx.x : ntiles - 1 - (int)blockIdx.x, h = blockIdx.y;
  const int kvh = h / (a.heads / a.kv_heads);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int ql = lane & 31, hh = lane >> 5;
  const int qrow = qt * PA_BQ + wave * 32 + ql;            // this lane's query row
  const int qr = min(qrow, a.T - 1);
  const int64_t qplace = a.p0 + qr;
  const int64_t last_key = a.p0 + min(qt * PA_BQ + PA_BQ, a.T) - 1;  // the workgroup's last key (its last row's place)
  const int nkt = (int)(last_key / PA_BK) + 1;
  // the wave's first row's place: a key tile wholly at or before it is visible to every row of the wave (no mask)
  const int64_t wave_first = a.p0 + min(qt * PA_BQ + wave * 32, a.T - 1);
  // scores kept in base 2 (scale times log2 e): the softmax's exponentials are then the chip's exp2 alone
  const float scale2 = a.scale * 1.44269504088896341f;

  // the lane's query, bf16, in the B-operand layout: step s holds dimensions 16 s + 8 hh .. + 7
  bf16x8 qf[HD / 16];
  {
    const float* qp = a.q + (int64_t)qr * a.ldq + (int64_t)h * HD;
#pragma unroll
    for (int s = 0; s < HD / 16; ++s) {
      const float4 u = *(const float4*)(qp + 16 * s + 8 * hh), v = *(const float4*)(qp + 16 * s + 8 * hh + 4);
      const float f[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[s][i] = (__bf16)f[i];
    }
  }

  floatx16 acc[HD / 32];
#pragma unroll
  for (int d = 0; d < HD / 32; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[d][r] = 0.f;
  float m = PA_MASKED, l = 0.f;

  const int64_t krow = (int64_t)kvh * a.cache_len + a.slot_row;
  const int64_t vrow = (int64_t)(a.kv_heads + kvh) * a.cache_len + a.slot_row;

  // a tile's loads: K, 64 rows x HD, a thread NK pieces of 8; V, a thread (past NVT threads none) 4 keys x 8 dimensions
  constexpr int NK = PA_BK * HD / 8 / 256, NVT = (PA_BK / 4) * (HD / 8);
  static_assert(NK * 256 == PA_BK * HD / 8 && NVT <= 256, "tile pieces a thread");
  CacheRaw kraw[NK], vraw[4];
  auto load_tile = [&](int kt) {
    const int64_t k0 = (int64_t)kt * PA_BK;
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int i = t + 256 * j, r = i / (HD / 8), c = (i % (HD / 8)) * 8;
      kraw[j] = cache_raw<HD, CF>(a, krow + min(k0 + r, last_key), c);
    }
    if (t < NVT) {
      const int kq = t % (PA_BK / 4), dg = t / (PA_BK / 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) vraw[j] = cache_raw<HD, CF>(a, vrow + min(k0 + 4 * kq + j, last_key), 8 * dg);
    }
  };
  // a tile's loads, as bf16, into buffer b: K rows; V^T, a thread's 4 keys x 8 dimensions as 8 rows of 4 keys. In a
  // V^T row each 16 keys lie as 0-3, 8-11, 4-7, 12-15, so that the 8 keys a lane multiplies at a 16-key step (4 hh ..
  // 4 hh + 3 and 8 + 4 hh .. 8 + 4 hh + 3, the score layout's) are one 16-byte read
  auto vt_col = [](int kq) { return 16 * (kq >> 2) + 4 * (((kq & 1) << 1) | ((kq >> 1) & 1)); };
  auto store_tile = [&](int b) {
    uint16_t* Ks = Ks2[b];
    uint16_t* Vt = Vt2[b];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int i = t + 256 * j, r = i / (HD / 8), c = (i % (HD / 8)) * 8;
      *(uint4*)(Ks + r * KLD + c) = raw_bf16x8<CF>(kraw[j]);
    }
    if (t < NVT) {
      const int kq = t % (PA_BK / 4), dg = t / (PA_BK / 4);
      uint32_t lo[4][4];  // [key][pair of dims]
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 w = raw_bf16x8<CF>(vraw[j]);
        lo[j][0] = w.x; lo[j][1] = w.y; lo[j][2] = w.z; lo[j][3] = w.w;
      }
#pragma unroll
      for (int d = 0; d < 8; ++d) {  // (a byte permute a word: dimension d's halves of two keys' words)
        const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u, p = d >> 1;
        const uint32_t k01 = __builtin_amdgcn_perm(lo[1][p], lo[0][p], sel);
        const uint32_t k23 = __builtin_amdgcn_perm(lo[3][p], lo[2][p], sel);
        *(uint2*)(Vt + (8 * dg + d) * VLD + vt_col(kq)) = make_uint2(k01, k23);
      }
    }
  };
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = (int64_t)kt * PA_BK;
    const uint16_t* Ks = Ks2[kt & 1];
    const uint16_t* Vt = Vt2[kt & 1];
    if (kt + 1 < nkt) load_tile(kt + 1);  // the next tile's loads in flight during this one's arithmetic

    // S^T for the tile's two blocks of 32 keys: block kb's value r of lane (ql, hh) is key 32 kb + 8 (r / 4) + 4 hh +
    // r % 4, query ql
    // (the two blocks' products interleaved, a 16-dimension step at a time: two independent MFMAs for each pair of
    // fragment reads, rather than one block's chain of 8 waiting on each read in turn)
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
    for (int st = 0; st < HD / 16; ++st)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf = *(const bf16x8*)(Ks + (32 * kb + ql) * KLD + 16 * st + 8 * hh);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kb], 0, 0, 0);
      }
    // mask past the query's place (only on a tile reaching past the wave's first row), and the online softmax: the
    // max of the raw scores (the scale is positive), and each exponent's scale and shift as one fused multiply-add
    float mt = PA_MASKED;
    if (k0 + PA_BK - 1 > wave_first) {
      const int kq = (int)(qplace - k0);  // (the key's offset in the tile: visible up to this)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = 32 * kb + 8 * (r >> 2) + 4 * hh + (r & 3);
          const float v = key <= kq ? s[kb][r] : PA_MASKED;
          s[kb][r] = v;
          mt = fmaxf(mt, v);
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt == PA_MASKED ? PA_MASKED : mt * scale2);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    float rsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], scale2, -mn));
        s[kb][r] = p;
        rsum += p;
      }
    rsum += __shfl_xor(rsum, 32, 64);
    l = l * alpha + rsum;
    m = mn;
#pragma unroll
    for (int d = 0; d < HD / 32; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[d][r] *= alpha;
    // O^T += V^T P^T, 16 keys a step: the keys of score registers 8 j .. 8 j + 7 of block kb, which are
    // 32 kb + 16 j + {4 hh .. 4 hh + 3, 8 + 4 hh .. 8 + 4 hh + 3}
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 pf;
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[i] = (__bf16)s[kb][8 * j + i];
        const int g = 32 * kb + 16 * j;
#pragma unroll
        for (int d = 0; d < HD / 32; ++d) {
          const uint4 vv = *(const uint4*)(Vt + (32 * d + ql) * VLD + g + 8 * hh);
          acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8*)&vv, pf, acc[d], 0, 0, 0);
        }
      }
    if (kt + 1 < nkt) store_tile((kt + 1) & 1);  // (the other buffer: its last readers passed the previous barrier)
    __syncthreads();
  }

  // o[row][h * HD + dim]: block d's value r of lane (ql, hh) is dimension 32 d + 8 (r / 4) + 4 hh + r % 4
  if (qrow < a.T) {
    const float inv = 1.f / l;
    const int64_t base = (int64_t)qrow * a.ldo + (int64_t)h * HD;
#pragma unroll
    for (int d = 0; d < HD / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dim = 32 * d + 8 * g + 4 * hh;
        const float v0 = acc[d][4 * g] * inv, v1 = acc[d][4 * g + 1] * inv, v2 = acc[d][4 * g + 2] * inv, v3 = acc[d][4 * g + 3] * inv;
        if (a.o_bf16) *(uint2*)((uint16_t*)a.o + base + dim) = make_uint2(pack2_rne(v0, v1), pack2_rne(v2, v3));
        else *(float4*)((float*)a.o + base + dim) = make_float4(v0, v1, v2, v3);
      }
  }
}

// out = x * rsqrt(mean(x^2) + eps) * w (w + 1 when centered), a workgroup a row (models/llama.py:82-85); a row of up
// to 4096 values is held in registers, read 16 bytes a load where the rows allow it (vec)
template <bool OBF16>
__global__ __launch_bounds__(256) void rms_rows_kernel(const float* x, int64_t ldx, int dim, const float* w, float eps,
                                                       int centered, void* out, int64_t ldo, int tiles, int vec) {
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  __shared__ float part[4];
  auto put = [&](int i, float xi, float rs) {
    const float g = centered ? w[i] + 1.f : w[i];
    const float v = xi * rs * g;
    if (OBF16) ((uint16_t*)out)[tiles ? tile16_at(row, i, ldo) : row * ldo + i] = (uint16_t)bf16_rne_f(v);
    else ((float*)out)[row * ldo + i] = v;
  };
  constexpr int R = 16;  // values a thread holds for a row of up to 256 R: all its loads issued at once, read once
  if (vec) {  // (dim a multiple of 4 up to 256 R, rows and w 16-byte aligned, out 8-byte aligned: 4 values a load)
    float4 xv[R / 4];
#pragma unroll
    for (int j = 0; j < R / 4; ++j) {
      const int i = 4 * (threadIdx.x + 256 * j);
      xv[j] = *(const float4*)(xr + (i < dim ? i : 0));
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < R / 4; ++j)
      if (4 * (threadIdx.x + 256 * j) < dim) s += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const float rs = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)dim + eps);
#pragma unroll
    for (int j = 0; j < R / 4; ++j) {
      const int i = 4 * (threadIdx.x + 256 * j);
      if (i >= dim) continue;
      float4 g = *(const float4*)(w + i);
      if (centered) { g.x += 1.f; g.y += 1.f; g.z += 1.f; g.w += 1.f; }
      const float v0 = xv[j].x * rs * g.x, v1 = xv[j].y * rs * g.y, v2 = xv[j].z * rs * g.z, v3 = xv[j].w * rs * g.w;
      if (OBF16) *(uint2*)((uint16_t*)out + (tiles ? tile16_at(row, i, ldo) : row * ldo + i)) = make_uint2(pack2_rne(v0, v1), pack2_rne(v2, v3));
      else *(float4*)((float*)out + row * ldo + i) = make_float4(v0, v1, v2, v3);
    }
    return;
  }
  if (dim <= 256 * R) {
    float xv[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int i = threadIdx.x + 256 * j;
      xv[j] = xr[i < dim ? i : 0];
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j)
      if (threadIdx.x + 256 * j < dim) s += xv[j] * xv[j];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const float rs = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)dim + eps);
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int i = threadIdx.x + 256 * j;
      if (i < dim) put(i, xv[j], rs);
    }
    return;
  }
  float s = 0.f;
  for (int i = threadIdx.x; i < dim; i += 256) s += xr[i] * xr[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float rs = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += 256) put(i, xr[i], rs);
}

template <int HD>
static void launch_prefill(int cf, dim3 g, dim3 b, hipStream_t s, const PrefArgs& a) {
  switch (cf) {
    case FH_F32: hipLaunchKernelGGL((attention_prefill_kernel<HD, FH_F32>), g, b, 0, s, a); break;
    case FH_BF16: hipLaunchKernelGGL((attention_prefill_kernel<HD, FH_BF16>), g, b, 0, s, a); break;
    case FH_BFP8: hipLaunchKernelGGL((attention_prefill_kernel<HD, FH_BFP8>), g, b, 0, s, a); break;
    default: hipLaunchKernelGGL((attention_prefill_kernel<HD, FH_BFP4>), g, b, 0, s, a); break;
  }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_attention_prefill(const float* q, int64_t ldq, const void* cache, int cache_dtype, int64_t cache_len,
                                    int T, int heads, int kv_heads, int head_dim, int64_t p0, int64_t slot_row, void* o,
                                    int o_dtype, int64_t ldo, void* stream) {
  if (!q || !cache || !o) return fail(FH_EINVAL, "fh_attention_prefill: null pointer");
  if (T < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads) return fail(FH_EINVAL, "fh_attention_prefill: need T >= 1, heads a multiple of kv_heads");
  if (head_dim != 64 && head_dim != 128) return fail(FH_EUNSUP, "fh_attention_prefill: head_dim 64 or 128");
  if (cache_dtype < FH_F32 || cache_dtype > FH_BFP4)
    return fail(FH_EUNSUP, "fh_attention_prefill: cache is FH_F32, FH_BF16, FH_BFP8 or FH_BFP4");
  if (o_dtype != FH_F32 && o_dtype != FH_BF16) return fail(FH_EINVAL, "fh_attention_prefill: o is FH_F32 or FH_BF16");
  if (ldq < (int64_t)heads * head_dim || ldo < (int64_t)heads * head_dim || ldq % 4 || ldo % 4)
    return fail(FH_EINVAL, "fh_attention_prefill: ldq and ldo at least heads * head_dim, multiples of 4");
  if (p0 < 0 || slot_row < 0 || slot_row + p0 + T > cache_len)
    return fail(FH_EINVAL, "fh_attention_prefill: the rows' keys (slot_row .. slot_row + p0 + T - 1) must lie in the cache");
  PrefArgs a = {};
  a.q = q; a.ldq = ldq; a.cache = cache; a.cache_len = cache_len;
  a.cache_exps = (const uint8_t*)cache + kv_exps_at(cache_dtype, kv_heads, cache_len, head_dim);
  a.T = T; a.heads = heads; a.kv_heads = kv_heads; a.scale = 1.0f / sqrtf((float)head_dim);
  a.p0 = p0; a.slot_row = slot_row; a.o = o; a.ldo = ldo; a.o_bf16 = o_dtype == FH_BF16;
  const dim3 g((T + PA_BQ - 1) / PA_BQ, heads), b(256);
  hipStream_t s = as_stream(stream);
  if (head_dim == 128) launch_prefill<128>(cache_dtype, g, b, s, a);
  else launch_prefill<64>(cache_dtype, g, b, s, a);
  return check_launch("fh_attention_prefill");
}

extern "C" int fh_rms_rows(const float* x, int64_t ldx, int64_t rows, int64_t dim, const float* norm_w, float eps,
                           int centered, void* out, int out_dtype, int64_t ldo, void* stream) {
  if (!x || !norm_w || !out) return fail(FH_EINVAL, "fh_rms_rows: null pointer");
  if (rows < 1 || dim < 1 || ldx < dim || ldo < dim) return fail(FH_EINVAL, "fh_rms_rows: need rows, dim >= 1, ldx and ldo >= dim");
  if (out_dtype != FH_F32 && out_dtype != FH_BF16 && out_dtype != FH_BF16_T16)
    return fail(FH_EINVAL, "fh_rms_rows: out is FH_F32, FH_BF16 or FH_BF16_T16");
  const int tiles = out_dtype == FH_BF16_T16;
  if (tiles && ldo % 8) return fail(FH_EINVAL, "fh_rms_rows: FH_BF16_T16 out needs ldo a multiple of 8");
  if (rows >= (1LL << 31)) return fail(FH_EUNSUP, "fh_rms_rows: too many rows");
  hipStream_t s = as_stream(stream);
  const int vec = dim % 4 == 0 && dim <= 4096 && ldx % 4 == 0 && ldo % 4 == 0 && !((uintptr_t)x & 15) && !((uintptr_t)norm_w & 15) &&
                  !((uintptr_t)out & (out_dtype == FH_F32 ? 15 : 7));
  if (out_dtype != FH_F32) hipLaunchKernelGGL((rms_rows_kernel<true>), dim3((unsigned)rows), dim3(256), 0, s, x, ldx, (int)dim, norm_w, eps, centered, out, ldo, tiles, vec);
  else hipLaunchKernelGGL((rms_rows_kernel<false>), dim3((unsigned)rows), dim3(256), 0, s, x, ldx, (int)dim, norm_w, eps, centered, out, ldo, 0, vec);
  return check_launch("fh_rms_rows");
}
