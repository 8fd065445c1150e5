// Decode attention over a KV cache, flash-decoding style, in two kernels. The first: a workgroup (two waves) takes a
// chunk of 128 cache rows of one batch row for one query head (grouped-query: its key head is h / (heads / kv_heads);
// the query heads that share a key head read the same rows, which the Infinity Cache serves after the first); each
// lane scores one row (its keys' loads all in flight), the wave takes its largest score and sum of exps, then each
// lane accumulates p * v for its dimensions (the wave's 64 rows of values loaded one row per instruction, all in
// flight); the waves meet in LDS and the chunk's (max, sum, p v) goes to the workspace, or, when the row's keys fit one
// chunk, o itself. The second kernel combines the chunks of each (row, head) by exp(max - the largest). A kernel
// boundary, not a fence, orders the two. A row reads only the cache rows its place reaches.
#include <math.h>
#include "fh_common.h"

namespace fh {

constexpr int ATT_WAVES = 2;                 // waves a workgroup, 64 cache rows each
constexpr int ATT_CHUNK = 64 * ATT_WAVES;    // cache rows a workgroup

struct AttArgs {
  const float* q; const void* cache; int64_t cache_len;
  int heads, kv_heads; float scale;
  const int32_t* places; const int32_t* first_row;
  int max_chunks;
  float* o;
  float* part;          // [batch][heads][max_chunks][hd + 2]: p v, then max, then sum
};

// the row's cache rows, kept inside the cache and the launch's chunks whatever the places say
__device__ inline void row_range(const AttArgs& a, int b, int64_t& row0, int64_t& length) {
  row0 = a.first_row[b];
  row0 = row0 < 0 ? 0 : (row0 >= a.cache_len ? a.cache_len - 1 : row0);
  length = (int64_t)a.places[b] + 1;
  const int64_t room = a.cache_len - row0 < (int64_t)a.max_chunks * ATT_CHUNK ? a.cache_len - row0 : (int64_t)a.max_chunks * ATT_CHUNK;
  length = length < 1 ? 1 : (length > room ? room : length);
}

template <int HD, bool BF>
__global__ __launch_bounds__(64 * ATT_WAVES) void attention_kernel(AttArgs a) {
  constexpr int DL = HD / 64;
  const int chunk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;  // h: the query head (its key head h / rep)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kvh = h / (a.heads / a.kv_heads);
  int64_t row0, length;
  row_range(a, b, row0, length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (chunk >= nchunks) return;  // past the row's place

  __shared__ float qs[HD];
  __shared__ float ps[ATT_WAVES][64];
  __shared__ float wm[ATT_WAVES], wl[ATT_WAVES];
  __shared__ float wo[ATT_WAVES][HD];
  const int64_t w0 = (int64_t)chunk * ATT_CHUNK + 64 * wave;  // the wave's first row
  const int n = (int)(length - w0 < 64 ? (length - w0 > 0 ? length - w0 : 0) : 64);
  const int64_t t = w0 + (lane < n ? lane : (n > 0 ? n - 1 : 0));  // (a lane past the rows reads the last, unused)
  const bool valid = lane < n;

  // every load at once: q, the lane's row of keys, and the wave's 64 rows of values (a lane its DL dimensions)
  float qv[(HD + 64 * ATT_WAVES - 1) / (64 * ATT_WAVES)];
#pragma unroll
  for (int i = 0; i < (int)(sizeof qv / sizeof qv[0]); ++i) {
    const int d = tid + 64 * ATT_WAVES * i;
    qv[i] = d < HD ? a.q[((int64_t)b * a.heads + h) * HD + d] : 0.f;
  }
  constexpr int EPL = BF ? 8 : 4;  // elements a 16-byte load
  uint4 kw[HD / EPL];
  const int64_t kb = ((int64_t)kvh * a.cache_len + row0 + t) * HD;
#pragma unroll
  for (int i = 0; i < HD / EPL; ++i) kw[i] = *(const uint4*)((const char*)a.cache + (kb + i * EPL) * (BF ? 2 : 4));
  // values kept as loaded (bf16 pairs stay packed: half the registers) and widened when used
  constexpr int VW = BF ? (DL + 1) / 2 : DL;  // 32-bit words a row a lane
  uint32_t v[64][VW];
  const int64_t vb = ((int64_t)(a.kv_heads + kvh) * a.cache_len + row0 + w0) * HD + DL * lane;
#pragma unroll
  for (int tt = 0; tt < 64; ++tt) {
    const int64_t at = vb + (int64_t)(tt < n ? tt : 0) * HD;
    if (BF && DL == 1) v[tt][0] = ((const uint16_t*)a.cache)[at];
    else if (BF && DL == 2) v[tt][0] = *(const uint32_t*)((const uint16_t*)a.cache + at);
    else if (BF) { const uint2 w = *(const uint2*)((const uint16_t*)a.cache + at); v[tt][0] = w.x; v[tt][VW - 1] = w.y; }
    else {
#pragma unroll
      for (int i = 0; i < VW; ++i) v[tt][i] = ((const uint32_t*)a.cache)[at + i];
    }
  }
#pragma unroll
  for (int i = 0; i < (int)(sizeof qv / sizeof qv[0]); ++i) {
    const int d = tid + 64 * ATT_WAVES * i;
    if (d < HD) qs[d] = qv[i];
  }
  __syncthreads();

  // the score of the lane's row: the dot with q (read from LDS, the same for every lane)
  float s2[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < HD / EPL; ++i) {
    const uint32_t w[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (BF) {
        s2[0] = fmaf(qs[i * EPL + 2 * j], __uint_as_float(w[j] << 16), s2[0]);
        s2[1] = fmaf(qs[i * EPL + 2 * j + 1], __uint_as_float(w[j] & 0xFFFF0000u), s2[1]);
      } else {
        s2[j & 1] = fmaf(qs[i * EPL + j], __uint_as_float(w[j]), s2[j & 1]);
      }
    }
  }
  float mx = -INFINITY, sm = 0.f;
  if (n > 0) {
    const float sc = valid ? (s2[0] + s2[1]) * a.scale : -INFINITY;
    mx = wave_max(sc);
    const float p = valid ? expf(sc - mx) : 0.f;
    sm = wave_sum(p);
    ps[wave][lane] = p;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // p v (rows past n have p = 0)
  float o[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) o[i] = 0.f;
  if (n > 0) {
#pragma unroll
    for (int tt = 0; tt < 64; ++tt) {
      const float p = ps[wave][tt];
#pragma unroll
      for (int i = 0; i < DL; ++i) {
        const float x = BF ? __uint_as_float(i % 2 ? v[tt][i / 2] & 0xFFFF0000u : v[tt][i / 2] << 16) : __uint_as_float(v[tt][i]);
        o[i] = fmaf(p, x, o[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < DL; ++i) wo[wave][DL * lane + i] = o[i];
  if (lane == 0) { wm[wave] = mx; wl[wave] = sm; }
  __syncthreads();

  // the workgroup's waves combined, a thread a dimension; o itself when the row has one chunk
  const bool alone = nchunks == 1;
  for (int d = tid; d < HD; d += 64 * ATT_WAVES) {
    float big = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) big = fmaxf(big, wm[w]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      if (wm[w] == -INFINITY) continue;  // a wave past the row's place
      const float e = expf(wm[w] - big);
      num = fmaf(e, wo[w][d], num);
      den = fmaf(e, wl[w], den);
    }
    if (alone) {
      a.o[((int64_t)b * a.heads + h) * HD + d] = num / den;
    } else {
      float* pp = a.part + (((int64_t)b * a.heads + h) * a.max_chunks + chunk) * (HD + 2);
      pp[d] = num;
      if (d == 0) { pp[HD] = big; pp[HD + 1] = den; }
    }
  }
}

// the chunks of row blockIdx.y, head blockIdx.x combined: a thread a dimension, every chunk's loads in flight
template <int HD>
__global__ __launch_bounds__(HD) void attention_combine(AttArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int64_t row0, length;
  row_range(a, b, row0, length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (nchunks == 1) return;  // the first kernel wrote o
  const float* pp = a.part + ((int64_t)b * a.heads + h) * a.max_chunks * (HD + 2);
  float big = -INFINITY, num = 0.f, den = 0.f;
  for (int c0 = 0; c0 < nchunks; c0 += 16) {  // 16 chunks' loads at once, the running sums rescaled to a new largest
    float m16[16], l16[16], v16[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool ok = c0 + j < nchunks;
      const float* q = pp + (int64_t)(ok ? c0 + j : c0) * (HD + 2);
      m16[j] = ok ? q[HD] : -INFINITY; l16[j] = q[HD + 1]; v16[j] = q[d];
    }
    float top = big;
#pragma unroll
    for (int j = 0; j < 16; ++j) top = fmaxf(top, m16[j]);
    if (big != -INFINITY) { const float f = expf(big - top); num *= f; den *= f; }
    big = top;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (m16[j] == -INFINITY) continue;
      const float e = expf(m16[j] - big);
      num = fmaf(e, v16[j], num);
      den = fmaf(e, l16[j], den);
    }
  }
  a.o[((int64_t)b * a.heads + h) * HD + d] = num / den;
}


}  // namespace fh

using namespace fh;

extern "C" size_t fh_attention_workspace_bytes(int batch, int heads, int head_dim, int64_t max_context) {
  if (batch < 1 || heads < 1 || head_dim < 1 || max_context < 1) return 0;
  const int64_t chunks = (max_context + ATT_CHUNK - 1) / ATT_CHUNK;
  return (size_t)batch * heads * chunks * (head_dim + 2) * sizeof(float);
}

extern "C" int fh_attention_decode(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch,
                                   int heads, int kv_heads, int head_dim, const int32_t* places, const int32_t* first_row,
                                   int64_t max_context, float* o, void* workspace, size_t ws_bytes, void* stream) {
  if (!q || !cache || !places || !first_row || !o) return fail(FH_EINVAL, "fh_attention_decode: null pointer");
  if (batch < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads)
    return fail(FH_EINVAL, "fh_attention_decode: heads must be a multiple of kv_heads");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail(FH_EUNSUP, "fh_attention_decode: head_dim 64, 128 or 256");
  if (cache_dtype != FH_F32 && cache_dtype != FH_BF16) return fail(FH_EUNSUP, "fh_attention_decode: cache is FH_F32 or FH_BF16");
  if (max_context < 1 || max_context > cache_len) return fail(FH_EINVAL, "fh_attention_decode: max_context outside 1..cache_len");
  const size_t need = fh_attention_workspace_bytes(batch, heads, head_dim, max_context);
  if (max_context > ATT_CHUNK && (!workspace || ws_bytes < need))
    return fail(FH_EINVAL, "fh_attention_decode: workspace smaller than fh_attention_workspace_bytes");
  AttArgs a;
  a.q = q; a.cache = cache; a.cache_len = cache_len;
  a.heads = heads; a.kv_heads = kv_heads; a.scale = 1.0f / sqrtf((float)head_dim);
  a.places = places; a.first_row = first_row;
  a.max_chunks = (int)((max_context + ATT_CHUNK - 1) / ATT_CHUNK);
  a.o = o;
  a.part = (float*)workspace;
  dim3 grid(a.max_chunks, heads, batch), block(64 * ATT_WAVES);
  hipStream_t s = as_stream(stream);
  const bool bf = cache_dtype == FH_BF16;
  const dim3 cgrid(heads, batch);
  switch (head_dim) {
    case 64: if (bf) hipLaunchKernelGGL((attention_kernel<64, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<64, false>), grid, block, 0, s, a);
             if (a.max_chunks > 1) hipLaunchKernelGGL(attention_combine<64>, cgrid, dim3(64), 0, s, a); break;
    case 128: if (bf) hipLaunchKernelGGL((attention_kernel<128, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<128, false>), grid, block, 0, s, a);
              if (a.max_chunks > 1) hipLaunchKernelGGL(attention_combine<128>, cgrid, dim3(128), 0, s, a); break;
    default: if (bf) hipLaunchKernelGGL((attention_kernel<256, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<256, false>), grid, block, 0, s, a);
             if (a.max_chunks > 1) hipLaunchKernelGGL(attention_combine<256>, cgrid, dim3(256), 0, s, a); break;
  }
  return check_launch("fh_attention_decode");
}
