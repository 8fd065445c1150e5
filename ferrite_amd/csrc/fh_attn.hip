// Decode attention over a KV cache, flash-decoding style. A workgroup (four waves) takes a chunk of 256 cache rows of one
// key/value head of one batch row and all the query heads that share it (grouped-query: heads / kv_heads of them):
// each lane scores one row against every query head, the wave takes the chunk's largest score and sum of exps, then
// each lane accumulates p * v over the chunk for its dimensions. A chunk's (max, sum, p v) goes to the workspace; the
// last chunk to finish (an atomic count per batch row and key head, reset by that workgroup) weights each chunk by
// exp(its max - the largest) and writes o. A row reads only the cache rows its place reaches.
#include <math.h>
#include "fh_common.h"

namespace fh {

constexpr int ATT_WAVES = 4;                 // waves a workgroup, 64 cache rows each
constexpr int ATT_CHUNK = 64 * ATT_WAVES;    // cache rows a workgroup
constexpr int ATT_MAX_REP = 8;

struct AttArgs {
  const float* q; const void* cache; int64_t cache_len;
  int heads, kv_heads; float scale;
  const int32_t* places; const int32_t* first_row;
  int max_chunks;
  float* o;
  unsigned* counters;   // [batch][kv_heads]
  float* part;          // [batch][heads][max_chunks][hd + 2]: p v, then max, then sum
};

template <bool BF> __device__ inline float cval(const void* c, int64_t i) {
  return BF ? bf16_to_f(((const uint16_t*)c)[i]) : ((const float*)c)[i];
}

// Rows first_row[b] .. first_row[b] + places[b] of kv head blockIdx.y for row b = blockIdx.z, chunk blockIdx.x of
// ATT_CHUNK rows: wave w scores rows 64 w .. 64 w + 63 (a lane a row, its keys' loads all in flight), takes their max
// and sum of exps, then p v with a lane on HD / 64 dimensions (the 64 rows' values loaded a row per instruction, all
// in flight); the waves' results meet in LDS, the workgroup's goes to the workspace, and the last workgroup of the
// row's chunks to finish combines them.
template <int HD, bool BF>
__global__ __launch_bounds__(64 * ATT_WAVES) void attention_kernel(AttArgs a) {
  constexpr int DL = HD / 64;
  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rep = a.heads / a.kv_heads;
  // the row's cache rows, kept inside the cache and the launch's chunks whatever the places say
  int64_t row0 = a.first_row[b];
  row0 = row0 < 0 ? 0 : (row0 >= a.cache_len ? a.cache_len - 1 : row0);
  int64_t length = (int64_t)a.places[b] + 1;
  const int64_t room = a.cache_len - row0 < (int64_t)a.max_chunks * ATT_CHUNK ? a.cache_len - row0 : (int64_t)a.max_chunks * ATT_CHUNK;
  length = length < 1 ? 1 : (length > room ? room : length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (chunk >= nchunks) return;  // past the row's place: not counted

  __shared__ float qs[ATT_MAX_REP][HD];
  __shared__ float ps[ATT_WAVES][ATT_MAX_REP][64];
  __shared__ float wm[ATT_WAVES][ATT_MAX_REP], wl[ATT_WAVES][ATT_MAX_REP];
  __shared__ float wo[ATT_WAVES][ATT_MAX_REP][HD];
  for (int i = tid; i < rep * HD; i += 64 * ATT_WAVES) qs[i / HD][i % HD] = a.q[((int64_t)b * a.heads + (int64_t)kvh * rep) * HD + i];
  __syncthreads();

  const int64_t w0 = (int64_t)chunk * ATT_CHUNK + 64 * wave;  // the wave's first row
  const int n = (int)(length - w0 < 64 ? (length - w0 > 0 ? length - w0 : 0) : 64);
  const int64_t t = w0 + lane;
  const bool valid = lane < n;

  // scores
  float s[ATT_MAX_REP];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r) s[r] = 0.f;
  if (valid) {
    const int64_t kb = ((int64_t)kvh * a.cache_len + row0 + t) * HD;
    constexpr int EPL = BF ? 8 : 4;  // elements a 16-byte load
    uint4 kw[HD / EPL];
#pragma unroll
    for (int i = 0; i < HD / EPL; ++i) kw[i] = *(const uint4*)((const char*)a.cache + (kb + i * EPL) * (BF ? 2 : 4));
#pragma unroll
    for (int i = 0; i < HD / EPL; ++i) {
      const uint32_t w[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
      float kv[EPL];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (BF) { kv[2 * j] = bf16_to_f(w[j] & 0xFFFFu); kv[2 * j + 1] = bf16_to_f(w[j] >> 16); }
        else kv[j] = __uint_as_float(w[j]);
      }
#pragma unroll
      for (int r = 0; r < ATT_MAX_REP; ++r)
        if (r < rep) {
#pragma unroll
          for (int j = 0; j < EPL; ++j) s[r] = fmaf(qs[r][i * EPL + j], kv[j], s[r]);
        }
    }
  }
  float mx[ATT_MAX_REP], sm[ATT_MAX_REP];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r) {
    mx[r] = -INFINITY; sm[r] = 0.f;
    if (r < rep && n > 0) {
      const float sc = valid ? s[r] * a.scale : -INFINITY;
      mx[r] = wave_max(sc);
      const float p = valid ? expf(sc - mx[r]) : 0.f;
      sm[r] = wave_sum(p);
      ps[wave][r][lane] = p;
    }
  }
  // p v: lane on dimensions DL lane .. DL lane + DL - 1, a row's values one load across the wave
  float o[ATT_MAX_REP][DL];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r)
#pragma unroll
    for (int i = 0; i < DL; ++i) o[r][i] = 0.f;
  if (n > 0) {
    const int64_t vb = ((int64_t)(a.kv_heads + kvh) * a.cache_len + row0 + w0) * HD + DL * lane;
    float v[64][DL];
#pragma unroll
    for (int tt = 0; tt < 64; ++tt) {
#pragma unroll
      for (int i = 0; i < DL; ++i) v[tt][i] = tt < n ? cval<BF>(a.cache, vb + (int64_t)tt * HD + i) : 0.f;
    }
#pragma unroll
    for (int tt = 0; tt < 64; ++tt) {
#pragma unroll
      for (int r = 0; r < ATT_MAX_REP; ++r)
        if (r < rep) {
          const float p = ps[wave][r][tt];
#pragma unroll
          for (int i = 0; i < DL; ++i) o[r][i] = fmaf(p, v[tt][i], o[r][i]);
        }
    }
  }
  for (int r = 0; r < rep; ++r) {
#pragma unroll
    for (int i = 0; i < DL; ++i) wo[wave][r][DL * lane + i] = o[r][i];
    if (lane == 0) { wm[wave][r] = mx[r]; wl[wave][r] = sm[r]; }
  }
  __syncthreads();

  // the workgroup's waves combined: thread on (r, d) pairs
  const bool alone = nchunks == 1;
  for (int i = tid; i < rep * HD; i += 64 * ATT_WAVES) {
    const int r = i / HD, d = i % HD;
    float big = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) big = fmaxf(big, wm[w][r]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      if (wm[w][r] == -INFINITY) continue;  // a wave past the row's place
      const float e = expf(wm[w][r] - big);
      num = fmaf(e, wo[w][r][d], num);
      den = fmaf(e, wl[w][r], den);
    }
    const int64_t h = (int64_t)kvh * rep + r;
    if (alone) {
      a.o[((int64_t)b * a.heads + h) * HD + d] = num / den;
    } else {
      float* pp = a.part + (((int64_t)b * a.heads + h) * a.max_chunks + chunk) * (HD + 2);
      pp[d] = num;
      if (d == 0) { pp[HD] = big; pp[HD + 1] = den; }
    }
  }
  if (alone) return;
  __threadfence();
  __syncthreads();
  __shared__ unsigned last;
  if (tid == 0) last = atomicAdd(&a.counters[b * a.kv_heads + kvh], 1u) == (unsigned)(nchunks - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  // the row's chunks combined by the last to finish: thread on (r, d) pairs, every chunk's loads in flight
  for (int i = tid; i < rep * HD; i += 64 * ATT_WAVES) {
    const int r = i / HD, d = i % HD;
    const float* pp = a.part + (((int64_t)b * a.heads + (int64_t)kvh * rep + r) * a.max_chunks) * (HD + 2);
    float big = -INFINITY;
    for (int c = 0; c < nchunks; ++c) big = fmaxf(big, pp[c * (HD + 2) + HD]);
    float num = 0.f, den = 0.f;
    for (int c0 = 0; c0 < nchunks; c0 += 8) {
      float m8[8], l8[8], v8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = c0 + j < nchunks;
        const float* q = pp + (int64_t)(c0 + j) * (HD + 2);
        m8[j] = ok ? q[HD] : -INFINITY; l8[j] = ok ? q[HD + 1] : 0.f; v8[j] = ok ? q[d] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (m8[j] == -INFINITY) continue;
        const float e = expf(m8[j] - big);
        num = fmaf(e, v8[j], num);
        den = fmaf(e, l8[j], den);
      }
    }
    a.o[((int64_t)b * a.heads + (int64_t)kvh * rep + r) * HD + d] = num / den;
  }
  if (tid == 0) atomicExch(&a.counters[b * a.kv_heads + kvh], 0u);  // ready for the next call
}

static size_t counter_bytes(int batch, int heads) { return ((size_t)batch * heads * sizeof(unsigned) + 255) / 256 * 256; }

}  // namespace fh

using namespace fh;

extern "C" size_t fh_attention_workspace_bytes(int batch, int heads, int head_dim, int64_t max_context) {
  if (batch < 1 || heads < 1 || head_dim < 1 || max_context < 1) return 0;
  const int64_t chunks = (max_context + ATT_CHUNK - 1) / ATT_CHUNK;
  return counter_bytes(batch, heads) + (size_t)batch * heads * chunks * (head_dim + 2) * sizeof(float);
}

extern "C" int fh_attention_decode(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch,
                                   int heads, int kv_heads, int head_dim, const int32_t* places, const int32_t* first_row,
                                   int64_t max_context, float* o, void* workspace, size_t ws_bytes, void* stream) {
  if (!q || !cache || !places || !first_row || !o) return fail(FH_EINVAL, "fh_attention_decode: null pointer");
  if (batch < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads || heads / kv_heads > ATT_MAX_REP)
    return fail(FH_EINVAL, "fh_attention_decode: heads must be a multiple of kv_heads, at most 8 query heads a key head");
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
  a.counters = (unsigned*)workspace;
  a.part = workspace ? (float*)((char*)workspace + counter_bytes(batch, heads)) : nullptr;
  dim3 grid(a.max_chunks, kv_heads, batch), block(64 * ATT_WAVES);
  hipStream_t s = as_stream(stream);
  const bool bf = cache_dtype == FH_BF16;
  switch (head_dim) {
    case 64: if (bf) hipLaunchKernelGGL((attention_kernel<64, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<64, false>), grid, block, 0, s, a); break;
    case 128: if (bf) hipLaunchKernelGGL((attention_kernel<128, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<128, false>), grid, block, 0, s, a); break;
    default: if (bf) hipLaunchKernelGGL((attention_kernel<256, true>), grid, block, 0, s, a); else hipLaunchKernelGGL((attention_kernel<256, false>), grid, block, 0, s, a); break;
  }
  return check_launch("fh_attention_decode");
}
