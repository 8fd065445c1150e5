// Decode attention over a KV cache, flash-decoding style. A workgroup (one wave) takes a chunk of 64 cache rows of one
// key/value head of one batch row and all the query heads that share it (grouped-query: heads / kv_heads of them):
// each lane scores one row against every query head, the wave takes the chunk's largest score and sum of exps, then
// each lane accumulates p * v over the chunk for its dimensions. A chunk's (max, sum, p v) goes to the workspace; the
// last chunk to finish (an atomic count per batch row and key head, reset by that workgroup) weights each chunk by
// exp(its max - the largest) and writes o. A row reads only the cache rows its place reaches.
#include <math.h>
#include "fh_common.h"

namespace fh {

constexpr int ATT_CHUNK = 64;
constexpr int ATT_MAX_REP = 8;

struct AttArgs {
  const float* q; const void* cache; int cache_bf16; int64_t cache_len;
  int heads, kv_heads, hd; float scale;
  const int32_t* places; const int32_t* first_row;
  int max_chunks;
  float* o;
  unsigned* counters;   // [batch][kv_heads]
  float* part;          // [batch][heads][max_chunks][hd + 2]: p v, then max, then sum
};

__device__ inline float cache_at(const void* c, int bf16, int64_t i) {
  return bf16 ? bf16_to_f(((const uint16_t*)c)[i]) : ((const float*)c)[i];
}

template <int HD>
__global__ __launch_bounds__(64) void attention_kernel(AttArgs a) {
  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int rep = a.heads / a.kv_heads;
  // rows first_row .. first_row + place, kept inside the cache and the launch's chunks whatever the places say
  int64_t row0 = a.first_row[b];
  row0 = row0 < 0 ? 0 : (row0 >= a.cache_len ? a.cache_len - 1 : row0);
  int64_t length = (int64_t)a.places[b] + 1;
  const int64_t room = a.cache_len - row0 < (int64_t)a.max_chunks * ATT_CHUNK ? a.cache_len - row0 : (int64_t)a.max_chunks * ATT_CHUNK;
  length = length < 1 ? 1 : (length > room ? room : length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (chunk >= nchunks) return;  // past the row's place: not counted
  const int64_t t0 = (int64_t)chunk * ATT_CHUNK;

  __shared__ float qs[ATT_MAX_REP][HD];
  __shared__ float ps[ATT_MAX_REP][ATT_CHUNK];
  for (int i = lane; i < rep * HD; i += 64) qs[i / HD][i % HD] = a.q[(int64_t)b * a.heads * HD + ((int64_t)kvh * rep) * HD + i];
  __syncthreads();

  // scores: a lane a cache row
  const int64_t t = t0 + lane;
  const bool valid = t < length;
  float s[ATT_MAX_REP];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r) s[r] = 0.f;
  if (valid) {
    const int64_t kbase = ((int64_t)kvh * a.cache_len + row0 + t) * HD;
    for (int d = 0; d < HD; d += 8) {
      float kv[8];
      if (a.cache_bf16) {
        uint4 w = *(const uint4*)((const uint16_t*)a.cache + kbase + d);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) { kv[2 * i] = bf16_to_f(ww[i] & 0xFFFFu); kv[2 * i + 1] = bf16_to_f(ww[i] >> 16); }
      } else {
        float4 w0 = *(const float4*)((const float*)a.cache + kbase + d), w1 = *(const float4*)((const float*)a.cache + kbase + d + 4);
        kv[0] = w0.x; kv[1] = w0.y; kv[2] = w0.z; kv[3] = w0.w; kv[4] = w1.x; kv[5] = w1.y; kv[6] = w1.z; kv[7] = w1.w;
      }
#pragma unroll
      for (int r = 0; r < ATT_MAX_REP; ++r) {
        if (r < rep) {
#pragma unroll
          for (int i = 0; i < 8; ++i) s[r] = fmaf(qs[r][d + i], kv[i], s[r]);
        }
      }
    }
  }
  float mx[ATT_MAX_REP], sum[ATT_MAX_REP];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r) {
    if (r < rep) {
      float sc = valid ? s[r] * a.scale : -INFINITY;
      mx[r] = wave_max(sc);
      float p = valid ? expf(sc - mx[r]) : 0.f;
      sum[r] = wave_sum(p);
      ps[r][lane] = p;
    }
  }
  __syncthreads();

  // p v: a lane HD / 64 dimensions
  constexpr int DL = HD / 64;
  float o[ATT_MAX_REP][DL];
#pragma unroll
  for (int r = 0; r < ATT_MAX_REP; ++r)
#pragma unroll
    for (int i = 0; i < DL; ++i) o[r][i] = 0.f;
  const int64_t vbase = ((int64_t)(a.kv_heads + kvh) * a.cache_len + row0 + t0) * HD;
  const int n = (int)(length - t0 < ATT_CHUNK ? length - t0 : ATT_CHUNK);
  for (int tt = 0; tt < n; ++tt) {
    float v[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) v[i] = cache_at(a.cache, a.cache_bf16, vbase + (int64_t)tt * HD + lane + 64 * i);
#pragma unroll
    for (int r = 0; r < ATT_MAX_REP; ++r) {
      if (r < rep) {
        const float p = ps[r][tt];
#pragma unroll
        for (int i = 0; i < DL; ++i) o[r][i] = fmaf(p, v[i], o[r][i]);
      }
    }
  }

  if (nchunks == 1) {  // the whole row in one chunk: no combine
    for (int r = 0; r < rep; ++r)
#pragma unroll
      for (int i = 0; i < DL; ++i) a.o[((int64_t)b * a.heads + kvh * rep + r) * HD + lane + 64 * i] = o[r][i] / sum[r];
    return;
  }
  for (int r = 0; r < rep; ++r) {
    float* pp = a.part + (((int64_t)b * a.heads + kvh * rep + r) * a.max_chunks + chunk) * (HD + 2);
#pragma unroll
    for (int i = 0; i < DL; ++i) pp[lane + 64 * i] = o[r][i];
    if (lane == 0) { pp[HD] = mx[r]; pp[HD + 1] = sum[r]; }
  }
  __threadfence();
  __shared__ unsigned last;
  if (lane == 0) last = atomicAdd(&a.counters[b * a.kv_heads + kvh], 1u) == (unsigned)(nchunks - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int r = 0; r < rep; ++r) {
    const float* pp = a.part + (((int64_t)b * a.heads + kvh * rep + r) * a.max_chunks) * (HD + 2);
    float big = -INFINITY;
    for (int c = 0; c < nchunks; ++c) big = fmaxf(big, pp[c * (HD + 2) + HD]);
    float acc[DL], den = 0.f;
#pragma unroll
    for (int i = 0; i < DL; ++i) acc[i] = 0.f;
    for (int c = 0; c < nchunks; ++c) {
      const float* q = pp + c * (HD + 2);
      const float w = expf(q[HD] - big);
      den = fmaf(w, q[HD + 1], den);
#pragma unroll
      for (int i = 0; i < DL; ++i) acc[i] = fmaf(w, q[lane + 64 * i], acc[i]);
    }
#pragma unroll
    for (int i = 0; i < DL; ++i) a.o[((int64_t)b * a.heads + kvh * rep + r) * HD + lane + 64 * i] = acc[i] / den;
  }
  if (lane == 0) atomicExch(&a.counters[b * a.kv_heads + kvh], 0u);  // ready for the next call
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
  a.q = q; a.cache = cache; a.cache_bf16 = cache_dtype == FH_BF16; a.cache_len = cache_len;
  a.heads = heads; a.kv_heads = kv_heads; a.hd = head_dim; a.scale = 1.0f / sqrtf((float)head_dim);
  a.places = places; a.first_row = first_row;
  a.max_chunks = (int)((max_context + ATT_CHUNK - 1) / ATT_CHUNK);
  a.o = o;
  a.counters = (unsigned*)workspace;
  a.part = workspace ? (float*)((char*)workspace + counter_bytes(batch, heads)) : nullptr;
  dim3 grid(a.max_chunks, kv_heads, batch), block(64);
  hipStream_t s = as_stream(stream);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(attention_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(attention_kernel<128>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(attention_kernel<256>, grid, block, 0, s, a); break;
  }
  return check_launch("fh_attention_decode");
}
