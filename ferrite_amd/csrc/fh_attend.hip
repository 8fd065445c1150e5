// The lazy Tensor's attend (ferrite/tensor.py:487-516): out[b][t] = softmax(q[b][t] k[b]^T + mask) v[b], the mask
// hiding every key after the row's place (and with a window, every key window or more before it). The general form,
// for any batch of query rows and keys (a model's decode step takes fh_attention_decode / fh_attention_prefill over
// its KV cache instead): a workgroup a query row, its q in LDS; its waves share the row's visible keys 64 at a time,
// a lane a key's score (q . k in fp32; its key row read 16 bytes a load where the rows allow it), an online softmax
// across a wave's chunks (running max and sum), and p v accumulated with a lane a dimension (head_dim up to 256; each
// key's p read from its lane by v_readlane); the waves' parts then combine in LDS. The result, p v over the sum of p,
// stored as bf16 (nearest even) or fp32.
#include <math.h>
#include <algorithm>
#include "fh_common.h"

namespace fh {

struct AttendArgs {
  const void* q; int q_f32; int64_t q_batch, ldq;
  const void* k; const void* v; int kv_f32; int64_t k_batch, ldk, v_batch, ldv;
  int64_t S, T; int hd;
  const int32_t* places; int64_t places_batch;
  int64_t window;
  void* out; int out_f32; int64_t out_batch, ldo;
  int k16;  // every key row starts on 16 bytes and head_dim fills whole 16-byte pieces: a lane reads its row 16 bytes a load
};

__device__ inline float at_load(const void* p, int f32, int64_t at) {
  return f32 ? ((const float*)p)[at] : bf16_to_f(((const uint16_t*)p)[at]);
}

template <int HDL>  // dimensions a lane holds: ceil(hd / 64)
__global__ __launch_bounds__(1024) void attend_kernel(AttendArgs a) {
  // a workgroup a query row (t, b), its NW waves sharing the row's visible keys: wave w takes the chunks of 64 keys
  // w, w + NW, ...; their (p v, max, sum) then meet in LDS (flash decoding inside the workgroup)
  __shared__ float qs[64 * HDL];
  __shared__ float part[16][64 * HDL + 2];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), NW = blockDim.x >> 6;
  const int64_t t = blockIdx.x, b = blockIdx.y;
  for (int d = threadIdx.x; d < 64 * HDL; d += blockDim.x) qs[d] = d < a.hd ? at_load(a.q, a.q_f32, b * a.q_batch + t * a.ldq + d) : 0.f;
  __syncthreads();
  const int64_t place = a.places[b * a.places_batch + t];
  const int64_t hi = place < a.S - 1 ? place : a.S - 1;
  int64_t lo = a.window > 0 ? place - a.window + 1 : 0;
  lo = lo < 0 ? 0 : lo;
  const char* kb = (const char*)a.k + b * a.k_batch * (a.kv_f32 ? 4 : 2);
  const char* vb = (const char*)a.v + b * a.v_batch * (a.kv_f32 ? 4 : 2);
  float m = -INFINITY, l = 0.f, acc[HDL];
#pragma unroll
  for (int i = 0; i < HDL; ++i) acc[i] = 0.f;
  for (int64_t j0 = lo + 64 * wave; j0 <= hi; j0 += 64 * NW) {
    const int64_t j = j0 + lane;
    const bool ok = j <= hi;
    float s = -INFINITY;
    if (ok && a.k16) {  // (16-byte pieces of the lane's key row: 8 bf16 or 4 fp32 values a load)
      s = 0.f;
      const uint4* kr = (const uint4*)(kb + j * a.ldk * (a.kv_f32 ? 4 : 2));
      const int pieces = a.hd / (a.kv_f32 ? 4 : 8);
      for (int pc = 0; pc < pieces; ++pc) {
        const uint4 w = kr[pc];
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
        if (a.kv_f32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) s = fmaf(qs[4 * pc + e], __uint_as_float(u[e]), s);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s = fmaf(qs[8 * pc + 2 * e], __uint_as_float(u[e] << 16), s);
            s = fmaf(qs[8 * pc + 2 * e + 1], __uint_as_float(u[e] & 0xFFFF0000u), s);
          }
        }
      }
    } else if (ok) {
      s = 0.f;
      for (int d = 0; d < a.hd; ++d) s = fmaf(qs[d], at_load(kb, a.kv_f32, j * a.ldk + d), s);
    }
    const float top = fmaxf(m, wave_max(s));
    const float p = ok ? expf(s - top) : 0.f;
    const float f = m == -INFINITY ? 0.f : expf(m - top);
    l = fmaf(l, f, wave_sum(p));
#pragma unroll
    for (int i = 0; i < HDL; ++i) acc[i] *= f;
    const int n = (int)(hi - j0 + 1 < 64 ? hi - j0 + 1 : 64);
    for (int jj = 0; jj < n; ++jj) {
      const float pj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), jj));  // (key jj's p, to every lane)
#pragma unroll
      for (int i = 0; i < HDL; ++i) {
        const int d = lane + 64 * i;
        if (d < a.hd) acc[i] = fmaf(pj, at_load(vb, a.kv_f32, (j0 + jj) * a.ldv + d), acc[i]);
      }
    }
    m = top;
  }
#pragma unroll
  for (int i = 0; i < HDL; ++i) part[wave][lane + 64 * i] = acc[i];
  if (lane == 0) { part[wave][64 * HDL] = m; part[wave][64 * HDL + 1] = l; }
  __syncthreads();
  if (wave != 0) return;
  float top = -INFINITY;
  for (int w = 0; w < NW; ++w) top = fmaxf(top, part[w][64 * HDL]);
  float den = 0.f, num[HDL];
#pragma unroll
  for (int i = 0; i < HDL; ++i) num[i] = 0.f;
  for (int w = 0; w < NW; ++w) {
    const float mw = part[w][64 * HDL];
    if (mw == -INFINITY) continue;  // (a wave that saw no key)
    const float c = expf(mw - top);
    den = fmaf(c, part[w][64 * HDL + 1], den);
#pragma unroll
    for (int i = 0; i < HDL; ++i) num[i] = fmaf(c, part[w][lane + 64 * i], num[i]);
  }
#pragma unroll
  for (int i = 0; i < HDL; ++i) {
    const int d = lane + 64 * i;
    if (d >= a.hd) continue;
    const float o = den > 0.f ? num[i] / den : 0.f;  // (a row that sees no key: zeros)
    const int64_t at = b * a.out_batch + t * a.ldo + d;
    if (a.out_f32) ((float*)a.out)[at] = o;
    else ((uint16_t*)a.out)[at] = (uint16_t)bf16_rne_f(o);
  }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_attend(const void* q, int q_dtype, int64_t q_batch_stride, int64_t ldq, const void* k, const void* v,
                         int kv_dtype, int64_t k_batch_stride, int64_t ldk, int64_t v_batch_stride, int64_t ldv, int64_t S,
                         int batch, int64_t T, int head_dim, const int32_t* places, int64_t places_batch_stride,
                         int64_t window, void* out, int out_dtype, int64_t out_batch_stride, int64_t ldo, void* stream) {
  if (!q || !k || !v || !places || !out) return fail(FH_EINVAL, "fh_attend: null pointer");
  if ((q_dtype != FH_F32 && q_dtype != FH_BF16) || (kv_dtype != FH_F32 && kv_dtype != FH_BF16) ||
      (out_dtype != FH_F32 && out_dtype != FH_BF16))
    return fail(FH_EINVAL, "fh_attend: q, k, v and out are FH_F32 or FH_BF16");
  if (batch < 1 || T < 1 || S < 1 || head_dim < 1 || head_dim > 256 || window < 0)
    return fail(FH_EINVAL, "fh_attend: need batch, T, S >= 1, 1 <= head_dim <= 256, window >= 0");
  if (ldq < head_dim || ldk < head_dim || ldv < head_dim || ldo < head_dim || q_batch_stride < 0 || k_batch_stride < 0 ||
      v_batch_stride < 0 || out_batch_stride < 0 || places_batch_stride < 0)
    return fail(FH_EINVAL, "fh_attend: a row stride below head_dim, or a negative batch stride");
  if (batch > 65535 || T > 0x7FFFFFFF) return fail(FH_EUNSUP, "fh_attend: batch or rows past the grid's limits");
  const int es = kv_dtype == FH_F32 ? 4 : 2;
  const int k16 = (uintptr_t)k % 16 == 0 && (k_batch_stride * es) % 16 == 0 && (ldk * es) % 16 == 0 && (head_dim * es) % 16 == 0;
  AttendArgs a = {q, q_dtype == FH_F32, q_batch_stride, ldq, k, v, kv_dtype == FH_F32, k_batch_stride, ldk, v_batch_stride,
                  ldv, S, T, head_dim, places, places_batch_stride, window, out, out_dtype == FH_F32, out_batch_stride, ldo, k16};
  // a workgroup a row, its waves sharing the keys: enough waves that each walks about 4 chunks of 64, at most 16
  const int64_t chunks = (S + 63) / 64;
  const int nw = (int)std::min<int64_t>(16, std::max<int64_t>(1, (chunks + 3) / 4));
  const dim3 grid((unsigned)T, (unsigned)batch), block(64 * nw);
  hipStream_t s = as_stream(stream);
  switch ((head_dim + 63) / 64) {
    case 1: hipLaunchKernelGGL(attend_kernel<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(attend_kernel<2>, grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL(attend_kernel<3>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(attend_kernel<4>, grid, block, 0, s, a); break;
  }
  return check_launch("fh_attend");
}
