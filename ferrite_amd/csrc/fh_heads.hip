// Logit heads (models/serve.py:31-47; Head.of, 23-27): each row's k largest logits, largest first and the first
// column of equal values first (numpy's stable argsort; topk_kernel, ferrite/compiler.py:1716-1838), and given the
// row's 1/temperature t, the log of the sum of exp(x t) over the row. Two kernels, as heads() splits a row: (1) a
// workgroup per (row, part of 4096 columns) selects the part's k best and its largest value and sum of exp((x - max)
// t); (2) a workgroup per row selects the k best of the parts' candidates and combines the sums. Selection is exact:
// each value becomes an order-preserving 32-bit key, a radix select (four passes of 8 bits over an LDS histogram)
// finds the k-th largest key, the keys above it and the first of those equal to it (in column order) are gathered in
// column order by a workgroup scan, and one wave sorts the k by (key descending, column ascending) with a bitonic
// network. A row is read once from HBM.
#include <math.h>
#include "fh_common.h"

namespace fh {

constexpr int HT = 256;               // threads a workgroup
constexpr int HE = 16;                // (key, id) pairs a thread, consecutive in the workgroup's order
constexpr int HWIDTH = HT * HE;       // a part's columns, and the most candidates the merge takes

// a float as a key whose unsigned order is the floats' order (negative values flipped whole, positive ones' sign set;
// -0 and +0 one key, as they compare equal); key 0 is padding, below every value
__device__ inline uint32_t order_key(float v) {
  const uint32_t u = v == 0.f ? 0u : __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline bool before(uint32_t ka, int32_t ia, uint32_t kb, int32_t ib) { return ka > kb || (ka == kb && ia < ib); }

struct HeadSmem {
  uint32_t hist[256];
  uint32_t sel_key[64];
  int32_t sel_id[64];
  int scan[2][HT / 64];
  uint32_t bin, above;
  float red[HT / 64];
};

// inclusive sum over a wave's lanes
__device__ inline int wave_scan_incl(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// exclusive sums of a and b over the workgroup's threads in order
__device__ inline void block_scan2(int a, int b, int& ea, int& eb, HeadSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ia = wave_scan_incl(a), ib = wave_scan_incl(b);
  if (lane == 63) { sm.scan[0][wave] = ia; sm.scan[1][wave] = ib; }
  __syncthreads();
  int oa = 0, ob = 0;
  for (int w = 0; w < wave; ++w) { oa += sm.scan[0][w]; ob += sm.scan[1][w]; }
  ea = oa + ia - a;
  eb = ob + ib - b;
  __syncthreads();
}

__device__ inline float block_max(float v, HeadSmem& sm) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) sm.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = sm.red[0];
#pragma unroll
  for (int w = 1; w < HT / 64; ++w) m = fmaxf(m, sm.red[w]);
  __syncthreads();
  return m;
}
__device__ inline float block_sum(float v, HeadSmem& sm) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) sm.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < HT / 64; ++w) s += sm.red[w];
  __syncthreads();
  return s;
}

// The k (<= 64) best of the workgroup's (key, id) pairs, thread t holding pairs t HE .. t HE + HE - 1 of its order:
// the largest keys, and of a key equal to the k-th largest the first in that order (with ids increasing along the
// order among equal keys, the smallest ids). Written as keys and ids, best first, to out_k / out_i [0, k).
__device__ void block_topk(const uint32_t (&key)[HE], const int32_t (&id)[HE], int k, uint32_t* out_k, int32_t* out_i,
                           HeadSmem& sm) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0, mask = 0;
  int remaining = k;  // how many of the k are still to be found below the bins fixed so far
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += HT) sm.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < HE; ++j)
      if ((key[j] & mask) == prefix) atomicAdd(&sm.hist[(key[j] >> shift) & 255u], 1u);
    __syncthreads();
    if (tid < 64) {  // the bin holding the remaining-th largest: lane l takes bins 255 - 4l .. 252 - 4l, top down
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = sm.hist[255 - 4 * lane - q];
      const int s = (int)(c[0] + c[1] + c[2] + c[3]);
      const int incl = wave_scan_incl(s), excl = incl - s;
      if (excl < remaining && remaining <= incl) {
        int acc = excl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (acc + (int)c[q] >= remaining) { sm.bin = 255 - 4 * lane - q; sm.above = acc; break; }
          acc += (int)c[q];
        }
      }
    }
    __syncthreads();
    prefix |= sm.bin << shift;
    mask |= 0xFFu << shift;
    remaining -= (int)sm.above;
  }
  // prefix is the k-th largest key; `remaining` of the keys equal to it are among the k
  int gt = 0, eq = 0;
#pragma unroll
  for (int j = 0; j < HE; ++j) { gt += key[j] > prefix; eq += key[j] == prefix; }
  int gt_before, eq_before;
  block_scan2(gt, eq, gt_before, eq_before, sm);
  int pos = gt_before + min(eq_before, remaining), eq_rank = eq_before;
#pragma unroll
  for (int j = 0; j < HE; ++j) {
    const bool take = key[j] > prefix || (key[j] == prefix && eq_rank < remaining);
    if (key[j] == prefix) ++eq_rank;
    if (take) { sm.sel_key[pos] = key[j]; sm.sel_id[pos] = id[j]; ++pos; }
  }
  __syncthreads();
  if (tid < 64) {  // one wave sorts the k: bitonic, best first
    uint32_t kk = lane < k ? sm.sel_key[lane] : 0u;
    int32_t ii = lane < k ? sm.sel_id[lane] : 0x7FFFFFFF;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
      for (int stride = size / 2; stride > 0; stride >>= 1) {
        const uint32_t pk = (uint32_t)__shfl_xor((int)kk, stride, 64);
        const int32_t pi = __shfl_xor(ii, stride, 64);
        const bool forward = (lane & size) == 0 || size == 64, lower = (lane & stride) == 0;
        const bool mine_first = before(kk, ii, pk, pi);
        if ((lower == forward) != mine_first) { kk = pk; ii = pi; }
      }
    }
    if (lane < k) { out_k[lane] = kk; out_i[lane] = ii; }
  }
}

struct HeadArgs {
  const float* logits; int64_t ldl; int64_t vocab; int k; int parts;
  const float* inv_temp;
  float* values; int32_t* ids; float* lse;
  uint32_t* cand_k; int32_t* cand_i; float2* stats;  // [rows][parts][k], [rows][parts][k], [rows][parts]
};

// (1) a part of a row: its k best (keys and columns) and (max, sum of exp((x - max) t)); with one part, the outputs
__global__ __launch_bounds__(HT) void heads_part(HeadArgs a) {
  __shared__ HeadSmem sm;
  const int part = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int64_t c0 = (int64_t)part * HWIDTH + (int64_t)tid * HE;
  const float* x = a.logits + (int64_t)row * a.ldl;
  float v[HE];
  if (c0 + HE <= a.vocab) {
#pragma unroll
    for (int q = 0; q < HE / 4; ++q) {
      const float4 f = *(const float4*)(x + c0 + 4 * q);
      v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < HE; ++j) v[j] = c0 + j < a.vocab ? x[c0 + j] : -INFINITY;
  }
  uint32_t key[HE];
  int32_t id[HE];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < HE; ++j) {
    const bool ok = c0 + j < a.vocab;
    key[j] = ok ? order_key(v[j]) : 0u;
    id[j] = ok ? (int32_t)(c0 + j) : 0x7FFFFFFF;
    if (ok) m = fmaxf(m, v[j]);
  }
  const bool one = a.parts == 1;
  const int64_t at = ((int64_t)row * a.parts + part) * a.k;
  uint32_t* ok_ = one ? (uint32_t*)(a.values + (int64_t)row * a.k) : a.cand_k + at;
  int32_t* oi = one ? a.ids + (int64_t)row * a.k : a.cand_i + at;
  block_topk(key, id, a.k, ok_, oi, sm);
  __syncthreads();
  if (one && tid < a.k) a.values[(int64_t)row * a.k + tid] = x[oi[tid]];  // (each pick's value as the row holds it)
  if (a.inv_temp) {
    const float t = a.inv_temp[row];
    m = block_max(m, sm);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < HE; ++j) s += c0 + j < a.vocab ? expf((v[j] - m) * t) : 0.f;
    s = block_sum(s, sm);
    if (tid == 0) {
      if (one) a.lse[row] = fmaf(m, t, logf(s));
      else a.stats[(int64_t)row * a.parts + part] = make_float2(m, s);
    }
  }
}

// (2) a row's parts merged: the k best of the parts' k each (laid out part by part, so equal keys stay in column
// order), and the sums combined at the largest max
__global__ __launch_bounds__(HT) void heads_merge(HeadArgs a) {
  __shared__ HeadSmem sm;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int n = a.parts * a.k;
  const uint32_t* ck = a.cand_k + (int64_t)row * n;
  const int32_t* ci = a.cand_i + (int64_t)row * n;
  uint32_t key[HE];
  int32_t id[HE];
#pragma unroll
  for (int j = 0; j < HE; ++j) {
    const int c = tid * HE + j;
    key[j] = c < n ? ck[c] : 0u;
    id[j] = c < n ? ci[c] : 0x7FFFFFFF;
  }
  uint32_t* out_k = (uint32_t*)(a.values + (int64_t)row * a.k);
  int32_t* out_i = a.ids + (int64_t)row * a.k;
  block_topk(key, id, a.k, out_k, out_i, sm);
  __syncthreads();
  if (tid < a.k) a.values[(int64_t)row * a.k + tid] = a.logits[(int64_t)row * a.ldl + out_i[tid]];
  if (a.inv_temp) {
    const float t = a.inv_temp[row];
    const float2* st = a.stats + (int64_t)row * a.parts;
    float m = -INFINITY;
    for (int p = tid; p < a.parts; p += HT) m = fmaxf(m, st[p].x);
    m = block_max(m, sm);
    float s = 0.f;
    for (int p = tid; p < a.parts; p += HT) s += st[p].y * expf((st[p].x - m) * t);
    s = block_sum(s, sm);
    if (tid == 0) a.lse[row] = fmaf(m, t, logf(s));
  }
}

static int64_t head_parts(int64_t vocab) { return (vocab + HWIDTH - 1) / HWIDTH; }

}  // namespace fh

using namespace fh;

extern "C" size_t fh_heads_workspace_bytes(int rows, int64_t vocab, int k) {
  if (rows < 1 || vocab < 1 || k < 1 || k > 64) return 0;
  const int64_t parts = head_parts(vocab);
  if (parts == 1) return 0;
  return (size_t)rows * parts * (k * 8 + sizeof(float2));
}

extern "C" int fh_logit_heads(const float* logits, int64_t ldl, int rows, int64_t vocab, int k, const float* inv_temp,
                              float* values, int32_t* ids, float* lse, void* workspace, size_t ws_bytes, void* stream) {
  if (!logits || !values || !ids) return fail(FH_EINVAL, "fh_logit_heads: null pointer");
  if (rows < 1 || k < 1 || k > 64 || vocab < k) return fail(FH_EINVAL, "fh_logit_heads: need rows >= 1, 1 <= k <= 64, vocab >= k");
  if (ldl < vocab || ldl % 4 || ((uintptr_t)logits & 15)) return fail(FH_EINVAL, "fh_logit_heads: rows 16-byte aligned, ldl >= vocab and a multiple of 4");
  if ((inv_temp == nullptr) != (lse == nullptr)) return fail(FH_EINVAL, "fh_logit_heads: lse and inv_temp go together");
  const int64_t parts = head_parts(vocab);
  if (parts * k > HWIDTH) return fail(FH_EUNSUP, "fh_logit_heads: vocabulary too wide for k (parts of 4096 columns, parts * k <= 4096)");
  if (rows > 65535) return fail(FH_EUNSUP, "fh_logit_heads: at most 65535 rows");
  const size_t need = fh_heads_workspace_bytes(rows, vocab, k);
  if (need && (!workspace || ws_bytes < need)) return fail(FH_EINVAL, "fh_logit_heads: workspace smaller than fh_heads_workspace_bytes");
  HeadArgs a = {};
  a.logits = logits; a.ldl = ldl; a.vocab = vocab; a.k = k; a.parts = (int)parts; a.inv_temp = inv_temp;
  a.values = values; a.ids = ids; a.lse = lse;
  if (parts > 1) {
    char* ws = (char*)workspace;
    a.cand_k = (uint32_t*)ws;
    a.cand_i = (int32_t*)(ws + (size_t)rows * parts * k * 4);
    a.stats = (float2*)(ws + (size_t)rows * parts * k * 8);
  }
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(heads_part, dim3((unsigned)parts, rows), dim3(HT), 0, s, a);
  if (parts > 1) hipLaunchKernelGGL(heads_merge, dim3(rows), dim3(HT), 0, s, a);
  return check_launch("fh_logit_heads");
}

namespace fh {

// out[r][j] = src[r][idx[r][j]] for 4-byte elements, an index outside [0, cols) read at the nearest column
__global__ __launch_bounds__(256) void gather_cols_kernel(const uint32_t* src, int64_t lds, int64_t cols, const int32_t* idx,
                                                          int64_t ldi, int64_t rows, int64_t k, uint32_t* out, int64_t ldo) {
  const int64_t n = rows * k;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / k, j = i % k;
    int64_t c = idx[r * ldi + j];
    c = c < 0 ? 0 : (c >= cols ? cols - 1 : c);
    out[r * ldo + j] = src[r * lds + c];
  }
}

}  // namespace fh

extern "C" int fh_gather_cols(const void* src, int64_t lds, int64_t cols, const int32_t* idx, int64_t ldi, int64_t rows,
                              int64_t k, void* out, int64_t ldo, void* stream) {
  if (!src || !idx || !out) return fail(FH_EINVAL, "fh_gather_cols: null pointer");
  if (rows < 1 || k < 1 || cols < 1 || lds < cols || ldi < k || ldo < k) return fail(FH_EINVAL, "fh_gather_cols: bad sizes");
  const int64_t blocks = (rows * k + 255) / 256;
  hipLaunchKernelGGL(gather_cols_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)src, lds, cols, idx, ldi, rows, k, (uint32_t*)out, ldo);
  return check_launch("fh_gather_cols");
}
