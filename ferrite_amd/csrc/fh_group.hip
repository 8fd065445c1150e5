// A mixture of experts' choices turned into the lists the lazy Tensor's indexed matmuls take (ferrite/tensor.py:389-416,
// Tensor.group and Tensor.touched; their kernels at compiler.py:1842-1945): integer bookkeeping over rows x k choices
// (values below n), one workgroup, in the choices' order (row by row, a row's choices in turn) so that every output is
// the reference's exactly.
#include "fh_common.h"

namespace fh {

// touched: the experts some row picks by a weight not 0, increasing, then n up to `slots` entries; weights[s][r] = the
// weight row r gave entry s's expert (0 if it did not pick it), as bf16 bits
__global__ __launch_bounds__(256) void touched_kernel(const int32_t* ids, int64_t ldi, const uint16_t* w, int64_t ldw, int rows,
                                                      int k, int n, int slots, int32_t* experts, uint16_t* weights) {
  extern __shared__ int32_t mark_list[];  // [n] marks, then [slots] the list
  int32_t* mark = mark_list;
  int32_t* list = mark_list + n;
  for (int e = threadIdx.x; e < n; e += 256) mark[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < rows * k; i += 256) {
    const int r = i / k, j = i % k, e = ids[(int64_t)r * ldi + j];
    if (w[(int64_t)r * ldw + j] && e >= 0 && e < n) mark[e] = 1;  // (a weight's bits not 0: +0 picks nothing)
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int count = 0;
    for (int e = 0; e < n && count < slots; ++e) if (mark[e]) list[count++] = e;
    for (; count < slots; ++count) list[count] = n;
  }
  __syncthreads();
  for (int s = threadIdx.x; s < slots; s += 256) experts[s] = list[s];
  for (int i = threadIdx.x; i < slots * rows; i += 256) {
    const int s = i / rows, r = i % rows, e = list[s];
    uint16_t v = 0;
    for (int j = 0; j < k; ++j) if (ids[(int64_t)r * ldi + j] == e) v = w[(int64_t)r * ldw + j];
    weights[i] = v;
  }
}

// group: each value's choices counted, its run of slots after the runs of the values before it, each rounded up to
// whole tiles of 32; each choice the next slot of its value's run. order[slot] = its row (0 for none), tiles[i] = tile
// i's value (n past those used), places[j rp + r] = the slot of row r's choice j (0 past the rows)
__global__ __launch_bounds__(64) void group_kernel(const int32_t* ids, int64_t ldi, int rows, int k, int n, int t, int rp,
                                                   int32_t* fill, int32_t* order, int32_t* tiles, int32_t* places) {
  for (int i = threadIdx.x; i < n; i += 64) fill[i] = 0;
  for (int i = threadIdx.x; i < 32 * t; i += 64) order[i] = 0;
  for (int i = threadIdx.x; i < t; i += 64) tiles[i] = n;
  for (int i = threadIdx.x; i < k * rp; i += 64) places[i] = 0;
  __syncthreads();
  if (threadIdx.x != 0) return;
  auto choice = [&](int r, int j) {
    const int e = ids[(int64_t)r * ldi + j];
    return e < 0 ? 0 : (e >= n ? n - 1 : e);  // (values below n; a bad one is kept inside the lists)
  };
  for (int r = 0; r < rows; ++r)
    for (int j = 0; j < k; ++j) fill[choice(r, j)]++;
  for (int e = 0, s = 0; e < n; ++e) {
    const int count = fill[e];
    fill[e] = s;
    for (const int end = s + (count + 31) / 32 * 32; s < end; s += 32) tiles[s / 32] = e;
  }
  for (int r = 0; r < rows; ++r)
    for (int j = 0; j < k; ++j) {
      const int s = fill[choice(r, j)]++;
      order[s] = r;
      places[j * rp + r] = s;
    }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_moe_touched(const int32_t* ids, int64_t ldi, const uint16_t* weights_in, int64_t ldw, int rows, int k,
                              int n, int32_t* experts, uint16_t* weights, void* stream) {
  if (!ids || !weights_in || !experts || !weights) return fail(FH_EINVAL, "fh_moe_touched: null pointer");
  if (rows < 1 || k < 1 || n < 1 || ldi < k || ldw < k) return fail(FH_EINVAL, "fh_moe_touched: bad sizes");
  const int64_t slots = (int64_t)rows * k < n ? (int64_t)rows * k : n;
  if ((int64_t)(n + slots) * 4 > 65536) return fail(FH_EUNSUP, "fh_moe_touched: at most ~8k experts");
  hipLaunchKernelGGL(touched_kernel, dim3(1), dim3(256), (size_t)(n + slots) * 4, as_stream(stream), ids, ldi, weights_in, ldw,
                     rows, k, n, (int)slots, experts, weights);
  return check_launch("fh_moe_touched");
}

extern "C" int fh_moe_group(const int32_t* ids, int64_t ldi, int rows, int k, int n, int32_t* order, int32_t* tiles,
                            int32_t* places, int32_t* workspace, void* stream) {
  if (!ids || !order || !tiles || !places || !workspace) return fail(FH_EINVAL, "fh_moe_group: null pointer");
  if (rows < 1 || k < 1 || n < 1 || ldi < k) return fail(FH_EINVAL, "fh_moe_group: bad sizes");
  const int64_t t = ((int64_t)rows * k + 31) / 32 + ((int64_t)rows * k < n ? (int64_t)rows * k : n), rp = ((int64_t)rows + 31) / 32 * 32;
  if (t * 32 > 0x7FFFFFFF || k * rp > 0x7FFFFFFF) return fail(FH_EUNSUP, "fh_moe_group: too many choices");
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(64), 0, as_stream(stream), ids, ldi, rows, k, n, (int)t, (int)rp, workspace,
                     order, tiles, places);
  return check_launch("fh_moe_group");
}
