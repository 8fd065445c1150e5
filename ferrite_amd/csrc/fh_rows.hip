// Rows by index, for the lazy Tensor's gather and put (ferrite/tensor.py:116-140: an embedding's lookup, a KV cache's
// put at each token's place) and for a block float's packed planes: a workgroup a (row, plane), its threads copying the
// row's bytes, 16 at a time where both rows allow it. Gather reads a bad index at the nearest row; put writes no row
// for an index outside the destination.
#include "fh_common.h"

namespace fh {

__global__ __launch_bounds__(256) void rows_kernel(const uint8_t* from, uint8_t* to, int64_t from_ld, int64_t from_plane,
                                                   int64_t to_ld, int64_t to_plane, int64_t row_bytes, const int32_t* ids,
                                                   int64_t limit, int put) {
  const int64_t j = blockIdx.x, p = blockIdx.y;
  int64_t id = ids[j];
  if (put && (id < 0 || id >= limit)) return;
  id = id < 0 ? 0 : (id >= limit ? limit - 1 : id);
  const uint8_t* src = from + p * from_plane + (put ? j : id) * from_ld;
  uint8_t* dst = to + p * to_plane + (put ? id : j) * to_ld;
  if ((((uintptr_t)src | (uintptr_t)dst | (uint64_t)row_bytes) & 15) == 0) {
    for (int64_t i = threadIdx.x; i < row_bytes / 16; i += 256) ((uint4*)dst)[i] = ((const uint4*)src)[i];
  } else {
    for (int64_t i = threadIdx.x; i < row_bytes; i += 256) dst[i] = src[i];
  }
}

static int rows_launch(const char* who, const void* from, void* to, int64_t from_ld, int64_t from_plane, int64_t to_ld,
                       int64_t to_plane, int64_t row_bytes, const int32_t* ids, int64_t n, int64_t limit, int64_t planes,
                       int put, void* stream) {
  char msg[128];
  if (!from || !to || !ids) { snprintf(msg, sizeof msg, "%s: null pointer", who); return fail(FH_EINVAL, msg); }
  if (n < 1 || limit < 1 || row_bytes < 1 || planes < 1 || from_ld < row_bytes || to_ld < row_bytes || from_plane < 0 || to_plane < 0) {
    snprintf(msg, sizeof msg, "%s: bad sizes", who);
    return fail(FH_EINVAL, msg);
  }
  if (n > 0x7FFFFFFF || planes > 65535) { snprintf(msg, sizeof msg, "%s: too many rows or planes", who); return fail(FH_EUNSUP, msg); }
  hipLaunchKernelGGL(rows_kernel, dim3((unsigned)n, (unsigned)planes), dim3(256), 0, as_stream(stream), (const uint8_t*)from,
                     (uint8_t*)to, from_ld, from_plane, to_ld, to_plane, row_bytes, ids, limit, put);
  return check_launch(who);
}

}  // namespace fh

using namespace fh;

extern "C" int fh_gather_rows(const void* src, int64_t src_rows, int64_t src_ld, int64_t src_plane, const int32_t* ids,
                              int64_t n, int64_t row_bytes, int64_t planes, void* out, int64_t out_ld, int64_t out_plane,
                              void* stream) {
  return rows_launch("fh_gather_rows", src, out, src_ld, src_plane, out_ld, out_plane, row_bytes, ids, n, src_rows, planes, 0, stream);
}

extern "C" int fh_put_rows(void* dst, int64_t dst_rows, int64_t dst_ld, int64_t dst_plane, const int32_t* ids, int64_t n,
                           int64_t row_bytes, int64_t planes, const void* src, int64_t src_ld, int64_t src_plane,
                           void* stream) {
  return rows_launch("fh_put_rows", src, dst, src_ld, src_plane, dst_ld, dst_plane, row_bytes, ids, n, dst_rows, planes, 1, stream);
}
