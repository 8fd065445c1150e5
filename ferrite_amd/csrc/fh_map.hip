// Lazy tensors' elementwise and reduction kernels: an fh_program evaluated at every element (fh_map), or folded along
// an axis (fh_reduce: sum or max). ferrite fuses the same trees into one Tensix kernel (fused_kernel,
// ferrite/compiler.py:699-1111; the reductions' FOLDS, 345-348); here each is one launch, memory-bound: a thread an
// element, its inputs read where the program's strides say (broadcasting by a stride of 0).
#include "fh_program.h"

namespace fh {

__global__ __launch_bounds__(256) void map_kernel(fh_program p, void* out, int out_dtype, int64_t batch, int64_t rows,
                                                  int64_t cols, int64_t ldb, int64_t ldo) {
  const int64_t n = batch * rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i % cols, r = (i / cols) % rows, b = i / (rows * cols);
    prog_store(out, out_dtype, b * ldb + r * ldo + c, prog_eval(p, 0.f, b, r, c));
  }
}

__device__ inline float fold(int kind, float a, float b) { return kind == FH_REDUCE_MAX ? fmaxf(a, b) : a + b; }

// along each row (axis 2): a workgroup a (batch, row), its threads striding the columns, then the wave and the
// workgroup folded in a fixed order
__global__ __launch_bounds__(256) void reduce_cols_kernel(fh_program p, int kind, int64_t rows, int64_t cols, void* out,
                                                          int out_dtype) {
  const int64_t r = blockIdx.x, b = blockIdx.y;
  const float id = kind == FH_REDUCE_MAX ? -INFINITY : 0.f;
  float acc = id;
  for (int64_t c = threadIdx.x; c < cols; c += 256) acc = fold(kind, acc, prog_eval(p, 0.f, b, r, c));
  acc = kind == FH_REDUCE_MAX ? wave_max(acc) : wave_sum(acc);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = part[0];
    for (int w = 1; w < 4; ++w) t = fold(kind, t, part[w]);
    prog_store(out, out_dtype, b * rows + r, t);
  }
}

// down the rows (axis 1) or over the batch (axis 0): a thread an output element, folding in order
__global__ __launch_bounds__(256) void reduce_lines_kernel(fh_program p, int kind, int axis, int64_t batch, int64_t rows,
                                                           int64_t cols, void* out, int out_dtype) {
  const int64_t outer = axis == 1 ? batch : rows;  // the other axis
  const int64_t n = outer * cols;
  const int64_t len = axis == 1 ? rows : batch;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i % cols, o = i / cols;
    float acc = kind == FH_REDUCE_MAX ? -INFINITY : 0.f;
    for (int64_t j = 0; j < len; ++j) {
      const int64_t b = axis == 1 ? o : j, r = axis == 1 ? j : o;
      acc = fold(kind, acc, prog_eval(p, 0.f, b, r, c));
    }
    prog_store(out, out_dtype, o * cols + c, acc);
  }
}

// a workgroup's fold of one value a thread, waves in order
__device__ inline float block_fold256(int kind, float v, float* part) {
  v = kind == FH_REDUCE_MAX ? wave_max(v) : wave_sum(v);
  __syncthreads();  // (part is reused)
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = part[0];
  for (int w = 1; w < 4; ++w) t = fold(kind, t, part[w]);
  return t;
}

// softmax (or log_softmax) along each row of the program's values: a workgroup a (batch, row), three passes over the
// row (its largest, the sum of exp(x - largest), the outputs), the program evaluated again each pass
__global__ __launch_bounds__(256) void softmax_rows_kernel(fh_program p, int log_form, int64_t rows, int64_t cols, void* out,
                                                           int out_dtype) {
  __shared__ float part[4];
  const int64_t r = blockIdx.x, b = blockIdx.y;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < cols; c += 256) m = fmaxf(m, prog_eval(p, 0.f, b, r, c));
  m = block_fold256(FH_REDUCE_MAX, m, part);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) s += expf(prog_eval(p, 0.f, b, r, c) - m);
  s = block_fold256(FH_REDUCE_SUM, s, part);
  if (out_dtype == FH_BF16) s = bf16_to_f(bf16_rne_f(s));  // (the composed form's sum is a tensor of the rows' dtype)
  const float ls = logf(s);
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float d = prog_eval(p, 0.f, b, r, c) - m;
    prog_store(out, out_dtype, (b * rows + r) * cols + c, log_form ? d - ls : expf(d) / s);
  }
}

static unsigned grid_for(int64_t n) {
  const int64_t g = (n + 255) / 256;
  return (unsigned)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace fh

using namespace fh;

extern "C" int fh_map(const fh_program* program, void* out, int out_dtype, int64_t batch, int64_t rows, int64_t cols,
                      int64_t ldb, int64_t ldo, void* stream) {
  if (int rc = check_program("fh_map", program, false)) return rc;
  // (each output element its own place: matrices one after another, or interleaved row by row: a merge's view)
  const bool apart = batch == 1 || ldb >= rows * ldo || (ldb >= cols && ldo >= batch * ldb);
  if (!out || batch < 1 || rows < 1 || cols < 1 || ldo < cols || ldb < 0 || !apart) return fail(FH_EINVAL, "fh_map: bad shape or strides");
  if (out_dtype != FH_F32 && out_dtype != FH_BF16 && out_dtype != FH_I32) return fail(FH_EINVAL, "fh_map: out is FH_F32, FH_BF16 or FH_I32");
  hipLaunchKernelGGL(map_kernel, dim3(grid_for(batch * rows * cols)), dim3(256), 0, as_stream(stream), *program, out,
                     out_dtype, batch, rows, cols, ldb, ldo);
  return check_launch("fh_map");
}

extern "C" int fh_reduce(const fh_program* program, int kind, int axis, int64_t batch, int64_t rows, int64_t cols,
                         void* out, int out_dtype, void* stream) {
  if (int rc = check_program("fh_reduce", program, false)) return rc;
  if (!out || batch < 1 || rows < 1 || cols < 1) return fail(FH_EINVAL, "fh_reduce: bad shape");
  if (kind != FH_REDUCE_SUM && kind != FH_REDUCE_MAX) return fail(FH_EINVAL, "fh_reduce: FH_REDUCE_SUM or FH_REDUCE_MAX");
  if (axis < 0 || axis > 2) return fail(FH_EINVAL, "fh_reduce: axis 0, 1 or 2");
  if (out_dtype != FH_F32 && out_dtype != FH_BF16 && out_dtype != FH_I32) return fail(FH_EINVAL, "fh_reduce: out is FH_F32, FH_BF16 or FH_I32");
  hipStream_t s = as_stream(stream);
  if (axis == 2) {
    if (rows >= (1LL << 31) || batch > 65535) return fail(FH_EUNSUP, "fh_reduce: too many rows");
    hipLaunchKernelGGL(reduce_cols_kernel, dim3((unsigned)rows, (unsigned)batch), dim3(256), 0, s, *program, kind, rows, cols, out, out_dtype);
  } else {
    const int64_t n = (axis == 1 ? batch : rows) * cols;
    hipLaunchKernelGGL(reduce_lines_kernel, dim3(grid_for(n)), dim3(256), 0, s, *program, kind, axis, batch, rows, cols, out, out_dtype);
  }
  return check_launch("fh_reduce");
}

extern "C" int fh_softmax_rows(const fh_program* program, int log_form, int64_t batch, int64_t rows, int64_t cols, void* out,
                               int out_dtype, void* stream) {
  if (int rc = check_program("fh_softmax_rows", program, false)) return rc;
  if (!out || batch < 1 || rows < 1 || cols < 1) return fail(FH_EINVAL, "fh_softmax_rows: bad shape");
  if (out_dtype != FH_F32 && out_dtype != FH_BF16) return fail(FH_EINVAL, "fh_softmax_rows: out is FH_F32 or FH_BF16");
  if (rows > 0x7FFFFFFF || batch > 65535) return fail(FH_EUNSUP, "fh_softmax_rows: too many rows");
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows, (unsigned)batch), dim3(256), 0, as_stream(stream), *program,
                     log_form, rows, cols, out, out_dtype);
  return check_launch("fh_softmax_rows");
}
