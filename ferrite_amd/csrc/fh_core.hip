// Errors, block-float packing and unpacking, embedding rows and argmax: the small kernels of libferrite_hip.so.
#include <stdarg.h>
#include <string.h>
#include "fh_common.h"

namespace fh {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
}

int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", kernel, hipGetErrorString(e));
    return FH_EHIP;
  }
  return FH_OK;
}

// ---- packing: one thread a block of 16 ---------------------------------------------------------------------------
// A block is (outer, inner): outer = the run of 16 (N/16 of them for FH_AXIS_N, K/16 for FH_AXIS_K), inner = the other
// axis's index. Its value j sits at src[inner * s_inner + outer * s_outer + j * s_elem]; its bytes go to
// mant[(outer * n_inner + inner) * (16 or 8)] and its exponent to exps[outer * n_inner + inner].
template <bool FOUR, bool BF16>
__global__ __launch_bounds__(256) void pack_kernel(const void* __restrict__ src, int64_t n_outer, int64_t n_inner,
                                                   int64_t s_outer, int64_t s_inner, int64_t s_elem,
                                                   uint8_t* __restrict__ mant, uint8_t* __restrict__ exps) {
  int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk >= n_outer * n_inner) return;
  int64_t outer = blk / n_inner, inner = blk % n_inner;
  const int64_t base = inner * s_inner + outer * s_outer;
  uint32_t bits[16];
  uint32_t top = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    uint32_t b;
    if (BF16) b = ((const uint16_t*)src)[base + j * s_elem];
    else b = bf16_rne(((const uint32_t*)src)[base + j * s_elem]);
    bits[j] = b;
    uint32_t e = (b >> 7) & 255u;
    top = e > top ? e : top;
  }
  exps[blk] = (uint8_t)top;
  if (!FOUR) {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      uint32_t q = bfp_magnitude(bits[j], top, false);
      int32_t sq = (bits[j] >> 15) && q ? -(int32_t)q : (int32_t)q;  // no sign on a zero
      w[j / 4] |= ((uint32_t)sq & 255u) << (8 * (j % 4));
    }
    *(uint4*)(mant + blk * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      uint32_t q = bfp_magnitude(bits[j], top, true);
      int32_t sq = (bits[j] >> 15) && q ? -(int32_t)q : (int32_t)q;
      w[j / 8] |= ((uint32_t)sq & 15u) << (4 * (j % 8));
    }
    *(uint2*)(mant + blk * 8) = make_uint2(w[0], w[1]);
  }
}

template <bool FOUR>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ mant, const uint8_t* __restrict__ exps,
                                                      int64_t n_outer, int64_t n_inner, int64_t s_outer, int64_t s_inner,
                                                      int64_t s_elem, uint16_t* __restrict__ out) {
  int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk >= n_outer * n_inner) return;
  int64_t outer = blk / n_inner, inner = blk % n_inner;
  const int64_t base = inner * s_inner + outer * s_outer;
  uint32_t top = exps[blk];
  // bfp4's q is worth q * 2^(top - 129) = (16 q) * 2^(top - 133)
  uint32_t w[4];
  if (!FOUR) {
    uint4 v = *(const uint4*)(mant + blk * 16);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    uint2 v = *(const uint2*)(mant + blk * 8);
    w[0] = v.x; w[1] = v.y;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    int32_t sq;
    if (!FOUR) sq = (int8_t)((w[j / 4] >> (8 * (j % 4))) & 255u);
    else sq = 16 * (((int32_t)((w[j / 8] >> (4 * (j % 8))) << 28)) >> 28);
    out[base + j * s_elem] = (uint16_t)bfp_value_bf16(sq, top);
  }
}

struct BlockGeom {
  int64_t n_outer, n_inner, s_outer, s_inner, s_elem;
};
static int geometry(int64_t K, int64_t N, int64_t ld, int axis, BlockGeom* g) {
  if (K <= 0 || N <= 0 || ld < N) return fail(FH_EINVAL, "bfp: need K > 0, N > 0 and ld >= N");
  if (axis == FH_AXIS_N) {
    if (N % 16) return fail(FH_EINVAL, "bfp along N: N must be a multiple of 16");
    *g = {N / 16, K, 16, ld, 1};
  } else if (axis == FH_AXIS_K) {
    if (K % 16) return fail(FH_EINVAL, "bfp along K: K must be a multiple of 16");
    *g = {K / 16, N, 16 * ld, 1, ld};
  } else {
    return fail(FH_EINVAL, "bfp: axis is FH_AXIS_N or FH_AXIS_K");
  }
  return FH_OK;
}

}  // namespace fh

using namespace fh;

extern "C" const char* fh_last_error(void) { return g_error; }

extern "C" const char* fh_version(void) { return "ferrite_hip 0.1 gfx950"; }

extern "C" int fh_bfp_bytes(int64_t K, int64_t N, int fmt, int axis, size_t* mant_bytes, size_t* exp_bytes) {
  BlockGeom g;
  if (int rc = geometry(K, N, N, axis, &g)) return rc;
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "bfp: fmt is FH_BFP8 or FH_BFP4");
  if (mant_bytes) *mant_bytes = (size_t)(K * N) / (fmt == FH_BFP8 ? 1 : 2);
  if (exp_bytes) *exp_bytes = (size_t)(K * N / 16);
  return FH_OK;
}

extern "C" int fh_bfp_pack(const void* src, int src_dtype, int64_t K, int64_t N, int64_t ld, int fmt, int axis,
                           void* mant, uint8_t* exps, void* stream) {
  BlockGeom g;
  if (int rc = geometry(K, N, ld, axis, &g)) return rc;
  if (!src || !mant || !exps) return fail(FH_EINVAL, "fh_bfp_pack: null pointer");
  if (src_dtype != FH_F32 && src_dtype != FH_BF16) return fail(FH_EINVAL, "fh_bfp_pack: src is FH_F32 or FH_BF16");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_bfp_pack: fmt is FH_BFP8 or FH_BFP4");
  int64_t blocks = g.n_outer * g.n_inner;
  dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
  hipStream_t s = as_stream(stream);
  auto m = (uint8_t*)mant;
  if (fmt == FH_BFP8) {
    if (src_dtype == FH_F32) hipLaunchKernelGGL((pack_kernel<false, false>), grid, block, 0, s, src, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, m, exps);
    else hipLaunchKernelGGL((pack_kernel<false, true>), grid, block, 0, s, src, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, m, exps);
  } else {
    if (src_dtype == FH_F32) hipLaunchKernelGGL((pack_kernel<true, false>), grid, block, 0, s, src, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, m, exps);
    else hipLaunchKernelGGL((pack_kernel<true, true>), grid, block, 0, s, src, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, m, exps);
  }
  return check_launch("fh_bfp_pack");
}

extern "C" int fh_bfp_dequant(const void* mant, const uint8_t* exps, int64_t K, int64_t N, int fmt, int axis,
                              uint16_t* out, int64_t ldo, void* stream) {
  BlockGeom g;
  if (int rc = geometry(K, N, ldo, axis, &g)) return rc;
  if (!mant || !exps || !out) return fail(FH_EINVAL, "fh_bfp_dequant: null pointer");
  if (fmt != FH_BFP8 && fmt != FH_BFP4) return fail(FH_EINVAL, "fh_bfp_dequant: fmt is FH_BFP8 or FH_BFP4");
  int64_t blocks = g.n_outer * g.n_inner;
  dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
  hipStream_t s = as_stream(stream);
  if (fmt == FH_BFP8) hipLaunchKernelGGL((dequant_kernel<false>), grid, block, 0, s, (const uint8_t*)mant, exps, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, out);
  else hipLaunchKernelGGL((dequant_kernel<true>), grid, block, 0, s, (const uint8_t*)mant, exps, g.n_outer, g.n_inner, g.s_outer, g.s_inner, g.s_elem, out);
  return check_launch("fh_bfp_dequant");
}

// ---- embedding rows: one workgroup a row, a thread a run of 16 columns ----------------------------------------------
// (each thread's run loaded at once, written, and its sum of squares taken from the registers: no barrier, no re-read)
template <bool BF16>
__global__ __launch_bounds__(256) void embed_kernel(const void* __restrict__ table, int64_t vocab, int64_t dim,
                                                    const int32_t* __restrict__ ids, float* __restrict__ x,
                                                    float* __restrict__ ssq) {
  const int b = blockIdx.x;
  int64_t id = ids[b];
  if (id < 0 || id >= vocab) id = 0;  // (the host checks ids it knows; one computed on the GPU reads row 0 rather than fault)
  for (int64_t run = threadIdx.x; run < dim / 16; run += blockDim.x) {
    float v[16];
    if (BF16) {
      const uint4* src = (const uint4*)((const uint16_t*)table + id * dim + run * 16);
      const uint4 lo = src[0], hi = src[1];
      const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) { v[2 * j] = __uint_as_float(w[j] << 16); v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u); }
    } else {
      const float4* src = (const float4*)((const float*)table + id * dim + run * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) { const float4 f = src[q]; v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w; }
    }
    float4* dst = (float4*)(x + b * dim + run * 16);
    float sq = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dst[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
#pragma unroll
      for (int j = 0; j < 4; ++j) sq = fmaf(v[4 * q + j], v[4 * q + j], sq);
    }
    if (ssq) ssq[b * (dim / 16) + run] = sq;
  }
}

extern "C" int fh_embed_rows(const void* table, int table_dtype, int64_t vocab, int64_t dim, const int32_t* ids,
                             int batch, float* x, float* ssq_out, void* stream) {
  if (!table || !ids || !x) return fail(FH_EINVAL, "fh_embed_rows: null pointer");
  if (vocab <= 0 || dim <= 0 || batch <= 0 || dim % 16) return fail(FH_EINVAL, "fh_embed_rows: bad sizes (dim a multiple of 16)");
  if (table_dtype != FH_F32 && table_dtype != FH_BF16) return fail(FH_EINVAL, "fh_embed_rows: table is FH_F32 or FH_BF16");
  if (((uintptr_t)table & 15) || ((uintptr_t)x & 15)) return fail(FH_EINVAL, "fh_embed_rows: table and x 16-byte aligned (runs of 16 loaded whole)");
  hipStream_t s = as_stream(stream);
  if (table_dtype == FH_BF16) hipLaunchKernelGGL((embed_kernel<true>), dim3(batch), dim3(256), 0, s, table, vocab, dim, ids, x, ssq_out);
  else hipLaunchKernelGGL((embed_kernel<false>), dim3(batch), dim3(256), 0, s, table, vocab, dim, ids, x, ssq_out);
  return check_launch("fh_embed_rows");
}

// ---- argmax of each row: one workgroup a row, the first of equal maxima ------------------------------------------
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t n, int32_t* __restrict__ ids) {
  const float* row = x + (int64_t)blockIdx.x * n;
  float best = -INFINITY;
  int64_t at = n;
  for (int64_t c = threadIdx.x; c < n; c += blockDim.x) {
    float v = row[c];
    if (v > best || (v == best && c < at)) { best = v; at = c; }  // (strictly greater keeps the first of equals)
  }
  // wave then workgroup: the larger value, the smaller column on a tie
  for (int m = 32; m >= 1; m >>= 1) {
    float ov = __shfl_xor(best, m, 64);
    int64_t oa = __shfl_xor(at, m, 64);
    if (ov > best || (ov == best && oa < at)) { best = ov; at = oa; }
  }
  __shared__ float bv[16];
  __shared__ int64_t ba[16];
  int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) { bv[w] = best; ba[w] = at; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < (int)(blockDim.x / 64); ++i)
      if (bv[i] > best || (bv[i] == best && ba[i] < at)) { best = bv[i]; at = ba[i]; }
    ids[blockIdx.x] = (int32_t)(at < n ? at : 0);
  }
}

extern "C" int fh_argmax_rows(const float* x, int64_t rows, int64_t n, int32_t* ids, void* stream) {
  if (!x || !ids || rows <= 0 || n <= 0 || n > INT32_MAX) return fail(FH_EINVAL, "fh_argmax_rows: bad arguments");
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, as_stream(stream), x, n, ids);
  return check_launch("fh_argmax_rows");
}

// ---- argmax from the GEMV's per-run pairs: one workgroup a row ---------------------------------------------------
// (1024 threads, each issuing its 8 loads of a round before comparing any: one memory round trip a round)
constexpr int AP_T = 1024, AP_U = 8;
__global__ __launch_bounds__(AP_T) void argmax_parts_kernel(const int2* __restrict__ parts, int64_t n, int32_t* __restrict__ ids) {
  const int2* row = parts + (int64_t)blockIdx.x * n;
  float best = -INFINITY;
  int at = INT32_MAX;
  for (int64_t c0 = 0; c0 < n; c0 += AP_T * AP_U) {
    int2 p[AP_U];
#pragma unroll
    for (int u = 0; u < AP_U; ++u) {
      const int64_t c = c0 + (int64_t)u * AP_T + threadIdx.x;
      p[u] = c < n ? row[c] : make_int2(__float_as_int(-INFINITY), INT32_MAX);
    }
#pragma unroll
    for (int u = 0; u < AP_U; ++u) {
      const float v = __int_as_float(p[u].x);
      if (v > best || (v == best && p[u].y < at)) { best = v; at = p[u].y; }
    }
  }
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(best, m, 64);
    const int oa = __shfl_xor(at, m, 64);
    if (ov > best || (ov == best && oa < at)) { best = ov; at = oa; }
  }
  __shared__ float bv[AP_T / 64];
  __shared__ int ba[AP_T / 64];
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) { bv[w] = best; ba[w] = at; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < AP_T / 64; ++i)
      if (bv[i] > best || (bv[i] == best && ba[i] < at)) { best = bv[i]; at = ba[i]; }
    ids[blockIdx.x] = at == INT32_MAX ? 0 : at;
  }
}

extern "C" int fh_argmax_parts(const void* parts, int64_t rows, int64_t nparts, int32_t* ids, void* stream) {
  if (!parts || !ids || rows <= 0 || nparts <= 0) return fail(FH_EINVAL, "fh_argmax_parts: bad arguments");
  hipLaunchKernelGGL(argmax_parts_kernel, dim3((unsigned)rows), dim3(AP_T), 0, as_stream(stream), (const int2*)parts, nparts, ids);
  return check_launch("fh_argmax_parts");
}

// The read floor a matmul's stream is measured against: `bytes` read once, 16 bytes a load, four loads in flight a
// thread, in a grid-stride walk of `blocks` workgroups of 256 threads; each workgroup's xor of every word it read
// goes to sink[block] (so that the loads are used)
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* src, int64_t n16, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) { const uint4 a = src[i]; acc ^= a.x ^ a.y ^ a.z ^ a.w; }
  for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// The matrix cores' own rate: each wave `iters` rounds of 8 independent accumulators, one MFMA each (32x32x16 bf16,
// form 0, or 16x16x32, form 1), operands from registers; each workgroup's sum of its results to sink[block]
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 probe_bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float probe_floatx16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float probe_floatx4;
template <int FORM>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, float* sink) {
  probe_bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(float)((threadIdx.x + i) & 7); b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7); }
  float total = 0.f;
  if constexpr (FORM == 0) {
    probe_floatx16 acc[8] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) total += acc[j][r];
  } else {
    probe_floatx4 acc[8] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) total += acc[j][r];
  }
  total = wave_sum(total);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = total;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// LDS read rate: each thread `iters` rounds of four 16-byte reads of a 16 KiB buffer at addresses that rotate with the
// round (every 16 lanes on distinct banks); each workgroup's xor of what it read to sink[block]
__global__ __launch_bounds__(256) void lds_probe_kernel(int iters, uint32_t* sink) {
  __shared__ __attribute__((aligned(16))) uint4 buf[1024];
  for (int i = threadIdx.x; i < 1024; i += 256) buf[i] = make_uint4(i, i * 3u, i * 5u, i * 7u);
  __syncthreads();
  uint32_t x = 0;
#pragma clang loop unroll(disable)
  for (int it = 0; it < iters; ++it) {  // (not unrolled: no round's reads can stand in for another's)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint4 v = buf[(threadIdx.x + 256 * u + 64 * it) & 1023];
      x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

extern "C" int fh_mfma_probe(int form, int iters, float* sink, int blocks, void* stream) {
  if (!sink || (form != 0 && form != 1) || iters < 1 || blocks < 1 || blocks > 65536)
    return fail(FH_EINVAL, "fh_mfma_probe: need sink, form 0 or 1, iters >= 1 and 1..65536 blocks");
  if (form == 0) hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(blocks), dim3(256), 0, as_stream(stream), iters, sink);
  else hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(blocks), dim3(256), 0, as_stream(stream), iters, sink);
  return check_launch("fh_mfma_probe");
}

extern "C" int fh_lds_probe(int iters, uint32_t* sink, int blocks, void* stream) {
  if (!sink || iters < 1 || blocks < 1 || blocks > 65536) return fail(FH_EINVAL, "fh_lds_probe: need sink, iters >= 1 and 1..65536 blocks");
  hipLaunchKernelGGL(lds_probe_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), iters, sink);
  return check_launch("fh_lds_probe");
}

extern "C" int fh_read_probe(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 || blocks < 1 || blocks > 65536)
    return fail(FH_EINVAL, "fh_read_probe: need src, sink, bytes a multiple of 16 and 1..65536 blocks");
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), (const uint4*)src,
                     (int64_t)(bytes / 16), sink);
  return check_launch("fh_read_probe");
}
