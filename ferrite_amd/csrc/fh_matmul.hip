// The lazy Tensor's matmul of plain operands on the matrix cores: C[b] = program(A[b] @ B[b]), A [M][K] and B [K][N]
// each bf16 or fp32 (ferrite/tensor.py:443-485 with a bf16 or fp32 B). bf16 x bf16 products, exact in fp32, summed in
// fp32; an fp32 operand goes in as two bf16 parts, hi (its value rounded to nearest even) and lo (what hi leaves,
// rounded), and the sum is hi@hi + hi@lo + lo@hi (lo@lo, about 2^-16 of the rest, left out), ferrite's bf16x3
// (tensor.py:674-689): about 16 significant bits of each operand.
//
// A workgroup of 4 waves computes a 64 x 64 tile in K steps of 32: each thread loads 8 elements of A (a row's 8
// consecutive k) and 8 of B (a row's 8 consecutive columns), bounds-checked (any M, K, N, strides and alignment),
// splits them into bf16 parts and writes them to LDS, A's rows K-contiguous and B transposed to K-contiguous columns,
// as v_mfma_f32_32x32x16_bf16 takes its operands; each wave owns a 32 x 32 quarter. The epilogue evaluates the
// elementwise program (the fused ops on top of the matmul) at each output and stores it. This is the general path
// (batches, broadcasting by a batch stride of 0, any shape), not the block-float weights' hot path.
#include "fh_program.h"

namespace fh {

constexpr int MM_T = 64, MM_BK = 32, MM_LD = MM_BK + 8;  // tile, K step, LDS row (bf16: 80 bytes, banks spread)

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 mm_bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float mm_floatx16;

struct MmArgs {
  const void* a; int64_t sa, lda;
  const void* b; int64_t sb, ldb;
  int64_t M, K, N;
  void* c; int c_dtype; int64_t sc, ldc;
  int prog;  // whether the program runs (else the sum is stored)
};

__device__ inline float mm_load(const void* p, bool f32, int64_t at) {
  return f32 ? ((const float*)p)[at] : bf16_to_f(((const uint16_t*)p)[at]);
}

template <bool AF, bool BF>  // fp32 A, fp32 B: their lo parts too
__global__ __launch_bounds__(256) void matmul_kernel(MmArgs m, fh_program p) {
  __shared__ __attribute__((aligned(16))) uint16_t Ah[MM_T * MM_LD], Bh[MM_T * MM_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Al[AF ? MM_T * MM_LD : 8], Bl[BF ? MM_T * MM_LD : 8];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t bi = blockIdx.z, m0 = (int64_t)blockIdx.y * MM_T, n0 = (int64_t)blockIdx.x * MM_T;
  const char* A = (const char*)m.a + bi * m.sa * (AF ? 4 : 2);
  const char* B = (const char*)m.b + bi * m.sb * (BF ? 4 : 2);
  const int ar = t >> 2, ak = 8 * (t & 3);    // A: row ar of the tile, k ak .. ak + 7 of the step
  const int bk = t >> 3, bn = 8 * (t & 7);    // B: k row bk of the step, columns bn .. bn + 7 of the tile
  const int wr = 32 * (wave >> 1), wc = 32 * (wave & 1);
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  mm_floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;

  for (int64_t k0 = 0; k0 < m.K; k0 += MM_BK) {
    float av[8], bv[8];
    const int64_t r = m0 + ar, kb = k0 + bk;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = k0 + ak + j, n = n0 + bn + j;
      av[j] = (r < m.M && k < m.K) ? mm_load(A, AF, r * m.lda + k) : 0.f;
      bv[j] = (kb < m.K && n < m.N) ? mm_load(B, BF, kb * m.ldb + n) : 0.f;
    }
    __syncthreads();  // the last step's readers are done with the tiles
    uint32_t ah[8], al[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ah[j] = bf16_rne_f(av[j]);
      al[j] = AF ? bf16_rne_f(av[j] - bf16_to_f(ah[j])) : 0u;
    }
    *(uint4*)(Ah + ar * MM_LD + ak) = make_uint4(ah[0] | ah[1] << 16, ah[2] | ah[3] << 16, ah[4] | ah[5] << 16, ah[6] | ah[7] << 16);
    if (AF) *(uint4*)(Al + ar * MM_LD + ak) = make_uint4(al[0] | al[1] << 16, al[2] | al[3] << 16, al[4] | al[5] << 16, al[6] | al[7] << 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t h = bf16_rne_f(bv[j]);
      Bh[(bn + j) * MM_LD + bk] = (uint16_t)h;
      if (BF) Bl[(bn + j) * MM_LD + bk] = (uint16_t)bf16_rne_f(bv[j] - bf16_to_f(h));
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < MM_BK; kk += 16) {
      const mm_bf16x8 a_h = *(const mm_bf16x8*)(Ah + (wr + fr) * MM_LD + kk + fk);
      const mm_bf16x8 b_h = *(const mm_bf16x8*)(Bh + (wc + fr) * MM_LD + kk + fk);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, b_h, acc, 0, 0, 0);
      if (BF) {
        const mm_bf16x8 b_l = *(const mm_bf16x8*)(Bl + (wc + fr) * MM_LD + kk + fk);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, b_l, acc, 0, 0, 0);
      }
      if (AF) {
        const mm_bf16x8 a_l = *(const mm_bf16x8*)(Al + (wr + fr) * MM_LD + kk + fk);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, b_h, acc, 0, 0, 0);
      }
    }
  }

  // value r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of the wave's quarter
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = m0 + wr + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3), col = n0 + wc + (lane & 31);
    if (row < m.M && col < m.N) {
      const float v = m.prog ? prog_eval(p, acc[i], bi, row, col) : acc[i];
      prog_store(m.c, m.c_dtype, bi * m.sc + row * m.ldc + col, v);
    }
  }
}

}  // namespace fh

using namespace fh;

extern "C" int fh_matmul(const void* a, int a_dtype, int64_t a_batch_stride, int64_t lda, const void* b, int b_dtype,
                         int64_t b_batch_stride, int64_t ldb, int64_t batch, int64_t M, int64_t K, int64_t N,
                         const fh_program* program, void* c, int c_dtype, int64_t c_batch_stride, int64_t ldc,
                         void* stream) {
  if (!a || !b || !c) return fail(FH_EINVAL, "fh_matmul: null pointer");
  if ((a_dtype != FH_F32 && a_dtype != FH_BF16) || (b_dtype != FH_F32 && b_dtype != FH_BF16))
    return fail(FH_EINVAL, "fh_matmul: A and B are FH_F32 or FH_BF16");
  if (c_dtype != FH_F32 && c_dtype != FH_BF16 && c_dtype != FH_I32) return fail(FH_EINVAL, "fh_matmul: C is FH_F32, FH_BF16 or FH_I32");
  if (batch < 1 || M < 1 || K < 1 || N < 1) return fail(FH_EINVAL, "fh_matmul: batch, M, K and N at least 1");
  if (lda < K || ldb < N || ldc < N || a_batch_stride < 0 || b_batch_stride < 0 || c_batch_stride < 0)
    return fail(FH_EINVAL, "fh_matmul: a row stride below its row's length, or a negative batch stride");
  if (batch > 65535 || (M + MM_T - 1) / MM_T > 65535 || (N + MM_T - 1) / MM_T > (1LL << 31) - 1)
    return fail(FH_EUNSUP, "fh_matmul: batch or tiles past the grid's limits");
  if (program) {
    if (int rc = check_program("fh_matmul", program, true)) return rc;
  }
  MmArgs m = {a, a_batch_stride, lda, b, b_batch_stride, ldb, M, K, N, c, c_dtype, c_batch_stride, ldc, program != nullptr};
  fh_program p = program ? *program : fh_program{};
  const dim3 grid((unsigned)((N + MM_T - 1) / MM_T), (unsigned)((M + MM_T - 1) / MM_T), (unsigned)batch), block(256);
  hipStream_t s = as_stream(stream);
  const bool af = a_dtype == FH_F32, bf = b_dtype == FH_F32;
  if (af && bf) hipLaunchKernelGGL((matmul_kernel<true, true>), grid, block, 0, s, m, p);
  else if (af) hipLaunchKernelGGL((matmul_kernel<true, false>), grid, block, 0, s, m, p);
  else if (bf) hipLaunchKernelGGL((matmul_kernel<false, true>), grid, block, 0, s, m, p);
  else hipLaunchKernelGGL((matmul_kernel<false, false>), grid, block, 0, s, m, p);
  return check_launch("fh_matmul");
}
