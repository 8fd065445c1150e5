// Elementwise programs (fh_program): ferrite's fused elementwise trees, evaluated per output element in fp32. Used by
// the map and reduce kernels and as the matmul kernels' FH_EP_PROGRAM epilogue.
#pragma once
#include <math.h>
#include "fh_common.h"

namespace fh {

// An input's element at (b, r, c) as fp32 (bf16 exactly, int32 by value: exact below 2^24, as ferrite's int32 goes
// through fp32 for what it does not do itself)
__device__ inline float prog_input(const fh_program& p, int k, int64_t b, int64_t r, int64_t c) {
  const int64_t at = b * p.in_stride[k][0] + r * p.in_stride[k][1] + c * p.in_stride[k][2];
  const int d = p.in_dtype[k];
  if (d == FH_BF16) return bf16_to_f(((const uint16_t*)p.in[k])[at]);
  if (d == FH_I32) return (float)((const int32_t*)p.in[k])[at];
  return ((const float*)p.in[k])[at];
}

__device__ inline float prog_apply(int op, float x, float y) {
  switch (op) {
    case FH_OP_ADD: return x + y;
    case FH_OP_SUB: return x - y;
    case FH_OP_MUL: return x * y;
    case FH_OP_MAX: return fmaxf(x, y);
    case FH_OP_CMPLT: return x < y ? 1.f : 0.f;
    case FH_OP_CMPNE: return x != y ? 1.f : 0.f;
    case FH_OP_KEEP: return x != 0.f ? y : 0.f;   // where(c, y, .)'s half: y where c is not 0 (c = x)
    case FH_OP_DROP: return x == 0.f ? y : 0.f;   // and its other half: y where c is 0
    case FH_OP_RELU: return fmaxf(x, 0.f);
    case FH_OP_EXP: return expf(x);
    case FH_OP_EXP2: return exp2f(x);
    case FH_OP_LOG: return logf(x);
    case FH_OP_LOG2: return log2f(x);
    case FH_OP_SIN: return sinf(x);
    case FH_OP_COS: return cosf(x);
    case FH_OP_RECIP: return 1.f / x;
    case FH_OP_SQRT: return sqrtf(x);
    case FH_OP_FTOB: return __uint_as_float((__float_as_uint(x) + 0x8000u) & 0xFFFF0000u);  // to bf16, half up
    case FH_OP_FTOI: return truncf(x);
    default: return x;  // FH_OP_ITOF, FH_OP_COPY
  }
}

// the program's value at (b, r, c); acc: the matmul's result in an epilogue (0 elsewhere)
__device__ inline float prog_eval(const fh_program& p, float acc, int64_t b, int64_t r, int64_t c) {
  float reg[FH_MAX_OPS];
  float last = acc;
#pragma unroll
  for (int i = 0; i < FH_MAX_OPS; ++i) {
    if (i < p.n_ops) {
      float xy[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int code = s ? p.b[i] : p.a[i];
        float v = 0.f;
        if (code == FH_OPND_ACC) v = acc;
        else if (code == FH_OPND_IMM) v = p.imm[i];
        else if (code >= 16) v = prog_input(p, code - 16, b, r, c);
        else {
#pragma unroll
          for (int j = 0; j < i; ++j) v = code == j ? reg[j] : v;  // (static indices: the registers stay registers)
        }
        xy[s] = v;
      }
      reg[i] = prog_apply(p.op[i], xy[0], xy[1]);
      last = reg[i];
    }
  }
  return last;
}

__device__ inline void prog_store(void* out, int dtype, int64_t at, float v) {
  if (dtype == FH_BF16) ((uint16_t*)out)[at] = (uint16_t)bf16_rne_f(v);
  else if (dtype == FH_I32) ((int32_t*)out)[at] = (int32_t)truncf(v);
  else ((float*)out)[at] = v;
}

// Host check: operands refer to earlier ops, inputs it has, the matmul's result only where allowed
inline int check_program(const char* who, const fh_program* p, bool acc_ok) {
  char msg[160];
  auto bad = [&](const char* what) { snprintf(msg, sizeof msg, "%s: %s", who, what); return fail(FH_EINVAL, msg); };
  if (!p) return bad("null program");
  if (p->n_ops < 1 || p->n_ops > FH_MAX_OPS) return bad("a program holds 1 to 15 ops");
  if (p->n_inputs < 0 || p->n_inputs > FH_MAX_INPUTS) return bad("a program reads at most 8 inputs");
  for (int k = 0; k < p->n_inputs; ++k) {
    if (!p->in[k]) return bad("null input");
    if (p->in_dtype[k] != FH_F32 && p->in_dtype[k] != FH_BF16 && p->in_dtype[k] != FH_I32) return bad("inputs are FH_F32, FH_BF16 or FH_I32");
  }
  for (int i = 0; i < p->n_ops; ++i) {
    if (p->op[i] < FH_OP_ADD || p->op[i] > FH_OP_COPY) return bad("unknown op");
    for (int s = 0; s < 2; ++s) {
      const int code = s ? p->b[i] : p->a[i];
      const bool ok = (code >= 0 && code < i) || (code >= 16 && code < 16 + p->n_inputs) || code == FH_OPND_IMM ||
                      (code == FH_OPND_ACC && acc_ok);
      if (!ok) return bad("an operand refers to nothing the op can read");
    }
  }
  return FH_OK;
}

}  // namespace fh
