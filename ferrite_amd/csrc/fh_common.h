// Shared by the kernels of libferrite_hip.so: errors, launches, bf16 and block-float bit work, wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include "../../include/ferrite_hip.h"

namespace fh {

// The last error on this thread, for fh_last_error().
void set_error(const char* fmt, ...);
inline int fail(int code, const char* what) { set_error("%s", what); return code; }

// After a launch: a HIP error becomes FH_EHIP with its message.
int check_launch(const char* kernel);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- bf16 and the block floats, bit for bit ---------------------------------------------------------------------

// fp32 to bf16 bits, rounded to nearest even (models/gpt2.py:16-18 without packer)
__host__ __device__ inline uint32_t bf16_rne(uint32_t b) { return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16; }
__device__ inline uint32_t bf16_rne_f(float f) { return bf16_rne(__float_as_uint(f)); }
__device__ inline float bf16_to_f(uint32_t h) { return __uint_as_float(h << 16); }
// FH_BF16_T16: element (r, c) of bf16 rows of length ld in tiles of 16 rows, 8 columns of the 16 rows together
__host__ __device__ inline int64_t tile16_at(int64_t r, int64_t c, int64_t ld) {
  return (r >> 4) * 16 * ld + (c >> 3) * 128 + (r & 15) * 8 + (c & 7);
}

// One bf16 value's magnitude under a block exponent `top` (>= its own), as models/gpt2.py:25-31 rounds it: q for bfp8
// (7 bits, half up, at most 127) or for bfp4 (3 bits, nearest with ties up, at most 7, 0 from a shift of 4 on).
__device__ inline uint32_t bfp_magnitude(uint32_t bits, uint32_t top, bool four) {
  uint32_t e = (bits >> 7) & 255u, m = (bits & 127u) | (e ? 128u : 0u);
  uint32_t shift = top - e;
  if (four) {
    if (shift >= 4) return 0;
    uint32_t q = (m + (16u << shift)) >> (shift + 5);
    return q > 7 ? 7 : q;
  }
  if (shift > 8) shift = 8;
  uint32_t q = (m + (1u << shift)) >> (shift + 1);
  return q > 127 ? 127 : q;
}

// The bf16 bits of sign * q * 2^(top - 133), exactly (q <= 127 has at most 7 significant bits; below 2^-126 it is a
// bf16 subnormal, q << top). The values tensor._bf16s gives (ferrite/tensor.py:718-727) wherever those are normal.
__host__ __device__ inline uint32_t bfp_value_bf16(int32_t sq, uint32_t top) {
  uint32_t s = sq < 0, q = (uint32_t)(sq < 0 ? -sq : sq);
  if (q == 0) return 0;
  int nb = 31 - __builtin_clz(q);          // the top bit's place, 0..6
  int eb = (int)top + nb - 6;              // the biased exponent of q * 2^(top - 133)
  uint32_t out = eb >= 1 ? ((uint32_t)eb << 7) | ((q << (7 - nb)) & 127u) : (q << top);
  return (s << 15) | out;
}

// the 16 magnitudes of a run's row as floats: bfp8's 16 bytes are the signed q; bfp4's 8 bytes give 16 q (the 16 is
// folded into the scale: q * 2^(e - 129) = 16 q * 2^(e - 133))
__device__ inline void magnitudes(const uint4& m, float (&f)[16]) {
  const uint32_t w[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = (float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 255u);
}
__device__ inline void magnitudes(const uint2& m, float (&f)[16]) {
  const uint32_t w[2] = {m.x, m.y};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t hi = w[d] & 0xF0F0F0F0u, lo = (w[d] << 4) & 0xF0F0F0F0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[8 * d + 2 * i] = (float)(int8_t)((lo >> (8 * i)) & 255u);
      f[8 * d + 2 * i + 1] = (float)(int8_t)((hi >> (8 * i)) & 255u);
    }
  }
}

// 8 of a run's 16 magnitudes (columns 8h .. 8h + 7 of a row): bfp8's 8 bytes, bfp4's 4 bytes (16 q as above)
__device__ inline void magnitudes8(const uint2& m, float (&f)[8]) {
  const uint32_t w[2] = {m.x, m.y};
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = (float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 255u);
}
__device__ inline void magnitudes8(const uint32_t& m, float (&f)[8]) {
  const uint32_t hi = m & 0xF0F0F0F0u, lo = (m << 4) & 0xF0F0F0F0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = (float)(int8_t)((lo >> (8 * i)) & 255u);
    f[2 * i + 1] = (float)(int8_t)((hi >> (8 * i)) & 255u);
  }
}

// bfp4's 16 magnitudes offset by 8, through the chip's fp8 converter: a nibble's two's-complement q XOR 8 is q + 8 in
// 0..15, and an fp8 (OCP E4M3) byte of 0..15 is that integer times 2^-9 exactly (subnormal below 8, exponent field 1
// above), so f[j] = (q_j + 8) 2^-9. Per 8 values: a shift, two three-input bit operations (mask, then XOR 8) and four
// conversions of two values each (v_cvt_pk_f32_fp8), against a convert a value for magnitudes(). The caller takes
// the 8 2^-9 back out (once for all 16 columns: the sum of its scales times 2^-6).
typedef float fh_float2 __attribute__((ext_vector_type(2)));
__device__ inline void magnitudes_off8(const uint2& m, float (&f)[16]) {
  const uint32_t w[2] = {m.x, m.y};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t lo = (w[d] & 0x0F0F0F0Fu) ^ 0x08080808u, hi = ((w[d] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
    const fh_float2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
    const fh_float2 c = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false), e = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
    f[8 * d + 0] = a.x; f[8 * d + 2] = a.y; f[8 * d + 4] = b.x; f[8 * d + 6] = b.y;  // (low nibbles: even columns)
    f[8 * d + 1] = c.x; f[8 * d + 3] = c.y; f[8 * d + 5] = e.x; f[8 * d + 7] = e.y;
  }
}

// N values of a run of a block float as bf16, two a word (value 2i low, 2i + 1 high), exactly: f holds q (bfp8) or
// 16 q (bfp4, so both scale by 2^(top - 133)). q times a normal power of 2 is exact in fp32 (at most 7 significant
// bits) and its upper half is its bf16; a scale below fp32's normals (top < 7) takes bfp_value_bf16's integer path.
template <int N>
__device__ inline void bfp_run_bf16(const float (&f)[N], uint32_t top, uint32_t (&w)[N / 2]) {
  if (top >= 7) {
    const float sc = __uint_as_float((top - 6) << 23);
#pragma unroll
    for (int i = 0; i < N / 2; ++i)
      w[i] = __builtin_amdgcn_perm(__float_as_uint(f[2 * i + 1] * sc), __float_as_uint(f[2 * i] * sc), 0x07060302u);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) w[i] = bfp_value_bf16((int32_t)f[2 * i], top) | (bfp_value_bf16((int32_t)f[2 * i + 1], top) << 16);
  }
}

// A KV cache in a block float, [2 kv_heads][cache_len][head_dim] in one buffer: each row's magnitudes (head_dim bytes
// of two's-complement q for bfp8; head_dim / 2 for bfp4, values 2i and 2i + 1 in a byte's low and high nibble), all
// rows, then each row's head_dim / 16 exponents (a byte a run of 16), all rows.
__host__ __device__ inline int64_t kv_mant_row(int fmt, int hd) { return fmt == FH_BFP4 ? hd / 2 : hd; }
__host__ __device__ inline int64_t kv_exps_at(int fmt, int kv_heads, int64_t cache_len, int hd) {
  return 2 * (int64_t)kv_heads * cache_len * kv_mant_row(fmt, hd);
}

// ---- wave64 reductions ------------------------------------------------------------------------------------------

// Sum V values held by every lane over the wave's 64 lanes, transposing as it goes: at each lane bit (32 down to 1)
// while a lane holds more than one value, lanes with the bit set keep the upper half and send the lower, so each
// exchange halves what a lane holds; once one is left the rest is a plain butterfly. Afterwards lane l holds
// R = max(1, V / 64) sums, a[r] being the total of value index reduce_index<V>(l, r).
template <int V>
__device__ inline void wave_reduce_transpose(float (&a)[V]) {
  const int lane = threadIdx.x & 63;
  int n = V;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    if (n > 1) {
      const bool up = lane & m;
      const int h = n / 2;
#pragma unroll
      for (int i = 0; i < V / 2; ++i) {
        if (i < h) {
          float send = up ? a[i] : a[i + h];
          float keep = up ? a[i + h] : a[i];
          a[i] = keep + __shfl_xor(send, m, 64);
        }
      }
      n = h;
    } else {
      a[0] += __shfl_xor(a[0], m, 64);
    }
  }
}
template <int V>
__device__ inline int reduce_index(int lane, int r) {
  int n = V, idx = r;
  for (int m = 32; m >= 1; m >>= 1) {
    if (n > 1) { n /= 2; if (lane & m) idx += n; }
  }
  return idx;
}
// Whether lane holds a copy nobody else is responsible for (V < 64 leaves 64 / V lanes with each sum).
template <int V>
__device__ inline bool reduce_owner(int lane) { return V >= 64 || (lane & (64 / V - 1)) == 0; }

// DPP and lane-swap moves of gfx950 (a row is 16 lanes)
template <int CTRL>
__device__ inline float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_ROW_MIRROR = 0x140, DPP_ROW_HALF_MIRROR = 0x141, DPP_QUAD_XOR2 = 0x4E, DPP_QUAD_XOR1 = 0xB1;
// x's upper 32 lanes swapped with y's lower 32; then x holds x[l] (l < 32), y[l - 32] (l >= 32)
__device__ inline void swap32(float& x, float& y) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  x = __uint_as_float(r[0]); y = __uint_as_float(r[1]);
}
// in each 32-lane half, x's upper 16 lanes swapped with y's lower 16
__device__ inline void swap16(float& x, float& y) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  x = __uint_as_float(r[0]); y = __uint_as_float(r[1]);
}

// The 16 values a[0..15] of every lane summed over the wave, transposing as it goes: lane l ends with the total of
// value reduce16_index(l) in a[0] (four lanes, l & 3 = 0..3, hold each). Lane halves swap whole rows for the first two
// steps (permlane32/16 swaps: no LDS), DPP mirrors pair the lanes of a row for the next two, DPP quad moves finish.
__device__ inline void wave_reduce16(float (&a)[16]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 8; ++i) { swap32(a[i], a[i + 8]); a[i] += a[i + 8]; }  // lanes >= 32: value i + 8
#pragma unroll
  for (int i = 0; i < 4; ++i) { swap16(a[i], a[i + 4]); a[i] += a[i + 4]; }  // lanes with bit 4: value i + 4
  {
    const bool up = lane & 8;  // partner 15 - l within the row: the other bit-3 half
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float send = up ? a[i] : a[i + 2], keep = up ? a[i + 2] : a[i];
      a[i] = keep + dpp<DPP_ROW_MIRROR>(send);
    }
  }
  {
    const bool up = lane & 4;  // partner 7 - l within the half-row: the other bit-2 half
    const float send = up ? a[0] : a[1], keep = up ? a[1] : a[0];
    a[0] = keep + dpp<DPP_ROW_HALF_MIRROR>(send);
  }
  a[0] += dpp<DPP_QUAD_XOR2>(a[0]);
  a[0] += dpp<DPP_QUAD_XOR1>(a[0]);
}
__device__ inline int reduce16_index(int lane) { return ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1); }

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

}  // namespace fh
