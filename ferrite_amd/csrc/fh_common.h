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
