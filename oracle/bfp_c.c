/* CPU restatement in C of ferrite's block-float rounding, models/gpt2.py:16-32 (bf16_bits, bfp): the same arithmetic
 * as oracle/bfp.py's numpy bfp_parts / bfp_values, run by run, for the multi-gigabyte weights of the full-width parity
 * tests (numpy takes about a minute for one 4096 x 28672 matrix; this, about a second).
 *
 * TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, as a
 * checker; the product (ferrite_amd) never does. Pinned in tests/test_oracle.py against oracle/bfp.py's bfp (itself
 * pinned by exact rational rounding of every (bf16 value, block exponent) pair), bit for bit. */
#include <stdint.h>
#include <math.h>

/* fp32 bits to bf16 bits, to nearest even (models/gpt2.py:16-18 without packer), in 64 bits as oracle/bfp.py does */
static inline uint32_t bf16_rne(uint32_t b) { return (uint32_t)((((uint64_t)b + 0x7FFFu + ((b >> 16) & 1u)) >> 16) & 0xFFFFu); }

/* One run of 16 bf16 values to its block float's values (models/gpt2.py:24-32): each value's magnitude under the run's
 * largest exponent `top`, 7 bits rounded half up and at most 127 (bfp8; a shift of 8 or more leaves 0), or 3 bits to the
 * nearest with ties up and at most 7, 0 from a shift of 4 (bfp4); the value q * 2^(top - 133) (bfp8), q * 2^(top - 129)
 * (bfp4), exactly (at most 7 significant bits, at least 2^-133: a float32, subnormal or not); a zero keeps no sign. */
static void run16(const uint32_t* bits, int four, float* out) {
  uint32_t top = 0;
  for (int i = 0; i < 16; ++i) { const uint32_t e = (bits[i] >> 7) & 255u; if (e > top) top = e; }
  for (int i = 0; i < 16; ++i) {
    const uint32_t b = bits[i], e = (b >> 7) & 255u, m = (b & 127u) | (e ? 128u : 0u);
    uint32_t shift = top - e, q;
    if (shift > 8) shift = 8;
    if (four) {
      if (shift < 4) { q = (m + (16u << shift)) >> (shift + 5); if (q > 7) q = 7; }
      else q = 0;
    } else {
      q = (m + (1u << shift)) >> (shift + 1);
      if (q > 127) q = 127;
    }
    const int ex = (int)top - (four ? 129 : 133);
    float v;
    if (ex >= -126) { const uint32_t sb = (uint32_t)(ex + 127) << 23; float sc; __builtin_memcpy(&sc, &sb, 4); v = (float)q * sc; }
    else v = ldexpf((float)q, ex);  /* (a scale below float32's normals) */
    out[i] = q == 0 ? 0.0f : ((b >> 15) ? -v : v);
  }
}

/* n values (a multiple of 16; runs of 16 consecutive values, the last axis of a row-major array) given as bf16 bits */
void oracle_bfp_bf16(const uint16_t* in, int64_t n, int four, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; r += 16) {
    uint32_t bits[16];
    for (int i = 0; i < 16; ++i) bits[i] = in[r + i];
    run16(bits, four, out + r);
  }
}

/* the same from fp32 values, each rounded to bf16 first (gpt2.bfp's bf16_bits) */
void oracle_bfp_f32(const float* in, int64_t n, int four, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; r += 16) {
    uint32_t bits[16];
    for (int i = 0; i < 16; ++i) { uint32_t u; __builtin_memcpy(&u, in + r + i, 4); bits[i] = bf16_rne(u); }
    run16(bits, four, out + r);
  }
}
