// Decode attention over a KV cache, flash-decoding style, in two kernels. The first: a workgroup takes one key head
// of one batch row, with a wave for each query head that reads it (grouped-query: query head h reads key head h /
// (heads / kv_heads)), and walks chunks of 64 cache rows: split, split + S, split + 2S, ... where S workgroups share
// the row's chunks (S sized so the whole grid is resident at once). Its threads stage each chunk's keys and values in
// LDS (each byte of the cache read once from HBM) and issue the next chunk's loads into registers before the waves
// compute on this one, so the loads of one chunk overlap the arithmetic of the one before. Each wave scores the 64
// rows against its head's q (a lane a row; q read through the scalar unit, one address for the whole wave, where a
// workgroup walks several chunks; where it takes one, q is staged in LDS with the chunk's loads instead), keeps a
// running max and sum of exps across its chunks (online softmax), and accumulates p * v (a lane HD / 64 dimensions,
// four rows' p a broadcast read). A row whose chunks all fall to one workgroup writes o directly; otherwise each
// workgroup's (p v, max, sum) goes to the workspace, and the second kernel combines the S parts of each (row, head):
// a thread a part's statistics and a dimension's values, all loaded in one round with the row's place, one exp(max -
// the largest) a thread. A kernel boundary, not a fence, orders the two: on MI355X an agent-scope release (an L2
// write-back on each XCD) and a counter cost more than the ~1.4 us boundary. A row of at most 4 chunks (a short
// context) is one workgroup's instead (attention_short): a group of waves a chunk, the parts combined in LDS. A row reads only the cache rows its
// place reaches. A block-float cache (bfp8 or bfp4) is decoded into the same bf16 tiles as it is staged, exactly (a
// run's values are bf16 values), so its results are bit for bit a bf16 cache's of those values.
#include <math.h>
#include <algorithm>
#include <mutex>
#include <type_traits>
#include "fh_common.h"

namespace fh {

constexpr int ATT_CHUNK = 64;                // cache rows a chunk (a lane a row)
constexpr int ATT_REP = 16;                  // query heads a key head, at most (a wave each)

struct AttArgs {
  const float* q; const void* cache; int64_t cache_len; const uint8_t* cache_exps;
  int heads, kv_heads; float scale;
  const int32_t* places; const int32_t* first_row;
  int max_chunks;       // the launch's context in chunks (a row reads at most this many)
  int splits;           // S: workgroups a (row, key head), = gridDim.x
  void* o; int o_bf16; int o_tiles;  // the output, fp32 or bf16 (rounded to nearest even), rows or FH_BF16_T16 tiles
  int64_t o_ld;         // its row length: heads * head_dim
  float* part;          // [batch][heads][splits][hd + 2]: p v, then max, then sum
};

__device__ inline void put_o(const AttArgs& a, int b, int64_t col, float v) {
  const int64_t at = a.o_tiles ? tile16_at(b, col, a.o_ld) : b * a.o_ld + col;
  if (a.o_bf16) ((uint16_t*)a.o)[at] = (uint16_t)bf16_rne_f(v);
  else ((float*)a.o)[at] = v;
}

// the row's cache rows, kept inside the cache and the launch's chunks whatever the places say
__device__ inline void row_range(const AttArgs& a, int b, int64_t& row0, int64_t& length) {
  row0 = a.first_row[b];
  row0 = row0 < 0 ? 0 : (row0 >= a.cache_len ? a.cache_len - 1 : row0);
  length = (int64_t)a.places[b] + 1;
  const int64_t room = a.cache_len - row0 < (int64_t)a.max_chunks * ATT_CHUNK ? a.cache_len - row0 : (int64_t)a.max_chunks * ATT_CHUNK;
  length = length < 1 ? 1 : (length > room ? room : length);
}

// LDS a workgroup: keys and values [64][row + 16 bytes] (bf16, or fp32 for an fp32 cache), the heads' p [rep][64],
// and where q is staged, the heads' q [rep][HD] fp32
__host__ __device__ constexpr int att_row_bytes(int hd, int es) { return hd * es + 16; }
static size_t att_lds(int hd, int es, int rep, bool q_lds) {
  return (size_t)2 * ATT_CHUNK * att_row_bytes(hd, es) + (size_t)rep * ATT_CHUNK * 4 + (q_lds ? (size_t)rep * hd * 4 : 0);
}

// A chunk's keys and values, a thread's share of one round (4 pieces of each; a piece is 16 bytes of an fp32 or bf16
// row, or a run of 16 of a block float with its exponent byte): load() issues the round's loads into registers,
// store() writes them into the LDS tiles (a block float's runs decoded to bf16). Rows past the chunk's n read its last
// row (unused); pieces past the tile read its last piece again.
template <int HD, int CF>
struct ChunkLoader {
  static constexpr bool BLOCK = CF == FH_BFP8 || CF == FH_BFP4;
  static constexpr int ES = CF == FH_F32 ? 4 : 2;                 // bytes an element in LDS
  static constexpr int RW = att_row_bytes(HD, ES);
  static constexpr int PER_ROW = BLOCK ? HD / 16 : HD * ES / 16;   // pieces a row
  static constexpr int PIECES = ATT_CHUNK * PER_ROW;
  using Piece = typename std::conditional<CF == FH_BFP4, uint2, uint4>::type;
  Piece kp[4], vp[4];
  uint32_t kx[4], vx[4];

  __device__ __forceinline__ void load(const AttArgs& a, int64_t krow, int64_t vrow, int n, int i0, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(i0 + u * nthreads + tid, PIECES - 1);
      const int r = i / PER_ROW, pc = i % PER_ROW, rr = r < n ? r : n - 1;
      if constexpr (BLOCK) {
        kp[u] = ((const Piece*)a.cache)[(krow + rr) * PER_ROW + pc]; kx[u] = a.cache_exps[(krow + rr) * PER_ROW + pc];
        vp[u] = ((const Piece*)a.cache)[(vrow + rr) * PER_ROW + pc]; vx[u] = a.cache_exps[(vrow + rr) * PER_ROW + pc];
      } else {
        kp[u] = *(const uint4*)((const char*)a.cache + (krow + rr) * (HD * ES) + 16 * pc);
        vp[u] = *(const uint4*)((const char*)a.cache + (vrow + rr) * (HD * ES) + 16 * pc);
      }
    }
  }
  __device__ __forceinline__ void store(char* ks, char* vs, int i0, int tid, int nthreads) const {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * nthreads + tid;
      if (i >= PIECES) continue;
      const int r = i / PER_ROW, pc = i % PER_ROW;
      if constexpr (BLOCK) {
        float f[16];
        uint32_t w[8];
        uint4* kd = (uint4*)(ks + r * RW + 32 * pc);
        uint4* vd = (uint4*)(vs + r * RW + 32 * pc);
        magnitudes(kp[u], f);
        bfp_run_bf16<16>(f, kx[u], w);
        kd[0] = make_uint4(w[0], w[1], w[2], w[3]); kd[1] = make_uint4(w[4], w[5], w[6], w[7]);
        magnitudes(vp[u], f);
        bfp_run_bf16<16>(f, vx[u], w);
        vd[0] = make_uint4(w[0], w[1], w[2], w[3]); vd[1] = make_uint4(w[4], w[5], w[6], w[7]);
      } else {
        *(uint4*)(ks + r * RW + 16 * pc) = make_uint4(kp[u].x, kp[u].y, kp[u].z, kp[u].w);
        *(uint4*)(vs + r * RW + 16 * pc) = make_uint4(vp[u].x, vp[u].y, vp[u].z, vp[u].w);
      }
    }
  }
};

// The fields a kernel's first loads need, passed ahead of AttArgs so that they arrive in SGPRs with the wave
// (kernel-argument preloading: the loads go out without waiting for the argument buffer, ~0.6 us a launch measured on
// MI355X); each kernel starts from a copy of its AttArgs with these in place. The attention kernels' (the row's range
// and the cache's rows) and the combine's (the row's range and the parts).
#define FH_ATT_PRELOAD const float* __restrict__ pq, const void* __restrict__ pcache, const int32_t* __restrict__ pplaces, \
                       const int32_t* __restrict__ pfirst, int64_t pcache_len, int pmax_chunks, int pheads, int pkv_heads
#define FH_ATT_ARGS(a) (a).q, (a).cache, (a).places, (a).first_row, (a).cache_len, (a).max_chunks, (a).heads, (a).kv_heads
#define FH_CMB_PRELOAD const float* __restrict__ ppart, const int32_t* __restrict__ pplaces, const int32_t* __restrict__ pfirst, \
                       int64_t pcache_len, int pmax_chunks, int pheads, int psplits
#define FH_CMB_ARGS(a) (a).part, (a).places, (a).first_row, (a).cache_len, (a).max_chunks, (a).heads, (a).splits
__device__ inline AttArgs att_preloaded(const AttArgs& a0, const float* q, const void* cache, const int32_t* places,
                                        const int32_t* first, int64_t cache_len, int max_chunks, int heads, int kv_heads) {
  AttArgs a = a0;
  a.q = q; a.cache = cache; a.places = places; a.first_row = first; a.cache_len = cache_len; a.max_chunks = max_chunks;
  a.heads = heads; a.kv_heads = kv_heads;
  return a;
}
__device__ inline AttArgs cmb_preloaded(const AttArgs& a0, const float* part, const int32_t* places, const int32_t* first,
                                        int64_t cache_len, int max_chunks, int heads, int splits) {
  AttArgs a = a0;
  a.part = (float*)part; a.places = places; a.first_row = first; a.cache_len = cache_len; a.max_chunks = max_chunks;
  a.heads = heads; a.splits = splits;
  return a;
}

// One chunk's arithmetic for a wave (its query head): the lane's row's score (its keys in LDS dotted with the head's
// q), the running max and sum of exps (online softmax), and p v into o, a lane dimensions DL lane .. DL lane + DL - 1;
// n rows of the chunk are the row's. ps: the wave's row of p in LDS.
template <int HD, int CF>
__device__ __forceinline__ void chunk_arith(const AttArgs& a, const char* ks, const char* vs, float* ps, const float* qh,
                                            int lane, int n, float& m, float& l, float (&o)[HD / 64]) {
  using Loader = ChunkLoader<HD, CF>;
  constexpr bool BF = CF != FH_F32;
  constexpr int DL = HD / 64, ES = Loader::ES, V16 = HD * ES / 16, RW = Loader::RW;
  // the lane's row's score: its keys (from LDS) dotted with the head's q
  float s2[2] = {0.f, 0.f};
  const char* krow = ks + lane * RW;
#pragma unroll
  for (int p = 0; p < V16; ++p) {
    const uint4 w4 = *(const uint4*)(krow + 16 * p);
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
    const float4 qa = *(const float4*)(qh + p * (16 / ES)), qb = BF ? *(const float4*)(qh + p * 8 + 4) : qa;
    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (BF) {
        s2[0] = fmaf(qv[2 * j], __uint_as_float(w[j] << 16), s2[0]);
        s2[1] = fmaf(qv[2 * j + 1], __uint_as_float(w[j] & 0xFFFF0000u), s2[1]);
      } else {
        s2[j & 1] = fmaf(qv[j], __uint_as_float(w[j]), s2[j & 1]);
      }
    }
  }
  const bool valid = lane < n;
  const float sc = valid ? (s2[0] + s2[1]) * a.scale : -INFINITY;
  const float mn = fmaxf(m, wave_max(sc));   // the running max (finite: the chunk has a row)
  const float p = valid ? expf(sc - mn) : 0.f;
  const float f = expf(m - mn);              // (0 on the first chunk)
  l = fmaf(l, f, wave_sum(p));
  m = mn;
  ps[lane] = p;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the wave's p visible to all its lanes

  // p v: a lane dimensions DL lane .. DL lane + DL - 1
#pragma unroll
  for (int i = 0; i < DL; ++i) o[i] *= f;
#pragma unroll 4
  for (int t4 = 0; t4 < ATT_CHUNK / 4; ++t4) {
    const float4 p4 = *(const float4*)(ps + 4 * t4);
    const float pt[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const char* vrw = vs + (4 * t4 + u) * RW + DL * ES * lane;
      if constexpr (BF && DL == 2) {
        const uint32_t w = *(const uint32_t*)vrw;
        o[0] = fmaf(pt[u], __uint_as_float(w << 16), o[0]);
        o[1] = fmaf(pt[u], __uint_as_float(w & 0xFFFF0000u), o[1]);
      } else {
#pragma unroll
        for (int i = 0; i < DL; ++i) {
          const float x = BF ? __uint_as_float((uint32_t)((const uint16_t*)vrw)[i] << 16) : ((const float*)vrw)[i];
          o[i] = fmaf(pt[u], x, o[i]);
        }
      }
    }
  }
}

template <int HD, int CF, bool QLDS>
__global__ __launch_bounds__(64 * ATT_REP) void attention_kernel(FH_ATT_PRELOAD, AttArgs a0) {
  const AttArgs a = att_preloaded(a0, pq, pcache, pplaces, pfirst, pcache_len, pmax_chunks, pheads, pkv_heads);
  using Loader = ChunkLoader<HD, CF>;
  constexpr int DL = HD / 64;                  // dimensions a lane (p v, the combine)
  constexpr int RW = Loader::RW;               // (16 more than the row: a lane's 16-byte reads of its own row spread
                                               // over the banks)
  extern __shared__ __attribute__((aligned(16))) char att_smem[];
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, S = a.splits;
  const int rep = a.heads / a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, nthreads = 64 * rep;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = kvh * rep + wave;              // this wave's query head
  int64_t row0, length;
  row_range(a, b, row0, length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (split >= nchunks) return;  // no chunk of the row falls to this workgroup
  const int parts = nchunks < S ? nchunks : S;  // workgroups with a share of the row
  char* ks = att_smem;
  char* vs = att_smem + ATT_CHUNK * RW;
  float* ps = (float*)(att_smem + 2 * ATT_CHUNK * RW) + wave * ATT_CHUNK;  // this wave's p
  float* qs = (float*)(att_smem + 2 * ATT_CHUNK * RW) + rep * ATT_CHUNK;   // (QLDS) the heads' q
  // q: one address for the wave (scalar loads), or the wave's row of the staged q
  const float* qh = QLDS ? qs + wave * HD : a.q + ((int64_t)b * a.heads + h) * HD;
  const int64_t krow0 = (int64_t)kvh * a.cache_len + row0, vrow0 = (int64_t)(a.kv_heads + kvh) * a.cache_len + row0;
  auto rows_of = [&](int c) { return (int)(length - (int64_t)c * ATT_CHUNK < ATT_CHUNK ? length - (int64_t)c * ATT_CHUNK : ATT_CHUNK); };

  Loader ld;
  ld.load(a, krow0 + (int64_t)split * ATT_CHUNK, vrow0 + (int64_t)split * ATT_CHUNK, rows_of(split), 0, tid, nthreads);
  if constexpr (QLDS) {  // q with the first chunk's loads (rep HD / 4 <= 16 HD / 4 <= 64 rep float4s: one each at most)
    const float* qrow = a.q + ((int64_t)b * a.heads + (int64_t)kvh * rep) * HD;
    const float4 qp = *(const float4*)(qrow + 4 * min(tid, rep * HD / 4 - 1));
    if (tid < rep * HD / 4) *(float4*)(qs + 4 * tid) = qp;
  }
  float m = -INFINITY, l = 0.f, o[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) o[i] = 0.f;
  for (int c = split; c < nchunks; c += S) {
    const int n = rows_of(c);
    const int64_t kr = krow0 + (int64_t)c * ATT_CHUNK, vr = vrow0 + (int64_t)c * ATT_CHUNK;
    ld.store(ks, vs, 0, tid, nthreads);
    for (int i0 = 4 * nthreads; i0 < Loader::PIECES; i0 += 4 * nthreads) {  // (tiles beyond a round a thread)
      ld.load(a, kr, vr, n, i0, tid, nthreads);
      ld.store(ks, vs, i0, tid, nthreads);
    }
    __syncthreads();
    if (c + S < nchunks)  // the next chunk's first round in flight during this one's arithmetic
      ld.load(a, kr + (int64_t)S * ATT_CHUNK, vr + (int64_t)S * ATT_CHUNK, rows_of(c + S), 0, tid, nthreads);

    chunk_arith<HD, CF>(a, ks, vs, ps, qh, lane, n, m, l, o);
    __syncthreads();  // the tiles and p are rewritten by the next chunk
  }
  if (parts == 1) {  // the row's only part: o itself
    const int64_t ob = (int64_t)h * HD + DL * lane;
#pragma unroll
    for (int i = 0; i < DL; ++i) put_o(a, b, ob + i, o[i] / l);
    return;
  }
  float* pp = a.part + (((int64_t)b * a.heads + h) * S + split) * (HD + 2);
#pragma unroll
  for (int i = 0; i < DL; ++i) pp[DL * lane + i] = o[i];
  if (lane == 0) { pp[HD] = m; pp[HD + 1] = l; }
}

// A short row (at most G chunks, G rep waves at most 16): one workgroup a (key head, batch row) takes the whole row,
// a group of rep waves a chunk (group g chunk g, in LDS of its own), each the chunk's arithmetic above; the groups'
// (p v, max, sum) then meet in LDS and group 0's waves write o: no second kernel (its launch is most of a short row's
// cost). The combine's arithmetic is attention_combine's (each part weighted by exp(its max - the largest)).
template <int HD, int CF>
__global__ __launch_bounds__(64 * ATT_REP) void attention_short(FH_ATT_PRELOAD, AttArgs a0) {
  const AttArgs a = att_preloaded(a0, pq, pcache, pplaces, pfirst, pcache_len, pmax_chunks, pheads, pkv_heads);
  using Loader = ChunkLoader<HD, CF>;
  constexpr int DL = HD / 64, RW = Loader::RW;
  extern __shared__ __attribute__((aligned(16))) char att_smem[];
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int rep = a.heads / a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, gthreads = 64 * rep;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave / rep, wq = wave - g * rep;  // this wave's chunk and query head of the key head
  const int gtid = tid - g * gthreads;
  const int h = kvh * rep + wq;
  int64_t row0, length;
  row_range(a, b, row0, length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);  // (at most G: the host's launch)
  const bool has = g < nchunks;
  const int64_t rest = length - (int64_t)g * ATT_CHUNK;
  const int n = has ? (int)(rest < ATT_CHUNK ? rest : ATT_CHUNK) : 0;
  char* base = att_smem + (size_t)g * (2 * ATT_CHUNK * RW + (size_t)rep * (ATT_CHUNK + HD) * 4);  // the group's
  char* ks = base;
  char* vs = base + ATT_CHUNK * RW;
  float* ps = (float*)(base + 2 * ATT_CHUNK * RW) + wq * ATT_CHUNK;
  float* qs = (float*)(base + 2 * ATT_CHUNK * RW) + rep * ATT_CHUNK;  // the key head's query heads' q
  const int64_t kr = (int64_t)kvh * a.cache_len + row0 + (int64_t)g * ATT_CHUNK;
  const int64_t vr = (int64_t)(a.kv_heads + kvh) * a.cache_len + row0 + (int64_t)g * ATT_CHUNK;

  Loader ld;
  if (has) {
    ld.load(a, kr, vr, n, 0, gtid, gthreads);
    const float* qrow = a.q + ((int64_t)b * a.heads + (int64_t)kvh * rep) * HD;
    const float4 qp = *(const float4*)(qrow + 4 * min(gtid, rep * HD / 4 - 1));
    if (gtid < rep * HD / 4) *(float4*)(qs + 4 * gtid) = qp;
    ld.store(ks, vs, 0, gtid, gthreads);
    for (int i0 = 4 * gthreads; i0 < Loader::PIECES; i0 += 4 * gthreads) {  // (tiles beyond a round a thread)
      ld.load(a, kr, vr, n, i0, gtid, gthreads);
      ld.store(ks, vs, i0, gtid, gthreads);
    }
  }
  __syncthreads();
  float m = -INFINITY, l = 0.f, o[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) o[i] = 0.f;
  if (has) chunk_arith<HD, CF>(a, ks, vs, ps, qs + wq * HD, lane, n, m, l, o);
  __syncthreads();  // (the tiles are free: each wave's part goes where its group's keys were)
  float* part = (float*)base + wq * (HD + 2);
  if (has) {
#pragma unroll
    for (int i = 0; i < DL; ++i) part[DL * lane + i] = o[i];
    if (lane == 0) { part[HD] = m; part[HD + 1] = l; }
  }
  __syncthreads();
  if (g != 0) return;
  const size_t gstride = (2 * ATT_CHUNK * RW + (size_t)rep * (ATT_CHUNK + HD) * 4) / 4;  // (floats between groups)
  const float* p0 = (const float*)att_smem + wq * (HD + 2);
  float top = -INFINITY;
  for (int c = 0; c < nchunks; ++c) top = fmaxf(top, p0[c * gstride + HD]);
  float den = 0.f, num[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) num[i] = 0.f;
  for (int c = 0; c < nchunks; ++c) {
    const float* pc = p0 + c * gstride;
    const float wc = nchunks == 1 ? 1.f : expf(pc[HD] - top);
    den = fmaf(wc, pc[HD + 1], den);
#pragma unroll
    for (int i = 0; i < DL; ++i) num[i] = fmaf(wc, pc[DL * lane + i], num[i]);
  }
  const int64_t ob = (int64_t)h * HD + DL * lane;
#pragma unroll
  for (int i = 0; i < DL; ++i) put_o(a, b, ob + i, num[i] / den);
}

// The same chunk walk on the matrix cores, for a workgroup that takes several chunks (the throughput case: many rows)
// of a bf16 or block-float cache: 4 waves, wave w the chunk's rows 16 w .. 16 w + 15 for every query head at once
// (v_mfma_f32_16x16x32_bf16, heads as N). Scores S = K q^T: A the keys' rows from the LDS tile, B q in two bf16
// terms (q to nearest, then the rest to nearest: their sum is q within 2^-16 |q|, and each product of bf16 values is
// exact in fp32). The softmax statistics of each head meet across the waves in LDS; p is written to LDS in two bf16
// terms the same way; O += p V with A p's terms and B the values' columns read transposed (ds_read_b64_tr_b16), wave w
// a quarter of the dimensions. Two terms rather than three keep the workgroup within 40 KB of LDS and 128 registers a
// lane, so that four of them fit a CU.
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 att_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float att_floatx4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short att_short4;
#define ATT_LDS __attribute__((address_space(3)))
constexpr int ATT_PS = ATT_CHUNK + 8;  // a head's row of p in LDS, bf16 (144 bytes)

constexpr int ATT_T = 2;  // bf16 terms of q and of p

__device__ inline float att_rne(float x) {  // x rounded to bf16 (nearest even), as a float
  const uint32_t u = __float_as_uint(x);
  return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}
// x as two floats with bf16 values: x to nearest, then the rest (exact in fp32) to nearest; |x - t0 - t1| <= 2^-16 |x|
__device__ inline void split2(float x, float (&t)[ATT_T]) {
  t[0] = att_rne(x);
  t[1] = att_rne(x - t[0]);
}
__device__ inline uint32_t pack_hi(float lo, float hi) {  // two floats with bf16 values: their high halves
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

static size_t att_mfma_lds(int hd) {
  return (size_t)2 * ATT_CHUNK * att_row_bytes(hd, 2) + (size_t)ATT_T * 16 * ATT_PS * 2 + (size_t)(2 * 4 * 16 + 3 * 16) * 4;
}

template <int HD, int CF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8)))  // (4 workgroups a CU: 128 registers)
void attention_mfma(FH_ATT_PRELOAD, AttArgs a0) {
  const AttArgs a = att_preloaded(a0, pq, pcache, pplaces, pfirst, pcache_len, pmax_chunks, pheads, pkv_heads);
  using Loader = ChunkLoader<HD, CF>;
  constexpr int RW = Loader::RW, RWS = RW / 2;   // a tile row in bytes and in bf16s
  constexpr int KS = HD / 32;                    // K steps of the scores
  constexpr int TPW = HD / 16 / 4;               // 16-column tiles of O a wave
  static_assert(CF != FH_F32 && TPW >= 1, "bf16 or block-float tiles, head_dim >= 64");
  extern __shared__ __attribute__((aligned(16))) char att_smem[];
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, S = a.splits;
  const int rep = a.heads / a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), g = lane >> 4, c16 = lane & 15;
  int64_t row0, length;
  row_range(a, b, row0, length);
  const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
  if (split >= nchunks) return;
  const int parts = nchunks < S ? nchunks : S;
  char* ks = att_smem;
  char* vs = att_smem + ATT_CHUNK * RW;
  uint16_t* ps = (uint16_t*)(att_smem + 2 * ATT_CHUNK * RW);          // [ATT_T][16 heads][ATT_PS]
  float* wmax_s = (float*)(ps + ATT_T * 16 * ATT_PS);                 // [4 waves][16 heads]
  float* wsum_s = wmax_s + 64;
  float* m_s = wsum_s + 64;                                           // [16] running max
  float* l_s = m_s + 16;                                              // [16] running sum
  float* f_s = l_s + 16;                                              // [16] this chunk's rescale
  if (tid < 16) { m_s[tid] = -INFINITY; l_s[tid] = 0.f; f_s[tid] = 0.f; }
  const int64_t krow0 = (int64_t)kvh * a.cache_len + row0, vrow0 = (int64_t)(a.kv_heads + kvh) * a.cache_len + row0;
  auto rows_of = [&](int c) { return (int)(length - (int64_t)c * ATT_CHUNK < ATT_CHUNK ? length - (int64_t)c * ATT_CHUNK : ATT_CHUNK); };

  Loader ld;
  ld.load(a, krow0 + (int64_t)split * ATT_CHUNK, vrow0 + (int64_t)split * ATT_CHUNK, rows_of(split), 0, tid, 256);

  // q as B: lane's head c16 (zero past rep), dimensions 32 s + 8 g .. + 7, ATT_T terms
  // scores kept in base 2 (scale times log2 e): each exponential the chip's exp2 alone
  const float scale2 = a.scale * 1.44269504088896341f;
  att_bf16x8 qb[KS][ATT_T];
  {
    const bool hv = c16 < rep;
    const float* qh = a.q + ((int64_t)b * a.heads + (int64_t)kvh * rep + (hv ? c16 : 0)) * HD + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const float4 u = *(const float4*)(qh + 32 * s), v = *(const float4*)(qh + 32 * s + 4);
      const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
      float t[ATT_T][8];
#pragma unroll
      for (int i = 0; i < 8; ++i) { float u[ATT_T]; split2(hv ? x[i] : 0.f, u); for (int j = 0; j < ATT_T; ++j) t[j][i] = u[j]; }
#pragma unroll
      for (int j = 0; j < ATT_T; ++j) {
        const uint4 pk = make_uint4(pack_hi(t[j][0], t[j][1]), pack_hi(t[j][2], t[j][3]), pack_hi(t[j][4], t[j][5]), pack_hi(t[j][6], t[j][7]));
        qb[s][j] = *(const att_bf16x8*)&pk;
      }
    }
  }
  att_floatx4 acc_o[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) acc_o[tt] = att_floatx4{0.f, 0.f, 0.f, 0.f};
  // the values' transposed reads: 16-lane group g reads rows 8 g .. of a 32-row step; lane 4 m + q of a group points
  // at row m, columns 4 q .. 4 q + 3 of a 16-column tile
  ATT_LDS att_short4* vtr = (ATT_LDS att_short4*)((uint16_t*)vs + (8 * g + ((lane & 15) >> 2)) * RWS + 4 * (lane & 3));

  for (int c = split; c < nchunks; c += S) {
    const int n = rows_of(c);
    const int64_t kr = krow0 + (int64_t)c * ATT_CHUNK, vr = vrow0 + (int64_t)c * ATT_CHUNK;
    ld.store(ks, vs, 0, tid, 256);
    for (int i0 = 4 * 256; i0 < Loader::PIECES; i0 += 4 * 256) {
      ld.load(a, kr, vr, n, i0, tid, 256);
      ld.store(ks, vs, i0, tid, 256);
    }
    __syncthreads();
    if (c + S < nchunks)  // the next chunk's first round in flight during this one's arithmetic
      ld.load(a, kr + (int64_t)S * ATT_CHUNK, vr + (int64_t)S * ATT_CHUNK, rows_of(c + S), 0, tid, 256);

    // scores: rows 16 w + 4 g + i (i < 4) of head c16 in lane's D
    att_floatx4 sc = att_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const att_bf16x8 ka = *(const att_bf16x8*)(ks + (16 * w + c16) * RW + (32 * s + 8 * g) * 2);
#pragma unroll
      for (int j = 0; j < ATT_T; ++j) sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[s][j], sc, 0, 0, 0);
    }
    const bool hv = c16 < rep;
    float sv[4], wm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = hv && 16 * w + 4 * g + i < n;
      sv[i] = ok ? sc[i] * scale2 : -INFINITY;
      wm = fmaxf(wm, sv[i]);
    }
    wm = fmaxf(wm, __shfl_xor(wm, 16, 64));
    wm = fmaxf(wm, __shfl_xor(wm, 32, 64));
    if (g == 0) wmax_s[w * 16 + c16] = wm;
    __syncthreads();
    float mn = m_s[c16];
#pragma unroll
    for (int v = 0; v < 4; ++v) mn = fmaxf(mn, wmax_s[v * 16 + c16]);
    float pv[4], wsum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) { pv[i] = sv[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[i] - mn); wsum += pv[i]; }
    wsum += __shfl_xor(wsum, 16, 64);
    wsum += __shfl_xor(wsum, 32, 64);
    if (g == 0) wsum_s[w * 16 + c16] = wsum;
    {  // p's terms: head c16, rows 16 w + 4 g .. + 3
      float t[ATT_T][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) { float u[ATT_T]; split2(pv[i], u); for (int j = 0; j < ATT_T; ++j) t[j][i] = u[j]; }
#pragma unroll
      for (int j = 0; j < ATT_T; ++j)
        *(uint2*)(ps + (j * 16 + c16) * ATT_PS + 16 * w + 4 * g) = make_uint2(pack_hi(t[j][0], t[j][1]), pack_hi(t[j][2], t[j][3]));
    }
    __syncthreads();
    if (tid < 16) {  // each head's running statistics
      float mh = m_s[tid], sum = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { mh = fmaxf(mh, wmax_s[v * 16 + tid]); sum += wsum_s[v * 16 + tid]; }
      const float f = tid < rep && mh != -INFINITY ? __builtin_amdgcn_exp2f(m_s[tid] - mh) : 0.f;  // (0 on the first chunk)
      l_s[tid] = fmaf(l_s[tid], f, sum);
      m_s[tid] = mh;
      f_s[tid] = f;
    }
    __syncthreads();
    // O (heads 4 g + i, dimensions of tile w TPW + tt) rescaled, then += p V over the chunk's two 32-row steps
    float fr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fr[i] = f_s[4 * g + i];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc_o[tt][i] *= fr[i];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      att_bf16x8 pa[ATT_T];
#pragma unroll
      for (int j = 0; j < ATT_T; ++j) pa[j] = *(const att_bf16x8*)(ps + (j * 16 + c16) * ATT_PS + 32 * s2 + 8 * g);
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) {
        const int col = 16 * (w * TPW + tt);
        const att_short4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vtr + (32 * s2 * RWS + col) / 4);
        const att_short4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vtr + (32 * s2 * RWS + 4 * RWS + col) / 4);
        const short v8[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        const att_bf16x8 vb = *(const att_bf16x8*)v8;
#pragma unroll
        for (int j = 0; j < ATT_T; ++j) acc_o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[j], vb, acc_o[tt], 0, 0, 0);
      }
    }
    __syncthreads();  // the tiles, p and the statistics are rewritten by the next chunk
  }
  // lane's outputs: heads 4 g + i, dimension 16 (w TPW + tt) + c16
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = 4 * g + i;
    if (hh >= rep) continue;
    const int64_t h = (int64_t)kvh * rep + hh;
    if (parts == 1) {
      const int64_t ob = h * HD;
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) put_o(a, b, ob + 16 * (w * TPW + tt) + c16, acc_o[tt][i] / l_s[hh]);
    } else {
      float* pp = a.part + (((int64_t)b * a.heads + h) * S + split) * (HD + 2);
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) pp[16 * (w * TPW + tt) + c16] = acc_o[tt][i];
      if (w == 0 && c16 == 0) { pp[HD] = m_s[hh] * 0.693147180559945309f; pp[HD + 1] = l_s[hh]; }  // (the max in e's base)
    }
  }
}

// The parts of row blockIdx.y, head blockIdx.x combined, HD threads: thread t holds part g0 + t's statistics and
// dimension t's values of CV parts at a time. The first round's loads (the row's place, the statistics, the values)
// go out together; the largest max and the sum of exp-weighted sums are workgroup reductions, each part's weight
// exp(max - the largest) is computed once (by its thread) and shared through LDS. Parts past the row's (left from
// other calls) are selected away, never multiplied by 0.
template <int HD>
__device__ inline float block_fold(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < HD / 64; ++w) t = is_max ? fmaxf(t, red[w]) : t + red[w];
  __syncthreads();
  return t;
}

template <int HD>
__global__ __launch_bounds__(HD) void attention_combine(FH_CMB_PRELOAD, AttArgs a0) {
  const AttArgs a = cmb_preloaded(a0, ppart, pplaces, pfirst, pcache_len, pmax_chunks, pheads, psplits);
  constexpr int CV = 32;
  __shared__ float w_s[HD];
  __shared__ float red_s[HD / 64];
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const float* hp = a.part + ((int64_t)b * a.heads + h) * a.splits * (HD + 2);
  const int last = a.splits - 1;
  auto values = [&](float (&v)[CV], int c0) {
#pragma unroll
    for (int j = 0; j < CV; ++j) v[j] = hp[(int64_t)min(c0 + j, last) * (HD + 2) + d];
  };
  float big = -INFINITY, den = 0.f, num = 0.f;
  int nparts = a.splits;  // (the row's own count, known after the first round)
  for (int g0 = 0; g0 < nparts; g0 += HD) {
    const float* pc = hp + (int64_t)min(g0 + d, last) * (HD + 2);
    const float mc = pc[HD], lc = pc[HD + 1];
    float v[CV];
    values(v, g0);
    if (g0 == 0) {
      int64_t row0, length;
      row_range(a, b, row0, length);
      const int nchunks = (int)((length + ATT_CHUNK - 1) / ATT_CHUNK);
      nparts = nchunks < a.splits ? nchunks : a.splits;
      if (nparts == 1) return;  // the first kernel wrote o
    }
    const bool ok = g0 + d < nparts;
    const float top = fmaxf(big, block_fold<HD>(ok ? mc : -INFINITY, true, red_s));
    const float wc = ok ? expf(mc - top) : 0.f;
    const float f = big == -INFINITY ? 0.f : expf(big - top);
    den = fmaf(den, f, block_fold<HD>(ok ? wc * lc : 0.f, false, red_s));
    num *= f;
    w_s[d] = wc;
    __syncthreads();
    const int n = min(HD, nparts - g0);
    for (int j0 = 0; j0 < n; j0 += CV) {
      if (j0 > 0) values(v, g0 + j0);
#pragma unroll
      for (int j = 0; j < CV; ++j) num = j0 + j < n ? fmaf(w_s[j0 + j], v[j], num) : num;
    }
    __syncthreads();  // (w_s is rewritten by the next group)
    big = top;
  }
  put_o(a, b, (int64_t)h * HD + d, num / den);
}

// the kernel, allowed its largest LDS (above 64 KiB for fp32 rows of 256 and 16 heads a key head) once
template <int HD, int CF, bool QLDS>
static void launch_attention(dim3 grid, dim3 block, size_t lds, hipStream_t s, const AttArgs& a) {
  static const hipError_t allowed = hipFuncSetAttribute((const void*)attention_kernel<HD, CF, QLDS>,
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)att_lds(HD, CF == FH_F32 ? 4 : 2, ATT_REP, QLDS));
  (void)allowed;  // (a refusal shows as the launch's error)
  hipLaunchKernelGGL((attention_kernel<HD, CF, QLDS>), grid, block, lds, s, FH_ATT_ARGS(a), a);
}

template <int HD, int CF>
static void launch_attention(bool q_lds, dim3 grid, dim3 block, size_t lds, hipStream_t s, const AttArgs& a) {
  if (q_lds) launch_attention<HD, CF, true>(grid, block, lds, s, a);
  else launch_attention<HD, CF, false>(grid, block, lds, s, a);
}

template <int HD>
static void launch_attention(int cf, bool q_lds, dim3 grid, dim3 block, size_t lds, hipStream_t s, const AttArgs& a) {
  switch (cf) {
    case FH_F32: launch_attention<HD, FH_F32>(q_lds, grid, block, lds, s, a); break;
    case FH_BF16: launch_attention<HD, FH_BF16>(q_lds, grid, block, lds, s, a); break;
    case FH_BFP8: launch_attention<HD, FH_BFP8>(q_lds, grid, block, lds, s, a); break;
    default: launch_attention<HD, FH_BFP4>(q_lds, grid, block, lds, s, a); break;
  }
  if (a.splits > 1) hipLaunchKernelGGL(attention_combine<HD>, dim3(a.heads, grid.z), dim3(HD), 0, s, FH_CMB_ARGS(a), a);
}

template <int HD, int CF>
static void launch_attention_short(dim3 grid, dim3 block, size_t lds, hipStream_t s, const AttArgs& a) {
  static const hipError_t allowed = hipFuncSetAttribute((const void*)attention_short<HD, CF>,
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)allowed;  // (a refusal shows as the launch's error)
  hipLaunchKernelGGL((attention_short<HD, CF>), grid, block, lds, s, FH_ATT_ARGS(a), a);
}

template <int HD>
static void launch_attention_short(int cf, dim3 grid, dim3 block, size_t lds, hipStream_t s, const AttArgs& a) {
  switch (cf) {
    case FH_F32: launch_attention_short<HD, FH_F32>(grid, block, lds, s, a); break;
    case FH_BF16: launch_attention_short<HD, FH_BF16>(grid, block, lds, s, a); break;
    case FH_BFP8: launch_attention_short<HD, FH_BFP8>(grid, block, lds, s, a); break;
    default: launch_attention_short<HD, FH_BFP4>(grid, block, lds, s, a); break;
  }
}

template <int HD, int CF>
static void launch_attention_mfma(dim3 grid, dim3 block, hipStream_t s, const AttArgs& a) {
  static const hipError_t allowed = hipFuncSetAttribute((const void*)attention_mfma<HD, CF>,
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)att_mfma_lds(HD));
  (void)allowed;
  hipLaunchKernelGGL((attention_mfma<HD, CF>), grid, block, att_mfma_lds(HD), s, FH_ATT_ARGS(a), a);
}

template <int HD>
static void launch_attention_mfma(int cf, dim3 grid, dim3 block, hipStream_t s, const AttArgs& a) {
  switch (cf) {
    case FH_BF16: launch_attention_mfma<HD, FH_BF16>(grid, block, s, a); break;
    case FH_BFP8: launch_attention_mfma<HD, FH_BFP8>(grid, block, s, a); break;
    default: launch_attention_mfma<HD, FH_BFP4>(grid, block, s, a); break;
  }
  if (a.splits > 1) hipLaunchKernelGGL(attention_combine<HD>, dim3(a.heads, grid.z), dim3(HD), 0, s, FH_CMB_ARGS(a), a);
}

}  // namespace fh

using namespace fh;

extern "C" size_t fh_attention_workspace_bytes(int batch, int heads, int head_dim, int64_t max_context) {
  if (batch < 1 || heads < 1 || head_dim < 1 || max_context < 1) return 0;
  const int64_t chunks = (max_context + ATT_CHUNK - 1) / ATT_CHUNK;
  return (size_t)batch * heads * chunks * (head_dim + 2) * sizeof(float);
}

extern "C" size_t fh_kv_cache_bytes(int cache_dtype, int kv_heads, int64_t cache_len, int head_dim) {
  if (kv_heads < 1 || cache_len < 1 || head_dim < 32 || head_dim % 32) return 0;
  const int64_t rows = 2 * (int64_t)kv_heads * cache_len;
  switch (cache_dtype) {
    case FH_F32: return (size_t)rows * head_dim * 4;
    case FH_BF16: return (size_t)rows * head_dim * 2;
    case FH_BFP8: case FH_BFP4: return (size_t)(kv_exps_at(cache_dtype, kv_heads, cache_len, head_dim) + rows * (head_dim / 16));
    default: return 0;
  }
}

namespace fh {

// The scratch of fh_attention_decode_noalloc: the chunks' partial results, in a fixed array the library holds on every
// GPU it runs on (one copy a device, at its own address, until the process ends). In host code `scratch` names a
// host-side stand-in, not device memory: host code uses only the per-device address hipGetSymbolAddress gives.
static __device__ __align__(256) unsigned char scratch[FH_ATTENTION_SCRATCH_BYTES];

// The current device's address of `scratch`, looked up once per device (with that device current) and kept.
static int scratch_address(void** out) {
  constexpr int MAX_DEVICES = 64;
  static std::mutex mu;
  static void* at[MAX_DEVICES] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FH_EHIP, "fh_attention_decode_noalloc: no current device");
  if (dev < 0 || dev >= MAX_DEVICES) return fail(FH_EUNSUP, "fh_attention_decode_noalloc: device index past 63");
  std::lock_guard<std::mutex> hold(mu);
  if (!at[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("fh_attention_decode_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return FH_EHIP;
    }
    at[dev] = p;
  }
  *out = at[dev];
  return FH_OK;
}

}  // namespace fh

extern "C" int fh_attention_decode_noalloc(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch,
                                           int heads, int kv_heads, int head_dim, const int32_t* places,
                                           const int32_t* first_row, int64_t max_context, void* o, int o_dtype,
                                           void* stream) {
  // (the bound first, on the host: a call past it is refused before any HIP call)
  if (batch >= 1 && heads >= 1 && head_dim >= 1 && max_context >= 1 &&
      fh_attention_workspace_bytes(batch, heads, head_dim, max_context) > FH_ATTENTION_SCRATCH_BYTES)
    return fail(FH_EINVAL, "fh_attention_decode_noalloc: batch x heads x context needs more scratch than "
                           "FH_ATTENTION_SCRATCH_BYTES (16 MiB): use fh_attention_decode with a workspace");
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  return fh_attention_decode(q, cache, cache_dtype, cache_len, batch, heads, kv_heads, head_dim, places, first_row,
                             max_context, o, o_dtype, ws, FH_ATTENTION_SCRATCH_BYTES, stream);
}

extern "C" int fh_attention_decode(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch,
                                   int heads, int kv_heads, int head_dim, const int32_t* places, const int32_t* first_row,
                                   int64_t max_context, void* o, int o_dtype, void* workspace, size_t ws_bytes,
                                   void* stream) {
  if (!q || !cache || !places || !first_row || !o) return fail(FH_EINVAL, "fh_attention_decode: null pointer");
  if (batch < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads)
    return fail(FH_EINVAL, "fh_attention_decode: heads must be a multiple of kv_heads");
  if (heads / kv_heads > ATT_REP) return fail(FH_EUNSUP, "fh_attention_decode: at most 16 query heads a key head");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail(FH_EUNSUP, "fh_attention_decode: head_dim 64, 128 or 256");
  if (cache_dtype < FH_F32 || cache_dtype > FH_BFP4)
    return fail(FH_EUNSUP, "fh_attention_decode: cache is FH_F32, FH_BF16, FH_BFP8 or FH_BFP4");
  if (max_context < 1 || max_context > cache_len) return fail(FH_EINVAL, "fh_attention_decode: max_context outside 1..cache_len");
  if (o_dtype != FH_F32 && o_dtype != FH_BF16 && o_dtype != FH_BF16_T16)
    return fail(FH_EINVAL, "fh_attention_decode: o is FH_F32, FH_BF16 or FH_BF16_T16");
  const size_t need = fh_attention_workspace_bytes(batch, heads, head_dim, max_context);
  if (max_context > ATT_CHUNK && (!workspace || ws_bytes < need))
    return fail(FH_EINVAL, "fh_attention_decode: workspace smaller than fh_attention_workspace_bytes");
  AttArgs a;
  a.q = q; a.cache = cache; a.cache_len = cache_len;
  a.cache_exps = (const uint8_t*)cache + kv_exps_at(cache_dtype, kv_heads, cache_len, head_dim);
  a.heads = heads; a.kv_heads = kv_heads; a.scale = 1.0f / sqrtf((float)head_dim);
  a.places = places; a.first_row = first_row;
  a.max_chunks = (int)((max_context + ATT_CHUNK - 1) / ATT_CHUNK);
  a.o = o; a.o_bf16 = o_dtype != FH_F32; a.o_tiles = o_dtype == FH_BF16_T16; a.o_ld = (int64_t)heads * head_dim;
  a.part = (float*)workspace;
  const int rep = heads / kv_heads;
  // S: workgroups a (row, key head), enough that the grid fills every CU as far as LDS and waves let it (all of it
  // resident at once, each workgroup walking its chunks), at most the launch's chunks; with one chunk a workgroup, q
  // is staged in LDS with the chunk (its scalar loads would wait behind the chunk's)
  // (the first call's device, read once: a function-local static is initialised once whatever the threads calling)
  struct CuShape { int cus, lds_cu; };
  static const CuShape shape = [] {
    CuShape c = {0, 0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c.cus < 1) c.cus = 256;
    if (hipDeviceGetAttribute(&c.lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess || c.lds_cu < 65536) c.lds_cu = 160 * 1024;
    return c;
  }();
  const int cus = shape.cus, lds_cu = shape.lds_cu;
  const int es = cache_dtype == FH_F32 ? 4 : 2;
  const int64_t pairs = (int64_t)kv_heads * batch;
  auto splits_for = [&](int64_t lds_bytes, int64_t waves) {
    const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(lds_cu / lds_bytes, 32 / waves));
    return (int)std::min<int64_t>(a.max_chunks, std::max<int64_t>(1, (cus * per_cu + pairs - 1) / pairs));
  };
  hipStream_t s = as_stream(stream);
  // a short context (2-4 chunks): each row in one workgroup, a group of waves a chunk, no combine launch
  const size_t glds = att_lds(head_dim, es, rep, true);
  if (a.max_chunks > 1 && a.max_chunks <= 4 && a.max_chunks * rep <= ATT_REP && a.max_chunks * glds <= (size_t)lds_cu) {
    a.splits = 1;
    const dim3 grid(1, kv_heads, batch), block(64 * rep * a.max_chunks);
    const size_t lds = a.max_chunks * glds;
    switch (head_dim) {
      case 64: launch_attention_short<64>(cache_dtype, grid, block, lds, s, a); break;
      case 128: launch_attention_short<128>(cache_dtype, grid, block, lds, s, a); break;
      default: launch_attention_short<256>(cache_dtype, grid, block, lds, s, a); break;
    }
    return check_launch("fh_attention_decode");
  }
  // the matrix cores where workgroups walk several chunks (many rows: throughput) of a bf16 or block-float cache
  if (cache_dtype != FH_F32 && head_dim <= 128) {
    const int sm = splits_for((int64_t)att_mfma_lds(head_dim), 4);
    if (sm < a.max_chunks) {
      a.splits = sm;
      const dim3 grid(a.splits, kv_heads, batch), block(256);
      if (head_dim == 64) launch_attention_mfma<64>(cache_dtype, grid, block, s, a);
      else launch_attention_mfma<128>(cache_dtype, grid, block, s, a);
      return check_launch("fh_attention_decode");
    }
  }
  a.splits = splits_for((int64_t)att_lds(head_dim, es, rep, false), rep);
  const bool q_lds = a.splits == a.max_chunks;
  const size_t lds = att_lds(head_dim, es, rep, q_lds);
  const dim3 grid(a.splits, kv_heads, batch), block(64 * rep);
  switch (head_dim) {
    case 64: launch_attention<64>(cache_dtype, q_lds, grid, block, lds, s, a); break;
    case 128: launch_attention<128>(cache_dtype, q_lds, grid, block, lds, s, a); break;
    default: launch_attention<256>(cache_dtype, q_lds, grid, block, lds, s, a); break;
  }
  return check_launch("fh_attention_decode");
}
