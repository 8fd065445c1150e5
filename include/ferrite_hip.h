/* ferrite_hip.h — the C-ABI of libferrite_hip.so: ferrite's block-float (bfp8/bfp4) weight matmul hot path as
 * hand-written HIP kernels for gfx950 (MI355X).
 *
 * Every entry point takes plain device pointers and sizes, enqueues its kernels on `stream` (a hipStream_t, NULL for the
 * default stream) and returns at once: 0 on success, a negative FH_E* code otherwise, with the reason in
 * fh_last_error() (thread-local). Nothing here allocates or frees device memory: the caller owns every buffer, and
 * scratch comes in through a `workspace` argument sized by the matching *_workspace_bytes call. A workspace needs no
 * clearing, ever: no call keeps state in it, and what a call reads there it wrote first in the same call (a freshly
 * allocated, uninitialised buffer is fine). Calls on one stream run in order; calls that share a workspace must not
 * overlap.
 *
 * The reference (alkinun/ferrite) has no C interface for this path: it builds Tensix kernels in Python
 * (ferrite/compiler.py) and launches them through ferrite/runtime.py. Each declaration below names the reference
 * function whose work it replaces.
 */
#ifndef FERRITE_HIP_H
#define FERRITE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes */
#define FH_OK 0
#define FH_EINVAL (-1)   /* bad argument: null pointer, bad size or shape */
#define FH_EUNSUP (-2)   /* a valid request this build does not support */
#define FH_EHIP (-3)     /* the HIP runtime reported an error (launch failure, bad stream) */

/* element types */
#define FH_F32 0
#define FH_BF16 1
#define FH_BFP8 2
#define FH_BFP4 3
#define FH_I32 4
/* bf16 rows in tiles of 16 rows: element (r, c) of rows of length ld (a multiple of 8) sits at
 * (r / 16) * 16 * ld + (c / 8) * 128 + (r % 16) * 8 + c % 8, so that 8 columns of 16 rows are 256 contiguous bytes,
 * and a buffer of M rows holds 16 * ceil(M / 16) rows (the rows past M are read and never used). The layout of the
 * bf16 rows that pass between the kernels of a decode step of 3 to 64 sequences: fh_gemm_bfp's matrix-core kernel for
 * up to 64 rows loads x's 8 columns of 16 rows in one wave-wide read of whole lines where a row-major x takes 16 half
 * lines. Taken as fh_gemm_bfp's x and y (up to 64 rows, K a multiple of 64), attention's o and fh_rms_rows' out, and
 * written by FH_EP_RESIDUAL's copy (copy_tiles). No counterpart in the reference (a device layout). */
#define FH_BF16_T16 5

/* which axis of a weight W[K][N] (x @ W, K rows, N columns) a block of 16 values runs along:
 * FH_AXIS_N, along a row (16 consecutive columns share an exponent): ferrite's own, gpt2.bfp on W (models/gpt2.py:27,
 *   models/llama.py:652-653);
 * FH_AXIS_K, down a column (16 consecutive rows share one): gpt2.bfp(W.T).T. */
#define FH_AXIS_N 0
#define FH_AXIS_K 1

/* The last error's message on this thread ("" if none). */
const char* fh_last_error(void);
/* The library's version string and the GPU target it was built for. */
const char* fh_version(void);

/* ---- block-float weights: packing and unpacking ----------------------------------------------------------------
 * Packed layout of W[K][N] (both axes; for FH_AXIS_K swap the roles of K and N, i.e. the layout of W^T):
 *   exps: uint8 [N/16][K]            the block's shared exponent (the largest bf16 biased exponent in it)
 *   mant: bfp8  int8  [N/16][K][16]  the signed magnitude q*sign, -127..127 (two's complement byte)
 *         bfp4  uint8 [N/16][K][8]   two signed 4-bit magnitudes -7..7 a byte, value 2i in the low nibble
 * A value is sign * q * 2^(e - 133) (bfp8) or sign * q * 2^(e - 129) (bfp4). */

/* Sizes in bytes of the two arrays for a K x N weight (returns FH_EINVAL for an impossible shape). */
int fh_bfp_bytes(int64_t K, int64_t N, int fmt, int axis, size_t* mant_bytes, size_t* exp_bytes);

/* Pack src[K][N] (row stride ld elements; FH_F32 or FH_BF16) into a block float: fp32 rounded to bf16 to nearest even,
 * then each block to its largest exponent, bfp8 keeping 7 bits of magnitude rounded half up and saturated at 127,
 * bfp4 3 bits rounded to nearest (ties up), saturated at 7, 0 past a shift of 4; a zero keeps no sign.
 * Replaces Tensor.cast("bfp8"/"bfp4") (ferrite/tensor.py:315-320): the packer's cast (ferrite/compiler.py:52-70) and
 * bfp4_kernel (ferrite/compiler.py:2038-2072), whose rounding models/gpt2.py:21-32 states. */
int fh_bfp_pack(const void* src, int src_dtype, int64_t K, int64_t N, int64_t ld, int fmt, int axis, void* mant,
                uint8_t* exps, void* stream);

/* Unpack to bf16 bits out[K][N] (row stride ldo): each value exactly (every block-float value is a bf16 value).
 * Replaces tensor._bf16s (ferrite/tensor.py:718-727), the host readback of a block-float tensor. */
int fh_bfp_dequant(const void* mant, const uint8_t* exps, int64_t K, int64_t N, int fmt, int axis, uint16_t* out,
                   int64_t ldo, void* stream);

/* ---- decode GEMV: y = x @ W with W a block float, a few rows, fused prologue and epilogue -------------------------
 * x: [batch][K] fp32 (row stride ldx). Products are exact and sums are fp32. Up to 8 rows (4 with a paired epilogue)
 * share one pass over W; more rows take more passes (fh_gemm_bfp is the kernel for many rows).
 * Replaces the bfp-B matmul of fused_kernel (ferrite/compiler.py:699-1111, matmul at 958-1022) for a token row
 * (compiler.py:838-845), with the elementwise ops models/llama.py puts after it fused into the same kernel. */

#define FH_EP_STORE 0      /* y = acc (fp32 or bf16 out, dtype y_dtype) */
#define FH_EP_RESIDUAL 1   /* y = residual + acc, and the sums of squares of y by 16 columns into ssq_out (if set) */
#define FH_EP_SILU_GATE 2  /* W's columns are [gate | up], each `split` wide: y[:, j] = silu(gate_j) * up_j, j < split */
#define FH_EP_ROPE_KV 3    /* W's columns are q, k and v heads: RoPE on q's and k's, q into y, k and v into the cache */
#define FH_EP_PROGRAM 4    /* y = program(acc): a chain of elementwise ops on the matmul's result (fh_program below) */

/* ---- elementwise programs: the ops ferrite fuses into one kernel (Tensor.realize's tree, ferrite/tensor.py:247-272,
 * 708-767; fused_kernel's SFPU programs, ferrite/compiler.py:274-340), at most FH_MAX_OPS of them ----------------
 * Op i computes r_i = op(a, b) in fp32 from operands: r_j (j < i), input k (its element at the output's (batch, row,
 * column) by its strides; a stride of 0 broadcasts), the matmul's result (an epilogue's), or the op's immediate. The
 * program's value is its last op's. keep/drop are where()'s halves: a if b != 0 else 0, and a if b == 0 else 0. */
#define FH_MAX_OPS 15
#define FH_MAX_INPUTS 8
#define FH_OPND_IN(k) (16 + (k))   /* operand codes: 0..14 an op's result, 16..23 an input */
#define FH_OPND_ACC 24             /* the matmul's result */
#define FH_OPND_IMM 25             /* the op's immediate */
enum {
  FH_OP_ADD = 0, FH_OP_SUB, FH_OP_MUL, FH_OP_MAX, FH_OP_CMPLT, FH_OP_CMPNE, FH_OP_KEEP, FH_OP_DROP,
  FH_OP_RELU, FH_OP_EXP, FH_OP_EXP2, FH_OP_LOG, FH_OP_LOG2, FH_OP_SIN, FH_OP_COS, FH_OP_RECIP, FH_OP_SQRT,
  FH_OP_FTOB, FH_OP_ITOF, FH_OP_FTOI, FH_OP_COPY
};
typedef struct fh_program {
  int32_t n_ops, n_inputs;
  int8_t op[16], a[16], b[16];
  float imm[16];
  const void* in[FH_MAX_INPUTS];
  int32_t in_dtype[FH_MAX_INPUTS];        /* FH_F32, FH_BF16 or FH_I32 */
  int64_t in_stride[FH_MAX_INPUTS][3];    /* elements between batches, rows, columns */
} fh_program;

typedef struct fh_epilogue {
  int kind;                 /* FH_EP_* */
  /* RMSNorm prologue (models/llama.py:82-85): x is replaced by x * rsqrt(mean(x^2) + eps) * w (n*w + n if centered).
   * The mean comes from ssq_in: per row, the sums of x^2 over each run of 16 columns ([batch][K/16]), which the
   * kernel that made x wrote (FH_EP_RESIDUAL's ssq_out, fh_embed_rows). norm_w NULL and ssq_in NULL: no prologue.
   * norm_w NULL with ssq_in: x's rows already hold x * w (FH_EP_RESIDUAL's copy_bf16 with copy_w), and each row is
   * scaled by rsqrt(mean(x^2) + eps) only, the mean of the unscaled rows that ssq_in holds. */
  const float* norm_w;      /* [K] */
  const float* ssq_in;      /* [batch][K/16] */
  float eps;
  int centered;
  /* FH_EP_RESIDUAL */
  const float* residual;    /* [batch][N], row stride ldy; may be y itself */
  float* ssq_out;           /* [batch][N/16] or NULL */
  /* FH_EP_SILU_GATE */
  int split;                /* columns of gate (= of up); y is [batch][split] */
  /* FH_EP_ROPE_KV (models/llama.py:111-128): heads of q, then k, then v, head_dim each */
  int heads, kv_heads, head_dim;
  const float* cos_tab;     /* [places][head_dim]: cos of each place's angles (bf16 values, as rotary makes them) */
  const float* sin_tab;     /* [places][head_dim] */
  const int32_t* places;    /* [batch]: each row's place (its rotary row) */
  const int32_t* cache_rows;/* [batch]: the cache row each row's k and v go to (its slot's first row + place) */
  void* cache;              /* [2*kv_heads][cache_len][head_dim]: keys' heads then values' (fh_kv_cache_bytes) */
  int cache_dtype;          /* FH_F32, FH_BF16, or a block float: FH_BFP8 or FH_BFP4, each run of 16 of a row
                             * rounded from bf16(k or v) as fh_bfp_pack rounds it (Tensor.put into a block-float
                             * cache, ferrite/compiler.py:1638-1714) */
  int64_t cache_len;
  /* FH_EP_STORE: each row's largest value of each run of 16 columns and its column (the first of equals), as
   * (float, int32) pairs [batch][N/16], for fh_argmax_parts: greedy decoding's pick without a second pass over y */
  void* argmax_parts;
  /* FH_EP_PROGRAM: the program, evaluated at each output (batch row, column) with the matmul's result as its acc */
  const struct fh_program* program;
  /* FH_EP_RESIDUAL: y also written as bf16 ([batch][N], row stride N; nearest even), times copy_w [N] where given
   * (the next RMSNorm's weight, its centered + 1 included): the next matmul's rows, which it takes with ssq_in =
   * this epilogue's ssq_out and norm_w NULL; or NULL. No counterpart in the reference: it saves the separate
   * normalising pass before a matrix-core matmul, and the products are the same as its RMSNorm prologue's
   * (bf16(x * w), then 1/rms on the sums). */
  void* copy_bf16;
  const float* copy_w;
  /* FH_EP_ROPE_KV: the rows of cos_tab and sin_tab (the places they cover). A place outside 0 .. rope_rows - 1 reads
   * the nearest row, and a cache row outside 0 .. cache_len - 1 is not written: the caller checks both, these keep a
   * bad value from reading or writing past the buffers. */
  int64_t rope_rows;
  /* FH_EP_RESIDUAL's copy_bf16 in tiles of 16 rows (FH_BF16_T16, row length N) rather than rows: nonzero for the
   * matrix-core kernel's x (fh_gemm_bfp, up to 64 rows) */
  int copy_tiles;
} fh_epilogue;

/* y (dtype y_dtype, row stride ldy) from x @ W and the epilogue. x: fp32. w_mant/w_exps: a packed [K][N] weight
 * (FH_AXIS_N). For FH_EP_ROPE_KV, y is q: [batch][heads*head_dim] fp32. K is split among the waves of a workgroup,
 * whose sums meet in a fixed order (results do not depend on timing); no scratch memory is needed. */
int fh_gemv_bfp(const void* x, int x_dtype, int64_t ldx, int batch, int64_t K, int64_t N, const void* w_mant,
                const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy, void* stream);

/* fh_gemv_bfp for a weight packed along K (FH_AXIS_K: each run of 16 consecutive rows of a column shares an
 * exponent, gpt2.bfp(W.T).T, models/gpt2.py:21-32 applied to W's transpose): y = epilogue(prologue(x) @ W), K a
 * multiple of 16, any N >= 1. Epilogues FH_EP_STORE (argmax_parts with N a multiple of 16), FH_EP_RESIDUAL and
 * FH_EP_PROGRAM, the RMSNorm prologue as fh_gemv_bfp's; the pairs (FH_EP_SILU_GATE, FH_EP_ROPE_KV) are
 * FH_EUNSUP. Products exact (each run's sum of x q in fp32, times the run's power of 2), waves' sums in a fixed order.
 * Replaces fused_kernel's matmul by a block-float B whose blocks run down its columns (ferrite/compiler.py:699-1111
 * with the tile's face rows along K: the benchmark's config 1 as stated, 16-element blocks along K). */
int fh_gemv_bfp_k(const void* x, int x_dtype, int64_t ldx, int batch, int64_t K, int64_t N, const void* w_mant,
                  const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy, void* stream);

/* ---- prefill GEMM: the same y = epilogue(prologue(x) @ W) for M rows, on the matrix cores ----------------------
 * x: [M][K] fp32 or bf16 (row stride ldx, a multiple of 8); K a multiple of 32. As ferrite's chip does (its unpacker
 * hands the matrix unit bf16; ferrite/tensor.py:443-485), the products are bf16 x bf16 with fp32 sums: x (times the
 * RMSNorm weight) is rounded to bf16 (nearest even), the weight's values are exact. Every epilogue of fh_gemv_bfp,
 * with [M] in place of [batch] (FH_EP_ROPE_KV: each row its own place and cache row, a prompt's tokens at once).
 * Replaces fused_kernel's matmul for prompt rows (ferrite/compiler.py:699-1111 over 32-row tiles; models/llama.py's
 * prefill, 498-504). Up to 64 rows with K a multiple of 64 (a decode step of many sequences) take a kernel that splits
 * K among a workgroup's waves as the GEMV does; more rows take 128 x 128 tiles. No scratch memory; results do not
 * depend on timing. */
int fh_gemm_bfp(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t N, const void* w_mant,
                const uint8_t* w_exps, int fmt, const fh_epilogue* ep, void* y, int y_dtype, int64_t ldy, void* stream);

/* ---- the rest of a decode step ------------------------------------------------------------------------------- */

/* Rows ids[batch] of an embedding table [vocab][dim] (fp32 or bf16) into x[batch][dim] fp32, with the sums of
 * squares by 16 columns into ssq_out[batch][dim/16] (for the first block's RMSNorm). table and x 16-byte aligned. Replaces the gather of
 * forward's first line (models/llama.py:472; Tensor.gather, ferrite/tensor.py:116-126). */
int fh_embed_rows(const void* table, int table_dtype, int64_t vocab, int64_t dim, const int32_t* ids, int batch,
                  float* x, float* ssq_out, void* stream);

/* Decode attention over a KV cache (models/llama.py:129-142; Tensor.attend, ferrite/tensor.py:487-516): for each
 * row b and query head h, softmax(q k^T / sqrt(head_dim)) v over the cache rows first_row[b] .. first_row[b] +
 * places[b] (those its place reaches), k and v the heads of kv head h / (heads / kv_heads) (grouped-query).
 * q: [batch][heads*head_dim] fp32; o the same shape, fp32 or bf16 (o_dtype: rounded to nearest even, the rows the
 * matrix-core matmuls take); heads / kv_heads at most 16. Flash decoding: the keys are shared out among
 * workgroups in chunks of 64 rows of one key head (each cache byte read once, for all the query heads that share it),
 * each writing its partial result and softmax statistics to the workspace, and a second kernel combines the chunks
 * by exp-weights (ferrite/compiler.py:1138-1145); a context of one chunk writes o directly, and one of 2-4 chunks is
 * one workgroup's a row (a group of waves a chunk, the parts combined in LDS, the workspace unused). Scores, softmax and sums
 * are fp32; where many rows make workgroups walk several chunks of a bf16 or block-float cache, the products run on
 * the matrix cores with q and the softmax weights each as two bf16 terms (within 2^-16 of their fp32 values). The
 * workspace holds no state between calls (what a call does not write, it does not read). */
size_t fh_attention_workspace_bytes(int batch, int heads, int head_dim, int64_t max_context);
/* A KV cache's bytes: [2*kv_heads][cache_len][head_dim] of fp32 or bf16; or a block float (models/llama.py:127-128,
 * a cache in bfp8 or bfp4), one buffer: every row's magnitudes (head_dim bytes of two's-complement q for FH_BFP8;
 * head_dim / 2 for FH_BFP4, columns 2i and 2i + 1 in a byte's low and high nibble), rows in order, then every row's
 * head_dim / 16 exponents (a byte a run of 16 columns), rows in order; the values are q * 2^(e - 133) (FH_BFP8),
 * q * 2^(e - 129) (FH_BFP4). All zero bytes are a cache of zeros. 0 for bad arguments (head_dim not a multiple of 32,
 * an unknown dtype). Attention decodes a block float's runs to bf16 exactly: its results are a bf16 cache's holding
 * the same values. No counterpart in the reference as a function (its cache is a Tensor of that dtype). */
size_t fh_kv_cache_bytes(int cache_dtype, int kv_heads, int64_t cache_len, int head_dim);
int fh_attention_decode(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch, int heads,
                        int kv_heads, int head_dim, const int32_t* places, const int32_t* first_row, int64_t max_context,
                        void* o, int o_dtype, void* workspace, size_t ws_bytes, void* stream);

/* fh_attention_decode with no workspace, for callers that cannot allocate (code under HIP graph capture, serving
 * loops and harnesses that forbid hipMalloc); no counterpart in the reference. It allocates nothing: the chunks'
 * partial results go to a scratch array of FH_ATTENTION_SCRATCH_BYTES (16 MiB) that the library holds on each GPU it
 * runs on, from the first call on that GPU until the process ends. A call whose
 * fh_attention_workspace_bytes(batch, heads, head_dim, max_context) exceeds that returns FH_EINVAL (an 8B model's 32
 * heads at context 2048 fit up to batch 16). Every call on one GPU shares that GPU's array: calls in order on one
 * stream are safe, calls that overlap on one GPU (several streams or threads at once) race. The array needs no
 * clearing (no call reads what it did not write). The stream's device must be the current device. The first call on
 * a GPU looks up the array's address there (hipGetSymbolAddress, no allocation): a caller that captures calls into a
 * HIP graph makes one call on that GPU before its capture, and the captured calls then replay as any other kernel. */
#define FH_ATTENTION_SCRATCH_BYTES (16u << 20)
int fh_attention_decode_noalloc(const float* q, const void* cache, int cache_dtype, int64_t cache_len, int batch,
                                int heads, int kv_heads, int head_dim, const int32_t* places, const int32_t* first_row,
                                int64_t max_context, void* o, int o_dtype, void* stream);

/* A prompt's causal attention (models/llama.py:129-142 over a chunk of consecutive places; prefill, 498-504): rows
 * t = 0 .. T-1 of q [T][ldq] (fp32) are places p0 + t of the sequence whose cache rows start at slot_row; row t
 * attends to cache rows slot_row .. slot_row + p0 + t, which must already hold its keys and values (the qkv GEMM's
 * FH_EP_ROPE_KV put them there). On the matrix cores: q, k, v and the softmax weights in bf16, scores and sums fp32;
 * head_dim 64 or 128. o: [T][ldo], fp32 or bf16 (for the next GEMM). No scratch memory. Replaces Tensor.attend's
 * prompt path (ferrite/tensor.py:487-516; attention_kernel, ferrite/compiler.py:1147-1316). */
int fh_attention_prefill(const float* q, int64_t ldq, const void* cache, int cache_dtype, int64_t cache_len, int T,
                         int heads, int kv_heads, int head_dim, int64_t p0, int64_t slot_row, void* o, int o_dtype,
                         int64_t ldo, void* stream);

/* out[rows][dim] = x * rsqrt(mean(x^2) + eps) * w (w + 1 when centered), fp32 or bf16 out: the RMSNorm before a
 * prefill GEMM (models/llama.py:82-85), which then takes bf16 rows. */
int fh_rms_rows(const float* x, int64_t ldx, int64_t rows, int64_t dim, const float* norm_w, float eps, int centered,
                void* out, int out_dtype, int64_t ldo, void* stream);

/* ---- mixture of experts (models/llama.py:277-329) ------------------------------------------------------------ */

/* Each row of x [rows][ldx] (fp32; RMSNorm'd first when norm_w is given, by its own sums of squares): the router's
 * logits x @ router (router [dim][experts], bf16 or fp32; fp32 sums), the k largest (the first of equals first:
 * numpy's stable argsort, models/llama.py:27; Tensor.topk, ferrite/tensor.py:373-388) and their weights: a softmax
 * over the k (norm_topk), or the softmax over all experts at the k. Out: ids [rows][k] int32, weights [rows][k] fp32,
 * and dense [rows][experts] fp32 (each row's weight for each expert, 0 where not picked; Tensor.touched's weights,
 * ferrite/tensor.py:403-416). experts <= 256, k <= 16. */
int fh_moe_route(const float* x, int64_t ldx, int rows, int64_t dim, const float* norm_w, float eps, int centered,
                 const void* router, int router_dtype, int experts, int k, int norm_topk, int32_t* ids, float* weights,
                 float* dense, void* stream);

/* The chosen experts' SwiGLUs, weighted and summed (numpy_experts / chip_experts' dense path, models/llama.py:294-321):
 * y = residual + sum_e dense[:, e] * (silu(h @ gate_e) * (h @ up_e)) @ down_e, h = x with the RMSNorm prologue
 * (norm_w, ssq_in as fh_gemv_bfp's). gate_up: the experts' [dim][2 ffn] weights packed one after another (FH_AXIS_N);
 * down: the experts' [ffn][dim] weights packed one after another. An expert no row picked reads no weight. residual
 * NULL: y is the sum alone; ssq_out: y's sums of squares by 16 columns. On the matrix cores, x and the SwiGLU outputs
 * in bf16 (fh_gemm_bfp's arithmetic); the experts' outputs summed in expert order. dim and ffn multiples of 64.
 * Workspace: fh_moe_workspace_bytes (a pass of 64 rows' gate_up and down outputs). */
size_t fh_moe_workspace_bytes(int rows, int experts, int64_t ffn, int64_t dim);
int fh_moe_experts(const float* x, int64_t ldx, int rows, int64_t dim, const float* norm_w, const float* ssq_in, float eps,
                   int centered, int experts, int64_t ffn, const void* gu_mant, const uint8_t* gu_exps, int gu_fmt,
                   const void* down_mant, const uint8_t* down_exps, int down_fmt, const float* dense, float* y,
                   const float* residual, float* ssq_out, void* workspace, size_t ws_bytes, void* stream);

/* ---- lazy tensors' kernels (ferrite/tensor.py: elementwise trees, reductions) ---------------------------------- */

/* out[b][r][c] = program at (b, r, c), out's dtype FH_F32, FH_BF16 (nearest even) or FH_I32; out rows ldo apart,
 * batches ldb apart (matrices one after another, ldb >= rows ldo, or interleaved row by row, ldo >= batch ldb). Replaces fused_kernel for an elementwise tree (ferrite/compiler.py:699). */
int fh_map(const fh_program* program, void* out, int out_dtype, int64_t batch, int64_t rows, int64_t cols, int64_t ldb,
           int64_t ldo, void* stream);

/* C[b] = program(A[b] @ B[b]) for plain operands (Tensor.matmul with a bf16 or fp32 B, ferrite/tensor.py:443-485):
 * A [M][K] rows lda apart, B [K][N] rows ldb apart, each FH_BF16 or FH_F32, batches a_batch_stride / b_batch_stride
 * elements apart (0: one matrix for every batch entry); C [M][N] rows ldc apart, FH_F32, FH_BF16 (nearest even) or
 * FH_I32. bf16 products summed in fp32; an FH_F32 operand as ferrite's bf16x3 (hi@hi + hi@lo + lo@hi, tensor.py:674-689).
 * program: the elementwise ops on the sum (FH_OPND_ACC), evaluated at (b, row, col); NULL stores the sum. */
int fh_matmul(const void* a, int a_dtype, int64_t a_batch_stride, int64_t lda, const void* b, int b_dtype,
              int64_t b_batch_stride, int64_t ldb, int64_t batch, int64_t M, int64_t K, int64_t N,
              const fh_program* program, void* c, int c_dtype, int64_t c_batch_stride, int64_t ldc, void* stream);

/* The program's values summed (FH_REDUCE_SUM) or their largest (FH_REDUCE_MAX) along an axis of (batch, rows, cols)
 * (0, 1 or 2), out holding the result with that axis 1 (ferrite/tensor.py's _reduce, 362-368; FOLDS and COMBINE,
 * ferrite/compiler.py:345-348). fp32 sums in a fixed order. */
#define FH_REDUCE_SUM 0
#define FH_REDUCE_MAX 1
int fh_reduce(const fh_program* program, int kind, int axis, int64_t batch, int64_t rows, int64_t cols, void* out,
              int out_dtype, void* stream);

/* Along each row of the program's values over (batch, rows, cols): softmax, exp(x - max) / sum exp(x - max), or with
 * log_form (x - max) - log sum exp(x - max), into out [batch][rows][cols] (FH_F32 or FH_BF16, nearest even):
 * Tensor.softmax / log_softmax along the last axis (ferrite/tensor.py:433-437) in one launch, the elementwise tree under
 * it evaluated in the same kernel. */
int fh_softmax_rows(const fh_program* program, int log_form, int64_t batch, int64_t rows, int64_t cols, void* out,
                    int out_dtype, void* stream);

/* For each row of x[rows][n] (fp32), its largest value's column (the first of equals), into ids[rows]: greedy
 * decoding's pick (models/llama.py:792, numpy's argmax). */
int fh_argmax_rows(const float* x, int64_t rows, int64_t n, int32_t* ids, void* stream);

/* The same pick from the (value, column) pairs an FH_EP_STORE epilogue left in argmax_parts: parts [rows][nparts]. */
int fh_argmax_parts(const void* parts, int64_t rows, int64_t nparts, int32_t* ids, void* stream);

/* ---- logit heads (models/serve.py:31-47; Head.of, 23-27) ------------------------------------------------------
 * Each row of logits [rows][ldl] (fp32, rows 16-byte aligned, ldl a multiple of 4): its k (1..64) largest values,
 * largest first, the first column of equal values first (numpy's stable argsort of -x; Tensor.topk's topk_kernel,
 * ferrite/compiler.py:1716-1838), into values [rows][k] and their columns into ids [rows][k]; and, given inv_temp
 * (each row's 1/temperature, [rows]), lse [rows] = log of the sum over the row of exp(x t), as max t + log sum
 * exp((x - max) t) in fp32. Selection is exact (no rounding of the values compared). A row is cut into parts of 4096
 * columns, a workgroup each, whose k best (and sums) a second kernel merges; at most 4096 / k parts (a vocabulary of
 * 262144 at k = 64). NaNs are not ordered as numpy orders them. Workspace: fh_heads_workspace_bytes (0 for one part),
 * no state kept between calls. */
size_t fh_heads_workspace_bytes(int rows, int64_t vocab, int k);
int fh_logit_heads(const float* logits, int64_t ldl, int rows, int64_t vocab, int k, const float* inv_temp,
                   float* values, int32_t* ids, float* lse, void* workspace, size_t ws_bytes, void* stream);

/* out[r][j] = src[r][idx[r][j]] (4-byte elements: int32 or fp32; rows lds, ldi, ldo apart), an index outside
 * [0, cols) read at the nearest column: Tensor.topk's labels, each pick's label instead of its column
 * (ferrite/tensor.py:373-388, topk_kernel's labels, compiler.py:1716-1838). */
int fh_gather_cols(const void* src, int64_t lds, int64_t cols, const int32_t* idx, int64_t ldi, int64_t rows, int64_t k,
                   void* out, int64_t ldo, void* stream);

/* Attention of a batch of query rows (Tensor.attend, ferrite/tensor.py:487-516): out[b][t] = softmax(q[b][t] k[b]^T +
 * mask) v[b] with q [batch][T][head_dim], k and v [batch][S][head_dim] (rows ld* apart, batches *_batch_stride apart,
 * q, k and v FH_BF16 or FH_F32, k and v alike), the scores in fp32; row t sees keys places[b][t] - window + 1 ..
 * places[b][t] (window 0: from key 0), clipped to the keys there are; a row seeing none is zeros. places int32, a
 * batch's places_batch_stride apart (0: one column for every matrix). head_dim up to 256. out FH_BF16 (nearest even) or
 * FH_F32. The general form; a decode step's attention over its KV cache is fh_attention_decode. */
int fh_attend(const void* q, int q_dtype, int64_t q_batch_stride, int64_t ldq, const void* k, const void* v, int kv_dtype,
              int64_t k_batch_stride, int64_t ldk, int64_t v_batch_stride, int64_t ldv, int64_t S, int batch, int64_t T,
              int head_dim, const int32_t* places, int64_t places_batch_stride, int64_t window, void* out, int out_dtype,
              int64_t out_batch_stride, int64_t ldo, void* stream);

/* A mixture of experts' choices ids [rows][k] (int32, values below n, rows ldi apart) as the lists an indexed matmul
 * takes (Tensor.touched / Tensor.group, ferrite/tensor.py:389-416; compiler.py:1842-1945). touched: experts [slots]
 * (slots = min(rows k, n)) the experts some row picks by a weight whose bits are not 0 (weights_in [rows][k] bf16, ldw
 * apart), increasing, then n; weights [slots][rows] bf16, the weight row r gave entry s's expert (0 if it did not pick
 * it). group: t = ceil(rows k / 32) + min(n, rows k) tiles of 32 slots, each value's choices a run of whole tiles after
 * the runs of the values before it, each choice (row by row, a row's in turn) the next slot of its value's run;
 * order [32 t] the row each slot holds (0 for none), tiles [t] each tile's value (n past those used), places
 * [k][rp] (rp = rows rounded up to 32) the slot of row r's choice j (0 past the rows). workspace: n int32. */
int fh_moe_touched(const int32_t* ids, int64_t ldi, const uint16_t* weights_in, int64_t ldw, int rows, int k, int n,
                   int32_t* experts, uint16_t* weights, void* stream);
int fh_moe_group(const int32_t* ids, int64_t ldi, int rows, int k, int n, int32_t* order, int32_t* tiles, int32_t* places,
                 int32_t* workspace, void* stream);

/* ---- rows by index (Tensor.gather / Tensor.put, ferrite/tensor.py:116-140) ----------------------------------
 * Rows of bytes in planes (a batch's matrices, or a block float's runs of 16 columns: its magnitudes' and exponents'
 * planes). Sizes and strides in bytes. gather: out[p][j] = src[p][ids[j]], an index outside [0, src_rows) read at the
 * nearest row; put: dst[p][ids[j]] = src[p][j], an index outside [0, dst_rows) writing nothing. A put with an index
 * twice writes one of the two rows. */
int fh_gather_rows(const void* src, int64_t src_rows, int64_t src_ld, int64_t src_plane, const int32_t* ids, int64_t n,
                   int64_t row_bytes, int64_t planes, void* out, int64_t out_ld, int64_t out_plane, void* stream);
int fh_put_rows(void* dst, int64_t dst_rows, int64_t dst_ld, int64_t dst_plane, const int32_t* ids, int64_t n,
                int64_t row_bytes, int64_t planes, const void* src, int64_t src_ld, int64_t src_plane, void* stream);

/* ---- measurement ------------------------------------------------------------------------------------------
 * The read floor a matmul's weight stream is measured against (bench.py's read_floor): `bytes` (a multiple of 16) of
 * src read once by `blocks` workgroups of 256 threads, 16 bytes a load and four loads in flight a thread, each
 * workgroup's xor of the 32-bit words it read into sink[block] ([blocks] uint32). No counterpart in the reference. */
int fh_read_probe(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream);
/* The matrix cores' own rate (bench.py's peaks): `blocks` workgroups of 4 waves, each wave `iters` rounds of 8
 * independent v_mfma_f32_32x32x16_bf16 (form 0; 32,768 FLOPs each) or v_mfma_f32_16x16x32_bf16 (form 1; 16,384),
 * operands in registers; each workgroup's sum of its results into sink[block] ([blocks] float). And the LDS read rate:
 * each of 256 threads a workgroup `iters` rounds of four 16-byte reads of a 16 KiB buffer, every 16 lanes on distinct
 * banks; each workgroup's xor into sink[block] ([blocks] uint32). No counterpart in the reference. */
int fh_mfma_probe(int form, int iters, float* sink, int blocks, void* stream);
int fh_lds_probe(int iters, uint32_t* sink, int blocks, void* stream);

#ifdef __cplusplus
}
#endif
#endif
