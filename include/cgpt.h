/*
 * cgpt.h — C ABI of libcgpt.so, the gfx950 (MI355X / CDNA4) kernels behind
 * cutilegpt_amd's drop-in replacements for cutileGPT's kernel functions.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and element strides (no
 *     framework types), and a HIP stream passed as `void*` (hipStream_t);
 *   - launches asynchronously on that stream and never allocates or frees;
 *   - validates its arguments before launching and returns a status:
 *       0            CGPT_OK
 *       < 0          an argument error (CGPT_E*), nothing was launched
 *       > 0          a hipError_t from the launch
 *   - keeps no state between calls except (a) per-device caches of the CU
 *     count and of kernel occupancies, filled on first use through atomics
 *     and read-only afterwards, safe from any thread, and (b) the per-GPU
 *     scratch array of cgpt_gemm_skinny_noalloc, which overlapping calls of
 *     that entry point on one GPU share and race on.  Every other entry point
 *     works only in the caller's buffers: concurrent calls on different
 *     streams are safe when their outputs (and workspaces) are distinct.
 *
 * Element types are CGPT_F32 (IEEE fp32), CGPT_BF16 (bfloat16 bit patterns)
 * and CGPT_F16 (IEEE binary16; the GEMM, LayerNorm, GELU, attention and
 * embedding entry points); all arithmetic is fp32, 16-bit outputs are rounded
 * to nearest even.
 *
 * Reference citations are relative to the falcons-eyes/cutileGPT checkout.
 */
#ifndef CGPT_H_
#define CGPT_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CGPT_ABI_VERSION 1

/* status codes */
#define CGPT_OK 0
#define CGPT_EINVAL (-1)       /* bad pointer, size, stride or alignment */
#define CGPT_EDTYPE (-2)       /* unsupported dtype combination */
#define CGPT_ESHAPE (-3)       /* shape outside what the kernels support */
#define CGPT_ESCRATCH (-4)     /* problem needs more than the static scratch holds */

/* element types */
#define CGPT_F32 0
#define CGPT_BF16 1
#define CGPT_F16 2

/* GEMM epilogues */
#define CGPT_EPI_NONE 0        /* C = A W^T                                  */
#define CGPT_EPI_BIAS 1        /* C = A W^T + bias                           */
#define CGPT_EPI_BIAS_GELU 2   /* C = gelu_tanh(A W^T + bias)                */
#define CGPT_EPI_BIAS_RESID 3  /* C = C + A W^T + bias (residual add in place) */

/* ABI version (CGPT_ABI_VERSION) of the loaded library. */
int cgpt_version(void);

/* Human-readable text for a status returned by any entry point. */
const char* cgpt_status_string(int status);

/*
 * Element-wise tanh-approximate GELU, y = 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))).
 * x and y hold n elements of `dtype`, contiguous; y may alias x.
 * Replaces cutile_gelu, cutile_gpt/kernels/gelu.py:71-110 (kernel :20-41).
 */
int cgpt_gelu(const void* x, void* y, int64_t n, int dtype, void* stream);

/*
 * Fused residual add + LayerNorm over rows of `cols` contiguous elements:
 *   s     = x + delta              (delta may be NULL: s = x)
 *   x_out = s                      (x_out may be NULL, or alias x)
 *   y     = (s - mean(s)) / sqrt(var(s) + eps) * gamma + beta   (biased var)
 * Row r of x / delta / x_out / y starts at r * cols.  gamma and beta hold
 * `cols` elements of `param_dtype`.  Statistics are accumulated in fp32.
 * Any cols >= 1 and any dtype mix of CGPT_F32 / CGPT_BF16 / CGPT_F16 with
 * element-aligned pointers: fp32 / bf16 rows (or all-fp16 rows with fp16 /
 * fp32 gamma and beta) of cols % 4 == 0, cols <= 4096, 16-byte (fp32) or
 * 8-byte (16-bit) aligned take the register-resident vector kernels, the rest
 * a block-per-row kernel (three passes over the row).
 * Replaces cutile_layer_norm, cutile_gpt/kernels/layernorm.py:77-135 (kernel
 * :24-74), fused with the residual adds at cutile_gpt/models/gpt.py:155,174.
 */
int cgpt_add_layernorm(const void* x, const void* delta, void* x_out,
                       const void* gamma, const void* beta, void* y,
                       int64_t rows, int64_t cols, float eps,
                       int x_dtype, int delta_dtype, int param_dtype, int y_dtype,
                       void* stream);

/*
 * cgpt_add_layernorm with delta given as a GEMM's split-K partial products
 * (cgpt_gemm_partials): delta[r][c] = P[0][r][c] + ... + P[n_parts-1][r][c]
 * + bias[c] (bias of param_dtype, may be NULL), added in that order and
 * rounded to delta_dtype — the value the GEMM's bias epilogue would have
 * stored — then s = x + delta, x_out, y as cgpt_add_layernorm.  P[s] row r at
 * partials + s * part_stride + r * ldp (16-byte aligned; ldp and part_stride
 * multiples of 4); 1 <= n_parts <= 16; x and x_out fp32.  Replaces
 * cutile_linear_bias + the residual add + cutile_layer_norm at decode shapes
 * (cutile_gpt/kernels/linear.py:112-222, layernorm.py:77-135,
 * cutile_gpt/models/gpt.py:155,174).
 */
int cgpt_add_layernorm_partials(const void* x, const float* partials, int64_t n_parts,
                                int64_t part_stride, int64_t ldp, const void* bias, void* x_out,
                                const void* gamma, const void* beta, void* y, int64_t rows,
                                int64_t cols, float eps, int x_dtype, int delta_dtype,
                                int param_dtype, int y_dtype, void* stream);

/*
 * The consumer of a split-K cgpt_gemm_partials whose output takes a bias and
 * an activation: out[r][c] = act(P[0][r][c] + ... + P[n_parts-1][r][c] +
 * bias[c]), the sums in fp32 in that order, rounded once to out_dtype — the
 * values the GEMM's own bias / GELU epilogue stores.  epilogue:
 * CGPT_EPI_BIAS (no activation) or CGPT_EPI_BIAS_GELU (tanh GELU).  P[s] row r
 * at partials + s * part_stride + r * ldp floats (16-byte aligned; ldp,
 * part_stride multiples of 4); 1 <= n_parts <= 16; cols % 4 == 0; bias of
 * bias_dtype, out of out_dtype (fp32 or bf16; 16- / 8-byte aligned), rows of
 * ldo >= cols elements, ldo % 4 == 0.  Replaces cutile_linear_bias +
 * cutile_gelu on the MLP up-projection at decode shapes
 * (cutile_gpt/models/gpt.py:161-167, kernels/linear.py:112-222,
 * kernels/gelu.py:20-41).
 */
int cgpt_partials_bias_act(const float* partials, int64_t n_parts, int64_t part_stride,
                           int64_t ldp, const void* bias, int bias_dtype, void* out, int64_t ldo,
                           int64_t rows, int64_t cols, int epilogue, int out_dtype, void* stream);

/*
 * C[M,N] = epilogue(A[M,K] * W[N,K]^T (+ bias[N])).
 * A row-major with leading dimension lda, W row-major (out_features, in_features)
 * with leading dimension ldw — the nn.Linear / cutileGPT `weight` layout, so no
 * transposed copy is needed — C row-major with leading dimension ldc.
 * in_dtype is the type of A and W (CGPT_BF16 -> bf16 MFMA, CGPT_F16 -> fp16
 * MFMA, CGPT_F32 -> fp32 MFMA); accumulation is fp32; bias (bias_dtype) is
 * added in fp32; C is written as out_dtype.  bias_dtype and out_dtype are
 * CGPT_F32 or the 16-bit type of the inputs' family (CGPT_F16 with fp16 inputs,
 * CGPT_BF16 otherwise).  Any K >= 1, lda >= K, ldw >= K and element-aligned
 * pointers: problems with K, lda and ldw multiples of 8 (16-bit) or 4 (fp32)
 * elements and 16-byte aligned A, W and bias take the vector kernels below;
 * others run a 64x64 register-staged kernel that loads element by element
 * (any tile id but CGPT_TILE_SKINNY is then ignored).  fp16 inputs run every
 * tile id as bf16 does, on the fp16 MFMA.
 * `tile` selects a tile configuration: CGPT_TILE_AUTO = library heuristic (the
 * skinny kernel when M <= 64, fp32 / bf16); CGPT_TILE_SKINNY = the
 * weight-streaming kernel for M <= 64 rows (decode steps: one row per
 * sequence), CGPT_ESHAPE above; fp32 and bf16 under the vector rules only.
 * With CGPT_EPI_BIAS_RESID (C += A W^T + bias in place, C usually the fp32
 * residual stream), tile 14 asks for the slab kernel's residual ring, 17-19
 * for those 4-wave pipeline tiles, a register-staged id (bf16 / fp16 0-4,
 * fp32 0-1) for that tile, and any other id means CGPT_TILE_AUTO.  A persistent launch (bf16 tile >= 5) over a
 * weight matrix of at least 32 MiB with M >= 1024 first reads W once on the
 * same stream (one extra kernel) so that the launch's repeated W band fetches
 * are served from the memory-side cache.
 * Replaces cutile_linear / cutile_linear_bias, cutile_gpt/kernels/linear.py:112-222
 * (kernels :37-109); CGPT_EPI_BIAS_GELU also absorbs cutile_gelu at
 * cutile_gpt/models/gpt.py:167.
 */
#define CGPT_TILE_AUTO (-1)
#define CGPT_TILE_SKINNY (-2)
int cgpt_gemm(const void* a, const void* w, const void* bias, void* c,
              int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
              int in_dtype, int bias_dtype, int out_dtype, int epilogue, int tile,
              void* stream);

/* Number of GEMM tile configurations compiled into the library. */
int cgpt_gemm_num_tiles(void);

/*
 * The skinny GEMM (M <= 64, e.g. one decode step's rows) with its K range also
 * split across blocks.  Same arguments and checks as cgpt_gemm, plus a caller
 * workspace (16-byte aligned, >= the bytes cgpt_gemm_skinny_workspace reports)
 * and n_counters ints that must be zero before the first call; every call
 * leaves them zero again, so they can be reused (and captured in a graph)
 * without clearing.  Partials are combined in a fixed order: results are
 * deterministic and identical to the tile = CGPT_TILE_SKINNY path's up to
 * summation order.  Calls sharing a workspace must not run concurrently.
 * workspace = NULL runs the unsplit kernel.  Replaces cutile_linear /
 * cutile_linear_bias at decode shapes (cutile_gpt/kernels/linear.py:112-222,
 * called per token by generate, cutile_gpt/models/gpt.py:185-229).
 */
int cgpt_gemm_skinny(const void* a, const void* w, const void* bias, void* c,
                     int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                     int in_dtype, int bias_dtype, int out_dtype, int epilogue,
                     void* workspace, int64_t workspace_bytes, int* counters,
                     int64_t n_counters, void* stream);

/* Workspace bytes and counters cgpt_gemm_skinny needs for (M, N, K, in_dtype). */
int cgpt_gemm_skinny_workspace(int64_t M, int64_t N, int64_t K, int in_dtype,
                               int64_t* workspace_bytes, int64_t* n_counters);

/*
 * cgpt_gemm_skinny with the split-K workspace and counters taken from a static
 * device array of the library (8 MiB + 1024 ints per GPU, held until the
 * process ends) instead of caller memory: allocates nothing (no hipMalloc,
 * hipFree or allocating library call), so it can run under HIP graph capture
 * and in loops that must not allocate.  No counterpart in the reference: it
 * exists for callers that cannot allocate.  Same arguments, checks and result
 * as cgpt_gemm_skinny given a workspace (bit-identical: the same kernels and
 * split); a problem whose workspace would exceed the array returns
 * CGPT_ESCRATCH (none with M <= 64 does).  The counters are cleared by a fill
 * kernel on `stream` at every call.  Every call on a GPU uses that GPU's one
 * array: calls that overlap in time on the same GPU (other streams or
 * threads) race.
 */
int cgpt_gemm_skinny_noalloc(const void* a, const void* w, const void* bias, void* c,
                             int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw,
                             int64_t ldc, int in_dtype, int bias_dtype, int out_dtype,
                             int epilogue, void* stream);

/*
 * Split-K partial products of a decode-shaped GEMM (M <= 64), left for the
 * consumer to add: P[s][m][n] = sum over k in chunk s of A[m,k] W[n,k] (fp32,
 * no bias), s < n_split, P[s] at partials + s * M * ldp (row stride ldp >= N
 * floats, partials 4-byte aligned).  K is cut into n_split chunks of
 * ceil(dslabs / n_split) double slabs (a double slab = 64 bf16 or 32 fp32 k);
 * 1 <= n_split <= dslabs.  Adding P[0] .. P[n_split-1] in order, plus the bias,
 * gives cgpt_gemm's result up to fp32 summation order; the decode step hands
 * them to cgpt_attention_decode_partials and cgpt_add_layernorm_partials, so
 * the GEMM is one memory round trip with no cross-block reduction.
 * A and W requirements as cgpt_gemm.  Replaces cutile_linear_bias at decode
 * shapes, cutile_gpt/kernels/linear.py:112-222 (split-K with a deferred
 * reduction has no counterpart in the reference).
 */
int cgpt_gemm_partials(const void* a, const void* w, float* partials, int64_t M, int64_t N,
                       int64_t K, int64_t lda, int64_t ldw, int64_t ldp, int64_t n_split,
                       int in_dtype, void* stream);

/* The n_split cgpt_gemm_partials is tuned for at (M, N, K, in_dtype); at most 16,
 * the most the partials consumers take. */
int cgpt_gemm_partials_plan(int64_t M, int64_t N, int64_t K, int in_dtype, int64_t* n_split);

/*
 * Causal (or full) softmax attention, O = softmax(Q K^T * scale + mask) V,
 * for B batches x H heads; Q has Tq rows, K/V have Tk rows (Tk >= Tq); query i
 * sits at absolute position Tk - Tq + i and, when `causal`, sees keys j <= that
 * position.  Every tensor is addressed as base + b*sb + h*sh + t*st + d with
 * unit stride along head_dim, so Q/K/V may be strided views into one fused QKV
 * projection buffer (B, T, 3, H, hd) and O may be written straight into
 * (B, T, H, hd).  Softmax statistics are fp32; P is rounded to `dtype` before
 * the P*V product.  head_dim in {16, 32, 64, 128}.
 * Replaces cutile_causal_attention, cutile_gpt/kernels/attention.py:119-175
 * (kernel :24-116) and the QKV split/transpose copies at
 * cutile_gpt/models/gpt.py:133-146.
 */
int cgpt_attention_fwd(const void* q, const void* k, const void* v, void* o,
                       int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t head_dim,
                       int64_t q_sb, int64_t q_sh, int64_t q_st,
                       int64_t k_sb, int64_t k_sh, int64_t k_st,
                       int64_t v_sb, int64_t v_sh, int64_t v_st,
                       int64_t o_sb, int64_t o_sh, int64_t o_st,
                       float scale, int causal, int dtype, void* stream);

/*
 * Token (+ position) embedding gather:
 *   out[i, :] = wte[idx[i], :] (+ wpe[pos0 + i % T, :])
 * for i < n_tokens; idx holds int64 token ids; wpe may be NULL (plain gather).
 * Ids outside [0, vocab) or positions outside [0, n_pos) are clamped into range
 * (so the kernel never reads out of bounds) and, when err_flag is not NULL,
 * set *err_flag (a device int) to 1.  Any D >= 1 with element-aligned
 * pointers (four-element vectors when D % 4 == 0 and rows are 16-byte (fp32) /
 * 8-byte (16-bit) aligned, else element by element); w_dtype CGPT_F32 or
 * CGPT_BF16 with out_dtype CGPT_F32 or CGPT_BF16, or CGPT_F16 with CGPT_F16 /
 * CGPT_F32.
 * Replaces cutile_embedding, cutile_gpt/kernels/embedding.py:54-109 (kernel
 * :23-51), fused with the token+position add at cutile_gpt/models/gpt.py:110-113.
 */
int cgpt_embedding(const int64_t* idx, const void* wte, const void* wpe, void* out,
                   int64_t n_tokens, int64_t T, int64_t D, int64_t vocab,
                   int64_t pos0, int64_t n_pos, int w_dtype, int out_dtype,
                   int* err_flag, void* stream);

/*
 * Embedding of one decode step: out[i, :] = wte[idx[i], :] + wpe[pos_base + *pos_dev, :]
 * for i < n_tokens (one token per sequence, all at the same position), with the
 * position read from device memory (an int) when the kernel runs, so a
 * captured step replays unchanged.  Clamping and err_flag as cgpt_embedding.
 * No reference counterpart: the reference re-embeds the whole prefix every
 * step (generate, cutile_gpt/models/gpt.py:185-229 calling forward :109-113).
 */
int cgpt_embedding_at(const int64_t* idx, const void* wte, const void* wpe, void* out,
                      int64_t n_tokens, int64_t D, int64_t vocab, int64_t pos_base,
                      const int* pos_dev, int64_t n_pos, int w_dtype, int out_dtype,
                      int* err_flag, void* stream);

/*
 * Token + position embedding fused with the first LayerNorm (ln_1 of layer 0):
 *   x_out[i, :] = wte[idx[i], :] + wpe[pos_i, :]                 (fp32 residual stream)
 *   y[i, :]     = (x_out[i, :] - mean) / sqrt(var + eps) * gamma + beta
 * with pos_i = pos0 + i % T, or pos0 + *pos_dev for every token when pos_dev is
 * not NULL (a decode step; T is then ignored).  wte, wpe, gamma and beta are
 * w_dtype, y is y_dtype; D % 4 == 0, D <= 4096.  Clamping and err_flag as
 * cgpt_embedding.  x_out and y equal, bit for bit, cgpt_embedding into an
 * fp32 buffer followed by cgpt_add_layernorm on it without a delta — one HBM
 * pass fewer (the LayerNorm does not read the rows back).
 * Replaces the embedding and the first LayerNorm of CutileGPT.forward,
 * cutile_gpt/models/gpt.py:110-113 and :120-122 (layer 0).
 */
int cgpt_embedding_layernorm(const int64_t* idx, const void* wte, const void* wpe,
                             const int* pos_dev, float* x_out, const void* gamma,
                             const void* beta, void* y, int64_t n_tokens, int64_t T, int64_t D,
                             int64_t vocab, int64_t pos0, int64_t n_pos, float eps, int w_dtype,
                             int y_dtype, int* err_flag, void* stream);

/*
 * Single-query attention over a KV cache, one decode step for B sequences x H
 * heads.  Cache element (b, h, t, d) lives at base + b*c_sb + h*c_sh + t*c_st + d
 * (k_cache and v_cache share the strides; 16-byte aligned rows).  With
 * pos = pos_base + (*pos_dev if pos_dev else 0): writes k_new / v_new (the
 * step's key and value, (b, h, d) at base + b*sb + h*sh + d) into cache row
 * pos, then o = softmax(q K[0..pos]^T * scale) V[0..pos] — the causal row of
 * position pos.  P is rounded to `dtype` before the P*V product, as in
 * cgpt_attention_fwd.  head_dim is a power-of-two number (2 to 32) of
 * 16-byte vectors: 16..256 (bf16), 8..128 (fp32); t_max * c_st * element
 * size < 2^31.
 * A device pos outside [0, t_max) is clamped and sets
 * *err_flag.  Replaces the per-token full recompute of cutile_causal_attention
 * inside generate (cutile_gpt/models/gpt.py:185-229, attention.py:119-175).
 */
int cgpt_attention_decode(const void* q, const void* k_new, const void* v_new,
                          void* k_cache, void* v_cache, void* o, int64_t B, int64_t H,
                          int64_t head_dim, int64_t t_max, int64_t pos_base,
                          const int* pos_dev, int64_t q_sb, int64_t q_sh,
                          int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh,
                          int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t o_sb,
                          int64_t o_sh, float scale, int dtype, int* err_flag,
                          void* stream);

/*
 * cgpt_attention_decode with the step's q, k and v given as the fused QKV
 * GEMM's split-K partial products (cgpt_gemm_partials over the c_attn weight):
 * value d of head h of sequence b is column off + h*head_dim + d of
 * P[0] + ... + P[n_parts-1] + qkv_bias (off = q_off / k_off / v_off; P[s] row
 * b at qkv_partials + s * part_stride + b * ldp; qkv_bias of `dtype`), added
 * in that order and rounded to `dtype` as the GEMM's output would be.
 * 1 <= n_parts <= 16.  Other arguments as cgpt_attention_decode.  Replaces
 * cutile_linear_bias on c_attn plus the attention of one generate step
 * (cutile_gpt/models/gpt.py:124-146,185-229).
 */
int cgpt_attention_decode_partials(const float* qkv_partials, int64_t n_parts,
                                   int64_t part_stride, int64_t ldp, const void* qkv_bias,
                                   int64_t q_off, int64_t k_off, int64_t v_off, void* k_cache,
                                   void* v_cache, void* o, int64_t B, int64_t H,
                                   int64_t head_dim, int64_t t_max, int64_t pos_base,
                                   const int* pos_dev, int64_t c_sb, int64_t c_sh, int64_t c_st,
                                   int64_t o_sb, int64_t o_sh, float scale, int dtype,
                                   int* err_flag, void* stream);

/*
 * Copy T positions of keys and values ((b, h, t, d) at base + b*sb + h*sh + t*st
 * + d, e.g. strided views into a fused QKV buffer) into cache rows
 * pos0 .. pos0+T-1 (cache strides as cgpt_attention_decode; pos0 + T <= t_max).
 * Fills the cache after a prefill.  No reference counterpart (the reference
 * keeps no cache, cutile_gpt/models/gpt.py:185-229).
 */
int cgpt_kv_store(const void* k, const void* v, void* k_cache, void* v_cache, int64_t B,
                  int64_t H, int64_t T, int64_t head_dim, int64_t pos0, int64_t t_max,
                  int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh,
                  int64_t v_st, int64_t c_sb, int64_t c_sh, int64_t c_st, int dtype,
                  void* stream);

/*
 * Greedy token per row: ids[r] = argmax_c x[r * ld + c] (the first maximum;
 * NaN entries are skipped), also stored at hist[r * hist_ld + *step_dev] when
 * hist is not NULL (step_dev NULL: column 0).  Replaces the top_k = 1 case of
 * generate's sampling, cutile_gpt/models/gpt.py:207-226.
 */
int cgpt_argmax(const void* x, int64_t rows, int64_t cols, int64_t ld, int dtype,
                int64_t* ids, int64_t* hist, int64_t hist_ld, const int* step_dev,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CGPT_H_ */
