/*
 * tkmi.h -- C ABI of libtkmi.so, the MI355X (gfx950) kernels of the
 * transformer-layer forward path.
 *
 * Conventions
 *   - Every entry point is extern "C", returns int: 0 on success, a negative
 *     TK_ERR_* code on a rejected argument, or TK_ERR_HIP when the HIP runtime
 *     reported an error at launch.  tk_last_error_string() describes the last
 *     failure on the calling thread.
 *   - All buffers are DEVICE pointers owned by the caller (the Python side
 *     allocates them with torch.empty).  No entry point allocates device or
 *     host memory, none synchronizes; each enqueues on `stream` (a
 *     hipStream_t passed as void*; NULL = the legacy default stream).
 *   - tk_half is IEEE binary16 storage.  Row-major layouts; leading
 *     dimensions (ld*) and strides are in ELEMENTS.
 *
 * The reference (danielfodgaard/transformer-kernel) exposes this path as
 * Python functions on torch tensors; each entry point below names the
 * reference interface it replaces (paths relative to the reference repo).
 */
#ifndef TKMI_H
#define TKMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TKMI_ABI_VERSION 3

typedef uint16_t tk_half;

enum tk_status {
  TK_OK = 0,
  TK_ERR_ARG = -1,         /* null pointer, bad size, bad stride, bad enum */
  TK_ERR_UNSUPPORTED = -2, /* valid request outside the kernels' envelope  */
  TK_ERR_HIP = -3          /* the HIP runtime rejected the launch          */
};

enum tk_dtype { TK_F32 = 0, TK_F16 = 1 };

/*
 * Padding masks.  `row_valid` arguments are nullable [rows] byte arrays
 * (nonzero = valid token; a torch bool tensor's storage); NULL means every
 * row is valid and the kernels take their unmasked path.  The row modes give
 * what an invalid row of a residual update becomes, following the baseline
 * block (src/torch_transformer_benchmark.py:119-120,141-142,170-171):
 */
enum tk_row_mode {
  TK_ROWS_KEEP_RESID = 1, /* s = resid: the attention output of a padded row is 0 */
  TK_ROWS_ZERO = 2,       /* s = 0: the block output of a padded row is 0           */
  TK_ROWS_ZERO_ALL = 3    /* s = 0 and the normalised output h = 0 (final norm)     */
};

enum tk_epilogue {
  TK_EPI_BIAS = 0,      /* C(f16)  = A.W^T + bias                          */
  TK_EPI_BIAS_GELU = 1, /* C(f16)  = gelu_erf(A.W^T + bias)                */
  TK_EPI_BIAS_RESID = 2 /* C(f32)  = resid + (A.W^T + bias); C may alias resid */
};

/* ABI version (TKMI_ABI_VERSION) of the loaded library. */
int tk_version(void);

/* Message for the last non-zero status returned on this thread ("" if none). */
const char *tk_last_error_string(void);

/*
 * LayerNorm over the last dim + cast.
 *   out[r, :] = (x[r,:] - mean) * rsqrt(var_pop + eps) * w + b   (fp32 math)
 * x: [rows, cols] f32 contiguous; w, b: [cols] f32; out: [rows, cols] of
 * out_dtype (TK_F16 or TK_F32).  cols in [1, 8192].  row_valid (nullable):
 * rows marked invalid are written as zeros (the final norm of a padded row,
 * src/torch_transformer_benchmark.py:170-171).
 * Replaces fused_kernels.ln_fwd / _ln_kernel (src/fused_kernels.py:164-193,
 * :80-112).
 */
int tk_ln_cast(const float *x, const float *w, const float *b, void *out,
               int out_dtype, int64_t rows, int64_t cols, float eps,
               const uint8_t *row_valid, void *stream);

/*
 * Residual add + LayerNorm + cast.
 *   s = x + y (added in fp32);  h = LN(s) (statistics of the fp32 sum) cast
 *   to h_dtype;  s stored in x's dtype.
 * x has x_dtype and y has y_dtype (TK_F16 or TK_F32 each); sum_out, when not
 * NULL, is [rows, cols] of x_dtype and may alias x (NULL: s not stored).
 * cols in [1, 8192].
 * Replaces fused_kernels.add_ln_fwd / _add_ln_kernel
 * (src/fused_kernels.py:196-238, :114-161; s = empty_like(x) at :216).
 */
int tk_add_ln_cast(const void *x, int x_dtype, const void *y, int y_dtype,
                   const float *w, const float *b, void *sum_out, void *h_out,
                   int h_dtype, int64_t rows, int64_t cols, float eps,
                   void *stream);

/*
 * GEMM  C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] )
 * A: [m, k] f16 (lda), W: [n, k] f16 (ldw) -- the nn.Linear weight layout,
 * bias: [n] f32 (may be NULL = 0), fp32 accumulation on MFMA.
 * epilogue TK_EPI_BIAS / TK_EPI_BIAS_GELU: C is f16 (ldc).
 * epilogue TK_EPI_BIAS_RESID: C is f32 (ldc), resid is f32 (ldr), C may
 * equal resid (in-place residual stream update).
 * Any k >= 0 with lda, ldw >= k; A and W 2-byte aligned.  When k, lda and
 * ldw are multiples of 8 and A, W 16-byte aligned the operands are read in
 * 16-byte vectors (the fast path); otherwise by element (odd d_model /
 * ffn_dim, which the reference's config validation accepts).
 * row_valid / row_mode (TK_EPI_BIAS_RESID only; row_valid nullable, m bytes):
 * an invalid row m is written as resid (TK_ROWS_KEEP_RESID) or 0
 * (TK_ROWS_ZERO, TK_ROWS_ZERO_ALL).
 * Replaces torch F.linear (+ F.gelu) in src/optimized.py:572,627,632-636.
 */
int tk_gemm(const tk_half *a, int64_t lda, const tk_half *w, int64_t ldw,
            const float *bias, const float *resid, int64_t ldr, void *c,
            int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue,
            const uint8_t *row_valid, int row_mode, void *stream);

/*
 * GEMM with the residual + LayerNorm + cast epilogue over full output rows:
 *   s = resid + A.W^T + bias (fp32);  h = LN(s; ln_w, ln_b, eps) -> h_dtype
 * sum_out (may be NULL, may alias resid) receives s.  Rows of n elements
 * must fit one tile: n in {128, 256, 512} (tk_gemm_ln_supported).
 * row_valid (nullable, m bytes) / row_mode: an invalid row takes s per
 * row_mode (tk_row_mode); h = LN(s), or 0 under TK_ROWS_ZERO_ALL.
 * Replaces F.linear followed by fused_kernels.add_ln_fwd
 * (src/optimized.py:523-553 with :627 / :636).
 */
int tk_gemm_bias_add_ln(const tk_half *a, int64_t lda, const tk_half *w,
                        int64_t ldw, const float *bias, const float *resid,
                        const float *ln_w, const float *ln_b, float *sum_out,
                        void *h_out, int h_dtype, int64_t m, int64_t n,
                        int64_t k, float eps, const uint8_t *row_valid,
                        int row_mode, void *stream);

/* 1 when tk_gemm_bias_add_ln handles rows of n elements, else 0. */
int tk_gemm_ln_supported(int64_t n);

/*
 * FlashAttention-2-style forward (online softmax, scores never stored).
 * q, k, v: logical [batch, heads, seq, head_dim] f16 with element strides
 * {b, h, s} given in *_strides[3] (head_dim stride is 1).  out: logical
 * [batch, heads, seq, head_dim] written through o_strides (pass
 * {S*H*hd, hd, H*hd} for the [B, S, H*hd] layout).
 * scores = (q.k^T) * scale in fp32, causal masks key > query, fp32 softmax,
 * fp16 P on MFMA for P.V, fp32 accumulation.
 * key_valid (nullable): key validity bytes, key s of batch b at
 * key_valid[b * key_valid_stride + s]; invalid keys are masked with -inf
 * like future keys (src/torch_transformer_benchmark.py:104-107).  A query
 * row with no valid key yields non-finite output (the baseline's NaN row);
 * callers zero such padded rows downstream.
 * Any head_dim <= 256 (tk_attention_supported) and any element strides;
 * q/k/v/out 2-byte aligned.  Head dims 16/32/64/128/256 with rows that are
 * 16-byte vectors (q, k; v too except at 128) and 8-byte vectors (out; v
 * at 128) take the tuned kernels; every other head dim or view runs on the
 * tile of the next power of two >= max(head_dim, 16) with element loads and
 * the head-dim tail read as zeros (src/kernels.py:262-263 pads the same way).
 * Replaces kernels.flash_attention / _flash_attn_fwd_kernel
 * (src/kernels.py:250-294, :137-247) and F.scaled_dot_product_attention
 * (src/optimized.py:615-626).
 */
int tk_flash_attn_fwd(const tk_half *q, const tk_half *k, const tk_half *v,
                      tk_half *out, int64_t batch, int64_t heads, int64_t seq,
                      int64_t head_dim, const int64_t *q_strides,
                      const int64_t *k_strides, const int64_t *v_strides,
                      const int64_t *o_strides, float scale, int causal,
                      const uint8_t *key_valid, int64_t key_valid_stride,
                      void *stream);

/* 1 when tk_flash_attn_fwd handles head_dim, else 0: the reference's rule
 * next_pow2(max(head_dim, 16)) <= 256, i.e. head_dim <= 256.
 * Replaces kernels.attention_supported (src/kernels.py:96-103). */
int tk_attention_supported(int64_t head_dim);

/*
 * Masked softmax over rows of materialised scores.
 * scores: [groups, seq, seq] f32 (query-major, one group per (b, h));
 * probs: same shape, f16.  causal masks key > query with -inf before the
 * fp32 softmax; key_len (may be NULL) gives per-batch valid key counts
 * (group g belongs to batch g / heads_per_batch) -- keys >= key_len masked.
 * A row whose keys are all masked yields zeros.
 * Replaces the masked softmax of the baseline attention
 * (src/torch_transformer_benchmark.py:99-111; src/optimized.py:658-666).
 */
int tk_masked_softmax(const float *scores, tk_half *probs, int64_t groups,
                      int64_t seq, int causal, const int32_t *key_len,
                      int64_t heads_per_batch, void *stream);

/*
 * The whole dense forward of a narrow model in one launch: for each of the
 * batch's sequences, every layer of
 *   h = LN1(x); qkv = h.W_qkv^T + b; ctx = attention(q, k, v);
 *   x += ctx.W_o^T + b_o; h = LN2(x); u = gelu(h.W_1^T + b_1);
 *   x += u.W_2^T + b_2
 * then out = LN_final(x), with the numerics of the layer-by-layer path
 * (fp16 operands, fp32 accumulation, residual and statistics).
 * x, out: [batch, seq, d_model] f32 (out may not alias x).
 * Weights stacked over the layers, each layer's block as the layer-by-layer
 * calls take it: w_qkv [L][3*heads*hd][d] f16 (head rows zero-padded to hd =
 * head_dim_padded), b_qkv [L][3*heads*hd] f32, w_o [L][d][heads*hd] f16,
 * b_o [L][d], w_1 [L][ffn][d] f16, b_1 [L][ffn], w_2 [L][d][ffn] f16,
 * b_2 [L][d], n1_w, n1_b, n2_w, n2_b [L][d] f32, nf_w, nf_b [d] f32; all
 * 16-byte aligned.
 * scale: the attention scale (1/sqrt(unpadded head_dim)).  Dense inputs only
 * (no padding mask).  Shapes: tk_small_forward_supported.
 * Causal sequences of more than 32 tokens run one 32-row block per
 * workgroup when batch * ceil(seq/32) workgroups fit on the device's CUs at
 * once and batch * layers * 4 <= 4096: the blocks of a sequence hand each
 * layer's K and V rows to one another through a workspace the library
 * allocates on the device the first time a call needs it (and replaces by a
 * larger one, keeping the old, when a call needs more; 16 KB per sequence,
 * layer and block, plus 16 KB), with
 * the same results bit for bit as one workgroup per sequence.  Calls that
 * overlap on one device share that workspace and must not run concurrently;
 * a call made while its stream is being captured into a graph, with no
 * workspace yet large enough, runs one workgroup per sequence instead.
 * Replaces the layer loop of OptimizedTransformer._run_layers_fused
 * (src/optimized.py:488-554) for the narrow configs (reference config 1 and
 * the appendix cases of src/configs/shapes.json with d_model 128).
 */
int tk_small_forward(const float *x, float *out, int64_t batch, int64_t seq,
                     int64_t d_model, int64_t heads, int64_t head_dim_padded,
                     int64_t ffn_dim, int64_t layers, int causal,
                     const tk_half *w_qkv, const float *b_qkv,
                     const tk_half *w_o, const float *b_o,
                     const tk_half *w_1, const float *b_1,
                     const tk_half *w_2, const float *b_2,
                     const float *n1_w, const float *n1_b,
                     const float *n2_w, const float *n2_b,
                     const float *nf_w, const float *nf_b, float n1_eps,
                     float n2_eps, float nf_eps, float scale, void *stream);

/* tk_small_forward without any allocation: the same arguments, work and
 * results (bit for bit), but a split launch hands its K/V rows through a
 * fixed per-device scratch array (16 MB + 16 KB, in the library's code
 * object: each device holds it from the library's load until the process
 * ends) instead of the library's allocated workspace, and its count table is
 * cleared by a small kernel at each call.  Returns TK_ERR_UNSUPPORTED when a
 * split launch would need more than 1024 hand-off slots (batch * layers * 4
 * row blocks, e.g. C1's B64 L4); shapes that run unsplit use no scratch.
 * Calls that overlap on one device share that device's array and race.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int tk_small_forward_noalloc(const float *x, float *out, int64_t batch,
                             int64_t seq, int64_t d_model, int64_t heads,
                             int64_t head_dim_padded, int64_t ffn_dim,
                             int64_t layers, int causal, const tk_half *w_qkv,
                             const float *b_qkv, const tk_half *w_o,
                             const float *b_o, const tk_half *w_1,
                             const float *b_1, const tk_half *w_2,
                             const float *b_2, const float *n1_w,
                             const float *n1_b, const float *n2_w,
                             const float *n2_b, const float *nf_w,
                             const float *nf_b, float n1_eps, float n2_eps,
                             float nf_eps, float scale, void *stream);

/* Fused QKV projection + attention for one-key-tile sequences:
 *   ctx[t, h*64 + :64] = attention_h( h . W_qkv^T + b_qkv )
 * i.e. tk_gemm(h, w_qkv, b_qkv) into a [T, 3*d_model] q|k|v buffer followed
 * by tk_flash_attn_fwd on its strided views, without the buffer: q, k and v
 * of one head for two sequences stay in LDS.  h: [batch*seq, ldh] fp16;
 * w_qkv: [3*d_model, ldw] fp16 (rows q, k, v, each head's 64 rows
 * contiguous); b_qkv: [3*d_model] fp32; ctx: [batch*seq, ldc] fp16;
 * d_model = heads * head_dim.  Dense inputs only.  Shapes:
 * tk_qkv_attention_supported (seq = 64, head_dim = 64, batch*seq a multiple
 * of 128).  Replaces F.linear + scaled_dot_product_attention of
 * OptimizedTransformer._attention_block (src/optimized.py:572-626) for those
 * shapes (the reference's config 2). */
int tk_qkv_attention(const tk_half *h, int64_t ldh, const tk_half *w_qkv,
                     int64_t ldw, const float *b_qkv, tk_half *ctx,
                     int64_t ldc, int64_t batch, int64_t seq, int64_t heads,
                     int64_t head_dim, float scale, int causal, void *stream);

/* 1 when tk_qkv_attention takes the shape, else 0.  No counterpart in the
 * reference (its attention block always materialises q, k, v). */
int tk_qkv_attention_supported(int64_t batch, int64_t seq, int64_t heads,
                               int64_t head_dim);

/* 1 when tk_small_forward takes the shape (seq <= 128, d_model = ffn_dim =
 * 128, heads * head_dim_padded = 128, head_dim_padded in {16, 32, 64, 128}),
 * else 0.  No counterpart in the reference (its narrow configs run the
 * layer loop). */
int tk_small_forward_supported(int64_t seq, int64_t d_model, int64_t heads,
                               int64_t head_dim_padded, int64_t ffn_dim);

#ifdef __cplusplus
}
#endif

#endif /* TKMI_H */
