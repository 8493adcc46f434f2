/*
 * libnsw — MI355X (gfx950) kernels for the shifted-window Swin block forward
 * of neural-scaling-weather, behind a plain C ABI.
 *
 * Conventions
 *  - All tensors are dense, row-major, device pointers; the caller allocates
 *    every input, output and workspace (no entry point allocates).
 *  - `dtype` is NSW_DTYPE_F32 (fp32 storage and arithmetic, the reference's
 *    inference precision) or NSW_DTYPE_BF16 (bf16 storage, fp32 accumulation).
 *  - `stream` is a hipStream_t passed as void*; kernels are enqueued
 *    asynchronously, no entry point synchronises the host.
 *  - Return value: NSW_OK (0) or an NSW_ERR_* code; nsw_last_error() returns
 *    the thread-local message of the last failure.
 *  - Image layout is the reference's channels-last [B, T, H, W, C]; the
 *    window-ordered layout is [B*nW, T*ws0*ws1, C] with window index
 *    b*nW + i*(W/ws1) + j (models/swin_helpers.py:26-51).
 *
 * The reference is pure Python; the entry points below replace the library
 * calls that its Swin block makes (file:line of the reference given for
 * each).  There is no C ABI in the reference to bind against.
 */
#ifndef NSW_H_
#define NSW_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSW_OK 0
#define NSW_ERR_INVALID 1     /* bad shape / argument */
#define NSW_ERR_UNSUPPORTED 2 /* valid for the reference but not implemented here */
#define NSW_ERR_HIP 3         /* a HIP runtime call failed */

#define NSW_DTYPE_F32 0
#define NSW_DTYPE_BF16 1

/* GEMM epilogues for nsw_linear. */
#define NSW_EPI_NONE 0          /* y = x W^T                                   */
#define NSW_EPI_BIAS 1          /* y = x W^T + b                               */
#define NSW_EPI_BIAS_GELU 2     /* y = gelu_erf(x W^T + b)                     */
#define NSW_EPI_BIAS_RESIDUAL 3 /* y = x W^T + b + residual                    */
#define NSW_EPI_BIAS_GELU_TANH 4 /* y = gelu_tanh(x W^T + b): the tanh-form GELU of
                                    the reference's TE block ("gelu" activation of
                                    te.LayerNormMLP, models/swin_helpers_te.py:318-323) */

const char* nsw_last_error(void);
int nsw_version(void);

/* torch.roll of [B,T,H,W,C] by (s0, s1) over dims (H, W):
 * y[b,t,h,w] = x[b,t,(h-s0) mod H,(w-s1) mod W].
 * Replaces RollForwardReverseRollBackward.forward
 * (distributed/mappings.py:121-132 -> distributed/helpers.py:210-212). */
int nsw_roll_hw(const void* x, void* y, int64_t B, int64_t T, int64_t H, int64_t W, int64_t C,
                int64_t s0, int64_t s1, int dtype, void* stream);

/* window_partition (models/swin_helpers.py:26-51):
 * [B,T,H,W,C] -> [B*nW, T, ws0, ws1, C]. */
int nsw_window_partition(const void* x, void* windows, int64_t B, int64_t T, int64_t H,
                         int64_t W, int64_t C, int64_t ws0, int64_t ws1, int dtype, void* stream);

/* window_reverse (models/swin_helpers.py:54-77):
 * [B*nW, T, ws0, ws1, C] -> [B,T,H,W,C]. */
int nsw_window_reverse(const void* windows, void* x, int64_t B, int64_t T, int64_t H,
                       int64_t W, int64_t C, int64_t ws0, int64_t ws1, int dtype, void* stream);

/* Fused roll by -shift + window_partition (models/swin_helpers.py:402-412):
 * windows[w, t, r, c] = x[b, t, (i*ws0 + r + s0) mod H, (j*ws1 + c + s1) mod W]. */
int nsw_roll_window_partition(const void* x, void* windows, int64_t B, int64_t T, int64_t H,
                              int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                              int64_t s1, int dtype, void* stream);

/* Fused window_reverse + roll by +shift (models/swin_helpers.py:420-431):
 * exact inverse of nsw_roll_window_partition. */
int nsw_window_reverse_roll(const void* windows, void* x, int64_t B, int64_t T, int64_t H,
                            int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                            int64_t s1, int dtype, void* stream);

/* nsw_roll_window_partition that also writes the partial sums of squares of
 * every window-order row it stores: row_sumsq [B*T*H*W, nparts] fp32, part p
 * = sum of the squares of the row's stored elements in bytes [512p, 512p+512)
 * (nparts = ceil(C * dtype size / 512)).  The pre-pass of
 * nsw_swin_blocks_forward: the tokens of models/swin.py:307-308's first
 * block in its window order plus the norm1 statistics its QKV GEMM reads. */
int nsw_window_partition_sumsq(const void* x, void* windows, float* row_sumsq, int64_t B, int64_t T,
                               int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                               int64_t s1, int dtype, void* stream);

/* Block._make_attention_mask (models/swin_helpers.py:322-397), one GPU,
 * causal=False: writes the additive fp32 mask [nW, T*wa, T*wa], values
 * {0, -100}. */
int nsw_make_attention_mask(float* mask, int64_t H, int64_t W, int64_t ws0, int64_t ws1,
                            int64_t s0, int64_t s1, int64_t T, void* stream);

/* Host-only self-check (no counterpart in the reference): the exact
 * division by launch constants that the window <-> token row maps use
 * (roll, partition, reverse, the fused gathers and the proj scatter), tested
 * against '/' over divisors 1..4096 and large ones at the numerators where an
 * off-by-one would show.  Returns the number of mismatches (0 = pass); needs
 * no GPU. */
int nsw_selftest_fastdiv(void);

/* Measurement only (no counterpart in the reference): copies the MFMA GEMM's
 * per-tile phase stamps of the last launch to host memory, 8 64-bit words
 * per tile (s_memtime at the tile's start, once its first stages have
 * landed, after the main loop, after the first epilogue phase is staged,
 * at its end; HW_ID; XCC_ID; workgroup id), for up to 65536 tiles.  Only a
 * library built with the stamps compiled in (build.py --stamps ->
 * nsw/libnsw_stamps.so) records them; the default library returns
 * NSW_ERR_UNSUPPORTED. */
int nsw_gemm_read_stamps(void* host, size_t bytes);

/* nn.RMSNorm over the last dim (models/layer_helpers.py:101-119):
 * y = x * rsqrt(mean(x^2) + eps) * w, rows x C. */
int nsw_rmsnorm(const void* x, const void* w, float eps, void* y, int64_t rows, int64_t C,
                int dtype, void* stream);

/* nn.LayerNorm over the last dim (NormLayer with norm_type="layer_norm",
 * models/layer_helpers.py:94-100,118-119): y = (x - mean) / sqrt(var + eps)
 * * w + b, biased variance, rows x C; w and b may be NULL (no affine). */
int nsw_layernorm(const void* x, const void* w, const void* b, float eps, void* y, int64_t rows,
                  int64_t C, int dtype, void* stream);

/* Fused norm1 + cyclic roll by -shift + window_partition
 * (models/swin_helpers.py:446 + :402-412): x [B,T,H,W,C] -> xw [B*nW*T*wa, C]. */
int nsw_rmsnorm_roll_partition(const void* x, const void* w, float eps, void* xw, int64_t B,
                               int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0,
                               int64_t ws1, int64_t s0, int64_t s1, int dtype, void* stream);

/* F.linear + BiasLayer (+ GELU / residual) (models/layer_helpers.py:41-42,71-72,
 * models/mlp.py:80-93): y[M,N] = epi(x[M,K] . w[N,K]^T).  bias / residual may
 * be NULL when the epilogue does not use them.  Requires K % 32 == 0 (bf16) or
 * K % 16 == 0 (f32) (one MFMA step of k), N % 8 == 0, 16-byte aligned x, w, y
 * and residual. */
int nsw_linear(const void* x, const void* w, const void* bias, const void* residual, void* y,
               int64_t M, int64_t N, int64_t K, int epilogue, int dtype, void* stream);

/* q/k/v projections with their biases and the per-head q/k RMSNorm
 * (models/swin_helpers.py:216-234): qkv[M, 3C] = x[M,C] . wqkv[3C,C]^T + bqkv,
 * then columns [0,C) (q) and [C,2C) (k) are RMS-normalised per head of hd
 * columns with weights qn_w[hd], kn_w[hd].  wqkv/bqkv are the q, k, v weights
 * / biases stacked in that order.  Requires C % 16 == 0, hd in {4,8,16,32,64}
 * and C (the GEMM's k) a multiple of 32 (bf16) / 16 (f32). */
int nsw_qkv_projection(const void* x, const void* wqkv, const void* bqkv, const void* qn_w,
                       const void* kn_w, float eps, void* qkv, int64_t M, int64_t C,
                       int64_t num_heads, int dtype, void* stream);

/* Attention core of WindowMultiHeadAttention.forward (models/swin_helpers.py:236-249):
 * per window and head, o = softmax(q k^T * scale + mask) v, heads merged back
 * into o[Bw*L, C].  qkv is the [Bw*L, 3C] output of nsw_qkv_projection.
 * Mask: if `mask` is non-NULL it is the additive fp32 [nW_mask, L, L] tensor
 * broadcast over windows (window w uses mask[w % nW_mask]); otherwise, when
 * (s0, s1) != (0, 0) the reference's latitude shift mask is computed from
 * indices for the geometry (H, W, ws0, ws1, s0, T), else no mask. */
int nsw_window_attention(const void* qkv, void* o, const float* mask, int64_t nW_mask,
                         int64_t Bw, int64_t L, int64_t C, int64_t num_heads, float scale,
                         int64_t H, int64_t W, int64_t ws0, int64_t ws1, int64_t s0,
                         int64_t s1, int64_t T, int dtype, void* stream);

/* proj + bias + window_reverse + roll by +shift + residual
 * (models/swin_helpers.py:250-254, :420-431, :449):
 * y[token(m)] = o[m] . wproj^T + bproj + skip[token(m)], y and skip [B,T,H,W,C]. */
int nsw_proj_reverse_residual(const void* o, const void* wproj, const void* bproj,
                              const void* skip, void* y, int64_t B, int64_t T, int64_t H,
                              int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                              int64_t s1, int dtype, void* stream);

/* Number of partial sums per row that nsw_proj_reverse_residual_sumsq writes
 * for rows of C elements: one per 512 bytes of row, ceil(C * esize / 512). */
int64_t nsw_row_sumsq_parts(int64_t C, int dtype);

/* nsw_proj_reverse_residual that also writes, for each output row (token t),
 * partial sums of the squares of the values it stores (after the residual,
 * in the output dtype): row_sumsq[t * P + p] = sum of y[t, c]^2 over the p-th
 * 512-byte segment of the row, P = nsw_row_sumsq_parts(C, dtype), fp32.
 * These are the statistics of Block.forward's norm2 (models/swin_helpers.py
 * :457, nn.RMSNorm over h1), so that the consumer GEMM (nsw_linear_rowscale)
 * normalises h1 without a separate pass over it. */
int nsw_proj_reverse_residual_sumsq(const void* o, const void* wproj, const void* bproj,
                                    const void* skip, void* y, float* row_sumsq, int64_t B,
                                    int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0,
                                    int64_t ws1, int64_t s0, int64_t s1, int dtype, void* stream);

/* Whole Block.forward (models/swin_helpers.py:435-459). */
typedef struct nsw_block_params {
  const void* norm1_w;   /* [C]          norm1.norm.weight                      */
  const void* wqkv;      /* [3C, C]      attn.{q,k,v}.weight stacked            */
  const void* bqkv;      /* [3C]         attn.bias{q,k,v}.bias stacked          */
  const void* qn_w;      /* [hd]         attn.q_norm.norm.weight                */
  const void* kn_w;      /* [hd]         attn.k_norm.norm.weight                */
  const void* wproj;     /* [C, C]       attn.proj.weight                       */
  const void* bproj;     /* [C]          attn.biasproj.bias                     */
  const void* norm2_w;   /* [C]          norm2.norm.weight                      */
  const void* w1;        /* [Hm, C]      mlp.fc1.weight                         */
  const void* b1;        /* [Hm]         mlp.bias1.bias                         */
  const void* w2;        /* [C, Hm]      mlp.fc2.weight                         */
  const void* b2;        /* [C]          mlp.bias2.bias                         */
  /* Optional norm-folded weights: w1_n2[n,k] = w1[n,k] * norm2_w[k] removes
   * the norm2 pass (the proj GEMM writes h1's row sums of squares, fc1 applies
   * the row scale); wqkv_n1[n,k] = wqkv[n,k] * norm1_w[k] folds norm1 into
   * the QKV GEMM.  Both given: the block runs as the one-block window-order
   * chain of nsw_swin_blocks_forward (partition + norm1 sums, QKV with norm1
   * as a row scale, attention, proj + norm2 sums in window order, fc1, fc2
   * scattering to tokens: 6 launches).  w1_n2 alone: norm1 gather, proj
   * scattering to tokens with the sums (6 launches, the default of
   * nsw.Block; both 6-launch forms measure the same at config 2).  Neither:
   * norm2 as a pass of its own (7 launches).  wqkv_n1 alone is refused
   * (NSW_ERR_INVALID). */
  const void* wqkv_n1;   /* [3C, C] or NULL                                     */
  const void* w1_n2;     /* [Hm, C] or NULL                                     */
} nsw_block_params;

typedef struct nsw_block_shape {
  int64_t B, T, H, W, C;   /* image [B,T,H,W,C]                                 */
  int64_t num_heads;
  int64_t ws0, ws1;        /* window_size                                       */
  int64_t s0, s1;          /* shift_size ((0,0) for unshifted blocks)          */
  int64_t hidden;          /* MLP hidden features = int(C * mlp_ratio)          */
  float eps;               /* RMSNorm eps (nn.RMSNorm eps=None: finfo(dtype).eps)*/
  int dtype;
  int gelu_tanh;           /* 0: exact-erf GELU (nn.GELU(), models/mlp.py:55);  */
                           /* 1: tanh form (the TE block's "gelu")              */
} nsw_block_shape;

/* Bytes of device workspace nsw_swin_block_forward needs (for any choice
 * of the optional weights). */
size_t nsw_block_workspace_size(const nsw_block_shape* s);

/* y = Block.forward(x); x and y [B,T,H,W,C] must not alias. */
int nsw_swin_block_forward(const void* x, void* y, const nsw_block_params* p,
                           const nsw_block_shape* s, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Bytes of device workspace nsw_swin_blocks_forward needs for depth blocks of
 * the shapes given (0 for a malformed shape). */
size_t nsw_blocks_workspace_size(const nsw_block_shape* shapes, int64_t depth);

/* The blocks loop of SwinTransformer.forward (models/swin.py:307-308,
 * `for blk in self.blocks: x = blk(x)`): y = blocks[depth-1](...blocks[0](x)),
 * x and y [B,T,H,W,C] in token order, must not alias.  The residual stream
 * stays in window order between the blocks (each block's last GEMM stores its
 * rows in the next block's window order together with their norm1
 * statistics), so the result equals depth nsw_swin_block_forward calls up to
 * the rounding of the folded norms.  Every block needs the norm-folded
 * weights wqkv_n1 and w1_n2; all blocks share B,T,H,W,C, heads, window,
 * hidden and dtype (shift and eps may differ).  1 + 5*depth launches. */
int nsw_swin_blocks_forward(const void* x, void* y, const nsw_block_params* params,
                            const nsw_block_shape* shapes, int64_t depth, void* workspace,
                            size_t workspace_bytes, void* stream);

/* nsw_swin_blocks_forward from block 0's input already in block 0's window
 * order with its norm1 statistics: xw [B*T*H*W, C] as nsw_roll_window_partition
 * (shift shapes[0].s0, s1) lays out the tokens, row_sumsq [B*T*H*W, nparts]
 * fp32 (16-byte aligned) as nsw_window_partition_sumsq writes them -- e.g. the
 * patch-embedding GEMM of models/swin.py:269-284 with nsw_linear_remap_residual
 * map mode 3.  xw and row_sumsq are read only; y in token order.  5*depth
 * launches. */
int nsw_swin_blocks_forward_windowed(const void* xw, const float* row_sumsq, void* y,
                                     const nsw_block_params* params, const nsw_block_shape* shapes,
                                     int64_t depth, void* workspace, size_t workspace_bytes, void* stream);

/* WeightedRMSE.forward (utils/losses.py:243-266) and the textbook weighted ACC.
 * pred/target fp32 [P, H, W] with P = B*T*Cch planes (channel = plane % Cch);
 * w float64 [H, w_cols] with w_cols = 1 (cos-lat weights, the inference path,
 * utils/dataloaders/era5hdf5.py:159) or w_cols = W (a full map, as the
 * reference's tests/test_metrics.py:62-63 uses); clim fp32 [Cch] or NULL (no
 * ACC).  Writes per-plane rmse[P] = sqrt(sum_hw w (p-t)^2 / (H*W)) and, when
 * clim != NULL, acc[P] = sum w af ao / sqrt(sum w af^2 * sum w ao^2)
 * (float64).  Deterministic (fixed reduction order). */
size_t nsw_weighted_metrics_workspace_size(int64_t P, int64_t H, int64_t W);
int nsw_weighted_metrics(const float* pred, const float* target, const double* w,
                         int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                         int64_t Cch, double* rmse, double* acc, void* workspace,
                         size_t workspace_bytes, void* stream);

/* The same metrics on unnormalised fields (the inference loop,
 * utils/inferencer.py:390-391,405-412): pred (fp32 or bf16, pred_dtype) and
 * target (fp32) are both mapped x -> x * std_c[c] + mean_c[c] (product and sum
 * rounded separately, as the reference's two tensor ops) before the
 * reduction.  std_c / mean_c fp32 [Cch]; workspace as above. */
int nsw_weighted_metrics_unnorm(const void* pred, int pred_dtype, const float* target,
                                const float* std_c, const float* mean_c, const double* w,
                                int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                int64_t Cch, double* rmse, double* acc, void* workspace,
                                size_t workspace_bytes, void* stream);

/* nsw_weighted_metrics_unnorm with float64 statistics (std_c / mean_c
 * float64 [Cch]): the reference's torch.as_tensor(stats) keeps the dtype of
 * the stats file (utils/dataloaders/era5hdf5.py:111-122, utils/inferencer.py
 * :390-391,405-412), and float64 statistics promote the unnormalised fields,
 * their difference and its square to float64; here they are computed in
 * float64 likewise. */
int nsw_weighted_metrics_unnorm_f64stats(const void* pred, int pred_dtype, const float* target,
                                         const double* std_c, const double* mean_c, const double* w,
                                         int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                         int64_t Cch, double* rmse, double* acc, void* workspace,
                                         size_t workspace_bytes, void* stream);

/* Allocation-free variant of nsw_weighted_metrics_unnorm.  No counterpart in
 * the reference: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops).  Same arguments without the workspace; the
 * partial sums live in a library-owned device array of
 * NSW_METRICS_SCRATCH_BYTES per GPU (held until the process ends), enough
 * for nsw_weighted_metrics_workspace_size(P, H, W) <= that size (e.g. every
 * P <= 32768 planes); larger inputs return NSW_ERR_INVALID.  The stream must
 * belong to the current device.  Calls that overlap on one GPU share the
 * array and race; calls in one stream's order are safe. */
#define NSW_METRICS_SCRATCH_BYTES (1 << 20)
int nsw_weighted_metrics_unnorm_noalloc(const void* pred, int pred_dtype, const float* target,
                                        const float* std_c, const float* mean_c, const double* w,
                                        int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                        int64_t Cch, double* rmse, double* acc, void* stream);

/* y = epi(RMSNorm(x; norm_w, eps) . W^T) (norm2 + MLP fc1, models/swin_helpers.py
 * :457, models/mlp.py:80-85) with the row statistics supplied by x's producer:
 * w_n[n,k] = W[n,k] * norm_w[k], rs[m] = 1/sqrt(sum_p row_sumsq[m*nparts + p] / K
 * + eps) applied to each row of x . w_n^T before the bias.  row_sumsq as
 * written by nsw_proj_reverse_residual_sumsq.  Epilogues and requirements as
 * nsw_linear. */
int nsw_linear_rowscale(const void* x, const void* w_n, const void* bias, const void* residual, void* y,
                        const float* row_sumsq, int64_t nparts, int64_t M, int64_t N, int64_t K,
                        int epilogue, float eps, int dtype, void* stream);

/* WindowMultiHeadAttention's q/k/v projections with their per-head q/k
 * RMSNorms (models/swin_helpers.py:212-241) on rows whose norm1
 * (swin_helpers.py:446, nn.RMSNorm) comes as a row scale from partial sums of
 * squares supplied by the rows' producer: qkv[m] = headnorm(rs[m] *
 * (x[m] . wqkv_n^T) + bqkv), wqkv_n = wqkv * norm1_w per input column, rs[m]
 * = 1/sqrt(sum_p row_sumsq[m*nparts + p] / C + eps).  x [M, C] in any row
 * order (window order in the blocks), qkv [M, 3C]; row_sumsq 16-byte
 * aligned.  Requires C % 16 == 0, hd in {4,8,16,32,64} and C (the GEMM's k)
 * a multiple of 32 (bf16) / 16 (f32). */
int nsw_qkv_projection_rowscale(const void* x, const void* wqkv_n, const void* bqkv, const void* qn_w,
                                const void* kn_w, float eps, void* qkv, const float* row_sumsq,
                                int64_t nparts, int64_t M, int64_t C, int64_t num_heads, int dtype,
                                void* stream);

/* The residual adds of Block.forward (models/swin_helpers.py:452-458: x +
 * attn-branch, h1 + mlp-branch) on window-ordered rows: y[map(m)] = x[m] .
 * w^T + bias + residual[m], and, for map modes 0 and 2, the stored rows'
 * partial sums of squares into row_sumsq [rows, nparts] at the same rows
 * (nparts = nsw_row_sumsq_parts(N, dtype): the statistics of the norm that
 * consumes y).  map_mode 0: map(m) = m; 1: the token of window row m of the
 * image (B,T,H,W, window ws, shift s) — window_reverse + roll by +shift,
 * :424-431; 2: that token's row in the window order of the same image with
 * shift (sa, sb) — the next block's roll + window_partition, :402-412; 3:
 * row m is token m and map(m) its row in the window order of the image with
 * shift s (roll + window_partition of token-ordered rows: the first block's
 * input).  row_sumsq NULL for mode 1, required otherwise.  Requirements as
 * nsw_linear; residual and y must not alias. */
int nsw_linear_remap_residual(const void* x, const void* w, const void* bias, const void* residual, void* y,
                              float* row_sumsq, int64_t M, int64_t N, int64_t K, int map_mode, int64_t B,
                              int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1, int64_t s0,
                              int64_t s1, int64_t sa, int64_t sb, int dtype, void* stream);

/* Patch matrix of the stride-p patch convolution (PatchEmbedLayer,
 * models/layer_helpers.py:120-172, as called by SwinTransformer.prepare_tokens,
 * models/swin.py:269-277, and for the coordinate embedding, :278-282).
 * x [B, T, C_x, H, W] (x_dtype); inv [C_inv, H, W] or NULL appended as extra
 * channels (the preprocessor's concatenation, utils/data_utils.py:185-189);
 * frame t is read from slot (t + frame0) mod T (a ring-buffered input
 * window, utils/inferencer.py:448-449).  out [B*T*(H/p)*(W/p), Kp]
 * (out_dtype), row (b, t, i, j), column (c*p + u)*p + v, zero for columns
 * >= (C_x + C_inv)*p*p.  Requires p | H, p | W, p <= 16, Kp a multiple of 8
 * (bf16) / 4 (f32), 16-byte aligned out. */
int nsw_patch_im2col(const void* x, const void* inv, int64_t B, int64_t T, int64_t C_x,
                     int64_t C_inv, int64_t H, int64_t W, int64_t p, int64_t frame0, int64_t Kp,
                     void* out, int x_dtype, int out_dtype, void* stream);

/* Head layout of SwinTransformer.forward_head (models/swin.py:293-299) for
 * one frame: y [B*(H/p)*(W/p), p*p*C_out] (in_dtype), row (b, i, j), column
 * (u*p + v)*C_out + c -> out[b*out_bstride + (c*H + i*p + u)*W + j*p + v]
 * (out_dtype).  Requires p | H, p | W, p <= 16, p*p*C_out a multiple of 8
 * (bf16) / 4 (f32), 16-byte aligned y. */
int nsw_unpatchify(const void* y, void* out, int64_t B, int64_t C_out, int64_t H, int64_t W,
                   int64_t p, int64_t out_bstride, int in_dtype, int out_dtype, void* stream);

/* The head GEMM with the head layout fused into its write-out: replaces
 * nsw_linear (no bias) followed by nsw_unpatchify in
 * SwinTransformer.forward_head (models/swin.py:286-299, the Linear E ->
 * C_out*p*p of :201-209, then the reshape + einsum).  x [B*(H/p)*(W/p), K]
 * (dtype) holds the tokens (row (b, i, j)); w_perm [C_out*p*p, K] is the
 * head weight with its rows permuted from the reference's (u*p + v)*C_out + c
 * to c*p*p + u*p + v; pixel (c, i*p + u, j*p + v) of frame b goes to
 * out[b*out_bstride + (c*H + i*p + u)*W + j*p + v] in out_dtype (dtype, or
 * float32 for a bf16 GEMM: the bf16-rounded values widened, as nsw_linear +
 * nsw_unpatchify give).  Requires p in {1, 2, 4, 8, 16}, p | H, p | W,
 * K a multiple of 32 (bf16) / 16 (f32), out_bstride >= C_out*H*W and a
 * multiple of p, out aligned to min(16, p * element size) bytes, x and
 * w_perm 16-byte aligned. */
int nsw_head_unpatchify(const void* x, const void* w_perm, void* out, int64_t B, int64_t C_out, int64_t H,
                        int64_t W, int64_t p, int64_t K, int64_t out_bstride, int dtype, int out_dtype,
                        void* stream);

/* SwinTransformer's big skip (use_big_skip_conv, models/swin.py:212-223 and
 * :310-319): skip_conv = Conv2d(C_in -> C_out, 1x1, no bias) of the input,
 * added to the head's image, of which the model returns the last frame.
 * In place on that frame: out[b*out_bstride + co*H*W + q] +=
 * sum_ci w[co*C_in + ci] * xin[b, ci, q], xin = frame (T - 1 + frame0) mod T
 * of x [B, T, C_x, H, W] (x_dtype) followed by the C_inv invariant planes
 * inv [C_inv, H, W] (same dtype), C_in = C_x + C_inv.  w is float32
 * [C_out, C_in].  The input values and the convolution are rounded to
 * model_dtype (the reference's conv runs on the model-dtype input and
 * returns that dtype, then the two model-dtype images are added), the sum to
 * out_dtype.  Requires H*W a multiple of 4, C_out*C_in <= 16384, out_bstride
 * >= C_out*H*W and a multiple of 4, x / inv / out aligned to 4 elements. */
int nsw_skip_conv_accumulate(const void* x, const void* inv, const float* w, void* out, int64_t B, int64_t T,
                             int64_t C_x, int64_t C_inv, int64_t C_out, int64_t H, int64_t W, int64_t frame0,
                             int64_t out_bstride, int x_dtype, int model_dtype, int out_dtype, void* stream);

/* HBM stream probe.  No counterpart in the reference: a measurement helper
 * for callers that report kernel rates against what the device sustains
 * (bench.py's achievable peaks).  dst == NULL: reads `bytes` from src with
 * 16-byte loads, four per lane in flight (their bits are folded into a
 * checksum that touches nothing outside the library); otherwise copies
 * `bytes` from src to dst.  bytes a multiple of 16, src / dst 16-byte
 * aligned; blocks = 0 picks 16384 workgroups of 256 threads. */
int nsw_hbm_stream(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSW_H_ */
