// Whole Block.forward (models/swin_helpers.py:435-459) as one C-ABI call:
//
//   K1  xw  = rmsnorm(x; norm1) gathered to window order with the roll by -shift
//   K2  qkv = xw . [Wq;Wk;Wv]^T + b, per-head RMSNorm of q and k   (MFMA GEMM)
//   K3  o   = window attention(qkv) with the shift mask from indices
//   K4  h1  = scatter_to_tokens(o . Wproj^T + bproj) + x           (MFMA GEMM)
//   K5  hn  = rmsnorm(h1; norm2)
//   K6  u   = gelu(hn . W1^T + b1)  (erf form, or the tanh form)   (MFMA GEMM)
//   K7  y   = u . W2^T + b2 + h1                                   (MFMA GEMM)
//
// With the norm-folded weight w1_n2 = W1 * norm2 (per input column), K5
// disappears: K4 also writes partial sums of squares of the h1 rows it
// stores (S, [M, nparts]) and
//
//   K6' u   = gelu(rs2 . (h1 . w1_n2^T) + b1),  rs2 = 1/sqrt(sum(S row) / C + eps)
//
// (6 launches, the default of nsw.Block).  With wqkv_n1 = Wqkv * norm1 as
// well, the block runs as a one-block window-order chain (below).
//
// Workspace: A [M*C] holds xw, then o, then hn; Q [M*max(3C, Hm)] holds qkv,
// then u; H1 [M*C] holds h1 (dtype elements); S [M*nparts] float.
// M = B*T*H*W tokens.
#include "nsw_common.h"

namespace nsw {
int gemm_qkv(const void* x, const void* wqkv, const void* bqkv, const void* qn_w, const void* kn_w,
             float eps, void* qkv, int64_t M, int64_t C, int64_t num_heads, int dtype, void* stream);
int gemm_proj_scatter(const void* o, const void* wproj, const void* bproj, const void* skip, void* y,
                      int64_t B, int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1,
                      int64_t s0, int64_t s1, int dtype, void* stream, float* row_sumsq);
int gemm_linear_rowscale(const void* x, const void* w_n, const void* bias, const void* residual, void* y,
                         const float* row_sumsq, int64_t nparts, int64_t M, int64_t N, int64_t K, int epilogue,
                         float eps, int dtype, void* stream);
int64_t sumsq_parts(int64_t C, int dtype);
int gemm_qkv_rowscale(const void* x, const void* wqkv_n, const void* bqkv, const void* qn_w, const void* kn_w,
                      float eps, void* qkv, const float* row_sumsq, int64_t nparts, int64_t M, int64_t C,
                      int64_t num_heads, int dtype, void* stream);
int gemm_linear_remap(const void* x, const void* w, const void* bias, const void* residual, void* y,
                      float* row_sumsq, int64_t M, int64_t N, int64_t K, int map_mode, int64_t B, int64_t T,
                      int64_t H, int64_t W, int64_t ws0, int64_t ws1, int64_t s0, int64_t s1, int64_t sa,
                      int64_t sb, int dtype, void* stream);

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct BlockLayout {
  size_t a, q, h1, ss, total;
};

static BlockLayout block_layout(const nsw_block_shape* s) {
  BlockLayout l{};
  const size_t es = dtype_size(s->dtype);
  const size_t M = (size_t)(s->B * s->T * s->H * s->W);
  const size_t C = (size_t)s->C;
  const size_t wq = (size_t)(3 * s->C > s->hidden ? 3 * s->C : s->hidden);
  l.a = 0;
  l.q = align256(M * C * es);
  l.h1 = l.q + align256(M * wq * es);
  l.ss = l.h1 + align256(M * C * es);
  l.total = l.ss + align256(M * (size_t)sumsq_parts(s->C, s->dtype) * sizeof(float));
  return l;
}
}  // namespace nsw

using namespace nsw;

namespace nsw {
static size_t chain_workspace(const nsw_block_shape* s);
}

extern "C" size_t nsw_block_workspace_size(const nsw_block_shape* s) {
  if (!s || s->B <= 0 || s->T <= 0 || s->H <= 0 || s->W <= 0 || s->C <= 0 || s->hidden <= 0) return 0;
  // the larger of the two forms (the one-block window-order chain runs when
  // both norm-folded weights are given)
  const size_t a = block_layout(s).total, b = chain_workspace(s);
  return a > b ? a : b;
}

extern "C" int nsw_swin_block_forward(const void* x, void* y, const nsw_block_params* p,
                                      const nsw_block_shape* s, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  const char* what = "nsw_swin_block_forward";
  NSW_CHECK_ARG(p && s && x && y, "%s: null argument", what);
  NSW_CHECK_ARG(x != (const void*)y, "%s: x and y must not alias", what);
  NSW_CHECK_ARG(s->num_heads > 0 && s->C % s->num_heads == 0, "%s: C not divisible by num_heads", what);
  NSW_CHECK_ARG(s->hidden > 0, "%s: hidden must be positive", what);
  const size_t need = nsw_block_workspace_size(s);
  NSW_CHECK_ARG(workspace && workspace_bytes >= need, "%s: workspace of %zu bytes needed", what, need);
  const BlockLayout lay = block_layout(s);
  char* ws = (char*)workspace;
  void* A = ws + lay.a;
  void* Q = ws + lay.q;
  void* H1 = ws + lay.h1;
  const int64_t M = s->B * s->T * s->H * s->W;
  const int64_t C = s->C;
  const int64_t L = s->T * s->ws0 * s->ws1;
  const int64_t hd = C / s->num_heads;
  float* S = (float*)(ws + lay.ss);
  const int64_t nparts = sumsq_parts(C, s->dtype);
  NSW_CHECK_ARG(s->gelu_tanh == 0 || s->gelu_tanh == 1, "%s: gelu_tanh must be 0 or 1", what);
  const int gelu_epi = s->gelu_tanh ? NSW_EPI_BIAS_GELU_TANH : NSW_EPI_BIAS_GELU;
  int rc;
  if (p->wqkv_n1 && p->w1_n2) {
    // both norms folded: the one-block window-order chain (h1 stays in
    // window order, fc2 scatters to tokens)
    return nsw_swin_blocks_forward(x, y, p, s, 1, workspace, workspace_bytes, stream);
  }
  NSW_CHECK_ARG(!p->wqkv_n1, "%s: wqkv_n1 (norm1 folded) needs w1_n2 as well (the one-block window-order chain)",
                what);
  // K1
  rc = nsw_rmsnorm_roll_partition(x, p->norm1_w, s->eps, A, s->B, s->T, s->H, s->W, C, s->ws0, s->ws1, s->s0,
                                  s->s1, s->dtype, stream);
  if (rc) return rc;
  // K2
  rc = gemm_qkv(A, p->wqkv, p->bqkv, p->qn_w, p->kn_w, s->eps, Q, M, C, s->num_heads, s->dtype, stream);
  if (rc) return rc;
  // K3 (o overwrites xw in A)
  rc = nsw_window_attention(Q, A, nullptr, 0, M / L, L, C, s->num_heads, 1.0f / sqrtf((float)hd), s->H,
                            s->W, s->ws0, s->ws1, s->s0, s->s1, s->T, s->dtype, stream);
  if (rc) return rc;
  // K4 (+ the row partial sums of squares of h1 when norm2 is folded)
  rc = gemm_proj_scatter(A, p->wproj, p->bproj, x, H1, s->B, s->T, s->H, s->W, C, s->ws0, s->ws1, s->s0,
                         s->s1, s->dtype, stream, p->w1_n2 ? S : nullptr);
  if (rc) return rc;
  if (p->w1_n2) {
    // K6' (u overwrites qkv in Q)
    rc = gemm_linear_rowscale(H1, p->w1_n2, p->b1, nullptr, Q, S, nparts, M, s->hidden, C, gelu_epi,
                              s->eps, s->dtype, stream);
    if (rc) return rc;
  } else {
    // K5 (hn overwrites o in A)
    rc = nsw_rmsnorm(H1, p->norm2_w, s->eps, A, M, C, s->dtype, stream);
    if (rc) return rc;
    // K6 (u overwrites qkv in Q)
    rc = nsw_linear(A, p->w1, p->b1, nullptr, Q, M, s->hidden, C, gelu_epi, s->dtype, stream);
    if (rc) return rc;
  }
  // K7
  rc = nsw_linear(Q, p->w2, p->b2, H1, y, M, C, s->hidden, NSW_EPI_BIAS_RESIDUAL, s->dtype, stream);
  return rc;
}

// ---------------------------------------------------------------------------
// The blocks loop of SwinTransformer.forward (models/swin.py:305-309:
// `for blk in self.blocks: x = blk(x)`) with the residual stream kept in
// window order from block to block, so that no block gathers or scatters
// whole rows on its own:
//
//   G   xw  = partition(x) in block 0's window order, S1 = its rows' partial
//             sums of squares                                  (row kernel)
//   for block i (rows in block i's window order):
//   K2  qkv = headnorm(rs(S1) . (xw . wqkv_n1^T) + b)           (MFMA GEMM)
//   K3  o   = window attention(qkv)
//   K4  h1  = xw + o . Wproj^T + bproj, S2 = h1's partial sums   (MFMA GEMM)
//   K6  u   = gelu(rs(S2) . (h1 . w1_n2^T) + b1)                 (MFMA GEMM)
//   K7  y   = h1 + u . W2^T + b2, each row stored at the same token's row of
//             block i+1's window order with S1 for block i+1, or at its
//             token (token order) after the last block          (MFMA GEMM)
//
// rs(S) = 1/sqrt(sum of the row's partials / C + eps): the RMSNorms norm1
// and norm2 as row scales of GEMMs whose weights carry the norm weights
// (wqkv_n1 = Wqkv * norm1, w1_n2 = W1 * norm2 per input column).  1 + 5 *
// depth launches.  Workspace: two window-order row buffers (ping-pong), qkv
// / u, o, h1 and the two sums-of-squares arrays.
namespace nsw {
struct ChainLayout {
  size_t xa, xb, q, o, h1, s1, s2, total;
};

static ChainLayout chain_layout(const nsw_block_shape* s) {
  ChainLayout l{};
  const size_t es = dtype_size(s->dtype);
  const size_t M = (size_t)(s->B * s->T * s->H * s->W);
  const size_t C = (size_t)s->C;
  const size_t wq = (size_t)(3 * s->C > s->hidden ? 3 * s->C : s->hidden);
  const size_t ss = align256(M * (size_t)sumsq_parts(s->C, s->dtype) * sizeof(float));
  l.xa = 0;
  l.xb = l.xa + align256(M * C * es);
  l.q = l.xb + align256(M * C * es);
  l.o = l.q + align256(M * wq * es);
  l.h1 = l.o + align256(M * C * es);
  l.s1 = l.h1 + align256(M * C * es);
  l.s2 = l.s1 + ss;
  l.total = l.s2 + ss;
  return l;
}

static size_t chain_workspace(const nsw_block_shape* s) { return chain_layout(s).total; }

static bool same_stack(const nsw_block_shape* a, const nsw_block_shape* b) {
  return a->B == b->B && a->T == b->T && a->H == b->H && a->W == b->W && a->C == b->C &&
         a->num_heads == b->num_heads && a->ws0 == b->ws0 && a->ws1 == b->ws1 && a->hidden == b->hidden &&
         a->dtype == b->dtype;
}
}  // namespace nsw

extern "C" size_t nsw_blocks_workspace_size(const nsw_block_shape* shapes, int64_t depth) {
  if (!shapes || depth <= 0) return 0;
  const nsw_block_shape* s = shapes;
  if (s->B <= 0 || s->T <= 0 || s->H <= 0 || s->W <= 0 || s->C <= 0 || s->hidden <= 0) return 0;
  return chain_layout(s).total;
}

// The chain from token-ordered x (partitioned here into block 0's window
// order with its norm1 row sums), or from x0w / s0w already in that form
// (read only: block 0 takes its rows and sums from there, later blocks from
// the workspace).
static int blocks_chain(const void* x, const void* x0w, const float* s0w, void* y, const nsw_block_params* params,
                        const nsw_block_shape* shapes, int64_t depth, void* workspace, size_t workspace_bytes,
                        void* stream, const char* what) {
  const void* in = x ? x : x0w;
  NSW_CHECK_ARG(in && y && params && shapes && depth > 0, "%s: null argument or depth <= 0", what);
  NSW_CHECK_ARG(in != (const void*)y, "%s: x and y must not alias", what);
  NSW_CHECK_ARG(x != nullptr || s0w != nullptr, "%s: the window-ordered input needs its row sums", what);
  const nsw_block_shape* s0 = shapes;
  NSW_CHECK_ARG(s0->num_heads > 0 && s0->C % s0->num_heads == 0 && s0->hidden > 0,
                "%s: C not divisible by num_heads, or hidden <= 0", what);
  for (int64_t i = 0; i < depth; ++i) {
    NSW_CHECK_ARG(same_stack(s0, shapes + i), "%s: block %lld differs from block 0 in shape or dtype", what,
                  (long long)i);
    NSW_CHECK_ARG(params[i].wqkv_n1 && params[i].w1_n2,
                  "%s: block %lld needs the norm-folded weights wqkv_n1 and w1_n2", what, (long long)i);
    NSW_CHECK_ARG(shapes[i].gelu_tanh == 0 || shapes[i].gelu_tanh == 1, "%s: gelu_tanh must be 0 or 1", what);
  }
  const size_t need = nsw_blocks_workspace_size(shapes, depth);
  NSW_CHECK_ARG(workspace && workspace_bytes >= need, "%s: workspace of %zu bytes needed", what, need);
  const ChainLayout lay = chain_layout(s0);
  char* ws = (char*)workspace;
  void* X[2] = {ws + lay.xa, ws + lay.xb};
  void* Q = ws + lay.q;
  void* O = ws + lay.o;
  void* H1 = ws + lay.h1;
  float* S1 = (float*)(ws + lay.s1);
  float* S2 = (float*)(ws + lay.s2);
  const int64_t B = s0->B, T = s0->T, H = s0->H, W = s0->W, C = s0->C;
  const int64_t M = B * T * H * W;
  const int64_t L = T * s0->ws0 * s0->ws1;
  const int64_t hd = C / s0->num_heads;
  const int dt = s0->dtype;
  const int64_t nparts = sumsq_parts(C, dt);
  int rc = NSW_OK;
  if (x) {
    rc = nsw_window_partition_sumsq(x, X[0], S1, B, T, H, W, C, s0->ws0, s0->ws1, shapes[0].s0, shapes[0].s1, dt,
                                    stream);
    if (rc) return rc;
  }
  for (int64_t i = 0; i < depth; ++i) {
    const nsw_block_shape* s = shapes + i;
    const nsw_block_params* p = params + i;
    void* xw = i == 0 && !x ? const_cast<void*>(x0w) : X[i & 1];
    const float* s1 = i == 0 && !x ? s0w : S1;
    const bool last = i + 1 == depth;
    // K2
    rc = gemm_qkv_rowscale(xw, p->wqkv_n1, p->bqkv, p->qn_w, p->kn_w, s->eps, Q, s1, nparts, M, C, s->num_heads,
                           dt, stream);
    if (rc) return rc;
    // K3
    rc = nsw_window_attention(Q, O, nullptr, 0, M / L, L, C, s->num_heads, 1.0f / sqrtf((float)hd), H, W,
                              s->ws0, s->ws1, s->s0, s->s1, T, dt, stream);
    if (rc) return rc;
    // K4
    rc = gemm_linear_remap(O, p->wproj, p->bproj, xw, H1, S2, M, C, C, 0, B, T, H, W, s->ws0, s->ws1, s->s0,
                           s->s1, 0, 0, dt, stream);
    if (rc) return rc;
    // K6
    rc = gemm_linear_rowscale(H1, p->w1_n2, p->b1, nullptr, Q, S2, nparts, M, s->hidden, C,
                              s->gelu_tanh ? NSW_EPI_BIAS_GELU_TANH : NSW_EPI_BIAS_GELU, s->eps, dt, stream);
    if (rc) return rc;
    // K7
    if (last) {
      rc = gemm_linear_remap(Q, p->w2, p->b2, H1, y, nullptr, M, C, s->hidden, 1, B, T, H, W, s->ws0, s->ws1,
                             s->s0, s->s1, 0, 0, dt, stream);
    } else {
      const nsw_block_shape* sn = shapes + i + 1;
      rc = gemm_linear_remap(Q, p->w2, p->b2, H1, X[(i + 1) & 1], S1, M, C, s->hidden, 2, B, T, H, W, s->ws0,
                             s->ws1, s->s0, s->s1, sn->s0, sn->s1, dt, stream);
    }
    if (rc) return rc;
  }
  return NSW_OK;
}

extern "C" int nsw_swin_blocks_forward(const void* x, void* y, const nsw_block_params* params,
                                       const nsw_block_shape* shapes, int64_t depth, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  if (!x) return set_error(NSW_ERR_INVALID, "nsw_swin_blocks_forward: x is null");
  return blocks_chain(x, nullptr, nullptr, y, params, shapes, depth, workspace, workspace_bytes, stream,
                      "nsw_swin_blocks_forward");
}

extern "C" int nsw_swin_blocks_forward_windowed(const void* xw, const float* row_sumsq, void* y,
                                                const nsw_block_params* params, const nsw_block_shape* shapes,
                                                int64_t depth, void* workspace, size_t workspace_bytes,
                                                void* stream) {
  if (!xw || !row_sumsq) return set_error(NSW_ERR_INVALID, "nsw_swin_blocks_forward_windowed: null input");
  NSW_CHECK_ARG(((uintptr_t)row_sumsq % 16) == 0, "%s: row_sumsq must be 16-byte aligned",
                "nsw_swin_blocks_forward_windowed");
  return blocks_chain(nullptr, xw, row_sumsq, y, params, shapes, depth, workspace, workspace_bytes, stream,
                      "nsw_swin_blocks_forward_windowed");
}
