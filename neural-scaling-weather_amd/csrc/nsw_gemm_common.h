// Helpers of the MFMA GEMM kernel (nsw_gemm.hip): epilogue / operand-fusion
// identifiers, the epilogue argument block, the GELU forms and the LDS row
// swizzle of the operand stages.
#pragma once

#include "nsw_common.h"

namespace nsw {

enum Epi {
  EPI_NONE = NSW_EPI_NONE,
  EPI_BIAS = NSW_EPI_BIAS,
  EPI_BIAS_GELU = NSW_EPI_BIAS_GELU,
  EPI_BIAS_RESIDUAL = NSW_EPI_BIAS_RESIDUAL,
  EPI_BIAS_GELU_TANH = NSW_EPI_BIAS_GELU_TANH,
  EPI_WINDOW_RESIDUAL = 10,  // bias, + residual[m], stored at row_of_token(m) (token -> window order), + row sums
  EPI_SCATTER_RESIDUAL = 11, // bias, row m -> token_of_row(m), + skip[token]
  EPI_REMAP_RESIDUAL = 12,   // bias, + residual[m], stored at row_of_row_shift(m), + row sums of squares
  EPI_RES_SUMSQ = 13,        // bias, + residual[m], stored at row m, + row sums of squares
  EPI_TOKEN_RESIDUAL = 14,   // bias, + residual[m], stored at token_of_row(m)
  EPI_UNPATCH = 15,          // no bias; row m (a token) and column c p^2 + dy p + dx go to
                             // pixel (dy, dx) of the token's patch in image plane c
  EPI_QKV_HN16 = 16,         // bias, then per-head RMSNorm of the q and k
  EPI_QKV_HN32 = 32,         // columns, for head dims 16 / 32 / 64
  EPI_QKV_HN64 = 64,
  EPI_QKV_HN4 = 68,          // the same for head dims 4 and 8: a head inside
  EPI_QKV_HN8 = 72           // one 16-column block (4 / 8 of its columns)
};

// Operand-side fusion (template parameter PRE):
//   PRE_NONE     y = epi(x . w^T)
//   PRE_ROWSCALE y = epi(rs . (x . w^T)) with rs[m] = 1/sqrt(sum_p P[m,p] / K + eps)
//                from per-row partial sums of squares P [M, nparts] written by
//                the producer of x (the proj scatter / remap epilogues): the
//                RMSNorm of the rows of x with its weight folded into w
//                (w[n,k] = W[n,k] * norm_w[k], prepared by the caller), at
//                one read per row instead of a pass over x.
enum Pre { PRE_NONE = 0, PRE_ROWSCALE = 3 };

constexpr int qkv_head_dim(int epi) {
  return (epi == EPI_QKV_HN16 || epi == EPI_QKV_HN32 || epi == EPI_QKV_HN64) ? epi
         : epi == EPI_QKV_HN4 ? 4 : epi == EPI_QKV_HN8 ? 8 : 0;
}

struct EpiArgs {
  const void* bias;
  const void* residual;
  const void* qn_w;
  const void* kn_w;
  float eps;
  int C;       // q/k/v width for the QKV epilogues
  WinGeom geom;  // EPI_SCATTER_RESIDUAL
  // [rows, nparts] row sums of squares: output of EPI_SCATTER_RESIDUAL
  // (optional), EPI_REMAP_RESIDUAL and EPI_RES_SUMSQ; input of PRE_ROWSCALE
  float* row_sumsq;
  int nparts;
  int dh, dw;   // EPI_REMAP_RESIDUAL: shift differences of geom.row_of_row_shift
  int group_m;  // row blocks per XCD tile group (0: GROUP_M)
  // EPI_UNPATCH: image [B, 1, img_C, img_H, img_W], frames img_bstride
  // elements apart, in float (img_f32) or the GEMM's dtype; patch img_p
  void* img;
  int64_t img_bstride;
  int img_C, img_H, img_W, img_p, img_f32;
};

// GELU with the exact-erf form of nn.GELU(): 0.5 v (1 + erf(v / sqrt 2)).
// erfc from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7):
//   erfc(x) = (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-x^2),
//   t = 1 / (1 + p x), x >= 0.
// With x = |v| / sqrt 2: 1 + erf(v / sqrt 2) is 2 - erfc(x) for v >= 0 and
// erfc(x) for v < 0, so GELU(v) = max(v, 0) - |v| erfc(x) / 2 for both signs
// (no select, no cancellation).  Constants folded: u = |v| sqrt(log2(e) / 2)
// gives exp(-x^2) = exp2(-u^2) and p x = (p / (sqrt(log2(e)/2) sqrt 2)) u;
// the polynomial coefficients carry the factor -1/2.  13 VALU instructions,
// two of them transcendental (v_exp_f32, v_rcp_f32).
__device__ __forceinline__ float gelu_erf(float v) {
  const float a = fabsf(v);
  const float u = a * 0.84932180028801907f;
  const float e = __builtin_amdgcn_exp2f(-(u * u));
  const float t = __builtin_amdgcn_rcpf(fmaf(0.27273748087922252f, u, 1.0f));
  float h = fmaf(-0.5307027145f, t, 0.7265760135f);
  h = fmaf(h, t, -0.7107068705f);
  h = fmaf(h, t, 0.142248368f);
  h = fmaf(h, t, -0.127414796f);
  h *= t;                                   // -erfc(x) / 2
  return fmaf(h * e, a, fmaxf(v, 0.0f));
}

// Exact-erf GELU for bfloat16 outputs: GELU(v) = max(v, 0) - |v| Phi(-|v|)
// with Phi(-a) = exp2(P(a)), P a degree-5 least-squares fit of log2 Phi(-a)
// on [0, 5.5] (csrc/gelu_fit.py, which prints the coefficients and the
// error).  Worst error on a dense grid of [-12, 12] against float64: 0.145
// of the bfloat16 half-ulp of the exact value (|GELU| >= 2^-24; about 0.13
// throughout v < 1, below 0.02 for v > 1); P keeps decreasing past 5.5, so
// the tail only shrinks.  8 VALU instructions, one transcendental
// (v_exp_f32), against 13 and two for gelu_erf, which stays the form for
// fp32 outputs.
__device__ __forceinline__ float gelu_erf_bf16(float v) {
  const float a = fabsf(v);
  float p = fmaf(-2.297039027e-04f, a, 4.821910989e-03f);
  p = fmaf(p, a, -4.437467828e-02f);
  p = fmaf(p, a, -4.701045752e-01f);
  p = fmaf(p, a, -1.145988584e+00f);
  p = fmaf(p, a, -1.000384808e+00f);
  return fmaf(-a, __builtin_amdgcn_exp2f(p), fmaxf(v, 0.0f));
}

// GELU with the tanh form (nn.GELU(approximate="tanh"), the "gelu" of the
// reference's Transformer-Engine block): 0.5 v (1 + tanh(u)),
// u = sqrt(2/pi) (v + 0.044715 v^3).  As 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)):
// GELU(v) = v / (1 + exp2(v (c1 + c3 v^2))) with c1 = -2 sqrt(2/pi) log2(e),
// c3 = 0.044715 c1.  Saturates cleanly: exp2 -> inf gives 0, exp2 -> 0 gives v.
__device__ __forceinline__ float gelu_tanh(float v) {
  const float z = v * v;
  const float a = v * fmaf(-0.10294324f, z, -2.3022082f);
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a));
}

// Row blocks per tile group of one XCD (tiles come from xcd_remap).
constexpr int GROUP_M = 8;

// Chunk swizzle of a 128-byte stage row (8 chunks of 16 bytes).
__device__ __forceinline__ int row_swizzle(int row) {
  const int r = row & 15;   // position inside the 16-row block
  return ((r >> 1) & 7) ^ ((r & 1) << 2);
}

}  // namespace nsw
