// Latitude-weighted RMSE / ACC reduction (WeightedRMSE.forward,
// utils/losses.py:243-266, plus the textbook weighted ACC).
//
// One pass over pred and target: each workgroup reduces a band of rows of one
// (b, t, c) plane into four float64 sums, in the dtypes the reference ends up
// with (fp32 difference and square, float64 area weights -> float64 product
// and sum).  A second tiny kernel adds the bands of each plane in a fixed
// order (deterministic; no atomics) and finishes rmse / acc.  HBM-bound:
// 8 bytes read per grid point.
#include "nsw_common.h"

namespace nsw {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// FULLW: weights are a [H, W] map instead of one value per latitude row.
template <bool VEC4, bool ACC, bool FULLW>
__global__ __launch_bounds__(256) void wsum_partial_kernel(const float* __restrict__ pred,
                                                           const float* __restrict__ tgt,
                                                           const double* __restrict__ wlat,
                                                           const float* __restrict__ clim, int H,
                                                           int W, int Cch, int rpc, int nchunk,
                                                           double* __restrict__ partial) {
  const int64_t plane = blockIdx.x / nchunk;
  const int ch = blockIdx.x - (int)(plane * nchunk);
  const int h0 = ch * rpc;
  const int h1 = min(H, h0 + rpc);
  const float cl = ACC ? clim[plane % Cch] : 0.f;
  const float* pp = pred + plane * (int64_t)H * W;
  const float* tp = tgt + plane * (int64_t)H * W;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  auto acc1 = [&](float p, float t, double w) {
    const float d = p - t;
    const float d2 = d * d;
    s0 += w * (double)d2;
    if constexpr (ACC) {
      const double af = (double)(p - cl), ao = (double)(t - cl);
      s1 += w * af * ao;
      s2 += w * af * af;
      s3 += w * ao * ao;
    }
  };
  if constexpr (VEC4) {
    const int wq = W >> 2;
    const int64_t n = (int64_t)(h1 - h0) * wq;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
      const int hr = (int)(i / wq);
      const int x4 = (int)(i - (int64_t)hr * wq);
      const int h = h0 + hr;
      const int64_t off = (int64_t)h * W + 4 * x4;
      const f32x4 p = *reinterpret_cast<const f32x4*>(pp + off);
      const f32x4 t = *reinterpret_cast<const f32x4*>(tp + off);
      if constexpr (FULLW) {
        acc1(p[0], t[0], wlat[off]); acc1(p[1], t[1], wlat[off + 1]);
        acc1(p[2], t[2], wlat[off + 2]); acc1(p[3], t[3], wlat[off + 3]);
      } else {
        const double w = wlat[h];
        acc1(p[0], t[0], w); acc1(p[1], t[1], w); acc1(p[2], t[2], w); acc1(p[3], t[3], w);
      }
    }
  } else {
    const int64_t n = (int64_t)(h1 - h0) * W;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
      const int hr = (int)(i / W);
      const int h = h0 + hr;
      const int64_t off = (int64_t)h * W + (i - (int64_t)hr * W);
      acc1(pp[off], tp[off], FULLW ? wlat[off] : wlat[h]);
    }
  }
  __shared__ double red[4][4];
  s0 = wave_sum_d(s0);
  if constexpr (ACC) { s1 = wave_sum_d(s1); s2 = wave_sum_d(s2); s3 = wave_sum_d(s3); }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { red[wave][0] = s0; red[wave][1] = s1; red[wave][2] = s2; red[wave][3] = s3; }
  __syncthreads();
  if (threadIdx.x < 4) {
    const int k = threadIdx.x;
    partial[(plane * nchunk + ch) * 4 + k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
  }
}

__global__ void wsum_final_kernel(const double* __restrict__ partial, int64_t P, int nchunk,
                                  double hw, bool has_acc, double* __restrict__ rmse,
                                  double* __restrict__ acc) {
  const int64_t plane = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (plane >= P) return;
  double s[4] = {0.0, 0.0, 0.0, 0.0};
  for (int c = 0; c < nchunk; ++c)
    for (int k = 0; k < 4; ++k) s[k] += partial[(plane * nchunk + c) * 4 + k];
  rmse[plane] = sqrt(s[0] / hw);
  if (has_acc) acc[plane] = s[1] / sqrt(s[2] * s[3]);
}

static void metrics_chunks(int64_t P, int64_t H, int* rpc, int* nchunk) {
  int64_t want = (2048 + P - 1) / P;
  if (want < 1) want = 1;
  if (want > H) want = H;
  int64_t r = (H + want - 1) / want;
  *rpc = (int)r;
  *nchunk = (int)((H + r - 1) / r);
}

}  // namespace nsw

using namespace nsw;

extern "C" size_t nsw_weighted_metrics_workspace_size(int64_t P, int64_t H, int64_t W) {
  (void)W;
  if (P <= 0 || H <= 0) return 0;
  int rpc, nchunk;
  metrics_chunks(P, H, &rpc, &nchunk);
  return (size_t)P * nchunk * 4 * sizeof(double);
}

template <bool FULLW>
static void launch_partial(bool vec4, bool acc, dim3 grid, hipStream_t st, const float* pred,
                           const float* target, const double* w, const float* clim, int H, int W,
                           int Cch, int rpc, int nchunk, double* partial) {
  dim3 block(256);
  if (vec4 && acc)
    hipLaunchKernelGGL((wsum_partial_kernel<true, true, FULLW>), grid, block, 0, st, pred, target, w, clim, H, W, Cch, rpc, nchunk, partial);
  else if (vec4)
    hipLaunchKernelGGL((wsum_partial_kernel<true, false, FULLW>), grid, block, 0, st, pred, target, w, clim, H, W, Cch, rpc, nchunk, partial);
  else if (acc)
    hipLaunchKernelGGL((wsum_partial_kernel<false, true, FULLW>), grid, block, 0, st, pred, target, w, clim, H, W, Cch, rpc, nchunk, partial);
  else
    hipLaunchKernelGGL((wsum_partial_kernel<false, false, FULLW>), grid, block, 0, st, pred, target, w, clim, H, W, Cch, rpc, nchunk, partial);
}

extern "C" int nsw_weighted_metrics(const float* pred, const float* target, const double* w,
                                    int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                    int64_t Cch, double* rmse, double* acc, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  const char* what = "nsw_weighted_metrics";
  NSW_CHECK_ARG(P > 0 && H > 0 && W > 0 && Cch > 0, "%s: P, H, W, Cch must be positive", what);
  NSW_CHECK_ARG(w_cols == 1 || w_cols == W, "%s: weights must be [H] / [H,1] or [H,W]", what);
  NSW_CHECK_ARG(P % Cch == 0, "%s: P=%lld is not a multiple of Cch=%lld", what, (long long)P, (long long)Cch);
  NSW_CHECK_ARG(H * W < (1LL << 31), "%s: plane too large", what);
  NSW_CHECK_ARG(rmse != nullptr && (clim == nullptr || acc != nullptr), "%s: missing output", what);
  const size_t need = nsw_weighted_metrics_workspace_size(P, H, W);
  NSW_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "%s: workspace of %zu bytes needed", what, need);
  int rpc, nchunk;
  metrics_chunks(P, H, &rpc, &nchunk);
  NSW_CHECK_ARG(P * nchunk < (1LL << 31), "%s: too many planes", what);
  hipStream_t st = (hipStream_t)stream;
  double* partial = (double*)workspace;
  const bool vec4 = (W % 4 == 0) && ((uintptr_t)pred % 16 == 0) && ((uintptr_t)target % 16 == 0);
  dim3 grid((unsigned)(P * nchunk));
  if (w_cols == 1 || W == 1)
    launch_partial<false>(vec4, clim != nullptr, grid, st, pred, target, w, clim, (int)H, (int)W, (int)Cch, rpc, nchunk, partial);
  else
    launch_partial<true>(vec4, clim != nullptr, grid, st, pred, target, w, clim, (int)H, (int)W, (int)Cch, rpc, nchunk, partial);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(wsum_final_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, st, partial, P,
                     nchunk, (double)(H * W), clim != nullptr, rmse, acc);
  return check_launch(what);
}
