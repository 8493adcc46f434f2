// Latitude-weighted RMSE / ACC reduction (WeightedRMSE.forward,
// utils/losses.py:243-266, plus the textbook weighted ACC).
//
// One pass over pred and target: each workgroup reduces a band of rows of one
// (b, t, c) plane into four float64 sums, in the dtypes the reference ends up
// with (fp32 difference and square, float64 area weights -> float64 product
// and sum).  A second tiny kernel adds the bands of each plane in a fixed
// order (deterministic; no atomics) and finishes rmse / acc.  HBM-bound:
// 8 bytes read per grid point.
#include <mutex>

#include "nsw_common.h"

namespace nsw {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// FULLW: weights are a [H, W] map instead of one value per latitude row.
// TP: prediction dtype (float, or bf16 for a model's raw output).
// AFFINE: both fields are first unnormalised per channel, x * std + mean,
// rounded after the product and after the sum as the reference's two
// separate tensor ops do (utils/inferencer.py:390-391,408-409).
// TS: dtype of std / mean and of the unnormalised fields.  float64 statistics
// (torch.as_tensor of float64 .h5 stats, utils/dataloaders/era5hdf5.py:111-122)
// promote the reference's unnormalised fields, their difference and its
// square to float64, so the whole per-point chain then runs in TS.
template <typename TP, typename TS, bool VEC4, bool ACC, bool FULLW, bool AFFINE>
__global__ __launch_bounds__(256) void wsum_partial_kernel(const TP* __restrict__ pred,
                                                           const float* __restrict__ tgt,
                                                           const double* __restrict__ wlat,
                                                           const float* __restrict__ clim,
                                                           const TS* __restrict__ std_c,
                                                           const TS* __restrict__ mean_c, int H,
                                                           int W, int Cch, int rpc, int nchunk, FastDiv dwq,
                                                           double* __restrict__ partial) {
  const int64_t plane = blockIdx.x / nchunk;
  const int ch = blockIdx.x - (int)(plane * nchunk);
  const int h0 = ch * rpc;
  const int h1 = min(H, h0 + rpc);
  const int cidx = (int)(plane % Cch);
  const TS cl = ACC ? (TS)clim[cidx] : (TS)0;
  const TS sc = AFFINE ? std_c[cidx] : (TS)1;
  const TS of = AFFINE ? mean_c[cidx] : (TS)0;
  const TP* pp = pred + plane * (int64_t)H * W;
  const float* tp = tgt + plane * (int64_t)H * W;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  auto acc1 = [&](float pf, float tf, double w) {
    TS p = (TS)pf, t = (TS)tf;
    if constexpr (AFFINE) {
      // two roundings, never an FMA (the device default contracts a*b+c)
#pragma clang fp contract(off)
      p = p * sc + of;
      t = t * sc + of;
    }
    const TS d = p - t;
    const TS d2 = d * d;
    s0 += w * (double)d2;
    if constexpr (ACC) {
      const double af = (double)(p - cl), ao = (double)(t - cl);
      s1 += w * af * ao;
      s2 += w * af * af;
      s3 += w * ao * ao;
    }
  };
  if constexpr (VEC4 && !FULLW) {
    // One latitude row per wave at a time (rows h0 + wave, + 4, ...): the
    // row's weight is wave-uniform, and the four sums are accumulated per
    // lane without it in float64 and scaled by it once per row.  Each lane
    // keeps U 16-byte vectors of each field in flight (W <= 64 U 4 in one
    // pass).
    constexpr int U = 6;
    const int wq = W >> 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int h = h0 + wave; h < h1; h += 4) {
      const TP* pr = pp + (int64_t)h * W;
      const float* tr = tp + (int64_t)h * W;
      double r0 = 0.0, r1 = 0.0, r2 = 0.0, r3 = 0.0;
      for (int f0 = 0; f0 < wq; f0 += 64 * U) {
        float p[U][4];
        f32x4 t[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int f = f0 + u * 64 + lane;
          if (f < wq) {
            // non-temporal: both fields are read once (580 MB at config 5,
            // twice the last-level cache): 108 -> 95 us per call
            if constexpr (sizeof(TP) == 4) {
              const f32x4 pv = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pr + 4 * f));
              p[u][0] = pv[0]; p[u][1] = pv[1]; p[u][2] = pv[2]; p[u][3] = pv[3];
            } else {
              const bf16x4 pv = __builtin_nontemporal_load(reinterpret_cast<const bf16x4*>(pr + 4 * f));
              p[u][0] = (float)pv[0]; p[u][1] = (float)pv[1]; p[u][2] = (float)pv[2]; p[u][3] = (float)pv[3];
            }
            t[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(tr + 4 * f));
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int f = f0 + u * 64 + lane;
          if (f < wq) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              TS pv = (TS)p[u][e], tv = (TS)t[u][e];
              if constexpr (AFFINE) {
#pragma clang fp contract(off)
                pv = pv * sc + of;
                tv = tv * sc + of;
              }
              const TS d = pv - tv;
              const TS d2 = d * d;
              r0 += (double)d2;
              if constexpr (ACC) {
                const double af = (double)(pv - cl), ao = (double)(tv - cl);
                r1 = fma(af, ao, r1);
                r2 = fma(af, af, r2);
                r3 = fma(ao, ao, r3);
              }
            }
          }
        }
      }
      const double w = wlat[h];
      s0 = fma(w, r0, s0);
      if constexpr (ACC) {
        s1 = fma(w, r1, s1);
        s2 = fma(w, r2, s2);
        s3 = fma(w, r3, s3);
      }
    }
  } else if constexpr (VEC4) {
    // The band's rows are contiguous in the plane: n4 vectors of 4 from row
    // h0 on.  Each thread keeps U vector loads of each field in flight (the
    // loads of a group are issued before its arithmetic); the row of vector
    // f is f / (W/4) by multiply-shift.
    constexpr int U = 4;
    const int wq = W >> 2;
    const uint32_t n4 = (uint32_t)(h1 - h0) * (uint32_t)wq;
    const TP* pb = pp + (int64_t)h0 * W;
    const float* tb = tp + (int64_t)h0 * W;
    auto consume = [&](uint32_t f, const float (&p)[4], const f32x4& t) {
      const int hr = (int)dwq.div(f);
      const int h = h0 + hr;
      if constexpr (FULLW) {
        const int64_t off = (int64_t)h * W + 4 * (int)(f - (uint32_t)hr * (uint32_t)wq);
        acc1(p[0], t[0], wlat[off]); acc1(p[1], t[1], wlat[off + 1]);
        acc1(p[2], t[2], wlat[off + 2]); acc1(p[3], t[3], wlat[off + 3]);
      } else {
        const double w = wlat[h];
        acc1(p[0], t[0], w); acc1(p[1], t[1], w); acc1(p[2], t[2], w); acc1(p[3], t[3], w);
      }
    };
    uint32_t i = threadIdx.x;
    for (; i + (U - 1) * 256 < n4; i += U * 256) {
      float p[U][4];
      f32x4 t[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        load4<TP>(pb + 4 * (int64_t)(i + u * 256), p[u]);
        t[u] = *reinterpret_cast<const f32x4*>(tb + 4 * (int64_t)(i + u * 256));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) consume(i + u * 256, p[u], t[u]);
    }
    for (; i < n4; i += 256) {
      float p[4];
      load4<TP>(pb + 4 * (int64_t)i, p);
      const f32x4 t = *reinterpret_cast<const f32x4*>(tb + 4 * (int64_t)i);
      consume(i, p, t);
    }
  } else {
    const int64_t n = (int64_t)(h1 - h0) * W;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
      const int hr = (int)(i / W);
      const int h = h0 + hr;
      const int64_t off = (int64_t)h * W + (i - (int64_t)hr * W);
      acc1(to_f32(pp[off]), tp[off], FULLW ? wlat[off] : wlat[h]);
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

template <typename TP, typename TS, bool FULLW, bool AFFINE>
static void launch_partial(bool vec4, bool acc, dim3 grid, hipStream_t st, const TP* pred,
                           const float* target, const double* w, const float* clim, const TS* sc,
                           const TS* of, int H, int W, int Cch, int rpc, int nchunk, double* partial) {
  dim3 block(256);
  const FastDiv dwq = FastDiv::make((uint32_t)(W >= 4 ? W / 4 : 1));
#define NSW_PARTIAL(V4, AC)                                                                                 \
  hipLaunchKernelGGL((wsum_partial_kernel<TP, TS, V4, AC, FULLW, AFFINE>), grid, block, 0, st, pred, target, \
                     w, clim, sc, of, H, W, Cch, rpc, nchunk, dwq, partial)
  if (vec4 && acc) NSW_PARTIAL(true, true);
  else if (vec4) NSW_PARTIAL(true, false);
  else if (acc) NSW_PARTIAL(false, true);
  else NSW_PARTIAL(false, false);
#undef NSW_PARTIAL
}

template <typename TP, typename TS, bool AFFINE>
static int run_metrics(const TP* pred, const float* target, const double* w, int64_t w_cols,
                       const float* clim, const TS* sc, const TS* of, int64_t P, int64_t H,
                       int64_t W, int64_t Cch, double* rmse, double* acc, void* workspace,
                       size_t workspace_bytes, hipStream_t st, const char* what) {
  NSW_CHECK_ARG(P > 0 && H > 0 && W > 0 && Cch > 0, "%s: P, H, W, Cch must be positive", what);
  NSW_CHECK_ARG(w_cols == 1 || w_cols == W, "%s: weights must be [H] / [H,1] or [H,W]", what);
  NSW_CHECK_ARG(P % Cch == 0, "%s: P=%lld is not a multiple of Cch=%lld", what, (long long)P, (long long)Cch);
  NSW_CHECK_ARG(H * W < (1LL << 31), "%s: plane too large", what);
  NSW_CHECK_ARG(rmse != nullptr && (clim == nullptr || acc != nullptr), "%s: missing output", what);
  NSW_CHECK_ARG(!AFFINE || (sc != nullptr && of != nullptr), "%s: std and mean are required", what);
  const size_t need = nsw_weighted_metrics_workspace_size(P, H, W);
  NSW_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "%s: workspace of %zu bytes needed", what, need);
  int rpc, nchunk;
  metrics_chunks(P, H, &rpc, &nchunk);
  NSW_CHECK_ARG(P * nchunk < (1LL << 31), "%s: too many planes", what);
  double* partial = (double*)workspace;
  const bool vec4 = (W % 4 == 0) && ((uintptr_t)pred % (4 * sizeof(TP)) == 0) && ((uintptr_t)target % 16 == 0);
  dim3 grid((unsigned)(P * nchunk));
  if (w_cols == 1 || W == 1)
    launch_partial<TP, TS, false, AFFINE>(vec4, clim != nullptr, grid, st, pred, target, w, clim, sc, of, (int)H,
                                      (int)W, (int)Cch, rpc, nchunk, partial);
  else
    launch_partial<TP, TS, true, AFFINE>(vec4, clim != nullptr, grid, st, pred, target, w, clim, sc, of, (int)H,
                                     (int)W, (int)Cch, rpc, nchunk, partial);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(wsum_final_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, st, partial, P,
                     nchunk, (double)(H * W), clim != nullptr, rmse, acc);
  return check_launch(what);
}

extern "C" int nsw_weighted_metrics(const float* pred, const float* target, const double* w,
                                    int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                    int64_t Cch, double* rmse, double* acc, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return run_metrics<float, float, false>(pred, target, w, w_cols, clim, nullptr, nullptr, P, H, W, Cch, rmse, acc,
                                   workspace, workspace_bytes, (hipStream_t)stream, "nsw_weighted_metrics");
}

extern "C" int nsw_weighted_metrics_unnorm(const void* pred, int pred_dtype, const float* target,
                                           const float* std_c, const float* mean_c, const double* w,
                                           int64_t w_cols, const float* clim, int64_t P, int64_t H, int64_t W,
                                           int64_t Cch, double* rmse, double* acc, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  const char* what = "nsw_weighted_metrics_unnorm";
  hipStream_t st = (hipStream_t)stream;
  if (pred_dtype == NSW_DTYPE_F32)
    return run_metrics<float, float, true>((const float*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                           Cch, rmse, acc, workspace, workspace_bytes, st, what);
  if (pred_dtype == NSW_DTYPE_BF16)
    return run_metrics<bf16, float, true>((const bf16*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                          Cch, rmse, acc, workspace, workspace_bytes, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, pred_dtype);
}

extern "C" int nsw_weighted_metrics_unnorm_f64stats(const void* pred, int pred_dtype, const float* target,
                                                    const double* std_c, const double* mean_c, const double* w,
                                                    int64_t w_cols, const float* clim, int64_t P, int64_t H,
                                                    int64_t W, int64_t Cch, double* rmse, double* acc,
                                                    void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "nsw_weighted_metrics_unnorm_f64stats";
  hipStream_t st = (hipStream_t)stream;
  if (pred_dtype == NSW_DTYPE_F32)
    return run_metrics<float, double, true>((const float*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                            Cch, rmse, acc, workspace, workspace_bytes, st, what);
  if (pred_dtype == NSW_DTYPE_BF16)
    return run_metrics<bf16, double, true>((const bf16*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                           Cch, rmse, acc, workspace, workspace_bytes, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, pred_dtype);
}

// ------------------------------------------------ allocation-free variant ----
// nsw_weighted_metrics_unnorm_noalloc keeps its per-(plane, band) partial sums
// in `scratch`, a device global of NSW_METRICS_SCRATCH_BYTES: each GPU the
// library runs on holds one copy until the process ends.  In host code the
// name `scratch` is only a handle; the device address of a GPU's copy comes
// from hipGetSymbolAddress with that GPU current, looked up on the first call
// on each device and kept per device.  Nothing in it has to start at zero
// (every partial the final kernel reads is written by the partial kernel of
// the same call), and it keeps the last call's contents.  Calls that overlap
// on one GPU (different streams, or other host threads) share the array and
// race; calls in stream order do not.
namespace nsw {

static __device__ __align__(256) double scratch[NSW_METRICS_SCRATCH_BYTES / sizeof(double)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_address(hipStream_t st, void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(NSW_ERR_HIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  if (st != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return set_error(NSW_ERR_HIP, "%s: hipStreamGetDevice: %s", what, hipGetErrorString(e));
    NSW_CHECK_ARG((int)sdev == dev, "%s: the stream belongs to device %d, the current device is %d", what,
                  (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(NSW_ERR_UNSUPPORTED, "%s: device %d beyond the %d supported", what, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(NSW_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NSW_OK;
}

}  // namespace nsw

extern "C" int nsw_weighted_metrics_unnorm_noalloc(const void* pred, int pred_dtype, const float* target,
                                                   const float* std_c, const float* mean_c, const double* w,
                                                   int64_t w_cols, const float* clim, int64_t P, int64_t H,
                                                   int64_t W, int64_t Cch, double* rmse, double* acc,
                                                   void* stream) {
  const char* what = "nsw_weighted_metrics_unnorm_noalloc";
  NSW_CHECK_ARG(P > 0 && H > 0 && W > 0, "%s: P, H, W must be positive", what);
  const size_t need = nsw_weighted_metrics_workspace_size(P, H, W);
  NSW_CHECK_ARG(need <= (size_t)NSW_METRICS_SCRATCH_BYTES,
                "%s: %lld planes of %lld rows need %zu bytes of partial sums, more than the %d-byte scratch", what,
                (long long)P, (long long)H, need, (int)NSW_METRICS_SCRATCH_BYTES);
  hipStream_t st = (hipStream_t)stream;
  void* ptr = nullptr;
  int rc = scratch_address(st, &ptr, what);
  if (rc) return rc;
  if (pred_dtype == NSW_DTYPE_F32)
    return run_metrics<float, float, true>((const float*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                           Cch, rmse, acc, ptr, NSW_METRICS_SCRATCH_BYTES, st, what);
  if (pred_dtype == NSW_DTYPE_BF16)
    return run_metrics<bf16, float, true>((const bf16*)pred, target, w, w_cols, clim, std_c, mean_c, P, H, W,
                                          Cch, rmse, acc, ptr, NSW_METRICS_SCRATCH_BYTES, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, pred_dtype);
}

// ------------------------------------------------------ HBM stream probe ----
// nsw_hbm_stream: a grid-stride pass over `bytes` with four 16-byte loads per
// lane in flight (the loads of a group are issued before any use), read-only
// or copying; the read-only form keeps its loads by folding them into an
// xor of their bits, stored into a device global only when it equals one
// particular value (harmless either way: the global is the probe's own).
namespace nsw {

__device__ uint32_t nsw_hbm_probe_sink;   // external linkage: its stores stay

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ p, int64_t n) {
  constexpr int U = 4;
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * 256 * U;
  for (int64_t i = (int64_t)blockIdx.x * 256 * U + threadIdx.x; i < n; i += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + u * 256;
      v[u] = j < n ? p[j] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  const uint32_t s = (acc[0] ^ acc[1]) ^ (acc[2] ^ acc[3]);
  if (s == 0x9e3779b9u) nsw_hbm_probe_sink = s;
}

__global__ __launch_bounds__(256) void hbm_copy_kernel(const f32x4* __restrict__ p, f32x4* __restrict__ q,
                                                       int64_t n) {
  constexpr int U = 4;
  const int64_t stride = (int64_t)gridDim.x * 256 * U;
  for (int64_t i = (int64_t)blockIdx.x * 256 * U + threadIdx.x; i < n; i += stride) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + u * 256;
      if (j < n) v[u] = p[j];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + u * 256;
      if (j < n) q[j] = v[u];
    }
  }
}

}  // namespace nsw

extern "C" int nsw_hbm_stream(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream) {
  const char* what = "nsw_hbm_stream";
  NSW_CHECK_ARG(src != nullptr && bytes > 0 && bytes % 16 == 0, "%s: src and a positive multiple of 16 bytes", what);
  NSW_CHECK_ARG(((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0, "%s: 16-byte aligned pointers", what);
  NSW_CHECK_ARG(blocks >= 0 && blocks < (1LL << 31), "%s: blocks out of range", what);
  const unsigned nb = blocks > 0 ? (unsigned)blocks : 16384u;
  hipStream_t st = (hipStream_t)stream;
  if (dst == nullptr)
    hipLaunchKernelGGL(hbm_read_kernel, dim3(nb), dim3(256), 0, st, (const u32x4*)src, bytes / 16);
  else
    hipLaunchKernelGGL(hbm_copy_kernel, dim3(nb), dim3(256), 0, st, (const f32x4*)src, (f32x4*)dst, bytes / 16);
  return check_launch(what);
}
