// Row-permutation kernels (roll, window partition / reverse, the fused
// norm1 + roll + partition gather) and RMSNorm, plus the shift-mask builder.
//
// All of them move whole C-contiguous rows: one wavefront per output row,
// 16-byte vector loads/stores (8 bf16 or 4 f32 per lane), so every row is read
// and written as full 64-byte-aligned segments.  HBM-bound: 2*C*sizeof(T)
// bytes per row.
#include "nsw_common.h"

namespace nsw {

enum RowMap { MAP_IDENTITY = 0, MAP_PARTITION = 1, MAP_REVERSE = 2, MAP_ROLL = 3 };

// Source row of output row m for each map.
template <int MAP>
__device__ __forceinline__ int64_t src_row(int64_t m, const WinGeom& g) {
  if constexpr (MAP == MAP_IDENTITY) {
    return m;
  } else if constexpr (MAP == MAP_PARTITION) {
    return g.token_of_row(m);          // window-ordered row <- token (roll by -s folded in)
  } else if constexpr (MAP == MAP_REVERSE) {
    return g.row_of_token(m);          // token <- window-ordered row (roll by +s folded in)
  } else {
    // torch.roll by (s0, s1): y[h, w] = x[(h - s0) mod H, (w - s1) mod W]
    const uint32_t mu = (uint32_t)m;
    const uint32_t bt = g.dHW.div(mu);
    const uint32_t hw = mu - bt * (uint32_t)g.H * (uint32_t)g.W;
    const uint32_t h = g.dW.div(hw), w = hw - h * (uint32_t)g.W;
    int hs = (int)h - g.s0; if (hs < 0) hs += g.H;
    int wsr = (int)w - g.s1; if (wsr < 0) wsr += g.W;
    return (int64_t)((bt * (uint32_t)g.H + (uint32_t)hs) * (uint32_t)g.W + (uint32_t)wsr);
  }
}

// RPW rows per wave; CH = number of 16-byte chunks per lane (C <= 64*CH*VEC).
// A wave issues the loads of all its rows (and the norm weight, shared by
// them) before any arithmetic, so that RPW * CH 16-byte loads per lane are in
// flight; the row sums of squares are reduced with DPP and permlane swaps.
template <typename T, int MAP, bool NORM, int CH, int RPW>
__global__ __launch_bounds__(256) void row_map_kernel(const T* __restrict__ x,
                                                      const T* __restrict__ w, float eps,
                                                      T* __restrict__ y, int64_t rows, int C,
                                                      WinGeom g) {
  constexpr int VEC = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t m0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (m0 >= rows) return;
  float wv[NORM ? CH : 1][VEC];
  if constexpr (NORM) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int c0 = (lane + 64 * k) * VEC;
      if (c0 < C) load16<T>(w + c0, wv[k]);
    }
  }
  float v[RPW][CH][VEC];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t m = m0 + r < rows ? m0 + r : rows - 1;   // a tail row re-reads the last row (not stored)
    const T* xr = x + src_row<MAP>(m, g) * C;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int c0 = (lane + 64 * k) * VEC;
      if (c0 < C) load16<T>(xr + c0, v[r][k]);
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t m = m0 + r;
    float rs = 1.f;
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int c0 = (lane + 64 * k) * VEC;
        if (c0 < C) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) ss += v[r][k][e] * v[r][k][e];
        }
      }
      ss = rows4_sum(row16_sum(ss));
      rs = 1.0f / sqrtf(ss / (float)C + eps);
    }
    if (m < rows) {
      T* yr = y + m * C;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int c0 = (lane + 64 * k) * VEC;
        if (c0 < C) {
          if constexpr (NORM) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[r][k][e] = (v[r][k][e] * rs) * wv[k][e];
          }
          store16<T>(yr + c0, v[r][k]);
        }
      }
    }
  }
}

// Window partition (the roll by -shift folded in) that also writes the
// rows' partial sums of squares, one float per 512 bytes of row (the layout
// the row-scaled GEMMs read): in chunk iteration k, lanes 0-31 and 32-63
// cover parts 2k and 2k+1 (32 lanes x 16 B), summed as the GEMM epilogues
// sum theirs (FMA chain per lane, DPP row sums, even row first).
template <typename T, int CH>
__global__ __launch_bounds__(256) void partition_sumsq_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                              float* __restrict__ ss, int nparts, int64_t rows,
                                                              int C, WinGeom g) {
  constexpr int VEC = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;   // whole waves: the DPP sums below see every lane
  const T* xr = x + g.token_of_row(m) * C;
  T* yr = y + m * C;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c0 = (lane + 64 * k) * VEC;
    float part = 0.f;
    if (c0 < C) {
      float v[VEC];
      load16<T>(xr + c0, v);
      store16<T>(yr + c0, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) part = fmaf(v[e], v[e], part);
    }
    float lo = row16_sum(part), hi = lo;
    permlane16_swap(lo, hi);
    const int p = 2 * k + (lane >> 5);
    if ((lane & 31) == 0 && p < nparts) ss[m * nparts + p] = lo + hi;
  }
}

template <typename T, int MAP, bool NORM>
static int launch_row_map(const void* x, const void* w, float eps, void* y, int64_t rows,
                          int64_t C, const WinGeom& g, hipStream_t st, const char* what) {
  constexpr int VEC = Vec16<T>::N;
  NSW_CHECK_ARG(C > 0 && C % VEC == 0, "%s: C=%lld must be a positive multiple of %d", what,
                (long long)C, VEC);
  NSW_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0 &&
                    (!NORM || ((uintptr_t)w % 16) == 0),
                "%s: pointers must be 16-byte aligned", what);
  if (rows == 0) return NSW_OK;
  const int64_t per_lane = (C / VEC + 63) / 64;
  const T* xp = (const T*)x;
  const T* wp = (const T*)w;
  T* yp = (T*)y;
  // rows of one chunk per lane (up to 1 KB: C <= 512 in bf16) go two to a
  // wave (config 4's gather: 95.3 -> 89.9 us standalone); longer rows one
  // to a wave (two were slower at C = 1024: 42.4 against 39.9 us)
  auto grid = [&](int rpw) { return dim3((unsigned)((rows + 4 * rpw - 1) / (4 * rpw))); };
  const dim3 block(256);
  if (per_lane <= 1)
    hipLaunchKernelGGL((row_map_kernel<T, MAP, NORM, 1, 2>), grid(2), block, 0, st, xp, wp, eps, yp, rows, (int)C, g);
  else if (per_lane <= 2)
    hipLaunchKernelGGL((row_map_kernel<T, MAP, NORM, 2, 1>), grid(1), block, 0, st, xp, wp, eps, yp, rows, (int)C, g);
  else if (per_lane <= 4)
    hipLaunchKernelGGL((row_map_kernel<T, MAP, NORM, 4, 1>), grid(1), block, 0, st, xp, wp, eps, yp, rows, (int)C, g);
  else if (per_lane <= 8)
    hipLaunchKernelGGL((row_map_kernel<T, MAP, NORM, 8, 1>), grid(1), block, 0, st, xp, wp, eps, yp, rows, (int)C, g);
  else if (per_lane <= 16)
    hipLaunchKernelGGL((row_map_kernel<T, MAP, NORM, 16, 1>), grid(1), block, 0, st, xp, wp, eps, yp, rows, (int)C, g);
  else
    return set_error(NSW_ERR_UNSUPPORTED, "%s: C=%lld too large (max %d)", what, (long long)C, 64 * 16 * VEC);
  return check_launch(what);
}

template <int MAP, bool NORM>
static int dispatch_row_map(int dtype, const void* x, const void* w, float eps, void* y,
                            int64_t rows, int64_t C, const WinGeom& g, void* stream,
                            const char* what) {
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSW_DTYPE_BF16) return launch_row_map<bf16, MAP, NORM>(x, w, eps, y, rows, C, g, st, what);
  if (dtype == NSW_DTYPE_F32) return launch_row_map<float, MAP, NORM>(x, w, eps, y, rows, C, g, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
}

int check_geom(int64_t B, int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1, const char* what) {
  NSW_CHECK_ARG(B > 0 && T > 0 && H > 0 && W > 0 && ws0 > 0 && ws1 > 0,
                "%s: all of B,T,H,W,ws0,ws1 must be positive", what);
  NSW_CHECK_ARG(H % ws0 == 0 && W % ws1 == 0, "%s: H=%lld, W=%lld not divisible by window (%lld,%lld)",
                what, (long long)H, (long long)W, (long long)ws0, (long long)ws1);
  NSW_CHECK_ARG(B * T * H * W < ((int64_t)1 << 31), "%s: B*T*H*W=%lld tokens, at most 2^31 - 1", what,
                (long long)(B * T * H * W));
  return NSW_OK;
}

// Additive shift mask [nW, L, L] (closed form of Block._make_attention_mask).
__global__ void make_mask_kernel(float* __restrict__ mask, WinGeom g, int64_t total) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t LL = (int64_t)g.L * g.L;
  const int wi = (int)(idx / LL);
  const int pq = (int)(idx - (int64_t)wi * LL);
  const int p = pq / g.L, q = pq - p * g.L;
  float v = 0.f;
  if ((g.s0 != 0 || g.s1 != 0) && wi / g.nwb == g.nhb - 1) {
    const int rp = (p % g.wa) / g.ws1, rq = (q % g.wa) / g.ws1;
    const int thr = g.ws0 - g.s0;
    if ((rp >= thr) != (rq >= thr)) v = -100.0f;
  }
  mask[idx] = v;
}

}  // namespace nsw

using namespace nsw;

// Host check of FastDiv (the divisions of the row maps) against the '/'
// operator: every divisor 1..4096 plus large ones, at the numerators where an
// off-by-one would show (multiples of d and their neighbours, powers of two,
// the 32-bit extremes) and a pseudo-random sweep.  Returns the failure count.
extern "C" int nsw_selftest_fastdiv(void) {
  int fails = 0;
  auto check = [&](uint32_t d, uint32_t n) {
    const FastDiv f = FastDiv::make(d);
    if (f.div(n) != n / d) ++fails;
  };
  uint64_t state = 0x9E3779B97F4A7C15ull;
  auto next = [&]() {
    state ^= state << 13; state ^= state >> 7; state ^= state << 17;
    return (uint32_t)(state >> 16);
  };
  uint32_t divisors[4096 + 8];
  int nd = 0;
  for (uint32_t d = 1; d <= 4096; ++d) divisors[nd++] = d;
  const uint32_t big[] = {64800u, 259200u, 1036800u, 65535u, 65537u, 2147483647u, 2147483648u, 4294967295u};
  for (uint32_t d : big) divisors[nd++] = d;
  for (int a = 0; a < nd; ++a) {
    const uint32_t d = divisors[a];
    const uint32_t fixed[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0x7FFFFFFFu, 0x80000000u,
                              0xFFFFFFFFu, 0xFFFFFFFEu};
    for (uint32_t n : fixed) check(d, n);
    for (int e = 0; e < 32; ++e) { check(d, 1u << e); check(d, (1u << e) - 1); }
    const uint64_t kmax = 0xFFFFFFFFull / d;
    for (int s = 0; s < 64; ++s) {
      const uint64_t k = (uint64_t)next() % (kmax + 1);
      const uint64_t n = k * d;
      check(d, (uint32_t)n);
      if (n > 0) check(d, (uint32_t)(n - 1));
      if (n + 1 <= 0xFFFFFFFFull) check(d, (uint32_t)(n + 1));
      check(d, next());
    }
  }
  return fails;
}

extern "C" int nsw_roll_hw(const void* x, void* y, int64_t B, int64_t T, int64_t H, int64_t W,
                           int64_t C, int64_t s0, int64_t s1, int dtype, void* stream) {
  int rc = check_geom(B, T, H, W, 1, 1, "nsw_roll_hw");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, 1, 1, (int)(s0 % H), (int)(s1 % W));
  return dispatch_row_map<MAP_ROLL, false>(dtype, x, nullptr, 0.f, y, B * T * H * W, C, g, stream, "nsw_roll_hw");
}

extern "C" int nsw_window_partition(const void* x, void* windows, int64_t B, int64_t T, int64_t H,
                                    int64_t W, int64_t C, int64_t ws0, int64_t ws1, int dtype,
                                    void* stream) {
  int rc = check_geom(B, T, H, W, ws0, ws1, "nsw_window_partition");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, 0, 0);
  return dispatch_row_map<MAP_PARTITION, false>(dtype, x, nullptr, 0.f, windows, B * T * H * W, C, g,
                                                stream, "nsw_window_partition");
}

extern "C" int nsw_window_reverse(const void* windows, void* x, int64_t B, int64_t T, int64_t H,
                                  int64_t W, int64_t C, int64_t ws0, int64_t ws1, int dtype,
                                  void* stream) {
  int rc = check_geom(B, T, H, W, ws0, ws1, "nsw_window_reverse");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, 0, 0);
  return dispatch_row_map<MAP_REVERSE, false>(dtype, windows, nullptr, 0.f, x, B * T * H * W, C, g,
                                              stream, "nsw_window_reverse");
}

extern "C" int nsw_roll_window_partition(const void* x, void* windows, int64_t B, int64_t T,
                                         int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1,
                                         int64_t s0, int64_t s1, int dtype, void* stream) {
  int rc = check_geom(B, T, H, W, ws0, ws1, "nsw_roll_window_partition");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  return dispatch_row_map<MAP_PARTITION, false>(dtype, x, nullptr, 0.f, windows, B * T * H * W, C, g,
                                                stream, "nsw_roll_window_partition");
}

extern "C" int nsw_window_reverse_roll(const void* windows, void* x, int64_t B, int64_t T, int64_t H,
                                       int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                                       int64_t s1, int dtype, void* stream) {
  int rc = check_geom(B, T, H, W, ws0, ws1, "nsw_window_reverse_roll");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  return dispatch_row_map<MAP_REVERSE, false>(dtype, windows, nullptr, 0.f, x, B * T * H * W, C, g,
                                              stream, "nsw_window_reverse_roll");
}

extern "C" int nsw_rmsnorm(const void* x, const void* w, float eps, void* y, int64_t rows,
                           int64_t C, int dtype, void* stream) {
  NSW_CHECK_ARG(rows >= 0, "nsw_rmsnorm: rows < 0");
  WinGeom g = WinGeom::make(1, 1, 1, 1, 1, 1, 0, 0);
  return dispatch_row_map<MAP_IDENTITY, true>(dtype, x, w, eps, y, rows, C, g, stream, "nsw_rmsnorm");
}

extern "C" int nsw_rmsnorm_roll_partition(const void* x, const void* w, float eps, void* xw,
                                          int64_t B, int64_t T, int64_t H, int64_t W, int64_t C,
                                          int64_t ws0, int64_t ws1, int64_t s0, int64_t s1,
                                          int dtype, void* stream) {
  int rc = check_geom(B, T, H, W, ws0, ws1, "nsw_rmsnorm_roll_partition");
  if (rc) return rc;
  WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  return dispatch_row_map<MAP_PARTITION, true>(dtype, x, w, eps, xw, B * T * H * W, C, g, stream,
                                               "nsw_rmsnorm_roll_partition");
}

namespace nsw {
int64_t sumsq_parts(int64_t C, int dtype);

template <typename T>
static int launch_partition_sumsq(const void* x, void* xw, float* ss, int64_t rows, int64_t C, int nparts,
                                  const WinGeom& g, hipStream_t st, const char* what) {
  constexpr int VEC = Vec16<T>::N;
  NSW_CHECK_ARG(C > 0 && C % VEC == 0, "%s: C=%lld must be a positive multiple of %d", what, (long long)C, VEC);
  NSW_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)xw % 16) == 0 && ((uintptr_t)ss % 4) == 0,
                "%s: pointers must be 16-byte (row_sumsq 4-byte) aligned", what);
  if (rows == 0) return NSW_OK;
  const int64_t per_lane = (C / VEC + 63) / 64;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  const T* xp = (const T*)x;
  T* yp = (T*)xw;
  if (per_lane <= 1)
    hipLaunchKernelGGL((partition_sumsq_kernel<T, 1>), grid, block, 0, st, xp, yp, ss, nparts, rows, (int)C, g);
  else if (per_lane <= 2)
    hipLaunchKernelGGL((partition_sumsq_kernel<T, 2>), grid, block, 0, st, xp, yp, ss, nparts, rows, (int)C, g);
  else if (per_lane <= 4)
    hipLaunchKernelGGL((partition_sumsq_kernel<T, 4>), grid, block, 0, st, xp, yp, ss, nparts, rows, (int)C, g);
  else if (per_lane <= 8)
    hipLaunchKernelGGL((partition_sumsq_kernel<T, 8>), grid, block, 0, st, xp, yp, ss, nparts, rows, (int)C, g);
  else
    return set_error(NSW_ERR_UNSUPPORTED, "%s: C=%lld too large", what, (long long)C);
  return check_launch(what);
}

}  // namespace nsw

extern "C" int nsw_window_partition_sumsq(const void* x, void* xw, float* row_sumsq, int64_t B, int64_t T,
                                          int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                                          int64_t s1, int dtype, void* stream) {
  const char* what = "nsw_window_partition_sumsq";
  int rc = check_geom(B, T, H, W, ws0, ws1, what);
  if (rc) return rc;
  NSW_CHECK_ARG(x && xw && row_sumsq && x != (const void*)xw, "%s: x, xw, row_sumsq required, x != xw", what);
  const WinGeom g = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  const int64_t rows = B * T * H * W;
  const int nparts = (int)sumsq_parts(C, dtype);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSW_DTYPE_BF16) return launch_partition_sumsq<bf16>(x, xw, row_sumsq, rows, C, nparts, g, st, what);
  if (dtype == NSW_DTYPE_F32) return launch_partition_sumsq<float>(x, xw, row_sumsq, rows, C, nparts, g, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
}

extern "C" int nsw_make_attention_mask(float* mask, int64_t H, int64_t W, int64_t ws0, int64_t ws1,
                                       int64_t s0, int64_t s1, int64_t T, void* stream) {
  int rc = check_geom(1, T, H, W, ws0, ws1, "nsw_make_attention_mask");
  if (rc) return rc;
  NSW_CHECK_ARG(s0 >= 0 && s0 < ws0 && s1 >= 0 && s1 < ws1,
                "nsw_make_attention_mask: shift must lie in [0, window)");
  WinGeom g = WinGeom::make(1, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)s0, (int)s1);
  const int64_t total = (int64_t)g.nW * g.L * g.L;
  if (total == 0) return NSW_OK;
  hipLaunchKernelGGL(make_mask_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, mask, g, total);
  return check_launch("nsw_make_attention_mask");
}

// ------------------------------------------------------------- LayerNorm ----
// nn.LayerNorm over the last dim (NormLayer with norm_type="layer_norm",
// models/layer_helpers.py:94-100,118-119): y = (x - mean) / sqrt(var + eps)
// * w + b with the biased variance, w / b optional (elementwise_affine).
// One wave per row, the row held in registers: mean first, then the
// variance of the centred values (two passes over registers, one over HBM).
namespace nsw {

template <typename T, int CH>
__global__ __launch_bounds__(256) void layernorm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                        const T* __restrict__ b, float eps,
                                                        T* __restrict__ y, int64_t rows, int C) {
  constexpr int VEC = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  const T* xr = x + m * C;
  T* yr = y + m * C;
  float v[CH][VEC];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c0 = (lane + 64 * k) * VEC;
    if (c0 < C) {
      load16<T>(xr + c0, v[k]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += v[k][e];
    }
  }
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c0 = (lane + 64 * k) * VEC;
    if (c0 < C) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        v[k][e] -= mean;
        q += v[k][e] * v[k][e];
      }
    }
  }
  const float rs = 1.0f / sqrtf(wave_sum(q) / (float)C + eps);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c0 = (lane + 64 * k) * VEC;
    if (c0 < C) {
      float wv[VEC], bv[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) { wv[e] = 1.f; bv[e] = 0.f; }
      if (w != nullptr) load16<T>(w + c0, wv);
      if (b != nullptr) load16<T>(b + c0, bv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[k][e] = (v[k][e] * rs) * wv[e] + bv[e];
      store16<T>(yr + c0, v[k]);
    }
  }
}

template <typename T>
static int launch_layernorm(const void* x, const void* w, const void* b, float eps, void* y, int64_t rows,
                            int64_t C, hipStream_t st) {
  const char* what = "nsw_layernorm";
  constexpr int VEC = Vec16<T>::N;
  NSW_CHECK_ARG(rows >= 0, "%s: rows < 0", what);
  NSW_CHECK_ARG(C > 0 && C % VEC == 0, "%s: C=%lld must be a positive multiple of %d", what, (long long)C, VEC);
  NSW_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0 && ((uintptr_t)w % 16) == 0 &&
                    ((uintptr_t)b % 16) == 0,
                "%s: pointers must be 16-byte aligned", what);
  if (rows == 0) return NSW_OK;
  const int64_t per_lane = (C / VEC + 63) / 64;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)b;
  T* yp = (T*)y;
  if (per_lane <= 1) hipLaunchKernelGGL((layernorm_kernel<T, 1>), grid, block, 0, st, xp, wp, bp, eps, yp, rows, (int)C);
  else if (per_lane <= 2) hipLaunchKernelGGL((layernorm_kernel<T, 2>), grid, block, 0, st, xp, wp, bp, eps, yp, rows, (int)C);
  else if (per_lane <= 4) hipLaunchKernelGGL((layernorm_kernel<T, 4>), grid, block, 0, st, xp, wp, bp, eps, yp, rows, (int)C);
  else if (per_lane <= 8) hipLaunchKernelGGL((layernorm_kernel<T, 8>), grid, block, 0, st, xp, wp, bp, eps, yp, rows, (int)C);
  else if (per_lane <= 16) hipLaunchKernelGGL((layernorm_kernel<T, 16>), grid, block, 0, st, xp, wp, bp, eps, yp, rows, (int)C);
  else return set_error(NSW_ERR_UNSUPPORTED, "%s: C=%lld too large (max %d)", what, (long long)C, 64 * 16 * VEC);
  return check_launch(what);
}

}  // namespace nsw

extern "C" int nsw_layernorm(const void* x, const void* w, const void* b, float eps, void* y, int64_t rows,
                             int64_t C, int dtype, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSW_DTYPE_BF16) return nsw::launch_layernorm<nsw::bf16>(x, w, b, eps, y, rows, C, st);
  if (dtype == NSW_DTYPE_F32) return nsw::launch_layernorm<float>(x, w, b, eps, y, rows, C, st);
  return nsw::set_error(NSW_ERR_INVALID, "nsw_layernorm: unknown dtype %d", dtype);
}
