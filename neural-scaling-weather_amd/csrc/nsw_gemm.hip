// MFMA GEMM y[M,N] = epilogue(x[M,K] . w[N,K]^T) for gfx950, with the Swin
// block's epilogues fused in.
//
// Tiling (both dtypes): 256 threads = 4 wavefronts, block tile 256 (m) x 128
// (n), k tile = 128 bytes per row (64 bf16 / 32 f32), LDS double buffered
// (2 x 384 rows x 144 B = 108 KB; the 16-byte row pad makes the 16-lane
// ds_read_b128 phases conflict-free).  Each wave owns a 128 (m) x 64 (n)
// sub-tile = 8 x 4 blocks of 16x16 fp32 accumulators.
//
// The MFMA is issued "transposed": the A operand is the weight fragment
// (rows n) and the B operand the activation fragment (rows m), so lane l of a
// 16x16 result block holds y[m = l%16][n = 4*(l/16) + r], r = 0..3: four
// consecutive output columns, written as one 8-byte (bf16) / 16-byte (f32)
// store, and a row's head-norm reduction needs only two cross-lane shuffles.
//
//   bf16: v_mfma_f32_16x16x32_bf16, one instruction per 16-byte fragment pair
//   f32 : v_mfma_f32_16x16x4_f32, four instructions per 16-byte fragment pair
//         (lane group g supplies k = 4*chunk + e to instruction e; A and B use
//          the same assignment, so the k-sum is exact)
//
// Workgroups are remapped so that each XCD (8 on MI355X, dispatched
// round-robin) works on a contiguous range of tiles, n fastest: the ~32 CUs of
// an XCD share a few m-row panels of x and the whole w in their L2.
#include "nsw_common.h"

namespace nsw {

enum Epi {
  EPI_NONE = NSW_EPI_NONE,
  EPI_BIAS = NSW_EPI_BIAS,
  EPI_BIAS_GELU = NSW_EPI_BIAS_GELU,
  EPI_BIAS_RESIDUAL = NSW_EPI_BIAS_RESIDUAL,
  EPI_QKV_HEADNORM = 10,     // bias, then per-head RMSNorm of the q and k columns
  EPI_SCATTER_RESIDUAL = 11  // bias, row m -> token_of_row(m), + skip[token]
};

constexpr int BM = 256;
constexpr int BN = 128;
constexpr int ROWB = 128;          // k-tile bytes per row
constexpr int LDS_STRIDE = 144;    // padded row stride in LDS (bytes)
constexpr int STAGE_BYTES = (BM + BN) * LDS_STRIDE;

struct EpiArgs {
  const void* bias;
  const void* residual;
  const void* qn_w;
  const void* kn_w;
  float eps;
  int C;       // q/k/v width for EPI_QKV_HEADNORM
  int hd;      // head dim for EPI_QKV_HEADNORM
  WinGeom geom;  // EPI_SCATTER_RESIDUAL
};

__device__ __forceinline__ float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

template <typename T>
__device__ __forceinline__ void mfma_chunk(f32x4& acc, const u32x4& a, const u32x4& b) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 av = __builtin_bit_cast(bf16x8, a);
    bf16x8 bv = __builtin_bit_cast(bf16x8, b);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  } else {
    f32x4 av = __builtin_bit_cast(f32x4, a);
    f32x4 bv = __builtin_bit_cast(f32x4, b);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[0], bv[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[1], bv[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[2], bv[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[3], bv[3], acc, 0, 0, 0);
  }
}

// Bijective remap of the hardware workgroup id so that XCD x (which receives
// ids x, x+8, x+16, ...) processes the contiguous logical range
// [x*q + min(x, rem), ...).
__device__ __forceinline__ int xcd_remap(int bid, int ntiles) {
  const int q = ntiles >> 3, rem = ntiles & 7;
  const int x = bid & 7, idx = bid >> 3;
  return x * q + (x < rem ? x : rem) + idx;
}

template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const T* __restrict__ X, const T* __restrict__ Wt,
                                                   T* __restrict__ Y, int M, int N, int K,
                                                   EpiArgs ea) {
  constexpr int VEC = 16 / sizeof(T);        // elements per 16-byte chunk
  constexpr int KT = ROWB / sizeof(T);       // elements per k tile
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int MT = (M + BM - 1) / BM, NT = (N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, MT * NT);
  const int mt = tile / NT, nt = tile - mt * NT;
  const int m0 = mt * BM, n0 = nt * BN;

  // ---- global -> register staging: 8 x-chunks and 4 w-chunks per thread
  const int lrow = tid >> 3, lchunk = tid & 7;
  const T* xsrc[8];
  const T* wsrc[4];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    int r = m0 + p * 32 + lrow;
    r = r < M ? r : M - 1;
    xsrc[p] = X + (int64_t)r * K + lchunk * VEC;
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    int r = n0 + p * 32 + lrow;
    r = r < N ? r : N - 1;
    wsrc[p] = Wt + (int64_t)r * K + lchunk * VEC;
  }
  u32x4 xr[8], wr[4];
#define NSW_GLOAD(kt_)                                                                   \
  do {                                                                                   \
    const int koff_ = (kt_) * KT;                                                        \
    _Pragma("unroll") for (int p = 0; p < 8; ++p)                                        \
      xr[p] = *reinterpret_cast<const u32x4*>(xsrc[p] + koff_);                          \
    _Pragma("unroll") for (int p = 0; p < 4; ++p)                                        \
      wr[p] = *reinterpret_cast<const u32x4*>(wsrc[p] + koff_);                          \
  } while (0)
#define NSW_LSTORE(stage_)                                                               \
  do {                                                                                   \
    char* base_ = smem + (stage_) * STAGE_BYTES;                                         \
    _Pragma("unroll") for (int p = 0; p < 8; ++p)                                        \
      *reinterpret_cast<u32x4*>(base_ + (p * 32 + lrow) * LDS_STRIDE + lchunk * 16) = xr[p]; \
    _Pragma("unroll") for (int p = 0; p < 4; ++p)                                        \
      *reinterpret_cast<u32x4*>(base_ + (BM + p * 32 + lrow) * LDS_STRIDE + lchunk * 16) = wr[p]; \
  } while (0)

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int frow = lane & 15, fg = lane >> 4;
  const int nk = K / KT;

  NSW_GLOAD(0);
  NSW_LSTORE(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int stage = kt & 1;
    if (kt + 1 < nk) NSW_GLOAD(kt + 1);
    const char* base = smem + stage * STAGE_BYTES;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int coff = (4 * s + fg) * 16;
      u32x4 af[4], bfr[8];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        af[nb] = *reinterpret_cast<const u32x4*>(base + (BM + wn * 64 + nb * 16 + frow) * LDS_STRIDE + coff);
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
        bfr[mb] = *reinterpret_cast<const u32x4*>(base + (wm * 128 + mb * 16 + frow) * LDS_STRIDE + coff);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) mfma_chunk<T>(acc[nb][mb], af[nb], bfr[mb]);
    }
    if (kt + 1 < nk) NSW_LSTORE(stage ^ 1);
    __syncthreads();
  }

#undef NSW_GLOAD
#undef NSW_LSTORE

  // ---------------------------------------------------------------- epilogue
  const int nw0 = n0 + wn * 64;           // first column of this wave
  const T* bias = (const T*)ea.bias;
  float bv[4][4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int n = nw0 + nb * 16 + fg * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[nb][r] = 0.f;
    if constexpr (EPI != EPI_NONE) {
      if (n < N) load4<T>(bias + n, bv[nb]);
    }
  }

  // per-head RMSNorm weights for this lane's columns (q or k region only)
  bool headnorm = false;
  float nwv[4][4];
  if constexpr (EPI == EPI_QKV_HEADNORM) {
    const int region = nw0 / ea.C;  // 0: q, 1: k, 2: v
    headnorm = region < 2;
    const T* nwp = (const T*)(region == 0 ? ea.qn_w : ea.kn_w);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int cin = (nb * 16 + fg * 4) % ea.hd;
      if (headnorm) load4<T>(nwp + cin, nwv[nb]);
    }
  }

#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int m = m0 + wm * 128 + mb * 16 + frow;
    float v[4][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[nb][r] = acc[nb][mb][r] + bv[nb][r];

    if constexpr (EPI == EPI_QKV_HEADNORM) {
      // head groups of (hd/16) consecutive 16-column blocks; all lanes take
      // part in the shuffles (the branch below is wave-uniform).
      if (headnorm) {
        const int nbh = ea.hd >> 4;  // 1, 2 or 4
        float ssb[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          float s = 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) s += v[nb][r] * v[nb][r];
          s += __shfl_xor(s, 16, 64);
          s += __shfl_xor(s, 32, 64);
          ssb[nb] = s;
        }
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          float ss = 0.f;
          const int h0 = (nb / nbh) * nbh;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q >= h0 && q < h0 + nbh) ss += ssb[q];
          const float rs = 1.0f / sqrtf(ss / (float)ea.hd + ea.eps);
#pragma unroll
          for (int r = 0; r < 4; ++r) v[nb][r] = (v[nb][r] * rs) * nwv[nb][r];
        }
      }
    }
    if constexpr (EPI == EPI_BIAS_GELU) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[nb][r] = gelu_erf(v[nb][r]);
    }
    if (m < M) {
      int64_t orow = m;
      if constexpr (EPI == EPI_SCATTER_RESIDUAL) orow = ea.geom.token_of_row(m);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int n = nw0 + nb * 16 + fg * 4;
        if (n < N) {
          if constexpr (EPI == EPI_BIAS_RESIDUAL || EPI == EPI_SCATTER_RESIDUAL) {
            float rv[4];
            load4<T>((const T*)ea.residual + orow * N + n, rv);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[nb][r] += rv[r];
          }
          store4<T>(Y + orow * N + n, v[nb]);
        }
      }
    }
  }
}

template <typename T, int EPI>
static int launch_gemm(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K,
                       const EpiArgs& ea, hipStream_t st, const char* what) {
  constexpr int KT = ROWB / sizeof(T);
  NSW_CHECK_ARG(M > 0 && N > 0 && K > 0, "%s: M, N, K must be positive", what);
  NSW_CHECK_ARG(K % KT == 0, "%s: K=%lld must be a multiple of %d", what, (long long)K, KT);
  NSW_CHECK_ARG(N % 4 == 0, "%s: N=%lld must be a multiple of 4", what, (long long)N);
  NSW_CHECK_ARG(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "%s: dims too large", what);
  NSW_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)y % 8) == 0,
                "%s: x and w must be 16-byte aligned, y 8-byte aligned", what);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  NSW_CHECK_ARG(tiles < (1LL << 31), "%s: too many tiles", what);
  hipLaunchKernelGGL((gemm_kernel<T, EPI>), dim3((unsigned)tiles), dim3(256), 0, st, (const T*)x,
                     (const T*)w, (T*)y, (int)M, (int)N, (int)K, ea);
  return check_launch(what);
}

template <int EPI>
static int dispatch_gemm(int dtype, const void* x, const void* w, void* y, int64_t M, int64_t N,
                         int64_t K, const EpiArgs& ea, void* stream, const char* what) {
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSW_DTYPE_BF16) return launch_gemm<bf16, EPI>(x, w, y, M, N, K, ea, st, what);
  if (dtype == NSW_DTYPE_F32) return launch_gemm<float, EPI>(x, w, y, M, N, K, ea, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
}

int check_geom(int64_t B, int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1, const char* what);

int gemm_qkv(const void* x, const void* wqkv, const void* bqkv, const void* qn_w, const void* kn_w,
             float eps, void* qkv, int64_t M, int64_t C, int64_t num_heads, int dtype, void* stream) {
  const char* what = "nsw_qkv_projection";
  NSW_CHECK_ARG(num_heads > 0 && C % num_heads == 0, "%s: C=%lld not divisible by num_heads=%lld", what,
                (long long)C, (long long)num_heads);
  const int64_t hd = C / num_heads;
  NSW_CHECK_ARG(C % 64 == 0, "%s: C=%lld must be a multiple of 64", what, (long long)C);
  NSW_CHECK_ARG(hd == 16 || hd == 32 || hd == 64, "%s: head_dim=%lld unsupported (16, 32, 64)", what,
                (long long)hd);
  NSW_CHECK_ARG(bqkv && qn_w && kn_w, "%s: bias and norm weights are required", what);
  EpiArgs ea{};
  ea.bias = bqkv; ea.qn_w = qn_w; ea.kn_w = kn_w; ea.eps = eps; ea.C = (int)C; ea.hd = (int)hd;
  return dispatch_gemm<EPI_QKV_HEADNORM>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
}

int gemm_proj_scatter(const void* o, const void* wproj, const void* bproj, const void* skip, void* y,
                      int64_t B, int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1,
                      int64_t s0, int64_t s1, int dtype, void* stream) {
  const char* what = "nsw_proj_reverse_residual";
  int rc = check_geom(B, T, H, W, ws0, ws1, what);
  if (rc) return rc;
  NSW_CHECK_ARG(bproj && skip, "%s: bias and skip are required", what);
  NSW_CHECK_ARG(skip != (const void*)y, "%s: skip and y must not alias (rows are permuted)", what);
  EpiArgs ea{};
  ea.bias = bproj; ea.residual = skip;
  ea.geom = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  return dispatch_gemm<EPI_SCATTER_RESIDUAL>(dtype, o, wproj, y, B * T * H * W, C, C, ea, stream, what);
}

}  // namespace nsw

using namespace nsw;

extern "C" int nsw_linear(const void* x, const void* w, const void* bias, const void* residual, void* y,
                          int64_t M, int64_t N, int64_t K, int epilogue, int dtype, void* stream) {
  const char* what = "nsw_linear";
  EpiArgs ea{};
  ea.bias = bias; ea.residual = residual;
  if (epilogue != NSW_EPI_NONE) NSW_CHECK_ARG(bias != nullptr, "%s: epilogue %d needs a bias", what, epilogue);
  switch (epilogue) {
    case NSW_EPI_NONE: return dispatch_gemm<EPI_NONE>(dtype, x, w, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS: return dispatch_gemm<EPI_BIAS>(dtype, x, w, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS_GELU: return dispatch_gemm<EPI_BIAS_GELU>(dtype, x, w, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS_RESIDUAL:
      NSW_CHECK_ARG(residual != nullptr, "%s: residual epilogue needs a residual", what);
      return dispatch_gemm<EPI_BIAS_RESIDUAL>(dtype, x, w, y, M, N, K, ea, stream, what);
    default: return set_error(NSW_ERR_INVALID, "%s: unknown epilogue %d", what, epilogue);
  }
}

extern "C" int nsw_qkv_projection(const void* x, const void* wqkv, const void* bqkv, const void* qn_w,
                                  const void* kn_w, float eps, void* qkv, int64_t M, int64_t C,
                                  int64_t num_heads, int dtype, void* stream) {
  return gemm_qkv(x, wqkv, bqkv, qn_w, kn_w, eps, qkv, M, C, num_heads, dtype, stream);
}

extern "C" int nsw_proj_reverse_residual(const void* o, const void* wproj, const void* bproj,
                                         const void* skip, void* y, int64_t B, int64_t T, int64_t H,
                                         int64_t W, int64_t C, int64_t ws0, int64_t ws1, int64_t s0,
                                         int64_t s1, int dtype, void* stream) {
  return gemm_proj_scatter(o, wproj, bproj, skip, y, B, T, H, W, C, ws0, ws1, s0, s1, dtype, stream);
}
