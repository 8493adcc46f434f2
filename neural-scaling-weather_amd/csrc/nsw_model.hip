// Model-level layout kernels around the Swin blocks: the patch matrix of the
// stride-p patch convolution (PatchEmbedLayer, models/layer_helpers.py:120-172,
// used by SwinTransformer.prepare_tokens, models/swin.py:269-284) and the
// head's unpatchify (SwinTransformer.forward_head, models/swin.py:286-299).
// Both are pure index permutations, HBM-bound, done as a transpose through
// LDS: a workgroup owns R consecutive patch rows, reads the image side along
// its contiguous rows (p consecutive pixels per patch row segment, adjacent
// patches adjacent in memory) and the patch-matrix side as whole contiguous
// rows with 16-byte vectors.  Float images with p = 2 or 4 (the models')
// take im2col_dma_kernel instead: image runs copied straight into LDS.
//
// Patch matrix: row (b, t, i, j) of [B*T*h*w, Kp], column k = (c*p + u)*p + v
// (the flattening order of a Conv2d weight [E, C, p, p]) holds
// src[b, t, c, i*p + u, j*p + v]; columns C*p*p .. Kp-1 are zero (Kp pads K to
// the GEMM's k granularity).  Channels c < C_x come from the frames of x, the
// others from the invariant fields (the preprocessor's channel concatenation,
// utils/data_utils.py:185-189, without materialising it), and frame t is read
// from slot (t + frame0) mod T of x, so that a ring buffer stands in for the
// inference loop's roll of the input window (utils/inferencer.py:448-449).
//
// Unpatchify: out[b, c, i*p + u, j*p + v] = y[(b, i, j), (u*p + v)*C_out + c].
#include "nsw_common.h"

#include <algorithm>

namespace nsw {

constexpr int MODEL_LDS = 64 * 1024;   // dynamic LDS per workgroup (at most)
#ifndef IM2COL_DMA_NB
#define IM2COL_DMA_NB 64                // 1 KB runs per workgroup of the direct-to-LDS patch matrix
#endif
// unpatchify's tile: smaller tiles, more workgroups per CU (measured at
// config 3: 24 KB tiles 70 us against 77 us with 64 KB)
constexpr int UNPATCH_LDS = 24 * 1024;

template <typename T> struct VecOf;
template <> struct VecOf<bf16> { using V = bf16x8; };
template <> struct VecOf<float> { using V = f32x4; };

template <typename TX, typename TO, int P>
__global__ __launch_bounds__(256) void im2col_kernel(const TX* __restrict__ x, const TX* __restrict__ inv,
                                                     int Cx, int Cinv, int T, int H, int W, int p,
                                                     int frame0, int Kp, int64_t M, int R,
                                                     TO* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  TO* tile = reinterpret_cast<TO*>(smem);
  constexpr int V = 16 / sizeof(TO);
  const int KS = Kp + V;                        // LDS row stride (16 B of padding)
  const int64_t m0 = (int64_t)blockIdx.x * R;
  const int rows = (int)min((int64_t)R, M - m0);
  const int h = H / p, w = W / p, pp = p * p;
  const int C = Cx + Cinv, Kc = C * pp;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;

  // per-row source offsets (channel 0, pixel (i*p, j*p)) of x and of inv
  __shared__ int64_t xbase[256];
  __shared__ int ibase[256];
  for (int r = tid; r < rows; r += 256) {
    const int64_t m = m0 + r;
    const int j = (int)(m % w);
    const int64_t q = m / w;
    const int i = (int)(q % h);
    const int64_t bt = q / h;
    const int t = (int)(bt % T);
    const int64_t b = bt / T;
    int ts = t + frame0;
    if (ts >= T) ts -= T;
    const int pix = (i * p) * W + j * p;
    xbase[r] = ((b * T + ts) * Cx) * HW + pix;
    ibase[r] = pix;
  }
  __syncthreads();

  // gather: one lane per tile row, one patch-row segment (p consecutive
  // pixels, contiguous in x) per lane and iteration; the lane groups split
  // the (c, u) pairs
  const int groups = 256 / R;
  const int r = tid % R, grp = tid / R;
  if (r < rows && grp < groups) {
    TO* trow = tile + r * KS;
    const int64_t xb = xbase[r];
    const int ib = ibase[r];
    if constexpr (P > 0) {
      // P consecutive elements per (c, u), aligned to P * sizeof(TX)
      // (host-checked); U loads in flight per lane before their LDS stores
      constexpr int SA = P * sizeof(TX) < 16 ? P * sizeof(TX) : 16;
      constexpr int DA = P * sizeof(TO) < 16 ? P * sizeof(TO) : 16;
      constexpr int UB = 128 / (P * (int)sizeof(TX));
      constexpr int U = UB < 1 ? 1 : (UB > 16 ? 16 : UB);
      const int total = C * P;
      for (int cu0 = grp; cu0 < total; cu0 += U * groups) {
        TX v[U][P];
#pragma unroll
        for (int q = 0; q < U; ++q) {
          const int cu = cu0 + q * groups;
          if (cu < total) {
            const int c = cu / P, u = cu - c * P;
            const TX* src = c < Cx ? x + xb + c * HW + (int64_t)u * W : inv + (int64_t)(c - Cx) * HW + ib + u * W;
            const TX* s_ = (const TX*)__builtin_assume_aligned(src, SA);
#pragma unroll
            for (int e = 0; e < P; ++e) v[q][e] = s_[e];
          }
        }
#pragma unroll
        for (int q = 0; q < U; ++q) {
          const int cu = cu0 + q * groups;
          if (cu < total) {
            TO* d_ = (TO*)__builtin_assume_aligned(trow + cu * P, DA);
#pragma unroll
            for (int e = 0; e < P; ++e) d_[e] = from_f32<TO>(to_f32(v[q][e]));
          }
        }
      }
    } else {
      for (int cu = grp; cu < C * p; cu += groups) {
        const int c = cu / p, u = cu - c * p;
        const TX* src = c < Cx ? x + xb + c * HW + (int64_t)u * W : inv + (int64_t)(c - Cx) * HW + ib + u * W;
        TO* dst = trow + cu * p;
        for (int e = 0; e < p; ++e) dst[e] = from_f32<TO>(to_f32(src[e]));
      }
    }
  }
  // zero padding columns
  const int padw = Kp - Kc;
  for (int e = tid; e < rows * padw; e += 256) {
    const int r = e / padw;
    tile[r * KS + Kc + (e - r * padw)] = from_f32<TO>(0.f);
  }
  __syncthreads();

  // write whole rows (contiguous in out) with 16-byte vectors
  using Vt = typename VecOf<TO>::V;
  const int vpr = Kp / V;
  Vt* orow = reinterpret_cast<Vt*>(out + m0 * Kp);
  for (int e = tid; e < rows * vpr; e += 256) {
    const int r = e / vpr, cc = e - r * vpr;
    orow[e] = *reinterpret_cast<const Vt*>(tile + r * KS + cc * V);
  }
}

// Patch matrix from float images with p = 2 or 4 (the models' patch sizes)
// through direct-to-LDS copies, so that a workgroup's loads are all in
// flight at once without register staging.  A workgroup owns TG = 256 / p
// consecutive patches (j0 ..) of patch row i of one frame and CG = NB / p
// channels (cg*CG ..): LDS block d = c' p + u (1 KB) receives the TG patches'
// run of image row i p + u of channel c' -- 64 lanes x 16 bytes, lane l
// loading the run's 16-byte chunk l ^ s(c', u), so that chunk q sits at
// slot q ^ s.  s(c', u) is the index of the patch-matrix row chunk that
// run's values land in, so the 16 lanes that write 16 consecutive chunks of
// one patch row read 16 distinct 16-byte slots (all 64 banks).  Chunks past
// the image row's end re-read its last chunk (never stored).  Then each
// thread writes 16-byte chunks of the patch rows (CG channels' p*p columns
// per row, the last group also the zero columns up to Kp).
template <int P, typename TO>
__device__ __forceinline__ int im2col_swz(int cl, int u) {
  return (((cl * P + u) * P * (int)sizeof(TO)) >> 4) & 15;
}

template <typename TO, int P, int NB>
__global__ __launch_bounds__(256) void im2col_dma_kernel(const float* __restrict__ x, const float* __restrict__ inv,
                                                         int Cx, int Cinv, int T, int H, int W, int frame0, int Kp,
                                                         int ncg, int ntg, TO* __restrict__ out) {
  constexpr int CG = NB / P;                 // channels per workgroup
  constexpr int TG = 64 * 4 / P;             // patches per workgroup: one 1 KB run per image row
  constexpr int V = 16 / (int)sizeof(TO);    // patch-matrix elements per 16-byte chunk
  constexpr int CPR = CG * P * P / V;        // chunks per patch-row segment
  static_assert(V % P == 0 && NB % 4 == 0, "im2col_dma_kernel layout");
  __shared__ __attribute__((aligned(1024))) char smem[NB * 1024];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = H / P, w = W / P, C = Cx + Cinv, Kc = C * P * P;
  int item = blockIdx.x;                     // channel group fastest, then patch group, patch row, frame
  const int cg = item % ncg;
  item /= ncg;
  const int jg = item % ntg;
  item /= ntg;
  const int i = item % h;
  const int bt = item / h;                   // b * T + t
  const int t = bt % T, b = bt / T;
  int ts = t + frame0;
  if (ts >= T) ts -= T;
  const int64_t HW = (int64_t)H * W;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
#pragma unroll
  for (int j = 0; j < NB / 4; ++j) {
    const int d = wave * (NB / 4) + j;
    const int cl = d / P, u = d - cl * P;
    int c = cg * CG + cl;
    c = c < C ? c : C - 1;                   // past C: a valid plane, never stored
    const float* plane = c < Cx ? x + ((int64_t)(b * T + ts) * Cx + c) * HW : inv + (int64_t)(c - Cx) * HW;
    int x0 = jg * TG * P + (lane ^ im2col_swz<P, TO>(cl, u)) * 4;
    x0 = x0 + 4 <= W ? x0 : W - 4;
    // non-temporal: the image is read once (290 MB at config 3); 82.1 ->
    // 73.4 us at config 3, bit-identical
    dma16<true>(make_rsrc(plane, (uint32_t)(HW * 4)), lds0 + (uint32_t)d * 1024u,
                (uint32_t)(((i * P + u) * W + x0) * 4), 0u);
  }
  NSW_WAIT_VMCNT(0);
  __syncthreads();

  const int k0 = cg * CG * P * P;
  for (int e = tid; e < TG * CPR; e += 256) {
    const int tt = e / CPR, ch = e - tt * CPR;
    const int j = jg * TG + tt;
    const int kk = k0 + ch * V;
    if (j >= w || kk >= Kp) continue;
    TO v[V];
#pragma unroll
    for (int r = 0; r < V / P; ++r) {
      const int kl = ch * V + r * P;         // column within the group: c' p^2 + u p
      const int cl = kl / (P * P), u = (kl / P) % P;
      float f[P];
      if (k0 + kl < Kc) {
        const int slot = ((tt * P) >> 2) ^ im2col_swz<P, TO>(cl, u);
        const char* src = smem + (cl * P + u) * 1024 + slot * 16 + ((tt * P * 4) & 15);
        if constexpr (P == 4) {
          const f32x4 q = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
          for (int k = 0; k < 4; ++k) f[k] = q[k];
        } else {
          const float2 q = *reinterpret_cast<const float2*>(src);
          f[0] = q.x;
          f[1] = q.y;
        }
      } else {
#pragma unroll
        for (int k = 0; k < P; ++k) f[k] = 0.f;   // zero columns Kc .. Kp-1
      }
#pragma unroll
      for (int k = 0; k < P; ++k) v[r * P + k] = from_f32<TO>(f[k]);
    }
    const int64_t m = ((int64_t)bt * h + i) * w + j;
    *reinterpret_cast<u32x4*>(out + m * Kp + kk) = __builtin_bit_cast(u32x4, v);
  }
}

template <typename TI, typename TO, int P>
__global__ __launch_bounds__(256) void unpatchify_kernel(const TI* __restrict__ y, int Co, int H, int W, int p,
                                                         int64_t out_bstride, int64_t M, int R, int pairs,
                                                         TO* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  TI* tile = reinterpret_cast<TI*>(smem);
  constexpr int V = 16 / sizeof(TI);
  const int N = p * p * Co;
  const int NS = N + V;
  const int64_t m0 = (int64_t)blockIdx.x * R;
  const int rows = (int)min((int64_t)R, M - m0);
  const int h = H / p, w = W / p;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;

  __shared__ int64_t obase[256];
  for (int r = tid; r < rows; r += 256) {
    const int64_t m = m0 + r;
    const int j = (int)(m % w);
    const int64_t q = m / w;
    const int i = (int)(q % h);
    const int64_t b = q / h;
    obase[r] = b * out_bstride + (int64_t)(i * p) * W + j * p;
  }
  // load whole rows (contiguous in y) with 16-byte vectors
  using Vt = typename VecOf<TI>::V;
  const int vpr = N / V;
  const Vt* yrow = reinterpret_cast<const Vt*>(y + m0 * N);
  for (int e = tid; e < rows * vpr; e += 256) {
    const int r = e / vpr, cc = e - r * vpr;
    *reinterpret_cast<Vt*>(tile + r * NS + cc * V) = yrow[e];
  }
  __syncthreads();

  // scatter: per iteration a lane writes the p consecutive pixels of its
  // patch in one output row (one vector store), or, with `pairs` (host:
  // even R and w, output aligned), the 2p pixels of two horizontally
  // adjacent patches (tile rows 2k, 2k + 1 of one image row)
  if constexpr (P > 0) {
    if (pairs) {
      const int RP = R / 2, rowsP = rows / 2;    // rows is even with pairs
      const int groups = 256 / RP;
      const int rp = tid % RP, grp = tid / RP;
      if (rp < rowsP && grp < groups) {
        constexpr int DA = 2 * P * sizeof(TO) < 16 ? 2 * P * sizeof(TO) : 16;
        const TI* t0 = tile + 2 * rp * NS;
        const TI* t1 = t0 + NS;
        const int64_t ob = obase[2 * rp];
        bool done = false;
        if constexpr (sizeof(TI) == 2) {
          if (Co % 2 == 0) {
          done = true;
          // two channels per lane: each LDS read (4 bytes) serves two planes
          const int Ch = Co / 2;
#pragma unroll 2
          for (int cu = grp; cu < Ch * P; cu += groups) {
            const int c = 2 * (cu / P), u = cu - (cu / P) * P;
            const int so = u * P * Co + c;
            TO v0[2 * P], v1[2 * P];
#pragma unroll
            for (int e = 0; e < P; ++e) {
              const uint32_t a = *reinterpret_cast<const uint32_t*>(t0 + so + e * Co);
              const uint32_t b = *reinterpret_cast<const uint32_t*>(t1 + so + e * Co);
              const bf16x2 pa = __builtin_bit_cast(bf16x2, a), pb = __builtin_bit_cast(bf16x2, b);
              v0[e] = from_f32<TO>((float)pa[0]);
              v1[e] = from_f32<TO>((float)pa[1]);
              v0[P + e] = from_f32<TO>((float)pb[0]);
              v1[P + e] = from_f32<TO>((float)pb[1]);
            }
            TO* d0 = (TO*)__builtin_assume_aligned(out + ob + c * HW + (int64_t)u * W, DA);
            TO* d1 = (TO*)__builtin_assume_aligned(out + ob + (c + 1) * HW + (int64_t)u * W, DA);
#pragma unroll
            for (int e = 0; e < 2 * P; ++e) d0[e] = v0[e];
#pragma unroll
            for (int e = 0; e < 2 * P; ++e) d1[e] = v1[e];
          }
          }
        }
        if (!done) {
#pragma unroll 2
          for (int cu = grp; cu < Co * P; cu += groups) {
            const int c = cu / P, u = cu - c * P;
            TO* d_ = (TO*)__builtin_assume_aligned(out + ob + c * HW + (int64_t)u * W, DA);
            const int so = u * P * Co + c;
            TO v[2 * P];
#pragma unroll
            for (int e = 0; e < P; ++e) {
              v[e] = from_f32<TO>(to_f32(t0[so + e * Co]));
              v[P + e] = from_f32<TO>(to_f32(t1[so + e * Co]));
            }
#pragma unroll
            for (int e = 0; e < 2 * P; ++e) d_[e] = v[e];
          }
        }
      }
      return;
    }
  }
  const int groups = 256 / R;
  const int r = tid % R, grp = tid / R;
  if (r < rows && grp < groups) {
    const int p_ = P > 0 ? P : p;
    const TI* trow = tile + r * NS;
    const int64_t ob = obase[r];
#pragma unroll 4
    for (int cu = grp; cu < Co * p_; cu += groups) {
      const int c = cu / p_, u = cu - c * p_;
      TO* dst = out + ob + c * HW + (int64_t)u * W;
      const TI* src = trow + u * p_ * Co + c;
      if constexpr (P > 0) {
        constexpr int DA = P * sizeof(TO) < 16 ? P * sizeof(TO) : 16;
        TO* d_ = (TO*)__builtin_assume_aligned(dst, DA);
        TO v[P];
#pragma unroll
        for (int e = 0; e < P; ++e) v[e] = from_f32<TO>(to_f32(src[e * Co]));
#pragma unroll
        for (int e = 0; e < P; ++e) d_[e] = v[e];
      } else {
        for (int e = 0; e < p_; ++e) dst[e] = from_f32<TO>(to_f32(src[e * Co]));
      }
    }
  }
}

// Rows per workgroup: at most 64 (four lane groups split the (c, u) pairs)
// and at most `budget` bytes of tile (at least one row).
static int rows_per_wg(int budget, int row_bytes) {
  int r = 64;
  const int lim = budget / row_bytes;
  if (lim < r) r = lim;
  return r < 1 ? 1 : r;
}

}  // namespace nsw

namespace nsw {

// SwinTransformer's big skip (use_big_skip_conv, models/swin.py:212-223,
// 310-319): a 1x1 convolution without bias from the input channels to the
// output channels, added to the head's image.  Only the predicted frame is
// returned (x[:, -1:]), so only the window's last frame is convolved:
//   out[b, co, q] = R_o(out[b, co, q] + R_m(sum_ci w[co, ci] R_m(xin[b, ci, q])))
// with xin = x's frame (T - 1 + frame0) mod T of the ring, then the invariant
// planes; R_m rounds to the model's dtype (the reference convolves the
// model-dtype input and returns the model dtype, then adds two model-dtype
// tensors), R_o to out's dtype.  A thread owns 4 consecutive pixels and CPT
// output channels (blockIdx.y), the weight [C_out, C_in] sits in LDS.
template <typename TX, typename TO, typename TM, int CPT>
__global__ __launch_bounds__(256) void skip_conv_kernel(const TX* __restrict__ x, const TX* __restrict__ inv,
                                                        const float* __restrict__ w, TO* __restrict__ out,
                                                        int C_x, int C_inv, int C_out, int T, int slot,
                                                        int64_t HW, int64_t out_bstride) {
  extern __shared__ float wl[];
  const int C = C_x + C_inv;
  for (int i = threadIdx.x; i < C_out * C; i += 256) wl[i] = w[i];
  __syncthreads();
  const int b = blockIdx.z;
  const int co0 = blockIdx.y * CPT;
  const int64_t q0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (q0 >= HW) return;
  float acc[CPT][4];
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[j][e] = 0.f;
  const TX* xb = x + ((int64_t)b * T + slot) * C_x * HW + q0;
  for (int ci = 0; ci < C; ++ci) {
    const TX* src = ci < C_x ? xb + (int64_t)ci * HW : inv + (int64_t)(ci - C_x) * HW + q0;
    float v[4];
    load4<TX>(src, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = to_f32(from_f32<TM>(v[e]));
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const float wv = co0 + j < C_out ? wl[(co0 + j) * C + ci] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j][e] = fmaf(wv, v[e], acc[j][e]);
    }
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    if (co0 + j >= C_out) break;
    TO* o = out + (int64_t)b * out_bstride + (int64_t)(co0 + j) * HW + q0;
    float cur[4], r[4];
    load4<TO>(o, cur);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = cur[e] + to_f32(from_f32<TM>(acc[j][e]));
    store4<TO>(o, r);
  }
}

}  // namespace nsw

using namespace nsw;

extern "C" int nsw_patch_im2col(const void* x, const void* inv, int64_t B, int64_t T, int64_t C_x,
                                int64_t C_inv, int64_t H, int64_t W, int64_t p, int64_t frame0,
                                int64_t Kp, void* out, int x_dtype, int out_dtype, void* stream) {
  const char* what = "nsw_patch_im2col";
  NSW_CHECK_ARG(B > 0 && T > 0 && C_x > 0 && C_inv >= 0 && H > 0 && W > 0 && p > 0,
                "%s: B, T, C_x, H, W, p must be positive (C_inv >= 0)", what);
  NSW_CHECK_ARG(p <= 16 && H % p == 0 && W % p == 0, "%s: H=%lld, W=%lld not divisible by p=%lld (p <= 16)",
                what, (long long)H, (long long)W, (long long)p);
  NSW_CHECK_ARG(C_inv == 0 || inv != nullptr, "%s: invariant channels without data", what);
  NSW_CHECK_ARG(frame0 >= 0 && frame0 < T, "%s: frame0 must lie in [0, T)", what);
  const int64_t Kc = (C_x + C_inv) * p * p;
  const int V = out_dtype == NSW_DTYPE_BF16 ? 8 : 4;
  NSW_CHECK_ARG(Kp >= Kc && Kp % V == 0, "%s: Kp=%lld must be >= C*p*p=%lld and a multiple of %d", what,
                (long long)Kp, (long long)Kc, V);
  NSW_CHECK_ARG(((uintptr_t)out % 16) == 0, "%s: out must be 16-byte aligned", what);
  NSW_CHECK_ARG(B * T * C_x * H * W < (1LL << 40) && H * W < (1LL << 31), "%s: too large", what);
  const int64_t M = B * T * (H / p) * (W / p);
  const size_t es = dtype_size(out_dtype);
  // float images with p = 2 or 4: the direct-to-LDS kernel (its buffer
  // ranges and byte offsets into one image plane are 32-bit: H*W*4 < 2^31)
  if (x_dtype == NSW_DTYPE_F32 && (p == 2 || p == 4) && W % 4 == 0 && H * W * 4 < (1LL << 31) &&
      ((uintptr_t)x % 16) == 0 &&
      (inv == nullptr || ((uintptr_t)inv % 16) == 0)) {
    constexpr int NB = IM2COL_DMA_NB;
    const int CG = NB / (int)p, TG = 256 / (int)p;
    const int64_t C = C_x + C_inv;
    const int64_t ncg = (C + CG - 1) / CG, ntg = (W / p + TG - 1) / TG;
    const int64_t items = B * T * (H / p) * ntg * ncg;
    if (ncg * CG * p * p >= Kp && items < (1LL << 31)) {
      hipStream_t st = (hipStream_t)stream;
#define NSW_IM2COL_DMA(TO, P)                                                                                  \
  hipLaunchKernelGGL((im2col_dma_kernel<TO, P, NB>), dim3((unsigned)items), dim3(256), 0, st, (const float*)x, \
                     (const float*)inv, (int)C_x, (int)C_inv, (int)T, (int)H, (int)W, (int)frame0, (int)Kp,   \
                     (int)ncg, (int)ntg, (TO*)out)
      if (out_dtype == NSW_DTYPE_BF16) {
        if (p == 4) NSW_IM2COL_DMA(bf16, 4); else NSW_IM2COL_DMA(bf16, 2);
      } else if (out_dtype == NSW_DTYPE_F32) {
        if (p == 4) NSW_IM2COL_DMA(float, 4); else NSW_IM2COL_DMA(float, 2);
      } else {
        return set_error(NSW_ERR_INVALID, "%s: unknown output dtype %d", what, out_dtype);
      }
#undef NSW_IM2COL_DMA
      return check_launch(what);
    }
  }
  const int row_bytes = (int)((Kp + V) * es);
  NSW_CHECK_ARG(row_bytes <= MODEL_LDS, "%s: Kp=%lld too large for one LDS row", what, (long long)Kp);
  const int R = rows_per_wg(MODEL_LDS, row_bytes);
  const int64_t grid = (M + R - 1) / R;
  NSW_CHECK_ARG(grid < (1LL << 31), "%s: too many rows", what);
  hipStream_t st = (hipStream_t)stream;
  const size_t shm = (size_t)R * row_bytes;
  const dim3 g((unsigned)grid), blk(256);
  // p-specialised instances move one aligned vector per patch-row segment
  const size_t xes = dtype_size(x_dtype);
  const bool vec = (p == 1 || p == 2 || p == 4 || p == 8 || p == 16) &&
                   ((uintptr_t)x % std::min<size_t>(16, p * xes)) == 0 &&
                   (inv == nullptr || ((uintptr_t)inv % std::min<size_t>(16, p * xes)) == 0);
#define NSW_IM2COL_P(TX, TO, P)                                                                              \
  hipLaunchKernelGGL((im2col_kernel<TX, TO, P>), g, blk, shm, st, (const TX*)x, (const TX*)inv, (int)C_x,   \
                     (int)C_inv, (int)T, (int)H, (int)W, (int)p, (int)frame0, (int)Kp, M, R, (TO*)out)
#define NSW_IM2COL(TX, TO)                                                                                   \
  do {                                                                                                       \
    if (!vec) NSW_IM2COL_P(TX, TO, 0);                                                                       \
    else if (p == 1) NSW_IM2COL_P(TX, TO, 1);                                                                \
    else if (p == 2) NSW_IM2COL_P(TX, TO, 2);                                                                \
    else if (p == 4) NSW_IM2COL_P(TX, TO, 4);                                                                \
    else if (p == 8) NSW_IM2COL_P(TX, TO, 8);                                                                \
    else NSW_IM2COL_P(TX, TO, 16);                                                                           \
  } while (0)
  if (x_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_BF16) NSW_IM2COL(float, bf16);
  else if (x_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_F32) NSW_IM2COL(float, float);
  else if (x_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_BF16) NSW_IM2COL(bf16, bf16);
  else if (x_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_F32) NSW_IM2COL(bf16, float);
  else return set_error(NSW_ERR_INVALID, "%s: unknown dtype pair %d -> %d", what, x_dtype, out_dtype);
#undef NSW_IM2COL_P
#undef NSW_IM2COL
  return check_launch(what);
}

extern "C" int nsw_unpatchify(const void* y, void* out, int64_t B, int64_t C_out, int64_t H, int64_t W,
                              int64_t p, int64_t out_bstride, int in_dtype, int out_dtype, void* stream) {
  const char* what = "nsw_unpatchify";
  NSW_CHECK_ARG(B > 0 && C_out > 0 && H > 0 && W > 0 && p > 0, "%s: B, C_out, H, W, p must be positive", what);
  NSW_CHECK_ARG(p <= 16 && H % p == 0 && W % p == 0, "%s: H=%lld, W=%lld not divisible by p=%lld (p <= 16)",
                what, (long long)H, (long long)W, (long long)p);
  NSW_CHECK_ARG(out_bstride >= C_out * H * W, "%s: out_bstride smaller than one sample", what);
  const int64_t N = p * p * C_out;
  const int V = in_dtype == NSW_DTYPE_BF16 ? 8 : 4;
  NSW_CHECK_ARG(N % V == 0, "%s: p*p*C_out=%lld must be a multiple of %d", what, (long long)N, V);
  NSW_CHECK_ARG(((uintptr_t)y % 16) == 0, "%s: y must be 16-byte aligned", what);
  NSW_CHECK_ARG(B * out_bstride < (1LL << 40), "%s: too large", what);
  const int64_t M = B * (H / p) * (W / p);
  const size_t es = dtype_size(in_dtype);
  const int row_bytes = (int)((N + V) * es);
  NSW_CHECK_ARG(row_bytes <= MODEL_LDS, "%s: p*p*C_out=%lld too large for one LDS row", what, (long long)N);
  int R = rows_per_wg(UNPATCH_LDS, row_bytes);
  const int64_t wp = W / p;
  if (R > 1) R &= ~1;                            // even: tile rows pair up inside image rows when wp is even
  const int64_t grid = (M + R - 1) / R;
  NSW_CHECK_ARG(grid < (1LL << 31), "%s: too many rows", what);
  hipStream_t st = (hipStream_t)stream;
  const size_t shm = (size_t)R * row_bytes;
  const dim3 g((unsigned)grid), blk(256);
  const size_t oes = dtype_size(out_dtype);
  const bool vec = (p == 1 || p == 2 || p == 4 || p == 8 || p == 16) &&
                   ((uintptr_t)out % std::min<size_t>(16, p * oes)) == 0 &&
                   ((out_bstride * (int64_t)oes) % (int64_t)std::min<size_t>(16, p * oes)) == 0;
  const size_t pa = std::min<size_t>(16, 2 * p * oes);
  const int pairs = vec && R % 2 == 0 && wp % 2 == 0 && ((uintptr_t)out % pa) == 0 &&
                    ((out_bstride * (int64_t)oes) % (int64_t)pa) == 0 && ((H * W * (int64_t)oes) % (int64_t)pa) == 0;
#define NSW_UNPATCH_P(TI, TO, P)                                                                           \
  hipLaunchKernelGGL((unpatchify_kernel<TI, TO, P>), g, blk, shm, st, (const TI*)y, (int)C_out, (int)H,    \
                     (int)W, (int)p, out_bstride, M, R, pairs, (TO*)out)
#define NSW_UNPATCH(TI, TO)                                                                                \
  do {                                                                                                     \
    if (!vec) NSW_UNPATCH_P(TI, TO, 0);                                                                    \
    else if (p == 1) NSW_UNPATCH_P(TI, TO, 1);                                                             \
    else if (p == 2) NSW_UNPATCH_P(TI, TO, 2);                                                             \
    else if (p == 4) NSW_UNPATCH_P(TI, TO, 4);                                                             \
    else if (p == 8) NSW_UNPATCH_P(TI, TO, 8);                                                             \
    else NSW_UNPATCH_P(TI, TO, 16);                                                                        \
  } while (0)
  if (in_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_BF16) NSW_UNPATCH(bf16, bf16);
  else if (in_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_F32) NSW_UNPATCH(bf16, float);
  else if (in_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_F32) NSW_UNPATCH(float, float);
  else if (in_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_BF16) NSW_UNPATCH(float, bf16);
  else return set_error(NSW_ERR_INVALID, "%s: unknown dtype pair %d -> %d", what, in_dtype, out_dtype);
#undef NSW_UNPATCH_P
#undef NSW_UNPATCH
  return check_launch(what);
}

extern "C" int nsw_skip_conv_accumulate(const void* x, const void* inv, const float* w, void* out, int64_t B,
                                        int64_t T, int64_t C_x, int64_t C_inv, int64_t C_out, int64_t H,
                                        int64_t W, int64_t frame0, int64_t out_bstride, int x_dtype,
                                        int model_dtype, int out_dtype, void* stream) {
  const char* what = "nsw_skip_conv_accumulate";
  NSW_CHECK_ARG(B > 0 && T > 0 && C_x > 0 && C_inv >= 0 && C_out > 0 && H > 0 && W > 0,
                "%s: B, T, C_x, C_out, H, W must be positive (C_inv >= 0)", what);
  NSW_CHECK_ARG(C_inv == 0 || inv != nullptr, "%s: invariant channels without data", what);
  NSW_CHECK_ARG(x != nullptr && w != nullptr && out != nullptr, "%s: missing pointer", what);
  NSW_CHECK_ARG(frame0 >= 0 && frame0 < T, "%s: frame0 must lie in [0, T)", what);
  NSW_CHECK_ARG((C_x + C_inv) * C_out <= 16384, "%s: C_out x C_in = %lld above 16384 (the weight lives in LDS)",
                what, (long long)((C_x + C_inv) * C_out));
  const int64_t HW = H * W;
  NSW_CHECK_ARG(HW % 4 == 0 && HW < (1LL << 31), "%s: H*W=%lld must be a multiple of 4 (below 2^31)", what,
                (long long)HW);
  NSW_CHECK_ARG(out_bstride >= C_out * HW, "%s: out_bstride smaller than one sample", what);
  const size_t xa = 4 * dtype_size(x_dtype), oa = 4 * dtype_size(out_dtype);
  NSW_CHECK_ARG(((uintptr_t)x % xa) == 0 && (inv == nullptr || ((uintptr_t)inv % xa) == 0) &&
                    ((uintptr_t)out % oa) == 0 && (out_bstride * (int64_t)dtype_size(out_dtype)) % (int64_t)oa == 0,
                "%s: x / inv / out must be aligned to 4 elements", what);
  NSW_CHECK_ARG(B * T * C_x * HW < (1LL << 40) && B * out_bstride < (1LL << 40), "%s: too large", what);
  NSW_CHECK_ARG(B < 65536, "%s: B=%lld too large", what, (long long)B);
  constexpr int CPT = 16;
  const dim3 g((unsigned)((HW / 4 + 255) / 256), (unsigned)((C_out + CPT - 1) / CPT), (unsigned)B), blk(256);
  const size_t shm = (size_t)(C_x + C_inv) * C_out * sizeof(float);
  const int slot = (int)((T - 1 + frame0) % T);
  hipStream_t st = (hipStream_t)stream;
#define NSW_SKIP(TX, TO, TM)                                                                                 \
  hipLaunchKernelGGL((skip_conv_kernel<TX, TO, TM, CPT>), g, blk, shm, st, (const TX*)x, (const TX*)inv, w,  \
                     (TO*)out, (int)C_x, (int)C_inv, (int)C_out, (int)T, slot, HW, out_bstride)
#define NSW_SKIP_M(TX, TO)                                                                                   \
  do {                                                                                                       \
    if (model_dtype == NSW_DTYPE_BF16) NSW_SKIP(TX, TO, bf16);                                               \
    else if (model_dtype == NSW_DTYPE_F32) NSW_SKIP(TX, TO, float);                                          \
    else return set_error(NSW_ERR_INVALID, "%s: unknown model dtype %d", what, model_dtype);                 \
  } while (0)
  if (x_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_BF16) NSW_SKIP_M(float, bf16);
  else if (x_dtype == NSW_DTYPE_F32 && out_dtype == NSW_DTYPE_F32) NSW_SKIP_M(float, float);
  else if (x_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_BF16) NSW_SKIP_M(bf16, bf16);
  else if (x_dtype == NSW_DTYPE_BF16 && out_dtype == NSW_DTYPE_F32) NSW_SKIP_M(bf16, float);
  else return set_error(NSW_ERR_INVALID, "%s: unknown dtype pair %d -> %d", what, x_dtype, out_dtype);
#undef NSW_SKIP_M
#undef NSW_SKIP
  return check_launch(what);
}
