// Shared device/host helpers of libnsw (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/nsw.h"

namespace nsw {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

// ---------------------------------------------------------------- errors ----
// Every C-ABI entry point returns NSW_OK or an error code and leaves a
// human-readable message in a thread-local buffer (nsw_last_error()).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define NSW_CHECK_ARG(cond, ...)                                  \
  do {                                                            \
    if (!(cond)) return ::nsw::set_error(NSW_ERR_INVALID, __VA_ARGS__); \
  } while (0)

inline size_t dtype_size(int dtype) { return dtype == NSW_DTYPE_BF16 ? 2 : 4; }

// ------------------------------------------------------------ conversions ---
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
// v_cvt_pk_bf16_f32: round to nearest even, as torch's float -> bfloat16 cast.
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// 16-byte vector of T (8 bf16 or 4 f32), the unit of every global load/store.
template <typename T> struct Vec16 { static constexpr int N = 16 / sizeof(T); };

template <typename T>
__device__ __forceinline__ void load16(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)v[i];
  } else {
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v[i];
  }
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (bf16)in[i];
    *reinterpret_cast<bf16x8*>(p) = v;
  } else {
    f32x4 v = {in[0], in[1], in[2], in[3]};
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// 4 consecutive values (8 B for bf16, 16 B for f32).
template <typename T>
__device__ __forceinline__ void load4(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    out[0] = (float)v[0]; out[1] = (float)v[1]; out[2] = (float)v[2]; out[3] = (float)v[3];
  } else {
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    bf16x4 v = {(bf16)in[0], (bf16)in[1], (bf16)in[2], (bf16)in[3]};
    *reinterpret_cast<bf16x4*>(p) = v;
  } else {
    f32x4 v = {in[0], in[1], in[2], in[3]};
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// ---------------------------------------------------------- wave helpers ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Reductions over the four 16-lane rows of a wavefront (lanes l, l^16, l^32,
// l^48), the lanes that hold one row / query in an MFMA 16x16 result block.
// v_permlane16_swap(x, x) returns {x of even row, x of odd row} of each row
// pair and v_permlane32_swap(x, x) {x of lower half, x of upper half}, so
// combining the two returned values gives the xor-16 / xor-32 partner result
// in the same operand order on every lane (pure VALU, no LDS traffic).
//
// Issued through inline asm: with the same value in both operands the
// compiler's builtin lowering (ROCm 7.2 clang) folds the two results into one
// register and returns 2x instead of x + partner.  The s_nop covers the
// VALU-write -> permlane-read hazard.
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ float rows4_sum(float x) {
  float a = x, b = x;
  permlane16_swap(a, b);
  const float s = a + b;
  float c = s, d = s;
  permlane32_swap(c, d);
  return c + d;
}

// Sum over the pair of 16-lane rows (lanes l, l^16) only.
__device__ __forceinline__ float rows2_sum(float x) {
  float a = x, b = x;
  permlane16_swap(a, b);
  return a + b;
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), on every lane:
// rotations by 8, 4, 2, 1 within the row.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return x;
}

__device__ __forceinline__ float rows4_max(float x) {
  float a = x, b = x;
  permlane16_swap(a, b);
  const float s = fmaxf(a, b);
  float c = s, d = s;
  permlane32_swap(c, d);
  return fmaxf(c, d);
}

// ------------------------------------------- direct-to-LDS copies, waits ----
// Buffer resource (V#) over a whole tensor: raw buffer, stride 0, 32-bit
// byte offsets, num_records = bytes, dword 3 = 0x00020000 (the gfx9 raw
// buffer format).  Built from wave-uniform values so it lives in SGPRs.
__device__ __forceinline__ u32x4 make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)p;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// One direct-to-LDS copy: every lane loads 16 bytes at rsrc + voff + soff and
// the wave's 64 x 16 B land contiguously at LDS byte address lds_addr.
// Issued as inline asm so that the compiler's wait-count insertion does not
// see an LDS write in flight (it would otherwise drain all copies before
// each fragment read); ordering is kept by the explicit vmcnt waits and
// barriers of the pipeline.  s_nop: M0 write -> LDS-DMA read hazard.
// The scalar operands pass through v_readfirstlane, which the compiler drops
// when they already live in SGPRs: a wave-uniform value computed along paths
// the divergence analysis cannot prove uniform would otherwise reach the
// "s" constraints in a VGPR (an assembler error).
// NT: the non-temporal form (`nt`), for data read exactly once, so that it
// does not displace reused lines in the caches.
template <bool NT = false>
__device__ __forceinline__ void dma16(const u32x4& rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  const u32x4 r = {(uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[0]),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[1]),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[2]),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[3])};
  const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr);
  const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(l), "v"(voff), "s"(r), "s"(so)
                 : "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r), "s"(so)
                 : "m0");
}

// Barrier between waves with no fence (a fence would wait for every copy)
// and compiler-level memory ordering on both sides.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(N) only (expcnt / lgkmcnt fields at their "no wait" maxima).
#define NSW_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14))
// s_waitcnt lgkmcnt(0) only.
#define NSW_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))


// ------------------------------------------------------- XCD placement ----
// Workgroups are dispatched round-robin over the 8 XCDs (XCD x receives ids
// x, x+8, x+16, ...), each with its own L2.  This bijection over [0, n) gives
// XCD x the contiguous logical range [x*q + min(x, rem), ...), q = n / 8,
// rem = n % 8, so that neighbouring logical items share one L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, rem = n & 7;
  const int x = bid & 7, idx = bid >> 3;
  return x * q + (x < rem ? x : rem) + idx;
}

// ------------------------------------------------- division by a constant ---
// Exact unsigned 32-bit division by a divisor fixed when a kernel is launched
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Figure 4.1): with l = ceil(log2 d) and
// mag = floor(2^32 (2^l - d) / d) + 1, every 32-bit n gives
//   q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0),  t = mulhi(mag, n).
// Five integer instructions instead of a division sequence.
struct FastDiv {
  uint32_t mag, sh;   // sh = min(l, 1) | max(l - 1, 0) << 8

  __host__ __device__ static FastDiv make(uint32_t d) {
    FastDiv f;
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    f.mag = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    f.sh = (l < 1 ? l : 1) | ((l > 0 ? l - 1 : 0) << 8);
    return f;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint32_t t = (uint32_t)(((uint64_t)mag * n) >> 32);
    return (t + ((n - t) >> (sh & 0xff))) >> (sh >> 8);
  }
};

// ------------------------------------------------------- window geometry ----
// Window-ordered row m of the [B*nW, T*ws0*ws1, C] matrix <-> token of the
// [B, T, H, W, C] image, with the cyclic shift folded in:
//   row m = ((b*nW + i*nwb + j)*T + t)*wa + r*ws1 + c
//   token = ((b*T + t)*H + (i*ws0 + r + s0) mod H)*W + (j*ws1 + c + s1) mod W
// (roll by -shift, window_partition; the inverse is window_reverse followed by
//  the roll by +shift).  Rows and tokens are below 2^31 (checked at launch),
// so the maps run in 32-bit arithmetic with the divisions by constants.
struct WinGeom {
  int B, T, H, W, ws0, ws1, s0, s1;
  int nhb, nwb, nW, wa, L;  // bands, windows per band, windows per image, ws0*ws1, T*wa
  FastDiv dL, dwa, dws0, dws1, dnW, dnwb, dHW, dW, dT;

  __host__ __device__ static WinGeom make(int B, int T, int H, int W, int ws0, int ws1, int s0, int s1) {
    WinGeom g;
    g.B = B; g.T = T; g.H = H; g.W = W; g.ws0 = ws0; g.ws1 = ws1;
    // normalise shifts into [0, H) / [0, W)
    g.s0 = ((s0 % H) + H) % H;
    g.s1 = ((s1 % W) + W) % W;
    g.nhb = H / ws0; g.nwb = W / ws1; g.nW = g.nhb * g.nwb; g.wa = ws0 * ws1; g.L = T * g.wa;
    g.dL = FastDiv::make(g.L); g.dwa = FastDiv::make(g.wa); g.dws0 = FastDiv::make(ws0);
    g.dws1 = FastDiv::make(ws1); g.dnW = FastDiv::make(g.nW); g.dnwb = FastDiv::make(g.nwb);
    g.dHW = FastDiv::make((uint32_t)H * (uint32_t)W); g.dW = FastDiv::make(W); g.dT = FastDiv::make(T);
    return g;
  }

  __device__ __forceinline__ int64_t token_of_row(int64_t m) const {
    const uint32_t mu = (uint32_t)m;
    const uint32_t win = dL.div(mu);
    const uint32_t p = mu - win * (uint32_t)L;
    const uint32_t t = dwa.div(p);
    const uint32_t rr = p - t * (uint32_t)wa;
    const uint32_t r = dws1.div(rr);
    const uint32_t c = rr - r * (uint32_t)ws1;
    const uint32_t b = dnW.div(win);
    const uint32_t wi = win - b * (uint32_t)nW;
    const uint32_t i = dnwb.div(wi);
    const uint32_t j = wi - i * (uint32_t)nwb;
    int h = (int)(i * ws0 + r) + s0; if (h >= H) h -= H;
    int w = (int)(j * ws1 + c) + s1; if (w >= W) w -= W;
    return (int64_t)(((b * (uint32_t)T + t) * (uint32_t)H + (uint32_t)h) * (uint32_t)W + (uint32_t)w);
  }

  __device__ __forceinline__ int64_t row_of_token(int64_t tok) const { return row_of_token_shift(tok, s0, s1); }

  // Window-ordered row m of this geometry -> the row of the same token in
  // the window order of the image rolled by (sa, sb) instead of (s0, s1),
  // with dh = (s0 - sa) mod H, dw = (s1 - sb) mod W: the token's rolled
  // position moves by (dh, dw), so row_of_token_shift(token_of_row(m), sa,
  // sb) without forming the token (7 divisions by constants instead of 10).
  __device__ __forceinline__ int64_t row_of_row_shift(int64_t m, int dh, int dw) const {
    const uint32_t mu = (uint32_t)m;
    const uint32_t win = dL.div(mu);
    const uint32_t p = mu - win * (uint32_t)L;
    const uint32_t t = dwa.div(p);
    const uint32_t rr = p - t * (uint32_t)wa;
    const uint32_t r = dws1.div(rr);
    const uint32_t c = rr - r * (uint32_t)ws1;
    const uint32_t b = dnW.div(win);
    const uint32_t wi = win - b * (uint32_t)nW;
    const uint32_t i = dnwb.div(wi);
    const uint32_t j = wi - i * (uint32_t)nwb;
    int h = (int)(i * ws0 + r) + dh; if (h >= H) h -= H;
    int w = (int)(j * ws1 + c) + dw; if (w >= W) w -= W;
    const uint32_t i2 = dws0.div((uint32_t)h), r2 = (uint32_t)h - i2 * (uint32_t)ws0;
    const uint32_t j2 = dws1.div((uint32_t)w), c2 = (uint32_t)w - j2 * (uint32_t)ws1;
    const uint32_t win2 = b * (uint32_t)nW + i2 * (uint32_t)nwb + j2;
    return (int64_t)((win2 * (uint32_t)T + t) * (uint32_t)wa + r2 * (uint32_t)ws1 + c2);
  }

  // row_of_token of the same geometry rolled by (sa, sb) in [0, H) x [0, W)
  // instead of (s0, s1): the window order of another block of the image.
  __device__ __forceinline__ int64_t row_of_token_shift(int64_t tok, int sa, int sb) const {
    const uint32_t tu = (uint32_t)tok;
    const uint32_t bt = dHW.div(tu);
    const uint32_t hw = tu - bt * (uint32_t)H * (uint32_t)W;
    const uint32_t h = dW.div(hw);
    const uint32_t w = hw - h * (uint32_t)W;
    const uint32_t b = dT.div(bt);
    const uint32_t t = bt - b * (uint32_t)T;
    int hs = (int)h - sa; if (hs < 0) hs += H;
    int wsft = (int)w - sb; if (wsft < 0) wsft += W;
    const uint32_t i = dws0.div((uint32_t)hs), r = (uint32_t)hs - i * (uint32_t)ws0;
    const uint32_t j = dws1.div((uint32_t)wsft), c = (uint32_t)wsft - j * (uint32_t)ws1;
    const uint32_t win = b * (uint32_t)nW + i * (uint32_t)nwb + j;
    return (int64_t)((win * (uint32_t)T + t) * (uint32_t)wa + r * (uint32_t)ws1 + c);
  }
};

}  // namespace nsw
