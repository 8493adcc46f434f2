// Window attention core: o = softmax(q k^T * scale + mask) v per (window, head)
// (the F.scaled_dot_product_attention call of models/swin_helpers.py:247).
//
// bf16, head dim 64, 9 x 18 windows, shift mask from indices or none
// (attn_dma_kernel, the model's case): K and V rows are copied straight into
// LDS and V^T fragments come from transposing LDS reads (see below the
// direct-to-LDS section); the per-block arithmetic is that of
// attn_mfma_kernel, in the same order, so the two give identical bits.
//
// bf16 path (attn_mfma_kernel, other head dims and window sizes, mask
// tensors): one 256-thread workgroup per (window, head).
// K [keys x hd] and V^T [hd x keys] of the window are staged in LDS (zero
// padded to a multiple of 32 keys).  Each wavefront takes 16-query blocks and
//   1. computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16, so that lane l
//      holds the logits of query l%16 for keys 16*kb + 4*(l/16) + r;
//   2. adds the additive mask (the reference's latitude shift mask, taken
//      from a per-window key-class bit set built with one ballot per 64 keys,
//      or a materialised mask), does the softmax in the exp2 domain (row max
//      by permlane reduction, row sum by the PV MFMA against a ones block);
//   3. reuses the probability registers directly as the B operand of
//      O^T = V^T P^T (the k order of a 32-key step is {4g+r, 16+4g+r} for lane
//      group g; V^T is stored with its keys in that order, so each A fragment
//      is one 16-byte LDS read), and
//   4. writes O[q][h*hd + d] in 16-byte chunks (lane pairs exchange halves
//      with v_permlane16_swap).
// Workgroup ids are remapped so that the heads of a window share one XCD.
// Padding keys get -inf logits; no FLOPs are counted for them.
//
// Generic path (attn_scalar_kernel, fp32 and any head dim): one thread per
// query, online softmax over 64-key chunks staged in LDS, fp32 throughout.
#include "nsw_common.h"

#include <utility>

namespace nsw {

enum MaskMode { MASK_NONE = 0, MASK_SHIFT = 1, MASK_TENSOR = 2 };

struct AttnArgs {
  const void* qkv;
  void* o;
  const float* mask;
  int nW_mask;
  int L, C, heads;
  float scale;
  int mask_mode;
  WinGeom g;
  // set by the host for attn_dma_kernel: scale * log2(e), -100 / scale (both
  // rounded as the kernels' own float expressions), the byte sizes of qkv
  // and o (below 2^31 there) and the division by heads
  float zscale, smask;
  uint32_t qkv_bytes, obytes;
  FastDiv dheads;
};

// Additive mask value for (window, query, key); key/query are tokens of the
// window's T*wa sequence.
__device__ __forceinline__ float mask_value(const AttnArgs& a, int64_t win, int q, int k,
                                            bool last_band) {
  if (a.mask_mode == MASK_SHIFT) {
    if (!last_band) return 0.f;
    const int thr = a.g.ws0 - a.g.s0;
    const int rq = (q % a.g.wa) / a.g.ws1, rk = (k % a.g.wa) / a.g.ws1;
    return ((rq >= thr) != (rk >= thr)) ? -100.0f : 0.0f;
  } else if (a.mask_mode == MASK_TENSOR) {
    const int64_t mw = win % a.nW_mask;
    return a.mask[(mw * a.L + q) * (int64_t)a.L + k];
  }
  return 0.f;
}

__device__ __forceinline__ bool window_in_last_band(const AttnArgs& a, int64_t win) {
  if (a.mask_mode != MASK_SHIFT) return false;
  const int wi = (int)(win % a.g.nW);
  return wi / a.g.nwb == a.g.nhb - 1;
}

// ------------------------------------------------------------ bf16 MFMA ----
// Column of key k in a V^T row.  Within each 32-key step the keys are stored
// in the order the probability registers hold them: lane group g carries keys
// 4g..4g+3 and 16+4g..16+4g+3, so position 8g + 4h + r holds key 16h + 4g + r
// and each lane reads its 8 V^T values with one 16-byte LDS read.
__device__ __forceinline__ int vt_pos(int k) {
  const int j = k & 31;
  return (k & ~31) | ((j & 15) >> 2) << 3 | (j >> 4) << 2 | (j & 3);
}

// 16-byte chunk slot of chunk ch in K row r (SW: 8 chunks per row, XOR
// swizzle ((r >> 1) & 7) ^ ((r & 1) << 2): the 16 rows of a fragment read, or
// two rows of 8 chunks in a staging write, cover all banks once whether LDS
// serves 16 lanes over 64 banks or 8 lanes over 32).  Depends on r mod 16
// only, so a fragment row fr can stand for kb * 16 + fr.
template <bool SW>
__device__ __forceinline__ int k_chunk(int r, int ch) { return SW ? ch ^ (((r >> 1) & 7) ^ ((r & 1) << 2)) : ch; }

// LDS row of head dim d in V^T: within each group of 8 dims the rows are
// rotated by the group index, so that the staging writes of one instruction
// (lane = 16-byte chunk ch of a key row, element e: dim 8 ch + e) land in
// different banks; a fragment read (16 consecutive dims) still covers 16
// distinct rows of the same 8-row groups, conflict-free as before.
__device__ __forceinline__ int vt_row(int d) { return (d & ~7) | ((d + (d >> 3)) & 7); }

// NKB = ceil(L / 16) exactly, so only the last 16-key block holds padding.
template <int HD, int NKB, bool MT>
__global__ __launch_bounds__(256, 3) void attn_mfma_kernel(AttnArgs a) {
  constexpr int KP = ((NKB * 16 + 31) / 32) * 32;  // padded keys (multiple of 32)
  // 128-byte K rows (hd 64) are stored unpadded with XOR-swizzled 16-byte
  // chunks (conflict-free staging writes and fragment reads); 64-byte rows
  // (hd 32) are padded by 16 bytes
  constexpr bool KSW = HD == 64;
  constexpr int KS_STRIDE = KSW ? HD : HD + 8;     // bf16 elements per K row in LDS
  constexpr int VT_STRIDE = KP + 8;                // bf16 elements per V^T row (4 banks mod 64 dwords)
  constexpr int NS = HD / 32;                      // k-steps of the QK^T product
  constexpr int NDB = HD / 16;                     // 16-wide head-dim blocks
  static_assert(NDB % 2 == 0, "output stores pair 16-wide head-dim blocks");
  constexpr int NKS = KP / 32;                     // 32-key steps of PV
  constexpr int CPR = HD / 8;                      // 16-byte chunks per K / V row
  constexpr int NCH = (KP * CPR + 255) / 256;      // chunks staged per thread
  constexpr int NCLS = (KP + 63) / 64;             // 64-bit words of the key-class set
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ __attribute__((aligned(16))) bf16 Ks[KP * KS_STRIDE];
  __shared__ __attribute__((aligned(16))) bf16 Vt[HD * VT_STRIDE];
  __shared__ uint64_t cls[NCLS];

  // The heads of a window run on one XCD at about the same time, so that the
  // window's qkv rows and output rows are read and written whole there.
  const int item = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int win = item / a.heads;
  const int head = item - win * a.heads;
  const int L = a.L, C = a.C;
  const int64_t ld = 3 * (int64_t)C;
  const bf16* base = (const bf16*)a.qkv + (int64_t)win * L * ld + head * HD;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;

  // Q fragments of all of this wave's query blocks (wave, wave + 4, ...),
  // issued before the staging so that their latency overlaps it.
  constexpr int QPW = (NKB + 3) / 4;
  bf16x8 qf[QPW][NS];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int q = (wave + 4 * i) * 16 + fr;
    const int qc = q < L ? q : L - 1;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[i][s] = *reinterpret_cast<const bf16x8*>(base + qc * ld + 32 * s + 8 * fg);
  }

  // ---- stage K and V^T (zero padded): all loads first, then the LDS stores
  bf16x8 kv[NCH], vv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int idx = tid + 256 * c;
    const int key = idx / CPR, ch = idx - key * CPR;
    if (idx < KP * CPR && key < L) {
      const bf16* rowp = base + key * ld + ch * 8;
      kv[c] = *reinterpret_cast<const bf16x8*>(rowp + C);
      vv[c] = *reinterpret_cast<const bf16x8*>(rowp + 2 * C);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { kv[c][e] = (bf16)0.f; vv[c][e] = (bf16)0.f; }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int idx = tid + 256 * c;
    const int key = idx / CPR, ch = idx - key * CPR;
    if (idx < KP * CPR) {
      *reinterpret_cast<bf16x8*>(&Ks[key * KS_STRIDE + k_chunk<KSW>(key, ch) * 8]) = kv[c];
      const int kpos = vt_pos(key);
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[vt_row(ch * 8 + e) * VT_STRIDE + kpos] = vv[c][e];
    }
  }
  // Shift mask of a last-band window: key class = (row within the window)
  // >= ws0 - s0; a query attends with -100 to keys of the other class.
  const bool shifted = !MT && window_in_last_band(a, win);
  if (shifted && wave == 0) {
    const int thr = (a.g.ws0 - a.g.s0) * a.g.ws1;
#pragma unroll
    for (int w = 0; w < NCLS; ++w) {
      const int key = 64 * w + lane;
      const uint64_t b = __ballot(key < L && (key % a.g.wa) >= thr);
      if (lane == 0) cls[w] = b;
    }
  }
  __syncthreads();

  // Additive masks are applied to the raw q.k products as mask / scale, so
  // that one FMA per logit, p = exp2(s * scale*log2(e) - max), finishes it.
  const float zscale = a.scale * LOG2E;
  const float smask = -100.0f / a.scale;

#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int qb = wave + 4 * i;
    if (qb >= NKB) break;
    const int q = qb * 16 + fr;
    const int qc = q < L ? q : L - 1;
    // S^T = K Q^T; K fragments run KD 16-key blocks ahead of the MFMAs
    constexpr int KD = NKB < 4 ? NKB : 4;
    f32x4 S[NKB];
    bf16x8 kf[KD][NS];
#pragma unroll
    for (int kb = 0; kb < KD; ++kb)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        kf[kb][s] = *reinterpret_cast<const bf16x8*>(&Ks[(kb * 16 + fr) * KS_STRIDE + k_chunk<KSW>(fr, 4 * s + fg) * 8]);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) S[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb % KD][s], qf[i][s], S[kb], 0, 0, 0);
      if (kb + KD < NKB) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
          kf[kb % KD][s] = *reinterpret_cast<const bf16x8*>(
              &Ks[((kb + KD) * 16 + fr) * KS_STRIDE + k_chunk<KSW>(fr, 4 * s + fg) * 8]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // lane: query fr, keys 16*kb + 4*fg + r
    if constexpr (MT) {
      const float* mrow = a.mask + ((int64_t)(win % a.nW_mask) * L + qc) * (int64_t)L;
      const float inv_scale = 1.0f / a.scale;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb * 16 + 4 * fg + r;
          if (kb < NKB - 1 || key < L) S[kb][r] += mrow[key] * inv_scale;
        }
    } else if (shifted) {
      const int qcls = (int)((cls[qc >> 6] >> (qc & 63)) & 1);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const unsigned bits = (unsigned)(cls[kb >> 2] >> (16 * (kb & 3) + 4 * fg)) & 0xFu;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((int)((bits >> r) & 1u) != qcls) S[kb][r] += smask;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if ((NKB - 1) * 16 + 4 * fg + r >= L) S[NKB - 1][r] = -INFINITY;
    float mx = S[0][0];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[kb][r]);
    mx = rows4_max(mx);
    const float off = -mx * zscale;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[kb][r] = __builtin_amdgcn_exp2f(fmaf(S[kb][r], zscale, off));

    // O^T = V^T P^T; V^T fragments double-buffered across 32-key steps.  An
    // extra all-ones A block gives the row sums of the (bf16) probabilities
    // on every lane of the query, the same values that weight V.
    f32x4 O[NDB], Z = {0.f, 0.f, 0.f, 0.f};
    const bf16x8 ones = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};
#pragma unroll
    for (int db = 0; db < NDB; ++db) O[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 vf[2][NDB];
    auto load_v = [&](int buf, int ks) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        vf[buf][db] = *reinterpret_cast<const bf16x8*>(&Vt[vt_row(db * 16 + fr) * VT_STRIDE + 32 * ks + 8 * fg]);
    };
    load_v(0, 0);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks + 1 < NKS) load_v((ks + 1) & 1, ks + 1);
      bf16x8 pf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pf[r] = (bf16)S[2 * ks][r];
        pf[4 + r] = (2 * ks + 1 < NKB) ? (bf16)S[2 * ks + 1][r] : (bf16)0.f;
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        O[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[ks & 1][db], pf, O[db], 0, 0, 0);
      }
      Z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, Z, 0, 0, 0);
    }
    // Lane (fr, fg) holds dims 16 db + 4 fg .. +3 of query fr.  A
    // v_permlane16_swap of (db = 2j, db = 2j+1) pairs lane groups fg = 2m and
    // 2m+1: afterwards the even group holds dims 16 db + 8m .. +7 of db = 2j
    // and the odd group those of db = 2j+1, so every lane writes 16 B chunks.
    const float inv = __builtin_amdgcn_rcpf(Z[0]);
    float lo[NDB / 2][2], hi[NDB / 2][2];
#pragma unroll
    for (int j = 0; j < NDB / 2; ++j) {
      const bf16x4 e = {(bf16)(O[2 * j][0] * inv), (bf16)(O[2 * j][1] * inv), (bf16)(O[2 * j][2] * inv),
                        (bf16)(O[2 * j][3] * inv)};
      const bf16x4 f = {(bf16)(O[2 * j + 1][0] * inv), (bf16)(O[2 * j + 1][1] * inv),
                        (bf16)(O[2 * j + 1][2] * inv), (bf16)(O[2 * j + 1][3] * inv)};
      const f32x2 ev = __builtin_bit_cast(f32x2, e), fv = __builtin_bit_cast(f32x2, f);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        lo[j][h] = ev[h];
        hi[j][h] = fv[h];
        permlane16_swap(lo[j][h], hi[j][h]);
      }
    }
    if (q < L) {
      bf16* orow = (bf16*)a.o + ((int64_t)win * L + q) * (int64_t)C + head * HD + 8 * (fg >> 1) + 16 * (fg & 1);
#pragma unroll
      for (int j = 0; j < NDB / 2; ++j)
        *reinterpret_cast<f32x4*>(orow + 32 * j) = f32x4{lo[j][0], lo[j][1], hi[j][0], hi[j][1]};
    }
  }
}

// ------------------------------------------- bf16 MFMA, direct-to-LDS ----
// K and V rows of a (window, head) item are copied straight into LDS with
// buffer_load ... lds, row-major (128 B per row for head dim 64), their
// 16-byte chunks XOR-swizzled by row (K: sw_chunk, conflict-free fragment
// reads, as k_chunk; V: v_chunk, below).  The PV product reads its V^T fragments with
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4
// of the 4-element vectors addressed by lanes i/4, 4 + i/4, 8 + i/4 and
// 12 + i/4, so lanes addressing rows 4g + i/4 at dims 16 db + 4 (i%4) yield
// column 16 db + i of rows 4g .. 4g+3; two such reads per 16-dim block give
// keys {4g+r, 16+4g+r}, the key order of the probability registers.
__device__ __forceinline__ int sw_chunk(int row, int ch) {
  return ch ^ (((row >> 1) & 7) ^ ((row & 1) << 2));
}

// Chunk placement of the V rows.  A transposing read of the PV product
// covers, per 32-lane half of the wave, 8 consecutive rows 8i .. 8i + 7 at
// the two chunks 2 db, 2 db + 1 (per 16-lane quarter, 4 consecutive rows).
// Rows of equal parity share the 128-byte bank half, so chunk c of row r
// sits at c ^ 2 f(r), f(r) = ((r >> 1) & 3) ^ 2 (r & 1): f is distinct on
// the four rows of either parity in 8 consecutive rows and on 4 consecutive
// rows, so both halves' and all quarters' 16 chunk pairs fall in distinct
// banks (with sw_chunk the even rows 2 apart collided: 2-way conflicts on
// every V^T read).
__device__ __forceinline__ int v_chunk(int row, int ch) {
  return ch ^ (2 * (((row >> 1) & 3) ^ ((row & 1) << 1)));
}

// The resource built from kernel arguments, pinned to SGPRs (the inline asm
// operands below require scalar registers).
__device__ __forceinline__ u32x4 uniform_rsrc(const void* p, uint32_t bytes) {
  const u32x4 r = make_rsrc(p, bytes);
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)r[0]), (uint32_t)__builtin_amdgcn_readfirstlane((int)r[1]),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)r[2]), (uint32_t)__builtin_amdgcn_readfirstlane((int)r[3])};
}

// 16-byte store from inline asm.  A VALU write to the data VGPRs of a 16-byte
// store needs 2 wait states after the store on gfx950; the compiler cannot
// see the store inside the asm, so the s_nop provides them.
__device__ __forceinline__ void store16_asm(const u32x4& rsrc, uint32_t voff, const f32x4& v) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen\n\ts_nop 1" : : "v"(v), "v"(voff), "s"(rsrc) : "memory");
}

// One 16-query block of a (window, head) item with head dim 64: K rows and V
// rows (KP of each, 128 B per row, 16-byte chunks placed by sw_chunk / v_chunk) in LDS,
// V rows past L zero (so that their zero probabilities give exact zeros), the
// block's Q fragments in registers.  Computes S^T = K Q^T, the masked
// softmax in the exp2 domain (row max by permlane reduction, row sums by an
// MFMA against a ones block), O^T = V^T P^T with V^T fragments from
// ds_read_b64_tr_b16, and stores the block's rows of o (NDB / 2 16-byte
// stores per lane, issued from inline asm; queries past L go to offset
// obytes, past the end of o, where they are dropped).
template <int NKB, bool SHIFTED>
__device__ __forceinline__ void attn_qblock64(const AttnArgs& a, const char* Ks, const char* Vs, const bf16x8 (&qf)[2],
                                              int q, uint32_t win, int head, const uint64_t* cls,
                                              const u32x4& ro, int fr, int fg) {
  constexpr int HD = 64;
  constexpr int KP = ((NKB * 16 + 31) / 32) * 32;
  constexpr int NS = HD / 32, NDB = HD / 16, NKS = KP / 32;
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_s4;
  const int L = a.L, C = a.C;
  const int qc = q < L ? q : L - 1;
  const float zscale = a.zscale;
  const float smask = a.smask;
  const uint32_t obytes = a.obytes;
  const bf16x8 ones = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};
  // S^T = K Q^T, K fragments KD blocks ahead
  constexpr int KD = NKB < 4 ? NKB : 4;
  f32x4 S[NKB];
  bf16x8 kf[KD][NS];
#pragma unroll
  for (int kb = 0; kb < KD; ++kb)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int r = kb * 16 + fr;
      kf[kb][s] = *reinterpret_cast<const bf16x8*>(Ks + r * 128 + sw_chunk(r, 4 * s + fg) * 16);
    }
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) S[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb % KD][s], qf[s], S[kb], 0, 0, 0);
    if (kb + KD < NKB) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int r = (kb + KD) * 16 + fr;
        kf[kb % KD][s] = *reinterpret_cast<const bf16x8*>(Ks + r * 128 + sw_chunk(r, 4 * s + fg) * 16);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // lane: query fr, keys 16 kb + 4 fg + r
  if constexpr (SHIFTED) {
    const int qcls = (int)((cls[qc >> 6] >> (qc & 63)) & 1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const unsigned bits = (unsigned)(cls[kb >> 2] >> (16 * (kb & 3) + 4 * fg)) & 0xFu;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if ((int)((bits >> r) & 1u) != qcls) S[kb][r] += smask;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if ((NKB - 1) * 16 + 4 * fg + r >= L) S[NKB - 1][r] = -INFINITY;
  float mx = S[0][0];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[kb][r]);
  mx = rows4_max(mx);
  const float off = -mx * zscale;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[kb][r] = __builtin_amdgcn_exp2f(fmaf(S[kb][r], zscale, off));

  // O^T = V^T P^T: V^T fragments of 32-key step ks from two transposed
  // reads (keys 32ks + 4fg + 0..3 and 32ks + 16 + 4fg + 0..3, dim 16db + fr)
  f32x4 O[NDB], Z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int db = 0; db < NDB; ++db) O[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 vf[2][NDB];
  auto load_v = [&](int b, int ks) {
    const int r0 = 32 * ks + 4 * fg + fr / 4;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int lc = 2 * db + (fr & 3) / 2;
      const int half = (fr & 1) * 8;
      const i16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s4*)(Vs + r0 * 128 + v_chunk(r0, lc) * 16 + half));
      const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s4*)(Vs + (r0 + 16) * 128 + v_chunk(r0 + 16, lc) * 16 + half));
      const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo4), h4 = __builtin_bit_cast(bf16x4, hi4);
      vf[b][db] = bf16x8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    }
  };
  load_v(0, 0);
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (ks + 1 < NKS) load_v((ks + 1) & 1, ks + 1);
    bf16x8 pf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pf[r] = (bf16)S[2 * ks][r];
      pf[4 + r] = (2 * ks + 1 < NKB) ? (bf16)S[2 * ks + 1][r] : (bf16)0.f;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) O[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[ks & 1][db], pf, O[db], 0, 0, 0);
    Z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, Z, 0, 0, 0);
  }
  // 16-byte pieces after pairing head-dim blocks (as attn_mfma_kernel);
  // queries past L (and whole padding blocks) go to an offset past the
  // end of o, where the store is dropped
  const float inv = __builtin_amdgcn_rcpf(Z[0]);
  static_assert(NDB == 4, "two 64-byte halves per row");
  f32x4 ch[2];
#pragma unroll
  for (int j = 0; j < NDB / 2; ++j) {
    const bf16x4 e = {(bf16)(O[2 * j][0] * inv), (bf16)(O[2 * j][1] * inv), (bf16)(O[2 * j][2] * inv),
                      (bf16)(O[2 * j][3] * inv)};
    const bf16x4 f = {(bf16)(O[2 * j + 1][0] * inv), (bf16)(O[2 * j + 1][1] * inv),
                      (bf16)(O[2 * j + 1][2] * inv), (bf16)(O[2 * j + 1][3] * inv)};
    const f32x2 ev = __builtin_bit_cast(f32x2, e), fv = __builtin_bit_cast(f32x2, f);
    float l0 = ev[0], l1 = ev[1], h0 = fv[0], h1 = fv[1];
    permlane16_swap(l0, h0);
    permlane16_swap(l1, h1);
    ch[j] = f32x4{l0, l1, h0, h1};
  }
  // lanes fr and fr ^ 8 trade halves (DPP row_ror:8 within each 16-lane
  // row), so that each store instruction writes 8 whole 128-byte rows
  // (first the block's queries 0-7, then 8-15) instead of 64-byte halves
  // of 16: bit-identical, 0.7% / 2.3% faster at configs 2 / 4.  Four
  // separate v_mov_dpp: the vector form of update_dpp was merged into one.
  const bool lo = fr < 8;
  const int s0 = __builtin_bit_cast(int, lo ? ch[1][0] : ch[0][0]);
  const int s1 = __builtin_bit_cast(int, lo ? ch[1][1] : ch[0][1]);
  const int s2 = __builtin_bit_cast(int, lo ? ch[1][2] : ch[0][2]);
  const int s3 = __builtin_bit_cast(int, lo ? ch[1][3] : ch[0][3]);
  const f32x4 recv = {__builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(s0, 0x128, 0xF, 0xF, false)),
                      __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(s1, 0x128, 0xF, 0xF, false)),
                      __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(s2, 0x128, 0xF, 0xF, false)),
                      __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(s3, 0x128, 0xF, 0xF, false))};
  const int q0 = q - fr;                               // the block's first query
  const uint32_t cb = (uint32_t)(head * HD + 8 * (fg >> 1) + 16 * (fg & 1)) * 2u + (lo ? 0u : 64u);
  const int qa = q0 + (fr & 7), qb = q0 + 8 + (fr & 7);
  const uint32_t oa = (((uint32_t)win * (uint32_t)L + (uint32_t)qa) * (uint32_t)C) * 2u + cb;
  const uint32_t ob = (((uint32_t)win * (uint32_t)L + (uint32_t)qb) * (uint32_t)C) * 2u + cb;
  store16_asm(ro, qa < L ? oa : obytes, lo ? ch[0] : recv);
  store16_asm(ro, qb < L ? ob : obytes, lo ? recv : ch[1]);
}

// One workgroup per (window, head) item, head dim 64, shift mask from indices
// or none (three workgroups per CU).  K and V rows go straight to LDS with
// buffer_load ... lds (row-major, chunks placed by sw_chunk / v_chunk: no VGPR staging,
// no transposing LDS writes); each wave's Q fragments are loaded into
// registers alongside.  Waves take query blocks wave, wave + 4, ...
template <int NKB>
__global__ __launch_bounds__(256, 3) void attn_dma_kernel(AttnArgs a) {
  constexpr int HD = 64;
  constexpr int KP = ((NKB * 16 + 31) / 32) * 32;
  constexpr int PART = KP * 128;
  constexpr int RG = KP / 8;
  static_assert((2 * RG) % 4 == 0, "copies split evenly over 4 waves");
  constexpr int NDMA = 2 * RG / 4;
  static_assert(RG % NDMA == 0, "each wave's copies lie in one of K and V");
  constexpr int QPW = (NKB + 3) / 4;
  constexpr int NS = HD / 32, NCLS = (KP + 63) / 64;
  __shared__ __attribute__((aligned(1024))) char smem[2 * PART];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int L = a.L, C = a.C;
  const uint32_t ld = 3u * (uint32_t)C;
  const uint32_t item = (uint32_t)xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const uint32_t win = a.dheads.div(item);
  const int head = (int)(item - win * (uint32_t)a.heads);
  const u32x4 rq = uniform_rsrc(a.qkv, a.qkv_bytes);
  const u32x4 ro = uniform_rsrc(a.o, a.obytes);

  // Q fragments of this wave's query blocks (rows past L re-read row L - 1)
  const bf16* base = (const bf16*)a.qkv + ((size_t)win * (uint32_t)L * ld + (uint32_t)head * HD);
  bf16x8 qf[QPW][NS];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int q = (wave + 4 * i) * 16 + fr;
    const int qc = q < L ? q : L - 1;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[i][s] = *reinterpret_cast<const bf16x8*>(base + qc * ld + 32 * s + 8 * fg);
  }
  // K rows to [0, PART), V rows to [PART, 2 PART): copy j of this wave is
  // 8-row group d = wave * NDMA + j, all of one part (K for waves 0 and 1).
  // Lane l copies chunk l % 8 of row 8 rg + l / 8; the row's chunk placement
  // depends on row % 16 (K) or row % 8 (V), so each lane has two K offsets
  // (even and odd groups) and one V offset, and a copy adds the group's row
  // offset, a scalar.
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const uint32_t soff = (win * (uint32_t)L * ld + (uint32_t)head * HD) * 2u;
  const int part = wave * NDMA / RG;                  // uniform
  const int rg0 = wave * NDMA - part * RG;
  const int lrow = lane >> 3;
  const uint32_t lbase = ((uint32_t)lrow * ld + (uint32_t)(part + 1) * (uint32_t)C) * 2u;
  const uint32_t gstride = 8u * ld * 2u;              // bytes per 8-row group
  const uint32_t lds0 = sbase + (uint32_t)(part * PART + rg0 * 1024);
  if (part == 0) {
    const uint32_t e0 = lbase + (uint32_t)sw_chunk(lrow, lane & 7) * 16u;
    const uint32_t e1 = lbase + (uint32_t)sw_chunk(8 + lrow, lane & 7) * 16u;
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
      const int rg = rg0 + j;
      dma16(rq, lds0 + (uint32_t)j * 1024u, ((rg & 1) ? e1 : e0) + (uint32_t)rg * gstride, soff);
    }
  } else {
    const uint32_t e = lbase + (uint32_t)v_chunk(lrow, lane & 7) * 16u;
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
      const int rg = rg0 + j;
      // V rows past L read from offset qkv_bytes, past the end of qkv: the
      // range check returns zeros, which land in LDS as the padding rows
      const uint32_t voff = rg * 8 + lrow < L ? e + (uint32_t)rg * gstride : a.qkv_bytes;
      dma16(rq, lds0 + (uint32_t)j * 1024u, voff, soff);
    }
  }

  // the key-class bit sets of the shift mask (last band of windows only)
  bool shifted = false;
  uint64_t cls[NCLS];
#pragma unroll
  for (int w = 0; w < NCLS; ++w) cls[w] = 0;
  if (a.mask_mode == MASK_SHIFT) {
    const uint32_t wi = win - a.g.dnW.div(win) * (uint32_t)a.g.nW;
    shifted = (int)a.g.dnwb.div(wi) == a.g.nhb - 1;
  }
  if (shifted) {
    const int thr = (a.g.ws0 - a.g.s0) * a.g.ws1;
#pragma unroll
    for (int w = 0; w < NCLS; ++w) {
      const uint32_t key = 64u * w + (uint32_t)lane;
      const uint32_t r = key - a.g.dwa.div(key) * (uint32_t)a.g.wa;
      cls[w] = __ballot(key < (uint32_t)L && (int)r >= thr);
    }
  }
  NSW_WAIT_VMCNT(0);
  wg_barrier();

  if (shifted) {
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int qb = wave + 4 * i;
      if (qb >= NKB) break;
      attn_qblock64<NKB, true>(a, smem, smem + PART, qf[i], qb * 16 + fr, win, head, cls, ro, fr, fg);
    }
  } else {
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int qb = wave + 4 * i;
      if (qb >= NKB) break;
      attn_qblock64<NKB, false>(a, smem, smem + PART, qf[i], qb * 16 + fr, win, head, cls, ro, fr, fg);
    }
  }
}

// ---------------------------------------------------------- fp32 MFMA ----
// fp32 (the reference's inference precision), head dim 64, 9 x 18 windows,
// shift mask from indices or none: one 512-thread workgroup per (window,
// head).  K and V rows (256 B of fp32) are copied straight into LDS with
// their 16-byte chunks XOR-swizzled by row: K chunk c of row r at
// c ^ (r & 15) (a fragment read, 16 rows x one chunk, covers every bank), V
// chunk c at c ^ (((r >> 2) & 3) << 2) (the rows 16kb + 4g + r' that lane
// groups g read in one PV step fall in different 64-byte bank groups).  With
// v_mfma_f32_16x16x4_f32:
//   S^T = K Q^T: four MFMAs per 16-byte K fragment (instruction e takes head
//     dims 16s + 4g + e from lane group g), so lane (i, g) holds the logits of
//     query i for keys 16kb + 4g + r as in the bf16 kernels, and the mask and
//     exp2-domain softmax are theirs (probabilities stay fp32);
//   O^T = V^T P^T: for key step (kb, r) lane (i, g) supplies V[16kb + 4g + r]
//     [16db + i] (A) and its own probability for key 16kb + 4g + r (B);
//   row sums of P on the VALU (lane sums, then across the four lane groups).
// Lane (i, g) ends with O[query i][16db + 4g .. +3]: one 16-byte store per
// dim block.  The eight waves (two per SIMD) take query blocks w and w + 8.
// Key rows past L are zero-filled by the copies' range check (V) or masked to
// -inf (K).
template <int NKB>
__global__ __launch_bounds__(512, 1) void attn_f32_kernel(AttnArgs a, int nitems) {
  constexpr int HD = 64;
  constexpr int KR = NKB * 16;                  // rows of K and of V in LDS
  constexpr int PART = KR * HD * 4;
  constexpr int NW = 8;
  constexpr int RG = KR / 4;                    // 4-row copies per part
  static_assert((2 * RG) % NW == 0, "copies split evenly over the waves");
  constexpr int NDMA = 2 * RG / NW;
  constexpr int QPW = (NKB + NW - 1) / NW;
  constexpr int NS = HD / 16, NDB = HD / 16, NCLS = (KR + 63) / 64;
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ __attribute__((aligned(1024))) char smem[2 * PART];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int L = a.L, C = a.C;
  const uint32_t ld = 3u * (uint32_t)C;
  const int item = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int win = item / a.heads, head = item - win * a.heads;
  const uint32_t qkv_bytes = (uint32_t)((uint64_t)nitems / a.heads * L * ld * 4u);
  const u32x4 rq = uniform_rsrc(a.qkv, qkv_bytes);

  // K rows to [0, PART), V rows to [PART, 2 PART)
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const uint32_t soff = ((uint32_t)win * (uint32_t)L * ld + (uint32_t)head * HD) * 4u;
#pragma unroll
  for (int j = 0; j < NDMA; ++j) {
    const int d = wave * NDMA + j;
    const int part = d / RG, rg = d - part * RG;
    const int row = rg * 4 + lane / 16;
    const int sw = part == 0 ? (row & 15) : (((row >> 2) & 3) << 2);
    const int c = (lane % 16) ^ sw;
    const uint32_t voff = part == 1 && row >= L
                              ? qkv_bytes
                              : ((uint32_t)row * ld + (uint32_t)(part + 1) * (uint32_t)C) * 4u + (uint32_t)c * 16u;
    dma16(rq, sbase + (uint32_t)(part * PART + rg * 1024), voff, soff);
  }

  const bool shifted = window_in_last_band(a, win);
  uint64_t cls[NCLS];
  {
    const int thr = shifted ? (a.g.ws0 - a.g.s0) * a.g.ws1 : 0;
    const int wa = shifted ? a.g.wa : 1;
#pragma unroll
    for (int w = 0; w < NCLS; ++w) {
      const int key = 64 * w + lane;
      cls[w] = __ballot(shifted && key < L && (key % wa) >= thr);
    }
  }
  NSW_WAIT_VMCNT(0);
  wg_barrier();

  const float* base = (const float*)a.qkv + (int64_t)win * L * ld + head * HD;
  const char* Ks = smem;
  const char* Vs = smem + PART;
  const float zscale = a.scale * LOG2E;
  const float smask = -100.0f / a.scale;
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int qb = wave + NW * i;
    if (qb >= NKB) break;
    const int q = qb * 16 + fr;
    const int qc = q < L ? q : L - 1;
    f32x4 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = *reinterpret_cast<const f32x4*>(base + (int64_t)qc * ld + 16 * s + 4 * fg);
    // S^T = K Q^T
    f32x4 S[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r = kb * 16 + fr;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(Ks + r * (HD * 4) + (((4 * s + fg) ^ (r & 15)) * 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[e], qf[s][e], S[kb], 0, 0, 0);
      }
    }
    // lane: query fr, keys 16 kb + 4 fg + r
    if (shifted) {
      const int qcls = (int)((cls[qc >> 6] >> (qc & 63)) & 1);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const unsigned bits = (unsigned)(cls[kb >> 2] >> (16 * (kb & 3) + 4 * fg)) & 0xFu;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((int)((bits >> r) & 1u) != qcls) S[kb][r] += smask;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if ((NKB - 1) * 16 + 4 * fg + r >= L) S[NKB - 1][r] = -INFINITY;
    float mx = S[0][0];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[kb][r]);
    mx = rows4_max(mx);
    const float off = -mx * zscale;
    float zl = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        S[kb][r] = __builtin_amdgcn_exp2f(fmaf(S[kb][r], zscale, off));
        zl += S[kb][r];
      }
    const float z = rows4_sum(zl);
    // O^T = V^T P^T
    f32x4 O[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) O[db] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = kb * 16 + 4 * fg + r;
        const char* vr = Vs + row * (HD * 4) + (fr & 3) * 4;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const float v = *reinterpret_cast<const float*>(vr + (((4 * db + fr / 4) ^ (fg << 2)) * 16));
          O[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(v, S[kb][r], O[db], 0, 0, 0);
        }
      }
    if (q < L) {
      const float inv = 1.0f / z;
      float* orow = (float*)a.o + ((int64_t)win * L + q) * (int64_t)C + head * HD + 4 * fg;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        *reinterpret_cast<f32x4*>(orow + 16 * db) =
            f32x4{O[db][0] * inv, O[db][1] * inv, O[db][2] * inv, O[db][3] * inv};
    }
  }
}

// ------------------------------------------------------- generic (fp32) ----
template <typename T, int HD>
__global__ __launch_bounds__(256) void attn_scalar_kernel(AttnArgs a) {
  constexpr int KC = 64;  // keys per LDS chunk
  __shared__ float Kc[KC][HD];
  __shared__ float Vc[KC][HD];
  const int64_t win = blockIdx.x / a.heads;
  const int head = blockIdx.x - (int)(win * a.heads);
  const int L = a.L, C = a.C;
  const int64_t ld = 3 * (int64_t)C;
  const T* base = (const T*)a.qkv + win * L * ld;
  const bool last_band = window_in_last_band(a, win);
  const int tid = threadIdx.x;

  for (int q0 = 0; q0 < L; q0 += 256) {
    const int q = q0 + tid;
    const bool active = q < L;
    const int qc = active ? q : L - 1;
    float qv[HD], acc[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) {
      qv[d] = to_f32(base[qc * ld + head * HD + d]) * a.scale;
      acc[d] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int k0 = 0; k0 < L; k0 += KC) {
      __syncthreads();
      for (int idx = tid; idx < KC * HD; idx += 256) {
        const int kk = idx / HD, d = idx - kk * HD;
        const int key = k0 + kk;
        float kv = 0.f, vv = 0.f;
        if (key < L) {
          kv = to_f32(base[key * ld + C + head * HD + d]);
          vv = to_f32(base[key * ld + 2 * C + head * HD + d]);
        }
        Kc[kk][d] = kv;
        Vc[kk][d] = vv;
      }
      __syncthreads();
      const int kn = min(KC, L - k0);
      for (int kk = 0; kk < kn; ++kk) {
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < HD; ++d) s += qv[d] * Kc[kk][d];
        if (a.mask_mode != MASK_NONE) s += mask_value(a, win, qc, k0 + kk, last_band);
        const float mn = fmaxf(m, s);
        // offsets taken from 0 while every logit so far is -inf (keys masked
        // by -inf): exp(-inf) = 0 instead of exp(-inf - -inf) = NaN
        const float mo = mn == -INFINITY ? 0.f : mn;
        const float corr = expf(m - mo);
        const float p = expf(s - mo);
        l = l * corr + p;
#pragma unroll
        for (int d = 0; d < HD; ++d) acc[d] = acc[d] * corr + p * Vc[kk][d];
        m = mn;
      }
    }
    if (active) {
      const float inv = 1.0f / l;
      T* orow = (T*)a.o + (win * L + q) * (int64_t)C + head * HD;
#pragma unroll
      for (int d = 0; d < HD; ++d) orow[d] = from_f32<T>(acc[d] * inv);
    }
  }
}

template <int HD, int NKB>
static void launch_nkb(const AttnArgs& a, int64_t grid, hipStream_t st) {
  if (a.mask_mode == MASK_TENSOR)
    hipLaunchKernelGGL((attn_mfma_kernel<HD, NKB, true>), dim3((unsigned)grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((attn_mfma_kernel<HD, NKB, false>), dim3((unsigned)grid), dim3(256), 0, st, a);
}

// One instance per 16-key block count, L <= 384 (24 blocks).
template <int HD, int... N>
static int launch_mfma_seq(const AttnArgs& a, int64_t grid, hipStream_t st, std::integer_sequence<int, N...>) {
  const int nkb = (a.L + 15) / 16;
  bool done = false;
  ((nkb == N + 1 ? (launch_nkb<HD, N + 1>(a, grid, st), done = true) : false), ...);
  return done ? 0 : -1;
}

template <int HD>
static int launch_mfma(const AttnArgs& a, int64_t grid, hipStream_t st) {
  return launch_mfma_seq<HD>(a, grid, st, std::make_integer_sequence<int, 24>{});
}

// Head dim 64 without a mask tensor, 9 x 18 windows (11 key blocks):
// attn_dma_kernel.  Returns -1 when it does not apply: the 32-bit byte
// offsets of the copies (qkv_bytes, the drop offset of the padding rows, plus
// the item's offset) must stay below 2^32, and the tensors must be 16-byte
// aligned.
static int launch_dma(const AttnArgs& a0, int64_t items, hipStream_t st) {
  const int nkb = (a0.L + 15) / 16;
  const uint64_t qkv_bytes = (uint64_t)items / a0.heads * a0.L * 3ull * a0.C * 2ull;
  if (nkb != 11 || qkv_bytes >= (1ull << 31) || items >= (1ll << 31) || items % a0.heads != 0) return -1;
  if ((uintptr_t)a0.qkv % 16 != 0 || (uintptr_t)a0.o % 16 != 0) return -1;
  AttnArgs a = a0;
  a.zscale = a.scale * 1.4426950408889634f;
  a.smask = -100.0f / a.scale;
  a.qkv_bytes = (uint32_t)qkv_bytes;
  a.obytes = (uint32_t)((uint64_t)items / a.heads * a.L * a.C * 2ull);
  a.dheads = FastDiv::make((uint32_t)a.heads);
  hipLaunchKernelGGL((attn_dma_kernel<11>), dim3((unsigned)items), dim3(256), 0, st, a);
  return 0;
}

// fp32, head dim 64 without a mask tensor, 9 x 18 windows: attn_f32_kernel
// (conditions as launch_dma, with 4-byte elements).
static int launch_f32(const AttnArgs& a, int64_t items, hipStream_t st) {
  const int nkb = (a.L + 15) / 16;
  const uint64_t qkv_bytes = (uint64_t)items / a.heads * a.L * 3ull * a.C * 4ull;
  if (nkb != 11 || qkv_bytes >= (1ull << 31) || items >= (1ll << 31) || items % a.heads != 0) return -1;
  if ((uintptr_t)a.qkv % 16 != 0 || (uintptr_t)a.o % 16 != 0) return -1;
  hipLaunchKernelGGL((attn_f32_kernel<11>), dim3((unsigned)items), dim3(512), 0, st, a, (int)items);
  return 0;
}

template <typename T>
static int launch_scalar(const AttnArgs& a, int hd, int64_t grid, hipStream_t st) {
  switch (hd) {
    case 4: hipLaunchKernelGGL((attn_scalar_kernel<T, 4>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    case 8: hipLaunchKernelGGL((attn_scalar_kernel<T, 8>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    case 16: hipLaunchKernelGGL((attn_scalar_kernel<T, 16>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    case 32: hipLaunchKernelGGL((attn_scalar_kernel<T, 32>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    case 64: hipLaunchKernelGGL((attn_scalar_kernel<T, 64>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    case 128: hipLaunchKernelGGL((attn_scalar_kernel<T, 128>), dim3((unsigned)grid), dim3(256), 0, st, a); return 0;
    default: return -1;
  }
}

int check_geom(int64_t B, int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1, const char* what);

}  // namespace nsw

using namespace nsw;

extern "C" int nsw_window_attention(const void* qkv, void* o, const float* mask, int64_t nW_mask,
                                    int64_t Bw, int64_t L, int64_t C, int64_t num_heads, float scale,
                                    int64_t H, int64_t W, int64_t ws0, int64_t ws1, int64_t s0,
                                    int64_t s1, int64_t T, int dtype, void* stream) {
  const char* what = "nsw_window_attention";
  NSW_CHECK_ARG(Bw > 0 && L > 0 && C > 0 && num_heads > 0, "%s: Bw, L, C, num_heads must be positive", what);
  NSW_CHECK_ARG(C % num_heads == 0, "%s: C not divisible by num_heads", what);
  NSW_CHECK_ARG(C % 8 == 0, "%s: C must be a multiple of 8", what);
  NSW_CHECK_ARG(Bw * L < (1LL << 40) && Bw * num_heads < (1LL << 31), "%s: too large", what);
  const int hd = (int)(C / num_heads);
  AttnArgs a{};
  a.qkv = qkv; a.o = o; a.mask = mask; a.nW_mask = (int)nW_mask;
  a.L = (int)L; a.C = (int)C; a.heads = (int)num_heads; a.scale = scale;
  if (mask) {
    NSW_CHECK_ARG(nW_mask > 0 && Bw % nW_mask == 0, "%s: Bw=%lld not a multiple of the mask's %lld windows",
                  what, (long long)Bw, (long long)nW_mask);
    a.mask_mode = MASK_TENSOR;
  } else if (s0 != 0 || s1 != 0) {
    int rc = check_geom(1, T, H, W, ws0, ws1, what);
    if (rc) return rc;
    NSW_CHECK_ARG(s0 >= 0 && s0 < ws0 && s1 >= 0 && s1 < ws1, "%s: shift must lie in [0, window)", what);
    NSW_CHECK_ARG(L == T * ws0 * ws1, "%s: L=%lld != T*ws0*ws1", what, (long long)L);
    a.g = WinGeom::make(1, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)s0, (int)s1);
    NSW_CHECK_ARG(Bw % a.g.nW == 0, "%s: Bw not a multiple of the image's windows", what);
    a.mask_mode = MASK_SHIFT;
  } else {
    a.mask_mode = MASK_NONE;
  }
  hipStream_t st = (hipStream_t)stream;
  const int64_t grid = Bw * num_heads;
  if (dtype == NSW_DTYPE_BF16) {
    int rc = -1;
    if (hd == 64 && a.mask_mode != MASK_TENSOR) rc = launch_dma(a, grid, st);
    if (rc != 0) {
      if (hd == 64) rc = launch_mfma<64>(a, grid, st);
      else if (hd == 32) rc = launch_mfma<32>(a, grid, st);
    }
    if (rc != 0) rc = launch_scalar<bf16>(a, hd, grid, st);
    if (rc != 0) return set_error(NSW_ERR_UNSUPPORTED, "%s: head_dim=%d, L=%lld unsupported", what, hd, (long long)L);
  } else if (dtype == NSW_DTYPE_F32) {
    if (hd == 64 && a.mask_mode != MASK_TENSOR && launch_f32(a, grid, st) == 0) return check_launch(what);
    if (launch_scalar<float>(a, hd, grid, st) != 0)
      return set_error(NSW_ERR_UNSUPPORTED, "%s: head_dim=%d unsupported (4, 8, 16, 32, 64, 128)", what, hd);
  } else {
    return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
  }
  return check_launch(what);
}
