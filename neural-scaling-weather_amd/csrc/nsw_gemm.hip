// MFMA GEMM y[M,N] = epilogue(x[M,K] . w[N,K]^T) for gfx950, with the Swin
// block's epilogues fused in.
//
// Workgroup tile 256 (m) x 256 (n), one workgroup of 8 wavefronts per CU
// (two per SIMD, so that one wave's MFMAs cover the other's LDS reads and
// waits) in a 2 (m) x 4 (n) grid, each owning a 128 x 64 sub-tile of 16x16
// fp32 accumulator blocks (128 accumulator registers per lane).  A stage holds
// 128 bytes of k (64 bf16) of the 256 x-rows and the 256 w-rows and is
// consumed as two MFMA steps of 32 bf16; x lives in a ring of 3 slots and w in
// a ring of 2 slots of 32 KB (all 160 KB of LDS), filled at a steady 4 copies
// per wave and MFMA step (schedule at mainloop_256).  Whole 128-byte lines
// per copy.
//
// Operand staging: global -> LDS copies use gfx950's buffer_load_dwordx4 ...
// lds (direct to LDS, no VGPR staging): each instruction writes 1 KB = 8 stage
// rows of one wave's share.  Rows are XOR-swizzled in 16-byte chunks so that a
// fragment read (16 rows, same chunk) is bank-conflict free whether
// ds_read_b128 is served in 8-lane phases over 32 banks or 16-lane phases over
// 64 banks: slot = chunk ^ g(row & 15), g(r) = ((r >> 1) & 7) ^ ((r & 1) << 2).
// The MFMAs of step k run from registers while the fragments of step k+1 are
// read between them: the MFMAs go n block by n block, and the next step's
// weight fragment of an n block is read into the registers that block's
// MFMAs have just released, so the x fragments are double-buffered and the
// w fragments take one set (the register file of two waves per SIMD has no
// room for two of both).  Barriers are bare
// s_barrier: __syncthreads() would add a fence that waits for every
// outstanding copy.
//
// The MFMA is issued "transposed": the A operand is the weight fragment
// (rows n) and the B operand the activation fragment (rows m), so lane l of a
// 16x16 result block holds y[m = l%16][n = 4*(l/16) + r], r = 0..3: four
// consecutive output columns, and a row's head-norm reduction needs only two
// cross-lane permutes.
//
//   bf16: v_mfma_f32_16x16x32_bf16, one instruction per 16-byte fragment pair
//   f32 : v_mfma_f32_16x16x4_f32, four instructions per 16-byte fragment pair
//         (lane group g supplies k = 4*chunk + e to instruction e; A and B use
//          the same assignment, so the k-sum is exact)
//
// Workgroups are remapped so that each XCD (8 on MI355X, dispatched
// round-robin) works on a contiguous range of tiles, in groups of GROUP_M
// row blocks x all column blocks (column-major inside a group), so that the
// tiles in flight on an XCD share both row panels and weight panels in its L2.
#include <algorithm>

#include "nsw_gemm_common.h"

// Per-tile phase stamps, compiled in only with -DNSW_GEMM_STAMPS=1 (build.py
// --stamps, which writes nsw/libnsw_stamps.so; the default library has
// none): thread 0 of each workgroup reads s_memtime when its tile starts,
// when the prologue's first stages have landed, after the main loop, after
// the first epilogue phase is staged and at the end, and stores them with
// HW_ID, XCC_ID and the workgroup id as 8 words at tile * 8 of
// nsw_gemm_stamps (the first NSW_STAMP_TILES tiles of each launch; every
// launch overwrites them).  nsw_gemm_read_stamps copies them to the host.
#ifndef NSW_GEMM_STAMPS
#define NSW_GEMM_STAMPS 0
#endif
#if NSW_GEMM_STAMPS
constexpr int NSW_STAMP_TILES = 65536;
__device__ uint64_t nsw_gemm_stamps[NSW_STAMP_TILES * 8];
#define NSW_STAMP(var) (var) = __builtin_amdgcn_s_memtime()
#else
#define NSW_STAMP(var) ((void)0)
#endif

namespace nsw {


constexpr int BM = 256;             // activation rows (m) per workgroup tile
constexpr int WTM = 128;            // wave tile (m)
constexpr int MB = WTM / 16;        // 16x16 result blocks per wave along m
constexpr int STEPB = 64;           // k bytes per row consumed by one MFMA step

constexpr int BN = 256;             // weight rows (n) per workgroup tile
constexpr int WTN = 64;             // wave tile (n)
constexpr int NB = WTN / 16;        // 16x16 result blocks per wave along n
constexpr int WGM = BM / WTM;       // wave grid along m (2)
constexpr int WGN = BN / WTN;       // wave grid along n (4)
constexpr int NW = WGM * WGN;       // wavefronts per workgroup: 8, two per SIMD
constexpr int ROWB = 128;           // k bytes per row and LDS stage (two MFMA steps)
// LDS of the operand ring: x in 3 slots and w in 2 slots of 256 rows x 128 B
constexpr int RING = 5 * 256 * ROWB;
constexpr int LDS_BUDGET = 160 * 1024;

// epilogue staging of the output tile in LDS, in the output dtype: the whole
// 256-row tile when it fits in the CU's 160 KB, else two halves; rows padded
// by 16 B so that the fragment-layout writes spread over the banks
template <typename T> struct Stg {
  static constexpr int STRIDE = BN * (int)sizeof(T) + 16;
  static constexpr int ROWS = BM * STRIDE <= LDS_BUDGET ? BM : BM / 2;
  static constexpr int PASSES = BM / ROWS;
  static constexpr int BYTES = ROWS * STRIDE;
  static constexpr int SMEM = RING > BYTES ? RING : BYTES;
  static_assert(SMEM <= LDS_BUDGET, "LDS use exceeds the CU's 160 KB");
};
// LDS floats at PARAM_LDS take the epilogue's parameters (above the staging
// rows of either dtype): bias [0, 256), q/k norm weights [PRM_NW, +128), row
// scales [PRM_RS, +256).
constexpr int PARAM_LDS = 140 * 1024;
constexpr int PRM_NW = 256, PRM_RS = 384;
static_assert(Stg<bf16>::BYTES <= PARAM_LDS && Stg<float>::BYTES <= PARAM_LDS &&
              PARAM_LDS + (PRM_RS + 256) * 4 <= RING, "epilogue parameters in LDS");




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

// Fragment read: 16 bytes of k chunk `chunk` of a stage row.
__device__ __forceinline__ u32x4 lds_frag(const char* stage, int row, int chunk) {
  const int slot = chunk ^ row_swizzle(row);
  return *reinterpret_cast<const u32x4*>(stage + row * ROWB + slot * 16);
}

// Main loop of the 256 x 256 tile.  Stage st holds 128 bytes of k of the 256
// x rows and the 256 w rows.  x lives in a ring of 3 slots and w in a ring of
// 2 slots of 32 KB (160 KB in all).  The copies are issued by the four waves
// of the first row half (waves 0-3, one per SIMD: NC = 8 copies of each
// operand per stage each, 64 rows); the other four waves run only LDS reads
// and MFMAs, so that on every SIMD one wave's MFMA stream is free of copy
// issue (bit-identical; 2-5% faster on the block's four GEMM shapes than
// 4 + 4 copies per wave, measured on one box; the copies on waves 4-7
// instead were 2-5% slower than 4 + 4).  A copying wave issues its copies of
// a step in the step's first two n blocks (4 each):
//   step 2s+1 (the second step of stage s, after the barrier that frees the
//              slots of stage s): w of stage s+2 into w slot s%2;
//   step 2s+2 (the first step of stage s+1): x of stage s+3 into x slot s%3,
// and the x copies (the operand with fewer sharers in L2) get 2-3 steps of
// lead, the w copies 1-2.  At the start of step 2s+1 a wave waits for its
// copies of stage s+1 (only x of stage s+2 may still be in flight), then
// barrier.  The fragments of step k+1 are read during step k, so a slot is
// free once the barrier at the start of the last step of its stage has
// passed.  NC = 0: a wave that copies nothing (same barriers).
template <typename T, int PRE, int NC>
__device__ __forceinline__ void mainloop_256(char* smem, const T* __restrict__ X, const T* __restrict__ Wt, int M,
                                             int N, int K, int m0, int n0, const EpiArgs& ea,
                                             f32x4 (&acc)[NB][MB], int wave, int lane, int rev,
                                             uint64_t& t_ready) {
  constexpr int SLOT = 256 * ROWB;        // one operand's stage: 32 KB
  constexpr int NCA = NC > 0 ? NC : 1;
  constexpr int WR = NC * 8;              // stage rows copied by one wave (64)
  constexpr int CG = 2;                   // n blocks of a step that issue its copies
  constexpr int CPG = NC / CG;            // copies per such n block
  constexpr int UNR = 12;                 // steps per loop iteration: 6 stages, a multiple of 3 and 2
  static_assert(MB == 8 && NB == 4, "the step's schedule assumes 8 x 4 result blocks per wave");
  static_assert(NC == 0 || (NC % CG == 0 && WR * 4 == 256), "four copying waves cover the 256 stage rows");
  const uint32_t rowbytes = (uint32_t)K * sizeof(T);
  const u32x4 rx = make_rsrc(X, (uint32_t)M * rowbytes);
  const u32x4 rw = make_rsrc(Wt, (uint32_t)N * rowbytes);
  // copy j of this wave covers slot rows wave*WR + 8j .. +7; lane i writes row
  // +i/8, 16-byte slot i%8, and loads global chunk slot ^ swizzle(row)
  uint32_t vx[NCA], vw[NCA];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int srow = wave * WR + j * 8 + lane / 8;
    const int chunk = (lane % 8) ^ row_swizzle(srow);
    int gx = m0 + srow;
    gx = gx < M ? gx : M - 1;   // rows past the edge re-read the last row (never stored)
    int gw = n0 + srow;
    gw = gw < N ? gw : N - 1;
    vx[j] = (uint32_t)gx * rowbytes + chunk * 16;
    vw[j] = (uint32_t)gw * rowbytes + chunk * 16;
  }
  const uint32_t cbase = (uint32_t)(uintptr_t)smem + wave * WR * ROWB;   // this wave's first slot row

#define NSW_XSLOT(s) (((s) % 3) * SLOT)
#define NSW_WSLOT(s) ((3 + (s) % 2) * SLOT)
// copy j of stage st (k bytes st*ROWB ..) into the slot of stage sl (sl == st
// modulo 6; sl is a compile-time constant)
// k offset of stage st: stages walked from the last one when rev_ is set
#define NSW_KOFF(st) ((uint32_t)(rev_ ? (nst - 1 - (st)) : (st)) * ROWB)
#define NSW_COPY_X(sl, st, j) dma16(rx, cbase + NSW_XSLOT(sl) + (j) * 1024, vx[j], NSW_KOFF(st))
#define NSW_COPY_W(sl, st, j) dma16(rw, cbase + NSW_WSLOT(sl) + (j) * 1024, vw[j], NSW_KOFF(st))

  const int nk = K / (STEPB / (int)sizeof(T));   // MFMA steps
  // stages; with an odd step count the last stage holds one step's k (its
  // second half is copied -- the next row's first bytes, or zeros past the
  // end of the operand -- and never read by an MFMA)
  const int nst = (nk + 1) / 2;
  // serpentine k: a tile of an odd round of its XCD walks the stages from
  // the last one, so that it starts on the k slabs the tiles before it on
  // the XCD finished with, still in L2 (odd step counts keep the half
  // stage last: forward)
  const bool rev_ = rev && (nk & 1) == 0;
  // prologue: x0 w0 x1 w1, then wait for x0 and w0 (step 0 issues x2)
#pragma unroll
  for (int j = 0; j < NC; ++j) NSW_COPY_X(0, 0, j);
#pragma unroll
  for (int j = 0; j < NC; ++j) NSW_COPY_W(0, 0, j);
  if (nst > 1) {
#pragma unroll
    for (int j = 0; j < NC; ++j) NSW_COPY_X(1, 1, j);
#pragma unroll
    for (int j = 0; j < NC; ++j) NSW_COPY_W(1, 1, j);
    NSW_WAIT_VMCNT(2 * NC);
  } else {
    NSW_WAIT_VMCNT(0);
  }
  wg_barrier();
  NSW_STAMP(t_ready);

  const int frow = lane & 15, fg = lane >> 4;
  const int wrow = (wave % WGN) * WTN + frow;  // w rows of this wave (A operand)
  const int xrow = (wave / WGN) * WTM + frow;  // x rows of this wave (B operand)
  u32x4 fa[2][NB], fb[2][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i) fa[0][i] = lds_frag(smem + NSW_WSLOT(0), wrow + i * 16, fg);
#pragma unroll
  for (int i = 0; i < MB; ++i) fb[0][i] = lds_frag(smem + NSW_XSLOT(0), xrow + i * 16, fg);

  // step k = kt + U of stage st = k/2; kt is a multiple of UNR, so the slots
  // of the stages touched by step U are compile-time constants.  Step k
  // copies stage st + 2 (x in its first step, w in its second) with no
  // condition: uniform branches around the copies cost ~7% of the loop.  Past
  // the last stage these copies re-read the last stage (L2-resident) into
  // slots nothing reads: x into the slot of stage st - 1,
  // w into the slot of stage st, which the barrier at the start of the step
  // has freed, except in the last step (no barrier): its w copies go to the
  // x slot of stage st + 1, unused.  The epilogue drains them before it
  // writes LDS.
#define NSW_STEP256(U)                                                                         \
  {                                                                                            \
    const int k = kt + U;                                                                      \
    if (k < nk) {                                                                              \
      constexpr int sub_ = (U) % 2, su_ = (U) / 2;                                             \
      constexpr int nsub_ = ((U) + 1) % 2, nsu_ = ((U) + 1) / 2;                               \
      const int st = k >> 1;                                                                   \
      if (sub_ == 1 && k + 1 < nk) {                                                           \
        NSW_WAIT_VMCNT(NC);                                                                    \
        NSW_WAIT_LGKMCNT0();                                                                   \
        wg_barrier();                                                                          \
      }                                                                                        \
      const uint32_t wdst_ = cbase + (k + 1 < nk ? NSW_WSLOT(su_ + 2) : NSW_XSLOT(su_ + 1));    \
      const int cst_ = st + 2 < nst ? st + 2 : nst - 1;   /* past the end: the last stage, in L2 */ \
      /* n-block-major: the first MFMAs of a step need only its first weight  */             \
      /* fragment.  Per n block: the copies (first CG blocks), MB/NB next-step */            \
      /* x fragments, MB MFMAs, then the next step's weight fragment nb into   */            \
      /* the registers the MFMAs have just released (two sets of x fragments, */             \
      /* one of w)                                                             */            \
      _Pragma("unroll") for (int nb = 0; nb < NB; ++nb) {                                      \
        if (nb < CG) {                                                                         \
          _Pragma("unroll") for (int c_ = 0; c_ < CPG; ++c_) {                                 \
            const int j_ = nb * CPG + c_;                                                      \
            if (sub_ == 1) dma16(rw, wdst_ + j_ * 1024, vw[j_], NSW_KOFF(cst_));                \
            else NSW_COPY_X(su_ + 2, cst_, j_);                                                \
          }                                                                                    \
        }                                                                                      \
        /* unconditional: after the last step these read stale slots (unused); a  */         \
        /* conditional read would make the wait-count pass drain all LDS reads   */         \
        _Pragma("unroll") for (int q = 0; q < MB / NB; ++q) {                                  \
          const int mq = nb * (MB / NB) + q;                                                   \
          fb[((U) + 1) & 1][mq] = lds_frag(smem + NSW_XSLOT(nsu_), xrow + mq * 16, nsub_ * 4 + fg); \
        }                                                                                      \
        _Pragma("unroll") for (int mb = 0; mb < MB; ++mb)                                      \
          mfma_chunk<T>(acc[nb][mb], fa[(U) & 1][nb], fb[(U) & 1][mb]);                        \
        fa[((U) + 1) & 1][nb] = lds_frag(smem + NSW_WSLOT(nsu_), wrow + nb * 16, nsub_ * 4 + fg); \
        /* the group's three fragment reads spread over its MFMAs: 1, 2 MFMAs, 1, */            \
        /* 3 MFMAs, 1, 3 MFMAs (bf16; four MFMA instructions per block in fp32)   */            \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * (sizeof(T) == 2 ? 1 : 4), 0);          \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x008, 3 * (sizeof(T) == 2 ? 1 : 4), 0);          \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x008, 3 * (sizeof(T) == 2 ? 1 : 4), 0);          \
      }                                                                                        \
    }                                                                                          \
  }

  for (int kt = 0; kt < nk; kt += UNR) {
    NSW_STEP256(0) NSW_STEP256(1) NSW_STEP256(2) NSW_STEP256(3)
    NSW_STEP256(4) NSW_STEP256(5) NSW_STEP256(6) NSW_STEP256(7)
    NSW_STEP256(8) NSW_STEP256(9) NSW_STEP256(10) NSW_STEP256(11)
  }
#undef NSW_STEP256
#undef NSW_COPY_X
#undef NSW_KOFF
#undef NSW_COPY_W
#undef NSW_XSLOT
#undef NSW_WSLOT
}

// P consecutive values between LDS / registers / global memory, as one
// access where P * sizeof(V) is 2, 4, 8 or 16 bytes (16-byte pieces above).
template <typename V, int P>
__device__ __forceinline__ void copy_run(V* __restrict__ dst, const V* __restrict__ src) {
  constexpr int B = P * (int)sizeof(V);
  if constexpr (B >= 16) {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(src)[i];
  } else if constexpr (B == 8) {
    *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
  } else if constexpr (B == 4) {
    *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
  } else {
    *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
  }
}

// EPI_UNPATCH write-out of the staged rows [r0, r0 + S::ROWS) of a tile: the
// head layout of models/swin.py:286-299 (reshape [b, h, w, p, p, c], einsum
// nthwpqc -> ntchpwq) with the head's output columns permuted to c p^2 +
// dy p + dx (host side), so that a tile's 256 columns are the whole p x p
// patches of 256 / p^2 channels.  A thread keeps one staged row (a token:
// frame b, patch row py, patch column px) and walks the (channel, dy)
// pairs; per pair one LDS read of the p values dx = 0 .. p-1 and one store
// of p pixels into image row py p + dy.  Consecutive lanes hold consecutive
// tokens, so a store instruction covers consecutive p-pixel runs of one
// image row.  Values are rounded to T at staging, then widened to float for
// a float image (as the separate GEMM + unpatchify would).
template <typename T, int P>
__device__ __forceinline__ void unpatch_copy_out(const char* stg, const EpiArgs& ea, int M, int N, int r0, int n0,
                                                 int tid) {
  using S = Stg<T>;
  constexpr int CPT = BN / (P * P);                   // channels per tile
  constexpr int TPR = NW * 64 / S::ROWS;              // threads per staged row (2 / 4)
  const int tl = tid % S::ROWS;                       // staged row of this thread
  const int m = r0 + tl;
  if (m >= M) return;
  const int wq = ea.img_W / P, hw = (ea.img_H / P) * wq;
  const int b = m / hw, rr = m - b * hw, py = rr / wq, px = rr - py * wq;
  const int64_t HW = (int64_t)ea.img_H * ea.img_W;
  const int64_t pix0 = (int64_t)b * ea.img_bstride + (int64_t)(py * P) * ea.img_W + px * P;
  const int c0 = n0 / (P * P);
  const T* row = reinterpret_cast<const T*>(stg + tl * S::STRIDE);
  for (int cd = tid / S::ROWS; cd < CPT * P; cd += TPR) {
    const int cl = cd / P, dy = cd - cl * P;
    const int c = c0 + cl;
    if (c * P * P >= N) break;                        // columns past N: channels past C_out
    const T* src = row + cl * P * P + dy * P;
    const int64_t off = pix0 + c * HW + (int64_t)dy * ea.img_W;
    if (ea.img_f32 && sizeof(T) == 2) {
      T v[P];
      copy_run<T, P>(v, src);
      float f[P];
#pragma unroll
      for (int e = 0; e < P; ++e) f[e] = to_f32(v[e]);
      copy_run<float, P>(reinterpret_cast<float*>(ea.img) + off, f);
    } else {
      copy_run<T, P>(reinterpret_cast<T*>(ea.img) + off, src);
    }
  }
}

template <typename T, int EPI, int PRE>
__global__ __launch_bounds__(NW * 64, 1) void gemm_kernel(const T* __restrict__ X, const T* __restrict__ Wt,
                                                     T* __restrict__ Y, int M, int N, int K, EpiArgs ea) {
  // the operand ring during the k loop, the output staging area in the
  // epilogue
  __shared__ __attribute__((aligned(1024))) char smem[Stg<T>::SMEM];

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  const int MT = (M + BM - 1) / BM, NT = (N + BN - 1) / BN;
  // Tiles of one XCD run in groups of GROUP_M row blocks x all column blocks,
  // column-major inside the group, so that the tiles in flight on an XCD
  // share both their row panels and their weight panels in its L2.
  // (ea.group_m row blocks when set: 4 for the QKV projection and 16 for
  // proj, each measured 1.5-3% faster there; fc1 is fastest at 8)
  const int GM = ea.group_m > 0 ? ea.group_m : GROUP_M;
  const int tile = xcd_remap(blockIdx.x, MT * NT);
  const int group = tile / (GM * NT);
  const int gm0 = group * GM;
  const int gsz = MT - gm0 < GM ? MT - gm0 : GM;
  const int tin = tile - group * GM * NT;
  const int mt = gm0 + tin % gsz, nt = tin / gsz;
  const int m0 = mt * BM, n0 = nt * BN;

  f32x4 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // waves 0-3 copy the operands, waves 4-7 do not (see mainloop_256).  The
  // XCD-local workgroup index (blockIdx / 8) over the XCD's 32 CUs counts
  // the rounds of tiles on an XCD; odd rounds walk k backwards (serpentine:
  // 7-8% less L2 fetch on the K = 1024 GEMMs of config 2, 1-1.5% faster)
  const int rev = ((int)(blockIdx.x >> 3) / 32) & 1;
  uint64_t ts[5] = {0, 0, 0, 0, 0};   // phase stamps (NSW_GEMM_STAMPS builds only)
  NSW_STAMP(ts[0]);
  {
    const int lane0 = (int)threadIdx.x & 63;
    if (wave < 4) mainloop_256<T, PRE, 8>(smem, X, Wt, M, N, K, m0, n0, ea, acc, wave, lane0, rev, ts[1]);
    else mainloop_256<T, PRE, 0>(smem, X, Wt, M, N, K, m0, n0, ea, acc, wave, lane0, rev, ts[1]);
  }
  NSW_STAMP(ts[2]);
  // the lane's ids for the epilogue, from the lane counter and the (scalar)
  // wave id: kept live across the k loop they were spilled to scratch (2-5
  // VGPRs per instantiation; with this, none spill, bit-identical, time
  // unchanged).  Inline asm, or the compiler folds the counter back into the
  // work-item id and keeps that live.
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  const int tid = wave * 64 + lane;
  const int frow = lane & 15, fg = lane >> 4;

  // ---------------------------------------------------------------- epilogue
  // lane (frow, fg) of block (nb, mb) holds y[m0 + wm*WTM + mb*16 + frow]
  //                                          [n0 + wn*WTN + nb*16 + 4*fg + r]
  const int nw0 = n0 + wn * WTN;           // first column of this wave
  constexpr int HDQ = qkv_head_dim(EPI);
  // With the head norm or the row scale, the bias, norm weights and row
  // scales reach the lanes through LDS (one element per thread, parked there
  // once the operand ring is free): loaded straight into the fragment layout,
  // their 16+ small loads went out one at a time, each behind the previous
  // one, because the accumulators copied out of the AGPRs fill the VGPRs
  // here.  The bias-only epilogues load it directly (one batch).
  constexpr bool PLDS = HDQ > 0 || PRE == PRE_ROWSCALE;
  const T* bias = (const T*)ea.bias;
  float bv[NB][4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = nw0 + nb * 16 + fg * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[nb][r] = 0.f;
    if constexpr (EPI != EPI_NONE && EPI != EPI_UNPATCH && !PLDS)
      load4<T>(bias + (n < N ? n : 0), bv[nb]);   // straight-line: one batch
  }

  // per-head RMSNorm (QKV epilogue): a head is HDQ/16 consecutive 16-column
  // blocks inside one of the q / k / v regions (C % 16 == 0 and HDQ | C), so
  // whether a head is normalised is uniform across its lanes.  Head dims 4
  // and 8 put 4 / 2 heads in one 16-column block: a lane's 4 columns are a
  // whole head (4) or half of one, the other half in the lane 16 apart (8);
  // then the flags below are kept per block (NBH = 1, "heads" = blocks).
  constexpr int NBH = HDQ >= 16 ? HDQ / 16 : 1;  // blocks per head
  constexpr int HSP = HDQ >= 16 ? HDQ : 16;      // columns per flag slot
  constexpr int NHW = NB / NBH;                  // flag slots per wave tile
  bool normed[NHW];
  int nwreg[NHW];                               // 0: q weights, 1: k weights
  float nwv[NB][4];
  if constexpr (HDQ > 0) {
#pragma unroll
    for (int h = 0; h < NHW; ++h) {
      const int c0 = nw0 + h * HSP;
      const int region = c0 / ea.C;  // 0: q, 1: k, 2: v
      normed[h] = region < 2 && c0 < N;
      nwreg[h] = region == 0 ? 0 : 1;
    }
  }

  // this thread's parameter element, loaded here and parked in LDS once the
  // operand ring is free (see the write-out)
  float p_bias = 0.f, p_nw = 0.f, p_rs = 1.f;
  if constexpr (EPI != EPI_NONE && PLDS) {
    const int n = n0 + tid;
    p_bias = tid < BN && n < N ? to_f32(((const T*)ea.bias)[n]) : 0.f;
  }
  if constexpr (HDQ > 0) {
    if (tid < 2 * HDQ) p_nw = to_f32(((const T*)(tid < HDQ ? ea.qn_w : ea.kn_w))[tid % HDQ]);
  }
  if constexpr (PRE == PRE_ROWSCALE) {
    // row m0 + tid's norm from the producer's partial sums of squares, added
    // in a fixed order (rows past M read row 0 and are never stored)
    const int m = m0 + (tid < BM ? tid : 0);
    const float* pp = ea.row_sumsq + (int64_t)(m < M ? m : 0) * ea.nparts;
    float ss = 0.f;
    int q = 0;
    if ((ea.nparts & 3) == 0) {
      for (; q < ea.nparts; q += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(pp + q);
        ss += (v[0] + v[1]) + (v[2] + v[3]);
      }
    }
    for (; q < ea.nparts; ++q) ss += pp[q];
    p_rs = 1.0f / sqrtf(ss / (float)K + ea.eps);
  }

  // PRE_ROWSCALE: the row scales of this lane's rows (from LDS, below)
  float rsr[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) rsr[mb] = 1.f;
  // 1. epilogue math of row block mb in the fragment layout (bias, row scale,
  // head norm, GELU), evaluated where the block is staged
  auto row_values = [&](int mb, float (&v)[NB][4]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[nb][r] = (PRE != PRE_NONE ? acc[nb][mb][r] * rsr[mb] : acc[nb][mb][r]) + bv[nb][r];

    if constexpr (HDQ > 0) {
      // sum of squares of each head: local over its blocks, then across the
      // four lane groups holding the same row (xor 16, xor 32)
      float ss[NHW];
#pragma unroll
      for (int h = 0; h < NHW; ++h) {
        float sh = 0.f;
#pragma unroll
        for (int b = 0; b < NBH; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) sh = fmaf(v[h * NBH + b][r], v[h * NBH + b][r], sh);
        if constexpr (HDQ >= 16) ss[h] = rows4_sum(sh);
        else if constexpr (HDQ == 8) ss[h] = rows2_sum(sh);
        else ss[h] = sh;
      }
#pragma unroll
      for (int h = 0; h < NHW; ++h) {
        if (normed[h]) {
          // x * rsqrt(mean(x^2) + eps), then * weight, as RMSNorm
          const float rs = __builtin_amdgcn_rsqf(ss[h] * (1.0f / (float)HDQ) + ea.eps);
#pragma unroll
          for (int b = 0; b < NBH; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[h * NBH + b][r] = (v[h * NBH + b][r] * rs) * nwv[h * NBH + b][r];
        }
      }
    }
    if constexpr (EPI == EPI_BIAS_GELU) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[nb][r] = sizeof(T) == 2 ? gelu_erf_bf16(v[nb][r]) : gelu_erf(v[nb][r]);
    } else if constexpr (EPI == EPI_BIAS_GELU_TANH) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[nb][r] = gelu_tanh(v[nb][r]);
    }
  };

  // 2. write-out through LDS: the waves owning the staged rows store their
  // values in the fragment layout (output dtype), which frees the
  // accumulators, then every wave copies whole rows out with 16-byte lane
  // accesses (fully coalesced) in batches of BATCH rows, adding the residual
  // there.  A batch's output rows (the window -> token map for the scatter)
  // and residual rows are loaded one batch ahead, the first batch's before
  // the staging writes; the loads use clamped addresses (no branches), only
  // the stores are predicated.
  using S = Stg<T>;
  constexpr int VEC = 16 / sizeof(T);                 // elements per 16-byte chunk
  constexpr int LPR = BN / VEC;                       // lanes per output row (32 bf16 / 64 f32)
  constexpr int RPI = 64 / LPR;                       // rows per copy instruction (2 / 1)
  constexpr int ITER = S::ROWS / NW / RPI;            // copy instructions per wave per pass
  constexpr int BATCH = 8;                            // rows loaded one batch ahead (at most)
  constexpr bool SCAT = EPI == EPI_SCATTER_RESIDUAL;
  constexpr bool REMAP = EPI == EPI_REMAP_RESIDUAL;
  constexpr bool TOK = EPI == EPI_TOKEN_RESIDUAL;
  constexpr bool TOWIN = EPI == EPI_WINDOW_RESIDUAL;
  constexpr bool RES = EPI == EPI_BIAS_RESIDUAL || SCAT || REMAP || TOK || TOWIN || EPI == EPI_RES_SUMSQ;
  // row sums of squares of the stored rows (optional for the scatter)
  constexpr bool SUMSQ = SCAT || REMAP || TOWIN || EPI == EPI_RES_SUMSQ;
  NSW_WAIT_VMCNT(0);                                  // the copies past the last stage
  NSW_WAIT_LGKMCNT0();
  wg_barrier();                                       // the operand ring is no longer read
  if constexpr (PLDS) {
    // epilogue parameters, one element per thread: the tile's 256 bias
    // values, the q and k norm weights, the 256 row scales
    float* prm = reinterpret_cast<float*>(smem + PARAM_LDS);
    if constexpr (EPI != EPI_NONE) {
      if (tid < BN) prm[tid] = p_bias;
    }
    if constexpr (HDQ > 0) {
      if (tid < 2 * HDQ) prm[PRM_NW + tid] = p_nw;
    }
    if constexpr (PRE == PRE_ROWSCALE) {
      if (tid < BM) prm[PRM_RS + tid] = p_rs;
    }
    NSW_WAIT_LGKMCNT0();
    wg_barrier();
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 b4 = EPI != EPI_NONE ? *reinterpret_cast<const f32x4*>(prm + wn * WTN + nb * 16 + fg * 4)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[nb][r] = b4[r];
    }
    if constexpr (HDQ > 0) {
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int b = 0; b < NBH; ++b) {
          const int dcol = HDQ >= 16 ? b * 16 + fg * 4 : (fg * 4) % HDQ;   // column within the head
          const f32x4 w4 = *reinterpret_cast<const f32x4*>(prm + PRM_NW + nwreg[h] * HDQ + dcol);
#pragma unroll
          for (int r = 0; r < 4; ++r) nwv[h * NBH + b][r] = w4[r];
        }
    }
    if constexpr (PRE == PRE_ROWSCALE) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) rsr[mb] = prm[PRM_RS + wm * WTM + mb * 16 + frow];
    }
  }
  char* stg = smem;
  const int lrow = lane / LPR;                        // row of this lane within an instruction
  const int col = (lane % LPR) * VEC;                 // first tile column of this lane
  const int n = n0 + col;
  const int nc = n < N ? n : 0;                       // clamped column for loads
  // Phases: with the whole tile staged at once (bf16), staging and copy-out
  // run in NPH phases of MB / NPH row blocks per wave-row half, and a
  // phase's copy-out (LDS reads, global stores in flight) is followed by
  // the staging of the next phase's rows, so that the epilogue math (VALU)
  // overlaps the stores of the rows before it.  Phase p covers the tile
  // rows [p RHP, (p + 1) RHP) of both wave-row halves; its copy-out gives
  // each wave 2 RHP / NW consecutive rows of one half.
  constexpr int NPH = (S::PASSES == 1 && EPI != EPI_UNPATCH) ? 4 : 1;
  constexpr int IPP = ITER / NPH;                     // copy instructions per wave and phase
  constexpr int BAT = IPP < BATCH ? IPP : BATCH;      // rows loaded one batch ahead
  constexpr int NBP = IPP / BAT;                      // batches per phase
  constexpr int NBT = NPH * NBP;                      // batches per pass
  constexpr int RHP = WTM / NPH;                      // rows of a wave-row half per phase
  static_assert(ITER % NPH == 0 && IPP % BAT == 0 && (NPH == 1 || NW * IPP * RPI == 2 * RHP), "phases");
#pragma unroll
  for (int pass = 0; pass < S::PASSES; ++pass) {
    const int prow0 = pass * S::ROWS;                 // first tile row of this pass
    // tile row of the j-th row of phase p's copy-out (j = wave IPP RPI + ...)
    auto tile_row = [&](int p, int j) {
      return prow0 + (NPH == 1 ? j : (j / RHP) * WTM + p * RHP + j % RHP);
    };
    int orow[2][BAT];                                 // output row (token for the scatter) per batch row
    u32x4 rres[2][RES ? BAT : 1];
    float ssacc = 0.f;                                // row sums of squares of the pass (SUMSQ)
    // Row maps: the wave copies ITER * RPI (<= 64) rows per pass, so lane l
    // maps the wave's l-th row once and every copy instruction takes its
    // rows' targets from those lanes (v_readlane) instead of all 32 or 64
    // lanes of a row evaluating the same map.
    constexpr bool MAPPED = SCAT || TOK || REMAP || TOWIN;
    constexpr int WROWS = ITER * RPI;                 // rows per wave per pass
    static_assert(WROWS <= 64, "one row per lane");
    // the wave's l-th row (l < WROWS): phase l / (IPP RPI), j = wave IPP RPI + l % (IPP RPI)
    auto wave_row = [&](int l) { return tile_row(l / (IPP * RPI), wave * IPP * RPI + l % (IPP * RPI)); };
    int lmap = 0;
    if constexpr (MAPPED) {
      int mm = m0 + wave_row(lane % WROWS);
      mm = mm < M ? mm : M - 1;
      if constexpr (REMAP) lmap = (int)ea.geom.row_of_row_shift(mm, ea.dh, ea.dw);
      else if constexpr (TOWIN) lmap = (int)ea.geom.row_of_token(mm);
      else lmap = (int)ea.geom.token_of_row(mm);
    }
    // batch g, row b: phase g / NBP, instruction qq of the phase; its rows
    // are the wave's rows ql and ql + 1 (bf16) in the order of wave_row
    auto prefetch = [&](int g, int slot) {
#pragma unroll
      for (int b = 0; b < BAT; ++b) {
        const int ph = g / NBP, qq = (g % NBP) * BAT + b;
        const int ql = (ph * IPP + qq) * RPI;         // lane of this instruction's first row
        int m = m0 + tile_row(ph, wave * IPP * RPI + qq * RPI + lrow);
        m = m < M ? m : M - 1;
        if constexpr (MAPPED) {
          const int a0 = __builtin_amdgcn_readlane(lmap, ql);
          if constexpr (RPI == 2) {
            const int a1 = __builtin_amdgcn_readlane(lmap, ql + 1);
            orow[slot][b] = lrow ? a1 : a0;
          } else {
            orow[slot][b] = a0;
          }
        } else {
          orow[slot][b] = m;
        }
        // the residual row: the output row for the scatter, row m otherwise
        const int rrow = SCAT ? orow[slot][b] : m;
        if constexpr (RES)
          rres[slot][b] = *reinterpret_cast<const u32x4*>((const T*)ea.residual + (int64_t)rrow * N + nc);
      }
    };
    // epilogue math of phase p's row blocks, stored in the fragment layout
    auto stage = [&](int p) {
#pragma unroll
      for (int mb = p * (MB / NPH); mb < (p + 1) * (MB / NPH); ++mb) {
        const int trow = wm * WTM + mb * 16 + frow - prow0;
        if (wm * WTM + mb * 16 - prow0 >= 0 && wm * WTM + mb * 16 - prow0 < S::ROWS) {   // wave-uniform
          float v[NB][4];
          row_values(mb, v);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) store4<T>(reinterpret_cast<T*>(stg + trow * S::STRIDE) + wn * WTN + nb * 16 + fg * 4, v[nb]);
        }
      }
    };
    prefetch(0, 0);
    stage(0);
    wg_barrier();
    if (pass == 0) NSW_STAMP(ts[3]);
    if constexpr (EPI == EPI_UNPATCH) {
      switch (ea.img_p) {
        case 1: unpatch_copy_out<T, 1>(stg, ea, M, N, m0 + prow0, n0, tid); break;
        case 2: unpatch_copy_out<T, 2>(stg, ea, M, N, m0 + prow0, n0, tid); break;
        case 4: unpatch_copy_out<T, 4>(stg, ea, M, N, m0 + prow0, n0, tid); break;
        case 8: unpatch_copy_out<T, 8>(stg, ea, M, N, m0 + prow0, n0, tid); break;
        default: unpatch_copy_out<T, 16>(stg, ea, M, N, m0 + prow0, n0, tid); break;
      }
      if (pass + 1 < S::PASSES) wg_barrier();        // before the next pass overwrites the staging rows
      continue;
    }
#pragma unroll
    for (int g = 0; g < NBT; ++g) {
      const int cur = g & 1;
      if (g + 1 < NBT) prefetch(g + 1, cur ^ 1);
      const int ph = g / NBP;
      u32x4 ov[BAT];
#pragma unroll
      for (int b = 0; b < BAT; ++b) {
        const int rl = tile_row(ph, wave * IPP * RPI + ((g % NBP) * BAT + b) * RPI + lrow) - prow0;
        ov[b] = *reinterpret_cast<const u32x4*>(stg + rl * S::STRIDE + col * (int)sizeof(T));
      }
#pragma unroll
      for (int b = 0; b < BAT; ++b) {
        const int qq = (g % NBP) * BAT + b;
        const int m = m0 + tile_row(ph, wave * IPP * RPI + qq * RPI + lrow);
        const bool ok = m < M && n < N;
        float ssq = 0.f;                              // sum of squares of this lane's stored values
        if constexpr (RES) {
          float o[VEC], rv[VEC];
          if constexpr (sizeof(T) == 2) {
            const bf16x8 ob = __builtin_bit_cast(bf16x8, ov[b]);
            const bf16x8 rb = __builtin_bit_cast(bf16x8, rres[cur][b]);
#pragma unroll
            for (int e = 0; e < VEC; ++e) { o[e] = (float)ob[e]; rv[e] = (float)rb[e]; }
          } else {
            const f32x4 of = __builtin_bit_cast(f32x4, ov[b]);
            const f32x4 rf = __builtin_bit_cast(f32x4, rres[cur][b]);
#pragma unroll
            for (int e = 0; e < VEC; ++e) { o[e] = of[e]; rv[e] = rf[e]; }
          }
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[e] += rv[e];
          if (ok) store16<T>(Y + (int64_t)orow[cur][b] * N + n, o);
          if constexpr (SUMSQ) {
            // only stored elements count (lanes past N or rows past M add 0)
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const float r = sizeof(T) == 2 ? (float)(T)o[e] : o[e];   // the stored value
              ssq = fmaf(r, r, ssq);
            }
            if (!ok) ssq = 0.f;
          }
        } else {
          // non-temporal: the tile is not read again by this kernel, and the
          // outputs without a residual (qkv, the MLP hidden rows: 398 / 531
          // MB at config 2) exceed the last-level cache; streaming them past
          // L2 made these GEMMs 4-5% faster (fc1 504 -> 481 us, bit-identical;
          // the residual epilogues, whose 133 MB outputs the next kernel
          // reads, showed no gain and keep ordinary stores)
          if (ok) __builtin_nontemporal_store(ov[b], reinterpret_cast<u32x4*>(Y + (int64_t)orow[cur][b] * N + n));
        }
        if constexpr (SUMSQ) {
          // partial sum of squares over 32 lanes (32 * VEC columns, one float
          // per 512 bytes of output row): the two 16-lane row sums of each
          // half wave, even row first, parked in lane ql + half (bf16: the
          // wave's rows ql, ql + 1; fp32: row ql, half = part) of ssacc,
          // which is stored once per pass
          if (!SCAT || ea.row_sumsq != nullptr) {
            const int ri = __builtin_bit_cast(int, row16_sum(ssq));
            const float sa = __builtin_bit_cast(float, __builtin_amdgcn_readlane(ri, 0)) +
                             __builtin_bit_cast(float, __builtin_amdgcn_readlane(ri, 16));
            const float sb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(ri, 32)) +
                             __builtin_bit_cast(float, __builtin_amdgcn_readlane(ri, 48));
            const int ql = (ph * IPP + qq) * RPI;
            constexpr int HB = RPI == 2 ? 1 : 32;       // lane offset of the upper half's value
            ssacc = lane == ql ? sa : ssacc;
            ssacc = lane == ql + HB ? sb : ssacc;
          }
        }
      }
      // the next phase's rows: their math runs while this phase's stores drain
      if ((g + 1) % NBP == 0 && g + 1 < NBT) {
        stage((g + 1) / NBP);
        wg_barrier();
      }
    }
    if constexpr (SUMSQ) {
      // one store of the pass's row sums per wave: bf16, lane l < WROWS
      // holds the wave's row l (part n0 / 256); fp32, lane l with l % 32 <
      // WROWS holds the wave's row l % 32, part n0 / 128 + l / 32
      if (!SCAT || ea.row_sumsq != nullptr) {
        const int rw = RPI == 2 ? lane : (lane & 31);
        const int m = m0 + wave_row(rw < WROWS ? rw : 0);
        const int pcol = n0 + (RPI == 2 ? 0 : (lane >> 5) * 32 * VEC);   // first column of the part
        const int orw = MAPPED ? lmap : m;                                 // lmap: row lane % WROWS (= rw here)
        if (rw < WROWS && m < M && pcol < N) ea.row_sumsq[(int64_t)orw * ea.nparts + pcol / (32 * VEC)] = ssacc;
      }
    }
    if (pass + 1 < S::PASSES) wg_barrier();          // before the next pass overwrites the staging rows
  }
#if NSW_GEMM_STAMPS
  NSW_STAMP(ts[4]);
  if (tid == 0 && tile < NSW_STAMP_TILES) {
    uint64_t* o = nsw_gemm_stamps + (size_t)tile * 8;
#pragma unroll
    for (int i = 0; i < 5; ++i) o[i] = ts[i];
    o[5] = (uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);    // HW_ID
    o[6] = (uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 20);   // XCC_ID
    o[7] = blockIdx.x;
  }
#endif
}

template <typename T, int EPI, int PRE = PRE_NONE>
static int launch_gemm(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K,
                       const EpiArgs& ea, hipStream_t st, const char* what) {
  constexpr int KT = STEPB / sizeof(T);   // one MFMA step of k: 32 (bf16) / 16 (f32)
  NSW_CHECK_ARG(M > 0 && N > 0 && K > 0, "%s: M, N, K must be positive", what);
  NSW_CHECK_ARG(K % KT == 0, "%s: K=%lld must be a multiple of %d", what, (long long)K, KT);
  NSW_CHECK_ARG(N % 8 == 0, "%s: N=%lld must be a multiple of 8", what, (long long)N);
  NSW_CHECK_ARG(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "%s: dims too large", what);
  NSW_CHECK_ARG((uint64_t)M * K * sizeof(T) < (1ULL << 31) && (uint64_t)N * K * sizeof(T) < (1ULL << 31),
                "%s: operands above 2 GiB are not supported (32-bit buffer offsets)", what);
  NSW_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)y % 16) == 0 &&
                    ((uintptr_t)ea.residual % 16) == 0,
                "%s: x, w, y and residual must be 16-byte aligned", what);
  NSW_CHECK_ARG(((M + BM - 1) / BM) * ((N + BN - 1) / BN) < (1LL << 31), "%s: too many tiles", what);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  EpiArgs eg = ea;
  if constexpr (EPI == EPI_BIAS_GELU || EPI == EPI_BIAS_GELU_TANH) {
    // the MLP's first GEMM: tile groups of ~128 tiles (8 row blocks x 16
    // column blocks at config 2, 16 x 8 at config 4: each measured 5% faster
    // than the other height on its shape)
    if (eg.group_m == 0) eg.group_m = (int)std::max<int64_t>(8, std::min<int64_t>(32, 128 / ((N + BN - 1) / BN)));
  }
  hipLaunchKernelGGL((gemm_kernel<T, EPI, PRE>), dim3((unsigned)tiles), dim3(NW * 64), 0, st, (const T*)x, (const T*)w,
                     (T*)y, (int)M, (int)N, (int)K, eg);
  return check_launch(what);
}

template <int EPI, int PRE = PRE_NONE>
static int dispatch_gemm(int dtype, const void* x, const void* w, void* y, int64_t M, int64_t N,
                         int64_t K, const EpiArgs& ea, void* stream, const char* what) {
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSW_DTYPE_BF16) return launch_gemm<bf16, EPI, PRE>(x, w, y, M, N, K, ea, st, what);
  if (dtype == NSW_DTYPE_F32) return launch_gemm<float, EPI, PRE>(x, w, y, M, N, K, ea, st, what);
  return set_error(NSW_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
}

int check_geom(int64_t B, int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1, const char* what);

int gemm_qkv(const void* x, const void* wqkv, const void* bqkv, const void* qn_w, const void* kn_w,
             float eps, void* qkv, int64_t M, int64_t C, int64_t num_heads, int dtype, void* stream) {
  const char* what = "nsw_qkv_projection";
  NSW_CHECK_ARG(num_heads > 0 && C % num_heads == 0, "%s: C=%lld not divisible by num_heads=%lld", what,
                (long long)C, (long long)num_heads);
  const int64_t hd = C / num_heads;
  NSW_CHECK_ARG(C % 16 == 0, "%s: C=%lld must be a multiple of 16", what, (long long)C);
  NSW_CHECK_ARG(hd == 4 || hd == 8 || hd == 16 || hd == 32 || hd == 64,
                "%s: head_dim=%lld unsupported (4, 8, 16, 32, 64)", what, (long long)hd);
  NSW_CHECK_ARG(bqkv && qn_w && kn_w, "%s: bias and norm weights are required", what);
  EpiArgs ea{};
  ea.bias = bqkv; ea.qn_w = qn_w; ea.kn_w = kn_w; ea.eps = eps; ea.C = (int)C;
  ea.group_m = 4;
  if (hd == 64) return dispatch_gemm<EPI_QKV_HN64>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 32) return dispatch_gemm<EPI_QKV_HN32>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 8) return dispatch_gemm<EPI_QKV_HN8>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 4) return dispatch_gemm<EPI_QKV_HN4>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
  return dispatch_gemm<EPI_QKV_HN16>(dtype, x, wqkv, qkv, M, 3 * C, C, ea, stream, what);
}

// Partial sums of squares per output row: one float per 512 bytes of row
// (32 lanes of 16-byte stores in the scatter epilogue).
int64_t sumsq_parts(int64_t C, int dtype) {
  const int64_t es = dtype == NSW_DTYPE_F32 ? 4 : 2;
  return (C * es + 511) / 512;
}

int gemm_proj_scatter(const void* o, const void* wproj, const void* bproj, const void* skip, void* y,
                      int64_t B, int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0, int64_t ws1,
                      int64_t s0, int64_t s1, int dtype, void* stream, float* row_sumsq) {
  const char* what = row_sumsq ? "nsw_proj_reverse_residual_sumsq" : "nsw_proj_reverse_residual";
  int rc = check_geom(B, T, H, W, ws0, ws1, what);
  if (rc) return rc;
  NSW_CHECK_ARG(bproj && skip, "%s: bias and skip are required", what);
  NSW_CHECK_ARG(skip != (const void*)y, "%s: skip and y must not alias (rows are permuted)", what);
  EpiArgs ea{};
  ea.bias = bproj; ea.residual = skip;
  ea.geom = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
  ea.row_sumsq = row_sumsq;
  ea.nparts = (int)sumsq_parts(C, dtype);
  ea.group_m = 16;   // proj's 4 column blocks: 16-row-block groups measured 2.5% faster than 8
  return dispatch_gemm<EPI_SCATTER_RESIDUAL>(dtype, o, wproj, y, B * T * H * W, C, C, ea, stream, what);
}

// y = epi(rs . (x . w_n^T)), rs[m] = 1/sqrt(sum_p row_sumsq[m, p] / K + eps):
// RMSNorm(x) folded into the GEMM with the row statistics from x's producer.
int gemm_linear_rowscale(const void* x, const void* w_n, const void* bias, const void* residual, void* y,
                         const float* row_sumsq, int64_t nparts, int64_t M, int64_t N, int64_t K, int epilogue,
                         float eps, int dtype, void* stream) {
  const char* what = "nsw_linear_rowscale";
  NSW_CHECK_ARG(row_sumsq != nullptr && nparts > 0 && nparts <= 4096, "%s: row_sumsq [M, nparts] is required",
                what);
  NSW_CHECK_ARG(((uintptr_t)row_sumsq % 16) == 0, "%s: row_sumsq must be 16-byte aligned", what);
  EpiArgs ea{};
  ea.bias = bias; ea.residual = residual; ea.eps = eps;
  ea.row_sumsq = const_cast<float*>(row_sumsq);
  ea.nparts = (int)nparts;
  if (epilogue != NSW_EPI_NONE) NSW_CHECK_ARG(bias != nullptr, "%s: epilogue %d needs a bias", what, epilogue);
  switch (epilogue) {
    case NSW_EPI_NONE: return dispatch_gemm<EPI_NONE, PRE_ROWSCALE>(dtype, x, w_n, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS: return dispatch_gemm<EPI_BIAS, PRE_ROWSCALE>(dtype, x, w_n, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS_GELU:
      return dispatch_gemm<EPI_BIAS_GELU, PRE_ROWSCALE>(dtype, x, w_n, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS_GELU_TANH:
      return dispatch_gemm<EPI_BIAS_GELU_TANH, PRE_ROWSCALE>(dtype, x, w_n, y, M, N, K, ea, stream, what);
    case NSW_EPI_BIAS_RESIDUAL:
      NSW_CHECK_ARG(residual != nullptr, "%s: residual epilogue needs a residual", what);
      return dispatch_gemm<EPI_BIAS_RESIDUAL, PRE_ROWSCALE>(dtype, x, w_n, y, M, N, K, ea, stream, what);
    default: return set_error(NSW_ERR_INVALID, "%s: unknown epilogue %d", what, epilogue);
  }
}

// QKV projection of rows whose RMSNorm (norm1) comes as a row scale from the
// producer's partial sums of squares: qkv[m] = headnorm(rs1[m] * (x[m] .
// wqkv_n^T) + b), wqkv_n = wqkv * norm1_w per input column, rs1 =
// 1/sqrt(sum_p row_sumsq[m, p] / C + eps).  Rows in any order.
int gemm_qkv_rowscale(const void* x, const void* wqkv_n, const void* bqkv, const void* qn_w, const void* kn_w,
                      float eps, void* qkv, const float* row_sumsq, int64_t nparts, int64_t M, int64_t C,
                      int64_t num_heads, int dtype, void* stream) {
  const char* what = "nsw_qkv_projection_rowscale";
  NSW_CHECK_ARG(num_heads > 0 && C % num_heads == 0, "%s: C=%lld not divisible by num_heads=%lld", what,
                (long long)C, (long long)num_heads);
  const int64_t hd = C / num_heads;
  NSW_CHECK_ARG(C % 16 == 0, "%s: C=%lld must be a multiple of 16", what, (long long)C);
  NSW_CHECK_ARG(hd == 4 || hd == 8 || hd == 16 || hd == 32 || hd == 64,
                "%s: head_dim=%lld unsupported (4, 8, 16, 32, 64)", what, (long long)hd);
  NSW_CHECK_ARG(bqkv && qn_w && kn_w, "%s: bias and norm weights are required", what);
  NSW_CHECK_ARG(row_sumsq != nullptr && nparts > 0 && nparts <= 4096 && ((uintptr_t)row_sumsq % 16) == 0,
                "%s: row_sumsq [M, nparts] (16-byte aligned) is required", what);
  EpiArgs ea{};
  ea.bias = bqkv; ea.qn_w = qn_w; ea.kn_w = kn_w; ea.eps = eps; ea.C = (int)C;
  ea.group_m = 4;
  ea.row_sumsq = const_cast<float*>(row_sumsq);
  ea.nparts = (int)nparts;
  if (hd == 64) return dispatch_gemm<EPI_QKV_HN64, PRE_ROWSCALE>(dtype, x, wqkv_n, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 32) return dispatch_gemm<EPI_QKV_HN32, PRE_ROWSCALE>(dtype, x, wqkv_n, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 8) return dispatch_gemm<EPI_QKV_HN8, PRE_ROWSCALE>(dtype, x, wqkv_n, qkv, M, 3 * C, C, ea, stream, what);
  if (hd == 4) return dispatch_gemm<EPI_QKV_HN4, PRE_ROWSCALE>(dtype, x, wqkv_n, qkv, M, 3 * C, C, ea, stream, what);
  return dispatch_gemm<EPI_QKV_HN16, PRE_ROWSCALE>(dtype, x, wqkv_n, qkv, M, 3 * C, C, ea, stream, what);
}

// y[remap(m)] = x[m] . w^T + bias + residual[m], the stored rows' partial
// sums of squares (one float per 512 bytes of row) into row_sumsq at the
// same rows where asked.  map_mode 0: remap(m) = m (row_sumsq required); 1:
// the token of window-order row m of the image geometry (B, T, H, W, ws,
// shift s) (no row sums); 2: that token's row in the window order of the
// same image rolled by (sa, sb), the next block's (row_sumsq required).
int gemm_linear_remap(const void* x, const void* w, const void* bias, const void* residual, void* y,
                      float* row_sumsq, int64_t M, int64_t N, int64_t K, int map_mode, int64_t B, int64_t T,
                      int64_t H, int64_t W, int64_t ws0, int64_t ws1, int64_t s0, int64_t s1, int64_t sa,
                      int64_t sb, int dtype, void* stream) {
  const char* what = "nsw_linear_remap_residual";
  NSW_CHECK_ARG(bias && residual, "%s: bias and residual are required", what);
  NSW_CHECK_ARG(residual != (const void*)y, "%s: residual and y must not alias", what);
  NSW_CHECK_ARG(map_mode >= 0 && map_mode <= 3, "%s: map_mode must be 0, 1, 2 or 3", what);
  NSW_CHECK_ARG((row_sumsq != nullptr) == (map_mode != 1),
                "%s: row sums of squares are written for map modes 0, 2 and 3, and required there", what);
  EpiArgs ea{};
  ea.bias = bias; ea.residual = residual;
  if (map_mode != 0) {
    int rc = check_geom(B, T, H, W, ws0, ws1, what);
    if (rc) return rc;
    NSW_CHECK_ARG(M == B * T * H * W, "%s: M must be B*T*H*W for a row map", what);
    ea.geom = WinGeom::make((int)B, (int)T, (int)H, (int)W, (int)ws0, (int)ws1, (int)(s0 % H), (int)(s1 % W));
    const int64_t a = ((sa % H) + H) % H, b = ((sb % W) + W) % W;
    ea.dh = (int)(((ea.geom.s0 - a) % H + H) % H);
    ea.dw = (int)(((ea.geom.s1 - b) % W + W) % W);
  }
  ea.row_sumsq = row_sumsq;
  ea.nparts = (int)sumsq_parts(N, dtype);
  if (row_sumsq) NSW_CHECK_ARG(((uintptr_t)row_sumsq % 4) == 0, "%s: row_sumsq must be 4-byte aligned", what);
  if (map_mode == 0) {
    ea.group_m = N <= 1024 ? 16 : 0;   // proj-shaped (few column blocks): 16-row-block groups
    return dispatch_gemm<EPI_RES_SUMSQ>(dtype, x, w, y, M, N, K, ea, stream, what);
  }
  if (map_mode == 1) return dispatch_gemm<EPI_TOKEN_RESIDUAL>(dtype, x, w, y, M, N, K, ea, stream, what);
  if (map_mode == 3) return dispatch_gemm<EPI_WINDOW_RESIDUAL>(dtype, x, w, y, M, N, K, ea, stream, what);
  return dispatch_gemm<EPI_REMAP_RESIDUAL>(dtype, x, w, y, M, N, K, ea, stream, what);
}

}  // namespace nsw

using namespace nsw;

extern "C" int nsw_gemm_read_stamps(void* host, size_t bytes) {
#if NSW_GEMM_STAMPS
  NSW_CHECK_ARG(host != nullptr && bytes <= sizeof(uint64_t) * 8 * NSW_STAMP_TILES,
                "nsw_gemm_read_stamps: at most %zu bytes", sizeof(uint64_t) * 8 * (size_t)NSW_STAMP_TILES);
  if (hipMemcpyFromSymbol(host, HIP_SYMBOL(nsw_gemm_stamps), bytes, 0, hipMemcpyDeviceToHost) != hipSuccess)
    return set_error(NSW_ERR_HIP, "nsw_gemm_read_stamps: hipMemcpyFromSymbol failed");
  return 0;
#else
  (void)host; (void)bytes;
  return set_error(NSW_ERR_UNSUPPORTED, "nsw_gemm_read_stamps: library built without phase stamps (build.py --stamps)");
#endif
}

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
    case NSW_EPI_BIAS_GELU_TANH:
      return dispatch_gemm<EPI_BIAS_GELU_TANH>(dtype, x, w, y, M, N, K, ea, stream, what);
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
  return gemm_proj_scatter(o, wproj, bproj, skip, y, B, T, H, W, C, ws0, ws1, s0, s1, dtype, stream, nullptr);
}

extern "C" int64_t nsw_row_sumsq_parts(int64_t C, int dtype) { return C > 0 ? sumsq_parts(C, dtype) : 0; }

extern "C" int nsw_proj_reverse_residual_sumsq(const void* o, const void* wproj, const void* bproj,
                                               const void* skip, void* y, float* row_sumsq, int64_t B,
                                               int64_t T, int64_t H, int64_t W, int64_t C, int64_t ws0,
                                               int64_t ws1, int64_t s0, int64_t s1, int dtype, void* stream) {
  NSW_CHECK_ARG(row_sumsq != nullptr, "nsw_proj_reverse_residual_sumsq: row_sumsq is required");
  return gemm_proj_scatter(o, wproj, bproj, skip, y, B, T, H, W, C, ws0, ws1, s0, s1, dtype, stream, row_sumsq);
}

extern "C" int nsw_linear_rowscale(const void* x, const void* w_n, const void* bias, const void* residual,
                                   void* y, const float* row_sumsq, int64_t nparts, int64_t M, int64_t N,
                                   int64_t K, int epilogue, float eps, int dtype, void* stream) {
  return gemm_linear_rowscale(x, w_n, bias, residual, y, row_sumsq, nparts, M, N, K, epilogue, eps, dtype, stream);
}

extern "C" int nsw_qkv_projection_rowscale(const void* x, const void* wqkv_n, const void* bqkv, const void* qn_w,
                                           const void* kn_w, float eps, void* qkv, const float* row_sumsq,
                                           int64_t nparts, int64_t M, int64_t C, int64_t num_heads, int dtype,
                                           void* stream) {
  return gemm_qkv_rowscale(x, wqkv_n, bqkv, qn_w, kn_w, eps, qkv, row_sumsq, nparts, M, C, num_heads, dtype,
                           stream);
}

// The forecast head with its layout fused in: image = unpatchify(x . w_perm^T)
// (models/swin.py:286-299), w_perm the head weight with its rows permuted
// from the reference's (dy p + dx) C_out + c to c p^2 + dy p + dx.
int gemm_head_unpatchify(const void* x, const void* w_perm, void* out, int64_t B, int64_t C_out, int64_t H,
                         int64_t W, int64_t p, int64_t K, int64_t out_bstride, int dtype, int out_dtype,
                         void* stream) {
  const char* what = "nsw_head_unpatchify";
  NSW_CHECK_ARG(B > 0 && C_out > 0 && H > 0 && W > 0 && K > 0, "%s: B, C_out, H, W, K must be positive", what);
  NSW_CHECK_ARG(p == 1 || p == 2 || p == 4 || p == 8 || p == 16, "%s: p=%lld must be 1, 2, 4, 8 or 16", what,
                (long long)p);
  NSW_CHECK_ARG(H % p == 0 && W % p == 0, "%s: H=%lld, W=%lld not divisible by p=%lld", what, (long long)H,
                (long long)W, (long long)p);
  NSW_CHECK_ARG(dtype == NSW_DTYPE_BF16 || dtype == NSW_DTYPE_F32, "%s: unknown dtype %d", what, dtype);
  NSW_CHECK_ARG(out_dtype == dtype || out_dtype == NSW_DTYPE_F32,
                "%s: the image is in the GEMM's dtype or float32 (got %d for %d)", what, out_dtype, dtype);
  NSW_CHECK_ARG(out_bstride >= C_out * H * W && out_bstride % p == 0,
                "%s: out_bstride must cover one frame and be a multiple of p", what);
  const int64_t oes = out_dtype == NSW_DTYPE_F32 ? 4 : 2;
  NSW_CHECK_ARG(((uintptr_t)out % (uintptr_t)std::min<int64_t>(16, p * oes)) == 0,
                "%s: out must be aligned to min(16, p * element size) bytes", what);
  NSW_CHECK_ARG(B * out_bstride < (1LL << 40) && H * W < (1LL << 31), "%s: image too large", what);
  EpiArgs ea{};
  ea.img = out;
  ea.img_bstride = out_bstride;
  ea.img_C = (int)C_out; ea.img_H = (int)H; ea.img_W = (int)W; ea.img_p = (int)p;
  ea.img_f32 = out_dtype == NSW_DTYPE_F32 && dtype == NSW_DTYPE_BF16;
  const int64_t M = B * (H / p) * (W / p);
  return dispatch_gemm<EPI_UNPATCH>(dtype, x, w_perm, nullptr, M, C_out * p * p, K, ea, stream, what);
}

extern "C" int nsw_head_unpatchify(const void* x, const void* w_perm, void* out, int64_t B, int64_t C_out,
                                   int64_t H, int64_t W, int64_t p, int64_t K, int64_t out_bstride, int dtype,
                                   int out_dtype, void* stream) {
  return gemm_head_unpatchify(x, w_perm, out, B, C_out, H, W, p, K, out_bstride, dtype, out_dtype, stream);
}

extern "C" int nsw_linear_remap_residual(const void* x, const void* w, const void* bias, const void* residual,
                                         void* y, float* row_sumsq, int64_t M, int64_t N, int64_t K, int map_mode,
                                         int64_t B, int64_t T, int64_t H, int64_t W, int64_t ws0, int64_t ws1,
                                         int64_t s0, int64_t s1, int64_t sa, int64_t sb, int dtype,
                                         void* stream) {
  return gemm_linear_remap(x, w, bias, residual, y, row_sumsq, M, N, K, map_mode, B, T, H, W, ws0, ws1, s0, s1,
                           sa, sb, dtype, stream);
}
