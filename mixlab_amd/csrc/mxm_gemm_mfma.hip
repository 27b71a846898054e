// Grouped expert FFN on bf16 MFMA (gfx950, v_mfma_f32_32x32x16_bf16).
//
// One workgroup computes a BM x BN tile of one expert's output.  A rows are
// the expert's permuted slots: for the up projections they are gathered from
// x through `perm` (each row is D contiguous bf16), for the down projection
// they are the contiguous rows of H.  B is the expert's weight stored
// transposed ([out, in], k contiguous) so both operands stream k-contiguous
// 16-byte chunks.
//
// Operand tiles move global -> LDS with global_load_lds_dwordx4 (no VGPR
// round trip) into a ring of NS stages of BK k each; each lane's 16-byte
// chunk lands at a swizzled position so the 16-lane phases of ds_read_b128
// hit distinct banks.  Waves wait for their own loads with explicit vmcnt
// counts and meet at s_barrier; the loads of the next stage are spread over
// the first k steps of the current one so the vector memory path fills in
// the background.  With three or more stages the barrier of stage kt+1 is
// taken before the last k step of stage kt, so it overlaps MFMA work.
//
// Tile families (flags select; the default is 256 x 256 where the columns
// allow): 256 x 256 x 64 (8 waves as 2 x 4, each 128 x 64 = 4 x 2 MFMA tiles,
// 2 stages), 256 x 128 x 32 (4 waves, 3 stages, 2 workgroups per CU) and
// 128 x 128 x 64 (4 waves, 2 stages).  The GLU weight rows are interleaved in
// groups of 32 (gate cols f..f+31, then up cols f..f+31), so a wave's two
// column MFMA tiles hold gate and up for the same 32 hidden units and the
// activation is applied straight from the accumulators.
//
// Ragged experts: the scan kernel writes `mstart`, the prefix over experts of
// ceil(count/BM) row tiles, so tile -> (expert, rows) is resolved on device
// (one round of loads and a ballot) and tiles past the end are skipped.
//
// The grid is persistent: as many workgroups as fit on the device at once,
// each walking launch indices w, w + gridDim.x, ...; a CU goes from one
// tile's epilogue straight to the next tile while the stores drain, instead
// of waiting for the workgroup to retire and a new one to be dispatched.
//
// Tile order: the hardware hands workgroup L to XCD L % 8.  Row tiles are
// grouped GM at a time with the column tiles of a group adjacent, and group g
// is placed on XCD g % 8, so each XCD's L2 sees a GM x (N/BN) block of tiles
// sharing A rows and B columns, and the empty tail tiles are spread over all
// XCDs.  The epilogue applies the activation (hardware exp2 / rcp and bf16
// conversion), stages each wave's bf16 tile through LDS (chunk-swizzled) and
// writes 16-byte row segments.
#include <algorithm>

#include "mxm_kernels.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Native vector type for 16-byte moves (HIP's uint4 wrapper class defeats
// scalar replacement of the prefetch registers).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

#ifndef MXM_DMA_STEPS
#define MXM_DMA_STEPS 2
#endif

#ifndef MXM_GM
#define MXM_GM 6
#endif
constexpr int GM = MXM_GM;        // row tiles per scheduling group

// Physical 16-byte chunk of logical chunk kc in tile row `row` (CH chunks per
// row).  ds_read_b128 is serviced 16 lanes (16 consecutive rows, one chunk)
// at a time over 64 four-byte banks = 16 groups of 16 bytes; rows r and
// r + 16/CH fall in the same groups, so the CH rows of a phase that share
// them get distinct chunks.
template <int CH>
__device__ __forceinline__ int swz_phys(int row, int kc) {
  return kc ^ ((row / (16 / CH)) % CH);
}
template <int CH>
__device__ __forceinline__ int swz(int row, int kc) {
  return row * CH + swz_phys<CH>(row, kc);
}

__device__ __forceinline__ int find_expert(const int32_t* mstart, int E, int mtile) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (mstart[mid] <= mtile)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// Row tile mtile -> its expert e, first row row0 and the expert's row end.
// Returns false for tiles past the last expert's.  For E <= 64 this is one
// round of independent loads: lane l reads mstart[l + 1], offsets[l] and
// offsets[l + 1]; since mstart is nondecreasing from mstart[0] = 0, e is the
// number of i in 1..E-1 with mstart[i] <= mtile (a ballot), and the rest are
// read from the lanes holding them.  A binary search would be log2(E)
// dependent loads, each a full L2 round trip, before the tile's first
// operand load could be issued.
__device__ __forceinline__ bool locate_tile(const int32_t* mstart, const int32_t* offsets, int E,
                                            int mtile, int BM, int& e, int& row0, int& rend) {
  if (E <= 64) {
    const int lane = threadIdx.x & 63;
    const bool in = lane < E;
    const int ms1 = in ? mstart[lane + 1] : 0x7fffffff;
    const int of0 = in ? offsets[lane] : 0;
    const int of1 = in ? offsets[lane + 1] : 0;
    if (mtile >= __builtin_amdgcn_readlane(ms1, E - 1)) return false;
    e = __popcll(__ballot(lane + 1 < E && ms1 <= mtile));
    const int ms_e = e == 0 ? 0 : __builtin_amdgcn_readlane(ms1, e - 1);
    row0 = __builtin_amdgcn_readlane(of0, e) + (mtile - ms_e) * BM;
    rend = __builtin_amdgcn_readlane(of1, e);
    return true;
  }
  if (mtile >= mstart[E]) return false;
  e = find_expert(mstart, E, mtile);
  row0 = offsets[e] + (mtile - mstart[e]) * BM;
  rend = offsets[e + 1];
  return true;
}

// Direct global->LDS load of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's data lands at LDS address `lds` + 16*l.  Issued as inline asm so
// the compiler does not track it: its conservative tracking of LDS DMA would
// otherwise drain every in-flight stage before the next LDS read.  The caller
// waits with explicit vmcnt counts (stage_barrier) before reading.  M0 holds
// the LDS base; nothing else in these kernels uses M0.
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
  const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(base)
               : "memory", "m0");
}

// The same load from a uniform 64-bit base in SGPRs plus the lane's 32-bit
// byte offset (the SGPR-base form: no 64-bit address arithmetic per load).
__device__ __forceinline__ void dma16s(const void* base, unsigned off_bytes, const void* lds) {
  const unsigned lb = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off_bytes), "s"(base), "s"(lb)
               : "memory", "m0");
}

// Wait until at most N of this thread's direct-to-LDS loads are in flight and
// its LDS reads are done, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Tile family: BM x BN workgroup tile, WM x WN waves, each wave
// (BM/WM) x (BN/WN) = TM x TN MFMA 32x32 tiles.
template <int BM, int BN, int WM, int WN, int WAVES_PER_SIMD, int NSTAGE, int BKK>
struct Tile {
  static constexpr int NS = NSTAGE;
  static constexpr int BK = BKK;      // k per LDS stage
  static constexpr int CH = BKK / 8;  // 16-byte chunks per tile row
  static constexpr int NT = 64 * WM * WN;
  static constexpr int TM = BM / WM / 32;
  static constexpr int TN = BN / WN / 32;
  static constexpr int A_CH = BM * CH;
  static constexpr int B_CH = BN * CH;
  static constexpr int BUF = A_CH + B_CH;
  static constexpr int LA = A_CH / NT;
  static constexpr int LB = B_CH / NT;
  static constexpr int WPS = WAVES_PER_SIMD;
  static_assert(TN % 2 == 0, "GLU epilogue pairs gate and up column tiles");
  static_assert(A_CH % NT == 0 && B_CH % NT == 0, "whole chunks per thread");
};

template <class TL, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(TL::NT, TL::WPS * 256 / TL::NT) void gemm_kernel(GemmArgs a,
                                                                            int ngroups,
                                                                            int nblocks) {
  constexpr int MODE = Epi<EPI>::MODE;
  constexpr bool DOWN_SPLIT = Epi<EPI>::DOWN_SPLIT;  // A = [hi | lo] planes, y in fp32
  // 32-bit A offsets (when A fits) for the forward's up projections only:
  // measured faster there, slower for the down projection and no faster
  // for the raw-keeping variant
  constexpr bool A_OFF32 = MODE != MXM_GEMM_DOWN && !Epi<EPI>::KEEP_RAW;
  constexpr bool H_SPLIT = Epi<EPI>::H_SPLIT;        // H stored as [hi | lo] planes
  constexpr int NT = TL::NT, TM = TL::TM, TN = TL::TN;
  constexpr int A_CH = TL::A_CH, BUF = TL::BUF;
  constexpr int NW = NT / 64;
  constexpr int NS = TL::NS;  // LDS stages in the ring (NS-1 in flight)
  constexpr int BK = TL::BK, CH = TL::CH;
  __shared__ u32x4_t lds[NS * BUF];

  // XCD-aware grouped schedule (see the file comment).
  const int ntile_n = a.Ncols / BN;
  const int per_group = GM * ntile_n;
  // The grid is persistent (as many workgroups as fit at once): workgroup w
  // takes launch indices w, w + gridDim.x, ..., so the CU goes straight from
  // one tile's epilogue to the next tile while the epilogue's stores drain.
  // gridDim.x is a multiple of 8, so every index keeps the workgroup's XCD.
  for (int L = blockIdx.x; L < nblocks; L += gridDim.x) {
  // every wave has read the previous tile's epilogue staging out of LDS
  // (plain s_barrier: no wait for that epilogue's stores)
  if (L != (int)blockIdx.x) asm volatile("s_barrier" ::: "memory");
  const int local = L >> 3;
  const int g = (local / per_group) * 8 + (L & 7);
  if (g >= ngroups) break;  // g only grows with L
  const int rr = local % per_group;
  const int mtile = g * GM + rr % GM;
  const int ntile = rr / GM;
  int e, row0, rend;
  if (!locate_tile(a.mstart, a.offsets, a.E, mtile, BM, e, row0, rend)) continue;
  const int rows = min(BM, rend - row0);
  const int n0 = ntile * BN;
  const int Kd = a.Kd;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // int8 weights (the bf16 B holds the integers q): this lane's output
  // columns' scales, read before the k loop so their latency is hidden.
  // Lane l's accumulators of column tile j are column j*32 + l%32 of the
  // wave's; GLU tiles alternate gate (scale0) and up (scale1) over the same
  // 32 hidden units.
  float scv[TN];
  if constexpr (Epi<EPI>::SCALED) {
    const int wc0 = n0 + wn * TN * 32;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (MODE == MXM_GEMM_GLU) {
        const int hc = a.Ncols / 2;
        const float* sp = (j & 1) ? a.scale1 : a.scale0;
        scv[j] = sp[(size_t)e * hc + wc0 / 2 + (j >> 1) * 32 + (lane & 31)];
      } else {
        scv[j] = a.scale0[(size_t)e * a.Ncols + wc0 + j * 32 + (lane & 31)];
      }
    }
  }

  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(a.a);
  // B rows hold Kb k values; the split down projection reads W_down [D][F]
  // twice along its reduction over the hi and lo planes (k wraps at F)
  const int Kb = DOWN_SPLIT ? Kd / 2 : Kd;
  const uint16_t* __restrict__ B =
      static_cast<const uint16_t*>(a.b0) + (size_t)e * a.Ncols * Kb;

  // Global->LDS: global_load_lds_dwordx4 writes lane l's 16 bytes to
  // LDS base + 16*l, so one wave-load fills 1 KB = 64/CH consecutive tile
  // rows.  Lane l lands in row (l/CH) of its group at physical chunk l%CH and
  // fetches the logical k-chunk stored there -- the swizzle is applied on the
  // global address.
  constexpr int RPW = 64 / CH;     // tile rows per wave-load
  constexpr int QA = BM / RPW / NW;  // A wave-loads per wave per stage
  constexpr int QB = BN / RPW / NW;
  constexpr int LDPS = QA + QB;      // direct-to-LDS loads per thread per stage
  static_assert(QA * RPW * NW == BM && QB * RPW * NW == BN, "whole wave-loads");
  const int lrow = lane / CH;  // row within the wave-load group
  // Logical chunk of this lane's physical slot (the swizzle is an involution).
  // It depends on the tile row modulo 16; the row of load i is
  // (wave + NW*i)*RPW + lrow, which is the same modulo 16 for every i because
  // NW*RPW is a multiple of 16.
  static_assert((NW * RPW) % 16 == 0, "swizzle phase is the same for every wave-load of a lane");
  const int lkc = swz_phys<CH>(wave * RPW + lrow, lane % CH);
  size_t aoff[QA];
#pragma unroll
  for (int i = 0; i < QA; ++i) {
    const int r = (wave + NW * i) * RPW + lrow;
    const int p = row0 + min(r, rows - 1);  // rows past the segment reload a valid row
    const int src = (MODE == MXM_GEMM_DOWN && !a.gather_a) ? p : a.perm[p];
    aoff[i] = 2 * ((size_t)src * Kd + lkc * 8);  // bytes
  }
  const size_t bstep = (size_t)(NW * RPW) * Kb;
  // the B loads as 32-bit byte offsets from the expert's matrix (one expert's
  // Ncols x Kb bf16 stays far below 4 GiB); the wave index in an SGPR keeps
  // every load's LDS destination scalar
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const unsigned boff = (unsigned)(2 * ((size_t)(n0 + wv * RPW + lrow) * Kb + lkc * 8));
  const unsigned bstep_b = (unsigned)(2 * bstep);

// Direct-to-LDS loads Q0 .. Q1-1 of one stage (load q < QA fills A rows,
// the rest B rows).
#define MXM_DMA_LOOP(STAGE, K0, Q0, Q1, ALOAD)                                                \
  _Pragma("unroll") for (int q_ = (Q0); q_ < (Q1); ++q_) {                                    \
    if (q_ < QA) {                                                                            \
      ALOAD;                                                                                  \
    } else {                                                                                  \
      dma16s(B + (DOWN_SPLIT && (K0) >= Kb ? (K0) - Kb : (K0)), boff + (q_ - QA) * bstep_b,   \
             STAGE + A_CH + (wv + NW * (q_ - QA)) * 64);                                      \
    }                                                                                         \
  }
#define MXM_DMA_PART(STAGE, K0, Q0, Q1)                                                       \
  do {                                                                                        \
    if (A_OFF32 && a.a_off32) {                                                               \
      MXM_DMA_LOOP(STAGE, K0, Q0, Q1,                                                         \
                   dma16s(A + (K0), (unsigned)aoff[q_], STAGE + (wv + NW * q_) * 64))         \
    } else {                                                                                  \
      MXM_DMA_LOOP(STAGE, K0, Q0, Q1,                                                         \
                   dma16(reinterpret_cast<const char*>(A + (K0)) + aoff[q_],                  \
                         STAGE + (wv + NW * q_) * 64))                                        \
    }                                                                                         \
  } while (0)
#define MXM_DMA(STAGE, K0) MXM_DMA_PART(STAGE, K0, 0, LDPS)
  // Stage barrier: this thread's loads of the current stage have landed (at
  // most AHEAD later stages still in flight), then the workgroup barrier --
  // the stage is complete for every wave and the stage consumed in the
  // previous step is free.
#define MXM_STAGE_BARRIER(AHEAD)              \
  do {                                        \
    if ((AHEAD) >= 3)                         \
      stage_barrier<3 * LDPS>();              \
    else if ((AHEAD) == 2)                    \
      stage_barrier<2 * LDPS>();              \
    else if ((AHEAD) == 1)                    \
      stage_barrier<LDPS>();                  \
    else                                      \
      stage_barrier<0>();                     \
  } while (0)
  static_assert(NS >= 2 && NS <= 5, "stage barrier counts cover up to three stages ahead");
  static_assert(3 * LDPS <= 63, "vmcnt holds at most 63 outstanding loads");

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Fragment registers are double-buffered across the 16-wide k steps: the
  // reads for step ks+1 are issued before the MFMAs of step ks.
  const int arow = wm * TM * 32 + (lane & 31);
  const int brow = wn * TN * 32 + (lane & 31);
  bf16x8_t af[2][TM], bfm[2][TN];

#define MXM_FRAGS(STAGE, P, KS)                                                               \
  do {                                                                                        \
    const int kc_ = (KS) * 2 + (lane >> 5);                                                   \
    /* B first: the first MFMA needs b0 and a0, so it waits for TN + 1 reads */               \
    _Pragma("unroll") for (int j = 0; j < TN; ++j) bfm[P][j] =                                \
        __builtin_bit_cast(bf16x8_t, (STAGE)[A_CH + swz<CH>(brow + j * 32, kc_)]);            \
    _Pragma("unroll") for (int i = 0; i < TM; ++i) af[P][i] =                                 \
        __builtin_bit_cast(bf16x8_t, (STAGE)[swz<CH>(arow + i * 32, kc_)]);                   \
  } while (0)
// Per 16-wide k step: the fragment reads of the next step are interleaved
// one by one between the MFMAs of this step (sched_group_barrier pins the
// order: 1 MFMA, 1 LDS read, ...), so LDS latency hides behind MFMAs.  After
// the stage barrier the first step's TM + TN reads are all issued before its
// first MFMA, so the stage start costs one LDS latency rather than a read,
// wait, MFMA chain.  After
// each step, a share of the direct-to-LDS loads of stage DSTAGE (k offset
// DK0) is issued, so the vector memory path fills in the background instead
// of stalling every wave right after the stage barrier.
#define MXM_COMPUTE(STAGE, DO_DMA, DSTAGE, DK0)                                               \
  do {                                                                                        \
    MXM_FRAGS(STAGE, 0, 0);                                                                   \
    _Pragma("unroll") for (int ks = 0; ks < BK / 16; ++ks) {                                  \
      if (ks + 1 < BK / 16) MXM_FRAGS(STAGE, (ks + 1) & 1, ks + 1);                           \
      _Pragma("unroll") for (int i = 0; i < TM; ++i)                                          \
          _Pragma("unroll") for (int j = 0; j < TN; ++j) acc[i][j] =                          \
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfm[ks & 1][j],          \
                                                      acc[i][j], 0, 0, 0);                    \
      if (ks + 1 < BK / 16) {                                                                 \
        if (ks == 0) /* the first step's fragments all go out before its MFMAs */             \
          __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);                            \
        _Pragma("unroll") for (int q = 0; q < TM * TN; ++q) {                                 \
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                  \
          if (q < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                 \
        }                                                                                     \
      }                                                                                       \
      if ((DO_DMA) && ks < DSTEPS)                                                            \
        MXM_DMA_PART(DSTAGE, DK0, ks * LDPS / DSTEPS, (ks + 1) * LDPS / DSTEPS);              \
    }                                                                                         \
  } while (0)

// One 16-wide k step on fragment set P; if DOFRAG, the fragments of k step
// FKS of stage FSTAGE are read into set P^1 in between the MFMAs.
#define MXM_KSTEP(P, FSTAGE, FKS, DOFRAG)                                                     \
  do {                                                                                        \
    if (DOFRAG) MXM_FRAGS(FSTAGE, (P) ^ 1, FKS);                                              \
    _Pragma("unroll") for (int i = 0; i < TM; ++i)                                            \
        _Pragma("unroll") for (int j = 0; j < TN; ++j) acc[i][j] =                            \
            __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[P][i], bfm[P][j], acc[i][j], 0, 0, 0); \
    if (DOFRAG) {                                                                             \
      _Pragma("unroll") for (int q = 0; q < TM * TN; ++q) {                                   \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                    \
        if (q < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                   \
      }                                                                                       \
    }                                                                                         \
  } while (0)

  // k steps over which the next stage's loads are spread
  constexpr int DSTEPS = (MXM_DMA_STEPS > 0 && MXM_DMA_STEPS < BK / 16) ? MXM_DMA_STEPS : BK / 16;
  constexpr int KS = BK / 16;
  const int nk = Kd / BK;
  // first stage: the weight rows go out first, they do not wait for perm
  if (nk > 0) {
    MXM_DMA_PART(lds, 0, QA, LDPS);
    MXM_DMA_PART(lds, 0, 0, QA);
  }
#pragma unroll
  for (int st = 1; st < NS - 1; ++st)
    if (st < nk) MXM_DMA(lds + st * BUF, st * BK);
  if constexpr (NS >= 3) {
    // Deep ring: the barrier of stage kt+1 is taken before the last k step
    // of stage kt, while that step's fragments are already in registers and
    // the MFMAs issued just before it are still executing, so the barrier
    // and the first fragment reads of the next stage overlap MFMA work.  At
    // that barrier stage kt+1 has landed and stage kt-1 is free; it receives
    // stage kt+NS-1.
    static_assert(KS % 2 == 0, "fragment set parity repeats every stage");
    MXM_STAGE_BARRIER(min(NS - 2, nk - 1));
    MXM_FRAGS(lds, 0, 0);
    // (the last stage is peeled so the accumulators flow through one path)
    for (int kt = 0; kt < nk - 1; ++kt) {
      const u32x4_t* cur = lds + (kt % NS) * BUF;
#pragma unroll
      for (int ks = 0; ks < KS - 1; ++ks) MXM_KSTEP(ks & 1, cur, ks + 1, true);
      MXM_STAGE_BARRIER(min(NS - 3, nk - 2 - kt));
      if (kt + NS - 1 < nk) MXM_DMA(lds + ((kt + NS - 1) % NS) * BUF, (kt + NS - 1) * BK);
      MXM_KSTEP((KS - 1) & 1, lds + ((kt + 1) % NS) * BUF, 0, true);
    }
    {
      const u32x4_t* cur = lds + ((nk - 1) % NS) * BUF;
#pragma unroll
      for (int ks = 0; ks < KS - 1; ++ks) MXM_KSTEP(ks & 1, cur, ks + 1, true);
      MXM_KSTEP((KS - 1) & 1, cur, 0, false);
    }
  } else {
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt is complete and the stage consumed at kt-1 is free; it
      // receives stage kt+NS-1 while the MFMAs of stage kt run
      MXM_STAGE_BARRIER(min(NS - 2, nk - 1 - kt));
      const u32x4_t* cur = lds + (kt % NS) * BUF;
      const bool more = kt + NS - 1 < nk;
      MXM_COMPUTE(cur, more, lds + ((kt + NS - 1) % NS) * BUF, (kt + NS - 1) * BK);
    }
  }
  MXM_STAGE_BARRIER(0);  // every wave is done reading before the staging reuse
#undef MXM_DMA
#undef MXM_DMA_PART
#undef MXM_STAGE_BARRIER
#undef MXM_FRAGS
#undef MXM_COMPUTE
#undef MXM_KSTEP

  if constexpr (Epi<EPI>::SCALED) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] *= scv[j];
  }
  if constexpr (Epi<EPI>::Y_F32) {
    // y in fp32, straight from the accumulators: register r of lane l holds
    // C[(r/4)*8 + (l/32)*4 + r%4][l%32], so each store instruction writes
    // 32 consecutive floats of two rows
    float* __restrict__ yo = static_cast<float*>(a.out);
    const int ycol = n0 + wn * TN * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = wm * TM * 32 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (lr < rows) {
#pragma unroll
          for (int j = 0; j < TN; ++j)
            __builtin_nontemporal_store(acc[i][j][r],
                                        yo + (size_t)(row0 + lr) * a.Ncols + ycol + j * 32);
        }
      }
    continue;
  }
  // ---- epilogue: activation, bf16, per-wave LDS staging, 16-byte stores ----
  // 32x32 accumulator layout: register r of lane l holds
  // C[(r/4)*8 + (l/32)*4 + r%4][l%32].  Registers r and r+1 (r even) hold two
  // consecutive rows of one column; they are converted together and staged
  // as one 32-bit word (low half the even row) of a row-pair line, so a wave
  // writes half as many LDS words as it has outputs.  Lines hold C words (the
  // wave's output columns).  Staging swizzle, with kp the row pair:
  //   C = 64: line kp, 16-byte chunk ch -> ch ^ (kp & 1) ^ ((kp >> 1 & 1) << 3)
  //   C = 32: line kp ^ (kp >> 1 & 1), chunk ch -> ch ^ (kp >> 1 & 1)
  // A write instruction covers 32 columns of row pairs kp and kp + 2 (the two
  // half-waves), which land in disjoint banks; a read instruction's 16-lane
  // phases take two 16-byte chunks of four (C = 32) or two (C = 64) row
  // pairs, also in disjoint banks.
  constexpr int WROWS = TM * 32;
  constexpr int C = (MODE == MXM_GEMM_GLU) ? TN * 16 : TN * 32;  // output columns per wave
  static_assert(C == 32 || C == 64, "staging swizzle covers 32 or 64 columns per wave");
  static_assert(NW * WROWS * C * 2 <= (int)sizeof(u32x4_t) * NS * BUF, "staging fits in LDS");
  uint32_t* stage = reinterpret_cast<uint32_t*>(lds) + (size_t)wave * (WROWS / 2) * C;
  auto word_at = [](int kp, int c) -> int {
    const int b1 = (kp >> 1) & 1;
    if constexpr (C == 64) {
      const int ch = (c >> 2) ^ (kp & 1) ^ (b1 << 3);
      return kp * C + ch * 4 + (c & 3);
    } else {
      const int ch = (c >> 2) ^ b1;
      return (kp ^ b1) * C + ch * 4 + (c & 3);
    }
  };
  const int col = lane & 31;
  if constexpr (Epi<EPI>::KEEP_RAW) {
    // the raw bf16 projections (all TN column tiles: gate and up interleaved
    // as W1's rows) to out2, through the same staging with 64 columns per
    // wave, before the activation overwrites the accumulators
    constexpr int CR = TN * 32;
    static_assert(CR == 64 && NW * WROWS * CR * 2 <= (int)sizeof(u32x4_t) * NS * BUF,
                  "raw staging fits in LDS");
    uint32_t* rst = reinterpret_cast<uint32_t*>(lds) + (size_t)wave * (WROWS / 2) * CR;
    auto rword = [](int kp, int c) -> int {
      const int b1 = (kp >> 1) & 1;
      const int ch = (c >> 2) ^ (kp & 1) ^ (b1 << 3);
      return kp * CR + ch * 4 + (c & 3);
    };
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const int kp = i * 16 + (r >> 2) * 4 + (lane >> 5) * 2 + ((r & 3) >> 1);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          rst[rword(kp, j * 32 + col)] = mxm_pack_bf2_fast(acc[i][j][r], acc[i][j][r + 1]);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint16_t* __restrict__ rout = static_cast<uint16_t*>(a.out2);
    constexpr int RSEGS = CR / 8;
#pragma unroll
    for (int it = 0; it < (WROWS / 2) * RSEGS / 64; ++it) {
      const int q = lane + 64 * it;
      const int kp = q / RSEGS, sg = q % RSEGS;
      const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(rst + rword(kp, sg * 8));
      const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(rst + rword(kp, sg * 8 + 4));
      const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      u32x4_t lo, hi;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        lo[m] = __builtin_amdgcn_perm(wv[2 * m + 1], wv[2 * m], 0x05040100u);
        hi[m] = __builtin_amdgcn_perm(wv[2 * m + 1], wv[2 * m], 0x07060302u);
      }
      const int grow = wm * WROWS + 2 * kp;
      const int c0r = n0 + wn * CR + sg * 8;
      if (grow < rows)
        *reinterpret_cast<u32x4_t*>(rout + (size_t)(row0 + grow) * a.Ncols + c0r) = lo;
      if (grow + 1 < rows)
        *reinterpret_cast<u32x4_t*>(rout + (size_t)(row0 + grow + 1) * a.Ncols + c0r) = hi;
    }
    // every wave's staging reads are done before the next tile's loads
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    continue;  // no hidden: the backward's activation pass derives it
  }
  // kinds whose hidden is fp32 store it as two bf16 planes (hi, then lo =
  // bf16(h - hi)) through the same staging, one plane after the other
  constexpr int NPLANE = H_SPLIT ? 2 : 1;
  if constexpr (H_SPLIT) {
    // the fp32 hidden, computed once in place: h overwrites the gate
    // accumulator (GLU) or the projection's (MLP), which are dead after it
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (MODE == MXM_GEMM_GLU) {
#pragma unroll
          for (int pj = 0; pj < TN / 2; ++pj)
            acc[i][2 * pj][r] = mxm_hidden_fast<true>(
                Epi<EPI>::ETYPE, Epi<EPI>::ACT, a.slope, mxm_rbf_fast(acc[i][2 * pj][r]),
                mxm_rbf_fast(acc[i][2 * pj + 1][r]));
        } else {
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j][r] = mxm_hidden_fast<true>(MXM_EXPERT_MLP, Epi<EPI>::ACT, a.slope, 0.0f,
                                                 mxm_rbf_fast(acc[i][j][r]));
        }
      }
  }
#pragma unroll
  for (int plane = 0; plane < NPLANE; ++plane) {
  if (plane > 0) {
    // this wave's reads of the previous plane's staging are complete
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const int kp = i * 16 + (r >> 2) * 4 + (lane >> 5) * 2 + ((r & 3) >> 1);
      if (MODE == MXM_GEMM_GLU) {
#pragma unroll
        for (int pj = 0; pj < TN / 2; ++pj) {
          float h[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            if constexpr (H_SPLIT) {  // h computed above; plane 1 holds h - bf16(h)
              h[q] = acc[i][2 * pj][r + q];
              if (plane == 1) h[q] = h[q] - mxm_rbf_fast(h[q]);
            } else {
              const float gg = mxm_rbf_fast(acc[i][2 * pj][r + q]);
              const float u = mxm_rbf_fast(acc[i][2 * pj + 1][r + q]);
              h[q] = mxm_hidden_fast<true>(Epi<EPI>::ETYPE, Epi<EPI>::ACT, a.slope, gg, u);
            }
          }
          stage[word_at(kp, pj * 32 + col)] = mxm_pack_bf2_fast(h[0], h[1]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            v[q] = acc[i][j][r + q];
            if constexpr (H_SPLIT) {  // h computed above
              if (plane == 1) v[q] = v[q] - mxm_rbf_fast(v[q]);
            } else if (MODE == MXM_GEMM_MLP) {
              v[q] = mxm_hidden_fast<true>(MXM_EXPERT_MLP, Epi<EPI>::ACT, a.slope, 0.0f,
                                           mxm_rbf_fast(v[q]));
            }
          }
          stage[word_at(kp, j * 32 + col)] = mxm_pack_bf2_fast(v[0], v[1]);
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // each lane takes 8 columns of one row pair: two 16-byte chunks, split by
  // byte permutes into the even row's and the odd row's 16-byte segments
  const int hcols = (MODE == MXM_GEMM_GLU) ? a.Ncols / 2 : a.Ncols;  // F (up) or D (down)
  const int ldo = H_SPLIT ? 2 * hcols : hcols;
  const int c0 = n0 / (MODE == MXM_GEMM_GLU ? 2 : 1) + wn * C + plane * hcols;
  uint16_t* __restrict__ out = static_cast<uint16_t*>(a.out);
  constexpr int SEGS = C / 8;  // 8-column segments per row pair
#pragma unroll
  for (int it = 0; it < (WROWS / 2) * SEGS / 64; ++it) {
    const int q = lane + 64 * it;
    const int kp = q / SEGS, sg = q % SEGS;
    const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(stage + word_at(kp, sg * 8));
    const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(stage + word_at(kp, sg * 8 + 4));
    const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    u32x4_t lo, hi;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      lo[m] = __builtin_amdgcn_perm(wv[2 * m + 1], wv[2 * m], 0x05040100u);  // low halves
      hi[m] = __builtin_amdgcn_perm(wv[2 * m + 1], wv[2 * m], 0x07060302u);  // high halves
    }
    const int grow = wm * WROWS + 2 * kp;
    // Y (down projection) is read once, by the combine, and is several times
    // the last-level cache: stored nontemporal.  H stays cached for the down
    // GEMM's re-reads.
    u32x4_t* d0 = reinterpret_cast<u32x4_t*>(out + (size_t)(row0 + grow) * ldo + c0 + sg * 8);
    u32x4_t* d1 = reinterpret_cast<u32x4_t*>(out + (size_t)(row0 + grow + 1) * ldo + c0 + sg * 8);
    if constexpr (MODE == MXM_GEMM_DOWN) {
      if (grow < rows) __builtin_nontemporal_store(lo, d0);
      if (grow + 1 < rows) __builtin_nontemporal_store(hi, d1);
    } else {
      if (grow < rows) *d0 = lo;
      if (grow + 1 < rows) *d1 = hi;
    }
  }
  }  // plane loop
  }  // tile loop
}

// Workgroups resident at once on the current device: CUs x workgroups per
// CU, rounded down to a multiple of 8 so a workgroup's tiles all map to the
// XCD it runs on.
static int persistent_grid(int per_cu) {
  static int ncu[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (ncu[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    ncu[dev] = n;
  }
  return std::max(8, ncu[dev] * per_cu / 8 * 8);
}

template <int BM, int BN, int WM, int WN, int WPS, int NSTG, int BKK, int EPI>
void launch_epi(const GemmArgs& a, hipStream_t s, int blocks, int ngroups) {
  using TL = Tile<BM, BN, WM, WN, WPS, NSTG, BKK>;
  // workgroups per CU: what the launch bounds allow, capped by LDS
  constexpr int lds_bytes = NSTG * TL::BUF * 16;
  constexpr int per_cu = std::min(TL::WPS * 256 / TL::NT, 160 * 1024 / lds_bytes);
  const int grid = std::min(blocks, persistent_grid(std::max(1, per_cu)));
  hipLaunchKernelGGL((gemm_kernel<TL, BM, BN, WM, WN, EPI>), dim3(grid), dim3(TL::NT), 0, s, a,
                     ngroups, blocks);
}

template <int BM, int BN, int WM, int WN, int WPS, int NSTG, int BKK>
void launch_family(const GemmArgs& a, hipStream_t s);

// An up projection that also keeps its raw projections (GemmArgs::out2),
// or whose weights are int8 integers with per-column scales (scale0).
template <int BM, int BN, int WM, int WN, int WPS, int NSTG, int BKK, int EPI>
void launch_up(const GemmArgs& a, hipStream_t s, int blocks, int ngroups) {
  if (a.out2)
    launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_KEEP + EPI>(a, s, blocks, ngroups);
  else if (a.scale0)
    launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_SCALE + EPI>(a, s, blocks, ngroups);
  else
    launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI>(a, s, blocks, ngroups);
}

template <int BM, int BN, int WM, int WN, int WPS, int NSTG, int BKK>
void launch_family(const GemmArgs& a, hipStream_t s) {
  const int ngroups = (a.max_mtiles + GM - 1) / GM;
  const int per_group = GM * (a.Ncols / BN);
  const int blocks = ((ngroups + 7) / 8) * 8 * per_group;
  if (a.mode == MXM_GEMM_DOWN) {
    if (a.scale0 && a.h_split)
      launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_SCALE + EPI_DOWN_F32>(a, s, blocks, ngroups);
    else if (a.scale0)
      launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_SCALE + EPI_DOWN>(a, s, blocks, ngroups);
    else if (a.h_split)
      launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_DOWN_F32>(a, s, blocks, ngroups);
    else if (a.f32_out)
      launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_F32>(a, s, blocks, ngroups);
    else
      launch_epi<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_DOWN>(a, s, blocks, ngroups);
    return;
  }
  switch (mxm_epi_kind(a.expert_type, a.activation)) {
    case EPI_GEGLU:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_GEGLU>(a, s, blocks, ngroups);
      break;
    case EPI_MLP_SILU:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_MLP_SILU>(a, s, blocks, ngroups);
      break;
    case EPI_MLP_GELU:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_MLP_GELU>(a, s, blocks, ngroups);
      break;
    case EPI_MLP_RELU:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_MLP_RELU>(a, s, blocks, ngroups);
      break;
    case EPI_MLP_LEAKY:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_MLP_LEAKY>(a, s, blocks, ngroups);
      break;
    default:
      launch_up<BM, BN, WM, WN, WPS, NSTG, BKK, EPI_SWIGLU>(a, s, blocks, ngroups);
      break;
  }
}

}  // namespace

int mxm_mfma_tile_rows(int Ncols, int Kd, int family) {
  if (Kd % 64 != 0) return 0;
  // B loads address one expert's matrix with 32-bit byte offsets
  if ((size_t)Ncols * Kd * 2 >= ((size_t)1 << 32)) return 0;
  const bool f256 = Ncols % 256 == 0, f128 = Ncols % 128 == 0;
  switch (family) {
    case MXM_TILE_256x128:
      return f128 ? 256 : 0;
    case MXM_TILE_128x128:
      return f128 ? 128 : 0;
    case MXM_TILE_256x256:
      return f256 ? 256 : 0;
    default:  // auto: 256 x 256 where it tiles, else 128 x 128
      return f256 ? 256 : f128 ? 128 : 0;
  }
}

// Family chosen for these dimensions (auto resolved).
static int resolve_family(const GemmArgs& a) {
  if (a.family != MXM_TILE_AUTO) return a.family;
  return a.Ncols % 256 == 0 ? MXM_TILE_256x256 : MXM_TILE_128x128;
}

void mxm_launch_gemm_mfma(const GemmArgs& args, hipStream_t s) {
  if (args.max_mtiles <= 0) return;
  GemmArgs a = args;
  a.a_off32 = !a.no_off32 && (size_t)a.rows_total * a.Kd * 2 < ((size_t)1 << 32);
  switch (resolve_family(a)) {
    case MXM_TILE_256x128:
      launch_family<256, 128, 2, 2, 2, 3, 32>(a, s);
      break;
    case MXM_TILE_128x128:
      launch_family<128, 128, 2, 2, 2, 2, 64>(a, s);
      break;
    default:
      launch_family<256, 256, 2, 4, 2, 2, 64>(a, s);
      break;
  }
}
