// Weight gradients of the grouped expert FFN on bf16 MFMA (gfx950).
//
//   Out[e][m][c] = sum_p sum_k A[k][p * aplane + m] * B[k][c]   (fp32)
//
// over expert e's rows k = offsets[e] .. offsets[e+1]-1 (the forward's
// permuted slot order) and the planes p of A (two for a hidden stored as
// bf16 hi and lo planes, else one).  This is dW1 = Xp^T dG|dU (A = x, row k
// read at the token index a_rows[k] of the slot, B = the activation
// backward's output) and dW_down = Hg^T dD (A = the gated hidden gate * h,
// rows in slot order, B = the upstream gradient's bf16 row of the slot's
// token, read through b_rows); the reduction runs over the expert's rows,
// whose count is only known on the device.
//
// Both operands are k-outer: a row of A or B is one k, its columns are
// contiguous.  Tiles move global -> LDS in that natural layout with
// global_load_lds_dwordx4 (a wave-load fills 1 KB = whole tile rows; rows
// past the expert's end load from a zero row, so they add exact zeros), and
// the MFMA fragments, which hold 8 consecutive k for one m (or c), come out
// of LDS through the gfx950 transposing read ds_read_b64_tr_b16.  Its lane
// layout (checked on the device): within each group of 16 lanes, lane 4r+q
// supplies the address of 4 consecutive 16-bit elements (row r of a 4 x 16
// block, columns 4q..4q+3); lane i receives column i of the block, rows 0..3.
// Two such reads give a lane the 8 k of its 32x32x16 operand.  The 16-byte
// chunks of tile row k are XOR-swizzled by 4 * (k % 4), so the 32 lanes of a
// read phase (4 rows x 4 chunks) hit 16 distinct chunk columns = all banks.
// The fragments of the next 16-wide k step are read between the MFMAs of the
// current one, and the next stage's loads go out over the first two k steps.
//
// Schedule.  A tile's cost is its expert's row count, so under skewed routing
// a few experts' tiles dominate.  The work items are (expert, chunk, tile):
// an expert's reduction may be cut into chunks of whole 64-row stages, each
// chunk a separate item.  Every workgroup computes the same plan from the
// device-side offsets (one wave per candidate): each candidate split (none,
// or chunks of about 1, 1/2 or 1/4 of one workgroup's average share) is
// scored by the makespan of its items dealt round-robin in cost order
// (largest first, ties to the lower expert) plus the cost of reducing its
// extra chunks.  Sorted round-robin keeps every workgroup within one item of
// the average.
// Chunk 0 of an item writes the output; chunks 1.. write fp32 partial tiles
// to scratch slots, and a second kernel adds them to the output in chunk
// order, so the result does not depend on timing.  Consecutive positions of
// the sorted list go to workgroups of one XCD (32 at a time on 256 CUs), so
// the tiles of one expert and chunk share that XCD's L2.  The epilogue writes
// fp32 straight from the accumulators, optionally de-interleaving GLU columns
// (groups of 32: gate, then up) into the gate and up matrices.
#include <algorithm>

#include "mxm_kernels.h"

namespace {

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t* lds_bf16x4_p;

// global_load_lds_dwordx4: lane l's 16 bytes land at LDS `lds` + 16 l.  Inline
// asm, so the compiler's conservative tracking of LDS DMA does not drain the
// ring; the waits are explicit.  M0 holds the LDS base.
__device__ __forceinline__ void wg_dma16(const void* g, const void* lds) {
  const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(base)
               : "memory", "m0");
}

// The same load from a uniform 64-bit base in SGPRs plus the lane's 32-bit
// byte offset (the SGPR-base form: no 64-bit address arithmetic per load).
__device__ __forceinline__ void wg_dma16s(const void* base, unsigned off_bytes, const void* lds) {
  const unsigned lb = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off_bytes), "s"(base), "s"(lb)
               : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wg_stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// 4 consecutive k of column `col` of a tile stored [BK][W] (W bf16 per row,
// chunks swizzled by 4 * (row % 4)), for the lane's position in the
// transposing read; `row` is a multiple of 4.
template <int W>
__device__ __forceinline__ bf16x4_t wg_read_tr(const unsigned char* tile, int row, int col,
                                               int lane) {
  const int li = lane & 15;
  const int r = row + (li >> 2);
  const int c = col + 4 * (li & 3);
  const int pc = (c >> 3) ^ ((r & 3) << 2);
  const unsigned char* p = tile + r * (W * 2) + pc * 16 + (c & 7) * 2;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_p)(p));
}

template <int BM, int BN, int WM, int WN, int BK, int NS>
struct WTile {
  static constexpr int NW = WM * WN;
  static constexpr int NT = 64 * NW;
  static constexpr int TM = BM / WM / 32;
  static constexpr int TN = BN / WN / 32;
  static constexpr int A_BYTES = BK * BM * 2;
  static constexpr int BUF = A_BYTES + BK * BN * 2;  // bytes per stage
  static constexpr int RPWA = 64 / (BM / 8);         // tile rows per wave-load
  static constexpr int RPWB = 64 / (BN / 8);
  static constexpr int QA = BK / RPWA / NW;          // wave-loads per wave per stage
  static constexpr int QB = BK / RPWB / NW;
  static constexpr int LDPS = QA + QB;
  static_assert(QA * RPWA * NW == BK && QB * RPWB * NW == BK, "whole wave-loads");
  static_assert(BM / 8 <= 64 && BN / 8 <= 64 && 64 % (BM / 8) == 0, "row of at most 1 KB");
  static_assert(BM % 32 == 0 && BN % 32 == 0 && BK % 16 == 0, "MFMA tiles");
  static_assert((NS - 1) * LDPS <= 63, "vmcnt counts");
};

constexpr int WG_BK = 64;       // rows of the reduction per stage
constexpr int WG_OV = 8;        // per-item cost beyond its stages (prologue, epilogue), in stages
// The reduction kernel's cost per scratch slot (a partial tile read) and per
// reduced output tile (read and written once more), in stage times of one
// workgroup (one tile transfer at about 5.7 TB/s over the whole GPU, measured,
// against one stage's MFMA work on one CU, times 256 CUs).  A split must
// also beat the best smaller split by 10 % (the partial stores and the
// shorter items cost more than the per-item overhead above models).
constexpr int WG_PEN = 7;
constexpr int WG_CAPMIN = 16;   // no chunk shorter than 16 stages (1024 rows)
constexpr int WG_SLOTS_PER_WG = 2;  // scratch slots per workgroup of the grid
constexpr int WG_HDR_BYTES = 4096;  // plan header at the head of the scratch

constexpr int WG_NC = 4;  // candidate splits: none, chunks of about avg, avg/2, avg/4 stages

// The schedule, built identically by every workgroup (LDS).  Candidate c is
// evaluated by wave c alone; the kernel then follows the best one.
struct WgPlan {
  int cost[MXM_MAX_EXPERTS];             // stages of expert e's whole reduction (all planes)
  int nch[WG_NC][MXM_MAX_EXPERTS];       // chunks of expert e
  int order[WG_NC][MXM_MAX_EXPERTS];     // experts by chunk cost descending, ties to the lower e
                                         // (e | chunk cost << 8, the cost saturating)
  int ipre[WG_NC][MXM_MAX_EXPERTS + 1];  // first list position of sorted group r
  int slot0[MXM_MAX_EXPERTS];            // scratch slot of expert e's chunk 1, tile 0 (best plan)
  long long score[WG_NC];                // estimated cost; < 0: needs too many slots
};

// LDS written by lanes of this wave is read by other lanes of it afterwards.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ long long wave_sum_ll(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ long long wave_max_ll(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (long long)__shfl_xor(v, o));
  return v;
}

// Exclusive prefix over the lanes of a wave.
__device__ __forceinline__ int wave_excl_scan(int v, int lane) {
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x - v;
}

__device__ __forceinline__ int chunk_cost(int cost, int n) { return (cost + n - 1) / n; }

// List position of workgroup w in round r (r * G .. r * G + G - 1): the
// round's R positions are dealt to the 8 XCDs in runs of ceil(R / 8), so
// consecutive positions share an XCD (workgroup w runs on XCD w % 8; G is a
// multiple of 8) and a partial last round still spreads over every XCD.
// Returns -1 if the workgroup has no position in that round.
__device__ __forceinline__ int plan_position(int w, int r, int G, int items) {
  const int R = min(G, items - r * G);
  const int per = (R + 7) / 8;
  const int q = (w % 8) * per + w / 8;
  return (w / 8 < per && q < R) ? r * G + q : -1;
}

// The lowest-scoring feasible candidate, a larger split taken only when it
// scores 10 % below the best smaller one; no split is always feasible.
__device__ __forceinline__ int plan_best(const WgPlan& P) {
  int best = 0;
#pragma unroll
  for (int c = 1; c < WG_NC; ++c)
    if (P.score[c] >= 0 && P.score[c] * 10 < P.score[best] * 9) best = c;
  return best;
}

__device__ void build_plan(WgPlan& P, const int32_t* __restrict__ offsets, int E, int per_e,
                           int planes, int G, int slot_max) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += blockDim.x) {
    const int cnt = offsets[e + 1] - offsets[e];
    P.cost[e] = (cnt + WG_BK - 1) / WG_BK * planes;
  }
  __syncthreads();
  if (wave < WG_NC) {
    const int c = wave;
    long long tot = 0;
    for (int e = lane; e < E; e += 64) tot += (long long)P.cost[e] * per_e;
    tot = wave_sum_ll(tot);
    const long long avg = max(1LL, (tot + G - 1) / G);  // stages per workgroup
    // c = 1, 2, 3: as many chunks as make them closest to avg / 1, 2, 4
    // stages, none shorter than WG_CAPMIN
    const long long f = c == 0 ? 0 : 1LL << (c - 1);
    int* nch = P.nch[c];
    int* order = P.order[c];
    int* ipre = P.ipre[c];
    long long slots = 0, pairs = 0;
    for (int e = lane; e < E; e += 64) {
      const int co = P.cost[e];
      const long long want = (2 * co * f + avg) / (2 * avg);
      const int n = (int)max(1LL, min(want, (long long)max(1, co / WG_CAPMIN)));
      nch[e] = n;
      slots += (long long)(n - 1) * per_e;
      pairs += n > 1 ? per_e : 0;
    }
    slots = wave_sum_ll(slots);
    pairs = wave_sum_ll(pairs);
    wave_lds_sync();
    for (int e = lane; e < E; e += 64) {
      const int ic = chunk_cost(P.cost[e], nch[e]);
      int r = 0;
      for (int g = 0; g < E; ++g) {
        const int jc = chunk_cost(P.cost[g], nch[g]);
        r += (jc > ic) || (jc == ic && g < e);
      }
      order[r] = e | min(ic, 0x7fffff) << 8;  // the cost saturates for the estimate only
    }
    wave_lds_sync();
    // items per sorted group, 4 consecutive groups per lane (E <= 256)
    int loc[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * lane + k;
      loc[k] = sum;
      sum += r < E ? per_e * nch[order[r] & 0xff] : 0;
    }
    const int base = wave_excl_scan(sum, lane);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * lane + k < E) ipre[4 * lane + k] = base + loc[k];
    if (lane == 63) ipre[E] = base + sum;
    wave_lds_sync();
    // makespan of the workgroups' actual positions, in stages (4 workgroups
    // per lane at a time, so the LDS lookups of their walks overlap)
    const int items = ipre[E];
    long long mx = 0;
    for (int w0 = lane; w0 < G; w0 += 256) {
      long long load[4] = {0, 0, 0, 0};
      int g[4] = {0, 0, 0, 0};
      for (int r = 0; r * G < items; ++r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int w = w0 + 64 * k;
          const int p = w < G ? plan_position(w, r, G, items) : -1;
          if (p < 0) continue;
          while (ipre[g[k] + 1] <= p) ++g[k];
          load[k] += (order[g[k]] >> 8) + WG_OV;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) mx = max(mx, load[k]);
    }
    mx = wave_max_ll(mx);
    if (lane == 0) P.score[c] = slots <= slot_max ? mx * G + (slots + pairs) * WG_PEN : -1;
  }
  __syncthreads();
  const int best = plan_best(P);
  if (wave == 0) {
    // scratch slots of the chosen plan, by expert id
    int loc[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 4 * lane + k;
      loc[k] = sum;
      sum += e < E ? (P.nch[best][e] - 1) * per_e : 0;
    }
    const int base = wave_excl_scan(sum, lane);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * lane + k < E) P.slot0[4 * lane + k] = base + loc[k];
  }
  __syncthreads();
}


// GATHER: bit 1 = A's rows gathered through a_rows, bit 2 = B's through b_rows.
// PAD: the output is smaller than the padded operands' M x C (WgradArgs::
// m_store): stores are masked (a variant of its own: the masks' registers
// would otherwise spill in every launch).
template <class TL, int BM, int BN, int WM, int WN, int BK, int NS, int GATHER, bool PAD>
__global__ __launch_bounds__(TL::NT, 1) void wgrad_kernel(WgradArgs a) {
  constexpr int NW = TL::NW, TM = TL::TM, TN = TL::TN;
  constexpr int QA = TL::QA, LDPS = TL::LDPS, QB = LDPS - QA;
  constexpr bool GA = (GATHER & 1) != 0, GB = (GATHER & 2) != 0;
  static_assert(!(GA && GB), "one gathered operand");
  constexpr int RPWA = TL::RPWA, RPWB = TL::RPWB;
  constexpr int BUF = TL::BUF, A_BYTES = TL::A_BYTES;
  static_assert(BK == WG_BK, "the plan counts 64-row stages");
  // the stage barrier waits for every load (vmcnt 0), the gathered row
  // indices included; a deeper ring would have to count them
  static_assert(NS == 2 || !GATHER, "gathered rows with a two-stage ring only");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[NS * BUF];
  __shared__ WgPlan P;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int ntm = a.M / BM, ntc = a.C / BN, per_e = ntm * ntc;
  const int G = gridDim.x;
  const int slot_max = G * WG_SLOTS_PER_WG;
  const uint16_t* __restrict__ A = a.a;
  const uint16_t* __restrict__ B = a.b;

  build_plan(P, a.offsets, a.E, per_e, a.planes, G, slot_max);
  // values read from the LDS plan are uniform: readfirstlane keeps them (and
  // what is derived from them) in scalar registers
  const int best = __builtin_amdgcn_readfirstlane(plan_best(P));
  const int* __restrict__ nch = P.nch[best];
  const int* __restrict__ order = P.order[best];
  const int* __restrict__ ipre = P.ipre[best];
  const int items = __builtin_amdgcn_readfirstlane(ipre[a.E]);
  if (blockIdx.x == 0) {
    // the plan for the reduction kernel (read after this kernel ends)
    int* hdr = reinterpret_cast<int*>(a.scratch);
    for (int e = tid; e < a.E; e += TL::NT) {
      hdr[e] = nch[e];
      hdr[MXM_MAX_EXPERTS + e] = P.slot0[e];
    }
  }
  float* __restrict__ slots =
      reinterpret_cast<float*>(reinterpret_cast<char*>(a.scratch) + WG_HDR_BYTES);

  int g = 0;  // sorted group of the current position (positions only grow)
  for (int r = 0; r * G < items; ++r) {
    const int pos = plan_position(blockIdx.x, r, G, items);
    if (pos < 0) continue;
    while (__builtin_amdgcn_readfirstlane(ipre[g + 1]) <= pos) ++g;
    const int e = __builtin_amdgcn_readfirstlane(order[g]) & 0xff;
    const int u = pos - __builtin_amdgcn_readfirstlane(ipre[g]);
    const int j = u / per_e, tile = u % per_e;
    const int ct = tile / ntm, mt = tile % ntm;
    const int m0 = mt * BM, c0 = ct * BN;
    const int row0 = a.offsets[e];
    const int cnt = a.offsets[e + 1] - row0;
    const int kpp = (cnt + BK - 1) / BK;  // stages per plane
    const int n = __builtin_amdgcn_readfirstlane(nch[e]);
    const int cost = __builtin_amdgcn_readfirstlane(P.cost[e]);
    const int s_lo = (int)((long long)j * cost / n);
    const int nk = (int)((long long)(j + 1) * cost / n) - s_lo;

    // this lane's slot in its wave-loads: tile row (within the load) and the
    // logical 16-byte chunk stored at its physical chunk (the swizzle is an
    // involution; it depends on row % 4, which is the same for every load of
    // the lane since NW * RPW is a multiple of 4)
    const int ra = lane / (BM / 8), rb = lane / (BN / 8);
    static_assert((NW * RPWA) % 4 == 0 && (NW * RPWB) % 4 == 0, "swizzle phase per lane");
    const int lca = (lane % (BM / 8)) ^ (((wave * RPWA + ra) & 3) << 2);
    const int lcb = (lane % (BN / 8)) ^ (((wave * RPWB + rb) & 3) << 2);

    // The item's stages are loaded in order; (dp, dkk) is the plane and the
    // first reduction row (within the expert) of the next stage to load,
    // advanced one stage at a time (no division in the loop).
    int dp = s_lo / kpp, dkk = (s_lo % kpp) * BK;
    const int kend = kpp * BK;
    auto next_stage = [&]() {
      dkk += BK;
      if (dkk >= kend) {
        dkk = 0;
        ++dp;
      }
    };
    // element offsets of this lane's loads within a whole stage, fixed for
    // the item: the stage adds a uniform base (rows row0 + dkk, plane dp)
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    int a_lane[QA], b_lane[LDPS - QA];
#pragma unroll
    for (int q = 0; q < QA; ++q) a_lane[q] = ((wv + NW * q) * RPWA + ra) * a.lda + m0 + lca * 8;
#pragma unroll
    for (int q = 0; q < LDPS - QA; ++q)
      b_lane[q] = ((wv + NW * q) * RPWB + rb) * a.ldb + c0 + lcb * 8;
    // a gathered operand below 4 GiB: the lane's column part in bytes and the
    // row pitch in bytes (rows are added per stage from the scalar row indices)
    const unsigned a_colb = 2u * (unsigned)(m0 + lca * 8);
    const unsigned a_pitch = 2u * (unsigned)a.lda;
    const unsigned b_colb = 2u * (unsigned)(c0 + lcb * 8);
    const unsigned b_pitch = 2u * (unsigned)a.ldb;
    const bool g32 = (GA && a.a_rows32) || (GB && a.b_rows32);

    // Gathered rows: A's (B's) row for reduction row j is a_rows[j] (b_rows[j])
    // -- the token of a slot, so x (or a per-token gradient) is read in place
    // instead of a gathered copy.  The rows of the stage to be loaded next
    // are fetched once the current stage's loads are out, as scalar loads
    // (the wave's rows per wave-load are uniform; the lane picks its own at
    // the DMA), so that waiting for them waits on lgkmcnt and never on the
    // direct-to-LDS loads in flight.  Rows past the expert's end read its
    // last index and are not used.
    using crow_t = const __attribute__((address_space(4))) int32_t;
    crow_t* __restrict__ arows = (crow_t*)a.a_rows;
    crow_t* __restrict__ brows = (crow_t*)a.b_rows;
    int srow[QA][RPWA], srowb[QB][RPWB];
    auto load_arows = [&](int kt) {  // rows of the next stage to load (dkk)
      if (kt >= nk) return;
      if constexpr (GA) {
#pragma unroll
        for (int q = 0; q < QA; ++q)
#pragma unroll
          for (int i = 0; i < RPWA; ++i)
            srow[q][i] = arows[row0 + min(dkk + (wv + NW * q) * RPWA + i, cnt - 1)];
      }
      if constexpr (GB) {
#pragma unroll
        for (int q = 0; q < QB; ++q)
#pragma unroll
          for (int i = 0; i < RPWB; ++i)
            srowb[q][i] = brows[row0 + min(dkk + (wv + NW * q) * RPWB + i, cnt - 1)];
      }
    };
    // the lane's own row among a wave-load's gathered rows
    auto pick = [](const int* rowsq, int rl, auto rpw) {
      int r = rowsq[0];
#pragma unroll
      for (int i = 1; i < decltype(rpw)::value; ++i)
        if (rl == i) r = rowsq[i];
      return r;
    };
    auto pick_off = [](const int* rowsq, int rl, auto rpw, unsigned pitch, unsigned colb) {
      unsigned off = (unsigned)rowsq[0] * pitch + colb;
#pragma unroll
      for (int i = 1; i < decltype(rpw)::value; ++i) {
        const unsigned oi = (unsigned)rowsq[i] * pitch + colb;
        if (rl == i) off = oi;
      }
      return off;
    };
    const std::integral_constant<int, RPWA> rpwa;
    const std::integral_constant<int, RPWB> rpwb;
    // direct-to-LDS loads q0 .. q1-1 (q < QA: A rows, else B rows) of the
    // next stage to load, into ring slot kt % NS
    auto dma_part = [&](int kt, int l0, int l1) {
      unsigned char* st = lds + (kt % NS) * BUF;
      const int p = dp, kk = dkk;
      if (kk + BK <= cnt) {
        // a whole stage of rows
        const uint16_t* as = A + (size_t)(row0 + kk) * a.lda + (size_t)p * a.aplane;
        const uint16_t* bs = B + (size_t)(row0 + kk) * a.ldb + (size_t)p * a.bplane;
        auto whole = [&](auto off32) {
#pragma unroll
          for (int q = 0; q < LDPS; ++q) {
            if (q < l0 || q >= l1) continue;
            if (q < QA) {
              // gathered rows: each candidate row's byte offset (scalar) plus
              // the lane's column, the lane taking its own row's
              if constexpr (GA && decltype(off32)::value) {
                wg_dma16s(A + (size_t)p * a.aplane, pick_off(srow[q], ra, rpwa, a_pitch, a_colb),
                          st + (wv + NW * q) * 1024);
              } else if constexpr (GA) {
                wg_dma16(A + (size_t)pick(srow[q], ra, rpwa) * a.lda + (size_t)p * a.aplane + m0 +
                             lca * 8,
                         st + (wv + NW * q) * 1024);
              } else {
                wg_dma16s(as, 2u * (unsigned)a_lane[q], st + (wv + NW * q) * 1024);
              }
            } else {
              const int qb = q - QA;
              if constexpr (GB && decltype(off32)::value) {
                wg_dma16s(B + (size_t)p * a.bplane, pick_off(srowb[qb], rb, rpwb, b_pitch, b_colb),
                          st + A_BYTES + (wv + NW * qb) * 1024);
              } else if constexpr (GB) {
                wg_dma16(B + (size_t)pick(srowb[qb], rb, rpwb) * a.ldb + (size_t)p * a.bplane + c0 +
                             lcb * 8,
                         st + A_BYTES + (wv + NW * qb) * 1024);
              } else {
                wg_dma16s(bs, 2u * (unsigned)b_lane[qb], st + A_BYTES + (wv + NW * qb) * 1024);
              }
            }
          }
        };
        if (g32) whole(std::true_type{});
        else whole(std::false_type{});
      } else {
        // the expert's last, partial stage: rows past its end load the zero row
#pragma unroll
        for (int q = 0; q < LDPS; ++q) {
          if (q < l0 || q >= l1) continue;
          if (q < QA) {
            const int k = kk + (wv + NW * q) * RPWA + ra;
            int arw = row0 + k;
            if constexpr (GA) arw = pick(srow[q], ra, rpwa);
            const uint16_t* src = k < cnt ? A + (size_t)arw * a.lda + (size_t)p * a.aplane + m0 + lca * 8
                                          : a.zero + lca * 8;
            wg_dma16(src, st + (wv + NW * q) * 1024);
          } else {
            const int qb = q - QA;
            const int k = kk + (wv + NW * qb) * RPWB + rb;
            int brw = row0 + k;
            if constexpr (GB) brw = pick(srowb[qb], rb, rpwb);
            const uint16_t* src = k < cnt ? B + (size_t)brw * a.ldb + (size_t)p * a.bplane + c0 +
                                                lcb * 8
                                          : a.zero + lcb * 8;
            wg_dma16(src, st + A_BYTES + (wv + NW * qb) * 1024);
          }
        }
      }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.0f;

    // fragment (k step ks) of a tile: the lane's 8 k are rows
    // ks*16 + 8*(lane/32) .. +7 of column base + (lane & 31); the two reads
    // take the 16-lane groups' 4 rows at a time
    const int lg = lane >> 4;
    const int fr = 8 * (lg >> 1);         // row offset of the lane's k half
    const int fc = 16 * (lg & 1);         // column offset of the lane's 16-lane group
    auto frag = [&](const unsigned char* t, auto W, int ks, int col) -> bf16x8_t {
      constexpr int WW = decltype(W)::value;
      const bf16x4_t lo = wg_read_tr<WW>(t, ks * 16 + fr, col + fc, lane);
      const bf16x4_t hi = wg_read_tr<WW>(t, ks * 16 + fr + 4, col + fc, lane);
      const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
      const u32x4_t v = {l2.x, l2.y, h2.x, h2.y};
      return __builtin_bit_cast(bf16x8_t, v);
    };

    // prologue: stages 0 .. NS-2 in flight
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
      load_arows(s);
      if (s < nk) dma_part(s, 0, LDPS);
      next_stage();
    }
    load_arows(NS - 1);
    constexpr int KS = BK / 16;
    constexpr int DSTEPS = KS >= 2 ? 2 : 1;  // k steps the next stage's loads are spread over
    bf16x8_t af[2][TM], bfm[2][TN];
    auto frags = [&](const unsigned char* at, const unsigned char* bt, int set, int ks) {
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
        bfm[set][jj] = frag(bt, std::integral_constant<int, BN>{}, ks, wn * TN * 32 + jj * 32);
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[set][i] = frag(at, std::integral_constant<int, BM>{}, ks, wm * TM * 32 + i * 32);
    };
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt has landed for this thread (at most NS-2 later stages in
      // flight), and after the barrier for every wave; the stage read at
      // kt-1 is free and receives stage kt+NS-1
      const int ahead = min(NS - 2, nk - 1 - kt);
      // the row indices' scalar loads are retired here (lgkmcnt(0), vmcnt and
      // expcnt left open), where the compiler sees it: with none outstanding,
      // its waits for the fragment reads below need not count to zero
      if constexpr (GATHER) __builtin_amdgcn_s_waitcnt(0xC07F);
      if (NS >= 3 && ahead >= 2) wg_stage_barrier<2 * LDPS>();
      else if (ahead >= 1) wg_stage_barrier<LDPS>();
      else wg_stage_barrier<0>();
      const bool more = kt + NS - 1 < nk;
      const unsigned char* at = lds + (kt % NS) * BUF;
      const unsigned char* bt = at + A_BYTES;
      // the fragments of k step ks+1 are read between the MFMAs of step ks
      frags(at, bt, 0, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) frags(at, bt, (ks + 1) & 1, ks + 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < TN; ++jj)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfm[ks & 1][jj],
                                                                 acc[i][jj], 0, 0, 0);
        if (ks + 1 < KS) {
          if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x100, 2 * (TM + TN), 0);
#pragma unroll
          for (int q = 0; q < TM * TN; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            const int nr = (2 * (TM + TN) * (q + 1)) / (TM * TN) - (2 * (TM + TN) * q) / (TM * TN);
            if (nr == 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            else if (nr == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            else if (nr == 3) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
            else if (nr >= 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
          }
        }
        if (more && ks < DSTEPS) {
          dma_part(kt + NS - 1, ks * LDPS / DSTEPS, (ks + 1) * LDPS / DSTEPS);
          if (ks == DSTEPS - 1) {  // all of stage kt+NS-1 is out
            next_stage();
            load_arows(kt + NS);
          }
        }
      }
    }
    // every wave is done reading the ring before the next item's prologue
    wg_stage_barrier<0>();

    // register r of lane l holds Out[(r/4)*8 + (l/32)*4 + r%4][l%32] of the
    // MFMA tile; each store instruction writes 32 consecutive floats of two
    // rows.  Chunk 0 stores into the output (GLU columns, groups of 32 gate
    // then up, de-interleaved into the gate and up matrices), chunks 1.. a
    // BM x BN fp32 row-major partial into their scratch slot.
    float* __restrict__ base;
    int ldr;
    // with padded operands, only the tiles that reach past the output's shape
    // take the masked stores (a uniform branch)
    bool whole = true;
    if constexpr (PAD) {
      const int cend = a.glu_f > 0 ? ((c0 + BN - 1) >> 6) * 32 + 32 : c0 + BN;
      const int cst = a.glu_f > 0 ? a.glu_f : a.c_store > 0 ? a.c_store : a.C;
      whole = j > 0 || ((a.m_store <= 0 || m0 + BM <= a.m_store) && cend <= cst);
    }
    if (!PAD || whole) {
      if (j == 0) {
        ldr = a.glu_f > 0 ? a.glu_f : (PAD && a.c_store > 0) ? a.c_store : a.C;
        base = a.out + (size_t)e * a.out_estride + (size_t)m0 * ldr;
      } else {
        const int slot = __builtin_amdgcn_readfirstlane(P.slot0[e]) + (j - 1) * per_e + tile;
        base = slots + (size_t)slot * (BM * BN);
        ldr = BN;
      }
#pragma unroll
      for (int jj = 0; jj < TN; ++jj) {
        const int cl = wn * TN * 32 + jj * 32 + (lane & 31);
        const int c = c0 + cl;
        const size_t cofs =
            j > 0 ? (size_t)cl
                  : a.glu_f > 0 ? (size_t)((c >> 5) & 1) * a.out_slot + (size_t)((c >> 6) * 32 + (c & 31))
                                : (size_t)c;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = wm * TM * 32 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            __builtin_nontemporal_store(acc[i][jj][r], base + (size_t)m * ldr + cofs);
          }
      }
    } else {
      // the stored region only (partials in scratch are whole tiles)
      int mlim = BM, cvalid = 1 << 30;
      if (j == 0) {
        ldr = a.glu_f > 0 ? a.glu_f : a.c_store > 0 ? a.c_store : a.C;
        base = a.out + (size_t)e * a.out_estride + (size_t)m0 * ldr;
        if (a.m_store > 0) mlim = min(BM, a.m_store - m0);
        cvalid = ldr;
      } else {
        const int slot = __builtin_amdgcn_readfirstlane(P.slot0[e]) + (j - 1) * per_e + tile;
        base = slots + (size_t)slot * (BM * BN);
        ldr = BN;
      }
#pragma unroll
      for (int jj = 0; jj < TN; ++jj) {
        const int cl = wn * TN * 32 + jj * 32 + (lane & 31);
        const int c = c0 + cl;
        // output column (GLU: the hidden unit) this lane stores
        const int cu = j > 0 ? 0 : a.glu_f > 0 ? (c >> 6) * 32 + (c & 31) : c;
        const size_t cofs =
            j > 0 ? (size_t)cl
                  : a.glu_f > 0 ? (size_t)((c >> 5) & 1) * a.out_slot + (size_t)cu : (size_t)c;
        const bool cok = cu < cvalid;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = wm * TM * 32 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (cok && m < mlim)
              __builtin_nontemporal_store(acc[i][jj][r], base + (size_t)m * ldr + cofs);
          }
      }
    }
  }
}

// out tile (e, tile) += the partials of chunks 1 .. nch-1, in chunk order.
// Work units are 16-row slices of the (split expert, tile) pairs; a thread
// takes 4 float4 of a slice (4 consecutive columns stay inside one GLU group
// of 32) and keeps their loads in flight together.
// VEC: whole float4 of the output (16-byte aligned rows, nothing past the
// stored region); else element by element within the stored region.
template <int BM, int BN, bool VEC>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(WgradArgs a) {
  constexpr int SR = 16;                       // rows per unit
  constexpr int V = SR * BN / 4 / 256;         // float4 per thread per unit
  static_assert(V * 256 * 4 == SR * BN, "whole float4 per thread");
  __shared__ int nch[MXM_MAX_EXPERTS], slot0[MXM_MAX_EXPERTS], ppre[MXM_MAX_EXPERTS + 1];
  const int tid = threadIdx.x;
  const int* hdr = reinterpret_cast<const int*>(a.scratch);
  for (int e = tid; e < a.E; e += 256) {
    nch[e] = hdr[e];
    slot0[e] = hdr[MXM_MAX_EXPERTS + e];
  }
  __syncthreads();
  const int ntm = a.M / BM, per_e = ntm * (a.C / BN);
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < a.E; ++e) {
      ppre[e] = acc;
      acc += nch[e] > 1 ? per_e : 0;
    }
    ppre[a.E] = acc;
  }
  __syncthreads();
  const int units = ppre[a.E] * (BM / SR);
  const float* __restrict__ slots =
      reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.scratch) + WG_HDR_BYTES);
  const int ld = a.glu_f > 0 ? a.glu_f : a.c_store > 0 ? a.c_store : a.C;
  const int mst = a.m_store > 0 ? a.m_store : a.M;
  int e = 0;
  for (int k = blockIdx.x; k < units; k += gridDim.x) {
    const int pair = k / (BM / SR), r0 = (k % (BM / SR)) * SR;
    while (ppre[e + 1] <= pair) ++e;
    const int tile = pair - ppre[e];
    const int m0 = (tile % ntm) * BM, c0 = (tile / ntm) * BN;
    float* __restrict__ out = a.out + (size_t)e * a.out_estride;
    if constexpr (!VEC) {
      // element by element: the four columns of a float4 of the partial, each
      // stored only inside the output's shape
      for (int q = 0; q < V; ++q) {
        const int i = tid + 256 * q;
        const int m = r0 + i / (BN / 4), cb = c0 + (i % (BN / 4)) * 4;
        if (m0 + m >= mst) continue;
        for (int t = 0; t < 4; ++t) {
          const int c = cb + t;
          const int cu = a.glu_f > 0 ? (c >> 6) * 32 + (c & 31) : c;
          if (cu >= ld) continue;
          const size_t cofs = a.glu_f > 0 ? (size_t)((c >> 5) & 1) * a.out_slot + (size_t)cu
                                          : (size_t)c;
          float* po = out + (size_t)(m0 + m) * ld + cofs;
          float v = *po;
          for (int jc = 1; jc < nch[e]; ++jc)
            v = v + slots[(size_t)(slot0[e] + (jc - 1) * per_e + tile) * (BM * BN) +
                          (size_t)r0 * BN + 4 * i + t];
          *po = v;
        }
      }
      continue;
    }
    float4* o[V];
    float4 v[V];
#pragma unroll
    for (int q = 0; q < V; ++q) {
      const int i = tid + 256 * q;
      const int m = r0 + i / (BN / 4), c = c0 + (i % (BN / 4)) * 4;
      const size_t cofs = a.glu_f > 0
                              ? (size_t)((c >> 5) & 1) * a.out_slot + (size_t)((c >> 6) * 32 + (c & 31))
                              : (size_t)c;
      o[q] = reinterpret_cast<float4*>(out + (size_t)(m0 + m) * ld + cofs);
      v[q] = *o[q];
    }
    const int n = nch[e];
    for (int jc = 1; jc < n; ++jc) {
      const float* sl = slots + (size_t)(slot0[e] + (jc - 1) * per_e + tile) * (BM * BN) +
                        (size_t)r0 * BN;
      float4 p[V];
#pragma unroll
      for (int q = 0; q < V; ++q) p[q] = *reinterpret_cast<const float4*>(sl + 4 * (tid + 256 * q));
#pragma unroll
      for (int q = 0; q < V; ++q) {
        v[q].x = v[q].x + p[q].x;
        v[q].y = v[q].y + p[q].y;
        v[q].z = v[q].z + p[q].z;
        v[q].w = v[q].w + p[q].w;
      }
    }
#pragma unroll
    for (int q = 0; q < V; ++q) *o[q] = v[q];
  }
}

int n_cus() {
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
  return ncu[dev];
}

template <int BM, int BN, int WM, int WN, int BK, int NS>
struct WFamily {
  using TL = WTile<BM, BN, WM, WN, BK, NS>;
  static constexpr int LDS_BYTES = NS * TL::BUF + (int)sizeof(WgPlan);
  static constexpr int PER_CU = std::max(1, 160 * 1024 / LDS_BYTES);
  static int grid() { return std::max(8, n_cus() * PER_CU / 8 * 8); }
  static size_t scratch_bytes() {
    return WG_HDR_BYTES + (size_t)grid() * WG_SLOTS_PER_WG * BM * BN * sizeof(float);
  }
  template <bool PAD>
  static void launch_main(const WgradArgs& a, hipStream_t s) {
    if (a.a_rows)
      hipLaunchKernelGGL((wgrad_kernel<TL, BM, BN, WM, WN, BK, NS, 1, PAD>), dim3(grid()),
                         dim3(TL::NT), 0, s, a);
    else if (a.b_rows)
      hipLaunchKernelGGL((wgrad_kernel<TL, BM, BN, WM, WN, BK, NS, 2, PAD>), dim3(grid()),
                         dim3(TL::NT), 0, s, a);
    else
      hipLaunchKernelGGL((wgrad_kernel<TL, BM, BN, WM, WN, BK, NS, 0, PAD>), dim3(grid()),
                         dim3(TL::NT), 0, s, a);
  }
  static void launch(const WgradArgs& a, hipStream_t s) {
    const bool pad = (a.m_store > 0 && a.m_store != a.M) ||
                     (a.glu_f > 0 ? 2 * a.glu_f != a.C : (a.c_store > 0 && a.c_store != a.C));
    if (pad)
      launch_main<true>(a, s);
    else
      launch_main<false>(a, s);
    // whole float4 when the output rows are 16-byte aligned and every column
    // of the padded operands is stored
    const int ld = a.glu_f > 0 ? a.glu_f : a.c_store > 0 ? a.c_store : a.C;
    const bool vec = ld % 4 == 0 && (a.m_store <= 0 || a.m_store == a.M) &&
                     (a.glu_f > 0 ? 2 * a.glu_f == a.C : (a.c_store <= 0 || a.c_store == a.C)) &&
                     reinterpret_cast<uintptr_t>(a.out) % 16 == 0 && a.out_estride % 4 == 0 &&
                     a.out_slot % 4 == 0;
    if (vec)
      hipLaunchKernelGGL((wgrad_reduce_kernel<BM, BN, true>), dim3(std::max(8, n_cus() * 2)),
                         dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((wgrad_reduce_kernel<BM, BN, false>), dim3(std::max(8, n_cus() * 2)),
                         dim3(256), 0, s, a);
  }
};
using WBig = WFamily<256, 256, 2, 4, 64, 2>;
using WSmall = WFamily<128, 128, 2, 2, 64, 2>;

bool wgrad_big(int M, int C) { return M % 256 == 0 && C % 256 == 0; }

}  // namespace

bool mxm_wgrad_fits(int M, int C) { return M > 0 && C > 0 && M % 128 == 0 && C % 128 == 0; }

size_t mxm_wgrad_scratch_bytes(int M, int C) {
  return wgrad_big(M, C) ? WBig::scratch_bytes() : WSmall::scratch_bytes();
}

void mxm_launch_wgrad(const WgradArgs& a, hipStream_t s) {
  if (a.E <= 0) return;
  if (wgrad_big(a.M, a.C))
    WBig::launch(a, s);
  else
    WSmall::launch(a, s);
}
