// Weight gradients of the grouped expert FFN on bf16 MFMA (gfx950).
//
//   Out[e][m][c] = sum_p sum_k A[k][p * aplane + m] * B[k][c]   (fp32)
//
// over expert e's rows k = offsets[e] .. offsets[e+1]-1 (the forward's
// permuted slot order) and the planes p of A (two for a hidden stored as
// bf16 hi and lo planes, else one).  This is dW1 = Xp^T dG|dU (A = the
// gathered x rows, B = the activation backward's output) and dW_down = H^T dY
// (A = the forward's hidden, B = the routed output gradient); the reduction
// runs over the expert's rows, whose count is only known on the device.
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
//
// Output tiles (e, c tile, m tile) are numbered with m fastest and dealt to
// the 8 XCDs in contiguous ranges, so tiles sharing an expert's B columns
// run on one XCD's L2.  The grid is persistent.  The epilogue writes fp32
// straight from the accumulators, optionally de-interleaving GLU columns
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

template <class TL, int BM, int BN, int WM, int WN, int BK, int NS>
__global__ __launch_bounds__(TL::NT, 1) void wgrad_kernel(WgradArgs a) {
  constexpr int NW = TL::NW, TM = TL::TM, TN = TL::TN;
  constexpr int QA = TL::QA, QB = TL::QB, LDPS = TL::LDPS;
  constexpr int RPWA = TL::RPWA, RPWB = TL::RPWB;
  constexpr int BUF = TL::BUF, A_BYTES = TL::A_BYTES;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[NS * BUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int ntm = a.M / BM, ntc = a.C / BN, per_e = ntm * ntc;
  const int T = a.E * per_e;
  const int T8 = (T + 7) / 8;
  const uint16_t* __restrict__ A = a.a;
  const uint16_t* __restrict__ B = a.b;

  // gridDim.x is a multiple of 8, so L % 8 (the XCD) is fixed per workgroup
  for (int L = blockIdx.x;; L += gridDim.x) {
    const int t = (L & 7) * T8 + (L >> 3);
    if ((L >> 3) >= T8 || t >= T) break;
    const int e = t / per_e, rem = t % per_e;
    const int ct = rem / ntm, mt = rem % ntm;
    const int m0 = mt * BM, c0 = ct * BN;
    const int row0 = a.offsets[e];
    const int cnt = a.offsets[e + 1] - row0;
    const int kpp = (cnt + BK - 1) / BK;  // stages per plane
    const int nk = kpp * a.planes;

    // this lane's slot in its wave-loads: tile row (within the load) and the
    // logical 16-byte chunk stored at its physical chunk (the swizzle is an
    // involution; it depends on row % 4, which is the same for every load of
    // the lane since NW * RPW is a multiple of 4)
    const int ra = lane / (BM / 8), rb = lane / (BN / 8);
    static_assert((NW * RPWA) % 4 == 0 && (NW * RPWB) % 4 == 0, "swizzle phase per lane");
    const int lca = (lane % (BM / 8)) ^ (((wave * RPWA + ra) & 3) << 2);
    const int lcb = (lane % (BN / 8)) ^ (((wave * RPWB + rb) & 3) << 2);

    auto dma_stage = [&](int kt) {
      unsigned char* st = lds + (kt % NS) * BUF;
      const int p = kt / kpp, kk = (kt % kpp) * BK;
#pragma unroll
      for (int q = 0; q < QA; ++q) {
        const int r = (wave + NW * q) * RPWA + ra;
        const int k = kk + r;
        const uint16_t* src = k < cnt ? A + (size_t)(row0 + k) * a.lda + p * a.aplane + m0 + lca * 8
                                      : a.zero + lca * 8;
        wg_dma16(src, st + (wave + NW * q) * 1024);
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int r = (wave + NW * q) * RPWB + rb;
        const int k = kk + r;
        const uint16_t* src =
            k < cnt ? B + (size_t)(row0 + k) * a.ldb + c0 + lcb * 8 : a.zero + lcb * 8;
        wg_dma16(src, st + A_BYTES + (wave + NW * q) * 1024);
      }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // fragment (k step ks) of a tile: the lane's 8 k are rows
    // ks*16 + 8*(lane/32) .. +7 of column base + (lane & 31); the two reads
    // take the 16-lane groups' 4 rows at a time
    const int g = lane >> 4;
    const int fr = 8 * (g >> 1);         // row offset of the lane's k half
    const int fc = 16 * (g & 1);         // column offset of the lane's 16-lane group
    auto frag = [&](const unsigned char* tile, auto W, int ks, int col) -> bf16x8_t {
      constexpr int WW = decltype(W)::value;
      const bf16x4_t lo = wg_read_tr<WW>(tile, ks * 16 + fr, col + fc, lane);
      const bf16x4_t hi = wg_read_tr<WW>(tile, ks * 16 + fr + 4, col + fc, lane);
      const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
      const u32x4_t v = {l2.x, l2.y, h2.x, h2.y};
      return __builtin_bit_cast(bf16x8_t, v);
    };

    // prologue: stages 0 .. NS-2 in flight
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < nk) dma_stage(s);
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt has landed for this thread (at most NS-2 later stages in
      // flight), and after the barrier for every wave; the stage read at
      // kt-1 is free and receives stage kt+NS-1
      const int ahead = min(NS - 2, nk - 1 - kt);
      if (NS >= 3 && ahead >= 2) wg_stage_barrier<2 * LDPS>();
      else if (ahead >= 1) wg_stage_barrier<LDPS>();
      else wg_stage_barrier<0>();
      if (kt + NS - 1 < nk) dma_stage(kt + NS - 1);
      const unsigned char* at = lds + (kt % NS) * BUF;
      const unsigned char* bt = at + A_BYTES;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_t af[TM], bfm[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfm[j] = frag(bt, std::integral_constant<int, BN>{}, ks, wn * TN * 32 + j * 32);
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = frag(at, std::integral_constant<int, BM>{}, ks, wm * TM * 32 + i * 32);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfm[j], acc[i][j], 0, 0, 0);
      }
    }
    // every wave is done reading the ring before the next tile's prologue
    wg_stage_barrier<0>();

    // register r of lane l holds Out[(r/4)*8 + (l/32)*4 + r%4][l%32] of the
    // MFMA tile; each store instruction writes 32 consecutive floats of two rows
    float* __restrict__ out = a.out + (size_t)e * a.out_estride;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = c0 + wn * TN * 32 + j * 32 + (lane & 31);
      // GLU columns: groups of 32, gate then up -> (slot, hidden unit f)
      const size_t cofs = a.glu_f > 0
                              ? (size_t)((c >> 5) & 1) * a.out_slot + (size_t)((c >> 6) * 32 + (c & 31))
                              : (size_t)c;
      const int ld = a.glu_f > 0 ? a.glu_f : a.C;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * TM * 32 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
          __builtin_nontemporal_store(acc[i][j][r], out + (size_t)m * ld + cofs);
        }
    }
  }
}

int wgrad_grid(int per_cu) {
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

template <int BM, int BN, int WM, int WN, int BK, int NS>
void launch_wgrad_t(const WgradArgs& a, hipStream_t s) {
  using TL = WTile<BM, BN, WM, WN, BK, NS>;
  constexpr int per_cu = std::max(1, 160 * 1024 / (NS * TL::BUF));
  const int T = a.E * (a.M / BM) * (a.C / BN);
  const int grid = std::min((T + 7) / 8 * 8, wgrad_grid(per_cu));
  hipLaunchKernelGGL((wgrad_kernel<TL, BM, BN, WM, WN, BK, NS>), dim3(grid), dim3(TL::NT), 0, s,
                     a);
}

}  // namespace

bool mxm_wgrad_fits(int M, int C) { return M > 0 && C > 0 && M % 128 == 0 && C % 128 == 0; }

void mxm_launch_wgrad(const WgradArgs& a, hipStream_t s) {
  if (a.E <= 0) return;
  if (a.M % 256 == 0 && a.C % 256 == 0)
    launch_wgrad_t<256, 256, 2, 4, 64, 2>(a, s);
  else
    launch_wgrad_t<128, 128, 2, 2, 64, 2>(a, s);
}
