// Grouped expert FFN on bf16 MFMA (gfx950, v_mfma_f32_32x32x16_bf16).
//
// One workgroup computes a BM x BN tile of one expert's output.  A rows are
// the expert's permuted slots: for the up projections they are gathered from
// x through `perm` (each row is D contiguous bf16), for the down projection
// they are the contiguous rows of H.  B is the expert's weight stored
// transposed ([out, in], k contiguous) so both operands stream k-contiguous
// 16-byte chunks.  Tiles are staged through LDS, double-buffered with
// register prefetch, with the 16-byte chunk index XOR-swizzled by (row & 7)
// so the 8-lane phases of ds_read_b128 hit distinct banks.
//
// Two tile families share one template: 256 x 256 (8 waves as 2 x 4, each
// wave 128 x 64 = 4 x 2 MFMA tiles) where the dimensions allow, else
// 128 x 128 (4 waves as 2 x 2, each 64 x 64).  The GLU weight rows are
// interleaved in groups of 32 (gate cols f..f+31, then up cols f..f+31), so a
// wave's two column MFMA tiles hold gate and up for the same 32 hidden units
// and the activation is applied straight from the accumulators.
//
// Ragged experts: the scan kernel writes `mstart`, the prefix over experts of
// ceil(count/BM) row tiles, so tile -> (expert, rows) is resolved on device
// and tiles past the end exit at once.
//
// Tile order: the hardware hands workgroup L to XCD L % 8.  Row tiles are
// grouped GM at a time with the column tiles of a group adjacent, and group g
// is placed on XCD g % 8, so each XCD's L2 sees a GM x (N/BN) block of tiles
// sharing A rows and B columns, and the empty tail tiles are spread over all
// XCDs.  The epilogue stages each wave's bf16 tile through LDS
// (chunk-swizzled) and writes 16-byte row segments.
#include "mxm_kernels.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Native vector type for 16-byte moves (HIP's uint4 wrapper class defeats
// scalar replacement of the prefetch registers).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int BK = 64;            // k per LDS stage
constexpr int CH = BK / 8;        // 16-byte chunks per tile row
constexpr int GM = 4;             // row tiles per scheduling group

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

// 16-byte chunk kc of tile row `row`, XOR-swizzled by (row & 7).
__device__ __forceinline__ int swz(int row, int kc) { return row * CH + (kc ^ (row & 7)); }

// Tile family: BM x BN workgroup tile, WM x WN waves, each wave
// (BM/WM) x (BN/WN) = TM x TN MFMA 32x32 tiles.
template <int BM, int BN, int WM, int WN>
struct Tile {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int TM = BM / WM / 32;
  static constexpr int TN = BN / WN / 32;
  static constexpr int A_CH = BM * CH;
  static constexpr int B_CH = BN * CH;
  static constexpr int BUF = A_CH + B_CH;
  static constexpr int LA = A_CH / NT;
  static constexpr int LB = B_CH / NT;
  static_assert(TN == 2, "GLU epilogue pairs gate and up in a wave's two column tiles");
  static_assert(A_CH % NT == 0 && B_CH % NT == 0, "whole chunks per thread");
};

// Epilogue kinds: the hidden activation (expert type x activation) of the up
// projections, or the plain bf16 store of the down projection.
enum { EPI_SWIGLU, EPI_GEGLU, EPI_MLP_SILU, EPI_MLP_GELU, EPI_MLP_RELU, EPI_MLP_LEAKY, EPI_DOWN };

template <int EPI>
struct Epi {
  static constexpr int MODE = EPI <= EPI_GEGLU ? MXM_GEMM_GLU
                              : EPI == EPI_DOWN ? MXM_GEMM_DOWN
                                                : MXM_GEMM_MLP;
  static constexpr int ETYPE = EPI == EPI_SWIGLU ? MXM_EXPERT_SWIGLU
                               : EPI == EPI_GEGLU ? MXM_EXPERT_GEGLU
                                                  : MXM_EXPERT_MLP;
  static constexpr int ACT = EPI == EPI_MLP_GELU    ? MXM_ACT_GELU
                             : EPI == EPI_MLP_RELU  ? MXM_ACT_RELU
                             : EPI == EPI_MLP_LEAKY ? MXM_ACT_LEAKY_RELU_SQ
                             : EPI == EPI_GEGLU     ? MXM_ACT_GELU
                                                    : MXM_ACT_SILU;
};

template <class TL, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(TL::NT) void gemm_kernel(GemmArgs a, int ngroups) {
  constexpr int MODE = Epi<EPI>::MODE;
  constexpr int NT = TL::NT, TM = TL::TM, TN = TL::TN, LA = TL::LA, LB = TL::LB;
  constexpr int A_CH = TL::A_CH, BUF = TL::BUF;
  __shared__ u32x4_t lds[2][BUF];

  // XCD-aware grouped schedule (see the file comment).
  const int ntile_n = a.Ncols / BN;
  const int per_group = GM * ntile_n;
  const int L = blockIdx.x;
  const int local = L >> 3;
  const int g = (local / per_group) * 8 + (L & 7);
  if (g >= ngroups) return;
  const int rr = local % per_group;
  const int mtile = g * GM + rr % GM;
  const int ntile = rr / GM;
  if (mtile >= a.mstart[a.E]) return;
  const int e = find_expert(a.mstart, a.E, mtile);
  const int row0 = a.offsets[e] + (mtile - a.mstart[e]) * BM;
  const int rows = min(BM, a.offsets[e + 1] - row0);
  const int n0 = ntile * BN;
  const int Kd = a.Kd;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(a.a);
  const uint16_t* __restrict__ B =
      static_cast<const uint16_t*>(a.b0) + (size_t)e * a.Ncols * Kd;

  // Global->LDS assignment: chunk c = tid + NT*i -> tile row c/8, k-chunk c%8.
  const int kc_ld = tid & (CH - 1);
  const int r_ld = tid / CH;  // + i * NT/CH
  size_t aoff[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int r = r_ld + i * (NT / CH);
    const int p = row0 + min(r, rows - 1);  // rows past the segment reload a valid row
    const int src = (MODE == MXM_GEMM_DOWN) ? p : a.perm[p];
    aoff[i] = (size_t)src * Kd + kc_ld * 8;
  }
  const size_t boff = (size_t)(n0 + r_ld) * Kd + kc_ld * 8;
  const size_t bstep = (size_t)(NT / CH) * Kd;

  u32x4_t ra[LA], rb[LB];
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = Kd / BK;
#pragma unroll
  for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const u32x4_t*>(A + aoff[i]);
#pragma unroll
  for (int i = 0; i < LB; ++i) rb[i] = *reinterpret_cast<const u32x4_t*>(B + boff + i * bstep);
#pragma unroll
  for (int i = 0; i < LA; ++i) lds[0][swz(r_ld + i * (NT / CH), kc_ld)] = ra[i];
#pragma unroll
  for (int i = 0; i < LB; ++i) lds[0][A_CH + swz(r_ld + i * (NT / CH), kc_ld)] = rb[i];
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = (kt + 1) * BK;
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const u32x4_t*>(A + aoff[i] + k0);
#pragma unroll
      for (int i = 0; i < LB; ++i)
        rb[i] = *reinterpret_cast<const u32x4_t*>(B + boff + i * bstep + k0);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      bf16x8_t af[TM], bfm[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = __builtin_bit_cast(bf16x8_t,
                                   lds[cur][swz(wm * TM * 32 + i * 32 + (lane & 31), kc)]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfm[j] = __builtin_bit_cast(
            bf16x8_t, lds[cur][A_CH + swz(wn * TN * 32 + j * 32 + (lane & 31), kc)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfm[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < LA; ++i) lds[cur ^ 1][swz(r_ld + i * (NT / CH), kc_ld)] = ra[i];
#pragma unroll
      for (int i = 0; i < LB; ++i) lds[cur ^ 1][A_CH + swz(r_ld + i * (NT / CH), kc_ld)] = rb[i];
    }
    __syncthreads();
  }

  // ---- epilogue: activation, bf16, per-wave LDS staging, 16-byte stores ----
  // 32x32 accumulator layout: register r of lane l holds
  // C[(r/4)*8 + (l/32)*4 + r%4][l%32].
  constexpr int WROWS = TM * 32;
  constexpr int C = (MODE == MXM_GEMM_GLU) ? 32 : 64;  // output columns per wave
  constexpr int CPR = C / 8;
  static_assert(WM * WN * WROWS * 64 * 2 <= (int)sizeof(u32x4_t) * 2 * BUF, "staging fits in LDS");
  uint16_t* stage = reinterpret_cast<uint16_t*>(&lds[0][0]) + (size_t)wave * WROWS * 64;
  const int col = lane & 31;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (MODE == MXM_GEMM_GLU) {
        const float gg = mxm_rbf(acc[i][0][r]);
        const float u = mxm_rbf(acc[i][1][r]);
        const float h = mxm_hidden<true>(Epi<EPI>::ETYPE, Epi<EPI>::ACT, a.slope, gg, u);
        stage[row * C + (((col >> 3) ^ (row & (CPR - 1))) << 3) + (col & 7)] = mxm_f2bf(h);
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v = acc[i][j][r];
          if (MODE == MXM_GEMM_MLP)
            v = mxm_hidden<true>(MXM_EXPERT_MLP, Epi<EPI>::ACT, a.slope, 0.0f, mxm_rbf(v));
          const int c = j * 32 + col;
          stage[row * C + (((c >> 3) ^ (row & (CPR - 1))) << 3) + (c & 7)] = mxm_f2bf(v);
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int ldo = (MODE == MXM_GEMM_GLU) ? a.Ncols / 2 : a.Ncols;
  const int c0 = (MODE == MXM_GEMM_GLU) ? n0 / 2 + wn * 32 : n0 + wn * 64;
  uint16_t* __restrict__ out = static_cast<uint16_t*>(a.out);
#pragma unroll
  for (int it = 0; it < WROWS * CPR / 64; ++it) {
    const int q = lane + 64 * it;
    const int row = q / CPR, cc = q % CPR;
    const int grow = wm * WROWS + row;
    if (grow < rows) {
      const u32x4_t v =
          *reinterpret_cast<const u32x4_t*>(stage + row * C + ((cc ^ (row & (CPR - 1))) << 3));
      *reinterpret_cast<u32x4_t*>(out + (size_t)(row0 + grow) * ldo + c0 + cc * 8) = v;
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI>
void launch_epi(const GemmArgs& a, hipStream_t s, int blocks, int ngroups) {
  using TL = Tile<BM, BN, WM, WN>;
  hipLaunchKernelGGL((gemm_kernel<TL, BM, BN, WM, WN, EPI>), dim3(blocks), dim3(TL::NT), 0, s, a,
                     ngroups);
}

template <int BM, int BN, int WM, int WN>
void launch_family(const GemmArgs& a, hipStream_t s) {
  const int ngroups = (a.max_mtiles + GM - 1) / GM;
  const int per_group = GM * (a.Ncols / BN);
  const int blocks = ((ngroups + 7) / 8) * 8 * per_group;
  if (a.mode == MXM_GEMM_DOWN) {
    launch_epi<BM, BN, WM, WN, EPI_DOWN>(a, s, blocks, ngroups);
  } else if (a.mode == MXM_GEMM_GLU) {
    if (a.expert_type == MXM_EXPERT_GEGLU)
      launch_epi<BM, BN, WM, WN, EPI_GEGLU>(a, s, blocks, ngroups);
    else
      launch_epi<BM, BN, WM, WN, EPI_SWIGLU>(a, s, blocks, ngroups);
  } else {
    switch (a.activation) {
      case MXM_ACT_GELU:
        launch_epi<BM, BN, WM, WN, EPI_MLP_GELU>(a, s, blocks, ngroups);
        break;
      case MXM_ACT_RELU:
        launch_epi<BM, BN, WM, WN, EPI_MLP_RELU>(a, s, blocks, ngroups);
        break;
      case MXM_ACT_LEAKY_RELU_SQ:
        launch_epi<BM, BN, WM, WN, EPI_MLP_LEAKY>(a, s, blocks, ngroups);
        break;
      default:
        launch_epi<BM, BN, WM, WN, EPI_MLP_SILU>(a, s, blocks, ngroups);
        break;
    }
  }
}

}  // namespace

int mxm_mfma_bm() { return 128; }

int mxm_mfma_tile_rows(int Ncols, int Kd, bool tile128) {
  return (!tile128 && Ncols % 256 == 0 && Kd % BK == 0) ? 256 : 128;
}

void mxm_launch_gemm_mfma(const GemmArgs& a, hipStream_t s) {
  if (a.max_mtiles <= 0) return;
  if (mxm_mfma_tile_rows(a.Ncols, a.Kd, a.tile128) == 256)
    launch_family<256, 256, 2, 4>(a, s);
  else
    launch_family<128, 128, 2, 2>(a, s);
}
