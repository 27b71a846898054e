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
// Four waves form a 2x2 grid of 64x64 wave tiles; each wave issues 2x2
// 32x32x16 MFMAs per 16-wide k step.  The GLU weight rows are interleaved in
// groups of 32 (gate cols f..f+31, then up cols f..f+31), so a wave's two
// column MFMA tiles hold gate and up for the same 32 hidden units and the
// activation is applied straight from the accumulators.
//
// Ragged experts: blockIdx.y walks the concatenated row tiles of all experts
// (prefix `mstart`, written on device by the scan kernel); tiles past the
// end exit at once.
#include "mxm_kernels.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64, NT = 256;
constexpr int CH_PER_ROW = BK / 8;               // 16-byte chunks per tile row
constexpr int A_CHUNKS = BM * CH_PER_ROW;        // 1024
constexpr int B_CHUNKS = BN * CH_PER_ROW;        // 1024
constexpr int BUF_CHUNKS = A_CHUNKS + B_CHUNKS;  // 32 KB per buffer
constexpr int LOADS_A = A_CHUNKS / NT;           // 4
constexpr int LOADS_B = B_CHUNKS / NT;           // 4

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

__device__ __forceinline__ int swz(int row, int kc) { return row * CH_PER_ROW + (kc ^ (row & 7)); }

template <int MODE>
__global__ __launch_bounds__(NT, 2) void gemm_mfma_kernel(GemmArgs a) {
  __shared__ uint4 lds[2][BUF_CHUNKS];

  const int mtile = blockIdx.y;
  if (mtile >= a.mstart[a.E]) return;
  const int e = find_expert(a.mstart, a.E, mtile);
  const int row0 = a.offsets[e] + (mtile - a.mstart[e]) * BM;
  const int rows = min(BM, a.offsets[e + 1] - row0);
  const int n0 = blockIdx.x * BN;
  const int Kd = a.Kd;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint16_t* A = static_cast<const uint16_t*>(a.a);
  const uint16_t* B = static_cast<const uint16_t*>(a.b0) + (size_t)e * a.Ncols * Kd;

  // Global->LDS assignment: chunk c = tid + NT*i -> row c/8, k-chunk c%8.
  const int kc_ld = tid & (CH_PER_ROW - 1);
  const uint16_t* asrc[LOADS_A];
  const uint16_t* bsrc[LOADS_B];
  int adst[LOADS_A], bdst[LOADS_B];
#pragma unroll
  for (int i = 0; i < LOADS_A; ++i) {
    const int r = (tid + NT * i) / CH_PER_ROW;
    const int rr = min(r, rows - 1);  // rows past the segment reload a valid row; never stored
    const int p = row0 + rr;
    const int src = (MODE == MXM_GEMM_DOWN) ? p : a.perm[p];
    asrc[i] = A + (size_t)src * Kd + kc_ld * 8;
    adst[i] = swz(r, kc_ld);
  }
#pragma unroll
  for (int i = 0; i < LOADS_B; ++i) {
    const int r = (tid + NT * i) / CH_PER_ROW;
    bsrc[i] = B + (size_t)(n0 + r) * Kd + kc_ld * 8;
    bdst[i] = A_CHUNKS + swz(r, kc_ld);
  }

  uint4 ra[LOADS_A], rb[LOADS_B];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) ra[i] = *reinterpret_cast<const uint4*>(asrc[i] + k0);
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) rb[i] = *reinterpret_cast<const uint4*>(bsrc[i] + k0);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) lds[buf][adst[i]] = ra[i];
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) lds[buf][bdst[i]] = rb[i];
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = Kd / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      bf16x8_t af[2], bfm[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = __builtin_bit_cast(bf16x8_t, lds[cur][swz(r, kc)]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = wn * 64 + j * 32 + (lane & 31);
        bfm[j] = __builtin_bit_cast(bf16x8_t, lds[cur][A_CHUNKS + swz(r, kc)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfm[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  32x32 accumulator layout: register r of lane l holds
  // C[(r/4)*8 + (l/32)*4 + r%4][l%32].
  uint16_t* out = static_cast<uint16_t*>(a.out);
  const int col = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= rows) continue;
      if (MODE == MXM_GEMM_GLU) {
        const int F = a.Ncols / 2;
        const int f = (n0 / 64 + wn) * 32 + col;
        const float g = mxm_rbf(acc[i][0][r]);
        const float u = mxm_rbf(acc[i][1][r]);
        const float h = mxm_hidden<true>(a.expert_type, a.activation, a.slope, g, u);
        out[(size_t)(row0 + row) * F + f] = mxm_f2bf(h);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int c = n0 + wn * 64 + j * 32 + col;
          float v = acc[i][j][r];
          if (MODE == MXM_GEMM_MLP)
            v = mxm_hidden<true>(MXM_EXPERT_MLP, a.activation, a.slope, 0.0f, mxm_rbf(v));
          out[(size_t)(row0 + row) * a.Ncols + c] = mxm_f2bf(v);
        }
      }
    }
  }
}

}  // namespace

int mxm_mfma_bm() { return BM; }

void mxm_launch_gemm_mfma(const GemmArgs& a, hipStream_t s) {
  if (a.max_mtiles <= 0) return;
  const dim3 grid(a.Ncols / BN, a.max_mtiles);
  switch (a.mode) {
    case MXM_GEMM_GLU:
      hipLaunchKernelGGL(gemm_mfma_kernel<MXM_GEMM_GLU>, grid, dim3(NT), 0, s, a);
      break;
    case MXM_GEMM_MLP:
      hipLaunchKernelGGL(gemm_mfma_kernel<MXM_GEMM_MLP>, grid, dim3(NT), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL(gemm_mfma_kernel<MXM_GEMM_DOWN>, grid, dim3(NT), 0, s, a);
      break;
  }
}
