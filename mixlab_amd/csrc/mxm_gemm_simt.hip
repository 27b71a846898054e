// Grouped expert FFN, SIMT family.  Used for the fp32 flow and for bf16
// shapes the MFMA family does not tile (D or F not a multiple of 128).
//
// Each output is accumulated by fmaf over k = 0..Kd-1 in ascending order, the
// order of the CPU restatement, and the epilogue follows the dtype flow of
// gpu/ir.cpp:1126-1145 (projections rounded to bf16 in the bf16 flow, the
// hidden activation per mxm_hidden, y rounded to bf16 when the reference's
// down projection produces bf16).  H and Y are kept in fp32 storage.
//
// Row tiles are ragged per expert: blockIdx.y indexes the concatenation of
// every expert's ceil(count/BM) row tiles (prefix `mstart`), so no host sync
// is needed between dispatch and the GEMM.
//
// Two tiles, 256 threads each: 64 x 64 outputs (4 x 4 per thread), and 32 x
// 32 (2 x 2 per thread) for launches whose 64 x 64 grid would leave CUs
// idle -- four times the workgroups, each thread's chain a quarter as long
// (GemmArgs::simt_bm picks; the schedule's row tiles must match).
#include "mxm_kernels.h"

namespace {

constexpr int NT = 256;

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

template <typename TA>
__device__ __forceinline__ float lda_f32(const TA* p);
template <>
__device__ __forceinline__ float lda_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float lda_f32<uint16_t>(const uint16_t* p) { return mxm_bf2f(*p); }

// T consecutive floats of LDS (T * 4-byte aligned) as one vector read.
template <int T>
__device__ __forceinline__ void lds_vec(const float* p, float (&v)[T]) {
  static_assert(T == 2 || T == 4, "float2 or float4");
  if constexpr (T == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
    const float2 q = *reinterpret_cast<const float2*>(p);
    v[0] = q.x;
    v[1] = q.y;
  }
}

// BM x BN tile, TM x TN outputs per thread (a 16 x 16 thread grid), k tiles
// of BK.
template <typename TA, bool BF16, int MODE, int BM, int BN, int BK>
__global__ __launch_bounds__(NT) void gemm_simt_kernel(GemmArgs a) {
  constexpr int NB = (MODE == MXM_GEMM_GLU) ? 2 : 1;
  constexpr int TM = BM / 16, TN = BN / 16;
  constexpr int LA = BM * BK / NT, LB = BK * BN / NT;  // loads per thread per k tile
  constexpr int LDA = BM + 4, LDB = BN + 4;
  static_assert(LA * NT == BM * BK && LB * NT == BK * BN, "whole loads per thread");
  __shared__ float As[BK][LDA];
  __shared__ float Bs[NB][BK][LDB];

  const int mtile = blockIdx.y;
  if (mtile >= a.mstart[a.E]) return;
  const int e = find_expert(a.mstart, a.E, mtile);
  const int row0 = a.offsets[e] + (mtile - a.mstart[e]) * BM;
  const int rows = min(BM, a.offsets[e + 1] - row0);
  const int n0 = blockIdx.x * BN;
  const int Kd = a.Kd, NC = a.Ncols;
  const int tid = threadIdx.x;
  const int ty = tid >> 4, tx = tid & 15;

  const TA* A = static_cast<const TA*>(a.a);
  const float* B0 = static_cast<const float*>(a.b0) + (size_t)e * Kd * NC;
  const float* B1 = (NB == 2) ? static_cast<const float*>(a.b1) + (size_t)e * Kd * NC : nullptr;

  // A-tile rows this thread loads: idx = tid + 256*r -> row idx/BK, k idx%BK
  const TA* arow[LA];
#pragma unroll
  for (int r = 0; r < LA; ++r) {
    const int row = (tid + NT * r) / BK;
    if (row < rows) {
      const int p = row0 + row;
      const int src = (MODE == MXM_GEMM_DOWN) ? p : a.perm[p];
      arow[r] = A + (size_t)src * Kd;
    } else {
      arow[r] = nullptr;
    }
  }

  float acc[NB][TM][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[b][i][j] = 0.0f;

  // The k tile after the current one is loaded into registers while the
  // current one is summed (its loads' latency is then hidden behind 16 k
  // steps); only the time of the loads changes, not the order of the sums.
  float pa[LA], pb[NB][LB];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int r = 0; r < LA; ++r) {
      const int idx = tid + NT * r;
      const int row = idx / BK, kk = idx % BK;
      const int k = k0 + kk;
      pa[r] = (arow[r] != nullptr && k < Kd) ? lda_f32<TA>(arow[r] + k) : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float* Bm = (b == 0) ? B0 : B1;
#pragma unroll
      for (int r = 0; r < LB; ++r) {
        const int idx = tid + NT * r;
        const int kk = idx / BN, col = idx % BN;
        const int k = k0 + kk, c = n0 + col;
        pb[b][r] = (k < Kd && c < NC) ? Bm[(size_t)k * NC + c] : 0.0f;
      }
    }
  };
  fetch(0);
  for (int k0 = 0; k0 < Kd; k0 += BK) {
    __syncthreads();  // every thread has finished reading the previous tile
#pragma unroll
    for (int r = 0; r < LA; ++r) {
      const int idx = tid + NT * r;
      As[idx % BK][idx / BK] = pa[r];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < LB; ++r) {
        const int idx = tid + NT * r;
        Bs[b][idx / BN][idx % BN] = pb[b][r];
      }
    __syncthreads();
    if (k0 + BK < Kd) fetch(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float ar[TM];
      lds_vec<TM>(&As[kk][ty * TM], ar);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float br[TN];
        lds_vec<TN>(&Bs[b][kk][tx * TN], br);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[b][i][j] = __builtin_fmaf(ar[i], br[j], acc[b][i][j]);
      }
    }
  }

  float* out = static_cast<float*>(a.out);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = ty * TM + i;
    if (row >= rows) continue;
    const size_t orow = (size_t)(row0 + row) * NC;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = n0 + tx * TN + j;
      if (c >= NC) continue;
      float v;
      if (MODE == MXM_GEMM_GLU) {
        float g = acc[0][i][j], u = acc[NB - 1][i][j];
        if (BF16) {
          g = mxm_rbf(g);
          u = mxm_rbf(u);
        }
        v = mxm_hidden<BF16>(a.expert_type, a.activation, a.slope, g, u);
      } else if (MODE == MXM_GEMM_MLP) {
        float u = acc[0][i][j];
        if (BF16) u = mxm_rbf(u);
        if (a.out2) static_cast<float*>(a.out2)[(size_t)(row0 + row) * a.ld2 + c] = u;
        v = mxm_hidden<BF16>(MXM_EXPERT_MLP, a.activation, a.slope, 0.0f, u);
      } else {
        v = acc[0][i][j];
        if (a.y_bf16) v = mxm_rbf(v);
      }
      if (out) out[orow + c] = v;
    }
  }
}

// k tiles of 16 for the 64 x 64 tile (each thread's 16 outputs per k step
// amortise the tile's barriers), 32 for the 32 x 32 tile (4 outputs per k
// step: half as many barrier and LDS round trips per k)
template <typename TA, bool BF16, int T>
void launch_t(const GemmArgs& a, hipStream_t s) {
  constexpr int BK = T == 64 ? 16 : 32;
  const dim3 grid((a.Ncols + T - 1) / T, a.max_mtiles);
  switch (a.mode) {
    case MXM_GEMM_GLU:
      hipLaunchKernelGGL((gemm_simt_kernel<TA, BF16, MXM_GEMM_GLU, T, T, BK>), grid, dim3(NT), 0,
                         s, a);
      break;
    case MXM_GEMM_MLP:
      hipLaunchKernelGGL((gemm_simt_kernel<TA, BF16, MXM_GEMM_MLP, T, T, BK>), grid, dim3(NT), 0,
                         s, a);
      break;
    default:
      hipLaunchKernelGGL((gemm_simt_kernel<float, BF16, MXM_GEMM_DOWN, T, T, BK>), grid, dim3(NT),
                         0, s, a);
      break;
  }
}

}  // namespace

int mxm_simt_bm(int64_t rows, int E, int ncols, int n_cu) {
  // the 64 x 64 tile where its grid gives every CU one, else 32 x 32
  // (measured: C1's down projection, 72 tiles of 64 x 64, is faster on 32 x
  // 32; a 2048-row fp32 down projection of 320 tiles, over k = 2048, is
  // faster on 64 x 64, whose threads reuse each LDS read for 4 outputs)
  const int64_t tiles = ((rows + 63) / 64 + E) * ((ncols + 63) / 64);
  return tiles >= (int64_t)n_cu ? 64 : 32;
}

void mxm_launch_gemm_simt(const GemmArgs& a, bool bf16, hipStream_t s) {
  if (a.max_mtiles <= 0) return;
  const bool small = a.simt_bm == 32;
  if (bf16) {
    if (small)
      launch_t<uint16_t, true, 32>(a, s);
    else
      launch_t<uint16_t, true, 64>(a, s);
  } else {
    if (small)
      launch_t<float, false, 32>(a, s);
    else
      launch_t<float, false, 64>(a, s);
  }
}
