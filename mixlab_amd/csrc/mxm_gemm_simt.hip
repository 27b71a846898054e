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
//
// The 64 x 64 tile's products run on the fp32 matrix cores (MF): each wave
// owns a 32 x 32 quarter as 2 x 2 blocks of v_mfma_f32_16x16x1_4b_f32, one
// instruction per k step and matrix.  That instruction adds one product per
// output, rounded once like fmaf, denormals kept (checked on the part
// against fmaf chains bit for bit), so each output is the same fmaf chain
// over the same k steps, zero padding included, as on the vector unit, at
// twice the non-packed fp32 rate.
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

typedef float mf_v16 __attribute__((ext_vector_type(16)));

// BM x BN tile, TM x TN outputs per thread (a 16 x 16 thread grid), k tiles
// of BK.  MF (BM = BN = 64): wave w owns rows 32 (w >> 1) .. + 31 and columns
// 32 (w & 1) .. + 31 of the tile; block b of its MFMA covers rows 16 (b >> 1)
// .. and columns 16 (b & 1) .. of that quarter, A from lanes 16 b + i (row
// i), B from lanes 16 b + j (column j); register 4 b + q of lane l holds row
// (l >> 4) * 4 + q, column l & 15 of block b.
template <typename TA, bool BF16, int MODE, int BM, int BN, int BK, bool MF = false>
__global__ __launch_bounds__(NT) void gemm_simt_kernel(GemmArgs a) {
  static_assert(!MF || (BM == 64 && BN == 64), "the matrix-core tile is 64 x 64");
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
  // MF: the wave's quarter and this lane's A row / B column in it
  mf_v16 accm[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) accm[b] = mf_v16{};
  const int wave = tid >> 6, lane = tid & 63;
  const int wr0 = 32 * (wave >> 1), wc0 = 32 * (wave & 1);
  const int arow_l = wr0 + 16 * ((lane >> 4) >> 1) + (lane & 15);
  const int bcol_l = wc0 + 16 * ((lane >> 4) & 1) + (lane & 15);

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
    if constexpr (MF) {
#pragma unroll
      for (int kk = 0; kk < BK; ++kk) {
        const float av = As[kk][arow_l];
#pragma unroll
        for (int b = 0; b < NB; ++b)
          accm[b] = __builtin_amdgcn_mfma_f32_16x16x1f32(av, Bs[b][kk][bcol_l], accm[b], 0, 0, 0);
      }
    } else {
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
            for (int j = 0; j < TN; ++j)
              acc[b][i][j] = __builtin_fmaf(ar[i], br[j], acc[b][i][j]);
        }
      }
    }
  }

  float* out = static_cast<float*>(a.out);
  // the outputs this thread holds: TM x TN of its 16 x 16 grid cell, or
  // (MF) 16 registers of the wave's quarter
  constexpr int OI = MF ? 16 : TM, OJ = MF ? 1 : TN;
#pragma unroll
  for (int i = 0; i < OI; ++i) {
    const int row = MF ? wr0 + 16 * ((i >> 2) >> 1) + (lane >> 4) * 4 + (i & 3) : ty * TM + i;
    if (row >= rows) continue;
    const size_t orow = (size_t)(row0 + row) * NC;
#pragma unroll
    for (int j = 0; j < OJ; ++j) {
      const int c = MF ? n0 + wc0 + 16 * ((i >> 2) & 1) + (lane & 15) : n0 + tx * TN + j;
      if (c >= NC) continue;
      auto A_ = [&](int b) { return MF ? accm[b][i] : acc[b][MF ? 0 : i][MF ? 0 : j]; };
      float v;
      if (MODE == MXM_GEMM_GLU) {
        float g = A_(0), u = A_(NB - 1);
        if (BF16) {
          g = mxm_rbf(g);
          u = mxm_rbf(u);
        }
        v = mxm_hidden<BF16>(a.expert_type, a.activation, a.slope, g, u);
      } else if (MODE == MXM_GEMM_MLP) {
        float u = A_(0);
        if (BF16) u = mxm_rbf(u);
        if (a.out2) static_cast<float*>(a.out2)[(size_t)(row0 + row) * a.ld2 + c] = u;
        v = mxm_hidden<BF16>(MXM_EXPERT_MLP, a.activation, a.slope, 0.0f, u);
      } else {
        v = A_(0);
        if (a.y_bf16) v = mxm_rbf(v);
      }
      if (out) out[orow + c] = v;
    }
  }
}

// k tiles of 16 for the 64 x 64 tile (each thread's 16 outputs per k step
// amortise the tile's barriers), 32 for the 32 x 32 tile (4 outputs per k
// step: half as many barrier and LDS round trips per k)
template <typename TA, bool BF16, int T, bool MF>
void launch_t(const GemmArgs& a, hipStream_t s) {
  constexpr int BK = T == 64 ? 16 : 32;
  const dim3 grid((a.Ncols + T - 1) / T, a.max_mtiles);
  switch (a.mode) {
    case MXM_GEMM_GLU:
      hipLaunchKernelGGL((gemm_simt_kernel<TA, BF16, MXM_GEMM_GLU, T, T, BK, MF>), grid, dim3(NT),
                         0, s, a);
      break;
    case MXM_GEMM_MLP:
      hipLaunchKernelGGL((gemm_simt_kernel<TA, BF16, MXM_GEMM_MLP, T, T, BK, MF>), grid, dim3(NT),
                         0, s, a);
      break;
    default:
      hipLaunchKernelGGL((gemm_simt_kernel<float, BF16, MXM_GEMM_DOWN, T, T, BK, MF>), grid,
                         dim3(NT), 0, s, a);
      break;
  }
}

template <typename TA, bool BF16>
void launch_tile(const GemmArgs& a, hipStream_t s) {
  if (a.simt_bm == 32)
    launch_t<TA, BF16, 32, false>(a, s);
  else if (a.simt_vec)
    launch_t<TA, BF16, 64, false>(a, s);
  else
    launch_t<TA, BF16, 64, true>(a, s);
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
  if (bf16)
    launch_tile<uint16_t, true>(a, s);
  else
    launch_tile<float, false>(a, s);
}
