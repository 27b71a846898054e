// Weight preparation, run once when weights are uploaded: dtype conversion
// to the flow's storage type and the transposed / GLU-interleaved layout of
// the MFMA family.  Source dtypes: 1 = fp32, 2 = bf16 bits, 3 = int8 (the
// integers of int8 weights, exact in bf16: |q| <= 128 needs 8 bits).
#include "mxm_kernels.h"

namespace {

__device__ __forceinline__ float src_at(const void* p, int dtype, size_t i) {
  if (dtype == 3) return (float)static_cast<const int8_t*>(p)[i];
  return dtype == 2 ? mxm_bf2f(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

__global__ void to_f32_kernel(const void* src, int dtype, float* dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = src_at(src, dtype, (size_t)i);
}

__global__ void to_bf16_kernel(const void* src, int dtype, uint16_t* dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = mxm_f2bf(src_at(src, dtype, (size_t)i));
}

// 32x32 LDS transpose: block (32, 8) covers source cols c0..c0+31 and
// k0..k0+31; the 32 destination rows of an aligned group of 32 source
// columns are consecutive in both layouts.  Destination rows are ldd
// elements apart (ldd >= Kd: a padded row's tail is not written).
__global__ void transpose_kernel(const void* src, int dtype, int Kd, int C, int slot,
                                 uint16_t* dst, int ldd) {
  __shared__ uint16_t tile[32][33];
  const int c0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
  for (int yy = threadIdx.y; yy < 32; yy += 8) {
    const int k = k0 + yy, c = c0 + threadIdx.x;
    tile[yy][threadIdx.x] = (k < Kd && c < C) ? mxm_f2bf(src_at(src, dtype, (size_t)k * C + c)) : 0;
  }
  __syncthreads();
  for (int yy = threadIdx.y; yy < 32; yy += 8) {
    const int c = c0 + yy, k = k0 + threadIdx.x;
    if (c < C && k < Kd) {
      const int q = slot < 0 ? c : (c >> 5) * 64 + slot * 32 + (c & 31);
      dst[(size_t)q * ldd + k] = tile[threadIdx.x][yy];
    }
  }
}

int grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace

void mxm_launch_to_f32(const void* src, int src_dtype, float* dst, int64_t n, hipStream_t s) {
  if (n > 0) hipLaunchKernelGGL(to_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, src_dtype, dst, n);
}

void mxm_launch_to_bf16(const void* src, int src_dtype, uint16_t* dst, int64_t n, hipStream_t s) {
  if (n > 0) hipLaunchKernelGGL(to_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, src_dtype, dst, n);
}

namespace {

__global__ void rows_to_f32_kernel(const void* src, int dtype, int64_t rows, int cols, int ld,
                                   float* dst) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols;
    const int c = (int)(i - r * cols);
    dst[i] = src_at(src, dtype, (size_t)r * ld + c);
  }
}

__global__ void pad_rows_bf16_kernel(const uint16_t* src, int64_t rows, int cols, int ldd,
                                     uint16_t* dst) {
  const int64_t n = rows * ldd;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ldd;
    const int c = (int)(i - r * ldd);
    dst[i] = c < cols ? src[(size_t)r * cols + c] : (uint16_t)0;
  }
}

}  // namespace

void mxm_launch_rows_to_f32(const void* src, int src_dtype, int64_t rows, int cols, int ld,
                            float* dst, hipStream_t s) {
  const int64_t n = rows * cols;
  if (n > 0)
    hipLaunchKernelGGL(rows_to_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, src_dtype, rows,
                       cols, ld, dst);
}

void mxm_launch_pad_rows_bf16(const uint16_t* src, int64_t rows, int cols, int ldd, uint16_t* dst,
                              hipStream_t s) {
  const int64_t n = rows * ldd;
  if (n > 0)
    hipLaunchKernelGGL(pad_rows_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, rows, cols,
                       ldd, dst);
}

namespace {

__global__ void shuffle_bf16_kernel(const void* src, int dtype, int Kd, int C, int Kdp, int Cp,
                                    uint16_t* __restrict__ dst) {
  const size_t total = (size_t)Kdp * Cp;
  const int ncb = Cp / 16;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
       o += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = o >> 10;
    const int within = (int)(o & 1023);
    // half h of the block holds value 8h + i' of every lane, lane l at 8 l
    const int h = within >> 9, l = (within >> 3) & 63, i = 8 * h + (within & 7);
    const int kb = (int)(blk / ncb), cb = (int)(blk % ncb);
    const int k = 64 * kb + 16 * (l >> 4) + i;
    const int c = 16 * cb + (l & 15);
    dst[o] = (k < Kd && c < C) ? mxm_f2bf(src_at(src, dtype, (size_t)k * C + c)) : (uint16_t)0;
  }
}

}  // namespace

void mxm_launch_shuffle_bf16(const void* src, int src_dtype, int Kd, int C, int Kdp, int Cp,
                             uint16_t* dst, hipStream_t s) {
  const size_t total = (size_t)Kdp * Cp;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 65536) blocks = 65536;
  if (blocks > 0)
    hipLaunchKernelGGL(shuffle_bf16_kernel, dim3(blocks), dim3(256), 0, s, src, src_dtype, Kd, C,
                       Kdp, Cp, dst);
}

void mxm_launch_transpose_bf16(const void* src, int src_dtype, int Kd, int C, int slot,
                               uint16_t* dst, hipStream_t s, int ldd) {
  const dim3 grid((C + 31) / 32, (Kd + 31) / 32);
  hipLaunchKernelGGL(transpose_kernel, grid, dim3(32, 8), 0, s, src, src_dtype, Kd, C, slot, dst,
                     ldd > 0 ? ldd : Kd);
}

namespace {

// router_w [D, E] (x.W layout, in the flow's dtype T) -> the decode router's
// lane-interleaved layout [ceil(E/64)][ldw/P][64][P], P = 16 / sizeof(T):
// element (g, c, l, q) = router_w[Pc + q][64g + l], zero past D or E.  Lane l
// of a wave for expert group g reads its expert's next P d values as one
// 16-byte piece, and the 64 lanes' pieces are one contiguous 1 KB line set.
template <typename T>
__global__ void router_t_kernel(const T* src, int D, int E, int ldw, T* dst) {
  constexpr int P = 16 / (int)sizeof(T);
  const int G = (E + 63) / 64;
  const int64_t n = (int64_t)G * ldw * 64;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int q = (int)(i % P), l = (int)((i / P) & 63);
    const int64_t gc = i / (64 * P);  // g * (ldw / P) + c
    const int c = (int)(gc % (ldw / P)), g = (int)(gc / (ldw / P));
    const int d = P * c + q, e = 64 * g + l;
    dst[i] = (d < D && e < E) ? src[(size_t)d * E + e] : T(0);
  }
}

}  // namespace

void mxm_launch_router_t(const void* src, bool bf16, int D, int E, int ldw, void* dst,
                         hipStream_t s) {
  const int64_t n = (int64_t)((E + 63) / 64) * ldw * 64;
  if (n <= 0) return;
  if (bf16)
    hipLaunchKernelGGL(router_t_kernel<uint16_t>, dim3(grid_for(n)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(src), D, E, ldw, static_cast<uint16_t*>(dst));
  else
    hipLaunchKernelGGL(router_t_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s,
                       static_cast<const float*>(src), D, E, ldw, static_cast<float*>(dst));
}

namespace {

// MFMA-family expert weights back to fp32 in x.W layout, for the backward of
// bf16 ops.  w1 holds per expert [NC][Dk] bf16 (NC = 2Fk, gate and up rows
// interleaved in groups of 32, or Fk for one matrix; Fk >= F and Dk >= D the
// padded widths); slot picks the matrix (0 gate, 1 up, -1 not interleaved).
// dst[e][d][f] = w1[e][q(f)][d].
__global__ void w1_to_xw_kernel(const uint16_t* w1, int E, int D, int F, int Dk, int Fk, int slot,
                                float* dst) {
  const int NC = slot < 0 ? Fk : 2 * Fk;
  const int64_t n = (int64_t)E * D * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int f = (int)(i % F);
    const int64_t ed = i / F;
    const int d = (int)(ed % D), e = (int)(ed / D);
    const int q = slot < 0 ? f : (f >> 5) * 64 + slot * 32 + (f & 31);
    dst[i] = mxm_bf2f(w1[((size_t)e * NC + q) * Dk + d]);
  }
}

// w2 [E][Dk][Fk] bf16 (the down projection, k = F contiguous) -> dst [E][F][D].
__global__ void w2_to_xw_kernel(const uint16_t* w2, int E, int D, int F, int Dk, int Fk,
                                float* dst) {
  const int64_t n = (int64_t)E * D * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    const int64_t ef = i / D;
    const int f = (int)(ef % F), e = (int)(ef / F);
    dst[i] = mxm_bf2f(w2[((size_t)e * Dk + d) * Fk + f]);
  }
}

}  // namespace

void mxm_launch_w1_to_xw(const uint16_t* w1, int E, int D, int F, int Dk, int Fk, int slot,
                         float* dst, hipStream_t s) {
  const int64_t n = (int64_t)E * D * F;
  if (n > 0)
    hipLaunchKernelGGL(w1_to_xw_kernel, dim3(grid_for(n)), dim3(256), 0, s, w1, E, D, F, Dk, Fk,
                       slot, dst);
}

void mxm_launch_w2_to_xw(const uint16_t* w2, int E, int D, int F, int Dk, int Fk, float* dst,
                         hipStream_t s) {
  const int64_t n = (int64_t)E * D * F;
  if (n > 0)
    hipLaunchKernelGGL(w2_to_xw_kernel, dim3(grid_for(n)), dim3(256), 0, s, w2, E, D, F, Dk, Fk,
                       dst);
}
