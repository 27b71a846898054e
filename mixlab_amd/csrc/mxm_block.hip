// Block-level pieces of the MoE block (arch/moe.go:152-166): the RMSNorm in
// front of op 74 (gpu/ir.cpp:4949-4960).  The residual add and the moe_scale
// multiply are fused into the combine kernel.
//
// The norm's arithmetic is fixed so the CPU restatement reproduces it bit
// for bit (the normalised rows feed the router, whose top-k must match): one
// wave per row; lane l accumulates s += x[d]*x[d] (product rounded, then the
// sum) over d = 256*i + 4*l + j, i ascending, then j = 0..3; the 64 lane sums
// meet in an xor butterfly over distances 32, 16, 8, 4, 2, 1 (the same
// butterfly as the router's softmax); ms = sum * inv_d with inv_d the fp32
// value of 1/D; r = 1 / sqrt(ms + eps), sqrt and division correctly rounded;
// y = (x * r) * scale, rounded to the output dtype (bf16 round-to-nearest-
// even, or fp32).
#include "mxm_kernels.h"

namespace {

template <bool BF>
__device__ __forceinline__ float ld_elem(const void* p, size_t i) {
  if (BF) return mxm_bf2f(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

template <bool XBF, bool SBF, bool OBF>
__global__ __launch_bounds__(256) void rmsnorm_kernel(RmsNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= a.N) return;  // wave-uniform
  const int D = a.D;
  const size_t row = (size_t)n * D;
  float acc = 0.0f;
  for (int d0 = 0; d0 < D; d0 += 256) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = d0 + 4 * lane + j;
      if (d < D) {
        const float v = ld_elem<XBF>(a.x, row + d);
        acc = acc + v * v;
      }
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc = acc + mxm_xor_lane_f(acc, s);
  const float ms = acc * a.inv_d;
  const float r = 1.0f / __builtin_sqrtf(ms + a.eps);
  for (int d0 = 0; d0 < D; d0 += 256) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = d0 + 4 * lane + j;
      if (d < D) {
        const float y = (ld_elem<XBF>(a.x, row + d) * r) * ld_elem<SBF>(a.scale, d);
        if (OBF)
          static_cast<uint16_t*>(a.out)[row + d] = mxm_f2bf(y);
        else
          static_cast<float*>(a.out)[row + d] = y;
      }
    }
  }
}

template <bool XBF, bool SBF>
void launch_o(const RmsNormArgs& a, hipStream_t s) {
  const int blocks = (a.N + 3) / 4;
  if (a.out_bf16)
    hipLaunchKernelGGL((rmsnorm_kernel<XBF, SBF, true>), dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<XBF, SBF, false>), dim3(blocks), dim3(256), 0, s, a);
}

template <bool XBF>
void launch_s(const RmsNormArgs& a, hipStream_t s) {
  if (a.scale_bf16)
    launch_o<XBF, true>(a, s);
  else
    launch_o<XBF, false>(a, s);
}

}  // namespace

void mxm_launch_rmsnorm(const RmsNormArgs& a, hipStream_t s) {
  if (a.N <= 0) return;
  if (a.x_bf16)
    launch_s<true>(a, s);
  else
    launch_s<false>(a, s);
}
