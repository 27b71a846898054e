// Dispatch (per-expert counts, offsets, stable token permutation) and the
// deterministic combine.
//
// The reference has no dispatch: it runs every expert densely and masks with
// `top_idx == e` (gpu/ir.cpp:1118-1148).  The grouping defined here is the
// one that mask implies: expert e's rows are the tokens n with e among
// top_idx[n, :], in ascending n, and experts follow in ascending e.
//   counts[e]      = #{n : e in top_idx[n, :]}
//   offsets        = exclusive scan of counts (offsets[E] = N*K)
//   perm[offsets[e] + r] = the r-th such token
// The router leaves per-tile counts and per-slot in-tile ranks; the scan
// kernel below turns the counts into offsets and per-(expert, tile) bases,
// and the scatter kernel places every slot.  Nothing here uses atomics, so
// the result does not depend on scheduling.
//
// The combine sums, per token, gate * y over its K slots in ascending expert
// id, multiply then add in fp32, starting from 0 -- the accumulation order of
// `out = out + expert_out * gate` over e = 0..E-1 in gpu/ir.cpp:1148
// (unselected experts add +0 there).  Y is read once and delta written once,
// so the vector paths use nontemporal loads and stores (at 65,536 tokens the
// two are 2.7 GB, ten times the last-level cache; 0.52 -> 0.47 ms).
#include "mxm_kernels.h"

#include <type_traits>

namespace {
// 16-byte vectors for the nontemporal builtins (which take clang vector
// types, not HIP's float4 / uint4 structs).
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef unsigned int vu4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum_fixed(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v = v + __shfl_xor(v, s, 64);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
  return v;
}

constexpr int SCAN_NT = 1024;

template <bool BF16>
__global__ __launch_bounds__(SCAN_NT) void scan_kernel(ScanArgs a) {
  __shared__ int cnt[MXM_MAX_EXPERTS];
  __shared__ int offs[MXM_MAX_EXPERTS + 1];
  __shared__ float pmean[MXM_MAX_EXPERTS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int NW = SCAN_NT / 64;
  const int T = a.ntiles;

  // pass 1: per-expert totals and probability sums (lane-strided sequential
  // partial sums, then a fixed butterfly); the loads of SB tiles per lane are
  // issued together
  constexpr int SB = 16;
  for (int e = wave; e < a.E; e += NW) {
    int c = 0;
    float ps = 0.0f;
    for (int t0 = lane; t0 < T; t0 += 64 * SB) {
      int cv[SB];
      float pv[SB];
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        const int t = t0 + 64 * b;
        cv[b] = t < T ? a.tile_counts[(size_t)e * T + t] : 0;
        pv[b] = t < T ? a.tile_psum[(size_t)e * T + t] : 0.0f;
      }
#pragma unroll
      for (int b = 0; b < SB; ++b)
        if (t0 + 64 * b < T) {
          c += cv[b];
          ps = ps + pv[b];
        }
    }
    c = wave_sum_int(c);
    ps = wave_sum_fixed(ps);
    if (lane == 0) {
      cnt[e] = c;
      const float mean = ps / (float)a.N;
      pmean[e] = BF16 ? mxm_rbf(mean) : mean;
    }
  }
  if (wave == NW - 1) {
    float s = 0.0f;
    for (int t0 = lane; t0 < T; t0 += 64 * SB) {
      float ev[SB];
#pragma unroll
      for (int b = 0; b < SB; ++b) ev[b] = t0 + 64 * b < T ? a.tile_ent[t0 + 64 * b] : 0.0f;
#pragma unroll
      for (int b = 0; b < SB; ++b)
        if (t0 + 64 * b < T) s = s + ev[b];
    }
    s = wave_sum_fixed(s);
    if (lane == 0) a.entropy[0] = -(s / (float)a.N);
  }
  __syncthreads();

  if (tid == 0) {
    int o = 0, m1 = 0, m2 = 0;
    float aux = 0.0f;
    for (int e = 0; e < a.E; ++e) {
      const int c = cnt[e];
      offs[e] = o;
      a.offsets[e] = o;
      a.counts[e] = c;
      a.mstart1[e] = m1;
      a.mstart2[e] = m2;
      o += c;
      m1 += (c + a.bm1 - 1) / a.bm1;
      m2 += (c + a.bm2 - 1) / a.bm2;
      const float frac = ((float)c / (float)a.K) / (float)a.N;
      const float term = pmean[e] * frac;
      aux = (e == 0) ? term : aux + term;
    }
    offs[a.E] = o;
    a.offsets[a.E] = o;
    a.mstart1[a.E] = m1;
    a.mstart2[a.E] = m2;
    const float raw = aux * (float)a.E;
    a.aux[0] = raw;
    if (a.aux_scaled) a.aux_scaled[0] = raw * a.aux_weight;
  }
  __syncthreads();

  // pass 2: exclusive scan over tiles, per expert (SB chunks of 64 tiles
  // loaded together, then scanned in order)
  for (int e = wave; e < a.E; e += NW) {
    int carry = offs[e];
    for (int c0 = 0; c0 < T; c0 += 64 * SB) {
      int cv[SB];
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        const int t = c0 + 64 * b + lane;
        cv[b] = t < T ? a.tile_counts[(size_t)e * T + t] : 0;
      }
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        if (c0 + 64 * b < T) {  // wave-uniform
          const int t = c0 + 64 * b + lane;
          int incl = cv[b];
#pragma unroll
          for (int s = 1; s < 64; s <<= 1) {
            const int up = __shfl_up(incl, s, 64);
            if (lane >= s) incl += up;
          }
          if (t < T) a.tile_base[(size_t)e * T + t] = carry + incl - cv[b];
          carry += __shfl(incl, 63, 64);
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void scatter_kernel(ScatterArgs a) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= (int64_t)a.N * a.K) return;
  const int n = (int)(s / a.K);
  const int e = a.top_idx[s];
  const int tile = n / MXM_ROUTER_TM;
  const int pos = a.tile_base[(size_t)e * a.ntiles + tile] + a.slot_rank[s];
  a.perm[pos] = n;
  a.slot_pos[s] = pos;
}

template <typename TY>
__device__ __forceinline__ void load_y(const TY* p, float* f, int vec);

template <typename TY, int VEC>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  __shared__ int sk[MXM_MAX_EXPERTS];  // the token's experts in top-k order
  __shared__ int sp[MXM_MAX_EXPERTS];  // slot positions, ascending expert id
  __shared__ float sg[MXM_MAX_EXPERTS];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int K = a.K;  // K <= E <= 256 = blockDim.x
  int e = 0, p = 0;
  float g = 0.0f;
  if (tid < K) {
    e = a.top_idx[(size_t)n * K + tid];
    g = a.gates[(size_t)n * K + tid];
    p = a.slot_pos[(size_t)n * K + tid];
    sk[tid] = e;
  }
  __syncthreads();
  // a token's K experts are distinct, so the number of smaller ones is the
  // slot's place in ascending expert order
  if (tid < K) {
    int r = 0;
    for (int j = 0; j < K; ++j) r += sk[j] < e;
    sp[r] = p;
    sg[r] = g;
  }
  __syncthreads();
  const TY* y = static_cast<const TY*>(a.y);
  for (int d = tid * VEC; d < a.D; d += 256 * VEC) {
    float acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = 0.0f;
    if constexpr ((sizeof(TY) == 2 && VEC == 8) || (sizeof(TY) == 4 && VEC == 4)) {
      // the rows of up to KC slots are requested together, then accumulated
      // in ascending expert order
      constexpr int KC = 8;
      typedef typename std::conditional<sizeof(TY) == 2, vu4, vf4>::type raw_t;
      for (int k0 = 0; k0 < K; k0 += KC) {
        const int kn = min(KC, K - k0);
        raw_t r[KC];
#pragma unroll
        for (int u = 0; u < KC; ++u)
          if (u < kn)
            r[u] = __builtin_nontemporal_load(
                reinterpret_cast<const raw_t*>(y + (size_t)sp[k0 + u] * a.D + d));
#pragma unroll
        for (int u = 0; u < KC; ++u) {
          if (u < kn) {
            float f[VEC];
            if constexpr (sizeof(TY) == 2) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                f[2 * q] = mxm_u2f(r[u][q] << 16);
                f[2 * q + 1] = mxm_u2f(r[u][q] & 0xffff0000u);
              }
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) f[q] = r[u][q];
            }
            const float g = sg[k0 + u];
#pragma unroll
            for (int q = 0; q < VEC; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(f[q], g));
          }
        }
      }
    } else {
      for (int k = 0; k < K; ++k) {
        const TY* src = y + (size_t)sp[k] * a.D + d;
        float f[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          if constexpr (sizeof(TY) == 2)
            f[q] = mxm_bf2f(reinterpret_cast<const uint16_t*>(src)[q]);
          else
            f[q] = reinterpret_cast<const float*>(src)[q];
        }
        const float g = sg[k];
#pragma unroll
        for (int q = 0; q < VEC; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(f[q], g));
      }
    }
    if (a.resid) {
      // block level: x + delta (* moe_scale), fp32
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const size_t i = (size_t)n * a.D + d + q;
        const float xr = a.resid_bf16 ? mxm_bf2f(static_cast<const uint16_t*>(a.resid)[i])
                                      : static_cast<const float*>(a.resid)[i];
        float v = acc[q];
        if (a.rscale) {
          const float sc = a.rscale_bf16 ? mxm_bf2f(static_cast<const uint16_t*>(a.rscale)[d + q])
                                         : static_cast<const float*>(a.rscale)[d + q];
          v = __fmul_rn(v, sc);
        }
        acc[q] = __fadd_rn(xr, v);
      }
    }
    float* dst = a.delta + (size_t)n * a.D + d;
    if constexpr (VEC == 4 || VEC == 8) {
#pragma unroll
      for (int q = 0; q < VEC; q += 4)
        __builtin_nontemporal_store(vf4{acc[q], acc[q + 1], acc[q + 2], acc[q + 3]},
                                    reinterpret_cast<vf4*>(dst + q));
    } else {
#pragma unroll
      for (int q = 0; q < VEC; ++q) dst[q] = acc[q];
    }
  }
}

}  // namespace

void mxm_launch_scan(const ScanArgs& a, bool bf16, hipStream_t s) {
  if (bf16)
    hipLaunchKernelGGL(scan_kernel<true>, dim3(1), dim3(SCAN_NT), 0, s, a);
  else
    hipLaunchKernelGGL(scan_kernel<false>, dim3(1), dim3(SCAN_NT), 0, s, a);
}

void mxm_launch_scatter(const ScatterArgs& a, hipStream_t s) {
  const int64_t slots = (int64_t)a.N * a.K;
  const int blocks = (int)((slots + 255) / 256);
  if (blocks > 0) hipLaunchKernelGGL(scatter_kernel, dim3(blocks), dim3(256), 0, s, a);
}

void mxm_launch_combine(const CombineArgs& a, bool y_bf16, hipStream_t s) {
  if (a.N <= 0) return;
  const bool aligned = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(a.delta) % 16 == 0);
  if (y_bf16) {
    if (aligned && a.D % 8 == 0)
      hipLaunchKernelGGL((combine_kernel<uint16_t, 8>), dim3(a.N), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((combine_kernel<uint16_t, 1>), dim3(a.N), dim3(256), 0, s, a);
  } else {
    if (aligned && a.D % 4 == 0)
      hipLaunchKernelGGL((combine_kernel<float, 4>), dim3(a.N), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((combine_kernel<float, 1>), dim3(a.N), dim3(256), 0, s, a);
  }
}
