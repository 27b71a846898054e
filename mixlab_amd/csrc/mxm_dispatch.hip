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
// kernel below turns the counts into offsets and per-(expert, tile) bases
// (one workgroup per expert), and the scatter kernel places every slot.  Nothing here uses atomics, so
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

constexpr int SCAN_NT = 256;

// Workgroup e < E: expert e's total, its mean probability and the exclusive
// prefix of its per-tile counts (relative to the expert's first row);
// workgroup E: the entropy.  The last expert workgroup to finish (agent-scope
// release fence, atomic ticket; agent-scope acquire) computes counts,
// offsets, both row-tile prefixes and aux from the per-expert totals and
// resets the ticket.  No workgroup waits for another, so the grid always
// drains.  The floating-point sums keep one fixed order: per expert (and for
// the entropy) lane-strided sequential partial sums over the tiles, then an
// xor butterfly over the wave; aux over experts in ascending order.
template <bool BF16>
__global__ __launch_bounds__(SCAN_NT) void scan_kernel(ScanArgs a) {
  __shared__ int wtot[SCAN_NT / 64];
  __shared__ int s_last;
  __shared__ int scount[MXM_MAX_EXPERTS];
  __shared__ float spmean[MXM_MAX_EXPERTS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int T = a.ntiles;
  const int e = blockIdx.x;
  constexpr int SB = 16;  // loads per lane issued together

  if (e == a.E) {
    if (wave == 0) {
      float sum = 0.0f;
      for (int t0 = lane; t0 < T; t0 += 64 * SB) {
        float ev[SB];
#pragma unroll
        for (int b = 0; b < SB; ++b) ev[b] = t0 + 64 * b < T ? a.tile_ent[t0 + 64 * b] : 0.0f;
#pragma unroll
        for (int b = 0; b < SB; ++b)
          if (t0 + 64 * b < T) sum = sum + ev[b];
      }
      sum = wave_sum_fixed(sum);
      if (lane == 0) a.entropy[0] = -(sum / (float)a.N);
    }
    return;
  }

  const int32_t* tc = a.tile_counts + (size_t)e * T;
  if (wave == 0) {
    const float* tp = a.tile_psum + (size_t)e * T;
    float ps = 0.0f;
    for (int t0 = lane; t0 < T; t0 += 64 * SB) {
      float pv[SB];
#pragma unroll
      for (int b = 0; b < SB; ++b) pv[b] = t0 + 64 * b < T ? tp[t0 + 64 * b] : 0.0f;
#pragma unroll
      for (int b = 0; b < SB; ++b)
        if (t0 + 64 * b < T) ps = ps + pv[b];
    }
    ps = wave_sum_fixed(ps);
    if (lane == 0) {
      const float mean = ps / (float)a.N;
      a.expert_pmean[e] = BF16 ? mxm_rbf(mean) : mean;
    }
  }
  // thread i owns tiles [i*R, i*R + R): its run total, the workgroup's
  // exclusive scan of the run totals, then the tiles' bases
  const int R = (T + SCAN_NT - 1) / SCAN_NT;
  const int t_lo = min(T, tid * R), t_hi = min(T, t_lo + R);
  int run = 0;
  for (int t = t_lo; t < t_hi; ++t) run += tc[t];
  int incl = run;
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) {
    const int up = __shfl_up(incl, sh, 64);
    if (lane >= sh) incl += up;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = incl - run;
  for (int w = 0; w < wave; ++w) base += wtot[w];
  for (int t = t_lo; t < t_hi; ++t) {
    a.tile_base[(size_t)e * T + t] = base;
    base += tc[t];
  }
  if (tid == SCAN_NT - 1) a.expert_count[e] = base;  // the expert's total

  // ---- ticket: the last expert workgroup continues ----
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(a.ticket, 1) == a.E - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  // every expert's total read in one round of loads
  for (int x = tid; x < a.E; x += SCAN_NT) {
    scount[x] = a.expert_count[x];
    spmean[x] = a.expert_pmean[x];
  }
  __syncthreads();
  if (tid == 0) {
    int o = 0, m1 = 0, m2 = 0;
    float aux = 0.0f;
    for (int x = 0; x < a.E; ++x) {
      const int c = scount[x];
      a.offsets[x] = o;
      a.counts[x] = c;
      a.mstart1[x] = m1;
      a.mstart2[x] = m2;
      o += c;
      m1 += (c + a.bm1 - 1) / a.bm1;
      m2 += (c + a.bm2 - 1) / a.bm2;
      const float frac = ((float)c / (float)a.K) / (float)a.N;
      const float term = spmean[x] * frac;
      aux = (x == 0) ? term : aux + term;
    }
    a.offsets[a.E] = o;
    a.mstart1[a.E] = m1;
    a.mstart2[a.E] = m2;
    const float raw = aux * (float)a.E;
    a.aux[0] = raw;
    if (a.aux_scaled) a.aux_scaled[0] = raw * a.aux_weight;
    __hip_atomic_store(a.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(256) void scatter_kernel(ScatterArgs a) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= (int64_t)a.N * a.K) return;
  const int n = (int)(s / a.K);
  const int e = a.top_idx[s];
  const int tile = n / MXM_ROUTER_TM;
  const int pos = a.offsets[e] + a.tile_base[(size_t)e * a.ntiles + tile] + a.slot_rank[s];
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
  const size_t ldy = a.ldy > 0 ? (size_t)a.ldy : (size_t)a.D;
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
                reinterpret_cast<const raw_t*>(y + (size_t)sp[k0 + u] * ldy + d));
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
        const TY* src = y + (size_t)sp[k] * ldy + d;
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


// The int8 decode flow's combine: y token-major, so a token's rows are known
// before its picks are read -- the first KC rows of each thread's first
// columns are requested first, then the gates are sorted into ascending
// expert order, then the sum runs multiply then add in fp32 in that order
// (the reference's e-loop, as combine_kernel).
template <typename TY, int VEC>
__global__ __launch_bounds__(256) void combine_tm_kernel(CombineArgs a) {
  __shared__ int sk[MXM_MAX_EXPERTS];
  __shared__ float sg[MXM_MAX_EXPERTS];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int K = a.K;
  const TY* y = static_cast<const TY*>(a.y);
  const size_t ldy = a.ldy > 0 ? (size_t)a.ldy : (size_t)a.D;
  const size_t row0 = (size_t)n * K;
  constexpr bool WIDE = (sizeof(TY) == 2 && VEC == 8) || (sizeof(TY) == 4 && VEC == 4);
  typedef typename std::conditional<sizeof(TY) == 2, vu4, vf4>::type raw_t;
  constexpr int KC = 8;
  const int d0 = tid * VEC;
  raw_t pre[KC];
  if constexpr (WIDE) {
    if (d0 < a.D) {
#pragma unroll
      for (int u = 0; u < KC; ++u)
        if (u < K) pre[u] = __builtin_nontemporal_load(
                       reinterpret_cast<const raw_t*>(y + (row0 + u) * ldy + d0));
    }
  }
  int e = 0;
  float g = 0.0f;
  if (tid < K) {
    e = a.top_idx[row0 + tid];
    g = a.gates[row0 + tid];
    sk[tid] = e;
  }
  __syncthreads();
  if (tid < K) {
    int r = 0;
    for (int j = 0; j < K; ++j) r += sk[j] < e;
    sg[r] = g;
  }
  __syncthreads();
  auto add_raw = [&](float (&acc)[VEC], const raw_t& v, float gg) {
    float f[VEC];
    if constexpr (sizeof(TY) == 2) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = mxm_u2f(v[q] << 16);
        f[2 * q + 1] = mxm_u2f(v[q] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) f[q] = v[q];
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(f[q], gg));
  };
  for (int d = d0; d < a.D; d += 256 * VEC) {
    float acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = 0.0f;
    if constexpr (WIDE) {
      for (int k0 = 0; k0 < K; k0 += KC) {
        const int kn = min(KC, K - k0);
        raw_t r[KC];
        if (d == d0 && k0 == 0) {
#pragma unroll
          for (int u = 0; u < KC; ++u) r[u] = pre[u];
        } else {
#pragma unroll
          for (int u = 0; u < KC; ++u)
            if (u < kn) r[u] = __builtin_nontemporal_load(
                            reinterpret_cast<const raw_t*>(y + (row0 + k0 + u) * ldy + d));
        }
#pragma unroll
        for (int u = 0; u < KC; ++u)
          if (u < kn) add_raw(acc, r[u], sg[k0 + u]);
      }
    } else {
      for (int k = 0; k < K; ++k) {
        const TY* src = y + (row0 + k) * ldy + d;
        float f[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          if constexpr (sizeof(TY) == 2)
            f[q] = mxm_bf2f(reinterpret_cast<const uint16_t*>(src)[q]);
          else
            f[q] = reinterpret_cast<const float*>(src)[q];
        }
#pragma unroll
        for (int q = 0; q < VEC; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(f[q], sg[k]));
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
    hipLaunchKernelGGL(scan_kernel<true>, dim3(a.E + 1), dim3(SCAN_NT), 0, s, a);
  else
    hipLaunchKernelGGL(scan_kernel<false>, dim3(a.E + 1), dim3(SCAN_NT), 0, s, a);
}

void mxm_launch_scatter(const ScatterArgs& a, hipStream_t s) {
  const int64_t slots = (int64_t)a.N * a.K;
  const int blocks = (int)((slots + 255) / 256);
  if (blocks > 0) hipLaunchKernelGGL(scatter_kernel, dim3(blocks), dim3(256), 0, s, a);
}

void mxm_launch_combine(const CombineArgs& a, bool y_bf16, hipStream_t s) {
  if (a.N <= 0) return;
  const int ldy = a.ldy > 0 ? a.ldy : a.D;
  const bool aligned = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(a.delta) % 16 == 0) && ldy % 8 == 0;
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

void mxm_launch_combine_tm(const CombineArgs& a, bool y_bf16, hipStream_t s) {
  if (a.N <= 0) return;
  const int ldy = a.ldy > 0 ? a.ldy : a.D;
  const bool aligned = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(a.delta) % 16 == 0) && ldy % 8 == 0;
  const dim3 grid(a.N);
  if (y_bf16) {
    if (aligned && a.D % 8 == 0)
      hipLaunchKernelGGL((combine_tm_kernel<uint16_t, 8>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((combine_tm_kernel<uint16_t, 1>), grid, dim3(256), 0, s, a);
  } else {
    if (aligned && a.D % 4 == 0)
      hipLaunchKernelGGL((combine_tm_kernel<float, 4>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((combine_tm_kernel<float, 1>), grid, dim3(256), 0, s, a);
  }
}
