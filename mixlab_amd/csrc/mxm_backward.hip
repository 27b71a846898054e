// Backward of the MoE feed-forward op (gpu/ir.cpp:1073-1164 differentiated
// as MLX's autodiff does; the reference checks it with
// gpu/moe_feed_forward_test.go:84-151), fp32 flow.
//
// With dD = dL/d(delta) and the routing of the forward held fixed:
//   gate gradient   dg[n,k]  = <dD[n], y_k[n]>
//   renorm          g_k = tp_k / max(S, 1e-12), S = sum_k tp_k:
//                   dtp_k = sum_j tp_j (dg_k - dg_j) / S^2  (S > 1e-12; else dg_k / 1e-12)
//   probabilities   dp[n,e] = sum_k [top_idx = e] dtp_k
//                           + d_aux * E * counts[e] / (K N) / N
//                           - d_ent / N * (log max(p, 1e-12) + [p > 1e-12])
//   softmax         dlogits = p * (dp - <p, dp>)
//   router          dWr = x^T dlogits,  dx += dlogits Wr^T
//   experts (per routed slot, y = h W_down, h = act(g) * u or act(u)):
//                   dY = gate * dD, dH = dY W_down^T, dW_down = H^T dY,
//                   (dG, dU) from the activation's derivative,
//                   dx += dG W_gate^T + dU W_up^T,
//                   dW_gate = X^T dG, dW_up = X^T dU.
// The router part runs here (dgates, router_bw, dy, the router's input and
// weight gradients; the weight gradient reduces over row chunks in a fixed
// order).  The experts' products run on the MFMA grouped GEMM and weight-
// gradient kernels (bf16, or fp32 values as bf16 planes), issued by the
// library's host code; the elementwise parts around them (activation
// derivatives, planes, dx sums) are the kernels here.  Every result is
// deterministic.
#include <algorithm>

#include "mxm_kernels.h"

namespace {

__device__ __forceinline__ float ld_x(const float* p) { return *p; }
__device__ __forceinline__ float ld_x(const uint16_t* p) { return mxm_bf2f(*p); }


// dst[b][c][r] = src[b][r][c]
__global__ void transpose_f32_kernel(const float* __restrict__ src, int R, int C,
                                     float* __restrict__ dst) {
  __shared__ float t[32][33];
  const size_t off = (size_t)blockIdx.z * R * C;
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + threadIdx.x;
    t[i][threadIdx.x] = (r < R && c < C) ? src[off + (size_t)r * C + c] : 0.0f;
  }
  __syncthreads();
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + threadIdx.x;
    if (r < R && c < C) dst[off + (size_t)c * R + r] = t[threadIdx.x][i];
  }
}

// One workgroup per token n, for each of its slots s = n*K + k in order:
// dgates[s] = <dD[n], Y[slot_pos[s]]> and dY[slot_pos[s]] = gates[s] * dD[n]
// (bf16 or fp32).  V = 4: 4 consecutive d per thread (16-byte dD loads, 8 or
// 16-byte Y loads and dY stores); V = 1 for shapes or pointers that do not
// allow it.  The dot product is reduced over the workgroup in a fixed order.
template <int V>
__global__ __launch_bounds__(256) void dgates_dy_kernel(BackwardArgs a) {
  __shared__ float red[4];
  const int n = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const int D = a.D, K = a.K;
  const float* dd = a.d_delta + (size_t)n * D;
  for (int k = 0; k < K; ++k) {
    const int s = n * K + k;
    const size_t o = (size_t)a.slot_pos[s] * D;
    const float g = a.gates[s];
    float acc = 0.0f;
    for (int d = tid * V; d < D; d += nt * V) {
      float dv[V], yv[V];
      if constexpr (V == 4) {
        const float4 t = *reinterpret_cast<const float4*>(dd + d);
        dv[0] = t.x; dv[1] = t.y; dv[2] = t.z; dv[3] = t.w;
        if (a.Yb16) {
          const uint2 w = *reinterpret_cast<const uint2*>(a.Yb16 + o + d);
          yv[0] = mxm_u2f(w.x << 16); yv[1] = mxm_u2f(w.x & 0xffff0000u);
          yv[2] = mxm_u2f(w.y << 16); yv[3] = mxm_u2f(w.y & 0xffff0000u);
        } else {
          const float4 y = *reinterpret_cast<const float4*>(a.Y + o + d);
          yv[0] = y.x; yv[1] = y.y; yv[2] = y.z; yv[3] = y.w;
        }
      } else {
        dv[0] = dd[d];
        yv[0] = a.Yb16 ? mxm_bf2f(a.Yb16[o + d]) : a.Y[o + d];
      }
#pragma unroll
      for (int q = 0; q < V; ++q) acc = __builtin_fmaf(dv[q], yv[q], acc);
      if (a.dyb16) {
        if constexpr (V == 4) {
          const uint32_t lo = (uint32_t)mxm_f2bf(g * dv[0]) | (uint32_t)mxm_f2bf(g * dv[1]) << 16;
          const uint32_t hi = (uint32_t)mxm_f2bf(g * dv[2]) | (uint32_t)mxm_f2bf(g * dv[3]) << 16;
          *reinterpret_cast<uint2*>(a.dyb16 + o + d) = uint2{lo, hi};
        } else {
          a.dyb16[o + d] = mxm_f2bf(g * dv[0]);
        }
      } else {
        if constexpr (V == 4)
          *reinterpret_cast<float4*>(a.dy + o + d) =
              float4{g * dv[0], g * dv[1], g * dv[2], g * dv[3]};
        else
          a.dy[o + d] = g * dv[0];
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + mxm_xor_lane_f(acc, m);
    if ((tid & 63) == 0) red[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) {
      float t = red[0];
      for (int w = 1; w < nt / 64; ++w) t = t + red[w];
      a.dgates[s] = t;
    }
    __syncthreads();
  }
}

// One wave per token (4 tokens per workgroup): renorm, aux / entropy and
// softmax backward.  The token's K slot gate gradients dg_k and selected
// probabilities go to LDS; lane k computes d(tp_k), which lands at its
// expert sel[k] (the K experts are distinct); lane e then forms
// dp_e = aux term - entropy term + d(tp) of e, and dlogits_e =
// p_e (dp_e - sum_e' p_e' dp_e') with the sum reduced over the wave.
__global__ __launch_bounds__(256) void router_bw_kernel(BackwardArgs a) {
  __shared__ float dgs[4][MXM_MAX_EXPERTS], tps[4][MXM_MAX_EXPERTS], add[4][MXM_MAX_EXPERTS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + wave;
  if (n >= a.N) return;  // (the whole wave; no workgroup barrier below)
  const int K = a.K, E = a.E;
  const float* p = a.probs + (size_t)n * E;
  const int32_t* sel = a.top_idx + (size_t)n * K;
  const int32_t* sp = a.slot_pos + (size_t)n * K;
  // gate gradient of slot k (by slot position when the caller computed them there)
  for (int k = lane; k < K; k += 64) {
    dgs[wave][k] = a.dgp ? a.dgp[sp[k]] : a.dgates[(size_t)n * K + k];
    tps[wave][k] = p[sel[k]];
  }
  for (int e = lane; e < E; e += 64) add[wave][e] = 0.0f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float S = 0.0f;
  for (int k = 0; k < K; ++k) S = S + tps[wave][k];
  const float Sc = fmaxf(S, 1e-12f);
  const bool renorm = S > 1e-12f;
  // d(tp_k) = dg_k / S - sum_j dg_j tp_j / S^2 = sum_j tp_j (dg_k - dg_j) / S^2,
  // the second form free of the cancellation of the first (exactly 0 at K = 1)
  for (int k = lane; k < K; k += 64) {
    const float dgk = dgs[wave][k];
    float d;
    if (!renorm) {
      d = dgk / Sc;
    } else {
      float t = 0.0f;
      for (int j = 0; j < K; ++j) t = t + tps[wave][j] * (dgk - dgs[wave][j]);
      d = t / (Sc * Sc);
    }
    add[wave][sel[k]] = d;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float inv_n = 1.0f / (float)a.N;
  const float aux_c = a.d_aux * (float)E * inv_n / ((float)K * (float)a.N);
  constexpr int EL = MXM_MAX_EXPERTS / 64;  // experts per lane
  float dp[EL], pe[EL];
  float ps = 0.0f;
#pragma unroll
  for (int i = 0; i < EL; ++i) {
    const int e = lane + 64 * i;
    dp[i] = 0.0f;
    pe[i] = 0.0f;
    if (e < E) {
      pe[i] = p[e];
      float v = aux_c * (float)a.counts[e];
      v = v - a.d_ent * inv_n * (logf(fmaxf(pe[i], 1e-12f)) + (pe[i] > 1e-12f ? 1.0f : 0.0f));
      dp[i] = v + add[wave][e];
      ps = __builtin_fmaf(pe[i], dp[i], ps);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ps = ps + mxm_xor_lane_f(ps, m);
  float* out = a.dlogits + (size_t)n * E;
#pragma unroll
  for (int i = 0; i < EL; ++i) {
    const int e = lane + 64 * i;
    if (e < E) out[e] = pe[i] * (dp[i] - ps);
  }
}

__device__ __forceinline__ float gelu_t(float v, float& deriv) {
  const float c = 0.7978845608f, k = 0.044715f;
  const float in = c * (v + k * v * v * v);
  const float t = tanhf(in);
  deriv = 0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * c * (1.0f + 3.0f * k * v * v);
  return 0.5f * v * (1.0f + t);
}

// The hidden unit of one routed row and its derivatives (fp32 flow): h, and
// dh/dg (GLU only) and dh/du.
__device__ __forceinline__ void act_eval(int etype, int act, float slope, float g, float u,
                                         float& h, float& cg, float& cu) {
  if (etype == MXM_EXPERT_MLP) {
    float d;
    switch (act) {
      case MXM_ACT_SILU: {
        const float sg = 1.0f / (1.0f + expf(-u));
        h = u * sg;
        d = sg * (1.0f + u * (1.0f - sg));
        break;
      }
      case MXM_ACT_GELU:
        h = gelu_t(u, d);
        break;
      case MXM_ACT_RELU:
        h = u > 0.0f ? u : 0.0f;
        d = u > 0.0f ? 1.0f : 0.0f;
        break;
      default: {
        const float y = u > 0.0f ? u : u * slope;
        h = y * y;
        d = 2.0f * y * (u > 0.0f ? 1.0f : slope);
        break;
      }
    }
    cg = 0.0f;
    cu = d;
  } else {
    float a, d;
    if (etype == MXM_EXPERT_SWIGLU) {
      a = 1.0f / (1.0f + expf(-g));
      d = a * (1.0f - a);
    } else {
      a = gelu_t(g, d);
    }
    h = a * u;
    cg = u * d;
    cu = a;
  }
}



// d router_w = x^T dlogits, a D x E output reduced over all N rows.  Row
// group c (one workgroup) produces part[c][d][e]; its 4 waves take 4
// consecutive quarters of the group's rows, each summing fmaf(x[n][d],
// dlogits[n][e], .) over its rows ascending, and the workgroup adds the
// waves' sums in wave order through LDS.  The work is a stream of x (N x D)
// against a few FMAs per element, so the kernel is built to keep loads in
// flight: 8 consecutive d per lane (one 16-byte bf16 or two 16-byte fp32
// loads per row), JT experts per wave (dlogits rows by scalar loads), 16
// (bf16) or 8 (fp32) rows' loads issued together before their FMAs.  Lanes
// past D store nothing; rows past a quarter reload its last row and add
// nothing; empty quarters add zeros.
template <typename TX, int JT>
__global__ __launch_bounds__(256) void router_wgrad_kernel(const TX* __restrict__ x, int D,
                                                           const float* __restrict__ dl, int E,
                                                           int rows, int rg,
                                                           float* __restrict__ part) {
  constexpr int DV = 8;                          // d per lane
  constexpr int RU = sizeof(TX) == 2 ? 16 : 8;   // rows in flight
  constexpr int W = DV * (int)sizeof(TX) / 16;   // 16-byte words per lane and row
  __shared__ float xch[DV * JT * 64];            // one wave's sums, [i][j][lane]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.y;
  const int e0 = blockIdx.z * JT;
  const int ne = min(JT, E - e0);
  const int d0 = blockIdx.x * (64 * DV) + lane * DV;
  const int rw = (rg + 3) / 4;
  const int g0 = c * rg, g1 = min(rows, g0 + rg);
  const int r0 = min(g1, g0 + wave * rw), r1 = min(g1, r0 + rw);
  // whole 16-byte words need the lane's 8 d inside the row and D % 8 == 0
  const bool vec = d0 + DV <= D && (D % DV) == 0;
  float acc[DV][JT];
#pragma unroll
  for (int i = 0; i < DV; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j) acc[i][j] = 0.0f;
  for (int n0 = r0; n0 < r1; n0 += RU) {
    uint4 raw[RU][W];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const TX* src = x + (size_t)min(n0 + u, r1 - 1) * D + d0;
      if (vec) {
#pragma unroll
        for (int q = 0; q < W; ++q) raw[u][q] = reinterpret_cast<const uint4*>(src)[q];
      } else {
        float f[DV];
#pragma unroll
        for (int i = 0; i < DV; ++i) f[i] = d0 + i < D ? ld_x(src + i) : 0.0f;
        if constexpr (sizeof(TX) == 4) {
          raw[u][0] = uint4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                            __float_as_uint(f[3])};
          raw[u][1] = uint4{__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]),
                            __float_as_uint(f[7])};
        } else {
          // bf16 values are exact in the high half of their fp32 words
          uint32_t wv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            wv[q] = (__float_as_uint(f[2 * q]) >> 16) | (__float_as_uint(f[2 * q + 1]) & 0xffff0000u);
          raw[u][0] = uint4{wv[0], wv[1], wv[2], wv[3]};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      if (n0 + u < r1) {
        float xv[DV];
        if constexpr (sizeof(TX) == 2) {
          const uint32_t ws[4] = {raw[u][0].x, raw[u][0].y, raw[u][0].z, raw[u][0].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            xv[2 * q] = mxm_u2f(ws[q] << 16);
            xv[2 * q + 1] = mxm_u2f(ws[q] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            xv[4 * q] = __uint_as_float(raw[u][q].x);
            xv[4 * q + 1] = __uint_as_float(raw[u][q].y);
            xv[4 * q + 2] = __uint_as_float(raw[u][q].z);
            xv[4 * q + 3] = __uint_as_float(raw[u][q].w);
          }
        }
        const float* dr = dl + (size_t)(n0 + u) * E + e0;
        float g[JT];
#pragma unroll
        for (int j = 0; j < JT; ++j) g[j] = (ne == JT || j < ne) ? dr[j] : 0.0f;
#pragma unroll
        for (int i = 0; i < DV; ++i)
#pragma unroll
          for (int j = 0; j < JT; ++j) acc[i][j] = __builtin_fmaf(xv[i], g[j], acc[i][j]);
      }
    }
  }
  // wave 0 adds the other waves' sums in wave order
  for (int w = 1; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int i = 0; i < DV; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) xch[(i * JT + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < DV; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) acc[i][j] = acc[i][j] + xch[(i * JT + j) * 64 + lane];
    }
    __syncthreads();
  }
  if (wave != 0) return;
#pragma unroll
  for (int i = 0; i < DV; ++i) {
    if (d0 + i < D) {
      float* o = part + ((size_t)c * D + d0 + i) * E + e0;
#pragma unroll
      for (int j = 0; j < JT; ++j)
        if (j < ne) o[j] = acc[i][j];
    }
  }
}

// out[q] = sum over the partials p of part[p][q], in a fixed order: thread
// group g (of 4) sums p = g, g + 4, ... ascending for 64 consecutive q, then
// out = ((s0 + s1) + s2) + s3.
__global__ __launch_bounds__(256) void wgrad_sum_kernel(const float* __restrict__ part, int np,
                                                        size_t n, float* __restrict__ out) {
  __shared__ float sg[4][64];
  const int g = threadIdx.x >> 6, l = threadIdx.x & 63;
  const size_t q = (size_t)blockIdx.x * 64 + l;
  float acc = 0.0f;
  if (q < n) {
    constexpr int U = 8;
    int p = g;
    for (; p + 4 * (U - 1) < np; p += 4 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = part[(size_t)(p + 4 * u) * n + q];
#pragma unroll
      for (int u = 0; u < U; ++u) acc = acc + v[u];
    }
    for (; p < np; p += 4) acc = acc + part[(size_t)p * n + q];
  }
  sg[g][l] = acc;
  __syncthreads();
  if (g == 0 && q < n) out[q] = ((sg[0][l] + sg[1][l]) + sg[2][l]) + sg[3][l];
}


void transpose_batch(const float* src, int batch, int R, int C, float* dst, hipStream_t s) {
  if (batch <= 0 || R <= 0 || C <= 0) return;
  hipLaunchKernelGGL(transpose_f32_kernel, dim3((C + 31) / 32, (R + 31) / 32, batch), dim3(32, 8),
                     0, s, src, R, C, dst);
}

void grouped(const float* A, const float* B, float* out, int Kd, int NC, const int32_t* offsets,
             const int32_t* mstart, int E, int max_mtiles, hipStream_t s) {
  GemmArgs g{};
  g.mode = MXM_GEMM_DOWN;
  g.a = A;
  g.b0 = B;
  g.out = out;
  g.offsets = offsets;
  g.mstart = mstart;
  g.E = E;
  g.Kd = Kd;
  g.Ncols = NC;
  g.max_mtiles = max_mtiles;
  g.y_bf16 = false;
  mxm_launch_gemm_simt(g, false, s);
}

// ---- bf16 flow on the MFMA family --------------------------------------------

// One thread per 8 columns of a row of out [N][2 Ep]: hi = bf16(dl) at
// columns e, lo = bf16(dl - hi) at Ep + e (dl - hi is exact in fp32), zeros
// past E.  hi + lo carries dl to about 2^-16 relative.
__global__ void dl_split_kernel(const float* __restrict__ dl, int E, int Ep,
                                uint16_t* __restrict__ out, size_t total) {
  const int nb = Ep / 8;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t n = i / nb;
    const int e0 = (int)(i % nb) * 8;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float h2[2], l2[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = e0 + 2 * q + r;
        const float v = e < E ? dl[n * E + e] : 0.0f;
        h2[r] = mxm_rbf_fast(v);
        l2[r] = v - h2[r];
      }
      hw[q] = mxm_pack_bf2_fast(h2[0], h2[1]);
      lw[q] = mxm_pack_bf2_fast(l2[0], l2[1]);
    }
    uint16_t* row = out + n * 2 * Ep;
    *reinterpret_cast<uint4*>(row + e0) = uint4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<uint4*>(row + Ep + e0) = uint4{lw[0], lw[1], lw[2], lw[3]};
  }
}

// dwr[d][e] = t[d][e] + t[d][Ep + e]: x^T hi plus x^T lo.
__global__ void dwr_halves_kernel(const float* __restrict__ t, int E, int Ep,
                                  float* __restrict__ dwr, size_t total) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t d = i / E;
    const int e = (int)(i % E);
    dwr[i] = t[d * 2 * Ep + e] + t[d * 2 * Ep + Ep + e];
  }
}

// dx[n] = dlogits[n] . Wr^T + sum_k dXe[slot_pos(n, k)], k ascending: the
// router's input gradient (e ascending, fmaf) fused with the sum over the
// token's slots.  A workgroup takes TT tokens; a thread 4 consecutive d of
// each 4 * blockDim.x wide block (Wr^T rows [E][D] as float4, shared by the
// TT tokens).  D % 4 == 0.  The workgroup's dlogits rows are staged in LDS
// once; Wr^T is read 4 experts at a time, one group ahead; the token's KK
// slot rows are requested together, token t+1's while token t's are summed,
// so a thread keeps up to 2 KK row loads in flight.  Every global load here
// is unconditional (the workgroup's tokens all exist, K = KK, the last
// group's Wr^T rows are clamped and their FMAs skipped): the compiler's
// wait counts are then exact instead of draining everything in flight.
// Tokens n_first + blockIdx.x * TT + (0 .. TT-1).
template <int TT, int KK>
__global__ __launch_bounds__(256) void dx_fused_bf16_kernel(const float* __restrict__ dlogits,
                                                            const float* __restrict__ wrt, int E,
                                                            const uint16_t* __restrict__ dxe,
                                                            const int32_t* __restrict__ slot_pos,
                                                            int n_first, int D,
                                                            float* __restrict__ dx) {
  __shared__ __attribute__((aligned(16))) float sdl[TT * MXM_MAX_EXPERTS];
  const int n0 = n_first + blockIdx.x * TT;
  const int E4 = (E + 3) & ~3;  // LDS row stride: 16-byte aligned rows
  for (int i = threadIdx.x; i < TT * E4; i += blockDim.x) {
    const int t = i / E4, e = i % E4;
    sdl[i] = e < E ? dlogits[(size_t)(n0 + t) * E + e] : 0.0f;
  }
  __syncthreads();
  for (int d = threadIdx.x * 4; d < D; d += blockDim.x * 4) {
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[t][q] = 0.0f;
    float4 wa[4], wb[4];
    auto wload = [&](int e0, float4* w) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = *reinterpret_cast<const float4*>(wrt + (size_t)min(e0 + j, E - 1) * D + d);
    };
    auto wfma = [&](int e0, const float4* w, auto full) {
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const float4 l = *reinterpret_cast<const float4*>(sdl + t * E4 + e0);
        const float lj[4] = {l.x, l.y, l.z, l.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!decltype(full)::value && e0 + j >= E) break;
          acc[t][0] = __builtin_fmaf(lj[j], w[j].x, acc[t][0]);
          acc[t][1] = __builtin_fmaf(lj[j], w[j].y, acc[t][1]);
          acc[t][2] = __builtin_fmaf(lj[j], w[j].z, acc[t][2]);
          acc[t][3] = __builtin_fmaf(lj[j], w[j].w, acc[t][3]);
        }
      }
    };
    // whole groups of 4 experts, the next group requested before the
    // current one's FMAs (a clamped group past the end is harmless), then
    // the E % 4 experts left
    const std::true_type full;
    const int EF = E & ~3;
    if (EF > 0) wload(0, wa);
    for (int e0 = 0; e0 < EF; e0 += 8) {
      wload(e0 + 4, wb);
      __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the FMAs
      wfma(e0, wa, full);
      if (e0 + 4 >= EF) break;
      wload(e0 + 8, wa);
      __builtin_amdgcn_sched_barrier(0);
      wfma(e0 + 4, wb, full);
    }
    if (EF < E) {
      wload(EF, wa);
      wfma(EF, wa, std::false_type{});
    }

    uint2 v[2][KK];
    auto issue = [&](int t, uint2* vv) {
      const int32_t* sp = slot_pos + (size_t)(n0 + t) * KK;
#pragma unroll
      for (int k = 0; k < KK; ++k)
        vv[k] = *reinterpret_cast<const uint2*>(dxe + (size_t)sp[k] * D + d);
    };
    issue(0, v[0]);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t + 1 < TT) issue(t + 1, v[(t + 1) & 1]);
#pragma unroll
      for (int k = 0; k < KK; ++k) {
        const uint2 x = v[t & 1][k];
        acc[t][0] = acc[t][0] + mxm_u2f(x.x << 16);
        acc[t][1] = acc[t][1] + mxm_u2f(x.x & 0xffff0000u);
        acc[t][2] = acc[t][2] + mxm_u2f(x.y << 16);
        acc[t][3] = acc[t][3] + mxm_u2f(x.y & 0xffff0000u);
      }
      *reinterpret_cast<float4*>(dx + (size_t)(n0 + t) * D + d) =
          float4{acc[t][0], acc[t][1], acc[t][2], acc[t][3]};
    }
  }
}

// The same sum, one token per workgroup, any K: the tokens a whole group of
// TT does not cover, and K > 8.  Tokens n_first + blockIdx.x.
__global__ __launch_bounds__(256) void dx_fused_one_bf16_kernel(
    const float* __restrict__ dlogits, const float* __restrict__ wrt, int E,
    const uint16_t* __restrict__ dxe, const int32_t* __restrict__ slot_pos, int n_first, int D,
    int K, float* __restrict__ dx) {
  const int n = n_first + blockIdx.x;
  for (int d = threadIdx.x * 4; d < D; d += blockDim.x * 4) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (int e = 0; e < E; ++e) {
      const float4 w = *reinterpret_cast<const float4*>(wrt + (size_t)e * D + d);
      const float l = dlogits[(size_t)n * E + e];
      a0 = __builtin_fmaf(l, w.x, a0);
      a1 = __builtin_fmaf(l, w.y, a1);
      a2 = __builtin_fmaf(l, w.z, a2);
      a3 = __builtin_fmaf(l, w.w, a3);
    }
    for (int k = 0; k < K; ++k) {
      const uint2 x =
          *reinterpret_cast<const uint2*>(dxe + (size_t)slot_pos[(size_t)n * K + k] * D + d);
      a0 = a0 + mxm_u2f(x.x << 16);
      a1 = a1 + mxm_u2f(x.x & 0xffff0000u);
      a2 = a2 + mxm_u2f(x.y << 16);
      a3 = a3 + mxm_u2f(x.y & 0xffff0000u);
    }
    *reinterpret_cast<float4*>(dx + (size_t)n * D + d) = float4{a0, a1, a2, a3};
  }
}

// dG and dU of one hidden unit from its gate and up projections g, u and dH
// (fp32; GLU: dG and dU, MLP: dU only).
__device__ __forceinline__ void act_bw_one(int etype, int act, float slope, float g, float u,
                                           float dh, float& dg, float& du) {
  if (etype == MXM_EXPERT_MLP) {
    float d;
    switch (act) {
      case MXM_ACT_SILU: {
        const float sg = 1.0f / (1.0f + expf(-u));
        d = sg * (1.0f + u * (1.0f - sg));
        break;
      }
      case MXM_ACT_GELU:
        (void)gelu_t(u, d);
        break;
      case MXM_ACT_RELU:
        d = u > 0.0f ? 1.0f : 0.0f;
        break;
      default: {
        const float y = u > 0.0f ? u : u * slope;
        d = 2.0f * y * (u > 0.0f ? 1.0f : slope);
        break;
      }
    }
    dg = 0.0f;
    du = dh * d;
  } else {
    float a, d;
    if (etype == MXM_EXPERT_SWIGLU) {
      a = 1.0f / (1.0f + expf(-g));
      d = a * (1.0f - a);
    } else {
      a = gelu_t(g, d);
    }
    dg = dh * u * d;
    du = dh * a;
  }
}

// One workgroup per token n: ddb[n] = bf16(dD[n]); for each slot s = n*K + k
// at position p = slot_pos[s]: gp[p] = gates[s] and, if dyb is set, dyb[p] =
// bf16(gates[s] * dD[n]).  V = 4: 4 consecutive d per thread (16-byte dD
// loads, 8-byte stores).
template <int V>
__global__ __launch_bounds__(256) void dy_gate_kernel(const float* __restrict__ dd,
                                                      const float* __restrict__ gates,
                                                      const int32_t* __restrict__ slot_pos, int D,
                                                      int K, uint16_t* __restrict__ ddb,
                                                      uint16_t* __restrict__ dyb,
                                                      float* __restrict__ gp) {
  const int n = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const float* src = dd + (size_t)n * D;
  for (int k = tid; k < K; k += nt) gp[slot_pos[(size_t)n * K + k]] = gates[(size_t)n * K + k];
  for (int d = tid * V; d < D; d += nt * V) {
    float v[V];
    if constexpr (V == 4) {
      const float4 t = *reinterpret_cast<const float4*>(src + d);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
      *reinterpret_cast<uint2*>(ddb + (size_t)n * D + d) =
          uint2{(uint32_t)mxm_f2bf(v[0]) | (uint32_t)mxm_f2bf(v[1]) << 16,
                (uint32_t)mxm_f2bf(v[2]) | (uint32_t)mxm_f2bf(v[3]) << 16};
    } else {
      v[0] = src[d];
      ddb[(size_t)n * D + d] = mxm_f2bf(v[0]);
    }
    for (int k = 0; k < K && dyb; ++k) {
      const float g = gates[(size_t)n * K + k];
      uint16_t* o = dyb + (size_t)slot_pos[(size_t)n * K + k] * D + d;
      if constexpr (V == 4)
        *reinterpret_cast<uint2*>(o) =
            uint2{(uint32_t)mxm_f2bf(g * v[0]) | (uint32_t)mxm_f2bf(g * v[1]) << 16,
                  (uint32_t)mxm_f2bf(g * v[2]) | (uint32_t)mxm_f2bf(g * v[3]) << 16};
      else
        *o = mxm_f2bf(g * v[0]);
    }
  }
}

// One wave per routed row p (4 rows per workgroup), 8 hidden units per lane
// and step, from the forward's raw bf16 projections gu [N*K, NC] (GLU: NC =
// 2F, gate and up columns interleaved in groups of 32 as the MFMA family's W1
// rows; MLP: NC = F, up only): the hidden h = mxm_hidden_fast of them, as the
// up GEMM's epilogue computes it; the gated hidden gp[p] * h stored to Hg in
// bf16 (two planes hi and lo = bf16(v - hi) for a split hidden), dW_down's
// left operand; dH = gp[p] * dhr (dhr = dD W_down^T for the row's token, not
// yet gated); dG and dU from dH, written to dgu at the columns of g and u in
// bf16; and the gate gradient dgp[p] = <dhr[p], h[p]> with h as the forward
// stores it (bf16, or hi + lo when split), summed per lane in f order and
// then over the wave by a fixed butterfly.
__global__ __launch_bounds__(256) void act_bw_gated_bf16_kernel(
    const uint16_t* __restrict__ gu, const uint16_t* __restrict__ dhr,
    uint16_t* __restrict__ Hg, bool hsplit, const float* __restrict__ gp, int rows, int F,
    int etype, int act, float slope, uint16_t* __restrict__ dgu, float* __restrict__ dgp) {
  const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (p >= rows) return;  // (the whole wave)
  const bool glu = etype != MXM_EXPERT_MLP;
  const int NC = glu ? 2 * F : F;
  const float gate = gp[p];
  float dot = 0.0f;
  const size_t hstride = hsplit ? 2 * (size_t)F : (size_t)F;
  // U steps of 8 hidden units per lane: their loads go out together
  constexpr int U = 4;
  for (int f0 = lane * 8; f0 < F; f0 += 512 * U) {
    uint4 hv[U], uv[U], gv[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int f = min(f0 + 512 * j, F - 8);  // (steps past F reload the last group)
      const size_t cu = (size_t)p * NC + (glu ? (size_t)(f >> 5) * 64 + 32 + (f & 31) : (size_t)f);
      hv[j] = *reinterpret_cast<const uint4*>(dhr + (size_t)p * F + f);
      uv[j] = *reinterpret_cast<const uint4*>(gu + cu);
      gv[j] = glu ? *reinterpret_cast<const uint4*>(gu + cu - 32) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int f = f0 + 512 * j;
      if (f >= F) break;
      const size_t cu = (size_t)p * NC + (glu ? (size_t)(f >> 5) * 64 + 32 + (f & 31) : (size_t)f);
      const uint32_t hw[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
      const uint32_t uw[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
      const uint32_t gw[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
      uint32_t og[4], ou[4], xw[4], lw[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float r0 = mxm_u2f(hw[q] << 16), r1 = mxm_u2f(hw[q] & 0xffff0000u);
        // the hidden as the up epilogue computes it (mxm_hidden_fast on the
        // bf16 projections), then as stored
        // (sigmoid-GLU: the one fast sigmoid serves h and the derivative)
        const bool sw = etype == MXM_EXPERT_SWIGLU;
        float h[2], sg[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const float gg = glu ? mxm_u2f(t ? gw[q] & 0xffff0000u : gw[q] << 16) : 0.0f;
          const float uu = mxm_u2f(t ? uw[q] & 0xffff0000u : uw[q] << 16);
          if (sw) {
            sg[t] = mxm_sigmoid_fast(gg);
            h[t] = mxm_rbf_fast(mxm_rbf_fast(sg[t]) * uu);  // as mxm_hidden_fast
          } else {
            h[t] = mxm_hidden_fast<true>(glu ? etype : MXM_EXPERT_MLP, act, slope, gg, uu);
          }
        }
        // h as the forward stores it, for the gate gradient
        float h0 = mxm_rbf_fast(h[0]), h1 = mxm_rbf_fast(h[1]);
        if (hsplit) {
          h0 = h0 + mxm_rbf_fast(h[0] - h0);
          h1 = h1 + mxm_rbf_fast(h[1] - h1);
        }
        dot = __builtin_fmaf(r0, h0, dot);
        dot = __builtin_fmaf(r1, h1, dot);
        // the gated hidden
        const float v0 = gate * h[0], v1 = gate * h[1];
        xw[q] = mxm_pack_bf2_fast(v0, v1);
        if (hsplit)
          lw[q] = mxm_pack_bf2_fast(v0 - mxm_u2f(xw[q] << 16), v1 - mxm_u2f(xw[q] & 0xffff0000u));
        float dg0, du0, dg1, du1;
        if (sw) {
          const float u0 = mxm_u2f(uw[q] << 16), u1 = mxm_u2f(uw[q] & 0xffff0000u);
          const float d0 = gate * r0, d1 = gate * r1;
          dg0 = d0 * u0 * (sg[0] * (1.0f - sg[0]));
          du0 = d0 * sg[0];
          dg1 = d1 * u1 * (sg[1] * (1.0f - sg[1]));
          du1 = d1 * sg[1];
        } else {
          act_bw_one(etype, act, slope, mxm_u2f(gw[q] << 16), mxm_u2f(uw[q] << 16), gate * r0,
                     dg0, du0);
          act_bw_one(etype, act, slope, mxm_u2f(gw[q] & 0xffff0000u),
                     mxm_u2f(uw[q] & 0xffff0000u), gate * r1, dg1, du1);
        }
        og[q] = (uint32_t)mxm_f2bf(dg0) | ((uint32_t)mxm_f2bf(dg1) << 16);
        ou[q] = (uint32_t)mxm_f2bf(du0) | ((uint32_t)mxm_f2bf(du1) << 16);
      }
      *reinterpret_cast<uint4*>(dgu + cu) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
      if (glu) *reinterpret_cast<uint4*>(dgu + cu - 32) = make_uint4(og[0], og[1], og[2], og[3]);
      *reinterpret_cast<uint4*>(Hg + (size_t)p * hstride + f) = make_uint4(xw[0], xw[1], xw[2], xw[3]);
      if (hsplit)
        *reinterpret_cast<uint4*>(Hg + (size_t)p * hstride + F + f) =
            make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) dot = dot + mxm_xor_lane_f(dot, m);
  if (lane == 0) dgp[p] = dot;
}

// One thread per 8 hidden units of a routed row: h = mxm_hidden_fast of the
// raw bf16 projections (GLU: gate and up columns interleaved in groups of
// 32), stored as the up GEMM's epilogue stores it.
__global__ void hidden_from_raw_bf16_kernel(const uint16_t* __restrict__ gu, int F, int etype,
                                            int act, float slope, bool hsplit,
                                            uint16_t* __restrict__ H, size_t total) {
  const bool glu = etype != MXM_EXPERT_MLP;
  const int NC = glu ? 2 * F : F, nb = F / 8;
  const size_t hstride = hsplit ? 2 * (size_t)F : (size_t)F;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t p = i / nb;
    const int f = (int)(i % nb) * 8;
    const size_t cu = p * NC + (glu ? (size_t)(f >> 5) * 64 + 32 + (f & 31) : (size_t)f);
    const uint4 uv = *reinterpret_cast<const uint4*>(gu + cu);
    const uint4 gv = glu ? *reinterpret_cast<const uint4*>(gu + cu - 32) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float h[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float gg = glu ? mxm_u2f(t ? gw[q] & 0xffff0000u : gw[q] << 16) : 0.0f;
        const float uu = mxm_u2f(t ? uw[q] & 0xffff0000u : uw[q] << 16);
        h[t] = mxm_hidden_fast<true>(glu ? etype : MXM_EXPERT_MLP, act, slope, gg, uu);
      }
      hw[q] = mxm_pack_bf2_fast(h[0], h[1]);
      lw[q] = mxm_pack_bf2_fast(h[0] - mxm_u2f(hw[q] << 16), h[1] - mxm_u2f(hw[q] & 0xffff0000u));
    }
    *reinterpret_cast<uint4*>(H + p * hstride + f) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    if (hsplit)
      *reinterpret_cast<uint4*>(H + p * hstride + F + f) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
}

// dx[n] = dxr[n] + sum_k dxe[slot_pos(n, k)] (bf16 rows), k ascending
__global__ void dx_bf16_kernel(const float* __restrict__ dxr, const uint16_t* __restrict__ dxe,
                               const int32_t* __restrict__ slot_pos, int D, int K,
                               float* __restrict__ dx) {
  const int n = blockIdx.x;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = dxr[(size_t)n * D + d];
    for (int k = 0; k < K; ++k)
      acc = acc + mxm_bf2f(dxe[(size_t)slot_pos[(size_t)n * K + k] * D + d]);
    dx[(size_t)n * D + d] = acc;
  }
}

// Threads for a row of D elements taken V at a time: whole waves, at most 256.
int block_for(int D, int V) {
  const int t = (D + V - 1) / V;
  return std::min(256, std::max(64, (t + 63) / 64 * 64));
}

int grid_of(size_t n) {
  size_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

// Row groups of the router's weight gradient (one partial each): at least
// 64 rows each, at most 256 groups and 8 M partial floats in all.
int wgrad_router_chunks_impl(int N, int D, int E) {
  long long c = ((long long)N + 63) / 64;
  const long long budget = (8LL << 20) / std::max(1LL, (long long)D * E);
  c = std::max(1LL, std::min(c, std::min(256LL, budget)));
  return (int)c;
}

// Row-tile prefix of a grouped GEMM family with tile height bm:
// mstart[e] = sum over e' < e of ceil(counts[e'] / bm), e = 0..E.
__global__ void tile_prefix_kernel(const int32_t* counts, int E, int bm, int32_t* mstart) {
  if (threadIdx.x != 0) return;
  int m = 0;
  for (int e = 0; e < E; ++e) {
    mstart[e] = m;
    m += (counts[e] + bm - 1) / bm;
  }
  mstart[E] = m;
}


// ---- the fp32 backward's products on the bf16 MFMA kernels ----
// An fp32 value v is carried as two bf16 planes, hi = bf16(v) and lo =
// bf16(v - hi) (|v - hi - lo| <= 2^-18 |v|), and an fp32 product A . B as
// the bf16 product of the k-concatenated planes [a0 | a1 | a2] . [b0 | b1 |
// b2] with (a, b) = (hi, hi), (hi, lo), (lo, hi): A . B to within about
// 3 * 2^-18 relative per term (the lo . lo term, below 2^-18, is dropped),
// accumulated in fp32 by the MFMA.  Operands that pair with A-side planes
// are laid out HHL = [hi | hi | lo], those on the B side HLH = [hi | lo | hi].

__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = mxm_f2bf(v);
  lo = mxm_f2bf(v - mxm_bf2f(hi));
}

// dst[r][p * ldq + c] = plane p (order hlh: HLH, else HHL) of src[r][c] for
// c < cols, 0 for cols <= c < ldq.
__global__ void planes3_kernel(const float* __restrict__ src, int64_t rows, int cols, int lds,
                               int ldq, int hlh, uint16_t* __restrict__ dst) {
  const int64_t n = rows * ldq;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ldq;
    const int c = (int)(i - r * ldq);
    uint16_t hi = 0, lo = 0;
    if (c < cols) split_bf16(src[(size_t)r * lds + c], hi, lo);
    uint16_t* d = dst + (size_t)r * 3 * ldq + c;
    d[0] = hi;
    d[ldq] = hlh ? lo : hi;
    d[2 * ldq] = hlh ? hi : lo;
  }
}

// One fp32 expert matrix of the x.W layout in the planes of an MFMA B
// operand [R][3 Kq] bf16 per expert: dst[e][r][p * Kq + k] = plane p of the
// source value at (r, k), 0 past the real extent.  For the up projections
// (gate, up: src0, src1 [D][F]) or the down one (src0 [F][D]); the row or the
// k index may be a GLU-interleaved column (groups of 32 gate then 32 up).
struct Planes3W {
  const float* src0;
  const float* src1;    // the up matrix of a GLU pair (interleaved index), else null
  int E, R, Kq;         // rows and padded k per expert
  int r_lim, k_lim;     // real extent of the decoded row and k indices
  int glu_r, glu_k;     // the row / k index is GLU-interleaved
  int64_t sr, sk;       // source strides of the decoded row and k indices
  int64_t es;           // source stride between experts
  int hlh;
  uint16_t* dst;
};

__global__ void planes3_w_kernel(Planes3W a) {
  const int64_t per = (int64_t)a.R * a.Kq;
  const int64_t n = (int64_t)a.E * per;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = (int)(i / per);
    const int64_t rk = i - (int64_t)e * per;
    const int r = (int)(rk / a.Kq), k = (int)(rk - (int64_t)r * a.Kq);
    int slot = 0, rr = r, kk = k;
    if (a.glu_r) {
      slot = (r >> 5) & 1;
      rr = (r >> 6) * 32 + (r & 31);
    }
    if (a.glu_k) {
      slot = (k >> 5) & 1;
      kk = (k >> 6) * 32 + (k & 31);
    }
    uint16_t hi = 0, lo = 0;
    if (rr < a.r_lim && kk < a.k_lim) {
      const float* src = slot ? a.src1 : a.src0;
      split_bf16(src[(size_t)e * a.es + (size_t)rr * a.sr + (size_t)kk * a.sk], hi, lo);
    }
    uint16_t* d = a.dst + ((size_t)e * a.R + r) * 3 * a.Kq + k;
    d[0] = hi;
    d[a.Kq] = a.hlh ? lo : hi;
    d[2 * (size_t)a.Kq] = a.hlh ? hi : lo;
  }
}

// The hidden units of the raw projections gu [rows][NC] fp32 (GLU: gate and
// up interleaved in groups of 32; NC = 2 Fq, else Fq), as the HHL planes of
// H [rows][3 Fq].
__global__ void hidden_planes3_kernel(const float* __restrict__ gu, int64_t rows, int Fq, int etype,
                                      int act, float slope, uint16_t* __restrict__ h3) {
  const bool glu = etype != MXM_EXPERT_MLP;
  const int NC = glu ? 2 * Fq : Fq;
  const int64_t n = rows * Fq;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / Fq;
    const int f = (int)(i - r * Fq);
    const float* row = gu + (size_t)r * NC;
    const int qg = (f >> 5) * 64 + (f & 31);
    const float g = glu ? row[qg] : 0.0f, u = glu ? row[qg + 32] : row[f];
    float h, cg, cu;
    act_eval(etype, act, slope, g, u, h, cg, cu);
    uint16_t hi, lo;
    split_bf16(h, hi, lo);
    uint16_t* d = h3 + (size_t)r * 3 * Fq + f;
    d[0] = hi;
    d[Fq] = hi;
    d[2 * (size_t)Fq] = lo;
  }
}

// The activation backward: from gu (as above) and dh [rows][Fq] fp32, dG and
// dU as the HLH planes of dGU [rows][3 NC] in gu's column order.
__global__ void act_bw_planes3_kernel(const float* __restrict__ gu, const float* __restrict__ dh,
                                      int64_t rows, int Fq, int etype, int act, float slope,
                                      uint16_t* __restrict__ dgu3) {
  const bool glu = etype != MXM_EXPERT_MLP;
  const int NC = glu ? 2 * Fq : Fq;
  const int64_t n = rows * Fq;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / Fq;
    const int f = (int)(i - r * Fq);
    const float* row = gu + (size_t)r * NC;
    const int qg = (f >> 5) * 64 + (f & 31);
    const float g = glu ? row[qg] : 0.0f, u = glu ? row[qg + 32] : row[f];
    float h, cg, cu;
    act_eval(etype, act, slope, g, u, h, cg, cu);
    const float d = dh[(size_t)r * Fq + f];
    uint16_t* base = dgu3 + (size_t)r * 3 * NC;
    auto put = [&](int q, float v) {
      uint16_t hi, lo;
      split_bf16(v, hi, lo);
      base[q] = hi;
      base[NC + q] = lo;
      base[2 * NC + q] = hi;
    };
    if (glu) {
      put(qg, d * cg);
      put(qg + 32, d * cu);
    } else {
      put(f, d * cu);
    }
  }
}

// dx[n] = dxr[n] + sum_k dxe[slot_pos[n, k]] (k ascending; dxe rows ld apart).
__global__ void dx_sum_kernel(const float* __restrict__ dxr, const float* __restrict__ dxe, int ld,
                              const int32_t* __restrict__ slot_pos, int D, int K,
                              float* __restrict__ dx) {
  const int n = blockIdx.x;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = dxr[(size_t)n * D + d];
    for (int k = 0; k < K; ++k) acc = acc + dxe[(size_t)slot_pos[(size_t)n * K + k] * ld + d];
    dx[(size_t)n * D + d] = acc;
  }
}

}  // namespace

int wgrad_router_chunks(int N, int D, int E) { return wgrad_router_chunks_impl(N, D, E); }

void mxm_launch_tile_prefix(const int32_t* counts, int E, int bm, int32_t* mstart, hipStream_t s) {
  hipLaunchKernelGGL(tile_prefix_kernel, dim3(1), dim3(64), 0, s, counts, E, bm, mstart);
}

void mxm_launch_dx_fused_bf16(const float* dlogits, const float* wrt, int E, const uint16_t* dxe,
                              const int32_t* slot_pos, int N, int D, int K, float* dx,
                              hipStream_t s) {
  // tokens per workgroup: each float4 of Wr^T is read once per workgroup
  // from L2, so wide routers want more tokens to share it
  if (N <= 0) return;
  const dim3 blk(block_for(D, 4));
  int done = 0;
  auto groups = [&](auto tt, auto kk) {
    constexpr int TT = decltype(tt)::value, KK = decltype(kk)::value;
    const int g = N / TT;
    if (g > 0)
      hipLaunchKernelGGL((dx_fused_bf16_kernel<TT, KK>), dim3(g), blk, 0, s, dlogits, wrt, E, dxe,
                         slot_pos, 0, D, dx);
    done = g * TT;
  };
  auto by_k = [&](auto tt) {
    switch (K) {
      case 1: groups(tt, std::integral_constant<int, 1>{}); break;
      case 2: groups(tt, std::integral_constant<int, 2>{}); break;
      case 3: groups(tt, std::integral_constant<int, 3>{}); break;
      case 4: groups(tt, std::integral_constant<int, 4>{}); break;
      case 5: groups(tt, std::integral_constant<int, 5>{}); break;
      case 6: groups(tt, std::integral_constant<int, 6>{}); break;
      case 7: groups(tt, std::integral_constant<int, 7>{}); break;
      case 8: groups(tt, std::integral_constant<int, 8>{}); break;
      default: break;  // K > 8: every token below
    }
  };
  if (E > 16) by_k(std::integral_constant<int, 16>{});
  else by_k(std::integral_constant<int, 4>{});
  if (done < N)
    hipLaunchKernelGGL(dx_fused_one_bf16_kernel, dim3(N - done), blk, 0, s, dlogits, wrt, E, dxe,
                       slot_pos, done, D, K, dx);
}

void mxm_launch_dl_split_bf16(const float* dl, int N, int E, int Ep, uint16_t* out, hipStream_t s) {
  const size_t total = (size_t)N * (Ep / 8);
  if (total > 0)
    hipLaunchKernelGGL(dl_split_kernel, dim3(grid_of(total)), dim3(256), 0, s, dl, E, Ep, out,
                       total);
}

void mxm_launch_dwr_halves(const float* t, int D, int E, int Ep, float* dwr, hipStream_t s) {
  const size_t total = (size_t)D * E;
  if (total > 0)
    hipLaunchKernelGGL(dwr_halves_kernel, dim3(grid_of(total)), dim3(256), 0, s, t, E, Ep, dwr,
                       total);
}

void mxm_launch_dy_gate(const float* dd, const float* gates, const int32_t* slot_pos, int N, int D,
                        int K, uint16_t* ddb, uint16_t* dyb, float* gp, hipStream_t s) {
  if (N <= 0) return;
  const bool vec = D % 4 == 0 && reinterpret_cast<uintptr_t>(dd) % 16 == 0;
  if (vec)
    hipLaunchKernelGGL(dy_gate_kernel<4>, dim3(N), dim3(block_for(D, 4)), 0, s, dd, gates,
                       slot_pos, D, K, ddb, dyb, gp);
  else
    hipLaunchKernelGGL(dy_gate_kernel<1>, dim3(N), dim3(block_for(D, 1)), 0, s, dd, gates,
                       slot_pos, D, K, ddb, dyb, gp);
}

void mxm_launch_hidden_from_raw_bf16(const uint16_t* gu, int rows, int F, int etype, int act,
                                     float slope, bool hsplit, uint16_t* H, hipStream_t s) {
  const size_t total = (size_t)rows * (F / 8);
  if (total > 0)
    hipLaunchKernelGGL(hidden_from_raw_bf16_kernel, dim3(grid_of(total)), dim3(256), 0, s, gu, F,
                       etype, act, slope, hsplit, H, total);
}

void mxm_launch_act_bw_gated_bf16(const uint16_t* gu, const uint16_t* dhr, uint16_t* Hg,
                                  bool hsplit, const float* gp, int rows, int F, int etype, int act,
                                  float slope, uint16_t* dgu, float* dgp, hipStream_t s) {
  // F is a multiple of 32 (the MFMA family's GLU interleave)
  if (rows > 0)
    hipLaunchKernelGGL(act_bw_gated_bf16_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, gu, dhr,
                       Hg, hsplit, gp, rows, F, etype, act, slope, dgu, dgp);
}

void mxm_launch_dx_bf16(const float* dxr, const uint16_t* dxe, const int32_t* slot_pos, int N,
                        int D, int K, float* dx, hipStream_t s) {
  if (N > 0) hipLaunchKernelGGL(dx_bf16_kernel, dim3(N), dim3(256), 0, s, dxr, dxe, slot_pos, D, K, dx);
}

// Gate, renorm, aux / entropy and softmax gradients, the router's products
// (dx's router term dxr, d router_w) and dY = gate * dD.
void mxm_launch_backward_router(const BackwardArgs& a, hipStream_t s) {
  const int N = a.N, D = a.D, E = a.E, K = a.K, NK = a.N * a.K;
  if (NK <= 0) return;
  transpose_batch(a.wr, 1, D, E, a.wrt, s);  // [E][D]
  const auto al = [](const void* p, int b) { return reinterpret_cast<uintptr_t>(p) % b == 0; };
  const bool vec = D % 4 == 0 && al(a.d_delta, 16) &&
                   (a.Yb16 ? al(a.Yb16, 8) : al(a.Y, 16)) &&
                   (a.dyb16 ? al(a.dyb16, 8) : al(a.dy, 16));
  if (!a.dgp) {  // (else the caller computed the gate gradients and dY)
    if (vec)
      hipLaunchKernelGGL(dgates_dy_kernel<4>, dim3(N), dim3(block_for(D, 4)), 0, s, a);
    else
      hipLaunchKernelGGL(dgates_dy_kernel<1>, dim3(N), dim3(block_for(D, 1)), 0, s, a);
  }
  hipLaunchKernelGGL(router_bw_kernel, dim3((N + 3) / 4), dim3(256), 0, s, a);
  // dx's router term; fused into the dx sum by the caller when dxr is unset
  if (a.dxr) grouped(a.dlogits, a.wrt, a.dxr, E, D, a.one, a.one + 2, 1, (N + 63) / 64, s);
  if (a.dwr_by_caller) return;
  // router: d router_w = x^T dlogits over all N rows -- a D x E output, so
  // the rows are split in chunks (fixed chunk order, rows ascending within a
  // chunk) to spread the reduction over the GPU
  const int nch = wgrad_router_chunks(N, D, E);
  const int rg = (N + nch - 1) / nch;
  const int dblk = (D + 511) / 512;
  if (E <= 8) {
    const dim3 wg(dblk, nch, 1);
    if (a.xb16)
      hipLaunchKernelGGL((router_wgrad_kernel<uint16_t, 8>), wg, dim3(256), 0, s, a.xb16, D,
                         a.dlogits, E, N, rg, a.wr_part);
    else
      hipLaunchKernelGGL((router_wgrad_kernel<float, 8>), wg, dim3(256), 0, s, a.x, D, a.dlogits,
                         E, N, rg, a.wr_part);
  } else {
    const dim3 wg(dblk, nch, (E + 15) / 16);
    if (a.xb16)
      hipLaunchKernelGGL((router_wgrad_kernel<uint16_t, 16>), wg, dim3(256), 0, s, a.xb16, D,
                         a.dlogits, E, N, rg, a.wr_part);
    else
      hipLaunchKernelGGL((router_wgrad_kernel<float, 16>), wg, dim3(256), 0, s, a.x, D, a.dlogits,
                         E, N, rg, a.wr_part);
  }
  const size_t n = (size_t)D * E;
  hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, s, a.wr_part,
                     nch, n, a.dwr);
  (void)K;
}

// The fp32 backward's operand planes and elementwise parts; its products run
// on the MFMA grouped GEMM and weight-gradient kernels over bf16 planes
// (three plane pairs per fp32 product, fp32 accumulation).
void mxm_launch_planes3(const float* src, int64_t rows, int cols, int lds, int ldq, bool hlh,
                        uint16_t* dst, hipStream_t s) {
  const int64_t n = rows * ldq;
  if (n > 0)
    hipLaunchKernelGGL(planes3_kernel, dim3(grid_of((size_t)n)), dim3(256), 0, s, src, rows, cols,
                       lds, ldq, hlh ? 1 : 0, dst);
}

void mxm_launch_planes3_weights(const float* w1, const float* w1b, const float* w2, int E, int D,
                                int F, int Dq, int Fq, bool glu, uint16_t* w1p, uint16_t* w1t,
                                uint16_t* w2p, uint16_t* w2t, hipStream_t s) {
  const int NCq = glu ? 2 * Fq : Fq;
  const int64_t DF = (int64_t)D * F;
  auto go = [&](Planes3W a) {
    const int64_t n = (int64_t)a.E * a.R * a.Kq;
    if (n > 0) hipLaunchKernelGGL(planes3_w_kernel, dim3(grid_of((size_t)n)), dim3(256), 0, s, a);
  };
  // up projections: B of G|U = X W1 is [NCq][3 Dq] HLH (row = column of W1)
  go(Planes3W{w1, glu ? w1b : nullptr, E, NCq, Dq, F, D, glu ? 1 : 0, 0, 1, F, DF, 1, w1p});
  // B of dX = dGU W1^T is [Dq][3 NCq] HHL (row = d, k = column of W1)
  go(Planes3W{w1, glu ? w1b : nullptr, E, Dq, NCq, D, F, 0, glu ? 1 : 0, F, 1, DF, 0, w1t});
  // down projection W2 [F][D]: B of Y = H W2 is [Dq][3 Fq] HLH (row = d, k = f)
  go(Planes3W{w2, nullptr, E, Dq, Fq, D, F, 0, 0, 1, D, DF, 1, w2p});
  // B of dH = dY W2^T is [Fq][3 Dq] HHL (row = f, k = d)
  go(Planes3W{w2, nullptr, E, Fq, Dq, F, D, 0, 0, D, 1, DF, 0, w2t});
}

void mxm_launch_hidden_planes3(const float* gu, int64_t rows, int Fq, int etype, int act,
                               float slope, uint16_t* h3, hipStream_t s) {
  const int64_t n = rows * Fq;
  if (n > 0)
    hipLaunchKernelGGL(hidden_planes3_kernel, dim3(grid_of((size_t)n)), dim3(256), 0, s, gu, rows,
                       Fq, etype, act, slope, h3);
}

void mxm_launch_act_bw_planes3(const float* gu, const float* dh, int64_t rows, int Fq, int etype,
                               int act, float slope, uint16_t* dgu3, hipStream_t s) {
  const int64_t n = rows * Fq;
  if (n > 0)
    hipLaunchKernelGGL(act_bw_planes3_kernel, dim3(grid_of((size_t)n)), dim3(256), 0, s, gu, dh,
                       rows, Fq, etype, act, slope, dgu3);
}

void mxm_launch_dx_sum(const float* dxr, const float* dxe, int ld, const int32_t* slot_pos, int N,
                       int D, int K, float* dx, hipStream_t s) {
  if (N > 0)
    hipLaunchKernelGGL(dx_sum_kernel, dim3(N), dim3(256), 0, s, dxr, dxe, ld, slot_pos, D, K, dx);
}
