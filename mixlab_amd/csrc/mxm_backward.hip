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
// order).  The experts' fp32 products are one rocBLAS GEMM per expert and
// product, issued by the library's host code; the elementwise parts (the
// gathered rows, the activation derivative, dx) are the launchers at the end.
// Every result is deterministic.
#include "mxm_kernels.h"

namespace {

__device__ __forceinline__ float ld_x(const float* p) { return *p; }
__device__ __forceinline__ float ld_x(const uint16_t* p) { return mxm_bf2f(*p); }

__global__ void gather_rows_kernel(const float* __restrict__ x, const int32_t* __restrict__ perm,
                                   int D, float* __restrict__ out) {
  const int s = blockIdx.x;
  const float* src = x + (size_t)perm[s] * D;
  float* dst = out + (size_t)s * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) dst[d] = src[d];
}

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

// one wave per slot: dgates[n*K+k] = <dD[n], Y[slot_pos]>
__global__ __launch_bounds__(256) void dgates_kernel(BackwardArgs a) {
  const int s = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (s >= a.N * a.K) return;
  const int n = s / a.K;
  const float* dd = a.d_delta + (size_t)n * a.D;
  const size_t yo = (size_t)a.slot_pos[s] * a.D;
  float acc = 0.0f;
  if (a.Yb16) {
    for (int d = lane; d < a.D; d += 64) acc = __builtin_fmaf(dd[d], mxm_bf2f(a.Yb16[yo + d]), acc);
  } else {
    for (int d = lane; d < a.D; d += 64) acc = __builtin_fmaf(dd[d], a.Y[yo + d], acc);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = acc + mxm_xor_lane_f(acc, m);
  if (lane == 0) a.dgates[s] = acc;
}

// one thread per token: renorm, aux / entropy and softmax backward
__global__ void router_bw_kernel(BackwardArgs a) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= a.N) return;
  const int K = a.K, E = a.E;
  const float* p = a.probs + (size_t)n * E;
  const int32_t* sel = a.top_idx + (size_t)n * K;
  const float* dg = a.dgates + (size_t)n * K;
  float S = 0.0f;
  for (int k = 0; k < K; ++k) S = S + p[sel[k]];
  const float Sc = fmaxf(S, 1e-12f);
  const bool renorm = S > 1e-12f;
  // d(tp_k) = dg_k / S - sum_j dg_j tp_j / S^2 = sum_j tp_j (dg_k - dg_j) / S^2,
  // the second form free of the cancellation of the first (exactly 0 at K = 1)
  auto dtp_of = [&](int k) {
    if (!renorm) return dg[k] / Sc;
    float t = 0.0f;
    for (int j = 0; j < K; ++j) t = t + p[sel[j]] * (dg[k] - dg[j]);
    return t / (Sc * Sc);
  };
  const float inv_n = 1.0f / (float)a.N;
  const float aux_c = a.d_aux * (float)E * inv_n / ((float)K * (float)a.N);
  auto dp_of = [&](int e) {
    const float pe = p[e];
    float v = aux_c * (float)a.counts[e];
    v = v - a.d_ent * inv_n * (logf(fmaxf(pe, 1e-12f)) + (pe > 1e-12f ? 1.0f : 0.0f));
    for (int k = 0; k < K; ++k)
      if (sel[k] == e) v = v + dtp_of(k);
    return v;
  };
  float s = 0.0f;
  for (int e = 0; e < E; ++e) s = s + p[e] * dp_of(e);
  float* out = a.dlogits + (size_t)n * E;
  for (int e = 0; e < E; ++e) out[e] = p[e] * (dp_of(e) - s);
}

// dY[slot_pos] = gate * dD[n]
__global__ void dy_kernel(BackwardArgs a) {
  const int s = blockIdx.x;
  const int n = s / a.K;
  const float g = a.gates[s];
  const float* dd = a.d_delta + (size_t)n * a.D;
  const size_t o = (size_t)a.slot_pos[s] * a.D;
  if (a.dyb16) {
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) a.dyb16[o + d] = mxm_f2bf(g * dd[d]);
  } else {
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) a.dy[o + d] = g * dd[d];
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

// activation backward per element of [N*K, F]; recomputes H
__global__ void act_bw_kernel(BackwardArgs a, size_t total) {
  const bool glu = a.etype != MXM_EXPERT_MLP;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const float dh = a.dh[i];
    float h, cg, cu;
    act_eval(a.etype, a.act, a.slope, glu ? a.g[i] : 0.0f, a.u[i], h, cg, cu);
    a.h[i] = h;
    if (glu) a.dg[i] = dh * cg;
    a.du[i] = dh * cu;
  }
}

// H per element of [N*K, F] from the projections (the forward's hidden
// units, for the backward's own expert forward)
__global__ void hidden_kernel(BackwardArgs a, size_t total) {
  const bool glu = a.etype != MXM_EXPERT_MLP;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    float h, cg, cu;
    act_eval(a.etype, a.act, a.slope, glu ? a.g[i] : 0.0f, a.u[i], h, cg, cu);
    a.h[i] = h;
  }
}

// d router_w = x^T dlogits, a D x E output reduced over all N rows: row
// chunk c's partial part[c][d][e] = sum over its rows n ascending of
// fmaf(x[n][d], dlogits[n][e], .).  Lane l of a workgroup takes column
// d = 64 * blockIdx.x + l (coalesced x reads), wave w experts
// 4 JT * blockIdx.z + JT w .. +JT-1 (wave-uniform, so dlogits comes in by scalar
// loads); JT = 8 experts per wave for E <= 8, else 16; idle waves (past E)
// return at once.
template <typename TX, int JT>
__global__ __launch_bounds__(256) void router_wgrad_kernel(const TX* __restrict__ x, int D,
                                                           const float* __restrict__ dl, int E,
                                                           int rows, int rc,
                                                           float* __restrict__ part) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e0 = blockIdx.z * (4 * JT) + wave * JT;
  if (e0 >= E) return;
  const int c = blockIdx.y;
  const int d = blockIdx.x * 64 + (threadIdx.x & 63);
  const int dc = min(d, D - 1);  // lanes past D read a valid column and store nothing
  const int r0 = c * rc, r1 = min(rows, r0 + rc);
  const int ne = min(JT, E - e0);
  float acc[JT];
#pragma unroll
  for (int j = 0; j < JT; ++j) acc[j] = 0.0f;
  // rows 8 at a time: the 8 loads go out together, then the FMAs in row order
  constexpr int RU = 8;
  for (int n0 = r0; n0 < r1; n0 += RU) {
    float xv[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) xv[u] = ld_x(x + (size_t)min(n0 + u, r1 - 1) * D + dc);
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      if (n0 + u < r1) {
        const float* dr = dl + (size_t)(n0 + u) * E + e0;
        if (ne == JT) {  // a full block: one contiguous scalar load of the row's JT values
#pragma unroll
          for (int j = 0; j < JT; ++j) acc[j] = __builtin_fmaf(xv[u], dr[j], acc[j]);
        } else {
#pragma unroll
          for (int j = 0; j < JT; ++j)
            if (j < ne) acc[j] = __builtin_fmaf(xv[u], dr[j], acc[j]);
        }
      }
    }
  }
  if (d < D) {
    float* o = part + ((size_t)c * D + d) * E + e0;
#pragma unroll
    for (int j = 0; j < JT; ++j)
      if (j < ne) o[j] = acc[j];
  }
}

// out[q] = sum over chunks c ascending of part[c][q]
__global__ void wgrad_sum_kernel(const float* __restrict__ part, int nchunks, size_t n,
                                 float* __restrict__ out) {
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n;
       q += (size_t)gridDim.x * blockDim.x) {
    float acc = part[q];
    for (int c = 1; c < nchunks; ++c) acc = acc + part[(size_t)c * n + q];
    out[q] = acc;
  }
}

// dx[n] = dxr[n] + sum_k (dxg + dxu)[slot_pos(n, k)], k ascending
__global__ void dx_kernel(BackwardArgs a) {
  const int n = blockIdx.x;
  const bool glu = a.etype != MXM_EXPERT_MLP;
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    float acc = a.dxr[(size_t)n * a.D + d];
    for (int k = 0; k < a.K; ++k) {
      const size_t p = (size_t)a.slot_pos[(size_t)n * a.K + k] * a.D + d;
      const float v = glu ? a.dxg[p] + a.dxu[p] : a.dxu[p];
      acc = acc + v;
    }
    a.dx[(size_t)n * a.D + d] = acc;
  }
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

// out[s] = x[perm[s]] (bf16 rows, permuted order)
__global__ void gather_rows_bf16_kernel(const uint16_t* __restrict__ x,
                                        const int32_t* __restrict__ perm, int D,
                                        uint16_t* __restrict__ out) {
  const int s = blockIdx.x;
  const uint16_t* src = x + (size_t)perm[s] * D;
  uint16_t* dst = out + (size_t)s * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) dst[d] = src[d];
}

// Activation backward on the forward's bf16 projections gu [N*K, NC] (GLU:
// NC = 2F, gate and up columns interleaved in groups of 32 as the MFMA
// family's W1 rows; MLP: NC = F, up only) and dH [N*K, F]: writes dG and dU
// into dgu at the columns of g and u, rounded to bf16.  One thread takes 8
// consecutive hidden units (16-byte loads and stores; F is a multiple of 32).
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

__global__ void act_bw_bf16_kernel(const uint16_t* __restrict__ gu, const uint16_t* __restrict__ dh,
                                   int F, int etype, int act, float slope, size_t total8,
                                   uint16_t* __restrict__ dgu) {
  const bool glu = etype != MXM_EXPERT_MLP;
  const int NC = glu ? 2 * F : F;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total8;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t e0 = i * 8;  // first element of [N*K, F]
    const size_t r = e0 / F;
    const int f = (int)(e0 % F);
    const uint4 hv = *reinterpret_cast<const uint4*>(dh + e0);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    const size_t cu = r * NC + (glu ? (size_t)(f >> 5) * 64 + 32 + (f & 31) : (size_t)f);
    const uint4 uv = *reinterpret_cast<const uint4*>(gu + cu);
    const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t gw[4] = {0u, 0u, 0u, 0u};
    if (glu) {
      const uint4 gv = *reinterpret_cast<const uint4*>(gu + cu - 32);
      gw[0] = gv.x;
      gw[1] = gv.y;
      gw[2] = gv.z;
      gw[3] = gv.w;
    }
    uint32_t og[4], ou[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float dg0, du0, dg1, du1;
      act_bw_one(etype, act, slope, mxm_u2f(gw[q] << 16), mxm_u2f(uw[q] << 16),
                 mxm_u2f(hw[q] << 16), dg0, du0);
      act_bw_one(etype, act, slope, mxm_u2f(gw[q] & 0xffff0000u), mxm_u2f(uw[q] & 0xffff0000u),
                 mxm_u2f(hw[q] & 0xffff0000u), dg1, du1);
      og[q] = (uint32_t)mxm_f2bf(dg0) | ((uint32_t)mxm_f2bf(dg1) << 16);
      ou[q] = (uint32_t)mxm_f2bf(du0) | ((uint32_t)mxm_f2bf(du1) << 16);
    }
    *reinterpret_cast<uint4*>(dgu + cu) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
    if (glu) *reinterpret_cast<uint4*>(dgu + cu - 32) = make_uint4(og[0], og[1], og[2], og[3]);
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

int grid_of(size_t n) {
  size_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

// Row chunks of the router's weight gradient: at most 64, of at least 256 rows.
int wgrad_router_chunks_impl(int N) {
  int c = (N + 255) / 256;
  return c < 1 ? 1 : (c > 64 ? 64 : c);
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

}  // namespace

int wgrad_router_chunks(int N) { return wgrad_router_chunks_impl(N); }

void mxm_launch_tile_prefix(const int32_t* counts, int E, int bm, int32_t* mstart, hipStream_t s) {
  hipLaunchKernelGGL(tile_prefix_kernel, dim3(1), dim3(64), 0, s, counts, E, bm, mstart);
}

void mxm_launch_gather_rows_bf16(const uint16_t* x, const int32_t* perm, int rows, int D,
                                 uint16_t* out, hipStream_t s) {
  if (rows > 0) hipLaunchKernelGGL(gather_rows_bf16_kernel, dim3(rows), dim3(256), 0, s, x, perm, D, out);
}

void mxm_launch_act_bw_bf16(const uint16_t* gu, const uint16_t* dh, int rows, int F, int etype,
                            int act, float slope, uint16_t* dgu, hipStream_t s) {
  // F is a multiple of 32 (the MFMA family's GLU interleave), so rows of 8
  // hidden units never straddle an interleave group or a row
  const size_t total8 = (size_t)rows * F / 8;
  if (total8 > 0)
    hipLaunchKernelGGL(act_bw_bf16_kernel, dim3(grid_of(total8)), dim3(256), 0, s, gu, dh, F, etype,
                       act, slope, total8, dgu);
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
  hipLaunchKernelGGL(dgates_kernel, dim3((NK + 3) / 4), dim3(256), 0, s, a);
  hipLaunchKernelGGL(router_bw_kernel, dim3((N + 127) / 128), dim3(128), 0, s, a);
  hipLaunchKernelGGL(dy_kernel, dim3(NK), dim3(256), 0, s, a);
  grouped(a.dlogits, a.wrt, a.dxr, E, D, a.one, a.one + 2, 1, (N + 63) / 64, s);
  // router: d router_w = x^T dlogits over all N rows -- a D x E output, so
  // the rows are split in chunks (fixed chunk order, rows ascending within a
  // chunk) to spread the reduction over the GPU
  const int nch = wgrad_router_chunks(N);
  const int rc = (N + nch - 1) / nch;
  if (E <= 8) {
    const dim3 wg((D + 63) / 64, nch, 1);
    if (a.xb16)
      hipLaunchKernelGGL((router_wgrad_kernel<uint16_t, 8>), wg, dim3(256), 0, s, a.xb16, D,
                         a.dlogits, E, N, rc, a.wr_part);
    else
      hipLaunchKernelGGL((router_wgrad_kernel<float, 8>), wg, dim3(256), 0, s, a.x, D, a.dlogits,
                         E, N, rc, a.wr_part);
  } else {
    const dim3 wg((D + 63) / 64, nch, (E + 63) / 64);
    if (a.xb16)
      hipLaunchKernelGGL((router_wgrad_kernel<uint16_t, 16>), wg, dim3(256), 0, s, a.xb16, D,
                         a.dlogits, E, N, rc, a.wr_part);
    else
      hipLaunchKernelGGL((router_wgrad_kernel<float, 16>), wg, dim3(256), 0, s, a.x, D, a.dlogits,
                         E, N, rc, a.wr_part);
  }
  const size_t n = (size_t)D * E;
  hipLaunchKernelGGL(wgrad_sum_kernel, dim3(grid_of(n)), dim3(256), 0, s, a.wr_part, nch, n, a.dwr);
  (void)K;
}

// The fp32 experts' elementwise parts; their products are per-expert rocBLAS
// GEMMs issued by the library's host code.
void mxm_launch_backward_gather(const BackwardArgs& a, hipStream_t s) {
  const int NK = a.N * a.K;
  if (NK > 0) hipLaunchKernelGGL(gather_rows_kernel, dim3(NK), dim3(256), 0, s, a.x, a.perm, a.D, a.xp);
}

void mxm_launch_backward_act(const BackwardArgs& a, hipStream_t s) {
  const size_t total = (size_t)a.N * a.K * a.F;
  if (total > 0)
    hipLaunchKernelGGL(act_bw_kernel, dim3(grid_of(total)), dim3(256), 0, s, a, total);
}

void mxm_launch_backward_hidden(const BackwardArgs& a, hipStream_t s) {
  const size_t total = (size_t)a.N * a.K * a.F;
  if (total > 0)
    hipLaunchKernelGGL(hidden_kernel, dim3(grid_of(total)), dim3(256), 0, s, a, total);
}

void mxm_launch_backward_dx(const BackwardArgs& a, hipStream_t s) {
  if (a.N > 0) hipLaunchKernelGGL(dx_kernel, dim3(a.N), dim3(256), 0, s, a);
}
