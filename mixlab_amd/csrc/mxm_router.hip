// Router: logits = x . Wr, softmax, stable top-k, renormalised gates
// (gpu/ir.cpp:1106-1111), fused with the per-tile pieces of dispatch and of
// the aux / entropy outputs (gpu/ir.cpp:1150-1162).
//
// One workgroup owns a tile of MXM_ROUTER_TM consecutive tokens and all E
// experts.  (Small batches compute the logits first with logits_small_kernel,
// one wave per token, and the tile kernel starts at phase 2.)  Phase 1 is a register-tiled SIMT product: each output logit is
// accumulated in fp32 by fmaf over d = 0..D-1 in ascending order, which is
// the order the CPU restatement uses, so logits are bit-identical.  Phase 2
// gives each wavefront 16 tokens: one lane per expert (lane l holds experts
// l, l+64, ...), softmax with a fixed xor-butterfly sum, top-k by K rounds of
// a wave-wide argmax under the total order (p desc, expert asc), i.e. the
// order of a stable argsort(-p).  Phase 3 writes, per tile, the per-expert
// token bitmasks' popcounts (the tile histogram) and each slot's rank among
// the tile's tokens routed to the same expert; the scan kernel turns these
// into the stable permutation.
#include "mxm_kernels.h"

namespace {

constexpr int TM = MXM_ROUTER_TM;  // tokens per tile
constexpr int BK = 64;             // d-chunk staged through LDS
constexpr int NT = 256;            // threads per workgroup

template <typename TX>
__device__ __forceinline__ float ld_as_f32(const TX* p);
template <>
__device__ __forceinline__ float ld_as_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld_as_f32<uint16_t>(const uint16_t* p) { return mxm_bf2f(*p); }

template <typename TX>
__device__ __forceinline__ void unpack16(const uint4 raw, float* f);
template <>
__device__ __forceinline__ void unpack16<float>(const uint4 raw, float* f) {
  f[0] = mxm_u2f(raw.x);
  f[1] = mxm_u2f(raw.y);
  f[2] = mxm_u2f(raw.z);
  f[3] = mxm_u2f(raw.w);
}
template <>
__device__ __forceinline__ void unpack16<uint16_t>(const uint4 raw, float* f) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = mxm_u2f(w[q] << 16);
    f[2 * q + 1] = mxm_u2f(w[q] & 0xffff0000u);
  }
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return mxm_xor_lane_f(v, m); }
__device__ __forceinline__ int shfl_xor_i(int v, int m) { return mxm_xor_lane_i(v, m); }

// EPT = experts per thread in phase 1 (E padded to 16*EPT).
template <typename TX, bool BF16, int EPT, bool VEC, bool PRE>
__global__ __launch_bounds__(PRE ? 1024 : NT) void router_kernel(
    const TX* __restrict__ x, const TX* __restrict__ wr, const float* __restrict__ logits_in,
    int N, int D, int E, int K,
    int32_t* __restrict__ top_idx, float* __restrict__ gates, int32_t* __restrict__ slot_rank,
    int32_t* __restrict__ tile_counts, float* __restrict__ tile_psum, float* __restrict__ tile_ent,
    float* __restrict__ probs_out, int ntiles) {
  constexpr int EP = 16 * EPT;
  constexpr int NJ = (EP + 63) / 64;  // experts per lane in phase 2
  constexpr int LG_STRIDE = EP + 1;
  constexpr int STAGE_FLOATS = BK * TM + BK * EP;
  constexpr int LG_FLOATS = TM * LG_STRIDE;
  constexpr int SMEM_FLOATS = STAGE_FLOATS > LG_FLOATS ? STAGE_FLOATS : LG_FLOATS;
  __shared__ float smem[SMEM_FLOATS];
  __shared__ uint32_t mask[EP][2];
  constexpr int THREADS = PRE ? 1024 : NT;
  constexpr int NWAVE = THREADS / 64;
  __shared__ float wave_psum[NWAVE][EP];
  __shared__ float wave_ent[NWAVE];

  float* xs = smem;            // [BK][TM]
  float* ws = smem + BK * TM;  // [BK][EP]
  float* lg = smem;            // [TM][LG_STRIDE] after phase 1

  const int tid = threadIdx.x;
  const int tile = blockIdx.x;
  const int n0 = tile * TM;
  for (int i = tid; i < EP * 2; i += THREADS) (&mask[0][0])[i] = 0u;

  // ---- phase 1: logits --------------------------------------------------
  if (PRE) {
    // logits computed by logits_small_kernel (same accumulation order)
    for (int i = tid; i < TM * EP; i += THREADS) {
      const int t = i / EP, e = i % EP;
      const int n = n0 + t;
      const float v = (n < N && e < E) ? logits_in[(size_t)n * E + e] : 0.0f;
      lg[t * LG_STRIDE + e] = BF16 ? mxm_rbf(v) : v;
    }
    __syncthreads();
  } else {
  const int ty = tid >> 4;  // tokens ty*4 .. ty*4+3
  const int tx = tid & 15;  // experts tx*EPT .. tx*EPT+EPT-1
  float acc[4][EPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < EPT; ++j) acc[i][j] = 0.0f;

  for (int d0 = 0; d0 < D; d0 += BK) {
    __syncthreads();
    if (VEC) {
      // 16-byte loads along d, token-fastest across lanes so the transposed
      // LDS store is conflict-free.
      constexpr int PER = 16 / sizeof(TX);
      for (int i = tid; i < TM * (BK / PER); i += NT) {
        const int t = i % TM, dc = i / TM;
        const int n = n0 + t, d = d0 + dc * PER;
        float f[PER];
        if (n < N && d < D) {
          const uint4 raw = *reinterpret_cast<const uint4*>(x + (size_t)n * D + d);
          unpack16<TX>(raw, f);
        } else {
#pragma unroll
          for (int q = 0; q < PER; ++q) f[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) xs[(dc * PER + q) * TM + t] = f[q];
      }
    } else {
      for (int i = tid; i < TM * BK; i += NT) {
        const int t = i % TM, dd = i / TM;
        const int n = n0 + t, d = d0 + dd;
        xs[dd * TM + t] = (n < N && d < D) ? ld_as_f32<TX>(x + (size_t)n * D + d) : 0.0f;
      }
    }
    for (int i = tid; i < BK * EP; i += NT) {
      const int dd = i / EP, e = i % EP;
      const int d = d0 + dd;
      ws[i] = (d < D && e < E) ? ld_as_f32<TX>(wr + (size_t)d * E + e) : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int dd = 0; dd < BK; ++dd) {
      const float4 xv = *reinterpret_cast<const float4*>(&xs[dd * TM + ty * 4]);
      float wv[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) wv[j] = ws[dd * EP + tx * EPT + j];
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        acc[0][j] = __builtin_fmaf(xv.x, wv[j], acc[0][j]);
        acc[1][j] = __builtin_fmaf(xv.y, wv[j], acc[1][j]);
        acc[2][j] = __builtin_fmaf(xv.z, wv[j], acc[2][j]);
        acc[3][j] = __builtin_fmaf(xv.w, wv[j], acc[3][j]);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const float v = acc[i][j];
      lg[(ty * 4 + i) * LG_STRIDE + tx * EPT + j] = BF16 ? mxm_rbf(v) : v;
    }
  __syncthreads();

  }

  // ---- phase 2: softmax, top-k, gates -----------------------------------
  const int lane = tid & 63;
  const int wave = tid >> 6;
  float psum[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) psum[j] = 0.0f;
  float ent_acc = 0.0f;

  for (int tt = 0; tt < TM / NWAVE; ++tt) {
    const int t = wave * (TM / NWAVE) + tt;
    const int n = n0 + t;
    if (n >= N) break;
    float v[NJ];
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      v[j] = (e < E) ? lg[t * LG_STRIDE + e] : -__builtin_inff();
      m = fmaxf(m, v[j]);
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, shfl_xor_f(m, s));
    float ex[NJ];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      ex[j] = (e < E) ? mxm_exp(v[j] - m) : 0.0f;
      sum = (j == 0) ? ex[j] : sum + ex[j];
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) sum = sum + shfl_xor_f(sum, s);
    float p[NJ];
    float ent_local = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      float q = mxm_ftz(ex[j] / sum);
      if (BF16) q = mxm_rbf(q);
      p[j] = (e < E) ? q : -1.0f;
      if (e < E) {
        psum[j] = psum[j] + q;
        const float term = q * logf(fmaxf(q, 1e-12f));
        ent_local = (j == 0) ? term : ent_local + term;
        if (probs_out) probs_out[(size_t)n * E + e] = q;
      }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) ent_local = ent_local + shfl_xor_f(ent_local, s);
    ent_acc = ent_acc + ent_local;

    // top-k: K rounds of argmax under (p desc, e asc).  The argmax is
    // wave-uniform, so every lane accumulates the same running sum of the
    // picked probabilities (k order), and lane k%64 keeps pick k in slot k/64.
    uint32_t taken = 0u;
    float s_top = 0.0f;
    float my_p[NJ];
    int my_e[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      my_p[j] = 0.0f;
      my_e[j] = 0;
    }
    for (int k = 0; k < K; ++k) {
      float bp = -2.0f;
      int be = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !((taken >> j) & 1u) && p[j] > bp) {
          bp = p[j];
          be = e;
        }
      }
#pragma unroll
      for (int s = 32; s >= 1; s >>= 1) {
        const float op = shfl_xor_f(bp, s);
        const int oe = shfl_xor_i(be, s);
        if (op > bp || (op == bp && oe < be)) {
          bp = op;
          be = oe;
        }
      }
      if ((be & 63) == lane) taken |= 1u << (be >> 6);
      s_top = (k == 0) ? bp : s_top + bp;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (k == lane + 64 * j) {
          my_p[j] = bp;
          my_e[j] = be;
        }
    }
    if (BF16) s_top = mxm_rbf(s_top);
    const float den = fmaxf(s_top, 1e-12f);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int k = lane + 64 * j;
      if (k < K) {
        top_idx[(size_t)n * K + k] = my_e[j];
        gates[(size_t)n * K + k] = my_p[j] / den;
        atomicOr(&mask[my_e[j]][t >> 5], 1u << (t & 31));
      }
    }
  }

  if (lane == 0) wave_ent[wave] = ent_acc;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + 64 * j;
    if (e < EP) wave_psum[wave][e] = psum[j];
  }
  __syncthreads();

  // ---- phase 3: tile histogram, slot ranks, aux partials -----------------
  for (int e = tid; e < E; e += THREADS) {
    tile_counts[(size_t)e * ntiles + tile] = __popc(mask[e][0]) + __popc(mask[e][1]);
    float ps = wave_psum[0][e];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) ps = ps + wave_psum[w][e];
    tile_psum[(size_t)e * ntiles + tile] = ps;
  }
  if (tid == 0) {
    float en = wave_ent[0];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) en = en + wave_ent[w];
    tile_ent[tile] = en;
  }
  for (int i = tid; i < TM * K; i += THREADS) {
    const int t = i / K;
    const int n = n0 + t;
    if (n >= N) continue;
    const int e = top_idx[(size_t)n * K + (i % K)];
    const uint32_t lo = mask[e][0], hi = mask[e][1];
    int r;
    if (t < 32)
      r = __popc(lo & ((1u << t) - 1u));
    else
      r = __popc(lo) + __popc(hi & ((1u << (t - 32)) - 1u));
    slot_rank[(size_t)n * K + (i % K)] = r;
  }
}

// Logits for small batches, where the tiled kernel would run on a handful of
// workgroups.  A workgroup takes four tokens, one per wave; lane l computes
// experts l, l+64, ...  Each logit is fmaf-accumulated over d = 0..D-1 in
// ascending order from 0, exactly as the tiled phase 1 does, so the bits are
// the same.  The router weights pass through LDS in chunks of BK rows (fp32,
// double-buffered: the next chunk's global loads are in flight while the
// current one is consumed); the tokens' x values travel the same way.
template <typename TX, int NJ, bool VEC>
__global__ __launch_bounds__(256) void logits_small_kernel(const TX* __restrict__ x,
                                                           const TX* __restrict__ wr, int N, int D,
                                                           int E, float* __restrict__ out) {
  constexpr int EP = 64 * NJ;
  constexpr int BK = 128 / NJ;             // one 32 KB fp32 buffer per chunk
  constexpr int VW = 16 / sizeof(TX);      // elements per 16-byte load
  constexpr int CPR = EP / VW;             // vectors per weight row
  constexpr int RPP = 256 / CPR;           // weight rows per loader pass
  constexpr int WPASS = BK / RPP;
  constexpr int XV = 4 * BK / VW;          // x vectors per chunk (4 tokens)
  static_assert(XV <= 256, "x chunk fits one loader pass");
  __shared__ __attribute__((aligned(16))) float ws[2][BK][EP];
  __shared__ __attribute__((aligned(16))) float xs[2][4][BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * 4;
  const int nchunks = (D + BK - 1) / BK;

  // Raw 16-byte pieces of the next chunk; they are converted (and the ones
  // outside [D, E] zeroed) only when written to LDS, after the current
  // chunk's arithmetic, so the loads stay in flight meanwhile.
  uint4 wraw[WPASS];
  uint4 xraw = make_uint4(0u, 0u, 0u, 0u);
  uint32_t wok = 0u;  // bit p*VW + q: element q of piece p lies inside [D, E]
  bool xok = false;
  auto load = [&](int c) {
    const int d0 = c * BK;
    wok = 0u;
#pragma unroll
    for (int p = 0; p < WPASS; ++p) {
      const int d = d0 + p * RPP + tid / CPR, e = (tid % CPR) * VW;
      if (VEC) {
        const bool ok = d < D && e < E;
        wraw[p] = *reinterpret_cast<const uint4*>(wr + (ok ? (size_t)d * E + e : 0));
        wok |= ok ? (((1u << VW) - 1u) << (p * VW)) : 0u;
      } else {
        TX v[VW];
#pragma unroll
        for (int q = 0; q < VW; ++q) {
          const bool ok = d < D && e + q < E;
          v[q] = wr[ok ? (size_t)d * E + e + q : 0];
          wok |= ok ? (1u << (p * VW + q)) : 0u;
        }
        wraw[p] = __builtin_bit_cast(uint4, v);
      }
    }
    if (tid < XV) {
      const int t = tid / (BK / VW), d = d0 + (tid % (BK / VW)) * VW;
      const int n = n0 + t;
      xok = n < N && d < D;
      if (VEC) {
        xraw = *reinterpret_cast<const uint4*>(x + (xok ? (size_t)n * D + d : 0));
      } else {
        TX v[VW];
#pragma unroll
        for (int q = 0; q < VW; ++q) v[q] = (xok && d + q < D) ? x[(size_t)n * D + d + q] : TX(0);
        xraw = __builtin_bit_cast(uint4, v);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < WPASS; ++p) {
      float f[VW];
      unpack16<TX>(wraw[p], f);
      float* dst = &ws[buf][p * RPP + tid / CPR][(tid % CPR) * VW];
#pragma unroll
      for (int q = 0; q < VW; ++q) dst[q] = ((wok >> (p * VW + q)) & 1u) ? f[q] : 0.0f;
    }
    if (tid < XV) {
      float f[VW];
      unpack16<TX>(xraw, f);
      float* dst = &xs[buf][tid / (BK / VW)][(tid % (BK / VW)) * VW];
#pragma unroll
      for (int q = 0; q < VW; ++q) dst[q] = xok ? f[q] : 0.0f;
    }
  };

  float acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = 0.0f;
  load(0);
  store(0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    if (c + 1 < nchunks) load(c + 1);
    // rows past D are zero in both buffers: fmaf(0, 0, acc) leaves acc's
    // value unchanged
    const float* xw = xs[buf][wave];
#pragma unroll 8
    for (int dd = 0; dd < BK; dd += 4) {
      const float4 xv = *reinterpret_cast<const float4*>(xw + dd);
      const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[j] = __builtin_fmaf(xa[q], ws[buf][dd + q][lane + 64 * j], acc[j]);
    }
    if (c + 1 < nchunks) store(buf ^ 1);
    __syncthreads();
  }
  const int n = n0 + wave;
  if (n < N) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (lane + 64 * j < E) out[(size_t)n * E + lane + 64 * j] = acc[j];
  }
}

template <typename TX, bool BF16, int EPT>
void launch_router_t(const RouterArgs& a, hipStream_t s) {
  if (a.logits_scratch) {
    constexpr int NJ = (16 * EPT + 63) / 64;
    constexpr int VW = 16 / (int)sizeof(TX);
    const bool vec = a.E % VW == 0 && a.D % VW == 0 &&
                     (reinterpret_cast<uintptr_t>(a.x) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.wr) % 16) == 0;
    if (vec)
      hipLaunchKernelGGL((logits_small_kernel<TX, NJ, true>), dim3((a.N + 3) / 4), dim3(256), 0, s,
                         static_cast<const TX*>(a.x), static_cast<const TX*>(a.wr), a.N, a.D, a.E,
                         a.logits_scratch);
    else
      hipLaunchKernelGGL((logits_small_kernel<TX, NJ, false>), dim3((a.N + 3) / 4), dim3(256), 0, s,
                         static_cast<const TX*>(a.x), static_cast<const TX*>(a.wr), a.N, a.D, a.E,
                         a.logits_scratch);
    const int ntiles = (a.N + TM - 1) / TM;
    hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, false, true>), dim3(ntiles), dim3(1024), 0, s,
                       static_cast<const TX*>(a.x), static_cast<const TX*>(a.wr),
                       a.logits_scratch, a.N, a.D, a.E, a.K, a.top_idx, a.gates, a.slot_rank,
                       a.tile_counts, a.tile_psum, a.tile_ent, a.probs_out, ntiles);
    return;
  }
  const int ntiles = (a.N + TM - 1) / TM;
  const bool vec = (a.D % (16 / (int)sizeof(TX))) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  if (vec)
    hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, true, false>), dim3(ntiles), dim3(NT), 0, s,
                       static_cast<const TX*>(a.x), static_cast<const TX*>(a.wr), nullptr, a.N, a.D, a.E,
                       a.K, a.top_idx, a.gates, a.slot_rank, a.tile_counts, a.tile_psum,
                       a.tile_ent, a.probs_out, ntiles);
  else
    hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, false, false>), dim3(ntiles), dim3(NT), 0, s,
                       static_cast<const TX*>(a.x), static_cast<const TX*>(a.wr), nullptr, a.N, a.D, a.E,
                       a.K, a.top_idx, a.gates, a.slot_rank, a.tile_counts, a.tile_psum,
                       a.tile_ent, a.probs_out, ntiles);
}

template <typename TX, bool BF16>
void launch_router_dt(const RouterArgs& a, hipStream_t s) {
  if (a.E <= 16)
    launch_router_t<TX, BF16, 1>(a, s);
  else if (a.E <= 32)
    launch_router_t<TX, BF16, 2>(a, s);
  else if (a.E <= 64)
    launch_router_t<TX, BF16, 4>(a, s);
  else if (a.E <= 128)
    launch_router_t<TX, BF16, 8>(a, s);
  else
    launch_router_t<TX, BF16, 16>(a, s);
}

}  // namespace

void mxm_launch_router(const RouterArgs& a, bool bf16, hipStream_t s) {
  if (bf16)
    launch_router_dt<uint16_t, true>(a, s);
  else
    launch_router_dt<float, false>(a, s);
}
