// Router: logits = x . Wr, softmax, stable top-k, renormalised gates
// (gpu/ir.cpp:1106-1111), fused with the per-tile pieces of dispatch and of
// the aux / entropy outputs (gpu/ir.cpp:1150-1162).
//
// One workgroup owns a tile of MXM_ROUTER_TM consecutive tokens and all E
// experts.  Phase 1 computes the logits in their summation order
// (mxm_numerics.h): per 64-d chunk of d, a partial by fmaf over the chunk's
// d ascending from +0, added to the logit in chunk order -- the order the
// CPU restatement uses, so logits are bit-identical.  For E > 32 the fmaf
// chains run on the fp32 matrix cores (logits_mfma, a pass per group of 64
// experts), otherwise as a register-tiled SIMT product on the vector unit.
// Phase 2
// gives each wavefront 16 tokens: one lane per expert (lane l holds experts
// l, l+64, ...), softmax with a fixed xor-butterfly sum, top-k by K rounds of
// a wave-wide argmax under the total order (p desc, expert asc), i.e. the
// order of a stable argsort(-p).  Phase 3 writes, per tile, the per-expert
// token bitmasks' popcounts (the tile histogram) and each slot's rank among
// the tile's tokens routed to the same expert; the scan kernel turns these
// into the stable permutation.
//
// Decode-sized batches take route_small_kernel instead (one launch for the
// router, scan and scatter; see below).  Both kernels run the per-token
// softmax / top-k / gate code of route_token, so their routing is the same
// bit for bit.
#include <type_traits>

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

// Per-wave LDS scratch of route_token's top-k for E <= 64.
struct RankScratch {
  uint64_t key[64];
  float pick_p[64];
  int pick_e[64];
};

// Softmax, stable top-k and renormalised gates of one token on one wave
// (gpu/ir.cpp:1107-1111).  Lane l holds experts l + 64 j (j < NJ); v[j] is
// that expert's logit (bf16-rounded in the bf16 flow), ignored past E.  On
// return p[j] is the expert's probability (-1 past E), lane k % 64 holds
// pick k's expert and gate in pick_e[k / 64] and pick_g[k / 64], and the
// result is the token's sum_e p log max(p, 1e-12) (gpu/ir.cpp:1161), summed
// lane-wise in j order and then by the xor butterfly.
template <bool BF16, int NJ>
__device__ __forceinline__ float route_token(const float (&v)[NJ], int lane, int E, int K,
                                             float (&p)[NJ], int (&pick_e)[NJ],
                                             float (&pick_g)[NJ], RankScratch* rsc) {
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    if (lane + 64 * j < E) m = fmaxf(m, v[j]);
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
  float ent_local = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + 64 * j;
    float q = mxm_ftz(ex[j] / sum);
    if (BF16) q = mxm_rbf(q);
    p[j] = (e < E) ? q : -1.0f;
    if (e < E) {
      const float term = q * logf(fmaxf(q, 1e-12f));
      ent_local = (j == 0) ? term : ent_local + term;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ent_local = ent_local + shfl_xor_f(ent_local, s);

  // top-k under (p desc, e asc) -- the order of a stable argsort(-p).  Every
  // lane accumulates the same running sum of the picked probabilities (k
  // order), and lane k%64 keeps pick k in slot k/64.  E > 64: K rounds of a
  // wave-wide argmax.
  uint32_t taken = 0u;
  float s_top = 0.0f;
  float my_p[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    my_p[j] = 0.0f;
    pick_e[j] = 0;
  }
  if constexpr (NJ == 1) {
    // E <= 64: each lane's rank under the same order, from the wave's 64
    // keys in LDS (broadcast reads): key = (bits of p + 2) << 6 | (63 - lane),
    // an integer order equal to (p desc, e asc) on p >= 0.  A NaN p (every p
    // of a token with a non-finite logit) takes 64 | (63 - lane) and a lane
    // past E (p = -1) 63 - lane, below every p >= 0: the 64 keys are distinct,
    // so the ranks are a permutation and the K <= E picks distinct experts
    // below E, whatever the inputs.  The lane of rank k < K leaves its
    // probability and expert in pick slot k; every lane then reads the K
    // picks in k order.  (One wave owns rsc; its LDS operations complete in
    // program order.)
    const float pl = p[0];
    const uint64_t lo = (uint64_t)(63 - lane);
    const uint64_t key = pl >= 0.0f ? (((uint64_t)__builtin_bit_cast(uint32_t, pl) + 2) << 6) | lo
                         : lane < E ? (64ull | lo)
                                    : lo;
    rsc->key[lane] = key;
    __builtin_amdgcn_wave_barrier();
    int rank = 0;
#pragma unroll
    for (int j2 = 0; j2 < 32; ++j2) {
      const ulonglong2 q = reinterpret_cast<const ulonglong2*>(rsc->key)[j2];
      rank += (q.x > key) ? 1 : 0;
      rank += (q.y > key) ? 1 : 0;
    }
    if (rank < K) {
      rsc->pick_p[rank] = pl;
      rsc->pick_e[rank] = lane;
    }
    __builtin_amdgcn_wave_barrier();
    for (int k = 0; k < K; ++k) {
      const float bp = rsc->pick_p[k];
      s_top = (k == 0) ? bp : s_top + bp;
    }
    if (lane < K) {
      my_p[0] = rsc->pick_p[lane];
      pick_e[0] = rsc->pick_e[lane];
    }
    __builtin_amdgcn_wave_barrier();  // rsc is free for the wave's next token
    (void)taken;
  } else {
    // a NaN p (every p of a token with a non-finite logit) competes as -1.5,
    // below every p >= 0, so each round picks an untaken expert below E
    for (int k = 0; k < K; ++k) {
      float bp = -2.0f;
      int be = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        const float c = p[j] >= 0.0f ? p[j] : -1.5f;
        if (e < E && !((taken >> j) & 1u) && c > bp) {
          bp = c;
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
      if (bp < 0.0f) bp = __builtin_nanf("");  // the NaN it stood for
      s_top = (k == 0) ? bp : s_top + bp;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (k == lane + 64 * j) {
          my_p[j] = bp;
          pick_e[j] = be;
        }
    }
  }
  if (BF16) s_top = mxm_rbf(s_top);
  const float den = fmaxf(s_top, 1e-12f);
#pragma unroll
  for (int j = 0; j < NJ; ++j) pick_g[j] = my_p[j] / den;
  return ent_local;
}

// route_token for E <= SEG < 64 with 64 / SEG tokens on one wave at once:
// lane l works on token slot l / SEG, expert e = l % SEG (SEG a power of
// two).  Per token these are route_token's operations in route_token's
// order: its butterfly steps of xor distance >= SEG only combine a lane
// with lanes past E, which hold -inf (the max) or +0 (the sums), so
// leaving them out changes no result (up to the sign of an all-zero
// entropy term), and the rank counts the same larger keys (lanes past E
// carry the lowest keys).  Returns the token's entropy term in every lane of its
// segment; p is -1 past E; lane e < K of a segment holds pick e.
template <bool BF16, int SEG>
__device__ __forceinline__ float route_token_seg(float v, int lane, int E, int K, float& p,
                                                 int& pick_e, float& pick_g, RankScratch* rsc) {
  const int e = lane & (SEG - 1), base = lane - e;
  float m = e < E ? v : -__builtin_inff();
#pragma unroll
  for (int s = SEG / 2; s >= 1; s >>= 1) m = fmaxf(m, shfl_xor_f(m, s));
  const float ex = e < E ? mxm_exp(v - m) : 0.0f;
  float sum = ex;
#pragma unroll
  for (int s = SEG / 2; s >= 1; s >>= 1) sum = sum + shfl_xor_f(sum, s);
  float q = mxm_ftz(ex / sum);
  if (BF16) q = mxm_rbf(q);
  p = e < E ? q : -1.0f;
  float ent = e < E ? q * logf(fmaxf(q, 1e-12f)) : 0.0f;
#pragma unroll
  for (int s = SEG / 2; s >= 1; s >>= 1) ent = ent + shfl_xor_f(ent, s);
  // rank under (p desc, e asc) among the segment's keys, as route_token
  // (distinct keys: NaN p below every p >= 0, lanes past E lowest)
  const uint64_t lo = (uint64_t)(63 - e);
  const uint64_t key = p >= 0.0f ? (((uint64_t)__builtin_bit_cast(uint32_t, p) + 2) << 6) | lo
                       : e < E ? (64ull | lo)
                               : lo;
  rsc->key[lane] = key;
  __builtin_amdgcn_wave_barrier();
  int rank = 0;
#pragma unroll
  for (int j2 = 0; j2 < SEG / 2; ++j2) {
    const ulonglong2 q2 = reinterpret_cast<const ulonglong2*>(rsc->key + base)[j2];
    rank += (q2.x > key) ? 1 : 0;
    rank += (q2.y > key) ? 1 : 0;
  }
  if (rank < K) {
    rsc->pick_p[base + rank] = p;
    rsc->pick_e[base + rank] = e;
  }
  __builtin_amdgcn_wave_barrier();
  float s_top = 0.0f;
  for (int k = 0; k < K; ++k) {
    const float bp = rsc->pick_p[base + k];
    s_top = (k == 0) ? bp : s_top + bp;
  }
  float my_p = 0.0f;
  pick_e = 0;
  if (e < K) {
    my_p = rsc->pick_p[base + e];
    pick_e = rsc->pick_e[base + e];
  }
  __builtin_amdgcn_wave_barrier();  // rsc is free for the wave's next tokens
  if (BF16) s_top = mxm_rbf(s_top);
  pick_g = my_p / fmaxf(s_top, 1e-12f);
  return ent;
}

// Phase 2 of the tiled router for E <= SEG: the wave's TPW tokens, 64 / SEG at
// a time.  The per-expert probability sums (lane e) and the entropy sum take
// the tokens one by one in token order, as the one-token-per-pass loop does.
template <bool BF16, int SEG, int TPW, int LGS, int EPP>
__device__ __forceinline__ void route_tile_seg(const float* lg, int wave, int lane, int n0, int N,
                                               int E, int K, float* probs_out, int32_t* top_idx,
                                               float* gates, uint32_t (*mask)[2], RankScratch* rsc,
                                               float& psum, float& ent_acc) {
  constexpr int S = 64 / SEG;  // tokens per pass
  static_assert(TPW % S == 0, "whole passes");
  const int sl = lane / SEG, e = lane & (SEG - 1);
  for (int tt0 = 0; tt0 < TPW; tt0 += S) {
    const int t = wave * TPW + tt0 + sl;
    const int n = n0 + t;
    const bool valid = n < N;
    const float v = (valid && e < E) ? lg[t * LGS + e] : -__builtin_inff();
    float p, pick_g;
    int pick_e;
    const float ent = route_token_seg<BF16, SEG>(v, lane, E, K, p, pick_e, pick_g, rsc);
    // the pass's tokens one by one: lane e (< E) adds token s's p of expert e
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (n0 + wave * TPW + tt0 + s >= N) break;  // (tokens past N end the wave's list)
      const float ps = __shfl(p, s * SEG + (lane & (SEG - 1)), 64);
      const float es = __shfl(ent, s * SEG, 64);
      if (lane < E) psum = psum + ps;
      ent_acc = ent_acc + es;
    }
    if (valid) {
      if (e < E && probs_out) probs_out[(size_t)n * E + e] = p;
      if (e < K) {
        top_idx[(size_t)n * K + e] = pick_e;
        gates[(size_t)n * K + e] = pick_g;
        atomicOr(&mask[pick_e][t >> 5], 1u << (t & 31));
      }
    }
  }
  (void)EPP;
}

// ---- logits on the fp32 matrix cores (E in 33..64) -------------------------
// v_mfma_f32_16x16x1_4b_f32 is four 16 x 16 blocks of fused multiply-adds
// with one product each: D = C + A B rounded once, to nearest even,
// denormals kept -- the fmaf of the logits' summation order, bit for bit
// (checked on the part against fmaf chains over bf16-valued, fp32, wide-
// exponent, denormal, signed-zero and cancelling operands).  A chain of them
// over a chunk's d from +0 is therefore the SIMT path's chunk partial, at
// twice the rate of the non-packed fp32 FMA.
//
// A wave computes 16 tokens x 64 experts.  A = tokens, broadcast to the four
// blocks from lane group k = lane / 16 (cbsz 2, abid k); B = experts, lane l
// holding expert l (blocks b = experts 16 b .. 16 b + 15).  The output's
// register 4 b + q in lane l is token (l / 16) * 4 + q, expert 16 b + l % 16.
// A round is 32 d: lane group k loads its token's d0 + 8k .. d0 + 8k + 7
// from x (one 16-byte piece in bf16, two in fp32), and every lane its
// expert's 32 d from the lane-interleaved router copy (4 or 8 pieces).
typedef float mxm_lg16 __attribute__((ext_vector_type(16)));

template <typename TX>
struct LgRound {
  static constexpr int P = 16 / (int)sizeof(TX);  // values per 16-byte piece
  uint4 xu[8 / P];
  uint4 wu[32 / P];
};

// value j (< P) of a 16-byte piece
template <typename TX>
__device__ __forceinline__ float lg_val(const uint4& u, int j) {
  const int wi = sizeof(TX) == 2 ? (j >> 1) : j;
  const uint32_t w = wi == 0 ? u.x : wi == 1 ? u.y : wi == 2 ? u.z : u.w;
  if constexpr (sizeof(TX) == 2) return mxm_u2f((j & 1) ? (w & 0xffff0000u) : (w << 16));
  else return mxm_u2f(w);
}

// x through a buffer descriptor over the wave's 16 token rows: the loads
// are unconditional (a range check in the load returns zeros), so every
// path leaves the same loads in flight and the wait before a round counts
// only the older round's.  Word 3 of a gfx9 raw buffer descriptor: 32-bit
// data format, no swizzle.
constexpr int LG_RSRC_W3 = 0x00020000;
constexpr int LG_OUT_OF_RANGE = 0x7ffffff0;  // above any wave's record count
typedef uint32_t lg_u4 __attribute__((ext_vector_type(4)));

// Round r's pieces.  x pieces at or past D (D % P == 0, so a piece is wholly
// in or out) take an offset past the records and tokens past N lie past
// them, so both load as zeros; the router copy is zero past D up to its
// ldw, a multiple of 64 >= 32 * rounds.
template <typename TX>
__device__ __forceinline__ void lg_load(LgRound<TX>& R, __amdgpu_buffer_rsrc_t xs, int xoff, int D,
                                        const uint4* wt, int lane, int r) {
  constexpr int P = LgRound<TX>::P;
  const int d0 = 32 * r + 8 * (lane >> 4);
#pragma unroll
  for (int h = 0; h < 8 / P; ++h) {
    const int d = d0 + P * h;
    const int off = d < D ? xoff + d * (int)sizeof(TX) : LG_OUT_OF_RANGE;
    const lg_u4 v = __builtin_amdgcn_raw_buffer_load_b128(xs, off, 0, 0);
    R.xu[h] = make_uint4(v.x, v.y, v.z, v.w);
  }
  const uint4* wp = wt + (size_t)(32 / P) * r * 64 + lane;
#pragma unroll
  for (int c = 0; c < 32 / P; ++c) R.wu[c] = wp[c * 64];
}

// the 8 d of lane group KK: d0 + 8 KK + t, t ascending
template <typename TX, int KK, bool FIRST>
__device__ __forceinline__ void lg_group(const LgRound<TX>& R, mxm_lg16& c) {
  constexpr int P = LgRound<TX>::P;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float a = lg_val<TX>(R.xu[t / P], t % P);
    const float b = lg_val<TX>(R.wu[(8 * KK + t) / P], (8 * KK + t) % P);
    if (FIRST && t == 0)
      c = __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, mxm_lg16{}, 2, KK, 0);
    else
      c = __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 2, KK, 0);
  }
}

// a round's 32 d in ascending order; FIRST starts the chunk partial at +0
template <typename TX, bool FIRST>
__device__ __forceinline__ void lg_round(const LgRound<TX>& R, mxm_lg16& c) {
  lg_group<TX, 0, FIRST>(R, c);
  lg_group<TX, 1, false>(R, c);
  lg_group<TX, 2, false>(R, c);
  lg_group<TX, 3, false>(R, c);
}

// The logits of tokens n0w .. n0w + 15 against the 64 (padded) experts: per
// 64-d chunk (two rounds) a partial from +0, added to the logit (from +0) in
// chunk order.  Both rounds of the last chunk run: past D the x pieces and
// the router copy (zero up to ldw) are zeros, and fma(0, 0, c) = c except
// that a -0 partial (a product that underflowed to -0) becomes +0, which
// the logit's addition absorbs (the logit, a sum from +0, is never -0, and
// adding either zero leaves it as it is).  The next round's
// pieces are loaded while a round computes (after the last chunk, its
// second round again, unused).  Needs 16 D sizeof(TX) < 2^30 (the launcher
// checks).
template <typename TX>
__device__ __forceinline__ mxm_lg16 logits_mfma(const TX* x, const TX* wr_t, int N, int D,
                                                int n0w, int lane) {
  // (readfirstlane: the clamp is computed on the vector unit, and a
  // descriptor in vector registers would be taken apart lane by lane)
  const int rows = __builtin_amdgcn_readfirstlane(N - n0w >= 16 ? 16 : N - n0w > 0 ? N - n0w : 0);
  const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<TX*>(rows > 0 ? x + (size_t)n0w * D : x), (short)0, rows * D * (int)sizeof(TX),
      LG_RSRC_W3);
  const int xoff = (lane & 15) * D * (int)sizeof(TX);
  const uint4* wt = reinterpret_cast<const uint4*>(wr_t);
  const int nch = (D + 63) / 64;
  mxm_lg16 lgt = {};
  LgRound<TX> ra, rb;
  // (the scheduling barriers keep each round's loads issued before the
  // other round's products instead of next to their own uses)
  lg_load<TX>(ra, xs, xoff, D, wt, lane, 0);
  for (int ch = 0; ch < nch; ++ch) {
    lg_load<TX>(rb, xs, xoff, D, wt, lane, 2 * ch + 1);
    __builtin_amdgcn_sched_barrier(0);
    mxm_lg16 part;
    lg_round<TX, true>(ra, part);
    __builtin_amdgcn_sched_barrier(0);
    lg_load<TX>(ra, xs, xoff, D, wt, lane, min(2 * ch + 2, 2 * nch - 1));
    __builtin_amdgcn_sched_barrier(0);
    lg_round<TX, false>(rb, part);
#pragma unroll
    for (int i = 0; i < 16; ++i) lgt[i] = lgt[i] + part[i];
  }
  return lgt;
}

// EPT = experts per thread in phase 1 (E padded to 16*EPT).  MF: phase 1 on
// the fp32 matrix cores (EPT 4, 8 or 16; wr_t is the lane-interleaved router
// copy [EPT/4][ldw/P][64][P], x 16-byte aligned with D % P == 0).
template <typename TX, bool BF16, int EPT, bool VEC, bool MF = false>
__global__ __launch_bounds__(NT) void router_kernel(
    const TX* __restrict__ x, const TX* __restrict__ wr, int N, int D, int E, int K,
    int32_t* __restrict__ top_idx, float* __restrict__ gates, int32_t* __restrict__ slot_rank,
    int32_t* __restrict__ tile_counts, float* __restrict__ tile_psum, float* __restrict__ tile_ent,
    float* __restrict__ probs_out, int ntiles,
    const TX* __restrict__ wr_t, int ldw) {
  constexpr int EP = 16 * EPT;
  constexpr int NJ = (EP + 63) / 64;  // experts per lane in phase 2
  constexpr int LG_STRIDE = EP + 1;
  constexpr int STAGE_FLOATS = BK * TM + BK * EP;
  constexpr int LG_FLOATS = TM * LG_STRIDE;
  constexpr int SMEM_FLOATS = MF ? LG_FLOATS : STAGE_FLOATS > LG_FLOATS ? STAGE_FLOATS : LG_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[SMEM_FLOATS];
  __shared__ uint32_t mask[EP][2];
  constexpr int THREADS = NT;
  constexpr int NWAVE = THREADS / 64;
  __shared__ float wave_psum[NWAVE][EP];
  __shared__ float wave_ent[NWAVE];
  __shared__ __attribute__((aligned(16))) RankScratch rank_scr[NWAVE];

  float* xs = smem;            // [BK][TM]
  float* ws = smem + BK * TM;  // [BK][EP]
  float* lg = smem;            // [TM][LG_STRIDE] after phase 1

  const int tid = threadIdx.x;
  const int tile = blockIdx.x;
  const int n0 = tile * TM;
  for (int i = tid; i < EP * 2; i += THREADS) (&mask[0][0])[i] = 0u;

  // ---- phase 1: logits --------------------------------------------------
  if constexpr (MF) {
    // one pass of 64 experts per group of the lane-interleaved copy (its
    // groups lie ldw * 64 elements apart); each pass reads the wave's x rows
    // again
    static_assert(EP % 64 == 0, "the matrix-core logits cover groups of 64 experts");
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), ln = tid & 63;  // wv: uniform
    for (int g = 0; g < EP / 64; ++g) {
      const mxm_lg16 v = logits_mfma<TX>(x, wr_t + (size_t)g * ldw * 64, N, D, n0 + 16 * wv, ln);
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int t = 16 * wv + (ln >> 4) * 4 + q;
          lg[t * LG_STRIDE + 64 * g + 16 * b + (ln & 15)] =
              BF16 ? mxm_rbf(v[4 * b + q]) : v[4 * b + q];
        }
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

    // products of one BK chunk held in LDS (BK is the logits' 64-d summation
    // chunk): a partial from +0, then added to the logit
    static_assert(BK == MXM_LOGIT_CHUNK, "one LDS chunk per summation chunk");
    auto compute = [&]() {
      float part[4][EPT];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < EPT; ++j) part[i][j] = 0.0f;
#pragma unroll 4
      for (int dd = 0; dd < BK; ++dd) {
        const float4 xv = *reinterpret_cast<const float4*>(&xs[dd * TM + ty * 4]);
        float wv[EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) wv[j] = ws[dd * EP + tx * EPT + j];
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          part[0][j] = __builtin_fmaf(xv.x, wv[j], part[0][j]);
          part[1][j] = __builtin_fmaf(xv.y, wv[j], part[1][j]);
          part[2][j] = __builtin_fmaf(xv.z, wv[j], part[2][j]);
          part[3][j] = __builtin_fmaf(xv.w, wv[j], part[3][j]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < EPT; ++j) acc[i][j] = acc[i][j] + part[i][j];
    };
    if constexpr (VEC) {
      // 16-byte pieces of x (token-fastest across lanes, so the transposed LDS
      // store is conflict-free) and of router_w rows.  The next chunk's pieces
      // are loaded into registers while the current chunk's products run;
      // pieces outside [N, D] x [D, E] are loaded from a valid address and
      // zeroed when stored.
      constexpr int PER = 16 / (int)sizeof(TX);
      constexpr int XPC = TM * BK / PER;  // x pieces per chunk
      constexpr int WPC = BK * EP / PER;  // router_w pieces per chunk
      constexpr int XP = (XPC + NT - 1) / NT, WP = (WPC + NT - 1) / NT;
      static_assert(WP <= 32 && XP <= 32, "validity masks are 32 bits");
      uint4 xr[XP], wrr[WP];
      uint32_t xok = 0u, wok = 0u;
      auto load = [&](int d0) {
        xok = 0u;
        wok = 0u;
#pragma unroll
        for (int p = 0; p < XP; ++p) {
          const int i = tid + p * NT;
          const int t = i % TM, dc = i / TM;
          const int n = n0 + t, d = d0 + dc * PER;
          const bool ok = i < XPC && n < N && d < D;
          xr[p] = *reinterpret_cast<const uint4*>(x + (ok ? (size_t)n * D + d : 0));
          xok |= ok ? (1u << p) : 0u;
        }
#pragma unroll
        for (int p = 0; p < WP; ++p) {
          const int j = tid + p * NT;
          const int dd = j / (EP / PER), ec = (j % (EP / PER)) * PER;
          const int d = d0 + dd;
          const bool ok = j < WPC && d < D && ec < E;
          wrr[p] = *reinterpret_cast<const uint4*>(wr + (ok ? (size_t)d * E + ec : 0));
          wok |= ok ? (1u << p) : 0u;
        }
      };
      auto store = [&]() {
#pragma unroll
        for (int p = 0; p < XP; ++p) {
          const int i = tid + p * NT;
          if (i < XPC) {
            const int t = i % TM, dc = i / TM;
            float f[PER];
            unpack16<TX>(xr[p], f);
            const bool ok = (xok >> p) & 1u;
#pragma unroll
            for (int q = 0; q < PER; ++q) xs[(dc * PER + q) * TM + t] = ok ? f[q] : 0.0f;
          }
        }
#pragma unroll
        for (int p = 0; p < WP; ++p) {
          const int j = tid + p * NT;
          if (j < WPC) {
            const int dd = j / (EP / PER), ec = (j % (EP / PER)) * PER;
            float f[PER];
            unpack16<TX>(wrr[p], f);
            const bool ok = (wok >> p) & 1u;
#pragma unroll
            for (int q = 0; q < PER; q += 4)
              *reinterpret_cast<float4*>(&ws[dd * EP + ec + q]) =
                  ok ? make_float4(f[q], f[q + 1], f[q + 2], f[q + 3]) : make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      };
      load(0);
      for (int d0 = 0; d0 < D; d0 += BK) {
        __syncthreads();  // the previous chunk's products are done with LDS
        store();
        __syncthreads();
        if (d0 + BK < D) load(d0 + BK);
        compute();
      }
    } else {
      for (int d0 = 0; d0 < D; d0 += BK) {
        __syncthreads();
        for (int i = tid; i < TM * BK; i += NT) {
          const int t = i % TM, dd = i / TM;
          const int n = n0 + t, d = d0 + dd;
          xs[dd * TM + t] = (n < N && d < D) ? ld_as_f32<TX>(x + (size_t)n * D + d) : 0.0f;
        }
        for (int i = tid; i < BK * EP; i += NT) {
          const int dd = i / EP, e = i % EP;
          const int d = d0 + dd;
          ws[i] = (d < D && e < E) ? ld_as_f32<TX>(wr + (size_t)d * E + e) : 0.0f;
        }
        __syncthreads();
        compute();
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

  // E <= 32 (the EPT 1 and 2 instantiations): several tokens on one wave at
  // once, a lane segment each
  bool seg_done = false;
  if constexpr (EPT <= 2) {
    if (E <= 32) {
      float ps = 0.0f;
      constexpr int TPW = TM / NWAVE;
      if (E <= 4)
        route_tile_seg<BF16, 4, TPW, LG_STRIDE, EP>(lg, wave, lane, n0, N, E, K, probs_out, top_idx,
                                                    gates, mask, &rank_scr[wave], ps, ent_acc);
      else if (E <= 8)
        route_tile_seg<BF16, 8, TPW, LG_STRIDE, EP>(lg, wave, lane, n0, N, E, K, probs_out, top_idx,
                                                    gates, mask, &rank_scr[wave], ps, ent_acc);
      else if (E <= 16)
        route_tile_seg<BF16, 16, TPW, LG_STRIDE, EP>(lg, wave, lane, n0, N, E, K, probs_out,
                                                     top_idx, gates, mask, &rank_scr[wave], ps,
                                                     ent_acc);
      else
        route_tile_seg<BF16, 32, TPW, LG_STRIDE, EP>(lg, wave, lane, n0, N, E, K, probs_out,
                                                     top_idx, gates, mask, &rank_scr[wave], ps,
                                                     ent_acc);
      psum[0] = ps;
      seg_done = true;
    }
  }
  for (int tt = 0; tt < TM / NWAVE && !seg_done; ++tt) {
    const int t = wave * (TM / NWAVE) + tt;
    const int n = n0 + t;
    if (n >= N) break;
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      v[j] = (e < E) ? lg[t * LG_STRIDE + e] : -__builtin_inff();
    }
    float p[NJ], pick_g[NJ];
    int pick_e[NJ];
    ent_acc = ent_acc + route_token<BF16, NJ>(v, lane, E, K, p, pick_e, pick_g, &rank_scr[wave]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        psum[j] = psum[j] + p[j];
        if (probs_out) probs_out[(size_t)n * E + e] = p[j];
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int k = lane + 64 * j;
      if (k < K) {
        top_idx[(size_t)n * K + k] = pick_e[j];
        gates[(size_t)n * K + k] = pick_g[j];
        atomicOr(&mask[pick_e[j]][t >> 5], 1u << (t & 31));
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

// Decode-sized batches: routing in one launch.  Workgroup n owns token n.
// Its x row is staged in LDS as fp32, zero-padded to whole 64-d chunks.  The
// logits follow the chunked summation order of mxm_numerics.h, so the bits
// are those of the tiled kernel: the waves of an expert group (one expert per
// lane) compute chunk partials in rounds, each an fmaf chain from +0 with x
// broadcast from LDS, and the group's first wave adds them in chunk order.
// The router weights are a copy in the flow's dtype, lane-interleaved (each
// wave load is 1 KB contiguous: 16 bytes = the lane's expert's next 4 or 8 d),
// and the next pieces are in flight while a chunk is summed.  Wave 0 then
// runs route_token and writes the token's picks, gates, probabilities and
// entropy term.  Every workgroup then takes a ticket (wave 0: agent-scope
// fence, atomic add); the one that takes the last ticket reads all tokens'
// results back and computes what the scan and scatter kernels compute for
// larger batches: per-expert counts (LDS histogram), offsets and row-tile
// prefixes (wave scans), aux and entropy, and the stable permutation (per
// 64-token chunk, the rank of a slot among the chunk's tokens on its expert
// from a 64-bit token mask, plus the running count of earlier chunks).  It
// resets the ticket for the next call.  No workgroup waits on another, so
// the kernel always drains.
constexpr int RS_NT = 1024;  // 16 waves: four per SIMD hide the LDS and load latency
constexpr int RS_WAVES = RS_NT / 64;
constexpr int RS_RING = 2;   // items in the logits' register ring (128 VGPRs a lane)
// LDS for a round's chunk partials [RPC][NJ * 64] and, in the last
// workgroup, the per-wave probability sums [RS_WAVES][MXM_MAX_EXPERTS]
constexpr int RS_PART_FLOATS = 4096;

__device__ __forceinline__ float rs_wave_sum(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v = v + shfl_xor_f(v, s);
  return v;
}

// The batch's dispatch from its per-token results (top_idx, probs,
// tok_ent): per-expert counts, offsets and row-tile prefixes, aux and
// entropy, and the stable permutation.  One workgroup of RS_NT threads; cnt,
// runc and msk zeroed before the call (ordered by a barrier); sidx holds
// N * K ints of LDS.
template <bool BF16, int NJ>
__device__ __forceinline__ void route_dispatch_body(const RouteSmallArgs& a, int* sidx,
                                                    float* rs_part, int* cnt, int* offs,
                                                    int* runc, uint32_t (*msk)[2]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N, E = a.E, K = a.K;
  // ---- dispatch, aux, entropy (one workgroup) -----------------------------
  // One round trip reads the batch's results back: each thread's first slots
  // (top_idx), its wave's tokens' probabilities and, on the last wave, the
  // entropy terms are loaded together.  Slots go to LDS and straight into the
  // per-expert counts and, for the first 64 tokens, the expert masks of the
  // stable permutation.  Probabilities are summed per wave over a fixed token
  // subset, then over the waves in wave order.
  const int NK = N * K;
  constexpr int SV = 4;  // slots per thread loaded in the first pass
  int sv[SV];
#pragma unroll
  for (int q = 0; q < SV; ++q) {
    const int sl = q * RS_NT + tid;
    sv[q] = sl < NK ? a.top_idx[sl] : 0;
  }
  float ps[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) ps[j] = 0.0f;
#pragma unroll 4
  for (int t = wave; t < N; t += RS_WAVES) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      if (e < E) ps[j] = ps[j] + a.probs[(size_t)t * E + e];
    }
  }
  constexpr int ENT_WAVE = RS_WAVES - 1;
  if (wave == ENT_WAVE) {
    float es = 0.0f;
    for (int t = lane; t < N; t += 64) es = es + a.tok_ent[t];
    es = rs_wave_sum(es);
    if (lane == 0) a.entropy[0] = -(es / (float)N);
  }
  auto take_slot = [&](int sl, int e) {
    sidx[sl] = e;
    atomicAdd(&cnt[e], 1);
    const int t = sl / K;
    if (t < 64) atomicOr(&msk[e][t >> 5], 1u << (t & 31));
  };
#pragma unroll
  for (int q = 0; q < SV; ++q) {
    const int sl = q * RS_NT + tid;
    if (sl < NK) take_slot(sl, sv[q]);
  }
  for (int sl = SV * RS_NT + tid; sl < NK; sl += RS_NT) take_slot(sl, a.top_idx[sl]);
  static_assert(RS_WAVES * MXM_MAX_EXPERTS <= RS_PART_FLOATS, "per-wave probability sums");
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + 64 * j;
    if (e < E) rs_part[wave * MXM_MAX_EXPERTS + e] = ps[j];
  }
  __syncthreads();

  if (wave == 0) {
    // expert e = lane + 64 j: exclusive prefixes of the counts and of the row
    // tiles of both GEMM families (one wave scan per j), the mean
    // probabilities and the aux terms
    int run0 = 0, run1 = 0, run2 = 0;
    float aux = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      const int c = e < E ? cnt[e] : 0;
      const int u1 = (c + a.bm1 - 1) / a.bm1, u2 = (c + a.bm2 - 1) / a.bm2;
      int i0 = c, i1 = u1, i2 = u2;
#pragma unroll
      for (int sh = 1; sh < 64; sh <<= 1) {
        const int v0 = __shfl_up(i0, sh, 64), v1 = __shfl_up(i1, sh, 64), v2 = __shfl_up(i2, sh, 64);
        if (lane >= sh) {
          i0 += v0;
          i1 += v1;
          i2 += v2;
        }
      }
      if (e < E) {
        const int o = run0 + i0 - c;
        offs[e] = o;
        a.offsets[e] = o;
        a.counts[e] = c;
        a.mstart1[e] = run1 + i1 - u1;
        a.mstart2[e] = run2 + i2 - u2;
        float pm = 0.0f;
#pragma unroll
        for (int w = 0; w < RS_WAVES; ++w) pm = pm + rs_part[w * MXM_MAX_EXPERTS + e];
        const float mean = pm / (float)N;
        const float frac = ((float)c / (float)K) / (float)N;
        aux = aux + (BF16 ? mxm_rbf(mean) : mean) * frac;
      }
      run0 += __shfl(i0, 63, 64);
      run1 += __shfl(i1, 63, 64);
      run2 += __shfl(i2, 63, 64);
    }
    aux = rs_wave_sum(aux);
    if (lane == 0) {
      a.offsets[E] = run0;
      a.mstart1[E] = run1;
      a.mstart2[E] = run2;
      const float raw = aux * (float)E;
      a.aux[0] = raw;
      if (a.aux_scaled) a.aux_scaled[0] = raw * a.aux_weight;
    }
  }
  __syncthreads();

  // stable permutation, 64 tokens at a time (chunk 0's masks are built above):
  // the rank of a slot among the chunk's tokens on its expert from the
  // expert's 64-bit token mask, plus the running count of earlier chunks
  for (int c0 = 0; c0 < N; c0 += 64) {
    const int ct = min(64, N - c0);
    if (c0 > 0) {
      for (int e = tid; e < E; e += RS_NT) {
        msk[e][0] = 0u;
        msk[e][1] = 0u;
      }
      __syncthreads();
      for (int i = tid; i < ct * K; i += RS_NT) {
        const int t = i / K;
        atomicOr(&msk[sidx[c0 * K + i]][t >> 5], 1u << (t & 31));
      }
      __syncthreads();
    }
    for (int i = tid; i < ct * K; i += RS_NT) {
      const int t = i / K, sl = c0 * K + i;
      const int e = sidx[sl];
      const uint32_t lo = msk[e][0], hi = msk[e][1];
      const int r = t < 32 ? __popc(lo & ((1u << t) - 1u))
                           : __popc(lo) + __popc(hi & ((1u << (t - 32)) - 1u));
      const int pos = offs[e] + runc[e] + r;
      a.perm[pos] = c0 + t;
      a.slot_pos[sl] = pos;
    }
    if (c0 + 64 < N) {
      __syncthreads();
      for (int e = tid; e < E; e += RS_NT) runc[e] += __popc(msk[e][0]) + __popc(msk[e][1]);
      __syncthreads();
    }
  }
}

template <typename TX, bool BF16, int NJ, bool VEC>
__global__ __launch_bounds__(RS_NT, 1) void route_small_kernel(RouteSmallArgs a) {
  extern __shared__ __attribute__((aligned(16))) float rs_dyn[];  // x row, then the slots
  __shared__ float lg[NJ * 64];
  __shared__ float rs_part[RS_PART_FLOATS];  // a round's chunk partials [RPC][NJ * 64]
  __shared__ __attribute__((aligned(16))) RankScratch rank_scr;
  __shared__ int cnt[MXM_MAX_EXPERTS];
  __shared__ int offs[MXM_MAX_EXPERTS];
  __shared__ int runc[MXM_MAX_EXPERTS];
  __shared__ uint32_t msk[MXM_MAX_EXPERTS][2];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = blockIdx.x;
  const int N = a.N, D = a.D, E = a.E, K = a.K;

  // ---- the token's x row -> LDS (fp32) ----------------------------------
  const TX* xrow = static_cast<const TX*>(a.x) + (size_t)n * D;
  float* xl = rs_dyn;
  if (VEC) {
    constexpr int PER = 16 / sizeof(TX);
    for (int i = tid; i < D / PER; i += RS_NT) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xrow + i * PER);
      float f[PER];
      unpack16<TX>(raw, f);
#pragma unroll
      for (int q = 0; q < PER; q += 4)
        *reinterpret_cast<float4*>(xl + i * PER + q) = make_float4(f[q], f[q + 1], f[q + 2], f[q + 3]);
    }
  } else {
    for (int d = tid; d < D; d += RS_NT) xl[d] = ld_as_f32<TX>(xrow + d);
  }
  // the dispatch's counters (used by the last workgroup only)
  for (int e = tid; e < E; e += RS_NT) {
    cnt[e] = 0;
    runc[e] = 0;
    msk[e][0] = 0u;
    msk[e][1] = 0u;
  }
  // zeros up to whole 64-d chunks (the padded weights are zero too)
  for (int d = D + tid; d < (D + MXM_LOGIT_CHUNK - 1) / MXM_LOGIT_CHUNK * MXM_LOGIT_CHUNK;
       d += RS_NT)
    xl[d] = 0.0f;
  __syncthreads();

  // ---- logits ---------------------------------------------------------------
  // The logits' summation order (mxm_numerics.h): 64-d chunks, each a partial
  // from +0, added in chunk order.  WPG = 16 / NJ waves share an expert group
  // (64 experts, one per lane).  Chunks go in rounds of up to RPC: wave
  // (g, sub) takes chunks sub, sub + WPG, ... of the round, streams their
  // weight pieces through a register ring of RS_RING items (an item is 32
  // registers of pieces: one bf16 chunk or half an fp32 chunk; the next item
  // is in flight while one is summed), and parks each chunk's partial in LDS.
  // After the round's barrier the group's first wave adds the partials in
  // chunk order.
  {
    constexpr int WPG = RS_WAVES / NJ;                  // waves per expert group
    constexpr int PER = 16 / (int)sizeof(TX);           // d per 16-byte weight piece
    constexpr int PPC = MXM_LOGIT_CHUNK / PER;          // pieces per chunk (8 or 16)
    constexpr int IP = 8;                               // pieces per item
    constexpr int IPC = PPC / IP;                       // items per chunk (1 or 2)
    constexpr int RPC = RS_PART_FLOATS / (NJ * 64);     // chunks per round
    static_assert(PPC % IP == 0 && RPC >= WPG, "items and rounds");
    // wave-uniform values in scalar registers, so every condition below is a
    // scalar branch and the loads sit outside divergent control flow
    const int swave = __builtin_amdgcn_readfirstlane(wave);
    const int g = swave / WPG, sub = swave % WPG;
    const bool active = g < NJ;  // NJ == 3 leaves the last wave idle
    const int nchunks = (D + MXM_LOGIT_CHUNK - 1) / MXM_LOGIT_CHUNK;
    // this lane's piece p of chunk c: wlane + (c * PPC + p) * 64 * PER
    const TX* wlane = static_cast<const TX*>(a.wr_t) +
                      ((size_t)(active ? g : 0) * (a.ldw / PER) * 64 + lane) * PER;
    float* part_lds = rs_part + g * 64 + lane;  // chunk i of the round at i * NJ * 64
    float acc = 0.0f;
    for (int r0 = 0; r0 < nchunks; r0 += RPC) {
      const int rc = min(RPC, nchunks - r0);               // chunks in this round
      const int mine = active && sub < rc ? (rc - sub + WPG - 1) / WPG : 0;
      const int nit = mine * IPC;                           // this wave's items
      // Workgroups n and n + 8 run on one XCD (round-robin dispatch); they
      // walk their chunk lists from different starting points, so the XCD's
      // L2 fills from HBM in parallel instead of every CU missing on the same
      // lines at once.  The partials land in chunk slots, so the order of the
      // walk does not change the sum.
      const int rot = (int)((blockIdx.x >> 3) & 7) * mine / 8;
      auto chunk_of = [&](int it) {  // chunk of the round of item it
        int j = it / IPC + rot;
        if (j >= mine) j -= mine;
        return sub + j * WPG;
      };
      uint4 ring[RS_RING][IP];
      // item it: chunk chunk_of(it), pieces (it % IPC) * IP ..
      auto load = [&](auto S, int it) {
        it = min(it, nit - 1);  // past the end: the last item again, unused
        const int c = r0 + chunk_of(it);
        const TX* p = wlane + ((size_t)c * PPC + (it % IPC) * IP) * 64 * PER;
#pragma unroll
        for (int q = 0; q < IP; ++q)
          ring[S()][q] = *reinterpret_cast<const uint4*>(p + (size_t)q * 64 * PER);
      };
      float part = 0.0f;
      auto step = [&](auto S, int it) {
        load(std::integral_constant<int, (S() + RS_RING - 1) % RS_RING>{}, it + RS_RING - 1);
        if (it < nit) {
          const int i = chunk_of(it), h = it % IPC;  // chunk of the round, half
          const float* xc = xl + (r0 + i) * MXM_LOGIT_CHUNK + h * IP * PER;
#pragma unroll
          for (int q = 0; q < IP; ++q) {
            float w[PER];
            unpack16<TX>(ring[S()][q], w);
#pragma unroll
            for (int t = 0; t < PER; ++t) part = __builtin_fmaf(xc[q * PER + t], w[t], part);
          }
          if (h == IPC - 1) {
            part_lds[i * NJ * 64] = part;
            part = 0.0f;
          }
        }
      };
      if (nit > 0) {
        load(std::integral_constant<int, 0>{}, 0);
        static_assert(RS_RING == 2, "two slots in the loop below");
        for (int it = 0; it < nit; it += RS_RING) {
          step(std::integral_constant<int, 0>{}, it);
          step(std::integral_constant<int, 1>{}, it + 1);
        }
      }
      __syncthreads();
      if (active && sub == 0) {
        for (int i = 0; i < rc; ++i) acc = acc + part_lds[i * NJ * 64];
      }
      if (r0 + RPC < nchunks) __syncthreads();  // the next round reuses the partials
    }
    if (active && sub == 0) lg[g * 64 + lane] = BF16 ? mxm_rbf(acc) : acc;
  }
  __syncthreads();

  // ---- softmax, top-k, gates ---------------------------------------------
  if (wave == 0) {
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = lg[lane + 64 * j];
    float p[NJ], pick_g[NJ];
    int pick_e[NJ];
    const float ent = route_token<BF16, NJ>(v, lane, E, K, p, pick_e, pick_g, &rank_scr);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + 64 * j;
      if (e < E) a.probs[(size_t)n * E + e] = p[j];
      if (e < K) {
        a.top_idx[(size_t)n * K + e] = pick_e[j];
        a.gates[(size_t)n * K + e] = pick_g[j];
      }
    }
    if (lane == 0) a.tok_ent[n] = ent;
  }

  // the int8 decode flow reads the per-token results directly; its dispatch
  // runs on demand (mxm_launch_route_dispatch)
  if (!a.dispatch) return;

  // ---- ticket: the last workgroup continues --------------------------------
  // Wave 0 wrote all of this token's results, so it alone releases them; in
  // the last workgroup wave 0 alone acquires the others' (the caches it
  // invalidates are the CU's and the XCD's, shared by the workgroup's waves,
  // and the barrier orders the other waves' reads after it).
  if (wave == 0) {
    __threadfence();
    if (lane == 0) s_last = atomicAdd(a.ticket, 1) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  if (wave == 0) __threadfence();
  __syncthreads();

  route_dispatch_body<BF16, NJ>(a, reinterpret_cast<int*>(rs_dyn), rs_part, cnt, offs, runc, msk);
  if (tid == 0) __hip_atomic_store(a.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename TX, bool BF16, int NJ>
void launch_route_small_t(const RouteSmallArgs& a, hipStream_t s) {
  constexpr int PER = 16 / (int)sizeof(TX);
  const bool vec = a.D % PER == 0 && (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  size_t lds = (size_t)(a.D + MXM_LOGIT_CHUNK - 1) / MXM_LOGIT_CHUNK * MXM_LOGIT_CHUNK * 4;
  const size_t slots = (size_t)a.N * a.K * 4;
  if (slots > lds) lds = slots;
  lds = (lds + 15) / 16 * 16;
  if (vec)
    hipLaunchKernelGGL((route_small_kernel<TX, BF16, NJ, true>), dim3(a.N), dim3(RS_NT), lds, s, a);
  else
    hipLaunchKernelGGL((route_small_kernel<TX, BF16, NJ, false>), dim3(a.N), dim3(RS_NT), lds, s, a);
}

template <typename TX, bool BF16>
void launch_route_small_dt(const RouteSmallArgs& a, hipStream_t s) {
  if (a.E <= 64)
    launch_route_small_t<TX, BF16, 1>(a, s);
  else if (a.E <= 128)
    launch_route_small_t<TX, BF16, 2>(a, s);
  else if (a.E <= 192)
    launch_route_small_t<TX, BF16, 3>(a, s);
  else
    launch_route_small_t<TX, BF16, 4>(a, s);
}

template <typename TX, bool BF16, int EPT>
void launch_router_t(const RouterArgs& a, hipStream_t s) {
  const int ntiles = (a.N + TM - 1) / TM;
  constexpr int PER = 16 / (int)sizeof(TX);
  const bool xvec = a.D % PER == 0 && (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  const bool vec = xvec && a.E % PER == 0 && (reinterpret_cast<uintptr_t>(a.wr) % 16) == 0;
  const TX* x = static_cast<const TX*>(a.x);
  const TX* wr = static_cast<const TX*>(a.wr);
  const TX* wr_t = static_cast<const TX*>(a.wr_t);
  if constexpr (EPT >= 4) {
    if (wr_t && xvec && a.E > 32 && a.D <= (1 << 24)) {
      hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, true, true>), dim3(ntiles), dim3(NT), 0, s,
                         x, wr, a.N, a.D, a.E, a.K, a.top_idx, a.gates, a.slot_rank,
                         a.tile_counts, a.tile_psum, a.tile_ent, a.probs_out, ntiles, wr_t, a.ldw);
      return;
    }
  }
  if (vec)
    hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, true>), dim3(ntiles), dim3(NT), 0, s, x, wr,
                       a.N, a.D, a.E, a.K, a.top_idx, a.gates, a.slot_rank, a.tile_counts,
                       a.tile_psum, a.tile_ent, a.probs_out, ntiles, nullptr, 0);
  else
    hipLaunchKernelGGL((router_kernel<TX, BF16, EPT, false>), dim3(ntiles), dim3(NT), 0, s, x, wr,
                       a.N, a.D, a.E, a.K, a.top_idx, a.gates, a.slot_rank, a.tile_counts,
                       a.tile_psum, a.tile_ent, a.probs_out, ntiles, nullptr, 0);
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

bool mxm_route_small_fits(int N, int D, int E, int K) {
  return N >= 1 && N <= MXM_SMALL_BATCH && (int64_t)N * K <= MXM_SMALL_SLOTS && D >= 1 &&
         D <= MXM_SMALL_D && E >= 1 && E <= MXM_MAX_EXPERTS;
}

void mxm_launch_route_small(const RouteSmallArgs& a, bool bf16, hipStream_t s) {
  if (bf16)
    launch_route_small_dt<uint16_t, true>(a, s);
  else
    launch_route_small_dt<float, false>(a, s);
}

namespace {

template <bool BF16, int NJ>
__global__ __launch_bounds__(RS_NT, 1) void route_dispatch_kernel(RouteSmallArgs a) {
  extern __shared__ __attribute__((aligned(16))) float rd_dyn[];  // the slots
  __shared__ float rs_part[RS_PART_FLOATS];
  __shared__ int cnt[MXM_MAX_EXPERTS];
  __shared__ int offs[MXM_MAX_EXPERTS];
  __shared__ int runc[MXM_MAX_EXPERTS];
  __shared__ uint32_t msk[MXM_MAX_EXPERTS][2];
  for (int e = threadIdx.x; e < a.E; e += RS_NT) {
    cnt[e] = 0;
    runc[e] = 0;
    msk[e][0] = 0u;
    msk[e][1] = 0u;
  }
  __syncthreads();
  route_dispatch_body<BF16, NJ>(a, reinterpret_cast<int*>(rd_dyn), rs_part, cnt, offs, runc, msk);
}

template <bool BF16>
void launch_route_dispatch_b(const RouteSmallArgs& a, hipStream_t s) {
  const size_t lds = ((size_t)a.N * a.K * 4 + 15) / 16 * 16;
  if (a.E <= 64)
    hipLaunchKernelGGL((route_dispatch_kernel<BF16, 1>), dim3(1), dim3(RS_NT), lds, s, a);
  else if (a.E <= 128)
    hipLaunchKernelGGL((route_dispatch_kernel<BF16, 2>), dim3(1), dim3(RS_NT), lds, s, a);
  else if (a.E <= 192)
    hipLaunchKernelGGL((route_dispatch_kernel<BF16, 3>), dim3(1), dim3(RS_NT), lds, s, a);
  else
    hipLaunchKernelGGL((route_dispatch_kernel<BF16, 4>), dim3(1), dim3(RS_NT), lds, s, a);
}

}  // namespace

void mxm_launch_route_dispatch(const RouteSmallArgs& a, bool bf16, hipStream_t s) {
  if (bf16)
    launch_route_dispatch_b<true>(a, s);
  else
    launch_route_dispatch_b<false>(a, s);
}
