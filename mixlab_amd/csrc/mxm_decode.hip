// Grouped expert FFN for int8 weights (symmetric, fp32 scale per output
// channel), shaped for decode: few rows per expert, so the kernel is a
// weight stream and its bound is HBM bandwidth.
//
// Weight layout (written at upload by mxm_launch_shuffle_q8): a matrix
// W[Kd][C] (x.W layout) is cut into blocks of 64 k x 16 output columns; block
// (cb, kb) occupies 1 KB at ((kb * C/16) + cb) * 1024 and holds, at bytes
// 16*l .. 16*l+15, the 16 signed bytes W[64kb + 16*(l/16) + i][16cb + l%16],
// i = 0..15.
// Lane l of a wave therefore reads one contiguous 16-byte piece, a wave-load
// is one coalesced 1 KB read, and the waves of a workgroup, which walk k in
// step, read adjacent 1 KB blocks (a k block of all columns is C/16 KB
// contiguous).
//
// MFMA: v_mfma_f32_16x16x32_bf16.  Within a 64-k block, lane group g = l/16
// owns k = 16g .. 16g+15; the first 8 feed one MFMA, the last 8 a second.
// The A operand (16 of the expert's rows, bf16) uses the same k assignment,
// so the sum over k is the plain dot product.  A signed byte converts to
// bf16 exactly (one sign-extending byte-select conversion to fp32 per byte,
// then a pair pack), so the accumulators are sums of x * q.  (Stored offset
// binary, q + 128, the stream needed two more MFMAs per block for the rows'
// sums that remove the offset, at the same conversion count.)
//
// bf16 weights (GemmArgs::w_bf16, bf16 ops at decode sizes): the same
// blocks at 2 bytes per weight (mxm_launch_shuffle_bf16), 2 KB each as two
// 1 KB halves, lane l's first 8 values at bytes 16*l of the first half and
// its last 8 at 16*l of the second (each wave-load one coalesced 1 KB); no
// conversion, no offset and no scale -- the accumulators are the bf16 flow's
// fp32 products.  The ring holds 4 blocks per matrix (against the int8
// stream's 6 and 8), so the bytes in flight and the registers stay close to
// the int8 stream's.
//
// Split hidden (kinds whose hidden is fp32 in the bf16 flow, GemmArgs::
// h_split): the up projection stores H as the planes hi | lo, and the down
// projection stages a pass's 16 rows twice -- row group 0 from the hi
// plane, row group 1 from the lo plane -- so each converted weight block
// feeds both, and y = (hi . W + lo . W) * scale is stored in fp32.
//
// Work split: a workgroup = NW waves = NW consecutive column blocks of one
// expert.  Each wave requests the first P blocks of its weight stream, the
// workgroup stages 16 of the expert's rows (all Kd) in LDS, and each wave
// then streams its column block's weights over the whole of Kd through a
// ring of P register slots (P block-loads per matrix in flight per wave), so
// there is no split-K reduction and no barrier inside the stream.  More
// than 16 rows take further passes.  Experts with no rows return at once, so
// their weights are never read.
#include "mxm_kernels.h"

#ifndef MXM_Q8_DEPTH_GLU
#define MXM_Q8_DEPTH_GLU 6
#endif
#ifndef MXM_Q8_DEPTH_ONE
#define MXM_Q8_DEPTH_ONE 8
#endif
// bf16 weights: 2 KB blocks.  Measured (64 tokens, D 2048, E 64, top-8):
// gate+up 143.3 us at a ring of 3, 140.1 at 4, 154.8 at 5; down 74.3 us at
// 4, 72.6 at 6, 72.6 at 8, but at ffn 1024 57.6 / 61.4 / 60.1
#ifndef MXM_D16_DEPTH_GLU
#define MXM_D16_DEPTH_GLU 4
#endif
#ifndef MXM_D16_DEPTH_ONE
#define MXM_D16_DEPTH_ONE 4
#endif
// 64 rows per pass once an expert averages more than this many rows (int8;
// bf16 weights: MXM_D16_RG4_MIN)
// int8 down projection at 16 rows per pass: two 16-column blocks per wave,
// with the ring depth divided by MXM_Q8_CPW_PDIV (the same bytes in
// flight).  Measured on the 64-token decode layer (D 2048, E 64, top-8, ffn
// 1408): down 39-40 -> 37-37.5 us, its 1,024 workgroups halved to one round
// on the 512 slots; for the gate+up projection it measured slower (67-69 ->
// 75-77 us at half the ring depth, 72-73 at a third: the two-block kernel
// needs more than the 128 registers of two workgroups per CU)
#ifndef MXM_Q8_CPW
#define MXM_Q8_CPW 2
#endif
#ifndef MXM_Q8_CPW_PDIV
#define MXM_Q8_CPW_PDIV 2
#endif
#ifndef MXM_Q8_RG4_MIN
#define MXM_Q8_RG4_MIN 24
#endif
#ifndef MXM_D16_RG4_MIN
#define MXM_D16_RG4_MIN 16
#endif
// 128 rows per pass (eight row groups) once an expert averages more than
// this many rows.  Measured (forwards, 64 against 128 rows per pass, D 2048
// / E 64 / K 8 / ffn 1408): int8 at N 640 0.481 / 0.399 ms, N 768 0.500 /
// 0.422, bf16 at N 512 0.488 / 0.402, N 768 0.623 / 0.439; at 64 rows per
// expert int8 measured mixed (D 1024 / E 32 / K 4 / ffn 1024, N 512: 0.095
// / 0.106 ms), at 128 slower on every shape (two passes either way)
#ifndef MXM_Q8_RG8_MIN
#define MXM_Q8_RG8_MIN 64
#endif
#ifndef MXM_D16_RG8_MIN
#define MXM_D16_RG8_MIN 48
#endif
// the split down projection: 32 rows per pass (four row groups) once an
// expert averages more than this many rows (bf16 weights; int8:
// MXM_SPLIT_Q8_RG4_MIN)
#ifndef MXM_SPLIT_RG4_MIN
#define MXM_SPLIT_RG4_MIN 12
#endif
#ifndef MXM_SPLIT_Q8_RG4_MIN
#define MXM_SPLIT_Q8_RG4_MIN 40
#endif

// Weight blocks are read once per forward, so they are loaded nontemporal
// (the load's nt bit): the stream then does not displace the router's and
// the rows' cache lines from L2 and the last-level cache.  Measured on the
// 64-token decode layer: int8 gate+up 69.6 -> 63.4 us, router 29.4 -> 25.6 us.
#define MXM_WLD(p) __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p))

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int NW = 8;          // waves (column blocks) per workgroup
// A staging: each row group's 16 rows x up to MAX_KD k bf16 per chunk in LDS
// (64 KB), half that k at four row groups (64 rows per pass, 128 KB) and a
// quarter at eight (128 rows per pass, 128 KB)
constexpr int MAX_KD = 2048;

// Eight signed bytes (two dwords) -> eight bf16 of their value, exact.
__device__ __forceinline__ bf16x8_t s8x8_to_bf16(unsigned lo, unsigned hi) {
  bf16x8_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (__bf16)(float)(signed char)((lo >> (8 * i)) & 0xffu);
    r[4 + i] = (__bf16)(float)(signed char)((hi >> (8 * i)) & 0xffu);
  }
  return r;
}

__device__ __forceinline__ int clamp_kb(int kb, int kblocks) {
  return kb < kblocks ? kb : kblocks - 1;
}

// aux and entropy of a decode batch from its per-token results, in the
// order of the one-launch router's dispatch: the probabilities of expert e
// summed in 16 strided token subsets (t = w, w + 16, ...), the subsets then
// added in order; aux over the experts lane-wise, then an xor butterfly; the
// entropy terms lane-strided, then a butterfly.  NW waves; `scratch` holds
// at least (MXM_MAX_EXPERTS * 17) words of LDS.
__device__ void decode_aux(const DecodeAux& a, void* scratch) {
  constexpr int SUBSETS = 16;
  int* cnt = static_cast<int*>(scratch);
  float* part = reinterpret_cast<float*>(cnt + MXM_MAX_EXPERTS);  // [SUBSETS][MXM_MAX_EXPERTS]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N, E = a.E, K = a.K, NK = N * K;
  for (int e = tid; e < E; e += NW * 64) cnt[e] = 0;
  __syncthreads();
  for (int sl = tid; sl < NK; sl += NW * 64) atomicAdd(&cnt[a.top_idx[sl]], 1);
  for (int w = wave; w < SUBSETS; w += NW) {
    for (int e = lane; e < E; e += 64) {
      float ps = 0.0f;
      for (int t = w; t < N; t += SUBSETS) ps = ps + a.probs[(size_t)t * E + e];
      part[w * MXM_MAX_EXPERTS + e] = ps;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float aux = 0.0f;
    for (int e = lane; e < E; e += 64) {
      float pm = 0.0f;
      for (int w = 0; w < SUBSETS; ++w) pm = pm + part[w * MXM_MAX_EXPERTS + e];
      const float mean = pm / (float)N;
      const float frac = ((float)cnt[e] / (float)K) / (float)N;
      aux = aux + (a.bf16 ? mxm_rbf(mean) : mean) * frac;
    }
    for (int s = 32; s >= 1; s >>= 1) aux = aux + __shfl_xor(aux, s, 64);
    if (lane == 0) {
      const float raw = aux * (float)E;
      a.aux[0] = raw;
      if (a.aux_scaled) a.aux_scaled[0] = raw * a.aux_weight;
    }
  } else if (wave == 1) {
    float es = 0.0f;
    for (int t = lane; t < N; t += 64) es = es + a.tok_ent[t];
    for (int s = 32; s >= 1; s >>= 1) es = es + __shfl_xor(es, s, 64);
    if (lane == 0) a.entropy[0] = -(es / (float)N);
  }
}

// P: weight blocks in flight per matrix per wave.  RG: groups of 16 rows per
// pass (each weight block, converted once, feeds RG MFMA row groups).
// TOPK (decode batches, GemmArgs::top_idx): the up projection's workgroups
// find their expert's rows themselves from the top-k picks -- the slots on
// the expert, tokens ascending (the stable permutation's order), at offset =
// the number of slots on lower experts -- so they do not wait for a
// dispatch; the expert's first workgroup hands the offset, the count and
// each row's token-major y row (n * K + j, j the expert's place among the
// token's experts in ascending order) to the down projection, which reads
// them as the dispatch's offsets would be read and stores y token-major.
// W16: bf16 weights (2 KB blocks, two 16-byte pieces per lane).  CPW: 16-column
// blocks per wave (int8: two adjacent blocks share each A fragment and halve
// the workgroups, whose fixed costs -- start, row scan, staging, ring fill --
// then weigh half as much; the arithmetic of every column is unchanged).
// (one row group with two column blocks: four waves per SIMD, i.e. two
// workgroups per CU, as the one-block kernel reaches by itself)
template <int EPI, int P, int RG, bool TOPK, bool W16, int CPW>
__global__ __launch_bounds__(NW * 64, (CPW == 2 && RG == 1) ? 4 : 1) void gemm_q8_kernel(
    GemmArgs a, int groups_per_expert) {
  constexpr int MODE = Epi<EPI>::MODE;
  constexpr int BW = W16 ? 2 : 1;    // bytes per weight
  constexpr int NPC = W16 ? 2 : 1;   // 16-byte pieces per lane per block
  static_assert(CPW == 1 || CPW == 2, "one or two column blocks per wave");
  constexpr bool H_SPLIT = Epi<EPI>::H_SPLIT;        // up: store H as hi | lo planes
  // down over both planes of a split H: row group 2p + plane holds rows
  // 16p .. 16p+15 of the pass from that plane; y fp32
  constexpr bool DOWN_SPLIT = Epi<EPI>::DOWN_SPLIT;
  static_assert(!DOWN_SPLIT || RG == 2 || RG == 4, "the split down projection stages both planes");
  constexpr int ROWS_PER_PASS = DOWN_SPLIT ? 8 * RG : 16 * RG;
  constexpr int NMAT = (MODE == MXM_GEMM_GLU) ? 2 : 1;
  constexpr int MAXK = RG >= 8 ? MAX_KD / 4 : RG >= 4 ? MAX_KD / 2 : MAX_KD;
  constexpr int ASZ = MAXK / 64 * 2 * 64;  // pieces of one row group
  constexpr int CH = MAXK / 64 / P * P;    // k blocks per staged chunk
  // A rows of the current pass, per row group: [kb][half][lane] 16-byte
  // pieces; lane 16g + m holds row m, k = 64kb + 16g + 8*half .. +7.
  __shared__ u32x4_t ash[RG * ASZ];
  // TOPK: the expert's rows (their tokens) and, for the down projection,
  // each row's token-major y row
  constexpr bool SCAN = TOPK && MODE != MXM_GEMM_DOWN;  // rows from the picks
  __shared__ int s_tok[SCAN ? MXM_SMALL_BATCH : 1];
  __shared__ int s_ypos[TOPK ? MXM_SMALL_BATCH : 1];
  __shared__ int s_wc[NW], s_wl[NW];
  static_assert((int)sizeof(ash) >= MXM_MAX_EXPERTS * 17 * 4, "decode_aux scratch");

  if (TOPK && a.daux.aux && (int)blockIdx.x == a.E * groups_per_expert) {
    decode_aux(a.daux, ash);  // the launch's extra workgroup
    return;
  }
  const int e = blockIdx.x / groups_per_expert;
  const int grp = blockIdx.x % groups_per_expert;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int row_begin = 0, count = 0;
  int tk0 = -1;  // SCAN: this thread's first slot, requested before the weights
  if constexpr (SCAN) {
    if (tid < a.rows_total) tk0 = a.top_idx[tid];
  } else if constexpr (TOPK) {
    // the up projection's handoff
    row_begin = a.offsets[e];
    count = a.tk_counts[e];
    if (count <= 0) return;
  } else {
    row_begin = a.offsets[e];
    count = a.offsets[e + 1] - row_begin;
    if (count <= 0) return;
  }
  const int Kd = a.Kd, NC = a.Ncols;  // NC: output columns per matrix
  const int kblocks = Kd / 64;
  const size_t kstride = (size_t)NC * 64 * BW;  // bytes between k blocks of one column block
  // rows are staged in chunks: all of Kd when it fits the LDS, else chunks of
  // CH k blocks (a multiple of the ring depth, so every chunk starts on ring
  // slot 0); the weight ring runs on across chunk boundaries
  const int chunk = kblocks <= MAXK / 64 ? kblocks : CH;
  const int ncb = NC / 16;
  const int cb0 = (grp * NW + wave) * CPW;  // this wave's first column block
  const bool active = cb0 < ncb;             // wave-uniform
  const int g = lane >> 4, m = lane & 15;

  // (a second column block past the matrix reads the first's weights and is
  // not stored)
  const uint8_t* W[NMAT][CPW];
  float sc[NMAT][CPW];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt) {
    const void* base = (mt == 0) ? a.b0 : a.b1;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int cbj = active ? min(cb0 + j, ncb - 1) : 0;
      W[mt][j] = static_cast<const uint8_t*>(base) + (size_t)e * NC * Kd * BW +
                 (size_t)cbj * 1024 * BW + 16 * lane;
      if constexpr (W16)
        sc[mt][j] = 1.0f;
      else
        sc[mt][j] = active ? ((mt == 0) ? a.scale0 : a.scale1)[(size_t)e * NC + cbj * 16 + m]
                           : 0.0f;
    }
  }
  const uint16_t* X = static_cast<const uint16_t*>(a.a);
  const size_t ldx = DOWN_SPLIT ? 2 * (size_t)Kd : (size_t)Kd;  // A row stride

  u32x4_t wb[P][NMAT][CPW][NPC];
  auto wload = [&](int s, int kbl) {
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int j = 0; j < CPW; ++j)
#pragma unroll
        for (int h = 0; h < NPC; ++h)
          wb[s][mt][j][h] = MXM_WLD(W[mt][j] + (size_t)kbl * kstride + 1024 * h);
  };
  auto prologue = [&]() {
#pragma unroll
    for (int s = 0; s < P; ++s) wload(s, clamp_kb(s, kblocks));
  };
  // the first blocks of the weight stream are requested before the rows are
  // staged, so HBM is busy from the workgroup's start (TOPK: when most experts
  // have rows, i.e. at least two slots per expert on average; else after the
  // expert's row count is known, so that experts without rows read nothing)
  const bool early = !SCAN || a.rows_total >= 2 * a.E;
  if (early && active) prologue();
  if constexpr (TOPK && !SCAN) {
    for (int i = tid; i < count; i += NW * 64) s_ypos[i] = a.tk_ypos[row_begin + i];
    // (ordered before the epilogue by the staging barriers)
  }
  if constexpr (SCAN) {
    // the slots on expert e, in slot order (= tokens ascending: a token's
    // picks are distinct), by wave ballots; `less` counts the slots on lower
    // experts
    const int NK = a.rows_total, Kt = a.topk;
    int less = 0, base = 0;
    for (int c0 = 0; c0 < NK; c0 += NW * 64) {
      const int sl = c0 + tid;
      const int ex = c0 == 0 ? tk0 : (sl < NK ? a.top_idx[sl] : -1);
      const bool lower = ex >= 0 && ex < e;
      less += lower ? 1 : 0;
      const bool hit = ex == e;
      const unsigned long long bal = __ballot(hit);
      // the down projection's y row n * K + j, j = the token's picks below e:
      // when K divides 64 a token's K slots are lanes of one wave
      const unsigned long long low = __ballot(lower);
      if (lane == 0) s_wc[wave] = __popcll(bal);
      __syncthreads();
      int before = 0, tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int v = s_wc[w];
        before += w < wave ? v : 0;
        tot += v;
      }
      if (hit) {
        const int r = base + before + __popcll(bal & ((1ull << lane) - 1ull));
        const int n = sl / Kt;
        s_tok[r] = n;
        if (grp == 0) {  // (the expert's first workgroup hands the y rows on)
          int j = 0;
          if (64 % Kt == 0) {
            const int l0 = lane - sl % Kt;  // the token's first slot's lane
            const unsigned long long tm = Kt == 64 ? ~0ull : ((1ull << Kt) - 1ull) << l0;
            j = __popcll(low & tm);
          } else {
            for (int k = 0; k < Kt; ++k) j += a.top_idx[(size_t)n * Kt + k] < e ? 1 : 0;
          }
          s_ypos[r] = n * Kt + j;
        }
      }
      base += tot;
      __syncthreads();  // s_wc is reused
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) less += __shfl_xor(less, sh, 64);
    if (lane == 0) s_wl[wave] = less;
    __syncthreads();
    row_begin = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) row_begin += s_wl[w];
    count = base;
    if (grp == 0) {
      // the handoff to the down projection (read after this launch ends)
      if (tid == 0) {
        a.tk_offsets[e] = row_begin;
        a.tk_counts[e] = count;
      }
      for (int i = tid; i < count; i += NW * 64) a.tk_ypos[row_begin + i] = s_ypos[i];
    }
    if (count <= 0) return;
    if (!early && active) prologue();
  }

  for (int rc = 0; rc < count; rc += ROWS_PER_PASS) {
    if (active && rc > 0) prologue();

    f32x4_t acc[RG][NMAT][CPW];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int j = 0; j < CPW; ++j) acc[rg][mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    for (int k0 = 0; k0 < kblocks; k0 += chunk) {
    const int k1 = min(k0 + chunk, kblocks);
    const int pieces = (k1 - k0) * 8;  // 16-byte pieces of a row's chunk
    __syncthreads();  // every wave has finished reading ash
    for (int i = tid; i < 16 * RG * pieces; i += NW * 64) {
      const int r = i / pieces, c8 = i - r * pieces;
      // staged row r: row group r / 16 (when split: rows 16 (r / 32) .. +15
      // of the pass from plane (r / 16) % 2), row r % 16
      const int rr = DOWN_SPLIT ? ((r >> 5) << 4) | (r & 15) : r;
      const int col0 = (DOWN_SPLIT ? ((r >> 4) & 1) * Kd : 0) + 64 * k0;
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (rc + rr < count) {
        const int p = row_begin + rc + rr;
        const int src = (MODE == MXM_GEMM_DOWN) ? p : TOPK ? s_tok[rc + rr] : a.perm[p];
        v = *reinterpret_cast<const u32x4_t*>(X + (size_t)src * ldx + col0 + 8 * c8);
      }
      ash[(r >> 4) * ASZ + ((c8 >> 3) * 2 + (c8 & 1)) * 64 + ((c8 >> 1) & 3) * 16 + (r & 15)] = v;
    }
    __syncthreads();
    if (!active) continue;

// (up to four row groups: every row group's A fragments first, then each
// matrix's converted block against all of them; eight: one row group's
// fragments at a time against both matrices' blocks, which keeps a quarter
// of the A registers live.  Each accumulator sees the same MFMAs in the same
// order either way.)
#define MXM_Q8_STEP(s, kbi)                                                                  \
  if constexpr (RG <= 4) {                                                                   \
    bf16x8_t a0[RG], a1[RG];                                                                 \
    _Pragma("unroll") for (int rg = 0; rg < RG; ++rg) {                                      \
      a0[rg] = __builtin_bit_cast(bf16x8_t, ash[rg * ASZ + ((kbi) * 2 + 0) * 64 + lane]);    \
      a1[rg] = __builtin_bit_cast(bf16x8_t, ash[rg * ASZ + ((kbi) * 2 + 1) * 64 + lane]);    \
    }                                                                                        \
    _Pragma("unroll") for (int mt = 0; mt < NMAT; ++mt)                                      \
    _Pragma("unroll") for (int j = 0; j < CPW; ++j) {                                        \
      const bf16x8_t b0 = W16 ? __builtin_bit_cast(bf16x8_t, wb[s][mt][j][0])                \
                              : s8x8_to_bf16(wb[s][mt][j][0].x, wb[s][mt][j][0].y);          \
      const bf16x8_t b1 = W16 ? __builtin_bit_cast(bf16x8_t, wb[s][mt][j][NPC - 1])          \
                              : s8x8_to_bf16(wb[s][mt][j][0].z, wb[s][mt][j][0].w);          \
      _Pragma("unroll") for (int rg = 0; rg < RG; ++rg) {                                    \
        acc[rg][mt][j] =                                                                     \
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[rg], b0, acc[rg][mt][j], 0, 0, 0);    \
        acc[rg][mt][j] =                                                                     \
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[rg], b1, acc[rg][mt][j], 0, 0, 0);    \
      }                                                                                      \
    }                                                                                        \
  } else {                                                                                   \
    bf16x8_t b0[NMAT][CPW], b1[NMAT][CPW];                                                   \
    _Pragma("unroll") for (int mt = 0; mt < NMAT; ++mt)                                      \
    _Pragma("unroll") for (int j = 0; j < CPW; ++j) {                                        \
      b0[mt][j] = W16 ? __builtin_bit_cast(bf16x8_t, wb[s][mt][j][0])                        \
                      : s8x8_to_bf16(wb[s][mt][j][0].x, wb[s][mt][j][0].y);                  \
      b1[mt][j] = W16 ? __builtin_bit_cast(bf16x8_t, wb[s][mt][j][NPC - 1])                  \
                      : s8x8_to_bf16(wb[s][mt][j][0].z, wb[s][mt][j][0].w);                  \
    }                                                                                        \
    _Pragma("unroll") for (int rg = 0; rg < RG; ++rg) {                                      \
      const bf16x8_t a0 =                                                                    \
          __builtin_bit_cast(bf16x8_t, ash[rg * ASZ + ((kbi) * 2 + 0) * 64 + lane]);         \
      const bf16x8_t a1 =                                                                    \
          __builtin_bit_cast(bf16x8_t, ash[rg * ASZ + ((kbi) * 2 + 1) * 64 + lane]);         \
      _Pragma("unroll") for (int mt = 0; mt < NMAT; ++mt)                                    \
      _Pragma("unroll") for (int j = 0; j < CPW; ++j) {                                      \
        acc[rg][mt][j] =                                                                     \
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0[mt][j], acc[rg][mt][j], 0, 0, 0); \
        acc[rg][mt][j] =                                                                     \
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[mt][j], acc[rg][mt][j], 0, 0, 0); \
      }                                                                                      \
    }                                                                                        \
  }

    int kb = k0;
    for (; kb + P < k1; kb += P) {
#pragma unroll
      for (int s = 0; s < P; ++s) {
        MXM_Q8_STEP(s, kb + s - k0);
        wload(s, clamp_kb(kb + P + s, kblocks));
      }
    }
    // the chunk's last group; its slots take the next chunk's first blocks
#pragma unroll
    for (int s = 0; s < P; ++s)
      if (kb + s < k1) {
        MXM_Q8_STEP(s, kb + s - k0);
        if (k1 < kblocks) wload(s, clamp_kb(kb + P + s, kblocks));
      }
    }  // k chunks
    if (!active) continue;
#undef MXM_Q8_STEP

    // 16x16 layout: lane l holds column l%16, rows 4*(l/16) + i.
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
    if (cb0 + j >= ncb) continue;  // (wave-uniform)
    const int c = (cb0 + j) * 16 + m;
    if constexpr (DOWN_SPLIT) {
#pragma unroll
      for (int pg = 0; pg < RG / 2; ++pg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rc + 16 * pg + 4 * g + i;
        if (r >= count) continue;
        const int h0 = 2 * pg, l0 = 2 * pg + 1;  // the hi and lo planes' row groups
        const float hi = acc[h0][0][j][i];
        const float lo = acc[l0][0][j][i];
        const int yr = TOPK ? s_ypos[r] : row_begin + r;
        static_cast<float*>(a.out)[(size_t)yr * NC + c] = (hi + lo) * sc[0][j];
      }
      continue;
    }
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rc + 16 * rg + 4 * g + i;
      if (r >= count) continue;
      float v[NMAT];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
        v[mt] = W16 ? acc[rg][mt][j][i] : acc[rg][mt][j][i] * sc[mt][j];
      float out;
      if (MODE == MXM_GEMM_GLU) {
        out = mxm_hidden_fast<true>(Epi<EPI>::ETYPE, Epi<EPI>::ACT, a.slope, mxm_rbf_fast(v[0]),
                               mxm_rbf_fast(v[NMAT - 1]));
      } else if (MODE == MXM_GEMM_MLP) {
        out = mxm_hidden_fast<true>(MXM_EXPERT_MLP, Epi<EPI>::ACT, a.slope, 0.0f, mxm_rbf_fast(v[0]));
      } else {
        out = v[0];
      }
      uint16_t* H = static_cast<uint16_t*>(a.out);
      if constexpr (H_SPLIT) {
        const size_t o = (size_t)(row_begin + r) * (2 * NC) + c;
        const float hi = mxm_rbf_fast(out);
        H[o] = mxm_f2bf_fast(hi);
        H[o + NC] = mxm_f2bf_fast(out - hi);
      } else {
        // (the down projection's y: token-major rows in the TOPK flow)
        const int yr = (TOPK && MODE == MXM_GEMM_DOWN) ? s_ypos[r] : row_begin + r;
        H[(size_t)yr * NC + c] = mxm_f2bf_fast(out);
      }
    }
    }  // column blocks
  }
}

template <int EPI, int P, int RG, bool W16, int CPW>
void launch_q8w(const GemmArgs& a, hipStream_t s) {
  const int ncb = a.Ncols / 16;
  const int gpe = (ncb + NW * CPW - 1) / (NW * CPW);
  if (a.top_idx)
    hipLaunchKernelGGL((gemm_q8_kernel<EPI, P, RG, true, W16, CPW>),
                       dim3(a.E * gpe + (a.daux.aux ? 1 : 0)), dim3(NW * 64), 0, s, a, gpe);
  else
    hipLaunchKernelGGL((gemm_q8_kernel<EPI, P, RG, false, W16, CPW>), dim3(a.E * gpe),
                       dim3(NW * 64), 0, s, a, gpe);
}
// P int8 blocks in flight per matrix, or P16 bf16 blocks
template <int EPI, int P, int P16, int RG>
void launch_q8(const GemmArgs& a, hipStream_t s) {
  if (a.w_bf16)
    launch_q8w<EPI, P16, RG, true, 1>(a, s);
  else if constexpr (RG == 1 && MXM_Q8_CPW == 2 && Epi<EPI>::MODE == MXM_GEMM_DOWN &&
                     !Epi<EPI>::DOWN_SPLIT)
    launch_q8w<EPI, (P + MXM_Q8_CPW_PDIV - 1) / MXM_Q8_CPW_PDIV, RG, false, 2>(a, s);
  else
    launch_q8w<EPI, P, RG, false, 1>(a, s);
}
template <int EPI>
void launch_epi(const GemmArgs& a, hipStream_t s) {
  constexpr bool two = Epi<EPI>::MODE == MXM_GEMM_GLU;
  constexpr int P = two ? MXM_Q8_DEPTH_GLU : MXM_Q8_DEPTH_ONE;
  constexpr int P16 = two ? MXM_D16_DEPTH_GLU : MXM_D16_DEPTH_ONE;
  // 32 rows per pass once an expert averages more than 12 rows, 64 once it
  // averages more than 24 (int8) or 16 (bf16): the weights of an expert with
  // r rows are streamed ceil(r / rows per pass) times; one row group keeps
  // the LDS at 64 KB, two workgroups per CU, and four stage half of the
  // reduction at a time.  The row group a row lands in does not change its
  // arithmetic: results are the same bits at every pass height.  Measured
  // (forwards, 32 against 64 rows per pass): D 2048 / E 64 / K 8 / ffn 1408
  // int8 at N 256 0.271 / 0.238 ms, N 384 0.330 / 0.276, bf16 at N 256 0.449
  // / 0.307, N 384 0.525 / 0.339; the switch at 16 rows measured better for
  // bf16 (N 192: 0.317 against 0.294 ms) and worse for int8 (0.191 against
  // 0.229)
  if (a.rows_total > (a.w_bf16 ? MXM_D16_RG8_MIN : MXM_Q8_RG8_MIN) * a.E)
    launch_q8<EPI, P, P16, 8>(a, s);
  else if (a.rows_total > (a.w_bf16 ? MXM_D16_RG4_MIN : MXM_Q8_RG4_MIN) * a.E)
    launch_q8<EPI, P, P16, 4>(a, s);
  else if (a.rows_total > 12 * a.E)
    launch_q8<EPI, P, P16, 2>(a, s);
  else
    launch_q8<EPI, P, P16, 1>(a, s);
}

// Reorder one int8 matrix src [Kd][C] into the 1 KB block layout of a
// [Kdp][Cp] matrix; entries past the source's rows or columns are 0.
__global__ void shuffle_q8_kernel(const int8_t* __restrict__ src, int Kd, int C, int Kdp, int Cp,
                                  uint8_t* __restrict__ dst) {
  const size_t total = (size_t)Kdp * Cp;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
       o += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = o >> 10;
    const int within = (int)(o & 1023);
    const int l = within >> 4, i = within & 15;
    const int ncb = Cp / 16;
    const int kb = (int)(blk / ncb), cb = (int)(blk % ncb);
    const int k = 64 * kb + 16 * (l >> 4) + i;
    const int c = 16 * cb + (l & 15);
    const int8_t q = (k < Kd && c < C) ? src[(size_t)k * C + c] : (int8_t)0;
    dst[o] = (uint8_t)q;
  }
}

}  // namespace


void mxm_launch_gemm_q8(const GemmArgs& a, hipStream_t s) {
  if (a.mode == MXM_GEMM_DOWN) {
    // split: 16 rows per pass from both planes, 32 once an expert averages
    // more than 12 rows (bf16) or 40 (int8), bit-identical.  Measured
    // (geglu, forwards, 16 against 32 rows per pass): D 2048 / E 64 / K 8 /
    // ffn 1408 bf16 at N 128 0.318 / 0.284 ms, N 384 0.542 / 0.444; int8 at
    // N 256 0.306 / 0.312, N 384 0.377 / 0.364; D 512 / E 8 / K 2 / ffn 2048
    // int8 at N 128 0.068 / 0.076, N 192 0.084 / 0.080
    if (a.h_split &&
        a.rows_total > (a.w_bf16 ? MXM_SPLIT_RG4_MIN : MXM_SPLIT_Q8_RG4_MIN) * a.E)
      launch_q8<EPI_DOWN_F32, MXM_Q8_DEPTH_ONE, MXM_D16_DEPTH_ONE, 4>(a, s);
    else if (a.h_split)
      launch_q8<EPI_DOWN_F32, MXM_Q8_DEPTH_ONE, MXM_D16_DEPTH_ONE, 2>(a, s);
    else
      launch_epi<EPI_DOWN>(a, s);
    return;
  }
  switch (mxm_epi_kind(a.expert_type, a.activation)) {
    case EPI_GEGLU:
      launch_epi<EPI_GEGLU>(a, s);
      break;
    case EPI_MLP_SILU:
      launch_epi<EPI_MLP_SILU>(a, s);
      break;
    case EPI_MLP_GELU:
      launch_epi<EPI_MLP_GELU>(a, s);
      break;
    case EPI_MLP_RELU:
      launch_epi<EPI_MLP_RELU>(a, s);
      break;
    case EPI_MLP_LEAKY:
      launch_epi<EPI_MLP_LEAKY>(a, s);
      break;
    default:
      launch_epi<EPI_SWIGLU>(a, s);
      break;
  }
}

void mxm_launch_shuffle_q8(const int8_t* src, int Kd, int C, int Kdp, int Cp, uint8_t* dst,
                           hipStream_t s) {
  const size_t total = (size_t)Kdp * Cp;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 65536) blocks = 65536;
  if (blocks > 0)
    hipLaunchKernelGGL(shuffle_q8_kernel, dim3(blocks), dim3(256), 0, s, src, Kd, C, Kdp, Cp, dst);
}
