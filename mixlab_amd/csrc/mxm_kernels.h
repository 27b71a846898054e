// Launchers of the libmixmoe kernels (one HIP stream per call).  Host code in
// mxm_abi.cpp owns every buffer; these structs carry raw device pointers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxm_numerics.h"

// Tokens per router tile; the dispatch bitmasks are two 32-bit words per
// expert and tile, so this is fixed at 64.
#define MXM_ROUTER_TM 64
// Largest expert count the router supports (4 experts per lane).
#define MXM_MAX_EXPERTS 256

// Value of v held by lane (lane ^ s) of the wave, s in {1, 2, 4, 8, 16, 32}
// (a compile-time constant after unrolling).  Cross-lane moves on the VALU:
// DPP quad permutes (1, 2), row shifts under bank masks (4), a row rotate
// (8), and gfx950's permlane16/permlane32 swaps (16, 32) -- no LDS round
// trip, unlike ds_bpermute.  Every lane of the wave must be active.
__device__ __forceinline__ uint32_t mxm_xor_lane(uint32_t v, int s) {
  const int lane = threadIdx.x & 63;
  switch (s) {
    case 1:
      return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    case 2:
      return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    case 4: {
      const uint32_t r = __builtin_amdgcn_update_dpp(0u, v, 0x104, 0xf, 0x5, false);  // row_shl:4
      return __builtin_amdgcn_update_dpp(r, v, 0x114, 0xf, 0xa, false);              // row_shr:4
    }
    case 8:
      return __builtin_amdgcn_update_dpp(0u, v, 0x128, 0xf, 0xf, false);  // row_ror:8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
  }
}
__device__ __forceinline__ float mxm_xor_lane_f(float v, int s) {
  return __builtin_bit_cast(float, mxm_xor_lane(__builtin_bit_cast(uint32_t, v), s));
}
__device__ __forceinline__ int mxm_xor_lane_i(int v, int s) {
  return (int)mxm_xor_lane((uint32_t)v, s);
}

struct RouterArgs {
  const void* x;   // [N, D], bf16 bits or fp32
  const void* wr;  // [D, E], same dtype
  int N, D, E, K;
  int32_t* top_idx;      // [N, K]
  float* gates;          // [N, K]
  int32_t* slot_rank;    // [N, K] rank of the slot among the tile's tokens on that expert
  int32_t* tile_counts;  // [E, ntiles]
  float* tile_psum;      // [E, ntiles] sum of probabilities over the tile
  float* tile_ent;       // [ntiles] sum over the tile of sum_e p log max(p, 1e-12)
  float* probs_out;      // optional [N, E]
  // optional: router_w lane-interleaved as RouteSmallArgs::wr_t (ldw a
  // multiple of 64 >= D); for E > 32 the logits then run on the fp32 matrix
  // cores (same bits)
  const void* wr_t;
  int ldw;
};
void mxm_launch_router(const RouterArgs& a, bool bf16, hipStream_t s);

// Decode-sized batches (N <= MXM_SMALL_BATCH, N*K <= MXM_SMALL_SLOTS,
// D <= MXM_SMALL_D) route in one launch: a workgroup per token computes its
// logits, softmax, top-k and gates, and the last workgroup to finish (an
// atomic ticket) computes counts, offsets, row-tile prefixes, the stable
// permutation, aux and entropy -- the work of the router, scan and scatter
// kernels of larger batches.
#define MXM_SMALL_BATCH 1024
#define MXM_SMALL_SLOTS 16384
#define MXM_SMALL_D 16384
struct RouteSmallArgs {
  const void* x;       // [N, D], bf16 bits or fp32
  const void* wr_t;    // the flow's dtype, [ceil(E/64)][ldw/P][64][P] with P = 16 bytes
                       // of it (4 fp32, 8 bf16): element (g, c, l, q) =
                       // router_w[Pc + q][64g + l], zero past D or E
  int ldw;             // D rounded up to a multiple of MXM_LOGIT_CHUNK
  int N, D, E, K;
  int bm1, bm2;        // row-tile heights of the two grouped GEMMs
  int32_t* top_idx;    // [N, K]
  float* gates;        // [N, K]
  float* probs;        // [N, E] probabilities (the caller's copy, or scratch)
  float* tok_ent;      // [N] per-token sum_e p log max(p, 1e-12)
  int32_t* counts;     // [E]
  int32_t* offsets;    // [E + 1]
  int32_t* mstart1;    // [E + 1]
  int32_t* mstart2;    // [E + 1]
  int32_t* perm;       // [N*K]
  int32_t* slot_pos;   // [N*K]
  float* aux;          // [1]
  float* entropy;      // [1]
  float aux_weight;
  float* aux_scaled;   // [1] or null
  int32_t* ticket;     // [1], zero between calls (the last workgroup resets it)
  // false: only the per-token results (top_idx, gates, probs, tok_ent); the
  // dispatch (counts .. slot_pos, aux, entropy) is left to
  // mxm_launch_route_dispatch and the int8 decode flow's own kernels
  bool dispatch;
};
bool mxm_route_small_fits(int N, int D, int E, int K);
void mxm_launch_route_small(const RouteSmallArgs& a, bool bf16, hipStream_t s);
// The dispatch of route_small_kernel's last workgroup as a launch of its own
// (one workgroup) from the per-token results already written.
void mxm_launch_route_dispatch(const RouteSmallArgs& a, bool bf16, hipStream_t s);

struct ScanArgs {
  const int32_t* tile_counts;  // [E, ntiles]
  const float* tile_psum;      // [E, ntiles]
  const float* tile_ent;       // [ntiles]
  int N, E, K, ntiles;
  int bm1, bm2;         // row-tile heights of the two grouped GEMMs
  int32_t* counts;      // [E]
  int32_t* offsets;     // [E + 1]
  int32_t* tile_base;   // [E, ntiles] first position of the tile's rows on e, relative to offsets[e]
  int32_t* mstart1;     // [E + 1] prefix of ceil(counts / bm1)
  int32_t* mstart2;     // [E + 1] prefix of ceil(counts / bm2)
  float* aux;           // [1]
  float* entropy;       // [1]
  float aux_weight;     // block level: aux_scaled = aux * aux_weight
  float* aux_scaled;    // [1] or null
  int32_t* expert_count;  // [E] scratch: each workgroup's expert total
  float* expert_pmean;    // [E] scratch: each workgroup's mean probability
  int32_t* ticket;        // [1], zero between calls (the last workgroup resets it)
};
void mxm_launch_scan(const ScanArgs& a, bool bf16, hipStream_t s);

struct ScatterArgs {
  const int32_t* top_idx;
  const int32_t* slot_rank;
  const int32_t* tile_base;  // relative to offsets[e]
  const int32_t* offsets;
  int N, K, ntiles;
  int32_t* perm;      // [N*K] permuted position -> token
  int32_t* slot_pos;  // [N*K] slot (n, k) -> permuted position
};
void mxm_launch_scatter(const ScatterArgs& a, hipStream_t s);

// aux and entropy of a decode batch from its per-token results (the int8
// decode flow computes them in one more workgroup of its gate+up launch).
struct DecodeAux {
  const int32_t* top_idx;  // [N, K]
  const float* probs;      // [N, E]
  const float* tok_ent;    // [N] sum_e p log max(p, 1e-12) per token
  int N, E, K;
  bool bf16;               // the bf16 flow (the mean probabilities rounded to bf16)
  float* aux;              // [1]; null: not computed
  float* entropy;          // [1]
  float aux_weight;
  float* aux_scaled;       // [1] or null
};

// Grouped expert FFN.  mode: 0 = gate+up with GLU epilogue, 1 = up with MLP
// activation, 2 = down projection.
enum { MXM_GEMM_GLU = 0, MXM_GEMM_MLP = 1, MXM_GEMM_DOWN = 2 };

struct GemmArgs {
  int mode;
  const void* a;          // mode 0/1: x [N, Kd]; mode 2: H [N*K, Kd]
  const int32_t* perm;    // mode 0/1: permuted position -> token
  const void* b0;         // weights, layout depends on the kernel family
  const void* b1;         // second weight (SIMT GLU up-projection)
  const float* scale0;    // int8 weights: per-output-channel scales
  const float* scale1;
  void* out;              // mode 0/1: H [N*K, F]; mode 2: Y [N*K, D]
  void* out2;             // MFMA up projections: if set, the raw bf16 projections too,
                          // [N*K, Ncols] in W1's column order (the backward's G|U);
                          // SIMT MLP up projection: the raw fp32 projections, rows
                          // ld2 apart (out may then be null: no hidden stored)
  int ld2;
  const int32_t* offsets; // [E + 1]
  const int32_t* mstart;  // [E + 1]
  int E, Kd, Ncols;       // reduction length, output columns (per matrix)
  int max_mtiles;         // grid bound on row tiles
  int expert_type, activation;
  float slope;
  bool y_bf16;            // SIMT down: round y to bf16
  int family;             // MFMA tile family (MXM_TILE_*), MXM_TILE_AUTO picks
  int simt_bm;            // SIMT family: tile height and width, 64 (0 too) or 32
  int simt_vec;           // SIMT family: 1 keeps the 64 x 64 tile's products on the
                          // vector unit (0: the fp32 matrix cores, same bits)
  int rows_total;         // N*K routed rows (int8 family: picks rows per pass)
  // Split hidden (MFMA and int8 families, kinds whose hidden is fp32 in the
  // bf16 flow, !mxm_hidden_is_bf16): the up GEMM stores each fp32 hidden
  // value h as two bf16 planes of H [rows][2F], hi = bf16(h) in columns
  // 0..F-1 and lo = bf16(h - hi) in F..2F-1, and the down GEMM (h_split)
  // reduces over both planes (Kd = 2F for the MFMA family, W_down's k index
  // wrapping at F) and stores y in fp32 -- the fp32 matmul of the reference
  // to within 2^-16 relative, since bf16 x bf16 products are exact in fp32.
  bool h_split;
  // MFMA down projections: gather the A rows through perm (as the up
  // projections do) instead of reading them in slot order
  bool gather_a;
  // set by the MFMA launcher: every A row lies within 4 GiB of a (rows_total
  // * Kd bf16 bound it), so A loads take 32-bit byte offsets ...
  bool a_off32;
  // ... unless the caller forbids it (64-bit addressing throughout)
  bool no_off32;
  // MFMA mode 2 (MXM_GEMM_DOWN): store the fp32 accumulators as they are,
  // out [rows][Ncols] fp32 (the products of the fp32 backward, each an
  // A . B^T over bf16 planes concatenated along k)
  bool f32_out;
  // decode kernels (mxm_launch_gemm_q8): the weights are bf16 in the 2 KB
  // block layout of mxm_launch_shuffle_bf16, without scales (bf16 ops at
  // decode sizes), instead of int8 with scale0 / scale1
  bool w_bf16;
  // int8 family, decode batches (N <= MXM_SMALL_BATCH): if set, the kernels
  // take each expert's rows from the top-k picks [rows_total = N * topk]
  // instead of offsets / perm (H at the same offsets as the dispatch's), and
  // the down projection stores y token-major, row n * topk + j for the j-th
  // smallest of token n's experts
  const int32_t* top_idx;
  int topk;
  // the up projection's handoff to the down projection in that flow: each
  // expert's first row (tk_offsets, the down projection reads it as
  // `offsets`), row count and the token-major y row of each of its rows
  int32_t* tk_offsets;  // [E]
  int32_t* tk_counts;   // [E]
  int32_t* tk_ypos;     // [N * topk]
  // ... and with daux.aux set, the up projection's launch has one more
  // workgroup that computes aux and entropy
  DecodeAux daux;
};
// SIMT family: weights in the reference layout (x . W, [in, out]) per expert,
// fp32 storage; H and Y are fp32.  Accumulation is fmaf in ascending k.
void mxm_launch_gemm_simt(const GemmArgs& a, bool bf16, hipStream_t s);
// MFMA family: bf16 weights stored transposed ([out, in]); GLU gate/up rows
// interleaved in groups of 32; H and Y are bf16 (split hidden: H is the two
// planes and Y fp32, see GemmArgs::h_split).
void mxm_launch_gemm_mfma(const GemmArgs& a, hipStream_t s);
enum { MXM_TILE_AUTO = 0, MXM_TILE_128x128 = 1, MXM_TILE_256x128 = 2, MXM_TILE_256x256 = 3 };
// Row-tile height the MFMA launcher uses for a GEMM with these dimensions
// (0: the family does not tile them).
int mxm_mfma_tile_rows(int Ncols, int Kd, int family);

// Weight gradients on MFMA (mxm_wgrad.hip): per expert e,
//   out[e][m][c] = sum_p sum_k A[k][p * aplane + m] * B[k][p * bplane + c]   (fp32)
// over rows k = offsets[e] .. offsets[e+1]-1 and planes p < planes.  With
// glu_f > 0 the C columns are GLU-interleaved in groups of 32 (gate, up) and
// land de-interleaved: column c -> out[e] + ((c/32) % 2) * out_slot +
// m * glu_f + (c/64)*32 + c%32; else out[e] + m * C + c.
struct WgradArgs {
  const uint16_t* a;        // bf16 [rows][lda]
  int lda, aplane, planes;
  const uint16_t* b;        // bf16 [rows][ldb]
  int ldb;
  int bplane;               // B's columns of plane p start at p * bplane (0: B is shared)
  const int32_t* offsets;   // [E + 1]
  const uint16_t* zero;     // 256 zero bf16 (rows past an expert's end)
  int E, M, C;
  float* out;
  size_t out_estride;       // floats between experts' outputs
  size_t out_slot;          // floats from the gate matrix to the up matrix (GLU)
  int glu_f;                // F for GLU de-interleaving, else 0
  void* scratch;            // mxm_wgrad_scratch_bytes(M, C): the schedule and split partials
  const int32_t* a_rows;    // if set: A's row for reduction row j is a_rows[j] (else j)
  bool a_rows32;            // with a_rows: all of A lies within 4 GiB of a (32-bit offsets)
  const int32_t* b_rows;    // the same for B (at most one of a_rows, b_rows)
  bool b_rows32;
  // Operands padded past the output's shape (an expert width rounded up to
  // the tiles): only rows m < m_store are stored (0: all M), and without the
  // GLU interleave only columns c < c_store, at row stride c_store instead
  // of C (0: all).  With the interleave, glu_f is the real width: hidden
  // units f >= glu_f are not stored.
  int m_store, c_store;
};
// M and C multiples of 128.
bool mxm_wgrad_fits(int M, int C);
size_t mxm_wgrad_scratch_bytes(int M, int C);
void mxm_launch_wgrad(const WgradArgs& a, hipStream_t s);
// The SIMT family's row-tile height (and tile width) for a launch of `rows`
// routed rows over E experts and ncols output columns: 64, or 32 when the
// 64 x 64 grid would not give every CU a tile.
int mxm_simt_bm(int64_t rows, int E, int ncols, int n_cu);

// Epilogue kinds: the hidden activation (expert type x activation) of the up
// projections, or the plain bf16 store of the down projection.
enum { EPI_SWIGLU, EPI_GEGLU, EPI_MLP_SILU, EPI_MLP_GELU, EPI_MLP_RELU, EPI_MLP_LEAKY, EPI_DOWN,
       EPI_DOWN_F32, EPI_F32 };

// EPI_KEEP + an up-projection kind: the raw bf16 projections to
// GemmArgs::out2 instead of the hidden (the MFMA backward derives H from
// them in its activation pass).
constexpr int EPI_KEEP = 16;
// EPI_SCALE + a kind: the accumulators are multiplied by a per-output-column
// fp32 scale (GemmArgs::scale0, and scale1 for the up matrix of a GLU pair,
// each [E][output columns]) before anything else; the int8 weights' flow on
// the MFMA kernels, whose bf16 weights hold the integers q.
constexpr int EPI_SCALE = 32;

template <int EPI_>
struct Epi {
  static constexpr int EPI = EPI_ & (EPI_KEEP - 1);
  static constexpr bool KEEP_RAW = (EPI_ & EPI_KEEP) != 0;
  static constexpr bool SCALED = (EPI_ & EPI_SCALE) != 0;
  static constexpr int MODE = EPI <= EPI_GEGLU ? MXM_GEMM_GLU
                              : (EPI == EPI_DOWN || EPI == EPI_DOWN_F32 || EPI == EPI_F32)
                                  ? MXM_GEMM_DOWN
                                  : MXM_GEMM_MLP;
  // up projections whose hidden is fp32 in the bf16 flow: H in two planes
  static constexpr bool H_SPLIT = EPI == EPI_GEGLU || EPI == EPI_MLP_GELU || EPI == EPI_MLP_LEAKY;
  // down projection over the two planes, y stored in fp32
  static constexpr bool DOWN_SPLIT = EPI == EPI_DOWN_F32;
  // the accumulators stored in fp32 (the split down projection's y, or a
  // plain product: GemmArgs::f32_out)
  static constexpr bool Y_F32 = EPI == EPI_DOWN_F32 || EPI == EPI_F32;
  static constexpr int ETYPE = EPI == EPI_SWIGLU ? MXM_EXPERT_SWIGLU
                               : EPI == EPI_GEGLU ? MXM_EXPERT_GEGLU
                                                  : MXM_EXPERT_MLP;
  static constexpr int ACT = EPI == EPI_MLP_GELU    ? MXM_ACT_GELU
                             : EPI == EPI_MLP_RELU  ? MXM_ACT_RELU
                             : EPI == EPI_MLP_LEAKY ? MXM_ACT_LEAKY_RELU_SQ
                             : EPI == EPI_GEGLU     ? MXM_ACT_GELU
                                                    : MXM_ACT_SILU;
};

// Epilogue kind of the up-projection GEMM for an (expert type, activation).
inline int mxm_epi_kind(int expert_type, int activation) {
  if (expert_type == MXM_EXPERT_SWIGLU) return EPI_SWIGLU;
  if (expert_type == MXM_EXPERT_GEGLU) return EPI_GEGLU;
  switch (activation) {
    case MXM_ACT_GELU:
      return EPI_MLP_GELU;
    case MXM_ACT_RELU:
      return EPI_MLP_RELU;
    case MXM_ACT_LEAKY_RELU_SQ:
      return EPI_MLP_LEAKY;
    default:
      return EPI_MLP_SILU;
  }
}

struct CombineArgs {
  const void* y;          // [N*K, D], fp32 or bf16
  const int32_t* top_idx; // [N, K]
  const float* gates;     // [N, K]
  const int32_t* slot_pos;
  int N, D, K;
  int ldy;                // y's row stride (0: D; a padded down projection's width)
  float* delta;           // [N, D]
  // Block level (null resid: plain op output): delta[n, d] = resid[n, d] +
  // combined * rscale[d] (or + combined when rscale is null), in fp32.
  const void* resid;      // [N, D], bf16 bits or fp32 (resid_bf16)
  bool resid_bf16;
  const void* rscale;     // [D], bf16 bits or fp32 (rscale_bf16)
  bool rscale_bf16;
};
void mxm_launch_combine(const CombineArgs& a, bool y_bf16, hipStream_t s);
// The int8 decode flow's combine: y token-major (token n's rows n*K ..
// n*K+K-1 in ascending expert id; slot_pos unused).
void mxm_launch_combine_tm(const CombineArgs& a, bool y_bf16, hipStream_t s);

// RMSNorm of gpu/ir.cpp:4949-4960 with a fixed summation order: one wave
// per row; lane l sums x[d]^2 (product rounded, then added) over
// d = 256*i + 4*l + j in (i, j) order, the 64 partial sums meet in an xor
// butterfly (distances 32, 16, ..., 1); ms = sum * inv_d; r = 1 / sqrt(ms +
// eps) (both correctly rounded); y = (x * r) * scale, rounded to the output
// dtype.
struct RmsNormArgs {
  const void* x;          // [N, D]
  bool x_bf16;
  const void* scale;      // [D]
  bool scale_bf16;
  int N, D;
  float eps, inv_d;       // inv_d = (float)(1.0 / D)
  void* out;              // [N, D]
  bool out_bf16;
};
void mxm_launch_rmsnorm(const RmsNormArgs& a, hipStream_t s);

// Weight preparation (run once at upload).
void mxm_launch_to_f32(const void* src, int src_dtype, float* dst, int64_t n, hipStream_t s);
// dst [rows][cols] fp32 = the first cols of each row of src [rows][ld]
// (fp32 or bf16 bits), e.g. a padded down projection's outputs.
void mxm_launch_rows_to_f32(const void* src, int src_dtype, int64_t rows, int cols, int ld,
                            float* dst, hipStream_t s);
// dst [rows][ldd] bf16 = src [rows][cols] (bf16 bits) with columns cols ..
// ldd-1 zero: the rows of x padded to the up projection's reduction length.
void mxm_launch_pad_rows_bf16(const uint16_t* src, int64_t rows, int cols, int ldd, uint16_t* dst,
                              hipStream_t s);
void mxm_launch_to_bf16(const void* src, int src_dtype, uint16_t* dst, int64_t n, hipStream_t s);
// Transposed bf16 copy of one weight matrix src [Kd, C] (x.W layout; fp32,
// bf16 or int8 by src_dtype, an MXM_DTYPE_* value):
// dst[q * ldd + k] = bf16(src[k, c]) with q = c (slot < 0), or, for the GLU
// interleave, q = (c/32)*64 + slot*32 + c%32 with slot 0 = gate, 1 = up;
// ldd = Kd by default (a larger ldd leaves each row's padded tail as it is).
void mxm_launch_transpose_bf16(const void* src, int src_dtype, int Kd, int C, int slot,
                               uint16_t* dst, hipStream_t s, int ldd = 0);
// The decode router's copy of router_w [D, E] (stored in the flow's dtype:
// bf16 when bf16, else fp32), in RouteSmallArgs::wr_t's layout.
void mxm_launch_router_t(const void* src, bool bf16, int D, int E, int ldw, void* dst,
                         hipStream_t s);
// MFMA-family expert weights (padded to Dk x Fk) back to fp32 x.W layout
// [E][D][F] / [E][F][D] (backward of bf16 ops).
void mxm_launch_w1_to_xw(const uint16_t* w1, int E, int D, int F, int Dk, int Fk, int slot,
                         float* dst, hipStream_t s);
void mxm_launch_w2_to_xw(const uint16_t* w2, int E, int D, int F, int Dk, int Fk, float* dst,
                         hipStream_t s);

// int8-weight family (decode shapes): weights in the 1 KB block layout of
// mxm_launch_shuffle_q8, fp32 scale per output channel (scale0/scale1),
// H and Y bf16.  Reduction length Kd must be a multiple of 64 (rows are
// staged in chunks of at most 2048); output columns a multiple of 16.
void mxm_launch_gemm_q8(const GemmArgs& a, hipStream_t s);
// src [Kd][C] int8 -> dst in the 1 KB block layout of a [Kdp][Cp] matrix
// (Kdp a multiple of 64, Cp of 16, both at least the source's): entries
// past the source's rows or columns are 0.
void mxm_launch_shuffle_q8(const int8_t* src, int Kd, int C, int Kdp, int Cp, uint8_t* dst,
                           hipStream_t s);
// src [Kd][C] (fp32 or bf16 by src_dtype, x.W layout) -> bf16 in the decode
// kernels' block layout of a [Kdp][Cp] matrix at 2 bytes per weight: block
// (cb, kb) of 64 k x 16 columns at element ((kb * Cp/16) + cb) * 1024, lane
// l's 16 values W[64kb + 16*(l/16) + i][16cb + l%16], i = 0..15, at elements
// 512*(i/8) + 8*l + i%8 (two halves, each lane's 8 values contiguous in
// each); entries past the source's rows or columns are 0.
void mxm_launch_shuffle_bf16(const void* src, int src_dtype, int Kd, int C, int Kdp, int Cp,
                             uint16_t* dst, hipStream_t s);

// Backward of op 74 (fp32 flow).  Uses the routing and probabilities of a
// forward on the same x and the expert outputs Y (the forward's, or under
// fp32 compute the backward's own per-expert products); the projections and
// hidden units are computed again.  All matrices are fp32 in the x.W layout
// of the forward's SIMT family.
struct BackwardArgs {
  int N, D, E, K, F, etype, act, wpe;
  float slope;
  // forward state
  const float* x;            // [N, D]
  const int32_t* top_idx;    // [N, K]
  const float* gates;        // [N, K]
  const int32_t* slot_pos;   // [N*K]
  const int32_t* perm;       // [N*K]
  const int32_t* counts;     // [E]
  const int32_t* offsets;    // [E + 1]
  const float* probs;        // [N, E]
  const float* Y;            // [N*K, D]
  // bf16 flow: x and Y as the forward holds them (bf16); when set, the router
  // part reads these instead of x and Y
  const uint16_t* xb16;      // [N, D]
  const uint16_t* Yb16;      // [N*K, D]
  const float* wr;           // [D, E]
  const float* w1;           // [E][D][F] gate (GLU) or up (MLP)
  const float* w1b;          // [E][D][F] up (GLU)
  const float* w2;           // [E][F][D] down
  // upstream gradients
  const float* d_delta;      // [N, D]
  float d_aux, d_ent;
  // scratch
  float* dy;                 // [N*K, D]: dY = gate * dD by slot position
  const float* dgp;          // [N*K] gate gradients by slot position (set: the caller computed
                             // them; dgates is then not used)
  float *dgates, *dlogits, *dxr;                          // [N*K], [N, E], [N, D] (dxr unset:
                                                          // the caller fuses dx's router term)
  uint16_t* dyb16;           // [N*K, D]: when set, dY is written here in bf16 instead of dy
  float* wrt;                                             // router_w transposed [E][D]
  int32_t* one;                                           // [4]: offsets/mstart of one segment
  float* wr_part;            // [wgrad_router_chunks(N, D, E)][D][E]: row-chunk partials of d router_w
  bool dwr_by_caller;        // set: the caller computes d router_w (wr_part is not used)
  // outputs
  float* dx;                 // [N, D]
  float* dwr;                // [D, E]
  float* dw;                 // per expert, Op.Inputs order, x.W layout
};
// Row chunks of d router_w's reduction (BackwardArgs::wr_part holds one D x E
// partial per chunk).
int wgrad_router_chunks(int N, int D, int E);
// The router part: gate/router gradients, dY, dx's router term and d router_w.
void mxm_launch_backward_router(const BackwardArgs& a, hipStream_t s);
// bf16 flow on the MFMA family (products by the MFMA grouped GEMM, weight
// gradients by mxm_launch_wgrad): dx from bf16 expert input gradients.
void mxm_launch_dx_bf16(const float* dxr, const uint16_t* dxe, const int32_t* slot_pos, int N,
                        int D, int K, float* dx, hipStream_t s);
// dx = dlogits . Wr^T (wrt = Wr^T [E][D]) + the bf16 expert input gradients
// summed over each token's slots; D % 4 == 0 and 16-byte aligned rows.
void mxm_launch_dx_fused_bf16(const float* dlogits, const float* wrt, int E, const uint16_t* dxe,
                              const int32_t* slot_pos, int N, int D, int K, float* dx,
                              hipStream_t s);
// d router_w on the weight-gradient kernel: dlogits [N][E] as bf16 halves
// hi = bf16(dl), lo = bf16(dl - hi) in out [N][2 Ep] (hi at column e, lo at
// Ep + e, zeros for e >= E; Ep = E rounded up to 64), so that x^T out holds
// x^T hi and x^T lo side by side ...
void mxm_launch_dl_split_bf16(const float* dl, int N, int E, int Ep, uint16_t* out, hipStream_t s);
// ... and dwr[d][e] = t[d][e] + t[d][Ep + e] from that product t [D][2 Ep].
void mxm_launch_dwr_halves(const float* t, int D, int E, int Ep, float* dwr, hipStream_t s);
// bf16 MFMA backward without the forward's down projection: per token,
// ddb[n] = bf16(dD[n]) and, per slot s at position p = slot_pos[s],
// gp[p] = gates[s] and (if dyb is set) dyb[p] = bf16(gates[s] * dD[n]).
void mxm_launch_dy_gate(const float* dd, const float* gates, const int32_t* slot_pos, int N, int D,
                        int K, uint16_t* ddb, uint16_t* dyb, float* gp, hipStream_t s);
// The hidden H [rows][F] (hi, and lo = bf16(h - hi) after F columns when
// hsplit) from raw bf16 up projections gu [rows][NC] with the up epilogue's
// own activation code: bit for bit what the epilogue would store.
void mxm_launch_hidden_from_raw_bf16(const uint16_t* gu, int rows, int F, int etype, int act,
                                     float slope, bool hsplit, uint16_t* H, hipStream_t s);
// ... then, per routed row p: the hidden h from the forward's raw bf16
// projections gu with the up epilogue's own activation code (bit for bit the
// forward's); the gated hidden gp[p] * h written to Hg (hi, and lo =
// bf16(v - hi) after F columns when hsplit) for dW_down = Hg^T dD over the
// slots' tokens; dH = gp[p] * dhr[p] (dhr = dD W_down^T of the row's token,
// ungated), dG and dU (the activation backward); and the gate gradient
// dgp[p] = <dhr[p], h[p]> with h as the forward stores it (hi + lo when
// hsplit).
void mxm_launch_act_bw_gated_bf16(const uint16_t* gu, const uint16_t* dhr, uint16_t* Hg,
                                  bool hsplit, const float* gp, int rows, int F, int etype, int act,
                                  float slope, uint16_t* dgu, float* dgp, hipStream_t s);
// Row-tile prefix of counts for tile height bm (mstart[0..E]).
void mxm_launch_tile_prefix(const int32_t* counts, int E, int bm, int32_t* mstart, hipStream_t s);

// fp32 products on the bf16 MFMA kernels (the fp32 backward): fp32 values
// as bf16 planes hi = bf16(v), lo = bf16(v - hi), concatenated along k as
// HHL = [hi | hi | lo] (A side) or HLH = [hi | lo | hi] (B side), so that one
// bf16 product gives hi.hi + hi.lo + lo.hi.
// dst [rows][3 ldq]: the planes of src [rows][cols] (row stride lds), zero
// for cols <= c < ldq.
void mxm_launch_planes3(const float* src, int64_t rows, int cols, int lds, int ldq, bool hlh,
                        uint16_t* dst, hipStream_t s);
// The four B operands of the experts' products from fp32 x.W weights (w1 /
// w1b [E][D][F], w2 [E][F][D]), padded to Dq x Fq (NCq = 2 Fq for GLU, GLU
// columns interleaved in groups of 32): w1p [E][NCq][3 Dq] (HLH) for
// G|U = X W1, w1t [E][Dq][3 NCq] (HHL) for dX = dGU W1^T, w2p [E][Dq][3 Fq]
// (HLH) for Y = H W2, w2t [E][Fq][3 Dq] (HHL) for dH = dY W2^T.
void mxm_launch_planes3_weights(const float* w1, const float* w1b, const float* w2, int E, int D,
                                int F, int Dq, int Fq, bool glu, uint16_t* w1p, uint16_t* w1t,
                                uint16_t* w2p, uint16_t* w2t, hipStream_t s);
// H [rows][3 Fq] (HHL) from the raw fp32 projections gu [rows][NC].
void mxm_launch_hidden_planes3(const float* gu, int64_t rows, int Fq, int etype, int act,
                               float slope, uint16_t* h3, hipStream_t s);
// dGU [rows][3 NC] (HLH) from gu and dH [rows][Fq] fp32.
void mxm_launch_act_bw_planes3(const float* gu, const float* dh, int64_t rows, int Fq, int etype,
                               int act, float slope, uint16_t* dgu3, hipStream_t s);
// dx[n] = dxr[n] + sum_k dxe[slot_pos[n, k]] (dxe rows ld apart).
void mxm_launch_dx_sum(const float* dxr, const float* dxe, int ld, const int32_t* slot_pos, int N,
                       int D, int K, float* dx, hipStream_t s);
