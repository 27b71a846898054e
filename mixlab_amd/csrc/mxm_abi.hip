// C ABI of libmixmoe (declared in include/mixmoe.h): handle table, weight
// upload, and the op-74 forward as a sequence of six kernels on one stream.
//
// Mirrors the reference bridge's conventions (gpu/mlx_bridge.cpp): a
// process-global mutex over the handle table (gpu/mlx_bridge.cpp:39-42,105),
// int64 handles with 0 = failure, and an exception fence around every entry
// point (gpu/mlx_bridge.cpp:64-82) that turns failures into status codes and
// a per-thread message.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/mixmoe.h"
#include "mxm_kernels.h"

namespace {

thread_local std::string g_last_error;
std::mutex g_mu;
std::map<int64_t, std::unique_ptr<struct MoeOp>> g_ops;
int64_t g_next_handle = 1;
std::string g_device_name = "uninitialised";

// Failure classes of the bridge's status codes (gpu/mlx_bridge.cpp:814-823):
// an argument the call cannot accept (MXM_ERR_ARGS), a runtime that is not
// initialised (MXM_ERR_INIT); every other failure -- a HIP error, a call out
// of sequence -- is MXM_ERR.
struct ArgError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct InitError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

template <class Ex>
[[noreturn]] void vthrow(const char* fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  throw Ex(buf);
}

// An argument error (shape, dtype, index, size limit, NULL pointer).
[[noreturn]] void fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vthrow<ArgError>(fmt, ap);
}
// A runtime failure or a call out of sequence.
[[noreturn]] void fail_rt(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vthrow<std::runtime_error>(fmt, ap);
}
// The HIP runtime or the device is not (or cannot be) initialised.
[[noreturn]] void fail_init(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vthrow<InitError>(fmt, ap);
}

#define HIPCK(expr)                                                                       \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess)                                                                 \
      fail_rt("HIP error %s at %s:%d", hipGetErrorString(_e), __FILE__, __LINE__);       \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { reset(); }
  void alloc(size_t n) {
    reset();
    if (n == 0) n = 256;
    HIPCK(hipMalloc(&p, n));
    bytes = n;
  }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  template <typename T>
  T* as() const { return static_cast<T*>(p); }
};

// Every device buffer a forward writes besides its outputs.  layout_workspace
// places the pieces at 256-byte aligned offsets from one base; the two
// tickets share the first piece and must be zero between calls (the kernels
// that take them leave them zero).
struct Workspace {
  int32_t* scan_ticket = nullptr;  // [1] scan kernel (N > 1024)
  int32_t* ticket = nullptr;       // [1] one-launch router (decode sizes)
  void* xcast = nullptr;           // [N, D] bf16 copy of fp32 x (bf16 compute)
  int32_t* top_idx = nullptr;      // [N*K]
  float* gates = nullptr;          // [N*K]
  int32_t* slot_rank = nullptr;    // [N*K]
  int32_t* slot_pos = nullptr;     // [N*K]
  int32_t* perm = nullptr;         // [N*K]
  int32_t* tile_counts = nullptr;  // [E, ntiles]
  float* tile_psum = nullptr;      // [E, ntiles]
  float* tile_ent = nullptr;       // [ntiles]
  int32_t* tile_base = nullptr;    // [E, ntiles]
  int32_t* counts = nullptr;       // [E]
  int32_t* offsets = nullptr;      // [E + 1]
  int32_t* mstart1 = nullptr;      // [E + 1]
  int32_t* mstart2 = nullptr;      // [E + 1]
  float* aux = nullptr;            // [1] when the caller passes none
  float* ent = nullptr;            // [1]
  int32_t* expert_count = nullptr; // [E]
  float* expert_pmean = nullptr;   // [E]
  void* xpad = nullptr;            // [N, Kx] bf16 x padded to the up projection's reduction
  void* H = nullptr;               // [N*K, Fk] (split hidden: [N*K, 2Fk])
  void* Y = nullptr;               // [N*K, Dk]
  float* probs = nullptr;          // [N, E] (MXM_FLAG_DEBUG_PROBS)
  float* small_probs = nullptr;    // [N, E] one-launch router's probabilities
  float* tok_ent = nullptr;        // [N]
  size_t bytes = 0;
};

struct MoeOp {
  // op parameters (arch/ir.go:697)
  int B = 0, T = 0, D = 0, E = 0, K = 0, etype = 0, F = 0, act = 0;
  float slope = 0.0f;
  int N = 0, wpe = 0, n_inputs = 0;
  // Widths the expert kernels run at (set at create; equal to F and D on the
  // SIMT family).  The MFMA tiles want the expert width a multiple of 128
  // and the model width a multiple of 128 (down projection's columns) and
  // 64 (up projection's reduction); the int8 kernels want 64 and 16.  Other
  // widths are padded with zero weights: Fk is F rounded up (zero gate / up
  // columns, zero W_down rows: the hidden of a zero projection is 0 for every
  // kind, so y is unchanged), Dk is the down projection's output width (zero
  // W_down columns; y and the combine read D of Dk columns), Kx the up
  // projection's reduction length (D, or Dk when D is not a multiple of 64:
  // x's rows are then copied with zero columns).
  int Fk = 0, Dk = 0, Kx = 0;
  bool bf16 = false, mfma = false, debug_probs = false, q8 = false;
  // MFMA / int8 families with a kind whose hidden is fp32 in the bf16 flow:
  // H holds two bf16 planes [N*K][2F] and Y is fp32 (GemmArgs::h_split)
  bool hsplit = false;
  int family = MXM_TILE_AUTO;
  hipStream_t stream = nullptr;
  int device = 0;  // the device current at create (the stream's)

  // weights.  SIMT family: w1 = gate (GLU) or up (MLP) fp32 [E][D][F], w1b =
  // up (GLU) fp32 [E][D][F], w2 = down fp32 [E][F][D].  MFMA family: w1 =
  // bf16 [E][2F or F][D] (GLU interleaved), w2 = bf16 [E][D][F].
  DevBuf router, w1, w1b, w2;
  // decode-sized batches, and the tiled router's matrix-core logits (E >
  // 32): router_w lane-interleaved (RouteSmallArgs::wr_t)
  bool small_route = false, mf_router = false;
  int ldw = 0;
  DevBuf router_t;
  // int8 family: q1 = gate (GLU) or up (MLP), q1b = up (GLU), q2 = down, in
  // the 1 KB block layout; s1, s1b, s2 = fp32 per-output-channel scales.
  DevBuf q1, q1b, q2, s1, s1b, s2;
  // int8 weights on the MFMA kernels (batches of 96 or more routed rows per
  // expert, which are compute-bound): w1 / w2 hold the
  // integers q as bf16 (exact) in the MFMA layout and s1 / s1b / s2 the
  // scales [E][Fk] / [E][Dk], which the epilogue applies to the fp32
  // accumulators; q1, q1b and q2 are not allocated
  bool q8_mfma = false;
  bool int8_kernels() const { return q8 && !q8_mfma; }
  // bf16 ops at decode sizes (few routed rows per expert): the expert
  // weights also in the decode kernels' block layout at 2 bytes per weight
  // (d1 = gate or up, d1b = up, d2 = down), which the forward streams
  // instead of running the MFMA tiles; the MFMA layout (w1, w2) stays for
  // the backward, whose own forwards keep the tiles
  bool dec16 = false;
  DevBuf d1, d1b, d2;
  int n_cu = 256;        // CUs of the op's device
  int fam1 = 0, fam2 = 0;  // MFMA tile families of the up and down GEMMs
  int fam_dh = 0;           // ... of the backward's dH = dY W_down^T (dX uses fam2)
  std::vector<char> have;

  // tile schedule of the forward (set at create from the op's parameters)
  int ntiles = 0, bm1 = 0, bm2 = 0, max_mtiles1 = 0, max_mtiles2 = 0;
  int simt_tile = 0;  // MXM_SIMT_TILE at creation: the SIMT family's tile (0 picks)
  int simt_vec = 0;   // MXM_SIMT_MFMA=0 at creation: 64 x 64 SIMT tiles on the vector unit
  // the op's own workspace, allocated at the first forward; `last` is the
  // workspace the latest forward used (the op's own, or the device scratch
  // of mxm_moe_forward_noalloc), which the routing queries read
  bool ws_ready = false, have_last = false;
  DevBuf wsbuf;
  Workspace ws, last;
  // the last forward took the int8 decode flow: its dispatch (counts,
  // offsets, perm, slot_pos) is computed when the routing is queried, from
  // its per-token results and the probabilities at last_probs
  bool last_decode = false;
  float* last_probs = nullptr;
  // the int8 decode flow (1, default) or the dispatch of the one-launch
  // router (0): MXM_DECODE_FLOW at creation, for measurements of the two
  bool decode_flow = true;
  DevBuf xn, blk_scales;  // block level: normalised rows; host-call copies of the scales
  DevBuf bw_probs;        // the backward's forward keeps its probabilities here
  // backward (fp32 flow): the experts' projections, gradients and scratch
  bool keep_probs = false, bw_ready = false;
  // set by the fp32 backward around its forward: stop after the routing
  // (router, scan, scatter); the backward computes the experts' products itself
  bool route_only = false;
  bool up_only = false;  // the forward stops after the up projection (MFMA backward)
  // MXM_FLAG_KEEP_FOR_BACKWARD: the last call was an mxm_moe_forward, which
  // kept its own copy of x and (MFMA backward family) its routing,
  // probabilities and raw up projections for mxm_moe_backward_kept
  bool train = false, kept = false;
  DevBuf kept_xbuf;
  int kept_dtype = -1;
  // d router_w in the MFMA backward: on the weight-gradient kernel (1), on
  // the SIMT kernel (0), or by size (-1); MXM_ROUTER_WGRAD_MFMA at creation
  int dwr_mode = -1;
  // 64-bit addressing where 32-bit byte offsets would do (operands below
  // 4 GiB): MXM_FORCE_64BIT_OFFSETS at creation, so that the paths larger
  // operands take can be checked on small ones
  bool force64 = false;
  DevBuf bw_delta, bw_dy, bw_dgates,
      bw_dlogits, bw_dxr, bw_wrt, bw_one, bw_wr_part;
  // bf16 ops: fp32 copies of the (bf16-valued) weights in x.W layout, of x
  // and of the forward's expert outputs, for the fp32 backward kernels
  bool bw_w32_ready = false;
  DevBuf bw_w1_32, bw_w1b_32, bw_w2_32, bw_wr32, bw_x32, bw_y32;
  // bf16 ops of the MFMA family: bf16 intermediates of the MFMA backward and
  // the weights re-laid for its products (W_down [F][D], W1 [D][NC])
  bool bw_wbf_ready = false;
  DevBuf bw_dhb, bw_gub, bw_dgub, bw_dxeb, bw_zero, bw_ms, bw_w2o, bw_w1u, bw_wscr,
      bw_ddb, bw_gp, bw_dgp, bw_dlb, bw_dwr2;
  // the fp32 backward's products (run_backward_x3): bf16 planes of the
  // operands at the padded widths Dq x Fq, fp32 products
  bool bx_w_ready = false;
  int bx_Dq = 0, bx_Fq = 0;
  DevBuf bx_w1p, bx_w1t, bx_w2p, bx_w2t, bx_x3, bx_gu, bx_h3, bx_y, bx_dy3, bx_dh, bx_dgu3, bx_dxe;
  int32_t bw_one_host[4] = {0, 0, 0, 0};

  // profiling: one set of MXM_NUM_STAGES+1 events per profiled forward
  bool profiling = false;
  int prof_reps = 1;  // launches of each stage between its events
  std::vector<std::array<hipEvent_t, MXM_NUM_STAGES + 1>> ev_sets;
  size_t ev_used = 0;

  ~MoeOp() {
    if (stream) {
      (void)hipStreamSynchronize(stream);
      (void)hipStreamDestroy(stream);
    }
    for (auto& set : ev_sets)
      for (auto& e : set)
        if (e) (void)hipEventDestroy(e);
  }
};

MoeOp* get_op(int64_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_ops.find(h);
  if (it == g_ops.end()) return nullptr;
  return it->second.get();
}

template <typename F>
int fenced(F&& f) {
  try {
    return f();
  } catch (const ArgError& e) {
    g_last_error = e.what();
    return MXM_ERR_ARGS;
  } catch (const InitError& e) {
    g_last_error = e.what();
    return MXM_ERR_INIT;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return MXM_ERR;
  } catch (...) {
    g_last_error = "unknown exception";
    return MXM_ERR;
  }
}

#define OP_OR_RETURN(h)                                 \
  MoeOp* op = get_op(h);                                \
  if (!op) {                                            \
    g_last_error = "OP_MOE_FEED_FORWARD invalid handle"; \
    return MXM_ERR_OP;                                  \
  }

// Whether a batch that the one-launch router can take is faster there than
// on the tiled router + scan + scatter.  The one-launch router's time grows
// with N (a workgroup per token, then one workgroup's dispatch of the N*K
// slots); the three-launch path's hardly does at these sizes.  So the one
// launch pays while each token brings enough logit work.  Measured on MI355X
// over N = 64-1024 and D*E = 512 .. 131072 (bf16 and fp32; results are bit
// for bit the same either way): where the tiled router's logits run on the
// matrix cores (mf) and E <= 64 it is the faster one for every N <= 640,
// up to N = 768 from D*E = 8192 on, up to N = 896 from D*E = 65536 on and
// up to N = 1024 from D*E = 98304 on; for E > 64 for every N <= 512, up to
// N = 768 from D*E = 4096 on and up to N = 1024 from D*E = 16384 on (with
// or without the matrix-core logits: the tiled router has only N / 64
// workgroups at these sizes); for
// E <= 32, where the tiled router routes several tokens per wave, the
// crossover lies near N = 200-300 for D*E = 512, ~400 for 4096, ~550 for
// 8192 and ~700 for 16384.  The int8 decode flow is built on the one-launch
// router and keeps it wherever it fits.
bool small_route_pays(int N, int D, int E, bool mf) {
  const int64_t de = (int64_t)D * E;
  if (mf && E <= 64)
    return N <= 640 || (N <= 768 && de >= 8192) || (N <= 896 && de >= 65536) || de >= 98304;
  if (E > 32) return N <= 512 || (N <= 768 && de >= 4096) || de >= 16384;
  return N <= 256 || (N <= 512 && de >= 8192) || (N <= 640 && de >= 16384) || de >= 65536;
}

// Whether an int8 op runs its expert GEMMs on the MFMA kernels (bf16 copies
// of the integers q, scales in the epilogue) rather than on the int8
// kernels.  The int8 kernels stream half the weight bytes and win while the
// weights are the traffic; with more routed rows per expert (N*K/E) the
// products turn compute-bound, where the int8 kernels reach 60-250 TFLOP/s
// and the MFMA tiles 0.8-1.1 PFLOP/s.  To first order the weight bytes
// cancel out of the comparison and the crossover is a number of rows per
// expert: measured on MI355X (whole forwards, with the int8 kernels' 128-row
// passes) near 96 for D 2048 / E 64 / K 8 / ffn 1408 (N 640: 0.399 against
// 0.409 ms, N 768: 0.422 / 0.422, N 1024: 0.677 / 0.437), D 512 / E 8 / K 2
// / ffn 2048 (N 384: 0.090 / 0.094, N 512: 0.149 / 0.094) and D 1024 / E 32
// / K 4 / ffn 1024 (N 768: 0.126 / 0.129, N 1024: 0.167 / 0.147), and
// 75-150 for D 256 with ffn 128-192, whose forwards are launch-bound either
// way.
bool q8_mfma_pays(int N, int E, int K) { return (int64_t)N * K >= 96 * (int64_t)E; }

// Whether a bf16 op at decode sizes streams its weights through the decode
// kernels rather than running the MFMA tiles.  Both read the same bf16
// bytes, but the tiles, built for compute-bound products, stream weights at
// about 3.4 TB/s, the decode kernels at 5.5-6.  The decode kernels take up
// to 128 rows per pass and stream an expert's weights once per pass, so with
// more routed rows per expert (N*K/E) the second passes make them the
// slower.  Measured on MI355X (whole forwards, tiles against stream): D 2048
// / E 64 / K 8 / ffn 1408 at N 64 0.347 against 0.186 ms, N 256 0.366 /
// 0.275, N 512 0.387 / 0.376, N 768 0.423 / 0.408; D 512 / E 8 / K 2 / ffn
// 2048 at N 64 0.071 / 0.038, N 256 0.081 / 0.071, N 384 0.093 / 0.081; D
// 1024 / E 32 / K 4 / ffn 1024 at N 64 0.069 / 0.049, N 512 0.099 / 0.103,
// N 768 0.129 / 0.121.
constexpr int DEC16_MAX_RPE = 96;
bool dec16_pays(int N, int E, int K) { return (int64_t)N * K < DEC16_MAX_RPE * (int64_t)E; }

// Row-tile heights and tile counts of the forward's kernels; a function of
// the op's parameters only.
void set_schedule(MoeOp& o) {
  const size_t NK = (size_t)o.N * o.K;
  o.ntiles = (int)(((size_t)o.N + MXM_ROUTER_TM - 1) / MXM_ROUTER_TM);
  const bool glu = o.etype != MXM_EXPERT_MLP;
  if (o.int8_kernels()) {
    o.bm1 = o.bm2 = 256;  // tile schedules are not used by the int8 kernels
  } else if (o.mfma) {
    // Unless a family was requested: 256 x 256 tiles where the columns allow
    // and the launch has at least two tiles per CU, else 128 x 128 (a grid
    // of one 256 x 256 tile per CU spends its time in each tile's ramp and
    // epilogue: C2's down projection 99 -> 92 us)
    auto pick = [&](int ncols) {
      if (o.family != MXM_TILE_AUTO) return o.family;
      if (ncols % 256 != 0) return (int)MXM_TILE_128x128;
      const int64_t tiles = ((int64_t)NK + 255) / 256 * (ncols / 256);
      return tiles < 2 * (int64_t)o.n_cu ? (int)MXM_TILE_128x128 : (int)MXM_TILE_256x256;
    };
    const int nc1 = glu ? 2 * o.Fk : o.Fk;
    o.fam1 = pick(nc1);
    o.fam2 = pick(o.Dk);
    o.fam_dh = pick(o.Fk);
    o.bm1 = mxm_mfma_tile_rows(nc1, o.Kx, o.fam1);
    o.bm2 = mxm_mfma_tile_rows(o.Dk, o.hsplit ? 2 * o.Fk : o.Fk, o.fam2);
  } else {
    // 64 x 64 tiles where their grid covers every CU, else 32 x 32 (C1's
    // down projection: 72 tiles of 64 x 64 for 256 CUs); MXM_SIMT_TILE (32
    // or 64, read at creation) overrides
    o.bm1 = mxm_simt_bm((int64_t)NK, o.E, o.F, o.n_cu);
    o.bm2 = mxm_simt_bm((int64_t)NK, o.E, o.D, o.n_cu);
    if (o.simt_tile == 32 || o.simt_tile == 64) o.bm1 = o.bm2 = o.simt_tile;
  }
  o.max_mtiles1 = (int)((NK + o.bm1 - 1) / o.bm1) + o.E;
  o.max_mtiles2 = (int)((NK + o.bm2 - 1) / o.bm2) + o.E;
}

// Place the forward's workspace for op o at base (nullptr: sizes only).
Workspace layout_workspace(const MoeOp& o, char* base) {
  const size_t N = (size_t)o.N, K = (size_t)o.K, E = (size_t)o.E, NK = N * K;
  const size_t T = (size_t)o.ntiles;
  Workspace w;
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return p;
  };
  char* tickets = take(8);
  w.scan_ticket = reinterpret_cast<int32_t*>(tickets);
  w.ticket = base ? reinterpret_cast<int32_t*>(tickets + 4) : nullptr;
  if (o.bf16) w.xcast = take(N * o.D * 2);
  w.top_idx = reinterpret_cast<int32_t*>(take(NK * 4));
  w.gates = reinterpret_cast<float*>(take(NK * 4));
  w.slot_rank = reinterpret_cast<int32_t*>(take(NK * 4));
  w.slot_pos = reinterpret_cast<int32_t*>(take(NK * 4));
  w.perm = reinterpret_cast<int32_t*>(take(NK * 4));
  w.tile_counts = reinterpret_cast<int32_t*>(take(E * T * 4));
  w.tile_psum = reinterpret_cast<float*>(take(E * T * 4));
  w.tile_ent = reinterpret_cast<float*>(take(T * 4));
  w.tile_base = reinterpret_cast<int32_t*>(take(E * T * 4));
  w.counts = reinterpret_cast<int32_t*>(take(E * 4));
  w.offsets = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  w.mstart1 = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  w.mstart2 = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  w.aux = reinterpret_cast<float*>(take(4));
  w.ent = reinterpret_cast<float*>(take(4));
  w.expert_count = reinterpret_cast<int32_t*>(take(E * 4));
  w.expert_pmean = reinterpret_cast<float*>(take(E * 4));
  const size_t esz = (o.mfma || o.q8) ? 2 : 4;
  if ((o.mfma || o.q8) && o.Kx != o.D) w.xpad = take(N * (size_t)o.Kx * 2);
  w.H = take(NK * (size_t)o.Fk * esz * (o.hsplit ? 2 : 1));
  w.Y = take(NK * (size_t)o.Dk * (o.hsplit ? 4 : esz));
  if (o.debug_probs) w.probs = reinterpret_cast<float*>(take(N * E * 4));
  if (o.small_route) {
    w.small_probs = reinterpret_cast<float*>(take(N * E * 4));
    w.tok_ent = reinterpret_cast<float*>(take(N * 4));
  }
  w.bytes = off;
  return w;
}

void alloc_workspace(MoeOp& o) {
  const size_t bytes = layout_workspace(o, nullptr).bytes;
  o.wsbuf.alloc(bytes);
  o.ws = layout_workspace(o, o.wsbuf.as<char>());
  HIPCK(hipMemsetAsync(o.ws.scan_ticket, 0, 8, o.stream));  // both tickets
  o.ws_ready = true;
}

// Refuse to launch a GEMM whose operands are not all allocated (a kernel
// would otherwise read through a null pointer).
void require_operands(const GemmArgs& g, bool second_matrix, bool scaled) {
  if (!g.a || !g.b0 || !g.out || !g.offsets || !g.mstart || (second_matrix && !g.b1) ||
      (scaled && (!g.scale0 || (g.mode == MXM_GEMM_GLU && !g.scale1))) ||
      (g.mode != MXM_GEMM_DOWN && !g.perm))
    fail_rt("OP_MOE_FEED_FORWARD internal error: expert GEMM operand not allocated (mode %d)", g.mode);
}

// Block-level extras of a forward (arch/moe.go:152-213): the rows before
// the norm (the residual), the optional moe_scale, and the aux weight.
struct BlockIO {
  const void* x;
  bool x_bf16;
  const void* moe_scale;
  bool scale_bf16;
  float aux_weight;
  float* aux_scaled;
};

// pre_out (MFMA family only): also keep the up projections' pre-activation
// products [N*K, NC] bf16 there (the backward's activation gradient reads
// them); H is then derived from them with the same activation code.
// w is the workspace the forward writes (the op's own, or the device
// scratch of the no-allocation entry point); with events = false no
// profiling events are recorded (they are created on demand).
void run_forward(MoeOp& o, const Workspace& w, const void* x, int x_dtype, float* delta, float* aux,
                 float* ent, const BlockIO* blk = nullptr, uint16_t* pre_out = nullptr,
                 bool events = true) {
  for (int i = 1; i < o.n_inputs; ++i)
    if (!o.have[i]) fail_rt("OP_MOE_FEED_FORWARD input w%d (Op.Inputs[%d]) is not set", i - 1, i);
  hipStream_t st = o.stream;
  o.last = w;
  o.have_last = true;
  o.kept = false;  // every forward overwrites what a kept one left
  // int8 weights at decode sizes: the router writes only the per-token
  // results; the expert kernels find their rows from the top-k picks, the
  // down projection stores y token-major and the combine computes aux and
  // entropy, so no launch waits for a dispatch (mxm_moe_routing computes it
  // on demand)
  // bf16 weights at decode sizes stream through the same kernels, except in
  // the backward's own forwards (which keep the tiles' raw projections)
  const bool dec16 = o.dec16 && !pre_out && !o.up_only && !o.route_only && !o.keep_probs;
  const bool stream = o.int8_kernels() || dec16;  // the decode kernels
  const bool decode_flow = stream && o.small_route && o.decode_flow;
  o.last_decode = decode_flow;
  const void* xin = x;
  if (o.bf16 && x_dtype == MXM_DTYPE_F32) {
    mxm_launch_to_bf16(x, MXM_DTYPE_F32, static_cast<uint16_t*>(w.xcast), (int64_t)o.N * o.D, st);
    xin = w.xcast;
  } else if ((o.bf16 && x_dtype != MXM_DTYPE_BF16) || (!o.bf16 && x_dtype != MXM_DTYPE_F32)) {
    fail("OP_MOE_FEED_FORWARD unsupported x dtype %d for this compute dtype", x_dtype);
  }
  float* aux_p = aux ? aux : w.aux;
  float* ent_p = ent ? ent : w.ent;
  hipEvent_t* evs = nullptr;
  if (o.profiling && events) {
    if (o.ev_used == o.ev_sets.size()) {
      std::array<hipEvent_t, MXM_NUM_STAGES + 1> set{};
      for (auto& e : set) HIPCK(hipEventCreate(&e));
      o.ev_sets.push_back(set);
    }
    evs = o.ev_sets[o.ev_used++].data();
  }
  auto mark = [&](int i) {
    if (evs) HIPCK(hipEventRecord(evs[i], st));
  };
  // profiled forwards may launch each stage several times between its events
  // (every stage is idempotent), so that short kernels are timed without the
  // events' own gaps
  const int reps = evs ? o.prof_reps : 1;

  mark(0);
  float* probs_keep = o.keep_probs ? o.bw_probs.as<float>() : w.probs;
  ScanArgs sa{};
  sa.counts = w.counts;
  sa.offsets = w.offsets;
  sa.mstart1 = w.mstart1;
  sa.mstart2 = w.mstart2;
  ScatterArgs sc{};
  sc.perm = w.perm;
  sc.slot_pos = w.slot_pos;
  if (o.small_route) {
    // one launch: router, scan and scatter (stages 1 and 2 are empty)
    RouteSmallArgs rs{};
    rs.x = xin;
    rs.wr_t = o.router_t.p;
    rs.ldw = o.ldw;
    rs.N = o.N;
    rs.D = o.D;
    rs.E = o.E;
    rs.K = o.K;
    rs.bm1 = o.bm1;
    rs.bm2 = o.bm2;
    rs.top_idx = w.top_idx;
    rs.gates = w.gates;
    rs.probs = probs_keep ? probs_keep : w.small_probs;
    rs.tok_ent = w.tok_ent;
    rs.counts = sa.counts;
    rs.offsets = sa.offsets;
    rs.mstart1 = sa.mstart1;
    rs.mstart2 = sa.mstart2;
    rs.perm = sc.perm;
    rs.slot_pos = sc.slot_pos;
    rs.aux = aux_p;
    rs.entropy = ent_p;
    rs.aux_weight = blk ? blk->aux_weight : 1.0f;
    rs.aux_scaled = blk ? blk->aux_scaled : nullptr;
    rs.ticket = w.ticket;
    rs.dispatch = !decode_flow;
    o.last_probs = rs.probs;
    for (int rep = 0; rep < reps; ++rep) mxm_launch_route_small(rs, o.bf16, st);
    HIPCK(hipGetLastError());
    mark(1);
    mark(2);
  } else {
    RouterArgs ra{};
    ra.x = xin;
    ra.wr = o.router.p;
    ra.N = o.N;
    ra.D = o.D;
    ra.E = o.E;
    ra.K = o.K;
    ra.top_idx = w.top_idx;
    ra.gates = w.gates;
    ra.slot_rank = w.slot_rank;
    ra.tile_counts = w.tile_counts;
    ra.tile_psum = w.tile_psum;
    ra.tile_ent = w.tile_ent;
    ra.probs_out = probs_keep;
    ra.wr_t = o.mf_router ? o.router_t.p : nullptr;
    ra.ldw = o.ldw;
    for (int rep = 0; rep < reps; ++rep) mxm_launch_router(ra, o.bf16, st);
    HIPCK(hipGetLastError());

    mark(1);
    sa.tile_counts = ra.tile_counts;
    sa.tile_psum = ra.tile_psum;
    sa.tile_ent = ra.tile_ent;
    sa.N = o.N;
    sa.E = o.E;
    sa.K = o.K;
    sa.ntiles = o.ntiles;
    sa.bm1 = o.bm1;
    sa.bm2 = o.bm2;
    sa.tile_base = w.tile_base;
    sa.aux = aux_p;
    sa.entropy = ent_p;
    sa.aux_weight = blk ? blk->aux_weight : 1.0f;
    sa.aux_scaled = blk ? blk->aux_scaled : nullptr;
    sa.expert_count = w.expert_count;
    sa.expert_pmean = w.expert_pmean;
    sa.ticket = w.scan_ticket;
    for (int rep = 0; rep < reps; ++rep) mxm_launch_scan(sa, o.bf16, st);
    HIPCK(hipGetLastError());

    mark(2);
    sc.top_idx = ra.top_idx;
    sc.slot_rank = ra.slot_rank;
    sc.tile_base = sa.tile_base;
    sc.offsets = sa.offsets;
    sc.N = o.N;
    sc.K = o.K;
    sc.ntiles = o.ntiles;
    for (int rep = 0; rep < reps; ++rep) mxm_launch_scatter(sc, st);
    HIPCK(hipGetLastError());
  }

  mark(3);
  if (o.route_only) return;
  const bool glu = o.etype != MXM_EXPERT_MLP;
  // the up projection reads x's rows Kx long: a zero-padded copy when D is
  // not a multiple of 64
  const void* xg = xin;
  if (w.xpad) {
    for (int rep = 0; rep < reps; ++rep)
      mxm_launch_pad_rows_bf16(static_cast<const uint16_t*>(xin), o.N, o.D, o.Kx,
                               static_cast<uint16_t*>(w.xpad), st);
    xg = w.xpad;
  }
  GemmArgs g1{};
  g1.no_off32 = o.force64;
  g1.mode = glu ? MXM_GEMM_GLU : MXM_GEMM_MLP;
  g1.a = xg;
  g1.perm = sc.perm;
  g1.b0 = o.w1.p;
  g1.b1 = o.w1b.p;
  g1.out = w.H;
  g1.offsets = sa.offsets;
  g1.mstart = sa.mstart1;
  g1.E = o.E;
  g1.Kd = o.Kx;
  g1.Ncols = (o.mfma && glu && !stream) ? 2 * o.Fk : o.Fk;
  g1.max_mtiles = o.max_mtiles1;
  g1.simt_bm = o.bm1;
  g1.simt_vec = o.simt_vec;
  g1.family = o.fam1;
  g1.expert_type = o.etype;
  g1.activation = o.act;
  g1.slope = o.slope;
  g1.rows_total = o.N * o.K;
  if (stream) {
    if (o.q8) {
      g1.b0 = o.q1.p;
      g1.b1 = o.q1b.p;
      g1.scale0 = o.s1.as<float>();
      g1.scale1 = o.s1b.as<float>();
    } else {
      g1.b0 = o.d1.p;
      g1.b1 = o.d1b.p;
      g1.w_bf16 = true;
    }
    if (decode_flow) {
      g1.top_idx = w.top_idx;
      g1.topk = o.K;
      g1.tk_offsets = w.offsets;
      g1.tk_counts = w.counts;
      g1.tk_ypos = w.slot_rank;
      // aux and entropy in one more workgroup of this launch
      g1.daux.top_idx = w.top_idx;
      g1.daux.probs = o.last_probs;
      g1.daux.tok_ent = w.tok_ent;
      g1.daux.N = o.N;
      g1.daux.E = o.E;
      g1.daux.K = o.K;
      g1.daux.bf16 = o.bf16;
      g1.daux.aux = aux_p;
      g1.daux.entropy = ent_p;
      g1.daux.aux_weight = blk ? blk->aux_weight : 1.0f;
      g1.daux.aux_scaled = blk ? blk->aux_scaled : nullptr;
    }
    require_operands(g1, glu, o.q8);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_q8(g1, st);
  } else if (o.mfma) {
    g1.out2 = pre_out;  // the backward keeps the raw projections (and no hidden)
    if (o.q8_mfma) {
      g1.scale0 = o.s1.as<float>();
      g1.scale1 = glu ? o.s1b.as<float>() : nullptr;
    }
    require_operands(g1, false, o.q8_mfma);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_mfma(g1, st);
    if (pre_out && !o.up_only)  // a kept forward: the hidden from them, as the epilogue would
      mxm_launch_hidden_from_raw_bf16(pre_out, o.N * o.K, o.Fk, o.etype, o.act, o.slope, o.hsplit,
                                      static_cast<uint16_t*>(w.H), st);
  } else {
    require_operands(g1, glu, false);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_simt(g1, o.bf16, st);
  }
  HIPCK(hipGetLastError());
  if (o.up_only) return;

  mark(4);
  GemmArgs g2{};
  g2.no_off32 = o.force64;
  g2.mode = MXM_GEMM_DOWN;
  g2.a = w.H;
  g2.b0 = o.w2.p;
  g2.out = w.Y;
  g2.offsets = sa.offsets;
  g2.mstart = sa.mstart2;
  g2.E = o.E;
  // the split MFMA down projection reduces over both planes of H
  g2.Kd = (o.hsplit && o.mfma && !stream) ? 2 * o.Fk : o.Fk;
  g2.h_split = o.hsplit;
  g2.Ncols = o.Dk;
  g2.max_mtiles = o.max_mtiles2;
  g2.simt_bm = o.bm2;
  g2.simt_vec = o.simt_vec;
  g2.family = o.fam2;
  g2.expert_type = o.etype;
  g2.activation = o.act;
  g2.slope = o.slope;
  g2.y_bf16 = o.bf16 && mxm_hidden_is_bf16(o.etype, o.act);
  g2.rows_total = o.N * o.K;
  if (stream) {
    if (o.q8) {
      g2.b0 = o.q2.p;
      g2.scale0 = o.s2.as<float>();
    } else {
      g2.b0 = o.d2.p;
      g2.w_bf16 = true;
    }
    if (decode_flow) {
      // the rows the up projection handed on (offsets, counts, y rows)
      g2.top_idx = w.top_idx;
      g2.topk = o.K;
      g2.tk_counts = w.counts;
      g2.tk_ypos = w.slot_rank;
    }
    require_operands(g2, false, o.q8);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_q8(g2, st);
  } else if (o.mfma) {
    if (o.q8_mfma) g2.scale0 = o.s2.as<float>();
    require_operands(g2, false, o.q8_mfma);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_mfma(g2, st);
  } else {
    require_operands(g2, false, false);
    for (int rep = 0; rep < reps; ++rep) mxm_launch_gemm_simt(g2, o.bf16, st);
  }
  HIPCK(hipGetLastError());

  mark(5);
  CombineArgs ca{};
  ca.y = w.Y;
  ca.top_idx = w.top_idx;
  ca.gates = w.gates;
  ca.slot_pos = sc.slot_pos;
  ca.N = o.N;
  ca.D = o.D;
  ca.ldy = o.Dk;
  ca.K = o.K;
  ca.delta = delta;
  if (blk) {
    ca.resid = blk->x;
    ca.resid_bf16 = blk->x_bf16;
    ca.rscale = blk->moe_scale;
    ca.rscale_bf16 = blk->scale_bf16;
  }
  if (decode_flow) {
    for (int rep = 0; rep < reps; ++rep) mxm_launch_combine_tm(ca, !o.hsplit, st);
  } else {
    for (int rep = 0; rep < reps; ++rep)
      mxm_launch_combine(ca, (o.mfma || o.q8) && !o.hsplit, st);
  }
  HIPCK(hipGetLastError());
  mark(6);
}

void set_weight(MoeOp& o, int idx, int dtype, const int64_t* shape, int ndim, const void* data,
                int on_device) {
  if (idx < 1 || idx >= o.n_inputs)
    fail("OP_MOE_FEED_FORWARD input index %d out of range [1,%d)", idx, o.n_inputs);
  if (o.q8 && idx != 1)
    fail("OP_MOE_FEED_FORWARD expert weights of an int8 op are bound with mxm_moe_set_input_q8");
  if (dtype != MXM_DTYPE_F32 && dtype != MXM_DTYPE_BF16)
    fail("OP_MOE_FEED_FORWARD weight dtype %d unsupported (want fp32 or bf16)", dtype);
  if (!data) fail("OP_MOE_FEED_FORWARD input w%d has no data", idx - 1);
  int rows, cols;
  int e = -1, j = -1;
  if (idx == 1) {
    rows = o.D;
    cols = o.E;
    if (ndim != 2 || shape[0] != o.D || shape[1] != o.E)
      fail("OP_MOE_FEED_FORWARD expects router_w shape [D,num_experts]");
  } else {
    e = (idx - 2) / o.wpe;
    j = (idx - 2) % o.wpe;
    const bool down = (j == o.wpe - 1);
    rows = down ? o.F : o.D;
    cols = down ? o.D : o.F;
    if (ndim != 2 || shape[0] != rows || shape[1] != cols) {
      if (o.wpe == 3) fail("OP_MOE_FEED_FORWARD expert GLU weights have invalid shapes");
      fail("OP_MOE_FEED_FORWARD expert MLP weights have invalid shapes");
    }
  }
  const size_t n = (size_t)rows * cols;
  const size_t src_bytes = n * (dtype == MXM_DTYPE_BF16 ? 2 : 4);
  hipStream_t st = o.stream;
  DevBuf staging;
  const void* src = data;
  if (!on_device) {
    staging.alloc(src_bytes);
    HIPCK(hipMemcpyAsync(staging.p, data, src_bytes, hipMemcpyHostToDevice, st));
    src = staging.p;
  }
  if (idx == 1) {
    if (o.bf16)
      mxm_launch_to_bf16(src, dtype, o.router.as<uint16_t>(), (int64_t)n, st);
    else
      mxm_launch_to_f32(src, dtype, o.router.as<float>(), (int64_t)n, st);
    if (o.small_route || o.mf_router)
      mxm_launch_router_t(o.router.p, o.bf16, o.D, o.E, o.ldw, o.router_t.p, st);
  } else if (o.mfma) {
    // rows of Fk (W_down [Dk][Fk]) and of Kx (W1 [NC][Kx]); the padding stays
    // zero from the allocation
    const bool glu = o.wpe == 3;
    if (j == o.wpe - 1) {
      uint16_t* dst = o.w2.as<uint16_t>() + (size_t)e * o.Dk * o.Fk;
      mxm_launch_transpose_bf16(src, dtype, o.F, o.D, -1, dst, st, o.Fk);
      if (o.dec16)
        mxm_launch_shuffle_bf16(src, dtype, o.F, o.D, o.Fk, o.Dk,
                                o.d2.as<uint16_t>() + (size_t)e * o.Fk * o.Dk, st);
    } else {
      const size_t ncols1 = glu ? 2 * (size_t)o.Fk : (size_t)o.Fk;
      uint16_t* dst = o.w1.as<uint16_t>() + (size_t)e * ncols1 * o.Kx;
      mxm_launch_transpose_bf16(src, dtype, o.D, o.F, glu ? j : -1, dst, st, o.Kx);
      if (o.dec16)
        mxm_launch_shuffle_bf16(src, dtype, o.D, o.F, o.Kx, o.Fk,
                                (j == 1 ? o.d1b : o.d1).as<uint16_t>() + (size_t)e * o.Kx * o.Fk,
                                st);
    }
  } else {
    // SIMT family keeps the reference layout in fp32 storage, values rounded
    // to bf16 first under bf16 compute.
    float* dst;
    if (j == o.wpe - 1)
      dst = o.w2.as<float>() + (size_t)e * o.F * o.D;
    else if (o.wpe == 3 && j == 1)
      dst = o.w1b.as<float>() + (size_t)e * o.D * o.F;
    else
      dst = o.w1.as<float>() + (size_t)e * o.D * o.F;
    if (o.bf16) {
      DevBuf tmp;
      tmp.alloc(n * 2);
      mxm_launch_to_bf16(src, dtype, tmp.as<uint16_t>(), (int64_t)n, st);
      mxm_launch_to_f32(tmp.p, MXM_DTYPE_BF16, dst, (int64_t)n, st);
      HIPCK(hipStreamSynchronize(st));
    } else {
      mxm_launch_to_f32(src, dtype, dst, (int64_t)n, st);
    }
  }
  HIPCK(hipGetLastError());
  HIPCK(hipStreamSynchronize(st));
  o.have[idx] = 1;
  o.bw_w32_ready = false;
  o.bw_wbf_ready = false;
  o.bx_w_ready = false;
  o.kept = false;  // a kept forward ran on the weights this call replaced
}

void set_weight_q8(MoeOp& o, int idx, const int8_t* q, const float* scales, const int64_t* shape,
                   int ndim, int on_device) {
  if (!o.q8) fail("OP_MOE_FEED_FORWARD op was not created with MXM_FLAG_INT8_WEIGHTS");
  if (idx < 2 || idx >= o.n_inputs)
    fail("OP_MOE_FEED_FORWARD int8 input index %d out of range [2,%d)", idx, o.n_inputs);
  if (!q || !scales) fail("OP_MOE_FEED_FORWARD int8 input w%d has no data", idx - 1);
  const int e = (idx - 2) / o.wpe, j = (idx - 2) % o.wpe;
  const bool down = (j == o.wpe - 1);
  const int rows = down ? o.F : o.D, cols = down ? o.D : o.F;
  if (ndim != 2 || shape[0] != rows || shape[1] != cols) {
    if (o.wpe == 3) fail("OP_MOE_FEED_FORWARD expert GLU weights have invalid shapes");
    fail("OP_MOE_FEED_FORWARD expert MLP weights have invalid shapes");
  }
  const size_t n = (size_t)rows * cols;
  hipStream_t st = o.stream;
  DevBuf sq;
  const int8_t* src = q;
  if (!on_device) {
    sq.alloc(n);
    HIPCK(hipMemcpyAsync(sq.p, q, n, hipMemcpyHostToDevice, st));
    src = sq.as<int8_t>();
  }
  DevBuf* sdst = down ? &o.s2 : (o.wpe == 3 && j == 1) ? &o.s1b : &o.s1;
  const int cols_k = down ? o.Dk : o.Fk;
  if (o.q8_mfma) {
    // the integers as bf16 in the MFMA layout (as mxm_moe_set_input's), the
    // padding zero from the allocation
    const bool glu = o.wpe == 3;
    if (down) {
      uint16_t* dst = o.w2.as<uint16_t>() + (size_t)e * o.Dk * o.Fk;
      mxm_launch_transpose_bf16(src, MXM_DTYPE_I8, o.F, o.D, -1, dst, st, o.Fk);
    } else {
      const size_t ncols1 = glu ? 2 * (size_t)o.Fk : (size_t)o.Fk;
      uint16_t* dst = o.w1.as<uint16_t>() + (size_t)e * ncols1 * o.Kx;
      mxm_launch_transpose_bf16(src, MXM_DTYPE_I8, o.D, o.F, glu ? j : -1, dst, st, o.Kx);
    }
  } else {
    DevBuf* qdst = down ? &o.q2 : (o.wpe == 3 && j == 1) ? &o.q1b : &o.q1;
    // padded to [Kx][Fk] (up) or [Fk][Dk] (down) with zero weights; the
    // padded columns' scales stay zero from the allocation
    const int rows_k = down ? o.Fk : o.Kx;
    mxm_launch_shuffle_q8(src, rows, cols, rows_k, cols_k,
                          qdst->as<uint8_t>() + (size_t)e * rows_k * cols_k, st);
  }
  HIPCK(hipMemcpyAsync(sdst->as<float>() + (size_t)e * cols_k, scales, (size_t)cols * 4,
                       on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
  HIPCK(hipGetLastError());
  HIPCK(hipStreamSynchronize(st));
  o.have[idx] = 1;
  o.bw_w32_ready = false;
  o.bw_wbf_ready = false;
  o.bx_w_ready = false;
  o.kept = false;  // a kept forward ran on the weights this call replaced
}

// ---- device scratch of the no-allocation forward ----
// One array per GPU (each device holds its own copy at its own address), kept
// until the process ends.  In host code `scratch` names a host-side stand-in,
// never device memory: host code uses only the address hipGetSymbolAddress
// returns for the current device (device_scratch below).
static __device__ __align__(256) unsigned char scratch[MXM_NOALLOC_MAX_BYTES];

__global__ void zero_words_kernel(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch[kMaxDevices] = {};

// This device's scratch address.  The first call on a device looks it up and
// clears the tickets (the first 256 bytes of every workspace layout; the
// kernels leave them zero after each call) with a fill kernel, then waits for
// the device, so it must not run under stream capture: mxm_init does it
// before any capture.
char* device_scratch(hipStream_t capturing) {
  int dev = 0;
  HIPCK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) fail_rt("OP_MOE_FEED_FORWARD device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    if (capturing) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      HIPCK(hipStreamIsCapturing(capturing, &cs));
      if (cs != hipStreamCaptureStatusNone)
        fail_init("OP_MOE_FEED_FORWARD no-allocation forward: call mxm_init on device %d before "
             "capturing",
             dev);
    }
    void* p = nullptr;
    HIPCK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail_rt("OP_MOE_FEED_FORWARD device scratch has no address on device %d", dev);
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, nullptr, static_cast<int32_t*>(p),
                       64);
    HIPCK(hipGetLastError());
    HIPCK(hipDeviceSynchronize());
    g_scratch[dev] = static_cast<char*>(p);
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

int mxm_init(void) {
  return fenced([&] {
    // every failure here is an initialisation failure (MXM_ERR_INIT)
    try {
      int n = 0;
      HIPCK(hipGetDeviceCount(&n));
      if (n <= 0) fail_init("no HIP device");
      int dev = 0;
      HIPCK(hipGetDevice(&dev));
      hipDeviceProp_t prop;
      HIPCK(hipGetDeviceProperties(&prop, dev));
      {
        std::lock_guard<std::mutex> lk(g_mu);
        g_device_name = std::string(prop.name) + " (" + prop.gcnArchName + ", " +
                        std::to_string(prop.multiProcessorCount) + " CUs)";
      }
      device_scratch(nullptr);  // the no-allocation forward's scratch on this device
    } catch (const std::exception& e) {
      throw InitError(e.what());
    }
    return MXM_OK;
  });
}

const char* mxm_device_name(void) { return g_device_name.c_str(); }

int mxm_last_error(char* buf, int n) {
  if (buf && n > 0) {
    std::strncpy(buf, g_last_error.c_str(), (size_t)n - 1);
    buf[n - 1] = '\0';
  }
  return (int)g_last_error.size();
}

int mxm_malloc(void** ptr, int64_t bytes) {
  return fenced([&] {
    if (!ptr || bytes < 0) fail("mxm_malloc: bad arguments");
    HIPCK(hipMalloc(ptr, bytes > 0 ? (size_t)bytes : 256));
    return MXM_OK;
  });
}

int mxm_free(void* ptr) {
  return fenced([&] {
    if (ptr) HIPCK(hipFree(ptr));
    return MXM_OK;
  });
}

int mxm_memcpy_h2d(void* dst, const void* src, int64_t bytes) {
  return fenced([&] {
    if (bytes > 0) HIPCK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
    return MXM_OK;
  });
}

int mxm_memcpy_d2h(void* dst, const void* src, int64_t bytes) {
  return fenced([&] {
    if (bytes > 0) HIPCK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
    return MXM_OK;
  });
}

int mxm_memcpy_d2d(void* dst, const void* src, int64_t bytes) {
  return fenced([&] {
    if (bytes > 0) HIPCK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice));
    return MXM_OK;
  });
}

int mxm_device_synchronize(void) {
  return fenced([&] {
    HIPCK(hipDeviceSynchronize());
    return MXM_OK;
  });
}

int64_t mxm_moe_create(const float* float_params, int n_float_params, const int32_t* int_params,
                       int n_int_params, int n_inputs, int compute_dtype, int flags) {
  int64_t handle = 0;
  const int rc = fenced([&] {
    // gpu/ir.cpp:1076-1104
    if (!int_params || n_int_params < 8)
      fail("OP_MOE_FEED_FORWARD requires B,T,D,E,topK,expertType,ffn,activation");
    auto o = std::make_unique<MoeOp>();
    if (const char* v = std::getenv("MXM_ROUTER_WGRAD_MFMA")) o->dwr_mode = std::atoi(v) != 0;
    if (const char* v = std::getenv("MXM_FORCE_64BIT_OFFSETS")) o->force64 = std::atoi(v) != 0;
    if (const char* v = std::getenv("MXM_DECODE_FLOW")) o->decode_flow = std::atoi(v) != 0;
    if (const char* v = std::getenv("MXM_SIMT_TILE")) o->simt_tile = std::atoi(v);
    if (const char* v = std::getenv("MXM_SIMT_MFMA")) o->simt_vec = std::atoi(v) == 0;
    o->B = int_params[0];
    o->T = int_params[1];
    o->D = int_params[2];
    o->E = int_params[3];
    o->K = int_params[4];
    o->etype = int_params[5];
    o->F = int_params[6];
    o->act = int_params[7];
    o->slope = (float_params && n_float_params > 0) ? float_params[0] : 0.0f;
    if (o->B <= 0 || o->T <= 0 || o->D <= 0 || o->E <= 0 || o->K <= 0 || o->K > o->E || o->F <= 0)
      fail("OP_MOE_FEED_FORWARD invalid dimensions");
    if ((int64_t)o->B * o->T > (int64_t)1 << 30) fail("OP_MOE_FEED_FORWARD invalid dimensions");
    // slot indices (perm, slot_pos, offsets, row tiles) are int32
    if ((int64_t)o->B * o->T * o->K > (int64_t)INT32_MAX)
      fail("OP_MOE_FEED_FORWARD B*T*topK = %lld routed slots exceeds %d",
           (long long)((int64_t)o->B * o->T * o->K), INT32_MAX);
    if (o->etype < MXM_EXPERT_SWIGLU || o->etype > MXM_EXPERT_MLP)
      fail("OP_MOE_FEED_FORWARD unsupported expert type");
    if (o->etype == MXM_EXPERT_MLP && (o->act < MXM_ACT_SILU || o->act > MXM_ACT_LEAKY_RELU_SQ))
      fail("OP_MOE_FEED_FORWARD unsupported activation");
    o->wpe = (o->etype == MXM_EXPERT_MLP) ? 2 : 3;
    if (n_inputs != 2 + o->E * o->wpe)
      fail("OP_MOE_FEED_FORWARD unexpected expert weight input count");
    if (o->E > MXM_MAX_EXPERTS)
      fail("OP_MOE_FEED_FORWARD supports at most %d experts (got %d)", MXM_MAX_EXPERTS, o->E);
    if (compute_dtype != MXM_DTYPE_F32 && compute_dtype != MXM_DTYPE_BF16)
      fail("OP_MOE_FEED_FORWARD compute dtype %d unsupported", compute_dtype);
    o->N = o->B * o->T;
    o->n_inputs = n_inputs;
    o->bf16 = compute_dtype == MXM_DTYPE_BF16;
    auto round_up = [](int v, int m) { return (v + m - 1) / m * m; };
    o->Fk = o->F;
    o->Dk = o->Kx = o->D;
    {
      // MFMA tiles on the padded widths (see MoeOp::Fk) once both widths span
      // at least one 128-wide tile; smaller ops keep the exact-order SIMT
      // kernels
      const int f = (flags & MXM_FLAG_MFMA_TILE_MASK) >> 2;
      const int Fk = round_up(o->F, 128), Dk = round_up(o->D, 128), Kx = round_up(o->D, 64);
      const int n1 = o->etype == MXM_EXPERT_MLP ? Fk : 2 * Fk;
      o->mfma = o->bf16 && !(flags & MXM_FLAG_FORCE_SIMT) && o->D >= 128 && o->F >= 128 &&
                mxm_mfma_tile_rows(n1, Kx, f) > 0 && mxm_mfma_tile_rows(Dk, Fk, f) > 0;
      if (o->mfma) {
        o->Fk = Fk;
        o->Dk = Dk;
        o->Kx = Kx;
      }
    }
    o->debug_probs = (flags & MXM_FLAG_DEBUG_PROBS) != 0;
    o->train = (flags & MXM_FLAG_KEEP_FOR_BACKWARD) != 0;
    o->q8 = (flags & MXM_FLAG_INT8_WEIGHTS) != 0;
    if (o->q8) {
      if (!o->bf16) fail("OP_MOE_FEED_FORWARD int8 weights need bf16 compute");
      // from 96 routed rows per expert on the MFMA kernels on the integers q,
      // where their tiles fit the padded widths (MXM_Q8_MFMA: 0 never, 1
      // whenever they fit)
      o->q8_mfma = o->mfma && q8_mfma_pays(o->N, o->E, o->K);
      if (const char* v = std::getenv("MXM_Q8_MFMA")) o->q8_mfma = o->mfma && std::atoi(v) != 0;
    }
    if (o->int8_kernels()) {
      // the int8 kernels: reduction lengths multiples of 64, output columns
      // multiples of 16; one expert's matrix addressed with 32-bit offsets
      o->mfma = false;
      o->Fk = round_up(o->F, 64);
      o->Dk = round_up(o->D, 16);
      o->Kx = round_up(o->D, 64);
      if ((int64_t)o->Kx * o->Fk >= ((int64_t)1 << 31) || (int64_t)o->Fk * o->Dk >= ((int64_t)1 << 31))
        fail("OP_MOE_FEED_FORWARD int8 weights: one expert's matrix must hold fewer than 2^31 "
             "entries (D=%d ffn=%d)", o->D, o->F);
    }
    o->family = (flags & MXM_FLAG_MFMA_TILE_MASK) >> 2;
    o->hsplit = (o->mfma || o->q8) && !mxm_hidden_is_bf16(o->etype, o->act);
    // bf16 weights at decode sizes: the decode kernels' weight stream
    // (MXM_BF16_DECODE: 0 never, 1 at every decode size); not for ops kept
    // for the backward, whose forward keeps the tiles' raw projections
    {
      const bool can = o->mfma && !o->q8 && !o->train && mxm_route_small_fits(o->N, o->D, o->E, o->K);
      o->dec16 = can && dec16_pays(o->N, o->E, o->K);
      if (const char* v = std::getenv("MXM_BF16_DECODE")) o->dec16 = can && std::atoi(v) != 0;
    }
    o->have.assign((size_t)n_inputs, 0);
    HIPCK(hipGetDevice(&o->device));
    HIPCK(hipDeviceGetAttribute(&o->n_cu, hipDeviceAttributeMultiprocessorCount, o->device));
    HIPCK(hipStreamCreateWithFlags(&o->stream, hipStreamNonBlocking));
    const size_t DE = (size_t)o->D * o->E, DF = (size_t)o->D * o->F, EE = (size_t)o->E;
    const size_t F1 = (size_t)o->Kx * o->Fk, F2 = (size_t)o->Fk * o->Dk;  // padded matrices
    o->router.alloc(DE * (o->bf16 ? 2 : 4));
    o->mf_router = o->E > 32;
    if (const char* v = std::getenv("MXM_ROUTER_MFMA")) o->mf_router = o->mf_router && std::atoi(v) != 0;
    // (the launcher also wants x 16-byte aligned; D decides it for the choice)
    const bool mf_logits = o->mf_router && o->D % (o->bf16 ? 8 : 4) == 0 && o->D <= (1 << 24);
    o->small_route = mxm_route_small_fits(o->N, o->D, o->E, o->K) &&
                     (o->int8_kernels() || o->dec16 ||
                      small_route_pays(o->N, o->D, o->E, mf_logits));
    if (const char* v = std::getenv("MXM_SMALL_ROUTE"))
      o->small_route = std::atoi(v) != 0 && mxm_route_small_fits(o->N, o->D, o->E, o->K);
    set_schedule(*o);
    if (o->small_route || o->mf_router) {
      o->ldw = (o->D + MXM_LOGIT_CHUNK - 1) / MXM_LOGIT_CHUNK * MXM_LOGIT_CHUNK;
      o->router_t.alloc((size_t)((o->E + 63) / 64) * o->ldw * 64 * (o->bf16 ? 2 : 4));
    }
    if (o->int8_kernels()) {
      o->q1.alloc(EE * F1);
      if (o->wpe == 3) o->q1b.alloc(EE * F1);
      o->q2.alloc(EE * F2);
      // padded output channels keep a zero scale
      o->s1.alloc(EE * o->Fk * 4);
      HIPCK(hipMemsetAsync(o->s1.p, 0, o->s1.bytes, o->stream));
      if (o->wpe == 3) {
        o->s1b.alloc(EE * o->Fk * 4);
        HIPCK(hipMemsetAsync(o->s1b.p, 0, o->s1b.bytes, o->stream));
      }
      o->s2.alloc(EE * o->Dk * 4);
      HIPCK(hipMemsetAsync(o->s2.p, 0, o->s2.bytes, o->stream));
      HIPCK(hipStreamSynchronize(o->stream));
    } else if (o->mfma) {
      // the padded rows and columns stay zero: uploads write only the real ones
      o->w1.alloc(EE * F1 * 2 * (o->wpe == 3 ? 2 : 1));
      o->w2.alloc(EE * F2 * 2);
      if (F1 != DF || F2 != DF) {
        HIPCK(hipMemsetAsync(o->w1.p, 0, o->w1.bytes, o->stream));
        HIPCK(hipMemsetAsync(o->w2.p, 0, o->w2.bytes, o->stream));
        HIPCK(hipStreamSynchronize(o->stream));
      }
      if (o->dec16) {
        // (every element, padding included, is written at binding)
        o->d1.alloc(EE * F1 * 2);
        if (o->wpe == 3) o->d1b.alloc(EE * F1 * 2);
        o->d2.alloc(EE * F2 * 2);
      }
      if (o->q8_mfma) {
        // padded output channels keep a zero scale (their weights are zero)
        o->s1.alloc(EE * o->Fk * 4);
        HIPCK(hipMemsetAsync(o->s1.p, 0, o->s1.bytes, o->stream));
        if (o->wpe == 3) {
          o->s1b.alloc(EE * o->Fk * 4);
          HIPCK(hipMemsetAsync(o->s1b.p, 0, o->s1b.bytes, o->stream));
        }
        o->s2.alloc(EE * o->Dk * 4);
        HIPCK(hipMemsetAsync(o->s2.p, 0, o->s2.bytes, o->stream));
        HIPCK(hipStreamSynchronize(o->stream));
      }
    } else {
      o->w1.alloc(EE * DF * 4);
      if (o->wpe == 3) o->w1b.alloc(EE * DF * 4);
      o->w2.alloc(EE * DF * 4);
    }
    std::lock_guard<std::mutex> lk(g_mu);
    handle = g_next_handle++;
    g_ops[handle] = std::move(o);
    return MXM_OK;
  });
  return rc == MXM_OK ? handle : 0;
}

int mxm_moe_destroy(int64_t h) {
  return fenced([&] {
    std::unique_ptr<MoeOp> victim;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      auto it = g_ops.find(h);
      if (it == g_ops.end()) {
        g_last_error = "OP_MOE_FEED_FORWARD invalid handle";
        return MXM_ERR_OP;
      }
      victim = std::move(it->second);
      g_ops.erase(it);
    }
    return MXM_OK;
  });
}

int mxm_moe_set_input(int64_t h, int input_index, int dtype, const int64_t* shape, int ndim,
                      const void* data, int on_device) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (!shape && ndim > 0) fail("OP_MOE_FEED_FORWARD shape is NULL");
    set_weight(*op, input_index, dtype, shape, ndim, data, on_device);
    return MXM_OK;
  });
}

int mxm_moe_set_input_q8(int64_t h, int input_index, const int8_t* q, const float* scales,
                         const int64_t* shape, int ndim, int on_device) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (!shape && ndim > 0) fail("OP_MOE_FEED_FORWARD shape is NULL");
    set_weight_q8(*op, input_index, q, scales, shape, ndim, on_device);
    return MXM_OK;
  });
}

bool mfma_backward_fits(const MoeOp& o);
static uint16_t* bw_gu_buffer(MoeOp& o);

int mxm_moe_forward(int64_t h, const void* x, int x_dtype, int64_t rows, float* delta, float* aux,
                    float* entropy) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !delta) fail("OP_MOE_FEED_FORWARD x and delta must be non-NULL");
    if (!op->ws_ready) alloc_workspace(*op);
    if (op->train) {
      // the forward runs on the op's own copy of x, so that the kept backward
      // differentiates at the x this forward saw whatever the caller's
      // buffer holds by then
      if (x_dtype != MXM_DTYPE_F32 && x_dtype != MXM_DTYPE_BF16)
        fail("OP_MOE_FEED_FORWARD unsupported x dtype %d for this compute dtype", x_dtype);
      const size_t xbytes = (size_t)op->N * op->D * (x_dtype == MXM_DTYPE_BF16 ? 2 : 4);
      if (op->kept_xbuf.bytes < xbytes) op->kept_xbuf.alloc(xbytes);
      op->kept = false;
      HIPCK(hipMemcpyAsync(op->kept_xbuf.p, x, xbytes, hipMemcpyDeviceToDevice, op->stream));
      const void* xk = op->kept_xbuf.p;
      if (mfma_backward_fits(*op)) {
        // keep what the backward's own forward would recompute
        op->keep_probs = true;
        try {
          run_forward(*op, op->ws, xk, x_dtype, delta, aux, entropy, nullptr, bw_gu_buffer(*op));
        } catch (...) {
          op->keep_probs = false;
          throw;
        }
        op->keep_probs = false;
        if (op->debug_probs)  // (mxm_moe_probs reads the workspace's copy)
          HIPCK(hipMemcpyAsync(op->ws.probs, op->bw_probs.p, (size_t)op->N * op->E * 4,
                               hipMemcpyDeviceToDevice, op->stream));
      } else {
        run_forward(*op, op->ws, xk, x_dtype, delta, aux, entropy);
      }
      op->kept = true;
      op->kept_dtype = x_dtype;
    } else {
      run_forward(*op, op->ws, x, x_dtype, delta, aux, entropy);
    }
    return MXM_OK;
  });
}

int mxm_moe_forward_host(int64_t h, const void* x, int x_dtype, int64_t rows, float* delta,
                         float* aux, float* entropy) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !delta) fail("OP_MOE_FEED_FORWARD x and delta must be non-NULL");
    const size_t xe = (x_dtype == MXM_DTYPE_BF16) ? 2 : 4;
    DevBuf dx, dd;
    dx.alloc((size_t)op->N * op->D * xe);
    dd.alloc((size_t)op->N * op->D * 4);
    HIPCK(hipMemcpyAsync(dx.p, x, dx.bytes, hipMemcpyHostToDevice, op->stream));
    if (!op->ws_ready) alloc_workspace(*op);
    run_forward(*op, op->ws, dx.p, x_dtype, dd.as<float>(), op->ws.aux, op->ws.ent);
    HIPCK(hipMemcpyAsync(delta, dd.p, (size_t)op->N * op->D * 4, hipMemcpyDeviceToHost, op->stream));
    if (aux) HIPCK(hipMemcpyAsync(aux, op->ws.aux, 4, hipMemcpyDeviceToHost, op->stream));
    if (entropy) HIPCK(hipMemcpyAsync(entropy, op->ws.ent, 4, hipMemcpyDeviceToHost, op->stream));
    HIPCK(hipStreamSynchronize(op->stream));
    return MXM_OK;
  });
}

int mxm_moe_forward_noalloc(int64_t h, const void* x, int x_dtype, int64_t rows, float* delta,
                            float* aux, float* entropy) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !delta) fail("OP_MOE_FEED_FORWARD x and delta must be non-NULL");
    int dev = 0;
    HIPCK(hipGetDevice(&dev));
    if (dev != op->device)
      fail("OP_MOE_FEED_FORWARD no-allocation forward called on device %d for an op of device %d",
           dev, op->device);
    const size_t need = layout_workspace(*op, nullptr).bytes;
    if (need > (size_t)MXM_NOALLOC_MAX_BYTES)
      fail("OP_MOE_FEED_FORWARD no-allocation forward needs %zu bytes of scratch for B*T=%d "
           "D=%d ffn=%d topK=%d, above the %zu-byte device scratch",
           need, op->N, op->D, op->F, op->K, (size_t)MXM_NOALLOC_MAX_BYTES);
    const Workspace w = layout_workspace(*op, device_scratch(op->stream));
    run_forward(*op, w, x, x_dtype, delta, aux, entropy, nullptr, nullptr, /*events=*/false);
    return MXM_OK;
  });
}

// Fused block forward (arch/moe.go:152-166, emitMoEDeltaIR :173-213):
// xn = RMSNorm(x, norm_scale, eps) (gpu/ir.cpp:4949-4960) in the compute
// dtype, op 74 on xn, delta *= moe_scale (if any), x_out = x + delta in fp32,
// aux_out = aux_weight * aux_raw.  All pointers are device memory.
void run_block(MoeOp& o, const void* x, int x_dtype, const void* norm_scale, const void* moe_scale,
               int scale_dtype, float eps, float aux_weight, float* x_out, float* aux, float* ent) {
  if (x_dtype != MXM_DTYPE_BF16 && x_dtype != MXM_DTYPE_F32)
    fail("OP_MOE_FEED_FORWARD unsupported x dtype %d for the block", x_dtype);
  if (scale_dtype != MXM_DTYPE_BF16 && scale_dtype != MXM_DTYPE_F32)
    fail("OP_RMSNORM scale dtype %d unsupported (want fp32 or bf16)", scale_dtype);
  if (!norm_scale) fail("OP_RMSNORM requires a scale input");
  if (!o.ws_ready) alloc_workspace(o);
  const size_t esz = o.bf16 ? 2 : 4;
  if (!o.xn.p) o.xn.alloc((size_t)o.N * o.D * esz);
  RmsNormArgs na{};
  na.x = x;
  na.x_bf16 = x_dtype == MXM_DTYPE_BF16;
  na.scale = norm_scale;
  na.scale_bf16 = scale_dtype == MXM_DTYPE_BF16;
  na.N = o.N;
  na.D = o.D;
  na.eps = eps;
  na.inv_d = (float)(1.0 / (double)o.D);
  na.out = o.xn.p;
  na.out_bf16 = o.bf16;
  mxm_launch_rmsnorm(na, o.stream);
  HIPCK(hipGetLastError());
  BlockIO b{};
  b.x = x;
  b.x_bf16 = na.x_bf16;
  b.moe_scale = moe_scale;
  b.scale_bf16 = na.scale_bf16;
  b.aux_weight = aux_weight;
  b.aux_scaled = aux;
  run_forward(o, o.ws, o.xn.p, o.bf16 ? MXM_DTYPE_BF16 : MXM_DTYPE_F32, x_out, nullptr, ent, &b);
}

int mxm_moe_block_forward(int64_t h, const void* x, int x_dtype, int64_t rows,
                          const void* norm_scale, const void* moe_scale, int scale_dtype, float eps,
                          float aux_weight, float* x_out, float* aux, float* entropy) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !x_out) fail("OP_MOE_FEED_FORWARD x and x_out must be non-NULL");
    run_block(*op, x, x_dtype, norm_scale, moe_scale, scale_dtype, eps, aux_weight, x_out, aux,
              entropy);
    return MXM_OK;
  });
}

int mxm_moe_block_forward_host(int64_t h, const void* x, int x_dtype, int64_t rows,
                               const void* norm_scale, const void* moe_scale, int scale_dtype,
                               float eps, float aux_weight, float* x_out, float* aux,
                               float* entropy) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !x_out) fail("OP_MOE_FEED_FORWARD x and x_out must be non-NULL");
    if (!norm_scale) fail("OP_RMSNORM requires a scale input");
    const size_t xe = (x_dtype == MXM_DTYPE_BF16) ? 2 : 4;
    const size_t se = (scale_dtype == MXM_DTYPE_BF16) ? 2 : 4;
    const size_t D = (size_t)op->D;
    DevBuf dx, dout, dres;
    dx.alloc((size_t)op->N * D * xe);
    dout.alloc((size_t)op->N * D * 4);
    dres.alloc(8);
    if (!op->blk_scales.p) op->blk_scales.alloc(2 * D * 4);
    char* sc = op->blk_scales.as<char>();
    HIPCK(hipMemcpyAsync(dx.p, x, dx.bytes, hipMemcpyHostToDevice, op->stream));
    HIPCK(hipMemcpyAsync(sc, norm_scale, D * se, hipMemcpyHostToDevice, op->stream));
    if (moe_scale)
      HIPCK(hipMemcpyAsync(sc + D * 4, moe_scale, D * se, hipMemcpyHostToDevice, op->stream));
    run_block(*op, dx.p, x_dtype, sc, moe_scale ? sc + D * 4 : nullptr, scale_dtype, eps,
              aux_weight, dout.as<float>(), dres.as<float>(), dres.as<float>() + 1);
    HIPCK(hipMemcpyAsync(x_out, dout.p, (size_t)op->N * D * 4, hipMemcpyDeviceToHost, op->stream));
    float res[2];
    HIPCK(hipMemcpyAsync(res, dres.p, 8, hipMemcpyDeviceToHost, op->stream));
    HIPCK(hipStreamSynchronize(op->stream));
    if (aux) *aux = res[0];
    if (entropy) *entropy = res[1];
    return MXM_OK;
  });
}

// Backward of op 74: a forward on x (keeping the router probabilities), then
// the gate / router gradients (mxm_launch_backward_router) and the experts'
// products.  fp32 ops and bf16 ops whose shapes the MFMA family does not
// tile run the experts' products on the fp32 SIMT kernels, the bf16 flow's
// values (x and weights rounded to bf16, the forward's bf16 expert outputs)
// converted to fp32.  bf16 ops of the MFMA family run them on MFMA
// (run_backward_mfma).  d_experts receives the expert weight gradients in
// Op.Inputs order (per expert gate, up, down -- or up, down -- in x.W layout).

// Shapes of the MFMA backward's three grouped products: dH = dY W_down^T
// (Fk columns, reduction D), the forward's kept projections (NC, D) and
// dX = dGU W1^T (D, NC), NC = 2Fk (GLU) or Fk; the activation backward takes
// hidden units 8 at a time within groups of 32 (Fk % 32 == 0).  The expert
// width may be padded (Fk > F: the padded units' gradients are zero and not
// stored), the model width not (D a multiple of 128: x, dD and dx are the
// caller's rows as they are).
bool mfma_backward_fits(const MoeOp& o) {
  const int NC = o.wpe == 3 ? 2 * o.Fk : o.Fk;
  return o.mfma && !o.q8 && o.Dk == o.D && o.Kx == o.D && o.Fk % 32 == 0 &&
         mxm_mfma_tile_rows(o.Fk, o.D, o.family) > 0 &&
         mxm_mfma_tile_rows(NC, o.D, o.family) > 0 && mxm_mfma_tile_rows(o.D, NC, o.family) > 0;
}


// The experts' products of the bf16 flow on MFMA.  Rows are in the forward's
// permuted order throughout (expert e owns rows offsets[e] ..).  The forward
// stops after its up projection: Y is never formed.
//   G|U = Xp W1                kept by the forward (its gate+up GEMM stores
//                              only the raw projections, GemmArgs::out2)
//   dH' = dD[token] W_down^T   MFMA grouped GEMM on the bf16 dD rows gathered
//                              through perm, W_down kept as [F][D] bf16; not
//                              yet gated
//   dgates = <dH', h>          (= <dD, Y>), dH = gate * dH', dG|dU and the
//                              gated hidden Hg = gate * h, h from G|U as the
//                              forward's epilogue computes it: one pass
//                              (act_bw_gated_bf16), then the router part
//   dXe = dG|dU W1^T           MFMA grouped GEMM, W1 kept as [D][NC] bf16
//   dx  = dlogits Wr^T + sum_k dXe   (dx_fused_bf16; with a dx that is not
//                              16-byte aligned: dxr + sum_k dXe, dx_bf16)
//   dW1 = Xp^T dG|dU, dW_down = Hg^T dD[token]   MFMA weight-gradient kernel
//                              (fp32 out; x and dD rows read through perm)
void run_backward_mfma(MoeOp& o, const void* xb, const BackwardArgs& b, float* dx, float* dw) {
  hipStream_t st = o.stream;
  const bool glu = o.wpe == 3;
  // F: the op's expert width (the layout of the gradients written to dw);
  // Fk: the kernels' (padded) width, NC its up-projection columns
  const int D = o.D, F = o.F, Fk = o.Fk, E = o.E, NC = glu ? 2 * Fk : Fk;
  const size_t NK = (size_t)o.N * o.K, DF = (size_t)D * F, DFk = (size_t)D * Fk,
               stride = (size_t)o.wpe * DF;
  // d router_w = x^T dlogits is N*D*E fmaf on the SIMT kernel: from 2^28 of
  // them on (C3's shape has 2^30, C2's 2^26) the weight-gradient kernel's
  // product is faster than that VALU work, below it its schedule and
  // reduction cost more
  const bool dwr_mfma =
      o.dwr_mode >= 0 ? o.dwr_mode == 1 : (double)o.N * D * E >= (double)(1 << 28);
  const int Ep = (E + 63) / 64 * 64;  // that product's hi and lo halves of Ep columns
  if (!o.bw_dhb.p) {
    o.bw_dhb.alloc(NK * Fk * 2);
    o.bw_dgub.alloc(NK * NC * 2);
    o.bw_dxeb.alloc(NK * D * 2);
    o.bw_zero.alloc(512);  // 256 zero bf16: the weight gradients' rows past an expert's end
    HIPCK(hipMemsetAsync(o.bw_zero.p, 0, 512, st));
    o.bw_ms.alloc(3 * ((size_t)E + 1) * 4);
    // the weight gradients' schedule and split-reduction partials (both
    // launches run in stream order and share it)
    o.bw_wscr.alloc(std::max({mxm_wgrad_scratch_bytes(D, NC), mxm_wgrad_scratch_bytes(Fk, D),
                              dwr_mfma ? mxm_wgrad_scratch_bytes(D, 2 * Ep) : 0}));
    if (dwr_mfma) {
      o.bw_dlb.alloc((size_t)o.N * 2 * Ep * 2);
      o.bw_dwr2.alloc((size_t)D * 2 * Ep * 4);
    }
    o.bw_w2o.alloc((size_t)E * DFk * 2);
    o.bw_w1u.alloc((size_t)E * D * NC * 2);
    o.bw_ddb.alloc((size_t)o.N * D * 2);
    o.bw_gp.alloc(NK * 4);
    o.bw_dgp.alloc(NK * 4);
  }
  if (!o.bw_wbf_ready) {
    for (int e = 0; e < E; ++e) {
      // W_down: forward [D][Fk] -> [Fk][D]; W1: forward [NC][D] -> [D][NC]
      mxm_launch_transpose_bf16(o.w2.as<uint16_t>() + (size_t)e * DFk, MXM_DTYPE_BF16, D, Fk, -1,
                                o.bw_w2o.as<uint16_t>() + (size_t)e * DFk, st);
      mxm_launch_transpose_bf16(o.w1.as<uint16_t>() + (size_t)e * NC * D, MXM_DTYPE_BF16, NC, D, -1,
                                o.bw_w1u.as<uint16_t>() + (size_t)e * D * NC, st);
    }
    HIPCK(hipGetLastError());
    o.bw_wbf_ready = true;
  }
  uint16_t *dhb = o.bw_dhb.as<uint16_t>(), *gub = o.bw_gub.as<uint16_t>(),
           *dgub = o.bw_dgub.as<uint16_t>(), *dxeb = o.bw_dxeb.as<uint16_t>(),
           *ddb = o.bw_ddb.as<uint16_t>();
  // dD in bf16 per token and the gates by slot position (dW_down takes the
  // gate on its left operand, so no per-slot dY = gate * dD is written)
  mxm_launch_dy_gate(b.d_delta, b.gates, b.slot_pos, o.N, D, o.K, ddb, nullptr,
                     o.bw_gp.as<float>(), st);
  // families as the forward picks them for the same output width (dX has
  // the down projection's, D)
  auto product = [&](int which, const uint16_t* A, const void* W, uint16_t* out, int Kd, int Ncols,
                     int family, bool gather) {
    const int bm = mxm_mfma_tile_rows(Ncols, Kd, family);
    int32_t* ms = o.bw_ms.as<int32_t>() + (size_t)which * (E + 1);
    mxm_launch_tile_prefix(b.counts, E, bm, ms, st);
    GemmArgs g{};
    g.no_off32 = o.force64;
    g.mode = MXM_GEMM_DOWN;
    g.a = A;
    g.b0 = W;
    g.out = out;
    g.offsets = b.offsets;
    g.mstart = ms;
    g.E = E;
    g.Kd = Kd;
    g.Ncols = Ncols;
    g.max_mtiles = (int)((NK + bm - 1) / bm) + E;
    g.family = family;
    g.gather_a = gather;  // A rows = token rows through perm
    g.perm = b.perm;
    g.rows_total = (int)NK;
    require_operands(g, false, false);
    mxm_launch_gemm_mfma(g, st);
    HIPCK(hipGetLastError());
  };
  // dH' = dD W_down^T for each slot's token, ungated: with H it gives the
  // gate gradients <dD, Y> = <dH', h>, and dH = gate * dH'
  product(0, ddb, o.bw_w2o.p, dhb, D, Fk, o.fam_dh, true);
  // gub holds G|U from the forward (run_forward's pre_out)
  mxm_launch_act_bw_gated_bf16(gub, dhb, static_cast<uint16_t*>(o.ws.H), o.hsplit,
                               o.bw_gp.as<float>(), (int)NK, Fk, o.etype, o.act, o.slope, dgub,
                               o.bw_dgp.as<float>(), st);
  HIPCK(hipGetLastError());
  // the router part from those gate gradients
  BackwardArgs br = b;
  br.dgp = o.bw_dgp.as<float>();
  br.dwr_by_caller = dwr_mfma;
  mxm_launch_backward_router(br, st);
  HIPCK(hipGetLastError());
  // d router_w = x^T dlogits on the weight-gradient kernel: one segment of
  // all N token rows (b.one = {0, N}), B = dlogits as bf16 hi and lo halves,
  // the two halves' products added at the end
  if (dwr_mfma && !mxm_wgrad_fits(D, 2 * Ep))
    fail("OP_MOE_FEED_FORWARD backward: router weight-gradient tiles need D a multiple of 128 "
         "(D=%d)", D);
  if (dwr_mfma) {
    mxm_launch_dl_split_bf16(b.dlogits, o.N, E, Ep, o.bw_dlb.as<uint16_t>(), st);
    WgradArgs ra{};
    ra.a = static_cast<const uint16_t*>(xb);
    ra.lda = D;
    ra.planes = 1;
    ra.b = o.bw_dlb.as<uint16_t>();
    ra.ldb = 2 * Ep;
    ra.offsets = b.one;
    ra.zero = o.bw_zero.as<uint16_t>();
    ra.E = 1;
    ra.M = D;
    ra.C = 2 * Ep;
    ra.out = o.bw_dwr2.as<float>();
    ra.scratch = o.bw_wscr.p;
    mxm_launch_wgrad(ra, st);
    mxm_launch_dwr_halves(o.bw_dwr2.as<float>(), D, E, Ep, b.dwr, st);
    HIPCK(hipGetLastError());
  }
  product(2, dgub, o.bw_w1u.p, dxeb, NC, D, o.fam2, false);
  if (b.dxr)
    mxm_launch_dx_bf16(b.dxr, dxeb, b.slot_pos, o.N, D, o.K, dx, st);
  else
    mxm_launch_dx_fused_bf16(b.dlogits, b.wrt, E, dxeb, b.slot_pos, o.N, D, o.K, dx, st);
  HIPCK(hipGetLastError());

  // weight gradients on MFMA, each reduced over its expert's rows (ragged,
  // from the device-side offsets): dW1 = Xp^T dG|dU, its GLU columns landing
  // de-interleaved in the gate and up matrices (x.W layout), and
  // dW_down = Hg^T dD[token] over the gated hidden's planes (hi and lo for a
  // split hidden)
  if (!mxm_wgrad_fits(D, NC) || !mxm_wgrad_fits(Fk, D))
    fail("OP_MOE_FEED_FORWARD backward: weight-gradient tiles need D, F multiples of 128 "
         "(D=%d F=%d)", D, Fk);
  WgradArgs wa{};
  wa.offsets = b.offsets;
  wa.zero = o.bw_zero.as<uint16_t>();
  wa.scratch = o.bw_wscr.p;
  wa.E = E;
  wa.out_estride = stride;
  // dW1's A rows are the tokens' x rows, read in place through perm
  wa.a = static_cast<const uint16_t*>(xb);
  wa.a_rows = b.perm;
  wa.a_rows32 = !o.force64 && (size_t)o.N * D * 2 < ((size_t)1 << 32);
  wa.lda = D;
  wa.planes = 1;
  wa.b = dgub;
  wa.ldb = NC;
  wa.M = D;
  wa.C = NC;
  wa.out = dw;
  wa.out_slot = DF;
  // the gradients land in the op's [D][F] layout; padded units are not stored
  wa.glu_f = glu ? F : 0;
  wa.c_store = (!glu && Fk != F) ? F : 0;
  mxm_launch_wgrad(wa, st);
  HIPCK(hipGetLastError());
  // dW_down = sum over slots of (gate h)^T dD[token]: A = the gated hidden
  // the activation pass wrote, B = bf16(dD) rows read in place through perm
  wa.a = static_cast<const uint16_t*>(o.ws.H);
  wa.a_rows = nullptr;
  wa.lda = o.hsplit ? 2 * Fk : Fk;
  wa.aplane = Fk;
  wa.planes = o.hsplit ? 2 : 1;
  wa.b = ddb;
  wa.b_rows = b.perm;
  wa.b_rows32 = !o.force64 && (size_t)o.N * D * 2 < ((size_t)1 << 32);
  wa.ldb = D;
  wa.M = Fk;
  wa.m_store = Fk != F ? F : 0;
  wa.C = D;
  wa.c_store = 0;
  wa.out = dw + (glu ? 2 : 1) * DF;
  wa.out_slot = 0;
  wa.glu_f = 0;
  mxm_launch_wgrad(wa, st);
  HIPCK(hipGetLastError());
}

// MFMA tile family for a product with Ncols output columns over `rows`
// rows: 256 x 256 where the columns allow and there are at least two tiles
// per CU, else 128 x 128 (as the forward's schedule picks them).
int product_family(const MoeOp& o, int ncols, size_t rows) {
  if (ncols % 256 != 0) return MXM_TILE_128x128;
  const int64_t tiles = ((int64_t)rows + 255) / 256 * (ncols / 256);
  return tiles < 2 * (int64_t)o.n_cu ? (int)MXM_TILE_128x128 : (int)MXM_TILE_256x256;
}

// The fp32 backward after the routing (fp32 compute, or the bf16 flow on
// fp32 copies where the MFMA backward does not apply).  Every product of the
// experts runs on the library's bf16 MFMA kernels as the product of the
// operands' bf16 planes (hi = bf16(v), lo = bf16(v - hi), concatenated along
// k so that one product sums hi.hi + hi.lo + lo.hi; mxm_launch_planes3):
// about 2^-16 relative per term, accumulated in fp32.  Operands are padded
// with zeros to Dq x Fq (multiples of 128); rows are in the forward's
// permuted order and every grouped product takes its experts' row ranges
// from the device-side offsets, so nothing waits for the host.
//   G|U = Xp W1                 grouped product, A = x's planes through perm
//   H = act(G, U)               planes of H
//   Y = H W_down                (own_forward: fp32 compute; else the op's
//                                forward's expert outputs)
//   the router part             (mxm_launch_backward_router: dgates .. dY,
//                                dx's router term, d router_w)
//   dH = dY W_down^T            grouped product on dY's planes
//   dG, dU                      the activation backward, as planes
//   dXe = dGU W1^T, dx = dxr + sum_k dXe
//   dW1 = Xp^T dGU, dW_down = H^T dY   the weight-gradient kernel, three
//                                plane pairs each, the gradients stored in
//                                the op's [D][F] / [F][D] layout
void run_backward_x3(MoeOp& o, BackwardArgs& b, bool own_forward) {
  hipStream_t st = o.stream;
  const bool glu = o.wpe == 3;
  const int D = o.D, F = o.F, E = o.E;
  const int Dq = (D + 127) / 128 * 128, Fq = (F + 127) / 128 * 128, NCq = glu ? 2 * Fq : Fq;
  const size_t N = o.N, NK = (size_t)o.N * o.K, DF = (size_t)D * F;
  if (o.bx_Dq != Dq || o.bx_Fq != Fq || !o.bx_x3.p) {
    o.bx_Dq = Dq;
    o.bx_Fq = Fq;
    o.bx_w1p.alloc((size_t)E * NCq * 3 * Dq * 2);
    o.bx_w1t.alloc((size_t)E * Dq * 3 * NCq * 2);
    o.bx_w2p.alloc((size_t)E * Dq * 3 * Fq * 2);
    o.bx_w2t.alloc((size_t)E * Fq * 3 * Dq * 2);
    o.bx_x3.alloc(N * 3 * Dq * 2);
    o.bx_gu.alloc(NK * NCq * 4);
    o.bx_h3.alloc(NK * 3 * Fq * 2);
    if (Dq != D) o.bx_y.alloc(NK * Dq * 4);
    o.bx_dy3.alloc(NK * 3 * Dq * 2);
    o.bx_dh.alloc(NK * Fq * 4);
    o.bx_dgu3.alloc(NK * 3 * NCq * 2);
    o.bx_dxe.alloc(NK * Dq * 4);
    if (!o.bw_zero.p) {
      o.bw_zero.alloc(512);  // 256 zero bf16: the weight gradients' rows past an expert's end
      HIPCK(hipMemsetAsync(o.bw_zero.p, 0, 512, st));
    }
    if (!o.bw_ms.p) o.bw_ms.alloc(3 * ((size_t)E + 1) * 4);
    o.bw_wscr.alloc(std::max(mxm_wgrad_scratch_bytes(Dq, NCq), mxm_wgrad_scratch_bytes(Fq, Dq)));
    o.bx_w_ready = false;
  }
  if (!o.bx_w_ready) {
    mxm_launch_planes3_weights(b.w1, glu ? b.w1b : nullptr, b.w2, E, D, F, Dq, Fq, glu,
                               o.bx_w1p.as<uint16_t>(), o.bx_w1t.as<uint16_t>(),
                               o.bx_w2p.as<uint16_t>(), o.bx_w2t.as<uint16_t>(), st);
    HIPCK(hipGetLastError());
    o.bx_w_ready = true;
  }
  uint16_t *x3 = o.bx_x3.as<uint16_t>(), *h3 = o.bx_h3.as<uint16_t>(),
           *dy3 = o.bx_dy3.as<uint16_t>(), *dgu3 = o.bx_dgu3.as<uint16_t>();
  float *gu = o.bx_gu.as<float>(), *dh = o.bx_dh.as<float>(), *dxe = o.bx_dxe.as<float>();
  // grouped product out [NK][Ncols] fp32 = A [NK][Kd] (rows through perm when
  // gather) . B_e^T (B_e [Ncols][Kd] per expert)
  auto product = [&](int which, const uint16_t* A, const uint16_t* W, float* out, int Kd,
                     int Ncols, bool gather) {
    const int family = product_family(o, Ncols, NK);
    const int bm = mxm_mfma_tile_rows(Ncols, Kd, family);
    if (bm <= 0)
      fail("OP_MOE_FEED_FORWARD backward: a %d x %d expert product exceeds the MFMA tiles' "
           "addressing", Ncols, Kd);
    int32_t* ms = o.bw_ms.as<int32_t>() + (size_t)which * (E + 1);
    mxm_launch_tile_prefix(b.counts, E, bm, ms, st);
    GemmArgs g{};
    g.no_off32 = o.force64;
    g.mode = MXM_GEMM_DOWN;
    g.f32_out = true;
    g.a = A;
    g.b0 = W;
    g.out = out;
    g.offsets = b.offsets;
    g.mstart = ms;
    g.E = E;
    g.Kd = Kd;
    g.Ncols = Ncols;
    g.max_mtiles = (int)((NK + bm - 1) / bm) + E;
    g.family = family;
    g.gather_a = gather;
    g.perm = b.perm;
    g.rows_total = (int)NK;
    require_operands(g, false, false);
    mxm_launch_gemm_mfma(g, st);
    HIPCK(hipGetLastError());
  };
  // x's planes (one row per token; the products gather them through perm)
  mxm_launch_planes3(b.x, (int64_t)N, D, D, Dq, false, x3, st);
  // G|U = Xp W1 (fp32, W1's interleaved column order), H's planes.  An fp32
  // ReLU expert takes U from the exact-order SIMT projection instead -- the
  // forward's own fp32 sums: ReLU's derivative jumps at 0, and the plane
  // products (about 2^-16 relative) would flip the mask of the units whose
  // pre-activation lies that close to 0, so the backward would not be the
  // gradient of the forward's function
  if (!o.bf16 && o.etype == MXM_EXPERT_MLP && o.act == MXM_ACT_RELU) {
    if (Fq != F) HIPCK(hipMemsetAsync(gu, 0, NK * Fq * 4, st));  // the padding columns
    GemmArgs g{};
    g.mode = MXM_GEMM_MLP;
    g.a = b.x;
    g.perm = b.perm;
    g.b0 = o.w1.p;
    g.out = nullptr;
    g.out2 = gu;
    g.ld2 = Fq;
    g.offsets = b.offsets;
    g.mstart = o.ws.mstart1;
    g.E = E;
    g.Kd = D;
    g.Ncols = F;
    g.max_mtiles = o.max_mtiles1;
    g.simt_bm = o.bm1;
    g.simt_vec = o.simt_vec;
    g.expert_type = o.etype;
    g.activation = o.act;
    g.slope = o.slope;
    if (!g.a || !g.b0 || !g.offsets || !g.mstart || !g.perm)
      fail_rt("OP_MOE_FEED_FORWARD backward: an operand of the exact up projection is missing");
    mxm_launch_gemm_simt(g, false, st);
    HIPCK(hipGetLastError());
  } else {
    product(0, x3, o.bx_w1p.as<uint16_t>(), gu, 3 * Dq, NCq, true);
  }
  mxm_launch_hidden_planes3(gu, (int64_t)NK, Fq, o.etype, o.act, o.slope, h3, st);
  HIPCK(hipGetLastError());
  if (own_forward) {
    // the expert outputs Y = H W_down, which the gate gradients read
    float* y = static_cast<float*>(o.ws.Y);
    product(1, h3, o.bx_w2p.as<uint16_t>(), Dq == D ? y : o.bx_y.as<float>(), 3 * Fq, Dq, false);
    if (Dq != D) mxm_launch_rows_to_f32(o.bx_y.p, MXM_DTYPE_F32, (int64_t)NK, D, Dq, y, st);
    HIPCK(hipGetLastError());
  }
  mxm_launch_backward_router(b, st);
  HIPCK(hipGetLastError());
  // dH = dY W_down^T, the activation backward, dXe = dGU W1^T, dx
  mxm_launch_planes3(b.dy, (int64_t)NK, D, D, Dq, true, dy3, st);
  product(1, dy3, o.bx_w2t.as<uint16_t>(), dh, 3 * Dq, Fq, false);
  mxm_launch_act_bw_planes3(gu, dh, (int64_t)NK, Fq, o.etype, o.act, o.slope, dgu3, st);
  HIPCK(hipGetLastError());
  product(2, dgu3, o.bx_w1t.as<uint16_t>(), dxe, 3 * NCq, Dq, false);
  mxm_launch_dx_sum(b.dxr, dxe, Dq, b.slot_pos, o.N, D, o.K, b.dx, st);
  HIPCK(hipGetLastError());
  // weight gradients: dW1 = Xp^T dGU over the plane pairs (x hi, dGU hi),
  // (x hi, dGU lo), (x lo, dGU hi); dW_down = H^T dY likewise
  WgradArgs wa{};
  wa.offsets = b.offsets;
  wa.zero = o.bw_zero.as<uint16_t>();
  wa.scratch = o.bw_wscr.p;
  wa.E = E;
  wa.out_estride = (size_t)o.wpe * DF;
  wa.planes = 3;
  wa.a = x3;
  wa.a_rows = b.perm;
  wa.a_rows32 = !o.force64 && N * 3 * Dq * 2 < ((size_t)1 << 32);
  wa.lda = 3 * Dq;
  wa.aplane = Dq;
  wa.b = dgu3;
  wa.ldb = 3 * NCq;
  wa.bplane = NCq;
  wa.M = Dq;
  wa.m_store = Dq != D ? D : 0;
  wa.C = NCq;
  wa.c_store = (!glu && Fq != F) ? F : 0;
  wa.out = b.dw;
  wa.out_slot = DF;
  wa.glu_f = glu ? F : 0;
  mxm_launch_wgrad(wa, st);
  HIPCK(hipGetLastError());
  wa.a = h3;
  wa.a_rows = nullptr;
  wa.a_rows32 = false;
  wa.lda = 3 * Fq;
  wa.aplane = Fq;
  wa.b = dy3;
  wa.ldb = 3 * Dq;
  wa.bplane = Dq;
  wa.M = Fq;
  wa.m_store = Fq != F ? F : 0;
  wa.C = Dq;
  wa.c_store = Dq != D ? D : 0;
  wa.out = b.dw + (glu ? 2 : 1) * DF;
  wa.out_slot = 0;
  wa.glu_f = 0;
  mxm_launch_wgrad(wa, st);
  HIPCK(hipGetLastError());
}

static uint16_t* bw_gu_buffer(MoeOp& o) {
  if (!o.bw_probs.p) o.bw_probs.alloc((size_t)o.N * o.E * 4);
  if (!o.bw_gub.p) o.bw_gub.alloc((size_t)o.N * o.K * (size_t)(o.wpe == 3 ? 2 * o.Fk : o.Fk) * 2);
  return o.bw_gub.as<uint16_t>();
}

// allow_kept (mxm_moe_backward_kept, x = the kept forward's copy): the kept
// routing and projections stand in for the backward's own forward
void run_backward(MoeOp& o, const void* x, int x_dtype, const float* d_delta, float d_aux,
                  float d_ent, float* dx, float* dwr, float* dw, bool allow_kept = false) {
  if (o.q8) fail("OP_MOE_FEED_FORWARD backward is not available for int8 expert weights");
  if (x_dtype != MXM_DTYPE_F32 && !(o.bf16 && x_dtype == MXM_DTYPE_BF16))
    fail("OP_MOE_FEED_FORWARD backward takes fp32 x (or bf16 x under bf16 compute)");
  if (!x || !d_delta || !dx || !dwr || !dw) fail("OP_MOE_FEED_FORWARD backward pointers must be non-NULL");
  if (!o.ws_ready) alloc_workspace(o);
  const size_t N = o.N, D = o.D, E = o.E, F = o.F, NK = (size_t)o.N * o.K;
  const bool mfma_bw = mfma_backward_fits(o);
  if (!o.bw_probs.p) o.bw_probs.alloc(N * E * 4);
  if (!o.bw_ready) {
    o.bw_delta.alloc(N * D * 4);
    if (!mfma_bw) o.bw_dy.alloc(NK * D * 4);  // (the MFMA backward keeps no dY)
    o.bw_dgates.alloc(NK * 4);
    o.bw_dlogits.alloc(N * E * 4);
    o.bw_wrt.alloc(D * E * 4);
    o.bw_wr_part.alloc((size_t)wgrad_router_chunks(o.N, D, E) * D * E * 4);
    o.bw_one.alloc(16);
    o.bw_one_host[1] = o.N;
    o.bw_one_host[3] = (o.N + 63) / 64;
    HIPCK(hipMemcpyAsync(o.bw_one.p, o.bw_one_host, 16, hipMemcpyHostToDevice, o.stream));
    o.bw_ready = true;
  }
  const float *w1 = o.w1.as<float>(), *w1b = o.w1b.as<float>(), *w2 = o.w2.as<float>();
  const float* wr = o.router.as<float>();
  const float* x32 = static_cast<const float*>(x);
  const float* y32 = static_cast<const float*>(o.ws.Y);
  if (o.bf16) {
    // The bf16 flow's values (x and weights rounded to bf16, the forward's
    // bf16 expert outputs) in fp32 for the fp32 kernels.
    if (!o.bw_w32_ready) {
      const size_t DF = D * F;
      if (!o.bw_wr32.p) o.bw_wr32.alloc(D * E * 4);
      mxm_launch_to_f32(o.router.p, MXM_DTYPE_BF16, o.bw_wr32.as<float>(), (int64_t)(D * E),
                        o.stream);
      if (o.mfma && !mfma_bw) {
        const bool glu = o.wpe == 3;
        if (!o.bw_w1_32.p) o.bw_w1_32.alloc(E * DF * 4);
        if (glu && !o.bw_w1b_32.p) o.bw_w1b_32.alloc(E * DF * 4);
        if (!o.bw_w2_32.p) o.bw_w2_32.alloc(E * DF * 4);
        const uint16_t* m1 = o.w1.as<uint16_t>();
        mxm_launch_w1_to_xw(m1, o.E, o.D, o.F, o.Kx, o.Fk, glu ? 0 : -1, o.bw_w1_32.as<float>(),
                            o.stream);
        if (glu)
          mxm_launch_w1_to_xw(m1, o.E, o.D, o.F, o.Kx, o.Fk, 1, o.bw_w1b_32.as<float>(), o.stream);
        mxm_launch_w2_to_xw(o.w2.as<uint16_t>(), o.E, o.D, o.F, o.Dk, o.Fk, o.bw_w2_32.as<float>(),
                            o.stream);
      }
      HIPCK(hipGetLastError());
      o.bw_w32_ready = true;
    }
    wr = o.bw_wr32.as<float>();
    if (o.mfma) {
      w1 = o.bw_w1_32.as<float>();
      w1b = o.bw_w1b_32.as<float>();
      w2 = o.bw_w2_32.as<float>();
    }
    if (!mfma_bw) {  // (the MFMA backward reads the bf16 x)
      if (!o.bw_x32.p) o.bw_x32.alloc(N * D * 4);
      x32 = o.bw_x32.as<float>();
    }
  }
  // the MFMA backward's G|U (pre-activation products) come from the forward
  uint16_t* gu = mfma_bw ? bw_gu_buffer(o) : nullptr;
  // the kept forward (MXM_FLAG_KEEP_FOR_BACKWARD) left the routing, the
  // probabilities and the raw projections where this forward puts them
  const bool reuse = mfma_bw && allow_kept && o.kept;
  // fp32 compute: the forward's routing only; the experts' forward products
  // are computed by run_backward_x3
  const bool own_forward = !o.bf16;
  if (!reuse) {
    o.keep_probs = true;
    o.route_only = own_forward;
    // the MFMA backward needs the routing and G|U only: its gate gradients
    // come from dD W_down^T (the product that also gives dH), not from Y
    o.up_only = mfma_bw;
    try {
      run_forward(o, o.ws, x, x_dtype, o.bw_delta.as<float>(), nullptr, nullptr, nullptr, gu);
    } catch (...) {
      o.keep_probs = o.route_only = o.up_only = false;
      throw;
    }
    o.keep_probs = o.route_only = o.up_only = false;
  }
  o.kept = false;  // (the backward overwrites the hidden)
  // x as the forward saw it (rounded to bf16 when given in fp32)
  const void* xb = (o.bf16 && x_dtype == MXM_DTYPE_BF16) ? x : o.ws.xcast;
  // The MFMA backward's router part reads x and a bf16 Y as they are; the
  // fp32 kernels of the other paths take fp32 copies.
  const bool read_bf16 = o.bf16 && mfma_bw;
  if (o.bf16 && !read_bf16) {
    mxm_launch_to_f32(xb, MXM_DTYPE_BF16, o.bw_x32.as<float>(), (int64_t)(N * D), o.stream);
    // y in fp32 [NK][D] (a split hidden's y is fp32 already; a padded down
    // projection's rows are Dk long)
    if (o.mfma && (!o.hsplit || o.Dk != o.D)) {
      if (!o.bw_y32.p) o.bw_y32.alloc(NK * D * 4);
      mxm_launch_rows_to_f32(o.ws.Y, o.hsplit ? MXM_DTYPE_F32 : MXM_DTYPE_BF16, (int64_t)NK,
                             (int)D, o.Dk, o.bw_y32.as<float>(), o.stream);
      y32 = o.bw_y32.as<float>();
    }
    HIPCK(hipGetLastError());
  }
  BackwardArgs b{};
  b.N = o.N;
  b.D = o.D;
  b.E = o.E;
  b.K = o.K;
  b.F = o.F;
  b.etype = o.etype;
  b.act = o.act;
  b.wpe = o.wpe;
  b.slope = o.slope;
  b.x = x32;
  b.top_idx = o.ws.top_idx;
  b.gates = o.ws.gates;
  b.slot_pos = o.ws.slot_pos;
  b.perm = o.ws.perm;
  b.counts = o.ws.counts;
  b.offsets = o.ws.offsets;
  b.probs = o.bw_probs.as<float>();
  b.Y = y32;
  if (read_bf16) {
    b.xb16 = static_cast<const uint16_t*>(xb);
    if (!o.hsplit) b.Yb16 = static_cast<const uint16_t*>(o.ws.Y);
  }
  b.wr = wr;
  b.d_delta = d_delta;
  b.d_aux = d_aux;
  b.d_ent = d_ent;
  b.dy = o.bw_dy.as<float>();
  b.dgates = o.bw_dgates.as<float>();
  b.dlogits = o.bw_dlogits.as<float>();
  // the MFMA path fuses dx's router term dlogits . Wr^T into the dx sum
  // (16-byte aligned dx); otherwise it is a separate product into dxr
  const bool fuse_dx = mfma_bw && reinterpret_cast<uintptr_t>(dx) % 16 == 0;
  if (!fuse_dx && !o.bw_dxr.p) o.bw_dxr.alloc(N * D * 4);
  b.dxr = fuse_dx ? nullptr : o.bw_dxr.as<float>();
  b.wrt = o.bw_wrt.as<float>();
  b.one = o.bw_one.as<int32_t>();
  b.wr_part = o.bw_wr_part.as<float>();
  b.dx = dx;
  b.dwr = dwr;
  b.dw = dw;
  if (mfma_bw) {
    run_backward_mfma(o, xb, b, dx, dw);
    return;
  }
  b.w1 = w1;
  b.w1b = w1b;
  b.w2 = w2;
  run_backward_x3(o, b, own_forward);
}

int mxm_moe_backward(int64_t h, const void* x, int x_dtype, int64_t rows, const float* d_delta,
                     float d_aux, float d_entropy, float* dx, float* d_router_w, float* d_experts) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    run_backward(*op, x, x_dtype, d_delta, d_aux, d_entropy, dx, d_router_w, d_experts);
    return MXM_OK;
  });
}

int mxm_moe_backward_kept(int64_t h, const float* d_delta, float d_aux, float d_entropy, float* dx,
                          float* d_router_w, float* d_experts) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (!op->train)
      fail("OP_MOE_FEED_FORWARD backward_kept needs an op created with "
           "MXM_FLAG_KEEP_FOR_BACKWARD");
    if (!op->kept)
      fail_rt("OP_MOE_FEED_FORWARD backward_kept: no kept forward (the op's last call must be "
              "mxm_moe_forward; another forward, a backward or a weight update drops it)");
    run_backward(*op, op->kept_xbuf.p, op->kept_dtype, d_delta, d_aux, d_entropy, dx, d_router_w,
                 d_experts, true);
    return MXM_OK;
  });
}

int mxm_moe_backward_host(int64_t h, const void* x, int x_dtype, int64_t rows,
                          const float* d_delta, float d_aux, float d_entropy, float* dx,
                          float* d_router_w, float* d_experts) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (rows != op->N) fail("OP_MOE_FEED_FORWARD expects x shape [B*T,D]");
    if (!x || !d_delta || !dx || !d_router_w || !d_experts)
      fail("OP_MOE_FEED_FORWARD backward pointers must be non-NULL");
    if (x_dtype != MXM_DTYPE_F32 && !(op->bf16 && x_dtype == MXM_DTYPE_BF16))
      fail("OP_MOE_FEED_FORWARD backward takes fp32 x (or bf16 x under bf16 compute)");
    const size_t ND = (size_t)op->N * op->D * 4;
    const size_t NDx = (size_t)op->N * op->D * (x_dtype == MXM_DTYPE_BF16 ? 2 : 4);
    const size_t nw = (size_t)op->E * op->wpe * op->D * op->F * 4;
    DevBuf dx_, dd_, ddx_, dwr_, dw_;
    dx_.alloc(NDx);
    dd_.alloc(ND);
    ddx_.alloc(ND);
    dwr_.alloc((size_t)op->D * op->E * 4);
    dw_.alloc(nw);
    HIPCK(hipMemcpyAsync(dx_.p, x, NDx, hipMemcpyHostToDevice, op->stream));
    HIPCK(hipMemcpyAsync(dd_.p, d_delta, ND, hipMemcpyHostToDevice, op->stream));
    run_backward(*op, dx_.p, x_dtype, dd_.as<float>(), d_aux, d_entropy, ddx_.as<float>(),
                 dwr_.as<float>(), dw_.as<float>());
    HIPCK(hipMemcpyAsync(dx, ddx_.p, ND, hipMemcpyDeviceToHost, op->stream));
    HIPCK(hipMemcpyAsync(d_router_w, dwr_.p, (size_t)op->D * op->E * 4, hipMemcpyDeviceToHost,
                         op->stream));
    HIPCK(hipMemcpyAsync(d_experts, dw_.p, nw, hipMemcpyDeviceToHost, op->stream));
    HIPCK(hipStreamSynchronize(op->stream));
    return MXM_OK;
  });
}

int mxm_moe_synchronize(int64_t h) {
  OP_OR_RETURN(h);
  return fenced([&] {
    HIPCK(hipStreamSynchronize(op->stream));
    return MXM_OK;
  });
}

int mxm_moe_routing(int64_t h, int32_t* top_idx, float* gates, int32_t* counts, int32_t* offsets,
                    int32_t* perm, int to_host) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (!op->have_last) fail_rt("OP_MOE_FEED_FORWARD routing requested before any forward");
    const hipMemcpyKind kind = to_host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    const size_t NK = (size_t)op->N * op->K;
    const Workspace& w = op->last;
    if (op->last_decode) {
      // the decode flow's dispatch, from the last forward's per-token results
      // (its aux and entropy go to the workspace's own slots)
      RouteSmallArgs rs{};
      rs.N = op->N;
      rs.D = op->D;
      rs.E = op->E;
      rs.K = op->K;
      rs.bm1 = op->bm1;
      rs.bm2 = op->bm2;
      rs.top_idx = w.top_idx;
      rs.gates = w.gates;
      rs.probs = op->last_probs;
      rs.tok_ent = w.tok_ent;
      rs.counts = w.counts;
      rs.offsets = w.offsets;
      rs.mstart1 = w.mstart1;
      rs.mstart2 = w.mstart2;
      rs.perm = w.perm;
      rs.slot_pos = w.slot_pos;
      rs.aux = w.aux;
      rs.entropy = w.ent;
      rs.aux_weight = 1.0f;
      rs.dispatch = true;
      mxm_launch_route_dispatch(rs, op->bf16, op->stream);
      HIPCK(hipGetLastError());
    }
    auto cp = [&](void* dst, const void* src, size_t bytes) {
      if (dst) HIPCK(hipMemcpyAsync(dst, src, bytes, kind, op->stream));
    };
    cp(top_idx, w.top_idx, NK * 4);
    cp(gates, w.gates, NK * 4);
    cp(counts, w.counts, (size_t)op->E * 4);
    cp(offsets, w.offsets, ((size_t)op->E + 1) * 4);
    cp(perm, w.perm, NK * 4);
    HIPCK(hipStreamSynchronize(op->stream));
    return MXM_OK;
  });
}

int mxm_moe_probs(int64_t h, float* probs) {
  OP_OR_RETURN(h);
  return fenced([&] {
    if (!op->debug_probs) fail("OP_MOE_FEED_FORWARD probabilities need MXM_FLAG_DEBUG_PROBS");
    if (!op->have_last) fail_rt("OP_MOE_FEED_FORWARD probabilities requested before any forward");
    HIPCK(hipMemcpyAsync(probs, op->last.probs, (size_t)op->N * op->E * 4, hipMemcpyDeviceToHost,
                         op->stream));
    HIPCK(hipStreamSynchronize(op->stream));
    return MXM_OK;
  });
}

int mxm_moe_set_profiling(int64_t h, int enable) {
  OP_OR_RETURN(h);
  return fenced([&] {
    HIPCK(hipStreamSynchronize(op->stream));
    op->profiling = enable != 0;
    op->prof_reps = enable > 1 ? enable : 1;
    op->ev_used = 0;
    return MXM_OK;
  });
}

int mxm_moe_stage_times(int64_t h, float* ms, int n) {
  OP_OR_RETURN(h);
  int count = 0;
  const int rc = fenced([&] {
    if (op->ev_used == 0) fail_rt("OP_MOE_FEED_FORWARD no profiled forward yet");
    for (int i = 0; i < n; ++i) ms[i] = 0.0f;
    for (size_t f = 0; f < op->ev_used; ++f) {
      auto& set = op->ev_sets[f];
      HIPCK(hipEventSynchronize(set[MXM_NUM_STAGES]));
      for (int i = 0; i < MXM_NUM_STAGES && i < n; ++i) {
        float t = 0.0f;
        HIPCK(hipEventElapsedTime(&t, set[i], set[i + 1]));
        ms[i] += t;
      }
    }
    for (int i = 0; i < MXM_NUM_STAGES && i < n; ++i)
      ms[i] /= (float)op->ev_used * (float)op->prof_reps;
    count = (int)op->ev_used;
    return MXM_OK;
  });
  return rc == MXM_OK ? count : rc;
}

int mxm_moe_info(int64_t h, int64_t* info, int n) {
  OP_OR_RETURN(h);
  const int64_t flow = !op->have_last ? -1 : op->last_decode ? 2 : op->small_route ? 1 : 0;
  const int64_t vals[8] = {op->q8_mfma ? 3 : op->q8 ? 2 : op->dec16 ? 4 : op->mfma ? 1 : 0,
                           (int64_t)layout_workspace(*op, nullptr).bytes, (int64_t)op->bm1,
                           (int64_t)((op->N + MXM_ROUTER_TM - 1) / MXM_ROUTER_TM),
                           (int64_t)op->Fk, (int64_t)op->Dk, (int64_t)op->Kx, flow};
  int w = 0;
  for (; w < n && w < 8; ++w) info[w] = vals[w];
  return w;
}

}  // extern "C"
