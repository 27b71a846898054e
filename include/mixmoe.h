/*
 * libmixmoe -- MI355X (gfx950) executor for mixlab's MoE feed-forward op
 * (IR op 74, OP_MOE_FEED_FORWARD).
 *
 * This is the C ABI that replaces, for op 74 only, the path
 *   gpu/lower.go:117-170 (LowerIRProgram)  ->  mlx_ir_program_create/add_op
 *   gpu/mlx_bridge.h:83-90                  ->  mlx_ir_eval_program_named_outputs
 *   gpu/mlx_bridge.h:172-181                ->  ir_interpret_outputs
 *   gpu/ir.cpp:4816-4824 (case OP_MOE_FEED_FORWARD) -> moe_feed_forward
 *   gpu/ir.cpp:1073-1164.
 * The op keeps the reference encoding (arch/ir.go:692-698):
 *   IntParams   = [B, T, D, E, topK, expertType, ffn, activation]
 *   FloatParams = [leakySlope]
 *   Inputs      = [x, router_w, then per expert (gate, up, down) or (up, down)]
 *   Outputs     = [delta [B*T, D] fp32, aux [1] fp32, entropy [1] fp32]
 *
 * Conventions follow gpu/mlx_bridge.h: opaque int64 handles with 0 meaning
 * failure (gpu/mlx_bridge.h:70-83), int status codes (gpu/mlx_bridge.cpp:
 * 814-823): 0 = OK, -10 = an argument the call cannot accept (shape, dtype,
 * index, size limit, NULL pointer), -11 = the HIP runtime or device could not
 * be initialised, -12 = not a live op handle, -1 = any other failure (a HIP
 * error, a call out of sequence); no C++ exception ever crosses the
 * boundary (gpu/mlx_bridge.cpp:64-82): the message of the last failure on the
 * calling thread is available from mxm_last_error.  Tensor dtype codes extend
 * mlx_tensor_input's (0 = int32, 1 = float32; gpu/mlx_bridge.h:92-99).
 *
 * Every call on one op handle is serialised by the caller (one HIP stream per
 * handle); distinct handles are independent.
 */
#ifndef MIXMOE_H
#define MIXMOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXM_OK 0
#define MXM_ERR -1       /* HIP error, call out of sequence */
#define MXM_ERR_ARGS -10 /* gpu/mlx_bridge.cpp:814-815: argument error */
#define MXM_ERR_INIT -11 /* gpu/mlx_bridge.cpp:818-819: runtime / device not initialised */
#define MXM_ERR_OP -12   /* gpu/mlx_bridge.cpp:821-822: bad op handle */

#define MXM_DTYPE_INT32 0 /* gpu/mlx_bridge.h:94 */
#define MXM_DTYPE_F32 1   /* gpu/mlx_bridge.h:94 */
#define MXM_DTYPE_BF16 2  /* compute_dtype "bf16" (gpu/ir_trainer.cpp:1395-1412) */
#define MXM_DTYPE_I8 3    /* symmetric int8 weights with fp32 per-output-channel scales */

#define MXM_OP_MOE_FEED_FORWARD 74 /* arch/ir.go:67, gpu/ir.h:81 */

/* mxm_moe_create flags */
#define MXM_FLAG_FORCE_SIMT 1 /* use the exact-order SIMT expert kernels even where MFMA tiles fit */
#define MXM_FLAG_DEBUG_PROBS 2 /* keep the router probabilities of the last forward */
/* MFMA tile family (bits 2-3); 0 picks 256x256 where the dimensions allow,
 * else 128x128 */
#define MXM_FLAG_MFMA_TILE128 4       /* 128 x 128 x 64 tiles, 4 waves, 2 LDS stages */
#define MXM_FLAG_MFMA_TILE256x128 8   /* 256 x 128 x 32 tiles, 4 waves, 3 LDS stages */
#define MXM_FLAG_MFMA_TILE256x256 12  /* 256 x 256 x 64 tiles, 8 waves, 2 LDS stages */
#define MXM_FLAG_MFMA_TILE_MASK 12
#define MXM_FLAG_INT8_WEIGHTS 16 /* expert weights are int8 + per-output-channel scales
                                    (mxm_moe_set_input_q8); bf16 compute */
/* Each mxm_moe_forward keeps the op's own copy of x and, under bf16 compute
 * on the MFMA family, its routing, router probabilities and raw up
 * projections, for mxm_moe_backward_kept: the backward of that forward,
 * which then does not run the forward again, as the reference's autodiff
 * keeps the forward's values for its backward.  No counterpart flag in the
 * reference (its graph keeps them implicitly). */
#define MXM_FLAG_KEEP_FOR_BACKWARD 32

/* Stages timed by mxm_moe_stage_times, in launch order. */
#define MXM_STAGE_ROUTER 0
#define MXM_STAGE_SCAN 1
#define MXM_STAGE_SCATTER 2
#define MXM_STAGE_GEMM_UP 3
#define MXM_STAGE_GEMM_DOWN 4
#define MXM_STAGE_COMBINE 5
#define MXM_NUM_STAGES 6

/* Initialise the HIP runtime on the current device.  Replaces mlx_init
 * (gpu/mlx_bridge.h:15).  0 on success, MXM_ERR_INIT on failure. */
int mxm_init(void);

/* Device name ("AMD Instinct MI355X ..."); replaces mlx_device_name
 * (gpu/mlx_bridge.h:53).  Never NULL. */
const char* mxm_device_name(void);

/* Copy the last failure message of the calling thread into buf (NUL
 * terminated, truncated to n bytes).  Returns the full message length.
 * Replaces the stderr logging of log_bridge_exception
 * (gpu/mlx_bridge.cpp:80-82). */
int mxm_last_error(char* buf, int n);

/* Device memory for callers that hold inputs and outputs in HBM (the cgo
 * side keeps these instead of MLX array handles, gpu/mlx_bridge.h:70-80). */
int mxm_malloc(void** ptr, int64_t bytes);
int mxm_free(void* ptr);
int mxm_memcpy_h2d(void* dst, const void* src, int64_t bytes);
int mxm_memcpy_d2h(void* dst, const void* src, int64_t bytes);
int mxm_memcpy_d2d(void* dst, const void* src, int64_t bytes);
int mxm_device_synchronize(void);

/* Create an op-74 executor.  Replaces mlx_ir_program_create(n_weights) +
 * mlx_ir_program_add_op(prog, 74, ...) (gpu/mlx_bridge.h:83-90) for one MoE
 * op.  int_params/float_params are the op's IntParams/FloatParams
 * (arch/ir.go:697); n_inputs is len(Op.Inputs).  Parameter checks and their
 * messages are those of gpu/ir.cpp:1076-1104.  compute_dtype is
 * MXM_DTYPE_F32 or MXM_DTYPE_BF16 (weights are cast to it, as
 * gpu/ir_trainer.cpp:1395-1412 does).  Returns a handle, 0 on failure. */
int64_t mxm_moe_create(const float* float_params, int n_float_params, const int32_t* int_params,
                       int n_int_params, int n_inputs, int compute_dtype, int flags);

/* Release an executor and its device memory; replaces
 * mlx_ir_program_destroy + mlx_free_handles (gpu/mlx_bridge.h:79-90). */
int mxm_moe_destroy(int64_t op);

/* Bind weight input `input_index` (position in Op.Inputs: 1 = router_w
 * [D, E], then expert e's matrices at 2 + e*wpe + j, in x.W layout
 * [in, out] as arch/moe.go:126-142 declares them).  dtype is MXM_DTYPE_F32
 * or MXM_DTYPE_BF16; data is host memory (on_device = 0) or device memory
 * (on_device = 1), copied and converted, so the caller keeps ownership.
 * Replaces mlx_from_data_shape (gpu/mlx_bridge.h:71) plus the w<i> name
 * lookup of gpu/ir.cpp:3730-3734; shape checks and messages are those of
 * gpu/ir.cpp:1098-1140. */
int mxm_moe_set_input(int64_t op, int input_index, int dtype, const int64_t* shape, int ndim,
                      const void* data, int on_device);

/* Bind expert weight input `input_index` (2 + e*wpe + j, as for
 * mxm_moe_set_input) as symmetric int8: q [in, out] in x.W layout and fp32
 * scales [out], i.e. W = q * scales[None, :] (per output channel).  Only for
 * ops created with MXM_FLAG_INT8_WEIGHTS.  This has no counterpart in the
 * reference, whose bridge takes fp32 weights only (gpu/mlx_bridge.cpp:210-217);
 * it serves decode-shaped serving, where the expert weights are the traffic.
 * Any D and ffn (widths that are not multiples of 64 are padded with zero
 * weights inside the library; one expert's matrix below 2^31 entries).  An
 * op whose batch routes 96 or more rows per expert (B*T*topK >= 96*E), which
 * is compute-bound, keeps the integers as bf16 (exact; twice the int8
 * bytes) for the bf16 MFMA tiles, which apply the scales to the fp32
 * accumulators: the same products and activation as the int8 kernels. */
int mxm_moe_set_input_q8(int64_t op, int input_index, const int8_t* q, const float* scales,
                         const int64_t* shape, int ndim, int on_device);

/* Run the op on x [rows = B*T, D] (dtype MXM_DTYPE_BF16 or MXM_DTYPE_F32;
 * fp32 x is rounded to bf16 first under bf16 compute), writing delta
 * [rows, D] fp32, aux [1] fp32 and entropy [1] fp32.  All pointers are
 * device memory; the call is asynchronous on the op's stream.  aux and
 * entropy may be NULL.  Replaces the case OP_MOE_FEED_FORWARD dispatch
 * (gpu/ir.cpp:4816-4824) of moe_feed_forward (gpu/ir.cpp:1073-1164).
 * A row whose logits are not finite (a NaN or infinity in x or router_w)
 * gets NaN probabilities and gates and still picks K distinct experts
 * (the lowest ids), so the dispatch of every other row is unaffected. */
int mxm_moe_forward(int64_t op, const void* x, int x_dtype, int64_t rows, float* delta,
                    float* aux, float* entropy);

/* Same with host buffers; synchronous (copies in, runs, copies out).  This
 * is the shape of mlx_ir_eval_program_named_outputs (gpu/mlx_bridge.h:172-181)
 * for the three outputs of op 74. */
int mxm_moe_forward_host(int64_t op, const void* x, int x_dtype, int64_t rows, float* delta,
                         float* aux, float* entropy);

/* Device scratch of mxm_moe_forward_noalloc, per GPU (64 MiB). */
#define MXM_NOALLOC_MAX_BYTES (64ll << 20)

/* mxm_moe_forward that allocates nothing.  It has no counterpart in the
 * reference: it is for callers that cannot call hipMalloc -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation.
 * Every buffer the forward writes besides its outputs (routing, dispatch,
 * H, Y) lives in one file-scope device array per GPU of
 * MXM_NOALLOC_MAX_BYTES, held until the process ends; an op whose workspace
 * is larger is rejected with an error.  Same arguments, kernels and results
 * as mxm_moe_forward (device pointers, asynchronous on the op's stream).
 * All calls on one GPU share that array: calls that overlap on one GPU (two
 * streams, two threads) race; each call leaves it ready for the next.  Call
 * mxm_init on each device before capturing (it looks up and clears the
 * array).  After this call mxm_moe_routing reads the array, which the next
 * no-allocation call on that GPU overwrites. */
int mxm_moe_forward_noalloc(int64_t op, const void* x, int x_dtype, int64_t rows, float* delta,
                            float* aux, float* entropy);

/* The whole MoE block of arch/moe.go:152-213 (emitMoEIR + emitMoEDeltaIR):
 *   xn     = RMSNorm(x, norm_scale, eps)        gpu/ir.cpp:4949-4960 (OP_RMSNORM)
 *   (delta, aux_raw, entropy) = op 74 on xn     gpu/ir.cpp:1073-1164
 *   delta *= moe_scale   (when moe_scale != NULL; block scales, arch/moe.go:199-204)
 *   x_out  = x + delta                          (the residual Add, arch/moe.go:164)
 *   aux    = aux_weight * aux_raw               (ScalarMul, arch/moe.go:197)
 * x [rows, D] is bf16 bits or fp32 (x_dtype); norm_scale and moe_scale [D]
 * have scale_dtype (fp32 or bf16 bits); x_out [rows, D], aux and entropy are
 * fp32.  xn is computed in the op's compute dtype.  The emitter uses
 * eps = 1e-5 and aux_weight = the block's effective load_balance_loss_weight.
 * Dropout (training only) is not applied.  Replaces the four IR ops the
 * emitter produces for one block (RMSNorm, op 74, ScalarMul, Add); device
 * pointers, asynchronous on the op's stream. */
int mxm_moe_block_forward(int64_t op, const void* x, int x_dtype, int64_t rows,
                          const void* norm_scale, const void* moe_scale, int scale_dtype, float eps,
                          float aux_weight, float* x_out, float* aux, float* entropy);

/* Same with host buffers; synchronous. */
int mxm_moe_block_forward_host(int64_t op, const void* x, int x_dtype, int64_t rows,
                               const void* norm_scale, const void* moe_scale, int scale_dtype,
                               float eps, float aux_weight, float* x_out, float* aux,
                               float* entropy);

/* Backward of op 74 (the gradients MLX's autodiff takes through
 * gpu/ir.cpp:1073-1164; the reference exercises them in
 * gpu/moe_feed_forward_test.go:84-151), computed in fp32.  Under bf16 compute
 * it uses the bf16 flow's values (x and weights rounded to bf16, the
 * forward's bf16 expert outputs); int8-weight ops have no backward.  Given
 * x [rows, D] (fp32, or bf16 bits under bf16 compute) and the upstream
 * gradients d_delta [rows, D] fp32, d_aux and
 * d_entropy (scalars), runs the forward on x (routing held fixed, as top-k
 * indices carry no gradient) and writes dx [rows, D], d_router_w [D, E] and
 * d_experts: the expert weight gradients in Op.Inputs order (per expert
 * w_gate, w_up, w_down -- or w_up, w_down -- each in x.W layout, as
 * mxm_moe_set_input takes them).  Device pointers; the call is asynchronous
 * on the op's stream (every expert product is a ragged grouped product whose
 * row ranges come from the device-side routing).  Under fp32 compute each
 * expert product runs as a bf16 MFMA product over the operands' hi / lo
 * planes (hi = bf16(v), lo = bf16(v - hi); about 2^-16 relative).  The first
 * call allocates the backward's workspace (on MI355X, 128 MiB of it holds the
 * weight gradients' split-reduction partials). */
int mxm_moe_backward(int64_t op, const void* x, int x_dtype, int64_t rows, const float* d_delta,
                     float d_aux, float d_entropy, float* dx, float* d_router_w, float* d_experts);

/* The backward of the op's last call, which must be an mxm_moe_forward on
 * an op created with MXM_FLAG_KEEP_FOR_BACKWARD: the gradients at the x that
 * forward read (the op kept its own copy, so the caller's buffer may have
 * changed since), from the routing and projections it kept.  Outputs as
 * mxm_moe_backward's.  Any other call that runs the op -- another forward
 * (plain, host, no-allocation or block), a backward -- or a weight update
 * with mxm_moe_set_input[_q8] drops the kept forward; without one this
 * returns MXM_ERR.  Replaces the backward half of the trainer's
 * value_and_grad over the graph (gpu/ir_trainer.cpp:2790-2816), which
 * differentiates the forward it just ran. */
int mxm_moe_backward_kept(int64_t op, const float* d_delta, float d_aux, float d_entropy, float* dx,
                          float* d_router_w, float* d_experts);

/* Same with host buffers; synchronous. */
int mxm_moe_backward_host(int64_t op, const void* x, int x_dtype, int64_t rows,
                          const float* d_delta, float d_aux, float d_entropy, float* dx,
                          float* d_router_w, float* d_experts);

/* Wait for all work queued on the op's stream. */
int mxm_moe_synchronize(int64_t op);

/* Routing of the last forward (synchronous copy): top_idx [rows, K] int32
 * (argsort(-probs)[:, :K], gpu/ir.cpp:1108-1109), gates [rows, K] fp32
 * (top_norm, gpu/ir.cpp:1110-1111), counts [E], offsets [E+1] and perm
 * [rows*K] (expert-grouped token ids).  Any pointer may be NULL.  to_host
 * selects host (1) or device (0) destinations.  A forward of the decode
 * flow (mxm_moe_info entry 7) computes only the per-token picks and
 * gates; this call then computes counts, offsets and perm from them on the
 * device first (the same tables, bit for bit). */
int mxm_moe_routing(int64_t op, int32_t* top_idx, float* gates, int32_t* counts,
                    int32_t* offsets, int32_t* perm, int to_host);

/* Router probabilities [rows, E] of the last forward; requires
 * MXM_FLAG_DEBUG_PROBS.  Host destination. */
int mxm_moe_probs(int64_t op, float* probs);

/* Per-stage HIP-event timing on the op's stream.  mxm_moe_set_profiling
 * (re)starts a recording: every later forward records events between its
 * kernels (enable = 0 stops it).  With enable = R > 1 each stage is launched
 * R times between its events (the stages are idempotent, so outputs are
 * unchanged), which times short kernels without the events' own gaps.
 * mxm_moe_stage_times waits for the recorded forwards and writes the mean
 * duration of one launch of each of the MXM_NUM_STAGES stages in
 * milliseconds; it returns the number of forwards averaged (> 0) or an error
 * code. */
int mxm_moe_set_profiling(int64_t op, int enable);
int mxm_moe_stage_times(int64_t op, float* ms, int n);

/* Executor facts: info[0] = expert kernel family (0 SIMT, 1 bf16 MFMA, 2 int8
 * weights on the int8 kernels, 3 int8 weights on the bf16 MFMA tiles: the
 * integers as bf16, the scales applied to the fp32 accumulators, for batches
 * past the decode sizes, 4 bf16 MFMA family whose forwards stream the
 * weights through the decode kernels: bf16 ops at decode sizes with fewer
 * than 96 routed rows per expert, not created with
 * MXM_FLAG_KEEP_FOR_BACKWARD; they hold the weights in both layouts, and
 * their backward runs on the tiles), info[1] = workspace bytes, info[2] = row-tile
 * height of the grouped GEMM, info[3] = number of router tiles, info[4] = the
 * expert width the kernels run at (ffn, or ffn rounded up to the tiles: 128
 * for MFMA, 64 for the int8 kernels, with zero weights in the padding),
 * info[5] = the down
 * projection's output width (D, or D rounded up to 128 / 16), info[6] = the
 * up projection's reduction length (D, or D rounded up to 64), info[7] = how
 * the last forward routed: 0 the tiled router, scan and scatter (three
 * launches), 1 the one-launch router (a workgroup per token, the dispatch in
 * its last workgroup), 2 the decode flow of the decode kernels (int8, or
 * bf16 streamed: the one-launch router's per-token results only; the expert
 * kernels find their rows from the top-k picks), -1 no forward yet.  Returns the number of entries written (at most
 * n, at most 8). */
int mxm_moe_info(int64_t op, int64_t* info, int n);

#ifdef __cplusplus
}
#endif

#endif /* MIXMOE_H */
