/*
 * xpool_amd.h -- C ABI of the MI355X (gfx950) FfnAgent Dense-FFN path.
 *
 * This library replaces the pybind11 extension `xpool.native` (src/cext-bindings/)
 * for the FfnAgent execution path only.  Every entry point takes plain device
 * pointers, sizes and a HIP stream (`void *` = hipStream_t; NULL = the legacy
 * default stream; a Lane's own stream comes from xp_lane_stream).
 * No torch types cross this boundary.  References are file:line in the
 * CrossPool checkout.
 *
 * Conventions
 *   - Every function returns an xp_status (0 = success).  On failure the
 *     calling thread's message is available through xp_last_error().
 *     (Replaces the synchronous TORCH_CHECK -> RuntimeError errors of
 *     src/cext/transport/instance.cpp:82-119 and src/cext-bindings/ops.cpp:17-26.)
 *   - Payload rows are bf16 or fp16 (`uint16_t` bit patterns, the dtype named by the call
 *     or the layer), rows contiguous, hidden and intermediate sizes multiples of 8,
 *     pointers 16-byte aligned.
 *   - Work is stream-ordered and never synchronises the host, except the
 *     functions documented as synchronous (health / synchronize).
 *   - Kernels that find a slot id outside the mailbox poison the gathered row
 *     with NaNs, skip the out-of-range write and OR XP_FAULT_SLOT_OUT_OF_RANGE
 *     into a sticky device fault word (the reference's NaN-poisoned, sticky
 *     canonical failure: src/cext/transport/instance.cu:28-31,75-77).
 *   - Caller-owned memory (weights, workspace, mailboxes, outputs) is borrowed:
 *     it must outlive every replay that reads it
 *     (docs/designs/ffn-execution.md:243-296 ownership rule).
 */
#ifndef XPOOL_AMD_H
#define XPOOL_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XP_ABI_VERSION 2

/* Status codes. */
enum {
  XP_OK = 0,
  XP_ERROR_INVALID_ARGUMENT = 1,
  XP_ERROR_HIP = 2,
  XP_ERROR_STATE = 3,
  XP_ERROR_NOT_FOUND = 4,
  XP_ERROR_CAPACITY = 5,
  XP_ERROR_UNSUPPORTED = 6
};

/* Closed FFN vocabulary, values identical to src/cext-include/xpool/ffn.hpp:15-54. */
enum { XP_FORWARD_PREFILL = 1, XP_FORWARD_DECODE = 2, XP_FORWARD_IDLE = 4 };
enum { XP_OUTPUT_PER_RANK_COMPLETE = 1, XP_OUTPUT_GROUP_SUM_COMPLETE = 2 };
enum { XP_DP_ROWS_NONE = 0, XP_DP_ROWS_UNIFORM_BY_RANK = 1, XP_DP_ROWS_PACKED_BY_RANK = 2 };
enum { XP_RESULT_OK = 0, XP_RESULT_SHUTDOWN = 1, XP_RESULT_PROTOCOL_MISMATCH = 2, XP_RESULT_TIMEOUT = 3 };
enum { XP_LAYER_DENSE = 1, XP_LAYER_MOE = 2 };
enum { XP_DTYPE_BF16 = 1, XP_DTYPE_F16 = 2, XP_DTYPE_F32 = 3 };
/* Activation functions (values of src/xpool/ffn.py:43-48 ActivationKind) and Gate/Up row
 * orders (ffn.py:51-68 GateUpOrder). */
enum { XP_ACTIVATION_NONE = 0, XP_ACTIVATION_SILU = 1, XP_ACTIVATION_RELU = 2, XP_ACTIVATION_GELU = 3 };
enum { XP_GATE_UP_CONCATENATED = 1, XP_GATE_UP_INTERLEAVED = 2 };

/* Sticky device fault bits. */
#define XP_FAULT_SLOT_OUT_OF_RANGE 1u

typedef void *xp_stream_t;

/* One activation with its optional Gate/Up combination (src/xpool/runtime/ffnagent/operators/
 * activation.py:87-173 Activation; ffn.py:118-151 SiluActivation / ReluActivation /
 * GeluActivation; ffn.py:130-137 GateTransform).  Gated: f(min(g, limit)) *
 * (clamp(u, -limit, limit) + up_offset) (clipping only with has_limit); ungated: f(v).
 * SiLU: v / (1 + exp(-alpha v)); ReLU keeps NaN payloads; GELU: erf form or, with
 * approximate_tanh, the tanh form. */
typedef struct {
  int function;         /* XP_ACTIVATION_SILU / RELU / GELU */
  int approximate_tanh; /* GELU only */
  int gated;
  int has_limit;
  float alpha;          /* SiLU slope (> 0) */
  float limit;          /* > 0 when has_limit */
  float up_offset;      /* gated only */
} xp_activation_desc;
typedef struct xp_agent *xp_agent_t;
typedef struct xp_lane *xp_lane_t;

/* ABI version of this library (XP_ABI_VERSION).  Replaces ABI_VERSION of
 * src/cext-bindings/module.cpp:16-79. */
int xp_abi_version(void);

/* Copy the calling thread's last error message; returns its full length. */
size_t xp_last_error(char *buffer, size_t size);

/* ------------------------------------------------------------------ kernels */

/* Byte copy of `bytes` from src to dst (non-overlapping), any alignment; a zero
 * length with NULL pointers is a no-op.  Replaces xpool::utils::cooperative::copy
 * (src/cext-include/xpool/utils/cooperative.cuh:37-55), the primitive behind the
 * Transport payload copies (src/cext/transport/instance.cu:83-84,184-186). */
int xp_copy_bytes(void *dst, const void *src, size_t bytes, xp_stream_t stream);

/* Fixed-order sum of tensor-parallel partials: out[i] = bf16(((0 + p0[i]) + p1[i]) + ...
 * + p_{count-1}[i]), accumulated in fp32 from +0 in partial order and rounded once to
 * nearest even.  `partials` is a host array of `count` (1..16) device pointers to bf16
 * arrays of `elements` values (a multiple of 8); every pointer is 16-byte aligned; `out`
 * may be one of the partials.  Replaces the fixed PE-order fold of the true-TP delivery
 * (src/cext/ffnagent/delivery.cu:74-127, ordered_sum / reduce_tp_partials) for partials
 * already in this device's memory; the exchange that brings peer partials there is not
 * part of this single-GPU build. */
int xp_reduce_partials(const void *const *partials, int count, void *out, int64_t elements, xp_stream_t stream);

/* out[i, :] = pool[slots[i], :] for i < rows, then, when norm_weight is not
 * NULL, out[i, :] = bf16(out_f32[i, :] / sqrt(mean(out_f32[i, :]^2) + eps) * w).
 * Without norm_weight the rows are copied bit-exactly.  Replaces the row-prefix
 * staging copy of src/cext/transport/instance.cu:83-84 and
 * src/cext/fabric/atnagent.cu:215 (identity slots reproduce it); the fused
 * RMSNorm replaces SGLang's post_attention_layernorm called before the shim
 * (src/xpool/integrations/sglang/models/qwen2.py:125-126).  fault_word may be NULL. */
int xp_gather_rmsnorm(const void *pool, int64_t pool_rows, int64_t hidden, const int32_t *slots, int64_t rows,
                      const void *norm_weight, float eps, void *out, uint32_t *fault_word, xp_stream_t stream);

/* pool[slots[i], :] = values[i, :] for i < rows, bit-exact.  Replaces the output
 * copies of src/cext/fabric/atnagent.cu:275 and src/cext/transport/instance.cu:184-186.
 * Slot ids must be distinct. */
int xp_scatter(const void *values, int64_t rows, int64_t hidden, const int32_t *slots, void *pool,
               int64_t pool_rows, uint32_t *fault_word, xp_stream_t stream);

/* activated[t, j] = bf16(act(bf16(x[t] . w[2j]), bf16(x[t] . w[2j+1]))) with
 * act(g, u) = silu_alpha(min(g, limit)) * (clamp(u, -limit, limit) + up_offset)
 * (limit <= 0: no clipping).  w is the INTERLEAVED i_proj [2*intermediate, hidden].
 * Replaces Gemm.run_into for i_proj with the fused epilogue
 * (src/xpool/runtime/ffnagent/operators/linear.py:163-257,
 *  operators/activation.py:112-173, operators/simt.py:13-45). */
int xp_gemm_gate_up_silu(const void *x, int64_t rows, int64_t hidden, const void *w_gate_up, int64_t intermediate,
                         void *activated, float alpha, float limit, float up_offset, void *workspace,
                         size_t workspace_bytes, xp_stream_t stream);

/* out[t, n] = bf16(activated[t] . w_down[n]), w_down [hidden, intermediate].
 * When slots is not NULL, row t is written to out + slots[t] * hidden instead
 * (the scatter fused into the epilogue; out then has out_rows rows).
 * Replaces Gemm.run_into for o_proj (operators/linear.py:163-257, dense.py:86). */
int xp_gemm_down(const void *activated, int64_t rows, int64_t intermediate, const void *w_down, int64_t hidden,
                 void *out, const int32_t *slots, int64_t out_rows, void *workspace, size_t workspace_bytes,
                 xp_stream_t stream);

/* General projection: out = epilogue(bias + x . w^T) with x [rows, k], w [n, k], out
 * [rows, n] (gated: [rows, n / 2] over INTERLEAVED Gate/Up rows), all of one payload dtype
 * (XP_DTYPE_BF16 / F16 / F32), bias fp32 [n] or NULL, any K and N, element-aligned rows.
 * The fp32 sum plus bias is stored rounded to the dtype; with an activation (NULL: none) it is
 * first rounded to the dtype (the projection rounding point), then activated in fp32, then
 * stored.  For the operator contract's shapes, dtypes and biases; bf16 SiLU projections of
 * aligned shapes without bias take xp_gemm_gate_up_silu / xp_gemm_down.  Replaces Gemm.run_into
 * for unquantized weights (src/xpool/runtime/ffnagent/operators/linear.py:163-257,
 * operators/simt.py:13-80) with the epilogue of operators/activation.py:112-173. */
int xp_projection(const void *x, int64_t rows, int64_t k, const void *w, int64_t n, const float *bias, void *out,
                  int dtype, const xp_activation_desc *activation, xp_stream_t stream);

/* Standalone activation over projected bf16 / fp16 values: gated, inputs [rows, 2 * width] in
 * the given Gate/Up order (INTERLEAVED: gate 2j, up 2j + 1; CONCATENATED: gate j, up width + j)
 * and output [rows, width], distinct storage; ungated, inputs and output [rows, width], which
 * may be the same storage.  Replaces activation_kernel / Activation.apply_into
 * (src/xpool/runtime/ffnagent/operators/activation.py:55-84, 175-207), which the CONCATENATED
 * Dense order runs between its projections (operators/dense.py:80-85). */
int xp_activation(const void *inputs, void *output, int64_t rows, int64_t width, int dtype, int order,
                  const xp_activation_desc *activation, xp_stream_t stream);

/* Scratch bytes the two projections above need for `rows` rows, n weight rows and
 * reduction length k (0 when the chosen kernel keeps the K reduction inside one
 * workgroup; pass workspace NULL then).  The scratch (16-byte aligned, contents irrelevant
 * on entry) holds fp32 partial sums of K slices; calls that may overlap in time must not
 * share one.  Replaces GemmPlan.split_k_workspace_bytes
 * (src/xpool/runtime/ffnagent/operators/linear.py:111-131). */
size_t xp_gemm_workspace_bytes(int64_t rows, int64_t n, int64_t k, int gated);

/* Bytes of Lane workspace one Dense step at `capacity` rows needs
 * (gathered batch + activated intermediate + K-slice partial sums).  Replaces DenseExecutionPlan's
 * WorkspaceLayout (src/xpool/runtime/ffnagent/operators/dense.py:24-52). */
size_t xp_dense_workspace_bytes(int64_t capacity, int64_t hidden, int64_t intermediate);

/* Byte offsets of that workspace's regions: [0] the gathered (normalised) batch
 * [capacity, hidden] bf16, [1] the activated intermediate [capacity, intermediate] bf16,
 * [2] gate_up's and [3] down's fp32 K-range partial sums (equal to [4] when the capacity
 * splits no K), [4] the total.  A Dense step leaves the batch and the activated rows of its
 * live rows there until the next step on the same workspace.  Replaces the region views of
 * WorkspaceLayout.views (src/xpool/runtime/ffnagent/execution.py:60-70), which the
 * reference's tests read directly. */
int xp_dense_workspace_layout(int64_t capacity, int64_t hidden, int64_t intermediate, size_t *offsets);

/* One eager mailbox step: gather(+RMSNorm) -> gate_up+SiLU -> down -> scatter to
 * pool_out rows slots[i] (pool_out may equal pool_in).  Same kernels as a replay.  The pool
 * (pool_rows * hidden * 2 bytes) must stay below 2 GiB, the 32-bit buffer range through which
 * the decode kernels gather it (XP_ERROR_INVALID_ARGUMENT otherwise; xp_replay likewise).
 * Replaces Dense.run_into (operators/dense.py:70-86) plus the Transport copies. */
int xp_dense_step(const void *pool_in, void *pool_out, int64_t pool_rows, const int32_t *slots, int64_t rows,
                  int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                  const void *norm_weight, float eps, void *workspace, size_t workspace_bytes, uint32_t *fault_word,
                  xp_stream_t stream);

/* xp_dense_step without a workspace argument: the step's workspace (gathered batch,
 * activated intermediate, K-range partial sums) is a static 64 MiB device array of the
 * library, one per device, held until the process ends.  It allocates nothing: no
 * hipMalloc / hipFree, no allocating library call.  Steps needing more than 64 MiB
 * (xp_dense_workspace_bytes(rows, hidden, intermediate) > 64 MiB, e.g. Qwen3-8B past about
 * 512 rows) fail with XP_ERROR_CAPACITY.  Every call on one device shares the array and
 * leaves its contents behind (no region needs to start cleared): calls that overlap in time
 * on one device race, so order them on one stream.  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under stream capture, tight serving
 * loops, harnesses that forbid allocation). */
int xp_dense_step_static(const void *pool_in, void *pool_out, int64_t pool_rows, const int32_t *slots, int64_t rows,
                         int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                         const void *norm_weight, float eps, uint32_t *fault_word, xp_stream_t stream);

/* Name of the kernel variant chosen for a projection ("split_..." / "stream_..." / "tile_...").
 * Returns the full name length. */
size_t xp_gemm_variant(int64_t capacity, int64_t n, int64_t k, int gated, char *buffer, size_t size);
/* Name of the gate_up variant of a Dense step (xp_dense_step, a Lane template) at `capacity`
 * rows: xp_gemm_variant's names, with "+gather" when the mailbox gather and RMSNorm run inside
 * that kernel (no separate gather launch).  Diagnostic only; no counterpart in the reference. */
size_t xp_dense_gate_up_variant(int64_t capacity, int64_t hidden, int64_t intermediate, char *buffer, size_t size);

/* ------------------------------------------------------------------ runtime */

/* FfnAgent execution state on one device: the layer table shared by its Lanes.
 * Replaces ExecutionRuntime::install's layer tables
 * (src/cext/ffnagent/runtime.cu:627-699, 1008-1039). */
int xp_agent_create(int device, xp_agent_t *out);
int xp_agent_destroy(xp_agent_t agent);

/* Register (or rebind) one Dense layer's borrowed weights.  payload_dtype is XP_DTYPE_BF16
 * or XP_DTYPE_F16 (is_supported_payload_dtype, src/cext-include/xpool/ffn.hpp:83-85), the
 * dtype of the weights, the norm weight and the mailboxes the layer is replayed on.  gate_up
 * is the INTERLEAVED i_proj [2*intermediate, hidden], down is o_proj [hidden,
 * intermediate], norm_weight [hidden] or NULL.  Replaces
 * LayerExecutionDescriptor + DenseBindingView (src/cext-bindings/ffnagent.cpp:44-210)
 * and the device-side weight rebinding of bind_compute (src/cext/ffnagent/runtime.cu:336-369). */
int xp_layer_register(xp_agent_t agent, int instance_index, int layer_ordinal, int64_t hidden, int64_t intermediate,
                      int payload_dtype, const void *gate_up, const void *down, const void *norm_weight, float eps);

/* Executor Lane: an owned HIP stream (default priority), a borrowed workspace
 * and a sticky device fault word.  Replaces LaneCaptureResources
 * (src/xpool/runtime/ffnagent/registry.py:25-137) and OwnedCudaStream
 * (src/cext-bindings/cuda.cpp:13-41). */
int xp_lane_create(xp_agent_t agent, void *workspace, size_t workspace_bytes, xp_lane_t *out);
int xp_lane_destroy(xp_lane_t lane);
int xp_lane_stream(xp_lane_t lane, xp_stream_t *out);
/* Synchronous: waits for the Lane stream, then reads the fault word. */
int xp_lane_check_health(xp_lane_t lane, uint32_t *fault_bits);
int xp_lane_clear_fault(xp_lane_t lane);
int xp_lane_synchronize(xp_lane_t lane);
/* Replay dispatch of this Lane: 0 (default) launches a template's kernels directly on the
 * stream, nonzero launches its instantiated hipGraph (rebinding only the kernel nodes whose
 * arguments changed).  Both run the same kernels with the same arguments.  No counterpart
 * in the reference, whose CUDA graphs are always launched (runtime.cu:701-1006); on MI355X a
 * hipGraphLaunch adds about 4-5 us of GPU time per Dense replay at decode sizes (measured on
 * the Qwen3-8B layer at 1 and 32 rows). */
int xp_lane_set_graph_dispatch(xp_lane_t lane, int use_graph);

/* GraphTemplate: build and instantiate this Lane's hipGraph for the Execution
 * Signature (payload dtype, capacity, hidden, intermediate).  Idempotent per signature.
 * Replaces capture_dense_signature (src/xpool/runtime/ffnagent/registry.py:189-239)
 * and materialize_lane's graph embedding (src/cext/ffnagent/runtime.cu:701-1006). */
int xp_template_capture(xp_lane_t lane, int64_t hidden, int64_t intermediate, int payload_dtype, int64_t capacity);
/* Number of captured templates; capacities of those matching (hidden, intermediate, dtype). */
int xp_template_capacities(xp_lane_t lane, int64_t hidden, int64_t intermediate, int payload_dtype,
                           int64_t *capacities, int max_count, int *count);

/* Replay the smallest captured capacity >= rows for the layer: gather rows
 * slots[0..rows) of pool_in (+ RMSNorm), the layer's FFN (Dense, or MoE from its
 * xp_moe_template_capture templates), write them to the same slots of pool_out on `stream` (NULL = the legacy default stream; the Lane's own stream is
 * xp_lane_stream's).  1 <= rows <= largest capacity.
 * Replaces wait_pre_compute's layer + capacity selection
 * (src/cext/ffnagent/runtime.cu:232-258), bind_compute (:336-369) and the
 * captured Dense body (registry.py:212-217). */
int xp_replay(xp_lane_t lane, int instance_index, int layer_ordinal, int64_t rows, const void *pool_in,
              void *pool_out, int64_t pool_rows, const int32_t *slots, xp_stream_t stream);

/* Device address of the Lane's sticky fault word, for xp_transport_evaluate.  Replaces the
 * Lane fault observation the reference's check_health reads (src/cext/ffnagent/runtime.cu
 * health path, src/cext-bindings/ffnagent.cpp:231). */
int xp_lane_fault_word(xp_lane_t lane, uint32_t **out);

/* ------------------------------------------------------------------ transport mailbox */

/* Mailbox lifecycle values (src/cext-include/xpool/transport/protocol.hpp:33-49). */
enum {
  XP_MAILBOX_DORMANT = 0,
  XP_MAILBOX_IDLE = 1,
  XP_MAILBOX_STAGING = 2,
  XP_MAILBOX_PUBLISHED = 3,
  XP_MAILBOX_EVALUATED = 4,
  XP_MAILBOX_CLOSED = 5
};

typedef struct xp_transport *xp_transport_t;

/* Host copy of one arena: the mailbox (protocol.hpp:52-62), the arena state words
 * (arena.hpp ArenaState: shutdown, generation_failure_code), the staged per-DP-rank rows,
 * and two words of this build: `violations` counts broken protocol preconditions (where the
 * reference traps with xpool::abort_if these kernels count and publish ProtocolMismatch),
 * `instance_outcome` is the last completed request's result (0xffffffff while one is in
 * flight). */
typedef struct {
  uint32_t mailbox_status;
  uint32_t result_code;
  uint64_t payload_rows;
  uint64_t layer_ordinal;
  uint32_t forward_mode;
  uint32_t output_requirement;
  uint32_t dp_row_layout;
  uint32_t shutdown;
  uint32_t generation_failure;
  uint32_t violations;
  uint32_t instance_outcome;
  uint32_t atn_dp_size;
  uint64_t payload_row_capacity;
  uint32_t dp_rank_payload_rows[64];
} xp_arena_snapshot;

/* A Transport resident on `device` serving `arena_count` arenas (one per Instance rank),
 * arena i with payload row capacity capacities[i] and attention DP size dp_sizes[i] (1..64).
 * Every mailbox starts Dormant.  Replaces the AtnAgent's arena allocation and
 * TransportResident (src/cext/transport/arena.cpp, atnagent.cpp). */
int xp_transport_create(int device, int arena_count, const int64_t *payload_row_capacities,
                        const int32_t *atn_dp_sizes, xp_transport_t *out);
/* Synchronous: waits for the device, then frees the arenas. */
int xp_transport_destroy(xp_transport_t transport);

/* Resident startup: every Dormant mailbox becomes Idle (src/cext/transport/atnagent.cu:124-129). */
int xp_transport_open(xp_transport_t transport, xp_stream_t stream);

/* Instance side, first half of one request (src/cext/transport/instance.cu:46-128 with the
 * host checks of instance.cpp:82-119): reject before staging on a canonical failure or
 * shutdown, else claim the mailbox (Idle -> Staging), stage the per-DP-rank rows (int32 or
 * int64 device vector of dp_rank_count entries, or NULL), write the request facts and
 * publish (Staging -> Published).  The payload itself is not copied: on one device the Lane
 * reads the caller's rows in place. */
int xp_transport_submit(xp_transport_t transport, int arena, int64_t payload_rows, int64_t layer_ordinal,
                        int forward_mode, int output_requirement, int dp_row_layout,
                        const void *dp_rank_payload_rows, int64_t dp_rank_count, int dp_rows_i64,
                        xp_stream_t stream);

/* Agent side, after the Lane's Dense step (src/cext/transport/atnagent.cu:34-90,155-170):
 * answer a Published request with OK, or PROTOCOL_MISMATCH when the request is invalid
 * (request_valid, atnagent.cu:34-46) or the Lane's fault word (may be NULL) is set; a
 * mismatch drains every arena of the transport. */
int xp_transport_evaluate(xp_transport_t transport, int arena, const uint32_t *fault_word, xp_stream_t stream);

/* Instance side, second half (src/cext/transport/instance.cu:130-201): wait up to timeout_ns
 * (<= 0: 5 s, wait.cuh:17) for the result; OK acknowledges (Evaluated -> Idle, request facts
 * reset) or, after shutdown, closes; any other result closes the mailbox and fills the
 * `output_elements` values of `output` (payload_dtype XP_DTYPE_BF16 or XP_DTYPE_F16) with
 * quiet NaNs of that dtype (instance.cu:28-31).  A wait that times out publishes TIMEOUT as
 * the canonical failure (the reference traps there). */
int xp_transport_complete(xp_transport_t transport, int arena, void *output, int64_t output_elements,
                          int payload_dtype, int64_t timeout_ns, xp_stream_t stream);

/* xp_transport_evaluate then xp_transport_complete in one launch on one stream, for a
 * request whose Dense step ran on that same stream (the completion then never waits). */
int xp_transport_settle(xp_transport_t transport, int arena, const uint32_t *fault_word, void *output,
                        int64_t output_elements, int payload_dtype, xp_stream_t stream);

/* Resident drain (atnagent.cu:92-147): publish shutdown to every arena, close Idle
 * mailboxes, answer Published ones with the canonical failure or SHUTDOWN. */
int xp_transport_drain(xp_transport_t transport, xp_stream_t stream);

/* Publish a canonical failure (PROTOCOL_MISMATCH or TIMEOUT) into one arena; the first one
 * sticks (src/cext-include/xpool/transport/arena.cuh:55-62). */
int xp_transport_publish_failure(xp_transport_t transport, int arena, int result_code, xp_stream_t stream);

/* Synchronous: waits for the device, then copies one arena to the host
 * (Arena::state / mailbox_status / read_generation_failure of transport/arena.hpp). */
int xp_transport_snapshot(xp_transport_t transport, int arena, xp_arena_snapshot *out);

/* Synchronous test entry: runs one of the reference's device-side protocol scenarios on one
 * arena and copies its observation words (unused ones read 0xffffffff) to `observed`
 * (at least 16 words): 0-4 tests/suites/cext/transport/view_test.cu:68-150, 5 and 6 the
 * producer and consumer kernels of tests/suites/cext/transport/shutdown_test.cu:173-191. */
int xp_transport_probe(xp_transport_t transport, int arena, int scenario, uint32_t *observed, int max_words);

/* ------------------------------------------------------------------ MoE */

/* Router vocabulary, values of src/xpool/ffn.py:78-115 (RouterAlgorithm,
 * RouterProjectionPrecision, TopKWeightRounding). */
enum { XP_ROUTER_SOFTMAX = 1, XP_ROUTER_SIGMOID = 2 };
enum { XP_ROUTER_PRECISION_PAYLOAD = 1, XP_ROUTER_PRECISION_FP32 = 2, XP_ROUTER_PRECISION_FP32_LOGITS = 3 };
enum { XP_TOPK_ROUNDING_NONE = 1, XP_TOPK_ROUNDING_LOGITS_DTYPE = 2 };

/* TopK over logits [rows, experts] of logits_dtype (XP_DTYPE_BF16, F16 or F32): scores are
 * softmax or sigmoid in fp32; selection = score (+ correction_bias[e], fp32, may be NULL;
 * sigmoid over 16-bit logits rounds the selection to the logits dtype); ties go to the lower
 * id for softmax and the higher id for sigmoid; the weight of a pick is its score (softmax
 * without correction: the selected maximum); renormalize divides by the sum of picked
 * weights when positive; LOGITS_DTYPE rounding then rounds weights through the dtype of
 * 16-bit logits.  Writes ids [rows, topk] int32 and weights [rows, topk] fp32.
 * experts <= 1024, topk <= 64.  Replaces router_topk_kernel
 * (src/xpool/runtime/ffnagent/operators/routing.py:21-89). */
int xp_moe_router_topk(const void *logits, int logits_dtype, int64_t rows, int64_t experts, int64_t topk,
                       int algorithm, const float *correction_bias, int renormalize, int weight_rounding,
                       int32_t *ids, float *weights, xp_stream_t stream);

/* Workspace bytes of xp_moe_router (the logits and the projection's K-slice scratch). */
size_t xp_moe_router_workspace_bytes(int64_t rows, int64_t hidden, int64_t experts, int precision);

/* Router: logits = hidden_states [rows, hidden] . router_weights^T, with hidden_states of
 * payload_dtype (XP_DTYPE_BF16 or F16) and weights [experts, hidden] of the payload dtype
 * (PAYLOAD: logits of the payload dtype, through the MFMA projection kernels when hidden and
 * experts are multiples of 8; FP32_LOGITS: fp32 logits) or fp32 (FP32: fp32 logits of the
 * widened input), then xp_moe_router_topk.  Replaces Router.run_into (routing.py:148-190). */
int xp_moe_router(const void *hidden_states, int64_t rows, int64_t hidden, const void *router_weights,
                  int64_t experts, int64_t topk, int algorithm, int precision, int payload_dtype,
                  const float *correction_bias, int renormalize, int weight_rounding, int32_t *ids, float *weights,
                  void *workspace, size_t workspace_bytes, xp_stream_t stream);

/* Final Routing Metadata [capacity, effective_topk]: routed slots copy the Router's ids and
 * weights, shared slots s name expert routed_expert_count + s with weight
 * 1 / routed_scaling_factor, rows at or past *payload_rows (a device int64) read -1 / 0.
 * Replaces finalize_moe_routing (routing.py:193-307). */
int xp_moe_finalize_routing(const int32_t *routed_ids, const float *routed_weights, int64_t capacity,
                            int64_t routed_topk, int32_t *final_ids, float *final_weights, int64_t effective_topk,
                            const int64_t *payload_rows, int64_t routed_expert_count, float routed_scaling_factor,
                            xp_stream_t stream);

/* Workspace bytes of xp_moe_experts for rows x topk routes. */
size_t xp_moe_workspace_bytes(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk);

/* Byte offsets of the Experts workspace regions, for inspection after a call (the workspace
 * keeps them until the next call): [0] expert ends (int32 [experts], one past each expert's
 * last sorted position), [1] sorted routes (int32 [rows * topk], route = row * topk + slot
 * at each sorted position), [2] tile experts and [3] tile first positions (int32), [4] the
 * activated routes ([rows * topk, intermediate] of the payload dtype, sorted order), [5] the
 * route outputs ([rows * topk, hidden] of the payload dtype, by route).  No counterpart in
 * the reference, whose test harness reads its workspace views directly (moe.py:181-215). */
int xp_moe_workspace_layout(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk,
                            size_t *offsets);

/* Experts: for every route (row, slot) with 0 <= e = topk_ids[row, slot] < experts,
 * h = p(act(p(x[row] . w_gate_up[e][2j] + bg[e][2j]), p(x[row] . w_gate_up[e][2j+1] + bg[e][2j+1])))
 * and r = p((h . w_down[e][n] + bd[e][n]) * topk_weights[row, slot]); then
 * output[row] = p(routed_scaling_factor * sum over slots in order of float(r)), 0 for
 * rows without routes, where p rounds to payload_dtype (XP_DTYPE_BF16 or F16), the dtype of
 * x, the weights and the output, and the fp32 biases bg = gate_up_bias [experts,
 * 2*intermediate] and bd = down_bias [experts, hidden] read as 0 when NULL.  w_gate_up is
 * [experts, 2*intermediate, hidden] (Gate/Up INTERLEAVED), w_down [experts, hidden,
 * intermediate].  act(g, u) = f(min(g, limit)) * (clamp(u, -limit, limit) + up_offset)
 * (no clipping for limit <= 0) with f of `activation`: XP_ACTIVATION_SILU (v / (1 +
 * exp(-alpha v))), XP_ACTIVATION_RELU (NaN kept) or XP_ACTIVATION_GELU (erf, or the tanh
 * approximation with approximate_tanh).  Replaces Experts.run_into
 * (src/xpool/runtime/ffnagent/operators/moe.py:168-343). */
int xp_moe_experts(const void *hidden_states, int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts,
                   int64_t topk, const void *w_gate_up, const void *w_down, const float *gate_up_bias,
                   const float *down_bias, const int32_t *topk_ids, const float *topk_weights,
                   float routed_scaling_factor, int activation, int approximate_tanh, float alpha, float limit,
                   float up_offset, int payload_dtype, void *output, void *workspace, size_t workspace_bytes,
                   xp_stream_t stream);

/* ---------------------------------------------------------------- MoE layer kind
 * One MoE layer's execution identity: the fields of MoeFfnExecutionSignature
 * (src/xpool/runtime/ffnagent/execution.py:98-123, router signature included) that the
 * captured body depends on, with the layer's MoeFfnSpec (src/xpool/ffn.py:251-275) and the
 * model's SiLU / GateTransform.  experts counts the routed experts and then the shared ones
 * (experts - routed_experts always-selected slots); effective topk = routed_topk + shared.
 * On one device the Lane owns the Router (the reference's TP rank 0 role,
 * src/cext/ffnagent/runtime.cu:649). */
typedef struct {
  int64_t hidden;
  int64_t intermediate;     /* one expert's intermediate width */
  int64_t experts;          /* routed + shared, <= 1024 */
  int64_t routed_experts;   /* Router output width */
  int64_t routed_topk;      /* <= min(routed_experts, 64) */
  int algorithm;            /* XP_ROUTER_SOFTMAX / SIGMOID */
  int precision;            /* XP_ROUTER_PRECISION_* */
  int renormalize;
  int weight_rounding;      /* XP_TOPK_ROUNDING_* */
  float routed_scaling_factor;
  float alpha;              /* SiLU slope */
  float limit;              /* Gate/Up clip, 0 = none */
  float up_offset;
  int payload;              /* XP_DTYPE_BF16 or XP_DTYPE_F16: the mailbox rows and weights */
  int activation;           /* XP_ACTIVATION_SILU / RELU / GELU (alpha is SiLU's slope) */
  int approximate_tanh;     /* GELU: the tanh approximation */
  int biases;               /* projection biases bound at registration: bit 0 gate_up, bit 1 down */
} xp_moe_layer_desc;

/* Register (or rebind) one MoE layer's borrowed weights, of desc->payload unless stated:
 * gate_up [experts, 2*intermediate, hidden] (Gate/Up INTERLEAVED per expert), down
 * [experts, hidden, intermediate], the fp32 projection biases gate_up_bias [experts,
 * 2*intermediate] and down_bias [experts, hidden] (given exactly as desc->biases says, else
 * NULL), router [routed_experts, hidden] (fp32 for the FP32 precision), correction_bias
 * [routed_experts] fp32 or NULL, norm_weight [hidden] or NULL.
 * Replaces LayerExecutionDescriptor + MoeBindingView (src/cext-bindings/ffnagent.cpp) and
 * the MoE branch of validate_layer_weights_against_layout (registry.py:153-174). */
int xp_moe_layer_register(xp_agent_t agent, int instance_index, int layer_ordinal, const xp_moe_layer_desc *desc,
                          const void *gate_up, const void *down, const float *gate_up_bias, const float *down_bias,
                          const void *router, const float *correction_bias, const void *norm_weight, float eps);

/* Lane workspace bytes of one MoE template at `capacity` rows (0 for an invalid
 * descriptor).  Replaces the MoE branch of the capture workspace sizing
 * (execution.py:124-149, plan.workspace). */
size_t xp_moe_step_workspace_bytes(const xp_moe_layer_desc *desc, int64_t capacity);

/* Byte offsets of the MoE step's workspace regions: [0] the gathered (normalised) batch
 * [capacity, hidden] of the payload dtype, [1] the Router logits ([capacity, routed_experts],
 * of the payload dtype for the PAYLOAD precision, fp32 otherwise), [2] routed ids int32 and [3] routed weights fp32
 * [capacity, routed_topk], [4] final ids int32 and [5] final weights fp32 [capacity,
 * effective topk] (the routed ones when there are no shared experts), [6] the Experts
 * workspace (xp_moe_workspace_layout's regions at capacity rows), [7] the total.  No
 * counterpart in the reference (its tests read workspace views directly). */
int xp_moe_step_workspace_layout(const xp_moe_layer_desc *desc, int64_t capacity, size_t *offsets);

/* GraphTemplate of the MoE kind: this Lane's hipGraph for (desc, capacity) -- gather
 * (+ RMSNorm), Router projection and TopK, routing finalisation when there are shared
 * experts, route sort, grouped gate_up and down, combine scattered to the slots.
 * Idempotent per signature.  xp_replay serves registered MoE layers from these templates
 * (smallest captured capacity >= rows among templates whose descriptor equals the layer's).
 * Replaces capture_moe_signature (src/xpool/runtime/ffnagent/registry.py:242-339). */
int xp_moe_template_capture(xp_lane_t lane, const xp_moe_layer_desc *desc, int64_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* XPOOL_AMD_H */
