// Kernel argument records and host-side launch builders shared by the C ABI
// and the Lane/GraphTemplate runtime.  Every kernel takes exactly one argument
// record by value, so a launch is (function, grid, block, LDS bytes, record):
// the same description drives an eager launch and a hipGraph kernel node, and
// rebinding a captured node is a record overwrite.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>

#include "xp_common.hpp"

namespace xp {

struct KernelLaunch {
  const void *func = nullptr;
  dim3 grid{1, 1, 1};
  dim3 block{1, 1, 1};
  unsigned shmem = 0;
  alignas(16) unsigned char args[256] = {};
  size_t args_size = 0;

  template <class Args>
  void set_args(const Args &value) {
    static_assert(sizeof(Args) <= sizeof(args), "kernel argument record too large");
    std::memcpy(args, &value, sizeof(Args));
    args_size = sizeof(Args);
  }
  bool empty() const { return func == nullptr || grid.x == 0; }
};

// Dynamic LDS above 64 KB must be allowed per function before a launch or a graph node
// uses it.  Sets the maximum once per (function, current device) under a lock and returns
// the runtime's status; a failed attempt is not remembered, so the next call retries.
hipError_t enable_large_lds(const void *func);

inline hipError_t launch(const KernelLaunch &kernel, hipStream_t stream) {
  if (kernel.empty()) {
    return hipSuccess;
  }
  if (kernel.shmem > 64 * 1024) {
    if (const hipError_t status = enable_large_lds(kernel.func); status != hipSuccess) {
      return status;
    }
  }
  void *params[] = {const_cast<unsigned char *>(kernel.args)};
  return hipLaunchKernel(kernel.func, kernel.grid, kernel.block, params, kernel.shmem, stream);
}

// ---------------------------------------------------------------- transport
struct CopyArgs {
  uint8_t *destination;
  const uint8_t *source;
  uint64_t bytes;
};

// Payload dtype of a Dense step's kernels (argument records are zero-initialised: bf16).
enum PayloadKind : int32_t { kPayloadBf16 = 0, kPayloadF16 = 1 };

struct GatherArgs {
  const uint16_t *pool;      // [pool_rows, hidden] payload-dtype mailbox
  const int32_t *slots;      // [rows] slot ids
  const uint16_t *norm;      // [hidden] RMSNorm weight, or null for a plain gather
  uint16_t *out;             // [rows, hidden] contiguous batch
  uint32_t *fault;           // sticky fault word, may be null
  int64_t pool_rows;
  int64_t hidden;
  int64_t rows;              // live rows
  float eps;
  int32_t payload;           // PayloadKind of the mailbox, norm weight and batch
};

struct ScatterArgs {
  const uint16_t *values;    // [rows, hidden] contiguous batch
  const int32_t *slots;      // [rows] slot ids
  uint16_t *pool;            // [pool_rows, hidden] mailbox
  uint32_t *fault;
  int64_t pool_rows;
  int64_t hidden;
  int64_t rows;
};

// Fixed-order sum of tensor-parallel partials: out[i] = bf16(sum over k in order of
// float(partials[k][i])), the fp32 sum starting from 0 and rounded once.
constexpr int kMaxPartials = 16;
struct ReduceArgs {
  const uint16_t *partials[kMaxPartials];  // count of them used
  uint16_t *out;
  uint64_t vectors;  // 16-byte groups of 8 bf16
  int count;
};

KernelLaunch make_copy(const CopyArgs &args);
KernelLaunch make_reduce_partials(const ReduceArgs &args);

// ---------------------------------------------------------------- mailbox protocol
// Device image of one Transport arena's control words and request mailbox, shared by the
// Instance side (submit / complete) and the Agent side (evaluate / drain).  Values of the
// status and result words follow src/cext-include/xpool/transport/protocol.hpp:33-49 and
// src/cext-include/xpool/ffn.hpp:43-48.
enum : uint32_t {
  kMailboxDormant = 0,
  kMailboxIdle = 1,
  kMailboxStaging = 2,
  kMailboxPublished = 3,
  kMailboxEvaluated = 4,
  kMailboxClosed = 5,
};
enum : uint32_t { kResultOk = 0, kResultShutdown = 1, kResultProtocolMismatch = 2, kResultTimeout = 3 };
// Instance outcome word while a request is between submit and complete.
constexpr uint32_t kOutcomePending = 0xffffffffu;
constexpr int kMaxDpRanks = 64;
// Liveness deadline of the completion's wait (the reference's kDefaultTimeoutNanoseconds,
// src/cext-include/xpool/utils/wait.cuh:17).
constexpr uint64_t kTransportDefaultTimeoutNs = 5000000000ull;

struct RequestMetadata {
  uint64_t layer_ordinal;
  uint32_t forward_mode;
  uint32_t output_requirement;
  uint32_t dp_row_layout;
  uint32_t reserved;
};

struct alignas(8) Mailbox {
  uint32_t status;       // MailboxStatus, accessed with system-scope acquire / release atomics
  uint32_t result_code;  // published with Evaluated
  uint64_t payload_rows;
  RequestMetadata request;
};

struct alignas(256) TransportArena {
  uint32_t shutdown;            // monotonic terminal fact (arena.hpp ArenaState)
  uint32_t generation_failure;  // sticky canonical failure (ResultCode)
  uint32_t violations;          // sticky count of protocol preconditions found broken
  uint32_t instance_outcome;    // Instance-private: kOutcomePending, then the last request's result
  uint64_t payload_row_capacity;
  uint32_t atn_dp_size;
  uint32_t reserved;
  Mailbox mailbox;
  uint32_t dp_rank_payload_rows[kMaxDpRanks];
};

struct TransportArgs {
  TransportArena *arenas;       // every arena of the resident (drain walks them all)
  int32_t arena;                // the arena this call serves
  int32_t arena_count;
  const void *dp_rows;          // submit: per-DP-rank physical rows (int32 or int64) or null
  uint16_t *output;             // complete: caller output, NaN-filled on failure; probe: observations
  const uint32_t *fault;        // evaluate: the Lane's sticky fault word, or null
  uint64_t output_elements;     // complete
  uint32_t output_nan2;         // complete: two quiet NaNs of the output's payload dtype
  uint64_t payload_rows;        // submit
  uint64_t timeout_ticks;       // complete: wall-clock ticks before the wait gives up
  RequestMetadata request;      // submit
  uint32_t dp_rows_i64;         // submit
  uint32_t dp_rows_count;       // submit: entries of dp_rows (0 = absent)
  uint32_t code;                // publish_failure: result code; probe: scenario
};

KernelLaunch make_transport_open(const TransportArgs &args);
KernelLaunch make_transport_submit(const TransportArgs &args);
KernelLaunch make_transport_evaluate(const TransportArgs &args);
KernelLaunch make_transport_complete(const TransportArgs &args);
KernelLaunch make_transport_settle(const TransportArgs &args);
KernelLaunch make_transport_drain(const TransportArgs &args);
KernelLaunch make_transport_publish_failure(const TransportArgs &args);
KernelLaunch make_transport_probe(const TransportArgs &args);
// ---------------------------------------------------------------- MoE
constexpr int kMoeMaxExperts = 1024;

// Router TopK over [rows, experts] logits (bf16 or fp32), one wavefront per row.
struct RouterTopkArgs {
  const void *logits;
  const float *correction_bias;  // [experts] selection-only bias, or null
  int32_t *ids;                  // [rows, topk]
  float *weights;                // [rows, topk]
  int64_t rows;
  int32_t experts;
  int32_t topk;
  int32_t logits_f32;
  int32_t softmax;  // 1: softmax scores, ties to the lower id; 0: sigmoid, ties to the higher id
  int32_t renormalize;
  int32_t round_to_logits;
  // The bf16 projection's K-slice sums [slices, rows, experts] (fp32), or null: the TopK
  // then adds each logit's slices in slice order, rounds the sum to bf16 once (the order and
  // rounding of stream_reduce_kernel, whose launch this replaces) and stores it at
  // logits_out (= logits) before selecting.
  const float *partials;
  uint16_t *logits_out;
  int32_t slices;
  int32_t payload;  // PayloadKind of 16-bit logits (logits_f32 == 0) and of their roundings
};

// Router logits[rows, experts] = x[rows, hidden] . w[experts, hidden] (w bf16 or fp32) as
// fp32 sums, stored as fp32 or rounded to bf16.
struct RouterLogitsArgs {
  const uint16_t *x;
  const void *w;
  void *logits;
  int64_t rows;
  int64_t hidden;
  int32_t experts;
  int32_t weights_f32;
  int32_t out_payload;  // logits stored in the payload dtype (else fp32)
  int32_t payload;      // PayloadKind of x, of w unless weights_f32, and of payload logits
};

struct FinalizeRoutingArgs {
  const int32_t *routed_ids;     // [capacity, routed_topk]
  const float *routed_weights;
  int32_t *final_ids;            // [capacity, effective_topk]
  float *final_weights;
  const int64_t *payload_rows;   // one device value: live rows; null: every row below capacity
  int64_t capacity;
  int32_t routed_topk;
  int32_t effective_topk;
  int32_t routed_experts;
  float shared_weight;           // 1 / routed_scaling_factor
};

// Route sort: routes (row * topk + slot) grouped by expert, and the expert tile table of
// the grouped projections.
// Rows up to which a MoE step's route sort (one 1024-thread workgroup, one wave per row) also
// runs the Router's TopK.
constexpr int64_t kMoeFusedTopkRows = 16;

struct MoeSortArgs {
  const int32_t *ids;        // [routes] expert of each route, -1 = no route
  const float *weights;      // [routes] route weights
  // Router TopK fused into the sort (fused_topk != 0, at most 16 rows): wave w first picks
  // row w's routes from topk.logits into topk.ids / topk.weights (= ids / weights above).
  RouterTopkArgs topk;
  int32_t fused_topk;
  float *sorted_weight;      // [routes] weight of the route at each sorted position
  int32_t *expert_end;       // [experts] one past the expert's last sorted position
  int32_t *sorted_route;     // [routes] route at each sorted position
  int32_t *tile_expert;      // [max_tiles] expert of each tile, -1 past the last tile
  int32_t *tile_row0;        // [max_tiles] first sorted position of each tile
  int64_t routes;
  int32_t experts;
  int32_t tile_rows;         // BM of the grouped projections
  int32_t max_tiles;
};

struct MoeCombineArgs {
  const uint16_t *routes;    // [rows * topk, hidden] route outputs
  const int32_t *ids;        // [rows, topk]
  uint16_t *out;             // [rows, hidden], or [out_rows, hidden] rows slots[0..rows)
  const int32_t *slots;      // [rows] output row of each row, or null (row r -> r)
  int64_t out_rows;          // rows of `out` when scattering
  int64_t rows;
  int64_t hidden;
  int32_t topk;
  int32_t experts;
  float scale;               // routed scaling factor
  int32_t payload;           // PayloadKind of routes and out
};

// Expert tiles of the grouped projections: Small (16 sorted positions, grouped split
// kernel) for few routes per expert, otherwise the grouped tile kernel on 64-, 128- or
// 256-row expert tiles (Rows128Stream: 128 rows with the weights loaded nontemporally).
enum class MoeTile : int { Small = 0, Rows64 = 1, Rows128Stream = 2, Rows128 = 3, Rows256 = 4 };
int moe_tile_rows(MoeTile tile);
MoeTile choose_moe_tile(int64_t routes, int64_t experts);

KernelLaunch make_router_topk(const RouterTopkArgs &args);
KernelLaunch make_router_logits(const RouterLogitsArgs &args);
KernelLaunch make_finalize_routing(const FinalizeRoutingArgs &args);
KernelLaunch make_moe_sort(const MoeSortArgs &args);
KernelLaunch make_moe_combine(const MoeCombineArgs &args);

// `capacity` sizes the grid (graph templates keep one grid per capacity);
// workgroups beyond the live rows exit immediately.
KernelLaunch make_gather(const GatherArgs &args, int64_t capacity);
KernelLaunch make_scatter(const ScatterArgs &args, int64_t capacity);
bool gather_supported(int64_t hidden);

// ---------------------------------------------------------------- general projection, activation
// Payload dtypes and activation functions of the operator contract (values of the C ABI's
// XP_DTYPE_* and of src/xpool/ffn.py ActivationKind: SILU 1, RELU 2, GELU 3).
constexpr int kDtypeBf16 = 1;
constexpr int kDtypeF16 = 2;
constexpr int kDtypeF32 = 3;
constexpr int kActivationNone = 0;
constexpr int kActivationSilu = 1;
constexpr int kActivationRelu = 2;
constexpr int kActivationGelu = 3;

struct ActivationArgs {
  int32_t function;          // kActivation*
  int32_t approximate_tanh;  // GELU: tanh approximation instead of erf
  int32_t gated;             // Gate/Up pairs: out = f(min(g, limit)) * (clamp(u) + up_offset)
  int32_t has_limit;
  float alpha;               // SiLU slope
  float limit;
  float up_offset;
};

// out = epilogue(bias + x . w^T): x [rows, k], w [n, k], out [rows, n] (gated: [rows, n / 2],
// weights INTERLEAVED), all of `dtype`; bias fp32 [n] or null.
struct ProjectionArgs {
  const void *x;
  const void *w;
  const float *bias;
  void *out;
  int64_t rows;
  int64_t n;
  int64_t k;
  int32_t dtype;
  ActivationArgs act;
};

// output [elements] = activation of inputs ([elements] ungated, [rows, 2 width] gated).
struct ActivationLaunchArgs {
  const void *inputs;
  void *output;
  int64_t elements;
  int64_t width;     // gated: output columns per row
  int32_t dtype;
  int32_t interleaved;
  ActivationArgs act;
};

KernelLaunch make_projection(const ProjectionArgs &args);
KernelLaunch make_activation(const ActivationLaunchArgs &args);

// ---------------------------------------------------------------- GEMMs
// out[t, :] = epilogue(sum_k x[t, k] * w[n, k]) for the live rows t < rows.
// With `gated`, w rows are interleaved Gate/Up (row 2j = gate_j, row 2j+1 = up_j)
// and out[t, j] = silu(gate_j) * up_j; otherwise out[t, n] is the projection.
// `scatter_slots`, when set, redirects output row t to out + slots[t] * ldo.
struct GemmArgs {
  const uint16_t *x;
  const uint16_t *w;
  uint16_t *out;
  const int32_t *scatter_slots;
  float *partials;   // fp32 partial sums [ranges, rows, n] when K is split across workgroups
  int64_t k_slice;   // K columns per range (a multiple of the kernel's load group)
  int64_t k_split;   // split kernel: K ranges per 16-row weight block (1, 2, 4 or 8);
                     // tile kernel: K ranges (grid z)
  int64_t ldx;
  int64_t ldo;
  int64_t rows;      // live rows
  int64_t capacity;  // rows the grid was sized for (>= rows)
  int64_t out_rows;  // bound on scatter slot ids (rows of `out` when scattering)
  int64_t n;         // weight rows
  int64_t k;         // reduction length
  GatedSilu act;
  // Gather fused into the gate_up of a Dense step at decode sizes (stream or split kernel):
  // when set, token row t is row gather_slots[t] of the mailbox `x` ([pool_rows, ldx]),
  // RMS-normalised with `norm` when that is set, bit for bit as gather_rows_kernel does;
  // an out-of-range slot gives a row of quiet NaNs and raises kFaultSlotOutOfRange.
  const int32_t *gather_slots;
  const uint16_t *norm;
  uint32_t *fault;
  int64_t pool_rows;
  float eps;
  // Split kernel with the gather fused (the MoE step's router projection): workgroup 0 also
  // stores the live normalised rows here ([rows, k], row stride k) for the later stages.
  uint16_t *gathered_out;
  // Grouped projection (MoE experts: the tile kernel without a K split, or the grouped
  // split kernel): grid row y is entry y of an expert tile table over rows sorted by
  // expert; the tile multiplies rows [tile_row0[y], min(tile_row0[y] + BM,
  // expert_end[e])) by the weights w + e n k of its
  // expert e = tile_expert[y] (-1: no tile).  With gather_slots set, tile row t reads row
  // gather_slots[t] / gather_divisor of x ([pool_rows, ldx]).  With row_scale set (together
  // with scatter_slots), output row t's fp32 result is multiplied by row_scale[t] before
  // rounding.
  const int32_t *tile_expert;
  const int32_t *tile_row0;
  const int32_t *expert_end;
  const float *row_scale;
  int64_t gather_divisor;
  int32_t payload;  // PayloadKind of x, w and out
  // Grouped projections: fp32 bias of expert e at bias + e bias_stride ([n] per expert), added
  // to the fp32 sum before the rounding point (and before the row scale), or null.
  const float *bias;
  int64_t bias_stride;
};

// SplitGathered: the split kernel's units walked by a persistent grid that gathers the token
// rows once per workgroup (gate_up of a Dense step at decode sizes only).  Resident: the token
// rows (9 to 32) held in registers by a one-workgroup-per-CU grid that walks 16-row weight
// blocks; variant = token groups of 8 (2 or 4), k_slice = the columns of one K part (8 waves
// x 128-wide chunks), k_split = K parts over the grid (more than one: fp32 partial sums and
// the ordered reduction).
enum class GemmKind : int { Split = 1, Tile = 2, Stream = 3, SplitGathered = 4, Resident = 5 };

struct GemmChoice {
  GemmKind kind;
  int variant;      // index into the kind's instantiation table
  int64_t k_slice;  // K columns per range
  int64_t k_split;  // split kernel: K ranges per weight-row block; tile kernel: K ranges
                    // (grid z); 1 for the stream kernel, whose ranges follow from k_slice
  // Tile kernel without a K split only: the last tail_columns weight rows (output columns)
  // go to a second launch on tile shape tail_variant, so that the first launch's grid is
  // whole rounds of one tile per CU and the second fills what would be a partial round.
  int tail_variant = -1;
  int64_t tail_columns = 0;
};

// `split_columns`: the caller launches GemmLaunch::tail, so a tile choice may split columns.
GemmChoice choose_gemm(int64_t capacity, int64_t n, int64_t k, bool gated, bool split_columns = true);
// The gate_up of a Dense step: at decode sizes the stream kernel with the mailbox gather
// fused (`fused` set), otherwise choose_gemm's kernel after a separate gather.
GemmChoice choose_dense_gate_up(int64_t capacity, int64_t n, int64_t k, bool &fused);
// Whether choose_gemm's kernel for an ungated projection at `capacity` rows can take the
// mailbox gather fused: the split kernel with one token group and K <= 4096 (the MoE step's
// router projection then gathers and normalises the rows itself).
bool split_gather_fusable(int64_t capacity, int64_t n, int64_t k);
// Device scratch (fp32 partial sums of the K slices) a projection at `capacity` rows
// needs; 0 when its kernel reduces K inside one workgroup.
size_t gemm_scratch_bytes(GemmChoice choice, int64_t capacity, int64_t n, int64_t k);

// A projection is one kernel, or a kernel writing the partial sums of K ranges (sliced
// stream, split tile) followed by the kernel that adds them in range order and applies the
// epilogue (`reduce`, empty otherwise).  The kernel boundary orders the partials: no cross-workgroup fences.
struct GemmLaunch {
  KernelLaunch main;
  KernelLaunch reduce;
  KernelLaunch tail;   // the trailing columns of a column-split tile choice (empty otherwise)
  bool usable = true;  // false: the choice names no launchable kernel (callers fail the call)
  int64_t slices = 1;  // K ranges summed by `reduce` (fp32 partials [slices, rows, n]); 1: none
};
// `fused_gather`: the gate_up of a Dense step whose choose_dense_gate_up decision fused the
// mailbox gather, or a projection for which split_gather_fusable holds (the kernel variant
// follows that decision, not whether the argument record already holds slot pointers, so a
// template captured with placeholder arguments has the nodes its replays launch).
GemmLaunch make_gemm(const GemmArgs &args, int64_t capacity, bool gated, GemmChoice choice,
                     bool fused_gather = false);
// The grouped projection over an expert tile table of `max_tiles` entries (a multiple of
// 8; otherwise an empty launch), on the grouped tile kernel for `tile` (not Small), whose BM
// is grouped_tile_rows(tile) (the table must be built for that BM).
KernelLaunch make_grouped_gemm(const GemmArgs &args, bool gated, int max_tiles, MoeTile tile);
int grouped_tile_rows(MoeTile tile);
// The grouped projection for few routes per expert, on the grouped split kernel: tiles of
// grouped_split_rows() sorted positions, `live_tiles` the expected number of table entries
// in use (it sizes the K split).
KernelLaunch make_grouped_split(const GemmArgs &args, bool gated, int max_tiles, int64_t live_tiles);
int grouped_split_rows();
std::string gemm_name(GemmChoice choice, bool gated);

}  // namespace xp
