// C ABI, FfnAgent layer table, Executor Lanes and GraphTemplates.
//
// Reference (CrossPool checkout): the native FfnAgent runtime embeds one
// captured CUDA graph per Execution Signature as a SWITCH branch inside a
// resident WHILE graph and patches weight pointers on the device
// (src/cext/ffnagent/runtime.cu:199-369, 701-1047).  HIP has neither
// conditional nor device-updatable graph nodes, so here a Lane owns one
// instantiated hipGraphExec per signature, built from explicit kernel nodes;
// the host selects the layer and the smallest capacity that holds the live rows
// (the rule of runtime.cu:246-253).  A replay either launches the template's kernel
// nodes directly on the stream (the default: a hipGraphLaunch adds about 4-5 us of GPU
// time per Dense replay at decode sizes on MI355X, direct launches none) or rebinds the
// nodes' argument records with hipGraphExecKernelNodeSetParams and launches the graph.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/xpool_amd.h"
#include "xp_kernels.hpp"

namespace xp {
namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

#define XP_HIP_CHECK(expr)                                                                   \
  do {                                                                                       \
    const hipError_t xp_error_ = (expr);                                                     \
    if (xp_error_ != hipSuccess) {                                                           \
      return fail(XP_ERROR_HIP, std::string(#expr) + " failed: " + hipGetErrorString(xp_error_)); \
    }                                                                                        \
  } while (0)

#define XP_REQUIRE(condition, message)                  \
  do {                                                  \
    if (!(condition)) {                                 \
      return fail(XP_ERROR_INVALID_ARGUMENT, message);  \
    }                                                   \
  } while (0)

bool aligned16(const void *pointer) { return (reinterpret_cast<uintptr_t>(pointer) & 15u) == 0; }

// Region alignment of the Lane workspace, the reference's OPERATOR_ALIGNMENT_BYTES
// (src/xpool/runtime/ffnagent/execution.py:16).
constexpr size_t kRegionAlignment = 16;

size_t align_up(size_t value, size_t alignment) { return (value + alignment - 1) / alignment * alignment; }

// Workspace regions of one Dense step at `capacity`: gathered batch [capacity, hidden],
// then the activated intermediate [capacity, intermediate], each 16-byte aligned; then,
// when a projection at this capacity splits K across workgroups (sliced stream or split
// tile kernel), the fp32 partial sums of its K ranges (256-byte aligned, gate_up's then
// down's).
struct DenseWorkspace {
  size_t batch_offset;
  size_t activated_offset;
  size_t gate_up_partials_offset;
  size_t down_partials_offset;
  size_t bytes;
};

DenseWorkspace dense_workspace(int64_t capacity, int64_t hidden, int64_t intermediate) {
  DenseWorkspace layout{};
  layout.batch_offset = 0;
  layout.activated_offset = align_up(static_cast<size_t>(capacity * hidden) * 2, kRegionAlignment);
  size_t cursor = layout.activated_offset + static_cast<size_t>(capacity * intermediate) * 2;
  bool fused = false;
  const size_t gate_up = gemm_scratch_bytes(choose_dense_gate_up(capacity, 2 * intermediate, hidden, fused),
                                            capacity, 2 * intermediate, hidden);
  const size_t down = gemm_scratch_bytes(choose_gemm(capacity, hidden, intermediate, false), capacity, hidden,
                                         intermediate);
  if (gate_up + down > 0) {
    cursor = align_up(cursor, 256);
    layout.gate_up_partials_offset = cursor;
    cursor += gate_up;
    layout.down_partials_offset = cursor;
    cursor += down;
  }
  layout.bytes = cursor;
  return layout;
}

// Buffer resources are 32-bit.  The split and stream kernels address a whole weight matrix
// through one resource, so choose_gemm gives them only matrices below 2^31 bytes and takes
// the tile kernel otherwise; the tile kernel's resources span one tile (at most 256 weight
// or token rows of the reduction length), which the bound on the intermediate size keeps
// below 2^30 bytes (hidden is bounded by the gather's 16384).
constexpr int64_t kMaxIntermediate = int64_t{1} << 21;

// The fused gathers (split, stream and grouped tile kernels) read mailbox rows through one
// buffer resource over the whole pool, and out-of-range lanes use offsets near 2^31, so the
// pool must stay below 2^31 bytes wherever a step may fuse its gather.
int validate_mailbox(int64_t pool_rows, int64_t hidden) {
  XP_REQUIRE(pool_rows * hidden * 2 < (int64_t{1} << 31),
             "mailbox pool must stay below 2 GiB (32-bit buffer range of the fused gathers)");
  return XP_OK;
}

int validate_geometry(int64_t hidden, int64_t intermediate) {
  XP_REQUIRE(hidden > 0 && hidden % 8 == 0, "hidden size must be a positive multiple of 8");
  XP_REQUIRE(intermediate > 0 && intermediate % 8 == 0, "intermediate size must be a positive multiple of 8");
  XP_REQUIRE(gather_supported(hidden), "hidden size exceeds the gather kernel's register row (16384)");
  XP_REQUIRE(intermediate <= kMaxIntermediate, "intermediate size exceeds 2^21 (32-bit tile buffer ranges)");
  return XP_OK;
}

GatedSilu default_activation() { return GatedSilu{1.0f, 0.0f, 0.0f}; }

// The Dense payload dtype of the ABI (XP_DTYPE_BF16 / XP_DTYPE_F16, ffn.hpp:83-85) as the
// kernels' PayloadKind.
int payload_kind(int dtype, int32_t &out) {
  XP_REQUIRE(dtype == XP_DTYPE_BF16 || dtype == XP_DTYPE_F16, "payload dtype must be bf16 or fp16");
  out = dtype == XP_DTYPE_F16 ? kPayloadF16 : kPayloadBf16;
  return XP_OK;
}

// The kernels of one mailbox step, for a given capacity: gather (+ RMSNorm), gate_up
// with the gated SiLU fused (+ its K-slice reduction), down with the scatter fused (+ its
// reduction).  At decode sizes the gather is fused into gate_up and has no launch of its
// own.  The sequence depends only on the capacity and geometry, so a template's node list
// matches every replay's.
struct DenseLaunches {
  KernelLaunch gather;
  GemmLaunch gate_up;
  GemmLaunch down;

  bool usable() const { return gate_up.usable && down.usable; }

  int chain(const KernelLaunch **out) const {
    int count = 0;
    for (const KernelLaunch *kernel :
         {&gather, &gate_up.main, &gate_up.reduce, &gate_up.tail, &down.main, &down.reduce, &down.tail}) {
      if (!kernel->empty()) {
        out[count++] = kernel;
      }
    }
    return count;
  }
};
constexpr int kMaxStepKernels = 7;

// The kernels of one template's step in launch order (a Dense step has at most 7; a MoE
// step at most 9: gather, Router projection and its reduction, TopK, finalisation, sort,
// gate_up, down, combine).
constexpr int kMaxTemplateKernels = 9;
struct StepChain {
  KernelLaunch kernels[kMaxTemplateKernels];
  int count = 0;
  bool usable = true;  // false: a projection of the step has no launchable kernel choice
  void add(const KernelLaunch &kernel) {
    if (!kernel.empty()) {
      kernels[count++] = kernel;
    }
  }
};

struct DenseBinding {
  const uint16_t *pool_in;
  uint16_t *pool_out;
  int64_t pool_rows;
  const int32_t *slots;
  int64_t rows;
  int64_t hidden;
  int64_t intermediate;
  const uint16_t *gate_up;
  const uint16_t *down;
  const uint16_t *norm;
  float eps;
  uint8_t *workspace;
  uint32_t *fault;
  int32_t payload;  // PayloadKind
};

DenseLaunches make_dense_launches(const DenseBinding &b, int64_t capacity) {
  const DenseWorkspace layout = dense_workspace(capacity, b.hidden, b.intermediate);
  uint16_t *batch = reinterpret_cast<uint16_t *>(b.workspace + layout.batch_offset);
  uint16_t *activated = reinterpret_cast<uint16_t *>(b.workspace + layout.activated_offset);
  DenseLaunches launches;

  bool fused = false;
  const GemmChoice gate_up_choice = choose_dense_gate_up(capacity, 2 * b.intermediate, b.hidden, fused);
  if (!fused) {
    GatherArgs gather{};
    gather.pool = b.pool_in;
    gather.slots = b.slots;
    gather.norm = b.norm;
    gather.out = batch;
    gather.fault = b.fault;
    gather.pool_rows = b.pool_rows;
    gather.hidden = b.hidden;
    gather.rows = b.rows;
    gather.eps = b.eps;
    gather.payload = b.payload;
    launches.gather = make_gather(gather, capacity);
  }

  GemmArgs gate_up{};
  gate_up.x = fused ? b.pool_in : batch;
  gate_up.w = b.gate_up;
  gate_up.out = activated;
  gate_up.scatter_slots = nullptr;
  gate_up.ldx = b.hidden;
  gate_up.ldo = b.intermediate;
  gate_up.rows = b.rows;
  gate_up.out_rows = capacity;
  gate_up.n = 2 * b.intermediate;
  gate_up.k = b.hidden;
  gate_up.act = default_activation();
  gate_up.payload = b.payload;
  gate_up.partials = reinterpret_cast<float *>(b.workspace + layout.gate_up_partials_offset);
  if (fused) {
    gate_up.gather_slots = b.slots;
    gate_up.norm = b.norm;
    gate_up.fault = b.fault;
    gate_up.pool_rows = b.pool_rows;
    gate_up.eps = b.eps;
  }
  launches.gate_up = make_gemm(gate_up, capacity, true, gate_up_choice, fused);

  GemmArgs down{};
  down.x = activated;
  down.w = b.down;
  down.out = b.pool_out;
  down.scatter_slots = b.slots;
  down.ldx = b.intermediate;
  down.ldo = b.hidden;
  down.rows = b.rows;
  down.out_rows = b.pool_rows;
  down.n = b.hidden;
  down.k = b.intermediate;
  down.act = default_activation();
  down.payload = b.payload;
  down.partials = reinterpret_cast<float *>(b.workspace + layout.down_partials_offset);
  launches.down = make_gemm(down, capacity, false, choose_gemm(capacity, down.n, down.k, false));
  return launches;
}

// Point a kernel-level projection at its caller-provided scratch for K-slice partials.
int bind_scratch(GemmArgs &args, GemmChoice choice, void *workspace, size_t workspace_bytes) {
  const size_t needed = gemm_scratch_bytes(choice, args.rows, args.n, args.k);
  if (needed == 0) {
    return XP_OK;
  }
  if (workspace == nullptr || workspace_bytes < needed) {
    return fail(XP_ERROR_CAPACITY, "projection workspace is smaller than xp_gemm_workspace_bytes (" +
                                       std::to_string(needed) + " bytes)");
  }
  XP_REQUIRE(aligned16(workspace), "projection workspace must be 16-byte aligned");
  args.partials = static_cast<float *>(workspace);
  return XP_OK;
}

constexpr const char *kUnusableChoice = "no launchable projection kernel for this geometry (empty K range)";

int launch_gemm(const GemmLaunch &kernels, hipStream_t stream) {
  if (!kernels.usable) {
    return fail(XP_ERROR_INVALID_ARGUMENT, kUnusableChoice);
  }
  XP_HIP_CHECK(launch(kernels.main, stream));
  XP_HIP_CHECK(launch(kernels.reduce, stream));
  XP_HIP_CHECK(launch(kernels.tail, stream));
  return XP_OK;
}

hipKernelNodeParams node_params(const KernelLaunch &kernel, void **params) {
  hipKernelNodeParams node{};
  node.func = const_cast<void *>(kernel.func);
  node.gridDim = kernel.grid;
  node.blockDim = kernel.block;
  node.sharedMemBytes = kernel.shmem;
  params[0] = const_cast<unsigned char *>(kernel.args);
  node.kernelParams = params;
  node.extra = nullptr;
  return node;
}

}  // namespace
}  // namespace xp

using namespace xp;

struct Layer {
  int instance_index;
  int layer_ordinal;
  int64_t hidden;
  int64_t intermediate;
  const uint16_t *gate_up;
  const uint16_t *down;
  const uint16_t *norm;
  float eps;
  int32_t payload = kPayloadBf16;  // PayloadKind of the weights, norm and mailbox (Dense and MoE)
  int kind = XP_LAYER_DENSE;
  // MoE layers: the execution identity, the Router projection and its correction bias.
  xp_moe_layer_desc moe{};
  const void *router = nullptr;
  const float *correction_bias = nullptr;
  const float *gate_up_bias = nullptr;  // fp32 projection biases (moe.biases), or null
  const float *down_bias = nullptr;
};

struct xp_agent {
  int device = 0;
  std::mutex mutex;
  std::vector<Layer> layers;
  int live_lanes = 0;
};

struct Template {
  int kind = XP_LAYER_DENSE;
  int64_t hidden = 0;
  int64_t intermediate = 0;
  int32_t payload = kPayloadBf16;
  int64_t capacity = 0;
  xp_moe_layer_desc moe{};  // MoE templates: the signature they were captured for
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipGraphNode_t nodes[kMaxTemplateKernels] = {};
  int node_count = 0;
  // Argument records last bound to each node: a replay rebinds only the nodes whose
  // record changed.
  KernelLaunch bound[kMaxTemplateKernels];
};

struct xp_lane {
  xp_agent *agent = nullptr;
  hipStream_t stream = nullptr;
  uint8_t *workspace = nullptr;
  size_t workspace_bytes = 0;
  uint32_t *fault = nullptr;
  std::mutex mutex;
  std::vector<std::unique_ptr<Template>> templates;  // sorted by (hidden, intermediate, capacity)
  // Replays launch the template's kernels directly on the stream unless graph dispatch is
  // selected: each hipGraphLaunch adds GPU time before the graph's first kernel (about
  // 4-5 us per Dense replay at decode sizes on MI355X), while back-to-back kernel launches
  // leave no gap.
  bool graph_dispatch = false;
};

// A Transport resident: the device array of arenas it serves (one per Instance rank) and
// the host facts the C ABI validates against.  Replaces the AtnAgent-owned arenas and the
// TransportResident of src/cext/transport/atnagent.cpp (one Resident block per arena).
struct xp_transport {
  int device = 0;
  int arena_count = 0;
  TransportArena *arenas = nullptr;
  std::vector<int64_t> capacities;
  std::vector<int32_t> atn_dp_sizes;
  uint64_t wall_clock_khz = 0;
  std::mutex mutex;  // serialises host calls, as the Attachment mutex does (instance.hpp:113-114)
};

namespace {

// Workspace of one Experts call: expert ends, sorted routes, the tile table (sized for the
// smaller tile, an upper bound for both), the activated routes [routes, intermediate] and
// the route outputs [routes, hidden], each 256-byte aligned.
struct MoeWorkspace {
  size_t expert_end;
  size_t sorted_route;
  size_t sorted_weight;
  size_t tile_expert;
  size_t tile_row0;
  size_t activated;
  size_t route_out;
  size_t bytes;
  int max_tiles;
};

// Entries of an expert tile table of `tile_rows`-route tiles: every expert with c >= 1
// routes takes ceil(c / tile_rows) <= c / tile_rows + 1 tiles, so the table needs at most
// ceil(routes / tile_rows) + min(experts, routes) entries; rounded up to a multiple of 8 for
// the grouped tile kernel's XCD mapping.  Grid rows past the table's live entries exit at
// once, so a tight bound keeps decode grids small.
int moe_tile_bound(int64_t routes, int64_t experts, int64_t tile_rows) {
  const int64_t live_experts = experts < routes ? experts : routes;
  return static_cast<int>(((routes + tile_rows - 1) / tile_rows + live_experts + 7) / 8 * 8);
}

MoeWorkspace moe_workspace(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk) {
  MoeWorkspace layout{};
  const int64_t routes = rows * topk;
  // Tile table entries: the bound for the smaller tile size covers both.
  layout.max_tiles = moe_tile_bound(routes, experts, moe_tile_rows(MoeTile::Small));
  size_t cursor = 0;
  auto region = [&](size_t bytes) {
    const size_t offset = cursor;
    cursor = align_up(cursor + bytes, 256);
    return offset;
  };
  layout.expert_end = region(static_cast<size_t>(experts) * 4);
  layout.sorted_route = region(static_cast<size_t>(routes) * 4);
  layout.sorted_weight = region(static_cast<size_t>(routes) * 4);
  layout.tile_expert = region(static_cast<size_t>(layout.max_tiles) * 4);
  layout.tile_row0 = region(static_cast<size_t>(layout.max_tiles) * 4);
  layout.activated = region(static_cast<size_t>(routes * intermediate) * 2);
  layout.route_out = region(static_cast<size_t>(routes * hidden) * 2);
  layout.bytes = cursor;
  return layout;
}

// Router workspace: the logits [rows, experts] (bf16 for the PAYLOAD precision, fp32
// otherwise), then the PAYLOAD projection's K-slice scratch.
struct RouterWorkspace {
  size_t logits;
  size_t scratch;
  size_t scratch_bytes;
  size_t bytes;
};

// PAYLOAD logits go through the MFMA projection kernels when their geometry allows it.
bool router_uses_mfma(int64_t hidden, int64_t experts, int precision) {
  return precision == XP_ROUTER_PRECISION_PAYLOAD && hidden % 8 == 0 && experts % 8 == 0;
}

RouterWorkspace router_workspace(int64_t rows, int64_t hidden, int64_t experts, int precision) {
  RouterWorkspace layout{};
  const bool payload = precision == XP_ROUTER_PRECISION_PAYLOAD;
  layout.logits = 0;
  layout.scratch = align_up(static_cast<size_t>(rows * experts) * (payload ? 2 : 4), 256);
  layout.scratch_bytes = router_uses_mfma(hidden, experts, precision)
                             ? gemm_scratch_bytes(choose_gemm(rows, experts, hidden, false, false), rows, experts, hidden)
                             : 0;
  layout.bytes = layout.scratch + layout.scratch_bytes;
  return layout;
}

int validate_router(int64_t experts, int64_t topk, int algorithm, int precision, int weight_rounding) {
  XP_REQUIRE(precision == XP_ROUTER_PRECISION_PAYLOAD || precision == XP_ROUTER_PRECISION_FP32 ||
                 precision == XP_ROUTER_PRECISION_FP32_LOGITS,
             "router projection precision is unknown");
  XP_REQUIRE(experts >= 1 && experts <= kMoeMaxExperts, "the router supports 1 to 1024 experts");
  XP_REQUIRE(topk >= 1 && topk <= experts && topk <= 64, "topk must be between 1 and min(experts, 64)");
  XP_REQUIRE(algorithm == XP_ROUTER_SOFTMAX || algorithm == XP_ROUTER_SIGMOID, "router algorithm is unknown");
  XP_REQUIRE(weight_rounding == XP_TOPK_ROUNDING_NONE || weight_rounding == XP_TOPK_ROUNDING_LOGITS_DTYPE,
             "TopK weight rounding is unknown");
  return XP_OK;
}

int validate_experts(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk) {
  XP_REQUIRE(hidden > 0 && hidden % 8 == 0 && intermediate > 0 && intermediate % 8 == 0,
             "hidden and intermediate sizes must be positive multiples of 8");
  XP_REQUIRE(experts >= 1 && experts <= kMoeMaxExperts, "Experts support 1 to 1024 experts");
  XP_REQUIRE(topk >= 1 && topk <= experts, "topk must be between 1 and the expert count");
  XP_REQUIRE(rows * topk <= (int64_t{1} << 30), "too many routes for one call");
  // The projections address the token rows, the activated routes and one expert's weights
  // through 32-bit buffer ranges.
  XP_REQUIRE(rows * hidden * 2 < (int64_t{1} << 31) && rows * topk * intermediate * 2 < (int64_t{1} << 31) &&
                 2 * intermediate * hidden * 2 < (int64_t{1} << 31),
             "Experts tensors must stay below 2 GiB per buffer range");
  XP_REQUIRE(moe_tile_bound(rows * topk, experts, moe_tile_rows(MoeTile::Small)) <= 65535,
             "too many expert tiles for one call");
  return XP_OK;
}

// Router kernels for `rows` live rows with grids for `capacity` rows (the kernels bound
// themselves by the live rows), so that one template's nodes serve every smaller replay.
struct RouterBinding {
  const uint16_t *x;
  const void *w;
  const float *correction_bias;
  int32_t *ids;
  float *weights;
  uint8_t *workspace;  // router_workspace(capacity, ...)
  int64_t rows;
  int64_t hidden;
  int64_t experts;
  int64_t topk;
  int algorithm;
  int precision;
  int renormalize;
  int weight_rounding;
  // Gather fused into the MFMA projection (router_gather_fusable): the rows are mailbox rows
  // slots[t] of pool, RMS-normalised with norm when set, and the projection also stores them
  // in batch_out (the step's batch, which x names).
  bool fused_gather = false;
  uint16_t *batch_out = nullptr;
  const uint16_t *pool = nullptr;
  const int32_t *slots = nullptr;
  const uint16_t *norm = nullptr;
  uint32_t *fault = nullptr;
  int64_t pool_rows = 0;
  float eps = 0.0f;
  int32_t payload = kPayloadBf16;  // PayloadKind of x, of the weights unless FP32, of PAYLOAD logits
};

struct RouterLaunches {
  KernelLaunch logits;         // MFMA projection or the fp32 logits kernel
  KernelLaunch logits_reduce;  // K-slice reduction of the MFMA projection (empty: the TopK sums the slices)
  KernelLaunch topk;
  RouterTopkArgs topk_args;    // the TopK launch's arguments (live rows)
};

// Whether a MoE step at `capacity` rows runs its gather inside the router projection: the
// MFMA projection on the split kernel with one token group.
bool router_gather_fusable(const xp_moe_layer_desc &d, int64_t capacity) {
  return router_uses_mfma(d.hidden, d.routed_experts, d.precision) &&
         split_gather_fusable(capacity, d.routed_experts, d.hidden);
}

RouterLaunches make_router_launches(const RouterBinding &b, int64_t capacity) {
  const RouterWorkspace layout = router_workspace(capacity, b.hidden, b.experts, b.precision);
  void *logits = b.workspace + layout.logits;
  RouterLaunches launches;
  const float *partials = nullptr;
  int64_t slices = 1;
  if (router_uses_mfma(b.hidden, b.experts, b.precision)) {
    // logits = bf16(x . w^T): the Dense projection kernels, no epilogue.
    GemmArgs args{};
    args.x = b.x;
    if (b.fused_gather) {
      args.x = b.pool;
      args.gather_slots = b.slots;
      args.norm = b.norm;
      args.fault = b.fault;
      args.pool_rows = b.pool_rows;
      args.eps = b.eps;
      args.gathered_out = b.batch_out;
    }
    args.w = static_cast<const uint16_t *>(b.w);
    args.out = static_cast<uint16_t *>(logits);
    args.payload = b.payload;
    args.partials = layout.scratch_bytes > 0 ? reinterpret_cast<float *>(b.workspace + layout.scratch) : nullptr;
    args.ldx = b.hidden;
    args.ldo = b.experts;
    args.rows = b.rows;
    args.out_rows = capacity;
    args.n = b.experts;
    args.k = b.hidden;
    args.act = default_activation();
    // (no column split: the Router's launch list has room for one projection kernel)
    const GemmLaunch gemm = make_gemm(args, capacity, false,
                                      choose_gemm(capacity, b.experts, b.hidden, false, false), b.fused_gather);
    launches.logits = gemm.main;
    if (gemm.slices > 1) {
      // The TopK adds the K slices itself and stores the logits: no reduction launch (at one
      // to sixteen rows a quarter of the Router's time, most of it the launch).
      partials = args.partials;
      slices = gemm.slices;
    }
  } else {
    RouterLogitsArgs args{};
    args.x = b.x;
    args.w = b.w;
    args.logits = logits;
    args.rows = capacity;
    args.hidden = b.hidden;
    args.experts = static_cast<int32_t>(b.experts);
    args.weights_f32 = b.precision == XP_ROUTER_PRECISION_FP32 ? 1 : 0;
    args.out_payload = b.precision == XP_ROUTER_PRECISION_PAYLOAD ? 1 : 0;
    args.payload = b.payload;
    launches.logits = make_router_logits(args);
    args.rows = b.rows;
    launches.logits.set_args(args);
  }
  RouterTopkArgs topk{};
  topk.logits = logits;
  topk.correction_bias = b.correction_bias;
  topk.ids = b.ids;
  topk.weights = b.weights;
  topk.rows = capacity;
  topk.experts = static_cast<int32_t>(b.experts);
  topk.topk = static_cast<int32_t>(b.topk);
  topk.logits_f32 = b.precision == XP_ROUTER_PRECISION_PAYLOAD ? 0 : 1;
  topk.softmax = b.algorithm == XP_ROUTER_SOFTMAX ? 1 : 0;
  topk.renormalize = b.renormalize != 0 ? 1 : 0;
  topk.round_to_logits = b.weight_rounding == XP_TOPK_ROUNDING_LOGITS_DTYPE ? 1 : 0;
  topk.partials = partials;
  topk.logits_out = partials != nullptr ? static_cast<uint16_t *>(logits) : nullptr;
  topk.slices = static_cast<int32_t>(slices);
  topk.payload = b.payload;
  launches.topk = make_router_topk(topk);
  topk.rows = b.rows;
  launches.topk.set_args(topk);
  launches.topk_args = topk;
  return launches;
}

// Experts kernels (route sort, grouped gate_up, grouped down, combine) for `rows` live rows,
// with the tile choice, the tile table bound and the grids of `capacity` rows.
struct ExpertsBinding {
  const uint16_t *x;  // [rows, hidden] token rows
  const uint16_t *w_gate_up;
  const uint16_t *w_down;
  const int32_t *ids;  // [rows, topk]
  const float *weights;
  uint16_t *out;             // [rows, hidden], or the mailbox when out_slots is set
  const int32_t *out_slots;  // mailbox row of each row, or null
  int64_t out_rows;
  uint8_t *workspace;  // moe_workspace(capacity, ...)
  int64_t rows;
  int64_t hidden;
  int64_t intermediate;
  int64_t experts;
  int64_t topk;
  float scale;
  GatedSilu act;
  int32_t payload = kPayloadBf16;  // PayloadKind of x, the weights, the routes and out
  // The Router's TopK run by the sort kernel (at most 16 rows, no shared experts), or null.
  const RouterTopkArgs *fused_topk = nullptr;
  // fp32 projection biases ([experts, 2 intermediate] and [experts, hidden]), or null.
  const float *bias_gate_up = nullptr;
  const float *bias_down = nullptr;
};

struct ExpertsLaunches {
  KernelLaunch sort;
  KernelLaunch gate_up;
  KernelLaunch down;
  KernelLaunch combine;
};

int make_experts_launches(const ExpertsBinding &b, int64_t capacity, ExpertsLaunches &out) {
  const MoeWorkspace layout = moe_workspace(capacity, b.hidden, b.intermediate, b.experts, b.topk);
  int32_t *expert_end = reinterpret_cast<int32_t *>(b.workspace + layout.expert_end);
  int32_t *sorted_route = reinterpret_cast<int32_t *>(b.workspace + layout.sorted_route);
  float *sorted_weight = reinterpret_cast<float *>(b.workspace + layout.sorted_weight);
  int32_t *tile_expert = reinterpret_cast<int32_t *>(b.workspace + layout.tile_expert);
  int32_t *tile_row0 = reinterpret_cast<int32_t *>(b.workspace + layout.tile_row0);
  uint16_t *activated = reinterpret_cast<uint16_t *>(b.workspace + layout.activated);
  uint16_t *route_out = reinterpret_cast<uint16_t *>(b.workspace + layout.route_out);
  const int64_t routes = b.rows * b.topk;
  const int64_t capacity_routes = capacity * b.topk;
  const MoeTile tile = choose_moe_tile(capacity_routes, b.experts);
  const int tile_rows = moe_tile_rows(tile);
  const int max_tiles = moe_tile_bound(capacity_routes, b.experts, tile_rows);
  XP_REQUIRE(max_tiles <= 65535, "too many expert tiles for one call");

  MoeSortArgs sort{};
  sort.ids = b.ids;
  sort.weights = b.weights;
  sort.sorted_weight = sorted_weight;
  sort.expert_end = expert_end;
  sort.sorted_route = sorted_route;
  sort.tile_expert = tile_expert;
  sort.tile_row0 = tile_row0;
  sort.routes = routes;
  sort.experts = static_cast<int32_t>(b.experts);
  sort.tile_rows = tile_rows;
  sort.max_tiles = max_tiles;
  if (b.fused_topk != nullptr) {
    // moe_sort_kernel runs the fused TopK with one wave per row.
    XP_REQUIRE(b.fused_topk->rows <= kMoeFusedTopkRows, "fused TopK rows exceed the route sort's waves");
    sort.topk = *b.fused_topk;
    sort.fused_topk = 1;
  }
  out.sort = make_moe_sort(sort);

  // gate_up gathers the token row of each sorted route (route / topk) itself and writes the
  // activated rows in sorted order; down scales each sorted row by its route weight and
  // writes it to the route's row.
  GemmArgs up{};
  up.x = b.x;
  up.gather_slots = sorted_route;
  up.gather_divisor = b.topk;
  up.pool_rows = b.rows;
  up.w = b.w_gate_up;
  up.out = activated;
  up.ldx = b.hidden;
  up.ldo = b.intermediate;
  up.rows = routes;
  up.capacity = routes;
  up.out_rows = routes;
  up.n = 2 * b.intermediate;
  up.k = b.hidden;
  up.act = b.act;
  up.tile_expert = tile_expert;
  up.tile_row0 = tile_row0;
  up.expert_end = expert_end;
  up.payload = b.payload;
  up.bias = b.bias_gate_up;
  up.bias_stride = 2 * b.intermediate;

  GemmArgs dn = up;
  dn.x = activated;
  dn.gather_slots = nullptr;
  dn.w = b.w_down;
  dn.out = route_out;
  dn.scatter_slots = sorted_route;
  dn.row_scale = sorted_weight;
  dn.ldx = b.intermediate;
  dn.ldo = b.hidden;
  dn.n = b.hidden;
  dn.k = b.intermediate;
  dn.act = default_activation();
  dn.bias = b.bias_down;
  dn.bias_stride = b.hidden;

  if (tile != MoeTile::Small) {
    // Many routes per expert: the Dense tile kernel in its grouped mode, on expert tiles of
    // moe_tile_rows(tile) rows (the table the sort builds).
    out.gate_up = make_grouped_gemm(up, true, max_tiles, tile);
    out.down = make_grouped_gemm(dn, false, max_tiles, tile);
    if (out.gate_up.empty() || out.down.empty()) {
      return fail(XP_ERROR_STATE, "no grouped tile kernel for this expert tile table");
    }
  } else {
    // Few routes per expert: each touched expert's weights streamed by the grouped split
    // kernel; about one tile per touched expert.
    if (moe_tile_rows(MoeTile::Small) != grouped_split_rows()) {
      return fail(XP_ERROR_STATE, "expert tile table and grouped split kernel disagree on the tile rows");
    }
    const int64_t live_tiles = b.experts < capacity_routes ? b.experts : capacity_routes;
    out.gate_up = make_grouped_split(up, true, max_tiles, live_tiles);
    out.down = make_grouped_split(dn, false, max_tiles, live_tiles);
  }

  MoeCombineArgs combine{};
  combine.routes = route_out;
  combine.ids = b.ids;
  combine.out = b.out;
  combine.slots = b.out_slots;
  combine.out_rows = b.out_rows;
  combine.rows = capacity;
  combine.hidden = b.hidden;
  combine.topk = static_cast<int32_t>(b.topk);
  combine.experts = static_cast<int32_t>(b.experts);
  combine.scale = b.scale;
  combine.payload = b.payload;
  out.combine = make_moe_combine(combine);
  combine.rows = b.rows;
  out.combine.set_args(combine);
  return XP_OK;
}

// ------------------------------------------------------------------ MoE step
int64_t effective_topk(const xp_moe_layer_desc &d) { return d.routed_topk + (d.experts - d.routed_experts); }

bool same_moe(const xp_moe_layer_desc &a, const xp_moe_layer_desc &b) {
  return a.hidden == b.hidden && a.intermediate == b.intermediate && a.experts == b.experts &&
         a.routed_experts == b.routed_experts && a.routed_topk == b.routed_topk && a.algorithm == b.algorithm &&
         a.precision == b.precision && (a.renormalize != 0) == (b.renormalize != 0) &&
         a.weight_rounding == b.weight_rounding && a.routed_scaling_factor == b.routed_scaling_factor &&
         a.alpha == b.alpha && a.limit == b.limit && a.up_offset == b.up_offset && a.payload == b.payload &&
         a.activation == b.activation && a.approximate_tanh == b.approximate_tanh && a.biases == b.biases;
}

int validate_moe_desc(const xp_moe_layer_desc *d) {
  XP_REQUIRE(d != nullptr, "MoE layer descriptor must be non-null");
  XP_REQUIRE(d->hidden > 0 && d->hidden % 8 == 0 && d->intermediate > 0 && d->intermediate % 8 == 0,
             "hidden and intermediate sizes must be positive multiples of 8");
  XP_REQUIRE(gather_supported(d->hidden), "hidden size exceeds the gather kernel's register row (16384)");
  XP_REQUIRE(d->experts >= 1 && d->experts <= kMoeMaxExperts, "Experts support 1 to 1024 experts");
  XP_REQUIRE(d->routed_experts >= 1 && d->routed_experts <= d->experts,
             "routed experts must be between 1 and the expert count");
  if (const int status = validate_router(d->routed_experts, d->routed_topk, d->algorithm, d->precision,
                                         d->weight_rounding);
      status != XP_OK) {
    return status;
  }
  XP_REQUIRE(d->routed_scaling_factor > 0.0f && d->routed_scaling_factor < __builtin_inff(),
             "routed scaling factor must be finite and positive");
  XP_REQUIRE(d->activation == XP_ACTIVATION_SILU || d->activation == XP_ACTIVATION_RELU ||
                 d->activation == XP_ACTIVATION_GELU,
             "MoE activation must be SiLU, ReLU or GELU");
  XP_REQUIRE(d->approximate_tanh == 0 || (d->activation == XP_ACTIVATION_GELU && d->approximate_tanh == 1),
             "the tanh approximation is GELU's only");
  XP_REQUIRE(d->biases >= 0 && d->biases <= 3, "MoE biases are bit 0 (gate_up) and bit 1 (down)");
  XP_REQUIRE(d->alpha > 0.0f && d->alpha < __builtin_inff(), "SiLU alpha must be positive and finite");
  XP_REQUIRE(d->limit >= 0.0f && d->limit < __builtin_inff() && std::isfinite(d->up_offset),
             "gate limit must be finite and non-negative (0 = none) and the up offset finite");
  XP_REQUIRE(2 * d->intermediate * d->hidden * 2 < (int64_t{1} << 31),
             "one expert's gate_up must stay below 2 GiB (32-bit buffer range)");
  int32_t payload = kPayloadBf16;
  return payload_kind(d->payload, payload);
}

// Lane workspace of a MoE step at `capacity`: the gathered batch, the Router workspace
// (logits first), routed ids and weights, final ids and weights when shared experts add
// slots, then the Experts workspace; each region 256-byte aligned.
struct MoeStepWorkspace {
  size_t batch;
  size_t router;
  size_t routed_ids;
  size_t routed_weights;
  size_t final_ids;
  size_t final_weights;
  size_t experts;
  size_t bytes;
};

MoeStepWorkspace moe_step_workspace(const xp_moe_layer_desc &d, int64_t capacity) {
  MoeStepWorkspace layout{};
  size_t cursor = 0;
  auto region = [&](size_t bytes) {
    const size_t offset = cursor;
    cursor = align_up(cursor + bytes, 256);
    return offset;
  };
  const int64_t topk = effective_topk(d);
  layout.batch = region(static_cast<size_t>(capacity * d.hidden) * 2);
  layout.router = region(router_workspace(capacity, d.hidden, d.routed_experts, d.precision).bytes);
  layout.routed_ids = region(static_cast<size_t>(capacity * d.routed_topk) * 4);
  layout.routed_weights = region(static_cast<size_t>(capacity * d.routed_topk) * 4);
  if (topk > d.routed_topk) {
    layout.final_ids = region(static_cast<size_t>(capacity * topk) * 4);
    layout.final_weights = region(static_cast<size_t>(capacity * topk) * 4);
  } else {
    layout.final_ids = layout.routed_ids;
    layout.final_weights = layout.routed_weights;
  }
  layout.experts = region(moe_workspace(capacity, d.hidden, d.intermediate, d.experts, topk).bytes);
  layout.bytes = cursor;
  return layout;
}

int validate_moe_capacity(const xp_moe_layer_desc &d, int64_t capacity) {
  XP_REQUIRE(capacity > 0, "template capacity must be positive");
  return validate_experts(capacity, d.hidden, d.intermediate, d.experts, effective_topk(d));
}

// One MoE mailbox step: gather (+ RMSNorm) into the batch, Router, finalisation (shared
// experts only), Experts with the combine scattered to the slots of pool_out.  Grids and
// kernel choices follow `capacity`; the argument records carry the live rows.
struct MoeStepBinding {
  const uint16_t *pool_in;
  uint16_t *pool_out;
  int64_t pool_rows;
  const int32_t *slots;
  int64_t rows;
  uint8_t *workspace;
  uint32_t *fault;
};

int make_moe_step(const Layer &layer, const MoeStepBinding &b, int64_t capacity, StepChain &chain) {
  const xp_moe_layer_desc &d = layer.moe;
  const MoeStepWorkspace layout = moe_step_workspace(d, capacity);
  uint16_t *batch = reinterpret_cast<uint16_t *>(b.workspace + layout.batch);
  int32_t *routed_ids = reinterpret_cast<int32_t *>(b.workspace + layout.routed_ids);
  float *routed_weights = reinterpret_cast<float *>(b.workspace + layout.routed_weights);
  int32_t *final_ids = reinterpret_cast<int32_t *>(b.workspace + layout.final_ids);
  float *final_weights = reinterpret_cast<float *>(b.workspace + layout.final_weights);
  const int64_t topk = effective_topk(d);

  // At decode sizes the gather runs inside the router projection and the TopK inside the
  // route sort (two launches fewer; the same kernels' code, so the same bits).  Both follow
  // from the capacity, so a template's node list matches every replay's.
  const bool fuse_gather = router_gather_fusable(d, capacity);
  const bool fuse_topk = capacity <= kMoeFusedTopkRows && topk == d.routed_topk;
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(d.payload, payload); status != XP_OK) {
    return status;
  }
  if (!fuse_gather) {
    GatherArgs gather{};
    gather.pool = b.pool_in;
    gather.slots = b.slots;
    gather.norm = layer.norm;
    gather.out = batch;
    gather.fault = b.fault;
    gather.pool_rows = b.pool_rows;
    gather.hidden = d.hidden;
    gather.rows = b.rows;
    gather.eps = layer.eps;
    gather.payload = payload;
    chain.add(make_gather(gather, capacity));
  }

  RouterBinding router{};
  router.x = batch;
  router.w = layer.router;
  router.correction_bias = layer.correction_bias;
  router.ids = routed_ids;
  router.weights = routed_weights;
  router.workspace = b.workspace + layout.router;
  router.rows = b.rows;
  router.hidden = d.hidden;
  router.experts = d.routed_experts;
  router.topk = d.routed_topk;
  router.algorithm = d.algorithm;
  router.precision = d.precision;
  router.renormalize = d.renormalize;
  router.weight_rounding = d.weight_rounding;
  router.payload = payload;
  if (fuse_gather) {
    router.fused_gather = true;
    router.batch_out = batch;
    router.pool = b.pool_in;
    router.slots = b.slots;
    router.norm = layer.norm;
    router.fault = b.fault;
    router.pool_rows = b.pool_rows;
    router.eps = layer.eps;
  }
  const RouterLaunches routing = make_router_launches(router, capacity);
  chain.add(routing.logits);
  chain.add(routing.logits_reduce);
  if (!fuse_topk) {
    chain.add(routing.topk);
  }

  if (topk > d.routed_topk) {
    // Shared experts: every live row also takes slots routed_experts + s (weight
    // 1 / scaling, which the combine's scale cancels).
    FinalizeRoutingArgs finalize{};
    finalize.routed_ids = routed_ids;
    finalize.routed_weights = routed_weights;
    finalize.final_ids = final_ids;
    finalize.final_weights = final_weights;
    finalize.payload_rows = nullptr;
    finalize.capacity = capacity;
    finalize.routed_topk = static_cast<int32_t>(d.routed_topk);
    finalize.effective_topk = static_cast<int32_t>(topk);
    finalize.routed_experts = static_cast<int32_t>(d.routed_experts);
    finalize.shared_weight = 1.0f / d.routed_scaling_factor;
    KernelLaunch kernel = make_finalize_routing(finalize);
    finalize.capacity = b.rows;
    kernel.set_args(finalize);
    chain.add(kernel);
  }

  ExpertsBinding experts{};
  experts.x = batch;
  experts.w_gate_up = layer.gate_up;
  experts.w_down = layer.down;
  experts.ids = final_ids;
  experts.weights = final_weights;
  experts.out = b.pool_out;
  experts.out_slots = b.slots;
  experts.out_rows = b.pool_rows;
  experts.workspace = b.workspace + layout.experts;
  experts.rows = b.rows;
  experts.hidden = d.hidden;
  experts.intermediate = d.intermediate;
  experts.experts = d.experts;
  experts.topk = topk;
  experts.scale = d.routed_scaling_factor;
  experts.act = GatedSilu{d.alpha, d.limit, d.up_offset,
                          d.activation == XP_ACTIVATION_RELU   ? kActivationRelu
                          : d.activation == XP_ACTIVATION_GELU ? kActivationGelu
                                                               : kActivationSilu,
                          d.approximate_tanh};
  experts.bias_gate_up = layer.gate_up_bias;
  experts.bias_down = layer.down_bias;
  experts.payload = payload;
  if (fuse_topk) {
    experts.fused_topk = &routing.topk_args;
  }
  ExpertsLaunches launches;
  if (const int status = make_experts_launches(experts, capacity, launches); status != XP_OK) {
    return status;
  }
  chain.add(launches.sort);
  chain.add(launches.gate_up);
  chain.add(launches.down);
  chain.add(launches.combine);
  return XP_OK;
}

TransportArgs transport_args(xp_transport_t transport, int arena) {
  TransportArgs args{};
  args.arenas = transport->arenas;
  args.arena = arena;
  args.arena_count = transport->arena_count;
  args.output_nan2 = Bf16Payload::kPoison2;
  return args;
}

int launch_transport(xp_transport_t transport, const KernelLaunch &kernel, xp_stream_t stream) {
  XP_HIP_CHECK(hipSetDevice(transport->device));
  XP_HIP_CHECK(launch(kernel, static_cast<hipStream_t>(stream)));
  return XP_OK;
}

bool valid_arena(xp_transport_t transport, int arena) {
  return transport != nullptr && arena >= 0 && arena < transport->arena_count;
}


void destroy_template(Template &t) {
  if (t.exec != nullptr) {
    (void)hipGraphExecDestroy(t.exec);
    t.exec = nullptr;
  }
  if (t.graph != nullptr) {
    (void)hipGraphDestroy(t.graph);
    t.graph = nullptr;
  }
}

StepChain dense_chain(const DenseBinding &binding, int64_t capacity) {
  const DenseLaunches launches = make_dense_launches(binding, capacity);
  const KernelLaunch *kernels[kMaxStepKernels];
  const int count = launches.chain(kernels);
  StepChain chain;
  chain.usable = launches.usable();
  for (int index = 0; index < count; ++index) {
    chain.add(*kernels[index]);
  }
  return chain;
}

// Build and instantiate a template's hipGraph: one kernel node per chain entry, each
// depending on the previous one.
int instantiate_template(Template &t, const StepChain &chain) {
  if (!chain.usable) {
    return fail(XP_ERROR_INVALID_ARGUMENT, kUnusableChoice);
  }
  XP_HIP_CHECK(hipGraphCreate(&t.graph, 0));
  t.node_count = chain.count;
  for (int index = 0; index < chain.count; ++index) {
    const KernelLaunch &kernel = chain.kernels[index];
    if (kernel.shmem > 64 * 1024) {
      const hipError_t enabled = enable_large_lds(kernel.func);
      if (enabled != hipSuccess) {
        destroy_template(t);
        return fail(XP_ERROR_HIP, std::string("enabling dynamic LDS above 64 KB failed: ") + hipGetErrorString(enabled));
      }
    }
    void *params[1];
    hipKernelNodeParams node = node_params(kernel, params);
    const hipGraphNode_t *dependencies = index == 0 ? nullptr : &t.nodes[index - 1];
    const hipError_t added = hipGraphAddKernelNode(&t.nodes[index], t.graph, dependencies, index == 0 ? 0 : 1, &node);
    if (added != hipSuccess) {
      destroy_template(t);
      return fail(XP_ERROR_HIP, std::string("hipGraphAddKernelNode failed: ") + hipGetErrorString(added));
    }
    t.bound[index] = kernel;
  }
  const hipError_t instantiated = hipGraphInstantiate(&t.exec, t.graph, nullptr, nullptr, 0);
  if (instantiated != hipSuccess) {
    destroy_template(t);
    return fail(XP_ERROR_HIP, std::string("hipGraphInstantiate failed: ") + hipGetErrorString(instantiated));
  }
  return XP_OK;
}

void insert_template(xp_lane *lane, std::unique_ptr<Template> t) {
  lane->templates.push_back(std::move(t));
  std::stable_sort(lane->templates.begin(), lane->templates.end(), [](const auto &left, const auto &right) {
    if (left->kind != right->kind) return left->kind < right->kind;
    if (left->hidden != right->hidden) return left->hidden < right->hidden;
    if (left->intermediate != right->intermediate) return left->intermediate < right->intermediate;
    return left->capacity < right->capacity;
  });
}

// Launch a replay's chain: directly on the stream, or (graph dispatch) by rebinding the
// template's nodes whose argument record changed and launching its graph.
int run_chain(xp_lane *lane, Template &t, const StepChain &chain, hipStream_t target) {
  if (!chain.usable) {
    return fail(XP_ERROR_INVALID_ARGUMENT, kUnusableChoice);
  }
  if (chain.count != t.node_count) {
    return fail(XP_ERROR_STATE, "replay kernel sequence differs from the captured template");
  }
  // Under an outer stream capture (a caller recording its decode step as a graph) the
  // kernels are launched directly, so that they become nodes of the caller's graph rather
  // than a graph launched inside a capture.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (lane->graph_dispatch) {
    XP_HIP_CHECK(hipStreamIsCapturing(target, &capture));
  }
  if (!lane->graph_dispatch || capture != hipStreamCaptureStatusNone) {
    for (int index = 0; index < chain.count; ++index) {
      XP_HIP_CHECK(launch(chain.kernels[index], target));
    }
    return XP_OK;
  }
  for (int index = 0; index < chain.count; ++index) {
    const KernelLaunch &kernel = chain.kernels[index];
    KernelLaunch &bound = t.bound[index];
    if (bound.func != kernel.func) {
      return fail(XP_ERROR_STATE, "replay kernel differs from the captured template's node");
    }
    if (bound.args_size == kernel.args_size && std::memcmp(bound.args, kernel.args, bound.args_size) == 0) {
      continue;
    }
    void *params[1];
    hipKernelNodeParams node = node_params(kernel, params);
    XP_HIP_CHECK(hipGraphExecKernelNodeSetParams(t.exec, t.nodes[index], &node));
    bound = kernel;
  }
  XP_HIP_CHECK(hipGraphLaunch(t.exec, target));
  return XP_OK;
}

const Layer *find_layer(const xp_agent *agent, int instance_index, int layer_ordinal) {
  for (const Layer &layer : agent->layers) {
    if (layer.instance_index == instance_index && layer.layer_ordinal == layer_ordinal) {
      return &layer;
    }
  }
  return nullptr;
}

}  // namespace

extern "C" {

int xp_abi_version(void) { return XP_ABI_VERSION; }

size_t xp_last_error(char *buffer, size_t size) {
  const std::string &message = g_last_error;
  if (buffer != nullptr && size > 0) {
    const size_t count = std::min(size - 1, message.size());
    std::memcpy(buffer, message.data(), count);
    buffer[count] = '\0';
  }
  return message.size();
}

// ------------------------------------------------------------------ kernels

int xp_copy_bytes(void *dst, const void *src, size_t bytes, xp_stream_t stream) {
  if (bytes == 0) {
    return XP_OK;
  }
  XP_REQUIRE(dst != nullptr && src != nullptr, "copy pointers must be non-null for a non-empty range");
  const uint8_t *s = static_cast<const uint8_t *>(src);
  uint8_t *d = static_cast<uint8_t *>(dst);
  XP_REQUIRE(d + bytes <= s || s + bytes <= d, "copy ranges must not overlap");
  CopyArgs args{d, s, bytes};
  XP_HIP_CHECK(launch(make_copy(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

int xp_reduce_partials(const void *const *partials, int count, void *out, int64_t elements, xp_stream_t stream) {
  XP_REQUIRE(count >= 1 && count <= kMaxPartials, "partial count must be between 1 and 16");
  XP_REQUIRE(elements >= 0 && elements % 8 == 0, "element count must be a non-negative multiple of 8");
  if (elements == 0) {
    return XP_OK;
  }
  XP_REQUIRE(partials != nullptr && out != nullptr, "reduction pointers must be non-null");
  ReduceArgs args{};
  for (int k = 0; k < count; ++k) {
    XP_REQUIRE(partials[k] != nullptr && aligned16(partials[k]), "partials must be non-null and 16-byte aligned");
    args.partials[k] = static_cast<const uint16_t *>(partials[k]);
  }
  XP_REQUIRE(aligned16(out), "the output must be 16-byte aligned");
  args.out = static_cast<uint16_t *>(out);
  args.vectors = static_cast<uint64_t>(elements / 8);
  args.count = count;
  XP_HIP_CHECK(launch(make_reduce_partials(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

int xp_gather_rmsnorm(const void *pool, int64_t pool_rows, int64_t hidden, const int32_t *slots, int64_t rows,
                      const void *norm_weight, float eps, void *out, uint32_t *fault_word, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0 && pool_rows >= 0, "row counts must be non-negative");
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(hidden > 0 && hidden % 8 == 0 && gather_supported(hidden),
             "hidden size must be a positive multiple of 8 and at most 16384");
  XP_REQUIRE(pool != nullptr && slots != nullptr && out != nullptr, "gather pointers must be non-null");
  XP_REQUIRE(aligned16(pool) && aligned16(out) && (norm_weight == nullptr || aligned16(norm_weight)),
             "gather rows must be 16-byte aligned");
  XP_REQUIRE(norm_weight == nullptr || eps >= 0.0f, "RMSNorm epsilon must be non-negative");
  GatherArgs args{};
  args.pool = static_cast<const uint16_t *>(pool);
  args.slots = slots;
  args.norm = static_cast<const uint16_t *>(norm_weight);
  args.out = static_cast<uint16_t *>(out);
  args.fault = fault_word;
  args.pool_rows = pool_rows;
  args.hidden = hidden;
  args.rows = rows;
  args.eps = eps;
  XP_HIP_CHECK(launch(make_gather(args, rows), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

int xp_scatter(const void *values, int64_t rows, int64_t hidden, const int32_t *slots, void *pool,
               int64_t pool_rows, uint32_t *fault_word, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0 && pool_rows >= 0, "row counts must be non-negative");
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(hidden > 0 && hidden % 8 == 0, "hidden size must be a positive multiple of 8");
  XP_REQUIRE(values != nullptr && slots != nullptr && pool != nullptr, "scatter pointers must be non-null");
  XP_REQUIRE(aligned16(values) && aligned16(pool), "scatter rows must be 16-byte aligned");
  ScatterArgs args{};
  args.values = static_cast<const uint16_t *>(values);
  args.slots = slots;
  args.pool = static_cast<uint16_t *>(pool);
  args.fault = fault_word;
  args.pool_rows = pool_rows;
  args.hidden = hidden;
  args.rows = rows;
  XP_HIP_CHECK(launch(make_scatter(args, rows), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

size_t xp_gemm_workspace_bytes(int64_t rows, int64_t n, int64_t k, int gated) {
  if (rows <= 0 || n <= 0 || k <= 0) {
    return 0;
  }
  return gemm_scratch_bytes(choose_gemm(rows, n, k, gated != 0), rows, n, k);
}

int xp_gemm_gate_up_silu(const void *x, int64_t rows, int64_t hidden, const void *w_gate_up, int64_t intermediate,
                         void *activated, float alpha, float limit, float up_offset, void *workspace,
                         size_t workspace_bytes, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0, "row count must be non-negative");
  if (rows == 0) {
    return XP_OK;
  }
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(x != nullptr && w_gate_up != nullptr && activated != nullptr, "projection pointers must be non-null");
  XP_REQUIRE(aligned16(x) && aligned16(w_gate_up) && aligned16(activated), "projection operands must be 16-byte aligned");
  XP_REQUIRE(alpha > 0.0f, "SiLU alpha must be positive");
  GemmArgs args{};
  args.x = static_cast<const uint16_t *>(x);
  args.w = static_cast<const uint16_t *>(w_gate_up);
  args.out = static_cast<uint16_t *>(activated);
  args.ldx = hidden;
  args.ldo = intermediate;
  args.rows = rows;
  args.out_rows = rows;
  args.n = 2 * intermediate;
  args.k = hidden;
  args.act = GatedSilu{alpha, limit, up_offset};
  const GemmChoice choice = choose_gemm(rows, args.n, args.k, true);
  if (const int status = bind_scratch(args, choice, workspace, workspace_bytes); status != XP_OK) {
    return status;
  }
  return launch_gemm(make_gemm(args, rows, true, choice), static_cast<hipStream_t>(stream));
}

int xp_gemm_down(const void *activated, int64_t rows, int64_t intermediate, const void *w_down, int64_t hidden,
                 void *out, const int32_t *slots, int64_t out_rows, void *workspace, size_t workspace_bytes,
                 xp_stream_t stream) {
  XP_REQUIRE(rows >= 0, "row count must be non-negative");
  if (rows == 0) {
    return XP_OK;
  }
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(activated != nullptr && w_down != nullptr && out != nullptr, "projection pointers must be non-null");
  XP_REQUIRE(aligned16(activated) && aligned16(w_down) && aligned16(out), "projection operands must be 16-byte aligned");
  XP_REQUIRE(slots == nullptr || out_rows >= 0, "scatter output rows must be non-negative");
  GemmArgs args{};
  args.x = static_cast<const uint16_t *>(activated);
  args.w = static_cast<const uint16_t *>(w_down);
  args.out = static_cast<uint16_t *>(out);
  args.scatter_slots = slots;
  args.ldx = intermediate;
  args.ldo = hidden;
  args.rows = rows;
  args.out_rows = slots != nullptr ? out_rows : rows;
  args.n = hidden;
  args.k = intermediate;
  args.act = default_activation();
  const GemmChoice choice = choose_gemm(rows, args.n, args.k, false);
  if (const int status = bind_scratch(args, choice, workspace, workspace_bytes); status != XP_OK) {
    return status;
  }
  return launch_gemm(make_gemm(args, rows, false, choice), static_cast<hipStream_t>(stream));
}

namespace {

size_t dtype_bytes(int dtype) {
  switch (dtype) {
    case XP_DTYPE_BF16:
    case XP_DTYPE_F16:
      return 2;
    case XP_DTYPE_F32:
      return 4;
    default:
      return 0;
  }
}

bool aligned_to(const void *pointer, size_t bytes) { return (reinterpret_cast<uintptr_t>(pointer) % bytes) == 0; }

// The activation descriptor of the C ABI as the kernels take it (checked).
int activation_record(const xp_activation_desc *desc, ActivationArgs &out) {
  out = ActivationArgs{};
  if (desc == nullptr) {
    out.function = kActivationNone;
    return XP_OK;
  }
  XP_REQUIRE(desc->function == XP_ACTIVATION_SILU || desc->function == XP_ACTIVATION_RELU ||
                 desc->function == XP_ACTIVATION_GELU,
             "activation function must be SiLU, ReLU or GELU");
  XP_REQUIRE(desc->function != XP_ACTIVATION_SILU || (desc->alpha > 0.0f && std::isfinite(desc->alpha)),
             "SiLU alpha must be positive and finite");
  XP_REQUIRE(!desc->has_limit || (desc->limit > 0.0f && std::isfinite(desc->limit)), "gate limit must be positive");
  XP_REQUIRE(std::isfinite(desc->up_offset), "up offset must be finite");
  XP_REQUIRE(desc->gated || (!desc->has_limit && desc->up_offset == 0.0f),
             "a gate transform needs a gated activation");
  out.function = desc->function;
  out.approximate_tanh = desc->approximate_tanh != 0;
  out.gated = desc->gated != 0;
  out.has_limit = desc->has_limit != 0;
  out.alpha = desc->alpha;
  out.limit = desc->has_limit ? desc->limit : 0.0f;
  out.up_offset = desc->up_offset;
  return XP_OK;
}

}  // namespace

int xp_projection(const void *x, int64_t rows, int64_t k, const void *w, int64_t n, const float *bias, void *out,
                  int dtype, const xp_activation_desc *activation, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0 && k > 0 && n > 0, "projection rows must be non-negative and K, N positive");
  const size_t element = dtype_bytes(dtype);
  XP_REQUIRE(element != 0, "payload dtype must be bf16, fp16 or fp32");
  ProjectionArgs args{};
  if (const int status = activation_record(activation, args.act); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(!args.act.gated || n % 2 == 0, "a gated projection needs an even number of (INTERLEAVED) weight rows");
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(x != nullptr && w != nullptr && out != nullptr, "projection pointers must be non-null");
  XP_REQUIRE(aligned_to(x, element) && aligned_to(w, element) && aligned_to(out, element) &&
                 (bias == nullptr || aligned_to(bias, 4)),
             "projection operands must be aligned to their element size");
  args.x = x;
  args.w = w;
  args.bias = bias;
  args.out = out;
  args.rows = rows;
  args.n = n;
  args.k = k;
  args.dtype = dtype;
  XP_HIP_CHECK(launch(make_projection(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

int xp_activation(const void *inputs, void *output, int64_t rows, int64_t width, int dtype, int order,
                  const xp_activation_desc *activation, xp_stream_t stream) {
  XP_REQUIRE(activation != nullptr, "activation descriptor must be non-null");
  XP_REQUIRE(rows >= 0 && width >= 0, "activation extents must be non-negative");
  XP_REQUIRE(dtype == XP_DTYPE_BF16 || dtype == XP_DTYPE_F16, "standalone activations take bf16 or fp16 payloads");
  ActivationLaunchArgs args{};
  if (const int status = activation_record(activation, args.act); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(!args.act.gated || order == XP_GATE_UP_INTERLEAVED || order == XP_GATE_UP_CONCATENATED,
             "gated activation requires a Gate/Up order");
  const int64_t elements = rows * width;
  if (elements == 0) {
    return XP_OK;
  }
  XP_REQUIRE(inputs != nullptr && output != nullptr, "activation pointers must be non-null");
  XP_REQUIRE(aligned_to(inputs, 2) && aligned_to(output, 2), "activation payloads must be 2-byte aligned");
  const uintptr_t in_begin = reinterpret_cast<uintptr_t>(inputs);
  const uintptr_t in_end = in_begin + static_cast<uintptr_t>(elements * (args.act.gated ? 2 : 1) * 2);
  const uintptr_t out_begin = reinterpret_cast<uintptr_t>(output);
  const uintptr_t out_end = out_begin + static_cast<uintptr_t>(elements * 2);
  const bool overlap = in_begin < out_end && out_begin < in_end;
  XP_REQUIRE(!overlap || (!args.act.gated && in_begin == out_begin),
             "only an ungated activation may run in place, and only on the same range");
  args.inputs = inputs;
  args.output = output;
  args.elements = elements;
  args.width = width;
  args.dtype = dtype;
  args.interleaved = order == XP_GATE_UP_INTERLEAVED;
  XP_HIP_CHECK(launch(make_activation(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

size_t xp_dense_workspace_bytes(int64_t capacity, int64_t hidden, int64_t intermediate) {
  if (capacity <= 0 || hidden <= 0 || intermediate <= 0) {
    return 0;
  }
  return dense_workspace(capacity, hidden, intermediate).bytes;
}

int xp_dense_workspace_layout(int64_t capacity, int64_t hidden, int64_t intermediate, size_t *offsets) {
  XP_REQUIRE(capacity > 0, "capacity must be positive");
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(offsets != nullptr, "offsets pointer must be non-null");
  const DenseWorkspace layout = dense_workspace(capacity, hidden, intermediate);
  const bool partials = layout.bytes > layout.activated_offset + static_cast<size_t>(capacity * intermediate) * 2;
  offsets[0] = layout.batch_offset;
  offsets[1] = layout.activated_offset;
  offsets[2] = partials ? layout.gate_up_partials_offset : layout.bytes;
  offsets[3] = partials ? layout.down_partials_offset : layout.bytes;
  offsets[4] = layout.bytes;
  return XP_OK;
}

namespace {

// Checks and launches shared by xp_dense_step and xp_dense_step_static: the same kernels
// on the same arguments, over a workspace the caller has already sized.
int dense_step_checks(const void *pool_in, const void *pool_out, int64_t pool_rows, const int32_t *slots,
                      int64_t rows, int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                      const void *norm_weight) {
  XP_REQUIRE(rows >= 0 && pool_rows >= 0, "row counts must be non-negative");
  if (rows == 0) {
    return XP_OK;
  }
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  if (const int status = validate_mailbox(pool_rows, hidden); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(pool_in != nullptr && pool_out != nullptr && slots != nullptr && w_gate_up != nullptr &&
                 w_down != nullptr,
             "dense step pointers must be non-null");
  XP_REQUIRE(aligned16(pool_in) && aligned16(pool_out) && aligned16(w_gate_up) && aligned16(w_down) &&
                 (norm_weight == nullptr || aligned16(norm_weight)),
             "dense step operands must be 16-byte aligned");
  return XP_OK;
}

int run_dense_step(const void *pool_in, void *pool_out, int64_t pool_rows, const int32_t *slots, int64_t rows,
                   int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                   const void *norm_weight, float eps, void *workspace, uint32_t *fault_word, xp_stream_t stream) {
  DenseBinding binding{};
  binding.pool_in = static_cast<const uint16_t *>(pool_in);
  binding.pool_out = static_cast<uint16_t *>(pool_out);
  binding.pool_rows = pool_rows;
  binding.slots = slots;
  binding.rows = rows;
  binding.hidden = hidden;
  binding.intermediate = intermediate;
  binding.gate_up = static_cast<const uint16_t *>(w_gate_up);
  binding.down = static_cast<const uint16_t *>(w_down);
  binding.norm = static_cast<const uint16_t *>(norm_weight);
  binding.eps = eps;
  binding.workspace = static_cast<uint8_t *>(workspace);
  binding.fault = fault_word;
  const DenseLaunches launches = make_dense_launches(binding, rows);
  XP_REQUIRE(launches.usable(), kUnusableChoice);
  const KernelLaunch *chain[kMaxStepKernels];
  const int count = launches.chain(chain);
  for (int index = 0; index < count; ++index) {
    XP_HIP_CHECK(launch(*chain[index], static_cast<hipStream_t>(stream)));
  }
  return XP_OK;
}

}  // namespace

int xp_dense_step(const void *pool_in, void *pool_out, int64_t pool_rows, const int32_t *slots, int64_t rows,
                  int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                  const void *norm_weight, float eps, void *workspace, size_t workspace_bytes, uint32_t *fault_word,
                  xp_stream_t stream) {
  if (const int status = dense_step_checks(pool_in, pool_out, pool_rows, slots, rows, hidden, intermediate, w_gate_up,
                                           w_down, norm_weight);
      status != XP_OK || rows == 0) {
    return status;
  }
  XP_REQUIRE(workspace != nullptr, "dense step pointers must be non-null");
  XP_REQUIRE(aligned16(workspace), "dense step operands must be 16-byte aligned");
  XP_REQUIRE(workspace_bytes >= dense_workspace(rows, hidden, intermediate).bytes,
             "workspace is smaller than xp_dense_workspace_bytes(rows, hidden, intermediate)");
  return run_dense_step(pool_in, pool_out, pool_rows, slots, rows, hidden, intermediate, w_gate_up, w_down,
                        norm_weight, eps, workspace, fault_word, stream);
}

// Workspace of xp_dense_step_static: a static device array, so that the step allocates
// nothing.  Every device the library runs on holds its own copy until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a stand-in, not a
// device address): it uses the device address that hipGetSymbolAddress returns for the
// current device, looked up once per device and kept in static_scratch_address.
constexpr size_t kStaticScratchBytes = size_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_static_scratch_mutex;
void *g_static_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call there).
int static_scratch_address(void **out) {
  int device = 0;
  XP_HIP_CHECK(hipGetDevice(&device));
  XP_REQUIRE(device >= 0 && device < kMaxDevices, "device ordinal exceeds the static scratch table (64 devices)");
  std::lock_guard<std::mutex> guard(g_static_scratch_mutex);
  if (g_static_scratch[device] == nullptr) {
    void *address = nullptr;
    XP_HIP_CHECK(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
    XP_REQUIRE(address != nullptr && (reinterpret_cast<uintptr_t>(address) & 255u) == 0,
               "static scratch address is not 256-byte aligned");
    g_static_scratch[device] = address;
  }
  *out = g_static_scratch[device];
  return XP_OK;
}

}  // namespace

int xp_dense_step_static(const void *pool_in, void *pool_out, int64_t pool_rows, const int32_t *slots, int64_t rows,
                         int64_t hidden, int64_t intermediate, const void *w_gate_up, const void *w_down,
                         const void *norm_weight, float eps, uint32_t *fault_word, xp_stream_t stream) {
  if (const int status = dense_step_checks(pool_in, pool_out, pool_rows, slots, rows, hidden, intermediate, w_gate_up,
                                           w_down, norm_weight);
      status != XP_OK || rows == 0) {
    return status;
  }
  const size_t needed = dense_workspace(rows, hidden, intermediate).bytes;
  if (needed > kStaticScratchBytes) {
    return fail(XP_ERROR_CAPACITY, "dense step needs " + std::to_string(needed) +
                                       " bytes of workspace, more than the static scratch holds (" +
                                       std::to_string(kStaticScratchBytes) + " bytes); use xp_dense_step");
  }
  void *workspace = nullptr;
  if (const int status = static_scratch_address(&workspace); status != XP_OK) {
    return status;
  }
  return run_dense_step(pool_in, pool_out, pool_rows, slots, rows, hidden, intermediate, w_gate_up, w_down,
                        norm_weight, eps, workspace, fault_word, stream);
}

size_t xp_gemm_variant(int64_t capacity, int64_t n, int64_t k, int gated, char *buffer, size_t size) {
  const std::string name = capacity > 0 ? gemm_name(choose_gemm(capacity, n, k, gated != 0), gated != 0) : "";
  if (buffer != nullptr && size > 0) {
    const size_t count = std::min(size - 1, name.size());
    std::memcpy(buffer, name.data(), count);
    buffer[count] = '\0';
  }
  return name.size();
}

size_t xp_dense_gate_up_variant(int64_t capacity, int64_t hidden, int64_t intermediate, char *buffer, size_t size) {
  std::string name;
  if (capacity > 0 && hidden > 0 && intermediate > 0) {
    bool fused = false;
    const GemmChoice choice = choose_dense_gate_up(capacity, 2 * intermediate, hidden, fused);
    name = gemm_name(choice, true) + (fused ? "+gather" : "");  // SplitGathered names itself
  }
  if (buffer != nullptr && size > 0) {
    const size_t count = std::min(size - 1, name.size());
    std::memcpy(buffer, name.data(), count);
    buffer[count] = '\0';
  }
  return name.size();
}

// ------------------------------------------------------------------ runtime

int xp_agent_create(int device, xp_agent_t *out) {
  XP_REQUIRE(out != nullptr, "agent output pointer must be non-null");
  int count = 0;
  XP_HIP_CHECK(hipGetDeviceCount(&count));
  XP_REQUIRE(device >= 0 && device < count, "device ordinal is out of range");
  auto agent = std::make_unique<xp_agent>();
  agent->device = device;
  *out = agent.release();
  return XP_OK;
}

int xp_agent_destroy(xp_agent_t agent) {
  if (agent == nullptr) {
    return XP_OK;
  }
  {
    std::lock_guard<std::mutex> guard(agent->mutex);
    if (agent->live_lanes != 0) {
      return fail(XP_ERROR_STATE, "destroy every Lane before its agent");
    }
  }
  delete agent;
  return XP_OK;
}

int xp_layer_register(xp_agent_t agent, int instance_index, int layer_ordinal, int64_t hidden, int64_t intermediate,
                      int payload_dtype, const void *gate_up, const void *down, const void *norm_weight, float eps) {
  XP_REQUIRE(agent != nullptr, "agent must be non-null");
  XP_REQUIRE(instance_index >= 0 && layer_ordinal >= 0, "instance index and layer ordinal must be non-negative");
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(gate_up != nullptr && down != nullptr, "layer weights must be non-null");
  XP_REQUIRE(aligned16(gate_up) && aligned16(down) && (norm_weight == nullptr || aligned16(norm_weight)),
             "layer weights must be 16-byte aligned");
  XP_REQUIRE(norm_weight == nullptr || eps >= 0.0f, "RMSNorm epsilon must be non-negative");
  std::lock_guard<std::mutex> guard(agent->mutex);
  Layer layer{instance_index,
              layer_ordinal,
              hidden,
              intermediate,
              static_cast<const uint16_t *>(gate_up),
              static_cast<const uint16_t *>(down),
              static_cast<const uint16_t *>(norm_weight),
              eps,
              payload};
  for (Layer &existing : agent->layers) {
    if (existing.instance_index == instance_index && existing.layer_ordinal == layer_ordinal) {
      existing = layer;
      return XP_OK;
    }
  }
  agent->layers.push_back(layer);
  return XP_OK;
}

int xp_lane_create(xp_agent_t agent, void *workspace, size_t workspace_bytes, xp_lane_t *out) {
  XP_REQUIRE(agent != nullptr && out != nullptr, "agent and output pointer must be non-null");
  XP_REQUIRE(workspace != nullptr || workspace_bytes == 0, "workspace must be non-null when sized");
  XP_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  XP_HIP_CHECK(hipSetDevice(agent->device));
  auto lane = std::make_unique<xp_lane>();
  lane->agent = agent;
  lane->workspace = static_cast<uint8_t *>(workspace);
  lane->workspace_bytes = workspace_bytes;
  XP_HIP_CHECK(hipStreamCreateWithFlags(&lane->stream, hipStreamNonBlocking));
  void *fault = nullptr;
  const hipError_t allocated = hipMalloc(&fault, sizeof(uint32_t));
  if (allocated != hipSuccess) {
    (void)hipStreamDestroy(lane->stream);
    return fail(XP_ERROR_HIP, std::string("hipMalloc of the Lane fault word failed: ") + hipGetErrorString(allocated));
  }
  lane->fault = static_cast<uint32_t *>(fault);
  const hipError_t cleared = hipMemset(lane->fault, 0, sizeof(uint32_t));
  if (cleared != hipSuccess) {
    (void)hipFree(lane->fault);
    (void)hipStreamDestroy(lane->stream);
    return fail(XP_ERROR_HIP, std::string("clearing the Lane fault word failed: ") + hipGetErrorString(cleared));
  }
  {
    std::lock_guard<std::mutex> guard(agent->mutex);
    agent->live_lanes += 1;
  }
  *out = lane.release();
  return XP_OK;
}

int xp_lane_destroy(xp_lane_t lane) {
  if (lane == nullptr) {
    return XP_OK;
  }
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  XP_HIP_CHECK(hipStreamSynchronize(lane->stream));
  for (auto &t : lane->templates) {
    destroy_template(*t);
  }
  lane->templates.clear();
  (void)hipFree(lane->fault);
  (void)hipStreamDestroy(lane->stream);
  {
    std::lock_guard<std::mutex> guard(lane->agent->mutex);
    lane->agent->live_lanes -= 1;
  }
  delete lane;
  return XP_OK;
}

int xp_lane_stream(xp_lane_t lane, xp_stream_t *out) {
  XP_REQUIRE(lane != nullptr && out != nullptr, "lane and output pointer must be non-null");
  *out = lane->stream;
  return XP_OK;
}

int xp_lane_set_graph_dispatch(xp_lane_t lane, int use_graph) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  std::lock_guard<std::mutex> guard(lane->mutex);
  lane->graph_dispatch = use_graph != 0;
  return XP_OK;
}

int xp_lane_synchronize(xp_lane_t lane) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  XP_HIP_CHECK(hipStreamSynchronize(lane->stream));
  return XP_OK;
}

int xp_lane_check_health(xp_lane_t lane, uint32_t *fault_bits) {
  XP_REQUIRE(lane != nullptr && fault_bits != nullptr, "lane and output pointer must be non-null");
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  XP_HIP_CHECK(hipStreamSynchronize(lane->stream));
  uint32_t value = 0;
  XP_HIP_CHECK(hipMemcpy(&value, lane->fault, sizeof value, hipMemcpyDeviceToHost));
  *fault_bits = value;
  return XP_OK;
}

int xp_lane_clear_fault(xp_lane_t lane) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  XP_HIP_CHECK(hipStreamSynchronize(lane->stream));
  XP_HIP_CHECK(hipMemset(lane->fault, 0, sizeof(uint32_t)));
  return XP_OK;
}

int xp_template_capture(xp_lane_t lane, int64_t hidden, int64_t intermediate, int payload_dtype, int64_t capacity) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  if (const int status = validate_geometry(hidden, intermediate); status != XP_OK) {
    return status;
  }
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(capacity > 0, "template capacity must be positive");
  const size_t needed = dense_workspace(capacity, hidden, intermediate).bytes;
  if (needed > lane->workspace_bytes) {
    return fail(XP_ERROR_CAPACITY, "Lane workspace is smaller than the template needs (" + std::to_string(needed) +
                                       " bytes)");
  }
  std::lock_guard<std::mutex> guard(lane->mutex);
  for (const auto &t : lane->templates) {
    if (t->kind == XP_LAYER_DENSE && t->hidden == hidden && t->intermediate == intermediate &&
        t->payload == payload && t->capacity == capacity) {
      return XP_OK;
    }
  }
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  // Placeholder binding: a replay rebinds every argument record before launching.
  DenseBinding binding{};
  binding.hidden = hidden;
  binding.intermediate = intermediate;
  binding.payload = payload;
  binding.rows = 0;
  binding.workspace = lane->workspace;
  binding.fault = lane->fault;
  auto t = std::make_unique<Template>();
  t->kind = XP_LAYER_DENSE;
  t->hidden = hidden;
  t->intermediate = intermediate;
  t->payload = payload;
  t->capacity = capacity;
  if (const int status = instantiate_template(*t, dense_chain(binding, capacity)); status != XP_OK) {
    return status;
  }
  insert_template(lane, std::move(t));
  return XP_OK;
}

int xp_template_capacities(xp_lane_t lane, int64_t hidden, int64_t intermediate, int payload_dtype,
                           int64_t *capacities, int max_count, int *count) {
  XP_REQUIRE(lane != nullptr && count != nullptr, "lane and count pointer must be non-null");
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  std::lock_guard<std::mutex> guard(lane->mutex);
  int found = 0;
  for (const auto &t : lane->templates) {
    if (t->kind == XP_LAYER_DENSE && t->hidden == hidden && t->intermediate == intermediate && t->payload == payload) {
      if (capacities != nullptr && found < max_count) {
        capacities[found] = t->capacity;
      }
      ++found;
    }
  }
  *count = found;
  return XP_OK;
}

int xp_replay(xp_lane_t lane, int instance_index, int layer_ordinal, int64_t rows, const void *pool_in,
              void *pool_out, int64_t pool_rows, const int32_t *slots, xp_stream_t stream) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  XP_REQUIRE(pool_in != nullptr && pool_out != nullptr && slots != nullptr, "replay pointers must be non-null");
  XP_REQUIRE(aligned16(pool_in) && aligned16(pool_out), "mailbox rows must be 16-byte aligned");
  XP_REQUIRE(pool_rows > 0, "mailbox must have rows");
  Layer layer{};
  {
    std::lock_guard<std::mutex> guard(lane->agent->mutex);
    const Layer *found = find_layer(lane->agent, instance_index, layer_ordinal);
    if (found == nullptr) {
      return fail(XP_ERROR_NOT_FOUND, "no layer is registered for (instance " + std::to_string(instance_index) +
                                          ", ordinal " + std::to_string(layer_ordinal) + ")");
    }
    layer = *found;
  }
  if (const int status = validate_mailbox(pool_rows, layer.kind == XP_LAYER_MOE ? layer.moe.hidden : layer.hidden);
      status != XP_OK) {
    return status;
  }
  std::lock_guard<std::mutex> guard(lane->mutex);
  Template *selected = nullptr;
  int64_t largest = 0;
  for (const auto &t : lane->templates) {
    const bool serves = t->kind == layer.kind &&
                        (layer.kind == XP_LAYER_MOE ? same_moe(t->moe, layer.moe)
                                                    : t->hidden == layer.hidden && t->intermediate == layer.intermediate &&
                                                          t->payload == layer.payload);
    if (serves) {
      largest = std::max(largest, t->capacity);
      if (selected == nullptr && rows <= t->capacity) {
        selected = t.get();
      }
    }
  }
  if (rows < 1 || selected == nullptr) {
    return fail(XP_ERROR_CAPACITY, "row count " + std::to_string(rows) + " is outside the installed capacities [1, " +
                                       std::to_string(largest) + "]");
  }
  // NULL is the legacy default stream, as for every other entry point.
  const hipStream_t target = static_cast<hipStream_t>(stream);
  if (layer.kind == XP_LAYER_MOE) {
    MoeStepBinding binding{};
    binding.pool_in = static_cast<const uint16_t *>(pool_in);
    binding.pool_out = static_cast<uint16_t *>(pool_out);
    binding.pool_rows = pool_rows;
    binding.slots = slots;
    binding.rows = rows;
    binding.workspace = lane->workspace;
    binding.fault = lane->fault;
    StepChain chain;
    if (const int status = make_moe_step(layer, binding, selected->capacity, chain); status != XP_OK) {
      return status;
    }
    return run_chain(lane, *selected, chain, target);
  }
  DenseBinding binding{};
  binding.pool_in = static_cast<const uint16_t *>(pool_in);
  binding.pool_out = static_cast<uint16_t *>(pool_out);
  binding.pool_rows = pool_rows;
  binding.slots = slots;
  binding.rows = rows;
  binding.hidden = layer.hidden;
  binding.intermediate = layer.intermediate;
  binding.gate_up = layer.gate_up;
  binding.down = layer.down;
  binding.norm = layer.norm;
  binding.eps = layer.eps;
  binding.workspace = lane->workspace;
  binding.fault = lane->fault;
  binding.payload = layer.payload;
  return run_chain(lane, *selected, dense_chain(binding, selected->capacity), target);
}


// ------------------------------------------------------------------ transport

int xp_lane_fault_word(xp_lane_t lane, uint32_t **out) {
  XP_REQUIRE(lane != nullptr && out != nullptr, "lane and output pointer must be non-null");
  *out = lane->fault;
  return XP_OK;
}

int xp_transport_create(int device, int arena_count, const int64_t *payload_row_capacities,
                        const int32_t *atn_dp_sizes, xp_transport_t *out) {
  XP_REQUIRE(out != nullptr, "output pointer must be non-null");
  XP_REQUIRE(arena_count >= 1 && arena_count <= 1024, "a transport serves 1 to 1024 arenas");
  XP_REQUIRE(payload_row_capacities != nullptr && atn_dp_sizes != nullptr, "arena geometry must be given");
  for (int index = 0; index < arena_count; ++index) {
    XP_REQUIRE(payload_row_capacities[index] > 0, "arena payload row capacity must be positive");
    XP_REQUIRE(atn_dp_sizes[index] >= 1 && atn_dp_sizes[index] <= kMaxDpRanks,
               "attention DP size must be between 1 and 64");
  }
  XP_HIP_CHECK(hipSetDevice(device));
  auto transport = std::make_unique<xp_transport>();
  transport->device = device;
  transport->arena_count = arena_count;
  int rate_khz = 0;
  XP_HIP_CHECK(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, device));
  XP_REQUIRE(rate_khz > 0, "device reports no wall clock rate");
  transport->wall_clock_khz = static_cast<uint64_t>(rate_khz);
  std::vector<TransportArena> image(static_cast<size_t>(arena_count));
  for (int index = 0; index < arena_count; ++index) {
    std::memset(&image[index], 0, sizeof(TransportArena));  // Dormant, Ok, no shutdown
    image[index].payload_row_capacity = static_cast<uint64_t>(payload_row_capacities[index]);
    image[index].atn_dp_size = static_cast<uint32_t>(atn_dp_sizes[index]);
    image[index].instance_outcome = kResultOk;
    transport->capacities.push_back(payload_row_capacities[index]);
    transport->atn_dp_sizes.push_back(atn_dp_sizes[index]);
  }
  void *memory = nullptr;
  XP_HIP_CHECK(hipMalloc(&memory, sizeof(TransportArena) * image.size()));
  const hipError_t copied = hipMemcpy(memory, image.data(), sizeof(TransportArena) * image.size(),
                                      hipMemcpyHostToDevice);
  if (copied != hipSuccess) {
    (void)hipFree(memory);
    return fail(XP_ERROR_HIP, std::string("initialising the transport arenas failed: ") + hipGetErrorString(copied));
  }
  transport->arenas = static_cast<TransportArena *>(memory);
  *out = transport.release();
  return XP_OK;
}

int xp_transport_destroy(xp_transport_t transport) {
  if (transport == nullptr) {
    return XP_OK;
  }
  XP_HIP_CHECK(hipSetDevice(transport->device));
  XP_HIP_CHECK(hipDeviceSynchronize());
  (void)hipFree(transport->arenas);
  delete transport;
  return XP_OK;
}


int xp_transport_open(xp_transport_t transport, xp_stream_t stream) {
  XP_REQUIRE(transport != nullptr, "transport must be non-null");
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_open(transport_args(transport, 0)), stream);
}

int xp_transport_submit(xp_transport_t transport, int arena, int64_t payload_rows, int64_t layer_ordinal,
                        int forward_mode, int output_requirement, int dp_row_layout,
                        const void *dp_rank_payload_rows, int64_t dp_rank_count, int dp_rows_i64,
                        xp_stream_t stream) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(layer_ordinal >= 0, "layer ordinal must be non-negative");
  XP_REQUIRE(forward_mode == XP_FORWARD_PREFILL || forward_mode == XP_FORWARD_DECODE || forward_mode == XP_FORWARD_IDLE,
             "forward mode is outside the FFN vocabulary");
  XP_REQUIRE(output_requirement == XP_OUTPUT_PER_RANK_COMPLETE || output_requirement == XP_OUTPUT_GROUP_SUM_COMPLETE,
             "output requirement is outside the FFN vocabulary");
  XP_REQUIRE(dp_row_layout >= XP_DP_ROWS_NONE && dp_row_layout <= XP_DP_ROWS_PACKED_BY_RANK,
             "DP row layout is outside the FFN vocabulary");
  const int64_t capacity = transport->capacities[arena];
  const int32_t dp_size = transport->atn_dp_sizes[arena];
  XP_REQUIRE(payload_rows > 0 && payload_rows <= capacity, "xpool FFN request row count exceeds Transport capacity");
  const bool present = dp_rank_payload_rows != nullptr && dp_rank_count != 0;
  if (dp_size == 1) {
    XP_REQUIRE(dp_row_layout == XP_DP_ROWS_NONE && !present,
               "xpool DP-one request must use NONE without a per-rank row vector");
  } else {
    XP_REQUIRE(dp_row_layout != XP_DP_ROWS_NONE, "xpool DP request requires UNIFORM_BY_RANK or PACKED_BY_RANK");
    XP_REQUIRE(present && dp_rank_count == dp_size,
               "xpool FFN shim DP-rank payload rows must have one entry per attention DP rank");
  }
  TransportArgs args = transport_args(transport, arena);
  args.payload_rows = static_cast<uint64_t>(payload_rows);
  args.request = RequestMetadata{static_cast<uint64_t>(layer_ordinal), static_cast<uint32_t>(forward_mode),
                                 static_cast<uint32_t>(output_requirement), static_cast<uint32_t>(dp_row_layout), 0};
  args.dp_rows = present ? dp_rank_payload_rows : nullptr;
  args.dp_rows_count = present ? static_cast<uint32_t>(dp_rank_count) : 0;
  args.dp_rows_i64 = dp_rows_i64 != 0 ? 1u : 0u;
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_submit(args), stream);
}

int xp_transport_evaluate(xp_transport_t transport, int arena, const uint32_t *fault_word, xp_stream_t stream) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  TransportArgs args = transport_args(transport, arena);
  args.fault = fault_word;
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_evaluate(args), stream);
}

int xp_transport_complete(xp_transport_t transport, int arena, void *output, int64_t output_elements,
                          int payload_dtype, int64_t timeout_ns, xp_stream_t stream) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(output_elements >= 0, "output element count must be non-negative");
  XP_REQUIRE(output != nullptr || output_elements == 0, "output must be non-null when it has elements");
  XP_REQUIRE((reinterpret_cast<uintptr_t>(output) & 1u) == 0, "output must be 2-byte aligned 16-bit values");
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  TransportArgs args = transport_args(transport, arena);
  args.output = static_cast<uint16_t *>(output);
  args.output_elements = static_cast<uint64_t>(output_elements);
  args.output_nan2 = payload == kPayloadF16 ? F16Payload::kPoison2 : Bf16Payload::kPoison2;
  const uint64_t nanoseconds = timeout_ns > 0 ? static_cast<uint64_t>(timeout_ns) : kTransportDefaultTimeoutNs;
  // ticks = ns * kHz / 1e6, kept in range for timeouts up to hours.
  args.timeout_ticks = nanoseconds / 1000 * transport->wall_clock_khz / 1000 + 1;
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_complete(args), stream);
}

int xp_transport_settle(xp_transport_t transport, int arena, const uint32_t *fault_word, void *output,
                        int64_t output_elements, int payload_dtype, xp_stream_t stream) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(output_elements >= 0, "output element count must be non-negative");
  XP_REQUIRE(output != nullptr || output_elements == 0, "output must be non-null when it has elements");
  XP_REQUIRE((reinterpret_cast<uintptr_t>(output) & 1u) == 0, "output must be 2-byte aligned 16-bit values");
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  TransportArgs args = transport_args(transport, arena);
  args.fault = fault_word;
  args.output = static_cast<uint16_t *>(output);
  args.output_elements = static_cast<uint64_t>(output_elements);
  args.output_nan2 = payload == kPayloadF16 ? F16Payload::kPoison2 : Bf16Payload::kPoison2;
  args.timeout_ticks = kTransportDefaultTimeoutNs / 1000 * transport->wall_clock_khz / 1000 + 1;
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_settle(args), stream);
}

int xp_transport_drain(xp_transport_t transport, xp_stream_t stream) {
  XP_REQUIRE(transport != nullptr, "transport must be non-null");
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_drain(transport_args(transport, 0)), stream);
}

int xp_transport_publish_failure(xp_transport_t transport, int arena, int result_code, xp_stream_t stream) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(result_code >= XP_RESULT_OK && result_code <= XP_RESULT_TIMEOUT, "result code is outside the vocabulary");
  TransportArgs args = transport_args(transport, arena);
  args.code = static_cast<uint32_t>(result_code);
  std::lock_guard<std::mutex> guard(transport->mutex);
  return launch_transport(transport, make_transport_publish_failure(args), stream);
}

int xp_transport_snapshot(xp_transport_t transport, int arena, xp_arena_snapshot *out) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(out != nullptr, "output pointer must be non-null");
  XP_HIP_CHECK(hipSetDevice(transport->device));
  XP_HIP_CHECK(hipDeviceSynchronize());
  TransportArena image{};
  XP_HIP_CHECK(hipMemcpy(&image, transport->arenas + arena, sizeof image, hipMemcpyDeviceToHost));
  std::memset(out, 0, sizeof *out);
  out->mailbox_status = image.mailbox.status;
  out->result_code = image.mailbox.result_code;
  out->payload_rows = image.mailbox.payload_rows;
  out->layer_ordinal = image.mailbox.request.layer_ordinal;
  out->forward_mode = image.mailbox.request.forward_mode;
  out->output_requirement = image.mailbox.request.output_requirement;
  out->dp_row_layout = image.mailbox.request.dp_row_layout;
  out->shutdown = image.shutdown;
  out->generation_failure = image.generation_failure;
  out->violations = image.violations;
  out->instance_outcome = image.instance_outcome;
  out->atn_dp_size = image.atn_dp_size;
  out->payload_row_capacity = image.payload_row_capacity;
  std::memcpy(out->dp_rank_payload_rows, image.dp_rank_payload_rows, sizeof out->dp_rank_payload_rows);
  return XP_OK;
}

int xp_transport_probe(xp_transport_t transport, int arena, int scenario, uint32_t *observed, int max_words) {
  XP_REQUIRE(valid_arena(transport, arena), "arena index is outside the transport");
  XP_REQUIRE(scenario >= 0 && scenario <= 6, "probe scenario must be between 0 and 6");
  XP_REQUIRE(observed != nullptr && max_words >= 16, "observation buffer must hold 16 words");
  XP_HIP_CHECK(hipSetDevice(transport->device));
  void *words = nullptr;
  XP_HIP_CHECK(hipMalloc(&words, 16 * sizeof(uint32_t)));
  TransportArgs args = transport_args(transport, arena);
  args.output = static_cast<uint16_t *>(words);
  args.code = static_cast<uint32_t>(scenario);
  hipError_t status = hipMemset(words, 0xff, 16 * sizeof(uint32_t));
  if (status == hipSuccess) {
    std::lock_guard<std::mutex> guard(transport->mutex);
    status = launch(make_transport_probe(args), nullptr);
  }
  if (status == hipSuccess) {
    status = hipDeviceSynchronize();
  }
  if (status == hipSuccess) {
    status = hipMemcpy(observed, words, 16 * sizeof(uint32_t), hipMemcpyDeviceToHost);
  }
  (void)hipFree(words);
  if (status != hipSuccess) {
    return fail(XP_ERROR_HIP, std::string("transport probe failed: ") + hipGetErrorString(status));
  }
  return XP_OK;
}


// ------------------------------------------------------------------ MoE

size_t xp_moe_router_workspace_bytes(int64_t rows, int64_t hidden, int64_t experts, int precision) {
  if (rows <= 0 || hidden <= 0 || experts <= 0) {
    return 0;
  }
  return router_workspace(rows, hidden, experts, precision).bytes;
}

int xp_moe_router_topk(const void *logits, int logits_dtype, int64_t rows, int64_t experts, int64_t topk,
                       int algorithm, const float *correction_bias, int renormalize, int weight_rounding,
                       int32_t *ids, float *weights, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0, "row count must be non-negative");
  XP_REQUIRE(logits_dtype == XP_DTYPE_BF16 || logits_dtype == XP_DTYPE_F16 || logits_dtype == XP_DTYPE_F32,
             "logits must be bf16, fp16 or fp32");
  XP_REQUIRE(experts >= 1 && experts <= kMoeMaxExperts, "the router supports 1 to 1024 experts");
  XP_REQUIRE(topk >= 1 && topk <= experts && topk <= 64, "topk must be between 1 and min(experts, 64)");
  XP_REQUIRE(algorithm == XP_ROUTER_SOFTMAX || algorithm == XP_ROUTER_SIGMOID, "router algorithm is unknown");
  XP_REQUIRE(weight_rounding == XP_TOPK_ROUNDING_NONE || weight_rounding == XP_TOPK_ROUNDING_LOGITS_DTYPE,
             "TopK weight rounding is unknown");
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(logits != nullptr && ids != nullptr && weights != nullptr, "router pointers must be non-null");
  RouterTopkArgs args{};
  args.logits = logits;
  args.correction_bias = correction_bias;
  args.ids = ids;
  args.weights = weights;
  args.rows = rows;
  args.experts = static_cast<int32_t>(experts);
  args.topk = static_cast<int32_t>(topk);
  args.logits_f32 = logits_dtype == XP_DTYPE_F32 ? 1 : 0;
  args.payload = logits_dtype == XP_DTYPE_F16 ? kPayloadF16 : kPayloadBf16;
  args.softmax = algorithm == XP_ROUTER_SOFTMAX ? 1 : 0;
  args.renormalize = renormalize != 0 ? 1 : 0;
  args.round_to_logits = weight_rounding == XP_TOPK_ROUNDING_LOGITS_DTYPE ? 1 : 0;
  XP_HIP_CHECK(launch(make_router_topk(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

int xp_moe_router(const void *hidden_states, int64_t rows, int64_t hidden, const void *router_weights,
                  int64_t experts, int64_t topk, int algorithm, int precision, int payload_dtype,
                  const float *correction_bias, int renormalize, int weight_rounding, int32_t *ids, float *weights,
                  void *workspace, size_t workspace_bytes, xp_stream_t stream) {
  XP_REQUIRE(rows >= 0, "row count must be non-negative");
  XP_REQUIRE(hidden > 0, "hidden size must be positive");
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  if (const int status = validate_router(experts, topk, algorithm, precision, weight_rounding); status != XP_OK) {
    return status;
  }
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(hidden_states != nullptr && router_weights != nullptr && ids != nullptr && weights != nullptr,
             "router pointers must be non-null");
  XP_REQUIRE(!router_uses_mfma(hidden, experts, precision) || (aligned16(hidden_states) && aligned16(router_weights)),
             "router inputs must be 16-byte aligned");
  const RouterWorkspace layout = router_workspace(rows, hidden, experts, precision);
  XP_REQUIRE(workspace != nullptr && workspace_bytes >= layout.bytes && aligned16(workspace),
             "router workspace is missing or smaller than xp_moe_router_workspace_bytes");
  RouterBinding binding{};
  binding.x = static_cast<const uint16_t *>(hidden_states);
  binding.w = router_weights;
  binding.correction_bias = correction_bias;
  binding.ids = ids;
  binding.weights = weights;
  binding.workspace = static_cast<uint8_t *>(workspace);
  binding.rows = rows;
  binding.hidden = hidden;
  binding.experts = experts;
  binding.topk = topk;
  binding.algorithm = algorithm;
  binding.precision = precision;
  binding.renormalize = renormalize;
  binding.weight_rounding = weight_rounding;
  binding.payload = payload;
  const RouterLaunches launches = make_router_launches(binding, rows);
  const hipStream_t hip_stream = static_cast<hipStream_t>(stream);
  for (const KernelLaunch *kernel : {&launches.logits, &launches.logits_reduce, &launches.topk}) {
    XP_HIP_CHECK(launch(*kernel, hip_stream));
  }
  return XP_OK;
}

int xp_moe_finalize_routing(const int32_t *routed_ids, const float *routed_weights, int64_t capacity,
                            int64_t routed_topk, int32_t *final_ids, float *final_weights, int64_t effective_topk,
                            const int64_t *payload_rows, int64_t routed_expert_count, float routed_scaling_factor,
                            xp_stream_t stream) {
  XP_REQUIRE(capacity >= 0 && routed_topk >= 1 && effective_topk >= routed_topk, "routing geometry is inconsistent");
  XP_REQUIRE(routed_expert_count >= routed_topk, "Routing Metadata Expert counts are inconsistent");
  XP_REQUIRE(routed_scaling_factor > 0.0f && routed_scaling_factor < __builtin_inff(),
             "routed scaling factor must be finite and positive");
  if (capacity == 0) {
    return XP_OK;
  }
  XP_REQUIRE(routed_ids != nullptr && routed_weights != nullptr && final_ids != nullptr && final_weights != nullptr &&
                 payload_rows != nullptr,
             "routing pointers must be non-null");
  FinalizeRoutingArgs args{};
  args.routed_ids = routed_ids;
  args.routed_weights = routed_weights;
  args.final_ids = final_ids;
  args.final_weights = final_weights;
  args.payload_rows = payload_rows;
  args.capacity = capacity;
  args.routed_topk = static_cast<int32_t>(routed_topk);
  args.effective_topk = static_cast<int32_t>(effective_topk);
  args.routed_experts = static_cast<int32_t>(routed_expert_count);
  args.shared_weight = 1.0f / routed_scaling_factor;
  XP_HIP_CHECK(launch(make_finalize_routing(args), static_cast<hipStream_t>(stream)));
  return XP_OK;
}

size_t xp_moe_workspace_bytes(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk) {
  if (rows <= 0 || hidden <= 0 || intermediate <= 0 || experts <= 0 || topk <= 0) {
    return 0;
  }
  return moe_workspace(rows, hidden, intermediate, experts, topk).bytes;
}

int xp_moe_workspace_layout(int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts, int64_t topk,
                            size_t *offsets) {
  XP_REQUIRE(rows > 0 && hidden > 0 && intermediate > 0 && experts > 0 && topk > 0, "geometry must be positive");
  XP_REQUIRE(offsets != nullptr, "output pointer must be non-null");
  const MoeWorkspace layout = moe_workspace(rows, hidden, intermediate, experts, topk);
  offsets[0] = layout.expert_end;
  offsets[1] = layout.sorted_route;
  offsets[2] = layout.tile_expert;
  offsets[3] = layout.tile_row0;
  offsets[4] = layout.activated;
  offsets[5] = layout.route_out;
  return XP_OK;
}

int xp_moe_experts(const void *hidden_states, int64_t rows, int64_t hidden, int64_t intermediate, int64_t experts,
                   int64_t topk, const void *w_gate_up, const void *w_down, const float *gate_up_bias,
                   const float *down_bias, const int32_t *topk_ids, const float *topk_weights,
                   float routed_scaling_factor, int activation, int approximate_tanh, float alpha, float limit,
                   float up_offset, int payload_dtype, void *output, void *workspace, size_t workspace_bytes,
                   xp_stream_t stream) {
  XP_REQUIRE(rows >= 0, "row count must be non-negative");
  int32_t payload = kPayloadBf16;
  if (const int status = payload_kind(payload_dtype, payload); status != XP_OK) {
    return status;
  }
  if (const int status = validate_experts(rows, hidden, intermediate, experts, topk); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(activation == XP_ACTIVATION_SILU || activation == XP_ACTIVATION_RELU || activation == XP_ACTIVATION_GELU,
             "Experts activation must be SiLU, ReLU or GELU");
  XP_REQUIRE(approximate_tanh == 0 || activation == XP_ACTIVATION_GELU, "the tanh approximation is GELU's only");
  XP_REQUIRE(activation != XP_ACTIVATION_SILU || alpha > 0.0f, "SiLU alpha must be positive");
  if (rows == 0) {
    return XP_OK;
  }
  XP_REQUIRE(hidden_states != nullptr && w_gate_up != nullptr && w_down != nullptr && topk_ids != nullptr &&
                 topk_weights != nullptr && output != nullptr,
             "Experts pointers must be non-null");
  XP_REQUIRE(aligned16(hidden_states) && aligned16(w_gate_up) && aligned16(w_down) && aligned16(output) &&
                 aligned16(gate_up_bias) && aligned16(down_bias),
             "Experts tensors must be 16-byte aligned");
  const MoeWorkspace layout = moe_workspace(rows, hidden, intermediate, experts, topk);
  XP_REQUIRE(workspace != nullptr && workspace_bytes >= layout.bytes && aligned16(workspace),
             "Experts workspace is missing or smaller than xp_moe_workspace_bytes");
  ExpertsBinding binding{};
  binding.x = static_cast<const uint16_t *>(hidden_states);
  binding.w_gate_up = static_cast<const uint16_t *>(w_gate_up);
  binding.w_down = static_cast<const uint16_t *>(w_down);
  binding.ids = topk_ids;
  binding.weights = topk_weights;
  binding.out = static_cast<uint16_t *>(output);
  binding.workspace = static_cast<uint8_t *>(workspace);
  binding.rows = rows;
  binding.hidden = hidden;
  binding.intermediate = intermediate;
  binding.experts = experts;
  binding.topk = topk;
  binding.scale = routed_scaling_factor;
  binding.act = GatedSilu{alpha, limit, up_offset,
                          activation == XP_ACTIVATION_RELU   ? kActivationRelu
                          : activation == XP_ACTIVATION_GELU ? kActivationGelu
                                                             : kActivationSilu,
                          approximate_tanh != 0 ? 1 : 0};
  binding.payload = payload;
  binding.bias_gate_up = gate_up_bias;
  binding.bias_down = down_bias;
  ExpertsLaunches launches;
  if (const int status = make_experts_launches(binding, rows, launches); status != XP_OK) {
    return status;
  }
  const hipStream_t hip_stream = static_cast<hipStream_t>(stream);
  for (const KernelLaunch *kernel : {&launches.sort, &launches.gate_up, &launches.down, &launches.combine}) {
    XP_HIP_CHECK(launch(*kernel, hip_stream));
  }
  return XP_OK;
}

// ------------------------------------------------------------------ MoE layer kind

int xp_moe_layer_register(xp_agent_t agent, int instance_index, int layer_ordinal, const xp_moe_layer_desc *desc,
                          const void *gate_up, const void *down, const float *gate_up_bias, const float *down_bias,
                          const void *router, const float *correction_bias, const void *norm_weight, float eps) {
  XP_REQUIRE(agent != nullptr, "agent must be non-null");
  XP_REQUIRE(instance_index >= 0 && layer_ordinal >= 0, "instance index and layer ordinal must be non-negative");
  if (const int status = validate_moe_desc(desc); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(gate_up != nullptr && down != nullptr && router != nullptr, "MoE layer weights must be non-null");
  XP_REQUIRE(aligned16(gate_up) && aligned16(down) && aligned16(router) &&
                 (norm_weight == nullptr || aligned16(norm_weight)) && aligned_to(correction_bias, 4),
             "MoE layer weights must be 16-byte aligned (the correction bias 4-byte aligned)");
  XP_REQUIRE((gate_up_bias != nullptr) == ((desc->biases & 1) != 0) && (down_bias != nullptr) == ((desc->biases & 2) != 0),
             "MoE projection biases must be given exactly as the descriptor's biases say");
  XP_REQUIRE(aligned16(gate_up_bias) && aligned16(down_bias), "MoE projection biases must be 16-byte aligned");
  XP_REQUIRE(norm_weight == nullptr || eps >= 0.0f, "RMSNorm epsilon must be non-negative");
  Layer layer{instance_index,
              layer_ordinal,
              desc->hidden,
              desc->intermediate,
              static_cast<const uint16_t *>(gate_up),
              static_cast<const uint16_t *>(down),
              static_cast<const uint16_t *>(norm_weight),
              eps};
  layer.kind = XP_LAYER_MOE;
  layer.moe = *desc;
  layer.moe.renormalize = desc->renormalize != 0 ? 1 : 0;
  if (const int status = payload_kind(desc->payload, layer.payload); status != XP_OK) {
    return status;
  }
  layer.router = router;
  layer.correction_bias = correction_bias;
  layer.gate_up_bias = gate_up_bias;
  layer.down_bias = down_bias;
  std::lock_guard<std::mutex> guard(agent->mutex);
  for (Layer &existing : agent->layers) {
    if (existing.instance_index == instance_index && existing.layer_ordinal == layer_ordinal) {
      existing = layer;
      return XP_OK;
    }
  }
  agent->layers.push_back(layer);
  return XP_OK;
}

size_t xp_moe_step_workspace_bytes(const xp_moe_layer_desc *desc, int64_t capacity) {
  if (validate_moe_desc(desc) != XP_OK || validate_moe_capacity(*desc, capacity) != XP_OK) {
    return 0;
  }
  return moe_step_workspace(*desc, capacity).bytes;
}

int xp_moe_step_workspace_layout(const xp_moe_layer_desc *desc, int64_t capacity, size_t *offsets) {
  if (const int status = validate_moe_desc(desc); status != XP_OK) {
    return status;
  }
  if (const int status = validate_moe_capacity(*desc, capacity); status != XP_OK) {
    return status;
  }
  XP_REQUIRE(offsets != nullptr, "output pointer must be non-null");
  const MoeStepWorkspace layout = moe_step_workspace(*desc, capacity);
  offsets[0] = layout.batch;
  offsets[1] = layout.router + router_workspace(capacity, desc->hidden, desc->routed_experts, desc->precision).logits;
  offsets[2] = layout.routed_ids;
  offsets[3] = layout.routed_weights;
  offsets[4] = layout.final_ids;
  offsets[5] = layout.final_weights;
  offsets[6] = layout.experts;
  offsets[7] = layout.bytes;
  return XP_OK;
}

int xp_moe_template_capture(xp_lane_t lane, const xp_moe_layer_desc *desc, int64_t capacity) {
  XP_REQUIRE(lane != nullptr, "lane must be non-null");
  if (const int status = validate_moe_desc(desc); status != XP_OK) {
    return status;
  }
  if (const int status = validate_moe_capacity(*desc, capacity); status != XP_OK) {
    return status;
  }
  xp_moe_layer_desc signature = *desc;
  signature.renormalize = desc->renormalize != 0 ? 1 : 0;
  const size_t needed = moe_step_workspace(signature, capacity).bytes;
  if (needed > lane->workspace_bytes) {
    return fail(XP_ERROR_CAPACITY, "Lane workspace is smaller than the template needs (" + std::to_string(needed) +
                                       " bytes)");
  }
  std::lock_guard<std::mutex> guard(lane->mutex);
  for (const auto &t : lane->templates) {
    if (t->kind == XP_LAYER_MOE && t->capacity == capacity && same_moe(t->moe, signature)) {
      return XP_OK;
    }
  }
  XP_HIP_CHECK(hipSetDevice(lane->agent->device));
  // Placeholder layer and binding: a replay rebinds every argument record before launching.
  Layer placeholder{};
  placeholder.kind = XP_LAYER_MOE;
  placeholder.moe = signature;
  placeholder.hidden = signature.hidden;
  placeholder.intermediate = signature.intermediate;
  MoeStepBinding binding{};
  binding.rows = capacity;
  binding.pool_rows = capacity;
  binding.workspace = lane->workspace;
  binding.fault = lane->fault;
  StepChain chain;
  if (const int status = make_moe_step(placeholder, binding, capacity, chain); status != XP_OK) {
    return status;
  }
  auto t = std::make_unique<Template>();
  t->kind = XP_LAYER_MOE;
  t->hidden = signature.hidden;
  t->intermediate = signature.intermediate;
  t->capacity = capacity;
  t->moe = signature;
  if (const int status = instantiate_template(*t, chain); status != XP_OK) {
    return status;
  }
  insert_template(lane, std::move(t));
  return XP_OK;
}

}  // extern "C"
