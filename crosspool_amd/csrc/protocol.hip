// Transport mailbox protocol on one device: the single-producer / single-consumer request
// mailbox between an Instance rank (the ffn_shim caller) and the agent that evaluates its
// requests, with the arena's sticky shutdown and canonical-failure words.
//
// Reference (CrossPool checkout):
//   * lifecycle Dormant -> Idle -> Staging -> Published -> Evaluated -> Idle | Closed and its
//     transitions: src/cext-include/xpool/transport/protocol.hpp:33-87, protocol.cuh:14-68;
//   * sticky arena words: src/cext-include/xpool/transport/arena.hpp (ArenaState),
//     arena.cuh:50-63 (publish_generation_failure);
//   * Instance transaction (claim, stage, publish, wait, acknowledge or close):
//     src/cext/transport/instance.cu:36-201;
//   * Resident service, request validation and drain: src/cext/transport/atnagent.cu:20-186.
//
// On one GPU both parties are in one process and the transaction is stream ordered:
// submit (Instance) -> Dense step -> evaluate (agent) -> complete (Instance), either all on
// the caller's stream with evaluate and complete in one launch (settle), or with the Dense
// step and evaluate on a Lane's stream between two events.  The reference's Instance
// kernel copies the payload into an IPC arena and polls for the result, because the agent
// is another process on another GPU; here the Lane reads the caller's rows and writes the
// caller's output directly, and the completion's bounded wait finds the result already
// published unless the agent side never ran.  Where the reference traps on a broken
// precondition (xpool::abort_if), these kernels count a violation in the arena, publish the
// canonical ProtocolMismatch failure and go on, so that every kernel exits.  Every access
// to a shared word is an atomic at system scope (the reference's cuda::atomic_ref default).

#include <type_traits>

#include "xp_kernels.hpp"

namespace xp {
namespace {

constexpr int kCompleteThreads = 256;
// Resident drain retries an Idle close that lost a race with a claiming Instance; the
// Instance then owns Staging, which ends the loop on the next observation.
constexpr int kDrainAttempts = 64;

__device__ __forceinline__ uint32_t load_acquire(const uint32_t *word) {
  return __hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_release(uint32_t *word, uint32_t value) {
  __hip_atomic_store(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
template <class T>
__device__ __forceinline__ T load_relaxed(const T *word) {
  return __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
template <class T>
__device__ __forceinline__ void store_relaxed(T *word, std::type_identity_t<T> value) {
  __hip_atomic_store(word, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Strong compare-exchange; returns the value observed (equal to `expected` on success).
__device__ __forceinline__ uint32_t compare_exchange(uint32_t *word, uint32_t expected, uint32_t desired) {
  __hip_atomic_compare_exchange_strong(word, &expected, desired, __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
  return expected;
}

// RequestMetadata::valid (protocol.hpp:25-28) over the closed vocabulary of ffn.hpp:56-70.
__device__ bool request_metadata_valid(const RequestMetadata &request) {
  const bool mode = request.forward_mode == 1 || request.forward_mode == 2 || request.forward_mode == 4;
  const bool requirement = request.output_requirement == 1 || request.output_requirement == 2;
  const bool layout = request.dp_row_layout <= 2;
  return mode && requirement && layout;
}

__device__ RequestMetadata load_request(const Mailbox &mailbox) {
  RequestMetadata request;
  request.layer_ordinal = load_relaxed(&mailbox.request.layer_ordinal);
  request.forward_mode = load_relaxed(&mailbox.request.forward_mode);
  request.output_requirement = load_relaxed(&mailbox.request.output_requirement);
  request.dp_row_layout = load_relaxed(&mailbox.request.dp_row_layout);
  request.reserved = 0;
  return request;
}

__device__ void store_request(Mailbox &mailbox, const RequestMetadata &request) {
  store_relaxed(&mailbox.request.layer_ordinal, request.layer_ordinal);
  store_relaxed(&mailbox.request.forward_mode, request.forward_mode);
  store_relaxed(&mailbox.request.output_requirement, request.output_requirement);
  store_relaxed(&mailbox.request.dp_row_layout, request.dp_row_layout);
  store_relaxed(&mailbox.request.reserved, 0u);
}

// A precondition the reference checks with xpool::abort_if does not hold: count it and
// publish the canonical ProtocolMismatch failure (first failure wins, as in arena.cuh:55-62).
__device__ void violate(TransportArena &arena) {
  __hip_atomic_fetch_add(&arena.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  (void)compare_exchange(&arena.generation_failure, kResultOk, kResultProtocolMismatch);
}

// ---- arena words (arena.hpp ArenaView, arena.cuh:50-63)
__device__ uint32_t generation_failure(TransportArena &arena) { return load_acquire(&arena.generation_failure); }

__device__ void publish_generation_failure(TransportArena &arena, uint32_t code) {
  if (code != kResultProtocolMismatch && code != kResultTimeout) {
    violate(arena);
    return;
  }
  const uint32_t observed = compare_exchange(&arena.generation_failure, kResultOk, code);
  if (observed != kResultOk && observed != code) {
    violate(arena);
  }
}

__device__ bool shutdown_requested(TransportArena &arena) { return load_acquire(&arena.shutdown) != 0; }
__device__ void publish_shutdown(TransportArena &arena) { store_release(&arena.shutdown, 1u); }

// ---- mailbox transitions (protocol.cuh:14-68)
__device__ uint32_t observe(TransportArena &arena) {
  const uint32_t value = load_acquire(&arena.mailbox.status);
  if (value > kMailboxClosed) {
    violate(arena);
  }
  return value;
}

__device__ void open_mailbox(TransportArena &arena) {
  if (observe(arena) != kMailboxDormant) {
    violate(arena);
    return;
  }
  store_release(&arena.mailbox.status, kMailboxIdle);
}

__device__ bool try_begin_staging(TransportArena &arena) {
  const uint32_t observed = compare_exchange(&arena.mailbox.status, kMailboxIdle, kMailboxStaging);
  if (observed > kMailboxClosed) {
    violate(arena);
  }
  return observed == kMailboxIdle;
}

__device__ bool publish_request(TransportArena &arena) {
  if (observe(arena) != kMailboxStaging || load_relaxed(&arena.mailbox.payload_rows) == 0 ||
      !request_metadata_valid(load_request(arena.mailbox))) {
    violate(arena);
    return false;
  }
  store_release(&arena.mailbox.status, kMailboxPublished);
  return true;
}

__device__ bool publish_result(TransportArena &arena, uint32_t code) {
  if (observe(arena) != kMailboxPublished) {
    violate(arena);
    return false;
  }
  store_relaxed(&arena.mailbox.result_code, code);
  store_release(&arena.mailbox.status, kMailboxEvaluated);
  return true;
}

// Request facts are cleared before Idle becomes visible to the next producer.
__device__ void acknowledge(TransportArena &arena) {
  if (observe(arena) != kMailboxEvaluated) {
    violate(arena);
    return;
  }
  store_relaxed(&arena.mailbox.result_code, kResultProtocolMismatch);
  store_relaxed(&arena.mailbox.payload_rows, uint64_t{0});
  store_request(arena.mailbox, RequestMetadata{});
  store_release(&arena.mailbox.status, kMailboxIdle);
}

__device__ void close_staging(TransportArena &arena) {
  if (observe(arena) != kMailboxStaging) {
    violate(arena);
    return;
  }
  store_release(&arena.mailbox.status, kMailboxClosed);
}

__device__ void close_evaluated(TransportArena &arena) {
  if (observe(arena) != kMailboxEvaluated) {
    violate(arena);
    return;
  }
  store_release(&arena.mailbox.status, kMailboxClosed);
}

__device__ bool try_close_idle(TransportArena &arena) {
  const uint32_t observed = compare_exchange(&arena.mailbox.status, kMailboxIdle, kMailboxClosed);
  if (observed > kMailboxClosed) {
    violate(arena);
  }
  return observed == kMailboxIdle;
}

// request_valid (atnagent.cu:34-46): the arena carries per-DP-rank rows exactly when its
// topology has more than one attention DP rank.
__device__ bool request_valid(TransportArena &arena) {
  const RequestMetadata request = load_request(arena.mailbox);
  const uint64_t rows = load_relaxed(&arena.mailbox.payload_rows);
  const uint32_t dp_size = arena.atn_dp_size;
  const bool layout_ok = dp_size == 1 ? request.dp_row_layout == 0
                                      : (request.dp_row_layout == 1 || request.dp_row_layout == 2);
  return request_metadata_valid(request) && rows != 0 && rows <= arena.payload_row_capacity && layout_ok;
}

// finish_terminal_mailbox (atnagent.cu:92-120): drive one mailbox towards Closed during
// drain, answering a request the agent side could already see.
__device__ void finish_terminal_mailbox(TransportArena &arena) {
  for (int attempt = 0; attempt < kDrainAttempts; ++attempt) {
    const uint32_t status = observe(arena);
    if (status == kMailboxIdle) {
      if (try_close_idle(arena)) {
        return;
      }
      continue;
    }
    if (status == kMailboxPublished) {
      const uint32_t failure = generation_failure(arena);
      (void)publish_result(arena, failure != kResultOk ? failure : kResultShutdown);
      return;
    }
    if (status == kMailboxDormant) {
      violate(arena);
    }
    return;
  }
}

// Drain of every arena the resident serves (atnagent.cu:136-147): shutdown first, then the
// mailbox.
__device__ void drain_all(const TransportArgs &a) {
  for (int index = 0; index < a.arena_count; ++index) {
    publish_shutdown(a.arenas[index]);
    finish_terminal_mailbox(a.arenas[index]);
  }
}

// ---------------------------------------------------------------- kernels
// Resident startup (atnagent.cu:124-129): every Dormant mailbox becomes Idle.
__global__ __launch_bounds__(64) void transport_open_kernel(TransportArgs a) {
  if (threadIdx.x == 0) {
    for (int index = 0; index < a.arena_count; ++index) {
      open_mailbox(a.arenas[index]);
    }
  }
}

// Instance claim, staging and publication (instance.cu:46-128).  The outcome word tells the
// completion whether the request reached Published (kOutcomePending) or ended before it.
__global__ __launch_bounds__(64) void transport_submit_kernel(TransportArgs a) {
  TransportArena &arena = a.arenas[a.arena];
  __shared__ uint32_t claim;
  const int lane = static_cast<int>(threadIdx.x);
  if (lane == 0) {
    // Claim: a canonical failure or shutdown rejects the request before staging.
    uint32_t outcome = kOutcomePending;
    const uint32_t failure = generation_failure(arena);
    if (failure != kResultOk || shutdown_requested(arena)) {
      outcome = failure != kResultOk ? failure : kResultShutdown;
    } else if (!try_begin_staging(arena)) {
      // Only a terminal arena may refuse the claim.
      if (observe(arena) != kMailboxClosed) {
        violate(arena);
      }
      const uint32_t terminal_failure = generation_failure(arena);
      if (terminal_failure == kResultOk && !shutdown_requested(arena)) {
        violate(arena);
      }
      const uint32_t settled = generation_failure(arena);
      outcome = settled != kResultOk ? settled : kResultShutdown;
    }
    claim = outcome;
  }
  __syncthreads();
  if (claim != kOutcomePending) {
    if (lane == 0) {
      store_relaxed(&arena.instance_outcome, claim);
    }
    return;
  }
  // Stage: per-DP-rank physical rows, range-checked into uint32 (instance.cu:86-103).
  bool bad_row = false;
  for (uint32_t index = static_cast<uint32_t>(lane); index < a.dp_rows_count; index += 64) {
    const int64_t value = a.dp_rows_i64 != 0 ? static_cast<const int64_t *>(a.dp_rows)[index]
                                             : static_cast<int64_t>(static_cast<const int32_t *>(a.dp_rows)[index]);
    bad_row = bad_row || value < 0 || value > static_cast<int64_t>(0xffffffffu);
    store_relaxed(&arena.dp_rank_payload_rows[index], static_cast<uint32_t>(value));
  }
  const bool any_bad_row = __ballot(bad_row) != 0;
  if (lane == 0) {
    // Publish: the staged facts become visible with the Staging -> Published release.
    store_relaxed(&arena.mailbox.payload_rows, a.payload_rows);
    store_request(arena.mailbox, a.request);
    const uint32_t failure = generation_failure(arena);
    const bool shutdown = shutdown_requested(arena);
    uint32_t outcome = kOutcomePending;
    if (any_bad_row) {
      violate(arena);
      store_relaxed(&arena.mailbox.result_code, kResultProtocolMismatch);
      close_staging(arena);
      outcome = kResultProtocolMismatch;
    } else if (failure != kResultOk || shutdown) {
      outcome = failure != kResultOk ? failure : kResultShutdown;
      store_relaxed(&arena.mailbox.result_code, outcome);
      close_staging(arena);
    } else if (!publish_request(arena)) {
      store_relaxed(&arena.mailbox.result_code, kResultProtocolMismatch);
      close_staging(arena);
      outcome = kResultProtocolMismatch;
    }
    store_relaxed(&arena.instance_outcome, outcome);
  }
}

// Agent side of one request (atnagent.cu:48-90, 155-170), after the Lane's Dense step: answer
// a Published request with Ok, or ProtocolMismatch when it is invalid or the Lane raised a
// fault, which also drains every arena of the resident.  A request the Instance closed before
// publishing has nothing to answer.
__device__ void evaluate_request(const TransportArgs &a) {
  TransportArena &arena = a.arenas[a.arena];
  const uint32_t status = observe(arena);
  if (status != kMailboxPublished) {
    if (status == kMailboxDormant) {
      violate(arena);
    }
    return;
  }
  uint32_t result = request_valid(arena) ? kResultOk : kResultProtocolMismatch;
  if (result == kResultOk && a.fault != nullptr && load_acquire(a.fault) != 0) {
    result = kResultProtocolMismatch;
  }
  (void)publish_result(arena, result);
  if (result != kResultOk) {
    drain_all(a);
  }
}

__global__ __launch_bounds__(64) void transport_evaluate_kernel(TransportArgs a) {
  if (threadIdx.x == 0) {
    evaluate_request(a);
  }
}

// Instance wait, result observation and acknowledgement (instance.cu:130-201).  Thread 0
// runs the protocol; on any result but Ok the workgroup fills the output with quiet NaNs,
// the reference's canonical failure output (instance.cu:28-31).
// Returns whether the output must carry the canonical failure.
__device__ bool complete_request(const TransportArgs &a) {
  TransportArena &arena = a.arenas[a.arena];
  const uint32_t outcome = load_relaxed(&arena.instance_outcome);
  uint32_t result = outcome;
  bool failed = true;
  if (outcome == kOutcomePending) {
    // Wait for the agent's terminal result within the deadline.
    const uint64_t started = wall_clock64();
    uint32_t status = observe(arena);
    bool timed_out = false;
    while (status != kMailboxEvaluated && status != kMailboxClosed) {
      if (wall_clock64() - started >= a.timeout_ticks) {
        timed_out = true;
        break;
      }
      __builtin_amdgcn_s_sleep(4);
      status = observe(arena);
    }
    if (timed_out) {
      // The reference traps unless a canonical failure explains the silence; this build
      // publishes Timeout as the canonical failure instead.
      if (generation_failure(arena) == kResultOk) {
        publish_generation_failure(arena, kResultTimeout);
      }
      result = generation_failure(arena);
    } else if (status != kMailboxEvaluated) {
      violate(arena);  // only the Instance closes a request it published
      result = generation_failure(arena);
    } else {
      const uint32_t failure = generation_failure(arena);
      const uint32_t mailbox_result = load_relaxed(&arena.mailbox.result_code);
      result = mailbox_result == kResultOk || failure == kResultOk ? mailbox_result : failure;
      if (result > kResultTimeout) {
        violate(arena);
        result = kResultProtocolMismatch;
      }
      if (result != kResultOk) {
        close_evaluated(arena);
      } else {
        failed = false;
        if (shutdown_requested(arena)) {
          close_evaluated(arena);  // the Ok output stands; the arena ends
        } else {
          acknowledge(arena);
        }
      }
    }
  }
  store_relaxed(&arena.instance_outcome, result);
  return failed;
}

// The canonical failure output: every value a quiet NaN of the payload dtype
// (static_cast<Scalar>(NAN), instance.cu:28-31).
__device__ void fill_failure_output(const TransportArgs &a) {
  const uint64_t elements = a.output_elements;
  const bool aligned = (reinterpret_cast<uintptr_t>(a.output) & 15u) == 0;
  const uint64_t vectors = aligned ? elements / 8 : 0;
  const u32x4 poison = {a.output_nan2, a.output_nan2, a.output_nan2, a.output_nan2};
  for (uint64_t index = threadIdx.x; index < vectors; index += kCompleteThreads) {
    store16(a.output + index * 8, poison);
  }
  for (uint64_t index = vectors * 8 + threadIdx.x; index < elements; index += kCompleteThreads) {
    a.output[index] = static_cast<uint16_t>(a.output_nan2 & 0xffffu);
  }
}

// Instance wait, result observation and acknowledgement (instance.cu:130-201).  Thread 0
// runs the protocol; on any result but Ok the workgroup fills the output with quiet NaNs.
__global__ __launch_bounds__(kCompleteThreads) void transport_complete_kernel(TransportArgs a) {
  __shared__ uint32_t fill;
  if (threadIdx.x == 0) {
    fill = complete_request(a) ? 1u : 0u;
  }
  __syncthreads();
  if (fill != 0 && a.output != nullptr) {
    fill_failure_output(a);
  }
}

// Agent answer and Instance completion in one launch, for a request whose Dense step ran on
// the caller's own stream: the evaluation is ordered before the completion's observation by
// program order within thread 0, so the completion never waits.
__global__ __launch_bounds__(kCompleteThreads) void transport_settle_kernel(TransportArgs a) {
  __shared__ uint32_t fill;
  if (threadIdx.x == 0) {
    evaluate_request(a);
    fill = complete_request(a) ? 1u : 0u;
  }
  __syncthreads();
  if (fill != 0 && a.output != nullptr) {
    fill_failure_output(a);
  }
}

// Host-requested drain (TransportResident drain, atnagent.cu:136-147).
__global__ __launch_bounds__(64) void transport_drain_kernel(TransportArgs a) {
  if (threadIdx.x == 0) {
    drain_all(a);
  }
}

// Agent side publication of a canonical failure into one arena (atnagent.cu:20-32).
__global__ __launch_bounds__(64) void transport_publish_failure_kernel(TransportArgs a) {
  if (threadIdx.x == 0) {
    publish_generation_failure(a.arenas[a.arena], a.code);
  }
}

// The reference's device-side protocol tests, one scenario per launch, each writing its
// observations as uint32 words to `output`:
//   0 lifecycle and body reset                 (view_test.cu:68-92, 154-179)
//   1 repeated canonical timeout               (view_test.cu:94-100, 181-196)
//   2 Instance closes Staging for shutdown     (view_test.cu:102-110, 198-213)
//   3 Instance closes an evaluated failure     (view_test.cu:112-131, 215-231)
//   4 successful result kept through shutdown  (view_test.cu:133-150, 233-248)
//   5 over-capacity request published          (shutdown_test.cu:173-184)
//   6 rejected request consumed and closed     (shutdown_test.cu:186-191)
__global__ __launch_bounds__(64) void transport_probe_kernel(TransportArgs a) {
  if (threadIdx.x != 0) {
    return;
  }
  TransportArena &arena = a.arenas[a.arena];
  uint32_t *observed = reinterpret_cast<uint32_t *>(a.output);
  const RequestMetadata decode_request{0, 2, 1, 0, 0};
  switch (a.code) {
    case 0: {
      observed[0] = observe(arena);
      open_mailbox(arena);
      observed[1] = observe(arena);
      observed[2] = try_begin_staging(arena) ? 1u : 0u;
      store_relaxed(&arena.mailbox.payload_rows, uint64_t{2});
      store_request(arena.mailbox, RequestMetadata{3, 2, 1, 0, 0});
      (void)publish_request(arena);
      observed[3] = observe(arena);
      (void)publish_result(arena, kResultOk);
      observed[4] = observe(arena);
      observed[5] = load_relaxed(&arena.mailbox.result_code);
      acknowledge(arena);
      observed[6] = observe(arena);
      observed[7] = load_relaxed(&arena.mailbox.result_code);
      observed[8] = static_cast<uint32_t>(load_relaxed(&arena.mailbox.payload_rows));
      observed[9] = try_close_idle(arena) ? 1u : 0u;
      observed[10] = observe(arena);
      break;
    }
    case 1: {
      publish_generation_failure(arena, kResultTimeout);
      publish_generation_failure(arena, kResultTimeout);
      observed[0] = generation_failure(arena);
      break;
    }
    case 2: {
      open_mailbox(arena);
      observed[0] = try_begin_staging(arena) ? 1u : 0u;
      store_relaxed(&arena.mailbox.result_code, kResultShutdown);
      close_staging(arena);
      observed[1] = observe(arena);
      observed[2] = load_relaxed(&arena.mailbox.result_code);
      break;
    }
    case 3: {
      open_mailbox(arena);
      observed[0] = try_begin_staging(arena) ? 1u : 0u;
      store_relaxed(&arena.mailbox.payload_rows, uint64_t{1});
      store_request(arena.mailbox, decode_request);
      (void)publish_request(arena);
      publish_generation_failure(arena, kResultProtocolMismatch);
      (void)publish_result(arena, kResultProtocolMismatch);
      close_evaluated(arena);
      observed[1] = observe(arena);
      observed[2] = load_relaxed(&arena.mailbox.result_code);
      observed[3] = generation_failure(arena);
      break;
    }
    case 4: {
      open_mailbox(arena);
      observed[0] = try_begin_staging(arena) ? 1u : 0u;
      store_relaxed(&arena.mailbox.payload_rows, uint64_t{1});
      store_request(arena.mailbox, decode_request);
      (void)publish_request(arena);
      (void)publish_result(arena, kResultOk);
      publish_shutdown(arena);
      close_evaluated(arena);
      observed[1] = observe(arena);
      observed[2] = load_relaxed(&arena.mailbox.result_code);
      observed[3] = shutdown_requested(arena) ? 1u : 0u;
      break;
    }
    case 5: {
      const bool acquired = try_begin_staging(arena);
      observed[0] = acquired ? 1u : 0u;
      if (!acquired) {
        violate(arena);
        break;
      }
      store_relaxed(&arena.mailbox.payload_rows, arena.payload_row_capacity + 1);
      store_request(arena.mailbox, decode_request);
      (void)publish_request(arena);
      observed[1] = observe(arena);
      break;
    }
    case 6: {
      observed[0] = observe(arena);
      observed[1] = load_relaxed(&arena.mailbox.result_code);
      if (observed[0] != kMailboxEvaluated || observed[1] != kResultProtocolMismatch) {
        violate(arena);
      }
      close_evaluated(arena);
      observed[2] = observe(arena);
      break;
    }
    default:
      violate(arena);
      break;
  }
}

template <class Kernel>
KernelLaunch single_workgroup(Kernel kernel, const TransportArgs &args, unsigned threads) {
  KernelLaunch launch;
  launch.func = reinterpret_cast<const void *>(kernel);
  launch.grid = dim3(1, 1, 1);
  launch.block = dim3(threads, 1, 1);
  launch.set_args(args);
  return launch;
}

}  // namespace

KernelLaunch make_transport_open(const TransportArgs &args) {
  return single_workgroup(transport_open_kernel, args, 64);
}
KernelLaunch make_transport_submit(const TransportArgs &args) {
  return single_workgroup(transport_submit_kernel, args, 64);
}
KernelLaunch make_transport_evaluate(const TransportArgs &args) {
  return single_workgroup(transport_evaluate_kernel, args, 64);
}
KernelLaunch make_transport_complete(const TransportArgs &args) {
  return single_workgroup(transport_complete_kernel, args, kCompleteThreads);
}
KernelLaunch make_transport_settle(const TransportArgs &args) {
  return single_workgroup(transport_settle_kernel, args, kCompleteThreads);
}
KernelLaunch make_transport_drain(const TransportArgs &args) {
  return single_workgroup(transport_drain_kernel, args, 64);
}
KernelLaunch make_transport_publish_failure(const TransportArgs &args) {
  return single_workgroup(transport_publish_failure_kernel, args, 64);
}
KernelLaunch make_transport_probe(const TransportArgs &args) {
  return single_workgroup(transport_probe_kernel, args, 64);
}

}  // namespace xp
