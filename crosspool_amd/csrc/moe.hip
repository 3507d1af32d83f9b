// MoE Router and Experts of the FfnAgent path on gfx950.
//
// Reference (CrossPool checkout):
//   * Router: src/xpool/runtime/ffnagent/operators/routing.py:21-89 (router_topk_kernel:
//     softmax or sigmoid scores, selection-only correction bias, tie policy, renormalisation,
//     optional rounding to the logits dtype) and :148-190 (Router.run_into: the projection at
//     the declared precision, then TopK);
//   * routing finalisation: routing.py:193-307 (routed plus always-selected shared experts,
//     invalid rows past the live count);
//   * Experts: src/xpool/runtime/ffnagent/operators/moe.py:168-343 (routes grouped by expert,
//     grouped i_proj with the row gather and the fused activation, grouped o_proj with the
//     route scatter and the route weight, sum over a row's routes with the routed scaling
//     factor), whose numerics the reference spells out in
//     tests/suites/integration/runtime/ffnagent/test_operators.py:255-281.
//
// The reference sorts routes with a bitmatrix and drives triton_kernels' ragged matmul;
// here one workgroup counts routes per expert in LDS, scans the counts into sorted offsets
// and an expert tile table, and places each route.  With many routes per expert the
// projections run on the Dense path's 256 x 128 tile kernel in its grouped mode (gate_up
// gathering each route's token row itself); with few (decode) on the grouped split kernel,
// which streams each touched expert's weight rows as the MFMA M operand against 16-route
// token blocks read from L2.  A route's output row depends only on its
// own token row and expert, so the order of routes within an expert does not change any bit.

#include "xp_kernels.hpp"

// Wavefront reductions of the ROCm device library (ockl), linked into every HIP device build.
extern "C" __device__ __attribute__((const)) float __ockl_wfred_max_f32(float);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_add_f32(float);
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);

namespace xp {
namespace {

constexpr float kNegativeInfinity = -__builtin_inff();

// Wavefront reductions through the device library's DPP sequences (a handful of cycles per
// step, where a shuffle goes through the LDS crossbar); every lane receives the result.
__device__ __forceinline__ float wave_max_f32(float value) { return __ockl_wfred_max_f32(value); }
__device__ __forceinline__ float wave_add_f32(float value) { return __ockl_wfred_add_f32(value); }
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long value) {
  return __ockl_wfred_max_u64(value);
}

// fp32 bits mapped to an unsigned integer of the same order (-inf lowest, +inf highest).
__device__ __forceinline__ uint32_t ordered_bits(float value) {
  const uint32_t bits = __float_as_uint(value);
  return (bits & 0x80000000u) != 0 ? ~bits : bits | 0x80000000u;
}

// One fp32 value rounded to the 16-bit payload P (bf16 or fp16, round to nearest even), as
// bits and back: the rounding points of the reference's payload-dtype logits and weights.
template <class P>
__device__ __forceinline__ uint32_t payload_bits(float value);
template <>
__device__ __forceinline__ uint32_t payload_bits<Bf16Payload>(float value) {
  return float_to_bf16(value);
}
template <>
__device__ __forceinline__ uint32_t payload_bits<F16Payload>(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f32_rounding_point(value)));
}
template <class P>
__device__ __forceinline__ float payload_round(float value) {
  return P::widen(payload_bits<P>(value));
}

// The same with the payload chosen at run time (PayloadKind), for the FP32-precision
// Router logits kernel, whose inner loop is LDS arithmetic.
__device__ __forceinline__ float payload_widen(uint32_t bits16, int32_t payload) {
  return payload == kPayloadF16 ? F16Payload::widen(bits16) : Bf16Payload::widen(bits16);
}
__device__ __forceinline__ uint32_t payload_bits(float value, int32_t payload) {
  return payload == kPayloadF16 ? payload_bits<F16Payload>(value) : payload_bits<Bf16Payload>(value);
}

// ------------------------------------------------------------------ router
// One wavefront per row; lane l holds experts l, l + 64, ... (PER_LANE each: the fewest of
// 2, 4, 8 or 16 that cover the expert count, so a 128-expert Router selects over two
// values per lane rather than sixteen).  Experts past the count are padding: a score of 0,
// which adds exactly nothing to the softmax sum, and a key of 0, which never wins, so the
// choice of PER_LANE changes no bit of the result.
constexpr int kTopkMaxPerLane = kMoeMaxExperts / kWave;

__host__ __device__ constexpr int topk_per_lane(int experts) {
  return experts <= 2 * kWave ? 2 : experts <= 4 * kWave ? 4 : experts <= 8 * kWave ? 8 : kTopkMaxPerLane;
}

// TopK of row `row` by the calling wavefront (all 64 lanes); experts <= PER_LANE * 64.
// P is the dtype of 16-bit logits (a.payload): their widening and rounding points.
template <int PER_LANE, class P>
__device__ void router_topk_row(const RouterTopkArgs &a, int64_t row, int lane) {
  constexpr int kTopkPerLane = PER_LANE;
  const int experts = a.experts;
  float logit[kTopkPerLane];
  float maximum = kNegativeInfinity;
  if (a.partials != nullptr) {
    // The projection's K slices, added here in slice order.  Every slice load of a batch,
    // for all of the lane's experts, is issued before the first addition (a load per
    // slice, each waiting for the last, would put the memory latency in series); a batch
    // keeps 32 values in flight per lane.
    constexpr int kBatch = 32 / kTopkPerLane > 1 ? 32 / kTopkPerLane : 2;
    const int64_t plane = a.rows * experts;
    float sum[kTopkPerLane];
    for (int first = 0; first < a.slices; first += kBatch) {
      float part[kTopkPerLane][kBatch];
#pragma unroll
      for (int i = 0; i < kTopkPerLane; ++i) {
        const int expert = lane + i * kWave;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          part[i][j] = expert < experts && first + j < a.slices ? a.partials[(first + j) * plane + row * experts + expert]
                                                                : 0.0f;
        }
      }
#pragma unroll
      for (int i = 0; i < kTopkPerLane; ++i) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          if (first + j < a.slices) {
            sum[i] = first + j == 0 ? part[i][j] : sum[i] + part[i][j];
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      const int expert = lane + i * kWave;
      float value = kNegativeInfinity;
      if (expert < experts) {
        // One rounding of the sum to the payload dtype, stored as the logit.
        const uint32_t bits = payload_bits<P>(sum[i]);
        a.logits_out[row * experts + expert] = static_cast<uint16_t>(bits);
        value = P::widen(bits);
      }
      logit[i] = value;
      maximum = fmaxf(maximum, value);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      const int expert = lane + i * kWave;
      float value = kNegativeInfinity;
      if (expert < experts) {
        const int64_t index = row * experts + expert;
        value = a.logits_f32 != 0 ? static_cast<const float *>(a.logits)[index]
                                  : P::widen(static_cast<const uint16_t *>(a.logits)[index]);
      }
      logit[i] = value;
      maximum = fmaxf(maximum, value);
    }
  }
  float score[kTopkPerLane];
  if (a.softmax != 0) {
    maximum = wave_max_f32(maximum);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      score[i] = lane + i * kWave < experts ? expf(logit[i] - maximum) : 0.0f;
      sum += score[i];
    }
    sum = wave_add_f32(sum);
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      score[i] = score[i] / sum;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      score[i] = 1.0f / (1.0f + expf(-logit[i]));
    }
  }
  // Selection keys: the selection's ordered bits above a tie-break field that favours the
  // lower id (softmax) or the higher id (sigmoid), so one 64-bit wavefront maximum picks the
  // expert.  Padding experts never win: their key is 0.
  unsigned long long key[kTopkPerLane];
#pragma unroll
  for (int i = 0; i < kTopkPerLane; ++i) {
    const int expert = lane + i * kWave;
    float value = score[i];
    if (expert < experts && a.correction_bias != nullptr) {
      value += a.correction_bias[expert];
    }
    // Sigmoid stores the selection into the logits buffer and reads it back
    // (routing.py:62-65): 16-bit logits round it there.
    if (a.softmax == 0 && a.logits_f32 == 0) {
      value = payload_round<P>(value);
    }
    const uint32_t tie = a.softmax != 0 ? static_cast<uint32_t>(kMoeMaxExperts - 1 - expert)
                                        : static_cast<uint32_t>(expert);
    key[i] = expert < experts ? (static_cast<unsigned long long>(ordered_bits(value)) << 32) | (tie + 1) : 0ull;
  }

  // Lane `slot` keeps slot `slot`'s id and weight (topk <= 64).
  float normalizer = 0.0f;
  float chosen_weight = 0.0f;
  int chosen_id = -1;
  for (int slot = 0; slot < a.topk; ++slot) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      best = key[i] > best ? key[i] : best;
    }
    best = wave_max_u64(best);
    const uint32_t tie = static_cast<uint32_t>(best & 0xffffffffull) - 1;
    const int expert = a.softmax != 0 ? kMoeMaxExperts - 1 - static_cast<int>(tie) : static_cast<int>(tie);
    float own = 0.0f;
#pragma unroll
    for (int i = 0; i < kTopkPerLane; ++i) {
      if (lane + i * kWave == expert) {
        own = score[i];
        key[i] = 0ull;
      }
    }
    // The weight is the picked expert's score (for softmax without correction that is the
    // selected maximum itself).
    const float weight = __shfl(own, expert & (kWave - 1), kWave);
    normalizer += weight;
    if (lane == slot) {
      chosen_weight = weight;
      chosen_id = expert;
    }
  }
  if (lane < a.topk) {
    float weight = chosen_weight;
    if (a.renormalize != 0) {
      weight = weight / (normalizer > 0.0f ? normalizer : 1.0f);
    }
    if (a.round_to_logits != 0 && a.logits_f32 == 0) {
      weight = payload_round<P>(weight);
    }
    a.ids[row * a.topk + lane] = chosen_id;
    a.weights[row * a.topk + lane] = weight;
  }
}

template <int PER_LANE, class P>
__global__ __launch_bounds__(256) void router_topk_kernel(RouterTopkArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row < a.rows) {
    router_topk_row<PER_LANE, P>(a, row, threadIdx.x & (kWave - 1));
  }
}

// Router logits for the FP32 and FP32_LOGITS precisions, and for PAYLOAD when the geometry
// does not suit the MFMA projection (hidden or expert count not a multiple of 8): a
// workgroup computes a 16-row x 64-expert block; thread t owns row t / 16 and experts
// 4 (t % 16) .. + 3, each a sequential fp32 sum over the hidden dimension staged through LDS
// 64 columns at a time, stored as fp32 or rounded once to the payload dtype.
__global__ __launch_bounds__(256) void router_logits_kernel(RouterLogitsArgs a) {
  constexpr int ROWS = 16;
  constexpr int EXPERTS = 64;
  constexpr int CHUNK = 64;
  __shared__ float xs[ROWS][CHUNK + 1];
  __shared__ float ws[EXPERTS][CHUNK + 1];
  const int tid = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.y) * ROWS;
  const int expert0 = static_cast<int>(blockIdx.x) * EXPERTS;
  const int my_row = tid / 16;
  const int my_expert = (tid % 16) * 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t k0 = 0; k0 < a.hidden; k0 += CHUNK) {
    for (int index = tid; index < ROWS * CHUNK; index += 256) {
      const int r = index / CHUNK;
      const int c = index % CHUNK;
      const int64_t row = row0 + r;
      xs[r][c] = row < a.rows && k0 + c < a.hidden ? payload_widen(a.x[row * a.hidden + k0 + c], a.payload) : 0.0f;
    }
    for (int index = tid; index < EXPERTS * CHUNK; index += 256) {
      const int e = index / CHUNK;
      const int c = index % CHUNK;
      const int expert = expert0 + e;
      float value = 0.0f;
      if (expert < a.experts && k0 + c < a.hidden) {
        const int64_t offset = static_cast<int64_t>(expert) * a.hidden + k0 + c;
        value = a.weights_f32 != 0 ? static_cast<const float *>(a.w)[offset]
                                   : payload_widen(static_cast<const uint16_t *>(a.w)[offset], a.payload);
      }
      ws[e][c] = value;
    }
    __syncthreads();
    const int columns = a.hidden - k0 < CHUNK ? static_cast<int>(a.hidden - k0) : CHUNK;
    for (int c = 0; c < columns; ++c) {
      const float x = xs[my_row][c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = fmaf(x, ws[my_expert + j][c], acc[j]);
      }
    }
    __syncthreads();
  }
  const int64_t row = row0 + my_row;
  if (row < a.rows) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int expert = expert0 + my_expert + j;
      if (expert < a.experts) {
        if (a.out_payload != 0) {
          static_cast<uint16_t *>(a.logits)[row * a.experts + expert] = static_cast<uint16_t>(payload_bits(acc[j], a.payload));
        } else {
          static_cast<float *>(a.logits)[row * a.experts + expert] = acc[j];
        }
      }
    }
  }
}

// finalize_moe_routing_kernel (routing.py:193-227): routed slots keep their ids and
// weights, shared slots name experts routed_experts + s with weight 1 / scaling, rows at or
// past the live count read -1 / 0.
__global__ __launch_bounds__(256) void finalize_routing_kernel(FinalizeRoutingArgs a) {
  const int64_t index = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (index >= a.capacity * a.effective_topk) {
    return;
  }
  const int64_t row = index / a.effective_topk;
  const int slot = static_cast<int>(index % a.effective_topk);
  const bool live = a.payload_rows == nullptr || row < *a.payload_rows;
  const bool routed = slot < a.routed_topk;
  int32_t id = -1;
  float weight = 0.0f;
  if (live) {
    if (routed) {
      id = a.routed_ids[row * a.routed_topk + slot];
      weight = a.routed_weights[row * a.routed_topk + slot];
    } else {
      id = a.routed_experts + slot - a.routed_topk;
      weight = a.shared_weight;
    }
  }
  a.final_ids[index] = id;
  a.final_weights[index] = weight;
}

// ------------------------------------------------------------------ route sort
// Inclusive scan of one value per thread over a 1024-thread workgroup.
__device__ int block_inclusive_scan(int value, int *wave_totals) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int offset = 1; offset < kWave; offset <<= 1) {
    const int other = __shfl_up(value, offset, kWave);
    if (lane >= offset) {
      value += other;
    }
  }
  if (lane == kWave - 1) {
    wave_totals[wave] = value;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int running = 0;
    for (int w = 0; w < 1024 / kWave; ++w) {
      const int total = wave_totals[w];
      wave_totals[w] = running;
      running += total;
    }
  }
  __syncthreads();
  return value + wave_totals[wave];
}

// Routes held in registers per thread between the count and the placement (16384 routes,
// 2048 rows at top-8, in one pass; more are read again).
constexpr int kSortRoutesPerThread = 16;
// Up to this many routes the placement goes to LDS first and leaves in contiguous stores:
// placed straight into global memory, each route is a 4-byte store to its own cache line,
// and one CU's memory path takes those a few lanes per cycle (2048 rows at top-8: 32768
// such stores, most of the kernel's time).
constexpr int kSortStagedRoutes = 1024 * kSortRoutesPerThread;

// The fused TopK gives each of the workgroup's waves one row.
static_assert(kMoeFusedTopkRows <= 1024 / kWave, "one wave of moe_sort_kernel per fused TopK row");

// P: the payload of the fused TopK's 16-bit logits (the sort itself is dtype-free).
template <class P>
__global__ __launch_bounds__(1024) void moe_sort_kernel(MoeSortArgs a) {
  __shared__ int counts[kMoeMaxExperts];
  __shared__ int offsets[kMoeMaxExperts + 1];
  __shared__ int tiles[kMoeMaxExperts + 1];
  __shared__ int totals[1024 / kWave];
  __shared__ int32_t staged_route[kSortStagedRoutes];
  __shared__ float staged_weight[kSortStagedRoutes];
  const int tid = threadIdx.x;
  if (a.fused_topk != 0) {
    // Decode sizes: the Router's TopK runs here, one wave per row (the same code as
    // router_topk_kernel), and the routes it writes are read back below by this workgroup.
    if ((tid >> 6) < a.topk.rows) {
      const int per_lane = topk_per_lane(a.topk.experts);
      if (per_lane == 2) {
        router_topk_row<2, P>(a.topk, tid >> 6, tid & (kWave - 1));
      } else if (per_lane == 4) {
        router_topk_row<4, P>(a.topk, tid >> 6, tid & (kWave - 1));
      } else if (per_lane == 8) {
        router_topk_row<8, P>(a.topk, tid >> 6, tid & (kWave - 1));
      } else {
        router_topk_row<kTopkMaxPerLane, P>(a.topk, tid >> 6, tid & (kWave - 1));
      }
    }
    __syncthreads();
  }
  counts[tid] = 0;
  int32_t held_expert[kSortRoutesPerThread];
  float held_weight[kSortRoutesPerThread];
#pragma unroll
  for (int i = 0; i < kSortRoutesPerThread; ++i) {
    const int64_t route = tid + static_cast<int64_t>(i) * 1024;
    held_expert[i] = route < a.routes ? a.ids[route] : -1;
    held_weight[i] = route < a.routes ? a.weights[route] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSortRoutesPerThread; ++i) {
    if (held_expert[i] >= 0 && held_expert[i] < a.experts) {
      atomicAdd(&counts[held_expert[i]], 1);
    }
  }
  for (int64_t route = tid + 1024 * kSortRoutesPerThread; route < a.routes; route += 1024) {
    const int expert = a.ids[route];
    if (expert >= 0 && expert < a.experts) {
      atomicAdd(&counts[expert], 1);
    }
  }
  __syncthreads();
  const int count = tid < a.experts ? counts[tid] : 0;
  const int row_end = block_inclusive_scan(count, totals);
  __syncthreads();
  const int tile_end = block_inclusive_scan((count + a.tile_rows - 1) / a.tile_rows, totals);
  offsets[tid + 1] = row_end;
  tiles[tid + 1] = tile_end;
  if (tid == 0) {
    offsets[0] = 0;
    tiles[0] = 0;
  }
  __syncthreads();
  if (tid < a.experts) {
    a.expert_end[tid] = offsets[tid + 1];
    counts[tid] = offsets[tid];  // placement cursor
  }
  const int total_tiles = tiles[a.experts];
  for (int tile = tid; tile < a.max_tiles; tile += 1024) {
    if (tile >= total_tiles) {
      a.tile_expert[tile] = -1;
      a.tile_row0[tile] = 0;
      continue;
    }
    // The last expert whose first tile is at or before this one owns it.
    int low = 0;
    int high = a.experts - 1;
    while (low < high) {
      const int middle = (low + high + 1) / 2;
      if (tiles[middle] <= tile) {
        low = middle;
      } else {
        high = middle - 1;
      }
    }
    a.tile_expert[tile] = low;
    a.tile_row0[tile] = offsets[low] + (tile - tiles[low]) * a.tile_rows;
  }
  __syncthreads();
  const bool staged = a.routes <= kSortStagedRoutes;  // uniform over the workgroup
#pragma unroll
  for (int i = 0; i < kSortRoutesPerThread; ++i) {
    if (held_expert[i] >= 0 && held_expert[i] < a.experts) {
      const int position = atomicAdd(&counts[held_expert[i]], 1);
      if (staged) {
        staged_route[position] = static_cast<int32_t>(tid + i * 1024);
        staged_weight[position] = held_weight[i];
      } else {
        a.sorted_route[position] = static_cast<int32_t>(tid + i * 1024);
        a.sorted_weight[position] = held_weight[i];
      }
    }
  }
  if (staged) {
    __syncthreads();
    const int placed = offsets[a.experts];
    for (int position = tid; position < placed; position += 1024) {
      a.sorted_route[position] = staged_route[position];
      a.sorted_weight[position] = staged_weight[position];
    }
    return;
  }
  for (int64_t route = tid + 1024 * kSortRoutesPerThread; route < a.routes; route += 1024) {
    const int expert = a.ids[route];
    if (expert >= 0 && expert < a.experts) {
      const int position = atomicAdd(&counts[expert], 1);
      a.sorted_route[position] = static_cast<int32_t>(route);
      a.sorted_weight[position] = a.weights[route];
    }
  }
}

// ------------------------------------------------------------------ combine
// out[row] = p(scale * sum over the row's live routes, in slot order, of float(route
// output)), p the payload rounding (bf16 or fp16) -- the route reduction with the routed
// scaling factor (moe.py:336-343); rows whose slots are all -1 read 0.  With slots the sum
// of row r goes to out row slots[r] (the mailbox scatter); a slot outside the mailbox is
// skipped (the gather that read it has raised the Lane's fault bit).
template <class P>
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeCombineArgs a) {
  const int64_t chunks = a.hidden / 8;
  const int64_t index = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (index >= a.rows * chunks) {
    return;
  }
  const int64_t row = index / chunks;
  const int64_t chunk = index % chunks;
  int64_t out_row = row;
  if (a.slots != nullptr) {
    out_row = a.slots[row];
    if (out_row < 0 || out_row >= a.out_rows) {
      return;
    }
  }
  float sum[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  // Slots in batches: the batch's ids first, then its route rows, then the sums in slot
  // order (two memory round trips per batch instead of two per slot).
  constexpr int BATCH = 8;
  for (int first = 0; first < a.topk; first += BATCH) {
    int32_t expert[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      expert[b] = first + b < a.topk ? a.ids[row * a.topk + first + b] : -1;
    }
    u32x4 values[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const bool live = expert[b] >= 0 && expert[b] < a.experts;
      values[b] = live ? load16(a.routes + (row * a.topk + first + b) * a.hidden + chunk * 8) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      if (expert[b] < 0 || expert[b] >= a.experts) {
        continue;
      }
#pragma unroll
      for (int word = 0; word < 4; ++word) {
        sum[2 * word] += P::widen(values[b][word] & 0xffffu);
        sum[2 * word + 1] += P::widen(values[b][word] >> 16);
      }
    }
  }
  u32x4 packed;
#pragma unroll
  for (int word = 0; word < 4; ++word) {
    packed[word] = P::pack2(sum[2 * word] * a.scale, sum[2 * word + 1] * a.scale);
  }
  store16(a.out + out_row * a.hidden + chunk * 8, packed);
}

template <class Args>
KernelLaunch launch_of(const void *kernel, dim3 grid, unsigned threads, const Args &args) {
  KernelLaunch launch;
  launch.func = kernel;
  launch.grid = grid;
  launch.block = dim3(threads, 1, 1);
  launch.set_args(args);
  return launch;
}

unsigned blocks_for(int64_t items, int64_t per_block) {
  return static_cast<unsigned>((items + per_block - 1) / per_block);
}

}  // namespace

int moe_tile_rows(MoeTile tile) { return tile == MoeTile::Small ? grouped_split_rows() : grouped_tile_rows(tile); }

// Few routes per expert (at most 4 on average) stream each expert's weights through the
// grouped split kernel in 16-route tiles; more take the grouped tile kernel on the shortest
// expert tile that holds most experts' routes.  An expert's weights are read once per tile
// of its routes, and the LDS a tile's token rows do not take holds weight slabs in flight
// (the grouped projections are bound by the weight bytes each CU has in flight), so:
// 64-row tiles (two workgroups per CU, each with two of its three 64 x 128 weight slabs in
// flight) up to 40 routes per expert on
// average, 128-row tiles with the weights loaded nontemporally up to 80, 128-row tiles with
// plain loads (an expert split over two tiles finds its weights in the last-level cache
// for the second) up to 160, 256-row tiles above.  Measured at the Qwen3-30B-A3B shape
// (128 experts, top-8), layer us against the 256-row tile everywhere: 256 tokens 335 -> 288,
// 512 357 -> 304, 1024 391 -> 332, 2048 431 -> 418, 4096 unchanged (647 against 652 on
// 128-row tiles); 128 tokens (8 routes per expert) 298 us on 16-route tiles -> 279 on 64-row
// tiles, while at 48 / 64 tokens (3 / 4 routes per expert) the 64-row tiles lost (254 / 263
// -> 263 / 270 us).  (Those 64-row figures are of a 64 x 256 tile, one workgroup per CU; the
// 64 x 128 tile at two per CU since took 256 / 512 tokens to 255 / 265 us, while in the
// 80-route regime it won below the capacity's 1024 tokens and lost at them: 377 against
// 319 us, so the thresholds stand.)
MoeTile choose_moe_tile(int64_t routes, int64_t experts) {
  if (routes <= 4 * experts) {
    return MoeTile::Small;
  }
  if (routes <= 40 * experts) {
    return MoeTile::Rows64;
  }
  if (routes <= 80 * experts) {
    return MoeTile::Rows128Stream;
  }
  return routes <= 160 * experts ? MoeTile::Rows128 : MoeTile::Rows256;
}

template <class P>
const void *router_topk_kernel_for(int per_lane) {
  return per_lane == 2   ? reinterpret_cast<const void *>(&router_topk_kernel<2, P>)
         : per_lane == 4 ? reinterpret_cast<const void *>(&router_topk_kernel<4, P>)
         : per_lane == 8 ? reinterpret_cast<const void *>(&router_topk_kernel<8, P>)
                         : reinterpret_cast<const void *>(&router_topk_kernel<kTopkMaxPerLane, P>);
}

KernelLaunch make_router_topk(const RouterTopkArgs &args) {
  const int per_lane = topk_per_lane(args.experts);
  const void *kernel = args.payload == kPayloadF16 ? router_topk_kernel_for<F16Payload>(per_lane)
                                                   : router_topk_kernel_for<Bf16Payload>(per_lane);
  return launch_of(kernel, dim3(blocks_for(args.rows, 4)), 256, args);
}

KernelLaunch make_router_logits(const RouterLogitsArgs &args) {
  return launch_of(reinterpret_cast<const void *>(&router_logits_kernel),
                   dim3(blocks_for(args.experts, 64), blocks_for(args.rows, 16)), 256, args);
}

KernelLaunch make_finalize_routing(const FinalizeRoutingArgs &args) {
  return launch_of(reinterpret_cast<const void *>(&finalize_routing_kernel),
                   dim3(blocks_for(args.capacity * args.effective_topk, 256)), 256, args);
}

KernelLaunch make_moe_sort(const MoeSortArgs &args) {
  const bool f16 = args.fused_topk != 0 && args.topk.payload == kPayloadF16;
  return launch_of(f16 ? reinterpret_cast<const void *>(&moe_sort_kernel<F16Payload>)
                       : reinterpret_cast<const void *>(&moe_sort_kernel<Bf16Payload>),
                   dim3(1), 1024, args);
}

KernelLaunch make_moe_combine(const MoeCombineArgs &args) {
  return launch_of(args.payload == kPayloadF16 ? reinterpret_cast<const void *>(&moe_combine_kernel<F16Payload>)
                                                : reinterpret_cast<const void *>(&moe_combine_kernel<Bf16Payload>),
                   dim3(blocks_for(args.rows * (args.hidden / 8), 256)), 256, args);
}

}  // namespace xp
