// Transport kernels: byte copy, mailbox gather (+ fused RMSNorm) and scatter.
//
// Reference behaviour (CrossPool checkout):
//   * row copies of the Transport/Fabric payload, src/cext/transport/instance.cu:83-84,184-186
//     and src/cext/fabric/atnagent.cu:215,275, all through xpool::utils::cooperative::copy
//     (src/cext-include/xpool/utils/cooperative.cuh:37-55);
//   * the reference copies one contiguous row prefix with one 256-thread CTA; here a row is
//     gathered from an arbitrary mailbox slot by one 64-lane wavefront with 16-byte loads, no
//     LDS, and the whole grid participates.
// RMSNorm has no counterpart on the reference path (SGLang applies it before the shim); it is
// fused here so the GEMM reads normalised rows straight from the gathered batch.

#include "xp_kernels.hpp"

namespace xp {
namespace {

__global__ __launch_bounds__(256) void copy_bytes_kernel(CopyArgs a) {
  const uint64_t thread = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  const bool aligned =
      ((reinterpret_cast<uintptr_t>(a.destination) | reinterpret_cast<uintptr_t>(a.source) | a.bytes) & 15u) == 0;
  if (aligned) {
    const uint64_t vectors = a.bytes >> 4;
    for (uint64_t index = thread; index < vectors; index += stride) {
      store16(a.destination + (index << 4), load16(a.source + (index << 4)));
    }
  } else {
    for (uint64_t index = thread; index < a.bytes; index += stride) {
      a.destination[index] = a.source[index];
    }
  }
}

// One wavefront per row; CHUNKS 16-byte chunks per lane stay in registers between the
// sum-of-squares reduction and the normalised store (hidden <= CHUNKS * 512).  The norm
// weights go to LDS once per workgroup (its four rows share them), requested right behind
// the rows, so a row still costs one memory round trip, and the registers hold the row
// only: with a copy of the weights per wave as well, hidden 4096 took 147 VGPRs (three
// waves per SIMD) and hidden 5120 or 8192 all 256 (one).
// 16-byte store through a buffer resource: offsets past the resource's end are dropped.
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset, u32x4 value) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, value),
                                         rsrc, static_cast<int>(offset), 0, 0);
}

template <int CHUNKS, class P>
__global__ __launch_bounds__(256) void gather_rows_kernel(GatherArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t norm_lds[CHUNKS * kWave * 8];
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t chunks = a.hidden >> 3;
  const bool live = row < a.rows;
  const int32_t slot = live ? a.slots[row] : 0;
  const bool bad = live && (slot < 0 || static_cast<int64_t>(slot) >= a.pool_rows);
  const uint32_t row_bytes = static_cast<uint32_t>(a.hidden * 2);
  // The row through a buffer resource of its own: chunk c of lane l sits at byte offset
  // 16 l + 1024 c, a constant per chunk, and chunks past the row read as zero.
  const __amdgpu_buffer_rsrc_t source =
      make_rsrc(a.pool + static_cast<int64_t>(live && !bad ? slot : 0) * a.hidden, live && !bad ? row_bytes : 0u);
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * 16);
  u32x4 values[CHUNKS];
#pragma unroll
  for (int index = 0; index < CHUNKS; ++index) {
    values[index] = buffer_load16(source, lane_bytes + index * kWave * 16);
  }
  if (a.norm != nullptr) {  // uniform: every wave reaches the barrier
    for (int64_t chunk = threadIdx.x; chunk < chunks; chunk += 256) {
      store16(norm_lds + chunk * 8, load16(a.norm + chunk * 8));
    }
    __syncthreads();
  }
  if (!live) {
    return;
  }
  const __amdgpu_buffer_rsrc_t destination = make_rsrc(a.out + row * a.hidden, row_bytes);
  if (bad) {
    // Canonical failure: poison the row with quiet NaNs and raise the sticky fault bit.
    const u32x4 poison = {P::kPoison2, P::kPoison2, P::kPoison2, P::kPoison2};
    for (int64_t chunk = lane; chunk < chunks; chunk += kWave) {
      buffer_store16(destination, static_cast<uint32_t>(chunk * 16), poison);
    }
    if (lane == 0) {
      raise_fault(a.fault, kFaultSlotOutOfRange);
    }
    return;
  }
  if (a.norm == nullptr) {
#pragma unroll
    for (int index = 0; index < CHUNKS; ++index) {
      buffer_store16(destination, lane_bytes + index * kWave * 16, values[index]);
    }
    return;
  }
  // Chunks past the row are zero and add nothing to the sum.
  float squares = 0.0f;
#pragma unroll
  for (int index = 0; index < CHUNKS; ++index) {
    add_squares<P>(values[index], squares);
  }
  const float inverse = rms_inverse(squares, a.hidden, a.eps);
  // The row's bits are opaque here, so the compiler widens them again rather than keeping
  // the sum of squares' fp32 copies (twice the registers) alive across the reduction.
#pragma unroll
  for (int index = 0; index < CHUNKS; ++index) {
    __asm__ volatile("" : "+v"(values[index]));
  }
#pragma unroll
  for (int index = 0; index < CHUNKS; ++index) {
    const int64_t chunk = lane + index * kWave;
    const u32x4 weight = chunk < chunks ? load16(norm_lds + chunk * 8) : u32x4{0u, 0u, 0u, 0u};
    buffer_store16(destination, lane_bytes + index * kWave * 16, normalize_chunk<P>(values[index], inverse, weight));
  }
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(ScatterArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) {
    return;
  }
  const int32_t slot = a.slots[row];
  if (slot < 0 || static_cast<int64_t>(slot) >= a.pool_rows) {
    if (lane == 0) {
      raise_fault(a.fault, kFaultSlotOutOfRange);
    }
    return;
  }
  const int64_t chunks = a.hidden >> 3;
  const uint16_t *source = a.values + row * a.hidden;
  uint16_t *destination = a.pool + static_cast<int64_t>(slot) * a.hidden;
  for (int64_t chunk = lane; chunk < chunks; chunk += kWave) {
    store16(destination + chunk * 8, load16(source + chunk * 8));
  }
}

constexpr int64_t kMaxGatherChunks = 32;

template <int CHUNKS>
const void *gather_kernel_for(int32_t payload) {
  return payload == kPayloadF16 ? reinterpret_cast<const void *>(&gather_rows_kernel<CHUNKS, F16Payload>)
                                : reinterpret_cast<const void *>(&gather_rows_kernel<CHUNKS, Bf16Payload>);
}

// Fixed-order TP partial sum (the exchange step's arithmetic, src/cext/ffnagent/
// delivery.cu:74-127): each thread takes 8 consecutive elements (16 bytes) of every
// partial, issues all the partials' loads before the first add, and folds them in partial
// order into fp32 sums that start from 0, then rounds once to bf16 (nearest even).  The
// vectorisation changes the memory traffic, not the association order.  HBM-bound:
// (count + 1) * 2 bytes per element.  STREAMING uses nontemporal loads and stores, for
// folds larger than the last-level cache (measured at 8 x 84 MB: 138 against 156 us;
// for a fold that fits the cache they cost 13 %).
template <bool STREAMING>
__global__ __launch_bounds__(256) void reduce_partials_kernel(ReduceArgs a) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t index = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; index < a.vectors;
       index += stride) {
    u32x4 chunks[kMaxPartials];
#pragma unroll
    for (int k = 0; k < kMaxPartials; ++k) {
      if (k < a.count) {
        chunks[k] = STREAMING ? load16_stream(a.partials[k] + index * 8) : load16(a.partials[k] + index * 8);
      }
    }
    float sums[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < kMaxPartials; ++k) {
      if (k < a.count) {
#pragma unroll
        for (int word = 0; word < 4; ++word) {
          sums[2 * word] += bf16_to_float(chunks[k][word] & 0xffffu);
          sums[2 * word + 1] += bf16_to_float(chunks[k][word] >> 16);
        }
      }
    }
    u32x4 packed;
#pragma unroll
    for (int word = 0; word < 4; ++word) {
      packed[word] = pack_bf16x2(sums[2 * word], sums[2 * word + 1]);
    }
    if constexpr (STREAMING) {
      __builtin_nontemporal_store(packed, reinterpret_cast<u32x4 *>(a.out + index * 8));
    } else {
      store16(a.out + index * 8, packed);
    }
  }
}

}  // namespace

KernelLaunch make_copy(const CopyArgs &args) {
  KernelLaunch kernel;
  kernel.func = reinterpret_cast<const void *>(&copy_bytes_kernel);
  const uint64_t units = (args.bytes + 15) / 16;
  uint64_t blocks = (units + 255) / 256;
  if (blocks > 2048) {
    blocks = 2048;
  }
  kernel.grid = dim3(static_cast<unsigned>(blocks), 1, 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

bool gather_supported(int64_t hidden) { return hidden > 0 && hidden % 8 == 0 && hidden <= kMaxGatherChunks * 512; }

KernelLaunch make_gather(const GatherArgs &args, int64_t capacity) {
  KernelLaunch kernel;
  const int64_t chunks_per_lane = (args.hidden / 8 + kWave - 1) / kWave;
  if (chunks_per_lane <= 1) {
    kernel.func = gather_kernel_for<1>(args.payload);
  } else if (chunks_per_lane <= 2) {
    kernel.func = gather_kernel_for<2>(args.payload);
  } else if (chunks_per_lane <= 4) {
    kernel.func = gather_kernel_for<4>(args.payload);
  } else if (chunks_per_lane <= 8) {
    kernel.func = gather_kernel_for<8>(args.payload);
  } else if (chunks_per_lane <= 16) {
    kernel.func = gather_kernel_for<16>(args.payload);
  } else {
    kernel.func = gather_kernel_for<32>(args.payload);
  }
  kernel.grid = dim3(static_cast<unsigned>((capacity + 3) / 4), 1, 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

KernelLaunch make_scatter(const ScatterArgs &args, int64_t capacity) {
  KernelLaunch kernel;
  kernel.func = reinterpret_cast<const void *>(&scatter_rows_kernel);
  kernel.grid = dim3(static_cast<unsigned>((capacity + 3) / 4), 1, 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

KernelLaunch make_reduce_partials(const ReduceArgs &args) {
  KernelLaunch kernel;
  constexpr uint64_t kLastLevelCacheBytes = 256ull << 20;
  const bool streaming = (static_cast<uint64_t>(args.count) + 1) * args.vectors * 16 > kLastLevelCacheBytes;
  kernel.func = streaming ? reinterpret_cast<const void *>(&reduce_partials_kernel<true>)
                          : reinterpret_cast<const void *>(&reduce_partials_kernel<false>);
  uint64_t blocks = (args.vectors + 255) / 256;
  if (blocks > 4096) {
    blocks = 4096;
  }
  kernel.grid = dim3(static_cast<unsigned>(blocks), 1, 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

}  // namespace xp
