// Hardware ceilings of the MI355X that the kernel design is measured against, launched by
// `bench.py --ceilings` (a separate library, libxpool_probes.so: none of this is on the
// FfnAgent path).
//
//  * probe_mfma: every wave issues rounds of 8 independent v_mfma_f32_32x32x16_bf16 on
//    register operands, no memory traffic: the sustained bf16 matrix rate of the chip at the
//    clock it holds under that load.  Two operand kinds: low-entropy constants (multiples
//    of 1/16, one A and one B fragment for every MFMA), and random bf16 values of GEMM-like
//    magnitude rotated over four A and four B fragments so that every MFMA's operands
//    differ from the previous one's, as in a GEMM's main loop.  The multipliers' switching
//    power, and with it the clock the chip can hold, depends on the operands.  Workgroup 0's
//    first wave records shader cycles (s_memtime) and 100 MHz ticks (s_memrealtime) over
//    its loop, from which the host reads the clock.
//  * probe_read_contiguous: a grid-stride read of a buffer, each wave instruction 1 KB of
//    consecutive bytes, UNROLL loads in flight per lane: the HBM read rate of the plainest
//    streaming pattern, with plain loads or with the nontemporal hint (`nt`), which the
//    tile kernels use for weights they read once.
//  * probe_read_rows: weight-streaming patterns of the decode projection kernels: a wave
//    owns 16 rows of a row-major matrix and reads 16 rows x 64 contiguous bytes (half
//    lines) or 8 rows x 128 bytes (whole lines) per instruction, 16 KB per wave in flight;
//    grid y splits each row into `ranges` contiguous parts (more workgroups for the same
//    bytes).
//  * probe_handoff: the cost of a grid-wide dependency.  `producers` workgroups each store
//    8 words; `consumers` workgroups then read all of them.  Three forms: two kernels back
//    to back (the stream orders them), or one launch in which the producers (the lower
//    workgroup ids, dispatched first, never waiting) publish with an agent-scope release
//    and an atomic increment, and the consumers wait for the count with a bounded, sleeping
//    poll and an agent-scope acquire; the count is one word, or one word per 8 producers on
//    lines of its own polled lane by lane.  Every consumer checks the words and sets `flag`
//    on a mismatch (1) or an expired wait (2).
//
// Each kernel folds what it reads (or computes) into registers and stores it only when
// `write` is set, which the host never does; the compiler cannot drop the work.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f32x16 = float __attribute__((ext_vector_type(16)));

constexpr int kMfmaChains = 8;

// A bf16 of magnitude 2^-3 .. 2^2 with random sign and mantissa from a hashed counter.
__device__ __forceinline__ __bf16 random_bf16(uint32_t seed) {
  uint32_t h = seed * 0x9e3779b9u;
  h ^= h >> 15;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  const uint32_t exponent = 124u + (h >> 24) % 6u;  // 2^-3 .. 2^2
  const uint32_t bits = ((h & 0x8000u) << 16) | (exponent << 23) | ((h & 0x7fu) << 16);
  return static_cast<__bf16>(__uint_as_float(bits));
}

template <bool RANDOM>
__global__ __launch_bounds__(256) void probe_mfma_kernel(int rounds, float *sink, int write, uint64_t *clocks) {
  constexpr int kSets = RANDOM ? 4 : 1;
  bf16x8 a[kSets];
  bf16x8 b[kSets];
#pragma unroll
  for (int s = 0; s < kSets; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (RANDOM) {
        const uint32_t id = (blockIdx.x * blockDim.x + threadIdx.x) * 64u + s * 8u + i;
        a[s][i] = random_bf16(2u * id);
        b[s][i] = random_bf16(2u * id + 1u);
      } else {
        a[s][i] = static_cast<__bf16>(static_cast<float>((threadIdx.x + i) & 7) * 0.125f);
        b[s][i] = static_cast<__bf16>(static_cast<float>((threadIdx.x * 3 + i) & 7) * 0.0625f);
      }
    }
  }
  f32x16 acc[kMfmaChains];
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc[c][r] = 0.0f;
    }
  }
  const uint64_t cycles0 = __builtin_readcyclecounter();
  const uint64_t ticks0 = __builtin_amdgcn_s_memrealtime();
  for (int round = 0; round < rounds; ++round) {
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c) {
      // RANDOM: chain c multiplies A set c % 4 by B set (c / 2) % 4, so consecutive MFMAs
      // never see the same operand pair.
      acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c % kSets], b[(c / 2) % kSets], acc[c], 0, 0, 0);
    }
  }
  if (clocks != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    // Reading the counters after the loop waits for nothing: the last MFMAs may still be in
    // the pipe, which is a few hundred cycles of a multi-millisecond loop.
    clocks[0] = __builtin_readcyclecounter() - cycles0;
    clocks[1] = __builtin_amdgcn_s_memrealtime() - ticks0;
  }
  if (write) {
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        total += acc[c][r];
      }
    }
    sink[blockIdx.x * blockDim.x + threadIdx.x] = total;
  }
}

template <int UNROLL, bool NONTEMPORAL>
__global__ __launch_bounds__(256) void probe_read_contiguous_kernel(const u32x4 *source, uint64_t vectors,
                                                                    uint32_t *sink, int write) {
  const uint64_t thread = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  u32x4 folded = {0u, 0u, 0u, 0u};
  for (uint64_t first = thread; first < vectors; first += stride * UNROLL) {
    u32x4 values[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint64_t index = first + u * stride;
      if constexpr (NONTEMPORAL) {
        values[u] = index < vectors ? __builtin_nontemporal_load(source + index) : u32x4{0u, 0u, 0u, 0u};
      } else {
        values[u] = index < vectors ? source[index] : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      folded ^= values[u];
    }
  }
  if (write) {
    sink[thread] = folded[0] ^ folded[1] ^ folded[2] ^ folded[3];
  }
}

// 8 waves per workgroup, wave w of workgroup x owns row block 8 x + w (16 rows); grid y is
// the part of each row (row_bytes / ranges bytes, a multiple of 1 KB).  LINES false: each
// instruction reads 16 rows x 64 contiguous bytes (the two halves of a 128-byte line in
// consecutive instructions).  LINES true: each instruction reads 8 rows x 128 bytes (lane
// l: row l & 7, 16-byte piece (l >> 4) + 4 ((l >> 3) & 1) of the line), whole lines.
template <bool LINES, bool NONTEMPORAL>
__global__ __launch_bounds__(512) void probe_read_rows_kernel(const char *matrix, int64_t rows, int64_t row_bytes,
                                                              int64_t part_bytes, uint32_t *sink, int write) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t block = static_cast<int64_t>(blockIdx.x) * 8 + wave;
  if (block * 16 >= rows) {
    return;
  }
  const int row_in_block = LINES ? (lane & 7) : (lane & 15);
  const int piece_bytes = LINES ? 16 * ((lane >> 4) + 4 * ((lane >> 3) & 1)) : 16 * (lane >> 4);
  const char *row = matrix + (block * 16 + row_in_block) * row_bytes + blockIdx.y * part_bytes + piece_bytes;
  u32x4 folded = {0u, 0u, 0u, 0u};
  for (int64_t column = 0; column < part_bytes; column += 1024) {
    u32x4 values[16];
#pragma unroll
    for (int chunk = 0; chunk < 4; ++chunk) {
#pragma unroll
      for (int piece = 0; piece < 4; ++piece) {
        // LINES: line 2 chunk + (piece >> 1) of rows 8 (piece & 1) + [0, 8).
        const int64_t offset = LINES ? (piece & 1) * 8 * row_bytes + chunk * 256 + (piece >> 1) * 128
                                     : chunk * 256 + piece * 64;
        const u32x4 *address = reinterpret_cast<const u32x4 *>(row + column + offset);
        if constexpr (NONTEMPORAL) {
          values[chunk * 4 + piece] = __builtin_nontemporal_load(address);
        } else {
          values[chunk * 4 + piece] = *address;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      folded ^= values[i];
    }
  }
  if (write) {
    sink[(blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x] = folded[0] ^ folded[1] ^ folded[2] ^ folded[3];
  }
}

__global__ __launch_bounds__(512) void probe_empty_kernel(uint32_t *sink) {
  if (blockIdx.x == 0x7fffffffu) {
    sink[0] = 1u;
  }
}

constexpr int kHandoffWords = 8;
constexpr int kHandoffSpinLimit = 1 << 22;  // polls of ~64 cycles each: ~0.1 s, then flag 2

__device__ __forceinline__ void handoff_produce(uint32_t *words, int producer, uint32_t salt) {
  if (threadIdx.x < kHandoffWords) {
    words[producer * kHandoffWords + threadIdx.x] = producer * kHandoffWords + threadIdx.x + salt;
  }
}

__device__ __forceinline__ void handoff_consume(const uint32_t *words, int producers, uint32_t salt,
                                                uint32_t *flag) {
  uint32_t bad = 0;
  for (int i = threadIdx.x; i < producers * kHandoffWords; i += blockDim.x) {
    bad |= words[i] != static_cast<uint32_t>(i) + salt ? 1u : 0u;
  }
  if (bad != 0) {
    atomicOr(flag, 1u);
  }
}

__global__ __launch_bounds__(512) void probe_produce_kernel(uint32_t *words, uint32_t salt) {
  handoff_produce(words, blockIdx.x, salt);
}

__global__ __launch_bounds__(512) void probe_consume_kernel(const uint32_t *words, int producers, uint32_t salt,
                                                            uint32_t *flag) {
  handoff_consume(words, producers, salt, flag);
}

// counters: SPREAD ? one word per 8 producers, 32 words (128 bytes) apart : one word.  Each
// counter grows by its producers' count per launch; `epoch` is the launch's 1-based number
// since the counters were zeroed.
template <bool SPREAD>
__global__ __launch_bounds__(512) void probe_handoff_kernel(uint32_t *words, int producers, uint32_t *counters,
                                                            uint32_t epoch, uint32_t salt, uint32_t *flag) {
  if (static_cast<int>(blockIdx.x) < producers) {
    handoff_produce(words, blockIdx.x, salt);
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_fetch_add(counters + (SPREAD ? (blockIdx.x / 8) * 32 : 0), 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  __shared__ int expired;
  if (threadIdx.x < 64) {
    const int groups = SPREAD ? (producers + 7) / 8 : 1;
    bool done = false;
    for (int spin = 0; spin < kHandoffSpinLimit; ++spin) {
      bool mine = true;
      for (int c = threadIdx.x; c < groups; c += 64) {
        const int members = SPREAD ? (producers - 8 * c < 8 ? producers - 8 * c : 8) : producers;
        mine = mine && __hip_atomic_load(counters + c * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
                           epoch * static_cast<uint32_t>(members);
      }
      done = __all(mine);
      if (done) {
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) {
      expired = done ? 0 : 1;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (expired != 0) {
    if (threadIdx.x == 0) {
      atomicOr(flag, 2u);
    }
    return;
  }
  handoff_consume(words, producers, salt, flag);
}

}  // namespace

extern "C" {

// rounds of 8 MFMAs per wave over `workgroups` 4-wave workgroups; operands low-entropy
// constants (random == 0) or rotating random bf16 values.  `clocks` (device, 2 words, may
// be NULL) receives the shader cycles and 100 MHz ticks of workgroup 0's loop.
int xp_probe_mfma(int workgroups, int rounds, int random, uint64_t *clocks, void *stream) {
  if (random != 0) {
    hipLaunchKernelGGL(probe_mfma_kernel<true>, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       rounds, static_cast<float *>(nullptr), 0, clocks);
  } else {
    hipLaunchKernelGGL(probe_mfma_kernel<false>, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       rounds, static_cast<float *>(nullptr), 0, clocks);
  }
  return static_cast<int>(hipGetLastError());
}

// Reads `bytes` (a multiple of 16) from `source` with `workgroups` 256-thread workgroups,
// with plain loads or (nontemporal != 0) with the nontemporal hint.
int xp_probe_read_contiguous(const void *source, uint64_t bytes, int workgroups, int nontemporal, void *stream) {
  if (nontemporal != 0) {
    hipLaunchKernelGGL((probe_read_contiguous_kernel<8, true>), dim3(workgroups), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const u32x4 *>(source), bytes / 16,
                       static_cast<uint32_t *>(nullptr), 0);
  } else {
    hipLaunchKernelGGL((probe_read_contiguous_kernel<8, false>), dim3(workgroups), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const u32x4 *>(source), bytes / 16,
                       static_cast<uint32_t *>(nullptr), 0);
  }
  return static_cast<int>(hipGetLastError());
}

// Reads a [rows, row_bytes] matrix (rows a multiple of 16, row_bytes a multiple of
// 1024 * ranges) in a weight-streaming pattern: 0 half lines, 1 whole lines, 2 whole lines
// with the nontemporal hint, 3 half lines with the nontemporal hint.
int xp_probe_read_rows(const void *matrix, int64_t rows, int64_t row_bytes, int ranges, int pattern, void *stream) {
  if (rows % 16 != 0 || ranges < 1 || row_bytes % (1024 * static_cast<int64_t>(ranges)) != 0 || pattern < 0 ||
      pattern > 3) {
    return -1;
  }
  const dim3 grid(static_cast<unsigned>((rows / 16 + 7) / 8), static_cast<unsigned>(ranges));
  auto kernel = pattern == 0   ? probe_read_rows_kernel<false, false>
                : pattern == 1 ? probe_read_rows_kernel<true, false>
                : pattern == 2 ? probe_read_rows_kernel<true, true>
                               : probe_read_rows_kernel<false, true>;
  hipLaunchKernelGGL(kernel, grid, dim3(512), 0, static_cast<hipStream_t>(stream), static_cast<const char *>(matrix),
                     rows, row_bytes, row_bytes / ranges, static_cast<uint32_t *>(nullptr), 0);
  return static_cast<int>(hipGetLastError());
}

// `workgroups` empty 512-thread workgroups.
int xp_probe_empty(int workgroups, void *stream) {
  hipLaunchKernelGGL(probe_empty_kernel, dim3(workgroups), dim3(512), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint32_t *>(nullptr));
  return static_cast<int>(hipGetLastError());
}

// One producer -> consumer handoff (mode 0 two kernels, 1 one launch with one counter, 2 one
// launch with a counter per 8 producers).  words: producers x 8 words; counters: zeroed
// before the first launch of a series, 32 x ceil(producers / 8) words (one in mode 1);
// epoch: the launch's 1-based number in its series; flag: one word, zeroed by the caller.
int xp_probe_handoff(int producers, int consumers, int mode, uint32_t *words, uint32_t *counters, uint32_t epoch,
                     uint32_t salt, uint32_t *flag, void *stream) {
  if (producers < 1 || consumers < 1 || mode < 0 || mode > 2) {
    return -1;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (mode == 0) {
    hipLaunchKernelGGL(probe_produce_kernel, dim3(producers), dim3(512), 0, s, words, salt);
    hipLaunchKernelGGL(probe_consume_kernel, dim3(consumers), dim3(512), 0, s, words, producers, salt, flag);
  } else {
    auto kernel = mode == 1 ? probe_handoff_kernel<false> : probe_handoff_kernel<true>;
    hipLaunchKernelGGL(kernel, dim3(producers + consumers), dim3(512), 0, s, words, producers, counters, epoch, salt,
                       flag);
  }
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
