// bf16 MFMA projections of the Dense FFN: gate_up (+ fused gated SiLU) and down.
//
// Reference behaviour (CrossPool checkout): Dense.run_into
// (src/xpool/runtime/ffnagent/operators/dense.py:70-86) runs Gemm.run_into
// (operators/linear.py:163-257) for i_proj with the fused epilogue of
// operators/activation.py:112-173 (projection rounded to the payload dtype,
// silu(gate) * up in fp32, stored as bf16), then for o_proj with no epilogue.
// Weights are [N, K] row-major with K contiguous; i_proj rows are interleaved
// Gate/Up (runtime/ffnagent/preparation.py:227).  Accumulation is fp32.
//
// Three kernel families, chosen per GraphTemplate capacity (choose_gemm):
//  * split (up to 8 rows, HBM-bound): weight rows are the MFMA M operand
//    (v_mfma_f32_16x16x32_bf16), read as whole 128-byte lines (8 rows x 128 bytes per load
//    instruction, nontemporal) with several 128-wide K chunks of loads in flight; the few
//    token rows are the N operand and come from L2 (or from LDS with the gather fused).  A
//    workgroup splits K across its waves and sums the ranges through LDS in a fixed order
//    (deterministic).  A Gate/Up pair lands in one lane's accumulator registers, so the
//    SiLU epilogue needs no data exchange.
//  * stream (up to 16 rows, HBM-bound): the same weight streaming with the token rows of
//    a K slice staged in LDS once per workgroup; sliced K goes through fp32 partial sums
//    and an ordered reduction kernel.
//  * tile (more rows: HBM-bound up to a few hundred, then MFMA-bound): BM x BN block
//    tiles from 64 x 128 to 256 x 256, BK = 64, 32x32x16 MFMA wave
//    tiles, direct global-to-LDS loads into a ring of stages with an XOR swizzle of
//    16-byte chunks (conflict-free ds_read_b128), and an optional K split across
//    workgroups (fp32 partials and the same ordered reduction) for grids smaller than
//    the chip.  For gate_up the weight tile is permuted while staging so that a wave's
//    Gate and Up columns for the same j sit in the same lane and register.

#include "xp_kernels.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <utility>

// Lambdas of the kernels below are forced inline: a lambda left out of line takes the
// accumulator array by reference, which then lives in scratch memory instead of registers.
#define XP_INLINE __attribute__((always_inline))

namespace xp {
namespace {

__device__ __forceinline__ uint16_t *output_row(const GemmArgs &a, int64_t token) {
  if (a.scatter_slots != nullptr) {
    const int32_t slot = a.scatter_slots[token];
    if (slot < 0 || static_cast<int64_t>(slot) >= a.out_rows) {
      return nullptr;
    }
    return a.out + static_cast<int64_t>(slot) * a.ldo;
  }
  return a.out + token * a.ldo;
}

// Offset that is always past a buffer resource's end (resources stay below 2^31 bytes, and
// adding a row's byte offset keeps it below 2^32).
constexpr uint32_t kOutOfRange = 0x7ffffff0u;

// Fused mailbox gather of token rows [0, TP) into LDS rows of stride `rs` (elements),
// columns [kbase, kbase + 8 vectors_per_row) of which the first kvalid hold data: token row
// t is mailbox row gather_slots[t] of a.x ([pool_rows, a.k]), RMS-normalised with a.norm when
// that is set, bit for bit as gather_rows_kernel computes it; rows past the live rows are
// zero and a slot outside the mailbox gives a row of quiet NaNs and raises the fault bit.
// Only rows [0, staged_rows) are written (the LDS holds no more; staged_rows <= TP covers
// the live rows).  All WAVES waves of the workgroup take part; the caller synchronises
// before reading.
template <int TP, int WAVES, class P = Bf16Payload>
__device__ __forceinline__ void stage_gathered_rows(const GemmArgs &a, uint16_t *xs, int64_t rs, int kbase,
                                                    int kvalid, int vectors_per_row, int wave, int lane,
                                                    int staged_rows) {
  const u32x4 zero = {0u, 0u, 0u, 0u};
  // Wave w finds rows w, w + WAVES, ... of the slot list and their inverse RMS over the
  // whole row (the gather kernel's wavefront reduction, so the same bits), then the columns
  // are staged from the mailbox rows, normalised.  Loads are issued in
  // batches of independent requests before their results are used, so the dependent
  // round trips are few (slot, row, and for rows longer than one batch the staging reads).
  constexpr int ROWS_PER_WAVE = TP / WAVES;
  constexpr int BATCH = 8;  // 16-byte chunks per lane and row in flight
  __shared__ float row_scale[TP];
  __shared__ int64_t row_source[TP];  // mailbox row; -1 past the live rows, -2 bad slot
  int64_t sources[ROWS_PER_WAVE];
#pragma unroll
  for (int r = 0; r < ROWS_PER_WAVE; ++r) {
    const int t = wave + r * WAVES;
    sources[r] = -1;
    if (t < a.rows) {
      const int32_t slot = a.gather_slots[t];
      sources[r] = slot < 0 || static_cast<int64_t>(slot) >= a.pool_rows ? -2 : slot;
    }
  }
  float squares[ROWS_PER_WAVE];
#pragma unroll
  for (int r = 0; r < ROWS_PER_WAVE; ++r) {
    squares[r] = 0.0f;
  }
  const int64_t row_chunks = a.k / 8;
  // Rows of at most BATCH * 64 chunks (hidden <= 4096) stay in registers between their sum
  // of squares and their normalised store into LDS: one round trip for the rows, none for
  // a second staging pass.  Longer rows are summed in batches and staged in a second pass.
  const bool one_batch = row_chunks <= BATCH * kWave;
  u32x4 values[ROWS_PER_WAVE][BATCH];
  u32x4 weights[BATCH];
  for (int64_t first = lane; first < row_chunks; first += BATCH * kWave) {
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int64_t chunk = first + b * kWave;
      weights[b] = one_batch && a.norm != nullptr && chunk < row_chunks ? load16(a.norm + chunk * 8) : zero;
#pragma unroll
      for (int r = 0; r < ROWS_PER_WAVE; ++r) {
        const bool live = sources[r] >= 0 && chunk < row_chunks && (one_batch || a.norm != nullptr);
        values[r][b] = live ? load16(a.x + sources[r] * a.ldx + chunk * 8) : zero;
      }
    }
    if (a.norm != nullptr) {
#pragma unroll
      for (int r = 0; r < ROWS_PER_WAVE; ++r) {
#pragma unroll
        for (int b = 0; b < BATCH; ++b) {
          add_squares<P>(values[r][b], squares[r]);  // chunk order lane, lane + 64, ...
        }
      }
    }
  }
  float scales[ROWS_PER_WAVE];
#pragma unroll
  for (int r = 0; r < ROWS_PER_WAVE; ++r) {
    const int t = wave + r * WAVES;
    scales[r] = a.norm != nullptr && sources[r] >= 0 ? rms_inverse(squares[r], a.k, a.eps) : 1.0f;
    if (lane == 0) {
      if (!one_batch) {
        row_scale[t] = scales[r];
        row_source[t] = sources[r];
      }
      if (sources[r] == -2 && blockIdx.x == 0) {
        raise_fault(a.fault, kFaultSlotOutOfRange);
      }
    }
  }
  const u32x4 poison = {P::kPoison2, P::kPoison2, P::kPoison2, P::kPoison2};
  if (one_batch) {
    // Each wave stores its own rows' part of the slice (zeros past the live rows).
#pragma unroll
    for (int r = 0; r < ROWS_PER_WAVE; ++r) {
      const int t = wave + r * WAVES;
      if (t >= staged_rows) {
        continue;
      }
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        const int64_t chunk = lane + b * kWave;
        const int64_t c = chunk - kbase / 8;  // chunk within this slice
        if (chunk >= row_chunks || c < 0 || c >= vectors_per_row) {
          continue;
        }
        u32x4 value = zero;
        if (sources[r] >= 0) {
          value = a.norm != nullptr ? normalize_chunk<P>(values[r][b], scales[r], weights[b]) : values[r][b];
        } else if (sources[r] == -2) {
          value = poison;
        }
        store16(xs + t * rs + c * 8, value);
      }
      // Slice columns past the row (the last slice's tail) are zero.
      for (int64_t c = row_chunks - kbase / 8 + lane; c < vectors_per_row; c += kWave) {
        if (c >= 0) {
          store16(xs + t * rs + c * 8, zero);
        }
      }
    }
  } else {
    __syncthreads();
    constexpr int STAGE_BATCH = 4;
    const int items = staged_rows * vectors_per_row;
    for (int first = threadIdx.x; first < items; first += STAGE_BATCH * 64 * WAVES) {
      u32x4 x_chunk[STAGE_BATCH];
      u32x4 w_chunk[STAGE_BATCH];
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int index = first + u * 64 * WAVES;
        const int t = index / vectors_per_row;
        const int c = index - t * vectors_per_row;
        const int64_t source = index < items ? row_source[t] : -1;
        const bool live = source >= 0 && c * 8 < kvalid;
        x_chunk[u] = live ? load16(a.x + source * a.ldx + kbase + c * 8) : zero;
        w_chunk[u] = live && a.norm != nullptr ? load16(a.norm + kbase + c * 8) : zero;
      }
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int index = first + u * 64 * WAVES;
        if (index >= items) {
          continue;
        }
        const int t = index / vectors_per_row;
        const int c = index - t * vectors_per_row;
        const int64_t source = row_source[t];
        u32x4 value = zero;
        if (c * 8 < kvalid) {
          if (source >= 0) {
            value = a.norm != nullptr ? normalize_chunk<P>(x_chunk[u], row_scale[t], w_chunk[u]) : x_chunk[u];
          } else if (source == -2) {
            value = poison;
          }
        }
        store16(xs + t * rs + c * 8, value);
      }
    }
  }
}

using lds_void_t = __attribute__((address_space(3))) void *;

// Direct global -> LDS load of 16 bytes per lane through a buffer resource: lane i's
// data lands at `lds_row_base + 16 i`; offsets past the resource's end write zeros.
template <int POLICY = 0>
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds_base, uint32_t voffset,
                                                  uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t)(lds_base), 16, static_cast<int>(voffset),
                                           static_cast<int>(soffset), 0, POLICY);
}

// s_waitcnt with vmcnt <= N and the LDS / export counters left unconstrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// ------------------------------------------------------------------ split (decode)
// Weight-streaming projection for at most 16 live rows (HBM-bound).  A workgroup of 8
// waves covers 8 / KSPLIT weight-row blocks of 16 rows; the KSPLIT waves of a block each
// stream one contiguous K range of `k_slice` columns, 128-wide K chunks with DEPTH chunks of
// loads in flight, multiplied on v_mfma_f32_16x16x32_bf16 with the weights as the M operand.
// The K ranges of a row block are summed through LDS in a fixed order (deterministic), all
// within the workgroup, so no partial sums leave the chip.
//
// Each weight load instruction reads whole 128-byte lines, 8 rows x 128 bytes, with the
// nontemporal hint (read once; measured on MI355X over Qwen3-8B gate_up: 6.4 TB/s, against
// 5.6 TB/s for 16 rows x 64 bytes per instruction, which the hint slows down).  Lane
// (i, q) = (lane & 15, lane >> 4) loads row i & 7 of the half, 16-byte piece p = 2 q + (i >> 3)
// of the line (K columns 8 p .. 8 p + 7).  As an MFMA operand, operand row i then holds the
// even pieces of weight row i (i < 8) or the odd pieces of weight row i - 8, and the token
// operand of token group g (tokens 8 g .. 8 g + 7) is laid out the same way: column j holds
// token 8 g + (j & 7) at piece 2 q + (j >> 3).  Products pair matching pieces only in the
// diagonal blocks, D[r][t] (even pieces) and D[r + 8][t + 8] (odd pieces) for r, t < 8,
// whose sum is the full dot product of weight row r with token 8 g + t; the off-diagonal
// blocks are discarded.  Half the MFMA work is thus wasted, which the decode sizes leave
// idle anyway (TG 16x16x32 per KB of weights).  Token pieces come from L2 (rows past the
// live rows cost no memory access).
constexpr int kSplitWaves = 8;
constexpr int kSplitGroupTokens = 8;
constexpr int kSplitMaxGroups = 2;

// GATHER (one token group, K <= 4096): the token rows are the mailbox rows gather_slots[t]
// of a.x, RMS-normalised with a.norm when that is set, staged once per workgroup into LDS
// (stage_gathered_rows, the gather kernel's bits) while the first DEPTH chunks of weights
// are in flight; the token pieces are then read from LDS instead of L2.  Dynamic LDS:
// min(capacity, 8) x (K + 16) bf16 (the 32-byte row padding puts the 16 pieces of one read
// in distinct bank slots).
template <int DEPTH, int TG, bool GATED, bool GATHER = false, class P = Bf16Payload>
__global__ __launch_bounds__(64 * kSplitWaves) void split_gemm_kernel(GemmArgs a) {
  static_assert(!GATHER || TG == 1, "the fused gather stages one token group");
  extern __shared__ __attribute__((aligned(16))) uint16_t staged[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int row = r16 & 7;                  // weight row within its half / token within its group
  const int piece = 2 * kq + (r16 >> 3);    // 16-byte piece of the 128-byte line
  const int ksplit = static_cast<int>(a.k_split);
  const int part = wave % ksplit;
  const int64_t rb = static_cast<int64_t>(blockIdx.x) * (kSplitWaves / ksplit) + wave / ksplit;
  const int64_t row_blocks = (a.n + 15) / 16;
  const bool active = rb < row_blocks;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  const int64_t rs = a.k + 16;  // staged row stride in elements (GATHER)
  // GATHER: rows staged in LDS, the capacity's: rows past them are zero.
  const int staged_rows = a.capacity < kSplitGroupTokens ? static_cast<int>(a.capacity) : kSplitGroupTokens;

  // acc[g][h]: token group g, weight rows 16 rb + 8 h + [0, 8).
  f32x4 acc[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    acc[g][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const int k0 = part * static_cast<int>(a.k_slice);
  // 128-wide chunks of this range (k_slice is a multiple of 128; the last range may be
  // shorter), rounded up to whole groups of DEPTH: the chunks past the range load through
  // an out-of-range offset, which reads zeros without a memory access.
  const int k_range = static_cast<int>(a.k - k0 < a.k_slice ? a.k - k0 : a.k_slice);
  const int chunks = (k_range + 127) / 128;  // >= 1: the host makes no empty range
  const int padded = (chunks + DEPTH - 1) / DEPTH * DEPTH;
  // Columns at or past K in the last chunk read the next row (or past the end): zero both
  // operands there.
  const int lane_valid = static_cast<int>(a.k) - k0 - piece * 8;
  // Row blocks start at different chunks of their range (stride-7 rotation), spreading the
  // concurrently streamed addresses over the memory channels.
  const int rotation = static_cast<int>((rb * 7) % chunks);
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w, static_cast<uint32_t>(a.n * a.k * 2));
  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(a.x, static_cast<uint32_t>(a.rows * a.ldx * 2));
  const uint32_t w_off = static_cast<uint32_t>(((rb * 16 + row) * a.k + k0 + piece * 8) * 2);
  const uint32_t w_half = static_cast<uint32_t>(8 * a.k * 2);  // rows 8 .. 15 of the block
  const uint32_t x_off = static_cast<uint32_t>((row * a.ldx + k0 + piece * 8) * 2);
  const uint32_t x_group = static_cast<uint32_t>(kSplitGroupTokens * a.ldx * 2);
  auto column_of = [&](int chunk) {
    const int c = chunk + rotation;
    return (c < chunks ? c : c - chunks) * 128;
  };

  // Per chunk: w[2 line + h] = line `line` (K columns 64 line .. 64 line + 63 of the chunk)
  // of rows 8 h + [0, 8); x[line][g] the matching pieces of token group g.
  constexpr int XG = GATHER ? 0 : TG;
  u32x4 wbuf[DEPTH][4];
  u32x4 xbuf[DEPTH][2][XG > 0 ? XG : 1];
  auto load_chunk = [&](int chunk, u32x4 (&w)[4], u32x4 (&x)[2][XG > 0 ? XG : 1]) {
    const bool in_range = chunk < chunks;
    const uint32_t column = static_cast<uint32_t>(column_of(chunk)) * 2;
#pragma unroll
    for (int line = 0; line < 2; ++line) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * line + h] = buffer_load16<kLoadNontemporal>(
            w_rsrc, in_range ? w_off + h * w_half + column + line * 128 : kOutOfRange);
      }
#pragma unroll
      for (int g = 0; g < XG; ++g) {
        x[line][g] = buffer_load16(x_rsrc, in_range ? x_off + g * x_group + column + line * 128 : kOutOfRange);
      }
    }
  };
  auto compute_chunk = [&](int chunk, const u32x4 (&w)[4], const u32x4 (&x)[2][XG > 0 ? XG : 1]) {
    const int column = chunk < chunks ? column_of(chunk) : 0;
#pragma unroll
    for (int line = 0; line < 2; ++line) {
      const bool valid = column + line * 64 < lane_valid;
      const u32x4 w0 = valid ? w[2 * line] : zero;
      const u32x4 w1 = valid ? w[2 * line + 1] : zero;
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        u32x4 xk;
        if constexpr (GATHER) {
          xk = valid && row < staged_rows ? load16(staged + row * rs + k0 + column + line * 64 + piece * 8) : zero;
        } else {
          xk = valid ? x[line][g] : zero;
        }
        acc[g][0] = P::mfma16(w0, xk, acc[g][0]);
        acc[g][1] = P::mfma16(w1, xk, acc[g][1]);
      }
    }
  };

  // Every load is unconditional and the trip count has no partial group, so the wait counts
  // track exactly DEPTH chunks in flight.
  if (active) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load_chunk(d, wbuf[d], xbuf[d]);
    }
  }
  if constexpr (GATHER) {
    const int vectors = static_cast<int>(a.k / 8);
    stage_gathered_rows<kSplitGroupTokens, kSplitWaves, P>(a, staged, rs, 0, static_cast<int>(a.k), vectors, wave,
                                                        lane, staged_rows);
    __syncthreads();
    if (a.gathered_out != nullptr && blockIdx.x == 0) {
      // The live rows' normalised bits for the stages after this projection.
      const int64_t live = a.rows < staged_rows ? a.rows : staged_rows;
      for (int64_t index = threadIdx.x; index < live * vectors; index += 64 * kSplitWaves) {
        const int64_t t = index / vectors;
        const int64_t c = index - t * vectors;
        store16(a.gathered_out + t * a.k + c * 8, load16(staged + t * rs + c * 8));
      }
    }
  }
  if (active) {
    int c0 = 0;
    for (; c0 < padded - DEPTH; c0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute_chunk(c0 + d, wbuf[d], xbuf[d]);
        load_chunk(c0 + d + DEPTH, wbuf[d], xbuf[d]);
        // Keep each refill right behind the chunk it replaces (DEPTH - 1 chunks stay in
        // flight) instead of letting the scheduler batch all refills at the loop end.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute_chunk(c0 + d, wbuf[d], xbuf[d]);
    }
  }

  // Fixed-order sum of the K ranges of each row block: range 0's wave adds ranges
  // 1 .. KSPLIT-1 in order.
  __shared__ f32x4 partial[kSplitWaves][TG][2][64];
  if (ksplit > 1) {
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      partial[wave][g][0][lane] = acc[g][0];
      partial[wave][g][1][lane] = acc[g][1];
    }
    __syncthreads();
    if (part != 0) {
      return;
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        for (int p = 1; p < ksplit; ++p) {
          acc[g][h] += partial[wave + p][g][h][lane];
        }
      }
    }
  }
  if (rb >= row_blocks) {
    return;
  }

  // Lane (i, q) holds D[4 q + v][i], v = 0 .. 3.  The lanes with q < 2 and i < 8 add the odd
  // pieces' block from lane + 40 (D[4 q + 8 + v][i + 8]) and then hold weight rows
  // 16 rb + 8 h + 4 q + v for token 8 g + i.
  f32x4 sum[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sum[g][h][v] = acc[g][h][v] + __shfl(acc[g][h][v], lane + 40, kWave);
      }
    }
  }
  if (kq >= 2 || r16 >= 8) {
    return;
  }
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int64_t token = kSplitGroupTokens * g + r16;
    if (token >= a.rows) {
      continue;
    }
    uint16_t *out = output_row(a, token);
    if (out == nullptr) {
      continue;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t n = rb * 16 + 8 * h + 4 * kq;
      if (n >= a.n) {
        continue;
      }
      if constexpr (GATED) {
        const float h0 = gated_silu_payload<P>(sum[g][h][0], sum[g][h][1], a.act);
        const float h1 = gated_silu_payload<P>(sum[g][h][2], sum[g][h][3], a.act);
        *reinterpret_cast<uint32_t *>(out + n / 2) = P::pack2(h0, h1);
      } else {
        u32x2 packed = {P::pack2(sum[g][h][0], sum[g][h][1]), P::pack2(sum[g][h][2], sum[g][h][3])};
        *reinterpret_cast<u32x2 *>(out + n) = packed;
      }
    }
  }
}

// The split kernel with the mailbox gather fused, for grids smaller than its unit count.
// A unit is the 8 / ksplit row blocks x ksplit K ranges one workgroup of the split kernel
// covers (wave w: row block unit * (8 / ksplit) + w / ksplit, K range w % ksplit);
// workgroup g takes units g, g + gridDim.x, ...  The token rows (one group of 8, K <=
// kSplitGatherMaxK) are gathered and RMS-normalised into LDS once per workgroup, so the
// gather costs one round trip per workgroup instead of one per unit, and one workgroup's
// K-range sum and stores overlap the other's weight stream.
//
// The gather runs under the first unit's weight stream: the first DEPTH weight chunks are
// requested first, then the slots, then the mailbox rows and the norm weights, which go
// straight into LDS (no registers beside the weight buffers, so two workgroups still fit
// on a CU).  Wave w then sums the squares of row w from LDS in the gather kernel's order
// (lane i over its chunks i, i + 64, ...; rms_inverse's wave reduction) and normalises the
// row in place, so the staged bits are gather_rows_kernel's.  The arithmetic per unit is
// split_gemm_kernel's (same chunk order, same fixed-order sum), so the results are bit for
// bit the split kernel's.
//
// Dynamic LDS: min(capacity, 8) rows of K + 16 bf16, then kSplitGatheredScratchBytes shared
// by the norm weights (while staging) and the K-range partial sums (after each unit).
constexpr int kSplitGatheredScratchBytes = (kSplitWaves - 1) * 2 * 64 * 16;

// The gated epilogue of the grouped MoE projections: SiLU exactly as the Dense kernels
// evaluate it (gated_silu_payload), or ReLU (NaN kept) / GELU (erf or tanh) of the rounded
// Gate, as compute_gated does (operators/activation.py:19-51), times the rounded Up plus
// the offset, with the same clipping.
template <class P, bool CLIP>
__device__ __forceinline__ float moe_gated_payload(float gate, float up, const GatedSilu &act) {
  if (act.function != kActivationRelu && act.function != kActivationGelu) {
    return gated_silu_payload<P, CLIP>(gate, up, act);
  }
  const uint32_t both = P::pack2(gate, up);
  float g = P::widen(both & 0xffffu);
  float u = P::widen(both >> 16);
  if constexpr (CLIP) {
    g = fminf(g, act.limit);
    u = fminf(fmaxf(u, -act.limit), act.limit);
  }
  float f;
  if (act.function == kActivationRelu) {
    f = (g > 0.0f || g != g) ? g : 0.0f;
  } else if (act.approximate_tanh != 0) {
    f = 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g)));
  } else {
    f = 0.5f * g * (1.0f + erff(g * 0.7071067811865476f));
  }
  return f * (u + act.up_offset);
}

template <class P>
__device__ __forceinline__ float moe_gated_payload(float gate, float up, const GatedSilu &act) {
  return act.limit > 0.0f ? moe_gated_payload<P, true>(gate, up, act) : moe_gated_payload<P, false>(gate, up, act);
}

template <int DEPTH, bool GATED, class P = Bf16Payload>
__global__ __launch_bounds__(64 * kSplitWaves) __attribute__((amdgpu_waves_per_eu(4))) void split_gathered_kernel(
    GemmArgs a) {
  static_assert(kSplitGroupTokens == kSplitWaves, "wave w stages token row w");
  extern __shared__ __attribute__((aligned(16))) uint16_t staged[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int row = r16 & 7;                // weight row within its half / token
  const int piece = 2 * kq + (r16 >> 3);  // 16-byte piece of the 128-byte line
  const int ksplit = static_cast<int>(a.k_split);
  const int part = wave % ksplit;
  const int block_in_unit = wave / ksplit;
  const int64_t per_unit = kSplitWaves / ksplit;
  const int64_t row_blocks = (a.n + 15) / 16;
  const int64_t units = (row_blocks + per_unit - 1) / per_unit;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  const int64_t rs = a.k + 16;  // staged row stride in elements
  const int staged_rows = a.capacity < kSplitGroupTokens ? static_cast<int>(a.capacity) : kSplitGroupTokens;
  uint16_t *scratch = staged + staged_rows * rs;  // norm weights, then partial sums
  f32x4(*partial)[2][64] = reinterpret_cast<f32x4(*)[2][64]>(scratch);
  const int k0 = part * static_cast<int>(a.k_slice);
  const int k_range = static_cast<int>(a.k - k0 < a.k_slice ? a.k - k0 : a.k_slice);
  const int chunks = (k_range + 127) / 128;
  const int padded = (chunks + DEPTH - 1) / DEPTH * DEPTH;
  const int lane_valid = static_cast<int>(a.k) - k0 - piece * 8;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w, static_cast<uint32_t>(a.n * a.k * 2));
  const uint32_t w_half = static_cast<uint32_t>(8 * a.k * 2);

  // The unit being worked on: its row block, whether this wave has one, its chunk rotation
  // and its weight offset.
  int64_t rb = 0;
  bool active = false;
  int rotation = 0;
  uint32_t w_off = 0;
  auto enter_unit = [&](int64_t unit) XP_INLINE {
    rb = unit * per_unit + block_in_unit;
    active = unit < units && rb < row_blocks;
    rotation = static_cast<int>((rb * 7) % chunks);
    w_off = static_cast<uint32_t>(((rb * 16 + row) * a.k + k0 + piece * 8) * 2);
  };
  auto column_of = [&](int chunk) XP_INLINE {
    const int c = chunk + rotation;
    return (c < chunks ? c : c - chunks) * 128;
  };
  u32x4 wbuf[DEPTH][4];
  auto load_chunk = [&](int chunk, u32x4 (&w)[4]) XP_INLINE {
    const bool in_range = chunk < chunks;
    const uint32_t column = static_cast<uint32_t>(column_of(chunk)) * 2;
#pragma unroll
    for (int line = 0; line < 2; ++line) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * line + h] = buffer_load16<kLoadNontemporal>(
            w_rsrc, in_range ? w_off + h * w_half + column + line * 128 : kOutOfRange);
      }
    }
  };

  // Wave w stages token row w: its mailbox row, -1 past the live rows, -2 for a slot outside
  // the mailbox.  The slot is read before the weight chunks are requested, so waiting for it
  // waits for nothing else.
  const int t = wave;
  int64_t source = -1;
  if (t < a.rows) {
    const int32_t slot = a.gather_slots[t];
    source = slot < 0 || static_cast<int64_t>(slot) >= a.pool_rows ? -2 : slot;
  }
  enter_unit(blockIdx.x);
  if (active) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load_chunk(d, wbuf[d]);
    }
  }

  // Gather (rows past the live rows are zero, a slot outside the mailbox gives a row of
  // quiet NaNs and raises the fault bit).
  {
    const int row_chunks = static_cast<int>(a.k / 8);  // <= 8 * 64
    uint16_t *token = staged + t * rs;
    if (source >= 0 && t < staged_rows) {
      const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(a.x, static_cast<uint32_t>(a.pool_rows * a.ldx * 2));
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        if (b * kWave < row_chunks && lane + b * kWave < row_chunks) {
          buffer_load_lds16(x_rsrc, token + b * kWave * 8,
                            static_cast<uint32_t>((source * a.ldx + (lane + b * kWave) * 8) * 2), 0u);
        }
      }
    }
    if (a.norm != nullptr && lane + wave * kWave < row_chunks) {
      const __amdgpu_buffer_rsrc_t n_rsrc = make_rsrc(a.norm, static_cast<uint32_t>(a.k * 2));
      buffer_load_lds16(n_rsrc, scratch + wave * kWave * 8, static_cast<uint32_t>((lane + wave * kWave) * 16), 0u);
    }
    wait_vmcnt<0>();  // the rows and norm weights (and the weight chunks issued before them)
    __syncthreads();
    if (t < staged_rows) {
      if (source >= 0) {
        if (a.norm != nullptr) {
          // Two LDS reads in flight at a time; chunks past the row read chunk 0 and count as
          // zeros (adding +0 to the non-negative sum leaves its bits unchanged).
          float squares = 0.0f;
#pragma unroll
          for (int pair = 0; pair < 4; ++pair) {
            u32x4 v[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int c = lane + (2 * pair + u) * kWave;
              v[u] = load16(token + (c < row_chunks ? c : 0) * 8);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              add_squares<P>(lane + (2 * pair + u) * kWave < row_chunks ? v[u] : zero, squares);
            }
          }
          const float scale = rms_inverse(squares, a.k, a.eps);
#pragma unroll
          for (int pair = 0; pair < 4; ++pair) {
            u32x4 v[2];
            u32x4 w[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int c = lane + (2 * pair + u) * kWave;
              v[u] = load16(token + (c < row_chunks ? c : 0) * 8);
              w[u] = load16(scratch + (c < row_chunks ? c : 0) * 8);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int c = lane + (2 * pair + u) * kWave;
              if (c < row_chunks) {
                store16(token + c * 8, normalize_chunk<P>(v[u], scale, w[u]));
              }
            }
          }
        }
      } else {
        const u32x4 poison = {P::kPoison2, P::kPoison2, P::kPoison2, P::kPoison2};
        const u32x4 fill = source == -2 ? poison : zero;
        for (int c = lane; c < row_chunks; c += kWave) {
          store16(token + c * 8, fill);
        }
      }
    }
    if (source == -2 && lane == 0 && blockIdx.x == 0) {
      raise_fault(a.fault, kFaultSlotOutOfRange);
    }
    __syncthreads();  // rows staged; the norm weights' space is free for the partial sums
  }
  const uint16_t *token_row = staged + row * rs + k0 + piece * 8;
  const bool token_live = row < staged_rows;

  for (int64_t unit = blockIdx.x; unit < units; unit += gridDim.x) {
    if (unit != blockIdx.x) {
      enter_unit(unit);
      if (active) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
          load_chunk(d, wbuf[d]);
        }
      }
    }
    f32x4 acc[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
    auto compute_chunk = [&](int chunk, const u32x4 (&w)[4]) XP_INLINE {
      const int column = chunk < chunks ? column_of(chunk) : 0;
#pragma unroll
      for (int line = 0; line < 2; ++line) {
        const bool valid = column + line * 64 < lane_valid;
        const u32x4 w0 = valid ? w[2 * line] : zero;
        const u32x4 w1 = valid ? w[2 * line + 1] : zero;
        const u32x4 xk = valid && token_live ? load16(token_row + column + line * 64) : zero;
        acc[0] = P::mfma16(w0, xk, acc[0]);
        acc[1] = P::mfma16(w1, xk, acc[1]);
      }
    };
    if (active) {
      int c0 = 0;
      for (; c0 < padded - DEPTH; c0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
          compute_chunk(c0 + d, wbuf[d]);
          load_chunk(c0 + d + DEPTH, wbuf[d]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute_chunk(c0 + d, wbuf[d]);
      }
    }
    // Fixed-order sum of the K ranges of each row block (range 0's wave adds 1 .. ksplit - 1
    // in order); the barriers wait for LDS only, nothing else is outstanding here.  Wave w
    // of range p > 0 writes slot w - w / ksplit - 1.
    if (ksplit > 1) {
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __asm__ volatile("s_barrier" ::: "memory");  // the previous unit's sums have been read
      if (part != 0) {
        partial[wave - block_in_unit - 1][0][lane] = acc[0];
        partial[wave - block_in_unit - 1][1][lane] = acc[1];
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __asm__ volatile("s_barrier" ::: "memory");
      if (part == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          for (int p = 1; p < ksplit; ++p) {
            acc[h] += partial[block_in_unit * (ksplit - 1) + p - 1][h][lane];
          }
        }
      }
    }
    if (part == 0 && active) {
      // As in split_gemm_kernel: lanes (i < 8, q < 2) add the odd pieces' block from lane + 40
      // and hold weight rows 16 rb + 8 h + 4 q + v for token i.
      f32x4 sum[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          sum[h][v] = acc[h][v] + __shfl(acc[h][v], lane + 40, kWave);
        }
      }
      uint16_t *out = kq < 2 && r16 < 8 && r16 < a.rows ? output_row(a, r16) : nullptr;
      if (out != nullptr) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t n = rb * 16 + 8 * h + 4 * kq;
          if (n >= a.n) {
            continue;
          }
          if constexpr (GATED) {
            const float h0 = gated_silu_payload<P>(sum[h][0], sum[h][1], a.act);
            const float h1 = gated_silu_payload<P>(sum[h][2], sum[h][3], a.act);
            *reinterpret_cast<uint32_t *>(out + n / 2) = P::pack2(h0, h1);
          } else {
            u32x2 packed = {P::pack2(sum[h][0], sum[h][1]), P::pack2(sum[h][2], sum[h][3])};
            *reinterpret_cast<u32x2 *>(out + n) = packed;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ grouped split (MoE decode)
// The split kernel over an expert tile table, for few routes per expert.  Grid y is entry y
// of the table: up to 16 sorted positions of one expert e (GemmArgs describes the table);
// grid x covers e's 16-row weight blocks and their K ranges as in split_gemm_kernel, and
// the weights are read and multiplied the same way: whole 128-byte lines, 8 rows x 128
// bytes per instruction with the nontemporal hint, on v_mfma_f32_16x16x32_bf16 with the
// even / odd piece pairing, here over two groups of 8 routes (route 8 g + i of the tile at
// sorted position p = tile_row0[y] + 8 g + i, live while p < expert_end[e]).  The token
// operand of route p is row gather_slots[p] / gather_divisor of x when gather_slots is set,
// else row p.  The result goes to row p of out, or to row scatter_slots[p] when that is
// set, times row_scale[p] when that is set.  A wave's chunk count is rounded up to whole
// groups of DEPTH; the chunks past its range load through an out-of-range offset, which
// reads zeros without a memory access.
template <int DEPTH, bool GATED, class P = Bf16Payload>
__global__ __launch_bounds__(64 * kSplitWaves) void grouped_split_kernel(GemmArgs a) {
  constexpr int TG = 2;  // groups of 8 routes
  // Both table words are loaded before the branch: the loads that follow depend on them,
  // and each dependent level costs a memory round trip before the weight stream starts.
  const int expert = __builtin_amdgcn_readfirstlane(a.tile_expert[blockIdx.y]);
  const int64_t m0 = __builtin_amdgcn_readfirstlane(a.tile_row0[blockIdx.y]);
  if (expert < 0) {
    return;  // uniform over the workgroup: no tile
  }
  const int64_t row_end = __builtin_amdgcn_readfirstlane(a.expert_end[expert]);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int row = r16 & 7;                // weight row within its half / route within its group
  const int piece = 2 * kq + (r16 >> 3);  // 16-byte piece of the 128-byte line
  const int ksplit = static_cast<int>(a.k_split);
  const int part = wave % ksplit;
  const int64_t rb = static_cast<int64_t>(blockIdx.x) * (kSplitWaves / ksplit) + wave / ksplit;
  const int64_t row_blocks = (a.n + 15) / 16;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // Route 8 g + row of the tile: its token row for the loads and, for the epilogue (whose
  // lanes r16 < 8 hold route 8 g + r16 = 8 g + row), its output row and factor, all loaded
  // before the stream starts.
  bool live[TG];
  int64_t x_row[TG];
  int64_t out_row[TG];
  float factor[TG];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int64_t position = m0 + 8 * g + row;
    live[g] = position < row_end;
    x_row[g] = position;
    if (a.gather_slots != nullptr) {
      x_row[g] = live[g] ? a.gather_slots[position] / a.gather_divisor : 0;
    }
    out_row[g] = position;
    if (a.scatter_slots != nullptr) {
      out_row[g] = live[g] ? a.scatter_slots[position] : -1;
    }
    factor[g] = live[g] && a.row_scale != nullptr ? a.row_scale[position] : 1.0f;
  }

  // acc[g][h]: route group g, weight rows 16 rb + 8 h + [0, 8).
  f32x4 acc[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    acc[g][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  if (rb < row_blocks) {
    const int k0 = part * static_cast<int>(a.k_slice);
    const int k_range = static_cast<int>(a.k - k0 < a.k_slice ? a.k - k0 : a.k_slice);
    const int chunks = (k_range + 127) / 128;  // >= 1: the host makes no empty range
    const int groups = (chunks + DEPTH - 1) / DEPTH;
    // Columns at or past K in the last chunk read the next row (or past the end): zero
    // both operands there.
    const int lane_valid = static_cast<int>(a.k) - k0 - piece * 8;
    const int rotation = static_cast<int>((rb * 7) % chunks);
    const uint16_t *weights = a.w + static_cast<int64_t>(expert) * a.n * a.k;
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(weights, static_cast<uint32_t>(a.n * a.k * 2));
    const __amdgpu_buffer_rsrc_t x_rsrc =
        make_rsrc(a.x, static_cast<uint32_t>((a.gather_slots != nullptr ? a.pool_rows : a.rows) * a.ldx * 2));
    const uint32_t w_off = static_cast<uint32_t>(((rb * 16 + row) * a.k + k0 + piece * 8) * 2);
    const uint32_t w_half = static_cast<uint32_t>(8 * a.k * 2);  // rows 8 .. 15 of the block
    uint32_t x_off[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      x_off[g] = static_cast<uint32_t>((x_row[g] * a.ldx + k0 + piece * 8) * 2);
    }
    auto column_of = [&](int chunk) XP_INLINE {
      const int c = chunk + rotation;
      return (c < chunks ? c : c - chunks) * 128;
    };

    // Per chunk: w[2 line + h] = line `line` (K columns 64 line .. 64 line + 63 of the
    // chunk) of rows 8 h + [0, 8); x[line][g] the matching pieces of route group g.
    u32x4 wbuf[DEPTH][4];
    u32x4 xbuf[DEPTH][2][TG];
    auto load_w = [&](int chunk, u32x4 (&w)[4]) XP_INLINE {
      const bool in_range = chunk < chunks;
      const uint32_t column = static_cast<uint32_t>(column_of(chunk)) * 2;
#pragma unroll
      for (int line = 0; line < 2; ++line) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          w[2 * line + h] = buffer_load16<kLoadNontemporal>(
              w_rsrc, in_range ? w_off + h * w_half + column + line * 128 : kOutOfRange);
        }
      }
    };
    auto load_x = [&](int chunk, u32x4 (&x)[2][TG]) XP_INLINE {
      const bool in_range = chunk < chunks;
      const uint32_t column = static_cast<uint32_t>(column_of(chunk)) * 2;
#pragma unroll
      for (int line = 0; line < 2; ++line) {
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          x[line][g] = buffer_load16(x_rsrc, in_range && live[g] ? x_off[g] + column + line * 128 : kOutOfRange);
        }
      }
    };
    auto compute_chunk = [&](int chunk, const u32x4 (&w)[4], const u32x4 (&x)[2][TG]) XP_INLINE {
      const int column = chunk < chunks ? column_of(chunk) : 0;
#pragma unroll
      for (int line = 0; line < 2; ++line) {
        const bool valid = column + line * 64 < lane_valid;
        const u32x4 w0 = valid ? w[2 * line] : zero;
        const u32x4 w1 = valid ? w[2 * line + 1] : zero;
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          const u32x4 xk = valid ? x[line][g] : zero;
          acc[g][0] = P::mfma16(w0, xk, acc[g][0]);
          acc[g][1] = P::mfma16(w1, xk, acc[g][1]);
        }
      }
    };

    // The weight loads of the first group go out before the token loads, whose offsets
    // wait on the gather slot loads.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load_w(d, wbuf[d]);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load_x(d, xbuf[d]);
    }
    for (int g = 1; g < groups; ++g) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int chunk = (g - 1) * DEPTH + d;
        compute_chunk(chunk, wbuf[d], xbuf[d]);
        load_w(chunk + DEPTH, wbuf[d]);
        load_x(chunk + DEPTH, xbuf[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute_chunk((groups - 1) * DEPTH + d, wbuf[d], xbuf[d]);
    }
  }

  // Fixed-order sum of the K ranges of each row block, as in split_gemm_kernel.
  __shared__ f32x4 partial[kSplitWaves][TG][2][64];
  if (ksplit > 1) {
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      partial[wave][g][0][lane] = acc[g][0];
      partial[wave][g][1][lane] = acc[g][1];
    }
    __syncthreads();
    if (part != 0) {
      return;
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        for (int p = 1; p < ksplit; ++p) {
          acc[g][h] += partial[wave + p][g][h][lane];
        }
      }
    }
  }

  // Lane (i, q) holds D[4 q + v][i], v = 0 .. 3.  The lanes with q < 2 and i < 8 add the odd
  // pieces' block from lane + 40 (D[4 q + 8 + v][i + 8]) and then hold weight rows
  // 16 rb + 8 h + 4 q + v for route 8 g + i.
  f32x4 sum[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sum[g][h][v] = acc[g][h][v] + __shfl(acc[g][h][v], lane + 40, kWave);
      }
    }
  }
  if (rb >= row_blocks || kq >= 2 || r16 >= 8) {
    return;
  }
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    if (!live[g] || out_row[g] < 0 || out_row[g] >= a.out_rows) {
      continue;
    }
    uint16_t *out = a.out + out_row[g] * a.ldo;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t n = rb * 16 + 8 * h + 4 * kq;
      if (n >= a.n) {
        continue;
      }
      f32x4 value = sum[g][h];
      if (a.bias != nullptr) {
        // Rows n .. n + 3 of the expert's bias (n + 3 < N: N is a multiple of 8).
        value += *reinterpret_cast<const f32x4 *>(a.bias + expert * a.bias_stride + n);
      }
      if constexpr (GATED) {
        const float h0 = moe_gated_payload<P>(value[0], value[1], a.act);
        const float h1 = moe_gated_payload<P>(value[2], value[3], a.act);
        *reinterpret_cast<uint32_t *>(out + n / 2) = P::pack2(h0, h1);
      } else {
        const float f = factor[g];
        u32x2 packed = {P::pack2(value[0] * f, value[1] * f), P::pack2(value[2] * f, value[3] * f)};
        *reinterpret_cast<u32x2 *>(out + n) = packed;
      }
    }
  }
}

// ------------------------------------------------------------------ stream (decode)
// Weight-streaming projection for up to 16 live rows.  Workgroup g works on K slice
// g / groups_per_slice: it stages the activations of that slice in LDS once, then each of
// its 8 waves streams one 16-row weight block of the slice with DEPTH 128-wide K chunks of
// loads in flight, multiplying on v_mfma_f32_16x16x32_bf16 with the weights as the M
// operand.  The weights are read as whole 128-byte lines with the nontemporal hint and the
// tokens as two groups of 8, with the even / odd piece pairing of the split kernel (see
// there): lane (i, q) loads row i & 7 of a half block, piece 2 q + (i >> 3) of the line,
// and reads token 8 g + (i & 7) at the same piece from LDS; the diagonal blocks of each
// MFMA are summed at the end.  LDS rows are padded by 32 bytes so that the 16 pieces one
// read touches fall in distinct bank slots.  With several slices the fp32 partial tiles go
// to scratch and stream_reduce_kernel, launched next on the same stream, finishes the
// projection.  (A last-arriver reduction inside this kernel would need an agent-scope
// release per wave, which writes back the XCD's whole L2 on this part and cost more than
// the stream itself.)
constexpr int kStreamWaves = 8;
constexpr int kStreamDepth = 4;
constexpr int kStreamTokens = 16;
constexpr int kStreamRowPad = 16;  // elements of LDS row padding

template <bool GATED, bool GATHER, class P = Bf16Payload>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_gemm_kernel(GemmArgs a) {
  constexpr int TP = kStreamTokens;
  constexpr int TG = TP / 8;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int row = r16 & 7;                // weight row within its half / token within its group
  const int piece = 2 * kq + (r16 >> 3);  // 16-byte piece of the 128-byte line
  const int64_t ks = a.k_slice;
  const int64_t slices = (a.k + ks - 1) / ks;
  const int64_t row_blocks = (a.n + 15) / 16;
  const int64_t groups_per_slice = (row_blocks + kStreamWaves - 1) / kStreamWaves;
  const int64_t slice = blockIdx.x / groups_per_slice;
  const int64_t rb = (blockIdx.x % groups_per_slice) * kStreamWaves + wave;
  const int64_t k0 = slice * ks;
  const int64_t klen = (a.k - k0) < ks ? (a.k - k0) : ks;
  const int64_t rs = ks + kStreamRowPad;  // LDS row stride in elements
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // Every slice runs ks / 128 chunks (a multiple of DEPTH, so the loop has no partial
  // group): weight loads go through a buffer resource over all N rows, rows past N read
  // as zero, and all loads are unconditional, which lets the wait counts track exactly
  // DEPTH chunks in flight.  Columns past K in the last slice are zeroed by a select.
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w, static_cast<uint32_t>(a.n * a.k * 2));
  const uint32_t w_off = static_cast<uint32_t>(((rb * 16 + row) * a.k + k0 + piece * 8) * 2);
  const uint32_t w_half = static_cast<uint32_t>(8 * a.k * 2);  // rows 8 .. 15 of the block
  const int chunks = static_cast<int>(ks / 128);
  const int lane_valid = static_cast<int>(klen) - piece * 8;
  // Waves start at different chunks of the slice (a stride-7 rotation by row block), so the
  // concurrently streamed addresses spread over the memory channels instead of every wave
  // reading the same column range of its rows at the same time.
  const int rotation = static_cast<int>((rb * 7) % chunks);
  auto rotated = [&](int chunk) { return chunk + rotation < chunks ? chunk + rotation : chunk + rotation - chunks; };

  // w[2 line + h]: line `line` of the chunk (K columns 64 line .. 64 line + 63), rows 8 h + [0, 8).
  u32x4 wbuf[kStreamDepth][4];
  auto load_chunk = [&](int chunk, u32x4 (&w)[4]) {
    const uint32_t column = static_cast<uint32_t>(rotated(chunk) * 128) * 2;
#pragma unroll
    for (int line = 0; line < 2; ++line) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * line + h] = buffer_load16<kLoadNontemporal>(w_rsrc, w_off + h * w_half + column + line * 128);
      }
    }
  };
  // The first DEPTH chunks of weights are requested before the activations are staged, so
  // their latency overlaps the staging (for the fused gather, several dependent round trips).
  if (rb < row_blocks) {
#pragma unroll
    for (int d = 0; d < kStreamDepth; ++d) {
      load_chunk(d, wbuf[d]);
    }
  }

  // Stage activations [0, TP) x [k0, k0 + ks) of this slice.  Rows past the live rows read
  // as zero; columns past K are zeroed explicitly.
  const int vectors_per_row = static_cast<int>(ks / 8);
  const int ldx = static_cast<int>(a.ldx);
  const int kbase = static_cast<int>(k0);
  const int kvalid = static_cast<int>(klen);
  if constexpr (GATHER) {
    stage_gathered_rows<TP, kStreamWaves, P>(a, xs, rs, kbase, kvalid, vectors_per_row, wave, lane, TP);
  } else {
    const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(a.x, static_cast<uint32_t>(a.rows * a.ldx * 2));
    for (int index = threadIdx.x; index < TP * vectors_per_row; index += 64 * kStreamWaves) {
      const int t = index / vectors_per_row;
      const int c = index - t * vectors_per_row;
      u32x4 value = buffer_load16(x_rsrc, static_cast<uint32_t>((t * ldx + kbase + c * 8) * 2));
      value = c * 8 < kvalid ? value : zero;
      store16(xs + t * rs + c * 8, value);
    }
  }
  __syncthreads();
  if (rb >= row_blocks) {
    return;
  }

  // acc[g][h]: token group g, weight rows 16 rb + 8 h + [0, 8).
  f32x4 acc[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    acc[g][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  auto compute_chunk = [&](int chunk, const u32x4 (&w)[4]) {
    const int column = rotated(chunk) * 128;
#pragma unroll
    for (int line = 0; line < 2; ++line) {
      const bool valid = column + line * 64 < lane_valid;
      const u32x4 w0 = valid ? w[2 * line] : zero;
      const u32x4 w1 = valid ? w[2 * line + 1] : zero;
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        const u32x4 x = load16(xs + (8 * g + row) * rs + column + line * 64 + piece * 8);
        acc[g][0] = P::mfma16(w0, x, acc[g][0]);
        acc[g][1] = P::mfma16(w1, x, acc[g][1]);
      }
    }
  };

  int c0 = 0;
  for (; c0 < chunks - kStreamDepth; c0 += kStreamDepth) {
#pragma unroll
    for (int d = 0; d < kStreamDepth; ++d) {
      compute_chunk(c0 + d, wbuf[d]);
      load_chunk(c0 + d + kStreamDepth, wbuf[d]);
      // Keep each refill right behind the chunk it replaces, so DEPTH - 1 chunks stay in
      // flight throughout instead of the scheduler batching all refills at the end.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < kStreamDepth; ++d) {
    compute_chunk(c0 + d, wbuf[d]);
  }

  // Lane (i, q) holds D[4 q + v][i]; the lanes with q < 2 and i < 8 add the odd pieces'
  // block from lane + 40 and then hold weight rows 16 rb + 8 h + 4 q + v for token 8 g + i.
  f32x4 sum[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sum[g][h][v] = acc[g][h][v] + __shfl(acc[g][h][v], lane + 40, kWave);
      }
    }
  }
  if (kq >= 2 || r16 >= 8) {
    return;
  }
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int64_t token = 8 * g + r16;
    if (token >= a.rows) {
      continue;
    }
    uint16_t *out = slices > 1 ? nullptr : output_row(a, token);
    if (slices == 1 && out == nullptr) {
      continue;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t n = rb * 16 + 8 * h + 4 * kq;
      if (n >= a.n) {
        continue;
      }
      if (slices > 1) {
        // Partial tile of this slice; stream_reduce_kernel sums the slices in order.
        *reinterpret_cast<f32x4 *>(a.partials + (slice * a.rows + token) * a.n + n) = sum[g][h];
      } else if constexpr (GATED) {
        const float h0 = gated_silu_payload<P>(sum[g][h][0], sum[g][h][1], a.act);
        const float h1 = gated_silu_payload<P>(sum[g][h][2], sum[g][h][3], a.act);
        *reinterpret_cast<uint32_t *>(out + n / 2) = P::pack2(h0, h1);
      } else {
        u32x2 packed = {P::pack2(sum[g][h][0], sum[g][h][1]), P::pack2(sum[g][h][2], sum[g][h][3])};
        *reinterpret_cast<u32x2 *>(out + n) = packed;
      }
    }
  }
}

// Sum of the split-K partials [slices, rows, n] in slice order (so results do not depend
// on which slice finished first), then the projection's epilogue.  One thread per four
// consecutive outputs of one row: 16-byte partial loads, coalesced along n.
template <bool GATED, class P = Bf16Payload>
__global__ __launch_bounds__(256) void stream_reduce_kernel(GemmArgs a) {
  const int64_t quads = a.n / 4;
  const int64_t index = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t token = index / quads;
  if (token >= a.rows) {
    return;
  }
  const int64_t n = (index - token * quads) * 4;
  const int64_t slices = (a.k + a.k_slice - 1) / a.k_slice;
  const int64_t plane = a.rows * a.n;
  const float *source = a.partials + token * a.n + n;
  auto partial = [&](int64_t slice) { return *reinterpret_cast<const f32x4 *>(source + slice * plane); };
  // Loads issued four slices at a time; the additions keep slice order.
  f32x4 sum = partial(0);
  int64_t slice = 1;
  for (; slice + 4 <= slices; slice += 4) {
    const f32x4 p0 = partial(slice), p1 = partial(slice + 1), p2 = partial(slice + 2), p3 = partial(slice + 3);
    sum += p0;
    sum += p1;
    sum += p2;
    sum += p3;
  }
  for (; slice < slices; ++slice) {
    sum += partial(slice);
  }
  uint16_t *row = output_row(a, token);
  if (row == nullptr) {
    return;
  }
  if constexpr (GATED) {
    const float h0 = gated_silu_payload<P>(sum[0], sum[1], a.act);
    const float h1 = gated_silu_payload<P>(sum[2], sum[3], a.act);
    *reinterpret_cast<uint32_t *>(row + n / 2) = P::pack2(h0, h1);
  } else {
    u32x2 packed = {P::pack2(sum[0], sum[1]), P::pack2(sum[2], sum[3])};
    *reinterpret_cast<u32x2 *>(row + n) = packed;
  }
}

// ------------------------------------------------------------------ resident (decode, 9-32 rows)
// Weight streaming for 9 to 32 live rows with the token rows resident in registers.  One
// workgroup of 8 waves per CU (256 VGPRs per wave, two waves per SIMD).  The K columns of a
// workgroup's part (k_slice = 8 CPW 128 columns; k_split parts over the grid) are split over
// its 8 waves, CPW 128-wide chunks each, and every wave loads the token rows' pieces of its
// own chunks once, in the split kernel's MFMA operand layout (token 8 g + i of group g at
// piece 2 q + (i >> 3) of each 64-column line), so the main loop reads no token data at all:
// past the prologue every load of the kernel is a weight load.
//
// Workgroup (part p, walker r) walks the 16-row weight blocks r, r + R, ... (R walkers per
// part).  For each block the 8 waves stream their chunks (whole 128-byte lines, nontemporal,
// the split kernel's even / odd piece pairing on v_mfma_f32_16x16x32_bf16), then sum their
// K ranges through LDS in wave order, i.e. in K order (deterministic), and the block's
// outputs are stored: activated bf16 for gate_up, bf16 (scattered by slot) for down, or,
// with several parts, fp32 partials [part, rows, n] that stream_reduce_kernel adds in part
// order.  The weight loads run a ring of chunks ahead across block boundaries: one
// workgroup per CU leaves no other workgroup to stream while a block is summed, so the stream
// must not stop there.
//
// GATHER (gate_up of a Dense step, one part): token row t is mailbox row gather_slots[t],
// RMS-normalised with a.norm.  Each wave sums the squares of its pieces of every row (lane
// order: chunk, then line), the 8 lanes holding a row's pieces add theirs by a butterfly, and
// the 8 waves' sums are added in the fixed tree ((w0 + w1) + (w2 + w3)) + ((w4 + w5) + (w6 +
// w7)) through LDS; the scale is 1 / sqrt(sum / K + eps) and each element becomes
// bf16((x * scale) * w), as in the gather kernel (whose sum of squares runs in another
// order, so the two agree within one bf16 ulp rather than bit for bit).  Rows past the live
// rows are zero; a slot outside the mailbox gives a row of quiet NaNs and raises the fault
// bit.  With gathered_out set, workgroup t stores normalised row t there.
constexpr int kResidentWaves = 8;
constexpr int kResidentWorkgroups = 256;  // one per CU
constexpr int kResidentChunk = 128;       // columns per chunk

// Weight chunks in flight per wave: 4 with two token groups (measured on MI355X for
// Qwen3-8B gate_up at 16 rows: 8 chunks were no faster than 4); 2 with four, whose token
// pieces take 128 registers per lane (at 4 in flight the kernel spilled; at 2 it takes 240
// VGPRs and none spill).  And the greatest common divisor for the loop's rounds.
constexpr int resident_depth(int groups) { return groups >= 4 ? 2 : 4; }
constexpr int gcd_int(int a, int b) { return b == 0 ? a : gcd_int(b, a % b); }

template <int TG>
struct ResidentLds {
  float row_squares[kResidentWaves][8 * TG];
  // Two buffers of block sums (alternating blocks): wave, token group, half, kq, token.
  f32x4 block[2][kResidentWaves][TG][2][2][8];
};

template <int TG, int CPW, bool GATED, bool GATHER, class P = Bf16Payload>
__global__ __launch_bounds__(64 * kResidentWaves) __attribute__((amdgpu_waves_per_eu(2))) void resident_gemm_kernel(
    GemmArgs a) {
  constexpr int D = resident_depth(TG);
  constexpr int L = D / gcd_int(D, CPW) * CPW;  // chunks per round of the loop: whole blocks and whole rings
  constexpr int TP = 8 * TG;
  __shared__ ResidentLds<TG> lds;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int row = r16 & 7;                // weight row within its half / token within its group
  const int piece = 2 * kq + (r16 >> 3);  // 16-byte piece of the 128-byte line
  const int parts = static_cast<int>(a.k_split);
  const int part = static_cast<int>(blockIdx.x) % parts;
  const int walkers = static_cast<int>(gridDim.x) / parts;
  const int walker = static_cast<int>(blockIdx.x) / parts;
  const int64_t row_blocks = (a.n + 15) / 16;
  const int units = walker < row_blocks ? static_cast<int>((row_blocks - 1 - walker) / walkers) + 1 : 0;
  const int64_t k0 = static_cast<int64_t>(part * kResidentWaves + wave) * CPW * kResidentChunk;
  // Columns [k0 + 128 c + 64 l + 8 piece, + 8) of this lane hold data iff 128 c + 64 l < lane_valid.
  const int64_t lane_valid = a.k - k0 - piece * 8;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  auto chunk_column = [](int c) XP_INLINE { return c * kResidentChunk; };

  // Weight chunk c of this wave's part of row block `unit`: w[2 l + h] = line l of rows
  // 16 rb + 8 h + [0, 8).  Each block is addressed through a buffer resource of its own
  // (wave-uniform, in scalar registers) whose size ends at the block's last row, so the
  // per-lane offsets are two constants (one per half) plus immediates, and rows past N,
  // chunks past K and blocks past the walker's read zeros without a memory access.
  const uint32_t lane_offset[2] = {static_cast<uint32_t>((row * a.k + k0 + piece * 8) * 2),
                                   static_cast<uint32_t>(((row + 8) * a.k + k0 + piece * 8) * 2)};
  auto load_chunk = [&](int unit, int c, u32x4 (&w)[4]) XP_INLINE {
    const int64_t rb = walker + static_cast<int64_t>(unit) * walkers;
    const int64_t block_rows = unit < units ? std::min<int64_t>(16, a.n - rb * 16) : 0;
    const __amdgpu_buffer_rsrc_t rsrc =
        make_rsrc(a.w + (unit < units ? rb * 16 * a.k : 0), static_cast<uint32_t>(block_rows * a.k * 2));
#pragma unroll
    for (int l = 0; l < 2; ++l) {
      const bool valid = chunk_column(c) + l * 64 < lane_valid;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * l + h] = buffer_load16<kLoadNontemporal>(
            rsrc, valid ? lane_offset[h] + static_cast<uint32_t>((chunk_column(c) + l * 64) * 2) : kOutOfRange);
      }
    }
  };

  // GATHER: mailbox row of token 8 g + row (-1 past the live rows, -2 for a slot outside the
  // mailbox); read before the weights are requested, so waiting for it waits for nothing else.
  int source[TG];
  int mine = -1;
  if constexpr (GATHER) {
    if (lane < TP && lane < a.rows) {
      const int32_t slot = a.gather_slots[lane];
      mine = slot < 0 || static_cast<int64_t>(slot) >= a.pool_rows ? -2 : slot;
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      source[g] = __shfl(mine, 8 * g + row, kWave);
    }
  } else {
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      source[g] = 8 * g + row;  // activation row
    }
  }

  // Token pieces of this wave's chunks: x[c][l][g] = token 8 g + row, columns k0 + 128 c +
  // 64 l + 8 piece.
  // The token pieces (and the norm weights) are requested before the weight ring, so the
  // gather's normalisation runs while the ring is in flight: the wait counts are in order,
  // and waiting for anything issued after the ring would wait for the ring as well.
  u32x4 x[CPW][2][TG];
  // GATHER: the norm weights go straight into LDS (the block buffers, unused until the first
  // block ends; K <= 8 CPW 128 columns fit them), so they take no registers.
  static_assert(sizeof(lds.block) >= kResidentWaves * CPW * kResidentChunk * 2, "the norm weights fit the block buffers");
  uint16_t *norm_lds = reinterpret_cast<uint16_t *>(&lds.block[0][0][0][0][0][0]);
  if constexpr (GATHER) {
    if (a.norm != nullptr) {
      const __amdgpu_buffer_rsrc_t n_rsrc = make_rsrc(a.norm, static_cast<uint32_t>(a.k * 2));
      for (int v = wave * kWave; v < (a.k + 7) / 8; v += kResidentWaves * kWave) {
        buffer_load_lds16(n_rsrc, norm_lds + v * 8, static_cast<uint32_t>((v + lane) * 16), 0u);
      }
    }
  }
  {
    // GATHER: mailbox rows by slot; otherwise activations [rows, k] (row stride ldx), rows past
    // the live rows reading as zero.
    const __amdgpu_buffer_rsrc_t x_rsrc =
        make_rsrc(a.x, static_cast<uint32_t>((GATHER ? a.pool_rows : a.rows) * a.ldx * 2));
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int l = 0; l < 2; ++l) {
        const bool valid = chunk_column(c) + l * 64 < lane_valid;
        const uint32_t column = static_cast<uint32_t>((k0 + piece * 8 + chunk_column(c) + l * 64) * 2);
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          const int64_t token_row = source[g];
          x[c][l][g] = buffer_load16(x_rsrc, valid && token_row >= 0
                                                 ? static_cast<uint32_t>(token_row * a.ldx * 2) + column
                                                 : kOutOfRange);  // (the pool is below 2 GiB)
        }
      }
    }
  }
  u32x4 wbuf[D][4];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    load_chunk(j / CPW, j % CPW, wbuf[j]);
  }

  if constexpr (GATHER) {
    wait_vmcnt<4 * D>();  // the token pieces and the norm weights; the ring stays in flight
    float scale[TG];
    if (a.norm != nullptr) {
      float squares[TG];
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        squares[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
#pragma unroll
          for (int l = 0; l < 2; ++l) {
            add_squares<P>(x[c][l][g], squares[g]);  // column order within the lane
          }
        }
        // The 8 lanes of token row (lane & 7) differ in lane bits 3 .. 5.
        squares[g] += __shfl_xor(squares[g], 8, kWave);
        squares[g] += __shfl_xor(squares[g], 16, kWave);
        squares[g] += __shfl_xor(squares[g], 32, kWave);
        if (lane < 8) {
          lds.row_squares[wave][8 * g + lane] = squares[g];
        }
      }
      __syncthreads();  // every wave's row sums and norm weights are in LDS
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        const float(*s)[TP] = lds.row_squares;
        const int t = 8 * g + row;
        const float total = ((s[0][t] + s[1][t]) + (s[2][t] + s[3][t])) + ((s[4][t] + s[5][t]) + (s[6][t] + s[7][t]));
        scale[g] = 1.0f / sqrtf(total / static_cast<float>(a.k) + a.eps);
      }
    }
    const u32x4 poison = {P::kPoison2, P::kPoison2, P::kPoison2, P::kPoison2};
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int l = 0; l < 2; ++l) {
        const bool valid = chunk_column(c) + l * 64 < lane_valid;
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          if (source[g] == -2) {
            x[c][l][g] = valid ? poison : zero;
          } else if (a.norm != nullptr) {
            const u32x4 weight = valid ? load16(norm_lds + k0 + piece * 8 + chunk_column(c) + l * 64) : zero;
            x[c][l][g] = normalize_chunk<P>(x[c][l][g], scale[g], weight);
          }
        }
      }
    }
    __syncthreads();  // every wave has read the norm weights before the block buffers are reused
    // Lane t < TP holds slot t's class (mine); one lane of workgroup 0 raises the fault bit.
    const bool any_bad = __ballot(mine == -2) != 0;
    if (blockIdx.x == 0 && wave == 0 && lane == 0 && any_bad) {
      raise_fault(a.fault, kFaultSlotOutOfRange);
    }
    if (a.gathered_out != nullptr && blockIdx.x < a.rows && static_cast<int>(blockIdx.x) < TP &&
        row == static_cast<int>(blockIdx.x % 8)) {
      // Workgroup t stores normalised row t (the lanes holding its pieces, every wave).
      const int g = static_cast<int>(blockIdx.x / 8);
#pragma unroll
      for (int gg = 0; gg < TG; ++gg) {
        if (gg != g) {
          continue;
        }
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
#pragma unroll
          for (int l = 0; l < 2; ++l) {
            if (chunk_column(c) + l * 64 < lane_valid) {
              store16(a.gathered_out + blockIdx.x * a.k + k0 + piece * 8 + chunk_column(c) + l * 64, x[c][l][gg]);
            }
          }
        }
      }
    }
  }

  f32x4 acc[TG][2];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    acc[g][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  auto compute_chunk = [&](int c, const u32x4 (&w)[4]) XP_INLINE {
#pragma unroll
    for (int l = 0; l < 2; ++l) {
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        acc[g][0] = P::mfma16(w[2 * l], x[c][l][g], acc[g][0]);
        acc[g][1] = P::mfma16(w[2 * l + 1], x[c][l][g], acc[g][1]);
      }
    }
  };

  // Block sums.  At the end of a block each wave's lanes (i < 8, q < 2) add the odd pieces'
  // block from lane + 40, which leaves weight rows 16 rb + 8 h + 4 q + v for token 8 g + i,
  // and store them to the block's LDS buffer; one chunk into the next block, behind a
  // barrier, 32 TG lanes (16 per wave) add the 8 waves' values in wave order and store the
  // outputs.  The weight loads in flight meanwhile keep the stream going.
  auto store_block = [&](int unit) XP_INLINE {
    f32x4(*block)[TG][2][2][8] = lds.block[unit & 1];
#pragma unroll
    for (int g = 0; g < TG; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          acc[g][h][v] += __shfl(acc[g][h][v], lane + 40, kWave);
        }
        if (kq < 2 && r16 < 8) {
          block[wave][g][h][kq][r16] = acc[g][h];
        }
        acc[g][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  };
  // The reducing lane's item (g, h, q, i) and its output row, looked up once: a dependent
  // load of the scatter slot inside the loop would wait for every weight load before it.
  const int item = wave * 16 + r16;
  const bool reducer = lane < 16 && item < 32 * TG;
  const int item_i = item & 7;
  const int item_q = (item >> 3) & 1;
  const int item_h = (item >> 4) & 1;
  const int item_g = item >> 5;
  const int64_t item_token = 8 * item_g + item_i;
  uint16_t *item_out = reducer && parts == 1 && item_token < a.rows ? output_row(a, item_token) : nullptr;
  auto reduce_block = [&](int unit) XP_INLINE {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __asm__ volatile("s_barrier" ::: "memory");
    if (!reducer) {
      return;
    }
    f32x4(*block)[TG][2][2][8] = lds.block[unit & 1];
    f32x4 sum = block[0][item_g][item_h][item_q][item_i];
#pragma unroll
    for (int w = 1; w < kResidentWaves; ++w) {
      sum += block[w][item_g][item_h][item_q][item_i];
    }
    const int64_t rb = walker + static_cast<int64_t>(unit) * walkers;
    const int64_t n = rb * 16 + 8 * item_h + 4 * item_q;
    if (item_token >= a.rows || n >= a.n) {
      return;
    }
    if (parts > 1) {
      *reinterpret_cast<f32x4 *>(a.partials + (part * a.rows + item_token) * a.n + n) = sum;
    } else if (item_out != nullptr) {
      if constexpr (GATED) {
        const float h0 = gated_silu_payload<P>(sum[0], sum[1], a.act);
        const float h1 = gated_silu_payload<P>(sum[2], sum[3], a.act);
        *reinterpret_cast<uint32_t *>(item_out + n / 2) = P::pack2(h0, h1);
      } else {
        u32x2 packed = {P::pack2(sum[0], sum[1]), P::pack2(sum[2], sum[3])};
        *reinterpret_cast<u32x2 *>(item_out + n) = packed;
      }
    }
  };

  // The wave's chunk stream: chunk f is chunk f % CPW of block f / CPW; ring slot f % D.  The
  // loop runs whole rounds of D chunks (a multiple of CPW); chunks past the last block read
  // zeros without a memory access, so every load is unconditional and the wait counts track
  // the chunks in flight exactly.  The block count is workgroup-uniform, so every wave
  // reaches every barrier.
  const int rounds = (units * CPW + L - 1) / L;
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int unit = r * (L / CPW) + j / CPW;
      const int c = j % CPW;
      compute_chunk(c, wbuf[j % D]);
      load_chunk(r * (L / CPW) + (j + D) / CPW, (j + D) % CPW, wbuf[j % D]);
      __builtin_amdgcn_sched_barrier(0);
      if (c == 0 && unit >= 1 && unit <= units) {
        reduce_block(unit - 1);
      }
      if (c == CPW - 1 && unit < units) {
        store_block(unit);
      }
    }
  }
  if (units > 0 && rounds * (L / CPW) == units) {
    reduce_block(units - 1);  // the last block had no next block to reduce it in
  }
}

// ------------------------------------------------------------------ tile
// LDS tiles are rows of 64 bf16 (128 bytes = eight 16-byte chunks).  gfx950 serves
// ds_read_b128 sixteen lanes at a time from a 256-byte bank line, i.e. two tile rows, so
// the 16 rows one MFMA fragment read touches must occupy 16 distinct 16-byte slots:
// logical chunk c of row r is stored at physical chunk c ^ ((r / 2) % 8).
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

// Calls f(std::integral_constant<int, 0>{}) .. f(std::integral_constant<int, N - 1>{}).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Weight tile tn and token tile tm of this workgroup (grid x spans the weight tiles, y the
// token tiles).  Workgroups go to the 8 XCDs round robin by linear id L = x + y gridDim.x,
// so XCD c runs L = c, c + 8, c + 16, ... in that order, 32 at a time (one per CU).  When
// the weight tiles split evenly over the XCDs and there are at most 8 token tiles, XCD c
// takes the weight tiles tn = c (mod 8) in blocks of J of them times every token tile,
// J * (token tiles) = 32: the workgroups an XCD runs together then share the slabs of a few
// token and weight tiles in its L2, and every weight tile is fetched by one XCD in one
// round (Qwen3-8B gate_up at 2048 rows: 612 instead of 968 MB fetched per launch, same
// time).  Otherwise the grid coordinates are used as they are (with 16 token tiles the
// blocks took 3 % longer).  The results are wave-uniform; readfirstlane keeps them (and the
// buffer resources built from them) in scalar registers.
__device__ __forceinline__ void tile_coordinates(int &tn, int &tm) {
  const int nx = static_cast<int>(gridDim.x);
  const int ny = static_cast<int>(gridDim.y);
  if (nx % 8 != 0 || ny > 8) {
    tn = static_cast<int>(blockIdx.x);
    tm = static_cast<int>(blockIdx.y);
    return;
  }
  const int linear = static_cast<int>(blockIdx.x) + nx * static_cast<int>(blockIdx.y);
  const int xcd = linear % 8;
  const int k = linear / 8;  // place in the XCD's dispatch order
  const int per_xcd = nx / 8;
  const int block_tiles = 32 / ny > per_xcd ? per_xcd : 32 / ny;
  const int block = k / (block_tiles * ny);
  const int rest = k - block * block_tiles * ny;
  const int tiles = per_xcd - block * block_tiles < block_tiles ? per_xcd - block * block_tiles : block_tiles;
  tm = __builtin_amdgcn_readfirstlane(rest / tiles);
  tn = __builtin_amdgcn_readfirstlane(xcd + 8 * (block * block_tiles + rest % tiles));
}

// Weight tile tn and expert tile tm of a grouped projection's workgroup.  Every weight tile
// of one expert tile reads the same rows, so they go to one XCD, one after another in its
// dispatch order: XCD c = L mod 8 takes expert tiles tm = c (mod 8), each with all its
// weight tiles, and fetches those rows into its L2 once (the grid's y extent is a multiple
// of 8, which makes the mapping a bijection).
__device__ __forceinline__ void grouped_tile_coordinates(int &tn, int &tm) {
  const int nx = static_cast<int>(gridDim.x);
  const int linear = static_cast<int>(blockIdx.x) + nx * static_cast<int>(blockIdx.y);
  const int k = linear / 8;  // place in the XCD's dispatch order
  tm = __builtin_amdgcn_readfirstlane(linear % 8 + 8 * (k / nx));
  tn = __builtin_amdgcn_readfirstlane(k % nx);
}

// Epilogue of a tile kernel whose waves each hold an MT x NT grid of 32x32 accumulator
// tiles (wave tile WTM x WTN at rows m0 + wm WTM, weight rows w0 + wn WTN).  With a K split
// the fp32 partial tile of this workgroup's range goes to scratch; otherwise the bf16
// result (gate_up: after the activation) goes out through `lds` (LDS_ELEMENTS bf16 of
// stage buffers that every wave is done with once this is called).
// Rows of a wave tile held per lane for the epilogue's row lookups (lane l: rows l, l + 64).
template <int WTM>
struct RowMeta {
  static constexpr int kPerLane = (WTM + 63) / 64;
  int32_t slot[kPerLane];   // scatter slot of the row, -1 for none
  float factor[kPerLane];   // row weight (grouped down projection), else 1
};

// Loads the scatter slots (and row weights) of wave tile rows [m0 + wm WTM, + WTM): one
// batch of independent loads, issued before the main loop so that they complete under it.
template <int WTM>
__device__ __forceinline__ void load_row_meta(const GemmArgs &a, int64_t m0, int64_t row_end, int wm,
                                              RowMeta<WTM> &meta) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < RowMeta<WTM>::kPerLane; ++i) {
    const int64_t token = m0 + wm * WTM + lane + 64 * i;
    const bool live = lane + 64 * i < WTM && token < row_end;
    meta.slot[i] = live ? a.scatter_slots[token] : -1;
    meta.factor[i] = live && a.row_scale != nullptr ? a.row_scale[token] : 1.0f;
  }
}

// Row `row`'s slot / weight from the lane that loaded it.  Every lane of the wave must call
// these together (no divergent branch around them): a shuffle only reads active lanes.
template <int WTM>
__device__ __forceinline__ int32_t row_slot(const RowMeta<WTM> &meta, int row) {
  int32_t value = __shfl(meta.slot[0], row & 63, kWave);
#pragma unroll
  for (int i = 1; i < RowMeta<WTM>::kPerLane; ++i) {
    const int32_t other = __shfl(meta.slot[i], row & 63, kWave);
    value = row >= 64 * i ? other : value;
  }
  return value;
}

template <int WTM>
__device__ __forceinline__ float row_factor(const RowMeta<WTM> &meta, int row) {
  float value = __shfl(meta.factor[0], row & 63, kWave);
#pragma unroll
  for (int i = 1; i < RowMeta<WTM>::kPerLane; ++i) {
    const float other = __shfl(meta.factor[i], row & 63, kWave);
    value = row >= 64 * i ? other : value;
  }
  return value;
}

template <int MT, int NT, int WTM, int WTN, int WAVES, int LDS_ELEMENTS, bool GATED, bool GROUPED, class P, bool EXTENDED>
__device__ __forceinline__ void tile_epilogue(const GemmArgs &a, const f32x16 (&acc)[MT][NT], uint16_t *lds,
                                              int64_t m0, int64_t row_end, int64_t w0, int wave, int wm, int wn,
                                              const RowMeta<WTM> &meta, int expert) {
  const int lane = threadIdx.x & 63;
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  if (a.k_split > 1) {
    // fp32 partial tile of this K range, [range][token][weight row]: for each (mt, r, nt)
    // the 32 lanes of a half-wave write 32 consecutive columns of one row (a Gate/Up pair
    // per lane for gate_up, in the weights' interleaved order).
    float *plane = a.partials + static_cast<int64_t>(blockIdx.z) * a.rows * a.n;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t token = m0 + wm * WTM + mt * 32 + 8 * (r >> 2) + 4 * frag_half + (r & 3);
        if (token >= a.rows) {
          continue;
        }
        float *row = plane + token * a.n;
        if constexpr (GATED) {
#pragma unroll
          for (int nt = 0; nt < NT / 2; ++nt) {
            const int64_t column = w0 + 2 * (wn * (WTN / 2) + nt * 32 + frag_row);
            if (column < a.n) {
              *reinterpret_cast<f32x2 *>(row + column) = f32x2{acc[mt][nt][r], acc[mt][nt + NT / 2][r]};
            }
          }
        } else {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const int64_t column = w0 + wn * WTN + nt * 32 + frag_row;
            if (column < a.n) {
              row[column] = acc[mt][nt][r];
            }
          }
        }
      }
    }
    return;
  }

  // Epilogue.  Lane holds D[8 (r / 4) + 4 (lane / 32) + r % 4][lane % 32] of each 32x32
  // tile.  Each wave rounds its tile to bf16 (gate_up: after the activation), writes it to
  // its own region of the now idle stage buffers and reads it back by rows, so results
  // leave in 16-byte chunks, 128 contiguous bytes per 8 lanes (to the slot rows when the
  // scatter is fused).  Bounds are checked per chunk on the way out.
  constexpr int OUT_N = GATED ? WTN / 2 : WTN;  // output columns of a wave tile
  constexpr int CPR = OUT_N / 8;                // 16-byte chunks per output row
  
  static_assert((WTM * CPR) % 64 == 0, "output chunks must split evenly over the lanes");
  static_assert(WTM * OUT_N * WAVES <= LDS_ELEMENTS, "epilogue tiles must fit the stage buffers");
  // With a scatter the rows' slots (and weights) come from `meta`, loaded at the start of the
  // kernel, so the epilogue does not wait on a dependent load per row.
  const bool scatter = a.scatter_slots != nullptr;
  __syncthreads();  // every wave is done reading the stage buffers
  uint16_t *out_tile = lds + wave * (WTM * OUT_N);
  // Chunk c of row r sits at physical chunk c ^ ((r / 4) % CPR): the two row groups one
  // write instruction covers (rows r and r + 4) then fall in different banks.
  auto slot_of = [](int row, int chunk) { return row * OUT_N + ((chunk ^ ((row >> 2) & (CPR - 1))) << 3); };
  // EXTENDED (grouped projections with a bias or a ReLU / GELU activation): the expert's
  // fp32 bias, indexed by weight row (gate_up: Gate and Up of output column c are weight
  // rows 2 c and 2 c + 1), and the first output column of this wave's tile.
  const float *bias = nullptr;
  int64_t bias_col0 = 0;
  if constexpr (EXTENDED) {
    bias = a.bias != nullptr ? a.bias + static_cast<int64_t>(expert) * a.bias_stride : nullptr;
    bias_col0 = GATED ? w0 / 2 + wn * (WTN / 2) : w0 + wn * WTN;
  }
  // The gated activation is the epilogue's VALU cost (two quarter-rate transcendentals per
  // output); its clipping is chosen once per tile, not per element.
  auto stage = [&](auto clip) XP_INLINE {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = mt * 32 + 8 * (r >> 2) + 4 * frag_half + (r & 3);
        // Row weight (grouped down projection); 1 elsewhere.
        float factor = 1.0f;
        if constexpr (GROUPED && !GATED) {
          factor = a.row_scale != nullptr ? row_factor(meta, row) : 1.0f;
        }
#pragma unroll
        for (int nt = 0; nt < OUT_N / 32; ++nt) {
          const int col = nt * 32 + frag_row;
          float value;
          if constexpr (GATED && EXTENDED) {
            float gate = acc[mt][nt][r];
            float up = acc[mt][nt + NT / 2][r];
            if (bias != nullptr) {
              const int64_t c = bias_col0 + col < a.n / 2 ? bias_col0 + col : 0;  // (columns past N are not stored)
              gate += bias[2 * c];
              up += bias[2 * c + 1];
            }
            value = moe_gated_payload<P, decltype(clip)::value>(gate, up, a.act);
          } else if constexpr (GATED) {
            value = gated_silu_payload<P, decltype(clip)::value>(acc[mt][nt][r], acc[mt][nt + NT / 2][r], a.act);
          } else if constexpr (EXTENDED) {
            float sum = acc[mt][nt][r];
            if (bias != nullptr) {
              sum += bias[bias_col0 + col < a.n ? bias_col0 + col : 0];
            }
            value = sum * factor;
          } else {
            value = acc[mt][nt][r] * factor;
          }
          out_tile[slot_of(row, col >> 3) + (col & 7)] = static_cast<uint16_t>(P::pack2(value, 0.0f) & 0xffffu);
        }
      }
    }
  };
  if (GATED && a.act.limit > 0.0f) {
    stage(std::true_type{});
  } else {
    stage(std::false_type{});
  }
  __syncthreads();
  const int64_t row0 = m0 + wm * WTM;
  const int64_t col0 = GATED ? w0 / 2 + wn * (WTN / 2) : w0 + wn * WTN;
  const int64_t out_cols = GATED ? a.n / 2 : a.n;
#pragma unroll 4
  for (int index = lane; index < WTM * CPR; index += 64) {
    const int row = index / CPR;
    const int chunk = index % CPR;
    const int64_t token = row0 + row;
    const int64_t col = col0 + chunk * 8;
    const int32_t slot = scatter ? row_slot(meta, row) : -1;  // all lanes, before the branch
    if (token < row_end && col < out_cols) {
      uint16_t *destination = a.out + token * a.ldo;
      if (scatter) {
        destination = slot >= 0 && static_cast<int64_t>(slot) < a.out_rows ? a.out + static_cast<int64_t>(slot) * a.ldo
                                                                            : nullptr;
      }
      if (destination != nullptr) {
        store16(destination + col, load16(out_tile + slot_of(row, chunk)));
      }
    }
  }
}

// BM x BN block tile, BK = 64, WAVES_M x WAVES_N waves (two per SIMD at 8 waves) each
// owning a (BM / WAVES_M) x (BN / WAVES_N) tile of 32x32x16 MFMA accumulators.  STAGES
// slabs of A and B live in LDS: while one is multiplied, the loads of the next STAGES - 1
// are in flight.  With 8 waves only waves 0-3 load: the refill issued after each barrier
// goes through the CU's one vector memory path at ~1 KB per 16 cycles and stalls the
// waves issuing it, and a SIMD whose other wave does not load keeps its matrix pipe fed
// meanwhile.  Grid z splits K into ranges of `k_slice` columns; with more than one
// range each workgroup writes the fp32 partial tile of its range and
// stream_reduce_kernel, launched next, adds the ranges in order and applies the epilogue.
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, bool GATED, bool GROUPED = false,
          bool STREAM_WEIGHTS = GROUPED, class PAYLOAD = Bf16Payload, bool EXTENDED = false>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void tile_gemm_kernel(GemmArgs a) {
  constexpr int BK = 64;
  constexpr int WAVES = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M;
  constexpr int WTN = BN / WAVES_N;
  constexpr int MT = WTM / 32;
  constexpr int NT = WTN / 32;
  constexpr int KSTEPS = BK / 16;                  // 16-wide k steps per slab
  constexpr int ROWS = BM + BN;                    // LDS rows per stage
  constexpr int STAGE = ROWS * BK;                 // bf16 elements per stage
  // LDS holds the A slabs of all stages, then the B slabs: a fragment read is then one
  // per-lane base per k step and operand plus an immediate offset below 64 KB (except for
  // A slabs past the first 64 KB), which keeps the address registers few.
  constexpr int B_REGION = STAGES * BM * BK;
  constexpr int LOAD_WAVES = WAVES == 8 ? 4 : WAVES;  // waves 0 .. LOAD_WAVES-1 fill the stages
  constexpr int A_LOADS = BM / 8 / LOAD_WAVES;     // 1 KB (8-row) load instructions per loading wave per stage
  constexpr int B_LOADS = BN / 8 / LOAD_WAVES;
  constexpr int LOADS = A_LOADS + B_LOADS;
  static_assert(MT >= 1 && NT >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  static_assert(!GATED || NT % 2 == 0, "gated tiles need whole Gate/Up column groups per wave");
  static_assert(BM % (8 * LOAD_WAVES) == 0 && BN % (8 * LOAD_WAVES) == 0, "stage rows must split evenly");
  static_assert(STAGES >= 2 && LOADS * (STAGES - 1) < 64, "in-flight loads must fit the vmcnt counter");
  static_assert(STAGES * STAGE * 2 <= 160 * 1024, "stages must fit the CU's LDS");

  __shared__ __attribute__((aligned(1024))) uint16_t lds[STAGES * STAGE];

  int tn;
  int tm;
  if constexpr (GROUPED) {
    grouped_tile_coordinates(tn, tm);
  } else {
    tile_coordinates(tn, tm);
  }
  // Rows [m0, row_end) and the weights of this tile: the live rows of the projection, or
  // for a grouped projection the rows of one expert tile and that expert's weights.
  int64_t m0 = static_cast<int64_t>(tm) * BM;
  int64_t row_end = a.rows;
  const uint16_t *weights = a.w;
  [[maybe_unused]] int expert = 0;
  if constexpr (GROUPED) {
    expert = __builtin_amdgcn_readfirstlane(a.tile_expert[tm]);
    if (expert < 0) {
      return;
    }
    m0 = __builtin_amdgcn_readfirstlane(a.tile_row0[tm]);
    row_end = __builtin_amdgcn_readfirstlane(a.expert_end[expert]);
    weights = a.w + static_cast<int64_t>(expert) * a.n * a.k;
  }
  if (m0 >= row_end) {
    return;
  }
  const int64_t w0 = static_cast<int64_t>(tn) * BN;
  const int64_t k_begin = static_cast<int64_t>(blockIdx.z) * a.k_slice;
  const int64_t k_end = a.k - k_begin < a.k_slice ? a.k : k_begin + a.k_slice;

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep it (and the load
  // descriptors and LDS bases derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  // A grouped 8-wave tile pairs each SIMD's two waves (w and w + 4) as one wave of the
  // upper half of the rows and one of the lower half: an expert tile's rows end anywhere,
  // and a wave whose rows are all past the end skips its fragment reads and MFMAs, which
  // leaves the SIMD's matrix pipe to its partner (at Qwen3-30B-A3B's ~128 routes per
  // expert, half of each 256-row tile).
  constexpr bool PAIRED = GROUPED && WAVES == 8 && WAVES_M % 2 == 0;
  constexpr int HALF_M = WAVES_M / 2;  // row bands per half
  const int wm = PAIRED ? (wave & 3) / WAVES_N + HALF_M * (wave >> 2) : wave % WAVES_M;
  const int wn = PAIRED ? (wave & 3) % WAVES_N : wave / WAVES_M;
  // Whether this wave's row band holds a live row (always outside grouped tiles).
  const bool wave_live = !GROUPED || __builtin_amdgcn_readfirstlane(static_cast<int>(m0 + wm * WTM < row_end)) != 0;

  // ---- loads: loading wave w fills A_LOADS 8-row groups of the A tile (rows from
  // w * BM / LOAD_WAVES) and B_LOADS of the B tile, so which resource a load uses is a
  // compile-time fact.  Lane i of a load writes LDS row r0 + i / 8, physical chunk i % 8,
  // which holds logical k chunk (i % 8) ^ swizzle(row): the swizzle is applied by choosing
  // the global chunk.
  const int64_t a_rows_left = row_end - m0;
  const int64_t b_rows_left = a.n - w0;
  // A grouped projection may gather its A rows: tile row r is row gather_slots[m0 + r] /
  // gather_divisor of x ([pool_rows, ldx]); otherwise the tile's rows are contiguous.
  const bool gathered = GROUPED && a.gather_slots != nullptr;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      gathered ? make_rsrc(a.x, static_cast<uint32_t>(a.pool_rows * a.ldx * 2))
               : make_rsrc(a.x + m0 * a.ldx, static_cast<uint32_t>((a_rows_left < BM ? a_rows_left : BM) * a.ldx * 2));
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(weights + w0 * a.k, static_cast<uint32_t>((b_rows_left < BN ? b_rows_left : BN) * a.k * 2));
  // Load q of a wave covers the 8-row group starting at LDS row g (a multiple of 8); lane
  // i takes row g + i / 8 and k chunk (i % 8) ^ swizzle(row).  Because g is a multiple of
  // 8, swizzle(g + i / 8) = (i / 16) ^ (4 if g / 8 is odd), so the per-lane part of every
  // offset takes one of two values and the group part is wave-uniform.
  const int a_first = (wave % LOAD_WAVES) * (BM / LOAD_WAVES);
  const int b_first = BM + (wave % LOAD_WAVES) * (BN / LOAD_WAVES);
  const bool loading_wave = wave < LOAD_WAVES;
  const int row_in_load = lane >> 3;
  const int lane_chunk[2] = {(lane & 7) ^ (row_in_load >> 1), (lane & 7) ^ (row_in_load >> 1) ^ 4};
  // Grouped tiles: byte offset of the A row each lane loads in load q (rows past the tile's
  // live rows of a gathered tile read as zeros through an out-of-range offset).
  uint32_t a_row_bytes[GROUPED ? A_LOADS : 1];
  if constexpr (GROUPED) {
#pragma unroll
    for (int q = 0; q < A_LOADS; ++q) {
      const int row = a_first + q * 8 + row_in_load;
      if (gathered) {
        a_row_bytes[q] = row < a_rows_left
                             ? static_cast<uint32_t>(a.gather_slots[m0 + row] / a.gather_divisor * a.ldx * 2)
                             : kOutOfRange;
      } else {
        a_row_bytes[q] = static_cast<uint32_t>(row * a.ldx * 2);
      }
    }
  }
  // B rows of a gated tile are permuted: LDS row p = wq * G + s * G / 2 + jj (G = BN /
  // WAVES_N) holds weight row 2 (wq * G / 2 + jj) + s, i.e. within an 8-row group the weight
  // row is the group's first weight row plus 2 (i / 8).
  constexpr int B_ROW_STEP = GATED ? 2 : 1;
  auto b_group_row = [](int p) XP_INLINE {
    if constexpr (GATED) {
      constexpr int group = BN / WAVES_N;
      return 2 * ((p / group) * (group / 2) + p % (group / 2)) + (p % group) / (group / 2);
    } else {
      return p;
    }
  };
  // Slab kt of this workgroup's K range.  Slabs at or past the range end (the prologue of
  // a short range, the refills after the last slab) load zeros without memory traffic.
  // PART selects the A loads (1), the B loads (2) or both (3).
  auto issue_part = [&](int64_t kt, int stage, auto part) XP_INLINE {
    constexpr int PART = decltype(part)::value;
    const int64_t k_pos = k_begin + kt * BK;
    const uint32_t k_bytes = static_cast<uint32_t>(k_pos * 2);
    // 16-byte chunks of this slab that lie inside the range (8 except in a ragged last slab).
    const int64_t chunks_left = (k_end - k_pos) >> 3;
    uint16_t *a_stage = lds + stage * BM * BK;
    uint16_t *b_stage = lds + B_REGION + stage * BN * BK - BM * BK;  // indexed by g >= BM
    // The scalar offset must stay wave-uniform; masking goes through the per-lane offset
    // (kOutOfRange + k_bytes is still past the resource end), as a select, not a branch.
    // A and B loads are separate loops so that each names one resource.
#pragma unroll
    for (int q = 0; q < ((PART & 1) ? A_LOADS : 0); ++q) {
      const int g = a_first + q * 8;
      const int chunk = lane_chunk[(g >> 3) & 1];
      uint32_t offset;
      if constexpr (GROUPED) {
        offset = a_row_bytes[q] + static_cast<uint32_t>(chunk * 16);
      } else {
        offset = static_cast<uint32_t>(((g + row_in_load) * a.ldx + chunk * 8) * 2);
      }
      buffer_load_lds16(a_rsrc, a_stage + g * BK, chunk < chunks_left ? offset : kOutOfRange, k_bytes);
    }
#pragma unroll
    for (int q = 0; q < ((PART & 2) ? B_LOADS : 0); ++q) {
      const int g = b_first + q * 8;
      const int chunk = lane_chunk[(g >> 3) & 1];
      const int weight_row = b_group_row(g - BM) + B_ROW_STEP * row_in_load;
      const uint32_t offset = static_cast<uint32_t>((weight_row * a.k + chunk * 8) * 2);
      buffer_load_lds16<STREAM_WEIGHTS ? kLoadNontemporal : 0>(b_rsrc, b_stage + g * BK,
                                                               chunk < chunks_left ? offset : kOutOfRange, k_bytes);
    }
  };
  auto issue_loads = [&](int64_t kt, int stage) XP_INLINE { issue_part(kt, stage, std::integral_constant<int, 3>{}); };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[mt][nt][r] = 0.0f;
      }
    }
  }

  // Fragment rows are frag_row plus multiples of 16 (wave and tile offsets), which leave
  // swizzle(row) unchanged, so one per-lane term per k step addresses every fragment.
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "fragment row offsets must keep the swizzle");
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  int frag_lane[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    frag_lane[ks] = frag_row * BK + (((ks * 2 + frag_half) ^ swizzle(frag_row)) << 3);
  }
  // Per-lane LDS byte bases of the fragment reads: one per k step, operand and 64 KB window
  // that the operand's stages reach.  They are opaque to the compiler, so every other term
  // of a read's address (stage, fragment, window remainder) goes into the instruction's
  // 16-bit offset instead of a register of its own.
  constexpr int A_SPAN = (STAGES - 1) * BM * BK * 2 + (MT - 1) * 32 * BK * 2;  // largest constant A offset
  constexpr int B_SPAN = B_REGION * 2 + (STAGES - 1) * BN * BK * 2 + (NT - 1) * 32 * BK * 2;
  constexpr int A_WINDOWS = A_SPAN / 65536 + 1;
  constexpr int B_WINDOWS = B_SPAN / 65536 + 1;
  uint32_t a_base[A_WINDOWS][KSTEPS];
  uint32_t b_base[B_WINDOWS][KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
    for (int w = 0; w < A_WINDOWS; ++w) {
      a_base[w][ks] = static_cast<uint32_t>((frag_lane[ks] + wm * WTM * BK) * 2 + w * 65536);
      __asm__ volatile("" : "+v"(a_base[w][ks]));
    }
#pragma unroll
    for (int w = 0; w < B_WINDOWS; ++w) {
      b_base[w][ks] = static_cast<uint32_t>((frag_lane[ks] + wn * WTN * BK) * 2 + w * 65536);
      __asm__ volatile("" : "+v"(b_base[w][ks]));
    }
  }
  const char *lds_bytes = reinterpret_cast<const char *>(lds);
  // Fragment slots.  With three, the fragments of k step g live in slot g % 3 and are read
  // two k steps ahead of their MFMAs, so a wave running alone on its SIMD (its partner
  // blocked on the barrier or on issuing loads) does not wait on LDS latency.  A wave tile of
  // 8 or more 32x32 accumulators (the 256 x 256 tiles) has 8 MFMAs (256 cycles) per k step
  // to cover one k step of read latency, and its accumulators take 128 of the 256 VGPRs two
  // waves per SIMD leave: it reads one k step ahead from two slots (slot g % 2), which frees
  // the 24 VGPRs of a third slot (with three it spilled 88 bytes per lane).
  static_assert(KSTEPS == 4, "the slab schedule below is written for four k steps");
  constexpr int SLOTS = MT * NT >= 8 ? 2 : 3;
  u32x4 af[SLOTS][MT];
  u32x4 bfrag[SLOTS][NT];
  // A grouped tile's wave whose rows all lie past the expert's last route reads no
  // fragments and issues no MFMAs (one wave-uniform branch around the unrolled loops).
  auto read_fragments = [&](int stage, int ks, int slot) XP_INLINE {
    if (!wave_live) {
      return;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int offset = stage * BM * BK * 2 + mt * 32 * BK * 2;
      af[slot][mt] = *reinterpret_cast<const u32x4 *>(lds_bytes + a_base[offset >> 16][ks] + (offset & 0xffff));
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int offset = B_REGION * 2 + stage * BN * BK * 2 + nt * 32 * BK * 2;
      bfrag[slot][nt] = *reinterpret_cast<const u32x4 *>(lds_bytes + b_base[offset >> 16][ks] + (offset & 0xffff));
    }
  };
  auto mfma_step = [&](int slot) XP_INLINE {
    if (!wave_live) {
      return;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        acc[mt][nt] = PAYLOAD::mfma32(af[slot][mt], bfrag[slot][nt], acc[mt][nt]);
      }
    }
  };
  // Workgroup barrier for the stage ring.  Before it each wave waits for its loads of the
  // next slab (leaving the STAGES - 2 younger slabs in flight, which a __syncthreads would
  // also drain) and for its own LDS reads, so that after it every wave may read the next
  // slab and refill the stage just read.  The memory clobber keeps the compiler from
  // moving LDS accesses across it; the scheduling barriers keep instructions on their side.
  auto stage_barrier = []() XP_INLINE {
    constexpr int N = LOADS * (STAGES - 2);
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4));  // vmcnt(N) lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    __asm__ volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Scatter slots and row weights of this wave's rows, for the epilogue (split-K tiles
  // write partials and need none).
  RowMeta<WTM> meta;
  if (a.scatter_slots != nullptr && a.k_split == 1) {
    load_row_meta<WTM>(a, m0, row_end, wm, meta);
  }
  // The chooser never makes an empty K range, so every workgroup runs at least one slab.
  const int64_t ktiles = (k_end - k_begin + BK - 1) / BK;
  // Prologue: slabs 0 .. STAGES-1 in flight, wait for slab 0, read its first fragments.
  if (loading_wave) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      issue_loads(s, s);
    }
  }
  wait_vmcnt<LOADS * (STAGES - 1)>();
  __syncthreads();
  read_fragments(0, 0, 0);
  if constexpr (SLOTS == 3) {
    read_fragments(0, 1, 1);
  }

  // Slab kt runs k steps 4 kt .. 4 kt + 3 from stage kt % STAGES, its fragment slots
  // starting at phase kt % 3.  After k step 1 every fragment of the slab has been read, so
  // the stage barrier sits there: past it slab kt+1 is in LDS (its first two fragment sets
  // are read during k steps 2 and 3) and this stage may be refilled with slab kt+STAGES
  // (zeros past the range end), which the loading waves issue interleaved with k step 2's
  // MFMAs.  The loop is unrolled over lcm(3, STAGES) slabs so that slots and stages, and
  // with them every LDS address but one per-lane term per k step, are compile-time
  // constants.  The loading and the other waves run the same loop (the same barriers),
  // with and without the refills, as separate code so that each has a fixed interleave.
  constexpr int UNROLL = SLOTS == 2 || STAGES % 3 == 0 ? STAGES : 3 * STAGES;
  // Two slots: k step g's fragments are read while k step g - 1's MFMAs run; the barrier
  // follows k step 2's MFMAs (every fragment of the slab read by then), and the refill goes
  // out under k step 3's.
  auto slab2 = [&](auto index, auto loads, int64_t kt) XP_INLINE {
    constexpr int S = decltype(index)::value % STAGES;
    constexpr int NEXT = (S + 1) % STAGES;
    constexpr bool LOADING = decltype(loads)::value;
    read_fragments(S, 1, 1);
    mfma_step(0);
    __builtin_amdgcn_sched_barrier(0);
    read_fragments(S, 2, 0);
    mfma_step(1);
    __builtin_amdgcn_sched_barrier(0);
    read_fragments(S, 3, 1);
    mfma_step(0);
    stage_barrier();
    read_fragments(NEXT, 0, 0);
    if constexpr (LOADING) {
      issue_part(kt + STAGES, S, std::integral_constant<int, 3>{});
    }
    mfma_step(1);
#pragma unroll
    for (int i = 0; i < MT * NT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      if constexpr (LOADING) {
        __builtin_amdgcn_sched_group_barrier(0x020, (LOADS + MT * NT - 1) / (MT * NT), 0);  // memory loads
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto slab = [&](auto index, auto loads, int64_t kt) XP_INLINE {
    if constexpr (SLOTS == 2) {
      slab2(index, loads, kt);
      return;
    }
    constexpr int P = decltype(index)::value % 3;
    constexpr int S = decltype(index)::value % STAGES;
    constexpr int NEXT = (S + 1) % STAGES;
    constexpr bool LOADING = decltype(loads)::value;
    read_fragments(S, 2, (P + 2) % 3);
    mfma_step(P);
    __builtin_amdgcn_sched_barrier(0);
    read_fragments(S, 3, P);
    mfma_step((P + 1) % 3);
    stage_barrier();
    // With three or more stages the A refill goes out under k step 2's MFMAs and the B
    // refill under k step 3's (one load per MFMA: Qwen3-8B down at 2048 rows on 256 x 128
    // tiles, 176 -> 169 us); the two-stage 256 x 256 tile issues both under k step 2
    // (spread, it was 1 % slower).
    constexpr bool SPREAD = STAGES >= 3;
    constexpr int FIRST_LOADS = SPREAD ? A_LOADS : LOADS;
    read_fragments(NEXT, 0, (P + 1) % 3);
    if constexpr (LOADING) {
      issue_part(kt + STAGES, S, std::integral_constant<int, SPREAD ? 1 : 3>{});
    }
    mfma_step((P + 2) % 3);
#pragma unroll
    for (int i = 0; i < MT * NT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      if constexpr (LOADING) {
        __builtin_amdgcn_sched_group_barrier(0x020, (FIRST_LOADS + MT * NT - 1) / (MT * NT), 0);  // memory loads
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    read_fragments(NEXT, 1, (P + 2) % 3);
    if constexpr (LOADING && SPREAD) {
      issue_part(kt + STAGES, S, std::integral_constant<int, 2>{});
    }
    mfma_step(P);
    if constexpr (SPREAD) {
#pragma unroll
      for (int i = 0; i < MT * NT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if constexpr (LOADING) {
          __builtin_amdgcn_sched_group_barrier(0x020, (B_LOADS + MT * NT - 1) / (MT * NT), 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int64_t kt = 0;
  auto main_loop = [&](auto loads) XP_INLINE {
    for (; kt + UNROLL < ktiles; kt += UNROLL) {
      static_for<UNROLL>([&](auto j) XP_INLINE { slab(j, loads, kt + decltype(j)::value); });
    }
    // The remaining slabs before the last (fewer than UNROLL), continuing the pattern.
    static_for<UNROLL - 1>([&](auto j) XP_INLINE {
      if (kt + decltype(j)::value + 1 < ktiles) {
        slab(j, loads, kt + decltype(j)::value);
      }
    });
  };
  if (loading_wave) {
    main_loop(std::true_type{});
  } else {
    main_loop(std::false_type{});
  }
  // Last slab (index ktiles - 1): no barrier and no refill.
  static_for<UNROLL>([&](auto j) XP_INLINE {
    if ((ktiles - 1) % UNROLL == decltype(j)::value) {
      constexpr int S = decltype(j)::value % STAGES;
      if constexpr (SLOTS == 2) {
        read_fragments(S, 1, 1);
        mfma_step(0);
        read_fragments(S, 2, 0);
        mfma_step(1);
        read_fragments(S, 3, 1);
        mfma_step(0);
        mfma_step(1);
      } else {
        constexpr int P = decltype(j)::value % 3;
        read_fragments(S, 2, (P + 2) % 3);
        mfma_step(P);
        read_fragments(S, 3, P);
        mfma_step((P + 1) % 3);
        mfma_step((P + 2) % 3);
        mfma_step(P);
      }
    }
  });
  // Past-the-end refills may still be landing in the stage buffers the epilogue reuses.
  __builtin_amdgcn_s_waitcnt(0);

  tile_epilogue<MT, NT, WTM, WTN, WAVES, STAGES * STAGE, GATED, GROUPED, PAYLOAD, EXTENDED>(a, acc, lds, m0, row_end, w0, wave, wm, wn,
                                                                         meta, expert);
}

// ------------------------------------------------------------------ tables
// Chunks of loads in flight per wave of the split kernel, by token groups (the register
// budget of two workgroups per CU).
constexpr int split_depth(int groups) { return groups == 1 ? 4 : 3; }

// The split kernel for `groups` token groups of 8 (1 or 2); the fused gather takes one.
// (Four groups, 32 tokens, were measured and dropped: the token pieces read from L2 for each
// weight line then cost more than the tile kernels, 60-77 us against 41-43 us for Qwen3-8B
// gate_up at 17-32 rows.)
// Every Dense and grouped MoE kernel is instantiated for both payload dtypes (bf16, fp16);
// `payload` (GemmArgs::payload) picks one.
template <bool GATED>
const void *split_kernel(int groups, bool gather, int32_t payload) {
  if (gather) {
    return payload == kPayloadF16
               ? reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(1), 1, GATED, true, F16Payload>)
               : reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(1), 1, GATED, true, Bf16Payload>);
  }
  if (payload == kPayloadF16) {
    return groups == 1 ? reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(1), 1, GATED, false, F16Payload>)
                       : reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(2), 2, GATED, false, F16Payload>);
  }
  return groups == 1 ? reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(1), 1, GATED, false, Bf16Payload>)
                     : reinterpret_cast<const void *>(&split_gemm_kernel<split_depth(2), 2, GATED, false, Bf16Payload>);
}

// The persistent split kernel with the gather fused (one token group).
template <bool GATED>
const void *split_gathered_kernel_ptr(int32_t payload) {
  return payload == kPayloadF16 ? reinterpret_cast<const void *>(&split_gathered_kernel<split_depth(1), GATED, F16Payload>)
                                : reinterpret_cast<const void *>(&split_gathered_kernel<split_depth(1), GATED, Bf16Payload>);
}

int split_groups(int64_t capacity) { return capacity <= kSplitGroupTokens ? 1 : 2; }

template <bool GATED, bool GATHER = false>
const void *stream_kernel(int32_t payload) {
  return payload == kPayloadF16 ? reinterpret_cast<const void *>(&stream_gemm_kernel<GATED, GATHER, F16Payload>)
                                : reinterpret_cast<const void *>(&stream_gemm_kernel<GATED, GATHER, Bf16Payload>);
}

template <bool GATED>
const void *stream_reduce(int32_t payload) {
  return payload == kPayloadF16 ? reinterpret_cast<const void *>(&stream_reduce_kernel<GATED, F16Payload>)
                                : reinterpret_cast<const void *>(&stream_reduce_kernel<GATED, Bf16Payload>);
}

// The resident kernel for 16 token rows (two groups of 8) and `cpw` chunks per wave (1 to
// 4), and for 32 (four groups, two chunks in flight per wave) as the gate_up of a Dense
// step with the gather fused.  Measured on MI355X, Qwen3 layers at 17-32 rows against the
// separate gather and the 64 x 64 tiles: 4B (19456 weight rows) 50.3 / 51.2 / 53.4 ->
// 45.6 / 46.7 / 49.4 us at 20 / 24 / 32 rows, 8B (24576) 71.9 / 72.4 / 74.0 -> 69.4 /
// 70.4 / 72.4; 1.7B (12288) and 0.6B (6144) within +-1 us either way, so four groups serve
// only projections of at least kResidentWideMinN weight rows.  (At 9-16 rows four groups
// were 1.2-4.3 us slower than two.)
constexpr int kResidentMaxChunksPerWave = 4;
constexpr int kResidentGroups = 2;
constexpr int kResidentWideGroups = 4;

template <int TG, bool GATED, bool GATHER, class P>
const void *resident_kernel(int cpw) {
  using Kernel = void (*)(GemmArgs);
  static const Kernel table[kResidentMaxChunksPerWave] = {
      &resident_gemm_kernel<TG, 1, GATED, GATHER, P>, &resident_gemm_kernel<TG, 2, GATED, GATHER, P>,
      &resident_gemm_kernel<TG, 3, GATED, GATHER, P>, &resident_gemm_kernel<TG, 4, GATED, GATHER, P>};
  return reinterpret_cast<const void *>(table[cpw - 1]);
}

// Null for a combination without an instantiation (four groups serve gate_up with the
// gather fused only).
template <class P>
const void *resident_kernel_for(bool gated, bool gather, int cpw, int groups) {
  if (groups == kResidentWideGroups) {
    return gated && gather ? resident_kernel<kResidentWideGroups, true, true, P>(cpw) : nullptr;
  }
  if (groups != kResidentGroups) {
    return nullptr;
  }
  if (gated) {
    return gather ? resident_kernel<kResidentGroups, true, true, P>(cpw)
                  : resident_kernel<kResidentGroups, true, false, P>(cpw);
  }
  return resident_kernel<kResidentGroups, false, false, P>(cpw);
}

const void *resident_kernel_for(bool gated, bool gather, int cpw, int32_t payload, int groups) {
  return payload == kPayloadF16 ? resident_kernel_for<F16Payload>(gated, gather, cpw, groups)
                                : resident_kernel_for<Bf16Payload>(gated, gather, cpw, groups);
}

struct TileShape {
  int bm;
  int bn;
  int waves;
  int stages;           // LDS slabs (STAGES - 1 of them in flight); one workgroup per CU
  double flops_per_us;  // one CU's rate on this shape with every CU busy, measured on MI355X
};
constexpr TileShape kTileShapes[] = {
    {256, 256, 8, 2, 4.6e6},
    {256, 128, 8, 3, 4.0e6},
    {128, 128, 4, 3, 3.4e6},
    {64, 128, 4, 6, 2.4e6},
    {64, 64, 2, 4, 1.2e6},
};
constexpr int kTileShapeCount = sizeof(kTileShapes) / sizeof(kTileShapes[0]);
// The cost model ranks the first four shapes.  The 64 x 64 gated tile (two waves, four
// stages, two workgroups per CU) replaces the 64 x 128 one for a one-token-tile grid that
// leaves CUs idle: twice the workgroups stream the weights.  Measured on MI355X with weights
// streamed cold: Qwen3-0.6B gate_up at 32 / 64 / 128 rows 11.2 / 12.0 / 11.8 -> 9.3 / 9.8 /
// 9.8 us (48-96 -> 96-192 workgroups), Qwen3-8B gate_up at 32 rows 44.5 -> 43.0 us.
constexpr int kRankedTileShapes = 4;
constexpr int kDecodeTile = 3;        // 64 x 128
constexpr int kNarrowDecodeTile = 4;  // 64 x 64

// STREAM: the grid has one token tile, so each weight tile has one reader and its loads
// carry the nontemporal hint (a compile-time policy: a per-load branch on an argument cost
// the loading waves ~2 % at 2048 rows).
template <bool GATED, class P>
const void *tile_kernel(int variant, bool stream) {
  using Kernel = void (*)(GemmArgs);
  static const Kernel table[][2] = {
      {&tile_gemm_kernel<256, 256, 2, 4, 2, GATED, false, false, P>, &tile_gemm_kernel<256, 256, 2, 4, 2, GATED, false, true, P>},
      {&tile_gemm_kernel<256, 128, 4, 2, 3, GATED, false, false, P>, &tile_gemm_kernel<256, 128, 4, 2, 3, GATED, false, true, P>},
      {&tile_gemm_kernel<128, 128, 2, 2, 3, GATED, false, false, P>, &tile_gemm_kernel<128, 128, 2, 2, 3, GATED, false, true, P>},
      {&tile_gemm_kernel<64, 128, 2, 2, 6, GATED, false, false, P>, &tile_gemm_kernel<64, 128, 2, 2, 6, GATED, false, true, P>},
      {&tile_gemm_kernel<64, 64, 2, 1, 4, GATED, false, false, P>, &tile_gemm_kernel<64, 64, 2, 1, 4, GATED, false, true, P>},
  };
  static_assert(sizeof(table) / sizeof(table[0]) == kTileShapeCount, "one kernel per tile shape");
  return reinterpret_cast<const void *>(table[variant][stream ? 1 : 0]);
}

template <bool GATED>
const void *tile_kernel(int variant, bool stream, int32_t payload) {
  return payload == kPayloadF16 ? tile_kernel<GATED, F16Payload>(variant, stream)
                                : tile_kernel<GATED, Bf16Payload>(variant, stream);
}

constexpr int kComputeUnits = 256;

// Decode sizes (up to 16 rows) take the split or the stream kernel, whichever a cost model
// in microseconds prefers.  Both stream the weights with 8-wave workgroups, each at a
// bounded rate (measured, the chip rate scales with the workgroup count up to the CU
// count), so a grid of few workgroups is the thing to avoid (Qwen3-4B down through the
// split kernel with 2 K ranges per row block has 80 workgroups: 41 us; with 8, 320: 16 us),
// workgroups past 256 run as further rounds, and the chip caps the total (both read whole
// 128-byte weight lines with the nontemporal hint).
// The split kernel reads its token pieces from L2, a little more per row and chunk of its
// K range; the stream kernel's K slices cost the reduction launch and their partial
// traffic.  The split kernel's rounds of 256 workgroups are priced one after another (each
// at the chip rate or at one workgroup's rate, whichever is slower, and never below one load
// round trip: short rounds are latency-bound).  Least-squares fit (relative error) to 498
// forced split (every K split) and stream (K slices of 512-4096 columns) timings on MI355X:
// the Qwen3 0.6B / 1.7B / 4B / 8B projections, the Qwen3-32B TP shard's and a hidden-1536
// down at 1 to 16 rows, the weights rotated over three copies (streamed from HBM).  Mean
// modelled error 7.4 % (26 % for the constants it replaced); summed over the 66
// (projection, rows) cases, its picks are 29 us slower than the fastest measured ones,
// against 79 us before.  Per layer (alternating builds on one box) that took the 9-16-row
// Dense steps of Qwen3-4B / 1.7B / the 32B shard from 47-51 / 34-38 / 42-47 us to 44-45 /
// 33-35 / 39-41 us and hidden 1536 at 1-8 rows from 27-31 to 26-27 us (Qwen3-8B at 9 rows:
// 61.4 -> 62.5 us, the one loss).
constexpr int64_t kDecodeMaxRows = 16;
constexpr int64_t kSplitMaxRows = kSplitGroupTokens * kSplitMaxGroups;
// Index: token groups - 1.  Two groups read twice the token pieces from L2 per weight line,
// which lowers the chip rate.
constexpr double kSplitWorkgroupBytesPerUs[kSplitMaxGroups] = {32.7e3, 27.6e3};
constexpr double kSplitBytesPerUs[kSplitMaxGroups] = {6.75e6, 5.06e6};
constexpr double kSplitFixedUs[kSplitMaxGroups] = {3.54, 4.19};
constexpr double kSplitRoundFloorUs = 2.7;  // no round of workgroups is shorter (one load round trip)
constexpr double kSplitTieMargin = 0.001;
// Per row past the first and 128-wide chunk of a range (padded to the load depth).
constexpr double kSplitRowUsPerChunk[kSplitMaxGroups] = {0.0406, 0.0314};
constexpr double kStreamWorkgroupBytesPerUs = 29.2e3;
constexpr double kStreamBytesPerUs = 6.1e6;
constexpr double kStreamFixedUs = 1.03;
constexpr double kStreamRowUs = 0.0071;  // per row past the first and 512 columns of the K slice
constexpr double kStreamReduceUs = 5.4;  // the reduction launch (it also ends the overlap of slices)
constexpr double kStreamPartialBytesPerUs = 6.0e6;
constexpr int kSplitDepth = 4;
constexpr double kGatherUs = 4.0;  // a separate gather launch at decode sizes (measured 3.8-4.0 us)
// The split kernel's fused gather runs in every workgroup, one per CU (its registers allow
// no second), beside only the first weight chunks: measured 2.3 us per round of 256
// workgroups for Qwen3-0.6B gate_up (one round), 3.3 and 4.4 us for Qwen3-8B (3 and 6).
constexpr double kSplitGatherRoundUs = 3.0;
// The same for the stream kernel's fused gather, per round of workgroups (measured: Qwen3-8B
// gate_up at 16 rows, 192 workgroups, 37.0 us plain and ~41 us with the gather fused).
constexpr double kStreamGatherUs = 3.5;
constexpr int64_t kSplitGatherMaxK = 4096;  // 8 staged rows of K + 16 bf16 (66 KB) beside the partial sums
static_assert(kSplitGatherMaxK * 2 <= kSplitGatheredScratchBytes, "the norm weights fit the partial sums' space");
static_assert(kSplitGatherMaxK / 8 <= 8 * 64, "a staged row is at most 8 chunks per lane");
// split_gathered_kernel: two workgroups per CU (128 VGPRs; at most 80 KB of LDS each, the
// 8 staged rows of 4096 + 16 bf16 and the space shared by the norm weights and the partial
// sums), for projections with at least that many units.  Its gather runs under the first
// weight chunks' round trip and its token pieces come from LDS (no per-row L2 reads); what
// the gather still adds is the normalisation pass over LDS and one barrier: measured on
// MI355X, the Qwen3-8B / 4B / 1.7B layer at one row 52.2 / 36.9 / 24.7 us against 55.0 /
// 37.7 / 26.6 us when the gather took its own round trip before the weight stream.
constexpr int64_t kSplitGatheredWorkgroups = 2 * kComputeUnits;
constexpr double kSplitPersistentGatherUs = 1.0;

double decode_stream_us(int64_t n, int64_t k, int64_t workgroups, double workgroup_bytes_per_us,
                        double chip_bytes_per_us, double fixed_us) {
  const int64_t rounds = (workgroups + kComputeUnits - 1) / kComputeUnits;
  const double bytes = 2.0 * static_cast<double>(n) * static_cast<double>(k);
  const double per_workgroup = static_cast<double>(rounds) * bytes / workgroups / workgroup_bytes_per_us;
  const double chip = bytes / chip_bytes_per_us;
  return (per_workgroup > chip ? per_workgroup : chip) + fixed_us;
}

// Candidate K splits of the split kernel (1, 2, 4 or 8 ranges per 16-row block, each range
// a whole number of 128-wide chunks and none empty) and their modelled cost at `capacity`
// rows, with the gather fused when `gather` is set.
GemmChoice choose_split(int64_t capacity, int64_t n, int64_t k, double &cost, bool gather = false,
                        bool persistent = false) {
  const int64_t quantum = 128;
  const int64_t row_blocks = (n + 15) / 16;
  const int groups = split_groups(capacity);
  const int64_t depth = split_depth(groups);
  GemmChoice best{GemmKind::Split, groups, 0, 1};
  cost = -1.0;
  for (int64_t ksplit = 1; ksplit <= kSplitWaves; ksplit *= 2) {
    const int64_t slice = ((k + ksplit - 1) / ksplit + quantum - 1) / quantum * quantum;
    if ((ksplit - 1) * slice >= k) {
      break;
    }
    const int64_t workgroups = (row_blocks * ksplit + kSplitWaves - 1) / kSplitWaves;
    const double workgroup_bytes = 2.0 * static_cast<double>(n) * static_cast<double>(k) / workgroups;
    double us = kSplitFixedUs[groups - 1];
    for (int64_t left = workgroups; left > 0; left -= kComputeUnits) {
      const double round_bytes = static_cast<double>(left < kComputeUnits ? left : kComputeUnits) * workgroup_bytes;
      const double chip_us = round_bytes / kSplitBytesPerUs[groups - 1];
      const double workgroup_us = workgroup_bytes / kSplitWorkgroupBytesPerUs[groups - 1];
      const double round_us = chip_us > workgroup_us ? chip_us : workgroup_us;
      us += round_us > kSplitRoundFloorUs ? round_us : kSplitRoundFloorUs;
    }
    us += kSplitRowUsPerChunk[groups - 1] *
                    static_cast<double>((slice / 128 + depth - 1) / depth * depth) *
                    static_cast<double>(capacity - 1);
    if (gather) {
      us += kSplitGatherRoundUs * static_cast<double>((workgroups + kComputeUnits - 1) / kComputeUnits);
    }
    // The persistent kernel walks units on a fixed grid, so it takes the most K ranges of
    // at least two chunks (the most units to balance) rather than the cheapest round count.
    // Otherwise a split whose cost equals the cheapest so far (within kSplitTieMargin, i.e.
    // rounding) takes its place: the most ranges among equal costs, shorter per-wave load
    // chains (Qwen3-8B gate_up at one row: 4 and 8 ranges model the same, and 8 is the
    // persistent kernel's split).
    if (persistent ? slice >= 2 * quantum : (cost < 0.0 || us < cost * (1.0 + kSplitTieMargin))) {
      best = {GemmKind::Split, groups, slice, ksplit};
      cost = us;
    }
  }
  return best;
}

constexpr int64_t kStreamLdsBytes = 160 * 1024 - 256;  // the fused gather's row table is static LDS
constexpr int64_t kStreamSliceQuantum = 128 * kStreamDepth;  // a whole number of load groups

int64_t stream_slices(int64_t k, int64_t k_slice) { return (k + k_slice - 1) / k_slice; }

// K slice of the stream kernel: workgroups are (8 row blocks) x (one slice), and the slice
// count minimising the modelled cost wins.
GemmChoice choose_stream(int64_t capacity, int64_t n, int64_t k, double &cost) {
  constexpr int64_t tp = 16;  // staged token rows
  const int64_t groups = ((n + 15) / 16 + kStreamWaves - 1) / kStreamWaves;
  GemmChoice best{GemmKind::Stream, 0, 0, 1};
  cost = -1.0;
  for (int64_t slices = 1; slices <= 64; ++slices) {
    const int64_t k_slice = ((k + slices - 1) / slices + kStreamSliceQuantum - 1) / kStreamSliceQuantum *
                            kStreamSliceQuantum;
    if (tp * (k_slice + kStreamRowPad) * 2 > kStreamLdsBytes || stream_slices(k, k_slice) != slices) {
      continue;  // does not fit LDS, or the same slice length as fewer slices
    }
    double us = decode_stream_us(n, k, slices * groups, kStreamWorkgroupBytesPerUs, kStreamBytesPerUs, kStreamFixedUs) +
                kStreamRowUs * static_cast<double>(capacity - 1) * static_cast<double>(k_slice) / 512.0;
    if (slices > 1) {
      us += kStreamReduceUs + 8.0 * static_cast<double>(slices * capacity * n) / kStreamPartialBytesPerUs;
    }
    if (cost < 0.0 || us < cost) {
      best = {GemmKind::Stream, 0, k_slice, 1};
      cost = us;
    }
  }
  return best;
}

// Tile shape and K split for a projection at `capacity` rows, from a cost model in
// microseconds.  Compute: whole rounds of one tile per CU at the shape's measured rate.
// Weights: streamed from HBM once.  The two overlap only in part (the slower counts fully,
// the faster by half).  A K split adds its fp32 partial traffic and the reduction launch;
// it fills the CUs when the tile grid is smaller than the chip (the down projection has 16
// to 32 weight tiles at H = 4096).  Fitted to forced-choice timings of the Qwen3 0.6B /
// 4B / 8B / 32B-shard projections at 32 to 4096 rows (weights streamed from HBM at the
// HBM-bound sizes), where it picks the fastest measured choice or one within 7 % of it.
constexpr double kWeightBytesPerUs = 4.5e6;   // weights streamed from HBM by the tile kernel
constexpr double kPartialBytesPerUs = 6.0e6;  // partial sums written, then read by the reduction
constexpr double kReduceLaunchUs = 4.0;
constexpr double kOverlap = 0.5;              // share of the faster of compute and streaming exposed
constexpr int64_t kMaxTileSplit = 16;

// A column split: the first n1 weight rows on shape `main` in whole rounds of one tile per
// CU, the other n - n1 on shape `tail` in a second launch, where one shape alone ends in a
// partial round (Qwen3-32B TP shard at 8192 rows: gate_up 800 tiles of 256 x 256, 3.125
// rounds).  Taken when the model prices it at least kColumnSplitGain below the best single
// shape, which keeps the choice away from near ties.
constexpr double kTailLaunchUs = 3.0;
constexpr double kColumnSplitGain = 0.05;

double tile_rounds_us(const TileShape &shape, int64_t rounds, int64_t k) {
  return static_cast<double>(rounds) * 2.0 * shape.bm * shape.bn * static_cast<double>(k) / shape.flops_per_us;
}

GemmChoice choose_tile(int64_t capacity, int64_t n, int64_t k, bool split_columns) {
  GemmChoice best{GemmKind::Tile, 0, k, 1};
  double best_cost = 0.0;
  for (int index = 0; index < kRankedTileShapes; ++index) {
    const TileShape &shape = kTileShapes[index];
    const int64_t base_tiles = ((capacity + shape.bm - 1) / shape.bm) * ((n + shape.bn - 1) / shape.bn);
    for (int64_t split = 1; split <= kMaxTileSplit; split *= 2) {
      const int64_t k_slice = ((k + split - 1) / split + 63) / 64 * 64;
      if ((split - 1) * k_slice >= k) {
        break;  // the last range would be empty
      }
      const int64_t rounds = (base_tiles * split + kComputeUnits - 1) / kComputeUnits;
      const double compute = static_cast<double>(rounds) * 2.0 * shape.bm * shape.bn *
                             static_cast<double>(k_slice) / shape.flops_per_us;
      const double stream = 2.0 * static_cast<double>(n) * static_cast<double>(k) / kWeightBytesPerUs;
      double cost = compute > stream ? compute + kOverlap * stream : stream + kOverlap * compute;
      if (split > 1) {
        cost += 8.0 * split * static_cast<double>(capacity) * static_cast<double>(n) / kPartialBytesPerUs +
                kReduceLaunchUs;
      }
      if ((index == 0 && split == 1) || cost < best_cost) {
        best = {GemmKind::Tile, index, k_slice, split};
        best_cost = cost;
      }
    }
  }
  if (!split_columns) {
    return best;
  }
  const double stream = 2.0 * static_cast<double>(n) * static_cast<double>(k) / kWeightBytesPerUs;
  GemmChoice split_best = best;
  double split_cost = best_cost * (1.0 - kColumnSplitGain);
  // The first launch runs on the 256 x 256 tile, the most efficient shape: with a 256 x 128
  // first launch the split measured slower than the best single shape (Qwen3-8B gate_up at
  // 512 rows 177 -> 186 us, the 32B shard's down at 2048 rows 228 -> 234 us per layer).
  for (int main = 0; main < 1; ++main) {
    const TileShape &shape = kTileShapes[main];
    const int64_t token_tiles = (capacity + shape.bm - 1) / shape.bm;
    for (int64_t weight_tiles = 1; weight_tiles * shape.bn < n; ++weight_tiles) {
      if ((token_tiles * weight_tiles) % kComputeUnits != 0) {
        continue;  // the first launch must be whole rounds
      }
      const int64_t n1 = weight_tiles * shape.bn;
      for (int tail = 0; tail < kRankedTileShapes; ++tail) {
        const TileShape &other = kTileShapes[tail];
        const int64_t tail_tiles = ((capacity + other.bm - 1) / other.bm) * ((n - n1 + other.bn - 1) / other.bn);
        const double compute =
            tile_rounds_us(shape, token_tiles * weight_tiles / kComputeUnits, k) +
            tile_rounds_us(other, (tail_tiles + kComputeUnits - 1) / kComputeUnits, k) + kTailLaunchUs;
        const double cost = compute > stream ? compute + kOverlap * stream : stream + kOverlap * compute;
        if (cost < split_cost) {
          split_cost = cost;
          split_best = {GemmKind::Tile, main, k, 1};
          split_best.tail_variant = tail;
          split_best.tail_columns = n - n1;
        }
      }
    }
  }
  return split_best;
}

// The resident kernel's K parts and chunks per wave at `capacity` rows (9 to 16, or 17 to
// 32 for a projection with the gather fused and at least kResidentWideMinN weight rows, on
// four token groups), with its modelled cost in microseconds (-1: not applicable).  Every workgroup streams its blocks'
// columns of its part at one workgroup's rate after a fixed prologue (launch, the token
// pieces, the first weight round trip), and the busiest workgroup sets the time; more than
// one part adds the partial sums and the reduction launch.  With the gather fused the part
// must cover K (a row's sum of squares needs every column).  Least-squares fit (relative
// error) to the kernel's durations on MI355X for the Qwen3 0.6B / 1.7B / 4B / 8B gate_up
// (gather fused) and the Qwen3 1.7B / 4B / 8B and 32B TP-shard down projections at 9 and 16
// rows, weights streamed from HBM: within 10 %.  The weight rows must fill the grid (N of at
// least 2048: a Router projection's few experts do not).
constexpr int64_t kResidentMinRows = 9;
constexpr int64_t kResidentMaxRows = 8 * kResidentGroups;
constexpr int64_t kResidentWideMaxRows = 8 * kResidentWideGroups;
constexpr int64_t kResidentMinN = 2048;
constexpr int64_t kResidentWideMinN = 16384;
constexpr double kResidentWorkgroupBytesPerUs[2] = {35.7e3, 24.8e3};  // index: gather fused
constexpr double kResidentFixedUs[2] = {7.8, 8.0};

GemmChoice choose_resident(int64_t capacity, int64_t n, int64_t k, bool gather, double &cost) {
  const bool wide = gather && capacity > kResidentMaxRows && capacity <= kResidentWideMaxRows && n >= kResidentWideMinN;
  const int groups = wide ? kResidentWideGroups : kResidentGroups;
  GemmChoice best{GemmKind::Resident, groups, 0, 0};
  cost = -1.0;
  if (capacity < kResidentMinRows || (capacity > kResidentMaxRows && !wide) || n < kResidentMinN ||
      n * k * 2 > INT32_MAX) {
    return best;
  }
  const int64_t chunks = (k + kResidentChunk - 1) / kResidentChunk;
  const int64_t row_blocks = (n + 15) / 16;
  for (int cpw = 1; cpw <= kResidentMaxChunksPerWave; ++cpw) {
    const int64_t part_chunks = static_cast<int64_t>(kResidentWaves) * cpw;
    const int64_t parts = (chunks + part_chunks - 1) / part_chunks;
    if ((gather && parts > 1) || parts > kResidentWorkgroups) {
      continue;
    }
    const int64_t walkers = std::min<int64_t>(kResidentWorkgroups / parts, row_blocks);
    const int64_t blocks = (row_blocks + walkers - 1) / walkers;
    const double columns = static_cast<double>(std::min<int64_t>(part_chunks * kResidentChunk, k));
    double us = kResidentFixedUs[gather ? 1 : 0] +
                static_cast<double>(blocks) * 16.0 * columns * 2.0 / kResidentWorkgroupBytesPerUs[gather ? 1 : 0];
    if (parts > 1) {
      us += kStreamReduceUs + 8.0 * static_cast<double>(parts * capacity * n) / kStreamPartialBytesPerUs;
    }
    if (cost < 0.0 || us < cost * (1.0 - kSplitTieMargin)) {
      best = {GemmKind::Resident, groups, part_chunks * kResidentChunk, parts};
      cost = us;
    }
  }
  return best;
}

}  // namespace

// The split or the stream kernel for a decode size, whichever the cost model prefers, and
// its modelled cost in microseconds.
GemmChoice choose_decode(int64_t capacity, int64_t n, int64_t k, double &cost) {
  const GemmChoice split = choose_split(capacity, n, k, cost);
  if (capacity <= kDecodeMaxRows) {
    double stream_us = 0.0;
    const GemmChoice stream = choose_stream(capacity, n, k, stream_us);
    if (stream_us < cost) {
      cost = stream_us;
      return stream;
    }
  }
  return split;
}

GemmChoice choose_gemm(int64_t capacity, int64_t n, int64_t k, bool gated, bool split_columns) {
  // 9 to 16 rows: the resident kernel where its model is cheaper than the split / stream
  // choice's.  Measured on MI355X (kernel durations, weights streamed from HBM): the Qwen3-32B
  // TP shard's down at 9 / 16 rows 12.8 / 13.3 us + a 4.0 us reduction (stream, 8 slices)
  // -> 12.3 / 13.2 us (one part, no reduction); Qwen3-4B and 1.7B down stay on the stream
  // kernel (resident 14.2 / 10.7 us + reduction against 12.5 / 8.5 us + reduction).
  // The split, stream and resident kernels address the weights through one 32-bit buffer range.
  if (capacity <= kDecodeMaxRows && n * k * 2 <= INT32_MAX) {
    double decode_us = 0.0;
    const GemmChoice decode = choose_decode(capacity, n, k, decode_us);
    double resident_us = 0.0;
    const GemmChoice resident = choose_resident(capacity, n, k, false, resident_us);
    return resident_us >= 0.0 && resident_us < decode_us ? resident : decode;
  }
  GemmChoice choice = choose_tile(capacity, n, k, split_columns);
  // Token tiles more than half full carry twice the MFMA work per weight byte, which the
  // two-wave tile's lower matrix rate turns into a loss once its grid passes the CU count
  // (Qwen3-8B at 64 rows: 81.2 -> 82.7 us per layer; Qwen3-0.6B at 256 rows: 30.1 -> 31.7).
  const TileShape &decode = kTileShapes[kDecodeTile];
  const int64_t decode_tiles = ((capacity + decode.bm - 1) / decode.bm) * ((n + decode.bn - 1) / decode.bn);
  const int64_t weight = capacity > decode.bm / 2 ? 2 : 1;
  if (gated && choice.variant == kDecodeTile && choice.k_split == 1 && choice.tail_variant < 0 &&
      decode_tiles * weight < kComputeUnits) {
    choice.variant = kNarrowDecodeTile;
  }
  return choice;
}

// The fused gather's prologue (slot list, full-row sums of squares, staging) runs in every
// workgroup, so the fused gate_up takes the fewest K slices that fit LDS (measured: 4
// slices of Qwen3-8B gate_up took 47 + 5 us against 38 us for one).  Up to kSplitMaxRows
// rows the split kernel can fuse the gather as well: each workgroup stages the rows' whole
// K (at most kSplitGatherMaxK columns) while its first weight chunks are in flight, which
// the model prices at kSplitGatherRoundUs per round of workgroups over the plain split
// kernel; for projections of many units, split_gathered_kernel gathers once per workgroup
// of a two-per-CU persistent grid instead.
GemmChoice choose_dense_gate_up(int64_t capacity, int64_t n, int64_t k, bool &fused) {
  // 9 to 16 rows: the resident kernel with the gather fused, wherever one part covers K.
  // Measured on MI355X (kernel durations at 9 / 16 rows, weights streamed from HBM) against
  // the choices of the decode models: Qwen3-8B 40.0 / 40.0 us (stream kernel, gather fused)
  // -> 37.9 / 38.9, Qwen3-4B 28.0 / 28.6 (the same) -> 24.0 / 24.7, Qwen3-1.7B 4.5 + 17.3 /
  // 4.6 + 19.0 (gather launch, split kernel) -> 17.1 / 17.8, Qwen3-0.6B 3.1 + 8.7 / 3.5 + 9.5
  // -> 10.0 / 10.4.
  double resident_us = 0.0;
  const GemmChoice resident = choose_resident(capacity, n, k, true, resident_us);
  if (resident_us >= 0.0) {
    fused = true;
    return resident;
  }
  fused = capacity <= kDecodeMaxRows && n * k * 2 <= INT32_MAX;
  if (!fused) {
    return choose_gemm(capacity, n, k, true);
  }
  GemmChoice fused_choice{GemmKind::Stream, 0, 0, 1};
  for (int64_t slices = 1;; ++slices) {
    const int64_t k_slice = ((k + slices - 1) / slices + kStreamSliceQuantum - 1) / kStreamSliceQuantum *
                            kStreamSliceQuantum;
    if (kStreamTokens * (k_slice + kStreamRowPad) * 2 <= kStreamLdsBytes) {
      fused_choice.k_slice = k_slice;
      break;
    }
  }
  // The fused launch streams the weights with one workgroup per 8 weight-row blocks (and K
  // slice); a separate gather launch lets the split kernel spread a small projection over
  // more workgroups (Qwen3-0.6B gate_up at one row: 48 fused workgroups, 13.6 us).
  const int64_t groups = ((n + 15) / 16 + kStreamWaves - 1) / kStreamWaves;
  const int64_t slices = stream_slices(k, fused_choice.k_slice);
  double fused_us = decode_stream_us(n, k, slices * groups, kStreamWorkgroupBytesPerUs, kStreamBytesPerUs,
                                     kStreamFixedUs) +
                    kStreamGatherUs * static_cast<double>((slices * groups + kComputeUnits - 1) / kComputeUnits);
  if (slices > 1) {
    fused_us += kStreamReduceUs + 8.0 * static_cast<double>(slices * capacity * n) / kStreamPartialBytesPerUs;
  }
  double separate_us = 0.0;
  const GemmChoice separate = choose_decode(capacity, n, k, separate_us);
  if (capacity <= kSplitGroupTokens && k <= kSplitGatherMaxK) {
    double split_us = 0.0;
    const GemmChoice split = choose_split(capacity, n, k, split_us, true);
    // The persistent variant prices as the split kernel at one row (its token pieces come
    // from LDS) plus its gather round trip, when the projection has units for every slot.
    // A reduction length of at most 128 has no K range of two chunks: choose_split then finds
    // no persistent split (k_slice 0, cost -1) and the persistent kernel is not a candidate.
    double persistent_us = 0.0;
    GemmChoice persistent = choose_split(1, n, k, persistent_us, false, true);
    const bool persistent_found = persistent.k_slice > 0 && persistent_us >= 0.0;
    persistent_us += kSplitPersistentGatherUs;
    const int64_t units = ((n + 15) / 16 * persistent.k_split + kSplitWaves - 1) / kSplitWaves;
    if (persistent_found && units >= kSplitGatheredWorkgroups && persistent_us < fused_us &&
        persistent_us < split_us && persistent_us < kGatherUs + separate_us) {
      persistent.kind = GemmKind::SplitGathered;
      return persistent;
    }
    if (split_us < fused_us && split_us <= kGatherUs + separate_us) {
      return split;  // fused into the split kernel
    }
  }
  if (kGatherUs + separate_us < fused_us) {
    fused = false;
    return separate;
  }
  return fused_choice;
}

bool split_gather_fusable(int64_t capacity, int64_t n, int64_t k) {
  const GemmChoice choice = choose_gemm(capacity, n, k, false);
  return choice.kind == GemmKind::Split && choice.variant == 1 && k <= kSplitGatherMaxK;
}

// K ranges whose fp32 partial sums go through scratch and the reduction kernel.
int64_t scratch_slices(GemmChoice choice, int64_t k) {
  switch (choice.kind) {
    case GemmKind::Stream:
      return stream_slices(k, choice.k_slice);
    case GemmKind::Tile:
    case GemmKind::Resident:
      return choice.k_split;
    default:
      return 1;  // the split kernel sums its K ranges in LDS
  }
}

size_t gemm_scratch_bytes(GemmChoice choice, int64_t capacity, int64_t n, int64_t k) {
  const int64_t slices = scratch_slices(choice, k);
  if (slices == 1) {
    return 0;
  }
  const size_t partial_bytes = static_cast<size_t>(slices * capacity * n) * sizeof(float);
  return (partial_bytes + 255) / 256 * 256;
}

hipError_t enable_large_lds(const void *func) {
  // (function, device) pairs already opted in: a few stream kernels on a few devices, kept in
  // a fixed table so that no launch path allocates.  Past its end the attribute is set again
  // on every launch (harmless, only slower).
  struct Enabled {
    const void *func;
    int device;
  };
  static std::mutex mutex;
  static Enabled enabled[128];
  static int count = 0;
  int device = 0;
  if (const hipError_t status = hipGetDevice(&device); status != hipSuccess) {
    return status;
  }
  std::lock_guard<std::mutex> guard(mutex);
  for (int index = 0; index < count; ++index) {
    if (enabled[index].func == func && enabled[index].device == device) {
      return hipSuccess;
    }
  }
  // The dynamic maximum is what the CU's 160 KB leave beside the function's static LDS (the
  // split kernel's partial sums, the fused gather's row table).
  hipFuncAttributes attributes{};
  if (const hipError_t status = hipFuncGetAttributes(&attributes, func); status != hipSuccess) {
    return status;
  }
  const int limit = 160 * 1024 - static_cast<int>(attributes.sharedSizeBytes);
  const hipError_t status = hipFuncSetAttribute(func, hipFuncAttributeMaxDynamicSharedMemorySize, limit);
  if (status == hipSuccess && count < static_cast<int>(sizeof(enabled) / sizeof(enabled[0]))) {
    enabled[count++] = Enabled{func, device};
  }
  return status;
}

GemmLaunch make_gemm(const GemmArgs &args, int64_t capacity, bool gated, GemmChoice choice, bool fused_gather) {
  GemmLaunch launches;
  KernelLaunch &kernel = launches.main;
  GemmArgs record = args;
  record.capacity = capacity;
  record.k_slice = choice.k_slice;
  record.k_split = choice.k_split;
  if ((choice.kind == GemmKind::Split || choice.kind == GemmKind::SplitGathered) &&
      (choice.k_slice <= 0 || choice.k_split <= 0)) {
    launches.usable = false;  // an empty K range would read nothing and store zeros
    return launches;
  }
  if (choice.kind == GemmKind::Split) {
    // choose_split is only consulted up to kSplitMaxRows rows (and the fused gather up to
    // one token group).
    const int64_t row_blocks = (args.n + 15) / 16;
    const int64_t per_group = kSplitWaves / choice.k_split;
    // The gather fuses into one token group (gate_up of a Dense step, the MoE router).
    const bool gather = fused_gather && choice.variant == 1;
    kernel.func = gated ? split_kernel<true>(choice.variant, gather, args.payload)
                        : split_kernel<false>(choice.variant, gather, args.payload);
    kernel.grid = dim3(static_cast<unsigned>((row_blocks + per_group - 1) / per_group), 1, 1);
    kernel.block = dim3(64 * kSplitWaves, 1, 1);
    // Dynamic LDS beyond 64 KB: launch() opts the function in (enable_large_lds).
    kernel.shmem = gather ? static_cast<unsigned>(
                                (capacity < kSplitGroupTokens ? capacity : kSplitGroupTokens) * (args.k + 16) * 2)
                          : 0u;
  } else if (choice.kind == GemmKind::SplitGathered) {
    // Chosen only for a Dense step's gate_up with the gather fused.
    const int64_t row_blocks = (args.n + 15) / 16;
    const int64_t units = (row_blocks * choice.k_split + kSplitWaves - 1) / kSplitWaves;
    kernel.func = gated ? split_gathered_kernel_ptr<true>(args.payload) : split_gathered_kernel_ptr<false>(args.payload);
    kernel.grid = dim3(static_cast<unsigned>(units < kSplitGatheredWorkgroups ? units : kSplitGatheredWorkgroups), 1, 1);
    kernel.block = dim3(64 * kSplitWaves, 1, 1);
    kernel.shmem = static_cast<unsigned>((capacity < kSplitGroupTokens ? capacity : kSplitGroupTokens) * (args.k + 16) * 2 +
                                         kSplitGatheredScratchBytes);
  } else if (choice.kind == GemmKind::Resident) {
    const int64_t row_blocks = (args.n + 15) / 16;
    const int cpw = static_cast<int>(choice.k_slice / (kResidentWaves * kResidentChunk));
    const int64_t walkers = std::min<int64_t>(kResidentWorkgroups / choice.k_split, row_blocks);
    kernel.func = resident_kernel_for(gated, fused_gather && gated, cpw, args.payload, choice.variant);
    if (kernel.func == nullptr) {
      launches.usable = false;
      return launches;
    }
    kernel.grid = dim3(static_cast<unsigned>(choice.k_split * walkers), 1, 1);
    kernel.block = dim3(64 * kResidentWaves, 1, 1);
  } else if (choice.kind == GemmKind::Stream) {
    const int64_t groups = ((args.n + 15) / 16 + kStreamWaves - 1) / kStreamWaves;
    const int64_t slices = stream_slices(args.k, choice.k_slice);
    const bool gather = fused_gather && gated;
    kernel.func = gather ? stream_kernel<true, true>(args.payload)
                         : (gated ? stream_kernel<true>(args.payload) : stream_kernel<false>(args.payload));
    kernel.grid = dim3(static_cast<unsigned>(slices * groups), 1, 1);
    kernel.block = dim3(64 * kStreamWaves, 1, 1);
    // Dynamic LDS beyond 64 KB: launch() opts the function in (enable_large_lds).
    kernel.shmem = static_cast<unsigned>(kStreamTokens * (choice.k_slice + kStreamRowPad) * 2);
  } else {
    // Tile grid over weight rows [0, n1) (all of them without a column split); the tail
    // launch takes [n1, n): its weights, and its output columns (half as many for gate_up).
    const int64_t n1 = args.n - choice.tail_columns;
    if (choice.tail_columns > 0) {
      if (choice.k_split != 1 || choice.tail_variant < 0 || n1 <= 0 || (gated && n1 % 2 != 0)) {
        launches.usable = false;
        return launches;
      }
      record.n = n1;
      const TileShape &other = kTileShapes[choice.tail_variant];
      GemmArgs tail_record = record;
      tail_record.n = choice.tail_columns;
      tail_record.w = args.w + n1 * args.k;
      tail_record.out = args.out + (gated ? n1 / 2 : n1);
      const bool tail_stream = capacity <= other.bm;
      launches.tail.func = gated ? tile_kernel<true>(choice.tail_variant, tail_stream, args.payload)
                                 : tile_kernel<false>(choice.tail_variant, tail_stream, args.payload);
      launches.tail.grid = dim3(static_cast<unsigned>((tail_record.n + other.bn - 1) / other.bn),
                                static_cast<unsigned>((capacity + other.bm - 1) / other.bm), 1);
      launches.tail.block = dim3(static_cast<unsigned>(64 * other.waves), 1, 1);
      launches.tail.set_args(tail_record);
    }
    const TileShape &shape = kTileShapes[choice.variant];
    const bool stream = capacity <= shape.bm;
    kernel.func = gated ? tile_kernel<true>(choice.variant, stream, args.payload)
                        : tile_kernel<false>(choice.variant, stream, args.payload);
    kernel.grid = dim3(static_cast<unsigned>((n1 + shape.bn - 1) / shape.bn),
                       static_cast<unsigned>((capacity + shape.bm - 1) / shape.bm),
                       static_cast<unsigned>(choice.k_split));
    kernel.block = dim3(static_cast<unsigned>(64 * shape.waves), 1, 1);
  }
  if (scratch_slices(choice, args.k) > 1) {
    launches.slices = scratch_slices(choice, args.k);
    KernelLaunch &reduce = launches.reduce;
    reduce.func = gated ? stream_reduce<true>(args.payload) : stream_reduce<false>(args.payload);
    reduce.grid = dim3(static_cast<unsigned>((capacity * (args.n / 4) + 255) / 256), 1, 1);
    reduce.block = dim3(256, 1, 1);
    reduce.set_args(record);
  }
  kernel.set_args(record);
  return launches;
}

// Grouped projections run on the tile kernel's grouped instantiations, one per expert
// tile height (choose_moe_tile picks it by routes per expert): 64 x 128 (four waves, three
// stages, 72 KB of LDS: two workgroups per CU), 128 x 256 (eight waves, three stages,
// nontemporal or plain weight loads) and 256 x 128 (eight waves, three stages, nontemporal),
// the last two at 144-147 KB of LDS, one workgroup per CU.  With few routes per expert a
// tile's K loop is short against its prologue and epilogue, and the second workgroup of a
// CU streams while the first fills or drains (Qwen3-30B-A3B layer at 256 / 512 tokens:
// 281 / 294 us on a 64 x 256 eight-wave tile with four stages, one per CU, against 255 /
// 265 us).  The nontemporal hint suits tiles whose expert's weights no other tile reads;
// with plain loads an expert split over two 128-row tiles reads its weights from the
// last-level cache the second time.
struct GroupedTile {
  int bm;
  int bn;
  int waves;
};

// The down projection (not gated) of the 128-row regimes takes 128 x 128 tiles of two
// stages (64 KB of LDS, two workgroups per CU): its K loop is short (Qwen3-30B-A3B: 768
// columns, 12 slabs), so a tile's fill and drain weigh on it, and the CU's second workgroup
// streams meanwhile.  Measured on that layer against 128 x 256 three-stage down tiles:
// 600 / 800 / 1024 tokens 306.8 / 311.6 / 319.6 -> 301.3 / 306.0 / 314.6 us, 1100 / 1400 /
// 1700 / 2048 tokens 346.3 / 350.2 / 385.1 / 396.4 -> 338.7 / 343.2 / 379.1 / 389.9 us.
// gate_up (K = 2048) lost on such tiles (2048 tokens: 410-421 against 397 us).
GroupedTile grouped_tile(MoeTile tile, bool gated) {
  switch (tile) {
    case MoeTile::Rows64:
      return {64, 128, 4};
    case MoeTile::Rows128Stream:
    case MoeTile::Rows128:
      return gated ? GroupedTile{128, 256, 8} : GroupedTile{128, 128, 8};
    case MoeTile::Rows256:
      return {256, 128, 8};
    default:
      return {0, 0, 0};
  }
}

// X: the EXTENDED epilogue (a bias or a ReLU / GELU activation), a separate instantiation so
// that the SiLU projections without bias keep their code (the general epilogue cost the
// 128-row gate_up tiles 3 % at 2048 tokens).
template <bool GATED, class P, bool X>
const void *grouped_tile_kernel(MoeTile tile) {
  switch (tile) {
    case MoeTile::Rows64:
      return reinterpret_cast<const void *>(&tile_gemm_kernel<64, 128, 2, 2, 3, GATED, true, true, P, X>);
    case MoeTile::Rows128Stream:
      return GATED ? reinterpret_cast<const void *>(&tile_gemm_kernel<128, 256, 2, 4, 3, GATED, true, true, P, X>)
                   : reinterpret_cast<const void *>(&tile_gemm_kernel<128, 128, 4, 2, 2, GATED, true, true, P, X>);
    case MoeTile::Rows128:
      return GATED ? reinterpret_cast<const void *>(&tile_gemm_kernel<128, 256, 2, 4, 3, GATED, true, false, P, X>)
                   : reinterpret_cast<const void *>(&tile_gemm_kernel<128, 128, 4, 2, 2, GATED, true, false, P, X>);
    case MoeTile::Rows256:
      return reinterpret_cast<const void *>(&tile_gemm_kernel<256, 128, 4, 2, 3, GATED, true, true, P, X>);
    default:
      return nullptr;
  }
}

template <bool GATED>
const void *grouped_tile_kernel(MoeTile tile, const GemmArgs &args) {
  const bool extended =
      args.bias != nullptr || args.act.function == kActivationRelu || args.act.function == kActivationGelu;
  if (args.payload == kPayloadF16) {
    return extended ? grouped_tile_kernel<GATED, F16Payload, true>(tile) : grouped_tile_kernel<GATED, F16Payload, false>(tile);
  }
  return extended ? grouped_tile_kernel<GATED, Bf16Payload, true>(tile) : grouped_tile_kernel<GATED, Bf16Payload, false>(tile);
}

int grouped_tile_rows(MoeTile tile) { return grouped_tile(tile, true).bm; }  // the same for down

KernelLaunch make_grouped_gemm(const GemmArgs &args, bool gated, int max_tiles, MoeTile tile) {
  const GroupedTile shape = grouped_tile(tile, gated);
  const void *func = gated ? grouped_tile_kernel<true>(tile, args) : grouped_tile_kernel<false>(tile, args);
  if (max_tiles % 8 != 0 || func == nullptr) {
    return KernelLaunch{};  // grouped_tile_coordinates needs a multiple of 8 (callers pad)
  }
  GemmArgs record = args;
  record.k_slice = args.k;
  record.k_split = 1;
  record.partials = nullptr;
  KernelLaunch kernel;
  kernel.func = func;
  kernel.grid = dim3(static_cast<unsigned>((args.n + shape.bn - 1) / shape.bn), static_cast<unsigned>(max_tiles), 1);
  kernel.block = dim3(static_cast<unsigned>(64 * shape.waves), 1, 1);
  kernel.set_args(record);
  return kernel;
}

// Routes per expert tile of the grouped split kernel: one 16-column MFMA token block.
int grouped_split_rows() { return 16; }

// Chunks in flight per wave of the grouped split kernel.  Its workgroups are short (a wave
// streams one 16-row block of one expert: 24 KB of Qwen3-30B-A3B's down projection), so
// the fixed cost of each (the tile table, the route slots, the first round trip) weighs
// more than the depth of its ring: at depth 2 the kernel takes 107 VGPRs and two
// workgroups share a CU, one streaming while the other starts or ends.  Qwen3-30B-A3B
// layer at 8 / 32 / 64 tokens: 121.5 / 215.7 / 238.1 us at depth 4 (160 VGPRs, one
// workgroup per CU), 115.0 / 201.2 / 223.3 at depth 2; depth 3 (128 VGPRs, two per CU, and
// chunk counts that do not divide into its groups) 122.4 / 217.0 / 238.7.
constexpr int kGroupedSplitDepth = 2;

// K ranges per weight block: the most (1, 2, 4 or 8) that keep the expected live tiles'
// workgroups within one round of one per CU, with every range at least two 128-wide chunks
// long.  A workgroup at decode sizes is latency-bound (the tile table, the route slots,
// then the weights and tokens, each a memory round trip), so a second round of
// workgroups costs nearly as much as the first (Qwen3-30B-A3B gate_up at 1 token: 384
// workgroups in two rounds 17.8 us).
KernelLaunch make_grouped_split(const GemmArgs &args, bool gated, int max_tiles, int64_t live_tiles) {
  const int64_t row_blocks = (args.n + 15) / 16;
  const int64_t chunks = (args.k + 127) / 128;
  auto nonempty = [&](int64_t ranges) { return (ranges - 1) * ((chunks + ranges - 1) / ranges) < chunks; };
  auto workgroups = [&](int64_t ranges) { return (row_blocks * ranges + kSplitWaves - 1) / kSplitWaves * live_tiles; };
  int64_t ksplit = 1;
  while (ksplit < kSplitWaves && 4 * ksplit <= chunks && nonempty(2 * ksplit) &&
         workgroups(2 * ksplit) <= kComputeUnits) {
    ksplit *= 2;
  }
  GemmArgs record = args;
  record.k_split = ksplit;
  record.k_slice = (chunks + ksplit - 1) / ksplit * 128;
  record.partials = nullptr;
  KernelLaunch kernel;
  if (args.payload == kPayloadF16) {
    kernel.func = gated ? reinterpret_cast<const void *>(&grouped_split_kernel<kGroupedSplitDepth, true, F16Payload>)
                        : reinterpret_cast<const void *>(&grouped_split_kernel<kGroupedSplitDepth, false, F16Payload>);
  } else {
    kernel.func = gated ? reinterpret_cast<const void *>(&grouped_split_kernel<kGroupedSplitDepth, true>)
                        : reinterpret_cast<const void *>(&grouped_split_kernel<kGroupedSplitDepth, false>);
  }
  kernel.grid = dim3(static_cast<unsigned>((row_blocks * ksplit + kSplitWaves - 1) / kSplitWaves),
                     static_cast<unsigned>(max_tiles), 1);
  kernel.block = dim3(64 * kSplitWaves, 1, 1);
  kernel.set_args(record);
  return kernel;
}

std::string gemm_name(GemmChoice choice, bool gated) {
  const std::string prefix = gated ? "_gated" : "";
  if (choice.kind == GemmKind::Split) {
    return "split" + prefix + "_t" + std::to_string(kSplitGroupTokens * choice.variant) + "_k" +
           std::to_string(choice.k_split);
  }
  if (choice.kind == GemmKind::SplitGathered) {
    return "split" + prefix + "_t8_k" + std::to_string(choice.k_split) + "_persistent";
  }
  if (choice.kind == GemmKind::Stream) {
    return "stream" + prefix + "_t16";
  }
  if (choice.kind == GemmKind::Resident) {
    std::string name = "resident" + prefix + "_t" + std::to_string(8 * choice.variant) + "_c" +
                       std::to_string(choice.k_slice / (kResidentWaves * kResidentChunk));
    if (choice.k_split > 1) {
      name += "_p" + std::to_string(choice.k_split);
    }
    return name;
  }
  const TileShape &shape = kTileShapes[choice.variant];
  std::string name = "tile" + prefix + "_" + std::to_string(shape.bm) + "x" + std::to_string(shape.bn);
  if (choice.k_split > 1) {
    name += "_k" + std::to_string(choice.k_split);
  }
  if (choice.tail_columns > 0) {
    const TileShape &other = kTileShapes[choice.tail_variant];
    name += "+" + std::to_string(other.bm) + "x" + std::to_string(other.bn) + "_n" + std::to_string(choice.tail_columns);
  }
  return name;
}

}  // namespace xp
