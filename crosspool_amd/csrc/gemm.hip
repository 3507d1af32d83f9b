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
// Two kernel families, chosen per GraphTemplate capacity:
//  * skinny (capacity <= 64, HBM-bound): weight rows are the MFMA M operand
//    (v_mfma_f32_16x16x32_bf16), each lane streams 64 contiguous bytes of one
//    weight row per 128-wide K chunk, the few token rows are the N operand
//    and come from L2.  A workgroup splits K across its waves and reduces the
//    partial tiles through LDS in a fixed order (deterministic).  A Gate/Up
//    pair lands in one lane's accumulator registers, so the SiLU epilogue
//    needs no data exchange.
//  * tile (capacity > 64, MFMA-bound): BMxBN block tiles, BK = 64, four waves
//    (2x2) each owning a (BM/2)x(BN/2) tile of v_mfma_f32_32x32x16_bf16
//    accumulators, register-staged global loads double-buffered through LDS
//    with an XOR swizzle of 16-byte chunks (conflict-free ds_read_b128), and
//    an XCD-major tile order for L2 reuse.  For gate_up the weight tile is
//    permuted while staging so that a wave's Gate and Up columns for the same
//    j sit in the same lane and register.

#include "xp_kernels.hpp"

namespace xp {
namespace {

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 value) { return __builtin_bit_cast(bf16x8, value); }

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

// ------------------------------------------------------------------ skinny
template <int TB, int WAVES, bool GATED>
__global__ __launch_bounds__(WAVES * 64) void skinny_gemm_kernel(GemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;

  const int64_t wn = n0 + r16;
  const bool w_ok = wn < a.n;
  const uint16_t *w_row = a.w + (w_ok ? wn : 0) * a.k + kq * 32;
  const uint16_t *x_row[TB];
  bool x_ok[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int64_t token = tb * 16 + r16;
    x_ok[tb] = token < a.rows;
    x_row[tb] = a.x + (x_ok[tb] ? token : 0) * a.ldx + kq * 32;
  }

  f32x4 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    acc[tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const int64_t chunks = (a.k + 127) >> 7;
  const bool whole = (a.k & 127) == 0;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  u32x4 wf[4], xf[TB][4];
  auto load_chunk = [&](int64_t chunk, u32x4 (&w)[4], u32x4 (&x)[TB][4]) {
    const int64_t kb = chunk * 128;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bool k_ok = whole || (kb + kq * 32 + s * 8 < a.k);
      w[s] = (w_ok && k_ok) ? load16_stream(w_row + kb + s * 8) : zero;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        x[tb][s] = (x_ok[tb] && k_ok) ? load16(x_row[tb] + kb + s * 8) : zero;
      }
    }
  };

  int64_t chunk = wave;
  if (chunk < chunks) {
    load_chunk(chunk, wf, xf);
  }
  for (; chunk < chunks; chunk += WAVES) {
    u32x4 wn_[4], xn_[TB][4];
    const bool more = chunk + WAVES < chunks;
    if (more) {
      load_chunk(chunk + WAVES, wn_, xn_);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        acc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[s]), as_bf16x8(xf[tb][s]), acc[tb], 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        wf[s] = wn_[s];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          xf[tb][s] = xn_[tb][s];
        }
      }
    }
  }

  // Fixed-order reduction of the K-split partial tiles.
  __shared__ float partial[WAVES > 1 ? WAVES : 1][TB * 4][64];
  if constexpr (WAVES > 1) {
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        partial[wave][tb * 4 + i][lane] = acc[tb][i];
      }
    }
    __syncthreads();
  }
  for (int tb = (WAVES > 1 ? wave : 0); tb < TB; tb += WAVES) {
    f32x4 sum;
    if constexpr (WAVES > 1) {
      sum = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int w = 0; w < WAVES; ++w) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sum[i] += partial[w][tb * 4 + i][lane];
        }
      }
    } else {
      sum = acc[tb];
    }
    const int64_t token = tb * 16 + r16;
    const int64_t n = n0 + 4 * kq;  // this lane holds weight rows n .. n+3
    if (token >= a.rows || n >= a.n) {
      continue;
    }
    uint16_t *row = output_row(a, token);
    if (row == nullptr) {
      continue;
    }
    if constexpr (GATED) {
      const float h0 = gated_silu(sum[0], sum[1], a.act);
      const float h1 = gated_silu(sum[2], sum[3], a.act);
      *reinterpret_cast<uint32_t *>(row + n / 2) = pack_bf16x2(h0, h1);
    } else {
      u32x2 packed = {pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3])};
      *reinterpret_cast<u32x2 *>(row + n) = packed;
    }
  }
}

// ------------------------------------------------------------------ tile
// Raw buffer resource over `bytes` bytes: loads past the end return zero, which
// masks rows beyond the live rows (activations) or beyond N (weights) without
// branches.  Word 3 is the gfx9 raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset), 0, 0));
}

using lds_void_t = __attribute__((address_space(3))) void *;

// Direct global -> LDS load of 16 bytes per lane through a buffer resource: lane i's
// data lands at `lds_row_base + 16 i`; offsets past the resource's end write zeros.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds_base, uint32_t voffset,
                                                  uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t)(lds_base), 16, static_cast<int>(voffset),
                                           static_cast<int>(soffset), 0, 0);
}

// LDS tiles are rows of 64 bf16 (128 bytes = eight 16-byte chunks).  gfx950 serves
// ds_read_b128 sixteen lanes at a time from a 256-byte bank line, i.e. two tile rows, so
// the 16 rows one MFMA fragment read touches must occupy 16 distinct 16-byte slots:
// logical chunk c of row r is stored at physical chunk c ^ ((r / 2) % 8).
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

// s_waitcnt with vmcnt <= N and the LDS / export counters left unconstrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Offset that is always past a tile resource's end (resources stay below 2^31 bytes).
constexpr uint32_t kOutOfRange = 0x7ffffff0u;

// BM x BN block tile, BK = 64, WAVES_M x WAVES_N waves (two per SIMD at 8 waves) each
// owning a (BM / WAVES_M) x (BN / WAVES_N) tile of 32x32x16 MFMA accumulators.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool GATED>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void tile_gemm_kernel(GemmArgs a) {
  constexpr int BK = 64;
  constexpr int WAVES = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M;
  constexpr int WTN = BN / WAVES_N;
  constexpr int MT = WTM / 32;
  constexpr int NT = WTN / 32;
  constexpr int ROWS = BM + BN;                    // LDS rows per stage (A rows then B rows)
  constexpr int STAGE = ROWS * BK;                 // bf16 elements per stage
  constexpr int LOADS = ROWS / 8 / WAVES;          // 1 KB (8-row) load instructions per wave per stage
  static_assert(MT >= 1 && NT >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  static_assert(!GATED || NT % 2 == 0, "gated tiles need whole Gate/Up column groups per wave");
  static_assert(ROWS % (8 * WAVES) == 0, "stage rows must split evenly over the waves");
  static_assert(BM % 8 == 0, "8-row load groups must not straddle the A/B boundary");

  __shared__ __attribute__((aligned(1024))) uint16_t lds[2 * STAGE];

  const int tiles_m = static_cast<int>((a.capacity + BM - 1) / BM);
  const int tile = xcd_major_tile(blockIdx.x, gridDim.x);
  const int tm = tile % tiles_m;
  const int tn = tile / tiles_m;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  if (m0 >= a.rows) {
    return;
  }
  const int64_t w0 = static_cast<int64_t>(tn) * BN;

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep it (and the load
  // descriptors and LDS bases derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wm = wave % WAVES_M;
  const int wn = wave / WAVES_M;

  // ---- loads: wave `wave` fills stage rows [wave * 8 * LOADS, +8 * LOADS).  Lane i of a load
  // writes LDS row r0 + i / 8, physical chunk i % 8, which holds logical k chunk
  // (i % 8) ^ swizzle(row): the swizzle is applied by choosing the global chunk.
  const int64_t a_rows_left = a.rows - m0;
  const int64_t b_rows_left = a.n - w0;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_rsrc(a.x + m0 * a.ldx, static_cast<uint32_t>((a_rows_left < BM ? a_rows_left : BM) * a.ldx * 2));
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(a.w + w0 * a.k, static_cast<uint32_t>((b_rows_left < BN ? b_rows_left : BN) * a.k * 2));
  const int first_row = wave * 8 * LOADS;
  const int row_in_load = lane >> 3;
  uint32_t load_offset[LOADS];
  bool load_is_a[LOADS];
  int load_chunk[LOADS];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) {
    const int group_row = first_row + q * 8;  // 8-row groups never straddle the A/B boundary
    const int row = group_row + row_in_load;
    const int k_chunk = (lane & 7) ^ swizzle(row);
    load_chunk[q] = k_chunk;
    load_is_a[q] = group_row < BM;
    if (load_is_a[q]) {
      load_offset[q] = static_cast<uint32_t>((row * a.ldx + k_chunk * 8) * 2);
    } else {
      const int p = row - BM;  // LDS row within the B tile
      int rr = p;              // weight row within the tile
      if constexpr (GATED) {
        // LDS row p = wq * (BN / WAVES_N) + s * (BN / WAVES_N / 2) + jj holds Gate (s = 0) or Up
        // (s = 1) of j = wq * (BN / WAVES_N / 2) + jj, i.e. weight row 2 j + s.
        constexpr int group = BN / WAVES_N;
        const int wq = p / group;
        const int s = (p % group) / (group / 2);
        const int jj = p % (group / 2);
        rr = 2 * (wq * (group / 2) + jj) + s;
      }
      load_offset[q] = static_cast<uint32_t>((rr * a.k + k_chunk * 8) * 2);
    }
  }
  const bool k_whole = (a.k % BK) == 0;
  auto issue_loads = [&](int64_t kt, int stage) {
    const uint32_t k_bytes = static_cast<uint32_t>(kt * BK * 2);
    uint16_t *base = lds + stage * STAGE + first_row * BK;
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const bool k_ok = k_whole || (kt * BK + load_chunk[q] * 8 < a.k);
      // The scalar offset must stay wave-uniform; masking goes through the per-lane offset
      // (kOutOfRange + k_bytes is still past the resource end).
      buffer_load_lds16(load_is_a[q] ? a_rsrc : b_rsrc, base + q * 8 * BK, k_ok ? load_offset[q] : kOutOfRange,
                        k_bytes);
    }
  };

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

  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  bf16x8 af[2][MT];
  bf16x8 bfrag[2][NT];
  auto read_fragments = [&](int stage, int ks, int slot) {
    const uint16_t *as = lds + stage * STAGE;
    const uint16_t *bs = as + BM * BK;
    const int chunk = ks * 2 + frag_half;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = wm * WTM + mt * 32 + frag_row;
      af[slot][mt] = as_bf16x8(load16(as + row * BK + ((chunk ^ swizzle(row)) << 3)));
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = wn * WTN + nt * 32 + frag_row;
      bfrag[slot][nt] = as_bf16x8(load16(bs + row * BK + ((chunk ^ swizzle(row)) << 3)));
    }
  };
  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][mt], bfrag[slot][nt], acc[mt][nt], 0, 0, 0);
      }
    }
  };

  // Prologue: tiles 0 and 1 in flight, wait for tile 0, read its first fragments.
  const int64_t ktiles = (a.k + BK - 1) / BK;
  issue_loads(0, 0);
  if (ktiles > 1) {
    issue_loads(1, 1);
    wait_vmcnt<LOADS>();  // tile 0 landed; tile 1 may still be in flight
  }
  __syncthreads();
  read_fragments(0, 0, 0);

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int stage = static_cast<int>(kt & 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) {
        read_fragments(stage, ks + 1, (ks + 1) & 1);
      }
      mfma_step(ks & 1);
    }
    if (kt + 1 < ktiles) {
      // Tile kt+1 (our loads) has landed; after the barrier everyone's has, and nobody reads
      // this stage any more, so tile kt+2 may refill it.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (kt + 2 < ktiles) {
        issue_loads(kt + 2, stage);
      }
      read_fragments(stage ^ 1, 0, 0);
    }
  }

  // Epilogue: lane holds D[8 (r / 4) + 4 (lane / 32) + r % 4][lane % 32] of each 32x32 tile.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t token = m0 + wm * WTM + mt * 32 + 8 * (r >> 2) + 4 * frag_half + (r & 3);
      if (token >= a.rows) {
        continue;
      }
      uint16_t *row = output_row(a, token);
      if (row == nullptr) {
        continue;
      }
      if constexpr (GATED) {
#pragma unroll
        for (int nt = 0; nt < NT / 2; ++nt) {
          const int64_t j = w0 / 2 + wn * (WTN / 2) + nt * 32 + frag_row;
          if (2 * j < a.n) {
            row[j] = static_cast<uint16_t>(float_to_bf16(gated_silu(acc[mt][nt][r], acc[mt][nt + NT / 2][r], a.act)));
          }
        }
      } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t n = w0 + wn * WTN + nt * 32 + frag_row;
          if (n < a.n) {
            row[n] = static_cast<uint16_t>(float_to_bf16(acc[mt][nt][r]));
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ tables
struct SkinnyShape {
  int token_blocks;  // 16-token MFMA column blocks (capacity <= 16 * token_blocks)
  int waves;         // K-split waves per workgroup
};
// 64-token tiles stop at 8 waves: 16 waves would cap a 1024-thread workgroup at
// 128 VGPRs and spill.
constexpr SkinnyShape kSkinnyShapes[] = {
    {1, 4}, {1, 8}, {1, 16}, {2, 4}, {2, 8}, {2, 16}, {4, 4}, {4, 8},
};
constexpr int kSkinnyShapeCount = sizeof(kSkinnyShapes) / sizeof(kSkinnyShapes[0]);

template <bool GATED>
const void *skinny_kernel(int variant) {
  using Kernel = void (*)(GemmArgs);
  static const Kernel table[] = {
      &skinny_gemm_kernel<1, 4, GATED>, &skinny_gemm_kernel<1, 8, GATED>, &skinny_gemm_kernel<1, 16, GATED>,
      &skinny_gemm_kernel<2, 4, GATED>, &skinny_gemm_kernel<2, 8, GATED>, &skinny_gemm_kernel<2, 16, GATED>,
      &skinny_gemm_kernel<4, 4, GATED>, &skinny_gemm_kernel<4, 8, GATED>,
  };
  static_assert(sizeof(table) / sizeof(table[0]) == kSkinnyShapeCount, "skinny table mismatch");
  return reinterpret_cast<const void *>(table[variant]);
}

struct TileShape {
  int bm;
  int bn;
  int waves;
  int per_cu;       // resident workgroups per CU (LDS-limited)
  double quality;   // relative per-CU efficiency of the tile shape
};
constexpr TileShape kTileShapes[] = {
    {256, 256, 8, 1, 1.00},
    {256, 128, 8, 1, 0.90},
    {128, 128, 4, 2, 0.80},
};

template <bool GATED>
const void *tile_kernel(int variant) {
  using Kernel = void (*)(GemmArgs);
  static const Kernel table[] = {
      &tile_gemm_kernel<256, 256, 2, 4, GATED>,
      &tile_gemm_kernel<256, 128, 4, 2, GATED>,
      &tile_gemm_kernel<128, 128, 2, 2, GATED>,
  };
  return reinterpret_cast<const void *>(table[variant]);
}

constexpr int kComputeUnits = 256;

}  // namespace

GemmChoice choose_gemm(int64_t capacity, int64_t n, int64_t k, bool gated) {
  (void)gated;
  if (capacity <= 64) {
    const int token_blocks = capacity <= 16 ? 1 : (capacity <= 32 ? 2 : 4);
    const int64_t blocks = (n + 15) / 16;
    const int64_t chunks = (k + 127) / 128;
    // Fewest K-split waves that still put >= 4096 waves in flight, without
    // leaving a wave fewer than four 128-wide K chunks.
    int chosen = -1;
    for (int index = 0; index < kSkinnyShapeCount; ++index) {
      const SkinnyShape &shape = kSkinnyShapes[index];
      if (shape.token_blocks != token_blocks) {
        continue;
      }
      chosen = index;
      if (blocks * shape.waves >= 4096 || chunks < 4 * shape.waves * 2) {
        break;
      }
    }
    return {GemmKind::Skinny, chosen};
  }
  int best = 0;
  double best_cost = 0.0;
  for (int index = 0; index < 3; ++index) {
    const TileShape &shape = kTileShapes[index];
    const int64_t tiles = ((capacity + shape.bm - 1) / shape.bm) * ((n + shape.bn - 1) / shape.bn);
    const int64_t slots = static_cast<int64_t>(kComputeUnits) * shape.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    // A round runs `per_cu` co-resident tiles on each CU, sharing its MFMA pipes.
    const double cost = static_cast<double>(rounds) * shape.per_cu * shape.bm * shape.bn / shape.quality;
    if (index == 0 || cost < best_cost) {
      best = index;
      best_cost = cost;
    }
  }
  return {GemmKind::Tile, best};
}

KernelLaunch make_gemm(const GemmArgs &args, int64_t capacity, bool gated, GemmChoice choice) {
  KernelLaunch kernel;
  if (choice.kind == GemmKind::Skinny) {
    const int waves = kSkinnyShapes[choice.variant].waves;
    kernel.func = gated ? skinny_kernel<true>(choice.variant) : skinny_kernel<false>(choice.variant);
    kernel.grid = dim3(static_cast<unsigned>((args.n + 15) / 16), 1, 1);
    kernel.block = dim3(static_cast<unsigned>(waves * 64), 1, 1);
  } else {
    const TileShape &shape = kTileShapes[choice.variant];
    kernel.func = gated ? tile_kernel<true>(choice.variant) : tile_kernel<false>(choice.variant);
    const int64_t tiles = ((capacity + shape.bm - 1) / shape.bm) * ((args.n + shape.bn - 1) / shape.bn);
    kernel.grid = dim3(static_cast<unsigned>(tiles), 1, 1);
    kernel.block = dim3(static_cast<unsigned>(64 * shape.waves), 1, 1);
  }
  GemmArgs record = args;
  record.capacity = capacity;
  kernel.set_args(record);
  return kernel;
}

const char *gemm_name(GemmChoice choice, bool gated) {
  static const char *skinny_names[2][kSkinnyShapeCount] = {
      {"skinny_t16_w4", "skinny_t16_w8", "skinny_t16_w16", "skinny_t32_w4", "skinny_t32_w8", "skinny_t32_w16",
       "skinny_t64_w4", "skinny_t64_w8"},
      {"skinny_gated_t16_w4", "skinny_gated_t16_w8", "skinny_gated_t16_w16", "skinny_gated_t32_w4",
       "skinny_gated_t32_w8", "skinny_gated_t32_w16", "skinny_gated_t64_w4", "skinny_gated_t64_w8"},
  };
  static const char *tile_names[2][3] = {
      {"tile_256x256", "tile_256x128", "tile_128x128"},
      {"tile_gated_256x256", "tile_gated_256x128", "tile_gated_128x128"},
  };
  return choice.kind == GemmKind::Skinny ? skinny_names[gated][choice.variant] : tile_names[gated][choice.variant];
}

}  // namespace xp
