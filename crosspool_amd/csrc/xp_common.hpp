// Shared device/host helpers for the CDNA4 (gfx950) FfnAgent kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace xp {

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Fault bits raised by kernels into a caller-provided device word.  The word is
// sticky: kernels only OR bits in, the host clears it explicitly.
constexpr uint32_t kFaultSlotOutOfRange = 1u;

__device__ __forceinline__ float bf16_to_float(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round-to-nearest-even fp32 -> bf16; NaN stays a quiet NaN of the same sign.
__device__ __forceinline__ uint32_t float_to_bf16(float value) {
  uint32_t bits = __float_as_uint(value);
  if ((bits & 0x7fffffffu) > 0x7f800000u) {
    return (bits >> 16) | 0x0040u;
  }
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return bits >> 16;
}

// Round through bf16 and back: the payload-dtype rounding point of the
// reference's projection epilogue.
__device__ __forceinline__ float round_bf16(float value) { return bf16_to_float(float_to_bf16(value)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return float_to_bf16(lo) | (float_to_bf16(hi) << 16);
}

// Gated activation parameters: silu(min(g, limit)) * (clamp(u, -limit, limit) + up_offset),
// with silu(v) = v / (1 + exp(-alpha v)); limit <= 0 disables clipping.
struct GatedSilu {
  float alpha;
  float limit;
  float up_offset;
};

// The projection is first rounded to bf16 (payload dtype), then evaluated in fp32.
__device__ __forceinline__ float gated_silu(float gate, float up, const GatedSilu &act) {
  float g = round_bf16(gate);
  float u = round_bf16(up);
  if (act.limit > 0.0f) {
    g = fminf(g, act.limit);
    u = fminf(fmaxf(u, -act.limit), act.limit);
  }
  return g / (1.0f + __expf(-act.alpha * g)) * (u + act.up_offset);
}

__device__ __forceinline__ u32x4 load16(const void *address) {
  return *reinterpret_cast<const u32x4 *>(address);
}

__device__ __forceinline__ u32x4 load16_stream(const void *address) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(address));
}

__device__ __forceinline__ void store16(void *address, u32x4 value) { *reinterpret_cast<u32x4 *>(address) = value; }

__device__ __forceinline__ float wave_sum(float value) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    value += __shfl_xor(value, offset, kWave);
  }
  return value;
}

__device__ __forceinline__ void raise_fault(uint32_t *fault, uint32_t bits) {
  if (fault != nullptr) {
    __hip_atomic_fetch_or(fault, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Map a linear workgroup id so that consecutive logical tiles land on the same
// XCD.  Workgroups are dispatched round-robin over the 8 XCDs of an MI355X, so
// workgroup b runs on XCD b % 8; the returned id enumerates tiles XCD-major.
__device__ __forceinline__ int xcd_major_tile(int block, int blocks) {
  constexpr int kXcds = 8;
  const int xcd = block % kXcds;
  const int index = block / kXcds;
  const int per = blocks / kXcds;
  const int extra = blocks % kXcds;
  return xcd < extra ? xcd * (per + 1) + index : extra * (per + 1) + (xcd - extra) * per + index;
}

}  // namespace xp
