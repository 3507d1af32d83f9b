// Shared device/host helpers for the CDNA4 (gfx950) FfnAgent kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace xp {

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f32x2 = float __attribute__((ext_vector_type(2)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Fault bits raised by kernels into a caller-provided device word.  The word is
// sticky: kernels only OR bits in, the host clears it explicitly.
constexpr uint32_t kFaultSlotOutOfRange = 1u;

__device__ __forceinline__ float bf16_to_float(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16, round to nearest even on the gfx950 converter (v_cvt_pk_bf16_f32); NaNs
// stay NaN.
__device__ __forceinline__ uint32_t float_to_bf16(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
}

// Round through bf16 and back: the payload-dtype rounding point of the
// reference's projection epilogue.
__device__ __forceinline__ float round_bf16(float value) { return bf16_to_float(float_to_bf16(value)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// Gated activation parameters: silu(min(g, limit)) * (clamp(u, -limit, limit) + up_offset),
// with silu(v) = v / (1 + exp(-alpha v)); limit <= 0 disables clipping.  The grouped MoE
// projections also take ReLU and GELU in place of SiLU (function: kActivationRelu /
// kActivationGelu; anything else is SiLU).
struct GatedSilu {
  float alpha;
  float limit;
  float up_offset;
  int32_t function;
  int32_t approximate_tanh;  // GELU: the tanh approximation instead of erf
};

// The projection is first rounded to bf16 (payload dtype), then evaluated in fp32.  CLIP is
// whether the gate transform clips (act.limit > 0), fixed at compile time so that tile
// epilogues without a limit carry no clamp or select per element; both bf16 roundings come
// from one packed conversion.
template <bool CLIP>
__device__ __forceinline__ float gated_silu_fixed(float gate, float up, const GatedSilu &act) {
  const uint32_t both = pack_bf16x2(gate, up);
  float g = __uint_as_float(both << 16);
  float u = __uint_as_float(both & 0xffff0000u);
  if constexpr (CLIP) {
    g = fminf(g, act.limit);
    u = fminf(fmaxf(u, -act.limit), act.limit);
  }
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-act.alpha * g)) * (u + act.up_offset);
}

__device__ __forceinline__ float gated_silu(float gate, float up, const GatedSilu &act) {
  float g = round_bf16(gate);
  float u = round_bf16(up);
  if (act.limit > 0.0f) {
    g = fminf(g, act.limit);
    u = fminf(fmaxf(u, -act.limit), act.limit);
  }
  // silu(g) = g / (1 + exp(-alpha g)) with the reciprocal instruction (1 ulp) instead of an
  // IEEE divide; exp overflow gives 1 / inf = 0, the limit of the quotient.
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-act.alpha * g)) * (u + act.up_offset);
}

// ------------------------------------------------------------------ payload dtypes
// The 16-bit float of a Dense layer's mailbox, weights and activations: bf16 or fp16 (the
// reference admits both, ffn.hpp:83-85).  Kernels take the payload as a template argument;
// everything dtype-specific goes through these: the widening of one 16-bit pattern, the
// round-to-nearest-even packing of two fp32 values, the quiet-NaN fill of a failed row
// (static_cast<Scalar>(NAN), instance.cu:28-31) and the MFMA tiles of the projections.
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));

struct Bf16Payload {
  static constexpr uint32_t kPoison2 = 0x7fc07fc0u;  // two bf16 quiet NaNs
  __device__ static __forceinline__ float widen(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
  }
  __device__ static __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

// An fp32 value at a rounding point, made opaque to the compiler before it is converted to
// fp16.  Without it the backend may fuse the multiply that produced the value into the
// conversion (v_fma_mix*_f16), which rounds the exact product to fp16 once instead of
// rounding it to fp32 first, as the reference (an fp32 product, then .to(float16)) does; at
// an fp16 tie the two results differ by one ulp.  (bf16 has no such fused form.)
__device__ __forceinline__ float f32_rounding_point(float value) {
  __asm__ volatile("" : "+v"(value));
  return value;
}

struct F16Payload {
  static constexpr uint32_t kPoison2 = 0x7e007e00u;  // two fp16 quiet NaNs
  __device__ static __forceinline__ float widen(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                            (f32x2_t{f32_rounding_point(lo), f32_rounding_point(hi)}), f16x2_t));
  }
  __device__ static __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ static __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
};

// Round through the payload dtype and back (the projection's rounding point).
template <class P>
__device__ __forceinline__ float round_payload(float value) {
  return P::widen(P::pack2(value, 0.0f) & 0xffffu);
}

// gated_silu_fixed / gated_silu with the rounding point in payload P.
template <class P, bool CLIP>
__device__ __forceinline__ float gated_silu_payload(float gate, float up, const GatedSilu &act) {
  const uint32_t both = P::pack2(gate, up);
  float g = P::widen(both & 0xffffu);
  float u = P::widen(both >> 16);
  if constexpr (CLIP) {
    g = fminf(g, act.limit);
    u = fminf(fmaxf(u, -act.limit), act.limit);
  }
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-act.alpha * g)) * (u + act.up_offset);
}

template <class P>
__device__ __forceinline__ float gated_silu_payload(float gate, float up, const GatedSilu &act) {
  return act.limit > 0.0f ? gated_silu_payload<P, true>(gate, up, act) : gated_silu_payload<P, false>(gate, up, act);
}

__device__ __forceinline__ u32x4 load16(const void *address) {
  return *reinterpret_cast<const u32x4 *>(address);
}

__device__ __forceinline__ u32x4 load16_stream(const void *address) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(address));
}

__device__ __forceinline__ void store16(void *address, u32x4 value) { *reinterpret_cast<u32x4 *>(address) = value; }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 value) { return __builtin_bit_cast(bf16x8, value); }

// Raw buffer resource over `bytes` bytes: loads past the end return zero without a memory
// access, which masks token rows beyond the live rows and weight rows beyond N without
// branches.  Word 3 is the gfx9 raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

template <int POLICY = 0>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset), 0, POLICY));
}

// Cache-policy bits of a buffer load: 2 is the nontemporal hint (`nt`), for data read once
// in whole 128-byte lines (the tile kernel's weight tiles).  Measured on MI355X: a 4 GiB
// read reaches 6.1-6.3 TB/s with plain loads and 6.8-7.1 TB/s with nontemporal ones.  The
// split and stream kernels read each line as two 64-byte halves in consecutive
// instructions; with the hint their decode layers took 10-12 us longer (the second half no
// longer found in L2), so they load plainly.
constexpr int kLoadNontemporal = 2;

__device__ __forceinline__ float wave_sum(float value) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    value += __shfl_xor(value, offset, kWave);
  }
  return value;
}

// RMSNorm of gathered mailbox rows, shared by the gather kernel and the gather fused into
// the decode projection so that both produce the same bits.  One wavefront takes a row's
// sum of squares, lane i over its 16-byte chunks i, i + 64, ... in that order (add_squares),
// reduced with wave_sum (rms_inverse); each element becomes bf16((x * inverse) * w).
template <class P = Bf16Payload>
__device__ __forceinline__ void add_squares(u32x4 chunk, float &squares) {
#pragma unroll
  for (int word = 0; word < 4; ++word) {
    const float lo = P::widen(chunk[word] & 0xffffu);
    const float hi = P::widen(chunk[word] >> 16);
    squares += lo * lo;
    squares += hi * hi;
  }
}

__device__ __forceinline__ float rms_inverse(float lane_squares, int64_t hidden, float eps) {
  const float squares = wave_sum(lane_squares);
  return 1.0f / sqrtf(squares / static_cast<float>(hidden) + eps);
}

template <class P = Bf16Payload>
__device__ __forceinline__ u32x4 normalize_chunk(u32x4 x, float inverse, u32x4 weight) {
  u32x4 result;
#pragma unroll
  for (int word = 0; word < 4; ++word) {
    const float lo = P::widen(x[word] & 0xffffu) * inverse;
    const float hi = P::widen(x[word] >> 16) * inverse;
    result[word] = P::pack2(lo * P::widen(weight[word] & 0xffffu), hi * P::widen(weight[word] >> 16));
  }
  return result;
}

// A gathered row whose slot is out of range reads as quiet NaNs (two bf16 per word).
constexpr uint32_t kPoisonBf16x2 = 0x7fc07fc0u;

__device__ __forceinline__ void raise_fault(uint32_t *fault, uint32_t bits) {
  if (fault != nullptr) {
    __hip_atomic_fetch_or(fault, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace xp
