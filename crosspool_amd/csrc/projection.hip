// General projections and the standalone activation: the FfnAgent operator cases that the
// bf16 MFMA kernels of gemm.hip do not take.
//
// Reference behaviour (CrossPool checkout):
//  * Gemm.run_into (src/xpool/runtime/ffnagent/operators/linear.py:163-257) with the
//    projection epilogue of operators/activation.py:112-173 and the IEEE kernels of
//    operators/simt.py:13-80: value = fp32 sum of x . w + the fp32 bias; with a fused
//    activation the value is first rounded to the payload dtype (projection_round_dtype,
//    linear.py:56-60), then activated in fp32 (gated: Gate/Up INTERLEAVED, Gate clipped above
//    at the limit, Up clamped to +-limit, plus up_offset); the store rounds to the output
//    dtype.
//  * activation_kernel / Activation.apply_into (operators/activation.py:55-84, 175-207):
//    the same activation over already-projected values, gated (INTERLEAVED or CONCATENATED)
//    or not; an ungated activation may run in place.  ReLU keeps NaN payloads and maps
//    every other non-positive value to +0 (activation.py:19-27).
//
// Payloads are bf16, fp16 or fp32 (activations: bf16 or fp16), any K and N, rows of any
// alignment: every element is loaded on its own, so these kernels are for the shapes, dtypes
// and biases of the reference's operator contract, not for the Qwen3 hot path (bf16, no bias,
// SiLU, aligned), which gemm.hip serves.

#include "xp_kernels.hpp"

#include <hip/hip_fp16.h>

namespace xp {
namespace {

__device__ __forceinline__ float load_value(const void *base, int64_t index, int dtype) {
  switch (dtype) {
    case kDtypeF16:
      return __half2float(reinterpret_cast<const __half *>(base)[index]);
    case kDtypeF32:
      return reinterpret_cast<const float *>(base)[index];
    default:
      return bf16_to_float(reinterpret_cast<const uint16_t *>(base)[index]);
  }
}

// Nearest-even rounding to the payload dtype, back in fp32.
__device__ __forceinline__ float round_to(float value, int dtype) {
  switch (dtype) {
    case kDtypeF16:
      return __half2float(__float2half_rn(f32_rounding_point(value)));
    case kDtypeF32:
      return value;
    default:
      return round_bf16(value);
  }
}

__device__ __forceinline__ void store_value(void *base, int64_t index, float value, int dtype) {
  switch (dtype) {
    case kDtypeF16:
      reinterpret_cast<__half *>(base)[index] = __float2half_rn(f32_rounding_point(value));
      break;
    case kDtypeF32:
      reinterpret_cast<float *>(base)[index] = value;
      break;
    default:
      reinterpret_cast<uint16_t *>(base)[index] = static_cast<uint16_t>(float_to_bf16(value));
      break;
  }
}

// ReLU that keeps NaN payloads: x for x > 0 or NaN, +0 otherwise.
__device__ __forceinline__ float relu_keep_nan(float value) { return (value > 0.0f || value != value) ? value : 0.0f; }

__device__ __forceinline__ float apply_function(float value, const ActivationArgs &act) {
  switch (act.function) {
    case kActivationRelu:
      return relu_keep_nan(value);
    case kActivationGelu:
      if (act.approximate_tanh) {
        const float inner = 0.7978845608028654f * (value + 0.044715f * value * value * value);
        return 0.5f * value * (1.0f + tanhf(inner));
      }
      return 0.5f * value * (1.0f + erff(value * 0.7071067811865476f));
    default:  // SiLU: v / (1 + exp(-alpha v)), IEEE divide
      return value / (1.0f + expf(-act.alpha * value));
  }
}

__device__ __forceinline__ float apply_gated(float gate, float up, const ActivationArgs &act) {
  if (act.has_limit) {
    gate = fminf(gate, act.limit);
    up = fminf(fmaxf(up, -act.limit), act.limit);
  }
  return apply_function(gate, act) * (up + act.up_offset);
}

// ------------------------------------------------------------------ general projection
// 64 x 64 output tile per 256-thread workgroup, each thread a 4 x 4 block of outputs
// (4 consecutive weight rows, so a Gate/Up pair of INTERLEAVED weights stays in one thread);
// K in slabs of 32 staged in LDS as fp32 (element loads, zero past the ends).  Each output is
// one fp32 sum in K order: deterministic.
constexpr int kProjTile = 64;
constexpr int kProjSlab = 32;

__global__ __launch_bounds__(256) void projection_kernel(ProjectionArgs a) {
  __shared__ float xs[kProjSlab][kProjTile + 4];
  __shared__ float ws[kProjSlab][kProjTile + 4];
  const int tx = threadIdx.x & 15;  // weight-row group: rows n0 + 4 tx .. + 3
  const int ty = threadIdx.x >> 4;  // token group: rows m0 + 4 ty .. + 3
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kProjTile;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kProjTile;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < a.k; k0 += kProjSlab) {
    for (int index = threadIdx.x; index < kProjTile * kProjSlab; index += 256) {
      const int row = index / kProjSlab;
      const int kk = index % kProjSlab;
      const int64_t k = k0 + kk;
      const int64_t token = m0 + row;
      const int64_t weight_row = n0 + row;
      xs[kk][row] = token < a.rows && k < a.k ? load_value(a.x, token * a.k + k, a.dtype) : 0.0f;
      ws[kk][row] = weight_row < a.n && k < a.k ? load_value(a.w, weight_row * a.k + k, a.dtype) : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < kProjSlab; ++kk) {
      float xv[4];
      float wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = xs[kk][4 * ty + i];
        wv[i] = ws[kk][4 * tx + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = fmaf(xv[i], wv[j], acc[i][j]);
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t token = m0 + 4 * ty + i;
    if (token >= a.rows) {
      continue;
    }
    float value[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + 4 * tx + j;
      value[j] = acc[i][j] + (a.bias != nullptr && n < a.n ? a.bias[n] : 0.0f);
    }
    if (a.act.gated) {
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        const int64_t n = n0 + 4 * tx + j;  // even: the Gate row of pair n / 2
        if (n < a.n) {
          const float h = apply_gated(round_to(value[j], a.dtype), round_to(value[j + 1], a.dtype), a.act);
          store_value(a.out, token * (a.n / 2) + n / 2, h, a.dtype);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + 4 * tx + j;
        if (n < a.n) {
          const float v = a.act.function == kActivationNone ? value[j] : apply_function(round_to(value[j], a.dtype), a.act);
          store_value(a.out, token * a.n + n, v, a.dtype);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ standalone activation
// One thread per output element (grid-stride): gated reads Gate and Up from the layout the
// order names; ungated ReLU works on the raw 16-bit patterns (bit-exact, in place allowed).
__global__ __launch_bounds__(256) void activation_kernel(ActivationLaunchArgs a) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t index = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; index < a.elements;
       index += stride) {
    if (!a.act.gated) {
      if (a.act.function == kActivationRelu) {
        const uint16_t bits = reinterpret_cast<const uint16_t *>(a.inputs)[index];
        const float value = load_value(a.inputs, index, a.dtype);
        reinterpret_cast<uint16_t *>(a.output)[index] = (value > 0.0f || value != value) ? bits : uint16_t{0};
      } else {
        store_value(a.output, index, apply_function(load_value(a.inputs, index, a.dtype), a.act), a.dtype);
      }
      continue;
    }
    const int64_t row = index / a.width;
    const int64_t column = index - row * a.width;
    const int64_t gate_at = a.interleaved ? row * 2 * a.width + 2 * column : row * 2 * a.width + column;
    const int64_t up_at = a.interleaved ? gate_at + 1 : gate_at + a.width;
    const float gate = load_value(a.inputs, gate_at, a.dtype);
    const float up = load_value(a.inputs, up_at, a.dtype);
    store_value(a.output, index, apply_gated(gate, up, a.act), a.dtype);
  }
}

}  // namespace

KernelLaunch make_projection(const ProjectionArgs &args) {
  KernelLaunch kernel;
  kernel.func = reinterpret_cast<const void *>(&projection_kernel);
  kernel.grid = dim3(static_cast<unsigned>((args.n + kProjTile - 1) / kProjTile),
                     static_cast<unsigned>((args.rows + kProjTile - 1) / kProjTile), 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

KernelLaunch make_activation(const ActivationLaunchArgs &args) {
  KernelLaunch kernel;
  kernel.func = reinterpret_cast<const void *>(&activation_kernel);
  const int64_t blocks = (args.elements + 255) / 256;
  kernel.grid = dim3(static_cast<unsigned>(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096), 1, 1);
  kernel.block = dim3(256, 1, 1);
  kernel.set_args(args);
  return kernel;
}

}  // namespace xp
