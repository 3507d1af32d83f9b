/*
 * Plain-C restatement of the FfnAgent Dense-FFN mailbox step.
 *
 * TEST INFRASTRUCTURE ONLY: the tests load this library to cross-check the
 * torch/numpy oracle (oracle/ffn_oracle.py).  Nothing in crosspool_amd links
 * or calls it.  Scalar loops, fp64 accumulation; bf16 is handled as raw
 * uint16 bit patterns so every rounding point is explicit.
 *
 * Reference behaviour restated (paths relative to the CrossPool checkout):
 *   copy   src/cext-include/xpool/utils/cooperative.cuh:37-55
 *   gather src/cext/transport/instance.cu:83-84 (prefix copy, generalised to slot ids)
 *   scatter src/cext/transport/instance.cu:184-186, src/cext/fabric/atnagent.cu:275
 *   dense  src/xpool-dev/xtest/harness/native/ffn/qualification.py:290-314
 *   silu   src/xpool/runtime/ffnagent/operators/activation.py:31-51
 *   rmsnorm (no reference counterpart; textbook formula, parity unpinned)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* float -> bf16, round to nearest even; NaN stays a quiet NaN of the same sign. */
uint16_t xpo_bf16_from_float(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0) {
    return (uint16_t)((bits >> 16) | 0x0040u);
  }
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

float xpo_float_from_bf16(uint16_t value) {
  uint32_t bits = (uint32_t)value << 16;
  float result;
  memcpy(&result, &bits, sizeof result);
  return result;
}

/* torch's fp64 -> bf16 conversion goes through fp32 (two roundings). */
static uint16_t bf16_from_double(double value) { return xpo_bf16_from_float((float)value); }

/* Byte copy of equal ranges; returns -1 on size mismatch (cooperative.cuh:40). */
int xpo_copy_bytes(uint8_t *destination, size_t destination_size, const uint8_t *source, size_t source_size) {
  if (destination_size != source_size) {
    return -1;
  }
  for (size_t index = 0; index < source_size; ++index) {
    destination[index] = source[index];
  }
  return 0;
}

/* out[i, :] = pool[slots[i], :]; returns -1 if a slot is outside the pool. */
int xpo_gather(const uint16_t *pool, int64_t pool_rows, int64_t hidden, const int32_t *slots, int64_t rows,
               uint16_t *out) {
  for (int64_t row = 0; row < rows; ++row) {
    if (slots[row] < 0 || slots[row] >= pool_rows) {
      return -1;
    }
    for (int64_t column = 0; column < hidden; ++column) {
      out[row * hidden + column] = pool[(int64_t)slots[row] * hidden + column];
    }
  }
  return 0;
}

/* pool[slots[i], :] = values[i, :]; returns -1 if a slot is outside the pool. */
int xpo_scatter(uint16_t *pool, int64_t pool_rows, int64_t hidden, const int32_t *slots, int64_t rows,
                const uint16_t *values) {
  for (int64_t row = 0; row < rows; ++row) {
    if (slots[row] < 0 || slots[row] >= pool_rows) {
      return -1;
    }
    for (int64_t column = 0; column < hidden; ++column) {
      pool[(int64_t)slots[row] * hidden + column] = values[row * hidden + column];
    }
  }
  return 0;
}

/* bf16(x * (1 / sqrt(mean(x^2) + eps)) * w); mean of squares accumulated in fp64, then fp32 math. */
void xpo_rmsnorm(const uint16_t *x, int64_t rows, int64_t hidden, const uint16_t *weight, float eps,
                 uint16_t *out) {
  for (int64_t row = 0; row < rows; ++row) {
    double sum = 0.0;
    for (int64_t column = 0; column < hidden; ++column) {
      const double value = xpo_float_from_bf16(x[row * hidden + column]);
      sum += value * value;
    }
    const float mean = (float)(sum / (double)hidden);
    const float inverse = 1.0f / sqrtf(mean + eps);
    for (int64_t column = 0; column < hidden; ++column) {
      const float value = xpo_float_from_bf16(x[row * hidden + column]) * inverse;
      out[row * hidden + column] = xpo_bf16_from_float(value * xpo_float_from_bf16(weight[column]));
    }
  }
}

/* silu(g) * (u + up_offset) with optional clipping, fp32, rounded to bf16 (activation.py:31-51). */
uint16_t xpo_gated_silu(uint16_t gate_bits, uint16_t up_bits, float alpha, float limit, float up_offset) {
  float gate = xpo_float_from_bf16(gate_bits);
  float up = xpo_float_from_bf16(up_bits);
  if (limit > 0.0f) {
    gate = gate < limit ? gate : limit;
    up = up < -limit ? -limit : (up > limit ? limit : up);
  }
  const float activated = gate / (1.0f + expf(-alpha * gate));
  return xpo_bf16_from_float(activated * (up + up_offset));
}

/*
 * Dense partial: x [T, H], interleaved w_gate_up [2I, H], w_down [H, I].
 * fp64 projections -> bf16 gate/up -> fp32 silu*mul -> bf16 h -> fp64 down -> bf16.
 * `activated` receives h [T, I] (may be NULL), `out` the result [T, H].
 */
void xpo_dense_partial(const uint16_t *x, int64_t rows, int64_t hidden, const uint16_t *w_gate_up,
                       const uint16_t *w_down, int64_t intermediate, uint16_t *activated, uint16_t *out) {
  for (int64_t row = 0; row < rows; ++row) {
    for (int64_t j = 0; j < intermediate; ++j) {
      double gate = 0.0;
      double up = 0.0;
      for (int64_t k = 0; k < hidden; ++k) {
        const double value = xpo_float_from_bf16(x[row * hidden + k]);
        gate += value * xpo_float_from_bf16(w_gate_up[(2 * j) * hidden + k]);
        up += value * xpo_float_from_bf16(w_gate_up[(2 * j + 1) * hidden + k]);
      }
      const uint16_t h = xpo_gated_silu(bf16_from_double(gate), bf16_from_double(up), 1.0f, 0.0f, 0.0f);
      if (activated != NULL) {
        activated[row * intermediate + j] = h;
      }
    }
  }
  for (int64_t row = 0; row < rows; ++row) {
    for (int64_t n = 0; n < hidden; ++n) {
      double sum = 0.0;
      for (int64_t j = 0; j < intermediate; ++j) {
        double h;
        if (activated != NULL) {
          h = xpo_float_from_bf16(activated[row * intermediate + j]);
        } else {
          h = 0.0; /* callers always pass the activated buffer; kept total for safety */
        }
        sum += h * xpo_float_from_bf16(w_down[n * intermediate + j]);
      }
      out[row * hidden + n] = bf16_from_double(sum);
    }
  }
}
