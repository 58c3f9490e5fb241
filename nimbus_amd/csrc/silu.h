// The SiLU gate of Llama's MLP on one element, as MLP.forward computes it in
// the model dtype (nimbus/model/llama.py:93-103: F.silu(gate) * up): silu in
// fp32 rounded to the model dtype, then the product rounded again. Shared by
// silu_mul_kernel and the INT8 gate_up projection's fused epilogue, so both
// give the same bits.
#pragma once

#include "common.h"

namespace nimbus {

// Contraction is off so that every kernel that inlines this forms 1 +
// exp(-gate), the quotient and the product as separate correctly rounded
// steps. The product s * up of two 16-bit values is exact in fp32, so the one
// rounding to the model dtype is the same whether the compiler multiplies in
// fp32 or in f16. The gate a caller passes must already be the model-dtype
// value (a 16-bit store read back), not a wider intermediate.
template <int DT>
__device__ __forceinline__ uint16_t silu_mul_value(float gate, float up) {
#pragma clang fp contract(off)
  const float s = Elem<DT>::to_f32(Elem<DT>::from_f32(gate / (1.f + expf(-gate))));
  return Elem<DT>::from_f32(s * up);
}

}  // namespace nimbus
