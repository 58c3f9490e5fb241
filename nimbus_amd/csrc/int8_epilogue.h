// The INT8 projection's output rounding, shared by the kernels that store it:
// the tiled matmuls, their split-K reduction, and the fused residual add +
// RMSNorm that folds a projection's split-K partials in itself.
#pragma once

#include "common.h"

namespace nimbus {

// dtype(acc * scale) as the reference forms it (nimbus/quant/int8.py:43-47):
// the fp32 product, then the conversion to the 16-bit type. Left to itself
// the compiler turns some of these into one v_fma_mixlo_f16 (the exact
// product rounded to 16 bits once) and others into a multiply and a
// conversion, picking per element and per kernel: about one output in 10^4
// then differs by an ulp between two kernels that store the same value
// (measured on the fused gate_up + SiLU launch against the projection and the
// gate run apart). The empty asm keeps the fp32 product in a register, so
// every store rounds twice, as the reference does.
template <int DT>
__device__ __forceinline__ uint16_t scaled(float acc, float scale) {
  float p = acc * scale;
  asm volatile("" : "+v"(p));
  return Elem<DT>::from_f32(p);
}

}  // namespace nimbus
