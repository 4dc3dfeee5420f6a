// quant_dev.h - device helpers shared by the kernels that write q8_0 activation codes (LayerNorm,
// the fc1 GELU epilogue, the attention output epilogue).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

// The q8_0 code of v at inverse scale id, as its two's-complement byte in the low 8 bits: x86 ggml's
// round-to-nearest-even(fl(v * id)), read from the float 1.5 * 2^23 + fl(v * id), whose unit in the
// last place is 1 (exact for |fl(v * id)| < 2^22); two VALU ops where rint, a clamp and a conversion
// took four. Every caller has |v| <= amax and id = fl(127 / amax), so |fl(v * id)| <= 127 (1 + 2^-23)
// and the quantizer's clamp to [-128, 127] never acts.
__device__ __forceinline__ uint32_t q8_byte(float v, float id) {
    return __float_as_uint(__fadd_rn(__fmul_rn(v, id), 12582912.0f)) & 0xffu;
}
