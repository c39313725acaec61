// Host-side entry points to the device fp8/bf16 codecs of smla_internal.h, for CPU tests.
#include "../../deepseek-v4-flash-mlx_amd/csrc/smla_internal.h"

extern "C" uint32_t host_f32_to_e4m3(float x) { return f32_to_e4m3(x); }
extern "C" float host_e4m3_to_f32(uint32_t c) { return e4m3_to_f32(c); }
extern "C" float host_pow2_ceil(float v) { return pow2_ceil(v); }
extern "C" uint16_t host_f32_to_bf16(float x) { return f32_to_bf16_bits(x); }
extern "C" uint32_t host_f32_to_e2m1(float z) { return f32_to_e2m1(z); }
extern "C" float host_e2m1_to_f32(uint32_t c) { return e2m1_to_f32(c); }
extern "C" int host_fp4_scale_exp(float amax) { return fp4_scale_exp(amax); }
extern "C" float host_hadamard_scale(int lg) { return hadamard_scale(lg); }
