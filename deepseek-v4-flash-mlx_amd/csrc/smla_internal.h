// Shared device helpers for the smla HIP kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/smla.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x32_t __attribute__((ext_vector_type(32)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ inline bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

#define SMLA_INF __builtin_inff()

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32 (bit level; fp32 -> bf16 rounds to nearest even, NaN stays NaN)
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
// device-side fp32 -> bf16, round to nearest even, with the gfx950 conversion instruction
// (v_cvt_pk_bf16_f32, two values per instruction).  The software form above, whose NaN test
// becomes divergent control flow, is kept for host code.
typedef float smla_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 smla_bf16x2_t __attribute__((ext_vector_type(2)));
// pack two fp32 into two bf16 (lo in bits 0..15)
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((smla_f32x2_t){lo, hi}, smla_bf16x2_t));
}
__device__ inline uint16_t bf16_rne(float f) { return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu); }
// fp32 rounded to the nearest bf16 value, back in fp32
__device__ inline float bf16_round(float f) { return __uint_as_float(pack_bf16x2(0.f, f) & 0xffff0000u); }

// ---------------------------------------------------------------------------------------------
// fp8 e4m3fn (OCP): decode and round-to-nearest-even encode, integer arithmetic only.
__host__ __device__ inline float e4m3_to_f32(uint32_t code) {
  uint32_t s = (code >> 7) & 1u, e = (code >> 3) & 0xFu, m = code & 7u;
  float v;
  if (e == 0) {
    v = (float)m * 0.001953125f;  // m * 2^-9
  } else if (e == 15 && m == 7) {
    v = __builtin_nanf("");
  } else {
    uint32_t bits = ((e + 120u) << 23) | (m << 20);  // 2^(e-7) * (1 + m/8)
    __builtin_memcpy(&v, &bits, 4);
  }
  return s ? -v : v;
}

// |x| <= 448 expected (callers clip); larger magnitudes saturate to 448.
__host__ __device__ inline uint32_t f32_to_e4m3(float x) {
  uint32_t u;
  __builtin_memcpy(&u, &x, 4);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t mag = u & 0x7fffffffu;
  if (mag >= 0x43e00000u) return sign | 0x7eu;  // >= 448 -> 448
  int32_t exp = (int32_t)(mag >> 23) - 127;
  if (exp < -10) return sign;  // < 2^-10: rounds to 0 (2^-10 itself is the 0/2^-9 midpoint)
  uint32_t man = (mag & 0x7fffffu) | 0x800000u;  // 24-bit significand, value = man * 2^(exp-23)
  if ((mag >> 23) == 0) return sign;              // fp32 subnormal
  // quantum of the e4m3 grid: 2^(max(exp,-6)-3);  q = value / quantum = man * 2^(exp-23-qe)
  int32_t qe = (exp < -6 ? -6 : exp) - 3;
  int32_t sh = qe - (exp - 23);  // >= 20 for normals, larger for subnormal range
  uint32_t q = man >> sh;
  uint32_t rem = man & ((1u << sh) - 1u);
  uint32_t half = 1u << (sh - 1);
  if (rem > half || (rem == half && (q & 1u))) q++;
  // q counts quanta at exponent qe: value = q * 2^qe.  Re-encode.
  if (qe == -9) {
    // quantum 2^-9 covers the subnormals (q < 8) and exponent field 1 (8 <= q < 16); q == 16
    // carries into exponent field 2.  Field/mantissa bits are contiguous, so code = q works for
    // q < 8 and code = 8 + (q - 8) = q for the rest: the code is q itself.
    return sign | q;
  }
  // normal: q in [8, 16]; q == 16 carries into the next binade
  uint32_t ef = (uint32_t)(qe + 3 + 7);
  if (q >= 16) { q >>= 1; ef += 1; }
  if (ef > 15 || (ef == 15 && (q - 8u) > 6u)) return sign | 0x7eu;
  return sign | (ef << 3) | (q - 8u);
}

// exact 2^ceil(log2(v)) for finite v > 0 (normal range)
__host__ __device__ inline float pow2_ceil(float v) {
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  uint32_t e = (u >> 23) & 0xffu;
  if (u & 0x7fffffu) e += 1;
  uint32_t r = e << 23;
  float f;
  __builtin_memcpy(&f, &r, 4);
  return f;
}

// ---------------------------------------------------------------------------------------------
// fp4 e2m1 (grid 0, 0.5, 1, 1.5, 2, 3, 4, 6; bit 3 the sign) with power-of-two block scales.
// Round to nearest, ties to the even code: the magnitude code counts the decision points passed,
// strict between an even code and the next, inclusive between an odd code and the next.
// |z| <= 6 expected (callers clip).
__host__ __device__ inline uint32_t f32_to_e2m1(float z) {
  const float a = fabsf(z);
  uint32_t m = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) + (uint32_t)(a >= 1.75f) +
               (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) + (uint32_t)(a > 5.0f);
  uint32_t u;
  __builtin_memcpy(&u, &z, 4);
  return m | ((u >> 28) & 8u);
}
__host__ __device__ inline float e2m1_to_f32(uint32_t code) {
  // magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6 = (code < 2 ? code / 2 : (2 + (code & 1)) * 2^((code >> 1) - 1) / 2)
  const uint32_t c = code & 7u;
  const float m = c < 2u ? 0.5f * (float)c : (float)(2u + (c & 1u)) * (float)(1u << ((c >> 1) - 1u)) * 0.5f;
  return (code & 8u) ? -m : m;
}
// exponent k of the fp4 block scale s = 2^k = 2^ceil(log2(max(amax, 6*2^-126) / 6)); the division
// is the float32 one of the definition (rounded), the ceiling is exact on its bits
__host__ __device__ inline int fp4_scale_exp(float amax) {
  const float a = fmaxf(amax, 6.0f * 0x1p-126f);
  const float v = a / 6.0f;  // >= 2^-126: a normal number
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return (int)((u >> 23) & 0xffu) - 127 + ((u & 0x7fffffu) ? 1 : 0);
}
// 2^k as float32 for -126 <= k <= 127
__host__ __device__ inline float exp2i_f32(int k) {
  const uint32_t u = (uint32_t)(k + 127) << 23;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
// ue8m0 scale byte b -> 2^(b-127) as float32: 0 gives the subnormal 2^-127, 255 the E8M0 NaN
__host__ __device__ inline float ue8m0_to_f32(uint32_t b) {
  // selects, not branches: inside unrolled loops a branch splits the schedule
  const uint32_t u = b == 0u ? 0x00400000u : (b == 255u ? 0x7fc00000u : b << 23);
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
// float32(n^-0.5) for n = 2^lg: 2^-(lg/2), times float32(sqrt(0.5)) = 0x3F3504F3 when lg is odd
__host__ __device__ inline float hadamard_scale(int lg) {
  const float p = exp2i_f32(-(lg >> 1));
  return (lg & 1) ? p * 0.707106769084930419921875f : p;
}

// ---------------------------------------------------------------------------------------------
// wave64 reductions
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// DPP forms (VALU lane moves, no LDS round trip): reductions inside each 16-lane row, then the
// four row results through readlane.  dpp controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140, row_shr:n = 0x110 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
template <int CTRL>
__device__ inline int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// wave-wide max / min (every lane gets the result)
__device__ inline float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ inline float wave_min_dpp(float v) { return -wave_max_dpp(-v); }
// wave-wide sum (every lane gets the same result, summed in a fixed order)
__device__ inline float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}
// inclusive prefix sum over the 64 lanes (lane order)
__device__ inline int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// ---------------------------------------------------------------------------------------------
// XCD pinning.  The workgroups of a launch are dealt to the 8 XCDs round-robin in linear order
// (workgroup L = x + gx (y + gy z) runs on XCD L mod 8) and each XCD has its own L2 (a hit in
// it costs about half the latency of a line served from another XCD's side and a third of HBM's).
// A launch over `rows` x `items` workgroups (rows a multiple of 8) that places every item of row r
// on XCD r mod 8 has all items of row r share its data in one L2: the attention splits of a query
// row fetch its q block and index list once per sequence instead of once per XCD.  Across kernel
// boundaries lines a kernel read stay in the L2; lines a kernel wrote are read back from memory
// (the merge fetches as many bytes as the split kernel wrote), so pinning a consumer to its
// producer's XCD saves no memory traffic.  The decode step pins its query rows the same way in
// the indexer, the selection, the attention splits and the merge.
constexpr int kXcds = 8;
__device__ inline int64_t linear_block_id() {
  return (int64_t)blockIdx.x + (int64_t)gridDim.x * ((int64_t)blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}
// (row, item) of this workgroup in a launch of rows * items workgroups: row-major when rows is not a
// multiple of 8, else pinned (row mod 8 == XCD).  Launches hold fewer than 2^32 workgroups, so the
// arithmetic is 32-bit: a 64-bit division by a launch-time value is a long dependent scalar
// sequence at the start of every workgroup.
__device__ inline void xcd_row_item(int64_t rows, int64_t items, int64_t& row, int64_t& item) {
  const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t n = (uint32_t)items;
  if ((uint32_t)rows % kXcds != 0) {
    const uint32_t q = L / n;
    row = q;
    item = L - q * n;
    return;
  }
  const uint32_t i = L / kXcds, q = i / n;
  row = (L % kXcds) + kXcds * q;
  item = i - q * n;
}
// batch entry of query row bs with S query rows per entry (bs < 2^32: a grid dimension)
__device__ inline int64_t batch_of(int64_t bs, int64_t S) {
  return S == 1 ? bs : (int64_t)((uint32_t)bs / (uint32_t)S);
}

// Launches whose grid has a query-row dimension (y: at most 65535) take at most kChunkRows query
// rows (a multiple of 8 keeps the XCD pinning of rows).  Longer calls run as launches over row
// chunks: whole batch entries while one entry fits, else pieces of one entry.  f(b0, s0, nb, ns)
// runs the chunk of query rows b0*S + s0 .. as a call of nb entries of ns rows each; the first
// nonzero return ends the walk.
constexpr int64_t kChunkRows = 65528;

template <class F>
inline int for_row_chunks(int64_t B, int64_t S, F&& f) {
  if (B * S <= kChunkRows) return f((int64_t)0, (int64_t)0, B, S);
  if (S <= kChunkRows) {
    const int64_t per = kChunkRows / S;
    for (int64_t b0 = 0; b0 < B; b0 += per)
      if (const int rc = f(b0, (int64_t)0, per < B - b0 ? per : B - b0, S); rc != 0) return rc;
    return 0;
  }
  for (int64_t b = 0; b < B; b++)
    for (int64_t s0 = 0; s0 < S; s0 += kChunkRows)
      if (const int rc = f(b, s0, (int64_t)1, kChunkRows < S - s0 ? kChunkRows : S - s0); rc != 0) return rc;
  return 0;
}

// ---------------------------------------------------------------------------------------------
// load one element of a given dtype as fp32
__device__ inline float load_as_f32(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case SMLA_F32: return ((const float*)p)[i];
    case SMLA_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case SMLA_FP8_E4M3: return e4m3_to_f32(((const uint8_t*)p)[i]);
    case SMLA_F16: return (float)((const _Float16*)p)[i];
  }
  return 0.f;
}
__device__ inline void store_from_f32(void* p, int64_t i, int dtype, float v) {
  if (dtype == SMLA_F32) ((float*)p)[i] = v;
  else if (dtype == SMLA_BF16) ((uint16_t*)p)[i] = bf16_rne(v);
  else if (dtype == SMLA_F16) ((_Float16*)p)[i] = (_Float16)v;
}

// tiled MFMA GEMM (gemm.hip): y [T, G*N] = grouped x [T, G*K] (row stride ldx) times w [G*N, K]^T,
// operands both bf16 or both fp32 (f32_operands), y bf16 or fp32; with pos, inverse RoPE of the
// last 64 dims of every head_dim-wide head of x (bf16) as it is loaded
int launch_gemm_tiled(const void* x, int64_t ldx, bool f32_operands, const void* w, int64_t T, int64_t G, int64_t N,
                      int64_t K, const int32_t* pos, const float* cos_t, const float* sin_t, int64_t head_dim,
                      void* y, int y_dtype, hipStream_t st);

#define SMLA_HIP_CHECK_LAUNCH()                         \
  do {                                                  \
    hipError_t _e = hipGetLastError();                  \
    if (_e != hipSuccess) return (int)_e;               \
  } while (0)

// Compute units of the current device, queried once per device id (256 if the query fails).
inline int smla_num_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Raises a kernel's dynamic LDS limit on the current device, once per device: `done` holds one bit
// per device id (ids from 64 up set the attribute on every call).  Safe to call from several host
// threads; a lost race only repeats the call.
inline hipError_t smla_set_dynamic_lds(const void* kern, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t{1} << dev) : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit != 0) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}
