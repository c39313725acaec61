// Indexer scoring (the build's definition; the reference attends every visible compressed row,
// oracle/decode_engine.py:112-114, and has no indexer).
//
//   dot_h = fma chain over d = 0..Di-1 of q[h,d]*k[n,d] (from +0)
//   r_h   = dot_h > 0 ? dot_h : +0
//   acc   = fma chain over h = 0..Hi-1 of w[h]*r_h (from +0)
//   score = acc * kscale[n]   (or acc when kscale == NULL);  -inf for n >= nvis
//
// The order is fixed so that every score is reproducible bit for bit by the CPU oracle; the top-k
// that follows can then be compared exactly.  One thread per key: the key row lives in VGPRs as
// fp32, q (fp32, [Hi][Di]) and w sit in LDS and are read as wave-wide broadcasts.  HBM traffic
// per (query row): N * (Di * sizeof(key) + 4) bytes of keys and scales, N * 4 bytes of scores.
#include "smla_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxDi = 128;
constexpr int kMaxQ = 64 * 128;  // Hi * Di fp32 in LDS (32 KiB)

template <int DI, int KDT>
__global__ __launch_bounds__(kThreads) void indexer_kernel(const void* __restrict__ q, int q_dtype,
                                                           const void* __restrict__ keys,
                                                           const float* __restrict__ kscale,
                                                           const float* __restrict__ weights,
                                                           const int32_t* __restrict__ nvis, int64_t S,
                                                           int Hi, int64_t N, float* __restrict__ scores) {
  __shared__ __align__(16) float sq[kMaxQ];
  __shared__ float sw[256];
  const int64_t bs = blockIdx.y;
  const int64_t b = bs / S;
  const int tid = threadIdx.x;
  for (int i = tid; i < Hi * DI; i += kThreads) sq[i] = load_as_f32(q, bs * Hi * DI + i, q_dtype);
  for (int i = tid; i < Hi; i += kThreads) sw[i] = weights[bs * Hi + i];
  __syncthreads();
  const int64_t n = (int64_t)blockIdx.x * kThreads + tid;
  if (n >= N) return;
  const int64_t nv = nvis ? (int64_t)nvis[bs] : N;
  float* out = scores + bs * N + n;
  if (n >= nv) {
    *out = -SMLA_INF;
    return;
  }
  float kr[DI];
  const int64_t row = b * N + n;
  if constexpr (KDT == SMLA_FP8_E4M3) {
    const u32x4_t* kp = (const u32x4_t*)((const uint8_t*)keys + row * DI);
#pragma unroll
    for (int v = 0; v < DI / 16; v++) {
      u32x4_t w = kp[v];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], false);
        f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], true);
        kr[16 * v + 4 * j + 0] = lo.x;
        kr[16 * v + 4 * j + 1] = lo.y;
        kr[16 * v + 4 * j + 2] = hi.x;
        kr[16 * v + 4 * j + 3] = hi.y;
      }
    }
  } else if constexpr (KDT == SMLA_BF16) {
    const u32x4_t* kp = (const u32x4_t*)((const uint16_t*)keys + row * DI);
#pragma unroll
    for (int v = 0; v < DI / 8; v++) {
      u32x4_t w = kp[v];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        kr[8 * v + 2 * j] = bf16_bits_to_f32((uint16_t)(w[j] & 0xffffu));
        kr[8 * v + 2 * j + 1] = bf16_bits_to_f32((uint16_t)(w[j] >> 16));
      }
    }
  } else {
    const f32x4_t* kp = (const f32x4_t*)((const float*)keys + row * DI);
#pragma unroll
    for (int v = 0; v < DI / 4; v++) {
      f32x4_t w = kp[v];
      kr[4 * v] = w[0];
      kr[4 * v + 1] = w[1];
      kr[4 * v + 2] = w[2];
      kr[4 * v + 3] = w[3];
    }
  }
  float acc = 0.f;
  for (int h = 0; h < Hi; h++) {
    const f32x4_t* qh = (const f32x4_t*)(sq + h * DI);
    float dot = 0.f;
#pragma unroll
    for (int v = 0; v < DI / 4; v++) {
      f32x4_t qq = qh[v];
      dot = __builtin_fmaf(qq[0], kr[4 * v], dot);
      dot = __builtin_fmaf(qq[1], kr[4 * v + 1], dot);
      dot = __builtin_fmaf(qq[2], kr[4 * v + 2], dot);
      dot = __builtin_fmaf(qq[3], kr[4 * v + 3], dot);
    }
    float r = dot > 0.f ? dot : 0.f;
    acc = __builtin_fmaf(sw[h], r, acc);
  }
  *out = kscale ? acc * kscale[row] : acc;
}

template <int DI>
int launch_di(const void* q, int q_dtype, const void* keys, int k_dtype, const float* kscale,
              const float* w, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi, int64_t N,
              float* scores, hipStream_t st) {
  dim3 grid((unsigned)((N + kThreads - 1) / kThreads), (unsigned)(B * S));
  if (k_dtype == SMLA_FP8_E4M3)
    hipLaunchKernelGGL((indexer_kernel<DI, SMLA_FP8_E4M3>), grid, dim3(kThreads), 0, st, q, q_dtype, keys,
                       kscale, w, nvis, S, (int)Hi, N, scores);
  else if (k_dtype == SMLA_BF16)
    hipLaunchKernelGGL((indexer_kernel<DI, SMLA_BF16>), grid, dim3(kThreads), 0, st, q, q_dtype, keys, kscale,
                       w, nvis, S, (int)Hi, N, scores);
  else
    hipLaunchKernelGGL((indexer_kernel<DI, SMLA_F32>), grid, dim3(kThreads), 0, st, q, q_dtype, keys, kscale,
                       w, nvis, S, (int)Hi, N, scores);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

}  // namespace

extern "C" int smla_indexer_score(const void* q, int q_dtype, const void* keys, int k_dtype, const float* kscale,
                                  const float* weights, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi,
                                  int64_t Di, int64_t N, float* scores, void* stream) {
  if (!q || !keys || !weights || !scores) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || Hi <= 0 || Di <= 0 || N <= 0) return SMLA_E_SHAPE;
  if (q_dtype != SMLA_F32 && q_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  if (k_dtype != SMLA_F32 && k_dtype != SMLA_BF16 && k_dtype != SMLA_FP8_E4M3) return SMLA_E_DTYPE;
  if (Hi > 256 || Hi * Di > kMaxQ || (N + kThreads - 1) / kThreads > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  switch (Di) {
    case 32: return launch_di<32>(q, q_dtype, keys, k_dtype, kscale, weights, nvis, B, S, Hi, N, scores, st);
    case 64: return launch_di<64>(q, q_dtype, keys, k_dtype, kscale, weights, nvis, B, S, Hi, N, scores, st);
    case 128: return launch_di<128>(q, q_dtype, keys, k_dtype, kscale, weights, nvis, B, S, Hi, N, scores, st);
  }
  return SMLA_E_UNSUPPORTED;
}
