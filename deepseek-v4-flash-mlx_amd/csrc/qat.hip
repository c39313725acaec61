// Indexer-key transform: normalised Walsh-Hadamard rotation and fp4 e2m1 block quantisation.
//
//  * rotate_fp4_kernel<N, XDT> : rows of N (32..1024, a power of two) float32 or bf16 values.
//      ROTATE: the butterfly of v4mlx/qat.py:8-20 (stages h = 1, 2, ..., N/2; at stage h the pair
//              (x[i], x[i+h]) of each group of 2h becomes (x[i] + x[i+h], x[i] - x[i+h]), one
//              float32 rounding each), then a float32 multiply by float32(N^-0.5);
//      FP4   : v4mlx/qat.py:23-31 per block of 32: s = 2^ceil(log2(max(amax, 6*2^-126) / 6)),
//              code = e2m1(clip(x / s, +-6)), round to nearest even; written as the round trip
//              (code value * s, float32) and/or the stored form (packed codes, element 2i in the
//              low nibble of byte i; one ue8m0 scale byte log2(s) + 127 per block).
//    Layout: a lane holds 32 consecutive values (one fp4 block), a row spans L = N / 32 lanes of
//    one wave, so 64 / L rows share a wave.  Butterfly stages h < 32 stay in registers; the
//    others pair lane l with lane l ^ (h / 32) through DPP (h / 32 < 4) or ds_bpermute.  The
//    block's abs-max is lane-local.  e2m1 rounding is the gfx950 conversion instruction
//    (v_cvt_scalef32_pk_fp4_f32 with scale 1, applied to x * 2^-k computed in float32), which
//    rounds to nearest even and saturates at +-6 like the definition.
//    HBM bound: reads N * 4 (or 2) bytes per row, writes N * 4 and/or N / 2 + N / 32 bytes.
#include "smla_internal.h"

namespace {

constexpr int kQatThreads = 256;

// value of lane (lane ^ M), M a power of two below 64
template <int M>
__device__ inline float lane_xor(float v) {
  if constexpr (M == 1) return dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
  else if constexpr (M == 2) return dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
  else return __shfl_xor(v, M, 64);
}

// one cross-lane butterfly stage: partner lane l ^ M.  The lane whose bit M is clear holds the
// lower element and keeps a + b; the other keeps a - b (a the partner's value).  Both as one
// fma(sgn, v, o) with sgn = +-1: v + o, or o - v, each rounded once like the sum it replaces
// (equal values give +0, as a - b does).
template <int M, int E>
__device__ inline void xstage(float (&v)[E], bool upper) {
  const float sgn = upper ? -1.0f : 1.0f;
#pragma unroll
  for (int r = 0; r < E; r++) {
    const float o = lane_xor<M>(v[r]);
    v[r] = fmaf(sgn, v[r], o);
  }
}

// A lane holds kQatE = 32 consecutive values of a row: one fp4 block.
constexpr int kQatE = 32;

template <int N, int XDT, bool OUT>
__global__ __launch_bounds__(kQatThreads) void rotate_fp4_kernel(const void* __restrict__ x, int64_t rows,
                                                                 int rotate, int fp4, float* __restrict__ out,
                                                                 uint8_t* __restrict__ codes,
                                                                 uint8_t* __restrict__ scales) {
  constexpr int E = kQatE;
  constexpr int L = N / E;     // lanes per row
  constexpr int RPW = 64 / L;  // rows per wave
  static_assert(N >= 32 && (N & (N - 1)) == 0 && N <= 1024, "row length");
  const int lane = threadIdx.x & 63;
  const int sub = lane % L;
  const int64_t row = ((int64_t)blockIdx.x * (kQatThreads / 64) + (threadIdx.x >> 6)) * RPW + lane / L;
  const bool live = row < rows;
  const int64_t rr = live ? row : rows - 1;  // rows past the end compute on the last row, store nothing
  const int64_t e0 = rr * N + (int64_t)sub * E;

  float v[E];
  if constexpr (XDT == SMLA_F32) {
#pragma unroll
    for (int q = 0; q < E / 4; q++) {
      const f32x4_t w = *(const f32x4_t*)((const float*)x + e0 + 4 * q);
#pragma unroll
      for (int k = 0; k < 4; k++) v[4 * q + k] = w[k];
    }
  } else {
#pragma unroll
    for (int q = 0; q < E / 8; q++) {
      const u32x4_t w = *(const u32x4_t*)((const uint16_t*)x + e0 + 8 * q);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        v[8 * q + 2 * k] = __uint_as_float(w[k] << 16);
        v[8 * q + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  }

  if (rotate) {
    // stages inside the lane: h = 1, 2, ..., 16
#pragma unroll
    for (int h = 1; h < E; h *= 2) {
#pragma unroll
      for (int i = 0; i < E; i++) {
        if (i & h) continue;
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
    }
    // stages across lanes: h = 32, 64, ..., N/2, partner lane sub ^ (h / 32)
    if constexpr (L > 1) xstage<1, E>(v, sub & 1);
    if constexpr (L > 2) xstage<2, E>(v, sub & 2);
    if constexpr (L > 4) xstage<4, E>(v, sub & 4);
    if constexpr (L > 8) xstage<8, E>(v, sub & 8);
    if constexpr (L > 16) xstage<16, E>(v, sub & 16);
    constexpr int LG = __builtin_ctz(N);
    const float sc = hadamard_scale(LG);
#pragma unroll
    for (int i = 0; i < E; i++) v[i] *= sc;
  }

  if (fp4) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < E; i++) a = fmaxf(a, fabsf(v[i]));
    const int kexp = fp4_scale_exp(a);
    const float inv = exp2i_f32(-kexp), s = exp2i_f32(kexp);
    // z = x * 2^-k (== x / 2^k, one rounding) in VALU arithmetic; the gfx950 conversion with
    // scale 1 then rounds z to e2m1 (nearest, ties to even, saturating at +-6), two per call,
    // element 2i into the low nibble of byte i
    u32x4_t packed;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      uint32_t word = 0;
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, v[8 * w] * inv, v[8 * w + 1] * inv, 1.0f, 0);
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, v[8 * w + 2] * inv, v[8 * w + 3] * inv, 1.0f, 1);
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, v[8 * w + 4] * inv, v[8 * w + 5] * inv, 1.0f, 2);
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, v[8 * w + 6] * inv, v[8 * w + 7] * inv, 1.0f, 3);
      packed[w] = word;
    }
    // outputs are not read back by this launch: nontemporal stores leave no dirty lines for the
    // kernel's end to write back (113.9 -> 110.4 us for 1M rows of 128; nontemporal loads of x,
    // 128 bytes per lane in 16-byte pieces, double the time)
    if (live && codes) __builtin_nontemporal_store(packed, (u32x4_t*)(codes + e0 / 2));
    if (live && scales) __builtin_nontemporal_store((uint8_t)(kexp + 127), scales + e0 / 32);
    if constexpr (OUT) {
      // decode (code value, exact) and rescale in VALU arithmetic
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const f32x2_t d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed[w], 1.0f, 0);
        const f32x2_t d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed[w], 1.0f, 1);
        const f32x2_t d2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed[w], 1.0f, 2);
        const f32x2_t d3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed[w], 1.0f, 3);
        v[8 * w] = d0[0] * s;
        v[8 * w + 1] = d0[1] * s;
        v[8 * w + 2] = d1[0] * s;
        v[8 * w + 3] = d1[1] * s;
        v[8 * w + 4] = d2[0] * s;
        v[8 * w + 5] = d2[1] * s;
        v[8 * w + 6] = d3[0] * s;
        v[8 * w + 7] = d3[1] * s;
      }
    }
  }
  if constexpr (OUT) {
    if (live) {
#pragma unroll
      for (int q = 0; q < E / 4; q++)
        __builtin_nontemporal_store((f32x4_t){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]}, (f32x4_t*)(out + e0 + 4 * q));
    }
  }
}

template <int N>
int launch_rotate_fp4(const void* x, int x_dtype, int64_t rows, int rotate, int fp4, float* out, uint8_t* codes,
                      uint8_t* scales, hipStream_t st) {
  constexpr int rows_per_wg = (kQatThreads / 64) * (64 / (N / kQatE));
  const int64_t nwg = (rows + rows_per_wg - 1) / rows_per_wg;
  if (nwg > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  const dim3 grid((unsigned)nwg), blk(kQatThreads);
  if (x_dtype == SMLA_F32) {
    if (out)
      hipLaunchKernelGGL((rotate_fp4_kernel<N, SMLA_F32, true>), grid, blk, 0, st, x, rows, rotate, fp4, out, codes, scales);
    else
      hipLaunchKernelGGL((rotate_fp4_kernel<N, SMLA_F32, false>), grid, blk, 0, st, x, rows, rotate, fp4, out, codes, scales);
  } else {
    if (out)
      hipLaunchKernelGGL((rotate_fp4_kernel<N, SMLA_BF16, true>), grid, blk, 0, st, x, rows, rotate, fp4, out, codes, scales);
    else
      hipLaunchKernelGGL((rotate_fp4_kernel<N, SMLA_BF16, false>), grid, blk, 0, st, x, rows, rotate, fp4, out, codes, scales);
  }
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

}  // namespace

extern "C" int smla_rotate_fp4(const void* x, int x_dtype, int64_t rows, int64_t n, int flags, float* out,
                               uint8_t* codes, uint8_t* scales, void* stream) {
  if (!x) return SMLA_E_NULL;
  if (rows < 0 || n <= 0) return SMLA_E_SHAPE;
  if (flags & ~(SMLA_QAT_ROTATE | SMLA_QAT_FP4)) return SMLA_E_UNSUPPORTED;
  const int rotate = (flags & SMLA_QAT_ROTATE) ? 1 : 0, fp4 = (flags & SMLA_QAT_FP4) ? 1 : 0;
  if (!out && !codes) return SMLA_E_NULL;                  // nothing to write
  if ((codes != nullptr) != (scales != nullptr)) return SMLA_E_NULL;
  if (codes && !fp4) return SMLA_E_UNSUPPORTED;            // the stored form is the fp4 one
  if (x_dtype != SMLA_F32 && x_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  if ((n & (n - 1)) != 0 || n < 32 || n > 1024) return SMLA_E_UNSUPPORTED;
  // vector accesses: 16-byte aligned x, out and codes (a lane's 32 values, 16 code bytes)
  if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)codes & 15))
    return SMLA_E_UNSUPPORTED;
  if (rows == 0) return SMLA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (n) {
    case 32: return launch_rotate_fp4<32>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
    case 64: return launch_rotate_fp4<64>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
    case 128: return launch_rotate_fp4<128>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
    case 256: return launch_rotate_fp4<256>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
    case 512: return launch_rotate_fp4<512>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
    default: return launch_rotate_fp4<1024>(x, x_dtype, rows, rotate, fp4, out, codes, scales, st);
  }
}
