// Projections of the decode step: few tokens (T <= 32) against a large bf16 weight, on MFMA.
//
//  * linear_kernel<TT, ROPE, YDT> : y[t, n] = sum_k x'[t, g*K + k] * W[n, k] for the rows n of
//      group g = n / N (G groups of N rows; G = 1 is a plain linear).  With ROPE, x is the
//      attention output [T, heads, head_dim] and x' has the last rd dims of every head rotated
//      back (the inverse RoPE of oracle/decode_engine.py:118: pairs (x0, x1) at position pos[t]
//      become (x0 c + x1 s, x1 c - x0 s) in float32, rounded to bf16 like the reference's cast
//      to o's dtype).  This is v4mlx/mla.py:42-56 (o_grouped: G = 8 groups of 1024 rows over
//      4096-wide slices of o) and v4mlx/mla.py:16-18 (linear) for decode shapes.
//    Layout: one workgroup of 8 waves per 16 weight rows; wave w takes the K-slice
//    [w K/8, (w+1) K/8).  Per 64-wide K step a lane loads 32 contiguous bytes of one weight row
//    (row l % 16, k 16(l / 16) .. +15) and the same k range of token l % 16, and issues two
//    v_mfma_f32_16x16x32_bf16 (weights as A = 16 rows, tokens as B = 16 columns; the first MFMA
//    takes k 16q .. 16q+7 of every lane group q, the second 16q+8 .. 16q+15, the same
//    assignment on both operands).  Eight steps of loads are issued before their MFMAs.  The
//    eight partial 16x16 tiles are summed through LDS in wave order (deterministic).
//    HBM bound on the weights: N*G*K*2 bytes per launch; x (T*G*K*2 bytes) is re-read from L2
//    by every workgroup.
//  * rope_kernel : in-place RoPE (or its inverse) of the last rd dims of every head of
//      x [T, heads, head_dim] at positions pos[t] (ref_torch/norm_rope.py:53-62 with inverse).
#include "smla_internal.h"

namespace {

constexpr int kLinWaves = 8;
constexpr int kLinSteps = 8;  // K steps of 64 whose loads are in flight together

// float32 ops that the compiler may not contract into fma (the reference rounds every product;
// HIP's __fmul_rn is a plain multiply, contractable under the default fp-contract)
__device__ inline float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ inline float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ inline float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// rotate 8 (x0, x1) pairs held as 16 bf16 in two u32x4 words: inverse RoPE with cos/sin of
// pairs p0 .. p0+7 at one position
__device__ inline void inv_rope16(u32x4_t& w0, u32x4_t& w1, const float* __restrict__ cs, const float* __restrict__ sn) {
  const f32x4_t c0 = *(const f32x4_t*)cs, c1 = *(const f32x4_t*)(cs + 4);
  const f32x4_t s0 = *(const f32x4_t*)sn, s1 = *(const f32x4_t*)(sn + 4);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t word = j < 4 ? w0[j] : w1[j - 4];
    const float x0 = __uint_as_float(word << 16), x1 = __uint_as_float(word & 0xffff0000u);
    const float c = j < 4 ? c0[j] : c1[j - 4], s = j < 4 ? s0[j] : s1[j - 4];
    const float o0 = add_rn(mul_rn(x0, c), mul_rn(x1, s));
    const float o1 = sub_rn(mul_rn(x1, c), mul_rn(x0, s));
    const uint32_t r = pack_bf16x2(o0, o1);
    if (j < 4) w0[j] = r;
    else w1[j - 4] = r;
  }
}

// the same for 4 pairs in one u32x4 word
__device__ inline void inv_rope8(u32x4_t& w, const float* __restrict__ cs, const float* __restrict__ sn) {
  const f32x4_t c = *(const f32x4_t*)cs, sv = *(const f32x4_t*)sn;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float x0 = __uint_as_float(w[j] << 16), x1 = __uint_as_float(w[j] & 0xffff0000u);
    const float o0 = add_rn(mul_rn(x0, c[j]), mul_rn(x1, sv[j]));
    const float o1 = sub_rn(mul_rn(x1, c[j]), mul_rn(x0, sv[j]));
    w[j] = pack_bf16x2(o0, o1);
  }
}

template <int TT, bool ROPE, int YDT>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int T, int N, int K, int64_t ldx,
    const int32_t* __restrict__ pos, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int head_dim,
    int rd, void* __restrict__ y, int64_t ldy) {
  __shared__ f32x4_t red[kLinWaves][TT][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = lane & 15, q = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int64_t g = row0 / N;
  const int KW = K / kLinWaves;
  const int kbeg = wave * KW;
  const uint16_t* wp = w + (row0 + m) * (int64_t)K + kbeg + 16 * q;
  const uint16_t* xp[TT];
  const float* csp[TT];
  const float* snp[TT];
#pragma unroll
  for (int tt = 0; tt < TT; tt++) {
    const int t = min(tt * 16 + m, T - 1);  // columns past T compute on token T-1 and are not stored
    xp[tt] = x + t * ldx + g * K + kbeg + 16 * q;
    if constexpr (ROPE) {
      const int64_t p = pos[t];
      csp[tt] = cos_t + p * (rd / 2) + 8 * q;
      snp[tt] = sin_t + p * (rd / 2) + 8 * q;
    }
  }
  f32x4_t acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; tt++) acc[tt] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  const int nsteps = KW / 64;
  const int nope = head_dim - rd;
  for (int s0 = 0; s0 < nsteps; s0 += kLinSteps) {
    const int nb = min(kLinSteps, nsteps - s0);
    u32x4_t wv[kLinSteps][2], xv[TT][kLinSteps][2];
    if (nb == kLinSteps) {
#pragma unroll
      for (int s = 0; s < kLinSteps; s++) {
        wv[s][0] = *(const u32x4_t*)(wp + (s0 + s) * 64);
        wv[s][1] = *(const u32x4_t*)(wp + (s0 + s) * 64 + 8);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
          xv[tt][s][0] = *(const u32x4_t*)(xp[tt] + (s0 + s) * 64);
          xv[tt][s][1] = *(const u32x4_t*)(xp[tt] + (s0 + s) * 64 + 8);
        }
      }
    } else {  // a short last batch (K/8 not a multiple of 512): guarded, indexes stay compile-time
#pragma unroll
      for (int s = 0; s < kLinSteps; s++) {
        if (s >= nb) break;
        wv[s][0] = *(const u32x4_t*)(wp + (s0 + s) * 64);
        wv[s][1] = *(const u32x4_t*)(wp + (s0 + s) * 64 + 8);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
          xv[tt][s][0] = *(const u32x4_t*)(xp[tt] + (s0 + s) * 64);
          xv[tt][s][1] = *(const u32x4_t*)(xp[tt] + (s0 + s) * 64 + 8);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < kLinSteps; s++) {
      if (s >= nb) break;
      if constexpr (ROPE) {
        const int d0 = (kbeg + (s0 + s) * 64) % head_dim;  // the step is all rope dims or none
        if (d0 >= nope) {
#pragma unroll
          for (int tt = 0; tt < TT; tt++)
            inv_rope16(xv[tt][s][0], xv[tt][s][1], csp[tt] + (d0 - nope) / 2, snp[tt] + (d0 - nope) / 2);
        }
      }
#pragma unroll
      for (int tt = 0; tt < TT; tt++) {
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[s][0]), as_bf16x8(xv[tt][s][0]), acc[tt], 0, 0, 0);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[s][1]), as_bf16x8(xv[tt][s][1]), acc[tt], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < TT; tt++) red[wave][tt][lane] = acc[tt];
  __syncthreads();
  // thread (tt, lane) of the first TT waves sums the eight partial tiles in wave order; lane holds
  // rows 4q .. 4q+3 of token column m
  if (wave >= TT) return;
  const int tt = wave;
  f32x4_t sum = red[0][tt][lane];
#pragma unroll
  for (int v = 1; v < kLinWaves; v++) {
    const f32x4_t p = red[v][tt][lane];
    sum[0] += p[0];
    sum[1] += p[1];
    sum[2] += p[2];
    sum[3] += p[3];
  }
  const int t = tt * 16 + m;
  if (t >= T) return;
  const int64_t n0 = row0 + 4 * q;
  if constexpr (YDT == SMLA_BF16) {
    *(u32x2_t*)((uint16_t*)y + t * ldy + n0) = (u32x2_t){pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3])};
  } else {
    *(f32x4_t*)((float*)y + t * ldy + n0) = sum;
  }
}

// The same product with x staged once per workgroup in LDS (T <= 8, K <= 8192): K / (64 STEPS)
// waves, each streaming STEPS steps of 64 (its K slice) of the workgroup's 16 weight rows.  The
// staging loads are issued before the weight loads and every load before the first wait (vmcnt
// counts in order, so the weights stay in flight while x is written to LDS); x rows are padded by
// 16 bytes so that the 16 token rows read by one b128 pass fall in distinct banks.  Per-lane x
// registers drop from 64 VGPRs to 8 (16 with STEPS = 16), so two workgroups fit on a CU for
// K = 4096.
constexpr int kLdsMaxBytes = 160 * 1024;

template <int TX, bool ROPE, int YDT, int STEPS>
__global__ __launch_bounds__(STEPS == 16 ? 512 : 1024) void linear_lds_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int T, int N, int K, int64_t ldx,
    const int32_t* __restrict__ pos, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int head_dim,
    int rd, void* __restrict__ y, int64_t ldy) {
  extern __shared__ __align__(16) uint16_t xs[];  // [T][K + 8] bf16, later the partial tiles
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = lane & 15, q = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int64_t g = row0 / N;
  const int xst = K + 8;  // padded LDS row (elements)
  // 1. this thread's 16-byte chunks k = 8 (threadIdx.x + j blockDim.x) of every token row
  // (nw * 64 * 8 * STEPS / 8 == K)
  constexpr int XJ = STEPS / 8;
  u32x4_t xr[TX][XJ];
#pragma unroll
  for (int c = 0; c < TX; c++)
#pragma unroll
    for (int j = 0; j < XJ; j++)
      xr[c][j] = *(const u32x4_t*)(x + (int64_t)min(c, T - 1) * ldx + g * K + 8 * (threadIdx.x + j * blockDim.x));
  // keep the x loads ahead of the weight loads: vmcnt counts in issue order, so the x rows can then
  // be written to LDS while the weights are still in flight (unpinned, the compiler may issue the
  // weights first, and the wait for x then drains every load)
  __builtin_amdgcn_sched_barrier(0);
  // 2. the wave's weight slice: STEPS steps of 64 (two MFMA K-blocks of 32 each); lane (m, q)
  // takes k 8q .. 8q+7 of both blocks, so each load instruction reads 64 contiguous bytes of 16 rows
  const int kbeg = wave * (STEPS * 64);
  const uint16_t* wp = w + (row0 + m) * (int64_t)K + kbeg + 8 * q;
  u32x4_t wv[STEPS][2];
#pragma unroll
  for (int s = 0; s < STEPS; s++) {
    wv[s][0] = *(const u32x4_t*)(wp + s * 64);
    wv[s][1] = *(const u32x4_t*)(wp + s * 64 + 32);
  }
  __builtin_amdgcn_sched_barrier(0);  // every weight load issued before the first wait for x
  // 3. x into LDS, all TX rows (rows past T repeat row T-1 and are not read); a guard here would
  // let the compiler sink the row's loads into it, behind the weight loads
#pragma unroll
  for (int c = 0; c < TX; c++)
#pragma unroll
    for (int j = 0; j < XJ; j++) *(u32x4_t*)(xs + c * xst + 8 * (threadIdx.x + j * blockDim.x)) = xr[c][j];
  __syncthreads();
  // 4. MFMAs: token column m reads its row (rows past T read row T-1 and are not stored)
  const uint16_t* xrow = xs + min(m, T - 1) * xst + kbeg + 8 * q;
  const float* csp = nullptr;
  const float* snp = nullptr;
  if constexpr (ROPE) {
    const int64_t p = pos[min(m, T - 1)];
    csp = cos_t + p * (rd / 2) + 4 * q;
    snp = sin_t + p * (rd / 2) + 4 * q;
  }
  const int nope = head_dim - rd;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < STEPS; s++) {
    u32x4_t x0 = *(const u32x4_t*)(xrow + s * 64), x1 = *(const u32x4_t*)(xrow + s * 64 + 32);
    if constexpr (ROPE) {
      const int d0 = (kbeg + s * 64) % head_dim;  // the step is all rope dims or none
      if (d0 >= nope) {  // pairs (d0 - nope)/2 + 4q .. +3 and 16 further
        inv_rope8(x0, csp + (d0 - nope) / 2, snp + (d0 - nope) / 2);
        inv_rope8(x1, csp + (d0 - nope) / 2 + 16, snp + (d0 - nope) / 2 + 16);
      }
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[s][0]), as_bf16x8(x0), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[s][1]), as_bf16x8(x1), acc, 0, 0, 0);
  }
  // 5. partial tiles through LDS (over the x rows, after every wave has read them), summed in wave order
  __syncthreads();
  f32x4_t* red = (f32x4_t*)xs;
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4_t sum = red[lane];
  for (int v = 1; v < nw; v++) {
    const f32x4_t p = red[v * 64 + lane];
    sum[0] += p[0];
    sum[1] += p[1];
    sum[2] += p[2];
    sum[3] += p[3];
  }
  if (m >= T) return;
  const int64_t n0 = row0 + 4 * q;
  if constexpr (YDT == SMLA_BF16) {
    *(u32x2_t*)((uint16_t*)y + m * ldy + n0) = (u32x2_t){pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3])};
  } else {
    *(f32x4_t*)((float*)y + m * ldy + n0) = sum;
  }
}

template <int TX, bool ROPE, int YDT, int STEPS>
int launch_linear_lds(const uint16_t* x, const uint16_t* w, int64_t T, int64_t G, int64_t N, int64_t K, int64_t ldx,
                      const int32_t* pos, const float* cos_t, const float* sin_t, int head_dim, int rd, void* y,
                      hipStream_t st) {
  auto kern = linear_lds_kernel<TX, ROPE, YDT, STEPS>;
  static std::atomic<uint64_t> lds_attr{0};  // devices whose limit is raised
  if (hipError_t e = smla_set_dynamic_lds((const void*)kern, kLdsMaxBytes, lds_attr); e != hipSuccess) return (int)e;
  const int nw = (int)(K / (STEPS * 64));
  const int64_t xbytes = TX * (K + 8) * 2, rbytes = (int64_t)nw * 64 * 16;
  const size_t lds = (size_t)(xbytes > rbytes ? xbytes : rbytes);
  hipLaunchKernelGGL(kern, dim3((unsigned)(G * N / 16)), dim3(64 * nw), lds, st, x, w, (int)T, (int)N, (int)K, ldx,
                     pos, cos_t, sin_t, head_dim, rd, y, G * N);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

// the LDS form applies: T <= 8, K a multiple of 512 of at most 16 waves (x then fits: 8 rows of
// at most 8200 bf16)
bool lds_form(int64_t T, int64_t K) { return T <= 8 && K % 512 == 0 && K / 512 <= 16; }
// K steps of 64 per wave: 16 for K = 8192 (8 waves of 512 threads, each with 32 weight loads in
// flight; the 16-wave form streams 6 % slower), else 8
int lds_steps(int64_t K) { return (K % 1024 == 0 && K / 1024 == 8) ? 16 : 8; }

// one thread per (token, head, pair)
template <int XDT>
__global__ __launch_bounds__(256) void rope_kernel(void* __restrict__ x, int64_t T, int heads, int head_dim, int rd,
                                                   const int32_t* __restrict__ pos, const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, int inverse) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int half = rd / 2;
  if (i >= T * heads * half) return;
  const int pr = (int)(i % half);
  const int64_t th = i / half;  // token * heads + head
  const int64_t t = th / heads;
  const int64_t e = th * head_dim + (head_dim - rd) + 2 * pr;
  const float c = cos_t[(int64_t)pos[t] * half + pr];
  const float s = inverse ? -sin_t[(int64_t)pos[t] * half + pr] : sin_t[(int64_t)pos[t] * half + pr];
  float x0, x1;
  if constexpr (XDT == SMLA_BF16) {
    const uint32_t wd = *(const uint32_t*)((const uint16_t*)x + e);
    x0 = __uint_as_float(wd << 16);
    x1 = __uint_as_float(wd & 0xffff0000u);
  } else {
    const f32x2_t v = *(const f32x2_t*)((const float*)x + e);
    x0 = v[0];
    x1 = v[1];
  }
  // ref_torch/norm_rope.py:53-62: (x0 + i x1) (c + i s), each product rounded
  const float o0 = sub_rn(mul_rn(x0, c), mul_rn(x1, s));
  const float o1 = add_rn(mul_rn(x0, s), mul_rn(x1, c));
  if constexpr (XDT == SMLA_BF16) *(uint32_t*)((uint16_t*)x + e) = pack_bf16x2(o0, o1);
  else *(f32x2_t*)((float*)x + e) = (f32x2_t){o0, o1};
}

template <bool ROPE, int YDT>
int launch_linear_t(const uint16_t* x, const uint16_t* w, int64_t T, int64_t G, int64_t N, int64_t K, int64_t ldx,
                    const int32_t* pos, const float* cos_t, const float* sin_t, int head_dim, int rd, void* y,
                    hipStream_t st) {
  if (lds_form(T, K))
    return lds_steps(K) == 16
               ? launch_linear_lds<8, ROPE, YDT, 16>(x, w, T, G, N, K, ldx, pos, cos_t, sin_t, head_dim, rd, y, st)
               : launch_linear_lds<8, ROPE, YDT, 8>(x, w, T, G, N, K, ldx, pos, cos_t, sin_t, head_dim, rd, y, st);
  const dim3 grid((unsigned)(G * N / 16)), blk(64 * kLinWaves);
  if (T <= 16)
    hipLaunchKernelGGL((linear_kernel<1, ROPE, YDT>), grid, blk, 0, st, x, w, (int)T, (int)N, (int)K, ldx, pos, cos_t,
                       sin_t, head_dim, rd, y, G * N);
  else
    hipLaunchKernelGGL((linear_kernel<2, ROPE, YDT>), grid, blk, 0, st, x, w, (int)T, (int)N, (int)K, ldx, pos, cos_t,
                       sin_t, head_dim, rd, y, G * N);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

int launch_linear(const void* x, const void* w, int64_t T, int64_t G, int64_t N, int64_t K, const int32_t* pos,
                  const float* cos_t, const float* sin_t, int head_dim, int rd, void* y, int y_dtype, hipStream_t st) {
  const uint16_t* xb = (const uint16_t*)x;
  const uint16_t* wb = (const uint16_t*)w;
  const int64_t ldx = G * K;
  if (pos) {
    if (y_dtype == SMLA_BF16)
      return launch_linear_t<true, SMLA_BF16>(xb, wb, T, G, N, K, ldx, pos, cos_t, sin_t, head_dim, rd, y, st);
    return launch_linear_t<true, SMLA_F32>(xb, wb, T, G, N, K, ldx, pos, cos_t, sin_t, head_dim, rd, y, st);
  }
  if (y_dtype == SMLA_BF16)
    return launch_linear_t<false, SMLA_BF16>(xb, wb, T, G, N, K, ldx, nullptr, nullptr, nullptr, 0, 0, y, st);
  return launch_linear_t<false, SMLA_F32>(xb, wb, T, G, N, K, ldx, nullptr, nullptr, nullptr, 0, 0, y, st);
}

// The decode form (the weight-streaming kernels above) takes up to 32 bf16 token rows with N % 16 == 0
// and K % 512 == 0; everything else goes to the tiled MFMA GEMM (gemm.hip): bf16 or fp32 operands,
// rows of a multiple of 16 bytes (K % 8 bf16, K % 4 fp32).
bool decode_form(int x_dtype, int64_t T, int64_t N, int64_t K) {
  return x_dtype == SMLA_BF16 && T <= 32 && N % 16 == 0 && K % (64 * kLinWaves) == 0;
}

int check_linear(const void* x, int x_dtype, const void* w, int w_dtype, int64_t T, int64_t G, int64_t N, int64_t K,
                 const void* y, int y_dtype) {
  if (!x || !w || !y) return SMLA_E_NULL;
  if (T <= 0 || G <= 0 || N <= 0 || K <= 0) return SMLA_E_SHAPE;
  if (x_dtype != w_dtype || (x_dtype != SMLA_BF16 && x_dtype != SMLA_F32) ||
      (y_dtype != SMLA_BF16 && y_dtype != SMLA_F32))
    return SMLA_E_DTYPE;
  if (G * N / 16 > 0x7fffffff || G * K > 0x7fffffff || T > 0x7fffffff / 2) return SMLA_E_UNSUPPORTED;
  if (!decode_form(x_dtype, T, N, K) && K % (x_dtype == SMLA_BF16 ? 8 : 4) != 0) return SMLA_E_UNSUPPORTED;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)y & 15)) return SMLA_E_UNSUPPORTED;
  return SMLA_OK;
}

int check_rope_args(const int32_t* pos, const float* cos_t, const float* sin_t, int64_t n_pos, int64_t heads,
                    int64_t head_dim, int64_t rd) {
  if (!pos || !cos_t || !sin_t) return SMLA_E_NULL;
  if (n_pos <= 0 || heads <= 0 || head_dim <= 0 || rd <= 0 || rd > head_dim || rd % 2 != 0) return SMLA_E_SHAPE;
  return SMLA_OK;
}

}  // namespace

extern "C" int smla_linear(const void* x, int x_dtype, const void* w, int w_dtype, int64_t T, int64_t G, int64_t N,
                           int64_t K, void* y, int y_dtype, void* stream) {
  int rc = check_linear(x, x_dtype, w, w_dtype, T, G, N, K, y, y_dtype);
  if (rc) return rc;
  if (!decode_form(x_dtype, T, N, K))
    return launch_gemm_tiled(x, G * K, x_dtype == SMLA_F32, w, T, G, N, K, nullptr, nullptr, nullptr, 0, y, y_dtype,
                             (hipStream_t)stream);
  return launch_linear(x, w, T, G, N, K, nullptr, nullptr, nullptr, 0, 0, y, y_dtype, (hipStream_t)stream);
}

extern "C" int smla_rope(void* x, int x_dtype, int64_t T, int64_t heads, int64_t head_dim, int64_t rd,
                         const int32_t* pos, const float* cos_t, const float* sin_t, int64_t n_pos, int inverse,
                         void* stream) {
  if (!x) return SMLA_E_NULL;
  if (T < 0) return SMLA_E_SHAPE;
  int rc = check_rope_args(pos, cos_t, sin_t, n_pos, heads, head_dim, rd);
  if (rc) return rc;
  if (x_dtype != SMLA_BF16 && x_dtype != SMLA_F32) return SMLA_E_DTYPE;
  if ((head_dim - rd) % 2 != 0 || ((uintptr_t)x & 7)) return SMLA_E_UNSUPPORTED;
  const int64_t n = T * heads * (rd / 2);
  if (n == 0) return SMLA_OK;
  if ((n + 255) / 256 > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (x_dtype == SMLA_BF16)
    hipLaunchKernelGGL(rope_kernel<SMLA_BF16>, grid, dim3(256), 0, (hipStream_t)stream, x, T, (int)heads, (int)head_dim,
                       (int)rd, pos, cos_t, sin_t, inverse);
  else
    hipLaunchKernelGGL(rope_kernel<SMLA_F32>, grid, dim3(256), 0, (hipStream_t)stream, x, T, (int)heads, (int)head_dim,
                       (int)rd, pos, cos_t, sin_t, inverse);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

extern "C" int smla_o_proj(const void* o, int o_dtype, const int32_t* pos, const float* cos_t, const float* sin_t,
                           int64_t n_pos, int64_t T, int64_t heads, int64_t head_dim, int64_t rd, int64_t G, int64_t R,
                           const void* wo_a, const void* wo_b, int w_dtype, int64_t dim, void* mid, void* y,
                           int y_dtype, void* stream) {
  if (!o || !wo_a || !wo_b || !mid || !y) return SMLA_E_NULL;
  if (T <= 0 || heads <= 0 || head_dim <= 0 || G <= 0 || R <= 0 || dim <= 0) return SMLA_E_SHAPE;
  if ((heads * head_dim) % G != 0) return SMLA_E_SHAPE;
  const int64_t Kg = heads * head_dim / G;  // width of one group's slice of o
  if (o_dtype != SMLA_BF16 || w_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  int rc = check_linear(o, o_dtype, wo_a, w_dtype, T, G, R, Kg, mid, SMLA_BF16);
  if (rc) return rc;
  rc = check_linear(mid, SMLA_BF16, wo_b, w_dtype, T, 1, dim, G * R, y, y_dtype);
  if (rc) return rc;
  const bool dform = decode_form(o_dtype, T, R, Kg);
  if (pos) {
    rc = check_rope_args(pos, cos_t, sin_t, n_pos, heads, head_dim, rd);
    if (rc) return rc;
    // every 64-wide K step lies inside one head, all rope dims or none; the tiled GEMM rotates
    // exactly the last 64 dims of each head
    if (head_dim % 64 != 0 || rd % 64 != 0 || Kg % head_dim != 0 || (!dform && rd != 64)) return SMLA_E_UNSUPPORTED;
  }
  hipStream_t st = (hipStream_t)stream;
  if (dform)
    rc = launch_linear(o, wo_a, T, G, R, Kg, pos, cos_t, sin_t, (int)head_dim, (int)rd, mid, SMLA_BF16, st);
  else
    rc = launch_gemm_tiled(o, G * Kg, false, wo_a, T, G, R, Kg, pos, cos_t, sin_t, head_dim, mid, SMLA_BF16, st);
  if (rc) return rc;
  if (!decode_form(SMLA_BF16, T, dim, G * R))
    return launch_gemm_tiled(mid, G * R, false, wo_b, T, 1, dim, G * R, nullptr, nullptr, nullptr, 0, y, y_dtype, st);
  return launch_linear(mid, wo_b, T, 1, dim, G * R, nullptr, nullptr, nullptr, 0, 0, y, y_dtype, st);
}
