// KV compressor kernels.
//
//  * block_mean_kernel : out[b,g,:] = (x[rg] + ... + x[rg+r-1]) * (1/r), fp32 in row order.
//                        HBM bound: reads N*D*es, writes N/r*D*es'.  16-byte vector lanes.
//  * gated_pool_kernel : ref_torch/compressor.py:41-49 from the projections — overlapped
//                        per-channel softmax over 2r slots (slots 0..r-1: previous group's first
//                        half channels, r..2r-1: own group's second half, ref_torch/compressor.py:
//                        12-18; group 0 has no previous slots), weighted sum, RMSNorm, RoPE of the
//                        last rd channels at position g*r, then optionally the fp8 round trip of
//                        the first d-rd channels (v4mlx/compressor.py:60-62) or, for the indexer
//                        compressor, the Hadamard rotation and fp4 round trip of all d channels
//                        (v4mlx/compressor.py:57-59).  One workgroup of d/2 threads per output row.
//  * ring_step_kernel  : oracle/decode_engine.py:96-105 — write the token into ring slot
//                        r + pos%r, and on a group boundary pool the ring into one row (same
//                        epilogue, RoPE position pos+1-r), append it to the compressed cache and
//                        shift the ring.  One workgroup per sequence; no host synchronisation.
//  * row_epilogue_kernel : the same epilogue on rows the caller projected (oracle/decode_engine.py:
//                        78-83: the q_a RMSNorm, the weightless per-head q norm + RoPE, the kv row's
//                        RMSNorm + RoPE + fp8 round trip written straight into its window-cache row).
//  * decode_ids_kernel : oracle/decode_engine.py:110-114, the decode id list (window rows, then every
//                        visible compressed row), plus the bf16 copy of a row the ring just emitted.
//  * quant_kernel      : act_quant_sim's stored form (v4mlx/compressor.py:11-20): per 64-block pow2
//                        scale and e4m3 codes, 16 lanes per block.
#include "smla_internal.h"

namespace {

constexpr int kPoolThreads = 256;

template <int XDT, int ODT>
__global__ void block_mean_kernel(const void* __restrict__ x, int64_t B, int64_t N, int64_t D, int ratio,
                                  void* __restrict__ out) {
  // one thread per 8 output elements.  Rows are read once and the pooled rows are not read back by
  // this launch: both go through nontemporal accesses, which are coalesced here (a wave reads and
  // writes 1 KB runs), so they stream past the L2 instead of filling it (and leave no dirty lines
  // for the kernel's end to write back): 69 -> 59 us for [8,32768,576] bf16, 5.4 -> 6.4 TB/s
  const int64_t G = N / ratio;
  const int64_t per_row = D / 8;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * G * per_row) return;
  int64_t c = i % per_row;
  int64_t bg = i / per_row;
  int64_t b = bg / G, g = bg % G;
  float acc[8];
  const float inv = 1.0f / (float)ratio;
  for (int j = 0; j < ratio; j++) {
    int64_t row = b * N + g * ratio + j;
    float v[8];
    if constexpr (XDT == SMLA_BF16) {
      u32x4_t w = __builtin_nontemporal_load((const u32x4_t*)((const uint16_t*)x + row * D + c * 8));
#pragma unroll
      for (int k = 0; k < 4; k++) {
        v[2 * k] = bf16_bits_to_f32((uint16_t)(w[k] & 0xffffu));
        v[2 * k + 1] = bf16_bits_to_f32((uint16_t)(w[k] >> 16));
      }
    } else {
      const f32x4_t* p = (const f32x4_t*)((const float*)x + row * D + c * 8);
      f32x4_t a = __builtin_nontemporal_load(p), bq = __builtin_nontemporal_load(p + 1);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        v[k] = a[k];
        v[4 + k] = bq[k];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = (j == 0) ? v[k] : acc[k] + v[k];
  }
  int64_t orow = b * G + g;
  if constexpr (ODT == SMLA_BF16) {
    u32x4_t w;
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = pack_bf16x2(acc[2 * k] * inv, acc[2 * k + 1] * inv);
    __builtin_nontemporal_store(w, (u32x4_t*)((uint16_t*)out + orow * D + c * 8));
  } else {
    f32x4_t a, bq;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      a[k] = acc[k] * inv;
      bq[k] = acc[4 + k] * inv;
    }
    f32x4_t* p = (f32x4_t*)((float*)out + orow * D + c * 8);
    __builtin_nontemporal_store(a, p);
    __builtin_nontemporal_store(bq, p + 1);
  }
}

__device__ inline float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); w++) s += red[w];
  __syncthreads();
  return s;
}

// Epilogue shared by the prefill pool, the ring step and the row epilogue: RMSNorm with the
// weights in `e`, RoPE of the last rd channels by the pair in `e` (the row's position), then the
// `sim` quantisation (SMLA_SIM_*).  Thread t owns channels 2t
// and 2t+1 (d == 2*blockDim.x).  `v0,v1` are the pooled values; the result is written to dst[2t],
// dst[2t+1].  `xch` (d floats of LDS) carries the rotation stages that cross waves.
struct EpiOperands {
  float w0, w1;  // norm weights of channels 2t, 2t+1 (1 for the weightless norm: an exact product)
  float cs, sn;  // rotation of the pair when it is a rope channel pair
};

// The epilogue's operands from memory, loaded by the caller ahead of (or beside) its own loads so
// that their latency overlaps them rather than following the norm's reduction.
__device__ inline EpiOperands epilogue_weights(const float* __restrict__ norm_w) {
  const int c0 = 2 * threadIdx.x;
  EpiOperands e{1.f, 1.f, 1.f, 0.f};
  if (norm_w) {
    e.w0 = norm_w[c0];
    e.w1 = norm_w[c0 + 1];
  }
  return e;
}

__device__ inline void epilogue_rotation(EpiOperands& e, int d, int rd, const float* __restrict__ cos_t,
                                         const float* __restrict__ sin_t, int64_t pos) {
  const int c0 = 2 * threadIdx.x;
  if (c0 >= d - rd) {
    const int64_t i = pos * (rd / 2) + ((c0 - (d - rd)) >> 1);
    e.cs = cos_t[i];
    e.sn = sin_t[i];
  }
}

__device__ inline void pool_epilogue(float v0, float v1, int d, int rd, float eps, int sim, const EpiOperands& e,
                                     float* red, float* xch, float* dst) {
  const int t = threadIdx.x;
  const int c0 = 2 * t;
  float ss = block_sum(v0 * v0 + v1 * v1, red);
  float inv = rsqrtf(ss / (float)d + eps);
  float y0 = e.w0 * (v0 * inv);
  float y1 = e.w1 * (v1 * inv);
  const int nope = d - rd;
  if (c0 >= nope) {
    const float cs = e.cs, sn = e.sn;
    float r0 = y0 * cs - y1 * sn;
    float r1 = y0 * sn + y1 * cs;
    y0 = r0;
    y1 = r1;
  }
  if (sim == SMLA_SIM_FP8 && c0 < nope) {
    // 64-channel blocks = 32 consecutive threads (half a wave)
    float a = fmaxf(fabsf(y0), fabsf(y1));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
    a = fmaxf(a, 1e-4f);
    float s = pow2_ceil(a / 448.0f);
    float z0 = fminf(fmaxf(y0 / s, -448.f), 448.f);
    float z1 = fminf(fmaxf(y1 / s, -448.f), 448.f);
    // e4m3 round trip by the gfx950 converters (round-to-nearest-even encode of the clamped
    // values, exact decode): the codes of f32_to_e4m3
    const f32x2_t q = __builtin_amdgcn_cvt_pk_f32_fp8(__builtin_amdgcn_cvt_pk_fp8_f32(z0, z1, 0, false), false);
    y0 = q[0] * s;
    y1 = q[1] * s;
  } else if (sim == SMLA_SIM_ROTATE_FP4) {
    // Hadamard butterfly over the d channels (v4mlx/qat.py:8-20): stage h pairs channels c and
    // c + h.  h = 1 is inside the thread; h = 2m pairs thread t with t ^ m, in the same wave for
    // m < 64, through LDS beyond.
    float a = y0 + y1, b = y0 - y1;
    y0 = a;
    y1 = b;
    for (int m = 1; m <= 32 && 4 * m <= d; m *= 2) {
      const float o0 = __shfl_xor(y0, m, 64), o1 = __shfl_xor(y1, m, 64);
      const bool up = t & m;
      y0 = up ? o0 - y0 : y0 + o0;
      y1 = up ? o1 - y1 : y1 + o1;
    }
    for (int m = 64; 4 * m <= d; m *= 2) {
      xch[c0] = y0;
      xch[c0 + 1] = y1;
      __syncthreads();
      const int pc = 2 * (t ^ m);
      const float o0 = xch[pc], o1 = xch[pc + 1];
      __syncthreads();
      const bool up = t & m;
      y0 = up ? o0 - y0 : y0 + o0;
      y1 = up ? o1 - y1 : y1 + o1;
    }
    const float hs = hadamard_scale(__builtin_ctz((unsigned)d));
    y0 *= hs;
    y1 *= hs;
    // fp4 round trip per 32-channel block = 16 threads (one DPP row), v4mlx/qat.py:23-31
    float am = fmaxf(fabsf(y0), fabsf(y1));
    am = fmaxf(am, dpp_f<0xB1>(am));
    am = fmaxf(am, dpp_f<0x4E>(am));
    am = fmaxf(am, dpp_f<0x141>(am));
    am = fmaxf(am, dpp_f<0x140>(am));
    const int k = fp4_scale_exp(am);
    const float si = exp2i_f32(-k), s = exp2i_f32(k);
    y0 = e2m1_to_f32(f32_to_e2m1(fminf(fmaxf(y0 * si, -6.f), 6.f))) * s;
    y1 = e2m1_to_f32(f32_to_e2m1(fminf(fmaxf(y1 * si, -6.f), 6.f))) * s;
  }
  dst[c0] = y0;
  dst[c0 + 1] = y1;
}

// slot-weighted pooling for one channel over `ns` (value, score) pairs held in registers
template <int MAXS>
__device__ inline float softmax_pool(const float* v, const float* s, int ns) {
  float m = -SMLA_INF;
  for (int j = 0; j < ns; j++) m = fmaxf(m, s[j]);
  float den = 0.f, num = 0.f;
  for (int j = 0; j < ns; j++) {
    float e = __expf(s[j] - m);
    den += e;
    num = fmaf(v[j], e, num);
  }
  return num / den;
}

constexpr int kMaxRatio = 8;

__global__ __launch_bounds__(kPoolThreads) void gated_pool_kernel(
    const float* __restrict__ kv, const float* __restrict__ score, const float* __restrict__ ape,
    const float* __restrict__ norm_w, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t N,
    int d, int ratio, int rd, float eps, int sim, float* __restrict__ out) {
  __shared__ float red[kPoolThreads / 64];
  __shared__ float xch[2 * kPoolThreads];
  const int64_t G = N / ratio;
  const int64_t bg = blockIdx.x;
  const int64_t b = bg / G, g = bg % G;
  const int t = threadIdx.x;
  const int64_t two_d = 2 * (int64_t)d;
  // channels c0 = 2t and c0 + 1 of every slot in one 8-byte load each (kv, score, ape)
  const int c0 = 2 * t;
  EpiOperands eo = epilogue_weights(norm_w);
  epilogue_rotation(eo, d, rd, cos_t, sin_t, g * ratio);
  float v0[2 * kMaxRatio], s0[2 * kMaxRatio], v1[2 * kMaxRatio], s1[2 * kMaxRatio];
  int ns = 0;
  auto slot = [&](int64_t row, int64_t off, int j) __attribute__((always_inline)) {
    const f32x2_t kvv = *(const f32x2_t*)(kv + row * two_d + off + c0);
    const f32x2_t sc = *(const f32x2_t*)(score + row * two_d + off + c0);
    const f32x2_t ap = *(const f32x2_t*)(ape + j * two_d + off + c0);
    v0[ns] = kvv[0];
    v1[ns] = kvv[1];
    s0[ns] = sc[0] + ap[0];
    s1[ns] = sc[1] + ap[1];
    ns++;
  };
  if (g > 0)
    for (int j = 0; j < ratio; j++) slot(b * N + (g - 1) * ratio + j, 0, j);
  for (int j = 0; j < ratio; j++) slot(b * N + g * ratio + j, d, j);
  float pooled[2];
  pooled[0] = softmax_pool<2 * kMaxRatio>(v0, s0, ns);
  pooled[1] = softmax_pool<2 * kMaxRatio>(v1, s1, ns);
  pool_epilogue(pooled[0], pooled[1], d, rd, eps, sim, eo, red, xch,
                out + bg * (int64_t)d);
}

// the ring step of sequence b, run by one workgroup of d/2 threads
__device__ __attribute__((always_inline)) inline void ring_step_body(int64_t b,
    float* __restrict__ ring_kv, float* __restrict__ ring_sc, const float* __restrict__ kv_p,
    const float* __restrict__ score_p, const int32_t* __restrict__ pos_arr, const float* __restrict__ ape,
    const float* __restrict__ norm_w, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int64_t n_pos, int d, int ratio, int rd, float eps, int sim, float* __restrict__ comp, int64_t comp_cap,
    int64_t ldp) {
  __shared__ float red[kPoolThreads / 64];
  __shared__ float xch[2 * kPoolThreads];
  const int t = threadIdx.x;
  const int64_t two_d = 2 * (int64_t)d;
  const int64_t pos = pos_arr[b];
  if (pos < 0 || pos + 1 - ratio >= n_pos) return;  // block-uniform guard
  float* rk = ring_kv + b * (2 * ratio) * two_d;
  float* rs = ring_sc + b * (2 * ratio) * two_d;
  const int ph = (int)(pos % ratio);
  const int slot = ratio + ph;
  // thread t owns channels c0 = 2t, 2t+1 of both halves (h = 0: c0, h = 1: d + c0) of every slot,
  // so no other thread reads or writes what it touches: every ring value it needs is loaded up
  // front (8-byte loads of its two channels, all independent) and the emit, pool and shift run
  // from registers
  const int c0 = 2 * t;
  f32x2_t nk[2], ns[2];  // the new token's slot
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int64_t cc = c0 + h * (int64_t)d;
    nk[h] = *(const f32x2_t*)(kv_p + b * ldp + cc);
    const f32x2_t sp = *(const f32x2_t*)(score_p + b * ldp + cc);
    const f32x2_t ap = *(const f32x2_t*)(ape + ph * two_d + cc);
    ns[h][0] = sp[0] + ap[0];
    ns[h][1] = sp[1] + ap[1];
  }
  if ((pos + 1) % ratio != 0) {  // block-uniform: no row completes, store the slot
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int64_t cc = c0 + h * (int64_t)d;
      *(f32x2_t*)(rk + slot * two_d + cc) = nk[h];
      *(f32x2_t*)(rs + slot * two_d + cc) = ns[h];
    }
    return;
  }
  EpiOperands eo = epilogue_weights(norm_w);
  epilogue_rotation(eo, d, rd, cos_t, sin_t, pos + 1 - ratio);
  // a row completes: slot 2r-1 is the new token; the pool reads the first halves of slots
  // 0..r-1 and the second halves of slots r..2r-1, the shift moves both halves of slots r..2r-1
  f32x2_t ok[kMaxRatio], os[kMaxRatio];                // first halves of slots 0..r-1
  f32x2_t hk[2][kMaxRatio], hs[2][kMaxRatio];          // both halves of slots r..2r-1
#pragma unroll
  for (int j = 0; j < kMaxRatio; j++) {
    if (j < ratio) {
      ok[j] = *(const f32x2_t*)(rk + j * two_d + c0);
      os[j] = *(const f32x2_t*)(rs + j * two_d + c0);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int64_t cc = c0 + h * (int64_t)d;
        if (j < ratio - 1) {
          hk[h][j] = *(const f32x2_t*)(rk + (ratio + j) * two_d + cc);
          hs[h][j] = *(const f32x2_t*)(rs + (ratio + j) * two_d + cc);
        } else {
          hk[h][j] = nk[h];
          hs[h][j] = ns[h];
        }
      }
    }
  }
  float pooled[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    float v[2 * kMaxRatio], sc[2 * kMaxRatio];
#pragma unroll
    for (int j = 0; j < kMaxRatio; j++) {
      if (j < ratio) {
        v[j] = ok[j][k];
        sc[j] = os[j][k];
        v[ratio + j] = hk[1][j][k];
        sc[ratio + j] = hs[1][j][k];
      }
    }
    pooled[k] = softmax_pool<2 * kMaxRatio>(v, sc, 2 * ratio);
  }
  // shift: slots r..2r-1 -> 0..r-1 (own channels only); slots r..2r-1 keep their values, the new
  // token included in slot 2r-1, as after a store-then-copy
#pragma unroll
  for (int j = 0; j < kMaxRatio; j++) {
    if (j < ratio) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int64_t cc = c0 + h * (int64_t)d;
        *(f32x2_t*)(rk + j * two_d + cc) = hk[h][j];
        *(f32x2_t*)(rs + j * two_d + cc) = hs[h][j];
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int64_t cc = c0 + h * (int64_t)d;
    *(f32x2_t*)(rk + (2 * ratio - 1) * two_d + cc) = nk[h];
    *(f32x2_t*)(rs + (2 * ratio - 1) * two_d + cc) = ns[h];
  }
  const int64_t grp = (pos + 1) / ratio - 1;
  __shared__ float rowbuf[2 * kPoolThreads];
  pool_epilogue(pooled[0], pooled[1], d, rd, eps, sim, eo, red, xch, rowbuf);
  if (grp < comp_cap) {
    float* dst = comp + (b * comp_cap + grp) * (int64_t)d;
    dst[2 * t] = rowbuf[2 * t];
    dst[2 * t + 1] = rowbuf[2 * t + 1];
  }
}

__global__ __launch_bounds__(kPoolThreads) void ring_step_kernel(
    float* __restrict__ ring_kv, float* __restrict__ ring_sc, const float* __restrict__ kv_p,
    const float* __restrict__ score_p, const int32_t* __restrict__ pos_arr, const float* __restrict__ ape,
    const float* __restrict__ norm_w, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int64_t n_pos, int d, int ratio, int rd, float eps, int sim, float* __restrict__ comp, int64_t comp_cap,
    int64_t ldp) {
  ring_step_body(blockIdx.x, ring_kv, ring_sc, kv_p, score_p, pos_arr, ape, norm_w, cos_t, sin_t, n_pos, d, ratio, rd, eps, sim, comp, comp_cap, ldp);
}

// 16 lanes per 64-element block (one DPP row), 4 elements per lane: vector loads, the block's
// abs-max by row reduction, x * (1/s) (exact: s is a power of two, so the product equals x / s),
// clamp to +-448, e4m3 round-to-nearest-even by the hardware converter
template <int XDT>
__global__ __launch_bounds__(256) void quant_kernel(const void* __restrict__ x, int64_t nblocks,
                                                    uint8_t* __restrict__ codes, float* __restrict__ scales) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk = t >> 4;
  const int sub = (int)(t & 15);
  const bool ok = blk < nblocks;
  const int64_t e0 = blk * 64 + sub * 4;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (ok) {
    if constexpr (XDT == SMLA_F32) {
      const f32x4_t w = *(const f32x4_t*)((const float*)x + e0);
      v[0] = w[0];
      v[1] = w[1];
      v[2] = w[2];
      v[3] = w[3];
    } else {
      const u32x2_t w = *(const u32x2_t*)((const uint16_t*)x + e0);
      v[0] = bf16_bits_to_f32((uint16_t)(w[0] & 0xffffu));
      v[1] = bf16_bits_to_f32((uint16_t)(w[0] >> 16));
      v[2] = bf16_bits_to_f32((uint16_t)(w[1] & 0xffffu));
      v[3] = bf16_bits_to_f32((uint16_t)(w[1] >> 16));
    }
  }
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  a = fmaxf(a, dpp_f<0xB1>(a));
  a = fmaxf(a, dpp_f<0x4E>(a));
  a = fmaxf(a, dpp_f<0x141>(a));
  a = fmaxf(a, dpp_f<0x140>(a));  // every lane of the 16-lane row: the block's abs-max
  a = fmaxf(a, 1e-4f);
  const float s = pow2_ceil(a / 448.0f);
  const float inv = 1.0f / s;
  if (!ok) return;
  // the gfx950 converter encodes OCP e4m3 with round-to-nearest-even; on the clamped values it
  // gives f32_to_e4m3's codes (checked on the device over every e4m3 value, every midpoint and
  // its neighbours, tiny values and signed zeros)
  float z[4];
#pragma unroll
  for (int by = 0; by < 4; by++) z[by] = fminf(fmaxf(v[by] * inv, -448.f), 448.f);
  int word = __builtin_amdgcn_cvt_pk_fp8_f32(z[0], z[1], 0, false);
  word = __builtin_amdgcn_cvt_pk_fp8_f32(z[2], z[3], word, true);
  *(uint32_t*)(codes + e0) = (uint32_t)word;
  if (sub == 0) scales[blk] = s;
}

}  // namespace

extern "C" int smla_block_mean_pool(const void* x, int x_dtype, int64_t B, int64_t N, int64_t D, int64_t ratio,
                                    void* out, int out_dtype, void* stream) {
  if (!x || !out) return SMLA_E_NULL;
  if (B <= 0 || N <= 0 || D <= 0 || ratio <= 0 || N < ratio) return SMLA_E_SHAPE;
  if (D % 8 != 0 || ratio > 64) return SMLA_E_UNSUPPORTED;
  if ((x_dtype != SMLA_F32 && x_dtype != SMLA_BF16) || (out_dtype != SMLA_F32 && out_dtype != SMLA_BF16))
    return SMLA_E_DTYPE;
  int64_t total = B * (N / ratio) * (D / 8);
  dim3 grid((unsigned)((total + 255) / 256)), blk(256);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == SMLA_BF16 && out_dtype == SMLA_BF16)
    hipLaunchKernelGGL((block_mean_kernel<SMLA_BF16, SMLA_BF16>), grid, blk, 0, st, x, B, N, D, (int)ratio, out);
  else if (x_dtype == SMLA_BF16)
    hipLaunchKernelGGL((block_mean_kernel<SMLA_BF16, SMLA_F32>), grid, blk, 0, st, x, B, N, D, (int)ratio, out);
  else if (out_dtype == SMLA_BF16)
    hipLaunchKernelGGL((block_mean_kernel<SMLA_F32, SMLA_BF16>), grid, blk, 0, st, x, B, N, D, (int)ratio, out);
  else
    hipLaunchKernelGGL((block_mean_kernel<SMLA_F32, SMLA_F32>), grid, blk, 0, st, x, B, N, D, (int)ratio, out);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

// d = 2 * threads with whole waves and at most kPoolThreads threads: 128, 256 or 512
static int check_pool_dims(int64_t d, int64_t ratio, int64_t rd, int sim) {
  if (d <= 0 || ratio <= 0 || rd <= 0 || rd > d || rd % 2 != 0) return SMLA_E_SHAPE;
  if ((d != 128 && d != 256 && d != 512) || ratio > kMaxRatio || (d - rd) % 64 != 0) return SMLA_E_UNSUPPORTED;
  if (sim != SMLA_SIM_NONE && sim != SMLA_SIM_FP8 && sim != SMLA_SIM_ROTATE_FP4) return SMLA_E_RANGE;
  return SMLA_OK;
}

extern "C" int smla_gated_pool(const float* kv, const float* score, const float* ape, const float* norm_w,
                               const float* cos_t, const float* sin_t, int64_t B, int64_t N, int64_t d, int64_t ratio,
                               int64_t rd, float eps, int sim, float* out, void* stream) {
  if (!kv || !score || !ape || !norm_w || !cos_t || !sin_t || !out) return SMLA_E_NULL;
  if (B <= 0 || N <= 0) return SMLA_E_SHAPE;
  int rc = check_pool_dims(d, ratio, rd, sim);
  if (rc) return rc;
  if (N % ratio != 0) return SMLA_E_SHAPE;
  // the kernel reads two adjacent channels of kv, score and ape in one 8-byte load
  if ((((uintptr_t)kv | (uintptr_t)score | (uintptr_t)ape) & 7) != 0) return SMLA_E_UNSUPPORTED;
  int64_t rows = B * (N / ratio);
  if (rows <= 0) return SMLA_OK;
  hipLaunchKernelGGL(gated_pool_kernel, dim3((unsigned)rows), dim3((unsigned)(d / 2)), 0, (hipStream_t)stream, kv,
                     score, ape, norm_w, cos_t, sin_t, N, (int)d, (int)ratio, (int)rd, eps, sim, out);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

// One workgroup of d/2 threads per input row r (fp32, d channels): pool_epilogue (RMSNorm with
// norm_w, or weightless when it is null; RoPE of the last rd channels at pos[r / rows_per_pos];
// the `sim` quantisation), written in out_dtype to row r of `out` or, when cache_rows > 0, to row
// pos mod cache_rows of sequence r / rows_per_pos of a cache [.., cache_rows, d]: a cache with a
// row per position keeps every row, a shorter one is a ring of the last cache_rows positions (the
// bounded window of oracle/v4_fast.py:93-96, winr[p % 128]).  A negative position, or one outside
// the rotation table, leaves the row unwritten.
// input row r, run by one workgroup of d/2 threads
__device__ __attribute__((always_inline)) inline void row_epilogue_body(int64_t r,
    const float* __restrict__ x, int d, int64_t ldx, int rows_per_pos,
    const int32_t* __restrict__ pos, const float* __restrict__ norm_w, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t n_pos, int rd, float eps, int sim, void* __restrict__ out, int out_dtype,
    int64_t cache_rows) {
  __shared__ float red[8];
  __shared__ float xch[1024];
  __shared__ float res[1024];
  const int t = threadIdx.x;
  // the row and the norm weights do not depend on the position: loaded beside it
  const float* xr = x + r * ldx;
  const float v0 = xr[2 * t], v1 = xr[2 * t + 1];
  EpiOperands eo = epilogue_weights(norm_w);
  const int64_t s = r / rows_per_pos;
  const int64_t p = pos ? (int64_t)pos[s] : 0;
  const bool ok = (rd == 0 || (p >= 0 && p < n_pos)) && (cache_rows == 0 || p >= 0);
  if (!ok) return;  // uniform over the workgroup
  if (rd) epilogue_rotation(eo, d, rd, cos_t, sin_t, p);
  pool_epilogue(v0, v1, d, rd, eps, sim, eo, red, xch, res);
  const int64_t orow = cache_rows > 0 ? s * cache_rows + p % cache_rows : r;
  if (out_dtype == SMLA_BF16)
    ((uint32_t*)out)[(orow * d) / 2 + t] = pack_bf16x2(res[2 * t], res[2 * t + 1]);
  else
    ((f32x2_t*)out)[(orow * d) / 2 + t] = f32x2_t{res[2 * t], res[2 * t + 1]};
}

__global__ __launch_bounds__(512) void row_epilogue_kernel(const float* __restrict__ x, int d, int64_t ldx, int rows_per_pos,
    const int32_t* __restrict__ pos, const float* __restrict__ norm_w, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t n_pos, int rd, float eps, int sim, void* __restrict__ out, int out_dtype,
    int64_t cache_rows) {
  row_epilogue_body(blockIdx.x, x, d, ldx, rows_per_pos, pos, norm_w, cos_t, sin_t, n_pos, rd, eps, sim, out, out_dtype, cache_rows);
}

// The decode step's kv row epilogue (into the window cache) and compressor ring step in one
// launch: both read only the input projection and share the thread layout (d/2 threads, channels
// 2t and 2t+1).  Workgroups 0..B-1 step the rings, workgroups B..2B-1 write the kv rows.
__global__ __launch_bounds__(kPoolThreads) void ring_kv_kernel(
    float* __restrict__ ring_kv, float* __restrict__ ring_sc, const float* __restrict__ kv_p,
    const float* __restrict__ score_p, const int32_t* __restrict__ pos_arr, const float* __restrict__ ape,
    const float* __restrict__ norm_w, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int64_t n_pos, int d, int ratio, int rd, float eps, int sim, float* __restrict__ comp, int64_t comp_cap,
    int64_t ldp, int64_t B,
    const float* __restrict__ kx, int64_t ldk, const float* __restrict__ k_norm, const float* __restrict__ k_cos,
    const float* __restrict__ k_sin, int64_t k_n_pos, int k_rd, float k_eps, int k_sim, void* __restrict__ k_cache,
    int k_dtype, int64_t k_cache_rows) {
  if ((int64_t)blockIdx.x < B)
    ring_step_body(blockIdx.x, ring_kv, ring_sc, kv_p, score_p, pos_arr, ape, norm_w, cos_t, sin_t, n_pos, d, ratio, rd, eps, sim, comp, comp_cap, ldp);
  else
    row_epilogue_body((int64_t)blockIdx.x - B, kx, d, ldk, 1, pos_arr, k_norm, k_cos, k_sin, k_n_pos, k_rd, k_eps,
                      k_sim, k_cache, k_dtype, k_cache_rows);
}

// ids [B, T] for sequences at positions pos[b]: columns 0..window-1 hold the rows of positions
// max(0, p-window+1)..p (then -1) in the raw source of n_raw rows, where position pp lives at row
// pp mod n_raw (a ring of n_raw >= window rows; the identity for a cache with a row per position),
// the rest n_raw + j for the (p+1)/ratio visible compressed rows j (then -1).  Workgroup column 0 also copies a row the ring emitted at this step
// ((p+1) % ratio == 0) from comp32 to comp_out in bf16.
// column block bx of sequence b's ids, run by one workgroup of 256 threads
__device__ __attribute__((always_inline)) inline void decode_ids_body(int64_t bx, int64_t b,
    const int32_t* __restrict__ pos, int window, int ratio, int64_t n_raw, int64_t ncomp, int64_t T,
    int32_t* __restrict__ ids, const float* __restrict__ comp32, uint16_t* __restrict__ comp_out, int d) {
  const int64_t p = pos[b];
  const int64_t j = bx * 256 + threadIdx.x;
  if (j < T) {
    int64_t id;
    if (j < window) {
      const int64_t lo = p - window + 1 > 0 ? p - window + 1 : 0;
      id = lo + j <= p ? (int64_t)((uint64_t)(lo + j) % (uint64_t)n_raw) : -1;
    } else {
      const int64_t c = j - window;
      id = (ratio > 0 && c < ncomp && c < (p + 1) / ratio) ? n_raw + c : -1;
    }
    ids[b * T + j] = (int32_t)id;
  }
  if (bx == 0 && comp_out && ratio > 0 && p >= 0 && (p + 1) % ratio == 0) {
    const int64_t row = (p + 1) / ratio - 1;
    if (row < ncomp)
      for (int c = threadIdx.x; c < d; c += 256)
        comp_out[(b * ncomp + row) * d + c] = bf16_rne(comp32[(b * ncomp + row) * d + c]);
  }
}

__global__ __launch_bounds__(256) void decode_ids_kernel(const int32_t* __restrict__ pos, int window, int ratio, int64_t n_raw, int64_t ncomp, int64_t T,
    int32_t* __restrict__ ids, const float* __restrict__ comp32, uint16_t* __restrict__ comp_out, int d) {
  decode_ids_body(blockIdx.x, blockIdx.y, pos, window, ratio, n_raw, ncomp, T, ids, comp32, comp_out, d);
}

// The decode step's per-head q epilogue (d = 512: 256 threads) and its id build in one launch:
// workgroups 0..rows-1 take the q rows, the next nx * B the id column blocks (nx = ceil(T/256)),
// sequence-major.
__global__ __launch_bounds__(256) void q_ids_kernel(
    const float* __restrict__ x, int d, int64_t ldx, int rows_per_pos, const int32_t* __restrict__ qpos,
    const float* __restrict__ norm_w, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t n_pos,
    int rd, float eps, int sim, void* __restrict__ out, int out_dtype, int64_t cache_rows, int64_t rows, int64_t nx,
    const int32_t* __restrict__ pos, int window, int ratio, int64_t n_raw, int64_t ncomp, int64_t T,
    int32_t* __restrict__ ids, const float* __restrict__ comp32, uint16_t* __restrict__ comp_out, int comp_d) {
  const int64_t blk = blockIdx.x;
  if (blk < rows) {
    row_epilogue_body(blk, x, d, ldx, rows_per_pos, qpos, norm_w, cos_t, sin_t, n_pos, rd, eps, sim, out, out_dtype,
                      cache_rows);
  } else {
    const int64_t i = blk - rows;
    decode_ids_body(i % nx, i / nx, pos, window, ratio, n_raw, ncomp, T, ids, comp32, comp_out, comp_d);
  }
}

static int check_ring_step(const float* ring_kv, const float* ring_sc, const float* kv_p, const float* score_p,
                           const int32_t* pos, const float* ape, const float* norm_w, const float* cos_t,
                           const float* sin_t, int64_t n_pos, int64_t B, int64_t d, int64_t ratio, int64_t rd,
                           int sim, const float* comp_cache, int64_t comp_cap, int64_t ld_p) {
  if (!ring_kv || !ring_sc || !kv_p || !score_p || !pos || !ape || !norm_w || !cos_t || !sin_t || !comp_cache)
    return SMLA_E_NULL;
  if (B <= 0 || comp_cap < 0 || n_pos <= 0 || (ld_p != 0 && ld_p < 2 * d)) return SMLA_E_SHAPE;
  int rc = check_pool_dims(d, ratio, rd, sim);
  if (rc) return rc;
  // two adjacent channels move in one 8-byte access
  if ((((uintptr_t)ring_kv | (uintptr_t)ring_sc | (uintptr_t)kv_p | (uintptr_t)score_p | (uintptr_t)ape) & 7) != 0 ||
      ld_p % 2 != 0)
    return SMLA_E_UNSUPPORTED;
  return SMLA_OK;
}

extern "C" int smla_ring_step(float* ring_kv, float* ring_sc, const float* kv_p, const float* score_p,
                              const int32_t* pos, const float* ape, const float* norm_w, const float* cos_t,
                              const float* sin_t, int64_t n_pos, int64_t B, int64_t d, int64_t ratio, int64_t rd,
                              float eps, int sim, float* comp_cache, int64_t comp_cap, int64_t ld_p, void* stream) {
  int rc = check_ring_step(ring_kv, ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, n_pos, B, d, ratio, rd,
                           sim, comp_cache, comp_cap, ld_p);
  if (rc) return rc;
  hipLaunchKernelGGL(ring_step_kernel, dim3((unsigned)B), dim3((unsigned)(d / 2)), 0, (hipStream_t)stream, ring_kv,
                     ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, n_pos, (int)d, (int)ratio, (int)rd,
                     eps, sim, comp_cache, comp_cap, ld_p ? ld_p : 2 * d);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

extern "C" int smla_quant_fp8_pow2(const void* x, int x_dtype, int64_t rows, int64_t D, uint8_t* codes,
                                   float* scales, void* stream) {
  if (!x || !codes || !scales) return SMLA_E_NULL;
  if (rows <= 0 || D <= 0 || D % 64 != 0) return SMLA_E_SHAPE;
  if (x_dtype != SMLA_F32 && x_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  const int64_t nb = rows * (D / 64);
  const int64_t nthreads = nb * 16;
  if ((nthreads + 255) / 256 > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  const dim3 grid((unsigned)((nthreads + 255) / 256));
  if (x_dtype == SMLA_F32)
    hipLaunchKernelGGL(quant_kernel<SMLA_F32>, grid, dim3(256), 0, (hipStream_t)stream, x, nb, codes, scales);
  else
    hipLaunchKernelGGL(quant_kernel<SMLA_BF16>, grid, dim3(256), 0, (hipStream_t)stream, x, nb, codes, scales);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

static int check_row_epilogue(const float* x, int64_t rows, int64_t d, int64_t ldx, int64_t rows_per_pos,
                              const int32_t* pos, const float* cos_t, const float* sin_t, int64_t n_pos, int64_t rd,
                              float eps, int sim, const void* out, int out_dtype, int64_t cache_rows) {
  if (!x || !out) return SMLA_E_NULL;
  if (rows <= 0 || d < 128 || d > 1024 || d % 64 != 0 || rows_per_pos <= 0 || rd < 0 || rd > d || rd % 2 != 0 ||
      cache_rows < 0 || rows > (int64_t)INT32_MAX || (ldx != 0 && ldx < d))
    return SMLA_E_SHAPE;
  if (rd > 0 && (!pos || !cos_t || !sin_t || n_pos <= 0)) return SMLA_E_NULL;
  if (cache_rows > 0 && !pos) return SMLA_E_NULL;
  if (sim != SMLA_SIM_NONE && sim != SMLA_SIM_FP8) return SMLA_E_UNSUPPORTED;
  if (sim == SMLA_SIM_FP8 && (d - rd) % 64 != 0) return SMLA_E_SHAPE;
  if (out_dtype != SMLA_F32 && out_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  if (!(eps >= 0.f)) return SMLA_E_RANGE;
  return SMLA_OK;
}

extern "C" int smla_row_epilogue(const float* x, int64_t rows, int64_t d, int64_t ldx, int64_t rows_per_pos,
                                 const int32_t* pos,
                                 const float* norm_w, const float* cos_t, const float* sin_t, int64_t n_pos,
                                 int64_t rd, float eps, int sim, void* out, int out_dtype, int64_t cache_rows,
                                 void* stream) {
  int rc = check_row_epilogue(x, rows, d, ldx, rows_per_pos, pos, cos_t, sin_t, n_pos, rd, eps, sim, out, out_dtype,
                              cache_rows);
  if (rc) return rc;
  hipLaunchKernelGGL(row_epilogue_kernel, dim3((unsigned)rows), dim3((unsigned)(d / 2)), 0, (hipStream_t)stream, x,
                     (int)d, ldx ? ldx : d, (int)rows_per_pos, pos, norm_w, cos_t, sin_t, n_pos, (int)rd, eps, sim, out, out_dtype,
                     cache_rows);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

extern "C" int smla_ring_step_kv(float* ring_kv, float* ring_sc, const float* kv_p, const float* score_p,
                                 const int32_t* pos, const float* ape, const float* norm_w, const float* cos_t,
                                 const float* sin_t, int64_t n_pos, int64_t B, int64_t d, int64_t ratio, int64_t rd,
                                 float eps, int sim, float* comp_cache, int64_t comp_cap, int64_t ld_p,
                                 const float* kv_x, int64_t ld_kv, const float* kv_norm, const float* kv_cos,
                                 const float* kv_sin, int64_t kv_n_pos, int64_t kv_rd, float kv_eps, int kv_sim,
                                 void* kv_cache, int kv_cache_dtype, int64_t kv_cache_rows, void* stream) {
  int rc = check_ring_step(ring_kv, ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, n_pos, B, d, ratio, rd,
                           sim, comp_cache, comp_cap, ld_p);
  if (rc) return rc;
  rc = check_row_epilogue(kv_x, B, d, ld_kv, 1, pos, kv_cos, kv_sin, kv_n_pos, kv_rd, kv_eps, kv_sim, kv_cache,
                          kv_cache_dtype, kv_cache_rows);
  if (rc) return rc;
  if (kv_cache_rows <= 0 || B > (int64_t)INT32_MAX / 2) return SMLA_E_SHAPE;
  hipLaunchKernelGGL(ring_kv_kernel, dim3((unsigned)(2 * B)), dim3((unsigned)(d / 2)), 0, (hipStream_t)stream, ring_kv,
                     ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, n_pos, (int)d, (int)ratio, (int)rd, eps,
                     sim, comp_cache, comp_cap, ld_p ? ld_p : 2 * d, B, kv_x, ld_kv ? ld_kv : d, kv_norm, kv_cos,
                     kv_sin, kv_n_pos, (int)kv_rd, kv_eps, kv_sim, kv_cache, kv_cache_dtype, kv_cache_rows);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

static int check_decode_ids(const int32_t* pos, int64_t B, int64_t window, int64_t ratio, int64_t n_raw,
                            int64_t ncomp, const int32_t* ids, int64_t T, const float* comp32,
                            const uint16_t* comp_out, int64_t d) {
  if (!pos || !ids) return SMLA_E_NULL;
  if (B <= 0 || B > 65535 || window <= 0 || ratio < 0 || n_raw <= 0 || ncomp < 0 || T < window || d < 0)
    return SMLA_E_SHAPE;
  if (window > n_raw) return SMLA_E_SHAPE;  // a ring shorter than the window would alias its rows
  if ((comp32 == nullptr) != (comp_out == nullptr)) return SMLA_E_NULL;
  if (comp_out && (ratio == 0 || d <= 0)) return SMLA_E_SHAPE;
  if (n_raw + ncomp > (int64_t)INT32_MAX) return SMLA_E_RANGE;
  return SMLA_OK;
}

extern "C" int smla_decode_ids(const int32_t* pos, int64_t B, int64_t window, int64_t ratio, int64_t n_raw,
                               int64_t ncomp, int32_t* ids, int64_t T, const float* comp32, uint16_t* comp_out,
                               int64_t d, void* stream) {
  int rc = check_decode_ids(pos, B, window, ratio, n_raw, ncomp, ids, T, comp32, comp_out, d);
  if (rc) return rc;
  const dim3 grid((unsigned)((T + 255) / 256), (unsigned)B);
  hipLaunchKernelGGL(decode_ids_kernel, grid, dim3(256), 0, (hipStream_t)stream, pos, (int)window, (int)ratio, n_raw,
                     ncomp, T, ids, comp32, comp_out, (int)d);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

extern "C" int smla_row_epilogue_ids(const float* x, int64_t rows, int64_t d, int64_t ldx, int64_t rows_per_pos,
                                     const int32_t* pos, const float* norm_w, const float* cos_t, const float* sin_t,
                                     int64_t n_pos, int64_t rd, float eps, int sim, void* out, int out_dtype,
                                     int64_t cache_rows, const int32_t* ids_pos, int64_t B, int64_t window,
                                     int64_t ratio, int64_t n_raw, int64_t ncomp, int32_t* ids, int64_t T,
                                     const float* comp32, uint16_t* comp_out, int64_t comp_d, void* stream) {
  int rc = check_row_epilogue(x, rows, d, ldx, rows_per_pos, pos, cos_t, sin_t, n_pos, rd, eps, sim, out, out_dtype,
                              cache_rows);
  if (rc) return rc;
  rc = check_decode_ids(ids_pos, B, window, ratio, n_raw, ncomp, ids, T, comp32, comp_out, comp_d);
  if (rc) return rc;
  if (d != 512) return SMLA_E_UNSUPPORTED;  // the id blocks' 256 threads are the rows' d/2
  const int64_t nx = (T + 255) / 256;
  if (rows + nx * B > (int64_t)INT32_MAX) return SMLA_E_SHAPE;
  hipLaunchKernelGGL(q_ids_kernel, dim3((unsigned)(rows + nx * B)), dim3(256), 0, (hipStream_t)stream, x, (int)d,
                     ldx ? ldx : d, (int)rows_per_pos, pos, norm_w, cos_t, sin_t, n_pos, (int)rd, eps, sim, out,
                     out_dtype, cache_rows, rows, nx, ids_pos, (int)window, (int)ratio, n_raw, ncomp, T, ids, comp32,
                     comp_out, (int)comp_d);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}
