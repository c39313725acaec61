// Indexer scoring (the build's definition; the reference attends every visible compressed row,
// oracle/decode_engine.py:112-114, and has no indexer).
//
//   dot_h = fma chain over d = 0..Di-1 of q[h,d]*k[n,d] (from +0)
//   r_h   = dot_h > 0 ? dot_h : +0
//   acc   = fma chain over h = 0..Hi-1 of w[h]*r_h (from +0)
//   score = acc * kscale[n]   (or acc when kscale == NULL);  -inf for n >= nvis
//
// The order is fixed so that every score is reproducible bit for bit by the CPU oracle; the top-k
// that follows can then be compared exactly.  Hi = Di = 64 (the decode shape) runs the dot-product
// chains on the matrix cores (indexer_mfma_kernel: K = 1 fp32 MFMAs, each one rounding, so the
// chain is the same sequence of fmas); other head counts run them on the vector ALUs
// (indexer_kernel: 64 keys per workgroup, one per lane, key row in VGPRs as fp32, waves splitting
// the heads 16 at a time with q and w staged in LDS as fp32 and read as wave-wide broadcasts).
// HBM traffic per query row: N * (Di * sizeof(key) + 4) bytes of keys and scales, N * 4 bytes of
// scores.  The fp32 multiply-add work (N * Hi * Di per query row) is the bound.
#include <type_traits>

#include "smla_internal.h"

namespace {

constexpr int kMaxQ = 64 * 128;  // Hi * Di fp32 in LDS (at most 32 KiB)
constexpr int kKeys = 64;        // keys per workgroup (one per lane)
// heads per wave of indexer_kernel: 16, or 4 / 8 for few heads, so a 64-key workgroup still
// spreads its dot products over four waves (at most 4 waves per workgroup)
inline int heads_per_wave(int64_t Hi) { return Hi <= 16 ? 4 : (Hi <= 32 ? 8 : 16); }
constexpr int kFp4 = 16;         // key type tag: packed e2m1 codes + one ue8m0 scale byte per 32

// Two code words of the gfx950 scaled fp4 converter, lanes of byte SEL: elements 2 SEL, 2 SEL + 1.
template <int SEL>
__device__ inline f32x2_t cvt_fp4_pair(uint32_t w, float s) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, s, SEL);
}

// scale bytes for which every e2m1 x 2^(sb - 127) is a normal finite float
__device__ inline bool fp4_scale_in_range(uint32_t sb) { return sb - 2u <= 250u; }

// 16 key values from two code words (element 2i in the low nibble of byte i, bit 3 the sign) of a
// block with scale byte sb: e2m1 x 2^(sb - 127), exact in fp32.  FOLD (sb in range): the scaled
// converter applies 2^(sb - 127) itself, two values per instruction; otherwise the converter gives
// the e2m1 value (all normal) and an fp32 multiply applies the scale (subnormal products, overflow
// to inf, the NaN byte).
template <bool FOLD>
__device__ inline void fp4_block16(uint32_t w0, uint32_t w1, uint32_t sb, float* o) {
  const float s = FOLD ? exp2i_f32((int)sb - 127) : 1.0f;
  const f32x2_t a0 = cvt_fp4_pair<0>(w0, s), a1 = cvt_fp4_pair<1>(w0, s), a2 = cvt_fp4_pair<2>(w0, s),
                a3 = cvt_fp4_pair<3>(w0, s);
  const f32x2_t b0 = cvt_fp4_pair<0>(w1, s), b1 = cvt_fp4_pair<1>(w1, s), b2 = cvt_fp4_pair<2>(w1, s),
                b3 = cvt_fp4_pair<3>(w1, s);
  o[0] = a0.x, o[1] = a0.y, o[2] = a1.x, o[3] = a1.y, o[4] = a2.x, o[5] = a2.y, o[6] = a3.x, o[7] = a3.y;
  o[8] = b0.x, o[9] = b0.y, o[10] = b1.x, o[11] = b1.y, o[12] = b2.x, o[13] = b2.y, o[14] = b3.x, o[15] = b3.y;
  if constexpr (!FOLD) {
    const float m = ue8m0_to_f32(sb);
#pragma unroll
    for (int e = 0; e < 16; e++) o[e] *= m;
  }
}

// One workgroup = 64 keys x all heads.  Wave w computes r_h = ReLU(dot_h) for heads
// hpw w .. hpw w + hpw - 1 (hpw = heads_per_wave: 4, 8 or 16; lane = key, key row in VGPRs, q rows
// read from LDS as wave-wide broadcasts);
// the r_h go through LDS and wave 0 runs the per-key chain over h = 0..Hi-1.  Each dot product is
// the same sequential fma chain over d as the oracle's, so scores are bit-identical.
template <int DI, int KDT, int QDT>
__global__ __launch_bounds__(256) void indexer_kernel(const void* __restrict__ q, int q_dtype,
                                                      const void* __restrict__ keys,
                                                      const uint8_t* __restrict__ kbs,
                                                      const float* __restrict__ kscale,
                                                      const float* __restrict__ weights,
                                                      const int32_t* __restrict__ nvis, int64_t S, int Hi,
                                                      int64_t N, float* __restrict__ scores) {
  __shared__ __align__(16) float sq[64 * DI];
  __shared__ float sw[256];
  __shared__ float sr[kKeys][65];  // r[key][head] (padded: lanes read different keys)
  int64_t bs, chunk;
  xcd_row_item(gridDim.y, gridDim.x, bs, chunk);
  const int64_t b = batch_of(bs, S);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int kHG = (Hi + nwaves - 1) / nwaves;  // heads per wave
  const int64_t n = chunk * kKeys + lane;
  const int64_t nv = nvis ? (int64_t)nvis[bs] : N;
  const bool live = n < N && n < nv;
  const int64_t nrow = n < N ? n : N - 1;

  // key row -> VGPRs (issued first so its latency overlaps the q staging)
  float kr[DI];
  const int64_t row = b * N + nrow;
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
  } else if constexpr (KDT == kFp4) {
    const u32x4_t* kp = (const u32x4_t*)((const uint8_t*)keys + row * (DI / 2));
#pragma unroll
    for (int v = 0; v < DI / 32; v++) {  // one 16-byte word = one 32-element scale block
      const u32x4_t w = kp[v];
      const uint32_t sb = kbs[row * (DI / 32) + v];
      fp4_block16<false>(w[0], w[1], sb, kr + 32 * v);
      fp4_block16<false>(w[2], w[3], sb, kr + 32 * v + 16);
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
  // q rows -> LDS as fp32, 8 elements per thread per step (Hi * DI is a multiple of 8 since DI is)
  {
    const int nq8 = Hi * DI / 8;
    if constexpr (QDT == SMLA_BF16) {
      const u32x4_t* qp = (const u32x4_t*)((const uint16_t*)q + bs * Hi * DI);
      for (int i = tid; i < nq8; i += blockDim.x) {
        const u32x4_t v = qp[i];
        f32x4_t lo, hi;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          lo[2 * j] = bf16_bits_to_f32((uint16_t)(v[j] & 0xffffu));
          lo[2 * j + 1] = bf16_bits_to_f32((uint16_t)(v[j] >> 16));
          hi[2 * j] = bf16_bits_to_f32((uint16_t)(v[j + 2] & 0xffffu));
          hi[2 * j + 1] = bf16_bits_to_f32((uint16_t)(v[j + 2] >> 16));
        }
        *(f32x4_t*)(sq + 8 * i) = lo;
        *(f32x4_t*)(sq + 8 * i + 4) = hi;
      }
    } else {
      const f32x4_t* qp = (const f32x4_t*)((const float*)q + bs * Hi * DI);
      for (int i = tid; i < nq8; i += blockDim.x) {
        const f32x4_t a = qp[2 * i], c = qp[2 * i + 1];
        *(f32x4_t*)(sq + 8 * i) = a;
        *(f32x4_t*)(sq + 8 * i + 4) = c;
      }
    }
    (void)q_dtype;
  }
  for (int i = tid; i < Hi; i += blockDim.x) sw[i] = weights[bs * Hi + i];
  __syncthreads();

  // r_h for this wave's heads
  for (int h0 = wave * kHG; h0 < Hi; h0 += nwaves * kHG) {
    const int hn = min(kHG, Hi - h0);
    int hh = 0;
    for (; hh + 1 < hn; hh += 2) {  // two independent chains per step
      const int h = h0 + hh;
      const f32x4_t* qa = (const f32x4_t*)(sq + h * DI);
      const f32x4_t* qb = (const f32x4_t*)(sq + (h + 1) * DI);
      float da = 0.f, db = 0.f;
#pragma unroll
      for (int v = 0; v < DI / 4; v++) {
        const f32x4_t xa = qa[v], xb = qb[v];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          da = __builtin_fmaf(xa[j], kr[4 * v + j], da);
          db = __builtin_fmaf(xb[j], kr[4 * v + j], db);
        }
      }
      sr[lane][h] = da > 0.f ? da : 0.f;
      sr[lane][h + 1] = db > 0.f ? db : 0.f;
    }
    if (hh < hn) {
      const int h = h0 + hh;
      const f32x4_t* qh = (const f32x4_t*)(sq + h * DI);
      float dot = 0.f;
#pragma unroll
      for (int v = 0; v < DI / 4; v++) {
        const f32x4_t qq = qh[v];
#pragma unroll
        for (int j = 0; j < 4; j++) dot = __builtin_fmaf(qq[j], kr[4 * v + j], dot);
      }
      sr[lane][h] = dot > 0.f ? dot : 0.f;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float acc = 0.f;
#pragma unroll 8
  for (int h = 0; h < Hi; h++) acc = __builtin_fmaf(sw[h], sr[lane][h], acc);
  if (n < N) scores[bs * N + n] = live ? (kscale ? acc * kscale[row] : acc) : -SMLA_INF;
}

// Hi = Di = 64 on the matrix cores.  v_mfma_f32_32x32x1_2b_f32 (K = 1) adds one product to each
// accumulator with a single rounding, so a chain of 64 of them over d = 0..63 is, element for
// element, the fma chain dot_h = fma(q[h,d], k[n,d], dot_h) of the definition above (bit for bit:
// checked against fmaf over 6.7e7 operand triples, subnormal, cancelling and overflowing ones
// included), at twice the rate of fp32 fma on the vector ALUs.  A wave computes a tile of 64 heads x
// 32 keys: A = q[h][d] with h = lane (block 0 takes heads 0..31 from lanes 0..31, block 1 heads
// 32..63 from lanes 32..63), B = k[n][d] with n = lane mod 32 (both blocks take the same 32 keys).
// Accumulator register r of lane l then holds head 32 (r / 16) + 8 ((r mod 16) / 4) + 4 (l / 32) +
// r mod 4 of key l mod 32.  The chain over the heads walks h = 0..63 in order: heads 8t..8t+3 sit
// in lanes 0..31 and heads 8t+4..8t+7 in lanes 32..63, both in registers 16 (t / 4) + 4 (t mod 4) +
// 0..3, so the running sum crosses between the two halves with a lane swap every four heads (the
// weights are wave-uniform scalars).  One tile per wave and two waves per SIMD (4-wave workgroups
// of 128 keys) measured faster than two interleaved tiles per wave at one wave per SIMD.
//
// KT = 16: tiles of 64 heads x 16 keys on v_mfma_f32_16x16x1_4b_f32 (also one rounding per product:
// checked against fmaf over 1.7e7 triples), for rows too few to give every CU a 128-key workgroup.
// A dependent step takes about 0.6 of the 32-key step, so a wave's chain ends sooner, at 0.8 of the
// 32-key form's throughput per product.  Block b takes heads 16b..16b+15 from lanes 16b..16b+15
// (h = lane again) and the key n = lane mod 16; register j of lane l holds head 16 (j / 4) + 4 (l / 16)
// + j mod 4.  The head chain walks the 16-lane rows: after the four heads of row g, every row takes
// row g's sum (two lane swaps).
template <int KDT, int QDT, int KT = 32>
__global__ __launch_bounds__(256) void indexer_mfma_kernel(const void* __restrict__ q, const void* __restrict__ keys,
                                                       const uint8_t* __restrict__ kbs,
                                                       const float* __restrict__ kscale,
                                                       const float* __restrict__ weights,
                                                       const int32_t* __restrict__ nvis, int64_t S, int64_t N,
                                                       float* __restrict__ scores) {
  constexpr int DI = 64;
  static_assert(KT == 32 || KT == 16, "key tiles of 32 or 16");
  constexpr int KEYS = 4 * KT;  // keys per workgroup: 4 waves x one tile of KT keys
  {
    const uint32_t gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    asm volatile("" ::"s"(gx), "s"(gy), "s"(gz), "s"(q), "s"(keys), "s"(kbs), "s"(kscale), "s"(weights), "s"(nvis),
                 "s"(S), "s"(N), "s"(scores));
  }
  int64_t bs, chunk;
  xcd_row_item(gridDim.y, gridDim.x, bs, chunk);
  const int64_t b = batch_of(bs, S);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t kb = chunk * KEYS + wave * KT;  // first key of this wave's tile

  // the row of key kb + lane mod KT in its storage type
  constexpr int KW = KDT == kFp4 ? 2 : KDT == SMLA_FP8_E4M3 ? 4 : (KDT == SMLA_BF16 ? 8 : 16);
  u32x4_t kr[KW];
  uint32_t ksb = 0;  // fp4: the row's two scale bytes
  {
    const int64_t n = kb + (lane & (KT - 1));
    const int64_t row = b * N + (n < N ? n : N - 1);
    const u32x4_t* pk = (const u32x4_t*)((const uint8_t*)keys + row * DI * KW / 4);
#pragma unroll
    for (int v = 0; v < KW; v++) kr[v] = pk[v];
    if constexpr (KDT == kFp4) ksb = ((const uint16_t*)kbs)[row];
  }
  // The row's q block (64 heads), its head weights and the key's scale come in once per workgroup
  // through LDS: each wave loading the whole q block itself moved 8 KB per wave through L2 (16 MB
  // per decode step), and the compiler placed each of those loads next to its first MFMA, a round
  // trip per 16 bytes inside the chain; the weights and the scale were loaded after the chain.  q
  // rows sit at a stride of QW + 1 16-byte words, so the 64 lanes' row reads spread over the banks.
  constexpr int QW = QDT == SMLA_BF16 ? 8 : 16;  // 16-byte words per head row
  constexpr int QV = 64 * QW / 256;              // words of the q block per thread
  __shared__ u32x4_t q_s[64 * (QW + 1)];
  __shared__ float w_s[64];
  float ksc = 1.f;  // the scale of key kb + lane (lanes < KT write)
  int nvl = 0;      // the row's visible count (nvis given)
  {
    const u32x4_t* qp = (const u32x4_t*)((const uint8_t*)q + bs * 64 * (int64_t)(QW * 16));
    u32x4_t qv[QV];
#pragma unroll
    for (int i = 0; i < QV; i++) qv[i] = qp[threadIdx.x + 256 * i];
    const float wv = weights[bs * 64 + lane];
    float ksc0 = 1.f;
    if (kscale) ksc0 = kscale[b * N + min(kb + (lane & (KT - 1)), N - 1)];
    if (nvis) nvl = nvis[bs];
    // one wait for every load of the wave (the keys were requested first)
#pragma unroll
    for (int v = 0; v < KW; v++) asm volatile("" ::"v"(kr[v]));
#pragma unroll
    for (int i = 0; i < QV; i++) asm volatile("" ::"v"(qv[i]));
    asm volatile("" ::"v"(wv), "v"(ksc0), "v"(nvl), "v"(ksb));
    ksc = ksc0;
#pragma unroll
    for (int i = 0; i < QV; i++) {
      const int k = threadIdx.x + 256 * i;  // word k: head k / QW, word k % QW
      q_s[(k / QW) * (QW + 1) + k % QW] = qv[i];
    }
    if (wave == 0) w_s[lane] = wv;
  }
  const int64_t nv = nvis ? (int64_t)nvl : N;
  __syncthreads();
  u32x4_t qw[QW];  // head `lane`'s q row, read whole before the chain starts
#pragma unroll
  for (int v = 0; v < QW; v++) qw[v] = q_s[lane * (QW + 1) + v];
#pragma unroll
  for (int v = 0; v < QW; v++) asm volatile("" : "+v"(qw[v]));
  auto wrow = [&](int h) -> float { return w_s[h]; };
  float qf[DI];
#pragma unroll
  for (int v = 0; v < QW; v++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if constexpr (QDT == SMLA_BF16) {
        qf[8 * v + 2 * j] = __uint_as_float(qw[v][j] << 16);
        qf[8 * v + 2 * j + 1] = __uint_as_float(qw[v][j] & 0xffff0000u);
      } else {
        qf[4 * v + j] = __uint_as_float(qw[v][j]);
      }
    }
  // 16 values of the key row starting at d0 = 16 db, as fp32 (fold: see fp4_block16)
  auto block16 = [&](int db, float (&o)[16], auto fold) {
    const u32x4_t(&row)[KW] = kr;
    if constexpr (KDT == kFp4) {
      const u32x4_t w = row[db >> 1];
      fp4_block16<decltype(fold)::value>(w[2 * (db & 1)], w[2 * (db & 1) + 1], (ksb >> (8 * (db >> 1))) & 0xffu, o);
    } else if constexpr (KDT == SMLA_FP8_E4M3) {
      const u32x4_t w = row[db];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], false);
        const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], true);
        o[4 * j] = lo.x;
        o[4 * j + 1] = lo.y;
        o[4 * j + 2] = hi.x;
        o[4 * j + 3] = hi.y;
      }
    } else if constexpr (KDT == SMLA_BF16) {
#pragma unroll
      for (int v = 0; v < 2; v++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t w = row[2 * db + v][j];
          o[8 * v + 2 * j] = __uint_as_float(w << 16);
          o[8 * v + 2 * j + 1] = __uint_as_float(w & 0xffff0000u);
        }
    } else {
#pragma unroll
      for (int v = 0; v < 4; v++)
#pragma unroll
        for (int j = 0; j < 4; j++) o[4 * v + j] = __uint_as_float(row[4 * db + v][j]);
    }
  };
  using Acc = typename std::conditional<KT == 32, f32x32_t, f32x16_t>::type;
  Acc acc;
#pragma unroll
  for (int r = 0; r < KT; r++) acc[r] = 0.f;
  auto run = [&](auto fold) {
#pragma unroll
    for (int db = 0; db < 4; db++) {
      float x[16];
      block16(db, x, fold);
#pragma unroll
      for (int dd = 0; dd < 16; dd++) {
        if constexpr (KT == 32)
          acc = __builtin_amdgcn_mfma_f32_32x32x1f32(qf[16 * db + dd], x[dd], acc, 0, 0, 0);
        else
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(qf[16 * db + dd], x[dd], acc, 0, 0, 0);
      }
    }
  };
  if constexpr (KDT == kFp4) {
    // the folded conversion when every scale byte of the wave's keys allows it (wave-uniform)
    const bool fold = fp4_scale_in_range(ksb & 0xffu) && fp4_scale_in_range(ksb >> 8);
    if (__all(fold)) run(std::true_type{});
    else run(std::false_type{});
  } else {
    run(std::true_type{});
  }
  // chain over the heads, then the key's scale; lanes l and l + 32 end with the same sum.  After
  // four heads in lanes 0..31 the swap hands every lane the low half's sum ([0]); after four in
  // lanes 32..63, the high half's ([1]).
  float sum = 0.f;
  if constexpr (KT == 32) {
#pragma unroll
    for (int tt = 0; tt < 8; tt++) {
      const int R = 16 * (tt >> 2) + 4 * (tt & 3);
      float r[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) r[rr] = acc[R + rr] > 0.f ? acc[R + rr] : 0.f;
#pragma unroll
      for (int rr = 0; rr < 4; rr++) sum = __builtin_fmaf(wrow(8 * tt + rr), r[rr], sum);
      sum = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(sum), false, false)[0]);
#pragma unroll
      for (int rr = 0; rr < 4; rr++) sum = __builtin_fmaf(wrow(8 * tt + 4 + rr), r[rr], sum);
      sum = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(sum), false, false)[1]);
    }
  } else {
    // heads 16bk + 4g .. +3 sit in row g = lane / 16, registers 4bk .. 4bk+3: each row adds its
    // four onto the running sum, then every row takes row g's result (permlane16_swap gives the
    // even or odd rows over each pair, permlane32_swap the low or high pair over both halves)
#pragma unroll
    for (int bk = 0; bk < 4; bk++) {
      float r[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) r[rr] = acc[4 * bk + rr] > 0.f ? acc[4 * bk + rr] : 0.f;
#pragma unroll
      for (int g = 0; g < 4; g++) {
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sum = __builtin_fmaf(wrow(16 * bk + 4 * g + rr), r[rr], sum);
        const uint32_t y =
            __builtin_amdgcn_permlane16_swap(__float_as_uint(sum), __float_as_uint(sum), false, false)[g & 1];
        sum = __uint_as_float(__builtin_amdgcn_permlane32_swap(y, y, false, false)[g >> 1]);
      }
    }
  }
  const int64_t n = kb + lane;
  if (lane < KT && n < N) scores[bs * N + n] = n < nv ? (kscale ? sum * ksc : sum) : -SMLA_INF;
}

// Hi > 64: one thread per key, sequential over all heads (same arithmetic order)
template <int DI, int KDT>
__global__ __launch_bounds__(256) void indexer_wide_kernel(const void* __restrict__ q, int q_dtype,
                                                           const void* __restrict__ keys,
                                                           const uint8_t* __restrict__ kbs,
                                                           const float* __restrict__ kscale,
                                                           const float* __restrict__ weights,
                                                           const int32_t* __restrict__ nvis, int64_t S, int Hi,
                                                           int64_t N, float* __restrict__ scores) {
  int64_t bs, chunk;
  xcd_row_item(gridDim.y, gridDim.x, bs, chunk);
  const int64_t b = batch_of(bs, S);
  const int64_t n = chunk * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t nv = nvis ? (int64_t)nvis[bs] : N;
  if (n >= nv) {
    scores[bs * N + n] = -SMLA_INF;
    return;
  }
  const int64_t row = b * N + n;
  auto key_at = [&](int d) -> float {
    if constexpr (KDT == kFp4) {
      const uint32_t c = (((const uint8_t*)keys)[row * (DI / 2) + d / 2] >> (4 * (d & 1))) & 15u;
      return e2m1_to_f32(c) * ue8m0_to_f32(kbs[row * (DI / 32) + d / 32]);
    } else {
      return load_as_f32(keys, row * DI + d, KDT);
    }
  };
  float acc = 0.f;
  for (int h = 0; h < Hi; h++) {
    float dot = 0.f;
    for (int d = 0; d < DI; d++) dot = __builtin_fmaf(load_as_f32(q, (bs * Hi + h) * DI + d, q_dtype), key_at(d), dot);
    acc = __builtin_fmaf(weights[bs * Hi + h], dot > 0.f ? dot : 0.f, acc);
  }
  scores[bs * N + n] = kscale ? acc * kscale[row] : acc;
}

template <int DI, int KDT>
int launch_k(const void* q, int q_dtype, const void* keys, const uint8_t* kbs, const float* kscale, const float* w,
             const int32_t* nvis, int64_t B, int64_t S, int64_t Hi, int64_t N, float* scores, hipStream_t st) {
  if (Hi == 64 && DI == 64) {
    // 128 keys per workgroup (a 64-head x 32-key tile per wave), or 64 (16-key tiles) when 128-key
    // workgroups would leave CUs idle
    const bool k16 = (N + 127) / 128 * B * S < smla_num_cus();
    const dim3 grid((unsigned)(k16 ? (N + 63) / 64 : (N + 127) / 128), (unsigned)(B * S));
#define SMLA_IDX_MFMA(QT, KTT)                                                                                  \
  hipLaunchKernelGGL((indexer_mfma_kernel<KDT, QT, KTT>), grid, dim3(256), 0, st, q, keys, kbs, kscale, w, nvis, S, \
                     N, scores)
    if (q_dtype == SMLA_BF16) {
      if (k16) SMLA_IDX_MFMA(SMLA_BF16, 16); else SMLA_IDX_MFMA(SMLA_BF16, 32);
    } else {
      if (k16) SMLA_IDX_MFMA(SMLA_F32, 16); else SMLA_IDX_MFMA(SMLA_F32, 32);
    }
#undef SMLA_IDX_MFMA
  } else if (Hi <= 64) {
    dim3 grid((unsigned)((N + kKeys - 1) / kKeys), (unsigned)(B * S));
    const int hpw = heads_per_wave(Hi);
    const int threads = (int)(((Hi + hpw - 1) / hpw) * 64);
    if (q_dtype == SMLA_BF16)
      hipLaunchKernelGGL((indexer_kernel<DI, KDT, SMLA_BF16>), grid, dim3(threads), 0, st, q, q_dtype, keys, kbs,
                         kscale, w, nvis, S, (int)Hi, N, scores);
    else
      hipLaunchKernelGGL((indexer_kernel<DI, KDT, SMLA_F32>), grid, dim3(threads), 0, st, q, q_dtype, keys, kbs,
                         kscale, w, nvis, S, (int)Hi, N, scores);
  } else {
    dim3 grid((unsigned)((N + 255) / 256), (unsigned)(B * S));
    hipLaunchKernelGGL((indexer_wide_kernel<DI, KDT>), grid, dim3(256), 0, st, q, q_dtype, keys, kbs, kscale, w, nvis,
                       S, (int)Hi, N, scores);
  }
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

template <int DI>
int launch_di(const void* q, int q_dtype, const void* keys, int k_dtype, const uint8_t* kbs, const float* kscale,
              const float* w, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi, int64_t N,
              float* scores, hipStream_t st) {
  if (k_dtype == kFp4) return launch_k<DI, kFp4>(q, q_dtype, keys, kbs, kscale, w, nvis, B, S, Hi, N, scores, st);
  if (k_dtype == SMLA_FP8_E4M3)
    return launch_k<DI, SMLA_FP8_E4M3>(q, q_dtype, keys, kbs, kscale, w, nvis, B, S, Hi, N, scores, st);
  if (k_dtype == SMLA_BF16)
    return launch_k<DI, SMLA_BF16>(q, q_dtype, keys, kbs, kscale, w, nvis, B, S, Hi, N, scores, st);
  return launch_k<DI, SMLA_F32>(q, q_dtype, keys, kbs, kscale, w, nvis, B, S, Hi, N, scores, st);
}

int indexer_score_any(const void* q, int q_dtype, const void* keys, int k_dtype, const uint8_t* kbs,
                      const float* kscale, const float* weights, const int32_t* nvis, int64_t B, int64_t S,
                      int64_t Hi, int64_t Di, int64_t N, float* scores, void* stream) {
  if (!q || !keys || !weights || !scores || (k_dtype == kFp4 && !kbs)) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || Hi <= 0 || Di <= 0 || N <= 0) return SMLA_E_SHAPE;
  if (q_dtype != SMLA_F32 && q_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  if (Hi > 256 || (Hi <= 64 && Hi * Di > kMaxQ) || (N + 63) / 64 > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  if (Di != 32 && Di != 64 && Di != 128) return SMLA_E_UNSUPPORTED;
  // q rows and key rows are read as 16-byte words, fp4 scale bytes of a row as one 2-byte word
  if (((uintptr_t)q & 15) || ((uintptr_t)keys & 15) || ((uintptr_t)kbs & 1)) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  // bytes of one key row and of one q element
  const int64_t krow = k_dtype == SMLA_F32 ? 4 * Di : k_dtype == SMLA_BF16 ? 2 * Di : k_dtype == kFp4 ? Di / 2 : Di;
  const int64_t qel = q_dtype == SMLA_BF16 ? 2 : 4;
  // the grid's y dimension is the query row: longer calls run as launches over row chunks, each
  // with its q rows, weights, nvis and scores and its sequences' keys
  return for_row_chunks(B, S, [&](int64_t b0, int64_t s0, int64_t nb, int64_t ns) -> int {
    const int64_t r0 = b0 * S + s0;
    const void* cq = (const uint8_t*)q + r0 * Hi * Di * qel;
    const void* ck = (const uint8_t*)keys + b0 * N * krow;
    const uint8_t* ckbs = kbs ? kbs + b0 * N * (Di / 32) : nullptr;
    const float* cks = kscale ? kscale + b0 * N : nullptr;
    const float* cw = weights + r0 * Hi;
    const int32_t* cnv = nvis ? nvis + r0 : nullptr;
    float* csc = scores + r0 * N;
    switch (Di) {
      case 32: return launch_di<32>(cq, q_dtype, ck, k_dtype, ckbs, cks, cw, cnv, nb, ns, Hi, N, csc, st);
      case 64: return launch_di<64>(cq, q_dtype, ck, k_dtype, ckbs, cks, cw, cnv, nb, ns, Hi, N, csc, st);
      default: return launch_di<128>(cq, q_dtype, ck, k_dtype, ckbs, cks, cw, cnv, nb, ns, Hi, N, csc, st);
    }
  });
}
}  // namespace

extern "C" int smla_indexer_score(const void* q, int q_dtype, const void* keys, int k_dtype, const float* kscale,
                                  const float* weights, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi,
                                  int64_t Di, int64_t N, float* scores, void* stream) {
  if (k_dtype != SMLA_F32 && k_dtype != SMLA_BF16 && k_dtype != SMLA_FP8_E4M3) return SMLA_E_DTYPE;
  return indexer_score_any(q, q_dtype, keys, k_dtype, nullptr, kscale, weights, nvis, B, S, Hi, Di, N, scores,
                           stream);
}

extern "C" int smla_indexer_score_fp4(const void* q, int q_dtype, const uint8_t* codes, const uint8_t* block_scales,
                                      const float* kscale, const float* weights, const int32_t* nvis, int64_t B,
                                      int64_t S, int64_t Hi, int64_t Di, int64_t N, float* scores, void* stream) {
  return indexer_score_any(q, q_dtype, codes, kFp4, block_scales, kscale, weights, nvis, B, S, Hi, Di, N, scores,
                           stream);
}
