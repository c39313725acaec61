// Sparse absorbed-MLA attention over gathered latent rows.
//
// Semantics follow ref_torch/sparse_attn.py:23-34 (sparse_attn): gather kv[idx] (idx < 0 masked),
// logits = scale * q.kv, softmax over valid rows with exp(sink - rowmax) added to the
// denominator, output = weighted sum of the first DV columns of the gathered rows.
//
// Two kernels:
//  * attn_generic_kernel — fp32 VALU, any dtype / shape; one workgroup per (b, s, head).  This
//    is the fp32 path (1e-5 parity) and the fallback for shapes the MFMA kernel does not cover.
//  * attn_mfma_kernel    — bf16 MFMA split-K kernel for H % 16 == 0, D in {576, 512}, DV = 512,
//    bf16 q, bf16 or fp8 (e4m3 + per-64 pow2 scale) rows.  One workgroup of 4 waves per
//    (query row, split, 64-head group).  Rows are staged in 32-row tiles through LDS twice: row
//    major (the A operand of S^T = K Q^T, rows as M, heads as N) and transposed (the A operand of
//    O^T = V^T P^T).  The K-dimension order of the P.V product is permuted so that each lane's
//    S^T accumulator registers are directly its B operand (no shuffles).  Tiles are double
//    buffered: tile i+1 is loaded from HBM into registers while tile i is computed.
//    Online softmax keeps a reference max per head that moves only when a tile's max exceeds it
//    by more than 8 (exact: numerator and denominator use the same reference).
//  * attn_merge_kernel   — log-sum-exp merge of the split partial states.
#include "attn_common.h"

namespace {

using smla_attn::kRescaleSlack;
using smla_attn::kThreads;
using smla_attn::kTileRows;
using smla_attn::RowSrc;

// pointer to row `r` (virtual concatenation [kv0; kv1]) of batch b; element size es bytes
__device__ inline const uint8_t* row_ptr(const RowSrc& src, int64_t b, int64_t r, int64_t D, int es,
                                         const float** scale_row) {
  if (r < src.n0) {
    if (scale_row) *scale_row = src.sc0 ? src.sc0 + (b * src.n0 + r) * (D / 64) : nullptr;
    return (const uint8_t*)src.kv0 + (b * src.n0 + r) * D * es;
  }
  int64_t r1 = r - src.n0;
  if (scale_row) *scale_row = src.sc1 ? src.sc1 + (b * src.n1 + r1) * (D / 64) : nullptr;
  return (const uint8_t*)src.kv1 + (b * src.n1 + r1) * D * es;
}

__device__ inline int dtype_size(int dt) { return dt == SMLA_F32 ? 4 : (dt == SMLA_FP8_E4M3 ? 1 : 2); }

// ---------------------------------------------------------------------------------------------
// Generic VALU kernel.
__global__ __launch_bounds__(kThreads) void attn_generic_kernel(
    const void* __restrict__ q, int q_dtype, RowSrc src, int kv_dtype,
    const float* __restrict__ sink, const int32_t* __restrict__ idx, int64_t T, int64_t S,
    int64_t H, int64_t D, int64_t DV, float scale, void* __restrict__ out, int out_dtype) {
  extern __shared__ float smem[];
  float* sq = smem;                 // [D]
  float* sp = sq + D;               // [256]
  int* sid = (int*)(sp + kThreads); // [256]
  __shared__ float red[kThreads / 64];

  const int tid = threadIdx.x;
  const int64_t h = blockIdx.x % H;
  const int64_t bs = blockIdx.x / H;
  const int64_t b = bs / S;
  const int64_t ntot = src.n0 + src.n1;
  const int es = dtype_size(kv_dtype);

  for (int64_t d = tid; d < D; d += kThreads) sq[d] = load_as_f32(q, (bs * H + h) * D + d, q_dtype);
  __syncthreads();

  constexpr int kMaxDvPerThread = 4;  // DV <= 1024
  float acc[kMaxDvPerThread];
#pragma unroll
  for (int j = 0; j < kMaxDvPerThread; j++) acc[j] = 0.f;
  float m_run = -SMLA_INF, l_run = 0.f;
  const int32_t* ids = idx + bs * T;

  for (int64_t t0 = 0; t0 < T; t0 += kThreads) {
    int64_t t = t0 + tid;
    float sc = -SMLA_INF;
    int rid = -1;
    if (t < T) {
      int64_t r = ids[t];
      if (r >= 0 && r < ntot) {
        const float* srow = nullptr;
        const uint8_t* row = row_ptr(src, b, r, D, es, &srow);
        float dot = 0.f;
        for (int64_t d = 0; d < D; d++) {
          float v = load_as_f32(row, d, kv_dtype);
          if (srow) v *= srow[d / 64];
          dot = fmaf(sq[d], v, dot);
        }
        sc = scale * dot;
        rid = (int)r;
      }
    }
    // block max
    float mx = wave_max(sc);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    float mt = red[0];
    for (int w = 1; w < kThreads / 64; w++) mt = fmaxf(mt, red[w]);
    __syncthreads();
    float m_new = fmaxf(m_run, mt);
    float p = (rid >= 0 && m_new > -SMLA_INF) ? __expf(sc - m_new) : 0.f;
    sp[tid] = p;
    sid[tid] = rid;
    float ps = wave_sum(p);
    if ((tid & 63) == 0) red[tid >> 6] = ps;
    __syncthreads();
    float psum = 0.f;
    for (int w = 0; w < kThreads / 64; w++) psum += red[w];
    if (m_new > -SMLA_INF) {
      float alpha = (m_run > -SMLA_INF) ? __expf(m_run - m_new) : 0.f;
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int j = 0; j < kMaxDvPerThread; j++) acc[j] *= alpha;
      int64_t nt = (T - t0) < kThreads ? (T - t0) : kThreads;
      for (int64_t tt = 0; tt < nt; tt++) {
        int r = sid[tt];
        if (r < 0) continue;
        float pt = sp[tt];
        const float* srow = nullptr;
        const uint8_t* row = row_ptr(src, b, r, D, es, &srow);
#pragma unroll
        for (int j = 0; j < kMaxDvPerThread; j++) {
          int64_t dv = tid + j * kThreads;
          if (dv < DV) {
            float v = load_as_f32(row, dv, kv_dtype);
            if (srow) v *= srow[dv / 64];
            acc[j] = fmaf(pt, v, acc[j]);
          }
        }
      }
      m_run = m_new;
    }
    __syncthreads();
  }
  float snk = sink ? sink[h] : -SMLA_INF;
  float den = l_run + ((m_run > -SMLA_INF) ? __expf(snk - m_run) : 0.f);
  bool empty = !(m_run > -SMLA_INF);
#pragma unroll
  for (int j = 0; j < kMaxDvPerThread; j++) {
    int64_t dv = tid + j * kThreads;
    if (dv < DV) {
      float o = empty ? __builtin_nanf("") : acc[j] / den;
      store_from_f32(out, (bs * H + h) * DV + dv, out_dtype, o);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// MFMA split-K kernel.
//
// LDS per buffer: K tile [32 rows][KS] bf16 (KS = D + 8: conflict-free 16-lane b128 reads) and
// V^T tile [DV][VS] bf16 (VS = 40 slots: 32 used, padded for conflict-free reads).
// Slot order of a tile row r: slot(r) = 8*((r%16)/4) + 4*(r/16) + r%4, so lane group g of the
// 16x16x32 MFMA owns slots 8g..8g+7 = rows {4g..4g+3} U {16+4g..16+4g+3} — exactly the rows of
// its two S^T accumulators.
template <int D, int DV>
struct MfmaCfg {
  static constexpr int KS = D + 8;
  static constexpr int VS = 40;
  static constexpr int KTILE_ELEMS = kTileRows * KS;
  static constexpr int VT_ELEMS = DV * VS;
  static constexpr int BUF_ELEMS = KTILE_ELEMS + VT_ELEMS;
  static constexpr size_t LDS_BYTES = 2 * BUF_ELEMS * 2 + 2 * kTileRows * 4;
  static constexpr int KSTEPS = D / 32;
  static constexpr int DVT = DV / 16;
};

__device__ inline int tile_slot(int r) { return 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3); }

// Per-thread staging registers for one tile.
// bf16 rows: unit = (row quad, 8-element chunk): 4 rows x 16 B.  units = 8 * D/8.
// fp8 rows : unit = (row quad, 16-element chunk): 4 rows x 16 B codes + 4 scales. units = 8 * D/16.
template <int D, bool FP8>
struct Stage {
  static constexpr int CH = FP8 ? 16 : 8;
  static constexpr int NCH = D / CH;
  static constexpr int UNITS = 8 * NCH;
  static constexpr int PER_THREAD = (UNITS + kThreads - 1) / kThreads;
  u32x4_t v[PER_THREAD][4];
  float s[FP8 ? PER_THREAD : 1][4];
  int vflag;  // validity of tile row `tid` (threads 0..31)
};

template <int D, int DV, bool FP8>
__device__ inline void stage_load(Stage<D, FP8>& st, const RowSrc& src, int64_t b, const int32_t* ids,
                                  int t_begin, int t_end, int tid) {
  using S = Stage<D, FP8>;
  const int64_t ntot = src.n0 + src.n1;
  st.vflag = 0;
  if (tid < kTileRows) {
    int t = t_begin + tid;
    if (t < t_end) {
      int64_t r = ids[t];
      st.vflag = (r >= 0 && r < ntot);
    }
  }
#pragma unroll
  for (int k = 0; k < S::PER_THREAD; k++) {
    int u = tid + k * kThreads;
    if (u < S::UNITS) {
      int rq = u / S::NCH, c = u % S::NCH;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int t = t_begin + rq * 4 + j;
        int64_t r = (t < t_end) ? (int64_t)ids[t] : -1;
        if (r >= 0 && r < ntot) {
          const float* srow = nullptr;
          const uint8_t* row = row_ptr(src, b, r, D, FP8 ? 1 : 2, FP8 ? &srow : nullptr);
          st.v[k][j] = *(const u32x4_t*)(row + (int64_t)c * 16);
          if constexpr (FP8) st.s[k][j] = srow[(c * 16) / 64];
        } else {
          st.v[k][j] = u32x4_t{0u, 0u, 0u, 0u};
          if constexpr (FP8) st.s[k][j] = 0.f;
        }
      }
    }
  }
}

template <int D, int DV, bool FP8>
__device__ inline void stage_store(const Stage<D, FP8>& st, uint16_t* buf, int* valid_out, int tid) {
  using C = MfmaCfg<D, DV>;
  using S = Stage<D, FP8>;
  if (tid < kTileRows) valid_out[tid] = st.vflag;
  uint16_t* kt = buf;
  uint16_t* vt = buf + C::KTILE_ELEMS;
#pragma unroll
  for (int k = 0; k < S::PER_THREAD; k++) {
    int u = tid + k * kThreads;
    if (u < S::UNITS) {
      int rq = u / S::NCH, c = u % S::NCH;
      int slot0 = tile_slot(rq * 4);
      if constexpr (!FP8) {
        // row-major K tile
#pragma unroll
        for (int j = 0; j < 4; j++) *(u32x4_t*)(kt + (rq * 4 + j) * C::KS + c * 8) = st.v[k][j];
        if (c * 8 < DV) {
          // transpose: element e of the chunk for rows rq*4..rq*4+3 -> 4 consecutive slots
#pragma unroll
          for (int e = 0; e < 8; e++) {
            int w = e >> 1, hi = e & 1;
            uint32_t x0 = st.v[k][0][w], x1 = st.v[k][1][w], x2 = st.v[k][2][w], x3 = st.v[k][3][w];
            uint32_t lo01, lo23;
            if (hi) {
              lo01 = (x0 >> 16) | (x1 & 0xffff0000u);
              lo23 = (x2 >> 16) | (x3 & 0xffff0000u);
            } else {
              lo01 = (x0 & 0xffffu) | (x1 << 16);
              lo23 = (x2 & 0xffffu) | (x3 << 16);
            }
            *(u32x2_t*)(vt + (c * 8 + e) * C::VS + slot0) = u32x2_t{lo01, lo23};
          }
        }
      } else {
        // dequantise 16 fp8 codes per row to bf16 (exact: pow2 scale, 4-bit significands)
        uint32_t outw[4][8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          float sc = st.s[k][j];
#pragma unroll
          for (int w = 0; w < 4; w++) {
            uint32_t word = st.v[k][j][w];
            f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
            f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true);
            outw[j][2 * w] = pack_bf16x2(lo.x * sc, lo.y * sc);
            outw[j][2 * w + 1] = pack_bf16x2(hi.x * sc, hi.y * sc);
          }
          uint16_t* dst = kt + (rq * 4 + j) * C::KS + c * 16;
          *(u32x4_t*)dst = u32x4_t{outw[j][0], outw[j][1], outw[j][2], outw[j][3]};
          *(u32x4_t*)(dst + 8) = u32x4_t{outw[j][4], outw[j][5], outw[j][6], outw[j][7]};
        }
        if (c * 16 < DV) {
#pragma unroll
          for (int e = 0; e < 16; e++) {
            int w = e >> 1, hi = e & 1;
            uint32_t x0 = outw[0][w], x1 = outw[1][w], x2 = outw[2][w], x3 = outw[3][w];
            uint32_t lo01, lo23;
            if (hi) {
              lo01 = (x0 >> 16) | (x1 & 0xffff0000u);
              lo23 = (x2 >> 16) | (x3 & 0xffff0000u);
            } else {
              lo01 = (x0 & 0xffffu) | (x1 << 16);
              lo23 = (x2 & 0xffffu) | (x3 << 16);
            }
            *(u32x2_t*)(vt + (c * 16 + e) * C::VS + slot0) = u32x2_t{lo01, lo23};
          }
        }
      }
    }
  }
}

template <int D, int DV, bool FP8>
__global__ __launch_bounds__(kThreads, 1) void attn_mfma_kernel(
    const uint16_t* __restrict__ q, RowSrc src, const float* __restrict__ sink,
    const int32_t* __restrict__ idx, int T, int S, int H, int rows_per_split, float scale,
    float* __restrict__ part, void* __restrict__ out, int out_dtype) {
  using C = MfmaCfg<D, DV>;
  extern __shared__ __align__(16) uint16_t lds[];
  int* valid = (int*)(lds + 2 * C::BUF_ELEMS);  // [2][32]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int split = blockIdx.x;
  const int nsplit = gridDim.x;
  const int64_t bs = blockIdx.y;
  const int hg = blockIdx.z;
  const int64_t b = bs / S;
  const int head = hg * 64 + wave * 16 + c;
  const bool head_ok = head < H;

  const int t_begin = split * rows_per_split;
  const int t_end = min(T, t_begin + rows_per_split);
  const int ntiles = (t_end - t_begin + kTileRows - 1) / kTileRows;
  const int32_t* ids = idx + bs * (int64_t)T;

  // Q^T fragments: lane (g, c) holds q[head c][32j + 8g .. +7]
  bf16x8_t qf[C::KSTEPS];
  {
    const uint16_t* qh = q + (bs * H + (head_ok ? head : 0)) * (int64_t)D + 8 * g;
#pragma unroll
    for (int j = 0; j < C::KSTEPS; j++) {
      u32x4_t w = head_ok ? *(const u32x4_t*)(qh + 32 * j) : u32x4_t{0u, 0u, 0u, 0u};
      qf[j] = __builtin_bit_cast(bf16x8_t, w);
    }
  }

  f32x4_t o[C::DVT];
#pragma unroll
  for (int i = 0; i < C::DVT; i++) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_ref = -SMLA_INF;  // per head (uniform over the 4 lane groups)
  float l_lane = 0.f;        // this lane's share of the denominator

  Stage<D, FP8> st;
  if (ntiles > 0) {
    stage_load<D, DV, FP8>(st, src, b, ids, t_begin, t_end, tid);
    stage_store<D, DV, FP8>(st, lds, valid, tid);
  }
  for (int it = 0; it < ntiles; it++) {
    const int cur = it & 1;
    uint16_t* buf = lds + cur * C::BUF_ELEMS;
    const int* vld = valid + cur * kTileRows;
    const bool more = it + 1 < ntiles;
    if (more) stage_load<D, DV, FP8>(st, src, b, ids, t_begin + (it + 1) * kTileRows, t_end, tid);
    __syncthreads();

    // ---- S^T = K Q^T for 32 rows x 16 heads
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    const uint16_t* kt0 = buf + c * C::KS + 8 * g;
    const uint16_t* kt1 = buf + (16 + c) * C::KS + 8 * g;
#pragma unroll
    for (int j = 0; j < C::KSTEPS; j++) {
      bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(kt0 + 32 * j));
      bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(kt1 + 32 * j));
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[j], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[j], s1, 0, 0, 0);
    }
    // ---- online softmax (rows 4g+i and 16+4g+i of this tile, head c)
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[i] = vld[4 * g + i] ? s0[i] * scale : -SMLA_INF;
      x[4 + i] = vld[16 + 4 * g + i] ? s1[i] * scale : -SMLA_INF;
    }
    float mt = x[0];
#pragma unroll
    for (int i = 1; i < 8; i++) mt = fmaxf(mt, x[i]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // move the reference max only when needed (wave-uniform decision)
    bool need = (mt > m_ref + kRescaleSlack) || (m_ref == -SMLA_INF && mt > -SMLA_INF);
    if (__builtin_amdgcn_ballot_w64(need)) {
      float m_new = need ? mt : m_ref;
      float alpha = (m_ref > -SMLA_INF) ? __expf(m_ref - m_new) : 0.f;
      if (need) {
        l_lane *= alpha;
#pragma unroll
        for (int i = 0; i < C::DVT; i++) o[i] *= alpha;
        m_ref = m_new;
      }
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float e = (m_ref > -SMLA_INF) ? __expf(x[i] - m_ref) : 0.f;
      p[i] = bf16_round(e);  // value used by the P.V product
      l_lane += p[i];
    }
    u32x4_t pw = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                  pack_bf16x2(p[6], p[7])};
    bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pw);

    // ---- O^T += V^T P^T
    const uint16_t* vt = buf + C::KTILE_ELEMS + c * C::VS + 8 * g;
#pragma unroll
    for (int i = 0; i < C::DVT; i++) {
      bf16x8_t a = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(vt + 16 * i * C::VS));
      o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[i], 0, 0, 0);
    }
    if (more) stage_store<D, DV, FP8>(st, lds + (cur ^ 1) * C::BUF_ELEMS, valid + (cur ^ 1) * kTileRows, tid);
  }

  // ---- finish: total denominator share over the 4 lane groups
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!head_ok) return;
  if (nsplit == 1) {
    float snk = sink ? sink[head] : -SMLA_INF;
    bool empty = !(m_ref > -SMLA_INF);
    float den = l_tot + (empty ? 0.f : __expf(snk - m_ref));
    float inv = 1.0f / den;
    int64_t obase = (bs * H + head) * (int64_t)DV;
#pragma unroll
    for (int i = 0; i < C::DVT; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float v = empty ? __builtin_nanf("") : o[i][r] * inv;
        int64_t dv = 16 * i + 4 * g + r;
        if (out_dtype == SMLA_BF16) ((uint16_t*)out)[obase + dv] = bf16_rne(v);
        else ((float*)out)[obase + dv] = v;
      }
    }
  } else {
    // partial state: [bs][H][nsplit] records of (m, l) and O[DV]
    int64_t rec = (bs * nsplit + split) * H + head;  // split-major partial records
    float* ml = part + rec * 2;
    float* op = part + (int64_t)gridDim.y * H * nsplit * 2 + rec * DV;
    if (g == 0) {
      ml[0] = m_ref;
      ml[1] = l_tot;
    }
#pragma unroll
    for (int i = 0; i < C::DVT; i++) *(f32x4_t*)(op + 16 * i + 4 * g) = o[i];
  }
}

// Merge of split partial states.  The nsplit states (m_j, l_j, O_j) of one (query row, head) are
// stored split-major ([row][split][head], so each split workgroup writes one contiguous block) and
// merge as
//   M = max m_j,  w_j = exp(m_j - M),  O = sum w_j O_j / (sum w_j l_j + exp(sink - M)).
// One workgroup of WAVES waves per (query row, head); thread t owns value columns
// CPL*t .. CPL*t+CPL-1 (CPL = 512 / (64 WAVES)).  The O loads of the first CHUNK splits (16 to 64)
// are issued before the (m, l) loads, so for up to CHUNK splits one memory round trip covers the
// whole merge;
// (m, l) and the weights pass through LDS, so any split count up to kMaxSplits takes the same path.
constexpr int kMaxSplits = 1024;

template <int WAVES, bool BF16P, int CH, int DVS = 1>
__global__ __launch_bounds__(WAVES * 64) void attn_merge_kernel(const float* __restrict__ part, int nsplit,
                                                                int64_t BS, int H, const float* __restrict__ sink,
                                                                void* __restrict__ out, int out_dtype) {
  constexpr int NT = WAVES * 64;
  constexpr int DV = 512;
  constexpr int CPL = DV / (DVS * NT);                // value columns per thread: 4, 2 or 1
  // DVS > 1: the row's columns are split over DVS workgroups (blockIdx.y), for row counts too small
  // to spread over the CUs otherwise
  constexpr int LW = BF16P ? (CPL + 1) / 2 : CPL;     // 32-bit words loaded per split
  constexpr int CHUNK = CH < 64 / LW ? CH : 64 / LW;  // splits in flight: at most 64 words per thread
  static_assert(CPL >= 1 && CPL <= 4 && DVS * NT * CPL == DV, "merge thread layout");
  static_assert(kMaxSplits % CHUNK == 0, "padded weights fit the table");
  __shared__ __align__(16) float m_s[kMaxSplits];
  __shared__ float l_s[kMaxSplits];
  __shared__ float red[2][WAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t rh = blockIdx.x;  // bs*H + head
  const int64_t bs = rh / H;
  const int head = (int)(rh % H);
  const int64_t rec0 = bs * nsplit * (int64_t)H + head;  // record of split 0; splits are H records apart
  const float* ml = part + rec0 * 2;
  const int dv0 = (int)blockIdx.y * (DV / DVS) + tid * CPL;
  const int64_t jstride = (int64_t)H * DV;  // elements between consecutive splits
  const float* obase = part + BS * H * nsplit * 2;

  uint32_t v[CHUNK][LW];
  // unconditional loads (an index past the last split re-reads the last one, whose weight in the
  // padded table is zero): a guarded load would become a branch with a full wait behind it
  auto load_chunk = [&](int j0) {
#pragma unroll
    for (int u = 0; u < CHUNK; u++) {
      const int j = min(j0 + u, nsplit - 1);
      if constexpr (BF16P) {
        const uint16_t* p = (const uint16_t*)obase + rec0 * DV + j * jstride + dv0;
        if constexpr (CPL == 4) {
          const u32x2_t t = *(const u32x2_t*)p;
          v[u][0] = t[0];
          v[u][1] = t[1];
        } else if constexpr (CPL == 2) {
          v[u][0] = *(const uint32_t*)p;
        } else {
          v[u][0] = (uint32_t)*p;
        }
      } else {
        const float* p = obase + rec0 * DV + j * jstride + dv0;
        if constexpr (CPL == 4) {
          const f32x4_t t = *(const f32x4_t*)p;
#pragma unroll
          for (int c = 0; c < 4; c++) v[u][c] = __float_as_uint(t[c]);
        } else if constexpr (CPL == 2) {
          const u32x2_t t = *(const u32x2_t*)p;
          v[u][0] = t[0];
          v[u][1] = t[1];
        } else {
          v[u][0] = __float_as_uint(*p);
        }
      }
    }
  };
  load_chunk(0);

  // (m, l) of every split to LDS; row max M
  float mx = -SMLA_INF;
  for (int j = tid; j < nsplit; j += NT) {
    const float m = ml[(int64_t)j * H * 2], l = ml[(int64_t)j * H * 2 + 1];
    m_s[j] = m;
    l_s[j] = l;
    mx = fmaxf(mx, m);
  }
  mx = wave_max_dpp(mx);
  if (lane == 0) red[0][wave] = mx;
  __syncthreads();
  float M = red[0][0];
#pragma unroll
  for (int w = 1; w < WAVES; w++) M = fmaxf(M, red[0][w]);
  const bool empty = !(M > -SMLA_INF);
  // weights w_j (in place of m_j) and the denominator L
  // (zero weights pad the last chunk, so the accumulation below runs whole chunks)
  float lsum = 0.f;
  const int npad = (nsplit + CHUNK - 1) / CHUNK * CHUNK;
  for (int j = tid; j < npad; j += NT) {
    const float m = j < nsplit ? m_s[j] : -SMLA_INF;
    const float w = m > -SMLA_INF ? __expf(m - M) : 0.f;
    m_s[j] = w;
    if (j < nsplit) lsum += w * l_s[j];
  }
  lsum = wave_sum_dpp(lsum);
  if (lane == 0) red[1][wave] = lsum;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; w++) L += red[1][w];

  float acc[CPL];
#pragma unroll
  for (int c = 0; c < CPL; c++) acc[c] = 0.f;
  for (int j0 = 0; j0 < nsplit; j0 += CHUNK) {
    if (j0 > 0) load_chunk(j0);
#pragma unroll
    for (int u = 0; u < CHUNK; u++) {
      const float w = m_s[j0 + u];
      if constexpr (BF16P) {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
          const uint32_t x = v[u][c >> 1];
          acc[c] += w * __uint_as_float((c & 1) ? (x & 0xffff0000u) : (x << 16));
        }
      } else {
#pragma unroll
        for (int c = 0; c < CPL; c++) acc[c] += w * __uint_as_float(v[u][c]);
      }
    }
  }
  const float snk = sink ? sink[head] : -SMLA_INF;
  if (!empty) L += __expf(snk - M);
  const float inv = 1.0f / L;
  const int64_t o = rh * DV + dv0;
  const float nan = __builtin_nanf("");
  if (out_dtype == SMLA_BF16) {
    uint16_t* po = (uint16_t*)out + o;
    if constexpr (CPL == 4) {
      *(u32x2_t*)po = empty ? u32x2_t{0x7fc07fc0u, 0x7fc07fc0u}
                            : u32x2_t{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
    } else if constexpr (CPL == 2) {
      *(uint32_t*)po = empty ? 0x7fc07fc0u : pack_bf16x2(acc[0] * inv, acc[1] * inv);
    } else {
      *po = empty ? (uint16_t)0x7fc0u : bf16_rne(acc[0] * inv);
    }
  } else {
    float* po = (float*)out + o;
#pragma unroll
    for (int c = 0; c < CPL; c++) po[c] = empty ? nan : acc[c] * inv;
  }
}

// ---------------------------------------------------------------------------------------------
// Launch planning (shared by the workspace query and the launcher).
struct Plan {
  bool mfma;
  int rows_per_split;
  int nsplit;
  int hgroups;
};

int g_target_wgs = 0;  // 0 = default (number of CUs); settable for tuning
hipEvent_t g_ev_before = nullptr, g_ev_after = nullptr;  // profiling: bracket the main kernel
bool g_main_only = false;  // profiling: launch the split kernel alone (partials, no merge)
int g_decode_kernel = 0;   // bf16 rows: 0 = role-split score/value waves, 1 = 64-head lockstep tiles

int num_cus() { return smla_num_cus(); }

Plan make_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t T, int q_dtype,
               int kv_dtype) {
  Plan p{};
  p.mfma = q_dtype == SMLA_BF16 && (kv_dtype == SMLA_BF16 || kv_dtype == SMLA_FP8_E4M3) &&
           H % 16 == 0 && DV == 512 && (D == 576 || D == 512) && T > 0 && T < (1ll << 30);
  if (!p.mfma) return p;
  p.hgroups = (int)((H + 63) / 64);
  int64_t rows = B * S * p.hgroups;
  int64_t tiles = (T + kTileRows - 1) / kTileRows;
  int64_t target = g_target_wgs > 0 ? g_target_wgs : num_cus();
  // tiles per split so that rows * nsplit ~ target workgroups
  int64_t per = (tiles * rows + target - 1) / target;
  if (per < 1) per = 1;
  // a split's fixed costs (its Q block, index table and partial record) outweigh one 32-row tile,
  // and every split adds a partial to merge: at least two tiles per split once the list has four
  // (the default plan; an explicit target is taken as given)
  if (g_target_wgs <= 0 && per < 2 && tiles >= 4) per = 2;
  if ((tiles + per - 1) / per > kMaxSplits) per = (tiles + kMaxSplits - 1) / kMaxSplits;
  if (per > tiles) per = tiles;
  // role-split kernel: splits of up to 8192 rows (the launcher picks the 4-tile ring for splits of
  // at most 256 rows, a 3-tile ring with a larger index table beyond)
  const bool v6 = (kv_dtype == SMLA_BF16 || kv_dtype == SMLA_FP8_E4M3) && g_decode_kernel == 0;
  const int max_rows = v6 ? smla_attn::kDecodeV6MaxRows : smla_attn::kDecodeMaxRowsPerSplit;
  if (per > max_rows / kTileRows) per = max_rows / kTileRows;
  p.rows_per_split = (int)(per * kTileRows);
  p.nsplit = (int)((tiles + per - 1) / per);
  if (p.nsplit > kMaxSplits) p.mfma = false;  // beyond the merge kernel's capacity: generic kernel
  return p;
}

int launch_merge(const Plan& p, int64_t B, int64_t S, int64_t H, const float* sink, void* out, int out_dtype,
                 void* ws, hipStream_t stream, int part_bf16) {
  if (p.nsplit <= 1) return SMLA_OK;
  const int64_t rows = B * S * H;
  // waves per (row, head): enough workgroups in flight to cover the partials' latency; below 256
  // rows, one wave per quarter of the row's columns (4-byte loads, 4 workgroups per row)
  const int waves = rows >= 1024 ? 2 : rows >= 256 ? 4 : 1;
  const dim3 grid((unsigned)rows, waves == 1 ? 4u : 1u), block(waves * 64);
  // splits in flight per chunk: the smallest of 16 / 32 / 64 that covers nsplit
  const int ch = p.nsplit <= 16 ? 16 : p.nsplit <= 32 ? 32 : 64;
#define SMLA_MERGE(W, BP, C) hipLaunchKernelGGL((attn_merge_kernel<W, BP, C, (W == 1 ? 4 : 1)>), grid, block, 0, \
                                                stream, (const float*)ws, p.nsplit, B * S, (int)H, sink, out, out_dtype)
#define SMLA_MERGE_CH(W, BP) \
  if (ch == 16) SMLA_MERGE(W, BP, 16); else if (ch == 32) SMLA_MERGE(W, BP, 32); else SMLA_MERGE(W, BP, 64)
  if (part_bf16) {
    if (waves == 2) {
      SMLA_MERGE_CH(2, true);
    } else if (waves == 4) {
      SMLA_MERGE_CH(4, true);
    } else {
      SMLA_MERGE_CH(1, true);
    }
  } else {
    if (waves == 2) {
      SMLA_MERGE_CH(2, false);
    } else if (waves == 4) {
      SMLA_MERGE_CH(4, false);
    } else {
      SMLA_MERGE_CH(1, false);
    }
  }
#undef SMLA_MERGE_CH
#undef SMLA_MERGE
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

template <int D, bool FP8>
int launch_mfma(const Plan& p, const void* q, RowSrc src, const float* sink, const int32_t* idx,
                int64_t T, int64_t B, int64_t S, int64_t H, float scale, void* out, int out_dtype,
                void* ws, hipStream_t stream) {
  if constexpr (!FP8) {
    int rc;
    if (g_decode_kernel == 0) {
      if (g_ev_before) (void)hipEventRecord(g_ev_before, stream);
      rc = smla_attn::launch_decode_v6(D, false, p.nsplit, p.rows_per_split, q, src, sink, idx, T, B, S, H, scale,
                                       out, out_dtype, (float*)ws, stream);
      if (g_ev_after) (void)hipEventRecord(g_ev_after, stream);
    } else {
      rc = smla_attn::launch_decode_bf16(D, p.nsplit, p.rows_per_split, q, src, sink, idx, T, B, S, H, scale, out,
                                         out_dtype, (float*)ws, stream, g_ev_before, g_ev_after);
    }
    if (rc != SMLA_OK || g_main_only) return rc;
    return launch_merge(p, B, S, H, sink, out, out_dtype, ws, stream, out_dtype == SMLA_BF16);
  }
  if (g_decode_kernel == 0) {  // fp8 rows on the role-split kernel
    int rc = smla_attn::launch_decode_v6(D, true, p.nsplit, p.rows_per_split, q, src, sink, idx, T, B, S, H, scale,
                                         out, out_dtype, (float*)ws, stream);
    if (rc != SMLA_OK || g_main_only) return rc;
    return launch_merge(p, B, S, H, sink, out, out_dtype, ws, stream, out_dtype == SMLA_BF16);
  }
  using C = MfmaCfg<D, 512>;
  auto kern = attn_mfma_kernel<D, 512, FP8>;
  static std::atomic<uint64_t> lds_attr{0};  // devices whose limit is raised
  if (hipError_t e = smla_set_dynamic_lds((const void*)kern, (int)C::LDS_BYTES, lds_attr); e != hipSuccess) return (int)e;
  dim3 grid(p.nsplit, (unsigned)(B * S), p.hgroups);
  if (g_ev_before) (void)hipEventRecord(g_ev_before, stream);
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), C::LDS_BYTES, stream, (const uint16_t*)q, src, sink,
                     idx, (int)T, (int)S, (int)H, p.rows_per_split, scale, (float*)ws, out, out_dtype);
  SMLA_HIP_CHECK_LAUNCH();
  if (g_ev_after) (void)hipEventRecord(g_ev_after, stream);
  return launch_merge(p, B, S, H, sink, out, out_dtype, ws, stream, 0);
}

}  // namespace

extern "C" size_t smla_sparse_attn_workspace(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV,
                                             int64_t T, int q_dtype, int kv_dtype) {
  Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype);
  if (!p.mfma || p.nsplit <= 1) return 0;
  return (size_t)(B * S * H) * p.nsplit * (2 + DV) * sizeof(float);
}

extern "C" int smla_sparse_attn(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1,
                                int64_t n1, int kv_dtype, const float* kv0_scale, const float* kv1_scale,
                                const float* attn_sink, const int32_t* topk_idxs, int64_t T, int64_t B,
                                int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out,
                                int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !kv0 || !topk_idxs || !out) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0 || DV <= 0 || DV > D || T <= 0 || n0 < 0 || n1 < 0 ||
      n0 + n1 <= 0)
    return SMLA_E_SHAPE;
  if (n1 > 0 && !kv1) return SMLA_E_NULL;
  if (q_dtype != SMLA_F32 && q_dtype != SMLA_BF16 && q_dtype != SMLA_F16) return SMLA_E_DTYPE;
  if (kv_dtype != SMLA_F32 && kv_dtype != SMLA_BF16 && kv_dtype != SMLA_F16 && kv_dtype != SMLA_FP8_E4M3)
    return SMLA_E_DTYPE;
  if (out_dtype != SMLA_F32 && out_dtype != SMLA_BF16) return SMLA_E_DTYPE;
  if (kv_dtype == SMLA_FP8_E4M3) {
    if (D % 64 != 0) return SMLA_E_SHAPE;
    if (!kv0_scale || (n1 > 0 && !kv1_scale)) return SMLA_E_NULL;
  }
  if (DV > 1024 || n0 + n1 > (1ll << 31) - 1) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  RowSrc src{kv0, kv1, kv_dtype == SMLA_FP8_E4M3 ? kv0_scale : nullptr,
             kv_dtype == SMLA_FP8_E4M3 ? kv1_scale : nullptr, n0, n1};
  Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype);
  if (p.mfma) {
    size_t need = smla_sparse_attn_workspace(B, S, H, D, DV, T, q_dtype, kv_dtype);
    if (need > 0 && (!workspace || workspace_bytes < need)) return SMLA_E_WORKSPACE;
    bool fp8 = kv_dtype == SMLA_FP8_E4M3;
    if (D == 576)
      return fp8 ? launch_mfma<576, true>(p, q, src, attn_sink, topk_idxs, T, B, S, H, scale, out, out_dtype, workspace, st)
                 : launch_mfma<576, false>(p, q, src, attn_sink, topk_idxs, T, B, S, H, scale, out, out_dtype, workspace, st);
    return fp8 ? launch_mfma<512, true>(p, q, src, attn_sink, topk_idxs, T, B, S, H, scale, out, out_dtype, workspace, st)
               : launch_mfma<512, false>(p, q, src, attn_sink, topk_idxs, T, B, S, H, scale, out, out_dtype, workspace, st);
  }
  size_t lds = (size_t)D * 4 + kThreads * 8;
  if (lds > 64 * 1024) return SMLA_E_UNSUPPORTED;
  hipLaunchKernelGGL(attn_generic_kernel, dim3((unsigned)(B * S * H)), dim3(kThreads), lds, st, q, q_dtype,
                     src, kv_dtype, attn_sink, topk_idxs, T, S, H, D, DV, scale, out, out_dtype);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

// tuning hook (not part of the public header): target number of workgroups for the split plan
extern "C" void smla_set_attn_target_wgs(int n) { g_target_wgs = n; }

// profiling hook (not part of the public header): when set, the MFMA attention path records
// `before` / `after` on its stream immediately around the main kernel (not the merge)
extern "C" void smla_profile_set_attn_events(void* before, void* after) {
  g_ev_before = (hipEvent_t)before;
  g_ev_after = (hipEvent_t)after;
}

// tuning hook (not part of the public header): bf16-row decode kernel, 0 = role-split score/value
// waves (default), 1 = 64-head lockstep tiles
extern "C" void smla_set_attn_decode_kernel(int k) { g_decode_kernel = k; }

// profiling hook (not part of the public header): when on, the MFMA attention path launches only
// its split kernel (the workspace partials are written, the output is not), so that a sequence of
// such launches times that kernel alone
extern "C" void smla_profile_set_attn_main_only(int on) { g_main_only = on != 0; }

// split plan of the MFMA path for these sizes: writes nsplit and rows per split (0 if the generic
// kernel would run)
extern "C" void smla_attn_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t T, int q_dtype,
                               int kv_dtype, int* nsplit, int* rows_per_split) {
  Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype);
  *nsplit = p.mfma ? p.nsplit : 0;
  *rows_per_split = p.mfma ? p.rows_per_split : 0;
}
