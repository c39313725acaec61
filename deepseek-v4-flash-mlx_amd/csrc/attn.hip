// Sparse absorbed-MLA attention over gathered latent rows.
//
// Semantics follow ref_torch/sparse_attn.py:23-34 (sparse_attn): gather kv[idx] (idx < 0 masked),
// logits = scale * q.kv, softmax over valid rows with exp(sink - rowmax) added to the
// denominator, output = weighted sum of the first DV columns of the gathered rows.
//
// This file holds:
//  * attn_generic_kernel — fp32 VALU, any dtype / shape; one workgroup of 16 waves per (b, s, head),
//    a wave per gathered row at a time.  This is the fp32 path (1e-5 parity) and the path for
//    shapes the MFMA kernel does not cover.
//  * attn_merge_kernel / attn_merge_frag_kernel — log-sum-exp merge of the split partial states
//    that the MFMA split kernel (attn_decode.hip) writes (fp32 rows / bf16 in MFMA fragment order).
//  * the split plan and the C entry points.
#include <algorithm>
#include <mutex>

#include "attn_common.h"

namespace {

using smla_attn::kRescaleSlack;
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

// ---------------------------------------------------------------------------------------------
// Generic VALU kernel: one workgroup of 16 waves per (query row, head).  Each wave takes a
// contiguous sixteenth of the index list and walks it R rows at a time: lane l holds columns
// l, l+64, ... of each row (coalesced row loads, 64 columns per load instruction), the dot with q
// is a DPP wave sum, and the wave keeps its own online-softmax state (m, l, O).  The 16 states merge
// through LDS at the end in a fixed order, so the result does not depend on timing.  The kernel is
// bound by each workgroup's own gather: every (query row, head) reads all T rows (1.2 MB for 512
// fp32 rows of 576), about the rate one CU takes in.
constexpr int kGenWaves = 16;
constexpr int kGenThreads = 64 * kGenWaves;

// a row element in its storage type (the register a load lands in) and its fp32 value
template <int KT>
using RawElem = typename std::conditional<
    KT == SMLA_F32, float,
    typename std::conditional<KT == SMLA_BF16, uint16_t,
                              typename std::conditional<KT == SMLA_F16, _Float16, uint8_t>::type>::type>::type;
template <int KT>
__device__ inline float raw_to_f32(RawElem<KT> x) {
  if constexpr (KT == SMLA_F32) return x;
  else if constexpr (KT == SMLA_BF16) return bf16_bits_to_f32(x);
  else if constexpr (KT == SMLA_F16) return (float)x;
  else return e4m3_to_f32(x);
}

template <int KT>
__device__ inline float load_elem(const uint8_t* row, int64_t i) {
  if constexpr (KT == SMLA_F32) return ((const float*)row)[i];
  else if constexpr (KT == SMLA_BF16) return bf16_bits_to_f32(((const uint16_t*)row)[i]);
  else if constexpr (KT == SMLA_F16) return (float)((const _Float16*)row)[i];
  else return e4m3_to_f32(row[i]);
}

// KT: row dtype; NC: 64-column chunks of a row held in registers; ONE: the whole row fits NC chunks
// (D <= 64 NC), so the value columns are taken from the registers the dot used; otherwise the dot
// runs over the row in blocks of NC chunks and the value columns (DV <= 1024) are loaded again.
// Grid (B*S*H, nsplit): with nsplit > 1 workgroup (row, head, split j) takes the j-th of nsplit
// equal runs of the index list and writes its partial state (m, l, unnormalised O) to `part`
// ([row, head][split] records of (m, l), then of DV values) for attn_generic_merge_kernel.
template <int KT, int NC, bool ONE>
__global__ __launch_bounds__(kGenThreads) void attn_generic_kernel(
    const void* __restrict__ q, int q_dtype, RowSrc src, const float* __restrict__ sink,
    const int32_t* __restrict__ idx, int64_t T, int64_t S, int64_t H, int64_t D, int64_t DV, float scale,
    void* __restrict__ out, int out_dtype, float* __restrict__ part) {
  // rows per batch: two batches in flight per wave when the row fits NC chunks (ONE), one
  // otherwise; sized to the 128 registers of a 16-wave workgroup (3 rows per batch at NC = 9
  // spill, and measured no faster)
  constexpr int R = ONE ? (NC <= 4 ? 8 : (NC <= 9 ? 2 : 1)) : 2;
  constexpr int NA = ONE ? NC : 16;                   // value chunks held (DV <= 1024)
  constexpr int ES = KT == SMLA_F32 ? 4 : (KT == SMLA_FP8_E4M3 ? 1 : 2);
  constexpr int HW = kGenWaves / 2;
  extern __shared__ float smem[];
  float* sq = smem;     // [D] the query row
  float* buf = sq + D;  // [HW][DV] weighted partial outputs
  __shared__ float sm[kGenWaves], sl[kGenWaves];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t h = blockIdx.x % H;
  const int64_t bs = blockIdx.x / H;
  const int64_t b = batch_of(bs, S);
  const int64_t ntot = src.n0 + src.n1;
  const int nch = (int)((D + 63) >> 6);

  for (int64_t d = tid; d < D; d += kGenThreads) sq[d] = load_as_f32(q, (bs * H + h) * D + d, q_dtype);
  __syncthreads();
  float qv[ONE ? NC : 1];
  if constexpr (ONE) {
#pragma unroll
    for (int c = 0; c < NC; c++) qv[c] = 64 * c + lane < D ? sq[64 * c + lane] : 0.f;
  }
  float acc[NA];
#pragma unroll
  for (int c = 0; c < NA; c++) acc[c] = 0.f;
  float m_run = -SMLA_INF, l_run = 0.f;

  const int32_t* ids = idx + bs * T;
  const int nsplit = gridDim.y, split = blockIdx.y;
  const int64_t tps = (T + nsplit - 1) / nsplit;  // list entries per split
  const int64_t t0 = split * tps, t1 = t0 + tps < T ? t0 + tps : T;
  const int64_t per = (t1 - t0 + kGenWaves - 1) / kGenWaves;
  const int64_t t_beg = t0 + wv * per;
  const int64_t t_end = t_beg + per < t1 ? t_beg + per : t1;
  // online-softmax update of the wave's state with R rows: scores s (-inf: masked), values in
  // x(k, c) for the NA value chunks
  auto update = [&](const float (&s)[R], auto&& x) {
    float mx = m_run;
#pragma unroll
    for (int k = 0; k < R; k++) mx = fmaxf(mx, s[k]);
    if (mx > -SMLA_INF) {
      const float alpha = m_run > -SMLA_INF ? __expf(m_run - mx) : 0.f;
      float p[R];
      float ps = 0.f;
#pragma unroll
      for (int k = 0; k < R; k++) {
        p[k] = s[k] > -SMLA_INF ? __expf(s[k] - mx) : 0.f;
        ps += p[k];
      }
      l_run = l_run * alpha + ps;
#pragma unroll
      for (int c = 0; c < NA; c++) {
        float a = acc[c] * alpha;
#pragma unroll
        for (int k = 0; k < R; k++) a = fmaf(p[k], x(k, c), a);
        acc[c] = a;
      }
      m_run = mx;
    }
  };
  if constexpr (ONE) {
    // Two batches of R rows in flight: a batch's loads are issued one batch ahead of their use.
    // Every fetch issues the same loads (masked rows read row 0, columns past D column D - 1,
    // rows past the block are masked), so the compiler's wait counts stay exact.
    struct Batch {
      RawElem<KT> v[R][NC];
      float sc[R][KT == SMLA_FP8_E4M3 ? NC : 1];
      bool ok[R];
    };
    for (int64_t tb = t_beg; tb < t_end; tb += 64) {
      const int nb = (int)(t_end - tb < 64 ? t_end - tb : 64);
      const int idv = lane < nb ? ids[tb + lane] : -1;
      auto fetch = [&](int j, Batch& bt) {
#pragma unroll
        for (int k = 0; k < R; k++) {
          const int r = j + k < nb ? __builtin_amdgcn_readlane(idv, (j + k) & 63) : -1;
          bt.ok[k] = r >= 0 && r < ntot;
          const float* sp = nullptr;
          const uint8_t* rp = row_ptr(src, b, bt.ok[k] ? r : 0, D, ES, &sp);
#pragma unroll
          for (int c = 0; c < NC; c++) {
            const int64_t d = 64 * c + lane < D ? 64 * c + lane : D - 1;
            bt.v[k][c] = ((const RawElem<KT>*)rp)[d];
            if constexpr (KT == SMLA_FP8_E4M3) bt.sc[k][c] = sp[c < nch ? c : nch - 1];
          }
        }
      };
      // element (k, c) of a fetched batch as fp32 (0 for masked rows and columns past D); computed
      // where it is used, so a batch holds only its loaded registers
      auto elem = [&](const Batch& bt, int k, int c) -> float {
        float x = 64 * c + lane < D ? raw_to_f32<KT>(bt.v[k][c]) : 0.f;
        if constexpr (KT == SMLA_FP8_E4M3) x *= bt.sc[k][c];
        return bt.ok[k] ? x : 0.f;
      };
      auto consume = [&](const Batch& bt) {
        float s[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
          float dt = 0.f;
#pragma unroll
          for (int c = 0; c < NC; c++) dt = fmaf(qv[c], elem(bt, k, c), dt);
          const float tot = wave_sum_dpp(dt);
          s[k] = bt.ok[k] ? scale * tot : -SMLA_INF;
        }
        update(s, [&](int k, int c) { return elem(bt, k, c); });
      };
      Batch ba, bb;
      fetch(0, ba);
      for (int j = 0; j < nb; j += 2 * R) {
        fetch(j + R, bb);
        consume(ba);
        fetch(j + 2 * R, ba);
        if (j + R < nb) consume(bb);
      }
    }
  }
  if constexpr (!ONE) {
    // rows longer than NC chunks: the dot in blocks of NC chunks, the value columns loaded again
    for (int64_t tb = t_beg; tb < t_end; tb += 64) {
      const int nb = (int)(t_end - tb < 64 ? t_end - tb : 64);
      const int idv = lane < nb ? ids[tb + lane] : -1;
      for (int j = 0; j < nb; j += R) {
        const uint8_t* rp[R];
        const float* sp[R];
        bool ok[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
          const int r = j + k < nb ? __builtin_amdgcn_readlane(idv, (j + k) & 63) : -1;
          ok[k] = r >= 0 && r < ntot;
          sp[k] = nullptr;
          rp[k] = ok[k] ? row_ptr(src, b, r, D, ES, &sp[k]) : nullptr;
        }
        float dot[R];
#pragma unroll
        for (int k = 0; k < R; k++) dot[k] = 0.f;
        for (int c0 = 0; c0 < nch; c0 += NC) {
          float w[R][NC];
#pragma unroll
          for (int k = 0; k < R; k++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
              const int cc = c0 + c;
              const int64_t d = 64 * (int64_t)cc + lane;
              float x = 0.f;
              if (ok[k] && cc < nch && d < D) {
                x = load_elem<KT>(rp[k], d);
                if constexpr (KT == SMLA_FP8_E4M3) x *= sp[k][cc];
              }
              w[k][c] = x;
            }
#pragma unroll
          for (int c = 0; c < NC; c++) {
            const int64_t d = 64 * (int64_t)(c0 + c) + lane;
            const float qd = d < D ? sq[d] : 0.f;
#pragma unroll
            for (int k = 0; k < R; k++) dot[k] = fmaf(qd, w[k][c], dot[k]);
          }
        }
        float s[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
          const float tot = wave_sum_dpp(dot[k]);
          s[k] = ok[k] ? scale * tot : -SMLA_INF;
        }
        update(s, [&](int k, int c) {
          const int64_t d = 64 * c + lane;
          float x = 0.f;
          if (ok[k] && d < DV) {
            x = load_elem<KT>(rp[k], d);
            if constexpr (KT == SMLA_FP8_E4M3) x *= sp[k][c];
          }
          return x;
        });
      }
    }
  }

  // merge of the 16 wave states: weights exp(m_w - M), partial outputs summed in wave order
  if (lane == 0) {
    sm[wv] = m_run;
    sl[wv] = l_run;
  }
  __syncthreads();
  float M = -SMLA_INF;
#pragma unroll
  for (int w = 0; w < kGenWaves; w++) M = fmaxf(M, sm[w]);
  const float wt = m_run > -SMLA_INF ? __expf(m_run - M) : 0.f;
  if (wv >= HW) {
#pragma unroll
    for (int c = 0; c < NA; c++)
      if (64 * c + lane < DV) buf[(wv - HW) * DV + 64 * c + lane] = acc[c] * wt;
  }
  __syncthreads();
  if (wv < HW) {
#pragma unroll
    for (int c = 0; c < NA; c++)
      if (64 * c + lane < DV) buf[wv * DV + 64 * c + lane] = fmaf(acc[c], wt, buf[wv * DV + 64 * c + lane]);
  }
  __syncthreads();
  float den = 0.f;
#pragma unroll
  for (int w = 0; w < kGenWaves; w++) den += (sm[w] > -SMLA_INF ? __expf(sm[w] - M) : 0.f) * sl[w];
  const int64_t rh = bs * H + h;
  if (nsplit > 1) {  // partial state: (M, l) and the unnormalised O of this split
    const int64_t rec = rh * nsplit + split;
    if (tid == 0) {
      part[rec * 2] = M;
      part[rec * 2 + 1] = den;
    }
    float* po = part + (int64_t)gridDim.x * nsplit * 2 + rec * DV;
    for (int64_t d = tid; d < DV; d += kGenThreads) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < HW; w++) o += buf[w * DV + d];
      po[d] = o;
    }
    return;
  }
  const bool empty = !(M > -SMLA_INF);
  const float snk = sink ? sink[h] : -SMLA_INF;
  if (!empty) den += __expf(snk - M);
  for (int64_t d = tid; d < DV; d += kGenThreads) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < HW; w++) o += buf[w * DV + d];
    store_from_f32(out, rh * DV + d, out_dtype, empty ? __builtin_nanf("") : o / den);
  }
}

// Merge of the generic kernel's split states: one workgroup per (query row, head); the weights
// w_j = exp(m_j - M) go through LDS, then thread t sums columns t, t + 256, .. over the splits in
// order: O = sum w_j O_j / (sum w_j l_j + exp(sink - M)), NaN when no split saw a valid row.
constexpr int kGenMergeMax = 64;  // splits of the generic kernel at most
__global__ __launch_bounds__(256) void attn_generic_merge_kernel(const float* __restrict__ part, int nsplit,
                                                                 int64_t H, int64_t DV,
                                                                 const float* __restrict__ sink,
                                                                 void* __restrict__ out, int out_dtype) {
  __shared__ float w_s[kGenMergeMax];
  const int64_t rh = blockIdx.x;
  const int h = (int)(rh % H);
  const float* ml = part + rh * nsplit * 2;
  float M = -SMLA_INF;
  for (int j = 0; j < nsplit; j++) M = fmaxf(M, ml[2 * j]);
  const bool empty = !(M > -SMLA_INF);
  float L = 0.f;
  for (int j = 0; j < nsplit; j++) {
    const float w = ml[2 * j] > -SMLA_INF ? __expf(ml[2 * j] - M) : 0.f;
    L += w * ml[2 * j + 1];
    if (threadIdx.x == j) w_s[j] = w;
  }
  if (!empty && sink) L += __expf(sink[h] - M);
  __syncthreads();
  const float* ob = part + (int64_t)gridDim.x * nsplit * 2 + rh * nsplit * DV;
  for (int64_t d = threadIdx.x; d < DV; d += 256) {
    float o = 0.f;
    for (int j = 0; j < nsplit; j++) o = fmaf(w_s[j], ob[j * DV + d], o);
    store_from_f32(out, rh * DV + d, out_dtype, empty ? __builtin_nanf("") : o / L);
  }
}

template <int KT>
void launch_generic_kt(int64_t D, dim3 grid, size_t lds, hipStream_t st, const void* q, int q_dtype, RowSrc src,
                       const float* sink, const int32_t* idx, int64_t T, int64_t S, int64_t H, int64_t DV,
                       float scale, void* out, int out_dtype, float* part) {
  const int64_t nch = (D + 63) / 64;
  if (nch <= 4)
    hipLaunchKernelGGL((attn_generic_kernel<KT, 4, true>), grid, dim3(kGenThreads), lds, st, q, q_dtype, src, sink,
                       idx, T, S, H, D, DV, scale, out, out_dtype, part);
  else if (nch <= 9)
    hipLaunchKernelGGL((attn_generic_kernel<KT, 9, true>), grid, dim3(kGenThreads), lds, st, q, q_dtype, src, sink,
                       idx, T, S, H, D, DV, scale, out, out_dtype, part);
  else if (nch <= 16)
    hipLaunchKernelGGL((attn_generic_kernel<KT, 16, true>), grid, dim3(kGenThreads), lds, st, q, q_dtype, src, sink,
                       idx, T, S, H, D, DV, scale, out, out_dtype, part);
  else
    hipLaunchKernelGGL((attn_generic_kernel<KT, 16, false>), grid, dim3(kGenThreads), lds, st, q, q_dtype, src, sink,
                       idx, T, S, H, D, DV, scale, out, out_dtype, part);
}

// the generic kernel over B*S*H x nsplit workgroups (nsplit > 1: partial states into `part`);
// LDS: the query row and half the waves' partial outputs
int launch_generic(const void* q, int q_dtype, RowSrc src, int kv_dtype, const float* sink, const int32_t* idx,
                   int64_t T, int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out,
                   int out_dtype, int nsplit, float* part, hipStream_t st) {
  const size_t lds = (size_t)D * 4 + (size_t)(kGenWaves / 2) * DV * 4;
  if (lds > 64 * 1024 || B * S * H > 0xffffffffll) return SMLA_E_UNSUPPORTED;
  const dim3 grid((unsigned)(B * S * H), (unsigned)nsplit);
  switch (kv_dtype) {
    case SMLA_F32:
      launch_generic_kt<SMLA_F32>(D, grid, lds, st, q, q_dtype, src, sink, idx, T, S, H, DV, scale, out, out_dtype,
                                  part);
      break;
    case SMLA_BF16:
      launch_generic_kt<SMLA_BF16>(D, grid, lds, st, q, q_dtype, src, sink, idx, T, S, H, DV, scale, out, out_dtype,
                                   part);
      break;
    case SMLA_F16:
      launch_generic_kt<SMLA_F16>(D, grid, lds, st, q, q_dtype, src, sink, idx, T, S, H, DV, scale, out, out_dtype,
                                  part);
      break;
    default:
      launch_generic_kt<SMLA_FP8_E4M3>(D, grid, lds, st, q, q_dtype, src, sink, idx, T, S, H, DV, scale, out,
                                      out_dtype, part);
  }
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
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
  // DVS > 1: the row's columns are split over DVS workgroups, for row counts too small
  // to spread over the CUs otherwise
  constexpr int LW = BF16P ? (CPL + 1) / 2 : CPL;     // 32-bit words loaded per split
  constexpr int CHUNK = CH < 64 / LW ? CH : 64 / LW;  // splits in flight: at most 64 words per thread
  static_assert(CPL >= 1 && CPL <= 4 && DVS * NT * CPL == DV, "merge thread layout");
  static_assert(kMaxSplits % CHUNK == 0, "padded weights fit the table");
  __shared__ __align__(16) float m_s[kMaxSplits];
  __shared__ float l_s[kMaxSplits];
  __shared__ float red[2][WAVES];
  // every launch argument read in one round trip of scalar loads
  {
    const uint32_t gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    asm volatile("" ::"s"(gx), "s"(gy), "s"(gz), "s"(part), "s"(nsplit), "s"(BS), "s"(H), "s"(sink), "s"(out),
                 "s"(out_dtype));
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // grid (B*S*H, DVS): every head and column slice of query row bs on XCD bs mod 8 (when B*S is a
  // multiple of 8), the XCD whose L2 holds that row's partials from the split kernel
  int64_t bs, item;
  xcd_row_item(BS, (int64_t)H * DVS, bs, item);
  const int head = DVS == 1 ? (int)item : (int)((uint32_t)item % (uint32_t)H);
  const int64_t rh = bs * H + head;
  const int64_t rec0 = bs * nsplit * (int64_t)H + head;  // record of split 0; splits are H records apart
  const float* ml = part + rec0 * 2;
  const int dv0 = (DVS == 1 ? 0 : (int)((uint32_t)item / (uint32_t)H)) * (DV / DVS) + tid * CPL;
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

// Merge of bf16 partial states in MFMA fragment order (attn_decode_kernel's value waves write
// them from their accumulators): per (query row bs, split j, head group hg) a 64 KB block in which
// the 1 KB piece ((vw * 4 + mb) * 2 + h) holds, in lane l's 16 bytes, value columns
// 128 (vw >> 1) + 32 mb + 16 h + 8 (l >> 5) .. +7 of head 64 hg + 32 (vw & 1) + (l & 31).
// One workgroup of NW waves per (query row, head group, 1 KB piece): lane l reads source lane l's
// 16 bytes of the piece in every split (8 values of one head) and the (m, l) record of that head
// (the split kernel's [row][split][head] fp32 pairs).  Wave w takes the w-th of NW equal runs of
// the splits, CH at a time: the compiler requests the chunk's (m, l) records, forms the maximum
// and the weights, then requests the O pieces and folds each in as it lands (loads return in
// order); requesting the O pieces first measured 0.5 us slower at 23 splits, the small records
// then queueing behind 24 KB of O per wave.  A later chunk whose maximum exceeds M rescales the
// running sums first.  Loads past the end of a run read its last split again (weight 0; spreading them over
// other splits costs SGPR spills of the per-load offsets and measured slower).  With NW > 1 the
// waves' states meet in LDS and wave 0 combines them in wave order.  Per split the weight and the
// sums follow attn_merge_kernel's formula.  (Against 4-wave workgroups reading 4 bytes per lane
// with the records staged in LDS: equal at 23 splits, 44.7 -> 42.4 us on the 64-sequence fp8
// batch, whose 4 splits per row take CH = 8.  Two waves of 17 splits instead of one wave taking
// 32 then 2 on the one-sequence 16384-key decode step, 34 splits per row: 32.9 -> 29.7 us per
// step.)
template <int CH, int NW = 1>
__global__ __launch_bounds__(64 * NW) void attn_merge_frag_kernel(const float* __restrict__ part, int nsplit,
                                                                    int64_t BS, int H, int HG,
                                                                    const float* __restrict__ sink,
                                                                    void* __restrict__ out, int out_dtype) {
  {
    const uint32_t gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    asm volatile("" ::"s"(gx), "s"(gy), "s"(gz), "s"(part), "s"(nsplit), "s"(BS), "s"(H), "s"(HG), "s"(sink),
                 "s"(out), "s"(out_dtype));
  }
  const int lane = threadIdx.x & 63;
  const int wq = NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  int64_t bs, item;
  xcd_row_item(BS, (int64_t)HG * 64, bs, item);
  const int hg = (int)((uint32_t)item >> 6), piece = (int)((uint32_t)item & 63u);
  const int vw = piece >> 3, mb = (piece >> 1) & 3, h = piece & 1;
  const int hl = 32 * (vw & 1) + (lane & 31);  // head within the group
  const int head = 64 * hg + hl;
  const int dv0 = 128 * (vw >> 1) + 32 * mb + 16 * h + 8 * (lane >> 5);
  const uint8_t* ob = (const uint8_t*)(part + BS * H * nsplit * 2) + (bs * nsplit * (int64_t)HG + hg) * 65536 +
                      piece * 1024 + 16 * lane;  // split j: + j * HG * 64 KB
  const int64_t job = (int64_t)HG * 65536;
  const float* mlb = part + (bs * nsplit * (int64_t)H + min(head, H - 1)) * 2;  // split j: + j * H * 2
  // this wave's run of splits [jb, je)
  const int per = (nsplit + NW - 1) / NW;
  const int jb = wq * per, je = min(nsplit, jb + per);
  float M = -SMLA_INF, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; e++) acc[e] = 0.f;
  for (int j0 = jb; j0 < je; j0 += CH) {
    u32x4_t v[CH];
    f32x2_t ml[CH];
    // split read by load u (past the run: its last split again)
    auto src = [&](int u) -> int64_t { return min(j0 + u, je - 1); };
#pragma unroll
    for (int u = 0; u < CH; u++) v[u] = *(const u32x4_t*)(ob + src(u) * job);
#pragma unroll
    for (int u = 0; u < CH; u++) ml[u] = *(const f32x2_t*)(mlb + src(u) * H * 2);
    float mc = M;
#pragma unroll
    for (int u = 0; u < CH; u++) mc = fmaxf(mc, j0 + u < je ? ml[u][0] : -SMLA_INF);
    if (mc > M && M > -SMLA_INF) {  // a later chunk raised the maximum (only past CH splits)
      const float r = __expf(M - mc);
      L *= r;
#pragma unroll
      for (int e = 0; e < 8; e++) acc[e] *= r;
    }
    M = mc;
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const float m = j0 + u < je ? ml[u][0] : -SMLA_INF;
      const float w = m > -SMLA_INF ? __expf(m - M) : 0.f;
      L += w * ml[u][1];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        acc[2 * e] += w * __uint_as_float(v[u][e] << 16);
        acc[2 * e + 1] += w * __uint_as_float(v[u][e] & 0xffff0000u);
      }
    }
  }
  if constexpr (NW > 1) {
    // waves 1.. hand their (M, L, acc) to wave 0, which folds them in wave order
    __shared__ float xs[NW - 1][10][64];
    if (wq > 0) {
      xs[wq - 1][0][lane] = M;
      xs[wq - 1][1][lane] = L;
#pragma unroll
      for (int e = 0; e < 8; e++) xs[wq - 1][2 + e][lane] = acc[e];
    }
    __syncthreads();
    if (wq > 0) return;
#pragma unroll
    for (int w = 0; w < NW - 1; w++) {
      const float m2 = xs[w][0][lane];
      const float mn = fmaxf(M, m2);
      const float r1 = M > -SMLA_INF ? __expf(M - mn) : 0.f;
      const float r2 = m2 > -SMLA_INF ? __expf(m2 - mn) : 0.f;
      L = L * r1 + xs[w][1][lane] * r2;
#pragma unroll
      for (int e = 0; e < 8; e++) acc[e] = acc[e] * r1 + xs[w][2 + e][lane] * r2;
      M = mn;
    }
  }
  if (head >= H) return;
  const bool empty = !(M > -SMLA_INF);
  const float snk = sink ? sink[head] : -SMLA_INF;
  if (!empty) L += __expf(snk - M);
  const float inv = 1.0f / L;
  const int64_t o = (bs * H + head) * 512 + dv0;
  if (out_dtype == SMLA_BF16) {
    u32x4_t w4;
#pragma unroll
    for (int e = 0; e < 4; e++) w4[e] = empty ? 0x7fc07fc0u : pack_bf16x2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
    *(u32x4_t*)((uint16_t*)out + o) = w4;
  } else {
    const float nan = __builtin_nanf("");
    f32x4_t a, c;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      a[e] = empty ? nan : acc[e] * inv;
      c[e] = empty ? nan : acc[4 + e] * inv;
    }
    *(f32x4_t*)((float*)out + o) = a;
    *(f32x4_t*)((float*)out + o + 4) = c;
  }
}

// ---------------------------------------------------------------------------------------------
// Launch planning (shared by the workspace queries and the launcher).  A pure function of its
// arguments and the device's compute-unit count.
struct Plan {
  bool mfma;
  int rows_per_split;
  int nsplit;
  int hgroups;
};

// splits of the vector-ALU kernel: enough (row, head, split) workgroups for about one per compute
// unit, at least 32 list entries per split, at most kGenMergeMax
int generic_splits(int64_t B, int64_t S, int64_t H, int64_t T) {
  const int64_t rows = B * S * H, cus = smla_num_cus();
  int64_t ns = rows >= cus ? 1 : (cus + rows - 1) / rows;
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, T / 32));
  return (int)std::min<int64_t>(ns, kGenMergeMax);
}

Plan make_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t T, int q_dtype, int kv_dtype,
               int64_t rps_req) {
  Plan p{};
  p.mfma = q_dtype == SMLA_BF16 && (kv_dtype == SMLA_BF16 || kv_dtype == SMLA_FP8_E4M3) &&
           H % 16 == 0 && DV == 512 && (D == 576 || D == 512) && T > 0 && T < (1ll << 30);
  if (!p.mfma) {
    p.nsplit = generic_splits(B, S, H, T);
    return p;
  }
  p.hgroups = (int)((H + 63) / 64);
  const int64_t rows = B * S * p.hgroups;
  const int64_t tiles = (T + kTileRows - 1) / kTileRows;
  int64_t per;
  if (rps_req > 0) {
    per = (rps_req + kTileRows - 1) / kTileRows;
  } else {
    // tiles per split so that rows * nsplit ~ one workgroup per compute unit; a split's fixed costs
    // (its Q block, index table and partial record) outweigh one 32-row tile, and every split adds
    // a partial to merge: at least two tiles per split once the list has four
    const int64_t target = smla_num_cus();
    per = (tiles * rows + target - 1) / target;
    if (per < 2 && tiles >= 4) per = 2;
  }
  if (per < 1) per = 1;
  if ((tiles + per - 1) / per > kMaxSplits) per = (tiles + kMaxSplits - 1) / kMaxSplits;
  if (per > tiles) per = tiles;
  // the split kernel takes splits of up to kDecodeV6MaxRows rows (a 4-tile ring for splits of at
  // most 256 rows, a 3-tile ring with a larger index table beyond)
  if (per > smla_attn::kDecodeV6MaxRows / kTileRows) per = smla_attn::kDecodeV6MaxRows / kTileRows;
  p.rows_per_split = (int)(per * kTileRows);
  p.nsplit = (int)((tiles + per - 1) / per);
  if (p.nsplit > kMaxSplits) {  // beyond the merge kernel's capacity: generic kernel
    p.mfma = false;
    p.nsplit = generic_splits(B, S, H, T);
  }
  return p;
}

// bytes of split partial states for a plan.  The MFMA kernel: (m, l) fp32 per (query row, head,
// split), then the partial O: bf16 blocks of 64 heads x 512 in fragment order per (query row,
// split, head group) (bf16 output), or fp32 rows per (query row, split, head).  The vector-ALU
// kernel: (m, l) and DV fp32 values per (query row, head, split).
size_t plan_workspace(const Plan& p, int64_t B, int64_t S, int64_t H, int64_t DV, int out_dtype) {
  if (p.nsplit <= 1) return 0;
  if (!p.mfma)  // the vector-ALU kernel's split states: (m, l) then DV fp32 values per record
    return (size_t)(B * S * H) * (size_t)p.nsplit * (size_t)(2 + DV) * sizeof(float);
  const size_t recs = (size_t)(B * S) * (size_t)p.nsplit;
  const size_t ml = recs * (size_t)H * 2 * sizeof(float);
  if (out_dtype == SMLA_BF16) return ml + recs * (size_t)p.hgroups * 65536;
  return ml + recs * (size_t)H * (size_t)DV * 4;
}

// the row sources of batch entries b0.. (rows of row_bytes bytes; fp8 rows with D/64 scales each)
RowSrc rows_from(const RowSrc& s, int64_t b0, int64_t row_bytes, int64_t scales_per_row) {
  auto adv = [](const void* p, int64_t bytes) -> const void* {
    return p ? (const void*)((const uint8_t*)p + bytes) : nullptr;
  };
  RowSrc r = s;
  r.kv0 = adv(s.kv0, b0 * s.n0 * row_bytes);
  r.kv1 = adv(s.kv1, b0 * s.n1 * row_bytes);
  r.sc0 = (const float*)adv(s.sc0, b0 * s.n0 * scales_per_row * (int64_t)sizeof(float));
  r.sc1 = (const float*)adv(s.sc1, b0 * s.n1 * scales_per_row * (int64_t)sizeof(float));
  return r;
}

int launch_merge(const Plan& p, int64_t B, int64_t S, int64_t H, const float* sink, void* out, int out_dtype,
                 const void* ws, hipStream_t stream) {
  if (p.nsplit <= 1) return SMLA_OK;
  const bool part_bf16 = out_dtype == SMLA_BF16;
  if (part_bf16) {  // fragment-order partials: one workgroup per (query row, head group, 1 KB piece)
    // waves per piece: one run of at most 32 splits each, up to 4 (more splits: 4 waves, several
    // chunks); CH: the smallest of 8 / 16 / 24 / 32 that covers a wave's run
    const dim3 grid((unsigned)(B * S * p.hgroups * 64));
    const int nw = p.nsplit <= 32 ? 1 : p.nsplit <= 64 ? 2 : 4;
    const int run = (p.nsplit + nw - 1) / nw;
    const int ch = run <= 8 ? 8 : run <= 16 ? 16 : run <= 24 ? 24 : 32;
#define SMLA_MERGE_FRAG(C, W)                                                                                      \
  hipLaunchKernelGGL((attn_merge_frag_kernel<C, W>), grid, dim3(64 * W), 0, stream, (const float*)ws, p.nsplit, \
                     B * S, (int)H, p.hgroups, sink, out, out_dtype)
#define SMLA_MERGE_FRAG_CH(W)        \
  if (ch == 8) SMLA_MERGE_FRAG(8, W); \
  else if (ch == 16) SMLA_MERGE_FRAG(16, W); \
  else if (ch == 24) SMLA_MERGE_FRAG(24, W); \
  else SMLA_MERGE_FRAG(32, W)
    if (nw == 1) {
      SMLA_MERGE_FRAG_CH(1);
    } else if (nw == 2) {
      SMLA_MERGE_FRAG_CH(2);
    } else {
      SMLA_MERGE_FRAG_CH(4);
    }
#undef SMLA_MERGE_FRAG_CH
#undef SMLA_MERGE_FRAG
    SMLA_HIP_CHECK_LAUNCH();
    return SMLA_OK;
  }
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

// host-side argument checks shared by the attention entry points
int check_attn_args(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1, int64_t n1,
                    int kv_dtype, const float* kv0_scale, const float* kv1_scale, const int32_t* topk_idxs,
                    int64_t T, int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, const void* out,
                    int out_dtype) {
  if (!q || !kv0 || !topk_idxs || !out) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0 || DV <= 0 || DV > D || T <= 0 || n0 < 0 || n1 < 0 || n0 + n1 <= 0)
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
  return SMLA_OK;
}

}  // namespace

// The launches of one attention call under plan p (phases: SMLA_ATTN_SPLIT and / or
// SMLA_ATTN_MERGE), with `ws` holding at least plan_workspace(p, ...) bytes.  Arguments are
// checked by the caller.  Calls of more query rows than one grid holds run chunk by chunk
// (for_row_chunks), each chunk's partial states in its own stretch of the workspace, so a merge
// alone finds what a split alone left.
static int attn_launch(const Plan& p, int phases, const void* q, int q_dtype, RowSrc src, int kv_dtype,
                     const float* attn_sink, const int32_t* topk_idxs, int64_t T, int64_t B, int64_t S, int64_t H,
                     int64_t D, int64_t DV, float scale, void* out, int out_dtype, void* ws, hipStream_t st,
                     smla_attn::SelectRows sr = smla_attn::SelectRows{}) {
  if (!p.mfma) {
    if (phases & SMLA_ATTN_SPLIT) {
      const int rc = launch_generic(q, q_dtype, src, kv_dtype, attn_sink, topk_idxs, T, B, S, H, D, DV, scale, out,
                                    out_dtype, p.nsplit, (float*)ws, st);
      if (rc != SMLA_OK) return rc;
    }
    if ((phases & SMLA_ATTN_MERGE) && p.nsplit > 1) {
      hipLaunchKernelGGL(attn_generic_merge_kernel, dim3((unsigned)(B * S * H)), dim3(256), 0, st, (const float*)ws,
                         p.nsplit, H, DV, attn_sink, out, out_dtype);
      SMLA_HIP_CHECK_LAUNCH();
    }
    return SMLA_OK;
  }
  const bool fp8 = kv_dtype == SMLA_FP8_E4M3;
  const int64_t row_bytes = fp8 ? D : 2 * D;
  const int64_t out_row = H * DV * (out_dtype == SMLA_BF16 ? 2 : 4);
  return for_row_chunks(B, S, [&](int64_t b0, int64_t s0, int64_t nb, int64_t ns) -> int {
    const int64_t r0 = b0 * S + s0;  // first query row of the chunk
    const void* cq = (const uint16_t*)q + r0 * H * D;
    const RowSrc csrc = rows_from(src, b0, row_bytes, fp8 ? D / 64 : 0);
    const int32_t* cidx = topk_idxs ? topk_idxs + r0 * T : nullptr;
    void* cout = (uint8_t*)out + r0 * out_row;
    void* cws = ws ? (uint8_t*)ws + plan_workspace(p, 1, r0, H, DV, out_dtype) : nullptr;
    smla_attn::SelectRows csr = sr;
    if (sr.enabled) {
      csr.scores = sr.scores + r0 * (int64_t)sr.N;
      csr.nvis = sr.nvis ? sr.nvis + r0 : nullptr;
      csr.pos = sr.pos + r0;
    }
    if (phases & SMLA_ATTN_SPLIT) {
      const int rc = smla_attn::launch_decode_v6((int)D, fp8, p.nsplit, p.rows_per_split, cq, csrc, attn_sink, cidx, T,
                                                 nb, ns, H, scale, cout, out_dtype, (float*)cws, st,
                                                 smla_attn::ImplicitRows{}, csr);
      if (rc != SMLA_OK) return rc;
    }
    if (phases & SMLA_ATTN_MERGE) return launch_merge(p, nb, ns, H, attn_sink, cout, out_dtype, cws, st);
    return SMLA_OK;
  });
}

// the checks and plan of one call, then its launches on `ws` (ws_bytes of it)
static int attn_call(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1, int64_t n1,
                     int kv_dtype, const float* kv0_scale, const float* kv1_scale, const float* attn_sink,
                     const int32_t* topk_idxs, int64_t T, int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV,
                     float scale, void* out, int out_dtype, int64_t rows_per_split, int phases, void* ws,
                     size_t ws_bytes, void* stream) {
  int rc = check_attn_args(q, q_dtype, kv0, n0, kv1, n1, kv_dtype, kv0_scale, kv1_scale, topk_idxs, T, B, S, H, D,
                           DV, out, out_dtype);
  if (rc != SMLA_OK) return rc;
  if (rows_per_split < 0 || rows_per_split % kTileRows != 0 || phases < 1 || phases > 3) return SMLA_E_RANGE;
  const RowSrc src{kv0, kv1, kv_dtype == SMLA_FP8_E4M3 ? kv0_scale : nullptr,
                   kv_dtype == SMLA_FP8_E4M3 ? kv1_scale : nullptr, n0, n1};
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, rows_per_split);
  const size_t need = plan_workspace(p, B, S, H, DV, out_dtype);
  if (need > 0 && (!ws || ws_bytes < need)) return SMLA_E_WORKSPACE;
  return attn_launch(p, phases, q, q_dtype, src, kv_dtype, attn_sink, topk_idxs, T, B, S, H, D, DV, scale, out,
                          out_dtype, ws, (hipStream_t)stream);
}

// Prompt attention with the row sets of oracle/decode_engine.py:107-117 computed in the kernel:
// one workgroup per (query, 64-head group), lists as ImplicitRows describes, queries longest first.
// With no index table in LDS the list length is not bounded by a table.
extern "C" int smla_prefill_attn(const void* q, int q_dtype, const void* kv_raw, int64_t n_raw, const void* kv_comp,
                                 int64_t n_comp, int kv_dtype, const float* attn_sink, int64_t q_pos0,
                                 int64_t window, int64_t ratio, int64_t B, int64_t S, int64_t H, int64_t D,
                                 int64_t DV, float scale, void* out, int out_dtype, void* stream) {
  if (!q || !kv_raw || !out || (ratio > 0 && n_comp > 0 && !kv_comp)) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || H <= 0 || n_raw <= 0 || n_comp < 0) return SMLA_E_SHAPE;
  if (q_dtype != SMLA_BF16 || kv_dtype != SMLA_BF16 || (out_dtype != SMLA_BF16 && out_dtype != SMLA_F32))
    return SMLA_E_DTYPE;
  if ((D != 576 && D != 512) || DV != 512 || H % 16 != 0) return SMLA_E_UNSUPPORTED;
  if (window <= 0 || ratio < 0 || q_pos0 < 0 || q_pos0 + S > n_raw) return SMLA_E_RANGE;
  if (((uintptr_t)q & 15) || ((uintptr_t)kv_raw & 15) || ((uintptr_t)kv_comp & 15) || ((uintptr_t)out & 15))
    return SMLA_E_UNSUPPORTED;
  const int64_t nc_max = ratio > 0 ? std::min((q_pos0 + S) / ratio, n_comp) : 0;
  const int64_t T = window + nc_max;
  const int64_t rows = (T + kTileRows - 1) / kTileRows * kTileRows;
  if (rows > (1 << 24) || window > (1 << 24)) return SMLA_E_UNSUPPORTED;
  const smla_attn::RowSrc src{kv_raw, nc_max > 0 ? kv_comp : nullptr, nullptr, nullptr, n_raw,
                              nc_max > 0 ? n_comp : 0};
  const int64_t out_row = H * DV * (out_dtype == SMLA_BF16 ? 2 : 4);
  // more query rows than one grid holds: launches over row chunks, the positions of a piece of a
  // sequence starting at q_pos0 + s0
  return for_row_chunks(B, S, [&](int64_t b0, int64_t s0, int64_t nb, int64_t ns) -> int {
    const int64_t r0 = b0 * S + s0;
    const smla_attn::ImplicitRows ir{q_pos0 + s0, (int)window, (int)ratio, 1};
    return smla_attn::launch_decode_v6((int)D, false, 1, (int)rows, (const uint16_t*)q + r0 * H * D,
                                       rows_from(src, b0, 2 * D, 0), attn_sink, nullptr, T, nb, ns, H, scale,
                                       (uint8_t*)out + r0 * out_row, out_dtype, nullptr, (hipStream_t)stream, ir);
  });
}

// Decode attention over the engine's index build (window ids of pos, then the top-k of the
// indexer scores: the list smla_select_decode writes), with the selection run by the attention
// workgroups themselves when the shape allows (bf16 rows, the short-split plan, N <= 18432): the
// list never goes through memory and the selection launch disappears.  Other shapes build the
// list in the workspace and run the list path.  Output bit-identical to smla_select_decode
// followed by smla_sparse_attn with the default plan.
namespace {
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
bool select_in_kernel(const Plan& p, int kv_dtype, int64_t N) {
  return p.mfma && kv_dtype == SMLA_BF16 && p.rows_per_split <= smla_attn::kDecodeV6ShortRows &&
         smla_attn::select_per(N) != 0;
}
}  // namespace

extern "C" size_t smla_decode_attn_workspace(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t window,
                                             int64_t k, int q_dtype, int kv_dtype, int out_dtype) {
  if (B <= 0 || S <= 0 || H <= 0 || window < 0 || k <= 0) return 0;
  const int64_t T = window + k;
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, 0);
  // the split partials, then room for the lists of the path that builds them in memory
  return align256(plan_workspace(p, B, S, H, DV, out_dtype)) + (size_t)(B * S * T) * sizeof(int32_t);
}

extern "C" int smla_decode_attn(const void* q, int q_dtype, const void* kv_raw, int64_t n_raw, const void* kv_comp,
                                int64_t n_comp, int kv_dtype, const float* attn_sink, const float* scores, int64_t N,
                                const int32_t* nvis, const int32_t* pos, int64_t window, int64_t k, int64_t B,
                                int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out, int out_dtype,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (!scores || !pos) return SMLA_E_NULL;
  if (N <= 0 || window < 0 || k <= 0 || window + k > 0x7fffffff || N > 0x7fffffff) return SMLA_E_SHAPE;
  if (window > n_raw) return SMLA_E_SHAPE;  // the raw ring must hold the window
  const int64_t T = window + k;
  // the list arguments are checked with a stand-in for the list pointer
  int rc = check_attn_args(q, q_dtype, kv_raw, n_raw, kv_comp, n_comp, kv_dtype, nullptr, nullptr, (const int32_t*)pos,
                           T, B, S, H, D, DV, out, out_dtype);
  if (rc != SMLA_OK) return rc;
  if (kv_dtype == SMLA_FP8_E4M3) return SMLA_E_DTYPE;  // fp8 rows carry scale arrays: the list entry takes them
  const size_t need = smla_decode_attn_workspace(B, S, H, D, DV, window, k, q_dtype, kv_dtype, out_dtype);
  if (!workspace || workspace_bytes < need) return SMLA_E_WORKSPACE;
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, 0);
  hipStream_t st = (hipStream_t)stream;
  const RowSrc src{kv_raw, kv_comp, nullptr, nullptr, n_raw, n_comp};
  if (select_in_kernel(p, kv_dtype, N)) {
    const smla_attn::SelectRows sr{scores, nvis, pos, (int)N, (int)window, (int)k, 1};
    return attn_launch(p, SMLA_ATTN_SPLIT | SMLA_ATTN_MERGE, q, q_dtype, src, kv_dtype, attn_sink, nullptr, T, B, S,
                       H, D, DV, scale, out, out_dtype, workspace, st, sr);
  }
  int32_t* ids = (int32_t*)((uint8_t*)workspace + align256(plan_workspace(p, B, S, H, DV, out_dtype)));
  rc = smla_select_decode(scores, B * S, N, nvis, k, pos, window, ids, T, (int32_t)n_raw, stream);
  if (rc != SMLA_OK) return rc;
  return attn_launch(p, SMLA_ATTN_SPLIT | SMLA_ATTN_MERGE, q, q_dtype, src, kv_dtype, attn_sink, ids, T, B, S, H, D,
                     DV, scale, out, out_dtype, workspace, st);
}

extern "C" size_t smla_sparse_attn_workspace(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV,
                                             int64_t T, int q_dtype, int kv_dtype) {
  // the larger of the two partial layouts, so it suffices for either output type
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, 0);
  return std::max(plan_workspace(p, B, S, H, DV, SMLA_F32), plan_workspace(p, B, S, H, DV, SMLA_BF16));
}

extern "C" size_t smla_sparse_attn_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t T,
                                        int q_dtype, int kv_dtype, int out_dtype, int64_t rows_per_split,
                                        int64_t* nsplit, int64_t* rows_per_split_out) {
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, rows_per_split > 0 ? rows_per_split : 0);
  if (nsplit) *nsplit = p.mfma ? p.nsplit : 0;
  if (rows_per_split_out) *rows_per_split_out = p.mfma ? p.rows_per_split : 0;
  return plan_workspace(p, B, S, H, DV, out_dtype);
}

extern "C" int smla_sparse_attn(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1,
                                int64_t n1, int kv_dtype, const float* kv0_scale, const float* kv1_scale,
                                const float* attn_sink, const int32_t* topk_idxs, int64_t T, int64_t B,
                                int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out,
                                int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return attn_call(q, q_dtype, kv0, n0, kv1, n1, kv_dtype, kv0_scale, kv1_scale, attn_sink, topk_idxs, T, B, S, H,
                   D, DV, scale, out, out_dtype, 0, SMLA_ATTN_SPLIT | SMLA_ATTN_MERGE, workspace, workspace_bytes,
                   stream);
}

extern "C" int smla_sparse_attn_ex(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1,
                                   int64_t n1, int kv_dtype, const float* kv0_scale, const float* kv1_scale,
                                   const float* attn_sink, const int32_t* topk_idxs, int64_t T, int64_t B,
                                   int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out,
                                   int out_dtype, int64_t rows_per_split, int phases, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  return attn_call(q, q_dtype, kv0, n0, kv1, n1, kv_dtype, kv0_scale, kv1_scale, attn_sink, topk_idxs, T, B, S, H,
                   D, DV, scale, out, out_dtype, rows_per_split, phases, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------------------------
// Allocation-free variant: the split partial states live in `scratch`, a buffer of
// SMLA_NOALLOC_SCRATCH_BYTES that every device the library runs on holds until the process ends.
// In host code `scratch` names a host-side stand-in, so its device address is taken once per
// device (hipGetSymbolAddress, with that device current) and only that address reaches kernels.
namespace {
static __device__ __align__(256) uint8_t scratch[SMLA_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// device address of the current device's `scratch` (resolved on the first call on that device)
int scratch_on_current_device(void** addr) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return SMLA_E_UNSUPPORTED;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (!p) {
      if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return (int)e;
      if (!p) return SMLA_E_UNSUPPORTED;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return SMLA_OK;
}
}  // namespace

extern "C" int smla_sparse_attn_noalloc(const void* q, int q_dtype, const void* kv0, int64_t n0, const void* kv1,
                                        int64_t n1, int kv_dtype, const float* kv0_scale, const float* kv1_scale,
                                        const float* attn_sink, const int32_t* topk_idxs, int64_t T, int64_t B,
                                        int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out,
                                        int out_dtype, void* stream) {
  int rc = check_attn_args(q, q_dtype, kv0, n0, kv1, n1, kv_dtype, kv0_scale, kv1_scale, topk_idxs, T, B, S, H, D,
                           DV, out, out_dtype);
  if (rc != SMLA_OK) return rc;
  // the default plan's partial states must fit the buffer (checked before anything runs)
  const Plan p = make_plan(B, S, H, D, DV, T, q_dtype, kv_dtype, 0);
  if (plan_workspace(p, B, S, H, DV, out_dtype) > SMLA_NOALLOC_SCRATCH_BYTES) return SMLA_E_WORKSPACE;
  void* ws = nullptr;
  rc = scratch_on_current_device(&ws);
  if (rc != SMLA_OK) return rc;
  return attn_call(q, q_dtype, kv0, n0, kv1, n1, kv_dtype, kv0_scale, kv1_scale, attn_sink, topk_idxs, T, B, S, H,
                   D, DV, scale, out, out_dtype, 0, SMLA_ATTN_SPLIT | SMLA_ATTN_MERGE, ws, SMLA_NOALLOC_SCRATCH_BYTES,
                   stream);
}
