// Top-k selection and index construction.
//
// smla_topk: per row, rank the first nvis scores by (score desc, index asc) with -0 == +0, keep
// min(k, nvis), emit ascending ids (+ id_offset), -1 padded to k.  One workgroup of 1024 threads
// per row; each thread owns a contiguous run of PER keys in registers.
//   1. key = order-preserving uint32 with larger score -> smaller key;
//   2. 4 radix passes (8-bit digits, per-wave LDS histograms) find the k-th smallest key K and the
//      number `need` of entries equal to K that still fit;
//   3. two block-wide exclusive scans in index order: rank the K-ties (lowest index first), then
//      place every selected id at its ascending position.
// Bit-exact by construction: only comparisons and counts.  When nvis <= k every visible id is
// taken (oracle/decode_engine.py:112-114, "all causally visible compressed rows").
//
// smla_window_topk_idxs mirrors ref_torch/sparse_attn.py:9-20; smla_decode_window_idxs builds the
// engine's decode window oracle/decode_engine.py:110-111 over an un-ringed raw cache.
#include "smla_internal.h"

namespace {

constexpr int kTopkThreads = 1024;
constexpr int kWaves = kTopkThreads / 64;

__device__ inline uint32_t desc_key(float f) {
  if (f == 0.f) f = 0.f;  // -0 -> +0
  uint32_t u = __float_as_uint(f);
  uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}

// exclusive scan of one value per thread over the block; returns the exclusive prefix and the
// block total.  `tmp` holds kWaves + 1 ints.
__device__ inline int block_excl_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int t = lane < kWaves ? tmp[lane] : 0;
    int s = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int y = __shfl_up(s, o, 64);
      if (lane >= o) s += y;
    }
    if (lane < kWaves) tmp[lane] = s - t;  // exclusive wave offsets
    if (lane == kWaves - 1) tmp[kWaves] = s;
  }
  __syncthreads();
  int res = tmp[wave] + x - v;
  *total = tmp[kWaves];
  __syncthreads();
  return res;
}

template <int PER>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores, int64_t N,
                                                            const int32_t* __restrict__ nvis, int k,
                                                            int32_t* __restrict__ out, int64_t out_stride,
                                                            int32_t id_offset) {
  __shared__ int hist[kWaves][256];
  __shared__ int tmp[kWaves + 1];
  __shared__ int sel_digit, sel_before;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t r = blockIdx.x;
  int64_t nv = nvis ? (int64_t)nvis[r] : N;
  if (nv > N) nv = N;
  if (nv < 0) nv = 0;
  const float* sr = scores + r * N;
  int32_t* orow = out + r * out_stride;
  const int take = (int)(nv < k ? nv : k);

  const int64_t base = (int64_t)tid * PER;
  if (nv <= k) {
    // take every visible id, already ascending
    for (int64_t j = tid; j < k; j += kTopkThreads) orow[j] = j < nv ? (int32_t)j + id_offset : -1;
    return;
  }
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    int64_t n = base + j;
    key[j] = n < nv ? desc_key(sr[n]) : 0xffffffffu;
  }
  // ---- radix select for the k-th smallest key among visible entries
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += 64) hist[wave][i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; j++) {
      int64_t n = base + j;
      if (n < nv && (key[j] & pmask) == prefix) atomicAdd(&hist[wave][(key[j] >> shift) & 255u], 1);
    }
    __syncthreads();
    if (wave == 0) {
      // bins lane*4 .. lane*4+3
      int c[4];
      int tot = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int s = 0;
        for (int w = 0; w < kWaves; w++) s += hist[w][lane * 4 + i];
        c[i] = s;
        tot += s;
      }
      int incl = tot;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      int before = incl - tot;
      // the digit where the cumulative count first reaches `remaining`
      if (before < remaining && remaining <= incl) {
        int cum = before;
        for (int i = 0; i < 4; i++) {
          if (remaining <= cum + c[i]) {
            sel_digit = lane * 4 + i;
            sel_before = cum;
            break;
          }
          cum += c[i];
        }
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sel_digit << shift;
    pmask |= 255u << shift;
    remaining -= sel_before;
    __syncthreads();
  }
  const uint32_t K = prefix;
  const int need = remaining;  // entries equal to K to take, lowest index first
  // ---- rank ties in index order
  int nt = 0;
#pragma unroll
  for (int j = 0; j < PER; j++) nt += (base + j < nv && key[j] == K);
  int tot_ties;
  int tie_rank = block_excl_scan(nt, tmp, &tot_ties);
  int nsel = 0;
  {
    int tr = tie_rank;
#pragma unroll
    for (int j = 0; j < PER; j++) {
      bool vis = base + j < nv;
      bool s = vis && (key[j] < K || (key[j] == K && tr < need));
      if (vis && key[j] == K) tr++;
      nsel += s;
    }
  }
  int tot_sel;
  int pos = block_excl_scan(nsel, tmp, &tot_sel);
  {
    int tr = tie_rank;
#pragma unroll
    for (int j = 0; j < PER; j++) {
      bool vis = base + j < nv;
      bool s = vis && (key[j] < K || (key[j] == K && tr < need));
      if (vis && key[j] == K) tr++;
      if (s) orow[pos++] = (int32_t)(base + j) + id_offset;
    }
  }
  for (int64_t j = take + tid; j < k; j += kTopkThreads) orow[j] = -1;
}

__global__ void window_idx_kernel(int64_t w, int64_t seqlen, int64_t start_pos, int64_t cols, int64_t total_per_b,
                                  int64_t bsz, int32_t* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total_per_b * bsz) return;
  int64_t e = i % total_per_b;
  int32_t v;
  if (start_pos >= w - 1) {
    int64_t p = start_pos % w;
    v = (int32_t)((p + 1 + e) % w);
  } else if (start_pos > 0) {
    v = e <= start_pos ? (int32_t)e : -1;
  } else {
    int64_t row = e / cols, j = e % cols;
    int64_t lo = row - w + 1;
    if (lo < 0) lo = 0;
    int64_t m = lo + j;
    v = m > row ? -1 : (int32_t)m;
  }
  (void)seqlen;
  out[i] = v;
}

__global__ void decode_window_kernel(const int32_t* __restrict__ pos, int64_t R, int64_t w, int32_t* __restrict__ out,
                                     int64_t out_stride) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * w) return;
  int64_t r = i / w, j = i % w;
  int64_t v = (int64_t)pos[r] - w + 1 + j;
  out[r * out_stride + j] = v < 0 ? -1 : (int32_t)v;
}

}  // namespace

extern "C" int smla_topk(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, void* stream) {
  if (!scores || !out) return SMLA_E_NULL;
  if (R <= 0 || N <= 0 || k <= 0 || out_stride < k) return SMLA_E_SHAPE;
  if (R > 0x7fffffff || k > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  int64_t per = (N + kTopkThreads - 1) / kTopkThreads;
  dim3 grid((unsigned)R), blk(kTopkThreads);
#define SMLA_TOPK_CASE(P)                                                                          \
  if (per <= P) {                                                                                  \
    hipLaunchKernelGGL(topk_kernel<P>, grid, blk, 0, st, scores, N, nvis, (int)k, out, out_stride, id_offset); \
    SMLA_HIP_CHECK_LAUNCH();                                                                       \
    return SMLA_OK;                                                                                \
  }
  SMLA_TOPK_CASE(2)
  SMLA_TOPK_CASE(4)
  SMLA_TOPK_CASE(8)
  SMLA_TOPK_CASE(16)
  SMLA_TOPK_CASE(32)
  SMLA_TOPK_CASE(64)
#undef SMLA_TOPK_CASE
  return SMLA_E_UNSUPPORTED;  // N > 65536
}

extern "C" int smla_window_topk_idxs(int64_t window_size, int64_t bsz, int64_t seqlen, int64_t start_pos,
                                     int32_t* out, void* stream) {
  if (!out) return SMLA_E_NULL;
  if (window_size <= 0 || bsz <= 0 || seqlen <= 0 || start_pos < 0) return SMLA_E_SHAPE;
  int64_t cols = seqlen < window_size ? seqlen : window_size;
  int64_t per_b = start_pos > 0 ? window_size : seqlen * cols;
  int64_t total = per_b * bsz;
  if (total > (1ll << 31)) return SMLA_E_UNSUPPORTED;
  hipLaunchKernelGGL(window_idx_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     window_size, seqlen, start_pos, cols, per_b, bsz, out);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

extern "C" int smla_decode_window_idxs(const int32_t* pos, int64_t R, int64_t window, int32_t* out, int64_t out_stride,
                                       void* stream) {
  if (!pos || !out) return SMLA_E_NULL;
  if (R <= 0 || window <= 0 || out_stride < window) return SMLA_E_SHAPE;
  int64_t total = R * window;
  if (total > (1ll << 31)) return SMLA_E_UNSUPPORTED;
  hipLaunchKernelGGL(decode_window_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     pos, R, window, out, out_stride);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}
