// Top-k selection and index construction.
//
// smla_topk: per row, rank the first nvis scores by (score desc, index asc) with -0 == +0, keep
// min(k, nvis), emit ascending ids (+ id_offset), -1 padded to k.  One workgroup of 1024 threads
// per row; each thread owns a contiguous run of PER keys in registers (key = order-preserving
// uint32, larger score -> smaller key).  The k-th best entry (Kt, It) is found by a bucket select
// (monotone value buckets, exact ranking of the boundary bucket) or, for degenerate spreads, by
// 4 radix passes plus a tie rank; a block-wide scan in index order then places every selected id
// at its ascending position.  Bit-exact by construction: only comparisons and counts.  When
// nvis <= k every visible id is taken (oracle/decode_engine.py:112-114, "all causally visible
// compressed rows").  smla_select_decode also writes the decode window ids in front (one launch
// for the engine's whole index build, oracle/decode_engine.py:110-114).
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
  const int x = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const int t = lane < kWaves ? tmp[lane] : 0;
    const int s = wave_incl_scan(t);
    if (lane < kWaves) tmp[lane] = s - t;  // exclusive wave offsets
    if (lane == kWaves - 1) tmp[kWaves] = s;
  }
  __syncthreads();
  const int res = tmp[wave] + x - v;
  *total = tmp[kWaves];
  __syncthreads();
  return res;
}

constexpr int kBuckets = 2048;
constexpr int kMaxCand = 256;

// inverse of desc_key (the score with -0 folded to +0)
__device__ inline float key_score(uint32_t key) {
  const uint32_t asc = ~key;
  return __uint_as_float((asc & 0x80000000u) ? (asc ^ 0x80000000u) : ~asc);
}

// monotone bucket of a finite score: 0 holds the largest scores
__device__ inline int bucket_of(uint32_t key, float lmax, float bscale) {
  int bb = (int)((lmax - key_score(key)) * bscale);
  return bb < 0 ? 0 : (bb >= kBuckets ? kBuckets - 1 : bb);
}

// Row selection.  Produces the threshold pair (Kt, It) of the k-th best entry in the order
// (key asc == score desc, index asc); entry n is selected iff key < Kt or (key == Kt && n <= It).
//  * fast path: monotone buckets of (max - s) * 2048 / (max - min); the bucket holding the k-th
//    entry is found from a histogram + scan, and its (few) candidates are ranked exactly;
//  * fallback (degenerate spreads, > 256 candidates in the boundary bucket): 4 radix passes of 8
//    bits over the keys, then the tie rank among entries equal to the k-th key.
// Output: window ids (optional), then the selected ids ascending (+ id_offset), then -1.
template <int PER>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores, int64_t N,
                                                            const int32_t* __restrict__ nvis, int k,
                                                            int32_t* __restrict__ out, int64_t out_stride,
                                                            int32_t id_offset, const int32_t* __restrict__ wpos,
                                                            int window) {
  __shared__ int hist[kWaves][256];
  __shared__ int bhist[kBuckets];
  __shared__ int tmp[kWaves + 1];
  __shared__ float redf[2 * kWaves];
  __shared__ uint32_t cand_key[kMaxCand];
  __shared__ int cand_idx[kMaxCand];
  __shared__ int s_int[4];
  __shared__ int s_nan[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t r = blockIdx.x;
  int64_t nv = nvis ? (int64_t)nvis[r] : N;
  if (nv > N) nv = N;
  if (nv < 0) nv = 0;
  const float* sr = scores + r * N;
  int32_t* orow = out + r * out_stride;
  if (wpos) {
    const int64_t p = wpos[r];
    for (int j = tid; j < window; j += kTopkThreads) {
      const int64_t v = p - window + 1 + j;
      orow[j] = v < 0 ? -1 : (int32_t)v;
    }
    orow += window;
  }
  const int take = (int)(nv < k ? nv : k);

  const int64_t base = (int64_t)tid * PER;
  if (nv <= k) {
    for (int64_t j = tid; j < k; j += kTopkThreads) orow[j] = j < nv ? (int32_t)j + id_offset : -1;
    return;
  }
  uint32_t key[PER];
  float lmin = SMLA_INF, lmax = -SMLA_INF;
  bool nan_seen = false;
  // this thread's PER contiguous scores: 16-byte loads when the run lies inside the row and is
  // 16-byte aligned (rows of N floats: N % 4 == 0), element loads otherwise
  float fv[PER];
  if (PER % 4 == 0 && (N & 3) == 0 && base + PER <= N) {
#pragma unroll
    for (int j = 0; j < PER; j += 4) {
      const f32x4_t v4 = *(const f32x4_t*)(sr + base + j);
      fv[j] = v4[0];
      fv[j + 1] = v4[1];
      fv[j + 2] = v4[2];
      fv[j + 3] = v4[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < PER; j++) fv[j] = base + j < N ? sr[base + j] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int64_t n = base + j;
    const float f = fv[j];
    key[j] = n < nv ? desc_key(f) : 0xffffffffu;
    if (n < nv) {
      lmin = fminf(lmin, f);
      lmax = fmaxf(lmax, f);
      nan_seen |= f != f;
    }
  }
  // ---- row min / max (and whether a NaN is visible)
  {
    const float a = wave_min_dpp(lmin), bmx = wave_max_dpp(lmax);
    const bool wnan = __builtin_amdgcn_ballot_w64(nan_seen) != 0;
    if (lane == 0) {
      redf[wave] = a;
      redf[kWaves + wave] = bmx;
      s_nan[wave] = wnan;
    }
    for (int i = tid; i < kBuckets; i += kTopkThreads) bhist[i] = 0;
    __syncthreads();
    // every wave reduces the kWaves per-wave results itself (one LDS read per lane)
    const int wl = lane < kWaves ? lane : 0;
    lmin = wave_min_dpp(redf[wl]);
    lmax = wave_max_dpp(redf[kWaves + wl]);
    nan_seen = __builtin_amdgcn_ballot_w64(lane < kWaves && s_nan[wl] != 0) != 0;
  }
  uint32_t Kt = 0;
  int It = -1;
  bool done = false;
  if (lmax == lmin && !nan_seen) {
    // every visible score equal: the k lowest indices
    Kt = desc_key(lmax);
    It = k - 1;
    done = true;
  }
  const float bscale = (float)kBuckets / (lmax - lmin);
  if (!done && !nan_seen && bscale < SMLA_INF && bscale > 0.f && lmin > -SMLA_INF && lmax < SMLA_INF) {
    // ---- bucket histogram (bucket 0 holds the largest scores)
#pragma unroll
    for (int j = 0; j < PER; j++)
      if (base + j < nv) atomicAdd(&bhist[bucket_of(key[j], lmax, bscale)], 1);
    __syncthreads();
    // thread t owns buckets 2t, 2t+1
    const int c0 = bhist[2 * tid], c1 = bhist[2 * tid + 1];
    int tot;
    const int before = block_excl_scan(c0 + c1, tmp, &tot);
    if (tid == 0) s_int[3] = 0;  // candidate counter
    if (before < k && k <= before + c0) {
      s_int[0] = 2 * tid;
      s_int[1] = k - before;
    } else if (before + c0 < k && k <= before + c0 + c1) {
      s_int[0] = 2 * tid + 1;
      s_int[1] = k - before - c0;
    }
    __syncthreads();
    const int bb = s_int[0], need = s_int[1];
    const int cb = bhist[bb];
    if (cb <= kMaxCand) {
      // gather the boundary bucket's entries and rank them exactly
      // candidates of the boundary bucket: per-thread count, wave offsets by scan, one LDS
      // atomic per wave
      int mine = 0;
#pragma unroll
      for (int j = 0; j < PER; j++) mine += (base + j < nv && bucket_of(key[j], lmax, bscale) == bb);
      const int incl = wave_incl_scan(mine);
      int wbase = 0;
      if (lane == 63 && incl > 0) wbase = atomicAdd(&s_int[3], incl);
      wbase = __builtin_amdgcn_readlane(wbase, 63);
      int slot = wbase + incl - mine;
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (base + j < nv && bucket_of(key[j], lmax, bscale) == bb) {
          if (slot < kMaxCand) {
            cand_key[slot] = key[j];
            cand_idx[slot] = (int)(base + j);
          }
          slot++;
        }
      }
      __syncthreads();
      if (tid < cb) {
        const uint32_t kk = cand_key[tid];
        const int ii = cand_idx[tid];
        int rank = 0;
#pragma unroll 4
        for (int j = 0; j < cb; j++) {
          const uint32_t k2 = cand_key[j];
          rank += (k2 < kk) || (k2 == kk && cand_idx[j] < ii);
        }
        if (rank == need - 1) {
          s_int[0] = (int)kk;
          s_int[1] = ii;
        }
      }
      __syncthreads();
      Kt = (uint32_t)s_int[0];
      It = s_int[1];
      done = true;
    }
    __syncthreads();
  }
  if (!done) {
    // ---- radix select over the 32-bit keys
    uint32_t prefix = 0, pmask = 0;
    int remaining = k;
#pragma unroll 1
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = lane; i < 256; i += 64) hist[wave][i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (base + j < nv && (key[j] & pmask) == prefix) atomicAdd(&hist[wave][(key[j] >> shift) & 255u], 1);
      }
      __syncthreads();
      if (wave == 0) {
        int cc[4];
        int t4 = 0;
#pragma unroll 1
        for (int i = 0; i < 4; i++) {
          int sacc = 0;
#pragma unroll 4
          for (int w = 0; w < kWaves; w++) sacc += hist[w][lane * 4 + i];
          cc[i] = sacc;
          t4 += sacc;
        }
        const int incl = wave_incl_scan(t4);
        const int bef = incl - t4;
        if (bef < remaining && remaining <= incl) {
          int cum = bef;
          for (int i = 0; i < 4; i++) {
            if (remaining <= cum + cc[i]) {
              s_int[0] = lane * 4 + i;
              s_int[1] = cum;
              break;
            }
            cum += cc[i];
          }
        }
      }
      __syncthreads();
      prefix |= (uint32_t)s_int[0] << shift;
      pmask |= 255u << shift;
      remaining -= s_int[1];
      __syncthreads();
    }
    // index of the `remaining`-th entry equal to the k-th key (index order)
    int nt = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) nt += (base + j < nv && key[j] == prefix);
    int tot_ties;
    const int trank = block_excl_scan(nt, tmp, &tot_ties);
    if (trank < remaining && remaining <= trank + nt) {
      int cnt = trank;
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (base + j < nv && key[j] == prefix) {
          cnt++;
          if (cnt == remaining) s_int[2] = (int)(base + j);
        }
      }
    }
    __syncthreads();
    Kt = prefix;
    It = s_int[2];
  }
  // ---- emit the selected ids in ascending order
  int nsel = 0;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int64_t n = base + j;
    nsel += (n < nv) && (key[j] < Kt || (key[j] == Kt && n <= It));
  }
  int tot_sel;
  int pos = block_excl_scan(nsel, tmp, &tot_sel);
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int64_t n = base + j;
    if ((n < nv) && (key[j] < Kt || (key[j] == Kt && n <= It))) {
      if (pos < take) orow[pos] = (int32_t)n + id_offset;
      pos++;
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

static int launch_select(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, const int32_t* wpos, int window, hipStream_t st);

extern "C" int smla_topk(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, void* stream) {
  if (!scores || !out) return SMLA_E_NULL;
  if (R <= 0 || N <= 0 || k <= 0 || out_stride < k) return SMLA_E_SHAPE;
  if (R > 0x7fffffff || k > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  return launch_select(scores, R, N, nvis, k, out, out_stride, id_offset, nullptr, 0, st);
}

static int launch_select(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, const int32_t* wpos, int window, hipStream_t st) {
  int64_t per = (N + kTopkThreads - 1) / kTopkThreads;
  dim3 grid((unsigned)R), blk(kTopkThreads);
#define SMLA_TOPK_CASE(P)                                                                          \
  if (per <= P) {                                                                                  \
    hipLaunchKernelGGL(topk_kernel<P>, grid, blk, 0, st, scores, N, nvis, (int)k, out, out_stride, id_offset, \
                       wpos, window);                                                              \
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

extern "C" int smla_select_decode(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k,
                                  const int32_t* pos, int64_t window, int32_t* out, int64_t out_stride,
                                  int32_t id_offset, void* stream) {
  if (!scores || !out || !pos) return SMLA_E_NULL;
  if (R <= 0 || N <= 0 || k <= 0 || window < 0 || out_stride < k + window) return SMLA_E_SHAPE;
  if (R > 0x7fffffff || k > 0x7fffffff || window > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  if ((N + kTopkThreads - 1) / kTopkThreads > 64) return SMLA_E_UNSUPPORTED;
  return launch_select(scores, R, N, nvis, k, out, out_stride, id_offset, pos, (int)window, (hipStream_t)stream);
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
