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

constexpr int kTopkThreads = 1024;  // the largest workgroup (sizes the per-thread run PER)

__device__ inline uint32_t desc_key(float f) {
  if (f == 0.f) f = 0.f;  // -0 -> +0
  uint32_t u = __float_as_uint(f);
  uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}

// exclusive scan of one value per thread over a block of NW waves; returns the exclusive prefix
// and the block total.  `tmp` holds NW ints.  One barrier: every wave scans the per-wave totals
// itself.  The caller separates two scans on the same `tmp` by a barrier.
template <int NW>
__device__ inline int block_excl_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  const int wi = wave_incl_scan(lane < NW ? tmp[lane] : 0);
  const int before = wave > 0 ? __builtin_amdgcn_readlane(wi, wave - 1) : 0;
  *total = __builtin_amdgcn_readlane(wi, NW - 1);
  return before + x - v;
}

constexpr int kBuckets = 2048;
constexpr int kMaxCand = 256;

// inverse of desc_key (the score with -0 folded to +0)
__device__ inline float key_score(uint32_t key) {
  const uint32_t asc = ~key;
  return __uint_as_float((asc & 0x80000000u) ? (asc ^ 0x80000000u) : ~asc);
}


// floor((lmax - s) * bscale) clamped to [0, kBuckets), as one fma (one rounding of the exact
// lmax bscale - s bscale, monotone non-increasing in s), a clamp in float and a conversion in range
__device__ inline int bucket_of_score(float s, float lmax, float bscale) {
  const float t = __builtin_fmaf(-s, bscale, lmax * bscale);
  return (int)__builtin_amdgcn_fmed3f(t, 0.f, (float)(kBuckets - 1));
}
// monotone bucket of a finite score: 0 holds the largest scores
__device__ inline int bucket_of(uint32_t key, float lmax, float bscale) {
  return bucket_of_score(key_score(key), lmax, bscale);
}

// Row selection.  Produces the threshold pair (Kt, It) of the k-th best entry in the order
// (key asc == score desc, index asc); entry n is selected iff key < Kt or (key == Kt && n <= It).
//  * fast path: monotone buckets of (max - s) * 2048 / (max - min); the bucket holding the k-th
//    entry is found from a histogram + scan, and its (few) candidates are ranked exactly;
//  * fallback (degenerate spreads, > 256 candidates in the boundary bucket): 4 radix passes of 8
//    bits over the keys, then the tie rank among entries equal to the k-th key.
// Output: window ids (optional), then the selected ids ascending (+ id_offset), then -1.
template <int PER, int NT>
__global__ __launch_bounds__(NT) void topk_kernel(const float* scores, int64_t N, const int32_t* __restrict__ nvis,
                                                  int k, int32_t* __restrict__ out, int64_t out_stride,
                                                  int32_t id_offset, const int32_t* __restrict__ wpos, int window) {
  constexpr int kWaves = NT / 64;
  constexpr int kBPT = kBuckets / NT;  // histogram buckets owned by each thread in the scan
  static_assert(kBPT * NT == kBuckets, "buckets per thread");
  static_assert(PER <= 64, "per-thread selection masks are 64 bits");
  __shared__ int hist[kWaves][256];
  __shared__ int bhist[kBuckets + 1];  // + a slot that absorbs the counts of entries past nvis
  __shared__ int tmp[kWaves + 1];
  __shared__ float redf[5 * kWaves];
  __shared__ uint64_t cand_pair[kMaxCand];  // (key << 32) | index: the selection order is the integer order
  __shared__ int cand_idx[kMaxCand];
  __shared__ int s_int[5];
  __shared__ int s_nan[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t r = blockIdx.x;
  // N <= 65536 (PER * NT): every index of the row fits 32 bits
  const int base = tid * PER;
  // this thread's PER contiguous scores: 16-byte loads when the run lies inside the row and is
  // 16-byte aligned (rows of N floats: N % 4 == 0), element loads otherwise.  Issued first: the
  // window-id stores below may alias the scores, so loads placed after them would wait for them.
  float fv[PER];
  auto load_scores = [&](const float* row) {
    if (PER % 4 == 0 && (N & 3) == 0 && base + PER <= N) {
#pragma unroll
      for (int j = 0; j < PER; j += 4) {
        const f32x4_t v4 = *(const f32x4_t*)(row + base + j);
        fv[j] = v4[0];
        fv[j + 1] = v4[1];
        fv[j + 2] = v4[2];
        fv[j + 3] = v4[3];
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; j++) fv[j] = base + j < N ? row[base + j] : 0.f;
    }
  };
  load_scores(scores + r * N);
  int nv = nvis ? nvis[r] : (int)N;
  if (nv > (int)N) nv = (int)N;
  if (nv < 0) nv = 0;
  int32_t* orow = out + r * out_stride;
  if (wpos) {
    const int64_t p = wpos[r];
    for (int j = tid; j < window; j += NT) {
      const int64_t v = p - window + 1 + j;
      orow[j] = v < 0 ? -1 : (int32_t)v;
    }
    orow += window;
  }
  const int take = (int)(nv < k ? nv : k);

  // this thread's entries j < nloc are visible (index base + j < nvis)
  const int nloc = nv - base < 0 ? 0 : (nv - base > PER ? PER : nv - base);
  if (nv <= k) {
    for (int j = tid; j < k; j += NT) orow[j] = j < nv ? j + id_offset : -1;
    return;
  }
  // the bucket holding the k-th entry (bucket 0 = largest scores) and how many of its entries the
  // selection takes: s_int[0], s_int[1].  Thread t owns buckets kBPT t .. kBPT t + kBPT - 1.
  auto find_boundary = [&](int t) {
    int c[kBPT], sum = 0;
#pragma unroll
    for (int i = 0; i < kBPT; i++) {
      c[i] = bhist[kBPT * t + i];
      sum += c[i];
    }
    int tot;
    int before = block_excl_scan<kWaves>(sum, tmp, &tot);
#pragma unroll
    for (int i = 0; i < kBPT; i++) {
      if (before < k && k <= before + c[i]) {
        s_int[0] = kBPT * t + i;
        s_int[1] = k - before;
      }
      before += c[i];
    }
  };
  // rank of candidate c among the first `total` in the order (key asc, index asc)
  auto rank_of = [&](int c, int total) -> int {
    const uint64_t me = cand_pair[c];
    int rank = 0;
#pragma unroll 16
    for (int j = 0; j < total; j++) rank += cand_pair[j] < me;
    return rank;
  };

  uint32_t key[PER];
  uint32_t Kt = 0;
  int It = -1;
  {
    float lmin = SMLA_INF, lmax = -SMLA_INF;
    bool nan_seen = false;
#pragma unroll
    for (int j = 0; j < PER; j++) {
      const bool vis = j < nloc;
      const float f = fv[j];
      key[j] = vis ? desc_key(f) : 0xffffffffu;
      lmin = fminf(lmin, vis ? f : SMLA_INF);
      lmax = fmaxf(lmax, vis ? f : -SMLA_INF);
      nan_seen |= vis && f != f;
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
      for (int i = tid; i <= kBuckets; i += NT) bhist[i] = 0;
      __syncthreads();
      // every wave reduces the kWaves per-wave results itself (one LDS read per lane)
      const int wl = lane < kWaves ? lane : 0;
      lmin = wave_min_dpp(redf[wl]);
      lmax = wave_max_dpp(redf[kWaves + wl]);
      nan_seen = __builtin_amdgcn_ballot_w64(lane < kWaves && s_nan[wl] != 0) != 0;
    }
    // The plain selection buckets the finite scores: -inf scores (the indexer's mark of masked
    // keys) go to the absorbing slot and are never selected as long as k finite scores are visible
    // (with fewer, the radix fallback ranks them).  The finite minimum and the -inf count are only
    // reduced when the row minimum is -inf (a block-uniform condition).
    float lminf = lmin, ninf = 0.f;
    if (lmin == -SMLA_INF && !nan_seen && lmax > -SMLA_INF) {
      float mf = SMLA_INF, ni = 0.f;
#pragma unroll
      for (int j = 0; j < PER; j++) {
        const bool vis = j < nloc;
        mf = fminf(mf, vis && fv[j] > -SMLA_INF ? fv[j] : SMLA_INF);
        ni += (vis && fv[j] == -SMLA_INF) ? 1.f : 0.f;
      }
      mf = wave_min_dpp(mf);
      ni = wave_sum_dpp(ni);
      if (lane == 0) {
        redf[3 * kWaves + wave] = mf;
        redf[4 * kWaves + wave] = ni;
      }
      __syncthreads();
      const int wl = lane < kWaves ? lane : 0;
      lminf = wave_min_dpp(redf[3 * kWaves + wl]);
      ninf = wave_sum_dpp(lane < kWaves ? redf[4 * kWaves + wl] : 0.f);  // exact: an integer <= 65536
    }
    const bool ninf_ok = (float)nv - ninf >= (float)k;
    const float lo = lminf;
    const float bscale = (float)kBuckets / (lmax - lo);
    const bool spread_ok = !nan_seen && ninf_ok && bscale < SMLA_INF && bscale > 0.f && lo > -SMLA_INF &&
                           lmax < SMLA_INF;
    bool done = false;
    if (lmax == lmin && !nan_seen) {
      // every visible score equal: the k lowest indices
      Kt = desc_key(lmax);
      It = k - 1;
      done = true;
    }
    if (!done && spread_ok) {
      // ---- bucket histogram (bucket 0 holds the largest scores).  Each entry's bucket is
      // computed once, from the score itself (key_score(key) only folds -0 to +0, which the
      // subtraction from lmax does not see); entries past nvis go to the absorbing slot.
      int bk[PER];
#pragma unroll
      for (int j = 0; j < PER; j++) bk[j] = (j < nloc && fv[j] > -SMLA_INF) ? bucket_of_score(fv[j], lmax, bscale) : kBuckets;
#pragma unroll
      for (int j = 0; j < PER; j++) atomicAdd(&bhist[bk[j]], 1);
      __syncthreads();
      find_boundary(tid);
      if (tid == 0) s_int[3] = 0;  // candidate counter
      __syncthreads();
      const int bb = s_int[0], need = s_int[1];
      const int cb = bhist[bb];
      if (cb <= kMaxCand) {
        // candidates of the boundary bucket: per-thread count, wave offsets by scan, one LDS
        // atomic per wave
        int mine = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) mine += bk[j] == bb;
        const int incl = wave_incl_scan(mine);
        int wbase = 0;
        if (lane == 63 && incl > 0) wbase = atomicAdd(&s_int[3], incl);
        wbase = __builtin_amdgcn_readlane(wbase, 63);
        int slot = wbase + incl - mine;
#pragma unroll
        for (int j = 0; j < PER; j++) {
          if (bk[j] == bb) {
            if (slot < kMaxCand) cand_pair[slot] = ((uint64_t)key[j] << 32) | (uint32_t)(base + j);
            slot++;
          }
        }
        __syncthreads();
        if (tid < cb && rank_of(tid, cb) == need - 1) {
          const uint64_t pr = cand_pair[tid];
          s_int[0] = (int)(uint32_t)(pr >> 32);
          s_int[1] = (int)(uint32_t)pr;
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
          if (j < nloc && (key[j] & pmask) == prefix) atomicAdd(&hist[wave][(key[j] >> shift) & 255u], 1);
        }
        __syncthreads();
        if (wave == 0) {
          int cc4[4];
          int t4 = 0;
#pragma unroll 1
          for (int i = 0; i < 4; i++) {
            int sacc = 0;
#pragma unroll 4
            for (int w = 0; w < kWaves; w++) sacc += hist[w][lane * 4 + i];
            cc4[i] = sacc;
            t4 += sacc;
          }
          const int incl = wave_incl_scan(t4);
          const int bef = incl - t4;
          if (bef < remaining && remaining <= incl) {
            int cum = bef;
            for (int i = 0; i < 4; i++) {
              if (remaining <= cum + cc4[i]) {
                s_int[0] = lane * 4 + i;
                s_int[1] = cum;
                break;
              }
              cum += cc4[i];
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
      for (int j = 0; j < PER; j++) nt += (j < nloc && key[j] == prefix);
      int tot_ties;
      const int trank = block_excl_scan<kWaves>(nt, tmp, &tot_ties);
      if (trank < remaining && remaining <= trank + nt) {
        int cnt = trank;
#pragma unroll
        for (int j = 0; j < PER; j++) {
          if (j < nloc && key[j] == prefix) {
            cnt++;
            if (cnt == remaining) s_int[2] = (int)(base + j);
          }
        }
      }
      __syncthreads();
      Kt = prefix;
      It = s_int[2];
    }
  }
  // ---- emit the selected ids in ascending order: the selection as a bit mask, evaluated once for
  // the count and the placement
  uint64_t selm = 0;  // PER <= 64
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int n = base + j;
    const bool sel = j < nloc && (key[j] < Kt || (key[j] == Kt && n <= It));
    selm |= (uint64_t)sel << j;
  }
  const int nsel = __builtin_popcountll(selm);
  int tot_sel;
  int pos = block_excl_scan<kWaves>(nsel, tmp, &tot_sel);
  // ids go straight to their output positions (each wave's selected ids fill one contiguous run)
#pragma unroll
  for (int j = 0; j < PER; j++) {
    if ((selm >> j) & 1ull) {
      if (pos < take) orow[pos] = (int32_t)(base + j) + id_offset;
      pos++;
    }
  }
  for (int j = take + tid; j < k; j += NT) orow[j] = -1;
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
  const dim3 grid((unsigned)R);
  // 1024 threads (16 waves: the per-entry phases are VALU-bound and need the waves to hide latency)
#define SMLA_TOPK_LAUNCH(P, T)                                                                            \
  {                                                                                                    \
    hipLaunchKernelGGL((topk_kernel<P, T>), grid, dim3(T), 0, st, scores, N, nvis, (int)k, out, out_stride, \
                       id_offset, wpos, window);                                                       \
    SMLA_HIP_CHECK_LAUNCH();                                                                           \
    return SMLA_OK;                                                                                    \
  }
  const int64_t per = (N + kTopkThreads - 1) / kTopkThreads;
  if (per <= 2) SMLA_TOPK_LAUNCH(2, kTopkThreads)
  if (per <= 4) SMLA_TOPK_LAUNCH(4, kTopkThreads)
  if (per <= 8) SMLA_TOPK_LAUNCH(8, kTopkThreads)
  if (per <= 16) SMLA_TOPK_LAUNCH(16, kTopkThreads)
  if (per <= 32) SMLA_TOPK_LAUNCH(32, kTopkThreads)
  if (per <= 64) SMLA_TOPK_LAUNCH(64, kTopkThreads)
#undef SMLA_TOPK_LAUNCH
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

extern "C" size_t smla_index_decode_workspace(int64_t B, int64_t S, int64_t N) {
  if (B <= 0 || S <= 0 || N <= 0) return 0;
  return (size_t)(B * S * N) * sizeof(float);  // the scores
}

extern "C" int smla_index_decode(const void* q, int q_dtype, const void* keys, int k_dtype, const float* kscale,
                                 const float* weights, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi,
                                 int64_t Di, int64_t N, int64_t k, const int32_t* pos, int64_t window,
                                 int32_t* out, int64_t out_stride, int32_t id_offset, int flags,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !keys || !weights || !out) return SMLA_E_NULL;
  if (window > 0 && !pos) return SMLA_E_NULL;
  if (B <= 0 || S <= 0 || Hi <= 0 || Di <= 0 || N <= 0 || k <= 0 || window < 0 || out_stride < k + window)
    return SMLA_E_SHAPE;
  if (flags & ~SMLA_INDEX_EXACT) return SMLA_E_RANGE;
  if (!workspace || workspace_bytes < smla_index_decode_workspace(B, S, N)) return SMLA_E_WORKSPACE;
  const int64_t R = B * S;
  if (R > 65535 || k > 0x7fffffff || window > 0x7fffffff || (N + kTopkThreads - 1) / kTopkThreads > 64)
    return SMLA_E_UNSUPPORTED;
  // the fixed-order scores (matrix-core chains for 64 heads x 64 dims) into the workspace, then the
  // exact selection; SMLA_INDEX_EXACT changes nothing (the scores are always the fixed-order ones)
  float* sc = (float*)workspace;
  const int rc = smla_indexer_score(q, q_dtype, keys, k_dtype, kscale, weights, nvis, B, S, Hi, Di, N, sc, stream);
  if (rc != SMLA_OK) return rc;
  return launch_select(sc, R, N, nvis, k, out, out_stride, id_offset, window > 0 ? pos : nullptr, (int)window,
                       (hipStream_t)stream);
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
