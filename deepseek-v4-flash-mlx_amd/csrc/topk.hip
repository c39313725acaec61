// Top-k selection and index construction.
//
// smla_topk: per row, rank the first nvis scores by (score desc, index asc) with -0 == +0, keep
// min(k, nvis), emit ascending ids (+ id_offset), -1 padded to k.  One workgroup of 1024 threads
// per row; each thread owns a contiguous run of PER keys in registers (key = order-preserving
// uint32, larger score -> smaller key).  The k-th best entry (Kt, It) comes from the row selection
// of select_row.h; a block-wide scan in index order then places every selected id at its
// ascending position.  Bit-exact by construction: only comparisons and counts.  When
// nvis <= k every visible id is taken (oracle/decode_engine.py:112-114, "all causally visible
// compressed rows").  smla_select_decode also writes the decode window ids in front (one launch
// for the engine's whole index build, oracle/decode_engine.py:110-114).
//
// smla_window_topk_idxs mirrors ref_torch/sparse_attn.py:9-20; smla_decode_window_idxs builds the
// engine's decode window oracle/decode_engine.py:110-111 over an un-ringed raw cache.
#include "select_row.h"
#include "smla_internal.h"

namespace {

using smla_select::block_excl_scan;

constexpr int kTopkThreads = 1024;  // the largest workgroup (sizes the per-thread run PER)

// One row per workgroup of NT threads: window ids (optional), then the selected ids ascending
// (+ id_offset), then -1.
template <int PER, int NT>
__global__ __launch_bounds__(NT) void topk_kernel(const float* scores, int64_t N, const int32_t* __restrict__ nvis,
                                                  int k, int32_t* __restrict__ out, int64_t out_stride,
                                                  int32_t id_offset, const int32_t* __restrict__ wpos, int window) {
  constexpr int kWaves = NT / 64;
  static_assert(PER <= 64, "per-thread selection masks are 64 bits");
  __shared__ smla_select::Lds<NT> sm;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  // N <= 65536 (PER * NT): every index of the row fits 32 bits
  const int base = tid * PER;
  // the row's visible count and this thread's PER contiguous scores, requested together (one
  // round trip): 16-byte loads when rows are 16-byte aligned (N % 4 == 0; a quad past the row end
  // reads the row's last quad, never visible), element loads otherwise.  No branch per thread
  // between the loads and their first use, so no wait lands before the window-id stores (issued
  // after the loads: they may alias the scores).
  int nv = nvis ? nvis[r] : (int)N;
  float fv[PER];
  {
    const float* row = scores + r * N;
    if (PER % 4 == 0 && (N & 3) == 0 && N >= 4) {  // uniform
#pragma unroll
      for (int j = 0; j < PER; j += 4) {
        const int64_t a = base + j < N ? base + j : N - 4;
        const f32x4_t v4 = *(const f32x4_t*)(row + a);
        fv[j] = v4[0];
        fv[j + 1] = v4[1];
        fv[j + 2] = v4[2];
        fv[j + 3] = v4[3];
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; j++) fv[j] = row[base + j < N ? base + j : N - 1];
    }
  }
  if (nv > (int)N) nv = (int)N;
  if (nv < 0) nv = 0;
  int32_t* orow = out + r * out_stride;
  if (wpos) {
    // position v of the window lives at raw row v mod id_offset (the raw source is a ring of
    // id_offset >= window rows; the identity for a cache with a row per position)
    const int64_t p = wpos[r];
    for (int j = tid; j < window; j += NT) {
      const int64_t v = p - window + 1 + j;
      orow[j] = v < 0 ? -1 : (int32_t)(id_offset > 0 ? (uint32_t)v % (uint32_t)id_offset : (uint32_t)v);
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
  uint32_t key[PER];
  uint32_t Kt;
  int It;
  smla_select::row_threshold<PER, NT>(fv, nloc, base, nv, k, sm, key, Kt, It);
  // ---- emit the selected ids in ascending order; ids go straight to their output positions
  // (each wave's selected ids fill one contiguous run)
  const auto selm = smla_select::selected_mask<PER>(key, nloc, base, Kt, It);
  int tot_sel;
  int pos = block_excl_scan<kWaves>(smla_select::sel_count<PER>(selm), sm.tmp, &tot_sel);
#pragma unroll
  for (int j = 0; j < PER; j++) {
    if ((selm >> j) & 1u) {
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
  if (id_offset > 0 && window > id_offset) return SMLA_E_SHAPE;  // a raw ring shorter than the window
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
  if (window > 0 && id_offset > 0 && window > id_offset) return SMLA_E_SHAPE;
  if (!workspace || workspace_bytes < smla_index_decode_workspace(B, S, N)) return SMLA_E_WORKSPACE;
  const int64_t R = B * S;
  if (R > 0x7fffffff || k > 0x7fffffff || window > 0x7fffffff || (N + kTopkThreads - 1) / kTopkThreads > 64)
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
