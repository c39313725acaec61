// Exact selection of the k best of one row of scores by a whole workgroup (the top-k of
// topk.hip and the selection the fused decode attention runs in its prologue).  Order: score
// descending, then index ascending, -0 == +0.  Every thread holds a contiguous run of PER
// scores; the threshold pair (Kt, It) of the k-th best entry comes from a bucket select
// (monotone value buckets, exact ranking of the boundary bucket) or, for degenerate spreads, 4
// radix passes plus a tie rank: only comparisons and counts, so the result is exact.
#pragma once
#include <type_traits>

#include "smla_internal.h"

namespace smla_select {

constexpr int kMaxCand = 256;  // boundary-bucket entries ranked exactly (more: the radix path)

// order-preserving key (larger score -> smaller key; -0 folded to +0): a non-negative score's bits
// with the 31 low bits inverted, a negative score's bits as they are
__device__ inline uint32_t desc_key(float f) {
  uint32_t u = __float_as_uint(f);
  u = u == 0x80000000u ? 0u : u;                              // -0 -> +0
  return u ^ (~(uint32_t)((int32_t)u >> 31) & 0x7fffffffu);  // sign clear: flip bits 0..30
}

// exclusive scan of one value per thread over a block of NW waves; returns the exclusive prefix
// and the block total.  `tmp` holds NW ints.  One barrier: every wave scans the per-wave totals
// itself.  The caller separates two scans on the same `tmp` by a barrier.
template <int NW, class IntPtr>
__device__ inline int block_excl_scan(int v, IntPtr tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  const int wi = wave_incl_scan(lane < NW ? tmp[lane] : 0);
  const int before = wave > 0 ? __builtin_amdgcn_readlane(wi, wave - 1) : 0;
  *total = __builtin_amdgcn_readlane(wi, NW - 1);
  return before + x - v;
}

// LDS of a selection by NT threads; 2 NT value buckets (two per thread in the boundary scan)
template <int NT>
struct Lds {
  static constexpr int kWaves = NT / 64;
  static constexpr int kBuckets = 2 * NT;
  int hist[kWaves][256];
  int bhist[kBuckets + 1];  // + a slot that absorbs the counts of entries past nvis
  int tmp[kWaves + 1];
  float redf[5 * kWaves];
  uint64_t cand_pair[kMaxCand];  // (key << 32) | index: the selection order is the integer order
  int s_int[5];
  int s_nan[kWaves];
};

// floor((lmax - s) * bscale) clamped to [0, NB), as one fma (one rounding of the exact
// lmax bscale - s bscale, monotone non-increasing in s), a clamp in float and a conversion in range
template <int NB>
__device__ inline int bucket_of_score(float s, float lmax, float bscale) {
  const float t = __builtin_fmaf(-s, bscale, lmax * bscale);
  return (int)__builtin_amdgcn_fmed3f(t, 0.f, (float)(NB - 1));
}

// The threshold pair (Kt, It) of the k-th best of the nv visible entries (k < nv): entry n is
// selected iff key < Kt or (key == Kt && n <= It).  fv: this thread's scores at indexes base ..
// base + PER - 1, the first nloc of them visible; key receives their order keys (0xffffffff past
// nloc).  The whole workgroup (NT threads) calls it.
//  * fast path: monotone buckets of (max - s) * 2 NT / (max - min); the bucket holding the k-th
//    entry is found from a histogram + scan, and its (few) candidates are ranked exactly;
//  * fallback (degenerate spreads, > 256 candidates in the boundary bucket): 4 radix passes of 8
//    bits over the keys, then the tie rank among entries equal to the k-th key.
template <int PER, int NT, class L>
__device__ inline void row_threshold(const float (&fv)[PER], int nloc, int base, int nv, int k, L& sm,
                                     uint32_t (&key)[PER], uint32_t& Kt, int& It) {
  constexpr int kWaves = NT / 64;
  constexpr int kBuckets = 2 * NT;
  constexpr int kBPT = 2;  // histogram buckets owned by each thread in the scan
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the bucket holding the k-th entry (bucket 0 = largest scores) and how many of its entries the
  // selection takes: s_int[0], s_int[1].  Thread t owns buckets kBPT t .. kBPT t + kBPT - 1.
  auto find_boundary = [&](int t) {
    int c[kBPT], sum = 0;
#pragma unroll
    for (int i = 0; i < kBPT; i++) {
      c[i] = sm.bhist[kBPT * t + i];
      sum += c[i];
    }
    int tot;
    int before = block_excl_scan<kWaves>(sum, sm.tmp, &tot);
#pragma unroll
    for (int i = 0; i < kBPT; i++) {
      if (before < k && k <= before + c[i]) {
        sm.s_int[0] = kBPT * t + i;
        sm.s_int[1] = k - before;
      }
      before += c[i];
    }
  };
  // rank of candidate c among the first `total` in the order (key asc, index asc).  The slots
  // from total up to the next multiple of 8 hold the largest pair (never below a candidate), so
  // the loads go 8 at a time and their latencies overlap (a loop over `total` alone runs its
  // remainder one dependent load at a time: ≈1.3 K cycles for the ≈10 candidates of a row)
  auto rank_of = [&](int c, int total) -> int {
    const uint64_t me = sm.cand_pair[c];
    int rank = 0;
    for (int j0 = 0; j0 < total; j0 += 8) {
      uint64_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = sm.cand_pair[j0 + u];
#pragma unroll
      for (int u = 0; u < 8; u++) rank += v[u] < me;
    }
    return rank;
  };

  Kt = 0;
  It = -1;
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
      sm.redf[wave] = a;
      sm.redf[kWaves + wave] = bmx;
      sm.s_nan[wave] = wnan;
    }
    for (int i = tid; i <= kBuckets; i += NT) sm.bhist[i] = 0;
    __syncthreads();
    // every wave reduces the kWaves per-wave results itself (one LDS read per lane)
    const int wl = lane < kWaves ? lane : 0;
    lmin = wave_min_dpp(sm.redf[wl]);
    lmax = wave_max_dpp(sm.redf[kWaves + wl]);
    nan_seen = __builtin_amdgcn_ballot_w64(lane < kWaves && sm.s_nan[wl] != 0) != 0;
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
      sm.redf[3 * kWaves + wave] = mf;
      sm.redf[4 * kWaves + wave] = ni;
    }
    __syncthreads();
    const int wl = lane < kWaves ? lane : 0;
    lminf = wave_min_dpp(sm.redf[3 * kWaves + wl]);
    ninf = wave_sum_dpp(lane < kWaves ? sm.redf[4 * kWaves + wl] : 0.f);  // exact: an integer <= 65536
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
    // ---- bucket histogram (bucket 0 holds the largest scores).  Each entry's bucket is computed
    // once, from the score itself (the order key only folds -0 to +0, which the subtraction from
    // lmax does not see); entries past nvis go to the absorbing slot.
    int bk[PER];
#pragma unroll
    for (int j = 0; j < PER; j++)
      bk[j] = (j < nloc && fv[j] > -SMLA_INF) ? bucket_of_score<kBuckets>(fv[j], lmax, bscale) : kBuckets;
#pragma unroll
    for (int j = 0; j < PER; j++) atomicAdd(&sm.bhist[bk[j]], 1);
    __syncthreads();
    find_boundary(tid);
    if (tid == 0) sm.s_int[3] = 0;  // candidate counter
    __syncthreads();
    const int bb = sm.s_int[0], need = sm.s_int[1];
    const int cb = sm.bhist[bb];
    if (cb <= kMaxCand) {
      // candidates of the boundary bucket: per-thread count, wave offsets by scan, one LDS atomic
      // per wave
      int mine = 0;
#pragma unroll
      for (int j = 0; j < PER; j++) mine += bk[j] == bb;
      const int incl = wave_incl_scan(mine);
      int wbase = 0;
      if (lane == 63 && incl > 0) wbase = atomicAdd(&sm.s_int[3], incl);
      wbase = __builtin_amdgcn_readlane(wbase, 63);
      int slot = wbase + incl - mine;
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (bk[j] == bb) {
          if (slot < kMaxCand) sm.cand_pair[slot] = ((uint64_t)key[j] << 32) | (uint32_t)(base + j);
          slot++;
        }
      }
      if (tid >= cb && tid < ((cb + 7) & ~7)) sm.cand_pair[tid] = ~0ull;  // rank_of's padding
      __syncthreads();
      if (tid < cb && rank_of(tid, cb) == need - 1) {
        const uint64_t pr = sm.cand_pair[tid];
        sm.s_int[0] = (int)(uint32_t)(pr >> 32);
        sm.s_int[1] = (int)(uint32_t)pr;
      }
      __syncthreads();
      Kt = (uint32_t)sm.s_int[0];
      It = sm.s_int[1];
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
      for (int i = lane; i < 256; i += 64) sm.hist[wave][i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (j < nloc && (key[j] & pmask) == prefix) atomicAdd(&sm.hist[wave][(key[j] >> shift) & 255u], 1);
      }
      __syncthreads();
      if (wave == 0) {
        int cc4[4];
        int t4 = 0;
#pragma unroll 1
        for (int i = 0; i < 4; i++) {
          int sacc = 0;
#pragma unroll 4
          for (int w = 0; w < kWaves; w++) sacc += sm.hist[w][lane * 4 + i];
          cc4[i] = sacc;
          t4 += sacc;
        }
        const int incl = wave_incl_scan(t4);
        const int bef = incl - t4;
        if (bef < remaining && remaining <= incl) {
          int cum = bef;
          for (int i = 0; i < 4; i++) {
            if (remaining <= cum + cc4[i]) {
              sm.s_int[0] = lane * 4 + i;
              sm.s_int[1] = cum;
              break;
            }
            cum += cc4[i];
          }
        }
      }
      __syncthreads();
      prefix |= (uint32_t)sm.s_int[0] << shift;
      pmask |= 255u << shift;
      remaining -= sm.s_int[1];
      __syncthreads();
    }
    // index of the `remaining`-th entry equal to the k-th key (index order)
    int nt = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) nt += (j < nloc && key[j] == prefix);
    int tot_ties;
    const int trank = block_excl_scan<kWaves>(nt, sm.tmp, &tot_ties);
    if (trank < remaining && remaining <= trank + nt) {
      int cnt = trank;
#pragma unroll
      for (int j = 0; j < PER; j++) {
        if (j < nloc && key[j] == prefix) {
          cnt++;
          if (cnt == remaining) sm.s_int[2] = (int)(base + j);
        }
      }
    }
    __syncthreads();
    Kt = prefix;
    It = sm.s_int[2];
  }
}

// this thread's selected entries as a bit mask (PER <= 64; 32-bit for PER <= 32)
template <int PER>
using SelMask = typename std::conditional<(PER <= 32), uint32_t, uint64_t>::type;
template <int PER>
__device__ inline SelMask<PER> selected_mask(const uint32_t (&key)[PER], int nloc, int base, uint32_t Kt, int It) {
  SelMask<PER> selm = 0;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const bool sel = j < nloc && (key[j] < Kt || (key[j] == Kt && base + j <= It));
    selm |= (SelMask<PER>)sel << j;
  }
  return selm;
}
template <int PER>
__device__ inline int sel_count(SelMask<PER> m) {
  if constexpr (PER <= 32) return __builtin_popcount(m);
  else return __builtin_popcountll(m);
}

}  // namespace smla_select
