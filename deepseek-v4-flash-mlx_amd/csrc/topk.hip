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
#include <type_traits>

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

// Context of a certified selection (smla_index_decode).  The scores are the approximations a_n of
// indexer_cert_kernel, ebound holds their per-chunk bounds (|a_n - s_n| <= bound, s_n the
// fixed-order score), and q / keys / kscale / w let the kernel recompute s_n for any key.
struct CertCtx {
  const float* ebound;  // [R, nchunk]
  int nchunk;
  const uint16_t* q;    // [R, 64, 64] bf16
  const uint8_t* keys;  // [B, N, 64] e4m3
  const float* kscale;  // [B, N] or null
  const float* w;       // [R, 64]
  int64_t S;            // query rows per batch entry: key rows of row r are batch r / S
  int force_exact;      // 1: skip certification, rescore every visible key (the slow path)
  float* rescored;      // [R, N]: the slow path's exact scores (the approximations' buffer itself)
};

constexpr int kQS = 68;  // LDS row stride (floats) of the staged q rows: 16-byte per-head reads hit all banks
constexpr int kRescoreChunk = 128;  // keys rescored per pass (their fp32 rows and ReLU values sit in LDS)
constexpr int kStageIds = 4096;   // selections up to this size are staged in LDS for coalesced stores

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
// Certified mode (CERT): the scores are approximations a_n with |a_n - s_n| <= E for the exact
// scores s_n.  With bb the bucket of the k-th largest a, an entry with bucket(a_n - 2E) < bb
// is certainly selected, one with bucket(a_n + 2E) > bb certainly not; the entries in between
// (the band: bucket bb and whatever lies within 2E of it) are rescored exactly and ranked.  The
// k-th largest s lies within E of the k-th largest a, which makes this the exact selection.  A
// row that cannot be certified (a bound that is not finite, a degenerate spread, more than 256
// band entries) is rescored in full and selected exactly.
// Output: window ids (optional), then the selected ids ascending (+ id_offset), then -1.
template <int PER, bool CERT, int NT>
__global__ __launch_bounds__(NT) void topk_kernel(const float* scores, int64_t N,
                                                            const int32_t* __restrict__ nvis, int k,
                                                            int32_t* __restrict__ out, int64_t out_stride,
                                                            int32_t id_offset, const int32_t* __restrict__ wpos,
                                                            int window, CertCtx cc) {
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
  __shared__ int out_s[kStageIds];           // the selected ids in output order, stored coalesced at the end
  __shared__ int s_int[5];
  __shared__ int s_nan[kWaves];
  __shared__ float q_s[CERT ? 64 * kQS : 1];
  __shared__ float w_s[CERT ? 64 : 1];
  __shared__ __align__(16) float kf_s[CERT ? kRescoreChunk * 64 : 1];  // key rows being rescored, fp32
  __shared__ float rl_s[CERT ? kRescoreChunk * 65 : 1];               // their ReLU(dot_h), [key][head]
  __shared__ float sc_s[CERT ? kRescoreChunk : 1];                     // their fixed-order sums over h
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
  const int64_t bkey = CERT ? r / cc.S : 0;  // batch entry of the key rows
  // the q row (4 bf16 per thread) and weights: loaded now, staged in LDS after the first barrier
  // (4096 / NT bf16 values per thread)
  constexpr int kQPT = 4096 / NT;
  static_assert(kQPT == 4 || kQPT == 8, "q values per thread");
  using QRawT = typename std::conditional<kQPT == 4, u32x2_t, u32x4_t>::type;
  QRawT qraw = {};
  float wraw = 0.f;
  if constexpr (CERT) {
    qraw = *(const QRawT*)(cc.q + r * 4096 + kQPT * tid);
    if (tid < 64) wraw = cc.w[r * 64 + tid];
  }
  // Fixed-order scores (the indexer's arithmetic, before the kscale product) of the cnt
  // <= kRescoreChunk keys whose fp32 rows are in kf_s, into sc_s.  Wave w takes keys w + kWaves i
  // (i < kKPW) and lane h runs head h's fma chain over d = 0..63 for all of them at once: per block
  // of 16 dims the q values are read from LDS once and each key's 16 values by LDS broadcast, so
  // every chain advances in d order.  The ReLU values go to rl_s; then one thread per key runs the
  // chain over the heads.  Ends with a barrier (sc_s complete).
  constexpr int kKPW = kRescoreChunk / kWaves;  // keys per wave (8 or 16)
  auto exact_chunk = [&](int cnt) {
    const float* qrow = &q_s[lane * kQS];
    const int mine = wave < cnt ? (cnt - wave + kWaves - 1) / kWaves : 0;  // this wave's keys
    float d[kKPW];
#pragma unroll
    for (int b = 0; b < kKPW; b++) d[b] = 0.f;
#pragma unroll 1
    for (int jb = 0; jb < 64; jb += 16) {
      f32x4_t q4[4];
#pragma unroll
      for (int e = 0; e < 4; e++) q4[e] = *(const f32x4_t*)&qrow[jb + 4 * e];
#pragma unroll
      for (int b = 0; b < kKPW; b++) {
        if (b < mine) {
          const float* kr = &kf_s[(wave + kWaves * b) * 64 + jb];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const f32x4_t kk = *(const f32x4_t*)&kr[4 * e];
            d[b] = __builtin_fmaf(q4[e][0], kk[0], d[b]);
            d[b] = __builtin_fmaf(q4[e][1], kk[1], d[b]);
            d[b] = __builtin_fmaf(q4[e][2], kk[2], d[b]);
            d[b] = __builtin_fmaf(q4[e][3], kk[3], d[b]);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < kKPW; b++)
      if (b < mine) rl_s[(wave + kWaves * b) * 65 + lane] = d[b] > 0.f ? d[b] : 0.f;
    __syncthreads();
    if (tid < cnt) {
      float acc = 0.f;
#pragma unroll 16
      for (int h = 0; h < 64; h++) acc = __builtin_fmaf(w_s[h], rl_s[tid * 65 + h], acc);
      sc_s[tid] = acc;
    }
    __syncthreads();
  };
  // a chunk's code rows are staged kCPT codes per thread: thread t converts codes
  // kCPT (t % kTPK) .. of key t / kTPK to fp32 in kf_s
  constexpr int kCPT = kRescoreChunk * 64 / NT;  // 8 or 16
  constexpr int kTPK = 64 / kCPT;                // threads per key row
  static_assert(kCPT == 8 || kCPT == 16, "codes per thread");
  using CodeT = typename std::conditional<kCPT == 8, u32x2_t, u32x4_t>::type;
  auto stage_key = [&](int c, CodeT codes) {
    f32x4_t* dst = (f32x4_t*)&kf_s[c * 64 + kCPT * (tid % kTPK)];
#pragma unroll
    for (int i = 0; i < kCPT / 4; i++) {
      const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[i], false);
      const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[i], true);
      dst[i] = f32x4_t{a.x, a.y, b.x, b.y};
    }
  };
  auto key_codes = [&](int64_t n) -> CodeT {
    return *(const CodeT*)(cc.keys + (bkey * N + n) * 64 + kCPT * (tid % kTPK));
  };
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

  float emax = 0.f;
  if constexpr (CERT) {
    for (int c = tid; c < cc.nchunk; c += NT) {
      const float e = cc.ebound[r * cc.nchunk + c];
      emax = fmaxf(emax, e == e ? e : SMLA_INF);
    }
  }
  uint32_t key[PER];
  uint32_t Kt = 0;
  int It = -1;
  // certified selection state (used by the emit when band_mode)
  bool band_mode = false;
  uint64_t in_mask = 0, band_mask = 0;
  int slot0 = 0;
  bool certified = CERT;
#pragma unroll 1
  for (int pass = 0; pass < 2; pass++) {
    if (pass > 0) __syncthreads();  // the previous pass's readers of redf / bhist are done
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
    // ---- row min / max (and whether a NaN is visible; the bound max on a certified pass)
    {
      const float a = wave_min_dpp(lmin), bmx = wave_max_dpp(lmax);
      const float em = CERT ? wave_max_dpp(emax) : 0.f;
      const bool wnan = __builtin_amdgcn_ballot_w64(nan_seen) != 0;
      if (lane == 0) {
        redf[wave] = a;
        redf[kWaves + wave] = bmx;
        redf[2 * kWaves + wave] = em;
        s_nan[wave] = wnan;
      }
      for (int i = tid; i <= kBuckets; i += NT) bhist[i] = 0;
      if (CERT && pass == 0) {
        const int h = (kQPT * tid) >> 6, d0 = (kQPT * tid) & 63;
#pragma unroll
        for (int i = 0; i < kQPT / 4; i++)
          *(f32x4_t*)&q_s[h * kQS + d0 + 4 * i] =
              f32x4_t{__uint_as_float(qraw[2 * i] << 16), __uint_as_float(qraw[2 * i] & 0xffff0000u),
                      __uint_as_float(qraw[2 * i + 1] << 16), __uint_as_float(qraw[2 * i + 1] & 0xffff0000u)};
        if (tid < 64) w_s[tid] = wraw;
      }
      __syncthreads();
      // every wave reduces the kWaves per-wave results itself (one LDS read per lane)
      const int wl = lane < kWaves ? lane : 0;
      lmin = wave_min_dpp(redf[wl]);
      lmax = wave_max_dpp(redf[kWaves + wl]);
      if (CERT) emax = wave_max_dpp(redf[2 * kWaves + wl]);
      nan_seen = __builtin_amdgcn_ballot_w64(lane < kWaves && s_nan[wl] != 0) != 0;
    }
    // The plain selection buckets the finite scores: -inf scores (the indexer's mark of masked
    // keys) go to the absorbing slot and are never selected as long as k finite scores are visible
    // (with fewer, the radix fallback ranks them).  The finite minimum and the -inf count are only
    // reduced when the row minimum is -inf (a block-uniform condition).  The certified pass keeps
    // the full range.
    const bool plain = !(CERT && certified);
    float lminf = lmin, ninf = 0.f;
    if (plain && lmin == -SMLA_INF && !nan_seen && lmax > -SMLA_INF) {
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
    const bool ninf_ok = !plain || (float)nv - ninf >= (float)k;
    const float lo = plain ? lminf : lmin;
    const float bscale = (float)kBuckets / (lmax - lo);
    const bool spread_ok = !nan_seen && ninf_ok && bscale < SMLA_INF && bscale > 0.f && lo > -SMLA_INF &&
                           lmax < SMLA_INF;
    if (CERT && certified) {
      // band half-width: twice the row bound, plus room for the rounding of a -+ E2
      const float E2 = 2.f * emax * (1.f + 0x1p-8f) + 0x1p-20f * fmaxf(fabsf(lmin), fabsf(lmax));
      if (cc.force_exact == 0 && spread_ok && E2 < SMLA_INF) {
        // ---- bucket histogram of the approximate scores
#pragma unroll
        for (int j = 0; j < PER; j++) atomicAdd(&bhist[j < nloc ? bucket_of(key[j], lmax, bscale) : kBuckets], 1);
        __syncthreads();
        find_boundary(tid);
        if (tid == 0) {
          s_int[3] = 0;
          s_int[4] = 0;
        }
        __syncthreads();
        const int bb = s_int[0], need = s_int[1];
        // ---- band: in (certainly selected), band (rescored), the rest certainly not selected
        int mine = 0, mine_u = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) {
          const float a = key_score(key[j]);
          const bool in = j < nloc && bucket_of_score(a - E2, lmax, bscale) < bb;
          const bool band = j < nloc && !in && bucket_of_score(a + E2, lmax, bscale) <= bb;
          in_mask |= (uint64_t)in << j;
          band_mask |= (uint64_t)band << j;
          mine += band;
          mine_u += band && bucket_of(key[j], lmax, bscale) < bb;
        }
        const int incl = wave_incl_scan(mine);
        const int incl_u = wave_incl_scan(mine_u);
        int wbase = 0;
        if (lane == 63) {
          if (incl > 0) wbase = atomicAdd(&s_int[3], incl);
          if (incl_u > 0) atomicAdd(&s_int[4], incl_u);
        }
        wbase = __builtin_amdgcn_readlane(wbase, 63);
        slot0 = wbase + incl - mine;
        int slot = slot0;
#pragma unroll
        for (int j = 0; j < PER; j++) {
          if ((band_mask >> j) & 1u) {
            if (slot < kMaxCand) cand_idx[slot] = (int)(base + j);
            slot++;
          }
        }
        __syncthreads();
        const int total = s_int[3], ucnt = s_int[4];
        if (total <= kMaxCand) {
          // exact scores of the band, kRescoreChunk keys per pass (one pass for the usual band):
          // their code rows to LDS as fp32, the fixed-order chains, then the kscale product
#pragma unroll 1
          for (int c0 = 0; c0 < total; c0 += kRescoreChunk) {
            const int cnt = total - c0 < kRescoreChunk ? total - c0 : kRescoreChunk;
            const int ck = tid / kTPK;
            float ksv = 1.f;
            if (ck < cnt) {
              const int n = cand_idx[c0 + ck];
              stage_key(ck, key_codes(n));
              if (cc.kscale) ksv = cc.kscale[bkey * N + n];
            }
            __syncthreads();
            exact_chunk(cnt);
            if (tid % kTPK == 0 && ck < cnt) {
              const float acc = sc_s[ck];
              const float sx = cc.kscale ? acc * ksv : acc;
              cand_pair[c0 + ck] = ((uint64_t)desc_key(sx) << 32) | (uint32_t)cand_idx[c0 + ck];
            }
          }
          __syncthreads();
          // the band supplies need + (its entries above bucket bb) of the selection
          const int need_b = need + ucnt;
          if (tid < total && rank_of(tid, total) == need_b - 1) {
            const uint64_t pr = cand_pair[tid];
            s_int[0] = (int)(uint32_t)(pr >> 32);
            s_int[1] = (int)(uint32_t)pr;
          }
          __syncthreads();
          Kt = (uint32_t)s_int[0];
          It = s_int[1];
          band_mode = true;
          break;
        }
        in_mask = band_mask = 0;
      }
      // not certifiable: every visible key's exact score (written over the approximations), then
      // the exact selection below; kRescoreChunk consecutive keys per pass, the next pass's code
      // rows loaded into registers while the current one is scored
      float* resc = cc.rescored + r * N;
      {
        const int ck = tid / kTPK;
        auto load_next = [&](int n0) -> CodeT { return key_codes(n0 + ck < nv ? n0 + ck : nv - 1); };
        CodeT nxt = load_next(0);
#pragma unroll 1
        for (int n0 = 0; n0 < nv; n0 += kRescoreChunk) {
          const int cnt = nv - n0 < kRescoreChunk ? nv - n0 : kRescoreChunk;
          stage_key(ck, nxt);
          if (n0 + kRescoreChunk < nv) nxt = load_next(n0 + kRescoreChunk);
          __syncthreads();
          exact_chunk(cnt);
          if (tid < cnt) {
            const int n = n0 + tid;
            resc[n] = cc.kscale ? sc_s[tid] * cc.kscale[bkey * N + n] : sc_s[tid];
          }
        }
      }
      __threadfence_block();
      __syncthreads();
      load_scores(resc);
      certified = false;
      continue;
    }
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
    break;
  }
  // ---- emit the selected ids in ascending order
  auto selected = [&](int j, int& slot) -> bool {
    const int n = base + j;
    if (j >= nloc) return false;
    if (CERT && band_mode) {
      if ((in_mask >> j) & 1u) return true;
      if (!((band_mask >> j) & 1u)) return false;
      const uint32_t ck = (uint32_t)(cand_pair[slot++] >> 32);
      return ck < Kt || (ck == Kt && n <= It);
    }
    return key[j] < Kt || (key[j] == Kt && n <= It);
  };
  // the selection as a bit mask, evaluated once for the count and the placement
  uint64_t selm = 0;  // PER <= 64
  int slot = slot0;
#pragma unroll
  for (int j = 0; j < PER; j++) selm |= (uint64_t)selected(j, slot) << j;
  const int nsel = __builtin_popcountll(selm);
  int tot_sel;
  int pos = block_excl_scan<kWaves>(nsel, tmp, &tot_sel);
  // ids go straight to their output positions (each wave's selected ids fill one contiguous run)
  const bool stage = false;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    if ((selm >> j) & 1ull) {
      if (pos < take) {
        if (stage) out_s[pos] = (int32_t)(base + j) + id_offset;
        else orow[pos] = (int32_t)(base + j) + id_offset;
      }
      pos++;
    }
  }
  if (stage) {
    __syncthreads();
    for (int j = tid; j < k; j += NT) orow[j] = j < take ? out_s[j] : -1;
  } else {
    for (int j = take + tid; j < k; j += NT) orow[j] = -1;
  }
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
                         int64_t out_stride, int32_t id_offset, const int32_t* wpos, int window, hipStream_t st,
                         const CertCtx* cert = nullptr);

extern "C" int smla_topk(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, void* stream) {
  if (!scores || !out) return SMLA_E_NULL;
  if (R <= 0 || N <= 0 || k <= 0 || out_stride < k) return SMLA_E_SHAPE;
  if (R > 0x7fffffff || k > 0x7fffffff) return SMLA_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  return launch_select(scores, R, N, nvis, k, out, out_stride, id_offset, nullptr, 0, st);
}

static int launch_select(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k, int32_t* out,
                         int64_t out_stride, int32_t id_offset, const int32_t* wpos, int window, hipStream_t st,
                         const CertCtx* cert) {
  const CertCtx cc = cert ? *cert : CertCtx{};
  const dim3 grid((unsigned)R);
  // 1024 threads (16 waves: the per-entry phases are VALU-bound and need the waves to hide latency)
#define SMLA_TOPK_LAUNCH(P, T)                                                                              \
  {                                                                                                      \
    if (cert)                                                                                            \
      hipLaunchKernelGGL((topk_kernel<P, true, T>), grid, dim3(T), 0, st, scores, N, nvis, (int)k, out,  \
                         out_stride, id_offset, wpos, window, cc);                                       \
    else                                                                                                 \
      hipLaunchKernelGGL((topk_kernel<P, false, T>), grid, dim3(T), 0, st, scores, N, nvis, (int)k, out, \
                         out_stride, id_offset, wpos, window, cc);                                       \
    SMLA_HIP_CHECK_LAUNCH();                                                                             \
    return SMLA_OK;                                                                                      \
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
  const int64_t R = B * S, nchunk = (N + 255) / 256;
  return (size_t)(R * N + R * nchunk) * sizeof(float);
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
  hipStream_t st = (hipStream_t)stream;
  float* approx = (float*)workspace;
  float* ebound = approx + R * N;
  const int32_t* wpos = window > 0 ? pos : nullptr;
  if (!(q_dtype == SMLA_BF16 && k_dtype == SMLA_FP8_E4M3 && Hi == 64 && Di == 64)) {
    // other shapes: the fixed-order scores themselves, then the exact selection
    const int rc = smla_indexer_score(q, q_dtype, keys, k_dtype, kscale, weights, nvis, B, S, Hi, Di, N, approx,
                                      stream);
    if (rc != SMLA_OK) return rc;
    return launch_select(approx, R, N, nvis, k, out, out_stride, id_offset, wpos, (int)window, st);
  }
  int rc = launch_indexer_cert((const uint16_t*)q, (const uint8_t*)keys, kscale, weights, nvis, B, S, N, approx,
                               ebound, st);
  if (rc != SMLA_OK) return rc;
  const CertCtx cc{ebound, (int)((N + 255) / 256), (const uint16_t*)q, (const uint8_t*)keys, kscale, weights, S,
                   (flags & SMLA_INDEX_EXACT) ? 1 : 0, approx};
  return launch_select(approx, R, N, nvis, k, out, out_stride, id_offset, wpos, (int)window, st, &cc);
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
