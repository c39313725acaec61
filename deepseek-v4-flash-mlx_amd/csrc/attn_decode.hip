// Split-K sparse decode attention over bf16 latent rows (ref_torch/sparse_attn.py:23-34 semantics;
// absorbed MLA: all heads read the same 576-wide rows, so a row is fetched once for 64 heads).
//
// One workgroup of 12 waves per (query row, split of its index list, 64-head group).  Roles:
//   * 4 score waves, one per 16-head group hg: S^T = K Q^T for a 32-row tile
//     (2 x 18 v_mfma_f32_16x16x32_bf16, rows as M, heads as N, Q^T in VGPRs), then the online
//     softmax of those 16 heads (lazy reference max) and P in bf16 to LDS, with the per-head
//     rescale factor of the tile;
//   * 8 value waves (head pair hp of 32 heads x value quarter dq of 128 columns):
//     O^T = alpha * O^T + V^T P^T with v_mfma_f32_32x32x16_bf16 (value columns as M, 32 heads as
//     N, V^T fragments by ds_read_b64_tr_b16, P^T rows straight from LDS).
// The two roles are skewed by one tile: iteration i scores tile i while the value waves consume
// tile i-1, so one workgroup barrier per tile suffices and no fp32 partial scores cross waves.
//
// Rows stream HBM -> LDS with global_load_lds_dwordx4 into a ring of 4 tiles (one instruction per
// row for columns 0..511, one per 8 rows for the 128-byte rope tails, XOR-swizzled by row; the 36
// instructions of a tile are dealt to the 8 value waves).  A tile is requested two iterations before
// it is scored.  The workgroup's 64 Q rows arrive the same way, laid out as two tiles of head rows
// in the two ring slots that are free until iteration 0, so their latency overlaps the first
// tiles' and the score waves read Q^T with the K-read pattern (free of bank conflicts).  Masked ids and rows past
// the split load row 0, so every LDS value an MFMA reads is finite.
//
// Output: final rows (one split) or (m, l, O) partial states in the layout the merge kernels read.
// bf16 partials leave the value waves' registers in MFMA fragment order (attn_merge_frag_kernel)
// with nontemporal stores: no staging through LDS, no barrier after the tile loop, and no dirty L2
// lines for the kernel's end to write back.
#include "attn_common.h"
#include "select_row.h"

namespace smla_attn {
namespace {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x4_t lds_i32x4_t;
typedef __attribute__((address_space(3))) float lds_f32_t;
typedef __attribute__((address_space(3))) u32x2_t lds_u32x2_t;

template <int D, int NBUF_, int MAXROWS_>
struct Geo6 {
  static constexpr int ROWB = D * 2;                    // bytes per bf16 row
  static constexpr bool TAIL = D > 512;
  static constexpr int MSTRIDE = 1056;                  // LDS bytes per row, columns 0..511
  static constexpr int MAIN_BYTES = kTileRows * MSTRIDE;        // 33792
  static constexpr int TAIL_BYTES = TAIL ? kTileRows * 128 : 0;  // 4096
  static constexpr int TILE_BYTES = MAIN_BYTES + TAIL_BYTES;
  static constexpr int NBUF = NBUF_;                    // ring slots (the last two stage Q first)
  static constexpr int PSTRIDE = 80;                    // bytes per head in a P buffer (32 rows + pad)
  static constexpr int PBUF = 64 * PSTRIDE;
  static constexpr int P_OFF = NBUF * TILE_BYTES;
  static constexpr int AL_OFF = P_OFF + 2 * PBUF;        // rescale factors: 2 x 64 floats
  static constexpr int IDS_OFF = AL_OFF + 2 * 64 * 4;
  static constexpr int MAX_ROWS = MAXROWS_;             // rows per split (index table in LDS; 0: none)
  static constexpr int LOOP_END = IDS_OFF + MAX_ROWS * 4;  // end of what the tile loop uses
  static constexpr int STAGE_BF16 = 64 * (1024 + 16);   // output staging after the loop
  static constexpr int STAGE_F32 = 64 * (2048 + 16);
  // (m, l) per head after the loop, past the output staging (which may reach past LOOP_END)
  static constexpr int ML_OFF = LOOP_END > STAGE_F32 ? LOOP_END : STAGE_F32;
  static constexpr int LDS_BYTES = ML_OFF + 64 * 2 * 4;
  static constexpr int NW = 12;
  static constexpr int KSTEPS = D / 32;                 // 18 / 16
  static constexpr int NDMA = kTileRows + (TAIL ? kTileRows / 8 : 0);   // 36 / 32 per tile
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static_assert(NBUF >= 3, "Q takes the last two slots; tile 0 needs one more");
  static_assert(STAGE_F32 <= ML_OFF, "output staging below the (m, l) table");
};

__device__ inline uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }

// Combine v over lanes l, l^16, l^32, l^48 (the four 16-lane rows of a wave) with the gfx950 lane
// swaps: permlane16_swap returns (even rows, odd rows) each duplicated over their pair, and
// permlane32_swap (low half, high half) likewise, so one op on the two results is the xor-16
// (resp. xor-32) step of a butterfly, in VALU registers instead of an LDS permute.
template <class Op>
__device__ inline float rows4_reduce(float v, Op op) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// The copies are dealt to the value waves only (wave 4 + v issues instructions v, v+8, v+16, ...):
// a wave whose copy waits at issue for the memory pipeline stalls with it, and the score waves
// carry the tile loop's critical path while the value waves have slack.
constexpr int kDmaWaves = 8;
template <class G>
__device__ inline int dma_count(int w) {
  return w < 4 ? 0 : (G::NDMA - (w - 4) + kDmaWaves - 1) / kDmaWaves;
}

// Workgroups are dealt to the 8 XCDs round-robin (workgroup L runs on XCD L mod 8), and each XCD
// has its own L2.  With one workgroup per query row (prefill), neighbouring rows share most of their
// window rows, so XCD x takes chunks of 128 consecutive rows: chunk position x in even rounds and
// 7 - x in odd rounds, because a row's work grows with its position and the snake keeps the XCDs
// even.  Other row counts keep the plain order.
__device__ inline int64_t query_row_of(int64_t L, int64_t n) {
  constexpr int64_t kX = 8, kC = 128;
  if (n % (kX * kC) != 0) return L;
  const int64_t x = L % kX, i = L / kX;
  const int64_t r = i / kC, j = i % kC;
  const int64_t pos = (r & 1) ? kX - 1 - x : x;
  return r * kX * kC + pos * kC + j;
}

template <int D, int NBUF, int MAXROWS, bool FP8, bool IMPL = false, int SELPER = 0>
__global__ __launch_bounds__(768) void attn_decode_kernel(
    const uint16_t* __restrict__ q, RowSrc src, const float* __restrict__ sink, const int32_t* __restrict__ idx,
    int T, int S, int H, int rows_per_split, float scale, float* __restrict__ part, void* __restrict__ out,
    int out_dtype, ImplicitRows ir, SelectRows sr) {
  using G = Geo6<D, NBUF, MAXROWS>;
  extern __shared__ __align__(16) uint8_t lds_generic[];
  lds_u8_t* lds = (lds_u8_t*)lds_generic;
  lds_i32_t* ids_s = (lds_i32_t*)(lds + G::IDS_OFF);
  lds_f32_t* al_s = (lds_f32_t*)(lds + G::AL_OFF);
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
  // every launch argument read in one round trip of scalar loads: left to the compiler, the grid
  // size, the index-list arguments and the row sources come in three dependent round trips
  {
    const uint32_t gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    asm volatile("" ::"s"(gx), "s"(gy), "s"(gz), "s"(q), "s"(src.kv0), "s"(src.kv1), "s"(src.n0), "s"(src.n1),
                 "s"(idx), "s"(T), "s"(S), "s"(H), "s"(rows_per_split), "s"(part), "s"(out), "s"(sink),
                 "s"(scale), "s"(out_dtype), "s"(ir.q_pos0), "s"(ir.window), "s"(ir.ratio), "s"(ir.enabled));
    if constexpr (SELPER > 0)
      asm volatile("" ::"s"(sr.scores), "s"(sr.nvis), "s"(sr.pos), "s"(sr.N), "s"(sr.window), "s"(sr.k));
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // grid (nsplit, B*S, head groups).  One split per query row and one head group (prefill): query
  // rows in XCD chunks (query_row_of); otherwise every split and head group of query row bs on XCD
  // bs mod 8 (when B*S is a multiple of 8), so that they share the row's q block and index list in
  // one L2
  const int nsplit = gridDim.x;
  int split = 0, hb = 0;  // hb: first head of this workgroup
  int64_t bs;
  if (nsplit == 1 && gridDim.z == 1) {
    bs = query_row_of(blockIdx.y, gridDim.y);
    if (ir.enabled) bs = gridDim.y - 1 - bs;  // prompt positions grow with s: longest lists first
  } else {
    int64_t item;
    xcd_row_item(gridDim.y, (int64_t)nsplit * gridDim.z, bs, item);
    if (gridDim.z == 1) {
      split = (int)item;
    } else {
      const uint32_t hg = (uint32_t)item / (uint32_t)nsplit;
      split = (int)((uint32_t)item - hg * nsplit);
      hb = (int)hg * 64;
    }
  }
  const int64_t b = batch_of(bs, S);
  const int nh = min(64, H - hb);                 // valid heads here
  const int t_begin = split * rows_per_split;
  const int t_end = min(T, t_begin + rows_per_split);
  const int nrows = max(0, t_end - t_begin);
  const int ntiles_all = (nrows + kTileRows - 1) / kTileRows;
  const int64_t n0 = src.n0, n1 = src.n1, ntot = n0 + n1;
  const int32_t* ig = idx ? idx + bs * (int64_t)T + t_begin : nullptr;
  // IMPL: no index table; entry e of the list of the query at position p (ImplicitRows) is
  //   e <= p - lo                       -> raw row lo + e       (window, lo = max(0, p - window + 1))
  //   window <= e < window + nc         -> compressed row e - window (id n0 + e - window)
  //   otherwise                         -> masked
  // with nc = min((p + 1) / ratio, n1), computed where it is needed, without branches
  const int64_t ip = ir.q_pos0 + (bs - b * S);
  const int64_t ilo = ip - ir.window + 1 > 0 ? ip - ir.window + 1 : 0;
  const int64_t incv = ir.ratio > 0 ? (ip + 1) / ir.ratio : 0;
  const int i_nc = (int)(incv < n1 ? incv : n1);
  const int i_wlast = (int)(ip - ilo);
  auto impl_ok = [&](int e) -> bool { return (e <= i_wlast) | ((unsigned)(e - ir.window) < (unsigned)i_nc); };
  const bool scorer = wave < 4;
  const int g = lane >> 4, c = lane & 15;

  const uint8_t* row0 = n0 > 0 ? (const uint8_t*)src.kv0 + b * n0 * (int64_t)G::ROWB
                               : (const uint8_t*)src.kv1 + b * n1 * (int64_t)G::ROWB;
  auto row_ptr = [&](int rid) -> const uint8_t* {
    const uint8_t* p0 = (const uint8_t*)src.kv0 + (b * n0 + rid) * (int64_t)G::ROWB;
    const uint8_t* p1 = (const uint8_t*)src.kv1 + (b * n1 + (rid - n0)) * (int64_t)G::ROWB;
    return rid < 0 ? row0 : (rid < n0 ? p0 : p1);
  };
  // IMPL: the row of list entry e (masked entries read row 0, like -1 ids); entry e of the window
  // is raw row lo + e, entry e of the compressed part compressed row e - window
  const uintptr_t i_wbase = (uintptr_t)src.kv0 + (uintptr_t)((b * n0 + ilo) * (int64_t)G::ROWB);
  const uintptr_t i_cbase = (uintptr_t)src.kv1 + (uintptr_t)((b * n1 - ir.window) * (int64_t)G::ROWB);
  auto impl_ptr = [&](int e) -> const uint8_t* {
    const uintptr_t a = (e < ir.window ? i_wbase : i_cbase) + (uintptr_t)((int64_t)e * G::ROWB);
    return impl_ok(e) ? (const uint8_t*)a : row0;
  };
  // this wave's share of the copies of one 32-row tile into ring slot `slot` (G::NDMA instructions
  // per tile, dealt round-robin over the value waves: one per row for columns 0..511, one per 8 rows
  // for the rope tails)
  auto issue_rows = [&](int slot, auto&& rowp, bool nt) {
    const uint32_t tbase = lds_base + (uint32_t)(slot * G::TILE_BYTES);
    if (wave < 4) return;
#pragma unroll
    for (int k = 0; k < (G::NDMA + kDmaWaves - 1) / kDmaWaves; k++) {
      const int x = wave - 4 + kDmaWaves * k;
      if (x < kTileRows) {
        const uint32_t ld = __builtin_amdgcn_readfirstlane(tbase + x * G::MSTRIDE);
        // IMPL: the row is wave-uniform; computed in scalar registers
        const int xr = IMPL ? __builtin_amdgcn_readfirstlane(x) : x;
        if (nt)
          dma16_nt(rowp(xr) + 16 * lane, ld);
        else
          dma16(rowp(xr) + 16 * lane, ld);
      } else if (x < G::NDMA) {
        const int r0 = (x - kTileRows) * 8;
        const int r = r0 + (lane >> 3);
        const int ch = (lane & 7) ^ (r & 7);  // rope tails XOR-swizzled by row
        const uint32_t ld = __builtin_amdgcn_readfirstlane(tbase + G::MAIN_BYTES + r0 * 128);
        if (nt)
          dma16_nt(rowp(r) + 1024 + 16 * ch, ld);
        else
          dma16(rowp(r) + 1024 + 16 * ch, ld);
      }
    }
  };
  // ---- the workgroup's 64 Q rows first (they do not depend on the index list, so their copies
  // overlap the id loads): two tiles of head rows in the last two ring slots, heads past H read
  // head 0
  constexpr int QS = G::NBUF - 2;  // first Q slot
  {
    const uint8_t* qrow0 = (const uint8_t*)(q + (bs * H + hb) * (int64_t)D);
    for (int qt = 0; qt < 2; qt++)
      issue_rows(
          QS + qt,
          [&](int r) {
            const int hl = 32 * qt + r;
            return qrow0 + (hl < nh ? hl : 0) * (int64_t)G::ROWB;
          },
          nsplit == 1);  // one workgroup per query row: its Q rows are read once
  }

  // ---- row ids -> LDS (-1: masked, out of range or past the split), whole tiles; the tiles
  // past the last live id are dropped (index lists padded with -1 at the end cost nothing)
  // The score waves load the table: they issue no row copies, so their id loads do not queue
  // behind the Q rows' copies (vmcnt counts in order), and the barriers below wait for LDS only.
  // Past 256 ids (one per score thread), four per thread are requested before any is written (one
  // round trip per 1024 ids; loads at clamped indexes, so none is conditional and none sinks
  // behind a wait).
  int last = -1;
  const int nt = ntiles_all * kTileRows;
  if constexpr (IMPL) {
    // the last live entry: the last visible compressed row, else the window's last (p itself)
    if (scorer) last = i_nc > 0 ? ir.window + i_nc - 1 : i_wlast;
  } else if constexpr (SELPER > 0) {
    // SelectRows: the window entries of the split, then (when the split reaches past the window)
    // the selection by the whole workgroup, its LDS in ring slot 0 (tile 0 is requested only after
    // the table is complete); each selected id lands at its list position if that is in the split
    using SL = smla_select::Lds<768>;
    static_assert(sizeof(SL) <= G::TILE_BYTES, "selection scratch fits a ring slot");
    SL& sm = *(SL*)lds_generic;
    const int p = sr.pos[bs];
    auto valid = [&](int64_t r) -> int { return (r >= 0 && r < ntot) ? (int)r : -1; };
    // window entry e: the row of position pp = p - window + 1 + e in the raw ring of n0 >= window
    // rows (row pp mod n0), -1 before the sequence start
    for (int t = tid; t < nt; t += 768) {
      const int e = t_begin + t;
      const int64_t pp = (int64_t)p - sr.window + 1 + e;
      ids_s[t] = (t < nrows && e < sr.window && pp >= 0) ? (int)((uint32_t)pp % (uint32_t)n0) : -1;
    }
    if (t_end > sr.window) {  // uniform over the workgroup
      int nv = sr.nvis ? sr.nvis[bs] : sr.N;
      nv = nv < 0 ? 0 : (nv > sr.N ? sr.N : nv);
      const int lo = t_begin - sr.window, hi = t_end - sr.window;  // selected ranks of this split
      if (nv <= sr.k) {
        // every visible row, in index order
        for (int t = tid; t < nrows; t += 768) {
          const int rk = t_begin + t - sr.window;
          if (rk >= 0 && rk < nv) ids_s[t] = valid(n0 + rk);
        }
      } else {
        const int base = tid * SELPER;
        const float* row = sr.scores + bs * (int64_t)sr.N;
        float fv[SELPER];
        if ((sr.N & 3) == 0 && base + SELPER <= sr.N) {
#pragma unroll
          for (int j = 0; j < SELPER; j += 4) {
            const f32x4_t v4 = *(const f32x4_t*)(row + base + j);
            fv[j] = v4[0];
            fv[j + 1] = v4[1];
            fv[j + 2] = v4[2];
            fv[j + 3] = v4[3];
          }
        } else {
#pragma unroll
          for (int j = 0; j < SELPER; j++) fv[j] = base + j < sr.N ? row[base + j] : 0.f;
        }
        const int nloc = nv - base < 0 ? 0 : (nv - base > SELPER ? SELPER : nv - base);
        uint32_t key[SELPER];
        uint32_t Kt;
        int It;
        smla_select::row_threshold<SELPER, 768>(fv, nloc, base, nv, sr.k, sm, key, Kt, It);
        const auto selm = smla_select::selected_mask<SELPER>(key, nloc, base, Kt, It);
        int tot;
        int rk = smla_select::block_excl_scan<12>(smla_select::sel_count<SELPER>(selm), sm.tmp, &tot);
#pragma unroll
        for (int j = 0; j < SELPER; j++) {
          if ((selm >> j) & 1u) {
            if (rk >= lo && rk < hi) ids_s[sr.window + rk - t_begin] = valid(n0 + base + j);
            rk++;
          }
        }
      }
    }
    __syncthreads();  // the table is complete; the selection scratch is no longer read
    if (scorer)
      for (int t = tid; t < nt; t += 4 * 64)
        if (ids_s[t] >= 0) last = t;
  } else if (MAXROWS <= 4 * 64 || nt <= 4 * 64) {
    if (scorer) {
      for (int t = tid; t < nt; t += 4 * 64) {
        int r = -1;
        if (t < nrows) {
          r = ig[t];
          r = (r >= 0 && r < ntot) ? r : -1;
        }
        ids_s[t] = r;
        if (r >= 0) last = t;
      }
    }
  } else if (scorer) {
    for (int t0 = tid; t0 < nt; t0 += 4 * 4 * 64) {
      int v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) v[u] = ig[min(t0 + u * 4 * 64, nrows - 1)];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int t = t0 + u * 4 * 64;
        if (t < nt) {
          int r = t < nrows ? v[u] : -1;
          r = (r >= 0 && r < ntot) ? r : -1;
          ids_s[t] = r;
          if (r >= 0) last = t;
        }
      }
    }
  }
  {
    const float wl = wave_max_dpp((float)last);
    if (lane == 0) al_s[wave] = wl;  // (the rescale buffer is free until iteration 0)
  }
  lds_barrier();
  const int last_live = (int)wave_max_dpp(lane < G::NW ? al_s[lane] : -1.f);
  const int ntiles = (last_live + kTileRows) / kTileRows;
  lds_barrier();  // al_s reads done before any later use

  auto issue_tile = [&](int tl) {
    if constexpr (!FP8) {
      if constexpr (IMPL) {
        issue_rows(tl % G::NBUF, [&](int r) { return impl_ptr(tl * kTileRows + r); }, false);
      } else {
        const lds_i32_t* tid_s = ids_s + tl * kTileRows;
        issue_rows(tl % G::NBUF, [&](int r) { return row_ptr(tid_s[r]); }, false);
      }
    }
  };
  // a data tile's DMA instructions of this wave (wave-uniform: the waits on it branch on scalars)
  const int my_dma = FP8 ? 0 : __builtin_amdgcn_readfirstlane(dma_count<G>(wave));

  // ---- fp8 rows (e4m3 codes + one fp32 power-of-two scale per 64 columns): the value waves load
  // a tile's 32 x D codes into registers (16 codes per lane-chunk, chunks dealt over the 512
  // value lanes) and write them to the ring slot as bf16 (exact: 4 significant bits times a power
  // of two), in the layout the DMA gives bf16 rows.  A wave's chunks are all main columns or all
  // rope columns (f8_chunk), so no wave runs both store paths (6 % faster on the 64-sequence fp8
  // batch than chunks dealt in row order); 8-code pieces, whose 16-byte stores are contiguous
  // over the lanes, measured 9 % slower (twice the load instructions).
  constexpr int F8_CH = D / 16;                       // 16-code chunks per row (36 / 32)
  constexpr int F8_K = (kTileRows * F8_CH + 511) / 512;  // chunks per value lane (3 / 2)
  struct F8Regs {
    u32x4_t v[F8_K];
    float s[F8_K];
  };
  // chunk k of value lane vl: k < 2 the main columns (row ci / 32, chunk ci % 32 with ci = vl + 512 k),
  // k = 2 the rope tail (lanes vl < 128: row vl / 4, chunk 32 + vl % 4), so no wave mixes the two
  auto f8_chunk = [&](int vl, int k, int& r, int& cc) -> bool {
    if (k < 2) {
      const int ci = vl + 512 * k;
      r = ci >> 5;
      cc = ci & 31;
      return true;
    }
    r = vl >> 2;
    cc = 32 + (vl & 3);
    return vl < 128;
  };
  auto f8_load = [&](int tl, F8Regs& fr) {
    const lds_i32_t* tid_s = ids_s + tl * kTileRows;
    const int vl = (wave - 4) * 64 + lane;
#pragma unroll
    for (int k = 0; k < F8_K; k++) {
      int r, cc;
      if (f8_chunk(vl, k, r, cc)) {
        const int rid = tid_s[r];
        const int64_t row = rid < 0 ? (n0 > 0 ? b * n0 : b * n1) : (rid < n0 ? b * n0 + rid : b * n1 + (rid - n0));
        const bool in0 = rid < 0 ? n0 > 0 : rid < n0;
        const uint8_t* cp = (const uint8_t*)(in0 ? src.kv0 : src.kv1) + row * D + 16 * cc;
        const float* sp = (in0 ? src.sc0 : src.sc1) + row * (D / 64) + (cc >> 2);
        fr.v[k] = *(const u32x4_t*)cp;
        fr.s[k] = *sp;
      }
    }
  };
  auto f8_store = [&](int tl, const F8Regs& fr) {
    lds_u8_t* slot = lds + (tl % G::NBUF) * G::TILE_BYTES;
    const int vl = (wave - 4) * 64 + lane;
#pragma unroll
    for (int k = 0; k < F8_K; k++) {
      int r, cc;
      if (f8_chunk(vl, k, r, cc)) {
        uint32_t w[8];
        // a normal power-of-two scale (the fp8 simulation's form): code x scale is a bf16 value,
        // which the scaled converter gives exactly, two per instruction (it applies the scale's
        // exponent only); any other scale: fp32 product rounded to bf16
        const uint32_t su = __float_as_uint(fr.s[k]);
        if ((su & 0x7fffffu) == 0 && su - 0x00800000u < 0x7f000000u) {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            w[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(fr.v[k][j], fr.s[k], false));
            w[2 * j + 1] =
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(fr.v[k][j], fr.s[k], true));
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)fr.v[k][j], false);
            const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)fr.v[k][j], true);
            w[2 * j] = pack_bf16x2(lo.x * fr.s[k], lo.y * fr.s[k]);
            w[2 * j + 1] = pack_bf16x2(hi.x * fr.s[k], hi.y * fr.s[k]);
          }
        }
        const u32x4_t w0 = {w[0], w[1], w[2], w[3]}, w1 = {w[4], w[5], w[6], w[7]};
        if (k < 2) {
          *(lds_u32x4_t*)(slot + r * G::MSTRIDE + 32 * cc) = w0;
          *(lds_u32x4_t*)(slot + r * G::MSTRIDE + 32 * cc + 16) = w1;
        } else {  // rope dims: 16-byte chunks 2(cc-32), 2(cc-32)+1 of the row's tail, swizzled
          const int l0 = 2 * (cc - 32);
          *(lds_u32x4_t*)(slot + G::MAIN_BYTES + r * 128 + 16 * (l0 ^ (r & 7))) = w0;
          *(lds_u32x4_t*)(slot + G::MAIN_BYTES + r * 128 + 16 * ((l0 + 1) ^ (r & 7))) = w1;
        }
      }
    }
  };

  // ---- prologue copies: tiles 0 .. NBUF-3 (the Q rows are already on their way)
  for (int tl = 0; tl < min(ntiles, QS); tl++) issue_tile(tl);
  F8Regs f8r;  // fp8: the value waves' registers of the next tile to write
  if constexpr (FP8) {
    if (!scorer) {
      for (int tl = 0; tl < min(ntiles, QS); tl++) {
        f8_load(tl, f8r);
        f8_store(tl, f8r);
      }
      if (QS < ntiles) f8_load(QS, f8r);
    }
  }
  // this wave's copies of Q and of tile 0 have landed (tiles 1 .. QS-1 may still fly)
  wait_vm(max(0, min(QS, ntiles) - 1) * my_dma);
  lds_barrier();

  // end of iteration it (same schedule in both roles): tile it+1 has landed, barrier, and the slot
  // of the consumed tile it-1 takes tile it+NBUF-1
  auto end_iteration = [&](int it) {
    if constexpr (!FP8) {
      if (it + 1 < ntiles) wait_vm(max(0, min(it + G::NBUF - 2, ntiles - 1) - (it + 1)) * my_dma);
    }
    lds_barrier();
    if (it + G::NBUF - 1 < ntiles) issue_tile(it + G::NBUF - 1);
  };
  lds_f32_t* ml_s = (lds_f32_t*)(lds + G::ML_OFF);  // (m, l) per head after the loop
  // output staging after the loop (the ring is free then): 64 head rows of 512 values in the output
  // element type (bf16 for bf16 output or bf16 partials, else fp32), padded against bank conflicts
  const bool out_bf16 = out_dtype == SMLA_BF16;
  // bf16 partial states: written in MFMA fragment order, no staging (attn_merge_frag_kernel)
  const bool frag_out = nsplit > 1 && out_bf16;
  const int row_bytes = out_bf16 ? 1024 : 2048;
  const int srow_bytes = row_bytes + 16;
  // the workgroup's nh x 512 output block is contiguous: final rows [bs][hb..][512] or the split's
  // partial O records [bs][split][hb..][512] (after the (m, l) records)
  auto copy_out = [&]() {
    uint8_t* dst = nsplit == 1
        ? (uint8_t*)out + (bs * H + hb) * (int64_t)row_bytes
        : (uint8_t*)(part + (int64_t)gridDim.y * H * nsplit * 2) + ((bs * nsplit + split) * (int64_t)H + hb) * row_bytes;
    const int chunks_per_row = row_bytes / 16;
    const int nchunks = nh * chunks_per_row;
    // nontemporal: neither final rows nor partial records are read back by this launch, and
    // streamed out they leave no dirty L2 lines for the kernel's end to write back
    for (int i = tid; i < nchunks; i += G::NW * 64) {
      const int hr = i / chunks_per_row, ch = i - hr * chunks_per_row;
      __builtin_nontemporal_store(*(const lds_u32x4_t*)(lds + hr * srow_bytes + ch * 16),
                                  (u32x4_t*)(dst + (int64_t)i * 16));
    }
  };

  if (scorer) {
    // ---------------- score waves: head group hg = wave
    const int hg = wave;
    // Q^T B operand from the Q tiles: head row hg*16 + c, K-step j holds elements 32j + 8g .. +7
    bf16x8_t qf[G::KSTEPS];
    {
      const lds_u8_t* qb = lds + (QS + (hg >> 1)) * G::TILE_BYTES;
      const int qr = (hg & 1) * 16 + c;
#pragma unroll
      for (int j = 0; j < G::KSTEPS; j++) {
        if (!G::TAIL || j < 16) {
          qf[j] = as_bf16x8(*(const lds_u32x4_t*)(qb + qr * G::MSTRIDE + 16 * g + 64 * j));
        } else {
          const int lch = 4 * (j - 16) + g;
          qf[j] = as_bf16x8(*(const lds_u32x4_t*)(qb + G::MAIN_BYTES + qr * 128 + 16 * (lch ^ (qr & 7))));
        }
      }
    }
    lds_barrier();  // Q slots free: they take tiles QS and QS+1 in turn
    if (ntiles > QS) issue_tile(QS);
    float m_ref = -SMLA_INF, l_lane = 0.f;
    const int kq_off = c * G::MSTRIDE + 16 * g;  // A operand, row c (block 0)
    for (int it = 0; it <= ntiles; it++) {
      if (it < ntiles) {
        const lds_u8_t* buf = lds + (it % G::NBUF) * G::TILE_BYTES;
        // K-operand reads run PF K-steps ahead of the MFMAs
        auto ldk = [&](int j, int blk) -> u32x4_t {
          if (!G::TAIL || j < 16) return *(const lds_u32x4_t*)(buf + kq_off + blk * 16 * G::MSTRIDE + 64 * j);
          const int r = 16 * blk + c, lch = 4 * (j - 16) + g;
          return *(const lds_u32x4_t*)(buf + G::MAIN_BYTES + r * 128 + 16 * (lch ^ (r & 7)));
        };
        constexpr int PF = 6;
        u32x4_t ka[PF], kb[PF];
#pragma unroll
        for (int j = 0; j < PF; j++) {
          ka[j] = ldk(j, 0);
          kb[j] = ldk(j, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int j = 0; j < G::KSTEPS; j++) {
          const u32x4_t a0 = ka[j % PF], a1 = kb[j % PF];
          if (j + PF < G::KSTEPS) {
            ka[j % PF] = ldk(j + PF, 0);
            kb[j % PF] = ldk(j + PF, 1);
          }
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), qf[j], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), qf[j], s1, 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);  // keep the reads PF steps ahead of their MFMAs
        }
        // online softmax over rows 4g+i and 16+4g+i for head hg*16 + c
        float x[8];
        if constexpr (IMPL) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            x[i] = impl_ok(it * kTileRows + 4 * g + i) ? s0[i] * scale : -SMLA_INF;
            x[4 + i] = impl_ok(it * kTileRows + 16 + 4 * g + i) ? s1[i] * scale : -SMLA_INF;
          }
        } else {
          const lds_i32_t* tid_s = ids_s + it * kTileRows;
          const i32x4_t v0 = *(const lds_i32x4_t*)(tid_s + 4 * g);
          const i32x4_t v1 = *(const lds_i32x4_t*)(tid_s + 16 + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            x[i] = v0[i] >= 0 ? s0[i] * scale : -SMLA_INF;
            x[4 + i] = v1[i] >= 0 ? s1[i] * scale : -SMLA_INF;
          }
        }
        float mt = x[0];
#pragma unroll
        for (int i = 1; i < 8; i++) mt = fmaxf(mt, x[i]);
        mt = rows4_reduce(mt, [](float x, float y) { return fmaxf(x, y); });
        float alpha = 1.f;
        if ((mt > m_ref + kRescaleSlack) || (m_ref == -SMLA_INF && mt > -SMLA_INF)) {
          alpha = (m_ref > -SMLA_INF) ? __expf(m_ref - mt) : 0.f;
          l_lane *= alpha;
          m_ref = mt;
        }
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float e = (m_ref > -SMLA_INF) ? __expf(x[i] - m_ref) : 0.f;
          p[i] = bf16_round(e);
          l_lane += p[i];
        }
        lds_u8_t* pb = lds + G::P_OFF + (it & 1) * G::PBUF + (hg * 16 + c) * G::PSTRIDE;
        *(lds_u32x2_t*)(pb + 8 * g) = u32x2_t{pack2(p[0], p[1]), pack2(p[2], p[3])};
        *(lds_u32x2_t*)(pb + 32 + 8 * g) = u32x2_t{pack2(p[4], p[5]), pack2(p[6], p[7])};
        if (g == 0) al_s[(it & 1) * 64 + hg * 16 + c] = alpha;
      }
      end_iteration(it);
    }
    // publish (m, l) per head: to LDS for the value waves' final scaling, and as the partial state
    const float l_tot = rows4_reduce(l_lane, [](float x, float y) { return x + y; });
    const int hl = hg * 16 + c;
    if (g == 0) {
      ml_s[hl * 2] = m_ref;
      ml_s[hl * 2 + 1] = l_tot;
      if (nsplit > 1 && hl < nh) {
        const int64_t rec = (bs * nsplit + split) * (int64_t)H + hb + hl;
        *(f32x2_t*)(part + rec * 2) = f32x2_t{m_ref, l_tot};
      }
    }
    if (frag_out) return;  // the value waves write their partial O without these values
    lds_barrier();  // (m, l) in LDS
    lds_barrier();  // the value waves' output block is staged
    copy_out();
    return;
  }

  // ---------------- value waves: head pair hp (32 heads) x value quarter dq (128 columns)
  const int vw = wave - 4;
  const int hp = vw & 1, dq = vw >> 1;
  lds_barrier();  // pairs with the score waves' barrier after their Q^T reads
  if (ntiles > QS) issue_tile(QS);
  f32x16_t o[4];
#pragma unroll
  for (int mb = 0; mb < 4; mb++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[mb][r] = 0.f;
  // V^T provider address inside a 16-row K-step: group j = lane>>4 covers value columns
  // 16*(j&1).. of a 32-column block and rows 8*(j>>1).. ; lane J = lane&15 supplies row J>>2,
  // columns 4*(J&3)..+3
  const int vj = lane >> 4, vJ = lane & 15;
  const int tr_off = (8 * (vj >> 1) + (vJ >> 2)) * G::MSTRIDE + 2 * (128 * dq + 16 * (vj & 1) + 4 * (vJ & 3));
  const int pr_off = (32 * hp + (lane & 31)) * G::PSTRIDE + 16 * (lane >> 5);  // P^T B operand
  for (int it = 0; it <= ntiles; it++) {
    if constexpr (FP8) {
      // tile it+NBUF-2 goes to the slot of tile it-2 (consumed before the last barrier); it is
      // scored NBUF-2 iterations later.  Then the next tile's codes are requested.
      if (it + G::NBUF - 2 < ntiles) {
        f8_store(it + G::NBUF - 2, f8r);
        if (it + G::NBUF - 1 < ntiles) f8_load(it + G::NBUF - 1, f8r);
      }
    }
    if (it >= 1) {
      const int tp = it - 1;  // tile consumed this iteration (scored in the previous one)
      const lds_u8_t* buf = lds + (tp % G::NBUF) * G::TILE_BYTES;
      const float a = al_s[(tp & 1) * 64 + 32 * hp + (lane & 31)];
      if (__builtin_amdgcn_ballot_w64(a != 1.f)) {
#pragma unroll
        for (int mb = 0; mb < 4; mb++) o[mb] *= a;
      }
      const lds_u8_t* pb = lds + G::P_OFF + (tp & 1) * G::PBUF + pr_off;
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const bf16x8_t pf = as_bf16x8(*(const lds_u32x4_t*)(pb + 32 * ks));
        const lds_u8_t* vb = buf + tr_off + 16 * ks * G::MSTRIDE;
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
          const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(vb + 64 * mb));
          const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(vb + 64 * mb + 4 * G::MSTRIDE));
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pf, o[mb], 0, 0, 0);
        }
      }
    }
    end_iteration(it);
  }
  if (frag_out) {
    // bf16 partial O^T straight from the accumulators: block (query row, split, head group) of
    // 64 KB holds, for value wave vw (head pair hp, value quarter dq), value block mb and half h,
    // 1 KB pieces at ((vw * 4 + mb) * 2 + h) * 1024 in which lane l's 16 bytes are the 8 values
    // 128 dq + 32 mb + 16 h + 8 (l >> 5) .. +7 of head 32 hp + (l & 31).  The accumulator holds
    // value columns 8 (r >> 2) + 4 (l >> 5) + (r & 3) of register r; one lane swap per register
    // pair gives each lane 8 contiguous columns.  Nontemporal stores: the merge launch reads the
    // partials from memory either way (the L2 does not keep a kernel's written lines for the next
    // launch), and streamed out they leave no dirty lines for the kernel's end to write back
    // (split kernel 13.5 -> 11.7 us at 8 x 23 splits; sc1 stores 12.8 us, plain ones 13.5 us).
    uint8_t* blk = (uint8_t*)(part + (int64_t)gridDim.y * H * nsplit * 2) +
                   ((bs * nsplit + split) * (int64_t)gridDim.z + (hb >> 6)) * 65536 + (int64_t)vw * 8192 + 16 * lane;
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
      uint32_t d[8];
#pragma unroll
      for (int k = 0; k < 8; k++) d[k] = pack2(o[mb][2 * k], o[mb][2 * k + 1]);
#pragma unroll
      for (int k = 0; k < 8; k += 4) {
        // lanes 32-63 of d[k], d[k+1] <-> lanes 0-31 of d[k+2], d[k+3]
        const auto s0 = __builtin_amdgcn_permlane32_swap(d[k], d[k + 2], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(d[k + 1], d[k + 3], false, false);
        const u32x4_t v4 = {s0[0], s1[0], s0[1], s1[1]};
        __builtin_nontemporal_store(v4, (u32x4_t*)(blk + (mb * 2 + (k >> 2)) * 1024));
      }
    }
    return;
  }
  lds_barrier();  // the score waves' (m, l) are in LDS

  // ---- epilogue: this wave's O^T block (value columns 128dq.. of 32 heads) -> LDS staging rows,
  // then all waves copy the workgroup's contiguous output block out with 16-byte stores
  {
    const int hl = 32 * hp + (lane & 31);  // head within the workgroup
    const float M = ml_s[hl * 2], L = ml_s[hl * 2 + 1];
    const bool empty = !(M > -SMLA_INF);
    float inv = 1.f;
    if (nsplit == 1) {
      const float snk = (sink && hl < nh) ? sink[hb + hl] : -SMLA_INF;
      inv = empty ? 0.f : 1.0f / (L + __expf(snk - M));
    }
    const bool nan_out = nsplit == 1 && empty;
    const int dvb = 128 * dq + 4 * (lane >> 5);  // + 32 mb + 8 qd + (r & 3)
    lds_u8_t* srow = lds + hl * srow_bytes;
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
      for (int qd = 0; qd < 4; qd++) {
        const int dv = dvb + 32 * mb + 8 * qd;
        const f32x4_t v = f32x4_t{o[mb][4 * qd], o[mb][4 * qd + 1], o[mb][4 * qd + 2], o[mb][4 * qd + 3]} * inv;
        if (out_bf16) {
          const uint32_t w0 = nan_out ? 0x7fc07fc0u : pack2(v[0], v[1]);
          const uint32_t w1 = nan_out ? 0x7fc07fc0u : pack2(v[2], v[3]);
          *(lds_u32x2_t*)(srow + 2 * dv) = u32x2_t{w0, w1};
        } else {
          const float nan = __builtin_nanf("");
          *(lds_f32x4_t*)(srow + 4 * dv) = nan_out ? f32x4_t{nan, nan, nan, nan} : v;
        }
      }
  }
  lds_barrier();
  copy_out();
}

template <int D, int NBUF, int MAXROWS, bool FP8, bool IMPL = false, int SELPER = 0>
int launch6(int nsplit, int rows_per_split, const void* q, RowSrc src, const float* sink, const int32_t* idx,
            int64_t T, int64_t B, int64_t S, int64_t H, float scale, void* out, int out_dtype, float* part,
            hipStream_t stream, ImplicitRows ir, SelectRows sr = SelectRows{}) {
  using G = Geo6<D, NBUF, MAXROWS>;
  auto kern = attn_decode_kernel<D, NBUF, MAXROWS, FP8, IMPL, SELPER>;
  static std::atomic<uint64_t> lds_attr{0};  // devices whose limit is raised
  if (hipError_t e = smla_set_dynamic_lds((const void*)kern, G::LDS_BYTES, lds_attr); e != hipSuccess) return (int)e;
  dim3 grid((unsigned)nsplit, (unsigned)(B * S), (unsigned)((H + 63) / 64));
  hipLaunchKernelGGL(kern, grid, dim3(G::NW * 64), G::LDS_BYTES, stream, (const uint16_t*)q, src, sink, idx, (int)T,
                     (int)S, (int)H, rows_per_split, scale, part, out, out_dtype, ir, sr);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

}  // namespace

// rows_per_split <= 256: 4-slot ring (deeper prefetch, for the short splits of decode);
// otherwise a 3-slot ring and an index table of up to 8192 rows (one split per query: prefill,
// long single-sequence lists)
int launch_decode_v6(int D, bool kv_fp8, int nsplit, int rows_per_split, const void* q, RowSrc src,
                     const float* sink, const int32_t* idx, int64_t T, int64_t B, int64_t S, int64_t H, float scale,
                     void* out, int out_dtype, float* part, hipStream_t stream, ImplicitRows ir,
                     SelectRows sr) {
  // decode lists selected in the kernel (SelectRows): bf16 rows, short splits (the 4-slot ring)
  if (sr.enabled) {
    const int per = select_per(sr.N);
    if (kv_fp8 || per == 0 || rows_per_split > kDecodeV6ShortRows || rows_per_split % kTileRows != 0 ||
        B * S > 65535 || T != (int64_t)sr.window + sr.k)
      return SMLA_E_UNSUPPORTED;
#define SMLA_V6S(DD, P)                                                                                            \
  return launch6<DD, 4, kDecodeV6ShortRows, false, false, P>(nsplit, rows_per_split, q, src, sink, nullptr, T, B, S, \
                                                             H, scale, out, out_dtype, part, stream, ir, sr);
    if (D == 576) {
      if (per == 12) SMLA_V6S(576, 12) else SMLA_V6S(576, 24)
    }
    if (D == 512) {
      if (per == 12) SMLA_V6S(512, 12) else SMLA_V6S(512, 24)
    }
#undef SMLA_V6S
    return SMLA_E_UNSUPPORTED;
  }
  // prefill with implicit row sets: no index table (any list length), one split per query; the
  // 3-slot ring (a 4th slot measured slower: 0.46 vs 0.45 ms over the 4096-query prompt)
  if (ir.enabled) {
    if (kv_fp8 || nsplit != 1 || rows_per_split % kTileRows != 0 || B * S > 65535) return SMLA_E_UNSUPPORTED;
    if (D == 576)
      return launch6<576, 3, 0, false, true>(1, rows_per_split, q, src, sink, idx, T, B, S, H, scale, out, out_dtype,
                                             part, stream, ir);
    if (D == 512)
      return launch6<512, 3, 0, false, true>(1, rows_per_split, q, src, sink, idx, T, B, S, H, scale, out, out_dtype,
                                             part, stream, ir);
    return SMLA_E_UNSUPPORTED;
  }
  if (rows_per_split > kDecodeV6MaxRows || rows_per_split % kTileRows != 0 || B * S > 65535) return SMLA_E_UNSUPPORTED;
  const bool sh = rows_per_split <= kDecodeV6ShortRows;
#define SMLA_V6(DD, F8)                                                                                           \
  return sh ? launch6<DD, 4, kDecodeV6ShortRows, F8>(nsplit, rows_per_split, q, src, sink, idx, T, B, S, H, scale, \
                                                     out, out_dtype, part, stream, ir)                             \
            : launch6<DD, 3, kDecodeV6MaxRows, F8>(nsplit, rows_per_split, q, src, sink, idx, T, B, S, H, scale,   \
                                                   out, out_dtype, part, stream, ir);
  if (D == 576) {
    if (kv_fp8) SMLA_V6(576, true) else SMLA_V6(576, false)
  }
  if (D == 512) {
    if (kv_fp8) SMLA_V6(512, true) else SMLA_V6(512, false)
  }
#undef SMLA_V6
  return SMLA_E_UNSUPPORTED;
}

}  // namespace smla_attn
