// Split-K sparse decode attention over bf16 latent rows (the HBM-bound gather).
//
// One workgroup of 16 waves per (query row, split of the index list, 64-head group).  Many waves
// per CU are what keeps enough row gathers in flight to approach HBM bandwidth; the work is cut
// so that each wave needs few registers.
//
//  * Tiles of 32 gathered rows are copied HBM -> LDS with global_load_lds_dwordx4 into a ring of
//    3 tile buffers: one instruction moves the first 1024 bytes (value columns 0..511) of one
//    row, with the row address in scalar registers; for 576-wide rows one more instruction per 8
//    rows moves their 128-byte rope tails.  Row stride in LDS is 1056 B (measured free of bank
//    conflicts for both read patterns below); rope tails are XOR-swizzled by row.
//  * Wave w = (head group hq = w>>2: 16 heads, one MFMA N-tile; quarter qt = w&3).  Quarter qt
//    computes the partial S^T = K Q^T over its quarter of the q.k K-steps
//    (v_mfma_f32_16x16x32_bf16, rows as M, heads as N, its Q^T slice in VGPRs); the 4 partials
//    meet through LDS and are summed in a fixed order, so all 4 waves hold bit-identical scores
//    and run the identical online softmax; quarter qt accumulates O^T = V^T P^T for value columns
//    [128qt, 128qt+128).  V^T fragments come from the row-major tile via ds_read_b64_tr_b16; the
//    K-order of P.V is chosen so that each lane's S^T accumulators are its P^T operand.
//  * The reference max of the online softmax moves only when exceeded by more than 8 (exact:
//    numerator and denominator share it).
//  * Nothing the compiler tracks is in flight while tiles stream: the prologue's vector loads
//    (row ids; Q^T via untracked asm loads) complete first or are covered by the tile waits.
//  * Output: final rows (one split) or (m, l, O) partial states for attn_merge_kernel.
#include "attn_common.h"

namespace smla_attn {
namespace {

template <int D>
struct Geo {
  static constexpr int ROWB = D * 2;                    // bytes per bf16 row
  static constexpr bool TAIL = D > 512;                 // 576: 64-wide rope tail beyond column 512
  static constexpr int MSTRIDE = 1056;                  // LDS bytes per row, columns 0..511
  static constexpr int MAIN_BYTES = kTileRows * MSTRIDE;   // 33792
  static constexpr int TAIL_BYTES = TAIL ? kTileRows * 128 : 0;
  static constexpr int TILE_BYTES = MAIN_BYTES + TAIL_BYTES;
  static constexpr int NBUF = 3;
  static constexpr int NW = 16;                              // waves per workgroup
  static constexpr int XS_OFF = NBUF * TILE_BYTES;           // S^T partial exchange: 16 waves x 2 KiB
  static constexpr int IDS_OFF = XS_OFF + NW * 2048;
  static constexpr int LDS_BYTES = IDS_OFF + kDecodeMaxRowsPerSplit * 4;
  static constexpr int KSTEPS = D / 32;                 // 18 / 16
  static constexpr int KQ = (KSTEPS + 3) / 4;           // max K-steps per quarter (5 / 4)
  static constexpr int NDMA = kTileRows + (TAIL ? kTileRows / 8 : 0);   // DMA instructions per tile
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  // K-steps of quarter qt: [kbeg(qt), kbeg(qt+1)); 576: 5,5,4,4; 512: 4,4,4,4
  __device__ static constexpr int kbeg(int qt) {
    return qt * (KSTEPS / 4) + (qt < (KSTEPS % 4) ? qt : (KSTEPS % 4));
  }
};

template <int D>
__global__ __launch_bounds__(1024, 1) void attn_decode_bf16_kernel(
    const uint16_t* __restrict__ q, RowSrc src, const float* __restrict__ sink, const int32_t* __restrict__ idx,
    int T, int S, int H, int rows_per_split, float scale, float* __restrict__ part, void* __restrict__ out,
    int out_dtype) {
  using G = Geo<D>;
  extern __shared__ __align__(16) uint8_t lds_generic[];
  lds_u8_t* lds = (lds_u8_t*)lds_generic;
  lds_i32_t* ids_s = (lds_i32_t*)(lds + G::IDS_OFF);
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int hq = wave >> 2, qt = wave & 3;
  const int split = blockIdx.x, nsplit = gridDim.x;
  const int64_t bs = blockIdx.y;
  const int64_t b = bs / S;
  const int t_begin = split * rows_per_split;
  const int t_end = min(T, t_begin + rows_per_split);
  const int nrows = t_end - t_begin;
  const int ntiles = (nrows + kTileRows - 1) / kTileRows;
  const int64_t n0 = src.n0, n1 = src.n1, ntot = n0 + n1;
  const int32_t* ig = idx + bs * (int64_t)T + t_begin;

  // ---- Q^T slice first (untracked loads; their latency overlaps the row-id fetch and they are
  // complete by the first tile wait): head h0 + c, K-steps kb .. kb+nk-1 of this quarter,
  // elements 32j + 8g .. +7
  const int head = blockIdx.z * 64 + hq * 16 + c;
  const bool head_ok = head < H;
  const int kb = G::kbeg(qt), nk = G::kbeg(qt + 1) - kb;
  bf16x8_t qf[G::KQ];
  {
    const uint16_t* qh = q + (bs * H + (head_ok ? head : H - 1)) * (int64_t)D + 32 * kb + 8 * g;
#pragma unroll
    for (int j = 0; j < G::KQ; j++)
      qf[j] = as_bf16x8(j < nk ? load16_untracked(qh + 32 * j) : u32x4_t{0u, 0u, 0u, 0u});
  }
  // ---- row ids of this split -> LDS (-1 for masked / out-of-range)
  for (int t = tid; t < nrows; t += G::NW * 64) {
    const int r = ig[t];
    ids_s[t] = (r >= 0 && r < ntot) ? r : -1;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): ids (and the Q loads issued before them)
  lds_barrier();

  const uint8_t* dummy = n0 > 0 ? (const uint8_t*)src.kv0 + b * n0 * (int64_t)G::ROWB
                                : (const uint8_t*)src.kv1 + b * n1 * (int64_t)G::ROWB;
  auto row_ptr = [&](int t_local) -> const uint8_t* {
    const int rid = ids_s[t_local];
    if (rid < 0) return dummy;
    if (rid < n0) return (const uint8_t*)src.kv0 + (b * n0 + rid) * (int64_t)G::ROWB;
    return (const uint8_t*)src.kv1 + (b * n1 + (rid - n0)) * (int64_t)G::ROWB;
  };
  // DMA of one tile; instructions are dealt round-robin to the waves.  Returns this wave's
  // instruction count.
  auto issue_tile = [&](int tl) -> int {
    const int rows_in_tile = min(kTileRows, nrows - tl * kTileRows);
    const uint32_t tbase = lds_base + (uint32_t)((tl % G::NBUF) * G::TILE_BYTES);
    int cnt = 0;
    for (int x = wave; x < G::NDMA; x += G::NW) {
      // rows past the split end load a real row too (masked by the softmax): every LDS value the
      // MFMAs read must be finite, since 0 * NaN from a stale row would poison the output
      if (x < kTileRows) {
        const int r = x;
        const uint8_t* rp = (r < rows_in_tile) ? row_ptr(tl * kTileRows + r) : dummy;
        dma16(rp + 16 * lane, __builtin_amdgcn_readfirstlane(tbase + r * G::MSTRIDE));
      } else {
        const int r0 = (x - kTileRows) * 8;
        const int r = r0 + (lane >> 3);
        const uint8_t* rp = (r < rows_in_tile) ? row_ptr(tl * kTileRows + r) : dummy;
        const int ch = (lane & 7) ^ (r & 7);
        dma16(rp + 1024 + 16 * ch, __builtin_amdgcn_readfirstlane(tbase + G::MAIN_BYTES + r0 * 128));
      }
      cnt++;
    }
    return cnt;
  };

  int cnt[G::NBUF] = {0, 0, 0};
  for (int tl = 0; tl < min(ntiles, G::NBUF); tl++) cnt[tl] = issue_tile(tl);

  f32x4_t o[8];
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_ref = -SMLA_INF, l_lane = 0.f;

  // per-lane LDS offsets
  const int kq_off = c * G::MSTRIDE + 16 * g;                 // QK A operand, main region, row c
  const int kt_off = G::MAIN_BYTES + c * 128;                  // rope tail region, row c
  const int j16 = lane & 15;
  const int prow = 4 * g + (j16 >> 2);
  const int tr_off = prow * G::MSTRIDE + 16 * ((j16 & 3) >> 1) + 8 * (j16 & 1) +
                     qt * 256;                                  // value columns [128 qt, ...)
  lds_f32x4_t* xs_w = (lds_f32x4_t*)(lds + G::XS_OFF + wave * 2048) + lane;
  const lds_f32x4_t* xs_g = (const lds_f32x4_t*)(lds + G::XS_OFF + hq * 4 * 2048) + lane;

  for (int it = 0; it < ntiles; it++) {
    int after = 0;
    const int last_issued = (it == 0) ? min(ntiles, G::NBUF) - 1 : min(ntiles - 1, it + G::NBUF - 2);
    for (int t2 = it + 1; t2 <= last_issued; t2++) after += cnt[t2 % G::NBUF];
    wait_vm(after);
    lds_barrier();
    if (it >= 1 && it + G::NBUF - 1 < ntiles) cnt[(it + G::NBUF - 1) % G::NBUF] = issue_tile(it + G::NBUF - 1);

    const lds_u8_t* buf = lds + (it % G::NBUF) * G::TILE_BYTES;
    const int rows_in_tile = min(kTileRows, nrows - it * kTileRows);
    // ---- partial S^T over this quarter's K-steps: rows {c, 16+c} x heads of this group
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int jj = 0; jj < G::KQ; jj++) {
      if (jj < nk) {
        const int j = kb + jj;  // global K-step (uniform per wave)
        u32x4_t a0w, a1w;
        if (!G::TAIL || j < 16) {
          a0w = *(const lds_u32x4_t*)(buf + kq_off + 64 * j);
          a1w = *(const lds_u32x4_t*)(buf + kq_off + 16 * G::MSTRIDE + 64 * j);
        } else {
          const int lch = 4 * (j - 16) + g;  // logical 16-byte chunk of the 128-byte tail
          a0w = *(const lds_u32x4_t*)(buf + kt_off + 16 * (lch ^ (c & 7)));
          a1w = *(const lds_u32x4_t*)(buf + kt_off + 16 * 128 + 16 * (lch ^ ((16 + c) & 7)));
        }
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0w), qf[jj], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1w), qf[jj], s1, 0, 0, 0);
      }
    }
    // ---- publish the partial; sum the group's 4 partials in quarter order (bit-identical in
    // all 4 waves of the group)
    xs_w[0] = s0;
    xs_w[64] = s1;
    lds_barrier();
    s0 = xs_g[0];
    s1 = xs_g[64];
#pragma unroll
    for (int k = 1; k < 4; k++) {
      s0 += xs_g[k * 128];
      s1 += xs_g[k * 128 + 64];
    }

    // ---- online softmax over this lane's rows 4g+i and 16+4g+i for head c
    const lds_i32_t* tid_s = ids_s + it * kTileRows;
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r0 = 4 * g + i, r1 = 16 + 4 * g + i;
      x[i] = (r0 < rows_in_tile && tid_s[r0] >= 0) ? s0[i] * scale : -SMLA_INF;
      x[4 + i] = (r1 < rows_in_tile && tid_s[r1] >= 0) ? s1[i] * scale : -SMLA_INF;
    }
    float mt = x[0];
#pragma unroll
    for (int i = 1; i < 8; i++) mt = fmaxf(mt, x[i]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const bool need = (mt > m_ref + kRescaleSlack) || (m_ref == -SMLA_INF && mt > -SMLA_INF);
    if (__builtin_amdgcn_ballot_w64(need)) {
      if (need) {
        const float alpha = (m_ref > -SMLA_INF) ? __expf(m_ref - mt) : 0.f;
        l_lane *= alpha;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] *= alpha;
        m_ref = mt;
      }
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float e = (m_ref > -SMLA_INF) ? __expf(x[i] - m_ref) : 0.f;
      p[i] = bf16_round(e);
      l_lane += p[i];
    }
    const bf16x8_t pb = as_bf16x8(u32x4_t{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                                          pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])});
    // ---- O^T[128 qt .. +128) += V^T P^T
    const lds_u8_t* tr0 = buf + tr_off;
    const lds_u8_t* tr1 = tr0 + 16 * G::MSTRIDE;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(tr0 + 32 * i));
      const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(tr1 + 32 * i));
      const bf16x8_t a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[i], 0, 0, 0);
    }
  }

  // ---- write out: value columns [128 qt, +128) of head h
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!head_ok) return;
  const bool empty = !(m_ref > -SMLA_INF);
  if (nsplit == 1) {
    const float snk = sink ? sink[head] : -SMLA_INF;
    const float inv = empty ? 0.f : 1.0f / (l_tot + __expf(snk - m_ref));
    const int64_t obase = (bs * H + head) * 512 + 128 * qt;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t dv = obase + 16 * i + 4 * g;
      if (out_dtype == SMLA_BF16) {
        const uint32_t w0 = empty ? 0x7fc07fc0u : pack_bf16x2(o[i][0] * inv, o[i][1] * inv);
        const uint32_t w1 = empty ? 0x7fc07fc0u : pack_bf16x2(o[i][2] * inv, o[i][3] * inv);
        *(u32x2_t*)((uint16_t*)out + dv) = u32x2_t{w0, w1};
      } else {
        const float nan = __builtin_nanf("");
        *(f32x4_t*)((float*)out + dv) = empty ? f32x4_t{nan, nan, nan, nan} : o[i] * inv;
      }
    }
  } else {
    const int64_t rec = (bs * nsplit + split) * H + head;  // split-major partial records
    if (g == 0 && qt == 0) {
      part[rec * 2] = m_ref;
      part[rec * 2 + 1] = l_tot;
    }
    const int64_t obase = (int64_t)gridDim.y * H * nsplit * 2;  // O records follow the (m, l) records
    if (out_dtype == SMLA_BF16) {
      // bf16 partial O (the output is bf16 anyway): half the store and merge traffic
      uint16_t* op = (uint16_t*)(part + obase) + rec * 512 + 128 * qt;
#pragma unroll
      for (int i = 0; i < 8; i++)
        *(u32x2_t*)(op + 16 * i + 4 * g) = u32x2_t{pack_bf16x2(o[i][0], o[i][1]), pack_bf16x2(o[i][2], o[i][3])};
    } else {
      float* op = part + obase + rec * 512 + 128 * qt;
#pragma unroll
      for (int i = 0; i < 8; i++) *(f32x4_t*)(op + 16 * i + 4 * g) = o[i];
    }
  }
}

template <int D>
int launch_d(int nsplit, int rows_per_split, const void* q, RowSrc src, const float* sink, const int32_t* idx,
             int64_t T, int64_t B, int64_t S, int64_t H, float scale, void* out, int out_dtype, float* part,
             hipStream_t stream, hipEvent_t ev_before, hipEvent_t ev_after) {
  using G = Geo<D>;
  auto kern = attn_decode_bf16_kernel<D>;
  static std::atomic<uint64_t> lds_attr{0};  // devices whose limit is raised
  if (hipError_t e = smla_set_dynamic_lds((const void*)kern, G::LDS_BYTES, lds_attr); e != hipSuccess) return (int)e;
  dim3 grid((unsigned)nsplit, (unsigned)(B * S), (unsigned)((H + 63) / 64));
  if (ev_before) (void)hipEventRecord(ev_before, stream);
  hipLaunchKernelGGL(kern, grid, dim3(G::NW * 64), G::LDS_BYTES, stream, (const uint16_t*)q, src, sink, idx, (int)T,
                     (int)S, (int)H, rows_per_split, scale, part, out, out_dtype);
  SMLA_HIP_CHECK_LAUNCH();
  if (ev_after) (void)hipEventRecord(ev_after, stream);
  return SMLA_OK;
}

}  // namespace

int launch_decode_bf16(int D, int nsplit, int rows_per_split, const void* q, RowSrc src, const float* sink,
                       const int32_t* idx, int64_t T, int64_t B, int64_t S, int64_t H, float scale, void* out,
                       int out_dtype, float* part, hipStream_t stream, hipEvent_t ev_before, hipEvent_t ev_after) {
  if (rows_per_split > kDecodeMaxRowsPerSplit) return SMLA_E_UNSUPPORTED;
  if (D == 576)
    return launch_d<576>(nsplit, rows_per_split, q, src, sink, idx, T, B, S, H, scale, out, out_dtype, part, stream,
                         ev_before, ev_after);
  if (D == 512)
    return launch_d<512>(nsplit, rows_per_split, q, src, sink, idx, T, B, S, H, scale, out, out_dtype, part, stream,
                         ev_before, ev_after);
  return SMLA_E_UNSUPPORTED;
}

}  // namespace smla_attn
