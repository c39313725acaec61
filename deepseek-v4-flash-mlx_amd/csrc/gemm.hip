// Tiled MFMA GEMM for the projections at prefill sizes (more than 32 token rows):
//   y[t, g*N + n] = sum_k x[t, g*K + k] * w[g*N + n, k]      (v4mlx/mla.py:16-18, and the grouped
//   product of v4mlx/mla.py:49-53 for G > 1; ref_torch/compressor.py:28-29 with fp32 operands)
//
// Both operands are K-contiguous (x rows, w rows), which is the operand order of the gfx950 MFMA:
// a lane's A fragment is 8 consecutive k of one token row, its B fragment 8 consecutive k of one
// weight row.  A workgroup of 4 waves computes a 128 (tokens) x 128 (outputs) tile, each wave a
// 64 x 64 quarter as 2 x 2 blocks of v_mfma_f32_32x32x16_bf16 (bf16 operands) or
// v_mfma_f32_32x32x2f32 (fp32 operands), accumulating in fp32.  K advances in steps of 128 bytes
// per row (64 bf16 / 32 fp32): the next step's tiles are loaded into registers while the current
// ones are multiplied out of LDS, two LDS stages, one barrier per step.  LDS rows are padded to
// 144 bytes so the 16-byte fragment reads of 32 consecutive rows spread over the banks.
// Rows past T or N are loaded clamped (finite) and never stored; K is a multiple of 16 bytes, and
// the 16-byte chunks of the last step that lie past K are zero.
//
// ROPE (bf16, the attention output projection of oracle/decode_engine.py:118-119): the K step that
// holds the last rd = 64 dims of a head has its (x0, x1) pairs rotated back to position 0 while it
// is loaded (inverse RoPE at pos[t], every product and sum rounded in float32, then bf16), the
// arithmetic of smla_rope.
//
// Large bf16 products (gemm_dma_kernel: K a multiple of 64 and enough 256 x 256 tiles for every
// CU, else 128 x 128 tiles of 4 waves, two workgroups per CU, when those suffice):
// 8 waves per 256 x 256 workgroup, each a 128 x 64 quarter-octant as 4 x 2 blocks of
// v_mfma_f32_32x32x16_bf16.  Operands go HBM -> LDS by global_load_lds_dwordx4 (no register
// staging) into a ring of two 64 KB stages; a K step (64 k) is 32 MFMAs per wave, two waves per
// SIMD, long enough to cover the next step's copies, with one barrier per step.  A copy
// instruction lands 64 x 16 bytes contiguously (8 rows of 128 bytes), so the rows cannot be
// padded: chunk c of row r is stored in slot c ^ ((r / 2) mod 8) instead, so that the fragment
// reads of 16 consecutive rows (two rows per 256-byte bank cycle) fall in distinct banks.  A
// 128 x 128 tile per workgroup with register staging (gemm_kernel) moves twice the operand bytes
// per product through LDS and had only 16 MFMAs per step to hide its next loads: 370-660 TFLOP/s
// on the prompt-size projections against 1.0-1.2 PFLOP/s here.  Measured and not kept: the same
// tile with register-staged operands (0.98-1.04), a 4-stage ring of 32-k steps (0.98-1.02),
// fragments of the next sub-step read ahead of the MFMAs (equal).
#include "attn_common.h"
#include "smla_internal.h"

namespace {

constexpr int kBM = 128, kBN = 128;   // tile: tokens x outputs
constexpr int kRowBytes = 128;        // bytes of one tile row per K step
constexpr int kLdsRow = 144;          // padded LDS row
constexpr int kTileLds = kBM * kLdsRow;
constexpr int kChunks = kBM * kRowBytes / 16 / 256;  // 16-byte chunks per thread per operand (4)

typedef float f32x16_t_g __attribute__((ext_vector_type(16)));

__device__ inline float mul_rn_g(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ inline float add_rn_g(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ inline float sub_rn_g(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// inverse RoPE of 4 (x0, x1) bf16 pairs held in one 16-byte chunk, pairs p0 .. p0+3 at one position
__device__ inline u32x4_t inv_rope4(u32x4_t v, const float* __restrict__ cs, const float* __restrict__ sn) {
  const f32x4_t c = *(const f32x4_t*)cs, s = *(const f32x4_t*)sn;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float x0 = __uint_as_float(v[j] << 16), x1 = __uint_as_float(v[j] & 0xffff0000u);
    const float o0 = add_rn_g(mul_rn_g(x0, c[j]), mul_rn_g(x1, s[j]));
    const float o1 = sub_rn_g(mul_rn_g(x1, c[j]), mul_rn_g(x0, s[j]));
    v[j] = pack_bf16x2(o0, o1);
  }
  return v;
}

template <bool BF16, int YDT, bool ROPE>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ x, int64_t ldx,
                                                   const uint8_t* __restrict__ w, int T, int N, int K, int ntn,
                                                   const int32_t* __restrict__ pos, const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, int head_dim,
                                                   void* __restrict__ y, int64_t ldy) {
  constexpr int ES = BF16 ? 2 : 4;              // element bytes
  constexpr int KSTEP = kRowBytes / ES;         // K per step: 64 / 32
  __shared__ __align__(16) uint8_t lds[2][2][kTileLds];  // [stage][A, B]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x / ntn;
  const int n0 = (blockIdx.x % ntn) * kBN;
  const int t0 = blockIdx.y * kBM;
  const int wm = wave & 1, wn = wave >> 1;

  // this thread's chunks: chunk c = tid + 256 i -> tile row c / 8, 16-byte column c % 8
  const uint8_t* ap[kChunks];
  const uint8_t* bp[kChunks];
  int lofs[kChunks];
  const float* csp[kChunks];
  const float* snp[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    const int c = tid + 256 * i, row = c >> 3, col = c & 7;
    const int t = min(t0 + row, T - 1);
    const int n = min(n0 + row, N - 1);
    ap[i] = x + ((int64_t)t * ldx + (int64_t)g * K) * ES + col * 16;
    bp[i] = w + ((int64_t)g * N + n) * K * ES + col * 16;
    lofs[i] = row * kLdsRow + col * 16;
    if constexpr (ROPE) {
      const int64_t p = pos[t];
      csp[i] = cos_t + p * 32 + 4 * col;   // rd / 2 = 32 pairs; this chunk holds pairs 4 col .. +3
      snp[i] = sin_t + p * 32 + 4 * col;
    }
  }
  u32x4_t ra[kChunks], rb[kChunks];
  const int kbytes = K * ES;
  const int ccol = (tid & 7) * 16;  // this thread's chunk column (the same for its kChunks chunks)
  auto load = [&](int ks) {
    const int64_t off = (int64_t)ks * kRowBytes;
    if (off + ccol < kbytes) {
#pragma unroll
      for (int i = 0; i < kChunks; i++) {
        ra[i] = *(const u32x4_t*)(ap[i] + off);
        rb[i] = *(const u32x4_t*)(bp[i] + off);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; i++) ra[i] = rb[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int stage, int ks) {
    if constexpr (ROPE) {
      if ((ks * KSTEP) % head_dim == head_dim - 64) {
#pragma unroll
        for (int i = 0; i < kChunks; i++) ra[i] = inv_rope4(ra[i], csp[i], snp[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < kChunks; i++) {
      *(u32x4_t*)&lds[stage][0][lofs[i]] = ra[i];
      *(u32x4_t*)&lds[stage][1][lofs[i]] = rb[i];
    }
  };

  f32x16_t_g acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; mb++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mb][nb][r] = 0.f;

  const int nk = (kbytes + kRowBytes - 1) / kRowBytes;
  load(0);
  store(0, 0);
  __syncthreads();
  // fragment rows of this lane: A row 64 wm + 32 mb + lane % 32, B row 64 wn + 32 nb + lane % 32
  const int arow = (64 * wm + (lane & 31)) * kLdsRow, brow = (64 * wn + (lane & 31)) * kLdsRow;
  const int khalf = lane >> 5;
  for (int ks = 0; ks < nk; ks++) {
    const int st = ks & 1;
    if (ks + 1 < nk) load(ks + 1);
    const uint8_t* A = lds[st][0];
    const uint8_t* B = lds[st][1];
    if constexpr (BF16) {
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {   // 16 k per MFMA: lane half h holds k = 16 kk + 8 h ..
        const int ko = kk * 32 + khalf * 16;
        bf16x8_t a[2], b[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
          a[j] = as_bf16x8(*(const u32x4_t*)&A[arow + 32 * j * kLdsRow + ko]);
          b[j] = as_bf16x8(*(const u32x4_t*)&B[brow + 32 * j * kLdsRow + ko]);
        }
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
          for (int nb = 0; nb < 2; nb++)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mb], b[nb], acc[mb][nb], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 16; kk++) {  // 2 k per MFMA: lane half h holds k = 2 kk + h
        const int ko = (2 * kk + khalf) * 4;
        float a[2], b[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
          a[j] = *(const float*)&A[arow + 32 * j * kLdsRow + ko];
          b[j] = *(const float*)&B[brow + 32 * j * kLdsRow + ko];
        }
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
          for (int nb = 0; nb < 2; nb++)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mb], b[nb], acc[mb][nb], 0, 0, 0);
      }
    }
    if (ks + 1 < nk) store(st ^ 1, ks + 1);
    __syncthreads();
  }

  // accumulator r of block (mb, nb): token 64 wm + 32 mb + 8 (r / 4) + 4 (lane / 32) + r % 4,
  // output 64 wn + 32 nb + lane % 32
#pragma unroll
  for (int mb = 0; mb < 2; mb++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int n = n0 + 64 * wn + 32 * nb + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = t0 + 64 * wm + 32 * mb + 8 * (r >> 2) + 4 * khalf + (r & 3);
        if (t < T) {
          const int64_t o = (int64_t)t * ldy + (int64_t)g * N + n;
          if constexpr (YDT == SMLA_BF16)
            __builtin_nontemporal_store((uint16_t)bf16_rne(acc[mb][nb][r]), (uint16_t*)y + o);
          else
            __builtin_nontemporal_store(acc[mb][nb][r], (float*)y + o);
        }
      }
    }
}

// BT x BT tiles (tokens x outputs): BT = 256 with 8 waves of 128 x 64, or BT = 128 with 4 waves of
// 64 x 64 (two workgroups per CU); either way 8 one-KB copy instructions per wave per stage
template <int BT>
struct DmaTile {
  static constexpr int NW = BT == 256 ? 8 : 4;        // waves
  static constexpr int WROWS = BT / 2;                 // rows per wave (2 row halves)
  static constexpr int MB = WROWS / 32;                // 32-row MFMA blocks per wave
  static constexpr int OPB = BT * kRowBytes;           // one operand's rows of one K step
  static constexpr int STAGE = 2 * OPB;                // A then B
  static constexpr int COPIES = STAGE / 1024 / NW;     // per wave per stage (8)
  static constexpr int ACH = BT * 8 / (64 * NW);       // A chunks per thread (rotation of a RoPE step: 4)
};

template <int YDT, bool ROPE, int BT>
__global__ __launch_bounds__(DmaTile<BT>::NW * 64) void gemm_dma_kernel(const uint8_t* __restrict__ x, int64_t ldx,
                                                       const uint8_t* __restrict__ w, int T, int N, int K, int ntn,
                                                       const int32_t* __restrict__ pos, const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t, int head_dim,
                                                       void* __restrict__ y, int64_t ldy) {
  using namespace smla_attn;
  using L = DmaTile<BT>;
  constexpr int kStageBytes = L::STAGE, kOperandBytes = L::OPB, kCopiesPerWave = L::COPIES;
  extern __shared__ __align__(16) uint8_t lds_g[];
  lds_u8_t* lds = (lds_u8_t*)lds_g;
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x / ntn;
  const int n0 = (blockIdx.x % ntn) * BT;
  const int t0 = blockIdx.y * BT;
  const int wm = wave & 1, wn = wave >> 1;  // row half, 64-column slice
  // copy instruction q = 8 wave + i covers stage bytes [1024 q, 1024 q + 1024): rows
  // 8 (q mod BT/8) .. +7 of A (q < BT/8) or of B; lane L takes row + L / 8, slot L mod 8 <- chunk
  // (L mod 8) ^ ((row / 2) mod 8)
  const uint8_t* src[kCopiesPerWave];
#pragma unroll
  for (int i = 0; i < kCopiesPerWave; i++) {
    const int q = wave * kCopiesPerWave + i;
    const int r = 8 * (q % (BT / 8)) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    if (q < BT / 8) {
      const int t = min(t0 + r, T - 1);
      src[i] = x + ((int64_t)t * ldx + (int64_t)g * K) * 2 + 16 * c;
    } else {
      const int n = min(n0 + r, N - 1);
      src[i] = w + ((int64_t)g * N + n) * (int64_t)K * 2 + 16 * c;
    }
  }
  auto issue = [&](int stage, int ks) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kCopiesPerWave; i++) {
      const uint32_t ld =
          __builtin_amdgcn_readfirstlane(lds_base + stage * kStageBytes + (wave * kCopiesPerWave + i) * 1024);
      dma16(src[i] + (int64_t)ks * kRowBytes, ld);
    }
  };

  f32x16_t_g acc[L::MB][2];
#pragma unroll
  for (int mb = 0; mb < L::MB; mb++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mb][nb][r] = 0.f;
  // fragment rows of this lane: A row 128 wm + 32 mb + lane % 32, B row 64 wn + 32 nb + lane % 32;
  // the lane half h holds k 16 kk + 8 h .. +7, chunk 2 kk + h of the row
  const int r32 = lane & 31, khalf = lane >> 5;
  // ROPE: the A chunks this thread rotates in a RoPE step, j = tid + 512 i (row j / 8, slot j mod 8),
  // and their rows' offsets in the cos / sin tables (32 pairs per position)
  int prow[L::ACH] = {};
  if constexpr (ROPE) {
#pragma unroll
    for (int i = 0; i < L::ACH; i++) prow[i] = pos[min(t0 + ((tid + 64 * L::NW * i) >> 3), T - 1)] * 32;
  }
  const int nk = K / 64;
  issue(0, 0);
  for (int ks = 0; ks < nk; ks++) {
    wait_vm(0);     // this wave's copies of step ks
    lds_barrier();  // everyone's copies of step ks landed; step ks - 1 is read by every wave
    if (ks + 1 < nk) issue((ks + 1) & 1, ks + 1);
    const lds_u8_t* A = lds + (ks & 1) * kStageBytes;
    const lds_u8_t* B = A + kOperandBytes;
    if constexpr (ROPE) {
      // the step holding a head's last 64 dims: every A chunk (4 (x0, x1) pairs, pairs 4c .. 4c + 3
      // of its row's position, c = slot ^ ((row / 2) mod 8)) rotated back in place, then a barrier
      if ((ks * 64) % head_dim == head_dim - 64) {
#pragma unroll
        for (int i = 0; i < L::ACH; i++) {
          const int j = tid + 64 * L::NW * i, r = j >> 3, sl = j & 7, c = sl ^ ((r >> 1) & 7);
          lds_u32x4_t* pa = (lds_u32x4_t*)(lds + (ks & 1) * kStageBytes + r * kRowBytes + 16 * sl);
          *pa = inv_rope4(*pa, cos_t + prow[i] + 4 * c, sin_t + prow[i] + 4 * c);
        }
        lds_barrier();
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const int c = 2 * kk + khalf;
      bf16x8_t a[L::MB], b[2];
#pragma unroll
      for (int mb = 0; mb < L::MB; mb++) {
        const int r = L::WROWS * wm + 32 * mb + r32;
        a[mb] = as_bf16x8(*(const lds_u32x4_t*)(A + r * kRowBytes + 16 * (c ^ ((r >> 1) & 7))));
      }
#pragma unroll
      for (int nb = 0; nb < 2; nb++) {
        const int r = 64 * wn + 32 * nb + r32;
        b[nb] = as_bf16x8(*(const lds_u32x4_t*)(B + r * kRowBytes + 16 * (c ^ ((r >> 1) & 7))));
      }
#pragma unroll
      for (int mb = 0; mb < L::MB; mb++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mb], b[nb], acc[mb][nb], 0, 0, 0);
    }
  }

  // accumulator r of block (mb, nb): token WROWS wm + 32 mb + 8 (r / 4) + 4 (lane / 32) + r % 4,
  // output 64 wn + 32 nb + lane % 32.  Nontemporal stores (the output is not read back by this
  // launch; 64-byte runs per half wave): the grouped 4096 x 8 x 1024 x 4096 product 287 -> 275 us,
  // the other prompt-size shapes equal.
#pragma unroll
  for (int mb = 0; mb < L::MB; mb++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int n = n0 + 64 * wn + 32 * nb + r32;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = t0 + L::WROWS * wm + 32 * mb + 8 * (r >> 2) + 4 * khalf + (r & 3);
        if (t < T) {
          const int64_t o = (int64_t)t * ldy + (int64_t)g * N + n;
          if constexpr (YDT == SMLA_BF16)
            __builtin_nontemporal_store((uint16_t)bf16_rne(acc[mb][nb][r]), (uint16_t*)y + o);
          else
            __builtin_nontemporal_store(acc[mb][nb][r], (float*)y + o);
        }
      }
    }
}

}  // namespace

template <int BT>
static int launch_gemm_dma(const void* x, int64_t ldx, const void* w, int64_t T, int64_t G, int64_t N, int64_t K,
                           const int32_t* pos, const float* cos_t, const float* sin_t, int64_t head_dim, void* y,
                           int y_dtype, hipStream_t st) {
  using L = DmaTile<BT>;
  const int64_t ntb = (N + BT - 1) / BT;
  const dim3 gb((unsigned)(ntb * G), (unsigned)((T + BT - 1) / BT));
  auto kern = pos ? (y_dtype == SMLA_BF16 ? gemm_dma_kernel<SMLA_BF16, true, BT> : gemm_dma_kernel<SMLA_F32, true, BT>)
                  : (y_dtype == SMLA_BF16 ? gemm_dma_kernel<SMLA_BF16, false, BT> : gemm_dma_kernel<SMLA_F32, false, BT>);
  // devices whose LDS limit is raised, one set per kernel (RoPE form x output type)
  static std::atomic<uint64_t> lds_attr[4] = {{0}, {0}, {0}, {0}};
  if (hipError_t e = smla_set_dynamic_lds((const void*)kern, 2 * L::STAGE,
                                          lds_attr[(pos ? 2 : 0) + (y_dtype == SMLA_BF16 ? 1 : 0)]);
      e != hipSuccess)
    return (int)e;
  hipLaunchKernelGGL(kern, gb, dim3(L::NW * 64), 2 * L::STAGE, st, (const uint8_t*)x, ldx, (const uint8_t*)w, (int)T,
                     (int)N, (int)K, (int)ntb, pos, cos_t, sin_t, (int)head_dim, y, G * N);
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}

// y [T, G*N] (row stride G*N) = grouped x [T, G*K] (row stride ldx elements) times w [G*N, K]^T.
// x and w both bf16 (x_f32 false) or both fp32; y bf16 or fp32.  With pos (bf16 only), inverse RoPE
// of the last 64 dims of every head_dim-wide head of x on load.  16-byte aligned rows (K % 8 for
// bf16, K % 4 for fp32).  Returns SMLA_OK or a hipError_t.
int launch_gemm_tiled(const void* x, int64_t ldx, bool f32_operands, const void* w, int64_t T, int64_t G, int64_t N,
                      int64_t K, const int32_t* pos, const float* cos_t, const float* sin_t, int64_t head_dim,
                      void* y, int y_dtype, hipStream_t st) {
  const int64_t ldy = G * N;
  // bf16 operands, 16-byte aligned, K a multiple of 64 (and the RoPE dims one K step per head): the
  // DMA tiles, 256 x 256 when they give every CU one, else 128 x 128 when those do
  if (!f32_operands && K % 64 == 0 && ldx % 8 == 0 && (!pos || head_dim % 64 == 0) &&
      (((uintptr_t)x | (uintptr_t)w) & 15) == 0) {
    const int64_t cus = smla_num_cus();
    auto tiles = [&](int64_t bt) { return (T + bt - 1) / bt * G * ((N + bt - 1) / bt); };
    if (tiles(256) >= cus)
      return launch_gemm_dma<256>(x, ldx, w, T, G, N, K, pos, cos_t, sin_t, head_dim, y, y_dtype, st);
    if (tiles(128) >= cus)
      return launch_gemm_dma<128>(x, ldx, w, T, G, N, K, pos, cos_t, sin_t, head_dim, y, y_dtype, st);
  }
  const int64_t ntn = (N + kBN - 1) / kBN;
  const dim3 grid((unsigned)(ntn * G), (unsigned)((T + kBM - 1) / kBM)), blk(256);
#define SMLA_GEMM(BF, YD, RP)                                                                                   \
  hipLaunchKernelGGL((gemm_kernel<BF, YD, RP>), grid, blk, 0, st, (const uint8_t*)x, ldx, (const uint8_t*)w,   \
                     (int)T, (int)N, (int)K, (int)ntn, pos, cos_t, sin_t, (int)head_dim, y, ldy)
  if (f32_operands) {
    if (y_dtype == SMLA_BF16) SMLA_GEMM(false, SMLA_BF16, false);
    else SMLA_GEMM(false, SMLA_F32, false);
  } else if (pos) {
    if (y_dtype == SMLA_BF16) SMLA_GEMM(true, SMLA_BF16, true);
    else SMLA_GEMM(true, SMLA_F32, true);
  } else {
    if (y_dtype == SMLA_BF16) SMLA_GEMM(true, SMLA_BF16, false);
    else SMLA_GEMM(true, SMLA_F32, false);
  }
#undef SMLA_GEMM
  SMLA_HIP_CHECK_LAUNCH();
  return SMLA_OK;
}
