// Declarations shared by the attention translation units.
#pragma once

#include "smla_internal.h"

namespace smla_attn {

constexpr int kTileRows = 32;
constexpr int kThreads = 256;
constexpr float kRescaleSlack = 8.0f;

struct RowSrc {
  const void* kv0;
  const void* kv1;
  const float* sc0;
  const float* sc1;
  int64_t n0, n1;
};

// Prefill row sets computed in the kernel instead of read from an index list: query s of a
// sequence sits at position p = q_pos0 + s; list entry t < window is raw row max(0, p-window+1) + t
// (-1 past p), entry window + c is compressed row c (id n0 + c) for c < (p+1)/ratio, else -1 --
// the lists oracle/decode_engine.py:110-114 builds for every position of a prompt.  Workgroups
// then take the queries longest first.
struct ImplicitRows {
  int64_t q_pos0;
  int window;
  int ratio;  // 0: window rows only
  int enabled;
};

// Decode lists built in the kernel from indexer scores: the engine's decode index build
// (oracle/decode_engine.py:110-114 with an indexer-ranked compressed part, the list
// smla_select_decode writes).  Entry t < window of query row r is raw row pos[r] - window + 1 + t
// (-1 below 0); entry window + j is the j-th of the selected compressed rows in ascending order
// (id n0 + c), where the selection is the min(k, nvis[r]) best of the first nvis[r] scores of row
// r (score descending, index ascending, -0 == +0), -1 past it.  Every workgroup whose split
// reaches past the window runs the selection itself, so no index list goes through memory.
struct SelectRows {
  const float* scores;   // [rows, N]
  const int32_t* nvis;   // [rows] or null (all N visible)
  const int32_t* pos;    // [rows]
  int N, window, k, enabled;
};

// bf16 or fp8 (e4m3 + per-64 pow2 scales) rows, D in {576, 512}, DV = 512, H % 16 == 0: 12-wave
// role-split kernel (4 score waves, 8 value waves, 64 heads per workgroup).  Writes the final
// output (nsplit == 1) or partial states: (m, l) fp32 per (query row, split, head), then the partial
// O rows (bf16 for bf16 output, else fp32) after all (m, l) records, split-major.
int launch_decode_v6(int D, bool kv_fp8, int nsplit, int rows_per_split, const void* q, RowSrc src,
                     const float* sink, const int32_t* idx, int64_t T, int64_t B, int64_t S, int64_t H, float scale,
                     void* out, int out_dtype, float* part, hipStream_t stream, ImplicitRows ir = ImplicitRows{},
                     SelectRows sr = SelectRows{});
// the selection's scores per thread of the 768-thread workgroup for N scores (0: not supported)
constexpr int select_per(int64_t N) { return N <= 768 * 12 ? 12 : N <= 768 * 24 ? 24 : 0; }
constexpr int kDecodeV6ShortRows = 256;  // up to here: 4-tile ring; its index table lives in LDS
constexpr int kDecodeV6MaxRows = 8192;   // beyond: 3-tile ring and a larger index table

// ---- device helpers shared by the LDS-DMA decode kernels
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;
typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
typedef __attribute__((address_space(3))) int lds_i32_t;

__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// wait until at most n vector-memory operations of this wave are outstanding
__device__ inline void wait_vm(int n) {
#define SMLA_VM_CASE(N) \
  case N:               \
    asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); \
    break;
  switch (n) {
    SMLA_VM_CASE(1) SMLA_VM_CASE(2) SMLA_VM_CASE(3) SMLA_VM_CASE(4) SMLA_VM_CASE(5) SMLA_VM_CASE(6)
    SMLA_VM_CASE(7) SMLA_VM_CASE(8) SMLA_VM_CASE(9) SMLA_VM_CASE(10) SMLA_VM_CASE(11) SMLA_VM_CASE(12)
    SMLA_VM_CASE(13) SMLA_VM_CASE(14) SMLA_VM_CASE(15) SMLA_VM_CASE(16) SMLA_VM_CASE(17) SMLA_VM_CASE(18)
    SMLA_VM_CASE(19) SMLA_VM_CASE(20) SMLA_VM_CASE(21) SMLA_VM_CASE(22) SMLA_VM_CASE(23) SMLA_VM_CASE(24)
    SMLA_VM_CASE(25) SMLA_VM_CASE(26) SMLA_VM_CASE(27) SMLA_VM_CASE(28) SMLA_VM_CASE(29) SMLA_VM_CASE(30)
    SMLA_VM_CASE(31) SMLA_VM_CASE(32) SMLA_VM_CASE(33) SMLA_VM_CASE(34) SMLA_VM_CASE(35) SMLA_VM_CASE(36)
    default:
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      break;
  }
#undef SMLA_VM_CASE
}

// 16-byte HBM -> LDS copy for every lane: lane l's bytes land at lds_dst + 16*l.  Untracked by the
// compiler (inline asm); callers wait with wait_vm().
__device__ inline void dma16(const void* gsrc, uint32_t lds_dst_uniform) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_dst_uniform), "v"(gsrc)
               : "memory", "m0");
}
// the same copy with the non-temporal hint: data read once (a query's own Q rows) should not push
// reused rows out of the L2
__device__ inline void dma16_nt(const void* gsrc, uint32_t lds_dst_uniform) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds_dst_uniform), "v"(gsrc)
               : "memory", "m0");
}

// 16-byte vector load that the compiler does not track (covered by a later wait_vm)
__device__ inline u32x4_t load16_untracked(const void* p) {
  u32x4_t r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}



}  // namespace smla_attn
