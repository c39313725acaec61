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

// bf16 rows, D in {576, 512}, DV = 512, H % 16 == 0.  Writes partial states (nsplit > 1) or the
// final output (nsplit == 1).  Returns SMLA_OK or a hipError_t.
int launch_decode_bf16(int D, int nsplit, int rows_per_split, const void* q, RowSrc src, const float* sink,
                       const int32_t* idx, int64_t T, int64_t B, int64_t S, int64_t H, float scale, void* out,
                       int out_dtype, float* part, hipStream_t stream, hipEvent_t ev_before, hipEvent_t ev_after);

// largest rows_per_split the bf16 decode kernel accepts (its index table lives in LDS)
constexpr int kDecodeMaxRowsPerSplit = 1024;

}  // namespace smla_attn
