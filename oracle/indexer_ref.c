/* Canonical indexer score and stable top-k selection — CPU oracle (TEST INFRASTRUCTURE ONLY).
 *
 * The reference has no indexer and no score-based top-k (its selection is "take every causally
 * visible compressed row", oracle/decode_engine.py:110-114).  This file defines the build's
 * indexer arithmetic exactly, so that the HIP kernels can reproduce every score bit for bit and
 * the selected index sets can be compared exactly:
 *
 *   dot[h]   = fmaf chain over d = 0..D-1 of q[s,h,d] * k[n,d], starting from +0
 *   r[h]     = dot[h] > 0 ? dot[h] : +0                                   (ReLU, -0 -> +0)
 *   acc      = fmaf chain over h = 0..H-1 of w[s,h] * r[h], starting from +0
 *   score    = acc * kscale[n]  (kscale == NULL: score = acc)
 *   score    = -inf for n >= nvis[s]
 *
 * q, k, w are fp32 here (bf16 / e4m3 inputs are decoded to fp32 exactly before the call).
 *
 * Selection: rank the visible positions by (score descending, index ascending), with -0 and +0
 * equal; keep the first min(k, nvis); emit them in ascending index order; pad with -1 to k.
 *
 * Pinning: brute force on tiny inputs (Python loops with math.fsum-free exact fma emulation via
 * fractions), the "take all" case nvis <= k equals the reference's index build, and the fp32
 * rounding of fmaf is glibc's correctly rounded fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_indexer_score(const float* q, const float* k, const float* kscale, const float* w,
                          int64_t S, int64_t H, int64_t D, int64_t N, const int32_t* nvis,
                          float* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t s = 0; s < S; s++) {
    for (int64_t n = 0; n < N; n++) {
      const float* qs = q + s * H * D;
      const float* ws = w + s * H;
      int64_t nv = nvis ? nvis[s] : N;
      if (n >= nv) { out[s * N + n] = -INFINITY; continue; }
      const float* kn = k + n * D;
      float acc = 0.0f;
      for (int64_t h = 0; h < H; h++) {
        float dot = 0.0f;
        for (int64_t d = 0; d < D; d++) dot = fmaf(qs[h * D + d], kn[d], dot);
        float r = dot > 0.0f ? dot : 0.0f;
        acc = fmaf(ws[h], r, acc);
      }
      out[s * N + n] = kscale ? acc * kscale[n] : acc;
    }
  }
}

/* order-preserving key: larger score -> smaller key; -0 and +0 map to the same key */
static uint32_t desc_key(float f) {
  if (f == 0.0f) f = 0.0f;
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}

static int cmp_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}
static int cmp_i32(const void* a, const void* b) {
  int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

void oracle_topk(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k,
                 int32_t* out) {
#pragma omp parallel for schedule(dynamic)
  for (int64_t r = 0; r < R; r++) {
    int64_t nv = nvis ? nvis[r] : N;
    if (nv > N) nv = N;
    if (nv < 0) nv = 0;
    int32_t* o = out + r * k;
    int64_t take = nv < k ? nv : k;
    uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (nv > 0 ? nv : 1));
    for (int64_t n = 0; n < nv; n++)
      keys[n] = ((uint64_t)desc_key(scores[r * N + n]) << 32) | (uint64_t)(uint32_t)n;
    qsort(keys, (size_t)nv, sizeof(uint64_t), cmp_u64);
    for (int64_t j = 0; j < take; j++) o[j] = (int32_t)(keys[j] & 0xffffffffu);
    qsort(o, (size_t)take, sizeof(int32_t), cmp_i32);
    for (int64_t j = take; j < k; j++) o[j] = -1;
    free(keys);
  }
}
