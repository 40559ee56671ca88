// IMROPE helpers and the per-head RMSNorm + IMROPE of the Qwen3.5
// attention prologue, shared by the prologue kernels (layer.hip) and the
// decode split kernel's fused prologue (decode.hip), so that both form the
// same values.
#pragma once
#include <math.h>

#include "alpx_common.h"

namespace alpx {

constexpr int kRopeMaxDim = 512;                // widest head a prologue wave stages
constexpr int kMaxPairs = kRopeMaxDim / 2;      // most rotary pairs

// IMROPE position lane of rotary pair p (interleaved T/H/W/E schedule).
__device__ __forceinline__ int imrope_lane(int p, const int (&sec)[4], int R) {
  const int sector = p % R;
  if (sector % 3 == 1 && sector < 3 * sec[1]) return 1;
  if (sector % 3 == 2 && sector < 3 * sec[2]) return 2;
  if (sector % 3 == 0 && sector < 3 * sec[0]) return 0;
  return 3;
}

// cos / sin of the angle pos * inv (inv = scale * base^(-2 p / (2 R)),
// formed on the host in double precision).  The angle reaches 10^4-10^6 rad
// at long contexts, where a float angle alone would be off by ~10^-3 rad,
// so it is reduced modulo 2 pi in double precision first; sin / cos of the
// reduced angle (|r| <= pi) are then taken in float.
__device__ __forceinline__ void rope_cs(double pos, double inv, float& c, float& s) {
  constexpr double kTwoPi = 6.283185307179586476925;
  const double theta = pos * inv;
  const double r = theta - kTwoPi * rint(theta * (1.0 / kTwoPi));
  sincosf((float)r, &s, &c);
}

// One rotated channel of an IMROPE pair: x c - xp s in the first half,
// xp s + x c in the second (xp: the pair partner), with the fused
// multiply-adds written out so every kernel that rotates forms the same
// bits (the prologue kernels, the split kernel's prelude and the prefill
// kernel's fused query prologue).
__device__ __forceinline__ float rope_pair(bool first, float x, float xp, float c, float s) {
  return first ? fmaf(x, c, -(xp * s)) : fmaf(xp, s, x * c);
}

__device__ __forceinline__ float rope_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// One head row by one wave: x (lane-strided, channel lane + 64 e, already
// loaded) is RMS-normalised over D with per-channel weights wt -- x times
// one correctly rounded 1 / sqrt(mean(x^2) + eps) per row, times wt (the
// reference divides each channel by the root, qwen35_cuda.py:920-931, which
// differs by at most an fp32 rounding before the T rounding) -- then the
// first 2 R channels are rotated as IMROPE pairs (p, p + R) at text
// position p (the last section's lane uses position 0); st is a D-float
// LDS row for the pair partners.  Channel i of the result goes to dst[i],
// rounded to T.
template <typename T, int kPer>
__device__ __forceinline__ void norm_rope(float (&x)[kPer], const float (&wt)[kPer], int D,
                                          float eps, const int (&sec)[4], int R,
                                          const double* inv, double p, float* st, T* dst,
                                          int lane) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e)
    if (lane + 64 * e < D) ss = fmaf(x[e], x[e], ss);
  ss = rope_wave_sum(ss);
  const float rinv = 1.f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i < D) {
      x[e] = x[e] * rinv * wt[e];
      st[i] = x[e];
    }
  }
  // LDS traffic of one wave is processed in issue order, so the partner
  // reads below see this wave's stores.
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i >= D) continue;
    float y = x[e];
    if (i < 2 * R) {
      const int pr = i < R ? i : i - R;
      const int ln = imrope_lane(pr, sec, R);
      float c, sn;
      rope_cs(ln == 3 ? 0.0 : p, inv[pr], c, sn);
      y = rope_pair(i < R, x[e], i < R ? st[i + R] : st[pr], c, sn);
    }
    dst[i] = from_f32<T>(y);
  }
}

// scale * base^(-2 p / (2 R)) for p < R, in double precision (host).
void inverse_frequencies(double* inv, int R, double base, double scale);
// The attention chunk prologue's key / value heads only (layer.hip), and
// rot_out [tokens, R] = the (cos, sin) of each token's rotary pairs: the
// caller forms the query rows itself with the same arithmetic.  With a
// table (the sequence's block-table row), the caches are page pools
// [num_pages, 2^page_shift, Hkv, D], capacity = max_pages << page_shift,
// cache_batch 1 and batch_index 0.
int attention_prologue_chunk_kv(const void* query_gate, const void* key, const void* value,
                                const float* q_norm, const float* k_norm, void* key_cache,
                                void* value_cache, int dtype, int64_t capacity, int cache_batch,
                                int batch_index, int tokens, int q_heads, int kv_heads,
                                int head_dim, int value_dim, int64_t position, const int* sections,
                                double frequency_base, float eps, float2* rot_out, void* stream,
                                const int32_t* table = nullptr, int page_shift = 0,
                                int num_pages = 0);
// R = the sum of the four IMROPE sections; true when they are unusable.
bool bad_sections(const int* sections, int& R);

}  // namespace alpx
