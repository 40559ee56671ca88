// Qwen3.5 layer primitives on either side of the attention / GDN kernels.
//
// Row norms (L2, RMS, RMS x SiLU gate), the depthwise causal convolution
// step, the recurrent parameters (beta, log decay), IMROPE, and two fused
// decode-step entry points built from them:
//  * the full-attention prologue: joint query/gate split, per-head Q/K
//    RMSNorm, IMROPE at the text position and the K/V cache append, one
//    wave per (sequence, head) in one launch;
//  * the recurrent-layer step: convolution + SiLU + split + Q/K L2 norm +
//    beta / log decay in one launch (one wave per head slot), the GDN step
//    kernel, and the gated RMSNorm.
// All of it is bandwidth / latency work: one wave owns one row (a head of
// 64..256 values), reductions are wave shuffles, and rotations stage the
// normalised row in LDS so every lane can read its pair partner.
#include <math.h>

#include "alpx_common.h"
#include "decode_internal.h"
#include "gdn_internal.h"
#include "rope_internal.h"
#include "timing.h"

namespace alpx {
namespace {

constexpr int kNormL2 = 0;        // x / max(||x||, eps)
constexpr int kNormRms = 1;       // x / sqrt(mean(x^2) + eps) * w
constexpr int kNormRmsGate = 2;   // rms_norm(x) * w * silu(gate)
constexpr int kMaxDim = 512;      // widest row a prologue / prep wave stages

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float silu_f(float x) { return x * stable_sigmoid(x); }

// Stable softplus log(1 + e^x) (two branches, as tensor.stable_softplus).
__device__ __forceinline__ float softplus_f(float x) {
  return x > 0.f ? x + log1pf(expf(-x)) : log1pf(expf(x));
}

static_assert(kMaxDim == kRopeMaxDim, "prologue rows and rope rows share one width");

// ---------------------------------------------------------------- row norm

struct NormArgs {
  const void* x;
  const float* w;
  const void* gate;
  void* out;
  int64_t rows;
  int64_t grp_rows, grp_stride;  // input row r at (r / grp_rows) * grp_stride + (r % grp_rows) * n
  int n;
  float eps;
};

// Row r of a row norm, by one wave, rows of at most 64 NPL values: every
// load of the row (x, and the weight and gate it needs) is issued from a
// clamped index before the reduction, so the row costs one memory round
// trip, and x stays in registers.  Lane l owns elements l + 64 j, summed in
// j order, as the strided loop below sums them: both forms give the same
// bits.
template <typename T, typename TO, int MODE, int NPL>
__device__ __forceinline__ void norm_row_regs(const NormArgs& a, int64_t r, int lane) {
  const T* x = (const T*)a.x + (r / a.grp_rows) * a.grp_stride + (r % a.grp_rows) * a.n;
  const T* g = (const T*)a.gate + r * a.n;
  float xv[NPL], wv[NPL], gv[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = min(lane + 64 * j, a.n - 1);
    xv[j] = to_f32(x[i]);
    if constexpr (MODE != kNormL2) wv[j] = a.w[i];
    if constexpr (MODE == kNormRmsGate) gv[j] = to_f32(g[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j)
    if (lane + 64 * j < a.n) ss = fmaf(xv[j], xv[j], ss);
  ss = wave_sum(ss);
  const float den = MODE == kNormL2 ? fmaxf(sqrtf(ss), a.eps) : sqrtf(ss / (float)a.n + a.eps);
  TO* o = (TO*)a.out + r * a.n;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = lane + 64 * j;
    if (i < a.n) {
      float v = xv[j] / den;
      if constexpr (MODE != kNormL2) v *= wv[j];
      if constexpr (MODE == kNormRmsGate) v *= silu_f(gv[j]);
      o[i] = from_f32<TO>(v);
    }
  }
}

// Row r of a row norm, by one wave (any width).
template <typename T, typename TO, int MODE>
__device__ __forceinline__ void norm_row(const NormArgs& a, int64_t r, int lane) {
  if (a.n <= 128) return norm_row_regs<T, TO, MODE, 2>(a, r, lane);
  if (a.n <= 256) return norm_row_regs<T, TO, MODE, 4>(a, r, lane);
  if (a.n <= 512) return norm_row_regs<T, TO, MODE, 8>(a, r, lane);
  const T* x = (const T*)a.x + (r / a.grp_rows) * a.grp_stride + (r % a.grp_rows) * a.n;
  float ss = 0.f;
  for (int i = lane; i < a.n; i += 64) {
    const float v = to_f32(x[i]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float den = MODE == kNormL2 ? fmaxf(sqrtf(ss), a.eps) : sqrtf(ss / (float)a.n + a.eps);
  TO* o = (TO*)a.out + r * a.n;
  const T* g = (const T*)a.gate + r * a.n;
  for (int i = lane; i < a.n; i += 64) {
    float v = to_f32(x[i]) / den;
    if (MODE != kNormL2) v *= a.w[i];
    if (MODE == kNormRmsGate) v *= silu_f(to_f32(g[i]));
    o[i] = from_f32<TO>(v);
  }
}

// kNormRows consecutive rows of at most 128 values by one wave: the loads of
// every row (and the weight, once) are issued before the first reduction,
// then each row is reduced and written with norm_row_regs's arithmetic
// (lane l owns elements l and l + 64, summed in that order): the same bits
// with a quarter of the waves, each with four rows' loads in flight.
constexpr int kNormRows = 4;

template <typename T, typename TO, int MODE>
__device__ __forceinline__ void norm_rows_128(const NormArgs& a, int64_t r0, int lane) {
  constexpr int NPL = 2, R = kNormRows;
  float xv[R][NPL], wv[NPL], gv[R][NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j)
    if constexpr (MODE != kNormL2) wv[j] = a.w[min(lane + 64 * j, a.n - 1)];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t r = min(r0 + k, a.rows - 1);
    const T* x = (const T*)a.x + (r / a.grp_rows) * a.grp_stride + (r % a.grp_rows) * a.n;
    const T* g = (const T*)a.gate + r * a.n;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = min(lane + 64 * j, a.n - 1);
      xv[k][j] = to_f32(x[i]);
      if constexpr (MODE == kNormRmsGate) gv[k][j] = to_f32(g[i]);
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t r = r0 + k;
    if (r >= a.rows) break;  // uniform across the wave
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (lane + 64 * j < a.n) ss = fmaf(xv[k][j], xv[k][j], ss);
    ss = wave_sum(ss);
    const float den =
        MODE == kNormL2 ? fmaxf(sqrtf(ss), a.eps) : sqrtf(ss / (float)a.n + a.eps);
    TO* o = (TO*)a.out + r * a.n;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = lane + 64 * j;
      if (i < a.n) {
        float v = xv[k][j] / den;
        if constexpr (MODE != kNormL2) v *= wv[j];
        if constexpr (MODE == kNormRmsGate) v *= silu_f(gv[k][j]);
        o[i] = from_f32<TO>(v);
      }
    }
  }
}

// ROWS = 1: one row per wave, any width; ROWS = kNormRows: rows of at most
// 128 values, kNormRows per wave (many-row calls: a prefill chunk's norms).
template <typename T, typename TO, int MODE, int ROWS>
__global__ void __launch_bounds__(256) row_norm_kernel(NormArgs a) {
  const int64_t r = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * ROWS;
  if (r >= a.rows) return;  // the whole wave leaves together
  if constexpr (ROWS == 1)
    norm_row<T, TO, MODE>(a, r, threadIdx.x & 63);
  else
    norm_rows_128<T, TO, MODE>(a, r, threadIdx.x & 63);
}

// Calls with at least this many rows of at most 128 values take the
// several-rows-per-wave kernel (fewer rows keep one row per wave, for
// parallelism).
constexpr int64_t kNormManyRows = 4096;

template <typename T, typename TO, int ROWS>
void launch_norm_rows(const NormArgs& a, int mode, hipStream_t s) {
  const dim3 grid((unsigned)((a.rows + 4 * ROWS - 1) / (4 * ROWS)));
  switch (mode) {
    case kNormL2:
      hipLaunchKernelGGL((row_norm_kernel<T, TO, kNormL2, ROWS>), grid, dim3(256), 0, s, a);
      break;
    case kNormRms:
      hipLaunchKernelGGL((row_norm_kernel<T, TO, kNormRms, ROWS>), grid, dim3(256), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((row_norm_kernel<T, TO, kNormRmsGate, ROWS>), grid, dim3(256), 0, s, a);
      break;
  }
}

template <typename T, typename TO>
int launch_norm(const NormArgs& a, int mode, hipStream_t s) {
  if (a.n <= 128 && a.rows >= kNormManyRows)
    launch_norm_rows<T, TO, kNormRows>(a, mode, s);
  else
    launch_norm_rows<T, TO, 1>(a, mode, s);
  return check_launch("alpx_row_norm");
}

template <typename T>
int launch_norm_to(const NormArgs& a, int mode, int out_dtype, hipStream_t s) {
  switch (out_dtype) {
    case ALPX_F32: return launch_norm<T, float>(a, mode, s);
    case ALPX_F16: return launch_norm<T, f16_t>(a, mode, s);
    default: return launch_norm<T, bf16_t>(a, mode, s);
  }
}

int run_norm(const NormArgs& a, int mode, int dtype, int out_dtype, hipStream_t s) {
  if (a.rows == 0) return ALPX_OK;
  switch (dtype) {
    case ALPX_F32: return launch_norm_to<float>(a, mode, out_dtype, s);
    case ALPX_F16: return launch_norm_to<f16_t>(a, mode, out_dtype, s);
    default: return launch_norm_to<bf16_t>(a, mode, out_dtype, s);
  }
}

// --------------------------------------------------------- conv step

struct ConvArgs {
  const float* cur;   // [B, C]
  const float* w;     // tap t, channel c at t * w_tap + c * w_ch
  float* hist;        // [B, K - 1, C], oldest first
  void* out;          // [B, C]
  int64_t w_tap, w_ch;
  int B, C, K;
  int silu;
};

template <typename TO>
__global__ void __launch_bounds__(256) conv_step_kernel(ConvArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.B * a.C) return;
  const int64_t b = i / a.C;
  const int c = (int)(i - b * a.C);
  float* h = a.hist + b * (int64_t)(a.K - 1) * a.C + c;
  const float x = a.cur[i];
  float acc = 0.f;
  for (int t = 0; t < a.K - 1; ++t) acc = fmaf(h[(int64_t)t * a.C], a.w[t * a.w_tap + c * a.w_ch], acc);
  acc = fmaf(x, a.w[(a.K - 1) * a.w_tap + c * a.w_ch], acc);
  for (int t = 0; t + 1 < a.K - 1; ++t) h[(int64_t)t * a.C] = h[(int64_t)(t + 1) * a.C];
  if (a.K > 1) h[(int64_t)(a.K - 2) * a.C] = x;
  ((TO*)a.out)[i] = from_f32<TO>(a.silu ? silu_f(acc) : acc);
}

// ------------------------------------------------- recurrent parameters

__global__ void __launch_bounds__(256)
recurrent_params_kernel(const float* __restrict__ bl, const float* __restrict__ al,
                        const float* __restrict__ dtb, const float* __restrict__ ssm,
                        float* beta, float* g, int64_t n, int heads) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int h = (int)(i % heads);
  beta[i] = stable_sigmoid(bl[i]);
  g[i] = softplus_f(al[i] + dtb[h]) * ssm[h];
}

// ------------------------------------------------------------- IMROPE

struct RopeArgs {
  const void* x;    // [rows, heads, dim]
  void* out;
  const int64_t* pos;  // lanes (T, H, W, E) of row r at pos + r * pos_stride
  int64_t rows, pos_stride;
  int heads, dim, R;
  int sec[4];
  double inv[kMaxPairs];  // scale * base^(-2 p / (2 R)) per pair p
};

// One thread per (row, head, j): j < R rotates the pair (j, j + R); the
// remaining j copy the unrotated tail coordinates 2 R .. dim - 1.
template <typename T, typename TO>
__global__ void __launch_bounds__(256) imrope_kernel(RopeArgs a) {
  const int per_head = a.dim - a.R;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.rows * a.heads * per_head) return;
  const int64_t rh = i / per_head;
  const int j = (int)(i - rh * per_head);
  const int64_t row = rh / a.heads;
  const T* x = (const T*)a.x + rh * a.dim;
  TO* o = (TO*)a.out + rh * a.dim;
  if (j < a.R) {
    const int lane = imrope_lane(j, a.sec, a.R);
    float c, s;
    rope_cs((double)a.pos[row * a.pos_stride + lane], a.inv[j], c, s);
    const float x0 = to_f32(x[j]), x1 = to_f32(x[j + a.R]);
    o[j] = from_f32<TO>(x0 * c - x1 * s);
    o[j + a.R] = from_f32<TO>(x0 * s + x1 * c);
  } else {
    const int e = j + a.R;
    o[e] = from_f32<TO>(to_f32(x[e]));
  }
}

template <typename T>
int launch_rope(const RopeArgs& a, int out_dtype, hipStream_t s) {
  const int64_t n = a.rows * a.heads * (a.dim - a.R);
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (out_dtype) {
    case ALPX_F32: hipLaunchKernelGGL((imrope_kernel<T, float>), grid, dim3(256), 0, s, a); break;
    case ALPX_F16: hipLaunchKernelGGL((imrope_kernel<T, f16_t>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((imrope_kernel<T, bf16_t>), grid, dim3(256), 0, s, a); break;
  }
  return check_launch("alpx_imrope");
}

// ---------------------------------------------- attention prologue (fused)

struct ProArgs {
  const void* qg;    // [B, Hq, 2 D]: per head D query then D gate values
  const void* k;     // [B, Hkv, D]
  const void* v;     // [B, Hkv, Dv]
  const float* qw;   // [D]
  const float* kw;   // [D]
  void* q_out;       // [B, Hq, D]
  void* g_out;       // [B, Hq, D], or null: the gate half is not copied
  void* kc;          // [capacity, B, Hkv, D]
  void* vc;          // [capacity, B, Hkv, Dv]
  const int32_t* positions;  // device [B] or null (then position + r pos_step for row r)
  int64_t position, capacity;
  int64_t pos_step;  // 0: one token per sequence; 1: the rows are one sequence's chunk
  int B, Hq, Hkv, D, Dv, R;
  int CB;            // cache batch count (cache row = pos * CB + cache sequence)
  int bsel;          // < 0: row r is cache sequence r; else every row is cache sequence bsel
  int sec[4];
  float eps;
  int slot0;         // first slot processed (Hq: key and value heads only)
  float2* rot_out;   // null, or [B, R]: (cos, sin) of each row's rotary pairs
  // Paged caches (table non-null): logical row pos of the one sequence is
  // row pos % 2^page_shift of page table[pos >> page_shift] of a pool
  // [num_pages, 2^page_shift, Hkv, D]; an entry outside the pool writes
  // nothing.
  const int32_t* table;
  int page_shift, num_pages;
  double inv[kMaxPairs];  // base^(-2 p / (2 R)) per pair p
};

// One wave per (sequence, slot): slots 0 .. Hq - 1 are query heads (RMSNorm
// + IMROPE, gate copy), Hq .. Hq + Hkv - 1 key heads (RMSNorm + IMROPE, to
// the key cache), the rest value heads (copied to the value cache).  Cache
// rows at a position outside [0, capacity) are not written.
template <typename T>
__global__ void __launch_bounds__(256) attn_prologue_kernel(ProArgs a) {
  __shared__ float stage[4][kMaxDim];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int slots = a.Hq + 2 * a.Hkv - a.slot0;
  const int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= (int64_t)a.B * slots) return;
  const int b = (int)(id / slots);
  const int j = a.slot0 + (int)(id - (int64_t)b * slots);
  const int64_t pos = a.positions ? (int64_t)a.positions[b] : a.position + b * a.pos_step;
  bool in_cache = pos >= 0 && pos < a.capacity;
  int64_t crow = pos * a.CB + (a.bsel < 0 ? b : a.bsel);  // cache row of this token
  if (a.table != nullptr && in_cache) {
    const int pg = a.table[pos >> a.page_shift];
    in_cache = pg >= 0 && pg < a.num_pages;
    crow = ((int64_t)pg << a.page_shift) + (pos & ((1 << a.page_shift) - 1));
  }
  if (j >= a.Hq + a.Hkv) {  // value head
    const int h = j - a.Hq - a.Hkv;
    if (!in_cache) return;
    const T* src = (const T*)a.v + ((int64_t)b * a.Hkv + h) * a.Dv;
    T* dst = (T*)a.vc + (crow * a.Hkv + h) * a.Dv;
    for (int i = lane; i < a.Dv; i += 64) dst[i] = src[i];
    return;
  }
  if (a.rot_out != nullptr && j == a.Hq) {
    // the rotation of this row's pairs, as norm_rope forms it, for a
    // kernel that rotates the query heads itself
    for (int pr = lane; pr < a.R; pr += 64) {
      float c, sn;
      rope_cs(imrope_lane(pr, a.sec, a.R) == 3 ? 0.0 : (double)pos, a.inv[pr], c, sn);
      a.rot_out[(int64_t)b * a.R + pr] = make_float2(c, sn);
    }
  }
  const bool is_q = j < a.Hq;
  const int h = is_q ? j : j - a.Hq;
  const T* src = is_q ? (const T*)a.qg + ((int64_t)b * a.Hq + h) * 2 * a.D
                      : (const T*)a.k + ((int64_t)b * a.Hkv + h) * a.D;
  const float* w = is_q ? a.qw : a.kw;
  // Every load first (row, weight, gate half), then the reduction.
  constexpr int kPer = kMaxDim / 64;
  float x[kPer], wt[kPer];
  T gv[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i < a.D) {
      x[e] = to_f32(src[i]);
      wt[e] = w[i];
      if (is_q && a.g_out != nullptr) gv[e] = src[a.D + i];
    }
  }
  T* dst;
  if (is_q) {
    dst = (T*)a.q_out + ((int64_t)b * a.Hq + h) * a.D;
    if (a.g_out != nullptr) {
      T* gd = (T*)a.g_out + ((int64_t)b * a.Hq + h) * a.D;
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        if (lane + 64 * e < a.D) gd[lane + 64 * e] = gv[e];
    }
  } else {
    if (!in_cache) return;
    dst = (T*)a.kc + (crow * a.Hkv + h) * a.D;
  }
  // text position lanes (p, p, p, 0)
  norm_rope<T, kPer>(x, wt, a.D, a.eps, a.sec, a.R, a.inv, (double)pos, stage[wave], dst, lane);
}

// --------------------------------------- recurrent-layer prep (fused)

struct PrepArgs {
  const float* cur;   // [B, C], C = 2 Hk Dk + Hv Dv
  const float* w;     // conv weights, tap t / channel c at t * w_tap + c * w_ch
  float* hist;        // [B, K - 1, C]
  const float* bl;    // [B, Hv]
  const float* al;    // [B, Hv]
  const float* dtb;   // [Hv]
  const float* ssm;   // [Hv]
  float* q;           // out [B, Hk, Dk]
  float* k;           // out [B, Hk, Dk]
  float* v;           // out [B, Hv, Dv]
  float* beta;        // out [B, Hv]
  float* g;           // out [B, Hv]
  int64_t w_tap, w_ch;
  int B, K, Hk, Hv, Dk, Dv;
  float eps;
};

// Convolution step of one head slot of sequence b (one wave): channels
// [c0, c0 + n) of the C = 2 Hk Dk + Hv Dv mixed channels.  Each lane
// convolves its channels (then SiLU) and shifts their history; `l2` slots
// (query / key) are L2-normalised over the head.  Results go to dst[0, n).
// `mid` runs between the slot's loads and its arithmetic (a caller issues
// further loads there, so that the slot's waits do not cover them).  Rows
// of up to 64 kPer channels.
template <int kPer, typename Mid>
__device__ __forceinline__ void prep_slot(const PrepArgs& a, int b, int c0, int n, bool l2,
                                          float* dst, int lane, Mid&& mid) {
  const int C = 2 * a.Hk * a.Dk + a.Hv * a.Dv;
  constexpr int kTaps = 4;  // history rows held in registers (longer kernels loop)
  const int64_t rowC = (int64_t)b * C;
  float* hist = a.hist + (int64_t)b * (a.K - 1) * C;
  // Every load of the lane's channels first: current sample, history taps
  // and weights; then the convolutions; then the history shift and outputs.
  float y[kPer], xc[kPer], hv[kPer][kTaps], wv[kPer][kTaps + 1];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i >= n) continue;
    const int c = c0 + i;
    xc[e] = a.cur[rowC + c];
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
      if (t < a.K - 1) hv[e][t] = hist[(int64_t)t * C + c];
#pragma unroll
    for (int t = 0; t <= kTaps; ++t)
      if (t < a.K) wv[e][t] = a.w[t * a.w_tap + c * a.w_ch];
  }
  mid();
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    y[e] = 0.f;
    if (i >= n) continue;
    const int c = c0 + i;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
      if (t < a.K - 1) acc = fmaf(hv[e][t], wv[e][t], acc);
    for (int t = kTaps; t < a.K - 1; ++t)  // kernels longer than kTaps + 1 taps
      acc = fmaf(hist[(int64_t)t * C + c], a.w[t * a.w_tap + c * a.w_ch], acc);
    float wl = 0.f;  // weight of the current sample (tap K - 1)
#pragma unroll
    for (int t = 0; t <= kTaps; ++t)
      if (t == a.K - 1) wl = wv[e][t];
    if (a.K - 1 > kTaps) wl = a.w[(a.K - 1) * a.w_tap + c * a.w_ch];
    acc = fmaf(xc[e], wl, acc);
    y[e] = silu_f(acc);
    ss = fmaf(y[e], y[e], ss);
  }
  float inv = 1.f;
  if (l2) inv = 1.f / fmaxf(sqrtf(wave_sum(ss)), a.eps);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i >= n) continue;
    const int c = c0 + i;
    dst[i] = l2 ? y[e] * inv : y[e];
    // shift the lane's history column: row t takes row t + 1, the last row
    // takes the current sample
#pragma unroll
    for (int t = 0; t + 1 < kTaps; ++t)
      if (t + 1 < a.K - 1) hist[(int64_t)t * C + c] = hv[e][t + 1];
    for (int t = kTaps - 1; t + 1 < a.K - 1; ++t)
      hist[(int64_t)t * C + c] = hist[(int64_t)(t + 1) * C + c];
    if (a.K > 1) hist[(int64_t)(a.K - 2) * C + c] = xc[e];
  }
}

// beta = sigmoid(b), log decay = softplus(a + dt_bias) * ssm_a of value head h.
__device__ __forceinline__ void recurrent_params(const PrepArgs& a, int b, int h, float& beta,
                                                 float& g) {
  const int64_t bh = (int64_t)b * a.Hv + h;
  beta = stable_sigmoid(a.bl[bh]);
  g = softplus_f(a.al[bh] + a.dtb[h]) * a.ssm[h];
}

// One wave per (sequence, head slot): Hk query slots, Hk key slots, Hv
// value slots; value slot h also forms beta and the log decay of value
// head h.
__global__ void __launch_bounds__(256) recurrent_prep_kernel(PrepArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int slots = 2 * a.Hk + a.Hv;
  const int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= (int64_t)a.B * slots) return;
  const int b = (int)(id / slots);
  const int j = (int)(id - (int64_t)b * slots);
  if (j < 2 * a.Hk) {
    float* dst = j < a.Hk ? a.q + ((int64_t)b * a.Hk + j) * a.Dk
                          : a.k + ((int64_t)b * a.Hk + (j - a.Hk)) * a.Dk;
    prep_slot<kMaxDim / 64>(a, b, j * a.Dk, a.Dk, true, dst, lane, [] {});
  } else {
    const int h = j - 2 * a.Hk;
    if (lane == 0) {
      const int64_t bh = (int64_t)b * a.Hv + h;
      recurrent_params(a, b, h, a.beta[bh], a.g[bh]);
    }
    prep_slot<kMaxDim / 64>(a, b, 2 * a.Hk * a.Dk + h * a.Dv, a.Dv, false,
              a.v + ((int64_t)b * a.Hv + h) * a.Dv, lane, [] {});
  }
}

// ------------------------------- recurrent-layer step in two launches
//
// Launch A, one block per (sequence, value head h, 16 state rows), the GDN
// step's geometry (recurrent_rows_kernel): the block recomputes the
// convolution + SiLU + L2 norm of h's query and key heads (key head
// h % Hk) from the history without writing it, forms the convolution of
// its own 16 value channels (and shifts their history: no other block
// touches them), beta and the log decay, then runs the GDN step on its
// rows and writes o.  Launch B (recurrent_finish_kernel): the gated
// RMSNorm of every o row and the history shift of the query / key
// channels, which every A block of the key head read.  Each value is
// formed with the arithmetic, in the order, of recurrent_prep_kernel,
// gdn_step_kernel and row_norm_kernel.

constexpr int kRowsThreads = 256;
constexpr int kRowsPerBlock = 16;  // 8 half-waves x kRowsPerHalf rows
constexpr int kRowsPerHalf = 2;
constexpr int kRowsDim = 256;      // widest key / value head of launch A

struct RowsArgs {
  PrepArgs p;   // q / k / v outputs unused; hist: value channels written
  float* state;  // [B, Hv, Dv, Dk]
  float* o;      // [B, Hv, Dv] fp32, scaled by 1 / sqrt(Dk)
  float scale;
};

// Convolution + SiLU of channel c of sequence b (taps from the history,
// the current sample last), as prep_slot: up to kTaps history rows and
// their weights are loaded together before any arithmetic (a loop over a
// run-time tap count would wait for each load in turn).
__device__ __forceinline__ float conv_silu(const PrepArgs& a, int64_t rowC, const float* hist,
                                           int C, int c) {
  constexpr int kTaps = 4;
  float hv[kTaps], wv[kTaps + 1];
  const float xc = a.cur[rowC + c];
#pragma unroll
  for (int t = 0; t < kTaps; ++t)
    if (t < a.K - 1) hv[t] = hist[(int64_t)t * C + c];
#pragma unroll
  for (int t = 0; t <= kTaps; ++t)
    if (t < a.K) wv[t] = a.w[t * a.w_tap + c * a.w_ch];
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < kTaps; ++t)
    if (t < a.K - 1) acc = fmaf(hv[t], wv[t], acc);
  for (int t = kTaps; t < a.K - 1; ++t)  // kernels longer than kTaps + 1 taps
    acc = fmaf(hist[(int64_t)t * C + c], a.w[t * a.w_tap + c * a.w_ch], acc);
  float wl = 0.f;  // weight of the current sample (tap K - 1)
#pragma unroll
  for (int t = 0; t <= kTaps; ++t)
    if (t == a.K - 1) wl = wv[t];
  if (a.K - 1 > kTaps) wl = a.w[(a.K - 1) * a.w_tap + c * a.w_ch];
  acc = fmaf(xc, wl, acc);
  return silu_f(acc);
}

template <int NV>
__global__ void __launch_bounds__(kRowsThreads) recurrent_rows_kernel(RowsArgs f) {
  const PrepArgs& a = f.p;
  __shared__ float qk[2][kRowsDim];  // SiLU(conv) of the query and key heads, then normalised
  __shared__ float inv[2];
  __shared__ float vs[kRowsPerBlock];
  __shared__ float bg[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, b = blockIdx.z, kh = h % a.Hk;
  const int Dk = a.Dk, Dv = a.Dv;
  const int C = 2 * a.Hk * Dk + a.Hv * Dv;
  const int64_t rowC = (int64_t)b * C;
  float* hist = a.hist + (int64_t)b * (a.K - 1) * C;
  const int rb = blockIdx.x * kRowsPerBlock;
  const int l32 = tid & 31, hw = tid >> 5;
  const int r0 = rb + hw * kRowsPerHalf;
  const int64_t bh = (int64_t)b * a.Hv + h;

  // The state rows first (rows rb + 2 hw + j, lane columns 4 l32 + 128 e +
  // 0..3, as gdn_step_kernel): they depend on nothing, so they are in
  // flight with the convolution loads and the block waits one round trip.
  float s[kRowsPerHalf][NV][4];
#pragma unroll
  for (int j = 0; j < kRowsPerHalf; ++j) {
    const float* row = f.state + (bh * Dv + min(r0 + j, Dv - 1)) * Dk;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int c0 = 4 * l32 + 128 * e;
      const f32x4 x = *(const f32x4*)(row + min(c0, Dk - 4));
#pragma unroll
      for (int c = 0; c < 4; ++c) s[j][e][c] = c0 < Dk ? x[c] : 0.f;
    }
  }

  // convolutions: query / key channel pairs, then the block's value rows
  for (int i = tid; i < 2 * Dk; i += kRowsThreads) {
    const int slot = i / Dk, d = i - slot * Dk;
    qk[slot][d] = conv_silu(a, rowC, hist, C, slot * a.Hk * Dk + kh * Dk + d);
  }
  if (tid < kRowsPerBlock && rb + tid < Dv) {
    const int c = 2 * a.Hk * Dk + h * Dv + rb + tid;
    const float xc = a.cur[rowC + c];
    vs[tid] = conv_silu(a, rowC, hist, C, c);
    // shift this value channel's history (only this block reads it)
    for (int t = 0; t + 1 < a.K - 1; ++t) hist[(int64_t)t * C + c] = hist[(int64_t)(t + 1) * C + c];
    if (a.K > 1) hist[(int64_t)(a.K - 2) * C + c] = xc;
  }
  if (tid == kRowsThreads - 1) recurrent_params(a, b, h, bg[0], bg[1]);
  __syncthreads();
  // L2 norms of the query (wave 0) and key (wave 1) heads, summed as
  // prep_slot sums them (lane-strided channels, then the wave sum)
  if (wave < 2) {
    float ss = 0.f;
    for (int d = lane; d < Dk; d += 64) ss = fmaf(qk[wave][d], qk[wave][d], ss);
    ss = wave_sum(ss);
    if (lane == 0) inv[wave] = 1.f / fmaxf(sqrtf(ss), a.eps);
  }
  __syncthreads();

  // GDN step on the block's rows, as gdn_step_kernel
  float kk[NV][4], qq[NV][4];
#pragma unroll
  for (int e = 0; e < NV; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = 4 * l32 + 128 * e + c;
      kk[e][c] = col < Dk ? qk[1][col] * inv[1] : 0.f;
      qq[e][c] = col < Dk ? qk[0][col] * inv[0] : 0.f;
    }
  const float decay = __expf(bg[1]);
  const float beta = bg[0];
  float p[kRowsPerHalf];
#pragma unroll
  for (int j = 0; j < kRowsPerHalf; ++j) {
    p[j] = 0.f;
#pragma unroll
    for (int e = 0; e < NV; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[j][e][c] *= decay;
        p[j] += s[j][e][c] * kk[e][c];
      }
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
    for (int j = 0; j < kRowsPerHalf; ++j) p[j] += __shfl_xor(p[j], off, 32);
  float o[kRowsPerHalf];
#pragma unroll
  for (int j = 0; j < kRowsPerHalf; ++j) {
    const float vv = vs[min(r0 + j, Dv - 1) - rb];
    const float delta = beta * (vv - p[j]);
    o[j] = 0.f;
#pragma unroll
    for (int e = 0; e < NV; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[j][e][c] += delta * kk[e][c];
        o[j] += s[j][e][c] * qq[e][c];
      }
  }
#pragma unroll
  for (int j = 0; j < kRowsPerHalf; ++j) {
    const int r = r0 + j;
    if (r >= Dv) break;
    float* row = f.state + (bh * Dv + r) * Dk;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int c0 = 4 * l32 + 128 * e;
      if (c0 < Dk) *(f32x4*)(row + c0) = (f32x4){s[j][e][0], s[j][e][1], s[j][e][2], s[j][e][3]};
    }
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
    for (int j = 0; j < kRowsPerHalf; ++j) o[j] += __shfl_xor(o[j], off, 32);
  if (l32 < kRowsPerHalf && r0 + l32 < Dv) {
    const float oj = l32 == 0 ? o[0] : o[1];
    f.o[bh * Dv + r0 + l32] = oj * f.scale;
  }
}

// Launch B: waves [0, norm_rows) take one gated-norm row each; the rest
// shift the history of the 2 Hk Dk query / key channels (one lane each).
struct FinishArgs {
  NormArgs norm;
  const float* cur;  // [B, C]
  float* hist;       // [B, K - 1, C]
  int B, C, K, qk_channels;
};

template <typename TO>
__global__ void __launch_bounds__(256) recurrent_finish_kernel(FinishArgs f) {
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w < f.norm.rows) {
    norm_row<float, TO, kNormRmsGate>(f.norm, w, lane);
    return;
  }
  const int64_t i = (w - f.norm.rows) * 64 + lane;
  if (i >= (int64_t)f.B * f.qk_channels) return;
  const int b = (int)(i / f.qk_channels), c = (int)(i - (int64_t)b * f.qk_channels);
  float* hist = f.hist + (int64_t)b * (f.K - 1) * f.C;
  for (int t = 0; t + 1 < f.K - 1; ++t) hist[(int64_t)t * f.C + c] = hist[(int64_t)(t + 1) * f.C + c];
  if (f.K > 1) hist[(int64_t)(f.K - 2) * f.C + c] = f.cur[(int64_t)b * f.C + c];
}

// ----------------------------------- recurrent-layer prep over a chunk

struct ChunkPrepArgs {
  const float* x;     // [T, C] convolution inputs of T consecutive tokens
  const float* w;     // conv weights, tap i / channel c at i * w_tap + c * w_ch
  const float* hist;  // [K - 1, C] history before token 0 (row 0 oldest)
  const float* bl;    // [T, Hv]
  const float* al;    // [T, Hv]
  const float* dtb;   // [Hv]
  const float* ssm;   // [Hv]
  void* q;            // out [T, Hk, Dk]
  void* k;            // out [T, Hk, Dk]
  void* v;            // out [T, Hv, Dv]
  float* beta;        // out [T, Hv]
  float* g;           // out [T, Hv]
  int64_t w_tap, w_ch;
  int T, K, Hk, Hv, Dk, Dv;
  float eps;
};

// One wave per (token, head slot), as recurrent_prep_kernel, with token t's
// convolution window taken from the extended sequence E = [history; x]:
// tap i reads E row t + i (tap K - 1 is x[t]).  The history is read only;
// conv_history_advance moves it on afterwards.
template <typename TO>
__global__ void __launch_bounds__(256) recurrent_chunk_prep_kernel(ChunkPrepArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int slots = 2 * a.Hk + a.Hv;
  const int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= (int64_t)a.T * slots) return;
  const int t = (int)(id / slots);
  const int j = (int)(id - (int64_t)t * slots);
  const int C = 2 * a.Hk * a.Dk + a.Hv * a.Dv;
  int c0, n;
  TO* dst;
  if (j < 2 * a.Hk) {
    c0 = j * a.Dk;
    n = a.Dk;
    dst = j < a.Hk ? (TO*)a.q + ((int64_t)t * a.Hk + j) * a.Dk
                   : (TO*)a.k + ((int64_t)t * a.Hk + (j - a.Hk)) * a.Dk;
  } else {
    const int h = j - 2 * a.Hk;
    c0 = 2 * a.Hk * a.Dk + h * a.Dv;
    n = a.Dv;
    dst = (TO*)a.v + ((int64_t)t * a.Hv + h) * a.Dv;
    if (lane == 0) {
      const int64_t th = (int64_t)t * a.Hv + h;
      a.beta[th] = stable_sigmoid(a.bl[th]);
      a.g[th] = softplus_f(a.al[th] + a.dtb[h]) * a.ssm[h];
    }
  }
  constexpr int kPer = kMaxDim / 64;
  constexpr int kTaps = 4;  // taps held in registers (longer kernels loop)
  float y[kPer], xv[kPer][kTaps], wv[kPer][kTaps];
  // every load first: the window rows and weights of the lane's channels
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i >= n) continue;
    const int c = c0 + i;
#pragma unroll
    for (int tap = 0; tap < kTaps; ++tap) {
      if (tap >= a.K) continue;
      const int er = t + tap;  // E row
      xv[e][tap] = er < a.K - 1 ? a.hist[(int64_t)er * C + c]
                                : a.x[(int64_t)(er - (a.K - 1)) * C + c];
      wv[e][tap] = a.w[tap * a.w_tap + c * a.w_ch];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    y[e] = 0.f;
    if (i >= n) continue;
    const int c = c0 + i;
    float acc = 0.f;
#pragma unroll
    for (int tap = 0; tap < kTaps; ++tap)
      if (tap < a.K) acc = fmaf(xv[e][tap], wv[e][tap], acc);
    for (int tap = kTaps; tap < a.K; ++tap) {  // kernels longer than kTaps taps
      const int er = t + tap;
      const float xe = er < a.K - 1 ? a.hist[(int64_t)er * C + c]
                                    : a.x[(int64_t)(er - (a.K - 1)) * C + c];
      acc = fmaf(xe, a.w[tap * a.w_tap + c * a.w_ch], acc);
    }
    y[e] = silu_f(acc);
    ss = fmaf(y[e], y[e], ss);
  }
  float inv = 1.f;
  if (j < 2 * a.Hk) inv = 1.f / fmaxf(sqrtf(wave_sum(ss)), a.eps);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = lane + 64 * e;
    if (i < n) dst[i] = from_f32<TO>(j < 2 * a.Hk ? y[e] * inv : y[e]);
  }
}

// Tiled form of the chunk prep for conv kernels of up to kTileTaps taps and
// head dims that are multiples of 4 (at most 256): one block per (64-token
// tile, head slot).  Thread (cg, tg) owns channels 4 cg .. 4 cg + 3 of the
// slot for P = 64 / TG consecutive tokens and holds the P + K - 1 window
// rows they need as 16-byte vectors, so each input element is loaded about
// once instead of K times by K different waves.  The L2 norm of a q / k row
// is a shuffle sum over the CG lanes that share the token (CG = channel
// groups rounded up to 16, 32 or 64; idle lanes add zero).  Per element the
// convolution, SiLU and scaling are the same operations, in the same order,
// as recurrent_chunk_prep_kernel.
constexpr int kTileTokens = 64;
constexpr int kTileTaps = 4;

inline bool aligned(const void* p, size_t bytes) { return (uintptr_t)p % bytes == 0; }

template <typename TO>
__device__ __forceinline__ void store4(TO* p, const float (&v)[4]) {
  if constexpr (sizeof(TO) == 4) {
    *(f32x4*)p = (f32x4){v[0], v[1], v[2], v[3]};
  } else {
    typedef TO T4 __attribute__((ext_vector_type(4)));
    *(T4*)p = (T4){from_f32<TO>(v[0]), from_f32<TO>(v[1]), from_f32<TO>(v[2]), from_f32<TO>(v[3])};
  }
}

template <typename TO>
__global__ void __launch_bounds__(256) recurrent_chunk_prep_tile(ChunkPrepArgs a) {
  constexpr int kMaxP = 16;
  const int tid = threadIdx.x;
  const int j = blockIdx.y;
  const int t0 = blockIdx.x * kTileTokens;
  const int C = 2 * a.Hk * a.Dk + a.Hv * a.Dv;
  const bool is_qk = j < 2 * a.Hk;
  int c0, n;
  TO* dst;
  int64_t dstride;
  if (is_qk) {
    c0 = j * a.Dk;
    n = a.Dk;
    dst = j < a.Hk ? (TO*)a.q + (int64_t)j * a.Dk : (TO*)a.k + (int64_t)(j - a.Hk) * a.Dk;
    dstride = (int64_t)a.Hk * a.Dk;
  } else {
    const int h = j - 2 * a.Hk;
    c0 = 2 * a.Hk * a.Dk + h * a.Dv;
    n = a.Dv;
    dst = (TO*)a.v + (int64_t)h * a.Dv;
    dstride = (int64_t)a.Hv * a.Dv;
    if (tid < kTileTokens && t0 + tid < a.T) {
      const int64_t th = (int64_t)(t0 + tid) * a.Hv + h;
      a.beta[th] = stable_sigmoid(a.bl[th]);
      a.g[th] = softplus_f(a.al[th] + a.dtb[h]) * a.ssm[h];
    }
  }
  const int ng = n >> 2;
  const int CG = ng <= 16 ? 16 : ng <= 32 ? 32 : 64;
  const int P = kTileTokens * CG / 256;  // 4, 8 or 16
  const int cg = tid & (CG - 1), tg = tid / CG;
  const bool act = cg < ng;
  const int c = c0 + 4 * (act ? cg : 0);
  const int tb = t0 + tg * P;
  const int K = a.K;

  float w[kTileTaps][4];
#pragma unroll
  for (int tap = 0; tap < kTileTaps; ++tap)
#pragma unroll
    for (int e = 0; e < 4; ++e) w[tap][e] = tap < K ? a.w[tap * a.w_tap + (c + e) * a.w_ch] : 0.f;
  // Window rows tb .. tb + P + K - 2 of E = [history; x]; rows past the
  // end of x read its last row (their tokens are not stored).
  f32x4 win[kMaxP + kTileTaps - 1];
#pragma unroll
  for (int r = 0; r < kMaxP + kTileTaps - 1; ++r) {
    win[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (r < P + K - 1) {
      const int er = tb + r;
      const int xr = er - (K - 1);
      const float* src = xr < 0 ? a.hist + (int64_t)er * C + c
                                : a.x + (int64_t)min(xr, a.T - 1) * C + c;
      win[r] = *(const f32x4*)src;
    }
  }
#pragma unroll
  for (int p = 0; p < kMaxP; ++p) {
    if (p < P) {
      float y[4];
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int tap = 0; tap < kTileTaps; ++tap)
          if (tap < K && p + tap < kMaxP + kTileTaps - 1) acc = fmaf(win[p + tap][e], w[tap][e], acc);
        y[e] = silu_f(acc);
        ss = fmaf(y[e], y[e], ss);
      }
      if (is_qk) {
        ss = act ? ss : 0.f;
        for (int off = CG >> 1; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        const float inv = 1.f / fmaxf(sqrtf(ss), a.eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] *= inv;
      }
      const int t = tb + p;
      if (act && t < a.T) store4(dst + (int64_t)t * dstride + 4 * cg, y);
    }
  }
}

// History after the chunk: the last K - 1 rows of E = [history; x].  One
// thread per channel walks the rows upward, so a history row it still has
// to read (row T + r > r) is never overwritten first.
__global__ void __launch_bounds__(256) conv_history_advance(float* hist, const float* x, int T,
                                                            int K, int C) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  for (int r = 0; r + 1 < K; ++r) {
    const int er = T + r;
    hist[(int64_t)r * C + c] =
        er < K - 1 ? hist[(int64_t)er * C + c] : x[(int64_t)(er - (K - 1)) * C + c];
  }
}

}  // namespace

void inverse_frequencies(double* inv, int R, double base, double scale) {
  for (int p = 0; p < R; ++p) inv[p] = scale * pow(base, -2.0 * (double)p / (double)(2 * R));
}

bool bad_sections(const int* sections, int& R) {
  if (!sections) return true;
  R = 0;
  for (int i = 0; i < 4; ++i) {
    if (sections[i] < 0) return true;
    R += sections[i];
  }
  return R <= 0;
}

}  // namespace alpx

// ------------------------------------------------------------- C-ABI

extern "C" int alpx_row_norm(const void* x, const float* weight, const void* gate, void* out,
                             int64_t rows, int n, int64_t group_rows, int64_t group_stride,
                             float eps, int mode, int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  if (!x || !out) return fail(ALPX_EINVAL, "alpx_row_norm: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_row_norm: unknown dtype");
  if (mode < kNormL2 || mode > kNormRmsGate) return fail(ALPX_EINVAL, "alpx_row_norm: unknown mode");
  if (rows < 0 || n <= 0) return fail(ALPX_EINVAL, "alpx_row_norm: rows must be >= 0 and width positive");
  if (!(eps > 0.f) || !isfinite(eps)) return fail(ALPX_EINVAL, "epsilon must be positive and finite");
  if (mode != kNormL2 && !weight) return fail(ALPX_EINVAL, "alpx_row_norm: RMSNorm needs a weight");
  if (mode == kNormRmsGate && !gate) return fail(ALPX_EINVAL, "alpx_row_norm: gated RMSNorm needs a gate");
  if (group_rows <= 0) {
    group_rows = rows > 0 ? rows : 1;
    group_stride = group_rows * n;
  }
  if (group_stride < group_rows * n) return fail(ALPX_EINVAL, "alpx_row_norm: group stride smaller than its rows");
  NormArgs a;
  a.x = x;
  a.w = weight;
  a.gate = gate;
  a.out = out;
  a.rows = rows;
  a.grp_rows = group_rows;
  a.grp_stride = group_stride;
  a.n = n;
  a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  return run_norm(a, mode, dtype, out_dtype, s);
}

extern "C" int alpx_conv_step(const float* current, const float* weight, float* history,
                              void* out, int batch, int channels, int kernel,
                              int64_t weight_tap_stride, int64_t weight_channel_stride,
                              int apply_silu, int out_dtype, void* stream) {
  using namespace alpx;
  if (!current || !weight || !out || (kernel > 1 && !history))
    return fail(ALPX_EINVAL, "alpx_conv_step: null buffer");
  if (!dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_conv_step: unknown dtype");
  if (batch <= 0 || channels <= 0 || kernel <= 0)
    return fail(ALPX_EINVAL, "alpx_conv_step: sizes must be positive");
  ConvArgs a;
  a.cur = current;
  a.w = weight;
  a.hist = history;
  a.out = out;
  a.w_tap = weight_tap_stride;
  a.w_ch = weight_channel_stride;
  a.B = batch;
  a.C = channels;
  a.K = kernel;
  a.silu = apply_silu ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  const dim3 grid((unsigned)(((int64_t)batch * channels + 255) / 256));
  switch (out_dtype) {
    case ALPX_F32: hipLaunchKernelGGL(conv_step_kernel<float>, grid, dim3(256), 0, s, a); break;
    case ALPX_F16: hipLaunchKernelGGL(conv_step_kernel<f16_t>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(conv_step_kernel<bf16_t>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch("alpx_conv_step");
}

extern "C" int alpx_recurrent_parameters(const float* beta_logits, const float* alpha_logits,
                                         const float* dt_bias, const float* ssm_a, float* beta,
                                         float* log_decay, int64_t count, int heads,
                                         void* stream) {
  using namespace alpx;
  if (!beta_logits || !alpha_logits || !dt_bias || !ssm_a || !beta || !log_decay)
    return fail(ALPX_EINVAL, "alpx_recurrent_parameters: null buffer");
  if (count < 0 || heads <= 0 || count % heads != 0)
    return fail(ALPX_EINVAL, "time-step bias and ssm_a must match value heads");
  if (count == 0) return ALPX_OK;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  hipLaunchKernelGGL(recurrent_params_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                     s, beta_logits, alpha_logits, dt_bias, ssm_a, beta, log_decay, count, heads);
  return check_launch("alpx_recurrent_parameters");
}

extern "C" int alpx_imrope(const void* x, void* out, const int64_t* positions,
                           int64_t position_stride, int64_t rows, int heads, int dim,
                           const int* sections, double frequency_base, double frequency_scale,
                           int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  if (!x || !out || !positions) return fail(ALPX_EINVAL, "alpx_imrope: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_imrope: unknown dtype");
  int R = 0;
  if (bad_sections(sections, R)) return fail(ALPX_EINVAL, "IMRoPE requires at least one rotary pair");
  if (rows < 0 || heads <= 0 || dim <= 0) return fail(ALPX_EINVAL, "alpx_imrope: sizes must be positive");
  if (dim < 2 * R) return fail(ALPX_EINVAL, "IMRoPE input is shorter than twice the section sum");
  if (R > kMaxPairs) return fail(ALPX_EUNSUPPORTED, "alpx_imrope: more than %d rotary pairs", kMaxPairs);
  if (!(frequency_base > 0.0) || !isfinite(frequency_base) || !(frequency_scale > 0.0) ||
      !isfinite(frequency_scale))
    return fail(ALPX_EINVAL, "frequency_base and frequency_scale must be positive and finite");
  if (position_stride < 0) return fail(ALPX_EINVAL, "alpx_imrope: negative position stride");
  if (rows == 0) return ALPX_OK;
  RopeArgs a;
  a.x = x;
  a.out = out;
  a.pos = positions;
  a.rows = rows;
  a.pos_stride = position_stride;
  a.heads = heads;
  a.dim = dim;
  a.R = R;
  for (int i = 0; i < 4; ++i) a.sec[i] = sections[i];
  inverse_frequencies(a.inv, R, frequency_base, frequency_scale);
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  switch (dtype) {
    case ALPX_F32: return launch_rope<float>(a, out_dtype, s);
    case ALPX_F16: return launch_rope<f16_t>(a, out_dtype, s);
    default: return launch_rope<bf16_t>(a, out_dtype, s);
  }
}

namespace {
// Shared by the decode (one token per sequence) and chunk (one sequence's
// consecutive tokens) forms of the attention prologue.
int attention_prologue_launch(const char* what, const void* query_gate, const void* key,
                              const void* value, const float* q_norm, const float* k_norm,
                              void* query_out, void* gate_out, void* key_cache,
                              void* value_cache, int dtype, int64_t capacity, int rows,
                              int cache_batch, int bsel, int64_t pos_step, int q_heads,
                              int kv_heads, int head_dim, int value_dim, int64_t position,
                              const int32_t* positions, const int* sections,
                              double frequency_base, float eps, void* stream,
                              bool kv_only = false, float2* rot_out = nullptr,
                              const int32_t* table = nullptr, int page_shift = 0,
                              int num_pages = 0) {
  using namespace alpx;
  if (!query_gate || !key || !value || !q_norm || !k_norm || (!query_out && !kv_only) ||
      (!gate_out && pos_step == 0) || !key_cache || !value_cache)
    return fail(ALPX_EINVAL, "%s: null buffer", what);
  if (!dtype_ok(dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", what);
  if (rows <= 0 || cache_batch <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      value_dim <= 0 || capacity <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", what);
  if (q_heads % kv_heads != 0) return fail(ALPX_EINVAL, "attention query heads must be a multiple of KV heads");
  if (head_dim > kMaxDim || value_dim > kMaxDim)
    return fail(ALPX_EUNSUPPORTED, "%s: head dims above %d", what, kMaxDim);
  int R = 0;
  if (bad_sections(sections, R)) return fail(ALPX_EINVAL, "IMRoPE requires at least one rotary pair");
  if (head_dim < 2 * R) return fail(ALPX_EINVAL, "IMRoPE input is shorter than twice the section sum");
  if (!(frequency_base > 0.0) || !isfinite(frequency_base))
    return fail(ALPX_EINVAL, "frequency_base must be positive and finite");
  if (!(eps > 0.f) || !isfinite(eps)) return fail(ALPX_EINVAL, "epsilon must be positive and finite");
  if (!positions && (position < 0 || position + pos_step * (rows - 1) >= capacity))
    return fail(ALPX_ERANGE, "attention cache position exceeds capacity");
  ProArgs a;
  a.qg = query_gate;
  a.k = key;
  a.v = value;
  a.qw = q_norm;
  a.kw = k_norm;
  a.q_out = query_out;
  a.g_out = gate_out;
  a.kc = key_cache;
  a.vc = value_cache;
  a.positions = positions;
  a.position = position;
  a.capacity = capacity;
  a.pos_step = pos_step;
  a.B = rows;
  a.CB = cache_batch;
  a.bsel = bsel;
  a.Hq = q_heads;
  a.Hkv = kv_heads;
  a.D = head_dim;
  a.Dv = value_dim;
  a.R = R;
  for (int i = 0; i < 4; ++i) a.sec[i] = sections[i];
  inverse_frequencies(a.inv, R, frequency_base, 1.0);
  a.eps = eps;
  a.slot0 = kv_only ? q_heads : 0;
  a.rot_out = rot_out;
  a.table = table;
  a.page_shift = page_shift;
  a.num_pages = num_pages;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  const int64_t waves = (int64_t)rows * (q_heads + 2 * kv_heads - a.slot0);
  const dim3 grid((unsigned)((waves + 3) / 4));
  switch (dtype) {
    case ALPX_F32: hipLaunchKernelGGL(attn_prologue_kernel<float>, grid, dim3(256), 0, s, a); break;
    case ALPX_F16: hipLaunchKernelGGL(attn_prologue_kernel<f16_t>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(attn_prologue_kernel<bf16_t>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch(what);
}
}  // namespace

extern "C" int alpx_attention_prologue(const void* query_gate, const void* key, const void* value,
                                       const float* q_norm, const float* k_norm, void* query_out,
                                       void* gate_out, void* key_cache, void* value_cache,
                                       int dtype, int64_t capacity, int batch, int q_heads,
                                       int kv_heads, int head_dim, int value_dim,
                                       int64_t position, const int32_t* positions,
                                       const int* sections, double frequency_base, float eps,
                                       void* stream) {
  return attention_prologue_launch("alpx_attention_prologue", query_gate, key, value, q_norm,
                                   k_norm, query_out, gate_out, key_cache, value_cache, dtype,
                                   capacity, batch, batch, -1, 0, q_heads, kv_heads, head_dim,
                                   value_dim, position, positions, sections, frequency_base, eps,
                                   stream);
}

extern "C" int alpx_attention_prologue_chunk(const void* query_gate, const void* key,
                                             const void* value, const float* q_norm,
                                             const float* k_norm, void* query_out,
                                             void* gate_out, void* key_cache, void* value_cache,
                                             int dtype, int64_t capacity, int cache_batch,
                                             int batch_index, int tokens, int q_heads,
                                             int kv_heads, int head_dim, int value_dim,
                                             int64_t position, const int* sections,
                                             double frequency_base, float eps, void* stream) {
  using namespace alpx;
  if (batch_index < 0 || batch_index >= cache_batch)
    return fail(ALPX_EINVAL, "batch_index exceeds the cache batch");
  return attention_prologue_launch("alpx_attention_prologue_chunk", query_gate, key, value,
                                   q_norm, k_norm, query_out, gate_out, key_cache, value_cache,
                                   dtype, capacity, tokens, cache_batch, batch_index, 1, q_heads,
                                   kv_heads, head_dim, value_dim, position, nullptr, sections,
                                   frequency_base, eps, stream);
}

namespace alpx {
// The chunk prologue's key and value heads only (the query heads are
// formed by the prefill kernel that reads them): cache rows written as
// alpx_attention_prologue_chunk writes them.
int attention_prologue_chunk_kv(const void* query_gate, const void* key, const void* value,
                                const float* q_norm, const float* k_norm, void* key_cache,
                                void* value_cache, int dtype, int64_t capacity, int cache_batch,
                                int batch_index, int tokens, int q_heads, int kv_heads,
                                int head_dim, int value_dim, int64_t position, const int* sections,
                                double frequency_base, float eps, float2* rot_out, void* stream,
                                const int32_t* table, int page_shift, int num_pages) {
  if (batch_index < 0 || batch_index >= cache_batch)
    return fail(ALPX_EINVAL, "batch_index exceeds the cache batch");
  return attention_prologue_launch(table ? "alpx_attention_layer_prefill_paged"
                                         : "alpx_attention_layer_prefill",
                                   query_gate, key, value, q_norm, k_norm, nullptr, nullptr,
                                   key_cache, value_cache, dtype, capacity, tokens, cache_batch,
                                   batch_index, 1, q_heads, kv_heads, head_dim, value_dim,
                                   position, nullptr, sections, frequency_base, eps, stream, true,
                                   rot_out, table, page_shift, num_pages);
}
}  // namespace alpx

namespace {

// Paged K/V pool of the layer step: pages [num_pages, page_size, Hkv, D],
// block_table [batch, max_pages].
struct LayerPages {
  const int32_t* table;
  int max_pages, page_size, num_pages;
};

// alpx_attention_layer_step over a contiguous cache (pages null) or a paged
// pool: same validation, prologue and split plan.
int layer_step_impl(const char* name, const void* query_gate, const void* key, const void* value,
                    const float* q_norm, const float* k_norm, void* key_cache, void* value_cache,
                    void* out, void* workspace, size_t workspace_bytes, int dtype, int out_dtype,
                    int64_t capacity, int batch, int q_heads, int kv_heads, int head_dim,
                    int64_t position, const int32_t* positions, const int* sections,
                    double frequency_base, float eps, float scale, void* stream,
                    const LayerPages* pages) {
  using namespace alpx;
  if (!query_gate || !key || !value || !q_norm || !k_norm || !key_cache || !value_cache ||
      !out || !workspace || (pages != nullptr && pages->table == nullptr))
    return fail(ALPX_EINVAL, "%s: null buffer", name);
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", name);
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || capacity <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", name);
  if (pages != nullptr && (pages->page_size < kDecodeWaveRows ||
                           (pages->page_size & (pages->page_size - 1)) != 0))
    return fail(ALPX_EINVAL, "page size must be a power of two of at least %d rows",
                kDecodeWaveRows);
  if (q_heads % kv_heads != 0)
    return fail(ALPX_EINVAL, "attention query heads must be a multiple of KV heads");
  if (position < 0 || position >= capacity)
    return fail(ALPX_ERANGE, "attention cache position exceeds capacity");
  if (position + 1 > INT32_MAX)
    return fail(ALPX_EUNSUPPORTED, "%s: cache length above 2^31 - 1", name);
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  int R = 0;
  if (bad_sections(sections, R)) return fail(ALPX_EINVAL, "IMRoPE requires at least one rotary pair");
  if (head_dim < 2 * R) return fail(ALPX_EINVAL, "IMRoPE input is shorter than twice the section sum");
  if (!(frequency_base > 0.0) || !isfinite(frequency_base))
    return fail(ALPX_EINVAL, "frequency_base must be positive and finite");
  if (!(eps > 0.f) || !isfinite(eps)) return fail(ALPX_EINVAL, "epsilon must be positive and finite");
  SplitPrologue pp = {};
  pp.qg = query_gate;
  pp.key = key;
  pp.value = value;
  pp.qw = q_norm;
  pp.kw = k_norm;
  pp.positions = positions;
  pp.position = position;
  pp.R = R;
  for (int i = 0; i < 4; ++i) pp.sec[i] = sections[i];
  pp.eps = eps;
  inverse_frequencies(pp.inv, R, frequency_base, 1.0);
  const int64_t D = head_dim;
  DecodeArgs a = {};
  a.q = query_gate;  // not read by the fused split; its alignment is checked with the rest
  a.k = key_cache;
  a.v = value_cache;
  a.gate = (const char*)query_gate + D * dtype_size(dtype);
  a.gate_stride = 2 * D;
  a.out = out;
  if (pages != nullptr) {  // rows of a page are [Hkv, D]
    a.ks_pos = a.vs_pos = (int64_t)kv_heads * D;
    a.ks_h = a.vs_h = D;
    a.ks_page = a.vs_page = (int64_t)pages->page_size * a.ks_pos;
    a.pages = pages->table;
    a.page_shift = __builtin_ctz((unsigned)pages->page_size);
    a.max_pages = pages->max_pages;
    a.num_pages = pages->num_pages;
  } else {
    a.ks_pos = a.vs_pos = (int64_t)batch * kv_heads * D;
    a.ks_b = a.vs_b = (int64_t)kv_heads * D;
    a.ks_h = a.vs_h = D;
  }
  a.causal_pos0 = -1;
  a.length = (int)(position + 1);
  if (positions != nullptr) {  // sequence b attends rows 0 .. positions[b]
    a.seq_lens = positions;
    a.len_bias = 1;
  }
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.group = q_heads / kv_heads;
  a.key_dim = head_dim;
  a.value_dim = head_dim;
  a.scale_log2 = scale * kLog2e;
  return run_decode(a, dtype, out_dtype, workspace, workspace_bytes, (hipStream_t)stream,
                    ALPX_T_DECODE, ALPX_T_DECODE_COMBINE, &pp);
}

}  // namespace

extern "C" int alpx_attention_layer_step(const void* query_gate, const void* key,
                                         const void* value, const float* q_norm,
                                         const float* k_norm, void* key_cache, void* value_cache,
                                         void* out, void* workspace, size_t workspace_bytes,
                                         int dtype, int out_dtype, int64_t capacity, int batch,
                                         int q_heads, int kv_heads, int head_dim,
                                         int64_t position, const int32_t* positions,
                                         const int* sections,
                                         double frequency_base, float eps, float scale,
                                         void* stream) {
  return layer_step_impl("alpx_attention_layer_step", query_gate, key, value, q_norm, k_norm,
                         key_cache, value_cache, out, workspace, workspace_bytes, dtype,
                         out_dtype, capacity, batch, q_heads, kv_heads, head_dim, position,
                         positions, sections, frequency_base, eps, scale, stream, nullptr);
}

extern "C" int alpx_attention_layer_step_paged(
    const void* query_gate, const void* key, const void* value, const float* q_norm,
    const float* k_norm, void* key_pages, void* value_pages, const int32_t* block_table,
    int max_pages, int page_size, int num_pages, void* out, void* workspace,
    size_t workspace_bytes, int dtype, int out_dtype, int batch, int q_heads, int kv_heads,
    int head_dim, int64_t position, const int32_t* positions, const int* sections,
    double frequency_base, float eps, float scale, void* stream) {
  using namespace alpx;
  if (max_pages <= 0 || num_pages <= 0 || page_size <= 0)
    return fail(ALPX_EINVAL, "alpx_attention_layer_step_paged: sizes must be positive");
  const LayerPages pages = {block_table, max_pages, page_size, num_pages};
  return layer_step_impl("alpx_attention_layer_step_paged", query_gate, key, value, q_norm,
                         k_norm, key_pages, value_pages, out, workspace, workspace_bytes, dtype,
                         out_dtype, (int64_t)max_pages * page_size, batch, q_heads, kv_heads,
                         head_dim, position, positions, sections, frequency_base, eps, scale,
                         stream, &pages);
}

extern "C" size_t alpx_recurrent_step_workspace_bytes(int batch, int key_heads, int value_heads,
                                                      int key_dim, int value_dim) {
  if (batch <= 0 || key_heads <= 0 || value_heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  const size_t b = (size_t)batch;
  const size_t floats = b * (2 * (size_t)key_heads * key_dim + 2 * (size_t)value_heads * value_dim +
                             2 * (size_t)value_heads);
  return floats * sizeof(float) + 256;
}

extern "C" int alpx_recurrent_step(const float* current, const float* conv_weight,
                                   int64_t weight_tap_stride, int64_t weight_channel_stride,
                                   float* conv_history, int conv_kernel, const float* gate,
                                   const float* beta_logits, const float* alpha_logits,
                                   const float* dt_bias, const float* ssm_a,
                                   const float* norm_weight, float* state, void* out,
                                   void* workspace, size_t workspace_bytes, int batch,
                                   int key_heads, int value_heads, int key_dim, int value_dim,
                                   float eps, int out_dtype, void* stream) {
  using namespace alpx;
  if (!current || !conv_weight || (conv_kernel > 1 && !conv_history) || !gate || !beta_logits ||
      !alpha_logits || !dt_bias || !ssm_a || !norm_weight || !state || !out || !workspace)
    return fail(ALPX_EINVAL, "alpx_recurrent_step: null buffer");
  if (!dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_recurrent_step: unknown dtype");
  if (batch <= 0 || key_heads <= 0 || value_heads <= 0 || key_dim <= 0 || value_dim <= 0 ||
      conv_kernel <= 0)
    return fail(ALPX_EINVAL, "alpx_recurrent_step: sizes must be positive");
  if (value_heads % key_heads != 0) return fail(ALPX_EINVAL, "GDN value heads must be a multiple of key heads");
  if (key_dim > 256 || value_dim > kMaxDim)
    return fail(ALPX_EUNSUPPORTED, "alpx_recurrent_step: key dim above 256 or value dim above %d", kMaxDim);
  if (!(eps > 0.f) || !isfinite(eps)) return fail(ALPX_EINVAL, "epsilon must be positive and finite");
  const size_t need = alpx_recurrent_step_workspace_bytes(batch, key_heads, value_heads, key_dim, value_dim);
  if (workspace_bytes < need)
    return fail(ALPX_EINVAL, "alpx_recurrent_step: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  float* base = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  PrepArgs a;
  a.cur = current;
  a.w = conv_weight;
  a.hist = conv_history;
  a.bl = beta_logits;
  a.al = alpha_logits;
  a.dtb = dt_bias;
  a.ssm = ssm_a;
  a.q = base;
  a.k = a.q + (size_t)batch * key_heads * key_dim;
  a.v = a.k + (size_t)batch * key_heads * key_dim;
  a.beta = a.v + (size_t)batch * value_heads * value_dim;
  a.g = a.beta + (size_t)batch * value_heads;
  float* o = a.g + (size_t)batch * value_heads;
  a.w_tap = weight_tap_stride;
  a.w_ch = weight_channel_stride;
  a.B = batch;
  a.K = conv_kernel;
  a.Hk = key_heads;
  a.Hv = value_heads;
  a.Dk = key_dim;
  a.Dv = value_dim;
  a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_RECURRENT_STEP, s);
  // Two launches (recurrent_rows_kernel, recurrent_finish_kernel) when the
  // heads fit launch A; otherwise prep, GDN step and norm separately.
  const bool rows_path = key_dim % 4 == 0 && key_dim <= kRowsDim && ((uintptr_t)state & 15) == 0 &&
                         override_value(ALPX_OVERRIDE_RECURRENT_UNFUSED) == 0;
  if (rows_path) {
    RowsArgs ra;
    ra.p = a;
    ra.state = state;
    ra.o = o;
    ra.scale = gdn_output_scale(key_dim);
    const dim3 grid((unsigned)((value_dim + kRowsPerBlock - 1) / kRowsPerBlock), value_heads, batch);
    if (key_dim <= 128)
      hipLaunchKernelGGL((recurrent_rows_kernel<1>), grid, dim3(kRowsThreads), 0, s, ra);
    else
      hipLaunchKernelGGL((recurrent_rows_kernel<2>), grid, dim3(kRowsThreads), 0, s, ra);
    int rc = check_launch("alpx_recurrent_step rows");
    if (rc != ALPX_OK) return rc;
    FinishArgs fa;
    fa.norm.x = o;
    fa.norm.w = norm_weight;
    fa.norm.gate = gate;
    fa.norm.out = out;
    fa.norm.rows = (int64_t)batch * value_heads;
    fa.norm.grp_rows = fa.norm.rows;
    fa.norm.grp_stride = fa.norm.rows * value_dim;
    fa.norm.n = value_dim;
    fa.norm.eps = eps;
    fa.cur = current;
    fa.hist = conv_history;
    fa.B = batch;
    fa.C = 2 * key_heads * key_dim + value_heads * value_dim;
    fa.K = conv_kernel;
    fa.qk_channels = 2 * key_heads * key_dim;
    const int64_t shift_waves = conv_kernel > 1 ? ((int64_t)batch * fa.qk_channels + 63) / 64 : 0;
    const int64_t fwaves = fa.norm.rows + shift_waves;
    const dim3 fgrid((unsigned)((fwaves + 3) / 4));
    switch (out_dtype) {
      case ALPX_F32: hipLaunchKernelGGL((recurrent_finish_kernel<float>), fgrid, dim3(256), 0, s, fa); break;
      case ALPX_F16: hipLaunchKernelGGL((recurrent_finish_kernel<f16_t>), fgrid, dim3(256), 0, s, fa); break;
      default: hipLaunchKernelGGL((recurrent_finish_kernel<bf16_t>), fgrid, dim3(256), 0, s, fa); break;
    }
    return check_launch("alpx_recurrent_step finish");
  }
  const int64_t waves = (int64_t)batch * (2 * key_heads + value_heads);
  hipLaunchKernelGGL(recurrent_prep_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, a);
  int rc = check_launch("alpx_recurrent_step prep");
  if (rc != ALPX_OK) return rc;
  rc = gdn_step_launch(state, a.q, a.k, a.v, a.beta, a.g, o, batch, key_heads, value_heads,
                       key_dim, value_dim, ALPX_F32, ALPX_F32, s);
  if (rc != ALPX_OK) return rc;
  NormArgs na;
  na.x = o;
  na.w = norm_weight;
  na.gate = gate;
  na.out = out;
  na.rows = (int64_t)batch * value_heads;
  na.grp_rows = na.rows;
  na.grp_stride = na.rows * value_dim;
  na.n = value_dim;
  na.eps = eps;
  return run_norm(na, kNormRmsGate, ALPX_F32, out_dtype, s);
}

extern "C" int alpx_recurrent_prefill_prep(const float* current, const float* conv_weight,
                                           int64_t weight_tap_stride, int64_t weight_channel_stride,
                                           float* conv_history, int conv_kernel,
                                           const float* beta_logits, const float* alpha_logits,
                                           const float* dt_bias, const float* ssm_a, void* q_out,
                                           void* k_out, void* v_out, float* beta_out,
                                           float* log_decay_out, int tokens, int key_heads,
                                           int value_heads, int key_dim, int value_dim, float eps,
                                           int out_dtype, void* stream) {
  using namespace alpx;
  if (!current || !conv_weight || (conv_kernel > 1 && !conv_history) || !beta_logits ||
      !alpha_logits || !dt_bias || !ssm_a || !q_out || !k_out || !v_out || !beta_out ||
      !log_decay_out)
    return fail(ALPX_EINVAL, "alpx_recurrent_prefill_prep: null buffer");
  if (!dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_recurrent_prefill_prep: unknown dtype");
  if (tokens <= 0 || key_heads <= 0 || value_heads <= 0 || key_dim <= 0 || value_dim <= 0 ||
      conv_kernel <= 0)
    return fail(ALPX_EINVAL, "alpx_recurrent_prefill_prep: sizes must be positive");
  if (value_heads % key_heads != 0) return fail(ALPX_EINVAL, "GDN value heads must be a multiple of key heads");
  if (key_dim > kMaxDim || value_dim > kMaxDim)
    return fail(ALPX_EUNSUPPORTED, "alpx_recurrent_prefill_prep: head dims above %d", kMaxDim);
  if (!(eps > 0.f) || !isfinite(eps)) return fail(ALPX_EINVAL, "epsilon must be positive and finite");
  ChunkPrepArgs a;
  a.x = current;
  a.w = conv_weight;
  a.hist = conv_history;
  a.bl = beta_logits;
  a.al = alpha_logits;
  a.dtb = dt_bias;
  a.ssm = ssm_a;
  a.q = q_out;
  a.k = k_out;
  a.v = v_out;
  a.beta = beta_out;
  a.g = log_decay_out;
  a.w_tap = weight_tap_stride;
  a.w_ch = weight_channel_stride;
  a.T = tokens;
  a.K = conv_kernel;
  a.Hk = key_heads;
  a.Hv = value_heads;
  a.Dk = key_dim;
  a.Dv = value_dim;
  a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_LAYER, s);
  const int slots = 2 * key_heads + value_heads;
  const size_t osz = dtype_size(out_dtype);
  const bool tiled = conv_kernel <= kTileTaps && key_dim % 4 == 0 && value_dim % 4 == 0 &&
                     key_dim <= 256 && value_dim <= 256 && aligned(current, 16) &&
                     (conv_kernel == 1 || aligned(conv_history, 16)) &&
                     aligned(q_out, 4 * osz) && aligned(k_out, 4 * osz) && aligned(v_out, 4 * osz);
  if (tiled) {
    const dim3 grid((unsigned)((tokens + kTileTokens - 1) / kTileTokens), (unsigned)slots);
    switch (out_dtype) {
      case ALPX_F32: hipLaunchKernelGGL(recurrent_chunk_prep_tile<float>, grid, dim3(256), 0, s, a); break;
      case ALPX_F16: hipLaunchKernelGGL(recurrent_chunk_prep_tile<f16_t>, grid, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL(recurrent_chunk_prep_tile<bf16_t>, grid, dim3(256), 0, s, a); break;
    }
  } else {
    const int64_t waves = (int64_t)tokens * slots;
    const dim3 grid((unsigned)((waves + 3) / 4));
    switch (out_dtype) {
      case ALPX_F32: hipLaunchKernelGGL(recurrent_chunk_prep_kernel<float>, grid, dim3(256), 0, s, a); break;
      case ALPX_F16: hipLaunchKernelGGL(recurrent_chunk_prep_kernel<f16_t>, grid, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL(recurrent_chunk_prep_kernel<bf16_t>, grid, dim3(256), 0, s, a); break;
    }
  }
  int rc = check_launch("alpx_recurrent_prefill_prep");
  if (rc != ALPX_OK || conv_kernel <= 1) return rc;
  const int C = 2 * key_heads * key_dim + value_heads * value_dim;
  hipLaunchKernelGGL(conv_history_advance, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s,
                     conv_history, current, tokens, conv_kernel, C);
  return check_launch("alpx_recurrent_prefill_prep (history)");
}
