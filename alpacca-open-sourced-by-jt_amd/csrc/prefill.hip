// Causal (optionally windowed) GQA prefill attention.
//
// fp16/bf16 with head_dim 64/128/256 (prefill_mfma): a flash-attention
// forward pass on v_mfma_f32_16x16x32_{f16,bf16}.  A block owns 16*NQB query
// columns per wave x 4 waves, where a column is one (token, query head) pair
// of one kv head's GQA group, so every K/V tile staged in LDS serves all the
// group's heads.  Per 64-key (32 for head_dim 256) tile each wave computes
// S^T = K Q^T (a lane owns one query column and 16 keys of each 16x16 block,
// so the softmax row max is local plus two xor shuffles), applies the causal
// mask only on tiles that straddle a row's diagonal, and accumulates
// O^T += V^T P^T with P taken straight from the score registers and V^T read
// from the row-major LDS tile with transposing reads.  K/V tiles are double
// buffered: the next tile's global loads are in flight while the current
// tile is multiplied.  Tiles entirely above the diagonal are never loaded;
// tiles entirely above one wave's diagonal are skipped by that wave.  Blocks
// are mapped so that one kv head's blocks share one XCD (and its L2), with
// the latest (most expensive) column tiles launched first.
//
// Everything else (fp32, odd head dims, unaligned rows) runs the split-K
// decode machinery in causal mode: query token t is a "sequence" whose
// visible rows are those at absolute positions <= pos0 + t (inside the
// window).
#include <math.h>

#include "alpx_common.h"
#include "decode_internal.h"
#include "timing.h"

namespace alpx {
namespace {

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t ks_pos, vs_pos;  // elements between cache rows (head stride = head_dim)
  int64_t pos0;            // absolute position of query token 0
  int64_t kv_start;        // absolute position of cache row 0
  int window;              // > 0: row at p sees keys in (p - window, p]
  int q_tokens, kv_tokens, q_heads, kv_heads, group;
  int col_tiles;           // column tiles per kv head
  int per_xcd;             // work items per XCD slice of the grid
  float scale_log2;
};

constexpr int kXcds = 8;  // MI355X: workgroup b is dispatched to XCD b % 8

// XCD-aware work mapping.  Work items (kv head, column tile) are ordered
// kv-head-major, heaviest column tile first, and cut into 8 contiguous
// slices, slice x running on XCD x, so the blocks of one kv head share one
// XCD's L2 and its K/V tiles are fetched from HBM once instead of once per
// XCD.  Inside a slice the first half of the dispatch order takes the heavy
// items in descending order and the second half the light items in
// ascending order, so the two blocks that share a CU (dispatched one slice
// pass apart) carry a heavy and a light tile.
__device__ __forceinline__ bool prefill_work(const PrefillArgs& a, int& kvh, int& ctile) {
  const int b = blockIdx.x;
  const int j = b / kXcds;
  const int half = (a.per_xcd + 1) / 2;
  const int rank = j < half ? j : a.per_xcd - 1 - (j - half);
  const int item = (b % kXcds) * a.per_xcd + rank;
  if (item >= a.kv_heads * a.col_tiles) return false;
  kvh = item / a.col_tiles;
  ctile = a.col_tiles - 1 - (item - kvh * a.col_tiles);
  return true;
}

// Scores are compared in the raw (unscaled) domain; the running max of a
// column is only moved when a tile's max exceeds it by more than
// kRescale / (scale log2 e), i.e. p = 2^((s - m) scale log2 e) stays <= 2^8.
// O and l share the stale scale, so the result is exact; the rescale
// multiplies (64 per tile) are skipped on almost every tile.
constexpr float kRescale = 8.0f;

template <typename T, typename TO, int D, int BK, int NQB>
__global__ void __launch_bounds__(256, 2)
prefill_mfma(PrefillArgs a) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec4<T>::type V4;
  // LDS row strides (elements).  K rows are read 16 B per lane, 16 rows at a
  // time: a 16-byte bank shift per row keeps 8 consecutive rows on distinct
  // banks.  V rows are read by 4-row transposing reads of 32 B per row: a
  // 32-byte shift keeps those 4 rows on distinct banks.
  constexpr int kStride = D + 8;
  constexpr int kVStride = D + 16;
  constexpr int kTileElems = BK * kVStride;
  constexpr int kUnits = D / 8;           // 16-byte units per row
  constexpr int kUPT = BK * kUnits / 256; // units per thread per tensor per tile
  constexpr int KB = BK / 16;
  constexpr int KK = BK / 32;
  constexpr int MB = D / 16;
  constexpr int KS = D / 32;
  constexpr int kWaveCols = 16 * NQB;
  constexpr int kCols = 4 * kWaveCols;
  static_assert(kUPT >= 1 && BK * kUnits % 256 == 0, "tile must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) T smem[4 * kTileElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane & 15;
  const int quad = lane >> 4;
  int kvh, ctile;
  if (!prefill_work(a, kvh, ctile)) return;
  const int G = a.group;
  const int cols = a.q_tokens * G;
  const int col0 = ctile * kCols;
  const int wcol0 = col0 + kWaveCols * wave;

  int tok[NQB], hq[NQB];
  bool cok[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int c = wcol0 + 16 * qb + hl;
    cok[qb] = c < cols;
    const int cc = cok[qb] ? c : cols - 1;
    tok[qb] = cc / G;
    hq[qb] = kvh * G + (cc - tok[qb] * G);
  }
  // Positions relative to the first cache row: key j is visible to query
  // token t iff j <= rel0 + t (and j > rel0 + t - window).
  const int rel0 = (int)(a.pos0 - a.kv_start);
  const int bt_first = col0 / G;
  const int bt_last = (min(col0 + kCols, cols) - 1) / G;
  const int wt_first = min(wcol0, cols - 1) / G;
  const int wt_last = (min(wcol0 + kWaveCols, cols) - 1) / G;

  // Key rows [lo, hi) that any column of the block can see.
  const int hi = max(0, min(a.kv_tokens, rel0 + bt_last + 1));
  int lo = 0;
  if (a.window > 0) lo = min(hi, max(0, rel0 + bt_first - a.window + 1)) / BK * BK;

  // B operand of S^T = K Q^T: lane holds Q[column][32 ks + 8 quad + 0..7].
  V8 qv[NQB][KS];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const T* qp = (const T*)a.q + ((int64_t)tok[qb] * a.q_heads + hq[qb]) * D + 8 * quad;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const V8 x = *(const V8*)(qp + 32 * ks);
      qv[qb][ks] = cok[qb] ? x : (V8){};
    }
  }

  f32x4 o[NQB][MB];  // O^T[d = 16 mb + 4 quad + i][column]
  float m[NQB], l[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) o[qb][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  const float c2 = a.scale_log2;
  const float thr = kRescale / c2;

  const T* kg = (const T*)a.k + (int64_t)kvh * D;
  const T* vg = (const T*)a.v + (int64_t)kvh * D;
  // Tile loads are raw buffer loads: a per-tile scalar resource (base = row
  // k0) plus per-thread constant byte offsets, so no per-tile vector address
  // arithmetic.  Rows at or past kv_tokens read as zero (masked anyway).
  int urow[kUPT];
  uint32_t kofs[kUPT], vofs[kUPT];
#pragma unroll
  for (int u = 0; u < kUPT; ++u) {
    const int idx = u * 256 + tid;
    urow[u] = idx / kUnits;
    const int c = idx - urow[u] * kUnits;
    kofs[u] = (uint32_t)((urow[u] * a.ks_pos + 8 * c) * (int64_t)sizeof(T));
    vofs[u] = (uint32_t)((urow[u] * a.vs_pos + 8 * c) * (int64_t)sizeof(T));
  }
  V8 kreg[kUPT], vreg[kUPT];
  auto gload = [&](int k0) {
    const uint32_t rows = (uint32_t)(a.kv_tokens - k0);
    const __amdgpu_buffer_rsrc_t kr =
        buffer_rsrc(kg + (int64_t)k0 * a.ks_pos, (uint32_t)(rows * a.ks_pos * sizeof(T)));
    const __amdgpu_buffer_rsrc_t vr =
        buffer_rsrc(vg + (int64_t)k0 * a.vs_pos, (uint32_t)(rows * a.vs_pos * sizeof(T)));
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      kreg[u] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(kr, kofs[u], 0, 0));
      vreg[u] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(vr, vofs[u], 0, 0));
    }
  };
  auto lstore = [&](int buf) {
    T* Kd = smem + 2 * buf * kTileElems;
    T* Vd = Kd + kTileElems;
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int idx = u * 256 + tid;
      const int r = urow[u];
      const int c = idx - r * kUnits;
      *(V8*)(Kd + r * kStride + 8 * c) = kreg[u];
      *(V8*)(Vd + r * kVStride + 8 * c) = vreg[u];
    }
  };

  if (lo < hi) {
    gload(lo);
    lstore(0);
  }
  __syncthreads();
  const int tr_row = 4 * quad + (hl >> 2);
  const int tr_col = 4 * (hl & 3);
  int buf = 0;
  for (int k0 = lo; k0 < hi; k0 += BK) {
    const bool next = k0 + BK < hi;
    if (next) gload(k0 + BK);
    const bool skip = k0 > rel0 + wt_last ||
                      (a.window > 0 && k0 + BK - 1 <= rel0 + wt_first - a.window);
    if (!skip) {
      // The mask is needed only on tiles that straddle a row's diagonal or
      // window edge, or run past the last row; the branch is wave-uniform.
      const bool need_mask = k0 + BK - 1 > rel0 + wt_first || k0 + BK > hi ||
                             (a.window > 0 && k0 <= rel0 + wt_last - a.window);
      const T* Ks = smem + 2 * buf * kTileElems;
      const T* Vs = Ks + kTileElems;
      f32x4 sc[KB][NQB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const V8 ka = *(const V8*)(Ks + (16 * kb + hl) * kStride + 8 * quad);
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
          sc[kb][qb] = mfma16x16x32(ka, qv[qb][0], (f32x4){0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int ks = 1; ks < KS; ++ks) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const V8 ka = *(const V8*)(Ks + (16 * kb + hl) * kStride + 32 * ks + 8 * quad);
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) sc[kb][qb] = mfma16x16x32(ka, qv[qb][ks], sc[kb][qb]);
        }
      }
      if (__builtin_expect(need_mask, 0)) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const int qrel = rel0 + tok[qb];
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = k0 + 16 * kb + 4 * quad + i;
              const bool ok = key < hi && key <= qrel && (a.window <= 0 || key > qrel - a.window);
              sc[kb][qb][i] = ok ? sc[kb][qb][i] : -INFINITY;
            }
          }
        }
      }
      V8 pv[KK][NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float mx = sc[0][qb][0];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][qb][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const bool grow = mx > m[qb] + thr;
        if (__ballot(grow) != 0) {  // rare: move the reference max and rescale
          const float mn = grow ? mx : m[qb];
          const float alpha = m[qb] == -INFINITY ? 0.f : fast_exp2((m[qb] - mn) * c2);
          l[qb] *= alpha;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) o[qb][mb] *= alpha;
          m[qb] = mn;
        }
        const float mc = m[qb] == -INFINITY ? 0.f : m[qb] * c2;
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(__builtin_fmaf(sc[kb][qb][i], c2, -mc));
            ps += p;
            pv[kb >> 1][qb][4 * (kb & 1) + i] = from_f32<T>(p);
          }
        }
        l[qb] += ps;
      }
      // O^T += V^T P^T; rows 32 kk + 16 h + 4 quad + 0..3 via transposing reads.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const V4 v0 = lds_read_tr4(Vs + (32 * kk + tr_row) * kVStride + 16 * mb + tr_col);
          const V4 v1 = lds_read_tr4(Vs + (32 * kk + 16 + tr_row) * kVStride + 16 * mb + tr_col);
          const V8 va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) o[qb][mb] = mfma16x16x32(va, pv[kk][qb], o[qb][mb]);
        }
      }
    }
    if (next) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    float lt = l[qb] + __shfl_xor(l[qb], 16);
    lt += __shfl_xor(lt, 32);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (!cok[qb]) continue;
    TO* op = (TO*)a.out + ((int64_t)tok[qb] * a.q_heads + hq[qb]) * D + 4 * quad;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) op[16 * mb + i] = from_f32<TO>(o[qb][mb][i] * inv);
    }
  }
}

template <typename T, typename TO>
const void* pick_kernel(int D) {
  switch (D) {
    case 64: return (const void*)prefill_mfma<T, TO, 64, 64, 2>;
    case 128: return (const void*)prefill_mfma<T, TO, 128, 64, 2>;
    case 256: return (const void*)prefill_mfma<T, TO, 256, 32, 1>;
  }
  return nullptr;
}

template <typename T>
const void* pick_kernel_out(int D, int out_dtype) {
  switch (out_dtype) {
    case ALPX_F32: return pick_kernel<T, float>(D);
    case ALPX_F16: return pick_kernel<T, f16_t>(D);
    default: return pick_kernel<T, bf16_t>(D);
  }
}

}  // namespace
}  // namespace alpx

extern "C" size_t alpx_prefill_workspace_bytes(int q_tokens, int q_heads, int kv_heads,
                                               int value_dim, int kv_tokens) {
  using namespace alpx;
  if (q_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || value_dim <= 0 || kv_tokens <= 0 ||
      q_heads % kv_heads != 0)
    return 0;
  return decode_workspace(q_tokens, q_heads, kv_heads, value_dim, kv_tokens);
}

extern "C" int alpx_prefill_causal(const void* q, const void* key, const void* value, void* out,
                                   void* workspace, size_t workspace_bytes, int q_tokens,
                                   int kv_tokens, int q_heads, int kv_heads, int key_dim,
                                   int value_dim, int64_t k_pos_stride, int64_t v_pos_stride,
                                   int64_t q_pos0, int window, int64_t kv_start, float scale,
                                   int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  if (!q || !key || !value || !out) return fail(ALPX_EINVAL, "alpx_prefill_causal: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(ALPX_EINVAL, "alpx_prefill_causal: unknown dtype");
  if (q_tokens <= 0 || kv_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || key_dim <= 0 ||
      value_dim <= 0)
    return fail(ALPX_EINVAL, "alpx_prefill_causal: sizes must be positive");
  if (q_heads % kv_heads != 0)
    return fail(ALPX_EINVAL, "attention query heads must be a multiple of KV heads");
  if (k_pos_stride < (int64_t)kv_heads * key_dim || v_pos_stride < (int64_t)kv_heads * value_dim)
    return fail(ALPX_EINVAL, "alpx_prefill_causal: row strides smaller than a row");
  if (q_pos0 < 0 || kv_start < 0 || window < 0)
    return fail(ALPX_EINVAL, "alpx_prefill_causal: negative position or window");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  if (key_dim > 256 || value_dim > 256)
    return fail(ALPX_EUNSUPPORTED, "alpx_prefill_causal: head dims above 256 are not supported");

  hipStream_t s = (hipStream_t)stream;
  const int group = q_heads / kv_heads;
  const size_t es = dtype_size(dtype);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)key | (uintptr_t)value |
                          (uintptr_t)(k_pos_stride * es) | (uintptr_t)(v_pos_stride * es);
  const bool mfma = dtype != ALPX_F32 && key_dim == value_dim &&
                    (key_dim == 64 || key_dim == 128 || key_dim == 256) && (align & 15) == 0 &&
                    getenv("ALPX_PREFILL_GENERIC") == nullptr;
  // the MFMA kernel forms per-tile row offsets in 32 bits
  const bool offsets_fit = (int64_t)kv_tokens * k_pos_stride * (int64_t)es < ((int64_t)1 << 31) &&
                           (int64_t)kv_tokens * v_pos_stride * (int64_t)es < ((int64_t)1 << 31) &&
                           q_pos0 - kv_start < ((int64_t)1 << 30) && q_pos0 - kv_start > -((int64_t)1 << 30);
  if (mfma && offsets_fit) {
    const void* kernel = nullptr;
    if (dtype == ALPX_F16)
      kernel = pick_kernel_out<f16_t>(key_dim, out_dtype);
    else
      kernel = pick_kernel_out<bf16_t>(key_dim, out_dtype);
    PrefillArgs a;
    a.q = q;
    a.k = key;
    a.v = value;
    a.out = out;
    a.ks_pos = k_pos_stride;
    a.vs_pos = v_pos_stride;
    a.pos0 = q_pos0;
    a.kv_start = kv_start;
    a.window = window;
    a.q_tokens = q_tokens;
    a.kv_tokens = kv_tokens;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.group = group;
    const int cols_per_block = key_dim == 256 ? 64 : 128;
    const int64_t cols = (int64_t)q_tokens * group;
    a.col_tiles = (int)((cols + cols_per_block - 1) / cols_per_block);
    const int64_t items = (int64_t)a.col_tiles * kv_heads;
    a.per_xcd = (int)((items + kXcds - 1) / kXcds);
    a.scale_log2 = scale * kLog2e;
    TimedRegion timed(ALPX_T_PREFILL, s);
    void* args[] = {(void*)&a};
    hipError_t err = hipLaunchKernel(kernel, dim3(a.per_xcd * kXcds), dim3(256), args, 0, s);
    if (err != hipSuccess)
      return fail(ALPX_EHIP, "prefill launch failed: %s", hipGetErrorString(err));
    return check_launch("prefill_mfma");
  }

  if (!workspace) return fail(ALPX_EINVAL, "alpx_prefill_causal: null workspace");
  DecodeArgs a = {};
  a.q = q;
  a.k = key;
  a.v = value;
  a.seq_lens = nullptr;
  a.gate = nullptr;
  a.out = out;
  a.ks_pos = k_pos_stride;
  a.ks_b = 0;
  a.ks_h = key_dim;
  a.vs_pos = v_pos_stride;
  a.vs_b = 0;
  a.vs_h = value_dim;
  a.causal_pos0 = q_pos0;
  a.kv_start = kv_start;
  a.window = window;
  a.length = kv_tokens;
  a.batch = q_tokens;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.group = group;
  a.key_dim = key_dim;
  a.value_dim = value_dim;
  a.scale_log2 = scale * kLog2e;
  return run_decode(a, dtype, out_dtype, workspace, workspace_bytes, s, ALPX_T_PREFILL,
                    ALPX_T_AUX);
}
