// Split-K flash-decode for single-token GQA attention, plus the combine pass.
//
// Pass 1 (split): the cache rows of one (sequence, kv head) are cut into
// chunks, one per block; each block streams its rows once and produces an
// online-softmax partial (running max m in the base-2 domain, running sum l,
// unnormalised accumulator acc[Dv]) for every query head of the GQA group.
// K and V are read exactly once per group, so the 4 (Llama-3-8B) or 8
// (Qwen3.5) query heads of a group share each byte.  The grid is sized from
// the occupancy API: one round of resident blocks, or (16-bit caches, two
// or more blocks per CU, long chunks) several rounds of shorter chunks that
// the dispatcher balances over the CUs.
//
//  * fp16/bf16, head_dim 64/128/256 (decode_split_mfma): 4 wavefronts per
//    block, 32 rows per wave step.  K and V rows are fetched row-major with
//    128-bit buffer loads (whole lines per load) and staged in a per-wave
//    LDS tile.  K is read back as the A operand of
//    v_mfma_f32_16x16x32_{f16,bf16} (S^T = K Q^T: 16 rows x 16 query heads
//    per instruction), so scores need no cross-lane dot-product reduction;
//    V is read back with transposing LDS reads as the A operand of
//    O^T = V^T P^T, so the probabilities never leave the registers the
//    score MFMA wrote them to.  The softmax max is a 2-step cross-lane
//    (xor 16, xor 32) reduction.
//  * everything else (fp32, odd head dims, unaligned caches):
//    decode_split_generic, one wavefront per block, VALU dot products.
//
// Pass 2 (combine): per (sequence, query head, 64 output columns), merge the
// block partials with weights 2^(m_s - M), divide by the merged sum, apply
// the optional sigmoid output gate and store in the output dtype.  (A
// single-launch variant where the last block of a group merges was measured
// 2.4x slower: the device-scope release/acquire fences it needs write back
// and invalidate the XCD L2 in every block.)
#include <math.h>

#include <mutex>

#include "alpx_common.h"
#include "decode_internal.h"
#include "rope_internal.h"
#include "timing.h"

namespace alpx {
namespace {

constexpr int kTile = kDecodeWaveRows;  // rows per wavefront step (MFMA path)
// Lazy softmax reference of the MFMA split kernel: P stays <= 2^8.
constexpr float kDecodeRescale = 8.0f;
// Buffer-load cache policy: nontemporal (V is streamed once per step).
constexpr int kAuxNontemporal = 2;
constexpr int kWaves = 4;   // wavefronts (= slots) per block (MFMA path)
constexpr int kGenericTile = 64;
constexpr int kMaxSlots = 2048;
// Wave tile rows of the fp32 MFMA split kernel.
constexpr int f32_tile_rows(int d) { return d == 64 ? 32 : 16; }
constexpr int kMaxResident = 8192;  // upper bound on resident blocks any plan assumes


// Rows [seq_lo, seq_len) of sequence b are attended.  Decode: [0, len_b).
// Causal mode (prefill through this path): "sequence" b is query token b at
// absolute position causal_pos0 + b; cache row j sits at kv_start + j and is
// visible iff kv_start + j <= pos and, with a window, > pos - window.
__device__ __forceinline__ int seq_len(const DecodeArgs& a, int b) {
  int64_t n;
  if (a.causal_pos0 >= 0)
    n = a.causal_pos0 + b + 1 - a.kv_start;
  else
    n = a.seq_lens == nullptr ? a.length : (int64_t)a.seq_lens[b] + a.len_bias;
  n = n < 0 ? 0 : n;
  return (int)(n > a.length ? a.length : n);
}

__device__ __forceinline__ int seq_lo(const DecodeArgs& a, int b, int hi) {
  if (a.causal_pos0 < 0 || a.window <= 0) return 0;
  int64_t n = a.causal_pos0 + b - a.window + 1 - a.kv_start;
  n = n < 0 ? 0 : n;
  return (int)(n > hi ? hi : n);
}

// ------------------------------------------------------------ balanced plan
//
// Ragged decode (device seq_lens) plans its split from the device lengths:
// the valid rows of all sequences are cut into chunks of one size C (the
// total over items_target, rounded up to a whole block step) and block x of
// a grid row takes the x-th (sequence, chunk) item, items listed in
// sequence order.  Every block streams at most C rows whatever the spread
// of the lengths, so the step time follows the total row count, not the
// longest sequence.  Since sum_b ceil(len_b / C) <= total / C + batch <=
// items_target + batch, the grid (items_max = items_target + batch) holds
// every item; blocks past the last item exit.  The functions below are
// wave-collective (every lane of the calling wave active) and every wave
// that calls them gets the same result.

__device__ __forceinline__ int64_t wave_sum(int64_t x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  return x;
}

// Common chunk size C of the balanced plan; n0 is the length of sequence
// `lane` (the first 64 sequences: most batches need no second load).
__device__ __forceinline__ int balanced_chunk(const DecodeArgs& a, int lane, int& n0) {
  n0 = lane < a.batch ? seq_len(a, lane) : 0;
  int64_t total = n0;
  for (int b0 = 64; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    if (b < a.batch) total += seq_len(a, b);
  }
  total = wave_sum(total);
  // 32-bit divisions where the row total allows (the 64-bit ones are long
  // instruction sequences on the path to every block's first tile loads)
  int64_t c;
  if (total <= 0x7fffffff - a.items_target) {
    const unsigned q = ((unsigned)total + (unsigned)a.items_target - 1u) / (unsigned)a.items_target;
    c = (q + (unsigned)a.unit - 1u) / (unsigned)a.unit * (unsigned)a.unit;
  } else {
    c = (total + a.items_target - 1) / a.items_target;
    c = (c + a.unit - 1) / a.unit * a.unit;
  }
  return c < a.unit ? a.unit : (int)c;
}

// Item `item` of the balanced plan: its sequence (-1 past the last item)
// and cache rows [start, end) (chunk start / C of its sequence).
__device__ __forceinline__ void balanced_item(const DecodeArgs& a, int item, int& b_out,
                                              int& start, int& end, int& chunk_out) {
  const int lane = threadIdx.x & 63;
  int n0;
  const int chunk = balanced_chunk(a, lane, n0);
  chunk_out = chunk;
  b_out = -1;
  start = end = 0;
  int base = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    const int n = b0 == 0 ? n0 : (b < a.batch ? seq_len(a, b) : 0);
    const int cnt = (n + chunk - 1) / chunk;
    const int incl = wave_inclusive_scan(cnt, lane);
    const int excl = incl - cnt;
    const bool mine = cnt > 0 && item >= base + excl && item < base + incl;
    const unsigned long long hit = __ballot(mine);
    if (hit != 0) {
      const int src = __ffsll((long long)hit) - 1;
      b_out = __shfl(b, src);
      start = (item - base - __shfl(excl, src)) * chunk;
      end = min(start + chunk, __shfl(n, src));
      return;
    }
    base += __shfl(incl, 63);
  }
}

// Item count of sequence b in the balanced plan.
__device__ __forceinline__ int balanced_count(const DecodeArgs& a, int want_b) {
  const int lane = threadIdx.x & 63;
  int n0;
  const int chunk = balanced_chunk(a, lane, n0);
  const int n = want_b < 64 ? __shfl(n0, want_b) : seq_len(a, want_b);
  return (n + chunk - 1) / chunk;
}

// The block's sequence, cache rows [start, end) (b < 0: nothing to do)
// and split slot: partial (b, h, slot) is written at (b * Hq + h) * nsplit
// + slot.  Uniform plan: slot = blockIdx.x.  Balanced plan: the chunk's
// index within its sequence (nsplit bounds the items of one sequence).
__device__ __forceinline__ void block_rows(const DecodeArgs& a, int& b, int& start, int& end,
                                           int& slot) {
  if (a.balanced) {
    int chunk;
    balanced_item(a, blockIdx.x, b, start, end, chunk);
    slot = b < 0 ? 0 : start / chunk;
  } else {
    b = blockIdx.z;
    const int len = seq_len(a, b);
    const int x = blockIdx.x;
    // with a skew, the even slot of each pair takes chunk + skew rows
    const int s0 = x * a.chunk + ((x & 1) ? a.skew : 0);
    const int e0 = x * a.chunk + a.chunk + ((x & 1) ? 0 : a.skew);
    start = max(s0, seq_lo(a, b, len));
    end = min(e0, len);
    slot = x;
  }
  b = __builtin_amdgcn_readfirstlane(b);
  start = __builtin_amdgcn_readfirstlane(start);
  end = __builtin_amdgcn_readfirstlane(end);
  slot = __builtin_amdgcn_readfirstlane(slot);
}

__device__ __forceinline__ int64_t partial_slot(const DecodeArgs& a, int b, int h, int slot) {
  return ((int64_t)b * a.q_heads + h) * a.nsplit + slot;
}

// Element offset of cache row `row` of sequence b, kv head kvh (page lookup
// for paged caches; a table entry outside [0, num_pages) is clamped, so a
// bad table reads a wrong page but never leaves the page pool).
__device__ __forceinline__ int64_t row_offset(const DecodeArgs& a, int b, int kvh, int row,
                                              int64_t s_pos, int64_t s_b, int64_t s_h,
                                              int64_t s_page) {
  if (a.pages == nullptr) return (int64_t)b * s_b + (int64_t)kvh * s_h + (int64_t)row * s_pos;
  int pg = a.pages[(int64_t)b * a.max_pages + (row >> a.page_shift)];
  pg = min(max(pg, 0), a.num_pages - 1);
  return (int64_t)pg * s_page + (int64_t)kvh * s_h +
         (int64_t)(row & ((1 << a.page_shift) - 1)) * s_pos;
}

__device__ __forceinline__ void wave_sync_lds() {
  // LDS operations of one wavefront complete in issue order; this only
  // stops the compiler from moving LDS accesses across the point.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// End of a split block: merge the four waves' online-softmax states (same
// lane layout: O^T[d = 16 mb + 4 quad + i][head hl]) through LDS into wave
// 0, which writes the block's partial (m, l, acc) for its live heads.
template <int D>
__device__ __forceinline__ void merge_waves(const DecodeArgs& a, char* smem, f32x4 (&o)[D / 16],
                                            float m, float l, int wave, int lane, bool head_ok,
                                            int b, int h, int slot) {
  constexpr int kMergeO = (kWaves - 1) * (D / 16) * 64 * 4;   // floats
  const int quad = lane >> 4;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  __syncthreads();
  float* mf = (float*)smem;
  float* mm = mf + kMergeO;
  float* ml = mm + (kWaves - 1) * 64;
  if (wave > 0) {
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb)
      *(f32x4*)(mf + (((wave - 1) * (D / 16) + mb) * 64 + lane) * 4) = o[mb];
    mm[(wave - 1) * 64 + lane] = m;
    ml[(wave - 1) * 64 + lane] = l;
  }
  __syncthreads();
  if (wave == 0) {
    float mw[kWaves - 1];
    float M = m;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) {
      mw[w] = mm[w * 64 + lane];
      M = fmaxf(M, mw[w]);
    }
    const bool any = M != -INFINITY;
    const float c0 = any ? fast_exp2(m - M) : 0.f;
    float L = l * c0;
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) o[mb] *= c0;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) {
      const float cw = any ? fast_exp2(mw[w] - M) : 0.f;
      L += ml[w * 64 + lane] * cw;
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb)
        o[mb] += cw * *(const f32x4*)(mf + ((w * (D / 16) + mb) * 64 + lane) * 4);
    }
    if (head_ok) {
      const int64_t pidx = partial_slot(a, b, h, slot);
      if (quad == 0) {
        a.part_m[pidx] = M;
        a.part_l[pidx] = L;
      }
      float* pa = a.part_acc + pidx * D + 4 * quad;
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) *(f32x4*)(pa + 16 * mb) = o[mb];
    }
  }
}

// Bytes of LDS a split block needs for the final merge.
template <int D>
constexpr int merge_lds_bytes() {
  return 4 * ((kWaves - 1) * (D / 16) * 64 * 4 + 2 * (kWaves - 1) * 64);
}

// ------------------------------------------------------------ MFMA split

// One block = 4 wavefronts sharing one chunk of rows of one (sequence, kv
// head, 16-head column block).  Wave w takes the 32-row tiles w, w+4, ...
// K and V rows are fetched row-major (16 lanes cover one 256-byte row at
// head_dim 128), so every 128-byte line is consumed by the instruction that
// fetches it; both tiles are staged in the wave's LDS slot, K read back as
// MFMA A operands, V with transposing reads.  V loads carry the nontemporal
// hint (V is read once per step); measured on C2, the hint on V alone gives
// the best rate, and adding it to K lowers it.
// The next tile's loads are issued as soon as the current tile is staged,
// so every wave keeps a tile in flight.  At the end the four waves' online
// softmax states are merged through LDS into one partial per block.
//
// PRO: the Qwen3.5 attention prologue runs in the same launch.  Every block
// forms its query heads from the joint projection (RMSNorm x weight, IMROPE
// at the new token's position, by norm_rope as in the prologue kernel) into
// LDS.  The blocks whose chunk holds the new row form that key row the same
// way and put it and the value row into their staged tile in LDS, over
// whatever their own loads fetched of that row; the one with head chunk 0
// also writes both rows to the cache.
template <typename T, int D, bool PAGED, bool PRO>
__device__ __forceinline__ void split_body(const DecodeArgs& a, const SplitPrologue* pp) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec4<T>::type V4;
  constexpr int kStride = D + 8;          // LDS row stride (elements), 16-byte aligned rows
  constexpr int kUnits = D / 8;           // 16-byte units per row
  constexpr int kIters = kTile * kUnits / 64;
  constexpr int kTileElems = kTile * kStride;
  constexpr int kTileBytes = 2 * kWaves * kTileElems * (int)sizeof(T);
  constexpr int kLdsBytes = kTileBytes > merge_lds_bytes<D>() ? kTileBytes : merge_lds_bytes<D>();
  // PRO: 16 query rows and the new key and value rows (T), then one float
  // row per wave for the rotation partners.
  constexpr int kProBytes = PRO ? (16 + 2) * D * (int)sizeof(T) + kWaves * D * 4 : 0;
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes + kProBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int b, start, end, slot;
  block_rows(a, b, start, end, slot);
  if (b < 0) return;  // past the last item of a balanced plan (whole block)
  const int hc = blockIdx.y % a.head_chunks;
  const int kvh = blockIdx.y / a.head_chunks;
  const int hl = lane & 15;  // query-head column (N index) of this lane
  const int quad = lane >> 4;
  const int g_in = hc * 16 + hl;
  const bool head_ok = g_in < a.group;
  const int h = kvh * a.group + (head_ok ? g_in : 0);

  // B operand of S^T = K Q^T: lane holds Q[h][32 ks + 8 quad + 0..7].
  V8 qv[D / 32];
  [[maybe_unused]] bool owns_new = false;  // PRO: the new row is in this block's chunk
  [[maybe_unused]] const T* new_kv = nullptr;  // PRO: new key row, then value row (LDS)
  if constexpr (PRO) {
    constexpr int kPer = D / 64;
    T* qrows = (T*)(smem + kLdsBytes);
    T* nkv = qrows + 16 * D;
    float* stage = (float*)(nkv + 2 * D) + wave * D;
    const int64_t pos = pp->positions ? (int64_t)pp->positions[b] : pp->position;
    owns_new = pos >= start && pos < end;
    new_kv = nkv;
    if (owns_new && wave < 2) {
      const int64_t src_row = ((int64_t)b * a.kv_heads + kvh) * D;  // [B, Hkv, D]
      if (wave == 0) {
        const T* src = (const T*)pp->key + src_row;
        float x[kPer], wt[kPer];
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
          x[e] = to_f32(src[lane + 64 * e]);
          wt[e] = pp->kw[lane + 64 * e];
        }
        norm_rope<T, kPer>(x, wt, D, pp->eps, pp->sec, pp->R, pp->inv, (double)pos, stage, nkv,
                           lane);
      } else {
        const T* src = (const T*)pp->value + src_row;
#pragma unroll
        for (int e = 0; e < kPer; ++e) nkv[D + lane + 64 * e] = src[lane + 64 * e];
      }
      if (hc == 0) {
        // this wave's own LDS stores above are done before these reads
        __builtin_amdgcn_wave_barrier();
        T* dst = nullptr;
        if constexpr (PAGED) {
          // the row's page; a table entry outside the pool writes nothing
          // (the reads clamp such entries, a write must not land elsewhere)
          const int pg = a.pages[(int64_t)b * a.max_pages + (int)(pos >> a.page_shift)];
          const int64_t in_page = pos & ((1 << a.page_shift) - 1);
          if (pg >= 0 && pg < a.num_pages)
            dst = wave == 0 ? (T*)a.k + pg * a.ks_page + in_page * a.ks_pos + (int64_t)kvh * a.ks_h
                            : (T*)a.v + pg * a.vs_page + in_page * a.vs_pos + (int64_t)kvh * a.vs_h;
        } else {
          dst = wave == 0 ? (T*)a.k + pos * a.ks_pos + (int64_t)b * a.ks_b + (int64_t)kvh * a.ks_h
                          : (T*)a.v + pos * a.vs_pos + (int64_t)b * a.vs_b + (int64_t)kvh * a.vs_h;
        }
        if (dst != nullptr) {
#pragma unroll
          for (int e = 0; e < kPer; ++e) dst[lane + 64 * e] = nkv[wave * D + lane + 64 * e];
        }
      }
    }
    // query heads hc * 16 + j of this kv group, one wave per head
    for (int j = wave; j < 16; j += kWaves) {
      const int g = hc * 16 + j;
      if (g >= a.group) break;
      const T* src = (const T*)pp->qg + ((int64_t)b * a.q_heads + kvh * a.group + g) * (2 * D);
      float x[kPer], wt[kPer];
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        x[e] = to_f32(src[lane + 64 * e]);
        wt[e] = pp->qw[lane + 64 * e];
      }
      norm_rope<T, kPer>(x, wt, D, pp->eps, pp->sec, pp->R, pp->inv, (double)pos, stage,
                         qrows + j * D, lane);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      const V8 x = *(const V8*)(qrows + hl * D + 32 * ks + 8 * quad);
      qv[ks] = head_ok ? x : (V8){};
    }
  } else {
    const T* qp = (const T*)a.q + ((int64_t)b * a.q_heads + h) * D + 8 * quad;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      V8 x = *(const V8*)(qp + 32 * ks);
      qv[ks] = head_ok ? x : (V8){};
    }
  }

  f32x4 o[D / 16];  // O^T[d = 16 mb + 4 quad + i][head hl]
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) o[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;
  float l = 0.f;

  const T* kbase = (const T*)a.k + (int64_t)b * a.ks_b + (int64_t)kvh * a.ks_h;
  const T* vbase = (const T*)a.v + (int64_t)b * a.vs_b + (int64_t)kvh * a.vs_h;
  T* ldsk = (T*)smem + 2 * wave * kTileElems;
  T* ldsv = ldsk + kTileElems;

  V8 kr[kIters];  // K rows, 16 bytes per lane, row-major
  V8 vr[kIters];  // V rows, same layout
  // Tile loads are raw buffer loads from the tile's first row: load `it`
  // covers rows kRowsPerLoad * it + lane / kUnits, 16-byte unit lane %
  // kUnits, so a lane's byte offset is its base plus it * (row step), one
  // add per load.  The buffer ends at row `end`: rows past it read as zero
  // (their scores are masked, their P is zero).
  constexpr int kRowsPerLoad = 64 / kUnits;
  const uint32_t koff = (uint32_t)(((lane / kUnits) * a.ks_pos + 8 * (lane % kUnits)) * (int64_t)sizeof(T));
  const uint32_t voff = (uint32_t)(((lane / kUnits) * a.vs_pos + 8 * (lane % kUnits)) * (int64_t)sizeof(T));
  const uint32_t kstep = (uint32_t)(kRowsPerLoad * a.ks_pos * (int64_t)sizeof(T));
  const uint32_t vstep = (uint32_t)(kRowsPerLoad * a.vs_pos * (int64_t)sizeof(T));
  auto load_tile = [&](int p) {
    // Paged: a wave tile starts at a multiple of kTile and never crosses a
    // page (page size a multiple of kTile), so its page is looked up once.
    const T* kt = kbase + (int64_t)p * a.ks_pos;
    const T* vt = vbase + (int64_t)p * a.vs_pos;
    if constexpr (PAGED) {
      kt = (const T*)a.k + row_offset(a, b, kvh, p, a.ks_pos, 0, a.ks_h, a.ks_page);
      vt = (const T*)a.v + row_offset(a, b, kvh, p, a.vs_pos, 0, a.vs_h, a.vs_page);
    }
    const int rows = min(end - p, kTile);
    const __amdgpu_buffer_rsrc_t kres = buffer_rsrc(kt, (uint32_t)(rows * a.ks_pos * (int64_t)sizeof(T)));
    const __amdgpu_buffer_rsrc_t vres = buffer_rsrc(vt, (uint32_t)(rows * a.vs_pos * (int64_t)sizeof(T)));
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      kr[it] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(kres, koff + it * kstep, 0, 0));
      vr[it] = __builtin_bit_cast(
          V8, __builtin_amdgcn_raw_buffer_load_b128(vres, voff + it * vstep, 0, kAuxNontemporal));
    }
  };

  int p0 = start + kTile * wave;
  if (p0 < end) load_tile(p0);
  while (p0 < end) {
    const int pn = p0 + kTile * kWaves;
    // Stage K and V in LDS (row-major, padded rows), then prefetch the next tile.
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int u = it * 64 + lane;
      const int r = u / kUnits;
      const int c = u - r * kUnits;
      *(V8*)(ldsk + r * kStride + 8 * c) = kr[it];
      *(V8*)(ldsv + r * kStride + 8 * c) = vr[it];
    }
    if constexpr (PRO) {
      const int64_t r = (pp->positions ? (int64_t)pp->positions[b] : pp->position) - p0;
      if (owns_new && r >= 0 && r < kTile) {
        for (int i = lane; i < D; i += 64) {
          ldsk[r * kStride + i] = new_kv[i];
          ldsv[r * kStride + i] = new_kv[D + i];
        }
      }
    }
    if (pn < end) load_tile(pn);
    wave_sync_lds();
    // Scores for 32 rows x 16 heads: lane holds S[pos = p0 + 16 blk + 4 quad + i][hl].
    f32x4 s[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      s[blk] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        const V8 ka = *(const V8*)(ldsk + (16 * blk + hl) * kStride + 32 * ks + 8 * quad);
        s[blk] = mfma16x16x32(ka, qv[ks], s[blk]);
      }
    }
    // Online softmax (base 2).  Slot j of this lane is row 16 (j/4) + 4 quad + j%4.
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pos = p0 + 16 * (j >> 2) + 4 * quad + (j & 3);
      const float x = pos < end ? s[j >> 2][j & 3] * a.scale_log2 : -INFINITY;
      sv[j] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy reference max: m moves only when the tile's max exceeds it by
    // more than kDecodeRescale (so P <= 2^kDecodeRescale), and O is rescaled
    // only on a step where some head of the wave moved.  Every tile holds at
    // least one live row, so the first tile always moves m off -inf.
    const bool grow = mx > m + kDecodeRescale;
    const float mn = grow ? mx : m;
    const float alpha = grow ? fast_exp2(m - mn) : 1.f;
    V8 pv;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = fast_exp2(sv[j] - mn);
      ps += p;
      pv[j] = from_f32<T>(p);
    }
    l = l * alpha + ps;
    m = mn;
    if (__builtin_expect(__ballot(grow) != 0, 0)) {
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) o[mb] *= alpha;
    }
    // O^T += V^T P^T.  A operand: lane holds V[row(quad, j)][16 mb + hl], j = 0..7,
    // gathered with two transposing reads of 4 rows (16 h + 4 quad + 0..3) each.
    const int tr_row = 4 * quad + (hl >> 2);
    const int tr_col = 4 * (hl & 3);
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) {
      const V4 lo = lds_read_tr4(ldsv + tr_row * kStride + 16 * mb + tr_col);
      const V4 hi = lds_read_tr4(ldsv + (16 + tr_row) * kStride + 16 * mb + tr_col);
      const V8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      o[mb] = mfma16x16x32(va, pv, o[mb]);
    }
    wave_sync_lds();
    p0 = pn;
  }

  merge_waves<D>(a, smem, o, m, l, wave, lane, head_ok, b, h, slot);
}

template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(256)
decode_split_mfma(DecodeArgs a) {
  split_body<T, D, PAGED, false>(a, nullptr);
}

template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(256)
decode_split_mfma_pro(DecodeArgs a, SplitPrologue pp) {
  split_body<T, D, PAGED, true>(a, &pp);
}

// fp32 caches: the same split structure on v_mfma_f32_16x16x4_f32 (fp32
// products and sums; P stays fp32).  A wave tile is R rows (32 at head_dim
// 64, 16 above, so two blocks' K and V tiles fit one CU's LDS at head_dim
// 64 and 128).  Both reductions run in a permuted order that lets each lane
// feed the values it already holds:
//   S^T = K Q^T, k-step (g, j): lane (hl, quad) supplies K[row hl][16 g +
//     4 quad + j] (one 16-byte LDS read per g) and Q[head hl][same d];
//   O^T = V^T P^T, k-step (blk, i): lane supplies P[16 blk + 4 quad + i]
//     [head hl] (its own score slot) and V[that row][16 mb + hl].
template <int D, int R, bool PAGED>
__global__ void __launch_bounds__(256)
decode_split_f32(DecodeArgs a) {
  constexpr int kStride = D + 4;  // floats: rows 4 apart sit 16 banks apart
  constexpr int kUnits = D / 4;   // 16-byte units per row
  constexpr int kIters = R * kUnits / 64;
  constexpr int kTileElems = R * kStride;
  constexpr int NB = R / 16;
  constexpr int kTileBytes = 2 * kWaves * kTileElems * 4;
  constexpr int kLdsBytes = kTileBytes > merge_lds_bytes<D>() ? kTileBytes : merge_lds_bytes<D>();
  static_assert(kIters >= 1 && R * kUnits % 64 == 0, "tile must split evenly over a wave");
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int b, start, end, slot;
  block_rows(a, b, start, end, slot);
  if (b < 0) return;  // past the last item of a balanced plan (whole block)
  const int hc = blockIdx.y % a.head_chunks;
  const int kvh = blockIdx.y / a.head_chunks;
  const int last = end - 1;
  const int hl = lane & 15;
  const int quad = lane >> 4;
  const int g_in = hc * 16 + hl;
  const bool head_ok = g_in < a.group;
  const int h = kvh * a.group + (head_ok ? g_in : 0);

  f32x4 qv[D / 16];  // Q[h][16 g + 4 quad + 0..3]
  {
    const float* qp = (const float*)a.q + ((int64_t)b * a.q_heads + h) * D + 4 * quad;
#pragma unroll
    for (int g = 0; g < D / 16; ++g) {
      const f32x4 x = *(const f32x4*)(qp + 16 * g);
      qv[g] = head_ok ? x : (f32x4){0.f, 0.f, 0.f, 0.f};
    }
  }
  f32x4 o[D / 16];
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) o[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;
  float l = 0.f;

  const float* kbase = (const float*)a.k + (int64_t)b * a.ks_b + (int64_t)kvh * a.ks_h;
  const float* vbase = (const float*)a.v + (int64_t)b * a.vs_b + (int64_t)kvh * a.vs_h;
  float* ldsk = (float*)smem + 2 * wave * kTileElems;
  float* ldsv = ldsk + kTileElems;

  f32x4 kr[kIters], vr[kIters];
  auto load_tile = [&](int p) {
    const float* kt = kbase;  // paged: one page per tile, as in decode_split_mfma
    const float* vt = vbase;
    if constexpr (PAGED) {
      kt = (const float*)a.k + row_offset(a, b, kvh, p, a.ks_pos, 0, a.ks_h, a.ks_page) -
           (int64_t)p * a.ks_pos;
      vt = (const float*)a.v + row_offset(a, b, kvh, p, a.vs_pos, 0, a.vs_h, a.vs_page) -
           (int64_t)p * a.vs_pos;
    }
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int u = it * 64 + lane;
      const int r = u / kUnits;
      const int c = u - r * kUnits;
      const int row = min(p + r, last);
      kr[it] = *(const f32x4*)(kt + (int64_t)row * a.ks_pos + 4 * c);
      vr[it] = __builtin_nontemporal_load((const f32x4*)(vt + (int64_t)row * a.vs_pos + 4 * c));
    }
  };

  int p0 = start + R * wave;
  if (p0 < end) load_tile(p0);
  while (p0 < end) {
    const int pn = p0 + R * kWaves;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int u = it * 64 + lane;
      const int r = u / kUnits;
      const int c = u - r * kUnits;
      *(f32x4*)(ldsk + r * kStride + 4 * c) = kr[it];
      *(f32x4*)(ldsv + r * kStride + 4 * c) = vr[it];
    }
    if (pn < end) load_tile(pn);
    wave_sync_lds();
    // lane holds S[pos = p0 + 16 blk + 4 quad + i][hl]
    f32x4 s[NB];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      s[blk] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < D / 16; ++g) {
        const f32x4 ka = *(const f32x4*)(ldsk + (16 * blk + hl) * kStride + 16 * g + 4 * quad);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[blk] = mfma16x16x4(ka[j], qv[g][j], s[blk]);
      }
    }
    float sv[NB][4];
    float mx = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = p0 + 16 * blk + 4 * quad + i;
        const float x = pos < end ? s[blk][i] * a.scale_log2 : -INFINITY;
        sv[blk][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);  // finite: every tile holds at least one live row
    const float alpha = fast_exp2(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[blk][i] = fast_exp2(sv[blk][i] - mn);
        ps += sv[blk][i];
      }
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) o[mb] *= alpha;
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb)
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float va = ldsv[(16 * blk + 4 * quad + i) * kStride + 16 * mb + hl];
          o[mb] = mfma16x16x4(va, sv[blk][i], o[mb]);
        }
    wave_sync_lds();
    p0 = pn;
  }
  merge_waves<D>(a, smem, o, m, l, wave, lane, head_ok, b, h, slot);
}

// ------------------------------------------------------------ generic split

template <typename T>
__global__ void __launch_bounds__(64)
decode_split_generic(DecodeArgs a) {
  __shared__ float qs[16][256];
  __shared__ float ps[kGenericTile][17];
  const int lane = threadIdx.x;
  int b, start, end, slot;
  block_rows(a, b, start, end, slot);
  if (b < 0) return;  // past the last item of a balanced plan (whole block)
  const int hc = blockIdx.y % a.head_chunks;
  const int kvh = blockIdx.y / a.head_chunks;
  const int D = a.key_dim, DV = a.value_dim;
  int gcount = a.group - hc * 16;
  gcount = gcount > 16 ? 16 : gcount;
  const int h0 = kvh * a.group + hc * 16;

  for (int i = lane; i < gcount * D; i += 64) {
    const int hh = i / D;
    const int d = i - hh * D;
    qs[hh][d] = to_f32(((const T*)a.q)[((int64_t)b * a.q_heads + h0 + hh) * D + d]);
  }
  __syncthreads();

  float m[16], l[16], acc[16][4];
#pragma unroll
  for (int hh = 0; hh < 16; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[hh][e] = 0.f;
  }
  for (int p0 = start; p0 < end; p0 += kGenericTile) {
    const int pos = p0 + lane;
    const bool live = pos < end;
    float s[16];
#pragma unroll
    for (int hh = 0; hh < 16; ++hh) s[hh] = 0.f;
    if (live) {
      const T* row = (const T*)a.k + row_offset(a, b, kvh, pos, a.ks_pos, a.ks_b, a.ks_h, a.ks_page);
      for (int d = 0; d < D; ++d) {
        const float kv = to_f32(row[d]);
#pragma unroll
        for (int hh = 0; hh < 16; ++hh)
          if (hh < gcount) s[hh] += qs[hh][d] * kv;
      }
    }
#pragma unroll
    for (int hh = 0; hh < 16; ++hh) {
      if (hh >= gcount) continue;
      const float x = live ? s[hh] * a.scale_log2 : -INFINITY;
      float mx = x;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      const float mn = fmaxf(m[hh], mx);
      const float alpha = fast_exp2(m[hh] - mn);
      const float p = fast_exp2(x - mn);
      l[hh] = l[hh] * alpha + p;
      m[hh] = mn;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[hh][e] *= alpha;
      ps[lane][hh] = p;
    }
    __syncthreads();
    const int n = min(kGenericTile, end - p0);
    for (int j = 0; j < n; ++j) {
      const T* vrow =
          (const T*)a.v + row_offset(a, b, kvh, p0 + j, a.vs_pos, a.vs_b, a.vs_h, a.vs_page);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < DV) {
          const float vv = to_f32(vrow[d]);
#pragma unroll
          for (int hh = 0; hh < 16; ++hh)
            if (hh < gcount) acc[hh][e] += ps[j][hh] * vv;
        }
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int hh = 0; hh < 16; ++hh) {
    if (hh >= gcount) continue;
    float lt = l[hh];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lt += __shfl_xor(lt, off);
    const int64_t pidx = partial_slot(a, b, h0 + hh, slot);
    if (lane == 0) {
      a.part_m[pidx] = m[hh];
      a.part_l[pidx] = lt;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      if (d < DV) a.part_acc[pidx * DV + d] = acc[hh][e];
    }
  }
}

// ------------------------------------------------------------ combine

// Pass 2: block (b*Hq + h, 64-column slice) merges the split partials of one
// query head for 64 output columns.  Wave w folds slots w, w+NW, ... into an
// online (m, l, acc) state; each group of slots has its max, sum and
// partial loads issued together (none depends on the running max), so the
// kernel pays about one memory round trip per group.  The NW wave states
// are then merged through LDS by wave 0.  NW = 1 (uniform plans of at most
// four splits, and every balanced plan, whose sequences hold a handful of
// items) folds groups of 16 in one wave with no LDS merge.
template <typename T, typename TO, int NW, int kGroup>
__global__ void __launch_bounds__(256)
decode_combine(DecodeArgs a) {
  // kGroup: partials per wave whose loads are issued together (one memory
  // round trip)
  __shared__ float red[3][NW > 1 ? NW - 1 : 1][64];
  const int64_t bh = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int DV = a.value_dim;
  const int d = blockIdx.y * 64 + lane;
  const int dc = d < DV ? d : DV - 1;
  // Partials of (b, h): slots s < ns of row bh.  A balanced plan's count
  // of slots for b is formed from the device lengths; the first group's
  // loads are issued over every slot the row can hold before the count is
  // known (one memory round trip for both), and slots past it are dropped.
  const int cap = a.nsplit;
  const float* pm = a.part_m + bh * cap;
  const float* pl = a.part_l + bh * cap;
  const float* pa = a.part_acc + bh * cap * DV + dc;
  int ns = cap;
  float m = -INFINITY, l = 0.f, acc = 0.f;
  for (int s0 = wave; s0 < ns; s0 += kGroup * NW) {
    float xm[kGroup], xl[kGroup], xa[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int s = s0 + u * NW;
      const bool ok = s < ns;
      xm[u] = ok ? pm[s] : -INFINITY;
      xl[u] = ok ? pl[s] : 0.f;
      xa[u] = ok ? pa[(int64_t)s * DV] : 0.f;
    }
    if (a.balanced && s0 == wave) {
      ns = balanced_count(a, (int)(bh / a.q_heads));
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        if (s0 + u * NW >= ns) {
          xm[u] = -INFINITY;
          xl[u] = 0.f;
          xa[u] = 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const float mn = fmaxf(m, xm[u]);
      if (mn == -INFINITY) continue;  // nothing live yet
      const float c_old = fast_exp2(m - mn);
      const float c_new = fast_exp2(xm[u] - mn);
      l = l * c_old + xl[u] * c_new;
      acc = acc * c_old + xa[u] * c_new;
      m = mn;
    }
  }
  if constexpr (NW > 1) {
    if (wave > 0) {
      red[0][wave - 1][lane] = m;
      red[1][wave - 1][lane] = l;
      red[2][wave - 1][lane] = acc;
    }
    __syncthreads();
  }
  if (wave != 0 || d >= DV) return;
  float M = m;
#pragma unroll
  for (int w = 0; w < NW - 1; ++w) M = fmaxf(M, red[0][w][lane]);
  float L = 0.f, A = 0.f;
  if (M != -INFINITY) {
    const float c0 = fast_exp2(m - M);
    L = l * c0;
    A = acc * c0;
#pragma unroll
    for (int w = 0; w < NW - 1; ++w) {
      const float cw = fast_exp2(red[0][w][lane] - M);
      L += red[1][w][lane] * cw;
      A += red[2][w][lane] * cw;
    }
  }
  float r = L > 0.f ? A / L : 0.f;
  if (a.gate != nullptr) r *= stable_sigmoid(to_f32(((const T*)a.gate)[bh * a.gate_stride + d]));
  ((TO*)a.out)[bh * DV + d] = from_f32<TO>(r);
}

// ------------------------------------------------------------ planning

struct Plan {
  int nsplit;   // partials per (b, h) == blocks along the split axis
  int chunk;    // rows per block
};

// Upper bound on partials per (b, h) for a cache of `length` rows; every
// plan stays within it, so the workspace size does not depend on the device.
int max_slots(int length) {
  int n = (length + kGenericTile - 1) / kGenericTile;
  return n < kMaxSlots ? (n < 1 ? 1 : n) : kMaxSlots;
}

// Size the split so the whole grid is resident at once (one round of blocks
// over the device), with each block's chunk a whole number of wave tiles.
Plan plan_split(int pairs, int length, int resident, int unit) {
  if (resident > kMaxResident) resident = kMaxResident;
  int want = (resident + pairs - 1) / pairs;
  const int most = (length + unit - 1) / unit;
  if (want > most) want = most;
  if (want < 1) want = 1;
  int chunk = (length + want - 1) / want;
  chunk = ((chunk + unit - 1) / unit) * unit;
  int n = (length + chunk - 1) / chunk;
  while (n > max_slots(length)) {
    chunk += unit;
    n = (length + chunk - 1) / chunk;
  }
  Plan p;
  p.nsplit = n;
  p.chunk = chunk;
  return p;
}

// One-round plans: the blocks a launch places on odd-numbered XCDs (block
// L of the grid runs on XCD L mod 8, and with an even split count the
// slot's parity is L's) streamed 7-11% slower than those on even XCDs in
// every per-block timing taken on MI355X boxes here (C4 shape: the odd XCDs'
// blocks end 3-4 us later on a 44 us split).  The even slot of each pair
// therefore takes a tenth of a chunk more rows (whole 32-row tiles) and the
// odd slot as many fewer, for chunks of at least kSkewMinUnits block steps.
constexpr int kSkewMinUnits = 4;

int plan_skew(const Plan& p, int unit) {
  if (p.nsplit % 2 != 0 || p.chunk < kSkewMinUnits * unit) return 0;
  return p.chunk / 10 / kDecodeWaveRows * kDecodeWaveRows;
}

// Several rounds of short chunks, for the 16-bit split kernels when two or
// more of their blocks fit on a CU.  With one round of long chunks the
// slowest CU sets the end of the launch (CUs, and whole XCDs, stream at
// rates up to ~20% apart under full load, and a CU that finishes its blocks
// early then idles).  Chunks of kRoundChunkUnits block steps, several per
// resident slot, let the dispatcher give a CU that finishes early the next
// block of its XCD.  At most kRoundMaxSlots partials per (sequence, head)
// keep the combine short, and plans whose one-round chunks are already
// short (fewer than kRoundMinUnits block steps) keep them: a block's start
// and merge would then weigh more than the balance gained.
constexpr int kRoundChunkUnits = 3;
constexpr int kRoundMinUnits = 8;
constexpr int kRoundMaxSlots = 32;

Plan plan_rounds(const Plan& one, int length, int unit, int bound) {
  if (one.chunk < kRoundMinUnits * unit) return one;
  const int cap = bound < kRoundMaxSlots ? bound : kRoundMaxSlots;
  int chunk = kRoundChunkUnits * unit;
  int n = (length + chunk - 1) / chunk;
  if (n > cap) {
    chunk = ((length + cap - 1) / cap + unit - 1) / unit * unit;
    n = (length + chunk - 1) / chunk;
  }
  if (n <= one.nsplit) return one;
  Plan p;
  p.nsplit = n;
  p.chunk = chunk;
  return p;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int slot_bound(int pairs, int length) {
  const int by_device = (kMaxResident + pairs - 1) / pairs;
  const int by_len = max_slots(length);
  return by_device < by_len ? by_device : by_len;
}

size_t partial_bytes(size_t n, int value_dim) {
  return 2 * align256(n * sizeof(float)) + align256(n * value_dim * sizeof(float));
}

size_t workspace_for(int batch, int q_heads, int value_dim, int nsplit) {
  return partial_bytes((size_t)batch * q_heads * nsplit, value_dim);
}

// Balanced plan: items_target blocks per grid row the chunk size is cut for
// (the resident blocks of one row, at most kMaxItemsPerRow), plus up to
// `batch` more for the sequences' last partial chunks.
constexpr int kMaxItemsPerRow = 256;
// items_target = resident blocks per grid row x NUM / DEN - batch x SUB / 2
// Two and a half rounds of blocks (measured on C2 ragged, same box: step
// 70.1-70.4% of HBM against 69.2-69.5% with two rounds and 66.8-67.0% with
// three, whose extra partials cost more in the combine than the finer
// balance gains; one round 64%).  Laying the padded sequences end to end and
// giving every block the same row count (blocks crossing a sequence boundary
// processing two segments) measured 64.7-66.1%: a segment's pipeline start
// and merge cost more than the tail imbalance it removes.
#ifndef ALPX_BALANCED_NUM
#define ALPX_BALANCED_NUM 5
#define ALPX_BALANCED_DEN 2
#define ALPX_BALANCED_SUB 0
#endif

// Grid x of the balanced plan: the item count is at most items_target +
// batch (see balanced_chunk) and at most batch * ceil(length / unit) (no
// chunk is shorter than unit rows unless it ends its sequence).
int balanced_items_max(int batch, int length, int unit, int items_target) {
  const int64_t by_len = (int64_t)batch * ((length + unit - 1) / unit);
  const int64_t by_target = (int64_t)items_target + batch;
  return (int)(by_len < by_target ? by_len : by_target);
}

// Partial slots per (b, h) of the balanced plan: the items one sequence can
// hold (C >= total / target gives ceil(len_b / C) <= target + 1, and C >=
// unit gives at most ceil(length / unit)).
int balanced_slots(int length, int unit, int items_target) {
  const int by_len = (length + unit - 1) / unit;
  return by_len < items_target + 1 ? by_len : items_target + 1;
}

template <typename T>
const void* split_kernel_pro(int D, bool paged) {
  if constexpr (sizeof(T) == 2) {
    switch (D) {
      case 64: return paged ? (const void*)decode_split_mfma_pro<T, 64, true>
                            : (const void*)decode_split_mfma_pro<T, 64, false>;
      case 128: return paged ? (const void*)decode_split_mfma_pro<T, 128, true>
                             : (const void*)decode_split_mfma_pro<T, 128, false>;
      case 256: return paged ? (const void*)decode_split_mfma_pro<T, 256, true>
                             : (const void*)decode_split_mfma_pro<T, 256, false>;
    }
  }
  return nullptr;
}

template <typename T>
const void* split_kernel(bool mfma, bool paged, int D) {
  if (mfma) {
    if constexpr (sizeof(T) == 2) {
      switch (D) {
        case 64: return paged ? (const void*)decode_split_mfma<T, 64, true>
                              : (const void*)decode_split_mfma<T, 64, false>;
        case 128: return paged ? (const void*)decode_split_mfma<T, 128, true>
                               : (const void*)decode_split_mfma<T, 128, false>;
        case 256: return paged ? (const void*)decode_split_mfma<T, 256, true>
                               : (const void*)decode_split_mfma<T, 256, false>;
      }
    } else {
      switch (D) {
        case 64: return paged ? (const void*)decode_split_f32<64, f32_tile_rows(64), true>
                              : (const void*)decode_split_f32<64, f32_tile_rows(64), false>;
        case 128: return paged ? (const void*)decode_split_f32<128, f32_tile_rows(128), true>
                               : (const void*)decode_split_f32<128, f32_tile_rows(128), false>;
        case 256: return paged ? (const void*)decode_split_f32<256, f32_tile_rows(256), true>
                               : (const void*)decode_split_f32<256, f32_tile_rows(256), false>;
      }
    }
    return nullptr;
  }
  return (const void*)decode_split_generic<T>;
}

template <typename T, int NW, int G>
void launch_combine_nw(int out_dtype, const DecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.batch * a.q_heads, (a.value_dim + 63) / 64), block(64 * NW);
  switch (out_dtype) {
    case ALPX_F32: hipLaunchKernelGGL((decode_combine<T, float, NW, G>), grid, block, 0, s, a); break;
    case ALPX_F16: hipLaunchKernelGGL((decode_combine<T, f16_t, NW, G>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((decode_combine<T, bf16_t, NW, G>), grid, block, 0, s, a); break;
  }
}

template <typename T>
int launch_combine(int out_dtype, const DecodeArgs& a, hipStream_t s) {
  // One wave folds up to four partials from one group of loads; with more
  // (uniform plans of many splits, balanced plans) four waves share them
  // (C2 ragged: the combine 0.6 us shorter than with one wave of 16-slot
  // groups, same box).  Uniform plans of more than 16 splits fold eight
  // partials per wave per group (C4's 32 in one round trip: step 0.3 us
  // shorter, same box); balanced plans keep groups of four (eight measured
  // 0.8 us slower on C2 ragged).
  if (a.nsplit <= 4)
    launch_combine_nw<T, 1, 16>(out_dtype, a, s);
  else if (a.nsplit > 16 && !a.balanced)
    launch_combine_nw<T, kWaves, 8>(out_dtype, a, s);
  else
    launch_combine_nw<T, kWaves, 4>(out_dtype, a, s);
  return check_launch("decode_combine");
}

int launch_split(const void* kernel, bool mfma, const DecodeArgs& a, const SplitPrologue* pro,
                 dim3 grid, hipStream_t s) {
  void* args[] = {(void*)&a, (void*)pro};
  hipError_t err = hipLaunchKernel(kernel, grid, dim3(mfma ? 256 : 64), args, 0, s);
  if (err != hipSuccess)
    return fail(ALPX_EHIP, "decode split launch failed: %s", hipGetErrorString(err));
  return check_launch("decode_split");
}

}  // namespace
}  // namespace alpx

extern "C" size_t alpx_decode_workspace_bytes(int batch, int q_heads, int kv_heads,
                                              int value_dim, int max_len) {
  using namespace alpx;
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || value_dim <= 0 || max_len <= 0 ||
      q_heads % kv_heads != 0)
    return 0;
  return decode_workspace(batch, q_heads, kv_heads, value_dim, max_len);
}

namespace alpx {

// Device-independent bound over both plans (split slots per (b, h) for a
// uniform length; item slots for device lengths).
size_t decode_workspace(int batch, int q_heads, int kv_heads, int value_dim, int length) {
  const int hc = (q_heads / kv_heads + 15) / 16;
  const size_t uniform =
      workspace_for(batch, q_heads, value_dim, slot_bound(batch * kv_heads * hc, length));
  // every split kernel steps at least kGenericTile rows per block step
  const size_t items = workspace_for(batch, q_heads, value_dim,
                                     balanced_slots(length, kGenericTile, kMaxItemsPerRow));
  return uniform > items ? uniform : items;
}

int run_decode(DecodeArgs a, int dtype, int out_dtype, void* workspace, size_t workspace_bytes,
               hipStream_t s, int split_timer, int combine_timer, const SplitPrologue* pro,
               const char* fixed_scratch) {
  const size_t es = dtype_size(dtype);
  const uintptr_t align = (uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v |
                          (uintptr_t)(a.ks_pos * es) | (uintptr_t)(a.ks_b * es) |
                          (uintptr_t)(a.ks_h * es) | (uintptr_t)(a.vs_pos * es) |
                          (uintptr_t)(a.vs_b * es) | (uintptr_t)(a.vs_h * es) |
                          (uintptr_t)(a.ks_page * es) | (uintptr_t)(a.vs_page * es);
  const int D = a.key_dim;
  // the MFMA kernels address a wave tile's rows with 32-bit byte offsets
  const int64_t max_pos = a.ks_pos > a.vs_pos ? a.ks_pos : a.vs_pos;
  const bool mfma = D == a.value_dim && (D == 64 || D == 128 || D == 256) && (align & 15) == 0 &&
                    (int64_t)kTile * max_pos * (int64_t)es < ((int64_t)1 << 31) &&
                    override_value(ALPX_OVERRIDE_DECODE_GENERIC) == 0;
  const size_t need = decode_workspace(a.batch, a.q_heads, a.kv_heads, a.value_dim, a.length);
  if (fixed_scratch == nullptr && workspace_bytes < need)
    return fail(ALPX_EINVAL, "decode workspace holds %zu bytes, needs %zu", workspace_bytes,
                need);
  const void* kernel = nullptr;
  const bool paged = a.pages != nullptr;
  if (pro != nullptr) {
    // fused prologue: 16-bit MFMA split over a contiguous or paged cache
    if (mfma && a.causal_pos0 < 0) {
      if (dtype == ALPX_F16) kernel = split_kernel_pro<f16_t>(D, paged);
      if (dtype == ALPX_BF16) kernel = split_kernel_pro<bf16_t>(D, paged);
    }
    if (kernel == nullptr)
      return fail(ALPX_EUNSUPPORTED,
                  "fused attention step: needs fp16/bf16 caches, key_dim == value_dim in "
                  "{64, 128, 256} and 16-byte aligned rows");
  } else {
    switch (dtype) {
      case ALPX_F32: kernel = split_kernel<float>(mfma, paged, D); break;
      case ALPX_F16: kernel = split_kernel<f16_t>(mfma, paged, D); break;
      default: kernel = split_kernel<bf16_t>(mfma, paged, D); break;
    }
  }
  if (kernel == nullptr) return fail(ALPX_EUNSUPPORTED, "decode: no kernel for this shape");
  if (a.gate_stride == 0) a.gate_stride = a.value_dim;
  const int unit =
      !mfma ? kGenericTile : (dtype == ALPX_F32 ? f32_tile_rows(D) : kTile) * kWaves;
  a.head_chunks = (a.group + 15) / 16;
  int resident = resident_blocks(kernel, mfma ? 256 : 64, 0);
  if (resident > kMaxResident) resident = kMaxResident;
  const int rows_y = a.kv_heads * a.head_chunks;
  size_t n;  // partial slots
  dim3 grid;
  if (a.seq_lens != nullptr && a.causal_pos0 < 0) {
    // device lengths: balanced plan (the chunk size is formed on the device)
    int target = resident * ALPX_BALANCED_NUM / (ALPX_BALANCED_DEN * rows_y) -
                 a.batch * ALPX_BALANCED_SUB / 2;
    target = target < 1 ? 1 : (target > kMaxItemsPerRow ? kMaxItemsPerRow : target);
    a.balanced = 1;
    a.items_target = target;
    a.items_max = balanced_items_max(a.batch, a.length, unit, target);
    a.unit = unit;
    a.nsplit = balanced_slots(a.length, unit, target);
    a.chunk = 0;
    n = (size_t)a.batch * a.q_heads * a.nsplit;
    grid = dim3(a.items_max, rows_y, 1);
  } else {
    Plan p = plan_split(a.batch * rows_y, a.length, resident, unit);
    const bool mfma16 = mfma && dtype != ALPX_F32 && a.causal_pos0 < 0;
    if (mfma16 && pro == nullptr && resident >= 2 * multiprocessor_count()) {
      const Plan r = plan_rounds(p, a.length, unit, slot_bound(a.batch * rows_y, a.length));
      // a fixed scratch that holds the one-round partials but not these
      // keeps the one-round plan
      if (fixed_scratch == nullptr ||
          partial_bytes((size_t)a.batch * a.q_heads * r.nsplit, a.value_dim) <= workspace_bytes)
        p = r;
    }
    a.skew = mfma16 && (int64_t)p.nsplit * a.batch * rows_y <= resident ? plan_skew(p, unit) : 0;
    a.balanced = 0;
    a.nsplit = p.nsplit;
    a.chunk = p.chunk;
    n = (size_t)a.batch * a.q_heads * p.nsplit;
    grid = dim3(p.nsplit, rows_y, a.batch);
  }
  if (fixed_scratch != nullptr && partial_bytes(n, a.value_dim) > workspace_bytes)
    return fail(ALPX_ERANGE,
                "%s: this call needs %zu bytes of split partials, more than the %zu-byte static "
                "scratch (call the entry point that takes a workspace)",
                fixed_scratch, partial_bytes(n, a.value_dim), workspace_bytes);
  char* ws = (char*)workspace;
  a.part_m = (float*)ws;
  a.part_l = (float*)(ws + align256(n * sizeof(float)));
  a.part_acc = (float*)(ws + 2 * align256(n * sizeof(float)));
  int rc;
  {
    TimedRegion timed(split_timer, s);
    rc = launch_split(kernel, mfma, a, pro, grid, s);
  }
  if (rc != ALPX_OK) return rc;
  TimedRegion timed(combine_timer, s);
  switch (dtype) {
    case ALPX_F32: return launch_combine<float>(out_dtype, a, s);
    case ALPX_F16: return launch_combine<f16_t>(out_dtype, a, s);
    default: return launch_combine<bf16_t>(out_dtype, a, s);
  }
}

}  // namespace alpx

namespace alpx {
namespace {

// ------------------------------------------------------------ static scratch

// Split partials of alpx_decode_gqa_noalloc.  Each GPU the library runs on
// holds its own copy of this array from the module's load until the process
// ends.  In host code `scratch` only names the symbol: its device address
// (one per GPU) comes from hipGetSymbolAddress, looked up once per device
// and kept in g_scratch_ptr.  Every split block writes its partial slot
// (an empty chunk writes m = -inf, l = 0, acc = 0) before the combine reads
// it, so nothing in the array has to start at zero and the previous call's
// contents never leak into a result.  Calls on one GPU share the array:
// calls that overlap in time on one GPU (different streams, no ordering)
// race on it.
static __device__ __align__(256) unsigned char scratch[ALPX_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream).
int scratch_address(hipStream_t stream, void** out) {
  int current = 0;
  hipError_t err = hipGetDevice(&current);
  if (err != hipSuccess) return fail(ALPX_EHIP, "hipGetDevice: %s", hipGetErrorString(err));
  int device = current;
  if (stream != nullptr) {
    err = hipStreamGetDevice(stream, &device);
    if (err != hipSuccess)
      return fail(ALPX_EHIP, "hipStreamGetDevice: %s", hipGetErrorString(err));
  }
  if (device < 0 || device >= kMaxDevices)
    return fail(ALPX_EUNSUPPORTED, "device %d is beyond the %d this library tracks", device,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    // the symbol lookup resolves on the current device: make it `device`
    if (device != current && (err = hipSetDevice(device)) != hipSuccess)
      return fail(ALPX_EHIP, "hipSetDevice(%d): %s", device, hipGetErrorString(err));
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (device != current) (void)hipSetDevice(current);
    if (err != hipSuccess || ptr == nullptr)
      return fail(ALPX_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(err));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return ALPX_OK;
}

// Validates and runs one contiguous-cache decode on `workspace`
// (fixed_scratch: see run_decode).
int decode_gqa(const char* who, const void* q, const void* key_cache, const void* value_cache,
               const int32_t* seq_lens, int length, const void* gate, void* out, void* workspace,
               size_t workspace_bytes, int batch, int q_heads, int kv_heads, int key_dim,
               int value_dim, int64_t k_pos_stride, int64_t k_batch_stride,
               int64_t k_head_stride, int64_t v_pos_stride, int64_t v_batch_stride,
               int64_t v_head_stride, float scale, int dtype, int out_dtype, hipStream_t stream,
               const char* fixed_scratch) {
  if (!q || !key_cache || !value_cache || !out || (!workspace && !fixed_scratch))
    return fail(ALPX_EINVAL, "%s: null buffer", who);
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", who);
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", who);
  if (length <= 0) return fail(ALPX_EINVAL, "attention cache length must be a positive integer");
  if (q_heads % kv_heads != 0)
    return fail(ALPX_EINVAL, "attention query heads must be a multiple of KV heads");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  if (key_dim > 256 || value_dim > 256)
    return fail(ALPX_EUNSUPPORTED, "%s: head dims above 256 are not supported", who);
  DecodeArgs a = {};
  a.q = q;
  a.k = key_cache;
  a.v = value_cache;
  a.seq_lens = seq_lens;
  a.gate = gate;
  a.out = out;
  a.ks_pos = k_pos_stride;
  a.ks_b = k_batch_stride;
  a.ks_h = k_head_stride;
  a.vs_pos = v_pos_stride;
  a.vs_b = v_batch_stride;
  a.vs_h = v_head_stride;
  a.causal_pos0 = -1;
  a.kv_start = 0;
  a.window = 0;
  a.length = length;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.group = q_heads / kv_heads;
  a.key_dim = key_dim;
  a.value_dim = value_dim;
  a.scale_log2 = scale * kLog2e;
  if (fixed_scratch != nullptr) {
    const int rc = scratch_address(stream, &workspace);
    if (rc != ALPX_OK) return rc;
    workspace_bytes = ALPX_DECODE_SCRATCH_BYTES;
  }
  return run_decode(a, dtype, out_dtype, workspace, workspace_bytes, stream, ALPX_T_DECODE,
                    ALPX_T_DECODE_COMBINE, nullptr, fixed_scratch);
}

}  // namespace
}  // namespace alpx

extern "C" int alpx_decode_gqa(const void* q, const void* key_cache, const void* value_cache,
                               const int32_t* seq_lens, int length, const void* gate, void* out,
                               void* workspace, size_t workspace_bytes, int batch, int q_heads,
                               int kv_heads, int key_dim, int value_dim, int64_t k_pos_stride,
                               int64_t k_batch_stride, int64_t k_head_stride,
                               int64_t v_pos_stride, int64_t v_batch_stride,
                               int64_t v_head_stride, float scale, int dtype, int out_dtype,
                               void* stream) {
  return alpx::decode_gqa("alpx_decode_gqa", q, key_cache, value_cache, seq_lens, length, gate,
                          out, workspace, workspace_bytes, batch, q_heads, kv_heads, key_dim,
                          value_dim, k_pos_stride, k_batch_stride, k_head_stride, v_pos_stride,
                          v_batch_stride, v_head_stride, scale, dtype, out_dtype,
                          (hipStream_t)stream, nullptr);
}

extern "C" int alpx_decode_gqa_noalloc(const void* q, const void* key_cache,
                                       const void* value_cache, const int32_t* seq_lens,
                                       int length, const void* gate, void* out, int batch,
                                       int q_heads, int kv_heads, int key_dim, int value_dim,
                                       int64_t k_pos_stride, int64_t k_batch_stride,
                                       int64_t k_head_stride, int64_t v_pos_stride,
                                       int64_t v_batch_stride, int64_t v_head_stride,
                                       float scale, int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  return decode_gqa("alpx_decode_gqa_noalloc", q, key_cache, value_cache, seq_lens, length, gate,
                    out, nullptr, 0, batch, q_heads, kv_heads, key_dim,
                    value_dim, k_pos_stride, k_batch_stride, k_head_stride, v_pos_stride,
                    v_batch_stride, v_head_stride, scale, dtype, out_dtype, (hipStream_t)stream,
                    "alpx_decode_gqa_noalloc");
}

extern "C" int alpx_decode_gqa_paged(const void* q, const void* key_pages,
                                     const void* value_pages, const int32_t* block_table,
                                     int max_pages, int page_size, int num_pages,
                                     const int32_t* seq_lens, int length, const void* gate,
                                     void* out, void* workspace, size_t workspace_bytes,
                                     int batch, int q_heads, int kv_heads, int key_dim,
                                     int value_dim, float scale, int dtype, int out_dtype,
                                     void* stream) {
  using namespace alpx;
  if (!q || !key_pages || !value_pages || !block_table || !out || !workspace)
    return fail(ALPX_EINVAL, "alpx_decode_gqa_paged: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(ALPX_EINVAL, "alpx_decode_gqa_paged: unknown dtype");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0 ||
      max_pages <= 0 || num_pages <= 0)
    return fail(ALPX_EINVAL, "alpx_decode_gqa_paged: sizes must be positive");
  if (page_size < kTile || (page_size & (page_size - 1)) != 0)
    return fail(ALPX_EINVAL, "page size must be a power of two of at least %d rows", kTile);
  if (length <= 0) return fail(ALPX_EINVAL, "attention cache length must be a positive integer");
  if ((int64_t)max_pages * page_size < length)
    return fail(ALPX_ERANGE, "the block table covers %lld rows, fewer than length %d",
                (long long)max_pages * page_size, length);
  if (q_heads % kv_heads != 0)
    return fail(ALPX_EINVAL, "attention query heads must be a multiple of KV heads");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  if (key_dim > 256 || value_dim > 256)
    return fail(ALPX_EUNSUPPORTED, "alpx_decode_gqa_paged: head dims above 256 are not supported");
  DecodeArgs a = {};
  a.q = q;
  a.k = key_pages;
  a.v = value_pages;
  a.seq_lens = seq_lens;
  a.gate = gate;
  a.out = out;
  a.ks_pos = (int64_t)kv_heads * key_dim;
  a.ks_h = key_dim;
  a.vs_pos = (int64_t)kv_heads * value_dim;
  a.vs_h = value_dim;
  a.ks_page = (int64_t)page_size * a.ks_pos;
  a.vs_page = (int64_t)page_size * a.vs_pos;
  a.pages = block_table;
  a.page_shift = __builtin_ctz((unsigned)page_size);
  a.max_pages = max_pages;
  a.num_pages = num_pages;
  a.causal_pos0 = -1;
  a.length = length;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.group = q_heads / kv_heads;
  a.key_dim = key_dim;
  a.value_dim = value_dim;
  a.scale_log2 = scale * kLog2e;
  return run_decode(a, dtype, out_dtype, workspace, workspace_bytes, (hipStream_t)stream,
                    ALPX_T_DECODE, ALPX_T_DECODE_COMBINE);
}
