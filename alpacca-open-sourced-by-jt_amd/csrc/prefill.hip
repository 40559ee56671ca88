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
// tile is multiplied.  One iteration's MFMA block holds PV of tile j - 1,
// the exp / convert work of tile j and QK of tile j + 1, at raised wave
// priority; the softmax max bookkeeping runs ahead of it (see grow_check).
// Tiles entirely above the diagonal are never loaded;
// tiles entirely above one wave's diagonal are skipped by that wave.  Blocks
// are mapped so that one kv head's blocks share one XCD (and its L2), with
// the latest (most expensive) column tiles launched first.
//
// Everything else (fp32, odd head dims, unaligned rows) runs the split-K
// decode machinery in causal mode: query token t is a "sequence" whose
// visible rows are those at absolute positions <= pos0 + t (inside the
// window).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "alpx_common.h"
#include "decode_internal.h"
#include "timing.h"

namespace alpx {
namespace {

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* gate;  // null, or q_tokens x q_heads rows of D in T: out *= sigmoid(gate)
  int64_t gate_stride;  // elements between the gate rows of (token, head)
  void* out;
  int64_t ks_pos, vs_pos;  // elements between cache rows (head stride = head_dim)
  int64_t pos0;            // absolute position of query token 0
  int64_t kv_start;        // absolute position of cache row 0
  int window;              // > 0: row at p sees keys in (p - window, p]
  int q_tokens, kv_tokens, q_heads, kv_heads, group;
  int col_tiles;           // column tiles per kv head
  int per_xcd;             // work items per XCD slice of the grid
  float scale_log2;
  // Paged caches (the PAGED kernels): cache row j lives in page
  // pages[j >> page_shift] (clamped to [0, num_pages)), at row
  // j & (page size - 1); ks_page / vs_page are the page strides in elements.
  const int32_t* pages;
  int page_shift;
  int num_pages;
  int64_t ks_page, vs_page;
  // Append mode (contiguous kernels): kn / vn hold the chunk's own K / V
  // rows, row i being cache row new0 + i (same row strides as the cache).
  // Tiles take rows >= new0 from them, and each block writes its tokens'
  // rows into the cache (k / v), so no launch has to append them first.
  const void* kn;
  const void* vn;
  int new0;
  // Fused query prologue (qw != null; the Qwen3.5 attention-layer chunk):
  // q holds the joint projection rows [T, Hq, 2 D], and each query row is
  // RMS-normalised with qw and rotated (IMROPE, q_R pairs, a multiple of
  // 32) with the attention prologue's arithmetic, then rounded to T, before
  // the softmax scale is applied.  q_rot [T, q_R] holds the (cos, sin) of
  // token t's pairs, formed by the prologue launch that writes the keys.
  int64_t q_stride;  // elements between the (token, head) rows of q
  const float* qw;
  const float2* q_rot;
  float q_eps;
  int q_R;
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

// K and V tiles sit unpadded in LDS, written by direct-to-LDS buffer loads
// (no staging registers, no LDS write instructions).  16-byte unit c of row r
// is stored at unit c ^ swz(r), with a swizzle per tile chosen from
// bank-conflict counter measurements on gfx950 of the two read patterns:
//   K operand reads (ds_read_b128: 16 consecutive rows, one unit each):
//     conflict-free with swz = r mod 16 (r mod 8 for 128-byte rows);
//   V transposing reads (ds_read_b64_tr_b16: 4-row groups, a unit pair
//     {2y, 2y+1} each): conflict-free with swz = ((r mod 8) << 1) | bit 3 of r
//     for rows of 256 bytes or more, r mod 8 for 128-byte rows.
// Every swizzle is below 16, so it only permutes units inside each aligned
// group of 16 units (256 bytes).
template <int ROW_BYTES>
__device__ __forceinline__ int swz_k(int r) {
  return ROW_BYTES >= 256 ? (r & 15) : (r & 7);
}
template <int ROW_BYTES>
__device__ __forceinline__ int swz_v(int r) {
  return ROW_BYTES >= 256 ? (((r & 7) << 1) | ((r >> 3) & 1)) : (r & 7);
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource words of a raw (stride 0) buffer of `bytes` bytes at
// `base`; loads at offsets past `bytes` return zero.
__device__ __forceinline__ i32x4 rsrc_words(uint64_t p, uint32_t bytes) {
  return (i32x4){(int)(uint32_t)p, (int)((uint32_t)(p >> 32) & 0xffffu), (int)bytes, 0x00020000};
}

// One direct-to-LDS 16-byte-per-lane buffer load: lane L's 16 bytes at
// buffer offset `voff` land at LDS byte `lds + 16 L` (`lds` wave-uniform).
// Written as inline assembly (the same three instructions the compiler
// emits for __builtin_amdgcn_raw_ptr_buffer_load_lds) because the
// compiler's wait insertion counts that builtin as an LDS store that may
// alias every later LDS read: it put a wait for all outstanding loads in
// front of the first LDS read of each iteration -- the reads of the other
// buffer -- which exposed the whole latency of the tile loads just issued.
// The kernel waits for these loads itself (s_waitcnt 0) before each
// barrier.  m0 is written here and nowhere else in the prefill kernels (no
// other instruction they contain reads it).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; the clobber is intended
__device__ __forceinline__ void lds_dma16(i32x4 r, uint32_t lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r)
               : "memory", "m0");
#else
  (void)r;
  (void)lds;
  (void)voff;
#endif
}
#pragma clang diagnostic pop

template <int V>
using Par = std::integral_constant<int, V>;

template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Par<B>());
    static_for<B + 1, E>(f);
  }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// LDS operand reads of the iteration block, issued as inline assembly so
// that their order, and the distance between a read and the MFMA that
// consumes it, is the kernel's and not the scheduler's (left to it, the
// scheduler placed each read right in front of its consumer and exposed
// the LDS latency on every MFMA pair).  The compiler does not track these
// reads: lds_wait<N> waits until at most N LDS operations of the wave are
// outstanding and, by taking the operand as a read-write register, keeps
// every use of the operand behind the wait.  Nothing else in the block
// issues LDS or scalar-memory operations, so the LDS counter holds exactly
// these reads, in issue order.
template <int OFS>
__device__ __forceinline__ u32x2 lds_tr64(uint32_t addr) {
  static_assert(OFS >= 0 && OFS < 65536, "LDS immediate offset is 16 bits");
  u32x2 r;
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFS));
#else
  (void)addr;
  r = (u32x2){0u, 0u};
#endif
  return r;
}
template <int OFS>
__device__ __forceinline__ u32x4 lds_b128(uint32_t addr) {
  static_assert(OFS >= 0 && OFS < 65536, "LDS immediate offset is 16 bits");
  u32x4 r;
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFS));
#else
  (void)addr;
  r = (u32x4){0u, 0u, 0u, 0u};
#endif
  return r;
}
template <int N, typename X>
__device__ __forceinline__ void lds_wait(X& x) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "n"(N));
#else
  (void)x;
#endif
}

// Marks a register value as used (and possibly changed) at this point, so
// the work producing it stays before it (the compiler would otherwise sink
// register-only work past the block barrier into the next iteration).
template <typename V>
__device__ __forceinline__ void pin(V& x) {
#if defined(__HIP_DEVICE_COMPILE__)  // the "v" constraint exists only for the GPU target
  asm volatile("" : "+v"(x));
#else
  (void)x;
#endif
}

// Append mode: copies the K and V rows (head kvh) of the tokens whose first
// column lies in column tile ct into the cache, 16 bytes per lane over 256
// threads, four loads in flight (clamped, so unconditional) before the
// stores.  No block of the launch reads those cache rows: tiles take them
// from kn / vn.
template <typename T, int D, int kCols>
__device__ __forceinline__ void copy_tile_rows(const PrefillArgs& a, int kvh, int ct, int tid) {
  constexpr int U = D / 8;
  const int G = a.group;
  const int t0 = (ct * kCols + G - 1) / G;
  const int t1 = min(a.q_tokens, ((ct + 1) * kCols + G - 1) / G);
  const int units = max(0, t1 - t0) * 2 * U;
  for (int u0 = 0; u0 < units; u0 += 4 * 256) {
    u32x4 x[4];
    T* dst[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = min(u0 + 256 * k + tid, units - 1);
      const int r = t0 + u / (2 * U), part = u % (2 * U);
      const bool val = part >= U;
      const int64_t pos = val ? a.vs_pos : a.ks_pos;
      const int64_t col = (int64_t)kvh * D + 8 * (part - (val ? U : 0));
      x[k] = *(const u32x4*)((const T*)(val ? a.vn : a.kn) + (int64_t)r * pos + col);
      // the caches are written here and nowhere else in the kernels
      dst[k] = (T*)const_cast<void*>(val ? a.v : a.k) + (int64_t)(a.new0 + r) * pos + col;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (u0 + 256 * k + tid < units) *(u32x4*)dst[k] = x[k];
  }
}

// Key tiles of a column tile: rows [lo, hi) that any of its columns can
// see, in nt tiles of BK rows starting at lo.
template <int BK, int kCols>
__device__ __forceinline__ void tile_keys(const PrefillArgs& a, int ctile, int& lo, int& hi,
                                          int& nt) {
  const int G = a.group;
  const int cols = a.q_tokens * G;
  const int col0 = ctile * kCols;
  const int rel0 = (int)(a.pos0 - a.kv_start);
  const int bt_first = col0 / G;
  const int bt_last = (min(col0 + kCols, cols) - 1) / G;
  hi = max(0, min(a.kv_tokens, rel0 + bt_last + 1));
  lo = 0;
  if (a.window > 0) lo = min(hi, max(0, rel0 + bt_first - a.window + 1)) / BK * BK;
  nt = (hi - lo + BK - 1) / BK;
}

// What a run does with its result: write the output; leave its partial
// state (O and this lane's share of l, with the column's m and offset mc)
// in LDS for the other group of the block; or merge that partial into its
// own and write the output.
constexpr int kRunWrite = 0, kRunPartial = 1, kRunMerge = 2;

// One run of a group of four waves (wave 0..3, tid 0..255 within the
// group): column tile ctile of kv head kvh over its key tiles [tb, te)
// (counted from the tile's first visible tile; te < 0: to its last), with
// the four K / V tile buffers at `smem` and `bar` as the group's barrier.
// prefill_mfma runs one per block; prefill_pair runs two groups per block.
// part_o / part_st: the partial's LDS home (written by kRunPartial, read by
// kRunMerge).
// The attention prologue's query half (norm_rope) for one column whose row
// a lane holds as q[ks] = channels 32 ks + 8 quad + 0..7 (the four lanes
// of a column hold quads 0..3), giving the prologue's bits.  The prologue
// wave sums squares per lane l over channels l + 64 e (e ascending) and
// then across lanes with xor offsets 32, 16, 8, 4, 2, 1; here lane
// l = 32 h + 8 quad + j lives in slot j of this lane's registers with
// ks = 2 e + h, offset 32 pairs h = 0 / 1 in place, 16 and 8 pair the lanes
// of quads quad ^ 2 and quad ^ 1 (this kernel's lanes ^ 32 and ^ 16), and
// 4, 2, 1 pair slots.  With q_R a multiple of 32 a channel's rotation
// partner (d +- q_R) sits in the same lane, q_R / 32 registers away; the
// (cos, sin) of its pair come from q_rot.
template <typename T, int D>
__device__ __forceinline__ void fused_query(const PrefillArgs& a, typename Vec8<T>::type (&q)[D / 32],
                                            int tok, int quad) {
  constexpr int KS = D / 32, E = D / 64;
  float x[KS][8];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int j = 0; j < 8; ++j) x[ks][j] = to_f32(q[ks][j]);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      s0 = fmaf(x[2 * e][j], x[2 * e][j], s0);
      s1 = fmaf(x[2 * e + 1][j], x[2 * e + 1][j], s1);
    }
    v[j] = s0 + s1;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = v[j] + __shfl_xor(v[j], 32);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = v[j] + __shfl_xor(v[j], 16);
  float w4[8], w2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w4[j] = v[j] + v[j ^ 4];
#pragma unroll
  for (int j = 0; j < 8; ++j) w2[j] = w4[j] + w4[j ^ 2];
  const float ss = w2[0] + w2[1];
  const float inv = 1.f / sqrtf(ss / (float)D + a.q_eps);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const f32x4 w0 = *(const f32x4*)(a.qw + 32 * ks + 8 * quad);
    const f32x4 w1 = *(const f32x4*)(a.qw + 32 * ks + 8 * quad + 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[ks][j] = x[ks][j] * inv * (j < 4 ? w0[j] : w1[j - 4]);
  }
  const int R = a.q_R, RK = R / 32;
  const float2* rot = a.q_rot + (int64_t)tok * R;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const bool rotated = 32 * ks < 2 * R;  // whole 32-channel groups rotate or not
    const bool first = 32 * ks < R;
    float2 cs[8];
    if (rotated) {
      const int pr0 = (first ? 32 * ks : 32 * ks - R) + 8 * quad;
#pragma unroll
      for (int j = 0; j < 8; ++j) cs[j] = rot[pr0 + j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = x[ks][j];
      if (rotated) {
        float xp = 0.f;  // the partner, RK registers away
#pragma unroll
        for (int k2 = 0; k2 < KS; ++k2)
          if (k2 == (first ? ks + RK : ks - RK)) xp = x[k2][j];
        y = rope_pair(first, x[ks][j], xp, cs[j].x, cs[j].y);
      }
      q[ks][j] = from_f32<T>(y);
    }
  }
}

template <typename T, typename TO, int D, int BK, int NQB, bool PAGED, int MODE, int NW,
          typename Bar>
__device__ __forceinline__ void prefill_run(const PrefillArgs& a, int kvh, int ctile, int tb,
                                            int te, char* smem, float* part_o, float* part_st,
                                            int wave, int tid, Bar& bar, int lw, int hi_blk,
                                            bool idle) {
  typedef typename Vec8<T>::type V8;
  constexpr int U = D / 8;                  // 16-byte units per row
  constexpr int kRowB = D * (int)sizeof(T);
  constexpr int kTileB = BK * kRowB;        // one K or V tile
  constexpr int kIW = BK * U / (64 * NW);   // direct-load instructions per wave per tile
  constexpr int KB = BK / 16;
  constexpr int KK = BK / 32;
  constexpr int MB = D / 16;
  constexpr int KS = D / 32;
  constexpr int kWaveCols = 16 * NQB;
  constexpr int kCols = 4 * kWaveCols;
  static_assert(kIW >= 1 && BK * U % (64 * NW) == 0, "tile must split evenly over the waves");
  static_assert(NW == 4 || (!PAGED && MODE == kRunWrite), "shared tiles: contiguous, one run");
  static_assert(kTileB % (64 * NW * 16) == 0, "the V buffer zeroing splits evenly");
  static_assert(U >= 8, "the row swizzle needs 8 units per row");
  // K tile buffers at smem and smem + kTileB, V tile buffers at 2 and 3 kTileB,
  // loaded and read by the NW waves that share them (lw = 0 .. NW - 1 among
  // them; `wave` = 0 .. 3 places this wave's columns in its column tile).

  const int lane = tid & 63;
  const int hl = lane & 15;
  const int quad = lane >> 4;
  const int G = a.group;
  const int cols = a.q_tokens * G;
  const int col0 = ctile * kCols;
  const int wcol0 = col0 + kWaveCols * wave;

  int tok[NQB], hq[NQB];
  bool cok[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int c = wcol0 + 16 * qb + hl;
    cok[qb] = c < cols && !idle;
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

  // Key rows [lo, hi) that any column of the block can see, in nt tiles.
  // Waves sharing tiles with a heavier column tile walk its key range
  // (hi_blk) but compute only over their own tiles (nt_own), then keep
  // loading and meeting the barrier.
  const int hi_own = max(0, min(a.kv_tokens, rel0 + bt_last + 1));
  const int hi = hi_blk >= 0 ? hi_blk : hi_own;
  int lo = 0;
  if (a.window > 0) lo = min(hi, max(0, rel0 + bt_first - a.window + 1)) / BK * BK;
  // Every wave walks all nt tiles of the block; keys a wave's columns cannot
  // see (past its diagonal, before its window) are masked, which costs at
  // most about one tile per wave and keeps the waves' pipelines in step.
  const int nt_all = (hi - lo + BK - 1) / BK;
  // This run's tiles are [tb, t_end) of them, its keys end at hi_r; inside
  // the run tiles are counted from tb.
  const int t_end = te < 0 ? nt_all : min(te, nt_all);
  const int nt = max(0, t_end - tb);
  const int hi_r = min(hi, lo + t_end * BK);
  const int nt_own = idle ? -1 : (hi_blk >= 0 ? (hi_own - lo + BK - 1) / BK : nt);

  // B operand of S^T = K Q^T: lane holds Q[column][32 ks + 8 quad + 0..7],
  // pre-multiplied by scale * log2(e) (and rounded once to T), so that the
  // product lands in the base-2 softmax domain.
  const float c2 = a.scale_log2;
  V8 qv[NQB][KS];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const T* qp = (const T*)a.q + ((int64_t)tok[qb] * a.q_heads + hq[qb]) * a.q_stride + 8 * quad;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qv[qb][ks] = *(const V8*)(qp + 32 * ks);
  }

  f32x4 o[NQB][MB];   // O^T[d = 16 mb + 4 quad + i][column]
  float lsum[NQB];    // this lane's share (its 4-key slices) of the column's sum of P
  // m: the column's reference max (base-2 domain); mc: the offset the QK
  // product subtracts through its accumulator input (m, or 0 while m is
  // -inf); lim: how far above mc a score may reach before m must move.
  float m[NQB], mc[NQB], lim[NQB], pend[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m[qb] = -INFINITY;
    mc[qb] = 0.f;
    lim[qb] = -INFINITY;
    pend[qb] = 1.f;
    lsum[qb] = 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) o[qb][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  bool pend_any = false;

  // Direct loads: wave-instruction q of a tile fills LDS bytes [1024 q,
  // 1024 q + 1024), lane L the 16 bytes at 1024 q + 16 L, i.e. row
  // (64 q + L) / U, stored unit (64 q + L) % U, which holds logical unit
  // stored ^ swz_k/swz_v(row).  Rows at or past kv_tokens read as zero.
  uint32_t kofs[kIW], vofs[kIW];
#pragma unroll
  for (int t = 0; t < kIW; ++t) {
    const int sl = (lw * kIW + t) * 64 + lane;
    const int row = sl / U;
    const int ck = (sl % U) ^ swz_k<kRowB>(row);
    const int cv = (sl % U) ^ swz_v<kRowB>(row);
    kofs[t] = (uint32_t)(((int64_t)row * a.ks_pos + 8 * ck) * (int64_t)sizeof(T));
    vofs[t] = (uint32_t)(((int64_t)row * a.vs_pos + 8 * cv) * (int64_t)sizeof(T));
  }
  const T* kg = (const T*)a.k + (int64_t)kvh * D;
  const T* vg = (const T*)a.v + (int64_t)kvh * D;
  const T* kgn = a.kn != nullptr ? (const T*)a.kn + (int64_t)kvh * D : nullptr;
  const T* vgn = a.vn != nullptr ? (const T*)a.vn + (int64_t)kvh * D : nullptr;
  // Paged: the block's page numbers (clamped) are staged in LDS once, so a
  // tile's page lookup is an LDS read rather than a global load on the
  // path to its tile loads; ranges of more than kPageSlots pages look up
  // the table directly.
  constexpr int kPageSlots = PAGED ? 1024 : 1;
  __shared__ int page_lds[kPageSlots];
  [[maybe_unused]] int page0 = 0;
  [[maybe_unused]] bool pages_in_lds = false;
  if constexpr (PAGED) {
    page0 = lo >> a.page_shift;
    const int np = nt > 0 ? ((hi - 1) >> a.page_shift) - page0 + 1 : 0;
    pages_in_lds = np <= kPageSlots;
    if (pages_in_lds) {
      for (int i = tid; i < np; i += 256) {
        const int pg = a.pages[page0 + i];
        page_lds[i] = pg < 0 ? 0 : (pg >= a.num_pages ? a.num_pages - 1 : pg);
      }
    }
    bar();
  }
  // A tile starts at a multiple of BK and a page holds a multiple of BK
  // rows, so a paged tile lies in one page, looked up once per tile (when
  // its K rows are loaded; its V rows reuse the number).
  [[maybe_unused]] auto tile_page = [&](int t) -> int {
    if constexpr (PAGED) {
      const int pi = (lo + (tb + t) * BK) >> a.page_shift;
      if (pages_in_lds) return __builtin_amdgcn_readfirstlane(page_lds[pi - page0]);
      const int pg = a.pages[pi];
      return pg < 0 ? 0 : (pg >= a.num_pages ? a.num_pages - 1 : pg);
    }
    return 0;
  };
  // gn: the chunk's own rows of this head (append mode), else null.
  auto load_tile = [&](const T* g, const T* gn, int64_t pos, int64_t page_stride,
                       const uint32_t (&ofs)[kIW], int t, int buf, int pg) {
    const int k0 = lo + (tb + t) * BK;
    const T* base = g + (int64_t)k0 * pos;
    if constexpr (PAGED)
      base = g + (int64_t)pg * page_stride + (int64_t)(k0 & ((1 << a.page_shift) - 1)) * pos;
    const uint32_t bytes = (uint32_t)((int64_t)(a.kv_tokens - k0) * pos * (int64_t)sizeof(T));
    const uint32_t lds0 =
        (uint32_t)(uintptr_t)(lds_void_t*)(smem + buf * kTileB + lw * kIW * 1024);
    if (!PAGED && gn != nullptr && k0 + BK > a.new0) {
      // Rows >= new0 come from the chunk's rows: a resource whose offset of
      // tile row i is the one of row k0 + i, based new0 - k0 rows before gn.
      const i32x4 rn = rsrc_words(
          (uint64_t)(uintptr_t)gn + (uint64_t)((int64_t)(k0 - a.new0) * pos * (int64_t)sizeof(T)),
          bytes);
      if (k0 >= a.new0) {
#pragma unroll
        for (int i = 0; i < kIW; ++i) lds_dma16(rn, lds0 + i * 1024, ofs[i]);
        return;
      }
      // A tile across new0: each lane loads from the side its row is on.
      const i32x4 rc = rsrc_words((uint64_t)(uintptr_t)base,
                                  (uint32_t)((int64_t)(a.new0 - k0) * pos * (int64_t)sizeof(T)));
#pragma unroll
      for (int i = 0; i < kIW; ++i) {
        if (((lw * kIW + i) * 64 + lane) / U < a.new0 - k0)
          lds_dma16(rc, lds0 + i * 1024, ofs[i]);
        else
          lds_dma16(rn, lds0 + i * 1024, ofs[i]);
      }
      return;
    }
    const i32x4 r = rsrc_words((uint64_t)(uintptr_t)base, bytes);
#pragma unroll
    for (int i = 0; i < kIW; ++i) lds_dma16(r, lds0 + i * 1024, ofs[i]);
  };

  // LDS read offsets (the swizzle only depends on a row's index mod 16, and
  // tile row bases are multiples of 16).  K operand: row 16 kb + hl,
  // logical unit 4 ks + quad.
  uint32_t kadr[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kadr[ks] = hl * kRowB + (((4 * ks + quad) ^ swz_k<kRowB>(hl)) * 16);
  // V transposing reads: row 32 kk + 16 h + tr_row, elements 16 mb + 4 (hl & 3)
  // + 0..3, i.e. logical unit 2 mb + cb (cb = (hl & 3) >> 1).  With mb = 4 x + y
  // that unit is 16 (x >> 1) + (8 (x & 1) + 2 y + cb), and the swizzle (< 16)
  // only touches the bracket, so x >> 1 becomes a constant 256-byte offset.
  const int tr_row = 4 * quad + (hl >> 2);
  constexpr int VXB = MB >= 8 ? 2 : 1;
  uint32_t vadr[VXB][4];
#pragma unroll
  for (int xb = 0; xb < VXB; ++xb)
#pragma unroll
    for (int y = 0; y < 4; ++y)
      vadr[xb][y] = tr_row * kRowB + (((8 * xb + 2 * y + ((hl & 3) >> 1)) ^ swz_v<kRowB>(tr_row)) * 16) +
                    (hl & 1) * 8;

  // Scores (S^T tiles) of one tile -- the block reads tile j's scores
  // before it writes tile j + 1's -- and P operands of two tiles, by parity.
  f32x4 sc[KB][NQB];
  V8 pv[2][KK][NQB];
  const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void_t*)smem;

  // QK of the first tile (before the loop), from K buffer 0.
  auto qk_first = [&]() __attribute__((always_inline)) {
    V8 ka[KS][KB];
    static_for<0, KS>([&](auto ks_) __attribute__((always_inline)) {
      constexpr int ks = decltype(ks_)::value;
      static_for<0, KB>([&](auto kb_) __attribute__((always_inline)) {
        constexpr int kb = decltype(kb_)::value;
        ka[ks][kb] = __builtin_bit_cast(V8, lds_b128<kb * 16 * kRowB>(lbase + kadr[ks]));
      });
    });
    lds_wait<0>(ka[0][0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) pin(ka[ks][kb]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
          sc[kb][qb] = mfma16x16x32(ka[ks][kb], qv[qb][ks],
                                    ks == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : sc[kb][qb]);
  };
  auto mask = [&](int t) __attribute__((always_inline)) {
    const int k0 = lo + (tb + t) * BK;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      const int qrel = rel0 + tok[qb];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * kb + 4 * quad + i;
          const bool ok = key < hi_r && key <= qrel && (a.window <= 0 || key > qrel - a.window);
          sc[kb][qb][i] = ok ? sc[kb][qb][i] : -INFINITY;
        }
    }
  };
  // Online softmax, base 2, with a lazy reference max: a column's m moves
  // only when one of its scores exceeds m by more than kRescale (so P stays
  // <= 2^kRescale), and the O / l rescale a move needs is applied before
  // the next PV step.  The QK product takes -mc as its accumulator input,
  // so scores arrive as s * scale * log2(e) - mc and P is exp2 of the score
  // as it stands.  The scores of tile j are in registers when iteration j
  // starts, so the growth check runs there, ahead of the interleaved block:
  // each lane compares the max of its own scores with lim, and only when some lane of the wave grew (rare after a
  // column's first tile) does the wave take the exact column max across the
  // four lanes of each column (l, l ^ 16, l ^ 32, l ^ 48) and move m.  The
  // block then forms P against the settled m.
  auto grow_check = [&]() __attribute__((always_inline)) {
    bool grow = false;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float mx = sc[0][qb][0];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][qb][i]);
      grow |= mx > lim[qb];
    }
    return __ballot(grow) != 0;
  };
  auto move_max = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float mx = sc[0][qb][0];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][qb][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const bool g = mx > lim[qb];
      const float mn = g ? mx + mc[qb] : m[qb];
      pend[qb] = g ? fast_exp2(m[qb] - mn) : 1.f;
      lsum[qb] *= pend[qb];  // l takes tile j's P next, formed against the moved m
      pend_any |= __ballot(g) != 0;
      // this tile's scores hold s - mc(old); shift them onto the new offset
      const float sh = g ? mx : 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[kb][qb][i] -= sh;
      m[qb] = mn;
      mc[qb] = g ? mn : mc[qb];
      lim[qb] = m[qb] - mc[qb] + kRescale;
    }
  };
  auto need_mask = [&](int t) {
    const int k0 = lo + (tb + t) * BK;
    return k0 + BK - 1 > rel0 + wt_first || k0 + BK > hi_r ||
           (a.window > 0 && k0 <= rel0 + wt_last - a.window);
  };

  // The interleaved block of iteration j (Q = parity of j - 1 and j + 1):
  // operands 0 .. NV-1 are the V^T operands of PV(j - 1) (two transposing
  // reads each, from V buffer 2 + Q), operands NV .. N-1 the K operands of
  // QK(j + 1) (one read each, from K buffer Q).  Reads run L operands ahead
  // of the MFMAs that consume them.  The softmax of tile j (scores in sc, P
  // into pv[P], row sums into lsum) is spread over the first KB * NQB
  // operand steps, all before the first QK MFMA overwrites sc.
  auto block = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    constexpr int Q = P ^ 1;
    constexpr int NV = KK * MB, NK = KS * KB, N = NV + NK;
    constexpr int NS = KB * NQB;
    constexpr int L = 4;
    static_assert(NS <= NV, "the softmax must read the scores before QK overwrites them");
    V8 opd[N];
    auto issue = [&](auto oo) __attribute__((always_inline)) {
      constexpr int O = decltype(oo)::value;
      if constexpr (O < NV) {
        constexpr int kk = O / MB, mb = O % MB;
        constexpr int base = (2 + Q) * kTileB + 32 * kk * kRowB + 256 * (mb >> 3);
        const uint32_t ad = lbase + vadr[(mb >> 2) & (VXB - 1)][mb & 3];
        const u32x2 v0 = lds_tr64<base>(ad);
        const u32x2 v1 = lds_tr64<base + 16 * kRowB>(ad);
        opd[O] = __builtin_bit_cast(V8, (u32x4){v0.x, v0.y, v1.x, v1.y});
      } else {
        constexpr int ks = (O - NV) / KB, kb = (O - NV) % KB;
        opd[O] = __builtin_bit_cast(V8, lds_b128<Q * kTileB + kb * 16 * kRowB>(lbase + kadr[ks]));
      }
    };
    static_for<0, L>(issue);
    static_for<0, N>([&](auto oo) __attribute__((always_inline)) {
      constexpr int O = decltype(oo)::value;
      if constexpr (O + L < N) issue(Par<O + L>());
      // reads issued after operand O's: one per later operand, two per later V operand
      constexpr int last = O + L < N ? O + L : N - 1;
      constexpr int later_v = O + 1 < NV ? (last < NV ? last : NV - 1) - O : 0;
      lds_wait<(last - O) + later_v>(opd[O]);
      if constexpr (O < NV) {
        constexpr int kk = O / MB, mb = O % MB;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) o[qb][mb] = mfma16x16x32(opd[O], pv[Q][kk][qb], o[qb][mb]);
      } else {
        constexpr int ks = (O - NV) / KB, kb = (O - NV) % KB;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
          sc[kb][qb] = mfma16x16x32(opd[O], qv[qb][ks],
                                    ks == 0 ? (f32x4){-mc[qb], -mc[qb], -mc[qb], -mc[qb]} : sc[kb][qb]);
      }
      if constexpr (O < NS) {
        constexpr int kb = O / NQB, qb = O % NQB;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(sc[kb][qb][i]);
          lsum[qb] += p;
          pv[P][kb >> 1][qb][4 * (kb & 1) + i] = from_f32<T>(p);
        }
      }
    });
  };

  // Paged: page of the K tile last loaded into buffer P (tile j + 2 - P's
  // parity partner), reused for that tile's V load two iterations later.
  int kpage[2] = {0, 0};

  // Iteration j: PV(j-1), softmax(j), QK(j+1) (tile indices), while the
  // direct loads of K(j+2) and V(j) land in the buffers iteration j-1 read.
  auto iteration = [&](auto par, int j) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;  // = j & 1
    // Nothing is outstanding here at run time (the previous iteration ended
    // with a full wait), but the compiler's wait tracking may still carry
    // memory operations from before the loop (a register spill store); left
    // pending, it answers them with a full memory wait in front of this
    // iteration's first LDS read, which would also wait for the tile loads
    // issued below.  An explicit wait here clears its scoreboard for free.
    __builtin_amdgcn_s_waitcnt(0);
    const int v_page = kpage[P];  // page of tile j, looked up with K(j)
    if (j + 2 < nt) {
      if constexpr (PAGED) kpage[P] = tile_page(j + 2);
      load_tile(kg, kgn, a.ks_pos, a.ks_page, kofs, j + 2, P, kpage[P]);
    }
    if (j < nt) load_tile(vg, vgn, a.vs_pos, a.vs_page, vofs, j, 2 + P, v_page);
    // Waves past their own key tiles (sharing a heavier tile's stream)
    // only load and meet the barrier.
    if (NW == 4 || j <= nt_own) {
      // Rescale for the m moved at tile j - 1 (O holds tiles <= j - 2 and is
      // about to take PV(j - 1), formed against the moved m; l was rescaled
      // at the move, before it took tile j - 1's P).
      if (__builtin_expect(pend_any, 0)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) o[qb][mb] *= pend[qb];
          pend[qb] = 1.f;
        }
        pend_any = false;
      }
      if (__builtin_expect(need_mask(j), 0)) mask(j);
      if (__builtin_expect(grow_check(), 0)) move_max();
      // One basic block of independent MFMA and VALU work.  At j = 0 the PV
      // step multiplies zeroed P by a zeroed V buffer; at j = nt the softmax
      // sees a fully masked tile (k0 >= hi_r) and its P is never used.
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      block(Par<P>());
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        pin(m[qb]);
        pin(mc[qb]);
        pin(lim[qb]);
        pin(pend[qb]);
        pin(lsum[qb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) pin(o[qb][mb]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) pin(pv[P][kk][qb]);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) pin(sc[kb][qb]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    bar();
  };

  // Zero V buffer 1 (read by the j = 0 PV step) and the P operands it uses.
#pragma unroll
  for (int i = 0; i < kTileB / (64 * NW * 16); ++i)
    *(u32x4*)(smem + 3 * kTileB + ((i * NW + lw) * 64 + lane) * 16) = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) pv[1][kk][qb] = (V8){};
  if (nt > 0) {
    if constexpr (PAGED) kpage[0] = tile_page(0);
    load_tile(kg, kgn, a.ks_pos, a.ks_page, kofs, 0, 0, kpage[0]);
  }
  if (nt > 1) {
    if constexpr (PAGED) kpage[1] = tile_page(1);
    load_tile(kg, kgn, a.ks_pos, a.ks_page, kofs, 1, 1, kpage[1]);
  }
  // The query columns' own work (the fused prologue, the scale) after the
  // first tile loads are issued, so that it overlaps their flight.
  if (a.qw != nullptr) {
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) fused_query<T, D>(a, qv[qb], tok[qb], quad);
  }
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      V8 x = qv[qb][ks];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = from_f32<T>(to_f32(x[e]) * c2);
      qv[qb][ks] = cok[qb] ? x : (V8){};
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  bar();
  qk_first();
  bar();  // K(0) fully read before iteration 0 refills its buffer
  for (int j = 0; j <= nt; j += 2) {
    iteration(Par<0>(), j);
    if (j + 1 <= nt) iteration(Par<1>(), j + 1);
  }

  // Partial layout: O as [wave][qb][mb][lane] f32x4 in part_o, then
  // [wave][qb][lane] l share, mc and m in part_st.
  constexpr int kPartO = NQB * MB * 64;  // f32x4 per wave
  if constexpr (MODE == kRunPartial) {
    // The loop ended with the group's barrier: no wave reads the tile
    // buffers any more, so part_o may overlay them.
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        ((f32x4*)part_o)[wave * kPartO + (qb * MB + mb) * 64 + lane] = o[qb][mb];
      float* st = part_st + ((wave * NQB + qb) * 3) * 64 + lane;
      st[0] = lsum[qb];
      st[64] = mc[qb];
      st[128] = m[qb];
    }
    __syncthreads();  // the block's one barrier: the merging group reads after it
    return;
  }
  if constexpr (MODE == kRunMerge) {
    __syncthreads();  // the block's one barrier: the partner's partial is in LDS
    // Both parts hold O and l relative to their own offset mc; a part whose
    // m is still -inf saw no visible key and weighs nothing.
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      const float* st = part_st + ((wave * NQB + qb) * 3) * 64 + lane;
      const float l1 = st[0], mc1 = st[64], m1 = st[128];
      const bool v0 = m[qb] != -INFINITY, v1 = m1 != -INFINITY;
      const float M = fmaxf(v0 ? mc[qb] : -INFINITY, v1 ? mc1 : -INFINITY);
      const float w0 = v0 ? fast_exp2(mc[qb] - M) : 0.f;
      const float w1 = v1 ? fast_exp2(mc1 - M) : 0.f;
      lsum[qb] = lsum[qb] * w0 + l1 * w1;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        o[qb][mb] = o[qb][mb] * w0 +
                    ((const f32x4*)part_o)[wave * kPartO + (qb * MB + mb) * 64 + lane] * w1;
    }
  }

#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    // the column's sum over its four lanes (l, l ^ 16, l ^ 32, l ^ 48)
    float lt = lsum[qb];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (!cok[qb]) continue;
    const int64_t ofs = ((int64_t)tok[qb] * a.q_heads + hq[qb]) * D + 4 * quad;
    TO* op = (TO*)a.out + ofs;
    if (a.gate != nullptr) {  // the sigmoid output gate, before the single rounding
      typedef typename Vec4<T>::type V4;
      const T* gp =
          (const T*)a.gate + ((int64_t)tok[qb] * a.q_heads + hq[qb]) * a.gate_stride + 4 * quad;
      V4 gv[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) gv[mb] = *(const V4*)(gp + 16 * mb);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          op[16 * mb + i] = from_f32<TO>(o[qb][mb][i] * inv * fast_sigmoid(to_f32(gv[mb][i])));
      }
      continue;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) op[16 * mb + i] = from_f32<TO>(o[qb][mb][i] * inv);
    }
  }
}

template <typename T, typename TO, int D, int BK, int NQB, bool PAGED = false>
__global__ void __launch_bounds__(256, 2)
prefill_mfma(PrefillArgs a) {
  constexpr int kTileB = BK * D * (int)sizeof(T);
  constexpr int kCols = 64 * NQB;
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileB];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int kvh, ctile;
  if (!prefill_work(a, kvh, ctile)) return;
  // The heavy column tiles (late tokens, many key tiles) set the kernel's
  // end time, so of each tile and its mirror col_tiles - 1 - ctile the
  // lighter one copies both tiles' rows (each tile's rows exactly once).
  if (!PAGED && a.kn != nullptr) {
    const int mirror = a.col_tiles - 1 - ctile;
    if (ctile <= mirror) copy_tile_rows<T, D, kCols>(a, kvh, ctile, tid);
    if (ctile < mirror) copy_tile_rows<T, D, kCols>(a, kvh, mirror, tid);
  }
  auto bar = []() __attribute__((always_inline)) { __syncthreads(); };
  prefill_run<T, TO, D, BK, NQB, PAGED, kRunWrite, 4>(a, kvh, ctile, 0, -1, smem, nullptr,
                                                      nullptr, wave, tid, bar, wave, -1, false);
}

// Work of a prefill_pair block: kv head kvh and the column tiles ta (light:
// earlier tokens) and tb = col_tiles - 1 - ta (heavy; equal to ta for the
// middle tile of an odd count).  Pairs are ordered kv-head-major and cut
// into 8 contiguous slices, slice x on XCD x, so one kv head's blocks share
// one XCD's L2.
__device__ __forceinline__ bool pair_work(const PrefillArgs& a, int& kvh, int& ta, int& tb) {
  const int b = blockIdx.x;
  const int item = (b % kXcds) * a.per_xcd + b / kXcds;
  const int pairs = (a.col_tiles + 1) / 2;
  if (item >= a.kv_heads * pairs) return false;
  kvh = item / pairs;
  ta = item - kvh * pairs;
  tb = a.col_tiles - 1 - ta;
  return true;
}

// Barrier of one four-wave group of a prefill_pair block: a counter in LDS
// that each wave raises once per barrier; the k-th barrier waits until it
// reads 4 k.  A polling wave spends its time waiting on its LDS read, so
// the other group's wave on the same SIMD keeps the issue slots (a sleep
// between polls measured slower: it delays the wake-up).  The wait gives
// up after 2^22 polls, a guard against a mismatched barrier count (never
// reached in a correct run: the waves of a workgroup are resident
// together, so all four arrive).
struct GroupBarrier {
  uint32_t* ctr;
  uint32_t target;
  __device__ __forceinline__ void operator()() {
    target += 4;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0)
      __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (int i = 0; i < (1 << 22); ++i) {
      const uint32_t v = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      if (v >= target) break;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};

// Causal imbalance removed: one block of eight waves per CU takes a light
// and a heavy column tile of one kv head.  Waves 0-3 (group 0) run the
// light tile over all its key tiles, then the heavy tile over its key
// tiles [s, nt_b); waves 4-7 (group 1) run the heavy tile over [0, s),
// with s chosen so that both groups walk about the same number of tiles.
// Each group has its own four tile buffers and its own barrier, so the two
// groups' pipelines run independently (as two co-resident blocks would);
// at the end group 0 leaves its heavy-tile partial in its LDS and group 1
// merges it into its own (one block barrier) and writes the heavy tile.
template <typename T, typename TO, int D, int BK, int NQB>
__global__ void __launch_bounds__(512, 1)
prefill_pair(PrefillArgs a) {
  constexpr int kTileB = BK * D * (int)sizeof(T);
  constexpr int kCols = 64 * NQB;
  constexpr int MB = D / 16;
  static_assert(NQB * MB * 64 * 16 * 4 <= 4 * kTileB, "the partial O must fit a group's buffers");
  __shared__ __attribute__((aligned(1024))) char smem[8 * kTileB];
  __shared__ float part_st[4 * NQB * 3 * 64];
  __shared__ uint32_t gctr[2];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  int kvh, ta, tbt;
  if (!pair_work(a, kvh, ta, tbt)) return;
  if (tid < 2) gctr[tid] = 0;
  __syncthreads();  // the group counters are zero before any group barrier
  int lo, hi, nta = 0, ntb;
  if (ta != tbt) tile_keys<BK, kCols>(a, ta, lo, hi, nta);
  tile_keys<BK, kCols>(a, tbt, lo, hi, ntb);
  // Group 0 also pays a second pipeline start: one tile's worth.
  const int split = min(ntb, (nta + ntb + (ta != tbt ? 1 : 0) + 1) / 2);
  GroupBarrier bar{gctr + grp, 0u};
  char* gsmem = smem + grp * 4 * kTileB;
  const int gw = wave & 3, gtid = tid & 255;
  if (grp == 0) {
    // the light tile, then the heavy tile's key tiles [split, nt_b)
    if (ta != tbt) {
      if (a.kn != nullptr) copy_tile_rows<T, D, kCols>(a, kvh, ta, gtid);
      prefill_run<T, TO, D, BK, NQB, false, kRunWrite, 4>(a, kvh, ta, 0, -1, gsmem, nullptr,
                                                          nullptr, gw, gtid, bar, gw, -1, false);
    }
    prefill_run<T, TO, D, BK, NQB, false, kRunPartial, 4>(a, kvh, tbt, split, -1, gsmem,
                                                          (float*)smem, part_st, gw, gtid, bar,
                                                          gw, -1, false);
  } else {
    // the heavy tile's key tiles [0, split), merged with group 0's part
    if (a.kn != nullptr) copy_tile_rows<T, D, kCols>(a, kvh, tbt, gtid);
    prefill_run<T, TO, D, BK, NQB, false, kRunMerge, 4>(a, kvh, tbt, 0, split, gsmem,
                                                        (float*)smem, part_st, gw, gtid, bar, gw,
                                                        -1, false);
  }
}

// One K/V tile stream for a light and a heavy column tile: one block of
// eight waves per CU takes column tile ta (waves 0-3) and its mirror
// tb = col_tiles - 1 - ta (waves 4-7) of one kv head.  Without a window
// both walk the key tiles from row 0, so one set of tile buffers, loaded
// by all eight waves, serves both tiles: half the direct-load bytes per
// FLOP of two four-wave blocks, which load the same tiles separately.  The
// loads' LDS writes and texture-path time are about a fifth of the
// four-wave kernel's loop at head_dim 128, where LDS reads (K operands at
// 244 B/clk per CU, transposing V reads at 131) and those writes come
// close to the MFMA time.  The light waves stop computing after their own
// last key tile and keep loading; the middle tile of an odd count goes to
// waves 4-7 alone.
template <typename T, typename TO, int D, int BK, int NQB>
__global__ void __launch_bounds__(512, 1)
prefill_shared(PrefillArgs a) {
  constexpr int kTileB = BK * D * (int)sizeof(T);
  constexpr int kCols = 64 * NQB;
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileB];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  int kvh, ta, tbt;
  if (!pair_work(a, kvh, ta, tbt)) return;
  int lo, hi_b, ntb;
  tile_keys<BK, kCols>(a, tbt, lo, hi_b, ntb);
  if (a.kn != nullptr && (grp == 1 || ta != tbt))
    copy_tile_rows<T, D, kCols>(a, kvh, grp == 0 ? ta : tbt, tid & 255);
  auto bar = []() __attribute__((always_inline)) { __syncthreads(); };
  prefill_run<T, TO, D, BK, NQB, false, kRunWrite, 8>(a, kvh, grp == 0 ? ta : tbt, 0, -1, smem,
                                                      nullptr, nullptr, wave & 3, tid, bar, wave,
                                                      hi_b, grp == 0 && ta == tbt);
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

// Paged caches: output in the cache dtype only.
template <typename T>
const void* pick_kernel_paged(int D) {
  switch (D) {
    case 64: return (const void*)prefill_mfma<T, T, 64, 64, 2, true>;
    case 128: return (const void*)prefill_mfma<T, T, 128, 64, 2, true>;
    case 256: return (const void*)prefill_mfma<T, T, 256, 32, 1, true>;
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

template <typename T, typename TO>
const void* pick_pair(int D) {
  switch (D) {
    case 64: return (const void*)prefill_pair<T, TO, 64, 64, 2>;
    case 128: return (const void*)prefill_pair<T, TO, 128, 64, 2>;
    case 256: return (const void*)prefill_pair<T, TO, 256, 32, 1>;
  }
  return nullptr;
}

template <typename T, typename TO>
const void* pick_shared(int D) {
  switch (D) {
    case 64: return (const void*)prefill_shared<T, TO, 64, 64, 2>;
    case 128: return (const void*)prefill_shared<T, TO, 128, 64, 2>;
    case 256: return (const void*)prefill_shared<T, TO, 256, 32, 1>;
  }
  return nullptr;
}

template <typename T>
const void* pick_shared_out(int D, int out_dtype) {
  switch (out_dtype) {
    case ALPX_F32: return pick_shared<T, float>(D);
    case ALPX_F16: return pick_shared<T, f16_t>(D);
    default: return pick_shared<T, bf16_t>(D);
  }
}

template <typename T>
const void* pick_pair_out(int D, int out_dtype) {
  switch (out_dtype) {
    case ALPX_F32: return pick_pair<T, float>(D);
    case ALPX_F16: return pick_pair<T, f16_t>(D);
    default: return pick_pair<T, bf16_t>(D);
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

namespace {

// Key tiles (of `rows` rows) that column tile ct walks: tile_keys on the host.
int host_tile_keys(int q_tokens, int kv_tokens, int group, int rel0, int window, int cols_per_block,
                   int rows, int ct) {
  const int cols = q_tokens * group;
  const int col0 = ct * cols_per_block;
  const int hi = std::max(0, std::min(kv_tokens, rel0 + (std::min(col0 + cols_per_block, cols) - 1) / group + 1));
  int lo = 0;
  if (window > 0) lo = std::min(hi, std::max(0, rel0 + col0 / group - window + 1)) / rows * rows;
  return (hi - lo + rows - 1) / rows;
}

// Kernel choice for contiguous caches.  The paired kernel gains the tail a
// heavy column tile runs alone and pays a second pipeline start (group 0)
// and the final merge.  Same-box sweep (2048 query tokens, 32/8 or 16/2
// heads, pair / single time): head_dim 128 at prefix 0, 512, 1024, 2048,
// 4096 -- 0.94, 0.98, 1.00, 1.04, 1.03; head_dim 256 at prefix 0, 2048,
// 8192 -- 0.75, 0.91, 1.04; head_dim 64 at prefix 0, 2048 -- 0.92, 0.98;
// 512 query tokens (64 pairs) 1.37; 8192 tokens at prefix 0 (four rounds
// of pairs) 1.02.  So: pairs must form one round that fills the device,
// and the heaviest column tile must walk at least R times the key tiles of
// the lightest, R = 3 at head_dim 128 and 1.8 at 64 and 256.  At head_dim
// 256 several rounds of pairs pay as well (16/2 heads, pair / single:
// 4096 tokens at prefix 0 -- 162 / 232 us, at prefix 1024 -- 240 / 292,
// 8192 tokens at prefix 0 -- 656 / 859).  The shared-stream kernel (one
// tile stream for both tiles of a pair, no window start inside the chunk)
// pays off at head_dim 256 with long prefixes only (2048 tokens, 16/2
// heads, shared / pair / single, us, one box: prefix 1024 -- 86.9 / 82.7 /
// 96.6, 1536 -- 101.8 / 99.4 / 113.0, 2048 -- 118.9 / 115.8 / 127.7, 8192
// -- 304.5 / 316.1 / 311.4; another box: 4096 -- 178.4 / 187.7 / 191.1;
// head_dim 128 at prefix 2048: 104.7 / 105.4 / 100.8, head_dim 64: 72.1 /
// 65.2 / 66.4), so it takes one round of pairs below a ratio of
// kSharedBelow10 / 10.
// ALPX_OVERRIDE_PREFILL_KERNEL (1 single, 2 paired, 3 shared-stream)
// overrides the choice (shared falls back to the single kernel where one
// stream cannot serve).
enum PrefillKernelChoice { kSingleKernel, kPairKernel, kSharedKernel };
constexpr int kSharedBelow10 = 16;

PrefillKernelChoice choose_prefill(int q_tokens, int kv_tokens, int kv_heads, int group, int rel0,
                                   int window, int cols_per_block, int rows, int col_tiles,
                                   int key_dim, const void* pair_kernel) {
  // both tiles of a pair walk the key rows from 0 when no window starts inside the chunk
  const bool one_stream = window <= 0 || (int64_t)window > (int64_t)rel0 + q_tokens;
  const int force = alpx::override_value(ALPX_OVERRIDE_PREFILL_KERNEL);
  if (force == 2) return kPairKernel;
  if (force == 1) return kSingleKernel;
  if (force == 3) return one_stream ? kSharedKernel : kSingleKernel;
  const int64_t pairs = (int64_t)kv_heads * ((col_tiles + 1) / 2);
  const int resident = alpx::resident_blocks(pair_kernel, 512, 0);
  if (resident <= 0) return kSingleKernel;
  const bool one_round = pairs <= resident && pairs * 10 >= (int64_t)resident * 9;
  if (!one_round && !(key_dim == 256 && pairs > resident)) return kSingleKernel;
  const int first = host_tile_keys(q_tokens, kv_tokens, group, rel0, window, cols_per_block, rows, 0);
  const int last =
      host_tile_keys(q_tokens, kv_tokens, group, rel0, window, cols_per_block, rows, col_tiles - 1);
  const int64_t ratio10 = (int64_t)last * 10 / std::max(1, first);
  if (key_dim == 256 && one_round && one_stream && ratio10 < kSharedBelow10) return kSharedKernel;
  const int r10 = key_dim == 128 ? 30 : 18;  // R x 10
  return ratio10 >= r10 ? kPairKernel : kSingleKernel;
}

// Whether prefill_impl runs these operands on the MFMA kernels: fp16 /
// bf16, equal head dims of 64, 128 or 256, 16-byte aligned buffers and row
// strides (`align` ORs their addresses and byte strides), and per-tile row
// offsets that fit 32 bits.  Otherwise it takes the split-K path, which
// needs a workspace of alpx_prefill_workspace_bytes.
bool mfma_prefill_applies(int dtype, int key_dim, int value_dim, uintptr_t align,
                          int64_t kv_tokens, int64_t k_pos_stride, int64_t v_pos_stride,
                          int64_t rel0) {
  const int64_t es = (int64_t)alpx::dtype_size(dtype);
  return dtype != ALPX_F32 && key_dim == value_dim &&
         (key_dim == 64 || key_dim == 128 || key_dim == 256) && (align & 15) == 0 &&
         alpx::override_value(ALPX_OVERRIDE_PREFILL_GENERIC) == 0 &&
         kv_tokens * k_pos_stride * es < ((int64_t)1 << 31) &&
         kv_tokens * v_pos_stride * es < ((int64_t)1 << 31) && rel0 < ((int64_t)1 << 30) &&
         rel0 > -((int64_t)1 << 30);
}

// The query prologue a prefill forms itself (alpx_attention_layer_prefill
// with no query_out): q is then the joint projection [T, Hq, 2 D].
struct QueryPrologue {
  const float* qw;
  const float2* rot;  // [T, R] (cos, sin) per token and pair
  float eps;
  int R;
};

int prefill_impl(const void* q, const void* key, const void* value, const void* gate, void* out,
                 void* workspace, size_t workspace_bytes, int q_tokens, int kv_tokens,
                 int q_heads, int kv_heads, int key_dim, int value_dim, int64_t k_pos_stride,
                 int64_t v_pos_stride, int64_t q_pos0, int window, int64_t kv_start, float scale,
                 int dtype, int out_dtype, void* stream, const int32_t* pages = nullptr,
                 int page_shift = 0, int num_pages = 0, const void* kn = nullptr,
                 const void* vn = nullptr, int64_t gate_stride = 0,
                 const QueryPrologue* qpro = nullptr) {
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
  // Append mode reads the chunk's rows through the cache's row strides.
  if (kn != nullptr && (k_pos_stride != (int64_t)kv_heads * key_dim ||
                        v_pos_stride != (int64_t)kv_heads * value_dim))
    return fail(ALPX_EINVAL, "alpx_prefill_append: cache rows must be contiguous");
  if (gate_stride == 0) gate_stride = value_dim;
  const int64_t q_stride = qpro != nullptr ? 2 * (int64_t)key_dim : key_dim;
  const uintptr_t align = (uintptr_t)q | (uintptr_t)(q_stride * es) | (uintptr_t)key |
                          (uintptr_t)value | (uintptr_t)gate |
                          (uintptr_t)(gate_stride * es) |
                          (uintptr_t)kn | (uintptr_t)vn | (uintptr_t)(k_pos_stride * es) |
                          (uintptr_t)(v_pos_stride * es);
  const bool mfma = mfma_prefill_applies(dtype, key_dim, value_dim, align, kv_tokens, k_pos_stride,
                                         v_pos_stride, q_pos0 - kv_start);
  if (pages != nullptr && !(mfma && out_dtype == dtype))
    return fail(ALPX_EUNSUPPORTED,
                "alpx_prefill_causal_paged: needs fp16/bf16 pages, head_dim in {64, 128, 256}, "
                "16-byte aligned rows and out_dtype == dtype");
  if (mfma) {
    const int cols_per_block = key_dim == 256 ? 64 : 128;
    const int tile_rows = key_dim == 256 ? 32 : 64;
    const int col_tiles = (int)(((int64_t)q_tokens * group + cols_per_block - 1) / cols_per_block);
    const PrefillKernelChoice choice =
        pages != nullptr
            ? kSingleKernel
            : choose_prefill(q_tokens, kv_tokens, kv_heads, group, (int)(q_pos0 - kv_start), window,
                             cols_per_block, tile_rows, col_tiles, key_dim,
                             dtype == ALPX_F16 ? pick_pair_out<f16_t>(key_dim, out_dtype)
                                               : pick_pair_out<bf16_t>(key_dim, out_dtype));
    const bool pair = choice == kPairKernel, shared = choice == kSharedKernel;
    const void* kernel = nullptr;
    if (pages != nullptr)
      kernel = dtype == ALPX_F16 ? pick_kernel_paged<f16_t>(key_dim)
                                 : pick_kernel_paged<bf16_t>(key_dim);
    else if (shared)
      kernel = dtype == ALPX_F16 ? pick_shared_out<f16_t>(key_dim, out_dtype)
                                 : pick_shared_out<bf16_t>(key_dim, out_dtype);
    else if (pair)
      kernel = dtype == ALPX_F16 ? pick_pair_out<f16_t>(key_dim, out_dtype)
                                 : pick_pair_out<bf16_t>(key_dim, out_dtype);
    else if (dtype == ALPX_F16)
      kernel = pick_kernel_out<f16_t>(key_dim, out_dtype);
    else
      kernel = pick_kernel_out<bf16_t>(key_dim, out_dtype);
    PrefillArgs a = {};
    a.kn = kn;
    a.vn = vn;
    a.new0 = (int)(q_pos0 - kv_start);
    a.pages = pages;
    a.page_shift = page_shift;
    a.num_pages = num_pages;
    a.ks_page = ((int64_t)1 << page_shift) * k_pos_stride;
    a.vs_page = ((int64_t)1 << page_shift) * v_pos_stride;
    a.q = q;
    a.q_stride = q_stride;
    if (qpro != nullptr) {
      a.qw = qpro->qw;
      a.q_rot = qpro->rot;
      a.q_eps = qpro->eps;
      a.q_R = qpro->R;
    }
    a.k = key;
    a.v = value;
    a.gate = gate;
    a.gate_stride = gate_stride;
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
    a.col_tiles = col_tiles;
    const bool paired = pair || shared;  // a light and a heavy column tile per block
    const int64_t items = (int64_t)(paired ? (a.col_tiles + 1) / 2 : a.col_tiles) * kv_heads;
    a.per_xcd = (int)((items + kXcds - 1) / kXcds);
    a.scale_log2 = scale * kLog2e;
    TimedRegion timed(ALPX_T_PREFILL, s);
    void* args[] = {(void*)&a};
    hipError_t err = hipLaunchKernel(kernel, dim3(a.per_xcd * kXcds), dim3(paired ? 512 : 256),
                                     args, 0, s);
    if (err != hipSuccess)
      return fail(ALPX_EHIP, "prefill launch failed: %s", hipGetErrorString(err));
    return check_launch("prefill_mfma");
  }

  if (qpro != nullptr)  // callers check the MFMA conditions before any launch
    return fail(ALPX_EUNSUPPORTED, "fused query prologue: MFMA prefill shapes only");
  if (!workspace) return fail(ALPX_EINVAL, "alpx_prefill_causal: null workspace");
  if (kn != nullptr) {  // append mode off the MFMA path: the append kernel first
    const int rc = alpx_kv_append(const_cast<void*>(key), const_cast<void*>(value), kn, vn, dtype,
                                  kv_tokens, 1, kv_heads, key_dim, value_dim, q_tokens,
                                  q_pos0 - kv_start, nullptr, stream);
    if (rc != ALPX_OK) return rc;
  }
  DecodeArgs a = {};
  a.q = q;
  a.k = key;
  a.v = value;
  a.seq_lens = nullptr;
  a.gate = gate;  // the combine pass applies it ([token][head][d] = [b][h][d])
  a.gate_stride = gate_stride;
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

}  // namespace

extern "C" int alpx_prefill_causal(const void* q, const void* key, const void* value, void* out,
                                   void* workspace, size_t workspace_bytes, int q_tokens,
                                   int kv_tokens, int q_heads, int kv_heads, int key_dim,
                                   int value_dim, int64_t k_pos_stride, int64_t v_pos_stride,
                                   int64_t q_pos0, int window, int64_t kv_start, float scale,
                                   int dtype, int out_dtype, void* stream) {
  return prefill_impl(q, key, value, nullptr, out, workspace, workspace_bytes, q_tokens, kv_tokens,
                      q_heads, kv_heads, key_dim, value_dim, k_pos_stride, v_pos_stride, q_pos0,
                      window, kv_start, scale, dtype, out_dtype, stream);
}

extern "C" int alpx_prefill_causal_gated(const void* q, const void* key, const void* value,
                                         const void* gate, void* out, void* workspace,
                                         size_t workspace_bytes, int q_tokens, int kv_tokens,
                                         int q_heads, int kv_heads, int key_dim, int value_dim,
                                         int64_t k_pos_stride, int64_t v_pos_stride,
                                         int64_t q_pos0, int window, int64_t kv_start,
                                         float scale, int dtype, int out_dtype, void* stream) {
  if (!gate) return alpx::fail(ALPX_EINVAL, "alpx_prefill_causal_gated: null gate");
  return prefill_impl(q, key, value, gate, out, workspace, workspace_bytes, q_tokens, kv_tokens,
                      q_heads, kv_heads, key_dim, value_dim, k_pos_stride, v_pos_stride, q_pos0,
                      window, kv_start, scale, dtype, out_dtype, stream);
}

extern "C" int alpx_prefill_append(const void* q, const void* key, const void* value,
                                   void* key_cache, void* value_cache, const void* gate, void* out,
                                   void* workspace, size_t workspace_bytes, int q_tokens,
                                   int64_t capacity, int q_heads, int kv_heads, int key_dim,
                                   int value_dim, int64_t position, int window, float scale,
                                   int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  if (!key || !value || !key_cache || !value_cache)
    return fail(ALPX_EINVAL, "alpx_prefill_append: null buffer");
  if (q_tokens <= 0 || capacity <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0)
    return fail(ALPX_EINVAL, "alpx_prefill_append: sizes must be positive");
  if (position < 0 || position > capacity - q_tokens)
    return fail(ALPX_ERANGE, "attention cache position exceeds capacity");
  if (position + q_tokens > INT32_MAX)
    return fail(ALPX_EUNSUPPORTED, "alpx_prefill_append: more than 2^31 - 1 cache rows");
  return prefill_impl(q, key_cache, value_cache, gate, out, workspace, workspace_bytes, q_tokens,
                      (int)(position + q_tokens), q_heads, kv_heads, key_dim, value_dim,
                      (int64_t)kv_heads * key_dim, (int64_t)kv_heads * value_dim, position, window,
                      0, scale, dtype, out_dtype, stream, nullptr, 0, 0, key, value);
}

extern "C" int alpx_attention_layer_prefill(
    const void* query_gate, const void* key, const void* value, const float* q_norm,
    const float* k_norm, void* query_out, void* key_cache, void* value_cache, void* out,
    void* workspace, size_t workspace_bytes, int dtype, int out_dtype, int64_t capacity,
    int cache_batch, int batch_index, int tokens, int q_heads, int kv_heads, int head_dim,
    int64_t position, const int* sections, double frequency_base, float eps, float scale,
    void* stream) {
  using namespace alpx;
  if (!out) return fail(ALPX_EINVAL, "alpx_attention_layer_prefill: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(ALPX_EINVAL, "alpx_attention_layer_prefill: unknown dtype");
  if (tokens <= 0 || head_dim <= 0 || kv_heads <= 0 || cache_batch <= 0)
    return fail(ALPX_EINVAL, "alpx_attention_layer_prefill: sizes must be positive");
  if (head_dim > 256)
    return fail(ALPX_EUNSUPPORTED, "alpx_prefill_causal: head dims above 256 are not supported");
  if (position + tokens > INT32_MAX)
    return fail(ALPX_EUNSUPPORTED, "alpx_attention_layer_prefill: more than 2^31 - 1 cache rows");
  // The prefill's checks that need no device work, first: a failing call
  // must not have written the caches.
  if (!workspace && !(dtype != ALPX_F32 && (head_dim == 64 || head_dim == 128 || head_dim == 256)))
    return fail(ALPX_EINVAL, "alpx_prefill_causal: null workspace");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  const size_t es = dtype_size(dtype);
  const int64_t row = (int64_t)cache_batch * kv_heads * head_dim;
  const int64_t seq = (int64_t)batch_index * kv_heads * head_dim;
  const void* kseq = (const char*)key_cache + seq * es;
  const void* vseq = (const char*)value_cache + seq * es;
  const void* gate = (const char*)query_gate + head_dim * es;
  if (query_out == nullptr) {
    // The prefill forms the query rows from query_gate (its Q load runs the
    // prologue's norm and rotation); the prologue launch writes the key and
    // value rows only.  Needs the MFMA prefill and rotary pairs in whole
    // 32-channel groups; checked before any launch.
    int R = 0;
    if (!query_gate || !q_norm || bad_sections(sections, R) || R % 32 != 0 || 2 * R > head_dim ||
        !(frequency_base > 0.0) || !isfinite(frequency_base))
      return fail(ALPX_EUNSUPPORTED,
                  "alpx_attention_layer_prefill without query_out: needs rotary sections summing "
                  "to a multiple of 32 and a valid frequency base");
    const uintptr_t align = (uintptr_t)query_gate | (uintptr_t)kseq | (uintptr_t)vseq |
                            (uintptr_t)q_norm | (uintptr_t)(row * es) |
                            (uintptr_t)(2 * head_dim * es);
    if (!((dtype == ALPX_F16 || dtype == ALPX_BF16) &&
          (head_dim == 64 || head_dim == 128 || head_dim == 256) && (align & 15) == 0 &&
          override_value(ALPX_OVERRIDE_PREFILL_GENERIC) == 0 &&
          (position + tokens) * row * (int64_t)es < ((int64_t)1 << 31)))
      return fail(ALPX_EUNSUPPORTED,
                  "alpx_attention_layer_prefill without query_out: needs fp16/bf16, head_dim in "
                  "{64, 128, 256}, 16-byte aligned rows and q_norm, and a cache under 2 GiB per "
                  "tensor");
    const size_t need = (size_t)tokens * R * sizeof(float2);
    if (!workspace || workspace_bytes < need)
      return fail(ALPX_EINVAL, "alpx_attention_layer_prefill: workspace of %zu bytes, %zu needed",
                  workspace ? workspace_bytes : (size_t)0, need);
    QueryPrologue qp = {};
    qp.qw = q_norm;
    qp.rot = (const float2*)workspace;
    qp.eps = eps;
    qp.R = R;
    const int rc = attention_prologue_chunk_kv(
        query_gate, key, value, q_norm, k_norm, key_cache, value_cache, dtype, capacity,
        cache_batch, batch_index, tokens, q_heads, kv_heads, head_dim, head_dim, position,
        sections, frequency_base, eps, (float2*)workspace, stream);
    if (rc != ALPX_OK) return rc;
    return prefill_impl(query_gate, kseq, vseq, gate, out, workspace, workspace_bytes, tokens,
                        (int)(position + tokens), q_heads, kv_heads, head_dim, head_dim, row, row,
                        position, 0, 0, scale, dtype, out_dtype, stream, nullptr, 0, 0, nullptr,
                        nullptr, 2 * (int64_t)head_dim, &qp);
  }
  // The query-buffer form: where the prefill will not take the MFMA
  // kernels, its split-K path needs a workspace, checked before the
  // prologue writes the caches.
  const uintptr_t qalign = (uintptr_t)query_out | (uintptr_t)(head_dim * es) | (uintptr_t)kseq |
                           (uintptr_t)vseq | (uintptr_t)gate | (uintptr_t)(2 * head_dim * es) |
                           (uintptr_t)(row * es);
  if (!mfma_prefill_applies(dtype, head_dim, head_dim, qalign, position + tokens, row, row,
                            position)) {
    const size_t need =
        alpx_prefill_workspace_bytes(tokens, q_heads, kv_heads, head_dim, (int)(position + tokens));
    if (need == 0) return fail(ALPX_EINVAL, "alpx_attention_layer_prefill: invalid sizes");
    if (!workspace || workspace_bytes < need)
      return fail(ALPX_EINVAL,
                  "alpx_attention_layer_prefill: the split-K prefill needs a workspace of %zu "
                  "bytes, %zu given (null workspace)",
                  need, workspace ? workspace_bytes : (size_t)0);
  }
  const int rc = alpx_attention_prologue_chunk(
      query_gate, key, value, q_norm, k_norm, query_out, nullptr, key_cache, value_cache, dtype,
      capacity, cache_batch, batch_index, tokens, q_heads, kv_heads, head_dim, head_dim, position,
      sections, frequency_base, eps, stream);
  if (rc != ALPX_OK) return rc;
  return prefill_impl(query_out, kseq, vseq, gate, out, workspace, workspace_bytes, tokens,
                      (int)(position + tokens), q_heads, kv_heads, head_dim, head_dim, row, row,
                      position, 0, 0, scale, dtype, out_dtype, stream, nullptr, 0, 0, nullptr,
                      nullptr, 2 * (int64_t)head_dim);
}

extern "C" int alpx_attention_layer_prefill_paged(
    const void* query_gate, const void* key, const void* value, const float* q_norm,
    const float* k_norm, void* key_pages, void* value_pages, const int32_t* block_table,
    int max_pages, int page_size, int num_pages, int batch_index, void* out, void* workspace,
    size_t workspace_bytes, int dtype, int tokens, int q_heads, int kv_heads, int head_dim,
    int64_t position, const int* sections, double frequency_base, float eps, float scale,
    void* stream) {
  using namespace alpx;
  const char* what = "alpx_attention_layer_prefill_paged";
  if (!query_gate || !key || !value || !q_norm || !k_norm || !key_pages || !value_pages ||
      !block_table || !out)
    return fail(ALPX_EINVAL, "%s: null buffer", what);
  if (!dtype_ok(dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", what);
  if (tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || max_pages <= 0 ||
      num_pages <= 0 || batch_index < 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", what);
  if (page_size < 64 || (page_size & (page_size - 1)) != 0)
    return fail(ALPX_EINVAL, "%s: page_size must be a power of two >= 64", what);
  if (position < 0 || position + tokens > (int64_t)max_pages * page_size)
    return fail(ALPX_ERANGE, "attention cache position exceeds capacity");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(ALPX_EINVAL, "attention scale must be positive and finite");
  // Everything the two launches check, first: a failing call writes no page.
  int R = 0;
  if (bad_sections(sections, R) || R % 32 != 0 || 2 * R > head_dim ||
      !(frequency_base > 0.0) || !isfinite(frequency_base))
    return fail(ALPX_EUNSUPPORTED,
                "%s: needs rotary sections summing to a multiple of 32 (at most head_dim / 2) "
                "and a valid frequency base", what);
  const size_t es = dtype_size(dtype);
  const int64_t row = (int64_t)kv_heads * head_dim;
  const uintptr_t align = (uintptr_t)query_gate | (uintptr_t)key_pages | (uintptr_t)value_pages |
                          (uintptr_t)q_norm | (uintptr_t)(row * es) |
                          (uintptr_t)(2 * head_dim * es);
  if (!((dtype == ALPX_F16 || dtype == ALPX_BF16) &&
        (head_dim == 64 || head_dim == 128 || head_dim == 256) && (align & 15) == 0 &&
        override_value(ALPX_OVERRIDE_PREFILL_GENERIC) == 0 && position < ((int64_t)1 << 30) &&
        (position + tokens) * row * (int64_t)es < ((int64_t)1 << 31)))
    return fail(ALPX_EUNSUPPORTED,
                "%s: needs fp16/bf16 pages, head_dim in {64, 128, 256}, 16-byte aligned rows and "
                "q_norm, and under 2 GiB of logical rows", what);
  const size_t need = (size_t)tokens * R * sizeof(float2);
  if (!workspace || workspace_bytes < need)
    return fail(ALPX_EINVAL, "%s: workspace of %zu bytes, %zu needed", what,
                workspace ? workspace_bytes : (size_t)0, need);
  const int page_shift = __builtin_ctz((unsigned)page_size);
  const int32_t* table = block_table + (int64_t)batch_index * max_pages;
  QueryPrologue qp = {};
  qp.qw = q_norm;
  qp.rot = (const float2*)workspace;
  qp.eps = eps;
  qp.R = R;
  const int rc = attention_prologue_chunk_kv(
      query_gate, key, value, q_norm, k_norm, key_pages, value_pages, dtype,
      (int64_t)max_pages * page_size, 1, 0, tokens, q_heads, kv_heads, head_dim, head_dim,
      position, sections, frequency_base, eps, (float2*)workspace, stream, table, page_shift,
      num_pages);
  if (rc != ALPX_OK) return rc;
  return prefill_impl(query_gate, key_pages, value_pages, (const char*)query_gate + head_dim * es,
                      out, nullptr, 0, tokens, (int)(position + tokens), q_heads, kv_heads,
                      head_dim, head_dim, row, row, position, 0, 0, scale, dtype, dtype, stream,
                      table, page_shift, num_pages, nullptr, nullptr, 2 * (int64_t)head_dim, &qp);
}

extern "C" int alpx_prefill_causal_paged(const void* q, const void* key_pages,
                                         const void* value_pages, const int32_t* block_table,
                                         int max_pages, int page_size, int num_pages,
                                         int batch_index, const void* gate, void* out,
                                         int q_tokens, int kv_tokens, int q_heads, int kv_heads,
                                         int head_dim, int64_t q_pos0, int window,
                                         int64_t kv_start, float scale, int dtype, void* stream) {
  using namespace alpx;
  if (!block_table) return fail(ALPX_EINVAL, "alpx_prefill_causal_paged: null block table");
  if (max_pages <= 0 || num_pages <= 0 || batch_index < 0)
    return fail(ALPX_EINVAL, "alpx_prefill_causal_paged: sizes must be positive");
  if (page_size < 64 || (page_size & (page_size - 1)) != 0)
    return fail(ALPX_EINVAL, "alpx_prefill_causal_paged: page_size must be a power of two >= 64");
  if ((int64_t)kv_tokens > (int64_t)max_pages * page_size)
    return fail(ALPX_ERANGE, "attention cache length exceeds capacity");
  const int64_t row = (int64_t)kv_heads * head_dim;
  return prefill_impl(q, key_pages, value_pages, gate, out, nullptr, 0, q_tokens, kv_tokens,
                      q_heads, kv_heads, head_dim, head_dim, row, row, q_pos0, window, kv_start,
                      scale, dtype, dtype, stream, block_table + (int64_t)batch_index * max_pages,
                      __builtin_ctz((unsigned)page_size), num_pages);
}
