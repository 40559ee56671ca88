// Gated delta-rule (GDN) recurrence: decode step and chunked prefill.
//
// Per value head h (key head kh = h % Hk), state S is Dv x Dk fp32:
//   S <- exp(g) S;  p = S k;  S <- S + beta (v - p) k^T;  o = S q / sqrt(Dk)
// Every row of S evolves independently (row r only needs v[r]), which both
// kernels exploit.
//
// Decode step (gdn_step): 32 lanes own one state row (Dk / 32 columns each);
// one pass reads the row, decays it, forms the prediction with a 5-step
// shuffle reduction, applies the rank-1 correction, forms the output with a
// second reduction and writes the row back: the state crosses HBM exactly
// once in each direction.
//
// Chunked prefill (bf16 inputs, chunks of 64 tokens, Dk 64/128/256):
//  phase A, gdn_prep, one block per (sequence, head, chunk), state-free:
//    Gc = cumsum(g); A = exp(Gc_t - Gc_i) k_t.k_i (i < t);
//    M = exp(Gc_t - Gc_i) q_t.k_i (i <= t); T = (I + diag(beta) A)^-1 by
//    16x16 forward substitution plus block recursion.  K K^T and Q K^T run
//    on bf16 MFMA (exact products of bf16 inputs, fp32 sums).  T and M are
//    stored split into hi and lo bf16 planes (the same bytes as fp32), with
//    Gc in base 2 and beta, so phase B loads its MFMA operands directly.
//  phase B, gdn_apply, one block per (sequence, head, 16 state rows),
//    sequential over chunks with the 16 x Dk state slice resident in LDS:
//    X = diag(beta) (V - diag(exp Gc) K S^T);  Delta = T X;
//    O = (diag(exp Gc) Q S^T + M Delta) / sqrt(Dk);
//    S <- exp(Gc_last) S + (diag(exp(Gc_last - Gc)) Delta)^T K.
//    (Delta = T X is Ub V - W S^T with Ub = T diag(beta) and
//    W = T diag(beta exp Gc) K folded together, so phase B reads T, 16 KiB
//    per head and chunk, instead of Ub and W, 48 KiB at Dk = 128.)
//    fp32 x fp32 products use three bf16 MFMAs (hi.hi + hi.lo + lo.hi),
//    fp32 x bf16 products two, so the state keeps ~fp32 accuracy.
// Tokens past the end of the last chunk are padded as k = q = v = 0,
// beta = 0, g = 0, which leaves every real quantity unchanged.
#include <math.h>

#include "alpx_common.h"
#include "gdn_internal.h"
#include "timing.h"

namespace alpx {
namespace {

constexpr int kC = 64;  // chunk length

struct GdnArgs {
  const void* q;      // [B, T, Hk, Dk]
  const void* k;      // [B, T, Hk, Dk]
  const void* v;      // [B, T, Hv, Dv]
  const float* beta;  // [B, T, Hv]
  const float* g;     // [B, T, Hv]  (log decay, <= 0)
  float* state;       // [B, Hv, Dv, Dk]
  void* out;          // [B, T, Hv, Dv]
  float* ws;          // phase A results per (b, h, chunk)
  int B, T, Hk, Hv, Dk, Dv, nchunks;
  float scale;        // 1 / sqrt(Dk)
};

// ------------------------------------------------------------ decode step

// A 32-lane half-wave updates kStepRows state rows; lane `lane` owns columns
// 4 lane + 128 e + 0..3 (e < NV, NV = ceil(Dk / 128)).  Every load is issued
// unconditionally from a clamped address and zeroed afterwards when out of
// range, so the whole working set (q, k, v, beta, g and the state rows) is in
// flight at once; a predicated load would be compiled as a branch with a
// wait after each load.  VEC: Dk % 4 == 0 and aligned rows, so each group of
// four columns is one vector load.
constexpr int kStepRows = 2;

template <typename T, bool VEC>
__device__ __forceinline__ void load4(const T* p, int c, int n, float (&x)[4]) {
  if constexpr (VEC) {
    typedef typename Vec4<T>::type V4;
    const bool ok = c < n;
    const V4 v = *(const V4*)(p + (ok ? c : 0));
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = ok ? to_f32(v[j]) : 0.f;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = to_f32(p[min(c + j, n - 1)]);
      x[j] = c + j < n ? v : 0.f;
    }
  }
}

template <typename T, typename TO, int NV, bool VEC>
__global__ void __launch_bounds__(256)
gdn_step_kernel(GdnArgs a) {
  const int lane = threadIdx.x & 31;
  const int hw = threadIdx.x >> 5;  // half-wave: 8 per block
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int kh = h % a.Hk;
  const int Dk = a.Dk;
  const int Dv = a.Dv;
  const int64_t bh = (int64_t)b * a.Hv + h;
  const T* kp = (const T*)a.k + ((int64_t)b * a.Hk + kh) * Dk;
  const T* qp = (const T*)a.q + ((int64_t)b * a.Hk + kh) * Dk;
  const int r0 = (blockIdx.x * 8 + hw) * kStepRows;

  float kk[NV][4], qq[NV][4], s[kStepRows][NV][4], vv[kStepRows];
#pragma unroll
  for (int e = 0; e < NV; ++e) {
    load4<T, VEC>(kp, 4 * lane + 128 * e, Dk, kk[e]);
    load4<T, VEC>(qp, 4 * lane + 128 * e, Dk, qq[e]);
  }
#pragma unroll
  for (int j = 0; j < kStepRows; ++j) {
    const int r = min(r0 + j, Dv - 1);
    const float* row = a.state + (bh * Dv + r) * Dk;
#pragma unroll
    for (int e = 0; e < NV; ++e) load4<float, VEC>(row, 4 * lane + 128 * e, Dk, s[j][e]);
    vv[j] = to_f32(((const T*)a.v)[bh * Dv + r]);
  }
  const float decay = __expf(a.g[bh]);
  const float beta = a.beta[bh];

  float p[kStepRows];
#pragma unroll
  for (int j = 0; j < kStepRows; ++j) {
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
    for (int j = 0; j < kStepRows; ++j) p[j] += __shfl_xor(p[j], off, 32);
  float o[kStepRows];
#pragma unroll
  for (int j = 0; j < kStepRows; ++j) {
    const float delta = beta * (vv[j] - p[j]);
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
  for (int j = 0; j < kStepRows; ++j) {
    const int r = r0 + j;
    if (r >= Dv) break;
    float* row = a.state + (bh * Dv + r) * Dk;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int c0 = 4 * lane + 128 * e;
      if constexpr (VEC) {
        if (c0 < Dk) *(f32x4*)(row + c0) = (f32x4){s[j][e][0], s[j][e][1], s[j][e][2], s[j][e][3]};
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c0 + c < Dk) row[c0 + c] = s[j][e][c];
      }
    }
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
    for (int j = 0; j < kStepRows; ++j) o[j] += __shfl_xor(o[j], off, 32);
  if (lane < kStepRows && r0 + lane < Dv) {
    const float oj = lane == 0 ? o[0] : o[1];
    ((TO*)a.out)[bh * Dv + r0 + lane] = from_f32<TO>(oj * a.scale);
  }
}

// ------------------------------------------------------------ helpers

__device__ __forceinline__ void split8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float v = x[j];
    const bf16_t h = static_cast<bf16_t>(v);
    hi[j] = h;
    lo[j] = static_cast<bf16_t>(v - static_cast<float>(h));
  }
}

// A/B operand rows in the order the transposing LDS read delivers them:
// k-slot j of lane group `quad` is row 16 (j / 4) + 4 quad + j % 4.
__device__ __forceinline__ int tr_slot(int quad, int j) { return 16 * (j >> 2) + 4 * quad + (j & 3); }

__host__ __device__ inline int64_t ws_per_chunk() { return 2 * kC + 2 * kC * kC; }

// Per-chunk workspace, in order: Gc * log2(e) [kC] fp32, beta [kC] fp32,
// then the hi and lo bf16 planes of T [kC x kC] and of M [kC x kC].  Each
// plane is stored fragment-major (frag_idx): the 16 bytes a lane feeds to one
// MFMA as its A operand are contiguous and the 64 lanes of a wave follow each
// other, so a wave's operand load is one contiguous 1 KiB access.  M's
// columns are additionally stored in k-slot order (slot_pos), matching the
// order in which phase B holds Delta.
struct ChunkWs {
  float* g;
  float* beta;
  bf16_t *t_hi, *t_lo, *m_hi, *m_lo;
};

__device__ __forceinline__ ChunkWs chunk_ws(float* base) {
  ChunkWs w;
  w.g = base;
  w.beta = base + kC;
  w.t_hi = (bf16_t*)(base + 2 * kC);
  w.t_lo = w.t_hi + kC * kC;
  w.m_hi = w.t_lo + kC * kC;
  w.m_lo = w.m_hi + kC * kC;
  return w;
}

// Column i of a kC-column operand -> its position when the columns are in
// k-slot order (position 32 ks + 8 quad + j holds column 32 ks + tr_slot(quad, j)).
__device__ __forceinline__ int slot_pos(int i) {
  const int ks = i >> 5, r = i & 31;
  return 32 * ks + 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
}

// Element (row t, column p) of a kC-row plane with `cols` columns -> its
// fragment-major index: (row tile t/16, k step p/32, lane
// 16 * ((p/8) % 4) + t % 16, element p % 8).
__device__ __forceinline__ int frag_idx(int t, int p, int cols) {
  return ((((t >> 4) * (cols >> 5) + (p >> 5)) * 4 + ((p >> 3) & 3)) * 16 + (t & 15)) * 8 + (p & 7);
}

__device__ __forceinline__ void store_split(bf16_t* hi, bf16_t* lo, int idx, float v) {
  const bf16_t h = static_cast<bf16_t>(v);
  hi[idx] = h;
  lo[idx] = static_cast<bf16_t>(v - static_cast<float>(h));
}

// ------------------------------------------------------------ phase A

template <int DK>
__global__ void __launch_bounds__(256)
gdn_prep(GdnArgs a) {
  constexpr int kS = DK + 8;   // bf16 LDS row stride
  constexpr int kF = kC + 4;   // fp32 LDS row stride
  constexpr int KS = DK / 32;
  __shared__ __attribute__((aligned(16))) bf16_t Ks[kC * kS];
  __shared__ __attribute__((aligned(16))) bf16_t Qs[kC * kS];
  __shared__ __attribute__((aligned(16))) float Bm[kC * kF];
  __shared__ __attribute__((aligned(16))) float Tm[kC * kF];
  __shared__ __attribute__((aligned(16))) float Xs[4][16 * 17];
  __shared__ float Gs[kC], Bs[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 15, quad = lane >> 4;
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kh = h % a.Hk;
  const int t0 = c * kC;

  // K, Q rows of the chunk (zero past the end)
  constexpr int kUnits = DK / 8;
#pragma unroll
  for (int u = 0; u < kC * kUnits / 256; ++u) {
    const int idx = u * 256 + tid;
    const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
    const int t = t0 + r;
    bf16x8 kv = {}, qv = {};
    if (t < a.T) {
      const int64_t off = (((int64_t)b * a.T + t) * a.Hk + kh) * DK + 8 * cc;
      kv = *(const bf16x8*)((const bf16_t*)a.k + off);
      qv = *(const bf16x8*)((const bf16_t*)a.q + off);
    }
    *(bf16x8*)(Ks + r * kS + 8 * cc) = kv;
    *(bf16x8*)(Qs + r * kS + 8 * cc) = qv;
  }
  if (wave == 0) {
    const int t = t0 + lane;
    const int64_t off = ((int64_t)b * a.T + t) * a.Hv + h;
    float gv = t < a.T ? a.g[off] : 0.f;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_up(gv, d);
      if (lane >= d) gv += y;
    }
    Gs[lane] = gv;
    Bs[lane] = t < a.T ? a.beta[off] : 0.f;
  }
  __syncthreads();

  const ChunkWs out = chunk_ws(a.ws + (((int64_t)b * a.Hv + h) * a.nchunks + c) * ws_per_chunk());
  if (tid < kC) {
    out.g[tid] = Gs[tid] * 1.4426950408889634f;
    out.beta[tid] = Bs[tid];
  }

  // Bm = diag(beta) (exp(Gc_t - Gc_i) k_t.k_i)_{i<t} and
  // M = (exp(Gc_t - Gc_i) q_t.k_i)_{i<=t}: wave w computes rows 16w..16w+15.
  {
    f32x4 kk[4], qk[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) kk[ib] = qk[ib] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 ka = *(const bf16x8*)(Ks + (16 * wave + hl) * kS + 32 * ks + 8 * quad);
      const bf16x8 qa = *(const bf16x8*)(Qs + (16 * wave + hl) * kS + 32 * ks + 8 * quad);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const bf16x8 kb = *(const bf16x8*)(Ks + (16 * ib + hl) * kS + 32 * ks + 8 * quad);
        kk[ib] = mfma16x16x32(ka, kb, kk[ib]);
        qk[ib] = mfma16x16x32(qa, kb, qk[ib]);
      }
    }
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * quad + r;
        const int i = 16 * ib + hl;
        const float dec = i <= t ? expf(Gs[t] - Gs[i]) : 0.f;
        Bm[t * kF + i] = i < t ? Bs[t] * dec * kk[ib][r] : 0.f;
        store_split(out.m_hi, out.m_lo, frag_idx(t, slot_pos(i), kC), dec * qk[ib][r]);
      }
    }
  }
  __syncthreads();

  // Diagonal 16x16 blocks of T = (I + Bm)^-1 by forward substitution:
  // wave w, lane j < 16 owns column j of block w.
  if (lane < 16) {
    const int base = 16 * wave;
    float col[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float acc = t == lane ? 1.f : 0.f;
#pragma unroll
      for (int i = 0; i < t; ++i) acc -= Bm[(base + t) * kF + base + i] * col[i];
      col[t] = acc;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) Tm[(base + t) * kF + base + lane] = col[t];
  }
  // Zero the strictly-upper blocks so the full 64 x 64 T can be read as is.
  for (int idx = tid; idx < kC * kC; idx += 256) {
    const int t = idx / kC, i = idx - (idx / kC) * kC;
    if ((i >> 4) > (t >> 4)) Tm[t * kF + i] = 0.f;
  }
  __syncthreads();

  // Off-diagonal blocks: T_ij = -T_ii sum_{j<=k<i} Bm_ik T_kj, block row by
  // block row; wave j computes block (i, j).
  for (int bi = 1; bi < 4; ++bi) {
    if (wave < bi) {
      const int bj = wave;
      float* X = Xs[wave];
      const int col = hl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * quad + e;
        float acc = 0.f;
        for (int k = bj; k < bi; ++k)
#pragma unroll
          for (int m = 0; m < 16; ++m)
            acc += Bm[(16 * bi + row) * kF + 16 * k + m] * Tm[(16 * k + m) * kF + 16 * bj + col];
        X[row * 17 + col] = acc;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * quad + e;
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < 16; ++m) acc += Tm[(16 * bi + row) * kF + 16 * bi + m] * X[m * 17 + col];
        Tm[(16 * bi + row) * kF + 16 * bj + col] = -acc;
      }
    }
    __syncthreads();
  }

  for (int idx = tid; idx < kC * kC; idx += 256) {
    const int t = idx / kC, i = idx - (idx / kC) * kC;
    store_split(out.t_hi, out.t_lo, frag_idx(t, i, kC), Tm[t * kF + i]);
  }
}

// ------------------------------------------------------------ phase B

// Block -> (16-row state slice, value head, batch).  Consecutive block ids
// run on consecutive XCDs, so the ids are permuted to give the slices of one
// head neighbouring positions on one XCD: they read the same per-chunk
// K/Q rows and T and share that XCD's L2.
__device__ __forceinline__ void apply_block(const GdnArgs& a, int& slice, int& h, int& b) {
  const int slices = a.Dv / 16;
  const int n = slices * a.Hv * a.B;
  int L = blockIdx.x;
  if (n % 8 == 0) L = (L % 8) * (n / 8) + L / 8;
  slice = L % slices;
  const int rest = L / slices;
  h = rest % a.Hv;
  b = rest / a.Hv;
}

// Global inputs of one chunk for one thread, in three groups fetched at
// different points of the chunk loop: the K/Q/V rows, decays and betas that
// are staged in LDS, and the rows of T and of M its lane feeds to the Delta
// and output MFMAs as A operands.
template <int DK>
struct StageIn {
  static constexpr int kUnitsPerThread = kC * (DK / 8) / 256;
  bf16x8 k[kUnitsPerThread], q[kUnitsPerThread];
  bf16x8 v;
  float g, beta;
};
struct TIn {
  bf16x8 t_hi[2], t_lo[2];
};
struct MIn {
  bf16x8 m_hi[2], m_lo[2];
};

template <typename TO, int DK>
__global__ void __launch_bounds__(256)
gdn_apply(GdnArgs a) {
  constexpr int kS = DK + 8;
  constexpr int kSF = DK + 4;
  constexpr int kDF = kC + 4;
  constexpr int KS = DK / 32;
  constexpr int kUnits = DK / 8;
  constexpr int kUPT = StageIn<DK>::kUnitsPerThread;
  __shared__ __attribute__((aligned(16))) bf16_t Ks[kC * kS];
  __shared__ __attribute__((aligned(16))) bf16_t Qs[kC * kS];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[kC * 24];  // [t][16 rows] + pad
  __shared__ __attribute__((aligned(16))) float Ss[16 * kSF];  // state slice [r][d]
  __shared__ __attribute__((aligned(16))) float Xt[16 * kDF];  // X^T [r][t]
  __shared__ __attribute__((aligned(16))) float Dt[16 * kDF];  // Delta^T [r][t]
  __shared__ __attribute__((aligned(16))) float Gs[kC];
  __shared__ __attribute__((aligned(16))) float Bs[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 15, quad = lane >> 4;
  int slice, h, b;
  apply_block(a, slice, h, b);
  const int r0 = slice * 16;
  const int kh = h % a.Hk;
  const int64_t bh = (int64_t)b * a.Hv + h;
  float* sg = a.state + (bh * a.Dv + r0) * DK;
  for (int idx = tid; idx < 16 * DK; idx += 256) {
    const int r = idx / DK, d = idx - (idx / DK) * DK;
    Ss[r * kSF + d] = sg[(int64_t)r * DK + d];
  }
  const int tr_row = 4 * quad + (hl >> 2);
  const int tr_col = 4 * (hl & 3);
  const int tw = 16 * wave;  // first token of this wave's 16-token tile

  // Every load reads a clamped row and is issued unconditionally; rows past
  // the end of the sequence are zeroed when staged, so a fetch puts its whole
  // group in flight without branches.
  auto fetch_stage = [&](StageIn<DK>& in, int c) __attribute__((always_inline)) {
    const int t0 = c * kC;
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int idx = u * 256 + tid;
      const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
      const int64_t off =
          (((int64_t)b * a.T + min(t0 + r, a.T - 1)) * a.Hk + kh) * DK + 8 * cc;
      in.k[u] = *(const bf16x8*)((const bf16_t*)a.k + off);
      in.q[u] = *(const bf16x8*)((const bf16_t*)a.q + off);
    }
    const int t = (tid & 127) >> 1, half = tid & 1;
    in.v = *(const bf16x8*)((const bf16_t*)a.v +
                            (((int64_t)b * a.T + min(t0 + t, a.T - 1)) * a.Hv + h) * a.Dv + r0 +
                            8 * half);
    const ChunkWs w = chunk_ws(a.ws + (bh * a.nchunks + c) * ws_per_chunk());
    in.g = w.g[tid & (kC - 1)];
    in.beta = w.beta[tid & (kC - 1)];
  };
  auto fetch_t = [&](TIn& in, int c) __attribute__((always_inline)) {
    const ChunkWs w = chunk_ws(a.ws + (bh * a.nchunks + c) * ws_per_chunk());
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int f = ((wave * 2 + ks) * 64 + lane) * 8;
      in.t_hi[ks] = *(const bf16x8*)(w.t_hi + f);
      in.t_lo[ks] = *(const bf16x8*)(w.t_lo + f);
    }
  };
  auto fetch_m = [&](MIn& in, int c) __attribute__((always_inline)) {
    const ChunkWs w = chunk_ws(a.ws + (bh * a.nchunks + c) * ws_per_chunk());
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int f = ((wave * 2 + ks) * 64 + lane) * 8;
      in.m_hi[ks] = *(const bf16x8*)(w.m_hi + f);
      in.m_lo[ks] = *(const bf16x8*)(w.m_lo + f);
    }
  };

  // Each group is re-fetched for chunk c + 1 right after its last use in
  // chunk c, into the same registers, so the loads overlap the rest of the
  // chunk without a second register set.  The last chunk re-reads itself
  // (unused) rather than branching, which would make the compiler wait for
  // every outstanding load at the top of the loop.  Issue order st, ti, mi
  // as in the loop (the loads complete in order, so the loop's first wait
  // for st must not also cover ti and mi).
  StageIn<DK> st;
  TIn ti;
  MIn mi;
  fetch_stage(st, 0);
  __builtin_amdgcn_sched_barrier(0);
  fetch_t(ti, 0);
  __builtin_amdgcn_sched_barrier(0);
  fetch_m(mi, 0);
  __builtin_amdgcn_sched_barrier(0);
  for (int c = 0; c < a.nchunks; ++c) {
    const int t0 = c * kC;
    const int cn = min(c + 1, a.nchunks - 1);
    const bf16x8 zero = {};
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int idx = u * 256 + tid;
      const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
      const bool ok = t0 + r < a.T;
      *(bf16x8*)(Ks + r * kS + 8 * cc) = ok ? st.k[u] : zero;
      *(bf16x8*)(Qs + r * kS + 8 * cc) = ok ? st.q[u] : zero;
    }
    if (tid < kC * 2)
      *(bf16x8*)(Vs + (tid >> 1) * 24 + 8 * (tid & 1)) = t0 + (tid >> 1) < a.T ? st.v : zero;
    if (tid < kC) {
      Gs[tid] = st.g;
      Bs[tid] = st.beta;
    }
    __syncthreads();
    fetch_stage(st, cn);

    // S^T operand (B: k = d, n = state row): lane holds S[hl][32 ks + 8 quad + 0..7].
    bf16x8 shi[KS], slo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) split8(Ss + hl * kSF + 32 * ks + 8 * quad, shi[ks], slo[ks]);
    // Q and K rows of this wave's tokens (A operands).
    bf16x8 qa[KS], ka[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qa[ks] = *(const bf16x8*)(Qs + (tw + hl) * kS + 32 * ks + 8 * quad);
      ka[ks] = *(const bf16x8*)(Ks + (tw + hl) * kS + 32 * ks + 8 * quad);
    }

    // (1a) X = diag(beta) (V - diag(exp Gc) K S^T), rows tw.. (lane: t = tw + 4 quad + r, row hl)
    f32x4 kst = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kst = mfma16x16x32(ka[ks], shi[ks], kst);
      kst = mfma16x16x32(ka[ks], slo[ks], kst);
    }
    {
      const bf16x4 v4 = lds_read_tr4(Vs + (tw + tr_row) * 24 + tr_col);
      const f32x4 g4 = *(const f32x4*)(Gs + tw + 4 * quad);
      const f32x4 b4 = *(const f32x4*)(Bs + tw + 4 * quad);
      f32x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = b4[r] * (static_cast<float>(v4[r]) - fast_exp2(g4[r]) * kst[r]);
      *(f32x4*)(Xt + hl * kDF + tw + 4 * quad) = x;
    }
    // (2a) Q S^T for the output rows of this wave
    f32x4 qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qs = mfma16x16x32(qa[ks], shi[ks], qs);
      qs = mfma16x16x32(qa[ks], slo[ks], qs);
    }
    __syncthreads();  // X complete; every wave has read Ss

    // (1b) Delta rows tw.. = T X.  T is lower triangular, so waves 0 and 1
    // (tokens < 32) skip the k step over tokens 32..63.
    f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks == 0 || wave >= 2) {
        bf16x8 xhi, xlo;
        split8(Xt + hl * kDF + 32 * ks + 8 * quad, xhi, xlo);
        dacc = mfma16x16x32(ti.t_hi[ks], xhi, dacc);
        dacc = mfma16x16x32(ti.t_hi[ks], xlo, dacc);
        dacc = mfma16x16x32(ti.t_lo[ks], xhi, dacc);
      }
    }
    *(f32x4*)(Dt + hl * kDF + tw + 4 * quad) = dacc;  // Delta^T[state row][t]
    fetch_t(ti, cn);
    __syncthreads();  // Dt complete; every wave has read Xt

    // Delta in the k-slot order of the transposing reads:
    // dv[ks][j] = Delta[32 ks + tr_slot(quad, j)][hl].
    float dv[2][8];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f32x4 d0 = *(const f32x4*)(Dt + hl * kDF + 32 * ks + 4 * quad);
      const f32x4 d1 = *(const f32x4*)(Dt + hl * kDF + 32 * ks + 16 + 4 * quad);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dv[ks][r] = d0[r];
        dv[ks][4 + r] = d1[r];
      }
    }

    // (2b) O = exp(Gc) Q S^T + M Delta (M's columns are stored in the same
    // k-slot order as dv; M is causal, so waves 0 and 1 skip tokens 32..63).
    f32x4 md = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks == 0 || wave >= 2) {
        bf16x8 dhi, dlo;
        split8(dv[ks], dhi, dlo);
        md = mfma16x16x32(mi.m_hi[ks], dhi, md);
        md = mfma16x16x32(mi.m_hi[ks], dlo, md);
        md = mfma16x16x32(mi.m_lo[ks], dhi, md);
      }
    }
    fetch_m(mi, cn);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tw + 4 * quad + r;
      if (t0 + t < a.T) {
        const float o = (fast_exp2(Gs[t]) * qs[r] + md[r]) * a.scale;
        ((TO*)a.out)[(((int64_t)b * a.T + t0 + t) * a.Hv + h) * a.Dv + r0 + hl] = from_f32<TO>(o);
      }
    }

    // (3) S <- exp(Gc_last) S + (diag(exp(Gc_last - Gc)) Delta)^T K  (Gs is in base 2)
    const float glast = Gs[kC - 1];
    bf16x8 dthi[2], dtlo[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = dv[ks][j] * fast_exp2(glast - Gs[32 * ks + tr_slot(quad, j)]);
      split8(x, dthi[ks], dtlo[ks]);
    }
    const float gl = fast_exp2(glast);
#pragma unroll
    for (int nq = 0; nq < DK / 64; ++nq) {
      const int nb = wave + 4 * nq;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x4 k0 = lds_read_tr4(Ks + (32 * ks + tr_row) * kS + 16 * nb + tr_col);
        const bf16x4 k1 = lds_read_tr4(Ks + (32 * ks + 16 + tr_row) * kS + 16 * nb + tr_col);
        const bf16x8 kb = __builtin_shufflevector(k0, k1, 0, 1, 2, 3, 4, 5, 6, 7);
        acc = mfma16x16x32(dthi[ks], kb, acc);
        acc = mfma16x16x32(dtlo[ks], kb, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float* sp = Ss + (4 * quad + r) * kSF + 16 * nb + hl;
        *sp = gl * *sp + acc[r];
      }
    }
    __syncthreads();
  }
  for (int idx = tid; idx < 16 * DK; idx += 256) {
    const int r = idx / DK, d = idx - (idx / DK) * DK;
    sg[(int64_t)r * DK + d] = Ss[r * kSF + d];
  }
}

template <int DK, typename TO>
int launch_chunk(const GdnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((gdn_prep<DK>), dim3(a.nchunks, a.Hv, a.B), dim3(256), 0, s, a);
  int rc = check_launch("gdn_prep");
  if (rc != ALPX_OK) return rc;
  hipLaunchKernelGGL((gdn_apply<TO, DK>), dim3(a.Dv / 16 * a.Hv * a.B), dim3(256), 0, s, a);
  return check_launch("gdn_apply");
}

template <typename TO>
int launch_chunk_dk(const GdnArgs& a, hipStream_t s) {
  switch (a.Dk) {
    case 64: return launch_chunk<64, TO>(a, s);
    case 128: return launch_chunk<128, TO>(a, s);
    default: return launch_chunk<256, TO>(a, s);
  }
}

template <typename T, typename TO, int NV>
void launch_step_nv(const GdnArgs& a, bool vec, dim3 grid, hipStream_t s) {
  if (vec)
    hipLaunchKernelGGL((gdn_step_kernel<T, TO, NV, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((gdn_step_kernel<T, TO, NV, false>), grid, dim3(256), 0, s, a);
}

template <typename T, typename TO>
void launch_step_to(const GdnArgs& a, bool vec, dim3 grid, hipStream_t s) {
  if (a.Dk > 128)
    launch_step_nv<T, TO, 2>(a, vec, grid, s);
  else
    launch_step_nv<T, TO, 1>(a, vec, grid, s);
}

template <typename T>
int launch_step(const GdnArgs& a, int out_dtype, hipStream_t s) {
  static_assert(kStepRows == 2, "output lane select assumes two rows per half-wave");
  const dim3 grid((a.Dv + 8 * kStepRows - 1) / (8 * kStepRows), a.Hv, a.B);
  const size_t vec_align = 4 * sizeof(T);
  const bool vec = a.Dk % 4 == 0 && (uintptr_t)a.state % 16 == 0 &&
                   (uintptr_t)a.q % vec_align == 0 && (uintptr_t)a.k % vec_align == 0;
  switch (out_dtype) {
    case ALPX_F32: launch_step_to<T, float>(a, vec, grid, s); break;
    case ALPX_F16: launch_step_to<T, f16_t>(a, vec, grid, s); break;
    default: launch_step_to<T, bf16_t>(a, vec, grid, s); break;
  }
  return check_launch("gdn_step");
}

int validate(const void* state, const void* q, const void* k, const void* v, const float* beta,
             const float* g, const void* out, int B, int Hk, int Hv, int Dk, int Dv, int dtype,
             int out_dtype, const char* who) {
  if (!state || !q || !k || !v || !beta || !g || !out)
    return fail(ALPX_EINVAL, "%s: null buffer", who);
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", who);
  if (B <= 0 || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", who);
  if (Hv % Hk != 0) return fail(ALPX_EINVAL, "GDN value heads must be a multiple of key heads");
  if (Dk > 256) return fail(ALPX_EUNSUPPORTED, "%s: key dimension above 256", who);
  return ALPX_OK;
}

}  // namespace
}  // namespace alpx

namespace alpx {

int gdn_step_launch(float* state, const void* q, const void* k, const void* v, const float* beta,
                    const float* log_decay, void* out, int batch, int key_heads,
                    int value_heads, int key_dim, int value_dim, int dtype, int out_dtype,
                    hipStream_t s) {
  int rc = validate(state, q, k, v, beta, log_decay, out, batch, key_heads, value_heads, key_dim,
                    value_dim, dtype, out_dtype, "alpx_gdn_step");
  if (rc != ALPX_OK) return rc;
  GdnArgs a = {};
  a.q = q;
  a.k = k;
  a.v = v;
  a.beta = beta;
  a.g = log_decay;
  a.state = state;
  a.out = out;
  a.B = batch;
  a.T = 1;
  a.Hk = key_heads;
  a.Hv = value_heads;
  a.Dk = key_dim;
  a.Dv = value_dim;
  a.scale = gdn_output_scale(key_dim);
  switch (dtype) {
    case ALPX_F32: return launch_step<float>(a, out_dtype, s);
    case ALPX_F16: return launch_step<f16_t>(a, out_dtype, s);
    default: return launch_step<bf16_t>(a, out_dtype, s);
  }
}

}  // namespace alpx

extern "C" int alpx_gdn_step(float* state, const void* q, const void* k, const void* v,
                             const float* beta, const float* log_decay, void* out, int batch,
                             int key_heads, int value_heads, int key_dim, int value_dim,
                             int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_GDN_STEP, s);
  return gdn_step_launch(state, q, k, v, beta, log_decay, out, batch, key_heads, value_heads,
                         key_dim, value_dim, dtype, out_dtype, s);
}

extern "C" size_t alpx_gdn_chunk_workspace_bytes(int batch, int tokens, int value_heads,
                                                 int key_dim) {
  using namespace alpx;
  if (batch <= 0 || tokens <= 0 || value_heads <= 0 || key_dim <= 0) return 0;
  const int64_t chunks = (tokens + kC - 1) / kC;
  return (size_t)batch * value_heads * chunks * ws_per_chunk() * sizeof(float);
}

extern "C" int alpx_gdn_chunk_prefill(float* state, const void* q, const void* k, const void* v,
                                      const float* beta, const float* log_decay, void* out,
                                      void* workspace, size_t workspace_bytes, int batch,
                                      int tokens, int key_heads, int value_heads, int key_dim,
                                      int value_dim, int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  int rc = validate(state, q, k, v, beta, log_decay, out, batch, key_heads, value_heads, key_dim,
                    value_dim, dtype, out_dtype, "alpx_gdn_chunk_prefill");
  if (rc != ALPX_OK) return rc;
  if (tokens <= 0) return fail(ALPX_EINVAL, "alpx_gdn_chunk_prefill: tokens must be positive");
  hipStream_t s = (hipStream_t)stream;
  GdnArgs a = {};
  a.q = q;
  a.k = k;
  a.v = v;
  a.beta = beta;
  a.g = log_decay;
  a.state = state;
  a.out = out;
  a.B = batch;
  a.T = tokens;
  a.Hk = key_heads;
  a.Hv = value_heads;
  a.Dk = key_dim;
  a.Dv = value_dim;
  a.nchunks = (tokens + kC - 1) / kC;
  a.scale = gdn_output_scale(key_dim);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v;
  const bool chunked = dtype == ALPX_BF16 && (key_dim == 64 || key_dim == 128 || key_dim == 256) &&
                       value_dim % 16 == 0 && (align & 15) == 0 &&
                       getenv("ALPX_GDN_SEQUENTIAL") == nullptr;
  TimedRegion timed(ALPX_T_GDN_CHUNK, s);
  if (chunked) {
    const size_t need = alpx_gdn_chunk_workspace_bytes(batch, tokens, value_heads, key_dim);
    if (!workspace || workspace_bytes < need)
      return fail(ALPX_EINVAL, "alpx_gdn_chunk_prefill: workspace holds %zu bytes, needs %zu",
                  workspace_bytes, need);
    a.ws = (float*)workspace;
    switch (out_dtype) {
      case ALPX_F32: return launch_chunk_dk<float>(a, s);
      case ALPX_F16: return launch_chunk_dk<f16_t>(a, s);
      default: return launch_chunk_dk<bf16_t>(a, s);
    }
  }
  // Token-sequential form (fp32/fp16 inputs, other shapes): the decode step
  // per token, exactly the reference's recurrence order.
  const size_t es = dtype_size(dtype);
  const size_t os = dtype_size(out_dtype);
  for (int t = 0; t < tokens; ++t) {
    GdnArgs st = a;
    st.T = 1;
    // per-token views of [B, T, H, D] tensors: batch stride differs, so walk
    // the batch inside by launching per (token) with B = 1 when batch > 1
    for (int bb = 0; bb < batch; ++bb) {
      st.B = 1;
      st.q = (const char*)q + (((size_t)bb * tokens + t) * key_heads) * key_dim * es;
      st.k = (const char*)k + (((size_t)bb * tokens + t) * key_heads) * key_dim * es;
      st.v = (const char*)v + (((size_t)bb * tokens + t) * value_heads) * value_dim * es;
      st.beta = beta + ((size_t)bb * tokens + t) * value_heads;
      st.g = log_decay + ((size_t)bb * tokens + t) * value_heads;
      st.state = state + (size_t)bb * value_heads * value_dim * key_dim;
      st.out = (char*)out + (((size_t)bb * tokens + t) * value_heads) * value_dim * os;
      switch (dtype) {
        case ALPX_F32: rc = launch_step<float>(st, out_dtype, s); break;
        case ALPX_F16: rc = launch_step<f16_t>(st, out_dtype, s); break;
        default: rc = launch_step<bf16_t>(st, out_dtype, s); break;
      }
      if (rc != ALPX_OK) return rc;
    }
  }
  return ALPX_OK;
}
