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
// Chunked prefill (bf16 inputs, chunks of 64 tokens, Dk 64/128/256).  With
// gamma_t = exp(Gc_t), Gc = cumsum(g) within the chunk, S the state entering
// the chunk, scale = 1 / sqrt(Dk), A = (gamma_t / gamma_i k_t.k_i)_{i<t},
// M = (gamma_t / gamma_i q_t.k_i)_{i<=t} and T = (I + diag(beta) A)^-1, the
// delta rule over the chunk is
//    X^T = V - diag(gamma) K S^T                       (L x Dv)
//    O   = scale diag(gamma) Q S^T + P X^T,            P = scale M T diag(beta)
//    S^T <- gamma_L S^T + K^T (W X^T),                 W = diag(gamma_L / gamma) T diag(beta)
//  phase A, gdn_prep, one block per (sequence, chunk, pair of value heads
//    sharing a key head), state-free: Gc, K K^T and Q K^T on bf16 MFMA
//    (exact products of bf16 inputs, fp32 sums), T by 16x16 forward
//    substitution plus a block recursion, then W and P; both are causal, and
//    their live 16 x 32 tiles are stored split into hi and lo bf16 planes
//    (the same bytes as fp32) as ready-made MFMA operands.
//  phase B, gdn_apply, one block per (sequence, head, 16 state rows),
//    sequential over chunks in three steps with a block barrier after each:
//    K S^T and X^T, then Y^T = W X^T, then the state update; Q S^T and
//    P X^T for the output ride alongside.  The state slice stays in fp32
//    registers of the wave that updates it and is published to the other
//    waves as hi / lo planes in LDS.
//    fp32 x fp32 products use three bf16 MFMAs (hi.hi + hi.lo + lo.hi),
//    fp32 x bf16 products two, so the state keeps ~fp32 accuracy.
// Tokens past the end of the last chunk are padded as k = q = v = 0,
// beta = 0, g = 0, which leaves every real quantity unchanged.
#include <math.h>

#include <type_traits>

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

// Operand planes.  An fp32 value x enters the bf16 MFMAs as N bf16 planes
// p0 = bf16(x), p1 = bf16(x - p0), p2 = bf16(x - p0 - p1): two planes hold
// x to about 2^-17 relative, three hold any fp32 value exactly (8 + 8 + 8
// significant bits).  Plane n is about 2^-8n of x, so a product of planed
// operands keeps the terms a_i b_j with i + j <= its order.
template <int N>
__device__ __forceinline__ void split_planes8(const float* x, bf16x8 (&p)[N]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float r = x[j];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const bf16_t h = static_cast<bf16_t>(r);
      p[n][j] = h;
      if (n + 1 < N) r = r - static_cast<float>(h);
    }
  }
}

template <int N>
__device__ __forceinline__ void split_planes4(f32x4 x, bf16x4 (&p)[N]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float r = x[j];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const bf16_t h = static_cast<bf16_t>(r);
      p[n][j] = h;
      if (n + 1 < N) r = r - static_cast<float>(h);
    }
  }
}

// acc + sum of a_i b_j over i + j <= ORD, accumulated in (i, j) order.
template <int NA, int NB, int ORD>
__device__ __forceinline__ f32x4 mfma_planes(const bf16x8 (&a)[NA], const bf16x8 (&b)[NB],
                                             f32x4 acc) {
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (i + j <= ORD) acc = mfma16x16x32(a[i], b[j], acc);
  return acc;
}

// Planes per operand by input type.  bf16 inputs (q, k, v) are one exact
// plane and the fp32 quantities derived from them (state, P, W, X, Y) two,
// products keeping the terms to order 1.  fp32 inputs take three planes
// everywhere, products to order 2: in a CPU model of the kernels on the
// Qwen3.5 recurrent-layer chain (small GDN outputs, formed with heavy
// cancellation, then RMS-normalised) two planes left 1.3e-4 after the gated
// norm against the fp64 chain, three planes 3e-5 (plain fp32 token by
// token: 5e-6).
template <typename TI>
struct Planes {
  static constexpr int in = 1, der = 2;
};
template <>
struct Planes<float> {
  static constexpr int in = 3, der = 3;
};

// Rows in the order the transposing LDS read delivers them: k-slot j of
// lane group `quad` is row 16 (j / 4) + 4 quad + j % 4.
__device__ __forceinline__ int tr_slot(int quad, int j) { return 16 * (j >> 2) + 4 * quad + (j & 3); }

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-chunk workspace (fp32 words), in order: Gc * log2(e) [kC], then the NS
// bf16 planes of P and the NS planes of W [kC x kC each].  Both are causal
// (row t is zero past column t), so of the eight 16 x 32 A-operand tiles (m
// tile mt, k step ks) only the six with 32 ks <= 16 mt + 15 are stored, in
// the order (0,0) (1,0) (2,0) (2,1) (3,0) (3,1).  Each tile is stored
// fragment-major: lane 16 quad + i holds row 16 mt + i, columns
// 32 ks + 8 quad + 0..7, as 16 contiguous bytes, and the 64 lanes follow
// each other, so a wave's operand load is one contiguous 1 KiB access.
constexpr int kTiles = 6;
constexpr int kTileElems = 64 * 8;
template <int NS>
__host__ __device__ constexpr int64_t ws_per_chunk() {
  return kC + 2 * NS * kTiles * kTileElems / 2;
}
__device__ __forceinline__ int tile_slot(int mt, int ks) { return mt < 2 ? mt : 2 * mt - 2 + ks; }
// Whether A-operand tile (mt, ks) of a causal kC x kC matrix is stored.
__device__ __forceinline__ bool tile_live(int mt, int ks) { return ks == 0 || mt >= 2; }

template <int NS>
struct ChunkWs {
  float* g;
  bf16_t* p[NS];
  bf16_t* w[NS];
};

template <int NS>
__device__ __forceinline__ ChunkWs<NS> chunk_ws(float* base) {
  ChunkWs<NS> c;
  c.g = base;
  bf16_t* const planes = (bf16_t*)(base + kC);
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    c.p[n] = planes + n * kTiles * kTileElems;
    c.w[n] = planes + (NS + n) * kTiles * kTileElems;
  }
  return c;
}

// Element offset of `lane`'s 16 bytes in stored tile (mt, ks).
__device__ __forceinline__ int tile_off(int mt, int ks, int lane) {
  return (tile_slot(mt, ks) * 64 + lane) * 8;
}

// ------------------------------------------------------------ phase A

// NG value heads of one key head per block (the value heads h with
// h % Hk = kh share K and Q): four waves per value head, one load of the
// chunk's K and Q rows for all of them.  bf16 inputs: the K and Q rows are
// staged in LDS as they are.  fp32 inputs: the K rows are staged as their
// three planes and each wave reads its own Q rows from global memory as A
// operands.
template <typename TI, int DK, int NG>
__global__ void __launch_bounds__(256 * NG)
gdn_prep(GdnArgs a) {
  constexpr bool F32IN = std::is_same<TI, float>::value;
  constexpr int NI = Planes<TI>::in, NS = Planes<TI>::der, ORD = NS - 1;
  constexpr int kS = DK + 8;   // bf16 LDS row stride
  constexpr int kF = kC + 4;   // fp32 LDS row stride
  constexpr int KS = DK / 32;
  constexpr int kUnits = DK / 8;
  constexpr int kUPT = kC * kUnits / (256 * NG);
  static_assert(kUPT * 256 * NG == kC * kUnits, "K / Q rows must split evenly over the block");
  __shared__ __attribute__((aligned(16))) bf16_t Ks[NI][kC * kS];             // K rows
  __shared__ __attribute__((aligned(16))) bf16_t Qs[F32IN ? 8 : kC * kS];     // Q rows
  // Per value head: diag(beta) A, then (per wave, its own 16 rows) M, P and
  // a staging tile; T; the block-recursion exchange; Gc; beta.
  __shared__ __attribute__((aligned(16))) float Bm_[NG][kC * kF];
  __shared__ __attribute__((aligned(16))) float Tm_[NG][kC * kF];
  __shared__ __attribute__((aligned(16))) float Xs_[NG][4][16 * 17];
  __shared__ __attribute__((aligned(16))) float Gs_[NG][kC];
  __shared__ __attribute__((aligned(16))) float Bs_[NG][kC];

  const int gtid = threadIdx.x;
  const int grp = __builtin_amdgcn_readfirstlane(gtid >> 8);  // value head of the block
  const int tid = gtid & 255, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 15, quad = lane >> 4;
  const int c = blockIdx.x, b = blockIdx.z;
  const int kh = (int)blockIdx.y % a.Hk;
  const int h = kh + a.Hk * (NG * ((int)blockIdx.y / a.Hk) + grp);
  const int t0 = c * kC;
  float* const Bm = Bm_[grp];
  float* const Tm = Tm_[grp];
  float (*const Xs)[16 * 17] = Xs_[grp];
  float* const Gs = Gs_[grp];
  float* const Bs = Bs_[grp];

  // K, Q rows of the chunk, g and beta: every load reads a clamped row and
  // is issued before any is used, so they are all in flight together; rows
  // past the end are zeroed when stored.
  bf16x8 kv[F32IN ? 1 : kUPT], qv[F32IN ? 1 : kUPT];
  f32x4 kf[F32IN ? kUPT : 1][2], qf[F32IN ? KS : 1][2];
  if constexpr (F32IN) {
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int idx = u * 256 * NG + gtid;
      const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
      const float* p =
          (const float*)a.k + (((int64_t)b * a.T + min(t0 + r, a.T - 1)) * a.Hk + kh) * DK + 8 * cc;
      kf[u][0] = *(const f32x4*)p;
      kf[u][1] = *(const f32x4*)(p + 4);
    }
    // this wave's Q rows in A-operand order: row 16 wave + hl, columns
    // 32 ks + 8 quad + 0..7
    const float* p = (const float*)a.q +
                     (((int64_t)b * a.T + min(t0 + 16 * wave + hl, a.T - 1)) * a.Hk + kh) * DK +
                     8 * quad;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks][0] = *(const f32x4*)(p + 32 * ks);
      qf[ks][1] = *(const f32x4*)(p + 32 * ks + 4);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int idx = u * 256 * NG + gtid;
      const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
      const int64_t off = (((int64_t)b * a.T + min(t0 + r, a.T - 1)) * a.Hk + kh) * DK + 8 * cc;
      kv[u] = *(const bf16x8*)((const bf16_t*)a.k + off);
      qv[u] = *(const bf16x8*)((const bf16_t*)a.q + off);
    }
  }
  const bool tok_ok = t0 + lane < a.T;
  const int64_t goff = ((int64_t)b * a.T + min(t0 + lane, a.T - 1)) * a.Hv + h;
  const float graw = a.g[goff], braw = a.beta[goff];
  // The strictly-upper blocks of T are zero (the full 64 x 64 T is read as
  // is below); they are cleared here, where the waves wait for their loads.
#pragma unroll
  for (int j = 0; j < kC * kC / 256; ++j) {
    const int idx = tid + 256 * j;
    const int t = idx / kC, i = idx - (idx / kC) * kC;
    if ((i >> 4) > (t >> 4)) Tm[t * kF + i] = 0.f;
  }
  const bf16x8 zero8 = {};
#pragma unroll
  for (int u = 0; u < kUPT; ++u) {
    const int idx = u * 256 * NG + gtid;
    const int r = idx / kUnits, cc = idx - (idx / kUnits) * kUnits;
    const bool ok = t0 + r < a.T;
    if constexpr (F32IN) {
      const float x[8] = {kf[u][0][0], kf[u][0][1], kf[u][0][2], kf[u][0][3],
                          kf[u][1][0], kf[u][1][1], kf[u][1][2], kf[u][1][3]};
      bf16x8 pl[NI];
      split_planes8<NI>(x, pl);
#pragma unroll
      for (int n = 0; n < NI; ++n) *(bf16x8*)(Ks[n] + r * kS + 8 * cc) = ok ? pl[n] : zero8;
    } else {
      *(bf16x8*)(Ks[0] + r * kS + 8 * cc) = ok ? kv[u] : zero8;
      *(bf16x8*)(Qs + r * kS + 8 * cc) = ok ? qv[u] : zero8;
    }
  }
  if (wave == 0) {
    float gv = tok_ok ? graw : 0.f;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_up(gv, d);
      if (lane >= d) gv += y;
    }
    Gs[lane] = gv;
    Bs[lane] = tok_ok ? braw : 0.f;
  }
  __syncthreads();

  const ChunkWs<NS> out =
      chunk_ws<NS>(a.ws + (((int64_t)b * a.Hv + h) * a.nchunks + c) * ws_per_chunk<NS>());
  if (tid < kC) out.g[tid] = Gs[tid] * kLog2e;

  // Bm = diag(beta) (exp(Gc_t - Gc_i) k_t.k_i)_{i<t} and
  // M = (exp(Gc_t - Gc_i) q_t.k_i)_{i<=t}: wave w computes rows 16w..16w+15.
  // M stays in registers until T is done and Bm's space is free.
  f32x4 mq[4];
  {
    f32x4 kk[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) kk[ib] = mq[ib] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const bool qok = t0 + 16 * wave + hl < a.T;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 ka[NI], qa[NI];
#pragma unroll
      for (int n = 0; n < NI; ++n)
        ka[n] = *(const bf16x8*)(Ks[n] + (16 * wave + hl) * kS + 32 * ks + 8 * quad);
      if constexpr (F32IN) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = qok ? qf[ks][0][j] : 0.f;
          x[4 + j] = qok ? qf[ks][1][j] : 0.f;
        }
        split_planes8<NI>(x, qa);
      } else {
        qa[0] = *(const bf16x8*)(Qs + (16 * wave + hl) * kS + 32 * ks + 8 * quad);
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        bf16x8 kb[NI];
#pragma unroll
        for (int n = 0; n < NI; ++n)
          kb[n] = *(const bf16x8*)(Ks[n] + (16 * ib + hl) * kS + 32 * ks + 8 * quad);
        kk[ib] = mfma_planes<NI, NI, ORD>(ka, kb, kk[ib]);
        mq[ib] = mfma_planes<NI, NI, ORD>(qa, kb, mq[ib]);
      }
    }
    // Decays and masks as selects over values already in registers (Gc is
    // non-increasing, so Gc_t - Gc_i <= 0 wherever i <= t).
    const f32x4 gt = *(const f32x4*)(Gs + 16 * wave + 4 * quad);
    const f32x4 bt = *(const f32x4*)(Bs + 16 * wave + 4 * quad);
    float gi[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) gi[ib] = Gs[16 * ib + hl];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * quad + r;
        const int i = 16 * ib + hl;
        const float e = fast_exp2(fminf(gt[r] - gi[ib], 0.f) * kLog2e);
        const float dec = i <= t ? e : 0.f;
        const float bm = bt[r] * dec * kk[ib][r];
        Bm[t * kF + i] = i < t ? bm : 0.f;
        mq[ib][r] *= dec;
      }
    }
  }
  __syncthreads();

  // Diagonal 16x16 blocks of T = (I + Bm)^-1 by forward substitution:
  // wave w, lane j < 16 owns column j of block w.  Column-oriented: once
  // entry i of the column is final it is subtracted from every later entry,
  // so each step's updates are independent of each other and the dependent
  // chain is 16 steps long instead of 120.
  if (lane < 16) {
    const int base = 16 * wave;
    float col[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) col[t] = t == lane ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < 15; ++i) {
#pragma unroll
      for (int t = i + 1; t < 16; ++t) col[t] -= Bm[(base + t) * kF + base + i] * col[i];
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) Tm[(base + t) * kF + base + lane] = col[t];
  }
  __syncthreads();

  // Off-diagonal blocks: T_ij = -T_ii sum_{k<i} Bm_ik T_kj (T_kj = 0 for
  // k < j), block row by block row; wave j computes block (i, j) on fp32
  // MFMAs (16x16x4: lane (hl, quad) feeds A[hl][quad] and B[quad][hl] of each
  // 4-wide k step and receives D[4 quad + e][hl]).
#pragma unroll
  for (int bi = 1; bi < 4; ++bi) {
    if (wave < bi) {
      const int bj = wave;
      float* X = Xs[wave];
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < bi; ++k) {
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const float av = Bm[(16 * bi + hl) * kF + 16 * k + 4 * s4 + quad];
          const float bv = Tm[(16 * k + 4 * s4 + quad) * kF + 16 * bj + hl];
          x = mfma16x16x4(av, bv, x);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) X[(4 * quad + e) * 17 + hl] = x[e];
      wave_sync_lds();
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float av = Tm[(16 * bi + hl) * kF + 16 * bi + 4 * s4 + quad];
        const float bv = X[(4 * s4 + quad) * 17 + hl];
        y = mfma16x16x4(av, bv, y);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[(16 * bi + 4 * quad + e) * kF + 16 * bj + hl] = -y[e];
    }
    __syncthreads();
  }

  // W = diag(exp(Gc_last - Gc)) T diag(beta), rows 16w..16w+15, straight
  // from T as soon as T is complete, so its stores drain while P is formed:
  // lane (hl, quad) forms row 16w + hl, columns 32 ks + 8 quad + 0..7.
  {
    const float rowf = fast_exp2((Gs[kC - 1] - Gs[16 * wave + hl]) * kLog2e);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (tile_live(wave, ks)) {
        const float* tr = Tm + (16 * wave + hl) * kF + 32 * ks + 8 * quad;
        const f32x4 x0 = *(const f32x4*)tr, x1 = *(const f32x4*)(tr + 4);
        const f32x4 b0 = *(const f32x4*)(Bs + 32 * ks + 8 * quad);
        const f32x4 b1 = *(const f32x4*)(Bs + 32 * ks + 8 * quad + 4);
        float x[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = rowf * x0[j] * b0[j];
          x[4 + j] = rowf * x1[j] * b1[j];
        }
        bf16x8 pl[NS];
        split_planes8<NS>(x, pl);
        const int o = tile_off(wave, ks, lane);
#pragma unroll
        for (int n = 0; n < NS; ++n)
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4, pl[n]), (u32x4*)(out.w[n] + o));
      }
    }
  }

  // From here each wave works on its own 16 rows of Bm's space (M, then P,
  // then a staging tile), so only wave-level ordering is needed.
  float* const Mw = Bm + 16 * wave * kF;
#pragma unroll
  for (int ib = 0; ib < 4; ++ib)
#pragma unroll
    for (int r = 0; r < 4; ++r) Mw[(4 * quad + r) * kF + 16 * ib + hl] = mq[ib][r];
  wave_sync_lds();

  // T's columns in the transposing read's token order (k-slot j of lane
  // group quad is token 32 ks + tr_slot(quad, j)), shared by P and Qm^T.
  float tc[4][2][8];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) tc[nt][ks][j] = Tm[(32 * ks + tr_slot(quad, j)) * kF + 16 * nt + hl];

  // P = scale M T diag(beta) for rows 16w..16w+15.  M (i <= t) and T
  // (lower triangular) are causal: waves 0 and 1 skip tokens 32..63 and
  // token tiles nt >= 2 get nothing from tokens < 32.
  {
    f32x4 pacc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) pacc[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f32x4 m0 = *(const f32x4*)(Mw + hl * kF + 32 * ks + 4 * quad);
      const f32x4 m1 = *(const f32x4*)(Mw + hl * kF + 32 * ks + 16 + 4 * quad);
      const float mrow[8] = {m0[0], m0[1], m0[2], m0[3], m1[0], m1[1], m1[2], m1[3]};
      bf16x8 mp[NS];
      split_planes8<NS>(mrow, mp);
      if (ks == 0 || wave >= 2) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          if (ks == 1 || nt < 2) {
            bf16x8 tp[NS];
            split_planes8<NS>(tc[nt][ks], tp);
            pacc[nt] = mfma_planes<NS, NS, ORD>(mp, tp, pacc[nt]);
          }
        }
      }
    }
    wave_sync_lds();  // M read before P overwrites it
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const float f = a.scale * Bs[16 * nt + hl];
#pragma unroll
      for (int e = 0; e < 4; ++e) Mw[(4 * quad + e) * kF + 16 * nt + hl] = f * pacc[nt][e];
    }
    wave_sync_lds();
    // P as planed fragments: the wave's live tiles, one unit per lane each.
    // Workspace stores are nontemporal: every block writes its fragments at
    // about the same late point, and streaming them out rather than leaving
    // them dirty in L2 shortens the drain at the end of the kernel.
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (tile_live(wave, ks)) {
        const f32x4 x0 = *(const f32x4*)(Mw + hl * kF + 32 * ks + 8 * quad);
        const f32x4 x1 = *(const f32x4*)(Mw + hl * kF + 32 * ks + 8 * quad + 4);
        const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        bf16x8 pl[NS];
        split_planes8<NS>(x, pl);
        const int o = tile_off(wave, ks, lane);
#pragma unroll
        for (int n = 0; n < NS; ++n)
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4, pl[n]), (u32x4*)(out.p[n] + o));
      }
    }
  }
}

// ------------------------------------------------------------ phase B

// Block -> (16-row state slice, value head, batch).  Consecutive block ids
// run on consecutive XCDs, so the ids are permuted to give the slices of one
// head neighbouring positions on one XCD: they read the same per-chunk
// K/Q rows, P and Qm^T and share that XCD's L2.
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

// Global inputs of one chunk, in three groups: what the K S^T / Q S^T step
// reads as A operands (K and Q rows of the lane's token), the P and W
// fragments of the wave's token rows, and the V rows and decays that waves
// 0..2 stage in LDS for everyone.  fp32 inputs keep the loaded fp32 values
// until their use, where they are split into planes.
template <typename TI, int DK>
struct KqIn {
  bf16x8 k[DK / 32], q[DK / 32];
};
template <int DK>
struct KqIn<float, DK> {
  f32x4 k[DK / 16], q[DK / 16];  // 32 ks + 8 quad + 0..3 in [2 ks], + 4..7 in [2 ks + 1]
};
template <int NS>
struct PwIn {
  bf16x8 p[2][NS], w[2][NS];  // [k step][plane]
};
template <typename TI>
struct VgIn {
  bf16x8 v;  // waves 0, 1: V[token tid / 2][16-column slice half tid % 2]
  f32x4 g;   // wave 2, lanes 0..15: Gc * log2(e) of tokens 4 lane .. 4 lane + 3
};
// fp32 V: one pair of registers holds either a wave's V halves (waves 0,
// 1) or the decays (wave 2, in v[0]), so no field is chosen by a branch
// (a branch-selected field is stored through a selected pointer, in
// scratch memory).
template <>
struct VgIn<float> {
  f32x4 v[2];
};
__device__ __forceinline__ f32x4& vg_decay(VgIn<bf16_t>& in) { return in.g; }
__device__ __forceinline__ f32x4& vg_decay(VgIn<float>& in) { return in.v[0]; }
__device__ __forceinline__ const f32x4& vg_decay(const VgIn<bf16_t>& in) { return in.g; }
__device__ __forceinline__ const f32x4& vg_decay(const VgIn<float>& in) { return in.v[0]; }

// The planes of fp32 operand elements 8 j .. 8 j + 7 held as two f32x4.
template <int N>
__device__ __forceinline__ void split_pair(const f32x4& x0, const f32x4& x1, bf16x8 (&p)[N]) {
  const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
  split_planes8<N>(x, p);
}

template <typename TI, typename TO, int DK>
__global__ void __launch_bounds__(256)
gdn_apply(GdnArgs a) {
  constexpr bool F32IN = std::is_same<TI, float>::value;
  constexpr int NI = Planes<TI>::in, NS = Planes<TI>::der, ORD = NS - 1;
  constexpr int KS = DK / 32;
  constexpr int MT = DK / 64;     // state d tiles per wave
  // chunks of operands in flight (fp32 operands take twice the registers)
  constexpr int PF = !F32IN && DK <= 128 ? 2 : 1;
  constexpr int kSB = DK + 8;     // bf16 row stride of the state planes
  // bf16 row stride of the K tile: 8 dwords past a multiple of 64 banks, so
  // the transposing reads of step (3) (four rows x four column groups per
  // 16 lanes) hit distinct banks
  constexpr int kSK = DK + 16;
  constexpr int kXB = kC + 8;     // bf16 row stride of the X^T and Y^T planes
  constexpr int kVB = 24;         // bf16 row stride of the V tile
  constexpr int kVF = 20;         // fp32 row stride of the V tile (fp32 inputs)
  constexpr int kOB = 16 + 16 / (int)sizeof(TO);  // TO row stride of the output tile
  __shared__ __attribute__((aligned(16))) bf16_t Sp[NS][16 * kSB];  // S [r][d]
  __shared__ __attribute__((aligned(16))) bf16_t Kt[NI][kC * kSK];  // K [t][d]
  __shared__ __attribute__((aligned(16))) bf16_t Xp[NS][16 * kXB];  // X^T [r][t]
  __shared__ __attribute__((aligned(16))) bf16_t Yp[NS][16 * kXB];  // Y^T [r][t]
  __shared__ __attribute__((aligned(16))) bf16_t Vs[F32IN ? 8 : kC * kVB];  // V [t][r]
  __shared__ __attribute__((aligned(16))) float Vf[F32IN ? kC * kVF : 4];   // V [t][r], fp32
  __shared__ __attribute__((aligned(16))) TO Os[kC * kOB];      // O [t][r]
  __shared__ __attribute__((aligned(16))) float Gs[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 15, quad = lane >> 4;
  int slice, h, b;
  apply_block(a, slice, h, b);
  const int r0 = slice * 16;
  const int kh = h % a.Hk;
  const int64_t bh = (int64_t)b * a.Hv + h;
  const int tw = 16 * wave;  // first token of this wave's 16-token tile
  const int tr_row = 4 * quad + (hl >> 2);
  const int tr_col = 4 * (hl & 3);

  // The wave keeps d tiles mt = wave + 4 i of S^T in fp32 (lane: state row
  // r0 + hl, d = 16 mt + 4 quad + e) and publishes them to every wave as
  // NS bf16 planes.
  float* const srow = a.state + (bh * a.Dv + r0 + hl) * DK;
  f32x4 sown[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) sown[i] = *(const f32x4*)(srow + 16 * (wave + 4 * i) + 4 * quad);
  auto put_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      bf16x4 pl[NS];
      split_planes4<NS>(sown[i], pl);
#pragma unroll
      for (int n = 0; n < NS; ++n)
        *(bf16x4*)(Sp[n] + hl * kSB + 16 * (wave + 4 * i) + 4 * quad) = pl[n];
    }
  };

  // Every load reads a clamped row and is issued unconditionally (per
  // wave); the rows of tokens past the end are zeroed where X^T is formed
  // and never stored, and their rows of W are zero.
  // Per-block bases; the per-token offsets are 24-bit products (a token
  // index below 2^24 times a row of fewer than 2^24 elements, whose product
  // the host also keeps below 2^32), so address arithmetic stays off the
  // quarter-rate 32 / 64-bit multiplies.
  const int krow = a.Hk * DK, vrow = a.Hv * a.Dv;
  const TI* const kbase = (const TI*)a.k + (int64_t)b * a.T * krow + kh * DK + 8 * quad;
  const TI* const qbase = (const TI*)a.q + (int64_t)b * a.T * krow + kh * DK + 8 * quad;
  const TI* const vbase = (const TI*)a.v + (int64_t)b * a.T * vrow + h * a.Dv + r0;
  TO* const obase = (TO*)a.out + (int64_t)b * a.T * vrow + h * a.Dv + r0;
  float* const wsbase = a.ws + bh * a.nchunks * ws_per_chunk<NS>();
  auto fetch_kq = [&](KqIn<TI, DK>& in, int c) __attribute__((always_inline)) {
    const unsigned off = __umul24((unsigned)min(c * kC + tw + hl, a.T - 1), (unsigned)krow);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (F32IN) {
        in.k[2 * ks] = *(const f32x4*)(kbase + off + 32 * ks);
        in.k[2 * ks + 1] = *(const f32x4*)(kbase + off + 32 * ks + 4);
        in.q[2 * ks] = *(const f32x4*)(qbase + off + 32 * ks);
        in.q[2 * ks + 1] = *(const f32x4*)(qbase + off + 32 * ks + 4);
      } else {
        in.k[ks] = *(const bf16x8*)(kbase + off + 32 * ks);
        in.q[ks] = *(const bf16x8*)(qbase + off + 32 * ks);
      }
    }
  };
  auto fetch_pw = [&](PwIn<NS>& in, int c) __attribute__((always_inline)) {
    const ChunkWs<NS> w = chunk_ws<NS>(wsbase + c * (int)ws_per_chunk<NS>());
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (tile_live(wave, ks)) {
        const int o = tile_off(wave, ks, lane);
#pragma unroll
        for (int n = 0; n < NS; ++n) in.p[ks][n] = *(const bf16x8*)(w.p[n] + o);
#pragma unroll
        for (int n = 0; n < NS; ++n) in.w[ks][n] = *(const bf16x8*)(w.w[n] + o);
      }
    }
  };
  auto fetch_vg = [&](VgIn<TI>& in, int c) __attribute__((always_inline)) {
    if (wave < 2) {
      const unsigned t = (unsigned)min(c * kC + (tid >> 1), a.T - 1);
      const TI* p = vbase + __umul24(t, (unsigned)vrow) + 8 * (tid & 1);
      if constexpr (F32IN) {
        in.v[0] = *(const f32x4*)p;
        in.v[1] = *(const f32x4*)(p + 4);
      } else {
        in.v = *(const bf16x8*)p;
      }
    } else if (wave == 2 && lane < 16) {
      vg_decay(in) = *(const f32x4*)(wsbase + c * (int)ws_per_chunk<NS>() + 4 * lane);
    }
  };
  auto stage_vg = [&](const VgIn<TI>& in, int c) __attribute__((always_inline)) {
    if (wave < 2) {
      const bool ok = c * kC + (tid >> 1) < a.T;
      if constexpr (F32IN) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        float* p = Vf + (tid >> 1) * kVF + 8 * (tid & 1);
        *(f32x4*)p = ok ? in.v[0] : zero;
        *(f32x4*)(p + 4) = ok ? in.v[1] : zero;
      } else {
        const bf16x8 zero = {};
        *(bf16x8*)(Vs + (tid >> 1) * kVB + 8 * (tid & 1)) = ok ? in.v : zero;
      }
    } else if (wave == 2 && lane < 16) {
      *(f32x4*)(Gs + 4 * lane) = vg_decay(in);
    }
  };
  // Output tile of chunk c (staged in LDS) -> global, 16 bytes per lane.
  auto flush_out = [&](int c) __attribute__((always_inline)) {
    constexpr int kPer = 16 / (int)sizeof(TO);  // elements per 16 bytes
    constexpr int kUnitsRow = 16 / kPer;
#pragma unroll
    for (int u0 = 0; u0 < kC * kUnitsRow; u0 += 256) {
      const int u = u0 + tid;
      const int t = u / kUnitsRow, part = u % kUnitsRow;
      if (u < kC * kUnitsRow && c * kC + t < a.T)
        *(u32x4*)(obase + __umul24((unsigned)(c * kC + t), (unsigned)vrow) + kPer * part) =
            *(const u32x4*)(Os + t * kOB + kPer * part);
    }
  };

  // Operands run PF chunks ahead: each set is re-fetched right after its
  // last use, into the same registers, so the loads overlap the following
  // chunks.  Chunks past the end re-read the last chunk (unused) rather
  // than branching.
  KqIn<TI, DK> kq[PF];
  PwIn<NS> pw[PF];
  VgIn<TI> vg[PF];
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    const int c = min(p, a.nchunks - 1);
    fetch_vg(vg[p], c);
    fetch_kq(kq[p], c);
    fetch_pw(pw[p], c);
  }
  put_state();
  stage_vg(vg[0], 0);
  fetch_vg(vg[0], min(PF, a.nchunks - 1));
  __syncthreads();

  auto chunk = [&](int c, KqIn<TI, DK>& kqc, PwIn<NS>& pwc, VgIn<TI>& vgn)
                   __attribute__((always_inline)) {
    const int t0 = c * kC;
    const int cf = min(c + PF, a.nchunks - 1);

    // (1) K S^T and Q S^T for this wave's tokens (B = S^T: lane holds
    // S[r0 + hl][32 ks + 8 quad + 0..7]); X^T = V - diag(exp Gc) K S^T.  The
    // wave's K rows also go to the K tile for step (3).
    bf16x8 sp[KS][NS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int n = 0; n < NS; ++n) sp[ks][n] = *(const bf16x8*)(Sp[n] + hl * kSB + 32 * ks + 8 * quad);
    f32x4 kst = {0.f, 0.f, 0.f, 0.f}, qst = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 kp[NI];
      if constexpr (F32IN) {
        split_pair<NI>(kqc.k[2 * ks], kqc.k[2 * ks + 1], kp);
#pragma unroll
        for (int n = 0; n < NI; ++n) *(bf16x8*)(Kt[n] + (tw + hl) * kSK + 32 * ks + 8 * quad) = kp[n];
      } else {
        kp[0] = kqc.k[ks];
      }
      kst = mfma_planes<NI, NS, ORD>(kp, sp[ks], kst);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 qp[NI];
      if constexpr (F32IN)
        split_pair<NI>(kqc.q[2 * ks], kqc.q[2 * ks + 1], qp);
      else
        qp[0] = kqc.q[ks];
      qst = mfma_planes<NI, NS, ORD>(qp, sp[ks], qst);
    }
    // The previous chunk's output tile goes out while the products run.
    if (c > 0) flush_out(c - 1);
    if constexpr (!F32IN) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        *(bf16x8*)(Kt[0] + (tw + hl) * kSK + 32 * ks + 8 * quad) = kqc.k[ks];
    }
    fetch_kq(kqc, cf);
    f32x4 v4;
    if constexpr (F32IN) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = Vf[(tw + 4 * quad + e) * kVF + hl];
    } else {
      const bf16x4 vb = lds_read_tr4(Vs + (tw + tr_row) * kVB + tr_col);
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = static_cast<float>(vb[e]);
    }
    const f32x4 g4 = *(const f32x4*)(Gs + tw + 4 * quad);
    const float glin = fast_exp2(Gs[kC - 1]);
    f32x4 gam, xt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gam[e] = fast_exp2(g4[e]);
      const bool ok = t0 + tw + 4 * quad + e < a.T;
      xt[e] = ok ? v4[e] - gam[e] * kst[e] : 0.f;
    }
    {
      bf16x4 pl[NS];
      split_planes4<NS>(xt, pl);
#pragma unroll
      for (int n = 0; n < NS; ++n) *(bf16x4*)(Xp[n] + hl * kXB + tw + 4 * quad) = pl[n];
    }
    __syncthreads();  // X^T and the K tile complete; every wave has read S, V and Gc

    // (2) Y^T = W X^T and O = scale exp(Gc) Q S^T + P X^T for this wave's
    // tokens (W and P are causal: waves 0 and 1, tokens < 32, skip tokens
    // 32..63).
    bf16x8 xp[2][NS];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int n = 0; n < NS; ++n) xp[ks][n] = *(const bf16x8*)(Xp[n] + hl * kXB + 32 * ks + 8 * quad);
    f32x4 yt = {0.f, 0.f, 0.f, 0.f}, po = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      if (tile_live(wave, ks)) yt = mfma_planes<NS, NS, ORD>(pwc.w[ks], xp[ks], yt);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      if (tile_live(wave, ks)) po = mfma_planes<NS, NS, ORD>(pwc.p[ks], xp[ks], po);
    {
      bf16x4 pl[NS];
      split_planes4<NS>(yt, pl);
#pragma unroll
      for (int n = 0; n < NS; ++n) *(bf16x4*)(Yp[n] + hl * kXB + tw + 4 * quad) = pl[n];
    }
    stage_vg(vgn, c + 1);
    fetch_vg(vgn, min(c + 1 + PF, a.nchunks - 1));
#pragma unroll
    for (int e = 0; e < 4; ++e)
      Os[(tw + 4 * quad + e) * kOB + hl] = from_f32<TO>(a.scale * gam[e] * qst[e] + po[e]);
    __syncthreads();  // Y^T, the output tile, V and Gc of the next chunk complete

    // (3) S^T <- exp(Gc_last) S^T + K^T Y^T: A = K^T through the transposing
    // read (k-slot j of lane group quad is token 32 ks + tr_slot(quad, j)),
    // B = Y^T in the same token order; then publish the new state.
    bf16x8 yp[2][NS];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        const bf16x4 h0 = *(const bf16x4*)(Yp[n] + hl * kXB + 32 * ks + 4 * quad);
        const bf16x4 h1 = *(const bf16x4*)(Yp[n] + hl * kXB + 32 * ks + 16 + 4 * quad);
        yp[ks][n] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int mt = wave + 4 * i;
      f32x4 acc = glin * sown[i];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 ka[NI];
#pragma unroll
        for (int n = 0; n < NI; ++n) {
          const bf16x4 k0 = lds_read_tr4(Kt[n] + (32 * ks + tr_row) * kSK + 16 * mt + tr_col);
          const bf16x4 k1 = lds_read_tr4(Kt[n] + (32 * ks + 16 + tr_row) * kSK + 16 * mt + tr_col);
          ka[n] = __builtin_shufflevector(k0, k1, 0, 1, 2, 3, 4, 5, 6, 7);
        }
        acc = mfma_planes<NI, NS, ORD>(ka, yp[ks], acc);
      }
      sown[i] = acc;
    }
    // P and W of chunk c + PF: issued here rather than with step (2)'s
    // other loads, so each step issues about a third of the chunk's loads.
    fetch_pw(pwc, cf);
    put_state();
    __syncthreads();  // new state published; every wave has read Y^T and the K tile
  };

  for (int c0 = 0; c0 < a.nchunks; c0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p)
      if (c0 + p < a.nchunks) chunk(c0 + p, kq[p], pw[p], vg[(p + 1) % PF]);
  }
  flush_out(a.nchunks - 1);
#pragma unroll
  for (int i = 0; i < MT; ++i) *(f32x4*)(srow + 16 * (wave + 4 * i) + 4 * quad) = sown[i];
}

template <typename TI, int DK, typename TO>
int launch_chunk(const GdnArgs& a, hipStream_t s) {
  // two value heads per phase-A block where the key head has an even
  // number of them; fp32 inputs at head_dim 256 stage three K planes, which
  // leave LDS for one head's matrices only
  constexpr bool kPairs = !(std::is_same<TI, float>::value && DK == 256);
  if constexpr (kPairs) {
    if ((a.Hv / a.Hk) % 2 == 0) {
      hipLaunchKernelGGL((gdn_prep<TI, DK, 2>), dim3(a.nchunks, a.Hv / 2, a.B), dim3(512), 0, s,
                         a);
      const int rc = check_launch("gdn_prep");
      if (rc != ALPX_OK) return rc;
      hipLaunchKernelGGL((gdn_apply<TI, TO, DK>), dim3(a.Dv / 16 * a.Hv * a.B), dim3(256), 0, s,
                         a);
      return check_launch("gdn_apply");
    }
  }
  hipLaunchKernelGGL((gdn_prep<TI, DK, 1>), dim3(a.nchunks, a.Hv, a.B), dim3(256), 0, s, a);
  int rc = check_launch("gdn_prep");
  if (rc != ALPX_OK) return rc;
  hipLaunchKernelGGL((gdn_apply<TI, TO, DK>), dim3(a.Dv / 16 * a.Hv * a.B), dim3(256), 0, s, a);
  return check_launch("gdn_apply");
}

template <typename TI, typename TO>
int launch_chunk_dk(const GdnArgs& a, hipStream_t s) {
  switch (a.Dk) {
    case 64: return launch_chunk<TI, 64, TO>(a, s);
    case 128: return launch_chunk<TI, 128, TO>(a, s);
    default: return launch_chunk<TI, 256, TO>(a, s);
  }
}

template <typename TI>
int launch_chunk_ti(const GdnArgs& a, int out_dtype, hipStream_t s) {
  switch (out_dtype) {
    case ALPX_F32: return launch_chunk_dk<TI, float>(a, s);
    case ALPX_F16: return launch_chunk_dk<TI, f16_t>(a, s);
    default: return launch_chunk_dk<TI, bf16_t>(a, s);
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

extern "C" int alpx_gdn_chunk_uses_mfma(int dtype, int tokens, int key_heads, int value_heads,
                                        int key_dim, int value_dim) {
  using namespace alpx;
  if (tokens <= 0 || key_heads <= 0 || value_heads <= 0 || key_dim <= 0 || value_dim <= 0 ||
      value_heads % key_heads != 0)
    return 0;
  const int64_t krow = (int64_t)key_heads * key_dim, vrow = (int64_t)value_heads * value_dim;
  // phase B forms per-token element offsets as unsigned 24 x 24-bit
  // products: token < 2^24, row < 2^24 and token x row < 2^32
  const bool offsets_fit = tokens < (1 << 24) && krow < (1 << 24) && vrow < (1 << 24) &&
                           (int64_t)tokens * (krow > vrow ? krow : vrow) <= (int64_t)UINT32_MAX;
  return (dtype == ALPX_BF16 || dtype == ALPX_F32) &&
                 (key_dim == 64 || key_dim == 128 || key_dim == 256) && value_dim % 16 == 0 &&
                 offsets_fit && override_value(ALPX_OVERRIDE_GDN_SEQUENTIAL) == 0
             ? 1
             : 0;
}

extern "C" size_t alpx_gdn_chunk_workspace_bytes(int batch, int tokens, int value_heads,
                                                 int key_dim) {
  using namespace alpx;
  if (batch <= 0 || tokens <= 0 || value_heads <= 0 || key_dim <= 0) return 0;
  const int64_t chunks = (tokens + kC - 1) / kC;
  // the fp32-input kernels' three planes of P and W (bf16 inputs use two)
  return (size_t)batch * value_heads * chunks * ws_per_chunk<3>() * sizeof(float);
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
  const uintptr_t align =
      (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)state | (uintptr_t)out;
  const bool chunked =
      alpx_gdn_chunk_uses_mfma(dtype, tokens, key_heads, value_heads, key_dim, value_dim) == 1 &&
      (align & 15) == 0;
  TimedRegion timed(ALPX_T_GDN_CHUNK, s);
  if (chunked) {
    const size_t need = alpx_gdn_chunk_workspace_bytes(batch, tokens, value_heads, key_dim);
    if (!workspace || workspace_bytes < need)
      return fail(ALPX_EINVAL, "alpx_gdn_chunk_prefill: workspace holds %zu bytes, needs %zu",
                  workspace_bytes, need);
    a.ws = (float*)workspace;
    return dtype == ALPX_F32 ? launch_chunk_ti<float>(a, out_dtype, s)
                             : launch_chunk_ti<bf16_t>(a, out_dtype, s);
  }
  // Token-sequential form (fp16 inputs, other shapes): the decode step per
  // token, exactly the reference's recurrence order.
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
