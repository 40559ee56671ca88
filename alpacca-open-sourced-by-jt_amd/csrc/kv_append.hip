// KV-cache append: a bit-exact, vectorised row copy into [C, B, Hkv, D].
//
// Every (token, sequence) pair owns one contiguous source row of Hkv*D
// elements and one contiguous destination row at cache row
// (position_b + t).  Rows are moved in the widest unit that divides the row
// and both base pointers (16, 8, 4 or 2 bytes), so an fp16/bf16 cache of
// head_dim 128 moves 16 bytes per lane with fully coalesced reads and
// writes.  K and V travel in one launch (blockIdx.y selects the tensor).
//
// With one host position for every sequence and a contiguous cache, row
// (t, b) lands at cache row (position + t) * batch + b: the destination of
// the whole append is one contiguous range, the source is another, and the
// append is a plain copy (kv_copy_kernel: no per-unit index arithmetic).  Device positions and
// paged destinations take kv_append_rows: one block per (token, sequence)
// row, which works out its destination once and streams the row's units.
#include "alpx_common.h"
#include "timing.h"

namespace alpx {
namespace {

// Paged destination (table != null): logical row p of sequence b is row
// (p & (page size - 1)) of page table[b * max_pages + (p >> shift)]; rows
// past the table or naming a page outside [0, num_pages) are skipped.
struct Paging {
  const int32_t* table;
  int max_pages, shift, num_pages;
};

// Copy of one unit.  NT: nontemporal loads and stores, for appends larger
// than the caches (measured on a 2 x 256 MiB copy: 6.59 TB/s, against 6.14
// with ordinary loads and stores and 5.72 with four units per lane).
// Smaller appends keep ordinary stores, so the rows stay in the caches for
// the attention launch that reads them next (the C3 prefill reads its 8 MiB
// of new rows right after the append).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool NT, typename U>
__device__ __forceinline__ void copy_unit(U* __restrict__ dst, const U* __restrict__ src) {
  if constexpr (NT)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src), dst);
  else
    *dst = *src;
}

constexpr int64_t kStreamingBytes = (int64_t)64 << 20;  // NT above this many bytes read

// dst[i] = src[i] for i < n (K: blockIdx.y 0, V: 1), one unit per lane.
template <bool NT, typename U>
__global__ void __launch_bounds__(256)
kv_copy_kernel(U* __restrict__ kd, U* __restrict__ vd, const U* __restrict__ ks,
               const U* __restrict__ vs, int64_t kn, int64_t vn) {
  const bool is_v = blockIdx.y != 0;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (is_v ? vn : kn)) copy_unit<NT>(is_v ? vd + i : kd + i, is_v ? vs + i : ks + i);
}

// One block per source row (blockIdx.x = t * batch + b; blockIdx.y = K/V):
// the destination row is found once per block, then the block's lanes copy
// the row's units.
template <bool NT, typename U>
__global__ void __launch_bounds__(256)
kv_append_rows(U* __restrict__ kc, U* __restrict__ vc, const U* __restrict__ k,
               const U* __restrict__ v, int64_t capacity, int batch, int k_units, int v_units,
               int64_t position, const int32_t* __restrict__ positions, Paging pg) {
  const bool is_v = blockIdx.y != 0;
  U* __restrict__ dst = is_v ? vc : kc;
  const U* __restrict__ src = is_v ? v : k;
  const int units = is_v ? v_units : k_units;
  const int64_t row = blockIdx.x;
  const int64_t t = row / batch;
  const int b = (int)(row - t * batch);
  const int64_t p = (positions != nullptr ? (int64_t)positions[b] : position) + t;
  if (p < 0 || p >= capacity) return;  // device positions: never write out of bounds
  int64_t drow;
  if (pg.table != nullptr) {
    const int page = pg.table[(int64_t)b * pg.max_pages + (p >> pg.shift)];
    if (page < 0 || page >= pg.num_pages) return;
    drow = ((int64_t)page << pg.shift) | (p & ((1 << pg.shift) - 1));
  } else {
    drow = p * batch + b;
  }
  U* __restrict__ d = dst + drow * units;
  const U* __restrict__ sr = src + row * units;
  for (int u = threadIdx.x; u < units; u += blockDim.x) copy_unit<NT>(d + u, sr + u);
}

template <typename U>
int launch(void* kc, void* vc, const void* k, const void* v, int64_t capacity, int batch,
           int64_t k_bytes_row, int64_t v_bytes_row, int tokens, int64_t position,
           const int32_t* positions, Paging pg, hipStream_t stream) {
  const int64_t ku = k_bytes_row / (int64_t)sizeof(U);
  const int64_t vu = v_bytes_row / (int64_t)sizeof(U);
  const int64_t rows = (int64_t)tokens * batch;
  if (positions == nullptr && pg.table == nullptr) {
    const int64_t kn = ku * rows, vn = vu * rows;
    const int64_t per_block = 256;
    const int64_t blocks = ((kn > vn ? kn : vn) + per_block - 1) / per_block;
    // a launch dimension holds fewer than 2^32 work-items
    if (blocks * 256 > 0xffffffffLL)
      return fail(ALPX_EUNSUPPORTED, "alpx_kv_append: append too large");
    const int64_t off = position * batch;  // first destination row
    if ((kn + vn) * (int64_t)sizeof(U) > kStreamingBytes)
      hipLaunchKernelGGL((kv_copy_kernel<true, U>), dim3((unsigned)blocks, 2), dim3(256), 0,
                         stream, (U*)kc + off * ku, (U*)vc + off * vu, (const U*)k,
                         (const U*)v, kn, vn);
    else
      hipLaunchKernelGGL((kv_copy_kernel<false, U>), dim3((unsigned)blocks, 2), dim3(256), 0,
                         stream, (U*)kc + off * ku, (U*)vc + off * vu, (const U*)k,
                         (const U*)v, kn, vn);
    return check_launch("alpx_kv_append");
  }
  const int64_t widest = ku > vu ? ku : vu;
  const int threads = widest >= 256 ? 256 : (int)((widest + 63) / 64) * 64;
  if (rows * threads > 0xffffffffLL || widest > 0x7fffffff)
    return fail(ALPX_EUNSUPPORTED, "alpx_kv_append: append too large");
  if (rows * (ku + vu) * (int64_t)sizeof(U) > kStreamingBytes)
    hipLaunchKernelGGL((kv_append_rows<true, U>), dim3((unsigned)rows, 2), dim3(threads), 0,
                       stream, (U*)kc, (U*)vc, (const U*)k, (const U*)v, capacity, batch,
                       (int)ku, (int)vu, position, positions, pg);
  else
    hipLaunchKernelGGL((kv_append_rows<false, U>), dim3((unsigned)rows, 2), dim3(threads), 0,
                       stream, (U*)kc, (U*)vc, (const U*)k, (const U*)v, capacity, batch,
                       (int)ku, (int)vu, position, positions, pg);
  return check_launch("alpx_kv_append");
}

}  // namespace
}  // namespace alpx

namespace {
int kv_append_any(void* key_cache, void* value_cache, const void* key, const void* value,
                  int dtype, int64_t capacity, int batch, int kv_heads, int key_dim,
                  int value_dim, int tokens, int64_t position, const int32_t* positions,
                  alpx::Paging pg, void* stream) {
  using namespace alpx;
  TimedRegion timed(ALPX_T_KV_APPEND, (hipStream_t)stream);
  const int64_t es = (int64_t)dtype_size(dtype);
  const int64_t kb = (int64_t)kv_heads * key_dim * es;
  const int64_t vb = (int64_t)kv_heads * value_dim * es;
  uintptr_t align = (uintptr_t)key_cache | (uintptr_t)value_cache | (uintptr_t)key |
                    (uintptr_t)value | (uintptr_t)kb | (uintptr_t)vb;
  hipStream_t s = (hipStream_t)stream;
  if ((align & 15) == 0)
    return launch<u32x4>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
                         position, positions, pg, s);
  if ((align & 7) == 0)
    return launch<u32x2>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
                         position, positions, pg, s);
  if ((align & 3) == 0)
    return launch<uint32_t>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
                            position, positions, pg, s);
  return launch<uint16_t>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
                          position, positions, pg, s);
}
}  // namespace

extern "C" int alpx_kv_append(void* key_cache, void* value_cache, const void* key,
                              const void* value, int dtype, int64_t capacity, int batch,
                              int kv_heads, int key_dim, int value_dim, int tokens,
                              int64_t position, const int32_t* positions, void* stream) {
  using namespace alpx;
  if (!key_cache || !value_cache || !key || !value)
    return fail(ALPX_EINVAL, "alpx_kv_append: null buffer");
  if (!dtype_ok(dtype)) return fail(ALPX_EINVAL, "alpx_kv_append: unknown dtype %d", dtype);
  if (capacity <= 0 || batch <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0 ||
      tokens <= 0)
    return fail(ALPX_EINVAL, "alpx_kv_append: sizes must be positive");
  if (positions == nullptr) {
    if (position < 0) return fail(ALPX_EINVAL, "alpx_kv_append: negative position");
    if (position + tokens > capacity)
      return fail(ALPX_ERANGE, "attention cache position exceeds capacity (%lld + %d > %lld)",
                  (long long)position, tokens, (long long)capacity);
  }
  return kv_append_any(key_cache, value_cache, key, value, dtype, capacity, batch, kv_heads,
                       key_dim, value_dim, tokens, position, positions,
                       alpx::Paging{nullptr, 0, 0, 0}, stream);
}

extern "C" int alpx_kv_append_paged(void* key_pages, void* value_pages, const void* key,
                                    const void* value, const int32_t* block_table,
                                    int max_pages, int page_size, int num_pages, int dtype,
                                    int batch, int kv_heads, int key_dim, int value_dim,
                                    int tokens, int64_t position, const int32_t* positions,
                                    void* stream) {
  using namespace alpx;
  if (!key_pages || !value_pages || !key || !value || !block_table)
    return fail(ALPX_EINVAL, "alpx_kv_append_paged: null buffer");
  if (!dtype_ok(dtype)) return fail(ALPX_EINVAL, "alpx_kv_append_paged: unknown dtype %d", dtype);
  if (batch <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0 || tokens <= 0 ||
      max_pages <= 0 || num_pages <= 0)
    return fail(ALPX_EINVAL, "alpx_kv_append_paged: sizes must be positive");
  if (page_size <= 0 || (page_size & (page_size - 1)) != 0)
    return fail(ALPX_EINVAL, "page size must be a power of two");
  const int64_t capacity = (int64_t)max_pages * page_size;  // rows the table can address
  if (positions == nullptr) {
    if (position < 0) return fail(ALPX_EINVAL, "alpx_kv_append_paged: negative position");
    if (position + tokens > capacity)
      return fail(ALPX_ERANGE, "attention cache position exceeds capacity (%lld + %d > %lld)",
                  (long long)position, tokens, (long long)capacity);
  }
  return kv_append_any(key_pages, value_pages, key, value, dtype, capacity, batch, kv_heads,
                       key_dim, value_dim, tokens, position, positions,
                       Paging{block_table, max_pages, __builtin_ctz((unsigned)page_size),
                              num_pages},
                       stream);
}
