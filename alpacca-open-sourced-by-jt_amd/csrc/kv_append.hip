// KV-cache append: a bit-exact, vectorised row copy into [C, B, Hkv, D].
//
// Every (token, sequence) pair owns one contiguous source row of
// Hkv*D elements and one contiguous destination row at cache row
// (position_b + t).  Rows are moved in the widest unit that divides the row
// and both base pointers (16, 8, 4 or 2 bytes), so an fp16/bf16 cache of
// head_dim 128 moves 16 bytes per lane with fully coalesced reads and
// writes.  K and V travel in one launch (blockIdx.y selects the tensor).
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

template <typename U>
__global__ void __launch_bounds__(256)
kv_append_kernel(U* __restrict__ kc, U* __restrict__ vc, const U* __restrict__ k,
                 const U* __restrict__ v, int64_t capacity, int batch, int64_t k_units,
                 int64_t v_units, int tokens, int64_t position,
                 const int32_t* __restrict__ positions, Paging pg) {
  const bool is_v = blockIdx.y != 0;
  U* __restrict__ dst = is_v ? vc : kc;
  const U* __restrict__ src = is_v ? v : k;
  const int64_t units = is_v ? v_units : k_units;  // units per (t, b) row
  const int64_t total = units * (int64_t)tokens * batch;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / units;
    const int64_t u = i - row * units;
    const int64_t t = row / batch;
    const int b = (int)(row - t * batch);
    const int64_t p = (positions != nullptr ? (int64_t)positions[b] : position) + t;
    if (p < 0 || p >= capacity) continue;  // device positions: never write out of bounds
    if (pg.table != nullptr) {
      const int page = pg.table[(int64_t)b * pg.max_pages + (p >> pg.shift)];
      if (page < 0 || page >= pg.num_pages) continue;
      const int64_t drow = ((int64_t)page << pg.shift) | (p & ((1 << pg.shift) - 1));
      dst[drow * units + u] = src[row * units + u];
    } else {
      dst[(p * batch + b) * units + u] = src[row * units + u];
    }
  }
}

template <typename U>
int launch(void* kc, void* vc, const void* k, const void* v, int64_t capacity, int batch,
           int64_t k_bytes_row, int64_t v_bytes_row, int tokens, int64_t position,
           const int32_t* positions, Paging pg, hipStream_t stream) {
  const int64_t ku = k_bytes_row / (int64_t)sizeof(U);
  const int64_t vu = v_bytes_row / (int64_t)sizeof(U);
  const int64_t work = (ku > vu ? ku : vu) * (int64_t)tokens * batch;
  int64_t blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(kv_append_kernel<U>, dim3((unsigned)blocks, 2), dim3(256), 0, stream,
                     (U*)kc, (U*)vc, (const U*)k, (const U*)v, capacity, batch, ku, vu, tokens,
                     position, positions, pg);
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
    return launch<uint4>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
                         position, positions, pg, s);
  if ((align & 7) == 0)
    return launch<uint2>(key_cache, value_cache, key, value, capacity, batch, kb, vb, tokens,
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
