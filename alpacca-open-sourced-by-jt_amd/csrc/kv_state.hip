// K/V cache state transfer: rows of one sequence between a device cache
// [capacity, B, Hkv, D] (fp32 / fp16 / bf16) and contiguous fp32 rows
// [rows, Hkv, D], the layout of the reference's attention state and of its
// snapshot record (FullAttentionState.key / value, FullAttentionSnapshot,
// memory.py:223-241, 385-475: float32, row-major, little-endian bytes).
// Export widens (exact); import narrows with round-to-nearest-even, as the
// reference's half-precision device mirror stores host rows
// (ALPACCAROO_KV_F16, cuda.py:1729-1738; _sync_mirror, cuda.py:1875-1900).
// Both are pure per-element moves: one thread per element, K and V in one
// launch (blockIdx.y selects the tensor).  The paged forms move the rows of
// one sequence of a paged pool ([num_pages, page_size, Hkv, D] under a
// block table [batch, max_pages]): logical row j is row j % page_size of
// page table[b][j / page_size]; a table entry outside the pool exports
// zeros and imports nothing.
#include "alpx_common.h"
#include "timing.h"

namespace alpx {
namespace {

// Cache slot of element e of logical row j (row-major [Hkv, D] rows):
// contiguous [capacity, batch, ...] or paged through the table.
struct PoolMap {
  const int32_t* table;  // null: contiguous
  int max_pages, page_shift, num_pages;
};

template <typename T, bool EXPORT>
__global__ void __launch_bounds__(256)
kv_transfer_kernel(T* kc, T* vc, float* kr, float* vr, int batch, int b, int64_t row0,
                   int64_t rows, int64_t k_row, int64_t v_row, PoolMap pm) {
  const bool is_v = blockIdx.y != 0;
  const int64_t n = is_v ? v_row : k_row;  // elements per cache row
  T* cache = is_v ? vc : kc;
  float* flat = is_v ? vr : kr;
  const int64_t total = rows * n;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / n;
    const int64_t e = i - r * n;
    const int64_t j = row0 + r;
    int64_t slot_row = j * batch + b;
    if (pm.table != nullptr) {
      const int pg = pm.table[(int64_t)b * pm.max_pages + (j >> pm.page_shift)];
      if (pg < 0 || pg >= pm.num_pages) {
        if (EXPORT) flat[i] = 0.f;
        continue;
      }
      slot_row = ((int64_t)pg << pm.page_shift) + (j & ((1 << pm.page_shift) - 1));
    }
    T* slot = cache + slot_row * n + e;
    if (EXPORT)
      flat[i] = to_f32(*slot);
    else
      *slot = from_f32<T>(flat[i]);
  }
}

template <typename T>
int transfer(bool exp, void* kc, void* vc, float* kr, float* vr, int batch, int b, int64_t row0,
             int64_t rows, int64_t k_row, int64_t v_row, const PoolMap& pm, hipStream_t s) {
  const int64_t work = rows * (k_row > v_row ? k_row : v_row);
  int64_t blocks = (work + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  const dim3 grid((unsigned)blocks, 2);
  if (exp)
    hipLaunchKernelGGL((kv_transfer_kernel<T, true>), grid, dim3(256), 0, s, (T*)kc, (T*)vc, kr,
                       vr, batch, b, row0, rows, k_row, v_row, pm);
  else
    hipLaunchKernelGGL((kv_transfer_kernel<T, false>), grid, dim3(256), 0, s, (T*)kc, (T*)vc, kr,
                       vr, batch, b, row0, rows, k_row, v_row, pm);
  return check_launch(exp ? "alpx_kv_export" : "alpx_kv_import");
}

int kv_transfer(bool exp, void* key_cache, void* value_cache, float* key_rows, float* value_rows,
                int dtype, int64_t capacity, int batch, int kv_heads, int key_dim, int value_dim,
                int batch_index, int64_t row0, int64_t rows, void* stream,
                const PoolMap& pm = PoolMap{nullptr, 0, 0, 0}) {
  const char* what = pm.table != nullptr ? (exp ? "alpx_kv_export_paged" : "alpx_kv_import_paged")
                                         : (exp ? "alpx_kv_export" : "alpx_kv_import");
  if (!key_cache || !value_cache || !key_rows || !value_rows)
    return fail(ALPX_EINVAL, "%s: null buffer", what);
  if (!dtype_ok(dtype)) return fail(ALPX_EINVAL, "%s: unknown dtype", what);
  if (capacity <= 0 || batch <= 0 || kv_heads <= 0 || key_dim <= 0 || value_dim <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", what);
  if (batch_index < 0 || batch_index >= batch)
    return fail(ALPX_EINVAL, "batch_index exceeds the cache batch");
  if (row0 < 0 || rows < 0 || row0 + rows > capacity)
    return fail(ALPX_ERANGE, "%s: rows [%lld, %lld) exceed the cache capacity %lld", what,
                (long long)row0, (long long)(row0 + rows), (long long)capacity);
  if (rows == 0) return ALPX_OK;
  hipStream_t s = (hipStream_t)stream;
  TimedRegion timed(ALPX_T_AUX, s);
  const int64_t kn = (int64_t)kv_heads * key_dim, vn = (int64_t)kv_heads * value_dim;
  switch (dtype) {
    case ALPX_F32:
      return transfer<float>(exp, key_cache, value_cache, key_rows, value_rows, batch,
                             batch_index, row0, rows, kn, vn, pm, s);
    case ALPX_F16:
      return transfer<f16_t>(exp, key_cache, value_cache, key_rows, value_rows, batch,
                             batch_index, row0, rows, kn, vn, pm, s);
    default:
      return transfer<bf16_t>(exp, key_cache, value_cache, key_rows, value_rows, batch,
                              batch_index, row0, rows, kn, vn, pm, s);
  }
}

}  // namespace
}  // namespace alpx

extern "C" int alpx_kv_export(const void* key_cache, const void* value_cache, float* key_rows,
                              float* value_rows, int dtype, int64_t capacity, int batch,
                              int kv_heads, int key_dim, int value_dim, int batch_index,
                              int64_t row0, int64_t rows, void* stream) {
  return alpx::kv_transfer(true, const_cast<void*>(key_cache), const_cast<void*>(value_cache),
                           key_rows, value_rows, dtype, capacity, batch, kv_heads, key_dim,
                           value_dim, batch_index, row0, rows, stream);
}

extern "C" int alpx_kv_import(const float* key_rows, const float* value_rows, void* key_cache,
                              void* value_cache, int dtype, int64_t capacity, int batch,
                              int kv_heads, int key_dim, int value_dim, int batch_index,
                              int64_t row0, int64_t rows, void* stream) {
  return alpx::kv_transfer(false, key_cache, value_cache, const_cast<float*>(key_rows),
                           const_cast<float*>(value_rows), dtype, capacity, batch, kv_heads,
                           key_dim, value_dim, batch_index, row0, rows, stream);
}

// Paged pools: `capacity` is max_pages * page_size logical rows of sequence
// batch_index of the block table [batch, max_pages].
static int kv_transfer_paged(bool exp, void* key_pages, void* value_pages,
                             const int32_t* block_table, int batch, int max_pages, int page_size,
                             int num_pages, float* key_rows, float* value_rows, int dtype,
                             int kv_heads, int key_dim, int value_dim, int batch_index,
                             int64_t row0, int64_t rows, void* stream) {
  using namespace alpx;
  const char* what = exp ? "alpx_kv_export_paged" : "alpx_kv_import_paged";
  if (!block_table) return fail(ALPX_EINVAL, "%s: null block table", what);
  if (max_pages <= 0 || num_pages <= 0 || page_size <= 0)
    return fail(ALPX_EINVAL, "%s: sizes must be positive", what);
  if ((page_size & (page_size - 1)) != 0)
    return fail(ALPX_EINVAL, "page size must be a power of two");
  const PoolMap pm = {block_table, max_pages, __builtin_ctz((unsigned)page_size), num_pages};
  return kv_transfer(exp, key_pages, value_pages, key_rows, value_rows, dtype,
                     (int64_t)max_pages * page_size, batch, kv_heads, key_dim, value_dim,
                     batch_index, row0, rows, stream, pm);
}

extern "C" int alpx_kv_export_paged(const void* key_pages, const void* value_pages,
                                    const int32_t* block_table, int batch, int max_pages,
                                    int page_size, int num_pages, float* key_rows,
                                    float* value_rows, int dtype, int kv_heads, int key_dim,
                                    int value_dim, int batch_index, int64_t row0, int64_t rows,
                                    void* stream) {
  return kv_transfer_paged(true, const_cast<void*>(key_pages), const_cast<void*>(value_pages),
                           block_table, batch, max_pages, page_size, num_pages, key_rows,
                           value_rows, dtype, kv_heads, key_dim, value_dim, batch_index, row0,
                           rows, stream);
}

extern "C" int alpx_kv_import_paged(const float* key_rows, const float* value_rows,
                                    void* key_pages, void* value_pages,
                                    const int32_t* block_table, int batch, int max_pages,
                                    int page_size, int num_pages, int dtype, int kv_heads,
                                    int key_dim, int value_dim, int batch_index, int64_t row0,
                                    int64_t rows, void* stream) {
  return kv_transfer_paged(false, key_pages, value_pages, block_table, batch, max_pages,
                           page_size, num_pages, const_cast<float*>(key_rows),
                           const_cast<float*>(value_rows), dtype, kv_heads, key_dim, value_dim,
                           batch_index, row0, rows, stream);
}
