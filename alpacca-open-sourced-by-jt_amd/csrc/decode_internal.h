// Split-K decode machinery shared by the decode and prefill entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rope_internal.h"

namespace alpx {

// Rows of one wavefront step of the 16-bit MFMA split kernel: a paged cache
// needs pages of a power-of-two size of at least this many rows, so a wave
// tile never crosses a page.
constexpr int kDecodeWaveRows = 32;

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* seq_lens;
  const void* gate;
  void* out;
  float* part_m;    // [B][Hq][nsplit]
  float* part_l;    // [B][Hq][nsplit]
  float* part_acc;  // [B][Hq][nsplit][Dv]
  int64_t ks_pos, ks_b, ks_h, vs_pos, vs_b, vs_h;
  int64_t causal_pos0;  // < 0: decode; >= 0: row b is query token b at this + b
  int64_t kv_start;     // absolute position of cache row 0 (causal mode)
  int window;           // > 0: sliding window (causal mode)
  int length;
  int batch, q_heads, kv_heads, group, key_dim, value_dim;
  int head_chunks;  // ceil(group / 16): 16 query heads per MFMA column block
  int nsplit;       // partial slots per (b, h)
  int chunk;        // rows per slot
  // Uniform plan, one round, even nsplit: rows moved from each odd slot to
  // the even slot before it (slot 2i covers chunk + skew rows, slot 2i + 1
  // chunk - skew); 0 = equal chunks.
  int skew;
  float scale_log2; // softmax scale * log2(e)
  // Paged caches (pages != null): cache row j of sequence b lives in page
  // pages[b * max_pages + (j >> page_shift)] (clamped to [0, num_pages)),
  // at row (j & (page size - 1)) of that page; ks_page / vs_page are the
  // page strides in elements, ks_b / vs_b are unused.
  const int32_t* pages;
  int page_shift;
  int max_pages;
  int num_pages;
  int64_t ks_page, vs_page;
  int64_t gate_stride;  // elements between the gate rows of (b, h); 0 = value_dim
  int len_bias;         // added to seq_lens[b] (decode mode)
  // Balanced plan (decode with device seq_lens): the split grid is
  // (items_max, kv_heads * head_chunks, 1); every block of one grid row
  // cuts the sequences' valid rows into chunks of a common size (the
  // total of the device lengths over items_target, rounded up to `unit`)
  // and takes the blockIdx.x-th (sequence, chunk) item of the list in
  // sequence order.  Chunk c of sequence b writes partial slot c of (b, h);
  // nsplit bounds the chunks of one sequence.
  int balanced;
  int items_target;  // blocks per grid row the chunk size is cut for
  int items_max;     // grid x: at least the item count
  int unit;          // rows per block step of the split kernel
};

// The Qwen3.5 attention prologue fused into the split launch: one new token
// per sequence, at cache row positions[b] (device) or, without positions,
// at `position` for every sequence.
struct SplitPrologue {
  const void* qg;      // [B, Hq, 2 D]: per head D query then D gate values
  const void* key;     // [B, Hkv, D] new key rows, before norm and rotation
  const void* value;   // [B, Hkv, D] new value rows
  const float* qw;     // [D] query RMSNorm weight
  const float* kw;     // [D] key RMSNorm weight
  const int32_t* positions;
  int64_t position;
  int R;               // rotary pairs
  int sec[4];
  float eps;
  double inv[kMaxPairs];  // base^(-2 p / (2 R)) per pair p
};

// Bytes of split partials for `batch` rows of `q_heads` heads over `length`
// cache rows.
size_t decode_workspace(int batch, int q_heads, int kv_heads, int value_dim, int length);

// Plans and launches split + combine for fully described args (pointers,
// strides, sizes, causal fields, scale_log2); fills the partial pointers,
// nsplit and chunk.  Validation is the caller's job.  A caller-owned
// workspace must hold decode_workspace() bytes (the device-independent
// bound); with `fixed_scratch` (the entry point's name) the workspace is a
// fixed-size static array and only the bytes of the plan actually chosen
// must fit.
int run_decode(DecodeArgs a, int dtype, int out_dtype, void* workspace, size_t workspace_bytes,
               hipStream_t stream, int split_timer, int combine_timer,
               const SplitPrologue* pro = nullptr, const char* fixed_scratch = nullptr);

}  // namespace alpx
