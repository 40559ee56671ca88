/*
 * alpx.h -- C-ABI of the MI355X (gfx950) attention library libalpx.so.
 *
 * The library replaces the attention hot path of alpaccaroo: KV-cache
 * append, GQA decode attention (with the optional Qwen3.5 sigmoid output
 * gate), causal prefill attention and the Qwen3.5 gated delta-rule (GDN)
 * recurrence.  Each entry point cites the reference interface it stands
 * behind (paths relative to the reference's alpaccaroo/ package).
 *
 * Conventions
 *  - Every pointer is a device pointer unless stated otherwise; the caller
 *    owns all buffers (caches, state, outputs, workspace).
 *  - Element strides are in ELEMENTS, not bytes.  The innermost (head
 *    dimension) axis is always contiguous.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Calls
 *    are asynchronous: they enqueue kernels and return.
 *  - Return value: ALPX_OK (0) or a negative status; the message of the
 *    last failing call on this host thread is alpx_last_error().
 *    Arguments are validated before anything is enqueued, so a failing
 *    call leaves every buffer untouched.
 *  - One caller at a time per stream; calls on one GPU that share a
 *    workspace must be ordered (same stream), as in the reference's
 *    single-generation lock (serve.py:326).
 */
#ifndef ALPX_H
#define ALPX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ALPX_ABI_VERSION 1

/* Element types (the reference's ROCm ops are float32 only,
 * qwen35_rocm_ops.py:153-158; fp16/bf16 are this library's extension). */
enum alpx_dtype { ALPX_F32 = 0, ALPX_F16 = 1, ALPX_BF16 = 2 };

enum alpx_status {
  ALPX_OK = 0,
  ALPX_EINVAL = -1,       /* contract violation: maps to ValueError/TypeError */
  ALPX_EUNSUPPORTED = -2, /* shape/dtype outside what the kernels cover */
  ALPX_EHIP = -3,         /* HIP runtime error (launch, device query) */
  ALPX_ERANGE = -4        /* position/length outside the cache capacity */
};

/* ABI version of the loaded library (must equal ALPX_ABI_VERSION). */
int alpx_abi_version(void);

/* Message of the last failing call on the calling host thread ("" if none). */
const char* alpx_last_error(void);

/* gcnArchName of `device` (e.g. "gfx950:sramecc+:xnack-") into a host buffer. */
int alpx_device_arch(int device, char* buf, int buf_len);

/* Device address of page-locked host memory allocated by the HIP runtime
 * (hipHostMalloc; torch's pin_memory), so that an entry point can write
 * its output straight to host memory over PCIe (the NumPy-facing decode
 * drop-in's mirror writes its 16-KiB output that way instead of a copy
 * back).  No counterpart in the reference.  ALPX_EINVAL for any other
 * pointer. */
int alpx_host_device_pointer(void* host, void** device_pointer);

/*
 * KV-cache append.
 * Replaces Qwen35RocmOps.attention_append_ (qwen35_rocm_ops.py:475-500),
 * qwen35_cuda._kv_append (qwen35_cuda.py:1001-1012), the llama-class cache
 * writes cache_k[li][pos0:pos0+n] = k (model.py:1335-1337, :1431-1432) and
 * FullAttentionState.append (memory.py:419-428).
 *
 * Caches are [capacity, batch, kv_heads, key_dim|value_dim]; key/value are
 * `tokens` rows [tokens, batch, kv_heads, key_dim|value_dim], contiguous.
 * Row (t, b) is written to cache row positions[b] + t when `positions`
 * (device int32 [batch]) is given, else to position + t.  The copy is
 * bit-exact.  With `positions` == NULL the call fails with ALPX_ERANGE
 * unless position + tokens <= capacity; with device `positions` the host
 * cannot see them, and rows that would fall outside [0, capacity) are
 * skipped by the kernel (never written out of bounds).
 */
int alpx_kv_append(void* key_cache, void* value_cache, const void* key, const void* value,
                   int dtype, int64_t capacity, int batch, int kv_heads, int key_dim,
                   int value_dim, int tokens, int64_t position, const int32_t* positions,
                   void* stream);

/* Paged K/V cache (an extension: the reference keeps one contiguous
 * [n_ctx, Hkv, D] array per layer, model.py:866-870, or growing host rows,
 * memory.py:385-475).  Pages are [num_pages, page_size, kv_heads,
 * key_dim|value_dim]; block_table [batch, max_pages] (device int32) maps
 * logical row j of sequence b to row (j % page_size) of page
 * block_table[b * max_pages + j / page_size].  page_size is a power of two
 * (at least 32 for decode).  alpx_kv_append_paged is alpx_kv_append
 * through the table (bit-exact; rows past the table or naming a page
 * outside [0, num_pages) are skipped); alpx_decode_gqa_paged is
 * alpx_decode_gqa over the table (same split plan and arithmetic, so its
 * result equals the contiguous cache's bit for bit; a page index outside
 * [0, num_pages) is clamped into the pool).  Workspace as
 * alpx_decode_workspace_bytes. */
int alpx_kv_append_paged(void* key_pages, void* value_pages, const void* key, const void* value,
                         const int32_t* block_table, int max_pages, int page_size, int num_pages,
                         int dtype, int batch, int kv_heads, int key_dim, int value_dim,
                         int tokens, int64_t position, const int32_t* positions, void* stream);
/* Causal prefill (as alpx_prefill_causal / _gated, with gate optional:
 * null = no gate) of q [q_tokens, Hq, D] at positions q_pos0 .. over the
 * first kv_tokens logical rows of sequence batch_index of a paged cache
 * (pages and block_table as above; page_size a power of two >= 64, so a
 * key tile never crosses a page).  The contiguous call's single-tile
 * kernel, tiling and arithmetic, so the same rows give its bits (and its
 * shared-stream kernel's; its paired kernel agrees within rounding).  fp16 / bf16
 * pages, head_dim = value width in {64, 128, 256}, output in `dtype`
 * (others: ALPX_EUNSUPPORTED).  No workspace. */
int alpx_prefill_causal_paged(const void* q, const void* key_pages, const void* value_pages,
                              const int32_t* block_table, int max_pages, int page_size,
                              int num_pages, int batch_index, const void* gate, void* out,
                              int q_tokens, int kv_tokens, int q_heads, int kv_heads,
                              int head_dim, int64_t q_pos0, int window, int64_t kv_start,
                              float scale, int dtype, void* stream);
int alpx_decode_gqa_paged(const void* q, const void* key_pages, const void* value_pages,
                          const int32_t* block_table, int max_pages, int page_size,
                          int num_pages, const int32_t* seq_lens, int length, const void* gate,
                          void* out, void* workspace, size_t workspace_bytes, int batch,
                          int q_heads, int kv_heads, int key_dim, int value_dim, float scale,
                          int dtype, int out_dtype, void* stream);

/* K/V state transfer for one sequence of a cache [capacity, batch, kv_heads,
 * key_dim|value_dim] (fp32 / fp16 / bf16, `dtype`): alpx_kv_export widens
 * cache rows [row0, row0 + rows) of sequence batch_index into contiguous
 * fp32 key_rows [rows, kv_heads, key_dim] and value_rows [rows, kv_heads,
 * value_dim]; alpx_kv_import writes such fp32 rows into the cache, rounding
 * to nearest even for fp16 / bf16 caches (bit-exact copies for fp32).  The
 * fp32 rows are the reference's attention state layout and snapshot record
 * (FullAttentionState.key / value and FullAttentionSnapshot, memory.py:
 * 223-241, 385-475, "f32-le"), so export + a device-to-host copy gives the
 * bytes of FullAttentionState.snapshot and a host-to-device copy + import
 * restores one; an fp16 cache stores rows as the reference's half-precision
 * device mirror does (ALPACCAROO_KV_F16, cuda.py:1729-1738; _sync_mirror,
 * cuda.py:1875-1900).  Rows outside [0, capacity) fail with ALPX_ERANGE. */
int alpx_kv_export(const void* key_cache, const void* value_cache, float* key_rows,
                   float* value_rows, int dtype, int64_t capacity, int batch, int kv_heads,
                   int key_dim, int value_dim, int batch_index, int64_t row0, int64_t rows,
                   void* stream);
int alpx_kv_import(const float* key_rows, const float* value_rows, void* key_cache,
                   void* value_cache, int dtype, int64_t capacity, int batch, int kv_heads,
                   int key_dim, int value_dim, int batch_index, int64_t row0, int64_t rows,
                   void* stream);
/* The same transfers for one sequence of a paged pool (an extension):
 * pages [num_pages, page_size, kv_heads, key_dim|value_dim], block_table
 * [batch, max_pages] (device int32, page_size a power of two); logical row
 * j of sequence batch_index is row j % page_size of page
 * block_table[batch_index][j / page_size].  A table entry outside
 * [0, num_pages) exports zeros and imports nothing.  Rows outside
 * [0, max_pages * page_size) fail with ALPX_ERANGE.  Same values as the
 * contiguous calls on the same rows. */
int alpx_kv_export_paged(const void* key_pages, const void* value_pages,
                         const int32_t* block_table, int batch, int max_pages, int page_size,
                         int num_pages, float* key_rows, float* value_rows, int dtype,
                         int kv_heads, int key_dim, int value_dim, int batch_index, int64_t row0,
                         int64_t rows, void* stream);
int alpx_kv_import_paged(const float* key_rows, const float* value_rows, void* key_pages,
                         void* value_pages, const int32_t* block_table, int batch, int max_pages,
                         int page_size, int num_pages, int dtype, int kv_heads, int key_dim,
                         int value_dim, int batch_index, int64_t row0, int64_t rows,
                         void* stream);

/*
 * Workspace size in bytes needed by alpx_decode_gqa for these sizes
 * (split-K partials: running max, running sum and the unnormalised
 * accumulator per query head and split).
 */
size_t alpx_decode_workspace_bytes(int batch, int q_heads, int kv_heads, int value_dim,
                                   int max_len);

/*
 * Single-token GQA decode attention (split-K flash-decode + combine).
 * Replaces kernels.attention_decode (kernels.py:1183-1200),
 * Model._attention_np (model.py:1231-1252),
 * qwen35_kernels.qwen35_full_attention_decode (qwen35_kernels.py:363-392),
 * Qwen35RocmOps.online_attention (qwen35_rocm_ops.py:502-564) and, with
 * `gate`, the sigmoid output gate of Qwen35Model._attention
 * (qwen35_runtime.py:653-660; Qwen35RocmOps.sigmoid_gate,
 * qwen35_rocm_ops.py:286-290).
 *
 *   out[b, h, :] = softmax_j(scale * q[b, h] . K[j, b, h // G]) . V[j, b, h // G]
 *                  (* sigmoid(gate[b, h, :]) when gate != NULL)
 * over cache rows j < len_b, where G = q_heads / kv_heads (contiguous
 * grouping) and len_b = seq_lens[b] (device int32 [batch], ragged
 * extension) or `length` when seq_lens == NULL.  Device lengths are
 * clamped to [0, length]; a sequence of length 0 yields zeros.
 *
 * q [batch, q_heads, key_dim] and gate/out [batch, q_heads, value_dim] are
 * contiguous.  K element (j, b, h, d) is at
 * key_cache[j*k_pos_stride + b*k_batch_stride + h*k_head_stride + d]
 * (likewise V with the v_* strides): [capacity, batch, kv_heads, D] is the
 * ROCm workspace layout, (t, kv_heads, D) with batch 1 the llama layout.
 * q, K, V and gate use `dtype`; out uses `out_dtype`; arithmetic is fp32.
 * workspace must hold alpx_decode_workspace_bytes(batch, q_heads,
 * kv_heads, value_dim, length) bytes; it is scratch (no initial contents
 * needed).  Calls sharing a workspace must be ordered on one stream.  One
 * call is two kernel launches: the split pass and the combine pass.
 */
int alpx_decode_gqa(const void* q, const void* key_cache, const void* value_cache,
                    const int32_t* seq_lens, int length, const void* gate, void* out,
                    void* workspace, size_t workspace_bytes, int batch, int q_heads,
                    int kv_heads, int key_dim, int value_dim, int64_t k_pos_stride,
                    int64_t k_batch_stride, int64_t k_head_stride, int64_t v_pos_stride,
                    int64_t v_batch_stride, int64_t v_head_stride, float scale, int dtype,
                    int out_dtype, void* stream);

/* Bytes of the static scratch array alpx_decode_gqa_noalloc keeps on each
 * GPU (32 MiB: the C2 ragged step needs 17 MB of partials). */
#define ALPX_DECODE_SCRATCH_BYTES ((size_t)32 << 20)

/*
 * alpx_decode_gqa without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments (minus workspace),
 * kernels, split plan and result (bit for bit) as alpx_decode_gqa, except
 * where alpx_decode_gqa's several-rounds plan (long 16-bit caches) needs
 * more partial bytes than the array: the call then keeps the one-round
 * plan (same result within rounding).  The split partials live in a
 * static device array of ALPX_DECODE_SCRATCH_BYTES per GPU, held from the
 * library's load until the process ends; its address on each device is
 * looked up on the first call there.  A call whose one-round plan needs
 * more partial bytes than that (many sequences x query heads x splits)
 * fails with ALPX_ERANGE before anything is enqueued; use alpx_decode_gqa
 * then.  Every call on one GPU
 * shares the array, so calls that overlap on one GPU (unordered streams)
 * race; calls ordered on one stream are safe.  Nothing in the array needs
 * initial contents.
 */
int alpx_decode_gqa_noalloc(const void* q, const void* key_cache, const void* value_cache,
                            const int32_t* seq_lens, int length, const void* gate, void* out,
                            int batch, int q_heads, int kv_heads, int key_dim, int value_dim,
                            int64_t k_pos_stride, int64_t k_batch_stride, int64_t k_head_stride,
                            int64_t v_pos_stride, int64_t v_batch_stride, int64_t v_head_stride,
                            float scale, int dtype, int out_dtype, void* stream);

/*
 * Workspace bytes alpx_prefill_causal may need (only its fallback path, for
 * fp32 or unsupported shapes, uses it).
 */
size_t alpx_prefill_workspace_bytes(int q_tokens, int q_heads, int kv_heads, int value_dim,
                                    int kv_tokens);

/*
 * Causal (optionally sliding-window) GQA prefill attention.
 * Replaces Model._attention_batch_np (model.py:1254-1272), its windowed form
 * _attention_batch_window_np (model.py:1567-1592), the device seam
 * cuda.attention_batch (cuda.py:1186-1244) and
 * qwen35_kernels.qwen35_full_attention_prefill (qwen35_kernels.py:395-411).
 *
 * q [q_tokens, q_heads, key_dim] and out [q_tokens, q_heads, value_dim] are
 * contiguous; cache row j of head h is key[j*k_pos_stride + h*key_dim + d]
 * (value likewise), so a (t, kv_heads, D) cache has k_pos_stride =
 * kv_heads*key_dim and one sequence of a [C, B, Hkv, D] cache is the base
 * pointer b*Hkv*D with k_pos_stride = B*Hkv*D.  Query token t sits at
 * absolute position q_pos0 + t, cache row j at kv_start + j; t sees row j
 * iff kv_start + j <= q_pos0 + t and (window == 0 or kv_start + j >
 * q_pos0 + t - window).  A row that sees no key yields zeros (the device
 * seam's convention, cuda.py:572-577).  Scale is usually 1/sqrt(key_dim).
 * fp16/bf16 with key_dim == value_dim in {64, 128, 256} and 16-byte aligned
 * rows run the MFMA flash kernel (no workspace); anything else runs the
 * split-K machinery and needs alpx_prefill_workspace_bytes of workspace.
 */
int alpx_prefill_causal(const void* q, const void* key, const void* value, void* out,
                        void* workspace, size_t workspace_bytes, int q_tokens, int kv_tokens,
                        int q_heads, int kv_heads, int key_dim, int value_dim,
                        int64_t k_pos_stride, int64_t v_pos_stride, int64_t q_pos0, int window,
                        int64_t kv_start, float scale, int dtype, int out_dtype, void* stream);

/*
 * alpx_prefill_causal with the Qwen3.5 sigmoid output gate applied before
 * the output is rounded: out = attention * sigmoid(gate), gate
 * [q_tokens, q_heads, value_dim] in `dtype`.  Replaces the pair
 * causal prefill + Qwen35RocmOps.sigmoid_gate (qwen35_rocm_ops.py:286-290;
 * gate placement qwen35_runtime.py:653-660) in a prefill chunk of the
 * full-attention layer.  The stable sigmoid is tensor.py:123-129's.
 */
int alpx_prefill_causal_gated(const void* q, const void* key, const void* value, const void* gate,
                              void* out, void* workspace, size_t workspace_bytes, int q_tokens,
                              int kv_tokens, int q_heads, int kv_heads, int key_dim,
                              int value_dim, int64_t k_pos_stride, int64_t v_pos_stride,
                              int64_t q_pos0, int window, int64_t kv_start, float scale, int dtype,
                              int out_dtype, void* stream);

/*
 * A prefill chunk's cache append and causal prefill in one call: key /
 * value [q_tokens, kv_heads, key_dim|value_dim] (contiguous) are written to
 * rows position .. position + q_tokens - 1 of a batch-1 cache [capacity, 1,
 * kv_heads, key_dim|value_dim] (bit-exact, as alpx_kv_append), and q
 * attends to cache rows 0 .. position + t as in alpx_prefill_causal with
 * q_pos0 = position, kv_start = 0 and kv_tokens = position + q_tokens
 * (gate optional, as alpx_prefill_causal_gated).  Replaces the sequence
 * "write the chunk's rows, then attend" of Model's batched prefill
 * (model.py:1335-1340: cache_k / cache_v rows, then _attention_batch_np,
 * model.py:1254-1272).  On the MFMA path this is one launch: the kernel
 * reads the chunk's rows from key / value and each block writes its own
 * tokens' rows into the cache; other shapes run alpx_kv_append and then
 * alpx_prefill_causal's fallback (workspace as alpx_prefill_causal).
 * position outside [0, capacity - q_tokens]: ALPX_ERANGE, nothing written.
 */
int alpx_prefill_append(const void* q, const void* key, const void* value, void* key_cache,
                        void* value_cache, const void* gate, void* out, void* workspace,
                        size_t workspace_bytes, int q_tokens, int64_t capacity, int q_heads,
                        int kv_heads, int key_dim, int value_dim, int64_t position, int window,
                        float scale, int dtype, int out_dtype, void* stream);

/*
 * Gated delta-rule (GDN) decode step, in place on the state.
 * Replaces Qwen35RocmOps.gated_delta_net_step_ (qwen35_rocm_ops.py:362-407),
 * qwen35_kernels.qwen35_gdn_step (qwen35_kernels.py:310-332) and
 * qwen35_cuda._gdn_step/_gdn_step_out (qwen35_cuda.py:239-293).
 *
 * state [batch, value_heads, value_dim, key_dim] fp32 (row-major value x
 * key, qwen35_ops.py:318-323); q, k [batch, key_heads, key_dim]; v and out
 * [batch, value_heads, value_dim]; beta and log_decay [batch, value_heads]
 * fp32.  Value head h reads key head h % key_heads (qwen35_ops.py:275-285):
 *   S <- exp(g) S; p = S k; S <- S + beta (v - p) k^T; out = S q / sqrt(key_dim)
 * q/k/v use `dtype`, out `out_dtype`; arithmetic is fp32.  key_dim <= 256.
 */
int alpx_gdn_step(float* state, const void* q, const void* k, const void* v, const float* beta,
                  const float* log_decay, void* out, int batch, int key_heads, int value_heads,
                  int key_dim, int value_dim, int dtype, int out_dtype, void* stream);

/* Workspace bytes for alpx_gdn_chunk_prefill (chunked path). */
size_t alpx_gdn_chunk_workspace_bytes(int batch, int tokens, int value_heads, int key_dim);

/* 1 when alpx_gdn_chunk_prefill runs these sizes on the chunked MFMA
 * kernels (given 16-byte aligned buffers), 0 when it runs them token by
 * token.  Host-only: no device work.  (No reference counterpart: it tells
 * a caller whether the call needs the chunk workspace.) */
int alpx_gdn_chunk_uses_mfma(int dtype, int tokens, int key_heads, int value_heads, int key_dim,
                             int value_dim);

/*
 * GDN over a `tokens`-long prefill, in place on the state: the same result
 * as `tokens` calls of alpx_gdn_step (the reference's only form, the
 * token-sequential scan of qwen35_ops.gated_delta_net_scan,
 * qwen35_ops.py:373-403, and Qwen35Model.prefill_state,
 * qwen35_runtime.py:777-810), computed in chunks of 64 tokens.
 *
 * q, k [batch, tokens, key_heads, key_dim]; v and out [batch, tokens,
 * value_heads, value_dim]; beta, log_decay [batch, tokens, value_heads] fp32;
 * state as in alpx_gdn_step.  bf16 or fp32 inputs with key_dim in {64,
 * 128, 256}, value_dim a multiple of 16 and 16-byte aligned rows run the
 * chunked MFMA kernels (workspace of alpx_gdn_chunk_workspace_bytes
 * needed; alpx_gdn_chunk_uses_mfma tells); fp32 inputs enter those
 * products as hi + lo bf16 pairs, so their result stays within fp32
 * accuracy (1e-4) of the token-sequential recurrence.  Anything else runs
 * the step kernel token by token (workspace unused).
 */
int alpx_gdn_chunk_prefill(float* state, const void* q, const void* k, const void* v,
                           const float* beta, const float* log_decay, void* out, void* workspace,
                           size_t workspace_bytes, int batch, int tokens, int key_heads,
                           int value_heads, int key_dim, int value_dim, int dtype, int out_dtype,
                           void* stream);

/*
 * Sigmoid output gate: out[i] = values[i] * sigmoid(gate[i]) for i < n, with
 * the stable two-branch sigmoid of tensor.stable_sigmoid (tensor.py:123-129).
 * Replaces Qwen35RocmOps.sigmoid_gate (qwen35_rocm_ops.py:286-290) and
 * qwen35_cuda._sigmoid_gate (qwen35_cuda.py:953-963).  values/gate use
 * `dtype`, out uses `out_dtype`; out may alias values when the dtypes match.
 */
int alpx_sigmoid_gate(const void* values, const void* gate, void* out, int64_t n, int dtype,
                      int out_dtype, void* stream);

/*
 * SiLU: out[i] = values[i] * sigmoid(values[i]) (stable sigmoid), the
 * activation between the convolution step and the split in the recurrent
 * layer.  Replaces Qwen35RocmOps.silu (qwen35_rocm_ops.py:276-278) and
 * qwen35_ops.silu (qwen35_ops.py:26-31).  out may alias values when the
 * dtypes match.
 */
int alpx_silu(const void* values, void* out, int64_t n, int dtype, int out_dtype, void* stream);

/*
 * Qwen3.5 layer primitives around the kernels above (the decomposed ROCm
 * operations of qwen35_rocm_ops.py and the NumPy/Numba helpers of
 * qwen35_kernels.py / qwen35_ops.py).  Inputs and outputs are contiguous
 * unless strides are given.
 */

/* Row-wise normalisation of `rows` rows of `n` values.  Input row r starts
 * at element (r / group_rows) * group_stride + (r % group_rows) * n
 * (group_rows <= 0: contiguous rows); gate and out rows are contiguous.
 *   mode 0 (L2):       out = x / max(||x||_2, eps)
 *     Qwen35RocmOps.l2_normalize (qwen35_rocm_ops.py:260-268),
 *     qwen35_normalize_qk (qwen35_kernels.py:277-287),
 *     tensor.l2_normalize (tensor.py:139-158);
 *   mode 1 (RMS):      out = x / sqrt(mean(x^2) + eps) * weight
 *     Qwen35RocmOps.rms_norm (qwen35_rocm_ops.py:251-258),
 *     qwen35_ops.rms_norm (qwen35_ops.py:46-76), the per-head Q/K norms
 *     of qwen35_runtime.py:625-630;
 *   mode 2 (gated):    out = rms_norm(x) * silu(gate)
 *     Qwen35RocmOps.recurrent_gate (qwen35_rocm_ops.py:292-296),
 *     qwen35_gated_rms (qwen35_kernels.py:335-352).
 * weight: fp32 [n] (modes 1, 2); x and gate use `dtype`, out `out_dtype`. */
int alpx_row_norm(const void* x, const float* weight, const void* gate, void* out, int64_t rows,
                  int n, int64_t group_rows, int64_t group_stride, float eps, int mode, int dtype,
                  int out_dtype, void* stream);

/* Depthwise causal convolution step, fp32 state:
 *   out[b, c] = sum_{t < K-1} history[b, t, c] w(t, c) + current[b, c] w(K-1, c)
 * then history[b] shifts by one row (oldest dropped, current appended) and,
 * with apply_silu, out = silu(out).  w(t, c) = weight[t * weight_tap_stride
 * + c * weight_channel_stride]: [K, C] (ROCm / GGUF order) is (C, 1), [C, K]
 * (qwen35_kernels order) is (1, K).  Replaces
 * Qwen35RocmOps.causal_convolution_step_ (qwen35_rocm_ops.py:320-341; no
 * SiLU), qwen35_conv_step (qwen35_kernels.py:53-68, :261-274; with SiLU)
 * and qwen35_ops.depthwise_causal_conv_step (qwen35_ops.py:218-258). */
int alpx_conv_step(const float* current, const float* weight, float* history, void* out,
                   int batch, int channels, int kernel, int64_t weight_tap_stride,
                   int64_t weight_channel_stride, int apply_silu, int out_dtype, void* stream);

/* GDN recurrent parameters for `count` = batch * heads entries (fp32):
 * beta = sigmoid(beta_logits), log_decay = softplus(alpha_logits +
 * dt_bias[i % heads]) * ssm_a[i % heads].  Replaces
 * Qwen35RocmOps.recurrent_parameters (qwen35_rocm_ops.py:343-360) and
 * qwen35_beta_decay (qwen35_kernels.py:290-307). */
int alpx_recurrent_parameters(const float* beta_logits, const float* alpha_logits,
                              const float* dt_bias, const float* ssm_a, float* beta,
                              float* log_decay, int64_t count, int heads, void* stream);

/* IMROPE (Qwen interleaved multi-section rotary embedding, NeoX half-split
 * pairs) of x [rows, heads, dim]: with R = sum(sections) (host int[4]),
 * pair p < R rotates coordinates (p, p + R) by theta = pos(lane(p)) *
 * frequency_scale * frequency_base^(-2p / (2R)); coordinates >= 2R are
 * copied.  positions: device int64, lanes (T, H, W, E) of row r at
 * positions + r * position_stride (stride 0: one lane vector for all rows).
 * Replaces Qwen35RocmOps.imrope (qwen35_rocm_ops.py:409-473) and
 * qwen35_ops.imrope_rotate (qwen35_ops.py:138-215). */
int alpx_imrope(const void* x, void* out, const int64_t* positions, int64_t position_stride,
                int64_t rows, int heads, int dim, const int* sections, double frequency_base,
                double frequency_scale, int dtype, int out_dtype, void* stream);

/* Qwen3.5 full-attention decode prologue, fused, one token per sequence
 * (qwen35_runtime.py:597-650): the joint projection query_gate [B, Hq, 2D]
 * is split (Qwen35RocmOps.split_query_gate, qwen35_rocm_ops.py:298-318)
 * into query_out [B, Hq, D] (RMSNorm with q_norm, then IMROPE) and
 * gate_out [B, Hq, D]; key [B, Hkv, D] is RMSNormed with k_norm, rotated
 * and written to key_cache[pos_b, b]; value [B, Hkv, Dv] is written to
 * value_cache[pos_b, b] (caches [capacity, B, Hkv, D|Dv], as
 * alpx_kv_append).  pos_b = positions[b] (device int32) or `position`;
 * the IMROPE lanes are the text lanes (pos_b, pos_b, pos_b, 0)
 * (qwen35_ops.imrope_text_position, qwen35_ops.py:102-108).  All tensors
 * use `dtype`; norm weights are fp32.  Device positions outside
 * [0, capacity) skip the cache writes. */
int alpx_attention_prologue(const void* query_gate, const void* key, const void* value,
                            const float* q_norm, const float* k_norm, void* query_out,
                            void* gate_out, void* key_cache, void* value_cache, int dtype,
                            int64_t capacity, int batch, int q_heads, int kv_heads, int head_dim,
                            int value_dim, int64_t position, const int32_t* positions,
                            const int* sections, double frequency_base, float eps, void* stream);

/* One decode token of the Qwen3.5 full-attention layer after its
 * projections (qwen35_runtime.py:597-665 for one token per sequence:
 * alpx_attention_prologue followed by alpx_decode_gqa with the sigmoid
 * gate), in two launches.  Sequence b's token sits at cache row pos_b =
 * positions[b] (device int32) or, with positions null, `position`; with
 * positions, `position` bounds them (a pos_b outside [0, position] writes
 * no cache row and attends rows 0 .. min(pos_b, position)).  The split-K
 * launch forms each block's query heads from query_gate [B, Hq, 2D]
 * (RMSNorm with q_norm, IMROPE at the text lanes (pos_b, pos_b, pos_b, 0))
 * and, in the blocks whose chunk holds row pos_b, the key row from key
 * [B, Hkv, D]; the rotated key and value [B, Hkv, D] are written to row
 * pos_b of the caches [capacity, B, Hkv, D].  Attention runs over rows
 * 0 .. pos_b with `scale`; the combine multiplies by sigmoid of the gate
 * half of query_gate and writes out [B, Hq, D] in out_dtype.  The values
 * equal those of alpx_attention_prologue + alpx_decode_gqa (seq_lens =
 * pos_b + 1, length position + 1) bit for bit.  fp16 / bf16 only, key width =
 * value width in {64, 128, 256}, 16-byte aligned buffers (others:
 * ALPX_EUNSUPPORTED).  workspace: alpx_decode_workspace_bytes(batch,
 * q_heads, kv_heads, head_dim, position + 1) bytes. */
int alpx_attention_layer_step(const void* query_gate, const void* key, const void* value,
                              const float* q_norm, const float* k_norm, void* key_cache,
                              void* value_cache, void* out, void* workspace,
                              size_t workspace_bytes, int dtype, int out_dtype, int64_t capacity,
                              int batch, int q_heads, int kv_heads, int head_dim,
                              int64_t position, const int32_t* positions, const int* sections,
                              double frequency_base, float eps, float scale, void* stream);

/* alpx_attention_layer_step over a paged K/V pool (an extension, as
 * alpx_decode_gqa_paged): pages [num_pages, page_size, Hkv, D],
 * block_table [batch, max_pages] (device int32), page_size a power of two
 * of at least 32.  Sequence b's rotated key and value land at logical row
 * pos_b (row pos_b % page_size of page block_table[b][pos_b / page_size]);
 * a table entry outside [0, num_pages) writes no row (reads clamp such an
 * entry into the pool, as alpx_decode_gqa_paged does).  `position` must be
 * below max_pages * page_size.  Same launches, split plan and arithmetic as
 * alpx_attention_layer_step, so the same rows give the same output bits.
 * fp16 / bf16 pages, head_dim in {64, 128, 256} (others:
 * ALPX_EUNSUPPORTED).  workspace: alpx_decode_workspace_bytes(batch,
 * q_heads, kv_heads, head_dim, position + 1) bytes. */
int alpx_attention_layer_step_paged(const void* query_gate, const void* key, const void* value,
                                    const float* q_norm, const float* k_norm, void* key_pages,
                                    void* value_pages, const int32_t* block_table, int max_pages,
                                    int page_size, int num_pages, void* out, void* workspace,
                                    size_t workspace_bytes, int dtype, int out_dtype, int batch,
                                    int q_heads, int kv_heads, int head_dim, int64_t position,
                                    const int32_t* positions, const int* sections,
                                    double frequency_base, float eps, float scale, void* stream);

/* Workspace bytes for alpx_recurrent_step. */
size_t alpx_recurrent_step_workspace_bytes(int batch, int key_heads, int value_heads, int key_dim,
                                           int value_dim);

/* One token of the Qwen3.5 recurrent (GDN) layer after its projections,
 * fused (qwen35_numpy.py:63-131, the recurrent half of
 * qwen35_recurrent_layer, qwen35_kernels.py:349-360): conv step + SiLU of
 * current [B, C] (C = 2 Hk Dk + Hv Dv) with conv_weight (strides as
 * alpx_conv_step) and conv_history [B, K-1, C]; split into q [Hk, Dk],
 * k [Hk, Dk], v [Hv, Dv]; L2-normalised q / k; beta / log decay from
 * beta_logits, alpha_logits [B, Hv], dt_bias, ssm_a [Hv]; the GDN step on
 * state [B, Hv, Dv, Dk] (alpx_gdn_step); then out [B, Hv * Dv] =
 * gated RMSNorm with norm_weight [Dv] and gate [B, Hv * Dv].  All inputs
 * fp32 (the reference's dtype); out in out_dtype.  Two launches (state
 * rows, then norm + query/key history shift) when key_dim is a multiple of
 * 4 up to 256 and the state is 16-byte aligned, three otherwise; both give
 * bit-identical results. */
int alpx_recurrent_step(const float* current, const float* conv_weight, int64_t weight_tap_stride,
                        int64_t weight_channel_stride, float* conv_history, int conv_kernel,
                        const float* gate, const float* beta_logits, const float* alpha_logits,
                        const float* dt_bias, const float* ssm_a, const float* norm_weight,
                        float* state, void* out, void* workspace, size_t workspace_bytes,
                        int batch, int key_heads, int value_heads, int key_dim, int value_dim,
                        float eps, int out_dtype, void* stream);

/* Qwen3.5 full-attention prologue for a prefill chunk of one sequence:
 * `tokens` consecutive tokens at positions position .. position + tokens - 1
 * of cache sequence batch_index (caches [capacity, cache_batch, Hkv, D|Dv]).
 * Row t of query_gate [T, Hq, 2D], key [T, Hkv, D], value [T, Hkv, Dv] is
 * processed as alpx_attention_prologue processes one sequence's token at
 * position + t, and its key / value rows land at cache row position + t.
 * Replaces the prologue half of the reference's token-sequential prefill,
 * one Qwen35Model._attention call per token (qwen35_runtime.py:597-650,
 * driven by prefill_state, qwen35_runtime.py:777-810); the chunk then runs
 * alpx_prefill_causal over the cache and alpx_sigmoid_gate.  gate_out may
 * be null (the gate half is then not copied; alpx_attention_layer_prefill
 * reads it in place). */
int alpx_attention_prologue_chunk(const void* query_gate, const void* key, const void* value,
                                  const float* q_norm, const float* k_norm, void* query_out,
                                  void* gate_out, void* key_cache, void* value_cache, int dtype,
                                  int64_t capacity, int cache_batch, int batch_index, int tokens,
                                  int q_heads, int kv_heads, int head_dim, int value_dim,
                                  int64_t position, const int* sections, double frequency_base,
                                  float eps, void* stream);

/* A prefill chunk of the Qwen3.5 full-attention layer after its
 * projections, in two launches: the chunk prologue (alpx_attention_prologue_
 * chunk, without the gate copy: query rows into query_out [T, Hq, D], key /
 * value rows into the caches) and the causal prefill over cache rows
 * 0 .. position + t with the sigmoid gate read in place from the second
 * half of each head's query_gate row (row stride 2 D) -- what
 * alpx_attention_prologue_chunk + alpx_prefill_causal_gated compute, bit
 * for bit, without the 2 x T x Hq x D gate copy.  Replaces the reference's
 * token-sequential Qwen35Model._attention calls of a prefill
 * (qwen35_runtime.py:597-665, prefill_state qwen35_runtime.py:777-810).
 * value_dim must equal head_dim (the gate has head_dim values per head);
 * workspace as alpx_prefill_causal (only its fallback path uses it).
 *
 * query_out may be null: the prefill then forms the query rows itself from
 * query_gate (the prologue's RMSNorm and IMROPE in its query load, same
 * bits) and the prologue launch writes only the key / value rows and each
 * token's rotary (cos, sin) pairs into workspace, which must hold
 * tokens x R x 8 bytes (R = the section sum).  Needs fp16 / bf16,
 * head_dim 64, 128 or 256, R a multiple of 32 with 2 R <= head_dim,
 * 16-byte aligned query_gate, q_norm and cache rows; otherwise
 * ALPX_EUNSUPPORTED before any launch. */
int alpx_attention_layer_prefill(const void* query_gate, const void* key, const void* value,
                                 const float* q_norm, const float* k_norm, void* query_out,
                                 void* key_cache, void* value_cache, void* out, void* workspace,
                                 size_t workspace_bytes, int dtype, int out_dtype,
                                 int64_t capacity, int cache_batch, int batch_index, int tokens,
                                 int q_heads, int kv_heads, int head_dim, int64_t position,
                                 const int* sections, double frequency_base, float eps,
                                 float scale, void* stream);

/* alpx_attention_layer_prefill over a paged pool (the form without a query
 * buffer): the key / value rows of the chunk's T tokens land at logical
 * rows position .. position + T - 1 of sequence batch_index, i.e. row
 * pos % page_size of page block_table[batch_index][pos / page_size] of
 * key_pages / value_pages [num_pages, page_size, Hkv, D] (a table entry
 * outside [0, num_pages) writes no row; the prefill's reads clamp it into
 * the pool, as alpx_prefill_causal_paged does), then the gated causal
 * prefill runs over logical rows 0 .. position + t, forming the query
 * heads from query_gate itself, on the prefill's single-tile kernel: the
 * same rows give the bits of the contiguous call on that kernel (within
 * rounding of its paired kernel, which splits a heavy tile's keys over two
 * wave groups and merges them).  fp16 / bf16,
 * head_dim 64, 128 or 256, rotary sections summing to a multiple of 32
 * (at most head_dim / 2), page_size a power of two >= 64, out in dtype;
 * workspace: tokens x R x 8 bytes (R = the section sum).  Every check
 * runs before the first launch. */
int alpx_attention_layer_prefill_paged(const void* query_gate, const void* key,
                                       const void* value, const float* q_norm,
                                       const float* k_norm, void* key_pages, void* value_pages,
                                       const int32_t* block_table, int max_pages, int page_size,
                                       int num_pages, int batch_index, void* out, void* workspace,
                                       size_t workspace_bytes, int dtype, int tokens, int q_heads,
                                       int kv_heads, int head_dim, int64_t position,
                                       const int* sections, double frequency_base, float eps,
                                       float scale, void* stream);

/* Qwen3.5 recurrent-layer inputs for a prefill chunk of one sequence: the
 * depthwise causal convolution + SiLU of current [T, C] (C = 2 Hk Dk +
 * Hv Dv; weights strided as alpx_conv_step) continuing conv_history
 * [K-1, C], split into q_out / k_out [T, Hk, Dk] (L2-normalised) and
 * v_out [T, Hv, Dv] in out_dtype, and beta_out / log_decay_out [T, Hv]
 * from beta_logits / alpha_logits [T, Hv], dt_bias and ssm_a [Hv]; the
 * history then advances to the chunk's last K-1 rows.  Token t's values
 * equal those alpx_recurrent_step forms for it after tokens 0 .. t-1 (the
 * per-token chain of qwen35_numpy.py:63-131 that the reference's
 * token-sequential prefill runs, qwen35_runtime.py:777-810); the chunk
 * then runs alpx_gdn_chunk_prefill and the gated alpx_row_norm.  All
 * inputs fp32.  Two launches. */
int alpx_recurrent_prefill_prep(const float* current, const float* conv_weight,
                                int64_t weight_tap_stride, int64_t weight_channel_stride,
                                float* conv_history, int conv_kernel, const float* beta_logits,
                                const float* alpha_logits, const float* dt_bias,
                                const float* ssm_a, void* q_out, void* k_out, void* v_out,
                                float* beta_out, float* log_decay_out, int tokens, int key_heads,
                                int value_heads, int key_dim, int value_dim, float eps,
                                int out_dtype, void* stream);

/*
 * Kernel timing (measurement support, no reference counterpart: it serves
 * the roofline measurement of bench.py).  While enabled, each entry point
 * records a pair of HIP events on its launch stream around the kernel named
 * by `kernel` below; alpx_timing_read synchronises the recorded events and
 * returns the summed duration and launch count.  alpx_timing_enable clears
 * the totals.  Timing adds two event records per launch.
 */
enum alpx_timed_kernel {
  ALPX_T_KV_APPEND = 0,
  ALPX_T_DECODE = 1,
  ALPX_T_DECODE_COMBINE = 2,
  ALPX_T_PREFILL = 3,
  ALPX_T_GDN_CHUNK = 4,
  ALPX_T_GDN_STEP = 5,
  ALPX_T_AUX = 6,
  ALPX_T_LAYER = 7,          /* layer primitives and the attention prologue */
  ALPX_T_RECURRENT_STEP = 8  /* the whole fused recurrent-layer step */
};
#define ALPX_TIMING_KERNELS 9
int alpx_timing_enable(int enable);
int alpx_timing_read(int kernel, double* total_ms, int64_t* launches);

/*
 * Kernel-choice overrides (test and A/B measurement support, no reference
 * counterpart).  Each starts from its environment variable, read once when
 * the library loads -- ALPX_DECODE_GENERIC, ALPX_PREFILL_GENERIC,
 * ALPX_PREFILL_KERNEL (single | pair | shared), ALPX_GDN_SEQUENTIAL,
 * ALPX_RECURRENT_UNFUSED -- and afterwards changes only through
 * alpx_set_override: no entry point reads the environment per call.
 * alpx_set_override returns the previous value, or ALPX_EINVAL for an
 * unknown override or value; alpx_get_override returns the value or
 * ALPX_EINVAL.  Set them between calls, not while calls are in flight on
 * another host thread.
 */
enum alpx_override {
  ALPX_OVERRIDE_DECODE_GENERIC = 0,    /* 1: decode on the VALU split kernel */
  ALPX_OVERRIDE_PREFILL_GENERIC = 1,   /* 1: prefill on the split-K decode path */
  ALPX_OVERRIDE_PREFILL_KERNEL = 2,    /* 0 auto, 1 single, 2 paired, 3 shared-stream */
  ALPX_OVERRIDE_GDN_SEQUENTIAL = 3,    /* 1: chunked GDN runs token by token */
  ALPX_OVERRIDE_RECURRENT_UNFUSED = 4  /* 1: recurrent step in three launches */
};
#define ALPX_OVERRIDES 5
int alpx_set_override(int which, int value);
int alpx_get_override(int which);

#ifdef __cplusplus
}
#endif

#endif /* ALPX_H */
