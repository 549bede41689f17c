/*
 * msattn.h -- C ABI of libmsattn.so, the MI355X (gfx950) paged-attention library.
 *
 * Every entry point takes plain device pointers, element strides and sizes, a
 * dtype code and a HIP stream (passed as void*, a hipStream_t). No entry point
 * allocates device memory except where stated, none throws, and all of them
 * return an msattn_status code. Work is enqueued on the given stream, so a
 * caller that is capturing that stream into a hipGraph records it.
 *
 * Layouts (all "contiguous" means row-major, innermost dimension last):
 *   query / out     [batch, q_len, num_heads, head_dim]                 contiguous
 *   k_cache/v_cache [num_blocks, block_size, num_kv_heads, head_dim]    strided, last dim contiguous
 *   block_table     int32 [batch, table_width]                          contiguous
 *   context_lens    int32 [batch]
 *   kv (write_kv)   [batch, tokens, num_kv_heads, head_dim]             contiguous
 *
 * Query heads h = kvh * group + g (group = num_heads / num_kv_heads) all read KV
 * head kvh. Query token i of row b sits at absolute position
 * q_pos = context_lens[b] - q_len + i; it attends to key positions k with
 * k < context_lens[b], k <= q_pos when causal, and k > q_pos - window when
 * window > 0. A row whose key set is empty produces zeros. Block-table entries
 * outside [0, num_blocks) are treated as holes: their tokens are neither read
 * nor written.
 */
#ifndef MSATTN_H
#define MSATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSATTN_ABI_VERSION 1

typedef enum msattn_dtype {
  MSATTN_F32 = 0,
  MSATTN_F16 = 1,
  MSATTN_BF16 = 2,
  MSATTN_FP8_E4M3 = 3, /* OCP float8 e4m3fn (torch.float8_e4m3fn) */
} msattn_dtype;

typedef enum msattn_status {
  MSATTN_OK = 0,
  MSATTN_ERR_INVALID_ARG = 1,  /* null pointer, bad size, misaligned pointer or stride */
  MSATTN_ERR_UNSUPPORTED = 2,  /* valid request outside the compiled kernel set */
  MSATTN_ERR_WORKSPACE = 3,    /* workspace smaller than msattn_workspace_bytes() */
  MSATTN_ERR_HIP = 4,          /* a HIP launch reported an error */
} msattn_status;

/* Kernel routes of msattn_paged_attention (msattn_paged_attention_route). */
typedef enum msattn_route {
  MSATTN_ROUTE_PREFILL = 1,          /* chunked-prefill MFMA kernel; output written directly */
  MSATTN_ROUTE_PARTITION_FUSED = 2,  /* MFMA partition kernel, split-K merged in-kernel */
  MSATTN_ROUTE_PARTITION = 3,        /* MFMA partition kernel, then the merge kernel */
  MSATTN_ROUTE_STREAMK = 4,          /* MFMA stream-K decode kernel, then the merge kernel */
  MSATTN_ROUTE_GENERIC = 5,          /* generic VALU kernel, then the merge kernel */
  MSATTN_ROUTE_PREFILL_STREAMK = 6,  /* prefill kernel, stream-K schedule (merge in-kernel) */
} msattn_route;

/* ABI version (MSATTN_ABI_VERSION). No reference counterpart. */
int msattn_abi_version(void);

/* Static, human-readable text for a status code. No reference counterpart. */
const char* msattn_status_string(int status);

/*
 * Context partition (tokens) the library uses for this geometry. The split-K
 * decomposition cuts every row's context into ceil(context_len / partition)
 * slices; max_context bounds every context_lens entry.
 * Replaces the host-side split policy of kernels/paged_attn_triton.py:80-84
 * (num_splits_for) and :313-314 (splits from lens.max()/lens.min()), which need
 * a device->host read; this one depends on sizes only, so it is capture-safe.
 */
int msattn_partition_tokens(int batch, int q_len, int num_heads, int num_kv_heads,
                            int head_dim, int max_context);

/*
 * Bytes of caller-owned device workspace msattn_paged_attention needs (a size
 * that depends on the geometry only). Replaces the per-call torch.empty partial buffers of
 * kernels/paged_attn_triton.py:320-323. A workspace must be all zeros when it is first
 * used (allocate it zeroed once): its header holds the arrival counters of the in-kernel
 * merge at a fixed offset, and every call leaves them zero, so one workspace serves any
 * sequence of calls and geometries that fit it. Calls that share a workspace must not
 * overlap in time.
 */
size_t msattn_workspace_bytes(int batch, int q_len, int num_heads, int num_kv_heads,
                              int head_dim, int max_context);

/*
 * Paged attention forward: out = softmax(scale * q k^T + mask) v over the paged
 * cache, for any q_len (decode q_len == 1, chunked prefill q_len > 1).
 * Replaces PagedAttention.forward (miniserve/attention.py:205-250: gather
 * :155-171, mask :135-153, GQA expansion :245-247, SDPA :249) and the split-K
 * launcher flash_decode (kernels/paged_attn_triton.py:286-344).
 * cache_*_stride are in elements and shared by k_cache and v_cache. The MFMA
 * kernels address a 16-token tile with 32-bit byte offsets; caches whose tile span
 * (15 * cache_slot_stride + head_dim elements) reaches 2^31 bytes take the generic
 * kernel, which addresses with 64-bit offsets.
 * max_context bounds context_lens (entries above it are clamped to it) and
 * sizes the launch grid; pass table_width * block_size for a capture-safe call.
 * window <= 0 means no sliding window. q_dtype and kv_dtype may differ: the cache is
 * cast to the query type as it is read (exact when widening, round to nearest even when
 * narrowing), as the reference casts the gathered K/V to query.dtype
 * (miniserve/attention.py:240-241). head_dim may be any even size up to 256. Decode
 * (q_len 1, or at most 16 query rows per KV head) runs on the MFMA kernels for a bf16/fp16
 * query over a cache of its type, fp8 e4m3 or fp32, and for an fp32 query over any cache
 * (head_dim 64 or 128, 16-byte aligned query, cache pointers and strides on 16-byte
 * boundaries, block_size a multiple of 16); an fp32 query's chunked prefill (more than 16
 * query rows per KV head) also runs there. Other pairs and shapes take the generic kernel,
 * which needs only element-aligned caches. msattn_paged_attention_route names the route.
 * Runs msattn_paged_attention_partials followed by msattn_merge_partials, except:
 * chunked prefill on the MFMA kernel (bf16/fp16 query 16-byte aligned, output 8-byte
 * aligned, cache of the query's type, fp8 e4m3 or fp32, head_dim 64 or 128, more than 16
 * query rows per KV head, and either more than 64 rows per KV head or enough
 * (sequence, KV head) pairs to fill the device; fewer go to the partition kernel, which
 * splits their keys over more workgroups), which writes the output directly; and decodes on the MFMA
 * partition kernel (those below the stream-K threshold, with batch x num_kv_heads x row
 * tiles <= 4096), which merge in-kernel in one launch: the last partition of each
 * (sequence, KV head, row tile) to finish folds the others' partials into `out`, and a
 * sequence of one partition writes `out` directly. The partials kernel's rounding and
 * the fold are those of the two-launch path, with the fold's sums in another order.
 * A prefill-kernel launch whose tasks (row blocks of 128 x KV heads x sequences) would
 * leave CUs idle in one-task-per-workgroup rounds runs stream-K when a cost model in sizes
 * only predicts it faster and the workspace is msattn_workspace_bytes() or more: one
 * workgroup per CU, each an equal share of all tasks' key steps, then a fold launch that
 * merges each task split between workgroups (its rows spread over many workgroups); the
 * fold sums the pieces in another order than one workgroup would.
 */
int msattn_paged_attention(const void* query, const void* k_cache, const void* v_cache,
                           int64_t cache_block_stride, int64_t cache_slot_stride,
                           int64_t cache_head_stride, const int32_t* block_table,
                           const int32_t* context_lens, void* out, void* workspace,
                           size_t workspace_bytes, int batch, int q_len, int num_heads,
                           int num_kv_heads, int head_dim, int block_size, int num_blocks,
                           int table_width, int max_context, int causal, int window,
                           float scale, int q_dtype, int kv_dtype, void* stream);

/*
 * msattn_paged_attention without the workspace arguments, for callers that cannot
 * allocate (code under hipGraph capture that must not call hipMalloc, tight serving
 * loops, harnesses that forbid allocation). No counterpart in the reference, whose
 * launcher allocates its partials per call (kernels/paged_attn_triton.py:320-323).
 * Same arguments, results and errors as msattn_paged_attention, with the same kernels;
 * the split-K partials go to a scratch array of MSATTN_NOALLOC_SCRATCH_BYTES that the
 * library holds on each device it runs on (allocated with the library's code object,
 * kept until the process ends); its address is looked up on the first call on a device.
 * A call whose msattn_workspace_bytes exceeds that size runs a chunked prefill on the
 * prefill kernel when that kernel can take it (it needs no scratch; this includes
 * chunked prefills msattn_paged_attention would send to the partition kernel), and
 * otherwise returns MSATTN_ERR_WORKSPACE; it calls no allocator. Every call on one device shares that device's scratch: calls that overlap
 * in time on one device (two streams, two threads) race and must be serialised by the
 * caller. The scratch keeps the last call's contents; nothing in it needs clearing.
 */
#define MSATTN_NOALLOC_SCRATCH_BYTES (64u << 20)
int msattn_paged_attention_noalloc(const void* query, const void* k_cache, const void* v_cache,
                                   int64_t cache_block_stride, int64_t cache_slot_stride,
                                   int64_t cache_head_stride, const int32_t* block_table,
                                   const int32_t* context_lens, void* out, int batch, int q_len,
                                   int num_heads, int num_kv_heads, int head_dim, int block_size,
                                   int num_blocks, int table_width, int max_context, int causal,
                                   int window, float scale, int q_dtype, int kv_dtype,
                                   void* stream);

/*
 * The kernel route (msattn_route) that msattn_paged_attention takes for a call with these
 * pointers, strides and sizes and a workspace of workspace_bytes (pass
 * MSATTN_NOALLOC_SCRATCH_BYTES for msattn_paged_attention_noalloc), written to *route.
 * The choice depends on sizes, types and alignment only (capture-safe), never on the
 * context lengths' values. Returns MSATTN_ERR_WORKSPACE when the call would need more
 * workspace than workspace_bytes, MSATTN_ERR_INVALID_ARG for an invalid geometry. No
 * reference counterpart: the reference has one path per backend
 * (miniserve/attention.py:231-235); this library picks among its kernels by shape.
 */
int msattn_paged_attention_route(const void* query, const void* out, const void* k_cache,
                                 const void* v_cache, int64_t cache_block_stride,
                                 int64_t cache_slot_stride, int64_t cache_head_stride, int batch,
                                 int q_len, int num_heads, int num_kv_heads, int head_dim,
                                 int block_size, int max_context, int q_dtype, int kv_dtype,
                                 size_t workspace_bytes, int* route);

/*
 * msattn_paged_attention for decode (q_len == 1) with rotate-half RoPE applied to
 * the query inside the attention kernels: row b's query becomes
 * q * cos[p] + rotate_half(q) * sin[p], p = position[b] (clamped to
 * [0, max_position)), computed in fp32 and rounded to q_dtype, then attends as
 * msattn_paged_attention. rope_cos / rope_sin: fp32 [max_position, head_dim],
 * 16-byte aligned; position: int32 [batch] on the device. Replaces the fused-RoPE
 * branch of the split kernel (kernels/paged_attn_triton.py:211-220) and of
 * flash_decode_reference (:135-139); the rotation is miniserve/attention.py:41-62.
 * Returns MSATTN_ERR_UNSUPPORTED for q_len != 1, as the reference's decode-only path.
 */
int msattn_paged_attention_rope(const void* query, const void* k_cache, const void* v_cache,
                                int64_t cache_block_stride, int64_t cache_slot_stride,
                                int64_t cache_head_stride, const int32_t* block_table,
                                const int32_t* context_lens, void* out, void* workspace,
                                size_t workspace_bytes, int batch, int q_len, int num_heads,
                                int num_kv_heads, int head_dim, int block_size, int num_blocks,
                                int table_width, int max_context, int causal, int window,
                                float scale, int q_dtype, int kv_dtype, const float* rope_cos,
                                const float* rope_sin, const int32_t* position,
                                int max_position, void* stream);

/*
 * First half of msattn_paged_attention: writes the split-K partials (running
 * max m, sum l and unnormalised accumulator per slice of context) into the
 * workspace, m in base-2 units (m = max of scale * log2(e) * q.k). The workspace
 * is opaque to the caller: a header naming the layout the launch chose (one slot
 * per context partition, closed by an end marker; or, for large decodes, stream-K
 * pieces located through a prefix sum of per-sequence tiles), then float (m, l)
 * pairs and float accumulators, each region 256-byte aligned. Only
 * msattn_merge_partials reads it, for the same geometry. Replaces _split_kernel
 * (kernels/paged_attn_triton.py:176-248).
 */
int msattn_paged_attention_partials(const void* query, const void* k_cache, const void* v_cache,
                                    int64_t cache_block_stride, int64_t cache_slot_stride,
                                    int64_t cache_head_stride, const int32_t* block_table,
                                    const int32_t* context_lens, void* workspace,
                                    size_t workspace_bytes, int batch, int q_len, int num_heads,
                                    int num_kv_heads, int head_dim, int block_size,
                                    int num_blocks, int table_width, int max_context, int causal,
                                    int window, float scale, int q_dtype, int kv_dtype,
                                    void* stream);

/*
 * Second half of msattn_paged_attention: log-sum-exp merge of the partials in
 * `workspace` into `out` (q_dtype). Rows with no key get zeros. The geometry must
 * be the one the partials call was given; context_lens is that call's array.
 * Replaces _merge_kernel (kernels/paged_attn_triton.py:250-284).
 */
int msattn_merge_partials(const void* workspace, size_t workspace_bytes,
                          const int32_t* context_lens, void* out, int batch, int q_len,
                          int num_heads, int num_kv_heads, int head_dim, int max_context,
                          int q_dtype, void* stream);

/*
 * Workspace bytes of msattn_paged_attention_prefix (at least msattn_workspace_bytes
 * of the same decode geometry); 0 for an invalid geometry. No reference counterpart.
 */
size_t msattn_prefix_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_context, int prefix_pages);

/*
 * Cascade decode (q_len == 1, causal, no window) over block tables whose first
 * prefix_pages entries are the same physical pages in every row, as
 * RadixPrefixCache.match hands them out (miniserve/prefix_cache.py:66-96) and the
 * scheduler forks them into each request's table (miniserve/scheduler.py:146-151).
 * Same result as msattn_paged_attention(q_len = 1, causal = 1, window = 0) within
 * float rounding. The shared pages are read once per KV head for the whole batch
 * (table row 0 names them) by one pass that takes every sequence's query as a row;
 * a second pass reads each sequence's own keys from prefix_pages * block_size on;
 * the merge folds both. A row whose context ends inside the prefix sees only its
 * own length. Types or head sizes without the cascade kernels (anything but a bf16 or
 * fp16 query over a cache of its type or of fp8 e4m3, head_dim 64 or 128, block_size a
 * multiple of 16), and
 * prefix_pages == 0, run msattn_paged_attention. The reference has no cascade
 * kernel: its decode re-reads the shared pages per sequence
 * (miniserve/attention.py:155-171).
 */
int msattn_paged_attention_prefix(const void* query, const void* k_cache, const void* v_cache,
                                  int64_t cache_block_stride, int64_t cache_slot_stride,
                                  int64_t cache_head_stride, const int32_t* block_table,
                                  const int32_t* context_lens, void* out, void* workspace,
                                  size_t workspace_bytes, int batch, int num_heads,
                                  int num_kv_heads, int head_dim, int block_size, int num_blocks,
                                  int table_width, int max_context, int prefix_pages, float scale,
                                  int q_dtype, int kv_dtype, void* stream);

/*
 * Scatter new keys/values into the paged cache: for row b, token t,
 * pos = starts[b] + t, cache[table[b, pos / block_size], pos % block_size] = kv[b, t]
 * converted to kv_dtype (round to nearest even). Replaces PagedAttention.write_kv
 * (miniserve/attention.py:111-133). Tokens whose page is a hole are skipped.
 */
int msattn_write_kv(void* k_cache, void* v_cache, int64_t cache_block_stride,
                    int64_t cache_slot_stride, int64_t cache_head_stride, const void* k,
                    const void* v, const int32_t* block_table, const int32_t* starts,
                    int batch, int tokens, int num_kv_heads, int head_dim, int block_size,
                    int num_blocks, int table_width, int src_dtype, int kv_dtype,
                    void* stream);

/*
 * Decode with the new token appended: msattn_write_kv of k_new / v_new at position
 * context_lens[b] - 1 of each row (rows with context_lens[b] <= 0 write nothing; holes
 * are skipped), followed by msattn_paged_attention (q_len 1, causal) over context_lens.
 * k_new / v_new are contiguous [batch, 1, num_kv_heads, head_dim] in the query dtype,
 * the token each row appends this step; context_lens already count it. With a bf16/fp16
 * query, at most 8 query rows per KV head and k_new and v_new 16-byte aligned, the append
 * runs inside the decode launch where the call takes the partition kernel merging
 * in-kernel (MSATTN_ROUTE_PARTITION_FUSED) or the stream-K kernel over a cache of 2 or 4
 * byte elements (MSATTN_ROUTE_STREAMK): the wave whose work holds the new position writes
 * the rows (cast to the cache type as msattn_write_kv casts them) and uses the same values
 * in place of the cache's row, so the output and the caches equal those of the two calls
 * bit for bit. Other routes run the two calls. No reference
 * counterpart as one call: the reference runner makes these two calls per layer
 * (miniserve/model_runner.py:70-76, attention.py:111-133 and 205-250); this entry
 * point is for callers, such as a bucketed decode graph, that want one launch per layer.
 */
int msattn_paged_attention_append(const void* query, const void* k_new, const void* v_new,
                                  void* k_cache, void* v_cache, int64_t cache_block_stride,
                                  int64_t cache_slot_stride, int64_t cache_head_stride,
                                  const int32_t* block_table, const int32_t* context_lens,
                                  void* out, void* workspace, size_t workspace_bytes, int batch,
                                  int num_heads, int num_kv_heads, int head_dim, int block_size,
                                  int num_blocks, int table_width, int max_context, int window,
                                  float scale, int q_dtype, int kv_dtype, void* stream);

/*
 * Block-table gather: out[b, p] = cache[table[b, p / block_size], p % block_size]
 * for p < context_lens[b]; positions p >= context_lens[b] read page 0 (as the
 * reference does), holes give zero rows. out is [batch, max_context,
 * num_kv_heads, head_dim] in the cache dtype, bytes copied unchanged.
 * Replaces PagedAttention._gather (miniserve/attention.py:155-171); used to
 * prove the kernels' page addressing bit-exact.
 */
int msattn_gather_kv(const void* cache, int64_t cache_block_stride, int64_t cache_slot_stride,
                     int64_t cache_head_stride, const int32_t* block_table,
                     const int32_t* context_lens, void* out, int batch, int max_context,
                     int num_kv_heads, int head_dim, int block_size, int num_blocks,
                     int table_width, int kv_dtype, void* stream);

/*
 * Measurement helper, with no counterpart in the reference: one launch of a plain
 * streaming-read kernel over `bytes` (a multiple of 16) of device memory at `buf`
 * (16-byte aligned), each workgroup reading a contiguous 64 KiB chunk with nontemporal
 * 16-byte loads. Timing it
 * gives the HBM read rate a plain kernel reaches on the device, beside which the
 * decode kernels' rates are reported. `sink` is device memory of
 * ceil(bytes / 65536) uint32 entries that the kernel may write (it keeps the loads
 * from being dropped); its contents carry no meaning.
 */
int msattn_probe_stream_read(const void* buf, size_t bytes, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSATTN_H */
