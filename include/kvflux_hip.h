/*
 * kvflux_hip.h - C ABI of the MI355X (gfx950) paged-KV data path.
 *
 * Everything that touches the GPU goes through these functions: the C++17
 * control plane (kvflux::v2, same API as the reference) calls them, and so
 * can any other host language through its FFI. No C++ or HIP types cross
 * the boundary: plain pointers, sizes, int status codes. Streams are passed
 * as `void*` holding a hipStream_t (NULL = the default stream).
 *
 * Device pointers are expected to be on the current device (see
 * kvflux_set_device). Every hot-path entry point only enqueues work on
 * `stream` and returns; it does not synchronise.
 *
 * Cache layout (reference include/kvflux/v2/paged_kv_layout.h:10-11):
 *   key_cache  [num_blocks][num_kv_heads][block_size][head_size]
 *   value_cache: same shape; element type `dtype`.
 * Page ids and slot numbers are 64-bit (reference PhysicalBlockID = size_t,
 * PhysicalSlot = uint64_t). Device kernels skip (never dereference) page ids
 * >= num_blocks and slots >= num_blocks * block_size.
 */
#ifndef KVFLUX_HIP_H
#define KVFLUX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the C++ layer maps each onto the exception type the
 * reference throws (reference src/v2/paged_kv_write.cu:15-19 and callers). */
enum kvflux_status {
    KVFLUX_OK = 0,
    KVFLUX_ERR_INVALID_ARGUMENT = 1, /* std::invalid_argument */
    KVFLUX_ERR_OUT_OF_RANGE = 2,     /* std::out_of_range */
    KVFLUX_ERR_OVERFLOW = 3,         /* std::overflow_error */
    KVFLUX_ERR_RUNTIME = 4,          /* std::runtime_error (HIP runtime failure) */
    KVFLUX_ERR_UNSUPPORTED = 5       /* shape or dtype a kernel does not handle */
};

/* Same values as kvflux::DType (reference include/kvflux/kv_layout.h:7). */
enum kvflux_dtype { KVFLUX_DTYPE_F16 = 0, KVFLUX_DTYPE_BF16 = 1, KVFLUX_DTYPE_F32 = 2 };

/* Message of the last failing call on this thread ("" if none). */
const char* kvflux_last_error(void);
int kvflux_abi_version(void);

/* ---------------------------------------------------------------------------
 * Runtime plumbing. These replace the CUDA runtime calls the reference makes
 * directly: cudaMalloc of the arena (reference src/gpu_memory_pool.cpp:38-50),
 * the DeviceGuard (src/v2/paged_kv_write.cu:28-37), cudaPointerGetAttributes
 * (src/v2/paged_kv_write.cu:52-60), metadata uploads (paged_kv_write.cu:122-124)
 * and cudaStreamSynchronize (paged_kv_write.cu:138).
 * ------------------------------------------------------------------------- */
int kvflux_device_count(int* count);
int kvflux_get_device(int* device);
int kvflux_set_device(int device);
int kvflux_device_malloc(void** ptr, size_t bytes);   /* on the current device */
int kvflux_device_free(void* ptr);
/* Page-locked host memory, mapped into the device address space. */
int kvflux_host_malloc_pinned(void** ptr, size_t bytes);
int kvflux_host_free_pinned(void* ptr);
/* Device-side address of a pointer returned by kvflux_host_malloc_pinned
 * (what kernels must be given to read or write that host memory). */
int kvflux_host_device_pointer(void* host_ptr, void** device_ptr);
/* *device = owning device id if `ptr` is device memory, else -1 (never fails
 * for host pointers; clears any sticky runtime error it provokes). */
int kvflux_pointer_device(const void* ptr, int* device);
/* Asynchronous copy in any direction (unified addressing). */
int kvflux_memcpy_async(void* dst, const void* src, size_t bytes, void* stream);
/* Synchronous copy in any direction (pageable host memory allowed). */
int kvflux_memcpy(void* dst, const void* src, size_t bytes);
/* Byte fill with a kernel (no memset node, safe under graph capture). */
int kvflux_fill_bytes(void* dst, int value, size_t bytes, void* stream);
int kvflux_stream_create(void** stream);
int kvflux_stream_destroy(void* stream);
int kvflux_stream_synchronize(void* stream);
int kvflux_device_synchronize(void);
int kvflux_event_create(void** event);
int kvflux_event_destroy(void* event);
int kvflux_event_record(void* event, void* stream);
int kvflux_event_elapsed_ms(float* ms, void* start, void* stop);
int kvflux_event_synchronize(void* event);
/* *complete = 1 when all work before the event has finished, else 0. */
int kvflux_event_query(void* event, int* complete);
/* Work enqueued on `stream` after this call waits for `event`. */
int kvflux_stream_wait_event(void* stream, void* event);

/* ---------------------------------------------------------------------------
 * Hot path 1: paged KV write (scatter by slot).
 * Replaces paged_kv_write_kernel + launch_write
 * (reference src/v2/paged_kv_write.cu:62-97), called from write_paged_kv
 * (paged_kv_write.cu:101-139).
 *   key_new/value_new: [num_tokens][num_kv_heads][head_size] of `dtype`.
 *   slots: device uint64 [num_tokens]; slot = page * block_size + offset.
 * Raw bit copy. Duplicate slots are the caller's responsibility (the C++
 * layer rejects them, as the reference does).
 * ------------------------------------------------------------------------- */
int kvflux_write_paged_kv(void* key_cache, void* value_cache, uint64_t num_blocks,
                          uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size,
                          int dtype, const void* key_new, const void* value_new,
                          const uint64_t* slots, uint64_t num_tokens, void* stream);

/* ---------------------------------------------------------------------------
 * Hot path 2: paged KV gather (BlockTable-driven read).
 * Replaces paged_kv_read_kernel + launch_read
 * (reference src/v2/paged_kv_read.cu:67-102), called from read_paged_kv
 * (paged_kv_read.cu:106-155), generalised to many sequences per launch.
 *   block_table: device uint64 [num_seqs][max_blocks_per_seq] (the reference's
 *                BatchBlockTable layout, include/kvflux/v2/batch_block_table.h:14-22)
 *   seq_lens:    device uint64 [num_seqs]
 *   out_offsets: device uint64 [num_seqs], first output token of each sequence
 *   max_seq_len: upper bound of seq_lens (sizes the grid)
 *   key_out/value_out: [sum of lengths][num_kv_heads][head_size] of `dtype`.
 * Only the valid tokens of a tail page are read or written.
 * ------------------------------------------------------------------------- */
int kvflux_gather_paged_kv(const void* key_cache, const void* value_cache,
                           uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                           uint64_t head_size, int dtype, const uint64_t* block_table,
                           uint64_t max_blocks_per_seq, const uint64_t* seq_lens,
                           const uint64_t* out_offsets, uint64_t num_seqs,
                           uint64_t max_seq_len, void* key_out, void* value_out,
                           void* stream);

/* kvflux_gather_paged_kv_live: the same gather with one workgroup per live
 * page. Replaces the same reference kernel (src/v2/paged_kv_read.cu:67-102,
 * whose grid is sized from the element count); used by the C++ read_paged_kv
 * and read_paged_kv_batch.
 *   page_starts: device uint64 [num_seqs], the exclusive scan of the
 *                per-sequence page counts: page_starts[i] =
 *                sum over j < i of ceil(seq_lens[j] / block_size)
 *   total_pages: sum of ceil(seq_lens[j] / block_size) over all sequences
 * Other arguments and the result as for kvflux_gather_paged_kv. No workgroup
 * is launched for a page past a sequence's end, whatever the spread of the
 * lengths. */
int kvflux_gather_paged_kv_live(const void* key_cache, const void* value_cache,
                                uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                                uint64_t head_size, int dtype, const uint64_t* block_table,
                                uint64_t max_blocks_per_seq, const uint64_t* seq_lens,
                                const uint64_t* out_offsets, const uint64_t* page_starts,
                                uint64_t num_seqs, uint64_t total_pages, void* key_out,
                                void* value_out, void* stream);

/* ---------------------------------------------------------------------------
 * Hot path 3a: paged attention, split-K (flash-decoding) kernel, FP32 math.
 * Replaces paged_attention_batch_kernel (reference src/v2/paged_attention.cu:130-153,
 * 173-189) and, for query_tokens small, paged_attention_kernel (:108-128, 155-171).
 * Rows: query/output device float [num_rows][query_heads][head_size].
 *   seq_lens != NULL: row r attends to tokens [0, seq_lens[r]) of table row r
 *                     (batch decode; kv_len = max over seq_lens).
 *   seq_lens == NULL: every row uses table row 0 and row r attends to tokens
 *                     [0, kv_len - num_rows + r] (causal trailing queries of one
 *                     sequence, reference paged_attention.cu:123).
 * scale = 1/sqrt(head_size). query_heads % num_kv_heads == 0.
 * workspace: device scratch of at least kvflux_paged_attention_workspace_size()
 *   bytes (no initialisation needed). Calls that share a workspace must be
 *   ordered (same stream).
 * Rows longer than one split take two launches: the split kernel and a
 * combine kernel that merges the split partials in ascending split order, so
 * results are deterministic. A split is 512 tokens; the block-size-16 kernel
 * (power-of-two block_size 1 to 256; head_size 64/128, and 256 with 16-bit
 * caches; any GQA group, as items of up to 16 heads) uses 512 to 4096 tokens
 * (pages of bs < 16 tokens: at most 256 * bs, and 256 at bs = 1), the
 * largest that leaves 8 work items per resident workgroup for num_rows rows
 * of kv_len tokens. The workspace is sized for 512-token splits (256 at
 * block_size 1), enough for either. Any group is accepted (num_rows and
 * kv_len below 2^32, at most 65535 kv heads); shapes outside these take the
 * split kernel (head_size 64/80/96/128/256) or a generic kernel (any other
 * head_size up to 512).
 * ------------------------------------------------------------------------- */
int kvflux_paged_attention_workspace_size(uint64_t num_rows, uint64_t kv_len,
                                          uint64_t num_kv_heads, uint64_t query_heads,
                                          uint64_t block_size, uint64_t head_size,
                                          size_t* bytes);
int kvflux_paged_attention(const void* key_cache, const void* value_cache,
                           uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                           uint64_t head_size, int dtype, const uint64_t* block_table,
                           uint64_t max_blocks_per_seq, const uint64_t* seq_lens,
                           uint64_t kv_len, uint64_t num_rows, uint64_t query_heads,
                           const float* query, float* output, void* workspace,
                           size_t workspace_bytes, void* stream);

/* kvflux_paged_attention_noalloc: kvflux_paged_attention without a workspace
 * argument and without any device allocation, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc, harnesses with a fixed memory budget). No counterpart in the
 * reference, whose paged_attention_batch allocates its metadata per call
 * (src/v2/paged_attention.cu:287-292). Same kernels, same results (bit for
 * bit) as kvflux_paged_attention. The chunk partials live in a static device
 * array of KVFLUX_NOALLOC_SCRATCH_BYTES that each device holds until the
 * process ends; a call whose partials exceed it fails with
 * KVFLUX_ERR_UNSUPPORTED (at the 128-row, 32K-token, 32 q-head, head_size 128
 * decode batch the partials take 17 MB). All calls on one device share that
 * array: calls that overlap on one device (different streams, or threads)
 * race and must be serialised by the caller. */
#define KVFLUX_NOALLOC_SCRATCH_BYTES (32ull << 20)
int kvflux_paged_attention_noalloc(const void* key_cache, const void* value_cache,
                                   uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                                   uint64_t head_size, int dtype, const uint64_t* block_table,
                                   uint64_t max_blocks_per_seq, const uint64_t* seq_lens,
                                   uint64_t kv_len, uint64_t num_rows, uint64_t query_heads,
                                   const float* query, float* output, void* stream);

/* ---------------------------------------------------------------------------
 * Hot path 3b: causal paged prefill on MFMA.
 * Replaces paged_attention_kernel for a whole-prompt call
 * (reference src/v2/paged_attention.cu:108-128, 193-246, query_tokens = Tq).
 * One sequence: block_table device uint64 [ceil(kv_len / block_size)],
 * query i attends to tokens [0, kv_len - query_tokens + i].
 * F16/BF16 caches: Q is rounded to the cache dtype and the softmax weights to
 * the cache dtype before the MFMA products; accumulation and softmax are
 * FP32. F32 caches: FP32 MFMAs on Q, K, V and the weights as they are (the
 * 1e-5 contract of kvflux_paged_prefill_exact, head_size 64 or 128).
 * KVFLUX_ERR_UNSUPPORTED unless head_size is 64, 128 or 256 (F32: 64 or
 * 128), block_size is a power of two up to 256 and kv_len is below 2^31.
 * Any GQA group query_heads / num_kv_heads: up to 512 at head_size 64, 256 at
 * 128 and 128 at 256 and in the exact and F32 variants in one launch, a
 * larger group as one launch per sub-group of heads (its largest divisor that
 * one launch takes).
 * ------------------------------------------------------------------------- */
int kvflux_paged_prefill(const void* key_cache, const void* value_cache,
                         uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                         uint64_t head_size, int dtype, const uint64_t* block_table,
                         uint64_t num_table_blocks, uint64_t kv_len, uint64_t query_tokens,
                         uint64_t query_heads, const float* query, float* output,
                         void* stream);

/* kvflux_paged_prefill_split: the same call with a device workspace, which
 * lets the kernel split the key range of each (query block, kv head) over
 * several workgroups when the call alone would not fill the GPU (a short
 * query block against a long prefix, as in chunked prefill), merged by a
 * second kernel. Same results within the bound (2e-2); same errors, plus
 * KVFLUX_ERR_INVALID_ARGUMENT for a workspace smaller than
 * kvflux_paged_prefill_workspace_size gives (0 bytes: no split is used, and
 * the workspace may be NULL). That size serves every variant of the call
 * (rounded, exact and FP32-cache kernels). No counterpart in the reference, whose
 * paged_attention_kernel runs one thread per output element
 * (src/v2/paged_attention.cu:108-128); the C++ paged_attention uses it. */
int kvflux_paged_prefill_workspace_size(uint64_t num_kv_heads, uint64_t head_size, uint64_t kv_len,
                                        uint64_t query_tokens, uint64_t query_heads, size_t* bytes);
int kvflux_paged_prefill_split(const void* key_cache, const void* value_cache,
                               uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                               uint64_t head_size, int dtype, const uint64_t* block_table,
                               uint64_t num_table_blocks, uint64_t kv_len, uint64_t query_tokens,
                               uint64_t query_heads, const float* query, float* output,
                               void* workspace, uint64_t workspace_bytes, void* stream);

/* kvflux_paged_prefill_exact: kvflux_paged_prefill_split with the reference's
 * arithmetic contract (1e-5 against a double-precision evaluation,
 * reference tests/paged_attention_test.cu:128) instead of 2e-2: Q (scale
 * folded in) and the softmax weights enter the MFMAs as three 16-bit parts
 * each, so every product is exact in FP32, and the row sums are FP32 sums of
 * the weights. About three times the MFMA work of kvflux_paged_prefill_split.
 * F32 caches run the FP32-MFMA prefill, as in kvflux_paged_prefill_split.
 * Same arguments, workspace and errors, except that head_size must be 64 or
 * 128 (256: KVFLUX_ERR_UNSUPPORTED). Replaces paged_attention_kernel
 * (reference src/v2/paged_attention.cu:108-128, 193-246) for the
 * reference's own paged_attention signature. */
int kvflux_paged_prefill_exact(const void* key_cache, const void* value_cache,
                               uint64_t num_blocks, uint64_t num_kv_heads, uint64_t block_size,
                               uint64_t head_size, int dtype, const uint64_t* block_table,
                               uint64_t num_table_blocks, uint64_t kv_len, uint64_t query_tokens,
                               uint64_t query_heads, const float* query, float* output,
                               void* workspace, uint64_t workspace_bytes, void* stream);

/* kvflux_paged_prefill_batch: kvflux_paged_prefill over num_seqs sequences in
 * one launch (a prefill batch). Sequence i: table row i of block_table
 * (device uint64 [num_seqs][max_blocks_per_seq], the reference's
 * BatchBlockTable layout), kv_lens[i] tokens of which the last
 * query_lens[i] are its queries, at token rows query_offsets[i] .. of query
 * and output ([total query tokens][query_heads][head_size] FP32); kv_lens,
 * query_lens, query_offsets are device uint64 [num_seqs]. max_query_tokens
 * and max_kv_len (host values) bound every query_lens[i] and kv_lens[i] and
 * size the grid; max_blocks_per_seq * block_size >= max_kv_len. Workgroups
 * take the heaviest query blocks of every sequence first. Same arithmetic,
 * errors and limits as kvflux_paged_prefill (each sequence's outputs are
 * bit-identical to that call's). Replaces one paged_attention call per
 * prompt (reference src/v2/paged_attention.cu:193-246) for a batch of
 * prompts. */
int kvflux_paged_prefill_batch(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                               uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                               const uint64_t* block_table, uint64_t max_blocks_per_seq,
                               const uint64_t* kv_lens, const uint64_t* query_lens,
                               const uint64_t* query_offsets, uint64_t num_seqs,
                               uint64_t max_query_tokens, uint64_t max_kv_len, uint64_t query_heads,
                               const float* query, float* output, void* stream);

/* ---------------------------------------------------------------------------
 * Callers of the hot path: copy-on-write and device-side batch metadata.
 *
 * kvflux_copy_pages: for every pair i of `pairs` (device uint64
 *   [num_pairs][2] = {source, destination}), the K page and the V page of
 *   `destination` (page_bytes = num_kv_heads * block_size * head_size * e
 *   each) become copies of those of `source`, in one launch. Replaces the two
 *   cudaMemcpyAsync of PagedKVStorage::copy_block
 *   (reference src/v2/paged_kv_storage.cpp:70-93), called once per shared
 *   tail page from append_token_cow (src/v2/copy_on_write.cpp:7-16), for a
 *   whole decode batch. Pairs with an id >= num_blocks or source ==
 *   destination are skipped. Destinations must be distinct and no
 *   destination may be a source of the same call (the C++ layer checks).
 *
 * kvflux_table_apply: brings a device batch block table (row-major uint64
 *   [num_rows][table_width], the reference's BatchBlockTable layout,
 *   include/kvflux/v2/batch_block_table.h:14-22) and its length array
 *   up to date in place. `updates` is device uint64 [num_updates][4] =
 *   {row, new_length, block_index, page_id}: seq_lens[row] = new_length and,
 *   when block_index < table_width, table[row][block_index] = page_id.
 *   Records of one row must carry the same length and distinct block
 *   indexes. Replaces the per-call host rebuild and upload of the batch
 *   table (reference src/v2/batch_block_table.cpp:18-48,
 *   src/v2/paged_attention.cu:248-313) with O(changed entries) work.
 *
 * kvflux_write_paged_kv_tail: kvflux_write_paged_kv for a decode step whose
 *   slots come from the device batch table: input row r (one token,
 *   [num_rows][num_kv_heads][head_size]) is written at position
 *   seq_lens[r] - 1 of table row r, i.e. slot
 *   table[r][(len - 1) / block_size] * block_size + (len - 1) % block_size
 *   (reference build_slot_mapping, src/v2/slot_mapping.cpp:8-31, evaluated on
 *   the device). Rows with a zero length, a block index >= table_width or a
 *   page id >= num_blocks are skipped.
 * ------------------------------------------------------------------------- */
int kvflux_copy_pages(void* key_cache, void* value_cache, uint64_t num_blocks,
                      uint64_t page_bytes, const uint64_t* pairs, uint64_t num_pairs,
                      void* stream);
int kvflux_table_apply(uint64_t* block_table, uint64_t table_width, uint64_t* seq_lens,
                       uint64_t num_rows, const uint64_t* updates, uint64_t num_updates,
                       void* stream);
int kvflux_write_paged_kv_tail(void* key_cache, void* value_cache, uint64_t num_blocks,
                               uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size,
                               int dtype, const void* key_new, const void* value_new,
                               const uint64_t* block_table, uint64_t table_width,
                               const uint64_t* seq_lens, uint64_t num_rows, void* stream);

/* ---------------------------------------------------------------------------
 * GPU <-> CPU chunk transfer (KV offload).
 *
 * kvflux_copy_chunks: for every pair i of `pairs` (device uint64
 *   [num_pairs][2] = {source address, destination address}), copies
 *   chunk_bytes bytes, all pairs in one launch. Either side may be device
 *   memory of the current device or pinned host memory from
 *   kvflux_host_malloc_pinned (mapped into the device address space), so one
 *   launch offloads (device -> host), onloads (host -> device) or moves a
 *   whole batch of chunks whose host slots are scattered. Every address must
 *   be aligned to the largest power of two (at most 16) dividing
 *   chunk_bytes; ranges must not overlap. Replaces one cudaMemcpyAsync per
 *   chunk of GpuCpuTransfer::begin_offload / begin_onload
 *   (reference src/v3/gpu_cpu_transfer.cpp:32-95) for a batch of chunks.
 *   Host addresses (in `pairs`, and `pairs` itself when it is host memory)
 *   are the device-side ones from kvflux_host_device_pointer.
 * ------------------------------------------------------------------------- */
int kvflux_copy_chunks(const uint64_t* pairs, uint64_t num_pairs, uint64_t chunk_bytes,
                       void* stream);

/* kvflux_copy_page_list: page i of `dst` (pages of page_bytes, i <
 *   num_pages) becomes a copy of page src_pages[i] of `src` (device uint64
 *   [num_pages]; ids >= num_src_blocks are skipped), one launch, raw bytes,
 *   no reordering inside a page. Stages a set of scattered KV pages (one
 *   cache's) in one contiguous device buffer, e.g. before a host transfer of
 *   a sequence's chunk (reference src/v3/gpu_cpu_transfer.cpp:32-95 copies
 *   one contiguous chunk per cudaMemcpyAsync). Ranges must not overlap. */
int kvflux_copy_page_list(void* dst, const void* src, uint64_t num_src_blocks, uint64_t page_bytes,
                          const uint64_t* src_pages, uint64_t num_pages, void* stream);

/* ---------------------------------------------------------------------------
 * kvflux_bandwidth_probe: HBM ceilings for the data-path kernels (no
 * counterpart in the reference; for benchmarks). Streams `bytes` bytes with
 * no page table: op 0 copies src -> dst, op 1 writes dst, op 2 reads src
 * (dst then takes a sink of threads * 16 bytes, almost never written).
 * threads 256/512/1024 per workgroup, vectors_per_thread 1/2/4/8 16-byte
 * vectors per thread per step, bytes a multiple of 16 * threads *
 * vectors_per_thread, 16-byte aligned buffers; grid 0 launches one
 * workgroup per step, otherwise `grid` workgroups walk the steps;
 * nontemporal selects the non-temporal form of the loads and stores.
 * ------------------------------------------------------------------------- */
int kvflux_bandwidth_probe(int op, void* dst, const void* src, uint64_t bytes, uint32_t threads,
                           uint32_t vectors_per_thread, uint32_t grid, int nontemporal, void* stream);

/* kvflux_bandwidth_probe_pages: read-only ceiling over scattered pages (no
 * counterpart in the reference; for benchmarks). Reads pages[0..num_pages)
 * of both caches (page_bytes each, ids >= num_blocks skipped) in list order,
 * one workgroup per (16 * threads * vectors_per_thread bytes of a page,
 * cache), and nothing else; page_bytes must be a multiple of that part.
 * sink: threads * 16 bytes, almost never written. */
int kvflux_bandwidth_probe_pages(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                 uint64_t page_bytes, const uint64_t* pages, uint64_t num_pages,
                                 uint32_t threads, uint32_t vectors_per_thread, int nontemporal,
                                 void* sink, void* stream);

/* ---------------------------------------------------------------------------
 * Test and benchmark support (not part of the reference API).
 * kvflux_fill_random writes `count` elements of `dtype` from a counter-based
 * generator: element i depends only on (seed, i), so a CPU checker can
 * recompute any element. distribution 0: uniform [-1, 1) on a 2^-23 grid;
 * 1: approximately N(0,1) as the sum of twelve 16-bit uniforms (Irwin-Hall).
 * 16-bit dtypes are rounded to nearest-even from the FP32 value.
 * kvflux_compare_bytes synchronously counts differing bytes of two device
 * buffers.
 * ------------------------------------------------------------------------- */
int kvflux_fill_random(void* dst, uint64_t count, int dtype, int distribution,
                       uint64_t seed, void* stream);
int kvflux_compare_bytes(const void* a, const void* b, uint64_t bytes, uint64_t* mismatches);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVFLUX_HIP_H */
