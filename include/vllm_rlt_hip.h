/*
 * vllm_rlt_hip.h — C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * One shared library (libvllm_rlt_hip.so) exports these entry points. They take
 * plain device pointers, element strides (int64, in elements of the storage
 * dtype unless the name says bytes) and a hipStream_t, launch asynchronously on
 * that stream, never synchronise and never allocate device memory (the one
 * standing reservation is the 96 MiB per-GPU array of vrh_paged_decode_noalloc,
 * made when the library's code object loads on a GPU). They return
 * VRH_OK or an error code; vrh_last_error() then holds a message for the
 * calling thread.
 *
 * Storage layout (the reference's KV pool, kv_cache_manager.py:143-145):
 *   key_cache, value_cache : [num_blocks, num_layers, block_size, kv_heads, head_dim]
 * Per-layer entry points receive the layer view K[:, layer], i.e. a base
 * pointer plus (block, token, head) strides; the head dimension is contiguous.
 * Block ids are int32 in tables and int64 in write addresses; every physical
 * offset is computed in 64-bit (pools beyond 2^31 elements).
 *
 * Index arguments (block ids, write offsets, slots, descriptors) are trusted,
 * as in the reference's Triton kernels: they are read on the device and not
 * range-checked there (the host cannot see them without a synchronisation).
 * An id outside the pool addresses memory outside it. Sizes, strides, dtypes
 * and pointers are checked on the host before any launch.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * vllm-rlt source tree):
 *   vrh_kv_append            kv_cache_manager.py:689-699 (index_put append),
 *                            kernels/routing.py:180-225 (masked_kv_store),
 *                            kernels/graph_kv.py:7-65 (write_graph_kv)
 *   vrh_paged_decode         kernels/paged_attention.py:12-71 (torch_paged_attention
 *                            and its windowed variant), kernels/triton_attention.py:150-202
 *   vrh_paged_decode_noalloc (none: see its declaration)
 *   vrh_paged_prefill        kernels/triton_attention.py:313-366 (paged_prefill_attention)
 *   vrh_kv_gather            kv_cache_manager.py:834-854 (read)
 *   vrh_kv_finalize          kernels/routing.py:147-177 (finalize_kernel),
 *                            worker/model_runner.py:1331-1346 (its launch)
 *   vrh_kv_finalize_token    kv_cache_manager.py:806-831 (finalize_token)
 *   vrh_kv_copy_blocks       kv_cache_manager.py:481-523 (snapshot/restore page
 *                            copies); also the copy-on-write block copy, which has
 *                            no counterpart in the reference
 *   vrh_expand_kv_addresses  kernels/metadata.py:7-24 (expand_kv_addresses)
 *   vrh_routing_metadata     kernels/routing.py:14-48 (metadata_kernel)
 *   vrh_routing_slots        kernels/routing.py:7-11 (slots_kernel)
 *   vrh_kv_blocks_to_host    kv_cache_manager.py:481-502 (snapshot page copies)
 *   vrh_kv_blocks_from_host  kv_cache_manager.py:504-523 (restore page copies)
 *   vrh_gather_rows          kernels/routing.py:51-66 (gather_kernel)
 *   vrh_scatter_rows         kernels/routing.py:69-83 (scatter_kernel)
 *   vrh_gather_segments      kernels/routing.py:86-113 (gather_segments_kernel)
 *   vrh_scatter_segments     kernels/routing.py:116-144 (scatter_segments_kernel)
 *   vrh_silu_and_mul         csrc/activation/silu_and_mul.cu:221-245 (silu_and_mul_cuda),
 *                            kernels/activation.py:20-33 (its Torch contract)
 */
#ifndef VLLM_RLT_HIP_H_
#define VLLM_RLT_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; 0 selects the null stream. */
typedef struct ihipStream_t* vrh_stream_t;

enum {
  VRH_OK = 0,
  VRH_ERROR_INVALID_ARG = 1,
  VRH_ERROR_LAUNCH = 2,
  VRH_ERROR_UNSUPPORTED = 3,
};

enum {
  VRH_DTYPE_F32 = 0,
  VRH_DTYPE_F16 = 1,
  VRH_DTYPE_BF16 = 2,
};

/* ABI version of this header; bumped on any signature change. */
int vrh_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* vrh_last_error(void);

/* ------------------------------------------------------------------ append
 * For every row r < rows that is enabled, and every layer l < layers:
 *   cache[write_blocks[r], l, write_offsets[r], h, d] = k[l, r, h, d]   (same for v)
 * A row is enabled when (active_rows == NULL || r < *active_rows) and
 * (write_mask == NULL || write_mask[r] != 0). Disabled rows are not touched.
 * `layers` > 1 batches the appends of several layers (k/v layer strides and
 * the cache layer stride select them); pass layers = 1 for one layer view.
 * With num_blocks > 0 (block_size > 0), a row whose block id lies outside
 * [0, num_blocks) (offset outside [0, block_size)) writes nothing, so a bad
 * address cannot write outside the pool; pass 0 to leave them unchecked.
 * Bit-exact copy. */
int vrh_kv_append(int dtype, void* key_cache, void* value_cache, int64_t cache_block_stride,
                  int64_t cache_token_stride, int64_t cache_head_stride,
                  int64_t cache_layer_stride, const void* k, const void* v, int64_t k_row_stride,
                  int64_t k_head_stride, int64_t k_layer_stride, int64_t v_row_stride,
                  int64_t v_head_stride, int64_t v_layer_stride, const int64_t* write_blocks,
                  const int64_t* write_offsets, const uint8_t* write_mask,
                  const int32_t* active_rows, int64_t rows, int32_t layers, int32_t kv_heads,
                  int32_t head_dim, int64_t num_blocks, int32_t block_size,
                  vrh_stream_t stream);

/* ------------------------------------------------------------ paged decode
 * Single-query attention per row over its own block table:
 *   out[r, h] = softmax(q[r, h] . K[t, h / G]^T / sqrt(D)) V[t, h / G],  t in window
 * where G = q_heads / kv_heads, t ranges over [max(0, n - window), n) with
 * n = context_lengths[r] (window = 0: the whole context), K[t] is
 * key_cache[block_tables[r, t / block_size], t % block_size]. Rows with n = 0
 * produce zeros. fp32 accumulation; the output is rounded to the storage dtype.
 * The result of a row depends only on that row's inputs (batch invariant).
 * block_tables holds `rows` rows of table_width readable entries (row stride
 * table_stride); entries past a row's ceil(n / block_size) pages are never used
 * as page ids (they may be -1), but are compared with the neighbouring rows'
 * entries at the same index, which only selects the cache policy of the loads.
 * `workspace` must hold vrh_paged_decode_workspace_bytes(rows, q_heads, head_dim)
 * bytes of device memory; it needs no initialisation. */
size_t vrh_paged_decode_workspace_bytes(int64_t rows, int32_t q_heads, int32_t head_dim);
int vrh_paged_decode(int dtype, void* out, const void* q, const void* key_cache,
                     const void* value_cache, const int32_t* block_tables,
                     const int32_t* context_lengths, int64_t rows, int32_t q_heads,
                     int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t table_width,
                     int64_t table_stride, int64_t q_row_stride, int64_t q_head_stride,
                     int64_t out_row_stride, int64_t out_head_stride, int64_t k_block_stride,
                     int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                     int64_t v_token_stride, int64_t v_head_stride, int32_t window,
                     void* workspace, size_t workspace_bytes, vrh_stream_t stream);

/* ------------------------------------------------- paged decode, no alloc
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP-graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same computation and kernels as vrh_paged_decode, with
 * the split partials in a built-in device array of
 * VRH_PAGED_DECODE_NOALLOC_MAX_BYTES per GPU (held until the process ends)
 * instead of a workspace argument. Calls needing more than that
 * (vrh_paged_decode_workspace_bytes(rows, q_heads, head_dim) > the limit, e.g.
 * more than 756 rows x 16 heads at head_dim 128) fail with
 * VRH_ERROR_INVALID_ARG before any launch. Every call on one GPU shares that
 * array: calls that overlap on one GPU (other streams, concurrent graph
 * replays) race. Nothing in it needs clearing between calls.
 * Fixed cost: the array is part of the library's code object, so its 96 MiB
 * are reserved on every GPU where the library is loaded, whether or not this
 * entry point is ever called (a caller sizing its KV pool to the last GiB
 * counts them). vrh_paged_decode_noalloc_max_bytes() also looks up the
 * current device's array address (once per device): a caller that captures
 * calls into a HIP graph calls it on each device before capture. */
#define VRH_PAGED_DECODE_NOALLOC_MAX_BYTES ((size_t)96 << 20)
size_t vrh_paged_decode_noalloc_max_bytes(void);
int vrh_paged_decode_noalloc(int dtype, void* out, const void* q, const void* key_cache,
                             const void* value_cache, const int32_t* block_tables,
                             const int32_t* context_lengths, int64_t rows, int32_t q_heads,
                             int32_t kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t table_width, int64_t table_stride, int64_t q_row_stride,
                             int64_t q_head_stride, int64_t out_row_stride,
                             int64_t out_head_stride, int64_t k_block_stride,
                             int64_t k_token_stride, int64_t k_head_stride,
                             int64_t v_block_stride, int64_t v_token_stride,
                             int64_t v_head_stride, int32_t window, vrh_stream_t stream);

/* ----------------------------------------------------------- paged prefill
 * Packed causal prefill, bottom-right aligned: sequence s owns query rows
 * [cu_seqlens_q[s], cu_seqlens_q[s+1]) and keys [0, context_lengths[s]) through
 * block_tables[s]; its query i sits at position n_s - q_s + i and attends keys
 * at positions <= that. bf16/f16 with head_dim 32, 64, 96 or 128 (and
 * 16-byte aligned rows) use MFMA tiles with fp32 accumulation; other cases
 * compute each query row with the decode kernel. With a workspace of
 * vrh_paged_prefill_workspace_bytes(num_seqs, max_seqlen_q, q_heads, head_dim)
 * bytes, sequences of one query (decode rows riding in a packed batch) use
 * split-KV decode, and the MFMA work items are dispatched longest sequence
 * first (batches of up to 64 sequences are ranked inside the kernel, larger
 * ones up to 2048 by a small ranking kernel writing the order into the
 * workspace). With none (NULL, 0) every sequence goes through the MFMA tiles
 * in batch order. Results do not depend on the order.
 * Decode exactness (the reference's packed_matches_decode, attention/backend.py:
 * 21-23): with the workspace and max_seqlen_q <= 8, every query runs as its own
 * split-KV decode row, and query i of sequence s equals, bit for bit, what
 * vrh_paged_decode returns for a row with the same q, table row and length
 * n_s - q_s + i + 1 (the decode partition depends only on that length). */
size_t vrh_paged_prefill_workspace_bytes(int64_t num_seqs, int32_t max_seqlen_q, int32_t q_heads,
                                         int32_t head_dim);
int vrh_paged_prefill(int dtype, void* out, const void* q, const void* key_cache,
                      const void* value_cache, const int32_t* block_tables,
                      const int32_t* context_lengths, const int32_t* cu_seqlens_q,
                      int64_t num_seqs, int64_t total_q, int32_t max_seqlen_q, int32_t q_heads,
                      int32_t kv_heads, int32_t head_dim, int32_t block_size,
                      int32_t table_width, int64_t table_stride, int64_t q_token_stride,
                      int64_t q_head_stride, int64_t out_token_stride, int64_t out_head_stride,
                      int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride,
                      int64_t v_block_stride, int64_t v_token_stride, int64_t v_head_stride,
                      void* workspace, size_t workspace_bytes, vrh_stream_t stream);

/* ------------------------------------------------------------------ gather
 * out_k[t] = K[table[t / block_size], t % block_size] for t < length (and V),
 * where K is a layer view; out rows are `channel_bytes` contiguous bytes
 * (kv_heads * head_dim * elem_size). Bit-exact. */
int vrh_kv_gather(void* out_k, void* out_v, const void* key_cache, const void* value_cache,
                  const int32_t* table, int64_t length, int32_t block_size,
                  int64_t block_stride_bytes, int64_t token_stride_bytes, int64_t channel_bytes,
                  vrh_stream_t stream);

/* ---------------------------------------------------------------- finalize
 * LAST_EXITED depth propagation from device descriptors. For each row r with
 * (slot, depth, pos) = descriptors[r, 0:3] and each plane p in (depth, planes):
 *   src = tables[(slot * planes + depth) * width + pos / block_size]
 *   dst = tables[(slot * planes + p) * width + pos / block_size]
 *   K[dst, l, pos % block_size, :] = K[src, l, pos % block_size, :]  for all l < layers
 * (same for V). Strides are in bytes; a (layer, token) slot is channel_bytes
 * contiguous bytes. Bit-exact. */
int vrh_kv_finalize(void* key_cache, void* value_cache, const int64_t* descriptors,
                    const int32_t* tables, int64_t rows, int32_t planes, int32_t width,
                    int32_t block_size, int32_t layers, int64_t block_stride_bytes,
                    int64_t layer_stride_bytes, int64_t token_stride_bytes,
                    int64_t channel_bytes, vrh_stream_t stream);

/* Host-described variant for one token: copies the slot `offset` of the
 * listed layers from block `src_block` into each of `dst_blocks[0:num_dst]`
 * (host arrays, num_dst <= 64, num_layers <= 256). */
int vrh_kv_finalize_token(void* key_cache, void* value_cache, int64_t src_block,
                          const int64_t* dst_blocks, int32_t num_dst, int32_t offset,
                          const int32_t* layer_ids, int32_t num_layers,
                          int64_t block_stride_bytes, int64_t layer_stride_bytes,
                          int64_t token_stride_bytes, int64_t channel_bytes,
                          vrh_stream_t stream);

/* -------------------------------------------------------------- block copy
 * For i < n: bytes [0, block_bytes) of block dst_blocks[i] = those of block
 * src_blocks[i], in both caches. Block ids index `block_stride_bytes`-strided
 * blocks of the whole pool (all layers). Source and destination sets must be
 * disjoint. Bit-exact. */
int vrh_kv_copy_blocks(void* key_cache, void* value_cache, int64_t block_stride_bytes,
                       int64_t block_bytes, const int64_t* src_blocks, const int64_t* dst_blocks,
                       int64_t n, vrh_stream_t stream);

/* ------------------------------------------------------- host offload
 * Preemption snapshot / restore of whole blocks (all layers) of both caches:
 * to_host copies block blocks[i] of key_cache / value_cache to row i of
 * host_keys / host_values (block_bytes per row); from_host copies row i back
 * into block blocks[i]. blocks is a device array. The host rows must be pinned
 * host memory (hipHostMalloc); the kernels access it through its device
 * mapping, so no device staging buffer is allocated. Other pointers are
 * rejected with VRH_ERROR_INVALID_ARG before any launch. Asynchronous on
 * `stream`: the host rows are complete (to_host) or may be reused (from_host)
 * once the stream has passed the call. Bit-exact. */
int vrh_kv_blocks_to_host(const void* key_cache, const void* value_cache,
                          int64_t block_stride_bytes, int64_t block_bytes, const int64_t* blocks,
                          void* host_keys, void* host_values, int64_t n, vrh_stream_t stream);
int vrh_kv_blocks_from_host(void* key_cache, void* value_cache, int64_t block_stride_bytes,
                            int64_t block_bytes, const int64_t* blocks, const void* host_keys,
                            const void* host_values, int64_t n, vrh_stream_t stream);

/* ------------------------------------------------------ hidden-state rows
 * Byte copies of `width_bytes`-wide rows (strides in bytes).
 * gather_rows: out[r] = r < n ? pool[slots[r]] : 0 for r < size.
 * scatter_rows: pool[slots[r]] = in[r] for r < count.
 * segments: int64 [num_segments, 5] = (state_slot, hidden_row_offset,
 * token_count, batch_row_start, keep_intermediate); pool row of segment row i
 * is state_slot * pool_rows + hidden_row_offset + i, batch row is
 * batch_row_start + i, i < token_count <= max_rows.
 * gather_segments: out[batch row] = pool[pool row].
 * scatter_segments: pool[pool row] = in[batch row] where keep_intermediate != 0. */
int vrh_gather_rows(const void* pool, const int64_t* slots, void* out, int64_t n, int64_t size,
                    int64_t width_bytes, int64_t pool_stride_bytes, int64_t out_stride_bytes,
                    vrh_stream_t stream);
int vrh_scatter_rows(const void* in, const int64_t* slots, void* pool, int64_t count,
                     int64_t width_bytes, int64_t in_stride_bytes, int64_t pool_stride_bytes,
                     vrh_stream_t stream);
int vrh_gather_segments(const void* pool, const int64_t* segments, void* out,
                        int64_t num_segments, int64_t max_rows, int64_t pool_rows,
                        int64_t width_bytes, int64_t pool_stride_bytes, int64_t out_stride_bytes,
                        vrh_stream_t stream);
int vrh_scatter_segments(const void* in, const int64_t* segments, void* pool,
                         int64_t num_segments, int64_t max_rows, int64_t pool_rows,
                         int64_t width_bytes, int64_t in_stride_bytes, int64_t pool_stride_bytes,
                         vrh_stream_t stream);

/* ------------------------------------------------------------ SiLU-and-Mul
 * out[i] = dtype(dtype(silu(gate[i])) * up[i]) for `count` contiguous elements
 * (f32, f16, bf16). silu is evaluated so that its rounding to the dtype equals
 * the double-precision value rounded to fp32 and then to the dtype; the
 * product is rounded once. Pointers need only their dtype's alignment: gate,
 * up and out may sit at different 16-byte offsets. */
int vrh_silu_and_mul(int dtype, void* out, const void* gate, const void* up, int64_t count,
                     vrh_stream_t stream);

/* --------------------------------------------------------------- addresses
 * blocks[i] = tables[sequences[i] * width + positions[i] / page],
 * offsets[i] = positions[i] % page, for i < n. */
int vrh_expand_kv_addresses(const int64_t* positions, const int32_t* sequences,
                            const int32_t* tables, int64_t* blocks, int64_t* offsets, int64_t n,
                            int32_t width, int32_t page, vrh_stream_t stream);

/* Per row r < size (valid when r < n), from descriptors[r] = (slot, depth, pos):
 *   plane = planes > 1 ? depth : 0; base = (slot * planes + plane) * width
 *   slots[r] = slot, positions[r] = pos, lengths[r] = valid ? pos + 1 : 0
 *   blocks[r] = tables[base + pos / page], offsets[r] = pos % page  (valid rows only)
 *   out_tables[r * width + c] = valid ? tables[base + c] : 0  for c < out_width
 * Invalid rows read slot = depth = pos = 0. */
int vrh_routing_metadata(const int64_t* descriptors, const int32_t* tables, int64_t* slots,
                         int64_t* positions, int32_t* lengths, int64_t* blocks,
                         int64_t* offsets, int32_t* out_tables, int64_t n, int64_t size,
                         int32_t width, int32_t page, int32_t planes, int32_t out_width,
                         vrh_stream_t stream);

/* slots[r] = r < n ? descriptors[r * 3] : 0 for r < size. */
int vrh_routing_slots(const int64_t* descriptors, int64_t* slots, int64_t n, int64_t size,
                      vrh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_RLT_HIP_H_ */
