/*
 * pagedcore_hip.h — C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * The library moves and reads the KV pool that PagedCore's Python layer owns:
 *
 *   pool: fp16, contiguous [22 layers][2 kinds: K, V][num_blocks][16 slots][4 kv heads][64 dims]
 *
 * Element (layer, kind, block, slot, head, dim) lives at
 *   ((((layer * 2 + kind) * num_blocks + block) * 16 + slot) * 256 + head * 64 + dim).
 *
 * Conventions shared by every entry point:
 *   - return 0 on success, a nonzero pc_status otherwise; pc_last_error() then names the
 *     problem (thread-local text, valid until the next call on the same thread);
 *   - every pointer is device memory, except where stated; nothing here allocates or frees;
 *   - work is only enqueued on `stream` (a hipStream_t passed as void*); no call synchronizes;
 *   - all arguments are validated before anything is enqueued, so a failed call leaves the
 *     pool untouched.
 */
#ifndef PAGEDCORE_HIP_H
#define PAGEDCORE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum pc_status {
  PC_OK = 0,
  PC_ERR_ARGUMENT = 1, /* a size, index, pointer or alignment is invalid */
  PC_ERR_LAUNCH = 2,   /* the HIP runtime rejected a kernel launch */
};

/* ABI revision; bumped whenever a signature or a layout contract changes. */
int pc_abi_version(void);

/* Text describing the last failure on the calling thread ("" if none). */
const char* pc_last_error(void);

/*
 * KV append: copy K and V token rows into the pool through a slot mapping.
 *
 * Replaces the chunked `Tensor.copy_` loop of KVAllocator.append
 * (reference src/pagedcore/kv_cache.py:161-172) and the per-row copies of
 * KVAllocator.write_decode_layer (reference src/pagedcore/kv_cache.py:242-245).
 *
 * For src layer l in [0, num_layers) and token t in [0, num_tokens):
 *   pool[layer_begin + l][0][slot / 16][slot % 16][:][:] = key  [l][t][:][:]
 *   pool[layer_begin + l][1][slot / 16][slot % 16][:][:] = value[l][t][:][:]
 * with slot = slot_mapping[t] = block * 16 + offset. A negative slot skips the token.
 * The copy moves raw 16-bit words, so the pool bytes equal the source bytes.
 *
 * key/value rows are [4][64] fp16 with contiguous heads and dims; the layer and token
 * strides (in fp16 elements) are free, so strided views need no staging copy.
 * Every slot must be < num_blocks * 16 (checked on the device; out-of-range tokens are
 * skipped, never written).
 */
int pc_kv_append(void* pool, int64_t num_blocks, int32_t layer_begin, int32_t num_layers,
                 const void* key, int64_t key_layer_stride, int64_t key_token_stride,
                 const void* value, int64_t value_layer_stride, int64_t value_token_stride,
                 const int64_t* slot_mapping, int64_t num_tokens, void* stream);

/*
 * Paged decode attention for one layer, one query token per sequence.
 *
 * Replaces the two page traversals of paged_attention
 * (reference src/pagedcore/attention.py:14-53) and the Python page generator that feeds
 * them, KVAllocator.iter_layer_blocks (reference src/pagedcore/kv_cache.py:248-270): the
 * block table is walked inside the kernel.
 *
 *   query        [batch][32][64] fp16, contiguous; q head h reads kv head h / 8
 *   out          [batch][32][64] fp16, contiguous, 16-byte aligned (query and pool too)
 *   block_tables [batch][max_blocks] int32 physical block ids (row b lists sequence b's
 *                blocks in logical order; only the first ceil(len/16) are read)
 *   context_lens [batch] int32, each in [1, max_blocks * 16] (0 or less: row not written)
 *   out[b][h] = softmax(q[b][h] . K[b][:len]^T / 8) . V[b][:len], computed in fp32 and
 *   rounded once to fp16. Slots past len are never multiplied, so poisoned (NaN) tail
 *   slots do not reach the output. A block id outside [0, num_blocks) is never
 *   dereferenced; its sequence's output rows become NaN.
 *
 * Split-K: a sequence's table is cut into work items of `partition_blocks` blocks (1, 2,
 * 4 or 8), one workgroup per item and one wave per block. A sequence covered by one item
 * is written directly; longer ones leave one partial per item in the workspace, merged
 * by a second kernel (flags = PC_ATTN_SEPARATE_REDUCE) or, flags = 0, by the last
 * workgroup of the sequence to finish (one launch).
 *   work_items  null: the grid covers batch * ceil(max_blocks / partition_blocks) item
 *               slots and the slots past a sequence's length exit at once; otherwise the
 *               host-built plan from pc_attn_plan() for the same context_lens,
 *               block_tables and partition_blocks (device copy, num_work_items records):
 *               the grid then holds only items that exist, and the item kernel takes
 *               block ids and lengths from the plan. A plan that does not match the
 *               tables gives wrong rows (never an out-of-pool read). One plan serves
 *               every layer of a decode step.
 *   workspace  fp32 partials, pc_attn_workspace_bytes() bytes, 256-byte aligned; scratch,
 *              nothing in it needs to survive between calls (unused, may be null, when
 *              max_blocks <= partition_blocks);
 *   tickets    int32 [batch], one merge ticket per sequence, only read by the fused merge:
 *              ZERO-FILLED BEFORE ITS FIRST USE; every call leaves the tickets at zero
 *              again, so one ticket array serves any number of later calls.
 * Calls that share a workspace or tickets must not overlap (use one set per stream).
 */
#define PC_ATTN_SEPARATE_REDUCE 1

int pc_paged_decode_attn(void* out, const void* query, const void* pool, int64_t num_blocks,
                         int32_t layer, const int32_t* block_tables, int32_t max_blocks,
                         const int32_t* context_lens, int32_t batch, int32_t partition_blocks,
                         const int32_t* work_items, int32_t num_work_items, void* workspace,
                         int32_t* tickets, int32_t flags, void* stream);

/* Workspace size in bytes for pc_paged_decode_attn; 0 on invalid arguments. */
int64_t pc_attn_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t partition_blocks);

/*
 * Host-side decode plan (no device access). context_lens [batch] and block_tables
 * [batch][max_blocks] are HOST copies of the tables the attention call will receive;
 * work_items is HOST memory. Writes one record of pc_attn_plan_record_ints() int32 per
 * work item that exists -- items of partition_blocks blocks first (sequence-major), then
 * the shorter tail items by descending block count, since workgroups are dispatched in
 * record order:
 *   {sequence, item, context length, 0, block ids of the item's partition_blocks blocks
 *    (0 past the sequence's last block), 0 padding}
 * and returns how many; returns -pc_status on invalid arguments or if `capacity` (in
 * records) is too small. pc_attn_plan_capacity() gives a capacity that always suffices
 * (-1 on invalid arguments). The kernel reads a record with one load, so the block
 * loads of a work item wait for one round trip instead of two.
 *
 * Replaces nothing in the reference: PagedCore walks each sequence's pages in Python
 * (reference src/pagedcore/attention.py:31-53); the plan is what lets one launch cover a
 * ragged batch without idle workgroups.
 */
int32_t pc_attn_plan(const int32_t* context_lens, const int32_t* block_tables, int32_t batch,
                     int32_t max_blocks, int32_t partition_blocks, int32_t* work_items, int64_t capacity);
int32_t pc_attn_plan_record_ints(int32_t partition_blocks);
int64_t pc_attn_plan_capacity(int32_t batch, int32_t max_blocks, int32_t partition_blocks);

/* Default blocks per work item (partition_blocks) used by the Python layer. */
int32_t pc_attn_default_partition_blocks(void);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDCORE_HIP_H */
