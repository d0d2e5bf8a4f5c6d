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
 * plan lists each sequence's blocks and the kernels read them from the pool directly.
 *
 *   query        [batch][32][64] fp16, contiguous; q head h reads kv head h / 8
 *   out          [batch][32][64] fp16, contiguous (query, out, pool and plan 16-byte aligned)
 *   context_lens [batch] int32 device copy of the lengths the plan was built from
 *                (0 or less: the row is not written); the kernel takes the lengths from
 *                the plan, which carries them
 *   plan         num_records rows of pc_attn_plan_record_ints() int32 from pc_attn_plan()
 *                for the same lengths and block tables (device copy), optionally followed
 *                by all-zero padding rows; one plan serves every layer of a decode step
 *   out[b][h] = softmax(q[b][h] . K[b][:len]^T / 8) . V[b][:len], computed in fp32 and
 *   rounded once to fp16. Slots past len are never multiplied, so poisoned (NaN) tail
 *   slots do not reach the output. A block id outside [0, num_blocks) is never
 *   dereferenced; its sequence's output rows become NaN. A plan that does not match
 *   context_lens gives wrong rows, never an access outside the buffers.
 *
 * One kernel launch, one workgroup per plan row (a bin of up to 256 blocks and 4
 * sequences). A sequence cut over several bins of one group leaves one fp32 partial per
 * part (all but its last) and kv head in `workspace`, with a ready flag; the bin holding
 * its last part waits for the flags (a bounded wait), folds the parts in order and writes
 * the row, then sets the flags back to zero. A flag value names the plan's epoch (each
 * pc_attn_plan result has its own) and the layer, so a flag left raised by an earlier call
 * is never taken for this call's partial. `workspace`: pc_attn_workspace_bytes() bytes,
 * 256-byte aligned, required (never null), ALL ZERO before its first use (hipMemset, or a
 * fill kernel under graph capture); every call leaves its flags at zero again, so it is
 * reused as is. Calls that share a workspace must not overlap in time.
 *
 * Faults fail closed. The first 4 bytes of the workspace are its fault word (int32). A
 * merge that finds a part flagged by another XCD (its partial may not be visible), or not
 * flagged within the bounded wait, and a block id outside the pool turn the affected rows
 * into NaN and OR a PC_ATTN_FAULT_* bit into the fault word; the call itself still returns
 * PC_OK (the failure happens on the device, after the launch). The kernels never clear the
 * word: the caller reads it after synchronizing and, when it is nonzero, treats every output
 * since it was last cleared as failed and zeroes the whole workspace before reusing it.
 */
#define PC_ATTN_WORKSPACE_HEADER_BYTES 256
#define PC_ATTN_FAULT_MERGE_TIMEOUT 1 /* a part's flag was not raised within the bounded wait */
#define PC_ATTN_FAULT_FOREIGN_XCD 2   /* a part's flag was raised on another XCD */
#define PC_ATTN_FAULT_BLOCK_ID 4      /* a block id outside [0, num_blocks) */
int pc_paged_decode_attn(void* out, const void* query, const void* pool, int64_t num_blocks, int32_t layer,
                         const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                         int32_t num_records, void* workspace, void* stream);

/*
 * KV append of each sequence's newest token fused with paged decode attention over it.
 *
 * Replaces the decode step's KVAllocator.write_decode_layer row copies followed by
 * paged_attention (reference src/pagedcore/decoder.py:187-190, kv_cache.py:221-246,
 * attention.py:14-53) when the key and value are already projected: one launch instead of
 * pc_kv_append + pc_paged_decode_attn, with the same results.
 *
 *   new_key, new_value  [batch][4][64] fp16, contiguous, 16-byte aligned: the token at
 *                       position context_lens[b] - 1 of sequence b
 *   other arguments     as pc_paged_decode_attn (pool writable)
 *
 * For each sequence b of the plan with length n > 0, the rows go to
 * pool[layer][0 / 1][table[b][(n - 1) / 16]][(n - 1) % 16] (the table as carried by the
 * plan; a block id outside [0, num_blocks) is not written, and its sequence's output rows
 * become NaN as in pc_paged_decode_attn), then out is what pc_paged_decode_attn gives on the
 * updated pool: bit-identical to pc_kv_append of those slots followed by
 * pc_paged_decode_attn. The block a new token goes into must not be read by another
 * sequence of the batch (a block taking new tokens belongs to one sequence); other layers
 * and other rows of the pool are not touched.
 */
int pc_kv_append_paged_decode_attn(void* out, const void* query, void* pool, int64_t num_blocks, int32_t layer,
                                   const int32_t* context_lens, int32_t batch, int32_t max_blocks,
                                   const int32_t* plan, int32_t num_records, const void* new_key,
                                   const void* new_value, void* workspace, void* stream);

/* Workspace size in bytes for pc_paged_decode_attn; 0 on invalid arguments. */
int64_t pc_attn_workspace_bytes(int32_t batch, int32_t max_blocks);

/*
 * pc_paged_decode_attn without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference, which allocates its score buffer
 * per call (src/pagedcore/attention.py:36).
 *
 * The split-K partials go to a device array inside the library, one per GPU, of
 * PC_ATTN_NOALLOC_SCRATCH_BYTES bytes, held until the process ends; its address is looked
 * up once per device (hipGetSymbolAddress) on the first call there. The call allocates and
 * frees nothing. Shapes whose workspace (pc_attn_workspace_bytes) exceeds the array are
 * refused with PC_ERR_ARGUMENT before any HIP call (32 MiB covers, e.g., batch 4096 with
 * 128-block tables, but not batch 8192). The array starts at zero when the library loads
 * and every call leaves its flags at zero. Its fault word is not readable by the caller:
 * a fault shows only as NaN rows. A merge that gave up waiting (a malformed plan, or a part
 * held back past the bounded wait) can leave a late part's flag raised: a call with a new
 * plan never takes it (the plan's epoch differs), a replay of the same plan could, so after
 * NaN rows build a new plan. `stream` must belong to the current device.
 * Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (concurrent streams,
 * threads) race and give wrong rows; calls ordered on one stream are safe. Arguments and
 * results are otherwise those of pc_paged_decode_attn.
 */
#define PC_ATTN_NOALLOC_SCRATCH_BYTES (32LL << 20)
int pc_paged_decode_attn_noalloc(void* out, const void* query, const void* pool, int64_t num_blocks, int32_t layer,
                                 const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                                 int32_t num_records, void* stream);

/*
 * Host-side decode plan (no device access). context_lens [batch] and block_tables
 * [batch][max_blocks] are HOST arrays (row b: sequence b's physical blocks in logical order,
 * only the first ceil(len / 16) read); plan is HOST memory of `capacity` rows of
 * pc_attn_plan_record_ints() (296) int32. Sequences are dealt, longest first, to the least
 * loaded of 8 groups (one per XCD); each group's blocks, taken sequence after sequence, are
 * cut into bins of equal block counts (about total / 256 blocks each, at least 8, at most
 * 256, and a bin also closes at 4 sequences). Row r holds bin r / 8 of group r % 8:
 *   {segments, blocks, plan epoch (nonzero, 22 bits, new for every call), 0 x 5},
 *   4 segments {sequence, context length, first block, blocks, row of the sequence's first
 *               bin, part index, parts, first partial slot (cut sequences) or 0},
 *   the bin's block ids in order (up to 256; 0 past them).
 * A cut sequence's part k is in row first + 8 k; only a bin's first and last segments can
 * be cut parts. Groups with fewer bins are padded with all-zero rows. Returns the row
 * count (a multiple of 8), or -pc_status on invalid arguments (including a context length
 * above 16 * max_blocks: its table cannot hold it) or if `capacity` is too small;
 * pc_attn_plan_capacity() always suffices (-1 on invalid arguments).
 *
 * Replaces nothing in the reference: PagedCore walks each sequence's pages in Python
 * (reference src/pagedcore/attention.py:31-53); the plan is what lets one launch cover a
 * ragged batch with every CU streaming the same number of blocks.
 */
int32_t pc_attn_plan(const int32_t* context_lens, const int32_t* block_tables, int32_t batch, int32_t max_blocks,
                     int32_t* plan, int64_t capacity);
int32_t pc_attn_plan_record_ints(void);
int64_t pc_attn_plan_capacity(int32_t batch, int32_t max_blocks);

/*
 * Decode-step kernels around paged attention. Each one rounds to fp16 exactly where the
 * reference's torch expression materialises an fp16 tensor (every fp16 torch op computes in
 * fp32 and rounds its result once), so only fp32 reduction order differs from the reference.
 */

/*
 * RoPE on one token's query and key, fused with the KV append of its rotated key and
 * unrotated value.
 *
 * Replaces apply_rope (reference src/pagedcore/dense.py:33-61) on decode and prefill
 * tokens, and the per-row KVAllocator.write_decode_layer copies of the rotated key and the
 * value (reference src/pagedcore/kv_cache.py:221-246, called at src/pagedcore/decoder.py:185-187).
 *
 *   qkv          [num_tokens][qkv_stride] fp16: columns 0..2047 are the 32 query heads,
 *                2048..2303 the 4 key heads, 2304..2559 the 4 value heads (qkv_stride >= 2560,
 *                a multiple of 8)
 *   positions    [num_tokens] int64: the token's absolute position, in [0, rope_positions)
 *   rope_table   [rope_positions][2][32] fp16: cos, then sin, of position * inv_freq[j] with
 *                inv_freq[j] = 1 / 10000^(2j / 64), computed in fp32 and rounded to fp16
 *   query_out    [num_tokens][32][64] fp16: the rotated queries
 *   key_out, value_out  [num_tokens][4][64] fp16 or null: the rotated keys / the values
 *   pool, slot_mapping  both null, or the KV pool and [num_tokens] int64 slots
 *                (block * 16 + offset; negative or >= num_blocks * 16: the token is not
 *                written): the rotated key and the value go to pool[layer][0 / 1][slot]
 *
 * For each head x and d < 32 (c, s the table row of the token's position):
 *   out[d]      = fp16(fp16(x[d] * c[d])      + fp16(-x[d + 32] * s[d]))
 *   out[d + 32] = fp16(fp16(x[d + 32] * c[d]) + fp16(x[d] * s[d]))
 * All buffers 16-byte aligned. A position outside the table is rejected by the callers;
 * inside the kernel it turns the token's rows to NaN and skips its pool write.
 */
int pc_rope_kv_append(void* query_out, void* key_out, void* value_out, const void* qkv, int64_t qkv_stride,
                      const int64_t* positions, const void* rope_table, int32_t rope_positions, void* pool,
                      int64_t num_blocks, int32_t layer, const int64_t* slot_mapping, int64_t num_tokens,
                      void* stream);

/*
 * Residual add fused with RMSNorm, over rows of `width` fp16 (a multiple of 8, <= 8192).
 *
 * Replaces the residual sums of the decoder (reference src/pagedcore/decoder.py:191-192 and
 * :238-239) followed by rms_norm (reference src/pagedcore/dense.py:17-21):
 *   if delta is not null: hidden = fp16(hidden + delta)   (in place)
 *   out = fp16(weight * fp16(hidden * rsqrt(mean(hidden^2) + eps)))   (mean in fp32)
 * hidden, delta, out: [rows][width]; weight: [width]; all 16-byte aligned; out must not
 * overlap hidden or delta.
 */
int pc_add_rms_norm(void* out, void* hidden, const void* delta, const void* weight, int64_t rows, int32_t width,
                    float eps, void* stream);

/*
 * SwiGLU activation. Replaces the elementwise part of swiglu
 * (reference src/pagedcore/dense.py:102-104):
 *   out[r][i] = fp16(fp16(silu(gate_up[r][i])) * gate_up[r][width + i]),  silu(x) = x / (1 + e^-x)
 * gate_up: [rows][2 * width] (the gate projection's outputs, then the up projection's);
 * out: [rows][width]; width a multiple of 8; both 16-byte aligned.
 */
int pc_silu_mul(void* out, const void* gate_up, int64_t rows, int32_t width, void* stream);

/*
 * Split-K forms of the two consumers above, for the partial sums of pc_gemm_m128's partials
 * epilogue: the fp16 input they replace is fp16(sum over s of parts[s]), added in split
 * order, and everything after that is the same computation.
 *
 *   pc_rope_kv_append_parts: qkv_parts [splits][num_tokens][2560] fp32 in place of qkv.
 *   pc_add_rms_norm_parts:   delta_parts [splits][rows][width] fp32 in place of delta;
 *                            hidden = fp16(hidden + fp16(sum of delta_parts)).
 * splits in [1, 64]; parts 16-byte aligned.
 */
int pc_rope_kv_append_parts(void* query_out, void* key_out, void* value_out, const float* qkv_parts, int32_t splits,
                            const int64_t* positions, const void* rope_table, int32_t rope_positions, void* pool,
                            int64_t num_blocks, int32_t layer, const int64_t* slot_mapping, int64_t num_tokens,
                            void* stream);
int pc_add_rms_norm_parts(void* out, void* hidden, const float* delta_parts, int32_t splits, const void* weight,
                          int64_t rows, int32_t width, float eps, void* stream);

/*
 * Projection GEMM of the decode step at up to 128 rows: Y[i][j] = sum_l x[i][l] * w[j][l],
 * fp16 inputs, fp32 accumulation.
 *
 * Replaces torch.nn.functional.linear on the decode step's activations (reference
 * src/pagedcore/dense.py:91-104, called per layer by src/pagedcore/decoder.py:156-199) for
 * the q|k|v, o_proj, gate|up and down projections at batch <= 128.
 *
 *   x    [m][k] fp16, m in [1, 128];  w [n][k] fp16 (the weight as stored, row-major)
 *   out, by epilogue:
 *     PC_GEMM_PARTIALS  [splits][m][n] fp32: split s sums l in [s k / splits, (s + 1) k / splits)
 *     PC_GEMM_HALF      [m][n] fp16, fp16(Y) (splits = 1)
 *     PC_GEMM_SWIGLU    [m][n / 2] fp16 (splits = 1), w the stacked [gate_proj | up_proj]
 *                       weight: out[i][j] = fp16(fp16(silu(fp16(Y[i][j]))) * fp16(Y[i][n/2 + j]))
 *                       (the rounding of pc_silu_mul applied to the fp16 projections)
 * k / splits a multiple of 64; n a multiple of 32 (of 64 for PC_GEMM_SWIGLU); all buffers
 * 16-byte aligned; out must not overlap x or w.
 */
#define PC_GEMM_PARTIALS 0
#define PC_GEMM_HALF 1
#define PC_GEMM_SWIGLU 2
int pc_gemm_m128(void* out, const void* x, const void* w, int32_t m, int32_t n, int32_t k, int32_t splits,
                 int32_t epilogue, void* stream);

/*
 * Causal attention of one prompt over its contiguous K/V (the prefill of one sequence).
 *
 * Replaces the prompt's dense_attention (reference src/pagedcore/dense.py:69-81, called by
 * the prefill forward at src/pagedcore/decoder.py:236-237):
 *   out[t][h] = softmax_{j <= t}(query[t][h] . key[j][h / 8] / 8) . value[j][h / 8]
 * query, out: [tokens][32][64] fp16; key, value: [tokens][4][64] fp16 (the rotated keys and
 * the values of pc_rope_kv_append's key_out / value_out); all contiguous, 16-byte aligned;
 * tokens in [0, 65536]. Scores, softmax and the weighted sum are fp32 (online softmax,
 * probabilities enter the PV product as fp16) with one final fp16 rounding, where the
 * reference rounds the scores and the normalised probabilities to fp16 (the accepted
 * difference is within the decoder tolerances).
 */
int pc_prefill_attention(void* out, const void* query, const void* key, const void* value, int32_t tokens,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDCORE_HIP_H */
