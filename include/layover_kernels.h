/*
 * layover_kernels.h: C ABI of the KV data-path kernels for MI355X (gfx950).
 *
 * The reference runs these as Triton kernels called from Python; each entry point below
 * replaces one of those call sites and keeps its argument meaning:
 *   lk_fp8_quantize    layover/kernels/fp8.py:349-367 quantize_blocks (_quantize_kernel :241-270)
 *   lk_fp8_dequantize  layover/kernels/fp8.py:370-384 dequantize_blocks (_dequantize_kernel :272-294)
 *   lk_fp8_encode      layover/kernels/fp8.py:319-323 encode_bits_triton (_encode_kernel :296-299)
 *   lk_fp8_decode      layover/kernels/fp8.py:326-329 decode_bits_triton (_decode_kernel :301-304)
 *   lk_paged_decode    layover/kernels/triton_decode.py:131-179 kernel_launch/run_kernel
 *                      (_paged_decode_kernel :39-119); the FP8-record KV format has no
 *                      reference counterpart (the reference decodes BF16 and FP32 pools only).
 *   lk_paged_prefill   layover/model.py:69-98 prefill_attention (gather + FlashAttention),
 *                      read in place instead of gathered.
 *   lk_kv_write        layover/model.py:139-140, the decode-time pool write, as one kernel.
 *   lk_fp8_append      no counterpart: the FP8-resident pool's version of the decode-time
 *                      pool write of layover/model.py:139-140.
 *
 * Conventions: plain device pointers and sizes; `stream` is a hipStream_t (a torch stream's
 * cuda_stream; null means the legacy default stream). Every entry point only enqueues work
 * and returns LK_OK, or returns LK_ERR_INVALID with nothing enqueued when the arguments do
 * not describe a launch the kernels support (the message is in lk_last_error). Block ids and
 * lengths are not read on the host: the caller has checked them (as the reference's trusted
 * decode path does, triton_decode.py:248-261).
 */
#ifndef LAYOVER_KERNELS_H
#define LAYOVER_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LK_ABI_VERSION 3

enum { LK_OK = 0, LK_ERR_INVALID = 1, LK_ERR_DEVICE = 2 };

/* Element formats of q/out and of the KV pool. */
enum {
    LK_BF16 = 0,      /* bfloat16 */
    LK_F32 = 1,       /* float32 */
    LK_FP8_RECORD = 2 /* KV only: FP8 E4M3 records with per-group int16 shifts (see below) */
};

int lk_abi_version(void);
const char* lk_last_error(void);

/* Quantize blocks ids[0..count) of a BF16 pool into `count` records at the front of `stage`.
 * A block is groups_per_block groups of group_elems consecutive BF16 values. Record i is
 * group_elems*groups_per_block E4M3 bytes (block ids[i], in pool order) followed by one
 * little-endian int16 shift per group: record_bytes = block_elems + 2*groups_per_block. Each
 * group is divided by 2**shift, shift = (largest finite nonzero BF16 exponent) - 134, or 0
 * for a group without one, and rounded to nearest even; see fp8.py:1-31 for the special
 * values. Bytes of `stage` past count*record_bytes are untouched. count 0 writes nothing and
 * accepts null pointers. */
int lk_fp8_quantize(const void* pool, const int32_t* ids, uint32_t count, void* stage, uint64_t group_elems,
                    uint32_t groups_per_block, void* stream);

/* The inverse: records 0..count) of `stage` decoded into pool blocks ids[0..count). */
int lk_fp8_dequantize(const void* stage, const int32_t* ids, uint32_t count, void* pool, uint64_t group_elems,
                      uint32_t groups_per_block, void* stream);

/* Elementwise codec at one shift, for exhaustive checks: n BF16 bit patterns -> n E4M3 bytes,
 * and n E4M3 bytes -> n BF16 bit patterns. */
int lk_fp8_encode(const uint16_t* bits, uint8_t* out, uint64_t n, int32_t shift, void* stream);
int lk_fp8_decode(const uint8_t* codes, uint16_t* out, uint64_t n, int32_t shift, void* stream);

/* Shape of one paged decode launch. Pool layout [block, kind(K=0,V=1), layer, kv_head, slot,
 * dim] (reference layover/kv/paged_cache.py:40-49); for LK_FP8_RECORD each block is one
 * record as produced by lk_fp8_quantize with group_elems = slots*head_dim and
 * groups_per_block = 2*layers*kv_heads, i.e. the same element order. */
typedef struct {
    uint32_t batch;
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t layers;
    uint32_t slots;       /* tokens per block */
    uint32_t layer;       /* the layer this launch reads */
    uint32_t table_width; /* blocks per table row */
    int32_t q_format;     /* LK_BF16 or LK_F32; out has the same format */
    int32_t kv_format;    /* LK_BF16, LK_F32 or LK_FP8_RECORD */
    float scale;          /* softmax scale, 1/sqrt(head_dim) in the reference */
    uint32_t table_stride;   /* int32 elements between table rows; 0 means table_width */
    uint32_t lengths_stride; /* int32 elements between lengths; 0 means 1 */
    uint32_t flags;          /* 0, or LK_DECODE_SHARED_BLOCKS */
} lk_decode_shape;

/* Decode flag: rows of the table share pool blocks (forked prefixes, or tables drawn from a
 * pool with fewer blocks than they list), so a block read by one row is likely read again by
 * another soon after. K/V tiles are then loaded so that they stay in the caches (the Infinity
 * Cache serves the repeats). Without it the tiles are streamed with the non-temporal hint,
 * the faster form when every block is read once per layer. Results are the same either way. */
#define LK_DECODE_SHARED_BLOCKS 1u

/* Bytes of device workspace lk_paged_decode needs for this shape (split-K partial results).
 * Depends only on the shape and on the current device's compute-unit count (a grid too small
 * to fill the GPU gets about one workgroup per CU), never on lengths, so it can be sized once
 * per batch layout. Its contents need no initialization. Calls that share a workspace must not
 * overlap in time. */
uint64_t lk_paged_decode_workspace(const lk_decode_shape* shape);

/* One decode step of one layer: out[b, h] = softmax(q[b,h] . K^T * scale) V over the first
 * lengths[b*lengths_stride] tokens of row b of `table` (int32, row b at b*table_stride, its
 * first table_width entries used; the strides let the columns of a packed row block, as
 * triton_decode.py takes them by stride, be passed without a copy), where query head h
 * reads KV head h / (query_heads / kv_heads). q and out are [batch, query_heads, head_dim]
 * contiguous. Tokens at or past lengths[b] never contribute, whatever their slots hold.
 * Accumulation is FP32; out is rounded to nearest even. Requires 1 <= lengths[b] <=
 * table_width*slots and every id in range, which the caller has checked. */
int lk_paged_decode(const lk_decode_shape* shape, const void* q, const void* pool, const int32_t* table,
                    const int32_t* lengths, void* out, void* workspace, uint64_t workspace_bytes, void* stream);

/* One prefill chunk of one sequence and one layer, causal: query token t of the chunk (absolute
 * position start + t) attends to keys 0 .. start + t, read in place from the pool through
 * block_ids (int32, the sequence's blocks in order; at least ceil((start + tokens) / slots)
 * of them, num_block_ids given for the check). q and out are BF16 [query_heads, tokens,
 * head_dim]; query head h reads KV head h / (query_heads / kv_heads). The chunk's own K/V
 * must already be in the pool. Replaces the reference's gather + FlashAttention
 * (layover/model.py:69-98, prefill_attention). Supported: 16 slots x 128 dims, BF16 q, BF16
 * or FP8-record pools. q and out 16-byte aligned; a pool read in place 16-byte aligned, its
 * blocks too. An FP8 record (2 x layers x kv_heads groups of 2,050 bytes) is aligned when
 * layers x kv_heads is a multiple of 4; lk_paged_prefill_split stages records of other
 * layouts as BF16 (they need only be 2-byte aligned), lk_paged_prefill refuses them. */
typedef struct {
    uint32_t tokens;      /* query tokens in the chunk */
    uint32_t start;       /* position of the chunk's first token */
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t layers;
    uint32_t slots;
    uint32_t layer;
    int32_t q_format;     /* LK_BF16 */
    int32_t kv_format;    /* LK_BF16 or LK_FP8_RECORD */
    float scale;
} lk_prefill_shape;

int lk_paged_prefill(const lk_prefill_shape* shape, const void* q, const void* pool, const int32_t* block_ids, uint32_t num_block_ids,
                     void* out, void* stream);

/* Bytes of device workspace lk_paged_prefill_split needs for this shape: for an FP8-record pool,
 * the chunk's history decoded to BF16 (one layer: 4 KiB per token at 8 KV heads) plus a block
 * index; split-K partials when the chunk's (KV head, 128-row tile) workgroups would not give
 * every CU two of them (short chunks against long histories); and, when they give exactly
 * that and causal tiles differ widely (chunks near the start of a sequence), the states of
 * heavy tiles whose key steps two workgroups of a CU divide (80 KiB per side) with a tag and a
 * ready word per CU pair. 0 when none applies.
 * No counterpart in the reference, whose prefill gathers the history and runs FlashAttention;
 * depends on the shape and the device's CU count (LAYOVER_PREFILL_SPLITS=n forces n splits;
 * LAYOVER_PREFILL_FP8=direct reads FP8 records in the attention kernel instead of staging
 * them). 0 also for a shape lk_paged_prefill refuses. */
uint64_t lk_paged_prefill_workspace(const lk_prefill_shape* shape);

/* lk_paged_prefill, staging an FP8-record history as BF16 first and splitting each tile's keys
 * over several workgroups when the plan above does (partials merged in a further launch), or
 * dividing heavy tiles within CU pairs (merged in the same launch). The workspace (at least
 * lk_paged_prefill_workspace bytes, 16-byte aligned; may be null when that is 0) needs no
 * initialization; calls that share one must not overlap in time. */
int lk_paged_prefill_split(const lk_prefill_shape* shape, const void* q, const void* pool, const int32_t* block_ids,
                           uint32_t num_block_ids, void* out, void* workspace, uint64_t workspace_bytes, void* stream);

/* One decode step's KV write into a BF16 pool, the reference's indexed assignment
 * (layover/model.py:139-140) as one launch: for row b, slot write_slot[b*row_stride] of block
 * write_block[b*row_stride], layer `layer`, takes k[b] (K) and v[b] (V), BF16 [batch,
 * kv_heads, head_dim] contiguous. head_dim a multiple of 8; pool, k and v 16-byte aligned.
 * Ids and slots are not checked. */
int lk_kv_write(void* pool, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride, uint32_t batch,
                const void* k, const void* v, uint32_t layer, uint32_t layers, uint32_t kv_heads, uint32_t slots,
                uint32_t head_dim, void* stream);

/* One decode step's KV write into an FP8-record pool: no reference counterpart (the
 * reference writes BF16 tokens into a BF16 pool, layover/model.py:139-140). For row b,
 * block write_block[b*row_stride] slot write_slot[b*row_stride] of layer `layer` takes
 * k[b] (K) and v[b] (V), BF16 [batch, kv_heads, head_dim]. Each of the 2*kv_heads groups a
 * row touches is re-encoded (as lk_fp8_quantize would encode it) from: the old codes decoded
 * at the old shift for earlier slots, the new values at the write slot, and zero for later
 * slots. Records are laid out as lk_fp8_quantize writes them, with group_elems =
 * slots*head_dim and groups_per_block = 2*layers*kv_heads. Rows must name distinct blocks;
 * ids and slots are not checked. */
int lk_fp8_append(void* records, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride, uint32_t batch,
                  const void* k, const void* v, uint32_t layer, uint32_t layers, uint32_t kv_heads, uint32_t slots,
                  uint32_t head_dim, void* stream);

/* lk_kv_write (BF16 pool) or lk_fp8_append (FP8 records) of each row's new token into layer
 * shape->layer, then lk_paged_decode of that layer, as one decode launch where the shape
 * allows (the wave that reads a row's last block for a KV head writes that head's token and
 * uses the written values for that block without re-reading them). No counterpart
 * in the reference, whose decode step writes the pool and then attends (layover/model.py:
 * 139-141); for small-batch steps, which are bound by launches. The write position must be
 * the row's last token: write_block[b*write_stride] = table[b][(lengths[b] - 1) / slots] and
 * write_slot[b*write_stride] = (lengths[b] - 1) % slots, as PagedKVCache.decode_rows packs
 * them; it is not checked. Rows must name distinct blocks. On the fused path the token is
 * written by the waves that read the row's last block, so a row is written only when
 * 1 <= lengths[b] <= table_width * slots (the range lk_paged_decode accepts); a row outside it
 * is neither read nor written. Other shapes run the two launches. */
int lk_paged_decode_append(const lk_decode_shape* shape, const void* q, void* pool, const int32_t* table, const int32_t* lengths,
                           const int32_t* write_block, const int32_t* write_slot, uint32_t write_stride, const void* k,
                           const void* v, void* out, void* workspace, uint64_t workspace_bytes, void* stream);

/* No counterpart in the reference. lk_paged_decode for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc): the same
 * arguments minus the workspace, whose split partials go to a file-scope device array of
 * 32 MiB per GPU (held until the process ends; its address is looked up on the first call
 * on each device). A shape whose lk_paged_decode_workspace exceeds 32 MiB is refused with
 * LK_ERR_INVALID. Calls on one GPU share the array, so they are ordered: a call on a stream
 * other than the previous call's first makes its stream wait for that call (an event recorded
 * after each call; one event per device, created on the first call). Under HIP graph capture
 * no event is used: captured calls are ordered by their graph, and replays of graphs holding
 * such calls must not overlap on one GPU. The stream must belong to the current device
 * (LK_ERR_INVALID otherwise). It calls no hipMalloc or hipFree. */
int lk_paged_decode_static(const lk_decode_shape* shape, const void* q, const void* pool, const int32_t* table,
                           const int32_t* lengths, void* out, void* stream);

/* Block gather and scatter between a paged pool and contiguous staging: the kernels behind
 * lt_out_gather / lt_in_scatter (the counterpart of the reference's gather_kernel /
 * scatter_kernel, native/transfer_cuda.cu:20-28, which its C ABI does not export), for callers
 * that stage blocks themselves and for measuring the kernels alone. lk_gather_blocks copies
 * pool block ids[i] to staging bytes [i * block_bytes, (i + 1) * block_bytes) for i < count;
 * lk_scatter_blocks copies the other way. ids are device uint32; pool and staging are device
 * memory, 8-byte aligned, and block_bytes a positive multiple of 8 (the transfer ABI's rules).
 * Block ids are not checked against the pool's size. count 0 copies nothing and accepts null
 * pointers. */
int lk_gather_blocks(const void* pool, const uint32_t* ids, uint32_t count, uint64_t block_bytes, void* staging, void* stream);
int lk_scatter_blocks(void* pool, const uint32_t* ids, uint32_t count, uint64_t block_bytes, const void* staging, void* stream);

/* Measurement support, no reference counterpart: stream `bytes` (a multiple of 16, 16-byte
 * aligned) from `src`, copying to `dst`, or only reading when dst is null (then `sink`, one
 * device uint32, is written only if the data hash to a value chosen never to occur). This is
 * the HBM ceiling bench.py reports beside the 8 TB/s specification. Reads move 4 KiB per wave,
 * copies 1 KiB per single-wave workgroup: the faster shape for each, measured on MI355X. */
int lk_stream_probe(const void* src, void* dst, uint64_t bytes, uint32_t* sink, void* stream);

/* Measurement support, no reference counterpart: the traffic mix of the FP8 record kernels.
 * Reads `src_bytes` from `src` and writes `dst_bytes` to `dst` (both 16-byte aligned), in the
 * ratio 2:1 (as lk_fp8_quantize: src_bytes a multiple of 16; output 8-byte word i is the two
 * halves of input 16-byte word i XORed) or 1:2 (as lk_fp8_dequantize: src_bytes a multiple of
 * 8; output 16-byte word i is input 8-byte word i twice), one single-wave workgroup per 64
 * words. The measured ceiling for those kernels' mix of reads and writes; LK_ERR_INVALID for
 * any other ratio. */
int lk_stream_probe_mix(const void* src, uint64_t src_bytes, void* dst, uint64_t dst_bytes, void* stream);

/* No counterpart in the reference; measurement only. Reads the K and V tiles that
 * lk_paged_decode would read for `shape` (BF16 or FP8-record pool, 16 slots x 128 dims; for
 * FP8 records also the two groups' shifts) and nothing else, in
 * the decode's order: the read rate of the decode's own access pattern on a given pool and
 * table, the ceiling the decode kernel is compared with. Writes *sink only if the data hash
 * to a value chosen never to occur. */
int lk_tile_probe(const lk_decode_shape* shape, const void* pool, const int32_t* table, const int32_t* lengths, void* sink,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAYOVER_KERNELS_H */
