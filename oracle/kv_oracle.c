/*
 * TEST INFRASTRUCTURE ONLY. This is the CPU oracle the HIP kernels are checked against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path (layover_amd/) never links, loads or calls anything here.
 *
 * A plain-C restatement of the reference's KV data path arithmetic:
 *
 *   - FP8 E4M3 codec on the uint16 bit view of BF16 with a per-group power-of-two shift:
 *       group shift  layover/kernels/fp8.py:86-92   (group_shifts)
 *       encode       layover/kernels/fp8.py:95-116  (encode_bits)
 *       decode       layover/kernels/fp8.py:119-137 (decode_bits)
 *   - Records of quantized blocks, data then int16 shifts, and their inverse:
 *       layover/kernels/fp8.py:58-80 (Fp8Layout), :179-187 (_quantize_torch),
 *       :190-198 (_dequantize_torch)
 *   - Byte gather/scatter of whole blocks in id order: native/pack.h:41-68
 *   - Paged GQA decode attention in float64: layover/kernels/decode_attention.py:9-37
 *     (the reference's own oracle), layover/kernels/triton_decode.py:39-119 for masking.
 *
 * Parity pins (each in tests/test_oracle.py): encode/decode against torch.float8_e4m3fn on
 * every pattern (test_fp8.py:40-59), the reference's known answers (test_fp8.py:62-153),
 * brute force of the round-trip error bound (fp8.py:25-27), record layout constants
 * (test_fp8.py:164-176), and decode attention against
 * torch's float64 scaled_dot_product_attention and a pure-Python softmax on tiny inputs.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>

#define ORACLE_EXPORT __attribute__((visibility("default")))

/* BF16 field masks and biases (fp8.py:45-55). */
enum { EXP_MASK = 0xFF, BF16_BIAS = 127, FP8_BIAS = 7, FP8_TARGET = 7, DROP = 4 };

/* fp8.py:86-92: largest finite nonzero biased exponent of the group, mapped to FP8 exponent
 * 7; a group with no such value keeps shift 0. */
ORACLE_EXPORT int32_t oracle_group_shift(const uint16_t* bits, uint64_t n) {
    int32_t largest = 0;
    for (uint64_t i = 0; i < n; ++i) {
        int32_t raw = (bits[i] >> 7) & EXP_MASK;
        if (raw > 0 && raw < EXP_MASK && raw > largest) largest = raw;
    }
    return largest > 0 ? largest - BF16_BIAS - FP8_TARGET : 0;
}

/* fp8.py:95-116. Divide by 2**shift and round the 8-bit significand to FP8's 4 bits, ties to
 * even; values that become FP8 subnormals lose one more bit per binade. */
ORACLE_EXPORT uint8_t oracle_encode(uint16_t bits, int32_t shift) {
    const int32_t sign = (bits >> 15) & 1;
    const int32_t raw = (bits >> 7) & EXP_MASK;
    const int32_t biased = raw - BF16_BIAS - shift + FP8_BIAS;
    const int32_t significand = (bits & 0x7F) | 0x80;
    int32_t below = 1 - biased;
    if (below < 0) below = 0;
    int32_t right = DROP + below;
    if (right > 15) right = 15;
    int32_t kept = significand >> right;
    const int32_t remainder = significand & ((1 << right) - 1);
    const int32_t half = 1 << (right - 1);
    if (remainder > half || (remainder == half && (kept & 1))) kept += 1;
    int32_t magnitude = biased > 0 ? ((biased - 1) << 3) + kept : kept;
    if (magnitude > 0x7E) magnitude = 0x7F;
    if (raw == 0) magnitude = 0;
    if (raw == EXP_MASK) magnitude = 0x7F;
    return (uint8_t)((sign << 7) | magnitude);
}

/* fp8.py:119-137. Multiply by 2**shift; saturate at BF16's largest finite, flush below its
 * smallest normal, NaN becomes the canonical 0x7FC0. */
ORACLE_EXPORT uint16_t oracle_decode(uint8_t byte, int32_t shift) {
    const int32_t sign = (byte >> 7) & 1;
    const int32_t magnitude = byte & 0x7F;
    const int32_t raw = magnitude >> 3;
    int32_t fraction = magnitude & 7;
    const int32_t top = fraction >= 4 ? 2 : (fraction >= 2 ? 1 : 0);
    const int32_t exponent = raw > 0 ? raw - FP8_BIAS : top - 9;
    if (raw == 0) fraction = (fraction << (3 - top)) & 7;
    const int32_t biased = exponent + shift + BF16_BIAS;
    int32_t out = (biased << 7) | (fraction << DROP);
    if (biased >= EXP_MASK) out = 0x7F7F;
    if (biased <= 0) out = 0;
    if (magnitude == 0) out = 0;
    out |= sign << 15;
    if (magnitude == 0x7F) out = 0x7FC0;
    return (uint16_t)out;
}

ORACLE_EXPORT void oracle_encode_array(const uint16_t* bits, uint8_t* out, uint64_t n, int32_t shift) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_encode(bits[i], shift);
}

ORACLE_EXPORT void oracle_decode_array(const uint8_t* bytes, uint16_t* out, uint64_t n, int32_t shift) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_decode(bytes[i], shift);
}

/* fp8.py:179-187. Record i = encoded block ids[i], then one little-endian int16 shift per
 * group. Groups are consecutive runs of group_elems in pool order. */
ORACLE_EXPORT void oracle_quantize_records(const uint16_t* pool, const int32_t* ids, uint32_t count, uint8_t* stage,
                                           uint64_t group_elems, uint32_t groups_per_block) {
    const uint64_t block_elems = group_elems * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    for (uint32_t i = 0; i < count; ++i) {
        const uint16_t* block = pool + (uint64_t)ids[i] * block_elems;
        uint8_t* out = stage + (uint64_t)i * record;
        for (uint32_t g = 0; g < groups_per_block; ++g) {
            const uint16_t* group = block + (uint64_t)g * group_elems;
            const int32_t shift = oracle_group_shift(group, group_elems);
            uint8_t* data = out + (uint64_t)g * group_elems;
            for (uint64_t e = 0; e < group_elems; ++e) data[e] = oracle_encode(group[e], shift);
            const int16_t stored = (int16_t)shift;
            memcpy(out + block_elems + 2ull * g, &stored, 2);
        }
    }
}

/* fp8.py:190-198. The inverse: record i decoded into pool block ids[i]. */
ORACLE_EXPORT void oracle_dequantize_records(const uint8_t* stage, const int32_t* ids, uint32_t count, uint16_t* pool,
                                             uint64_t group_elems, uint32_t groups_per_block) {
    const uint64_t block_elems = group_elems * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    for (uint32_t i = 0; i < count; ++i) {
        const uint8_t* in = stage + (uint64_t)i * record;
        uint16_t* block = pool + (uint64_t)ids[i] * block_elems;
        for (uint32_t g = 0; g < groups_per_block; ++g) {
            int16_t stored;
            memcpy(&stored, in + block_elems + 2ull * g, 2);
            const uint8_t* data = in + (uint64_t)g * group_elems;
            uint16_t* target = block + (uint64_t)g * group_elems;
            for (uint64_t e = 0; e < group_elems; ++e) target[e] = oracle_decode(data[e], stored);
        }
    }
}

/* pack.h:56-68: block ids[i] of the pool <-> slot i of a contiguous buffer, whole blocks. */
ORACLE_EXPORT void oracle_gather(const uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, uint8_t* out) {
    for (uint32_t i = 0; i < count; ++i) memcpy(out + (uint64_t)i * block_bytes, pool + (uint64_t)ids[i] * block_bytes, block_bytes);
}

ORACLE_EXPORT void oracle_scatter(uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const uint8_t* in) {
    for (uint32_t i = 0; i < count; ++i) memcpy(pool + (uint64_t)ids[i] * block_bytes, in + (uint64_t)i * block_bytes, block_bytes);
}

static double bf16_to_double(uint16_t bits) {
    uint32_t wide = (uint32_t)bits << 16;
    float value;
    memcpy(&value, &wide, 4);
    return (double)value;
}

/* Paged decode attention in float64 over a BF16 pool [block, 2, layers, kv_heads, slots,
 * dim] (paged_cache.py:40-49). q is float64 [batch, query_heads, dim]; out likewise. Query
 * head h reads KV head h / kv_groups (triton_decode.py:77). Slots at or past a sequence's
 * length are excluded entirely, so whatever they hold cannot reach the result
 * (triton_decode.py:100-109). The softmax is the textbook two-pass one: maximum, then
 * weights, then the weighted mean, all in double. */
ORACLE_EXPORT int oracle_decode_attention(const double* q, const uint16_t* pool, uint32_t layers, uint32_t kv_heads,
                                          uint32_t slots, uint32_t dim, uint32_t layer, const int32_t* table,
                                          uint32_t table_width, const int32_t* lengths, uint32_t batch,
                                          uint32_t query_heads, double scale, double* out) {
    if (kv_heads == 0 || query_heads % kv_heads) return 1;
    const uint32_t groups = query_heads / kv_heads;
    const uint64_t head_stride = (uint64_t)slots * dim;
    const uint64_t layer_stride = kv_heads * head_stride;
    const uint64_t kind_stride = layers * layer_stride;
    const uint64_t block_stride = 2 * kind_stride;
    for (uint32_t b = 0; b < batch; ++b) {
        const int32_t length = lengths[b];
        if (length < 1 || (uint64_t)length > (uint64_t)table_width * slots) return 2;
        double* scores = (double*)malloc(sizeof(double) * (size_t)length);
        if (!scores) return 3;
        for (uint32_t h = 0; h < query_heads; ++h) {
            const double* qh = q + ((uint64_t)b * query_heads + h) * dim;
            const uint64_t head_offset = (uint64_t)layer * layer_stride + (uint64_t)(h / groups) * head_stride;
            double top = -INFINITY;
            for (int32_t t = 0; t < length; ++t) {
                const uint64_t block = (uint64_t)table[(uint64_t)b * table_width + t / slots];
                const uint16_t* k = pool + block * block_stride + head_offset + (uint64_t)(t % slots) * dim;
                double dot = 0.0;
                for (uint32_t d = 0; d < dim; ++d) dot += qh[d] * bf16_to_double(k[d]);
                scores[t] = dot * scale;
                if (scores[t] > top) top = scores[t];
            }
            double total = 0.0;
            for (int32_t t = 0; t < length; ++t) {
                scores[t] = exp(scores[t] - top);
                total += scores[t];
            }
            double* oh = out + ((uint64_t)b * query_heads + h) * dim;
            for (uint32_t d = 0; d < dim; ++d) oh[d] = 0.0;
            for (int32_t t = 0; t < length; ++t) {
                const uint64_t block = (uint64_t)table[(uint64_t)b * table_width + t / slots];
                const uint16_t* v = pool + block * block_stride + kind_stride + head_offset + (uint64_t)(t % slots) * dim;
                const double w = scores[t] / total;
                for (uint32_t d = 0; d < dim; ++d) oh[d] += w * bf16_to_double(v[d]);
            }
        }
        free(scores);
    }
    return 0;
}
