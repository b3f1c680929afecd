/* CPU oracle, byte / integer / selection work -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain C restatement of the reference's packed-KV codec and of its selection rules,
 * used by tests/ (through oracle/codec.py) to check the HIP kernels bit-exactly.
 * Nothing in the product library links or loads this file.
 *
 * Reference (brain-lab-research/MaskAhead, src/maskahead):
 *   pack/unpack       reference.py:35-55   element 2i in bits 0-3, 2i+1 in bits 4-7
 *   key dequant       reference.py:168-179 x = f32(code) * f32(scale) + f32(zero), then bf16
 *   value dequant     reference.py:259-268 same rule, groups along channels
 *   read-set top-k    session.py:1429-1438 topk of rank, indices sorted ascending
 *   keep set          eviction.py:325-409  W newest + sinks/pins + top (C - W), sorted by pos
 *   compaction        cache.py:342-367     survivors gathered in keep order
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -shared -fPIC).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar conversions, written from the IEEE-754 binary16 / bfloat16 definitions */

float oc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t expo = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    float mag;
    if (expo == 0) {
        mag = ldexpf((float)mant, -24); /* subnormal: mant * 2^-24 */
    } else if (expo == 31) {
        mag = mant ? NAN : INFINITY;
    } else {
        mag = ldexpf((float)(mant | 0x400u), (int)expo - 25);
    }
    return sign ? -mag : mag;
}

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* round-to-nearest-even to bfloat16; NaN stays a quiet NaN */
uint16_t oc_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float oc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* ---- nibble packing: byte = code[2i] | code[2i+1] << 4 (reference.py:35-55) */

void oc_pack4(const uint8_t *codes, int64_t n_codes, uint8_t *out) {
    for (int64_t i = 0; i < n_codes / 2; ++i) {
        out[i] = (uint8_t)((codes[2 * i] & 15u) | ((codes[2 * i + 1] & 15u) << 4));
    }
}

void oc_unpack4(const uint8_t *bytes, int64_t n_bytes, uint8_t *codes) {
    for (int64_t i = 0; i < n_bytes; ++i) {
        codes[2 * i] = bytes[i] & 15u;
        codes[2 * i + 1] = bytes[i] >> 4;
    }
}

static float dq(uint32_t code, uint16_t scale, uint16_t zero) {
    /* code * scale is exact in f32 (4-bit code times 11-bit significand); one rounding
       on the add, matching the two torch ops of reference.py:170-171 */
    float prod = (float)code * oc_f16_to_f32(scale);
    return prod + oc_f16_to_f32(zero);
}

/* Keys, channel mode.  payload [G][D][KG/2] bytes, scale/zero [G][D] f16 bits, all
 * contiguous.  Output token-major [G*KG][D]: f32 (out32) and bf16 bits (out16); either
 * may be NULL.  Token t of group g sits in byte (t/2) of channel row d, nibble t%2. */
void oc_dequant_keys4(const uint8_t *payload, const uint16_t *scale, const uint16_t *zero,
                      int64_t groups, int64_t d, int64_t kg, float *out32, uint16_t *out16) {
    for (int64_t g = 0; g < groups; ++g) {
        for (int64_t c = 0; c < d; ++c) {
            const uint8_t *row = payload + (g * d + c) * (kg / 2);
            uint16_t s = scale[g * d + c], z = zero[g * d + c];
            for (int64_t t = 0; t < kg; ++t) {
                uint32_t code = (t & 1) ? (row[t / 2] >> 4) : (row[t / 2] & 15u);
                float x = dq(code, s, z);
                int64_t o = (g * kg + t) * d + c;
                if (out32) out32[o] = x;
                if (out16) out16[o] = oc_f32_to_bf16(x);
            }
        }
    }
}

/* Values, per token over channel groups.  payload [N][D/VG][VG/2], scale/zero [N][D/VG]. */
void oc_dequant_values4(const uint8_t *payload, const uint16_t *scale, const uint16_t *zero,
                        int64_t n, int64_t d, int64_t vg, float *out32, uint16_t *out16) {
    int64_t ng = d / vg;
    for (int64_t t = 0; t < n; ++t) {
        for (int64_t c = 0; c < d; ++c) {
            int64_t grp = c / vg, w = c % vg;
            uint8_t byte = payload[(t * ng + grp) * (vg / 2) + w / 2];
            uint32_t code = (w & 1) ? (byte >> 4) : (byte & 15u);
            float x = dq(code, scale[t * ng + grp], zero[t * ng + grp]);
            if (out32) out32[t * d + c] = x;
            if (out16) out16[t * d + c] = oc_f32_to_bf16(x);
        }
    }
}

/* ---- selection ------------------------------------------------------------------ */

/* Total order used for every selection: larger value first; -0.0 equals +0.0; NaN is
 * above +inf (torch.topk ranks NaN first); equal values by ascending index. */
static uint32_t order_key(float f) {
    if (f != f) return 0xffffffffu;
    if (f == 0.0f) f = 0.0f;
    uint32_t u = f32_bits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
    uint32_t key;
    int64_t idx;
} ranked_t;

static int cmp_ranked(const void *a, const void *b) {
    const ranked_t *x = (const ranked_t *)a, *y = (const ranked_t *)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return x < y ? -1 : (x > y);
}

/* Read set (session.py:1429-1438): the k largest of rank[0..n) (dead slots, mask == 0,
 * ranked as -inf), returned as ascending indices.  mask may be NULL. */
int oc_topk_ascending(const float *rank, const uint8_t *mask, int64_t n, int64_t k,
                      int64_t *out_idx) {
    if (k < 0 || k > n) return -1;
    ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)(n ? n : 1));
    if (!r) return -2;
    for (int64_t i = 0; i < n; ++i) {
        float v = (mask && !mask[i]) ? -INFINITY : rank[i];
        r[i].key = order_key(v);
        r[i].idx = i;
    }
    qsort(r, (size_t)n, sizeof(ranked_t), cmp_ranked);
    for (int64_t i = 0; i < k; ++i) out_idx[i] = r[i].idx;
    qsort(out_idx, (size_t)k, sizeof(int64_t), cmp_i64);
    free(r);
    return 0;
}

typedef struct {
    int64_t pos;
    int64_t idx;
} posidx_t;

static int cmp_posidx(const void *a, const void *b) {
    const posidx_t *x = (const posidx_t *)a, *y = (const posidx_t *)b;
    if (x->pos != y->pos) return x->pos < y->pos ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

/* Keep set of one (layer, batch, KV head) lane, eviction.py:355-409 (score-ranked
 * policies): the W = min(window, C) entries with the largest positions, plus the top
 * (C - W) of score among the rest, where positions < sink_tokens and pinned positions
 * [pin_lo, pin_hi) rank +inf; result = live-axis indices ordered by position.
 * Returns 0, or -1 on bad sizes. */
int oc_keep_select(const int64_t *pos, const float *score, int64_t n, int64_t capacity,
                   int64_t window, int64_t sink_tokens, int has_pin, int64_t pin_lo,
                   int64_t pin_hi, int64_t *out_idx) {
    if (capacity < 0 || capacity > n || window < 0) return -1;
    int64_t w = window < capacity ? window : capacity;
    int64_t rest = capacity - w;
    posidx_t *bypos = (posidx_t *)malloc(sizeof(posidx_t) * (size_t)(n ? n : 1));
    ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)(n ? n : 1));
    uint8_t *recent = (uint8_t *)calloc((size_t)(n ? n : 1), 1);
    posidx_t *kept = (posidx_t *)malloc(sizeof(posidx_t) * (size_t)(capacity ? capacity : 1));
    if (!bypos || !r || !recent || !kept) return -2;
    for (int64_t i = 0; i < n; ++i) {
        bypos[i].pos = pos[i];
        bypos[i].idx = i;
    }
    qsort(bypos, (size_t)n, sizeof(posidx_t), cmp_posidx);
    for (int64_t i = 0; i < w; ++i) recent[bypos[n - 1 - i].idx] = 1;
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (recent[i]) {
            kept[m].pos = pos[i];
            kept[m].idx = i;
            ++m;
        }
    }
    for (int64_t i = 0; i < n; ++i) {
        float v = score[i];
        if (pos[i] < sink_tokens) v = INFINITY;
        if (has_pin && pos[i] >= pin_lo && pos[i] < pin_hi) v = INFINITY;
        if (recent[i]) v = -INFINITY;
        r[i].key = order_key(v);
        r[i].idx = i;
    }
    qsort(r, (size_t)n, sizeof(ranked_t), cmp_ranked);
    for (int64_t i = 0; i < rest; ++i) {
        kept[m].pos = pos[r[i].idx];
        kept[m].idx = r[i].idx;
        ++m;
    }
    qsort(kept, (size_t)m, sizeof(posidx_t), cmp_posidx);
    for (int64_t i = 0; i < m; ++i) out_idx[i] = kept[i].idx;
    free(bypos);
    free(r);
    free(recent);
    free(kept);
    return 0;
}

/* Compaction of one lane (cache.py:342-367): rows dst[i] = src[keep[i]] for row_bytes
 * each; src and dst must not alias (the oracle copies out of place). */
void oc_compact_rows(const uint8_t *src, const int64_t *keep, int64_t c, int64_t row_bytes,
                     uint8_t *dst) {
    for (int64_t i = 0; i < c; ++i) {
        memcpy(dst + i * row_bytes, src + keep[i] * row_bytes, (size_t)row_bytes);
    }
}
