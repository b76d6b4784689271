/*
 * ORACLE -- test infrastructure, not product code.  See oracle.h for the contract.
 *
 * Pinning (what each function is checked against, in tests/):
 *   orc_f16_to_f32        reference KATs (tests/test_phase2a.cpp:94-100) + all 65536 inputs
 *                         against numpy's IEEE binary16 conversion
 *   orc_decode_q5_k_block reference KATs (test_phase2a.cpp:132-148) + the compiled reference
 *                         (oracle/_ref) on seeded random blocks, bit for bit
 *   orc_decode_q6_k_block reference KATs (test_phase2a.cpp:150-167), single-hot fixtures and
 *                         the compiled reference on random blocks
 *   orc_decode_q8_0_block reference KATs (test_phase2a.cpp:171-221) + compiled reference
 *   orc_decode_q4_k_block invariant: equals Q5_K decode of the same block with qh = 0
 *                         (checked against the compiled reference's Q5_K decoder) +
 *                         derived KATs (0.25 / 1.25 / -0.75) + single-hot scale packing
 *   orc_storage_dot/matvec reference KATs (4288, 8576, -192, 4480, 14, 64) + bitwise equality
 *                         with the compiled reference on random rows
 *   orc_storage_matmul_mt  m > 1: each output row bit-equal to the matvec of that activation
 *                         row (and to the compiled reference), for 1 and 4 threads
 *   orc_storage_dot_stats / orc_storage_matvec_stats  numpy float64 sums of w*x and |w*x| over
 *                         the decoded rows, every type, ragged sizes; planted wrong normalisers
 *                         (sum|w| max|x|, |sum w x|, half a row) are rejected by the same check
 *   orc_fnv1a64           the published FNV-1a-64 vectors ("", "a", "foobar")
 *   orc_quantize_row_q8_k  hand KATs and GGML invariants (|q| <= 127, q[argmax] = -127,
 *                         bsums, |d q - x| <= |d|/2, zero block, first-index tie break)
 *   orc_vec_dot_q8_k       algebraic identity with orc_storage_dot on the dequantized Q8_K
 *                         row (tolerance) + brute-force integer sums on tiny rows
 *   orc_rope              reference KATs (tests/test_phase1e.cpp:92-142) + the compiled
 *                         reference on seeded heads at text, multimodal and far positions, bit
 *                         for bit + identity at position 0 and per-pair norm preservation
 *   orc_attention_step    reference KATs (test_phase1e.cpp:144-186) + the compiled reference
 *                         over multi-step caches, bit for bit + one-token / equal-key / float64
 *                         softmax checks and the query-head to KV-head map
 *   orc_attention_block_step  the compiled reference block (qwen35_block.cpp:607-756) on
 *                         in-memory views, bit for bit (K-quant projections through its override
 *                         bridge) + the block KAT of test_phase2c.cpp:284-310
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_error[256];

static int fail(int code, const char* message) {
    snprintf(g_error, sizeof g_error, "%s", message);
    return code;
}

const char* orc_last_error(void) { return g_error; }

/* ---------------------------------------------------------------- registry */
/* GGML layout table: type id -> name, elements per block, bytes per block, quantized.
   The ids and geometries are GGML's on-disk format (ggml_type.cpp:12-54); ids with zero
   geometry are deprecated/removed and are reported as unregistered (ggml_type.cpp:69-75). */
typedef struct {
    const char* name;
    uint32_t block_elements;
    uint32_t bytes_per_block;
    int quantized;
} orc_layout_t;

static const orc_layout_t k_layouts[] = {
    {"f32", 1, 4, 0},         {"f16", 1, 2, 0},          {"q4_0", 32, 18, 1},
    {"q4_1", 32, 20, 1},      {"deprecated_q4_2", 0, 0, 0}, {"deprecated_q4_3", 0, 0, 0},
    {"q5_0", 32, 22, 1},      {"q5_1", 32, 24, 1},       {"q8_0", 32, 34, 1},
    {"q8_1", 32, 36, 1},      {"q2_K", 256, 84, 1},      {"q3_K", 256, 110, 1},
    {"q4_K", 256, 144, 1},    {"q5_K", 256, 176, 1},     {"q6_K", 256, 210, 1},
    {"q8_K", 256, 292, 1},    {"iq2_xxs", 256, 66, 1},   {"iq2_xs", 256, 74, 1},
    {"iq3_xxs", 256, 98, 1},  {"iq1_s", 256, 50, 1},     {"iq4_nl", 32, 18, 1},
    {"iq3_s", 256, 110, 1},   {"iq2_s", 256, 82, 1},     {"iq4_xs", 256, 136, 1},
    {"i8", 1, 1, 0},          {"i16", 1, 2, 0},          {"i32", 1, 4, 0},
    {"i64", 1, 8, 0},         {"f64", 1, 8, 0},          {"iq1_m", 256, 56, 1},
    {"bf16", 1, 2, 0},        {"removed_q4_0_4_4", 0, 0, 0}, {"removed_q4_0_4_8", 0, 0, 0},
    {"removed_q4_0_8_8", 0, 0, 0}, {"tq1_0", 256, 54, 1}, {"tq2_0", 256, 66, 1},
    {"removed_iq4_nl_4_4", 0, 0, 0}, {"removed_iq4_nl_4_8", 0, 0, 0},
    {"removed_iq4_nl_8_8", 0, 0, 0}, {"mxfp4", 32, 17, 1}, {"nvfp4", 64, 36, 1},
    {"q1_0", 128, 18, 1},     {"q2_0", 64, 18, 1},
};
#define ORC_LAYOUT_COUNT ((uint32_t)(sizeof k_layouts / sizeof k_layouts[0]))

/* ggml_type.cpp:69-75 */
int orc_type_layout(uint32_t type, uint64_t* block_elements, uint64_t* bytes_per_block,
                    int* quantized, const char** name) {
    if (type >= ORC_LAYOUT_COUNT || k_layouts[type].block_elements == 0 ||
        k_layouts[type].bytes_per_block == 0) {
        return fail(ORC_RUNTIME_ERROR, "unsupported GGML tensor type");
    }
    if (block_elements) *block_elements = k_layouts[type].block_elements;
    if (bytes_per_block) *bytes_per_block = k_layouts[type].bytes_per_block;
    if (quantized) *quantized = k_layouts[type].quantized;
    if (name) *name = k_layouts[type].name;
    return ORC_OK;
}

/* ggml_type.cpp:77-94: unknown type -> runtime_error; zero elements -> invalid_argument;
   ragged row -> runtime_error; overflow -> overflow_error */
int orc_row_byte_size(uint64_t row_elements, uint32_t type, uint64_t* out) {
    uint64_t be = 0, bpb = 0;
    int rc = orc_type_layout(type, &be, &bpb, NULL, NULL);
    if (rc != ORC_OK) return rc;
    if (row_elements == 0) {
        return fail(ORC_INVALID_ARGUMENT, "GGML tensor row must contain at least one element");
    }
    if (row_elements % be != 0) {
        return fail(ORC_RUNTIME_ERROR, "GGML tensor row length is not divisible by block size");
    }
    const uint64_t blocks = row_elements / be;
    if (blocks != 0 && bpb > UINT64_MAX / blocks) {
        return fail(ORC_OVERFLOW, "GGML row byte size overflow");
    }
    *out = blocks * bpb;
    return ORC_OK;
}

/* ---------------------------------------------------------------- scalars */
static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | ((uint16_t)p[1] << 8)); }

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* storage_decode.cpp:150-176: exact binary16 -> binary32, subnormals renormalised,
   infinities and NaN payloads kept by shifting the mantissa into place */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp5 = (h >> 10) & 0x1Fu;
    uint32_t frac = h & 0x3FFu;
    if (exp5 == 0x1Fu) return bits_to_f32(sign | 0x7F800000u | (frac << 13));
    if (exp5 != 0) return bits_to_f32(sign | ((exp5 + 112u) << 23) | (frac << 13));
    if (frac == 0) return bits_to_f32(sign);
    /* subnormal: value = frac * 2^-24; normalise so the leading one lands on bit 10 */
    uint32_t e = 113u; /* biased exponent of 2^-14 */
    while ((frac & 0x400u) == 0) {
        frac <<= 1;
        --e;
    }
    return bits_to_f32(sign | (e << 23) | ((frac & 0x3FFu) << 13));
}

/* storage_decode.cpp:178-180 */
float orc_bf16_to_f32(uint16_t bits) { return bits_to_f32((uint32_t)bits << 16); }

/* ---------------------------------------------------------------- block codecs */
/* storage_decode.cpp:44-61: 12 bytes hold eight 6-bit (scale, min) pairs.  Pairs 0..3 are the
   low six bits of bytes 0..3 (scale) and 4..7 (min); pairs 4..7 take their low nibbles from
   bytes 8..11 and their top two bits from the spare bits 6..7 of bytes 0..7. */
void orc_unpack_scale_min_k4(int j, const uint8_t* p, uint8_t* scale, uint8_t* minimum) {
    if (j < 4) {
        *scale = (uint8_t)(p[j] & 63u);
        *minimum = (uint8_t)(p[j + 4] & 63u);
    } else {
        *scale = (uint8_t)((p[j + 4] & 15u) | ((p[j - 4] >> 6) << 4));
        *minimum = (uint8_t)((p[j + 4] >> 4) | ((p[j] >> 6) << 4));
    }
}

/* GGML block_q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]} (144 B, registry
   ggml_type.cpp:25).  Not decoded by the reference (storage_decode.cpp:192-193 rejects it);
   this follows GGML's dequantize_row_q4_K, which is the reference's Q5_K decoder
   (storage_decode.cpp:63-94) without the high-bit plane and with qs at byte 16:
   element i -> group g = i/64, byte g*32 + i%32, low nibble if i%64 < 32 else high nibble,
   sub-block 2g (+1 for the high nibble); y = (d*sc)*q - dmin*m. */
void orc_decode_q4_k_block(const uint8_t* b, float* y) {
    const float d = orc_f16_to_f32(rd_u16(b));
    const float dmin = orc_f16_to_f32(rd_u16(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qs = b + 16;
    for (int g = 0; g < 4; ++g) {
        for (int half = 0; half < 2; ++half) {
            uint8_t s, m;
            orc_unpack_scale_min_k4(2 * g + half, sc, &s, &m);
            const float ds = d * (float)s;
            const float mm = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = qs[g * 32 + l];
                const unsigned q = half ? (unsigned)(byte >> 4) : (unsigned)(byte & 15u);
                y[g * 64 + half * 32 + l] = ds * (float)q - mm;
            }
        }
    }
}

/* storage_decode.cpp:63-94: {d@0, dmin@2, scales@4, qh[32]@16, qs[128]@48}; the fifth bit of
   element i is bit (2g + nibble) of qh[i%32]. */
void orc_decode_q5_k_block(const uint8_t* b, float* y) {
    const float d = orc_f16_to_f32(rd_u16(b));
    const float dmin = orc_f16_to_f32(rd_u16(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int g = 0; g < 4; ++g) {
        for (int half = 0; half < 2; ++half) {
            uint8_t s, m;
            orc_unpack_scale_min_k4(2 * g + half, sc, &s, &m);
            const float ds = d * (float)s;
            const float mm = dmin * (float)m;
            const unsigned bit = 1u << (2 * g + half);
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = qs[g * 32 + l];
                unsigned q = half ? (unsigned)(byte >> 4) : (unsigned)(byte & 15u);
                if (qh[l] & bit) q += 16u;
                y[g * 64 + half * 32 + l] = ds * (float)q - mm;
            }
        }
    }
}

/* storage_decode.cpp:96-125: {ql[128]@0, qh[64]@128, i8 sc[16]@192, f16 d@208}.  Element i:
   half h = i/128, segment s = (i%128)/32, lane l = i%32; low nibble from
   ql[64h + l + 32*(s&1)] (high nibble when s >= 2), two high bits (qh[32h + l] >> 2s) & 3,
   q = (low | high<<4) - 32, scale sc[8h + l/16 + 2s], y = (d*sc)*q. */
void orc_decode_q6_k_block(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = orc_f16_to_f32(rd_u16(b + 208));
    for (int h = 0; h < 2; ++h) {
        for (int s = 0; s < 4; ++s) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t lowbyte = ql[64 * h + l + 32 * (s & 1)];
                const unsigned low = (s >= 2) ? (unsigned)(lowbyte >> 4) : (unsigned)(lowbyte & 15u);
                const unsigned high = (unsigned)(qh[32 * h + l] >> (2 * s)) & 3u;
                const int q = (int)(low | (high << 4)) - 32;
                const int scale = sc[8 * h + l / 16 + 2 * s];
                y[128 * h + 32 * s + l] = d * (float)scale * (float)q;
            }
        }
    }
}

/* storage_decode.cpp:132-139: {f16 d; i8 qs[32]}, y = d*q */
void orc_decode_q8_0_block(const uint8_t* b, float* y) {
    const float d = orc_f16_to_f32(rd_u16(b));
    const int8_t* q = (const int8_t*)(b + 2);
    for (int i = 0; i < 32; ++i) y[i] = d * (float)q[i];
}

/* ---------------------------------------------------------------- rows */
static int decoder_supports(uint32_t type) {
    /* storage_decode.cpp:192-193 whitelist, plus Q4_K (the format the drop-in adds) */
    return type == ORC_TYPE_F32 || type == ORC_TYPE_F16 || type == ORC_TYPE_BF16 ||
           type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K || type == ORC_TYPE_Q6_K ||
           type == ORC_TYPE_Q8_0;
}

/* storage_decode.cpp:182-198: byte size checked first, then the type whitelist */
int orc_check_row(uint32_t type, uint64_t row_elements, uint64_t nbytes) {
    uint64_t expected = 0;
    int rc = orc_row_byte_size(row_elements, type, &expected);
    if (rc != ORC_OK) return rc;
    if (nbytes != expected) return fail(ORC_INVALID_ARGUMENT, "storage row byte size mismatch");
    if (!decoder_supports(type)) {
        return fail(ORC_INVALID_ARGUMENT, "storage decoder does not support GGML type");
    }
    return ORC_OK;
}

static uint32_t k_block_bytes(uint32_t type) {
    switch (type) {
        case ORC_TYPE_Q4_K: return ORC_Q4_K_BYTES;
        case ORC_TYPE_Q5_K: return ORC_Q5_K_BYTES;
        case ORC_TYPE_Q6_K: return ORC_Q6_K_BYTES;
        default: return 0;
    }
}

static void decode_kquant_block(uint32_t type, const uint8_t* b, float* y) {
    if (type == ORC_TYPE_Q4_K) orc_decode_q4_k_block(b, y);
    else if (type == ORC_TYPE_Q5_K) orc_decode_q5_k_block(b, y);
    else orc_decode_q6_k_block(b, y);
}

/* storage_decode.cpp:244-294 */
int orc_decode_row(uint32_t type, uint64_t n, const uint8_t* bytes, uint64_t nbytes, float* out) {
    int rc = orc_check_row(type, n, nbytes);
    if (rc != ORC_OK) return rc;
    if (type == ORC_TYPE_F32) {
        for (uint64_t i = 0; i < n; ++i) {
            uint32_t u;
            memcpy(&u, bytes + 4 * i, 4); /* little-endian host */
            out[i] = bits_to_f32(u);
        }
        return ORC_OK;
    }
    if (type == ORC_TYPE_F16 || type == ORC_TYPE_BF16) {
        for (uint64_t i = 0; i < n; ++i) {
            const uint16_t h = rd_u16(bytes + 2 * i);
            out[i] = type == ORC_TYPE_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
        }
        return ORC_OK;
    }
    if (type == ORC_TYPE_Q8_0) {
        for (uint64_t blk = 0; blk < n / 32; ++blk) {
            orc_decode_q8_0_block(bytes + blk * ORC_Q8_0_BYTES, out + blk * 32);
        }
        return ORC_OK;
    }
    const uint32_t bb = k_block_bytes(type);
    for (uint64_t blk = 0; blk < n / ORC_QK_K; ++blk) {
        decode_kquant_block(type, bytes + blk * bb, out + blk * ORC_QK_K);
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------- dot / matvec */
/* quantized_reference.cpp:24-82.  After validation, each block is decoded to F32 and
   accumulated lane by lane into a single F32 sum: sum = sum + w*x, in element order. */
static float dot_unchecked(uint32_t type, uint64_t n, const uint8_t* bytes, const float* x) {
    float sum = 0.0f;
    if (type == ORC_TYPE_F32 || type == ORC_TYPE_F16 || type == ORC_TYPE_BF16) {
        const unsigned width = type == ORC_TYPE_F32 ? 4u : 2u;
        for (uint64_t i = 0; i < n; ++i) {
            float w;
            if (type == ORC_TYPE_F32) {
                uint32_t u;
                memcpy(&u, bytes + 4 * i, 4);
                w = bits_to_f32(u);
            } else {
                const uint16_t h = rd_u16(bytes + (uint64_t)width * i);
                w = type == ORC_TYPE_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
            }
            sum += w * x[i];
        }
        return sum;
    }
    if (type == ORC_TYPE_Q8_0) {
        float w[32];
        for (uint64_t blk = 0; blk < n / 32; ++blk) {
            orc_decode_q8_0_block(bytes + blk * ORC_Q8_0_BYTES, w);
            const float* xb = x + blk * 32;
            for (int l = 0; l < 32; ++l) sum += w[l] * xb[l];
        }
        return sum;
    }
    float w[ORC_QK_K];
    const uint32_t bb = k_block_bytes(type);
    for (uint64_t blk = 0; blk < n / ORC_QK_K; ++blk) {
        decode_kquant_block(type, bytes + blk * bb, w);
        const float* xb = x + blk * ORC_QK_K;
        for (int l = 0; l < ORC_QK_K; ++l) sum += w[l] * xb[l];
    }
    return sum;
}

int orc_storage_dot(uint32_t type, uint64_t n, const uint8_t* bytes, uint64_t nbytes,
                    const float* x, float* out) {
    int rc = orc_check_row(type, n, nbytes);
    if (rc != ORC_OK) return rc;
    *out = dot_unchecked(type, n, bytes, x);
    return ORC_OK;
}

/* quantized_reference.cpp:128-153: argument checks before any write */
static int check_matvec(uint32_t type, uint64_t rows, uint64_t cols, uint64_t nbytes,
                        uint64_t* row_bytes) {
    if (rows == 0 || cols == 0) {
        return fail(ORC_INVALID_ARGUMENT, "reference matvec dimensions must be non-zero");
    }
    int rc = orc_row_byte_size(cols, type, row_bytes);
    if (rc != ORC_OK) return rc;
    if (*row_bytes != 0 && rows > UINT64_MAX / *row_bytes) {
        return fail(ORC_OVERFLOW, "reference matvec matrix size overflow");
    }
    if (nbytes != rows * *row_bytes) {
        return fail(ORC_INVALID_ARGUMENT, "reference matvec matrix byte size mismatch");
    }
    return orc_check_row(type, cols, *row_bytes);
}

int orc_storage_matvec(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                       uint64_t nbytes, const float* x, float* y) {
    uint64_t rb = 0;
    int rc = check_matvec(type, rows, cols, nbytes, &rb);
    if (rc != ORC_OK) return rc;
    for (uint64_t r = 0; r < rows; ++r) y[r] = dot_unchecked(type, cols, matrix + r * rb, x);
    return ORC_OK;
}

typedef struct {
    uint32_t type;
    uint64_t cols, row_bytes, rows;
    uint64_t job_begin, job_end; /* flat index over (m, row) */
    const uint8_t* matrix;
    const float* x;
    float* y;
    double* dot_f64;
    double* abs_sum;
} orc_job_t;

static void* matvec_worker(void* arg) {
    orc_job_t* j = (orc_job_t*)arg;
    for (uint64_t t = j->job_begin; t < j->job_end; ++t) {
        const uint64_t m = t / j->rows, r = t % j->rows;
        j->y[t] = dot_unchecked(j->type, j->cols, j->matrix + r * j->row_bytes, j->x + m * j->cols);
    }
    return NULL;
}

static int run_jobs(orc_job_t* base, uint64_t total, int threads, void* (*fn)(void*)) {
    if (threads < 1) threads = 1;
    if ((uint64_t)threads > total) threads = (int)total;
    pthread_t tid[256];
    orc_job_t jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        jobs[t] = *base;
        jobs[t].job_begin = total * (uint64_t)t / (uint64_t)threads;
        jobs[t].job_end = total * (uint64_t)(t + 1) / (uint64_t)threads;
    }
    int started = 0;
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tid[t], NULL, fn, &jobs[t]) != 0) break;
        started = t;
    }
    fn(&jobs[0]);
    for (int t = 1; t <= started; ++t) pthread_join(tid[t], NULL);
    for (int t = started + 1; t < threads; ++t) fn(&jobs[t]); /* threads that failed to start */
    return ORC_OK;
}

int orc_storage_matvec_mt(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                          uint64_t nbytes, const float* x, float* y, int threads) {
    return orc_storage_matmul_mt(type, rows, cols, matrix, nbytes, 1, x, y, threads);
}

int orc_storage_matmul_mt(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                          uint64_t nbytes, uint64_t m, const float* x, float* y, int threads) {
    uint64_t rb = 0;
    int rc = check_matvec(type, rows, cols, nbytes, &rb);
    if (rc != ORC_OK) return rc;
    if (m == 0) return fail(ORC_INVALID_ARGUMENT, "matmul batch must be non-zero");
    orc_job_t base = {type, cols, rb, rows, 0, 0, matrix, x, y, NULL, NULL};
    return run_jobs(&base, m * rows, threads, matvec_worker);
}

/* decoded row . x in double, and sum |w x| (the per-output normaliser of the tolerance) */
static void dot_stats_unchecked(uint32_t type, uint64_t n, const uint8_t* bytes, const float* x,
                                double* dot, double* abs_sum) {
    double s = 0.0, a = 0.0;
    float w[ORC_QK_K];
    uint64_t step = (type == ORC_TYPE_Q8_0) ? 32 : ORC_QK_K;
    if (type == ORC_TYPE_F32 || type == ORC_TYPE_F16 || type == ORC_TYPE_BF16) step = 1;
    uint64_t bb = 0;
    orc_row_byte_size(step, type, &bb);
    for (uint64_t blk = 0; blk < n / step; ++blk) {
        orc_decode_row(type, step, bytes + blk * bb, bb, w);
        for (uint64_t l = 0; l < step; ++l) {
            const double p = (double)w[l] * (double)x[blk * step + l];
            s += p;
            a += fabs(p);
        }
    }
    *dot = s;
    *abs_sum = a;
}

int orc_storage_dot_stats(uint32_t type, uint64_t n, const uint8_t* bytes, uint64_t nbytes,
                          const float* x, double* dot_f64, double* abs_sum) {
    int rc = orc_check_row(type, n, nbytes);
    if (rc != ORC_OK) return rc;
    dot_stats_unchecked(type, n, bytes, x, dot_f64, abs_sum);
    return ORC_OK;
}

static void* stats_worker(void* arg) {
    orc_job_t* j = (orc_job_t*)arg;
    for (uint64_t t = j->job_begin; t < j->job_end; ++t) {
        dot_stats_unchecked(j->type, j->cols, j->matrix + t * j->row_bytes, j->x, &j->dot_f64[t],
                            &j->abs_sum[t]);
    }
    return NULL;
}

int orc_storage_matvec_stats(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                             uint64_t nbytes, const float* x, double* dot_f64, double* abs_sum,
                             int threads) {
    uint64_t rb = 0;
    int rc = check_matvec(type, rows, cols, nbytes, &rb);
    if (rc != ORC_OK) return rc;
    orc_job_t base = {type, cols, rb, rows, 0, 0, matrix, x, NULL, dot_f64, abs_sum};
    return run_jobs(&base, rows, threads, stats_worker);
}

/* ---------------------------------------------------------------- Q8_K */
/* GGML quantize_row_q8_K (published algorithm; the reference registers the layout only,
   ggml_type.cpp:28).  Per 256-block: amax = max |x|, `max` = the x at the FIRST index that
   reaches amax; amax == 0 -> d = 0 and all-zero qs (bsums are defined as 0 here; GGML leaves
   them unwritten).  Otherwise iscale = -127/max, q = min(127, nearest(iscale*x)),
   bsums[j] = sum of q[16j..16j+15], d = 1/iscale.  nearest() is GGML's round-to-nearest-even
   by adding 1.5*2^23 and reading the low mantissa bits, valid for |v| < 2^22. */
static int nearest_int(float v) {
    const float t = v + 12582912.0f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007FFFFF) - 0x00400000;
}

int orc_quantize_row_q8_k(const float* x, uint64_t k, uint8_t* out) {
    if (k == 0 || k % ORC_QK_K != 0) {
        return fail(ORC_INVALID_ARGUMENT, "Q8_K quantization needs a multiple of 256 values");
    }
    for (uint64_t blk = 0; blk < k / ORC_QK_K; ++blk) {
        const float* xb = x + blk * ORC_QK_K;
        uint8_t* ob = out + blk * ORC_Q8_K_BYTES;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < ORC_QK_K; ++i) {
            const float ax = fabsf(xb[i]);
            if (ax > amax) {
                amax = ax;
                max = xb[i];
            }
        }
        int8_t q[ORC_QK_K];
        int16_t bsums[16];
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(q, 0, sizeof q);
            memset(bsums, 0, sizeof bsums);
        } else {
            const float iscale = -127.0f / max;
            for (int i = 0; i < ORC_QK_K; ++i) {
                const int v = nearest_int(iscale * xb[i]);
                q[i] = (int8_t)(v < 127 ? v : 127);
            }
            for (int j = 0; j < 16; ++j) {
                int s = 0;
                for (int i = 0; i < 16; ++i) s += q[16 * j + i];
                bsums[j] = (int16_t)s;
            }
            d = 1.0f / iscale;
        }
        memcpy(ob, &d, 4);
        memcpy(ob + 4, q, 256);
        memcpy(ob + 260, bsums, 32);
    }
    return ORC_OK;
}

int orc_dequantize_row_q8_k(const uint8_t* blocks, uint64_t k, float* out) {
    if (k == 0 || k % ORC_QK_K != 0) {
        return fail(ORC_INVALID_ARGUMENT, "Q8_K row needs a multiple of 256 values");
    }
    for (uint64_t blk = 0; blk < k / ORC_QK_K; ++blk) {
        const uint8_t* b = blocks + blk * ORC_Q8_K_BYTES;
        float d;
        memcpy(&d, b, 4);
        const int8_t* q = (const int8_t*)(b + 4);
        for (int i = 0; i < ORC_QK_K; ++i) out[blk * ORC_QK_K + i] = d * (float)q[i];
    }
    return ORC_OK;
}

/* GGML vec_dot_q{4,5,6}_K_q8_K and vec_dot_q8_0 semantics, restated per super-block:
   Q4_K/Q5_K: d_w*d_x * sum_j sc_j * (sum_32 q*q8)  -  dmin_w*d_x * sum_j m_j * (bsum_2j + bsum_2j+1)
   Q6_K:      d_w*d_x * sum_16groups sc_g * sum_16 (q-32)*q8
   Super-block partials are summed in F32 in block order. */
int orc_vec_dot_q8_k(uint32_t type, uint64_t k, const uint8_t* w, const uint8_t* q8k, float* out) {
    if (type != ORC_TYPE_Q4_K && type != ORC_TYPE_Q5_K && type != ORC_TYPE_Q6_K) {
        return fail(ORC_RUNTIME_ERROR, "integer Q8_K dot supports q4_K, q5_K and q6_K");
    }
    if (k == 0 || k % ORC_QK_K != 0) return fail(ORC_INVALID_ARGUMENT, "bad row length");
    const uint32_t bb = k_block_bytes(type);
    float sum = 0.0f;
    for (uint64_t blk = 0; blk < k / ORC_QK_K; ++blk) {
        const uint8_t* b = w + blk * bb;
        const uint8_t* a = q8k + blk * ORC_Q8_K_BYTES;
        float dx;
        memcpy(&dx, a, 4);
        const int8_t* q8 = (const int8_t*)(a + 4);
        int16_t bs[16];
        memcpy(bs, a + 260, 32);
        if (type == ORC_TYPE_Q6_K) {
            const float d = orc_f16_to_f32(rd_u16(b + 208));
            const int8_t* sc = (const int8_t*)(b + 192);
            int32_t isum = 0;
            for (int i = 0; i < ORC_QK_K; ++i) {
                const int h = i / 128, s = (i % 128) / 32, l = i % 32;
                const uint8_t lb = b[64 * h + l + 32 * (s & 1)];
                const unsigned low = (s >= 2) ? (unsigned)(lb >> 4) : (unsigned)(lb & 15u);
                const unsigned high = (unsigned)(b[128 + 32 * h + l] >> (2 * s)) & 3u;
                const int q = (int)(low | (high << 4)) - 32;
                isum += sc[8 * h + l / 16 + 2 * s] * q * q8[i];
            }
            sum += d * dx * (float)isum;
        } else {
            const float d = orc_f16_to_f32(rd_u16(b));
            const float dmin = orc_f16_to_f32(rd_u16(b + 2));
            const uint8_t* qs = b + (type == ORC_TYPE_Q4_K ? 16 : 48);
            int32_t isum = 0, imin = 0;
            for (int j = 0; j < 8; ++j) {
                uint8_t s, m;
                orc_unpack_scale_min_k4(j, b + 4, &s, &m);
                int32_t part = 0;
                for (int l = 0; l < 32; ++l) {
                    const int i = 64 * (j / 2) + 32 * (j & 1) + l;
                    const uint8_t byte = qs[32 * (j / 2) + l];
                    int q = (j & 1) ? (byte >> 4) : (byte & 15);
                    if (type == ORC_TYPE_Q5_K && (b[16 + l] & (1u << j))) q += 16;
                    part += q * q8[i];
                }
                isum += (int32_t)s * part;
                imin += (int32_t)m * (bs[2 * j] + bs[2 * j + 1]);
            }
            sum += d * dx * (float)isum - dmin * dx * (float)imin;
        }
    }
    *out = sum;
    return ORC_OK;
}

uint64_t orc_fnv1a64(const void* data, uint64_t n) {
    const uint8_t* p = (const uint8_t*)data;
    uint64_t h = 14695981039346656037ull;
    for (uint64_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

/* ---------------------------------------------------------------- Gated DeltaNet decode block */

/* qwen35_block.cpp:138-145: branch on the sign so exp never overflows */
float orc_sigmoid(float v) {
    if (v >= 0.0f) {
        const float e = expf(-v);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(v);
    return e / (1.0f + e);
}

/* qwen35_block.cpp:147-155 */
float orc_softplus(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

/* qwen35_block.cpp:157-159 */
float orc_silu(float v) { return v * orc_sigmoid(v); }

/* qwen35_block.cpp:161-186: sum of squares in double, inverse_rms rounded to F32, then
   (x * inverse_rms) * weight in F32 */
int orc_rms_norm_rows(const float* in, const float* weight, uint64_t n, uint64_t width, float eps,
                      float* out) {
    if (width == 0 || n % width != 0) return fail(ORC_INVALID_ARGUMENT, "Qwen3.5 RMSNorm dimensions are incompatible");
    if (!(eps > 0.0f) || !isfinite(eps)) return fail(ORC_INVALID_ARGUMENT, "Qwen3.5 RMSNorm epsilon must be positive and finite");
    for (uint64_t r = 0; r < n / width; ++r) {
        const float* x = in + r * width;
        double ss = 0.0;
        for (uint64_t c = 0; c < width; ++c) ss += (double)x[c] * (double)x[c];
        const double mean = ss / (double)width;
        const float inv = (float)(1.0 / sqrt(mean + (double)eps));
        for (uint64_t c = 0; c < width; ++c) out[r * width + c] = x[c] * inv * weight[c];
    }
    return ORC_OK;
}

/* reference_kernels.cpp:197-225: shift the channel's history left, append the input, dot in
   double with the channel's kernel taps */
int orc_conv_step(const float* input, const float* weights, uint64_t channels, uint64_t kernel,
                  float* history, float* out, int apply_silu) {
    if (channels == 0 || kernel == 0) return fail(ORC_INVALID_ARGUMENT, "depthwise convolution dimensions do not match SSM state");
    for (uint64_t c = 0; c < channels; ++c) {
        float* h = history + c * kernel;
        for (uint64_t i = 1; i < kernel; ++i) h[i - 1] = h[i];
        h[kernel - 1] = input[c];
        double sum = 0.0;
        for (uint64_t i = 0; i < kernel; ++i) sum += (double)h[i] * (double)weights[c * kernel + i];
        const float v = (float)sum;
        out[c] = apply_silu ? v * orc_sigmoid(v) : v;
    }
    return ORC_OK;
}

/* reference_kernels.cpp:227-335, per head: L2-normalise q and k (norms in double,
   1 / max(norm, eps) rounded to F32, q also scaled by 1/sqrt(dk)); decay the state by
   exp(log_decay); memory = state^T k (F32, key order); delta = (v - memory) * beta;
   state += k outer delta; out = state^T q (double accumulation, key order) */
int orc_gated_delta_step(const float* q, const float* k, const float* v, const float* beta,
                         const float* log_decay, uint64_t heads, uint64_t dk, uint64_t dv,
                         float eps, float* state, float* out) {
    if (!(eps > 0.0f)) return fail(ORC_INVALID_ARGUMENT, "gated delta normalization epsilon must be positive");
    if (heads == 0 || dk == 0 || dv == 0) return fail(ORC_INVALID_ARGUMENT, "gated_delta_step dimensions do not match SSM state");
    float* nq = (float*)malloc(dk * sizeof(float));
    float* nk = (float*)malloc(dk * sizeof(float));
    float* mem = (float*)malloc(dv * sizeof(float));
    float* delta = (float*)malloc(dv * sizeof(float));
    if (!nq || !nk || !mem || !delta) {
        free(nq); free(nk); free(mem); free(delta);
        return fail(ORC_RUNTIME_ERROR, "out of memory");
    }
    const float query_scale = 1.0f / sqrtf((float)dk);
    int rc = ORC_OK;
    for (uint64_t h = 0; h < heads; ++h) {
        if (!(beta[h] >= 0.0f && beta[h] <= 1.0f) || !isfinite(beta[h]) || !isfinite(log_decay[h])) {
            rc = fail(ORC_INVALID_ARGUMENT, "gated delta beta/decay values are invalid");
            break;
        }
        const float* qh = q + h * dk;
        const float* kh = k + h * dk;
        double qn = 0.0, kn = 0.0;
        for (uint64_t d = 0; d < dk; ++d) {
            qn += (double)qh[d] * (double)qh[d];
            kn += (double)kh[d] * (double)kh[d];
        }
        const double ql = sqrt(qn), kl = sqrt(kn);
        const float iq = (float)(1.0 / (ql > (double)eps ? ql : (double)eps));
        const float ik = (float)(1.0 / (kl > (double)eps ? kl : (double)eps));
        for (uint64_t d = 0; d < dk; ++d) {
            nq[d] = qh[d] * iq * query_scale;
            nk[d] = kh[d] * ik;
        }
        const float decay = expf(log_decay[h]);
        float* s = state + h * dk * dv;
        for (uint64_t i = 0; i < dk * dv; ++i) s[i] *= decay;
        for (uint64_t j = 0; j < dv; ++j) mem[j] = 0.0f;
        for (uint64_t d = 0; d < dk; ++d)
            for (uint64_t j = 0; j < dv; ++j) mem[j] += s[d * dv + j] * nk[d];
        for (uint64_t j = 0; j < dv; ++j) delta[j] = (v[h * dv + j] - mem[j]) * beta[h];
        for (uint64_t d = 0; d < dk; ++d)
            for (uint64_t j = 0; j < dv; ++j) s[d * dv + j] += nk[d] * delta[j];
        for (uint64_t j = 0; j < dv; ++j) {
            double sum = 0.0;
            for (uint64_t d = 0; d < dk; ++d) sum += (double)s[d * dv + j] * (double)nq[d];
            out[h * dv + j] = (float)sum;
        }
    }
    free(nq); free(nk); free(mem); free(delta);
    return rc;
}

static int is_kquant(uint32_t type) {
    return type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K || type == ORC_TYPE_Q6_K;
}

/* one projection of the block: rows x cols weight against x (see oracle.h for the semantics) */
static int block_matvec(uint32_t type, const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                        float* y, int threads) {
    uint64_t rb = 0;
    int rc = orc_row_byte_size(cols, type, &rb);
    if (rc != ORC_OK) return rc;
    const float* xin = x;
    float* xhat = NULL;
    if (is_kquant(type)) {
        uint8_t* blocks = (uint8_t*)malloc(cols / ORC_QK_K * ORC_Q8_K_BYTES);
        xhat = (float*)malloc(cols * sizeof(float));
        if (!blocks || !xhat) {
            free(blocks); free(xhat);
            return fail(ORC_RUNTIME_ERROR, "out of memory");
        }
        rc = orc_quantize_row_q8_k(x, cols, blocks);
        if (rc == ORC_OK) rc = orc_dequantize_row_q8_k(blocks, cols, xhat);
        free(blocks);
        if (rc != ORC_OK) {
            free(xhat);
            return rc;
        }
        xin = xhat;
    }
    rc = orc_storage_matvec_mt(type, rows, cols, w, rows * rb, xin, y, threads);
    free(xhat);
    return rc;
}

uint64_t orc_deltanet_trace_size(const orc_deltanet_block* b) {
    const uint64_t C = 2 * b->key_heads * b->key_dim + b->value_heads * b->value_dim;
    const uint64_t V = b->value_heads * b->value_dim;
    return 2 * C + 3 * V + 4 * b->value_heads + 4 * b->embedding + 3 * b->ffn;
}

/* qwen35_block.cpp:406-605 (recurrent block), :326-352 (finish_block), :296-324 (MLP) */
int orc_deltanet_step(const orc_deltanet_block* b, float* conv_history, float* state,
                      const float* x, float* y, float* trace, int threads) {
    const uint64_t E = b->embedding, Hk = b->key_heads, Hv = b->value_heads, dk = b->key_dim,
                   dv = b->value_dim, F = b->ffn;
    if (E == 0 || Hk == 0 || Hv == 0 || dk == 0 || dv == 0 || F == 0 || b->conv_kernel == 0 || Hv % Hk != 0)
        return fail(ORC_INVALID_ARGUMENT, "Qwen3.5 recurrent block dimensions are incompatible");
    const uint64_t KW = Hk * dk, V = Hv * dv, C = 2 * KW + V;
    float* buf = (float*)calloc(orc_deltanet_trace_size(b) + E + 2 * Hv * dk, sizeof(float));
    if (!buf) return fail(ORC_RUNTIME_ERROR, "out of memory");
    float *qkv = buf, *z = qkv + C, *beta = z + V, *alpha = beta + Hv, *conv = alpha + Hv, *rec = conv + C,
          *gated = rec + V, *branch = gated + V, *resid = branch + E, *post = resid + E, *gate = post + E,
          *up = gate + F, *act = up + F, *ffn = act + F, *beta_s = ffn + E, *log_decay = beta_s + Hv,
          *normed = log_decay + Hv, *query = normed + E, *key = query + Hv * dk;
    int rc = orc_rms_norm_rows(x, b->input_norm, E, E, b->eps, normed);
    if (rc == ORC_OK) rc = block_matvec(b->qkv_type, b->qkv, C, E, normed, qkv, threads);
    if (rc == ORC_OK) rc = block_matvec(b->z_type, b->z, V, E, normed, z, threads);
    if (rc == ORC_OK) rc = block_matvec(b->beta_type, b->beta, Hv, E, normed, beta, threads);
    if (rc == ORC_OK) rc = block_matvec(b->alpha_type, b->alpha, Hv, E, normed, alpha, threads);
    if (rc == ORC_OK) {
        for (uint64_t h = 0; h < Hv; ++h) {
            beta_s[h] = orc_sigmoid(beta[h]);
            log_decay[h] = orc_softplus(alpha[h] + b->dt_bias[h]) * b->decay[h];
        }
        rc = orc_conv_step(qkv, b->conv_weight, C, b->conv_kernel, conv_history, conv, 0);
    }
    if (rc == ORC_OK) {
        for (uint64_t c = 0; c < C; ++c) conv[c] = orc_silu(conv[c]);
        /* repeat_heads_tiled (qwen35_block.cpp:233-251): value head t takes key head t % Hk */
        for (uint64_t t = 0; t < Hv; ++t) {
            memcpy(query + t * dk, conv + (t % Hk) * dk, dk * sizeof(float));
            memcpy(key + t * dk, conv + KW + (t % Hk) * dk, dk * sizeof(float));
        }
        rc = orc_gated_delta_step(query, key, conv + 2 * KW, beta_s, log_decay, Hv, dk, dv, b->eps, state, rec);
    }
    if (rc == ORC_OK) rc = orc_rms_norm_rows(rec, b->out_norm, V, dv, b->eps, gated);
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < V; ++i) gated[i] *= orc_silu(z[i]);
        rc = block_matvec(b->out_type, b->out, E, V, gated, branch, threads);
    }
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < E; ++i) resid[i] = x[i] + branch[i];
        rc = orc_rms_norm_rows(resid, b->post_norm, E, E, b->eps, post);
    }
    if (rc == ORC_OK) rc = block_matvec(b->gate_type, b->gate, F, E, post, gate, threads);
    if (rc == ORC_OK) rc = block_matvec(b->up_type, b->up, F, E, post, up, threads);
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < F; ++i) act[i] = orc_silu(gate[i]) * up[i];
        rc = block_matvec(b->down_type, b->down, E, F, act, ffn, threads);
    }
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < E; ++i) y[i] = resid[i] + ffn[i];
        if (trace) memcpy(trace, buf, orc_deltanet_trace_size(b) * sizeof(float));
    }
    free(buf);
    return rc;
}

/* ---------------------------------------------------------------- full-attention decode */

/* reference_kernels.cpp:28-40: frequency f takes the height coordinate when f % 3 == 1 and
   f / 3 < sections[1], the width coordinate when f % 3 == 2 and f / 3 < sections[2], else the
   temporal one */
static uint64_t rope_coordinate(uint64_t f, const uint64_t position[3], const int32_t sections[4]) {
    if (f % 3 == 1 && f / 3 < (uint64_t)sections[1]) return position[1];
    if (f % 3 == 2 && f / 3 < (uint64_t)sections[2]) return position[2];
    return position[0];
}

/* reference_kernels.cpp:77-125 */
int orc_rope(float* heads, uint64_t n_heads, uint64_t head_dim, uint64_t rotary_dim, const int32_t sections[4],
             float base, const uint64_t position[3]) {
    if (rotary_dim == 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim)
        return fail(ORC_INVALID_ARGUMENT, "RoPE dimension must be non-zero, even, and within head width");
    if (!(base > 0.0f) || !isfinite(base))
        return fail(ORC_INVALID_ARGUMENT, "RoPE frequency base must be positive and finite");
    int64_t total = 0;
    for (int i = 0; i < 4; ++i) {
        if (sections[i] < 0) return fail(ORC_INVALID_ARGUMENT, "RoPE dimension sections must be non-negative");
        total += sections[i];
    }
    if (total != (int64_t)(rotary_dim / 2))
        return fail(ORC_INVALID_ARGUMENT, "RoPE dimension sections must sum to half the rotary dimension");
    const uint64_t half = rotary_dim / 2;
    for (uint64_t h = 0; h < n_heads; ++h) {
        float* x = heads + h * head_dim;
        for (uint64_t f = 0; f < half; ++f) {
            const double exponent = (2.0 * (double)f) / (double)rotary_dim;
            const double inv_freq = 1.0 / pow((double)base, exponent);
            const double angle = (double)rope_coordinate(f, position, sections) * inv_freq;
            const float c = (float)cos(angle), s = (float)sin(angle);
            const float a = x[f], b = x[half + f];
            x[f] = a * c - b * s;
            x[half + f] = b * c + a * s;
        }
    }
    return ORC_OK;
}

/* reference_kernels.cpp:127-195 with KvCache::append (hybrid_cache.cpp:154-169) */
int orc_attention_step(const float* q, uint64_t q_heads, const float* k, const float* v, orc_kv_cache* c,
                       float* out) {
    const uint64_t Hkv = c->kv_heads, dk = c->key_dim, dv = c->value_dim;
    if (Hkv == 0 || q_heads % Hkv != 0) return fail(ORC_INVALID_ARGUMENT, "causal_attention_step dimensions are incompatible");
    if (c->length >= c->capacity) return fail(ORC_OVERFLOW, "KV cache capacity exceeded");
    memcpy(c->keys + c->length * Hkv * dk, k, Hkv * dk * sizeof(float));
    memcpy(c->values + c->length * Hkv * dv, v, Hkv * dv * sizeof(float));
    c->length += 1;
    const uint64_t T = c->length, rep = q_heads / Hkv;
    const float scale = 1.0f / sqrtf((float)dk);
    float* scores = (float*)malloc(T * sizeof(float));
    if (!scores) return fail(ORC_RUNTIME_ERROR, "out of memory");
    for (uint64_t i = 0; i < q_heads * dv; ++i) out[i] = 0.0f;
    int rc = ORC_OK;
    for (uint64_t h = 0; h < q_heads && rc == ORC_OK; ++h) {
        const uint64_t g = h / rep;
        const float* qh = q + h * dk;
        float maximum = -INFINITY;
        for (uint64_t t = 0; t < T; ++t) {
            const float* kt = c->keys + (t * Hkv + g) * dk;
            double dot = 0.0;
            for (uint64_t d = 0; d < dk; ++d) dot += (double)qh[d] * (double)kt[d];
            scores[t] = (float)dot * scale;
            if (scores[t] > maximum) maximum = scores[t];
        }
        double denominator = 0.0;
        for (uint64_t t = 0; t < T; ++t) {
            scores[t] = expf(scores[t] - maximum);
            denominator += (double)scores[t];
        }
        if (!(denominator > 0.0) || !isfinite(denominator)) {
            rc = fail(ORC_RUNTIME_ERROR, "causal attention softmax normalization failed");
            break;
        }
        float* oh = out + h * dv;
        for (uint64_t t = 0; t < T; ++t) {
            const float p = (float)((double)scores[t] / denominator);
            const float* vt = c->values + (t * Hkv + g) * dv;
            for (uint64_t d = 0; d < dv; ++d) oh[d] += p * vt[d];
        }
    }
    free(scores);
    return rc;
}

uint64_t orc_attention_trace_size(const orc_attention_block* b) {
    const uint64_t Q = b->q_heads * b->head_dim, KV = b->kv_heads * b->head_dim;
    return 6 * Q + 3 * KV + 4 * b->embedding + 3 * b->ffn;
}

/* qwen35_block.cpp:607-756 (attention block), :326-352 (finish_block), :296-324 (MLP) */
int orc_attention_block_step(const orc_attention_block* b, orc_kv_cache* cache, const uint64_t position[3],
                             const float* x, float* y, float* trace, int threads) {
    const uint64_t E = b->embedding, Hq = b->q_heads, Hkv = b->kv_heads, D = b->head_dim, F = b->ffn;
    if (E == 0 || Hq == 0 || Hkv == 0 || D == 0 || F == 0)
        return fail(ORC_INVALID_ARGUMENT, "Qwen3.5 attention block dimensions are incompatible");
    if (cache->kv_heads != Hkv || cache->key_dim != D || cache->value_dim != D)
        return fail(ORC_INVALID_ARGUMENT, "Qwen3.5 attention cache dimensions do not match the manifest");
    const uint64_t Q = Hq * D, KV = Hkv * D;
    float* buf = (float*)calloc(orc_attention_trace_size(b) + E, sizeof(float));
    if (!buf) return fail(ORC_RUNTIME_ERROR, "out of memory");
    float *qfull = buf, *kp = qfull + 2 * Q, *vp = kp + KV, *qcur = vp + KV, *kcur = qcur + Q, *pregate = kcur + KV,
          *gate_s = pregate + Q, *gated = gate_s + Q, *branch = gated + Q, *resid = branch + E, *post = resid + E,
          *gate = post + E, *up = gate + F, *act = up + F, *ffn = act + F, *normed = ffn + E;
    int rc = orc_rms_norm_rows(x, b->input_norm, E, E, b->eps, normed);
    if (rc == ORC_OK) rc = block_matvec(b->q_type, b->q, 2 * Q, E, normed, qfull, threads);
    if (rc == ORC_OK) rc = block_matvec(b->k_type, b->k, KV, E, normed, kp, threads);
    if (rc == ORC_OK) rc = block_matvec(b->v_type, b->v, KV, E, normed, vp, threads);
    if (rc == ORC_OK) {
        /* per head: D query values, then D gate values (qwen35_block.cpp:671-685) */
        for (uint64_t h = 0; h < Hq; ++h) {
            memcpy(qcur + h * D, qfull + h * 2 * D, D * sizeof(float));
            memcpy(gate_s + h * D, qfull + h * 2 * D + D, D * sizeof(float));
        }
        rc = orc_rms_norm_rows(qcur, b->q_norm, Q, D, b->eps, qcur);
    }
    if (rc == ORC_OK) rc = orc_rms_norm_rows(kp, b->k_norm, KV, D, b->eps, kcur);
    if (rc == ORC_OK) rc = orc_rope(qcur, Hq, D, b->rope_dim, b->rope_sections, b->rope_base, position);
    if (rc == ORC_OK) rc = orc_rope(kcur, Hkv, D, b->rope_dim, b->rope_sections, b->rope_base, position);
    if (rc == ORC_OK) rc = orc_attention_step(qcur, Hq, kcur, vp, cache, pregate);
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < Q; ++i) {
            const float g = orc_sigmoid(gate_s[i]);
            gate_s[i] = g;
            gated[i] = pregate[i] * g;
        }
        rc = block_matvec(b->out_type, b->out, E, Q, gated, branch, threads);
    }
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < E; ++i) resid[i] = x[i] + branch[i];
        rc = orc_rms_norm_rows(resid, b->post_norm, E, E, b->eps, post);
    }
    if (rc == ORC_OK) rc = block_matvec(b->gate_type, b->gate, F, E, post, gate, threads);
    if (rc == ORC_OK) rc = block_matvec(b->up_type, b->up, F, E, post, up, threads);
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < F; ++i) act[i] = orc_silu(gate[i]) * up[i];
        rc = block_matvec(b->down_type, b->down, E, F, act, ffn, threads);
    }
    if (rc == ORC_OK) {
        for (uint64_t i = 0; i < E; ++i) y[i] = resid[i] + ffn[i];
        if (trace) memcpy(trace, buf, orc_attention_trace_size(b) * sizeof(float));
    }
    free(buf);
    return rc;
}
