/*
 * CPU oracle for the quantized-linear hot path. TEST INFRASTRUCTURE ONLY:
 * it is loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg as a checker, never by the product library or its Python package.
 *
 * Plain C restatements of the reference's device arithmetic, in the
 * reference's association order. Built with -ffp-contract=off so the only
 * fused multiply-adds are the explicit fmaf() calls (glibc's fmaf is the
 * correctly rounded IEEE operation), and with default round-to-nearest-even.
 *
 * Citations are to /root/reference/src/venturi/ops/csrc/.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---- IEEE half / bfloat16 conversions (round to nearest even) ---------- */

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { ++e; man <<= 1; } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan */
        return sign | 0x7c00u | (ax > 0x7f800000u ? (uint16_t)(0x200u | ((ax >> 13) & 0x3ffu)) : 0);
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) { /* result is subnormal or zero in fp16 */
        if (ax < 0x33000000u) return sign; /* < 2^-25: rounds to 0 (tie at 2^-25 -> even 0) */
        const int e = (int)(ax >> 23);
        const uint32_t man = (ax & 0x7fffffu) | 0x800000u;
        /* value = man * 2^(e-150); in units of 2^-24 that is man >> (126-e) */
        const int shift = 126 - e;
        uint32_t q = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return sign | (uint16_t)q;
    }
    /* normal */
    uint32_t m = ax + 0xc8000000u; /* rebias exponent: (e-127+15)<<23 */
    const uint32_t rem = m & 0x1fffu;
    m >>= 13;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) ++m;
    return sign | (uint16_t)m;
}

static float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    const uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

EXPORT uint16_t oracle_f32_to_f16(float f) { return f32_to_f16(f); }
EXPORT float oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
EXPORT uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }

static float act(const uint16_t* x, int64_t i, int dtype) {
    return dtype == 0 ? f16_to_f32(x[i]) : bf16_to_f32(x[i]);
}
static uint16_t cast_out(float v, int dtype) { return dtype == 0 ? f32_to_f16(v) : f32_to_bf16(v); }

/* ---- the reference's reduction trees ------------------------------------ */

/* shfl_down 16/8/4/2/1 over 32 lanes; result of lane 0. */
static float warp_tree(float v[32]) {
    for (int delta = 16; delta; delta >>= 1)
        for (int lane = 0; lane < delta; ++lane) v[lane] = v[lane] + v[lane + delta];
    return v[0];
}

/* block_sum over 256 threads (cuda_common.cuh:38-51). */
static float block_sum256(const float acc[256]) {
    float part[32];
    float second[32];
    for (int w = 0; w < 8; ++w) {
        float v[32];
        for (int l = 0; l < 32; ++l) v[l] = acc[32 * w + l];
        part[w] = warp_tree(v);
    }
    for (int l = 0; l < 32; ++l) second[l] = l < 8 ? part[l] : 0.0f;
    return warp_tree(second);
}

/* ---- Q8 A16 projection, canonical order (blocks.cu:306-321) ------------- */

EXPORT void oracle_q8_linear(const uint16_t* x, int dtype, const int8_t* codes, const uint16_t* scales,
                             uint16_t* out, int tokens, int n, int k, int padded) {
    const int groups = padded / 32;
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < n; ++row) {
            float acc[256];
            for (int j = 0; j < 256; ++j) {
                float a = 0.0f;
                for (int c = j; c < k; c += 256) {
                    const float w = (float)codes[(int64_t)row * padded + c] *
                                    f16_to_f32(scales[(int64_t)row * groups + c / 32]);
                    a = fmaf(act(x, (int64_t)t * k + c, dtype), w, a);
                }
                acc[j] = a;
            }
            out[(int64_t)t * n + row] = cast_out(block_sum256(acc), dtype);
        }
}

/* ---- A8 quantizer (q8_dp4a.cuh:15-34) ------------------------------------ */

static void quantize_group(const float in[32], int passes, int64_t count, int64_t index, int8_t* codes,
                           float* scales) {
    float r[32];
    int invalid = 0;
    for (int l = 0; l < 32; ++l) {
        r[l] = in[l];
        if (!isfinite(r[l])) invalid = 1;
    }
    for (int p = 0; p < passes; ++p) {
        float m = 0.0f;
        for (int l = 0; l < 32; ++l) m = fmaxf(m, fabsf(r[l]));
        const float scale = m / 127.0f;
        const float inverse = m > 0 ? 127.0f / m : 0.0f;
        for (int l = 0; l < 32; ++l) {
            int code = 0;
            if (!invalid) {
                const float q = rintf(r[l] * inverse);
                code = q > 127.0f ? 127 : (q < -127.0f ? -127 : (int)q);
            }
            codes[(p * count + index) * 32 + l] = (int8_t)code;
            r[l] = fmaf(-(float)code, scale, r[l]);
        }
        scales[p * count + index] = invalid ? NAN : scale;
    }
}

EXPORT void oracle_a8_quantize(const uint16_t* x, int tokens, int k, int passes, int8_t* codes, float* scales) {
    const int groups = (k + 31) / 32;
    const int64_t count = (int64_t)tokens * groups;
    for (int t = 0; t < tokens; ++t)
        for (int g = 0; g < groups; ++g) {
            float in[32];
            for (int l = 0; l < 32; ++l) {
                const int col = g * 32 + l;
                in[l] = col < k ? f16_to_f32(x[(int64_t)t * k + col]) : 0.0f;
            }
            quantize_group(in, passes, count, (int64_t)t * groups + g, codes, scales);
        }
}

/* ---- W8A8 projection, reference order (q8_dp4a.cuh:36-70) --------------- */

EXPORT void oracle_a8_linear(const int8_t* acodes, const float* ascales, const int8_t* codes,
                             const uint16_t* wscales, uint16_t* out, int tokens, int n, int k, int padded,
                             int passes) {
    const int groups = (k + 31) / 32;
    const int64_t count = (int64_t)tokens * groups;
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < n; ++row) {
            float lanes[32];
            for (int l = 0; l < 32; ++l) {
                float sum = 0.0f;
                for (int g = l; g < groups; g += 32) {
                    const float ws = f16_to_f32(wscales[(int64_t)row * (padded / 32) + g]);
                    for (int p = 0; p < passes; ++p) {
                        const int64_t gi = p * count + (int64_t)t * groups + g;
                        int32_t d = 0;
                        for (int e = 0; e < 32; ++e)
                            d += (int32_t)codes[(int64_t)row * padded + g * 32 + e] * (int32_t)acodes[gi * 32 + e];
                        sum = fmaf((float)d, ws * ascales[gi], sum);
                    }
                }
                lanes[l] = sum;
            }
            out[(int64_t)t * n + row] = f32_to_f16(warp_tree(lanes));
        }
}

/* Exact integer group dot products d[t][row][g] (pass 0) for bit checks. */
EXPORT void oracle_a8_group_dots(const int8_t* acodes, const int8_t* codes, int32_t* dots, int tokens, int n, int k,
                                 int padded) {
    const int groups = (k + 31) / 32;
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < n; ++row)
            for (int g = 0; g < groups; ++g) {
                int32_t d = 0;
                for (int e = 0; e < 32; ++e)
                    d += (int32_t)codes[(int64_t)row * padded + g * 32 + e] *
                         (int32_t)acodes[((int64_t)t * groups + g) * 32 + e];
                dots[((int64_t)t * n + row) * groups + g] = d;
            }
}

/* ---- RMSNorm (blocks.cu:31-54, with 1/sqrt in place of rsqrtf) ---------- */

static float inverse_rms(const float* v, int k, float epsilon) {
    float acc[256];
    for (int j = 0; j < 256; ++j) {
        float a = 0.0f;
        for (int c = j; c < k; c += 256) a = fmaf(v[c], v[c], a);
        acc[j] = a;
    }
    const float sum = block_sum256(acc);
    return 1.0f / sqrtf(sum / (float)k + epsilon);
}

/* dtype 0 = fp16, 1 = bf16, 2 = fp32 for x/out. */
EXPORT void oracle_rms(const void* x, int dtype, const float* w, void* out, int tokens, int k, float epsilon,
                       float* row_buffer) {
    for (int t = 0; t < tokens; ++t) {
        for (int c = 0; c < k; ++c) {
            const int64_t i = (int64_t)t * k + c;
            row_buffer[c] = dtype == 2 ? ((const float*)x)[i] : act((const uint16_t*)x, i, dtype);
        }
        const float inv = inverse_rms(row_buffer, k, epsilon);
        for (int c = 0; c < k; ++c) {
            const float y = (row_buffer[c] * inv) * w[c];
            const int64_t i = (int64_t)t * k + c;
            if (dtype == 2) ((float*)out)[i] = y;
            else ((uint16_t*)out)[i] = cast_out(y, dtype);
        }
    }
}

/* RMSNorm -> fp16 -> A8 (q8_rms_producer.cuh:8-53, any pass count). */
EXPORT void oracle_rms_a8(const uint16_t* x, const float* w, int tokens, int k, float epsilon, int passes,
                          int8_t* codes, float* scales, uint16_t* intermediate, float* row_buffer) {
    const int groups = (k + 31) / 32;
    const int64_t count = (int64_t)tokens * groups;
    for (int t = 0; t < tokens; ++t) {
        for (int c = 0; c < k; ++c) row_buffer[c] = f16_to_f32(x[(int64_t)t * k + c]);
        const float inv = inverse_rms(row_buffer, k, epsilon);
        for (int g = 0; g < groups; ++g) {
            float in[32];
            for (int l = 0; l < 32; ++l) {
                const int c = g * 32 + l;
                in[l] = 0.0f;
                if (c < k) {
                    const uint16_t y = f32_to_f16((row_buffer[c] * inv) * w[c]);
                    if (intermediate) intermediate[(int64_t)t * k + c] = y;
                    in[l] = f16_to_f32(y);
                }
            }
            quantize_group(in, passes, count, (int64_t)t * groups + g, codes, scales);
        }
    }
}

/* ---- W4A16 expert GEMV (flash_next_q4.cu:7-34) ---------------------------
 * weight = fp16(q * scale) (RNE), lane l sums columns l, l+32, ... with
 * fmaf in increasing order, then a 32-lane shfl_down tree, fp16 output. */

static float q4_weight(const uint8_t* codes, const uint16_t* scales, int row, int col, int padded) {
    const uint8_t byte = codes[(int64_t)row * (padded / 2) + col / 2];
    int q = (col & 1) ? (byte >> 4) : (byte & 15);
    q = q < 8 ? q : q - 16;
    return f16_to_f32(f32_to_f16((float)q * f16_to_f32(scales[(int64_t)row * (padded / 64) + col / 64])));
}

EXPORT void oracle_q4_linear(const uint16_t* x, const uint8_t* codes, const uint16_t* scales, uint16_t* out,
                             int tokens, int rows, int cols, int padded) {
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < rows; ++row) {
            float lanes[32];
            for (int l = 0; l < 32; ++l) {
                float sum = 0.0f;
                for (int c = l; c < cols; c += 32)
                    sum = fmaf(q4_weight(codes, scales, row, c, padded), f16_to_f32(x[(int64_t)t * cols + c]), sum);
                lanes[l] = sum;
            }
            out[(int64_t)t * rows + row] = f32_to_f16(warp_tree(lanes));
        }
}

/* fp16 decode of a Q4 matrix (flash_next_q4.cu:16-21). */
EXPORT void oracle_q4_decode(const uint8_t* codes, const uint16_t* scales, uint16_t* out, int rows, int cols,
                             int padded) {
    for (int row = 0; row < rows; ++row)
        for (int c = 0; c < cols; ++c)
            out[(int64_t)row * cols + c] = f32_to_f16(q4_weight(codes, scales, row, c, padded));
}

/* ---- Q4 plugin GEMV q4_generic (q4_linear.cu:21-56) ----------------------
 * Lane l owns byte l of each 32-byte group: columns 64g+2l (low nibble) and
 * 64g+2l+1 (high); FP32 weights w = f32(q) * f32(scale) (exact); per token
 * sum = fmaf(x0, w0, sum) then fmaf(x1, w1, sum) for columns < k, groups in
 * order; 32-lane tree; RNE cast to the activation type. */
EXPORT void oracle_q4_generic(const uint16_t* x, const uint8_t* codes, const uint16_t* scales, uint16_t* out, int n,
                              int k, int padded, int tokens, int dtype) {
    const int groups = (k + 63) / 64;
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < n; ++row) {
            float lanes[32];
            for (int l = 0; l < 32; ++l) {
                float sum = 0.0f;
                for (int g = 0; g < groups; ++g) {
                    const unsigned byte = codes[(int64_t)row * (padded / 2) + (int64_t)g * 32 + l];
                    const float scale = f16_to_f32(scales[(int64_t)row * (padded / 64) + g]);
                    const float w0 = (float)((int)((byte & 15) ^ 8) - 8) * scale;
                    const float w1 = (float)((int)((byte >> 4) ^ 8) - 8) * scale;
                    const int col = g * 64 + 2 * l;
                    if (col < k) sum = fmaf(act(x, (int64_t)t * k + col, dtype), w0, sum);
                    if (col + 1 < k) sum = fmaf(act(x, (int64_t)t * k + col + 1, dtype), w1, sum);
                }
                lanes[l] = sum;
            }
            out[(int64_t)t * n + row] = cast_out(warp_tree(lanes), dtype);
        }
}

/* ---- research fused Q4 GEMV (q4_fused.cuh:10-89) -------------------------
 * Lane l: for every padded group g, term = RNE(lo*x0 + hi*x1) (both products
 * are exact in fp32, so the fma contraction of either is the same value),
 * acc = fmaf(scale, term, acc); x past k reads 0; 32-lane tree; fp16. */
EXPORT void oracle_q4_fused(const uint16_t* x, const uint8_t* codes, const uint16_t* scales, uint16_t* out,
                            int tokens, int rows, int k, int padded) {
    const int groups = padded / 64;
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < rows; ++row) {
            float lanes[32];
            for (int l = 0; l < 32; ++l) {
                float acc = 0.0f;
                for (int g = 0; g < groups; ++g) {
                    const unsigned byte = codes[(int64_t)row * (padded / 2) + (int64_t)g * 32 + l];
                    int lo = byte & 15, hi = byte >> 4;
                    lo = lo >= 8 ? lo - 16 : lo;
                    hi = hi >= 8 ? hi - 16 : hi;
                    const int col = g * 64 + 2 * l;
                    const float x0 = col < k ? f16_to_f32(x[(int64_t)t * k + col]) : 0.0f;
                    const float x1 = col + 1 < k ? f16_to_f32(x[(int64_t)t * k + col + 1]) : 0.0f;
                    const float term = fmaf((float)hi, x1, (float)lo * x0);
                    acc = fmaf(f16_to_f32(scales[(int64_t)row * groups + g]), term, acc);
                }
                lanes[l] = acc;
            }
            out[(int64_t)t * rows + row] = f32_to_f16(warp_tree(lanes));
        }
}

/* ---- Q4/Q5/Q6 row codecs (weight_dequant.cuh:1-51, weights.py:175-190) ----
 * Column c of a row: low four bits = nibble (c & 1) of code byte c/2; the
 * hb = bits-4 upper bits are bits [c*hb, c*hb + hb) of the row's high plane
 * read as one LSB-first bit stream; q is the bits-wide two's complement;
 * w = fp16(q * scale[c / 64]), one RNE rounding. */
static float row_weight(const uint8_t* codes, const uint8_t* high, const uint16_t* scales, int64_t row, int col,
                        int padded, int bits) {
    const int hb = bits - 4;
    const uint8_t byte = codes[row * (padded / 2) + col / 2];
    int raw = (col & 1) ? (byte >> 4) : (byte & 15);
    for (int b = 0; b < hb; ++b) {
        const int64_t bit = (int64_t)col * hb + b;
        const int value = (high[row * ((int64_t)padded * hb / 8) + bit / 8] >> (bit % 8)) & 1;
        raw |= value << (4 + b);
    }
    const int q = raw >= (1 << (bits - 1)) ? raw - (1 << bits) : raw;
    return f16_to_f32(f32_to_f16((float)q * f16_to_f32(scales[row * (padded / 64) + col / 64])));
}

/* venturi_row_dequant_rows / _indexed: out[i][c] = w(ids[i], c), ld = k. */
EXPORT void oracle_row_decode(const uint8_t* codes, const uint8_t* high, const uint16_t* scales, const int64_t* ids,
                              uint16_t* out, int count, int k, int padded, int bits) {
    for (int i = 0; i < count; ++i)
        for (int c = 0; c < k; ++c)
            out[(int64_t)i * k + c] = f32_to_f16(row_weight(codes, high, scales, ids[i], c, padded, bits));
}

/* ---- W5A16 GEMV (flash_next_q5.cu:9-38) -----------------------------------
 * weight_at = fp16(q * scale); lane l sums columns l, l+32, ... with fmaf in
 * increasing order (nvcc contracts sum += w*x), 32-lane shfl_down tree,
 * fp16 output. */
EXPORT void oracle_q5_linear(const uint16_t* x, const uint8_t* codes, const uint8_t* high, const uint16_t* scales,
                             uint16_t* out, int tokens, int rows, int cols, int padded) {
    for (int t = 0; t < tokens; ++t)
        for (int row = 0; row < rows; ++row) {
            float lanes[32];
            for (int l = 0; l < 32; ++l) {
                float sum = 0.0f;
                for (int c = l; c < cols; c += 32)
                    sum = fmaf(row_weight(codes, high, scales, row, c, padded, 5), f16_to_f32(x[(int64_t)t * cols + c]),
                               sum);
                lanes[l] = sum;
            }
            out[(int64_t)t * rows + row] = f32_to_f16(warp_tree(lanes));
        }
}
