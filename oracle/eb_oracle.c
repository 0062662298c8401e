/*
 * ElasticBit CPU oracle -- TEST INFRASTRUCTURE ONLY (see eb_oracle.h).
 *
 * Built with -ffp-contract=off so every float expression rounds exactly as
 * written, matching the reference's host code compiled for x86-64 without FMA.
 * Reference paths are relative to the MLBricks repository root; "runtime.cu"
 * is mlbricks/elasticbit/csrc/elasticbit_runtime.cu.
 */
#include "eb_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16 from the IEEE-754 definition                                     */
/* ------------------------------------------------------------------------ */

uint16_t ebo_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof(x));
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t mag = x & 0x7fffffffu;
    const uint32_t exp32 = mag >> 23;
    const uint32_t man32 = mag & 0x7fffffu;

    if (exp32 == 0xffu) {                     /* inf / nan */
        if (man32 == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man32 >> 13));
    }
    if (exp32 >= 143u) return (uint16_t)(sign | 0x7c00u);  /* >= 2^16 */
    if (exp32 >= 113u) {                      /* normal binary16 range */
        uint32_t h = ((exp32 - 112u) << 10) | (man32 >> 13);
        const uint32_t rem = man32 & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;  /* carry may reach inf */
        return (uint16_t)(sign | h);
    }
    if (exp32 == 0) return sign;              /* f32 subnormal: < 2^-126 */
    /* binary16 subnormal: value = m * 2^-24, m = mant24 * 2^(exp32-126) */
    {
        const uint32_t shift = 126u - exp32;  /* >= 14 */
        const uint32_t mant24 = man32 | 0x800000u;
        if (shift > 24u) return sign;         /* < 2^-25: rounds to zero */
        uint32_t m = mant24 >> shift;
        const uint32_t rem = mant24 & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (m & 1u))) m += 1u;
        return (uint16_t)(sign | m);
    }
}

float ebo_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else {                                  /* subnormal: m * 2^-24 */
        const float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&x, &v, sizeof(x));
        x |= sign;
    }
    float out;
    memcpy(&out, &x, sizeof(out));
    return out;
}

void ebo_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ebo_f32_to_f16(in[i]);
}

void ebo_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ebo_f16_to_f32(in[i]);
}

static float round_fp16(float v) { return ebo_f16_to_f32(ebo_f32_to_f16(v)); }

/* ------------------------------------------------------------------------ */
/* canonical storage                                                         */
/* ------------------------------------------------------------------------ */

uint32_t ebo_qmax(int bits) {                 /* runtime.cu:64-67 */
    return (1u << (bits - 1)) - 1u;
}

size_t ebo_packed_bytes(size_t count, int bits) {  /* runtime.cu:69-71 */
    return (count * (size_t)bits + 7u) / 8u;
}

int32_t ebo_quantize(float value, float scale, int bits) {  /* runtime.cu:77-81 */
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    const float ratio = value / scale;
    int32_t q = (int32_t)nearbyintf(ratio);
    if (q > qmax) q = qmax;
    if (q < -qmax) q = -qmax;
    return q;
}

void ebo_row_scales(const float* w, int rows, int cols, int bits, float* scales) {
    /* runtime.cu:83-101 */
    if (bits == 16) return;
    const float qmax = (float)ebo_qmax(bits);
    for (int r = 0; r < rows; ++r) {
        float max_abs = 0.0f;
        for (int c = 0; c < cols; ++c) {
            const float a = fabsf(w[(size_t)r * cols + c]);
            if (a > max_abs) max_abs = a;
        }
        scales[r] = max_abs > 0.0f ? max_abs / qmax : 1.0f;
    }
}

static void or_code(uint8_t* payload, size_t payload_bytes, size_t index, int bits, uint32_t code) {
    /* runtime.cu:171-184: OR three bytes of (code << shift) at byte offset */
    const size_t bit = index * (size_t)bits;
    const size_t byte = bit >> 3;
    const uint64_t shifted = (uint64_t)code << (bit & 7u);
    for (int k = 0; k < 3; ++k) {
        if (byte + (size_t)k < payload_bytes) {
            payload[byte + (size_t)k] |= (uint8_t)((shifted >> (8 * k)) & 0xffu);
        }
    }
}

int ebo_pack_codes(const int16_t* codes, size_t count, int bits, uint8_t* payload) {
    /* runtime.cu:150-186 */
    const size_t nbytes = ebo_packed_bytes(count, bits);
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    memset(payload, 0, nbytes);
    for (size_t i = 0; i < count; ++i) {
        const int32_t q = codes[i];
        if (q < -qmax || q > qmax) return -1;
        or_code(payload, nbytes, i, bits, (uint32_t)(q + qmax));
    }
    return 0;
}

void ebo_pack_weights(const float* w, int rows, int cols, int bits,
                      const float* scales, uint8_t* payload) {
    /* runtime.cu:103-148 */
    const size_t count = (size_t)rows * cols;
    if (bits == 16) {
        for (size_t i = 0; i < count; ++i) {
            const uint16_t h = ebo_f32_to_f16(w[i]);
            payload[2 * i] = (uint8_t)(h & 0xffu);
            payload[2 * i + 1] = (uint8_t)(h >> 8);
        }
        return;
    }
    const size_t nbytes = ebo_packed_bytes(count, bits);
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    memset(payload, 0, nbytes);
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) {
            const size_t i = (size_t)r * cols + c;
            const int32_t q = ebo_quantize(w[i], scales[r], bits);
            or_code(payload, nbytes, i, bits, (uint32_t)(q + qmax));
        }
    }
}

uint32_t ebo_extract(const uint8_t* payload, size_t payload_bytes, size_t index, int bits) {
    /* runtime.cu:188-206 */
    const size_t bit = index * (size_t)bits;
    const size_t byte = bit >> 3;
    uint32_t word = 0;
    for (int k = 0; k < 3; ++k) {
        if (byte + (size_t)k < payload_bytes) word |= (uint32_t)payload[byte + (size_t)k] << (8 * k);
    }
    return (word >> (bit & 7u)) & ((1u << bits) - 1u);
}

void ebo_unpack_codes(const uint8_t* payload, size_t payload_bytes, size_t count,
                      int bits, int16_t* codes) {
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    for (size_t i = 0; i < count; ++i) {
        codes[i] = (int16_t)((int32_t)ebo_extract(payload, payload_bytes, i, bits) - qmax);
    }
}

static uint16_t stored_f16(const uint8_t* payload, size_t i) {
    return (uint16_t)(payload[2 * i] | ((uint16_t)payload[2 * i + 1] << 8));
}

void ebo_dequantize(const uint8_t* payload, size_t payload_bytes, const float* scales,
                    int rows, int cols, int bits, float* out, uint16_t* out16) {
    /* runtime.cu:208-238 */
    const size_t count = (size_t)rows * cols;
    if (bits == 16) {
        for (size_t i = 0; i < count; ++i) {
            const uint16_t h = stored_f16(payload, i);
            if (out) out[i] = ebo_f16_to_f32(h);
            if (out16) out16[i] = h;
        }
        return;
    }
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    for (int r = 0; r < rows; ++r) {
        const float s = scales[r];
        for (int c = 0; c < cols; ++c) {
            const size_t i = (size_t)r * cols + c;
            const int32_t q = (int32_t)ebo_extract(payload, payload_bytes, i, bits) - qmax;
            const float prod = (float)q * s;
            const uint16_t h = ebo_f32_to_f16(prod);
            if (out) out[i] = ebo_f16_to_f32(h);
            if (out16) out16[i] = h;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* output semantics                                                          */
/* ------------------------------------------------------------------------ */

void ebo_linear_intdot(const uint8_t* payload, size_t payload_bytes, const float* scales,
                       int rows, int cols, int bits, const uint16_t* x16, int M, double* y) {
    if (bits == 16) {
        ebo_linear_w16(payload, payload_bytes, scales, rows, cols, bits, x16, M, y);
        return;
    }
    const int32_t qmax = (int32_t)ebo_qmax(bits);
    for (int m = 0; m < M; ++m) {
        for (int r = 0; r < rows; ++r) {
            double acc = 0.0;
            for (int c = 0; c < cols; ++c) {
                const size_t i = (size_t)r * cols + c;
                const int32_t q = (int32_t)ebo_extract(payload, payload_bytes, i, bits) - qmax;
                acc += (double)q * (double)ebo_f16_to_f32(x16[(size_t)m * cols + c]);
            }
            y[(size_t)m * rows + r] = acc * (double)scales[r];
        }
    }
}

void ebo_linear_w16(const uint8_t* payload, size_t payload_bytes, const float* scales,
                    int rows, int cols, int bits, const uint16_t* x16, int M, double* y) {
    const int32_t qmax = bits == 16 ? 0 : (int32_t)ebo_qmax(bits);
    for (int m = 0; m < M; ++m) {
        for (int r = 0; r < rows; ++r) {
            double acc = 0.0;
            for (int c = 0; c < cols; ++c) {
                const size_t i = (size_t)r * cols + c;
                float w;
                if (bits == 16) {
                    w = ebo_f16_to_f32(stored_f16(payload, i));
                } else {
                    const int32_t q = (int32_t)ebo_extract(payload, payload_bytes, i, bits) - qmax;
                    w = round_fp16((float)q * scales[r]);
                }
                acc += (double)w * (double)ebo_f16_to_f32(x16[(size_t)m * cols + c]);
            }
            y[(size_t)m * rows + r] = acc;
        }
    }
}

int ebo_gemv_f32_baseline(const uint8_t* payload, size_t payload_bytes, const float* scales,
                          int rows, int cols, int bits, const uint16_t* x16,
                          int row_begin, int row_end, uint16_t* y16, int threads) {
    if (row_begin < 0 || row_end > rows || row_begin > row_end) return -1;
    float* xf = (float*)malloc(sizeof(float) * (size_t)cols);
    if (!xf) return -1;
    for (int c = 0; c < cols; ++c) xf[c] = ebo_f16_to_f32(x16[c]);
    const int32_t qmax = bits == 16 ? 0 : (int32_t)ebo_qmax(bits);
    int used = 1;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
    used = threads;
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
    for (int r = row_begin; r < row_end; ++r) {
        float acc = 0.0f;
        if (bits == 16) {
            for (int c = 0; c < cols; ++c) {
                acc += ebo_f16_to_f32(stored_f16(payload, (size_t)r * cols + c)) * xf[c];
            }
            y16[r - row_begin] = ebo_f32_to_f16(acc);
        } else if (bits <= 8) {               /* runtime.cu:538-558 */
            for (int c = 0; c < cols; ++c) {
                const int32_t q = (int32_t)ebo_extract(payload, payload_bytes, (size_t)r * cols + c, bits) - qmax;
                acc += (float)q * xf[c];
            }
            y16[r - row_begin] = ebo_f32_to_f16(acc * scales[r]);
        } else {                              /* runtime.cu:635-647 */
            const float s = scales[r];
            for (int c = 0; c < cols; ++c) {
                const int32_t q = (int32_t)ebo_extract(payload, payload_bytes, (size_t)r * cols + c, bits) - qmax;
                acc += round_fp16((float)q * s) * xf[c];
            }
            y16[r - row_begin] = ebo_f32_to_f16(acc);
        }
    }
    free(xf);
    return used;
}

/* ------------------------------------------------------------------------ */
/* host analyzer, runtime.cu:280-436                                         */
/* ------------------------------------------------------------------------ */

static void analyze_one(const float* w, int rows, int cols, const float* calib, int samples,
                        const float* refs, const float* xh, int bits, ebo_analysis* out) {
    /* runtime.cu:312-392 */
    float* scales = NULL;
    if (bits != 16) {
        scales = (float*)malloc(sizeof(float) * (size_t)rows);
        ebo_row_scales(w, rows, cols, bits, scales);
    }
    long double hw_num = 0.0L, full_num = 0.0L, denom = 0.0L;
    for (int s = 0; s < samples; ++s) {
        const float* in = xh + (size_t)s * cols;
        for (int r = 0; r < rows; ++r) {
            const float* row = w + (size_t)r * cols;
            float hw = 0.0f, full = 0.0f;
            if (bits == 16) {
                for (int c = 0; c < cols; ++c) {
                    const float wh = round_fp16(row[c]);
                    const float p = wh * in[c];
                    hw = hw + p;
                }
                full = hw;
            } else if (bits <= 8) {
                const float scale = scales[r];
                float idot = 0.0f;
                for (int c = 0; c < cols; ++c) {
                    const int32_t q = ebo_quantize(row[c], scale, bits);
                    const float p = (float)q * in[c];
                    idot = idot + p;
                    const float deq = round_fp16((float)q * scale);
                    const float p2 = deq * in[c];
                    full = full + p2;
                }
                hw = idot * scale;
            } else {
                const float scale = scales[r];
                for (int c = 0; c < cols; ++c) {
                    const int32_t q = ebo_quantize(row[c], scale, bits);
                    const float deq = round_fp16((float)q * scale);
                    const float p = deq * in[c];
                    hw = hw + p;
                }
                full = hw;
            }
            const double ref = (double)refs[(size_t)s * rows + r];
            const double hd = (double)hw - ref;
            const double fd = (double)full - ref;
            hw_num += (long double)hd * hd;
            full_num += (long double)fd * fd;
            denom += (long double)ref * ref;
        }
    }
    (void)calib;
    const long double safe = denom > 1.0e-30L ? denom : 1.0e-30L;
    out->bits = bits;
    out->hardware_native_error = sqrt((double)(hw_num / safe));
    out->full_precision_error = sqrt((double)(full_num / safe));
    out->error = out->hardware_native_error > out->full_precision_error
        ? out->hardware_native_error : out->full_precision_error;
    const size_t count = (size_t)rows * cols;
    out->storage_bytes = bits == 16 ? (uint64_t)(count * 2u)
        : (uint64_t)(ebo_packed_bytes(count, bits) + (size_t)rows * 4u);
    free(scales);
}

int ebo_analyze(const float* w, int rows, int cols, const float* calib, int samples,
                ebo_analysis* out14) {
    if (rows <= 0 || cols <= 0 || samples <= 0) return -1;
    /* runtime.cu:280-310 fp16_reference_outputs */
    float* xh = (float*)malloc(sizeof(float) * (size_t)samples * cols);
    float* wh = (float*)malloc(sizeof(float) * (size_t)rows * cols);
    float* refs = (float*)malloc(sizeof(float) * (size_t)samples * rows);
    for (size_t i = 0; i < (size_t)samples * cols; ++i) xh[i] = round_fp16(calib[i]);
    for (size_t i = 0; i < (size_t)rows * cols; ++i) wh[i] = round_fp16(w[i]);
    for (int s = 0; s < samples; ++s) {
        for (int r = 0; r < rows; ++r) {
            float sum = 0.0f;
            for (int c = 0; c < cols; ++c) {
                const float p = wh[(size_t)r * cols + c] * xh[(size_t)s * cols + c];
                sum = sum + p;
            }
            refs[(size_t)s * rows + r] = sum;
        }
    }
    for (int b = 3; b <= 16; ++b) {
        analyze_one(w, rows, cols, calib, samples, refs, xh, b, &out14[b - 3]);
    }
    free(xh);
    free(wh);
    free(refs);
    return 0;
}

int ebo_select(const ebo_analysis* a, int n, double threshold) {
    /* runtime.cu:408-427 */
    if (!isfinite(threshold) || threshold < 0.0) return -1;
    for (int i = 0; i < n; ++i) {
        if (a[i].bits <= 15 && a[i].error <= threshold) return i;
    }
    return n - 1;
}

/* ------------------------------------------------------------------------ */
/* FNV-1a and MLB4                                                           */
/* ------------------------------------------------------------------------ */

uint64_t ebo_fnv1a64(const void* data, size_t size) {
    /* published FNV-1a 64-bit: offset basis 0xcbf29ce484222325, prime 0x100000001b3 */
    const uint8_t* p = (const uint8_t*)data;
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < size; ++i) {
        h ^= (uint64_t)p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

static void put_le(uint8_t* dst, uint64_t v, int n) {
    for (int i = 0; i < n; ++i) dst[i] = (uint8_t)(v >> (8 * i));
}

size_t ebo_mlb4_write(uint8_t* buf, int rows, int cols, int bits,
                      const float* scales, const uint8_t* payload, size_t payload_bytes,
                      double threshold, double selected_error) {
    /* header layout runtime.cu:692-712; writer :1024-1049 */
    const uint32_t scale_count = bits == 16 ? 0u : (uint32_t)rows;
    const uint64_t scale_bytes = (uint64_t)scale_count * 4u;
    memset(buf, 0, 80);
    memcpy(buf, "MLB4", 4);
    put_le(buf + 4, 4, 2);
    put_le(buf + 6, 80, 2);
    put_le(buf + 8, (uint32_t)rows, 4);
    put_le(buf + 12, (uint32_t)cols, 4);
    buf[16] = (uint8_t)bits;
    put_le(buf + 20, scale_count, 4);
    put_le(buf + 24, scale_bytes, 8);
    put_le(buf + 32, payload_bytes, 8);
    put_le(buf + 40, (uint64_t)rows * (uint64_t)cols * 2u, 8);
    put_le(buf + 48, ebo_fnv1a64(scales, scale_count ? scale_bytes : 0), 8);
    put_le(buf + 56, ebo_fnv1a64(payload, payload_bytes), 8);
    memcpy(buf + 64, &threshold, 8);
    memcpy(buf + 72, &selected_error, 8);
    if (scale_count) memcpy(buf + 80, scales, scale_bytes);
    memcpy(buf + 80 + scale_bytes, payload, payload_bytes);
    return 80u + (size_t)scale_bytes + payload_bytes;
}

/* ------------------------------------------------------------------------ */
/* legacy group-scale op, bolt/ops_cuda.cu:2708-2750                          */
/* ------------------------------------------------------------------------ */

void ebo_packed_linear(const double* x, int M, const uint8_t* packed, const double* scales,
                       const double* bias, int bits, int group_size, int out_features,
                       int in_features, double* y) {
    const int qmin = -(1 << (bits - 1));
    const uint32_t mask = (1u << bits) - 1u;
    for (int m = 0; m < M; ++m) {
        for (int o = 0; o < out_features; ++o) {
            double acc = 0.0;
            for (int k = 0; k < in_features; ++k) {
                const size_t wi = (size_t)o * in_features + k;
                const size_t bit = wi * (size_t)bits;
                uint32_t word = packed[bit >> 3];
                if ((int)(bit & 7u) + bits > 8) word |= (uint32_t)packed[(bit >> 3) + 1] << 8;
                const int q = (int)((word >> (bit & 7u)) & mask) + qmin;
                acc += x[(size_t)m * in_features + k] * ((double)q * scales[wi / (size_t)group_size]);
            }
            if (bias) acc += bias[o];
            y[(size_t)m * out_features + o] = acc;
        }
    }
}
