/*
 * ElasticBit CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the MLBricks ElasticBit host algorithm, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker.  Nothing in mlbricks_amd/ links, loads or calls this code; the
 * product path is the HIP library under mlbricks_amd/csrc.
 *
 * Every function names the reference file:line it restates
 * (paths relative to the MLBricks repository root).
 */
#ifndef EB_ORACLE_H
#define EB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary16 conversions written from the format definition:
 * round-to-nearest-even, subnormals preserved, overflow to infinity. */
uint16_t ebo_f32_to_f16(float value);
float ebo_f16_to_f32(uint16_t bits);
void ebo_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void ebo_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* elasticbit_runtime.cu:64-67 / :69-71 */
uint32_t ebo_qmax(int bits);
size_t ebo_packed_bytes(size_t count, int bits);

/* elasticbit_runtime.cu:77-81 (quantize_scalar) */
int32_t ebo_quantize(float value, float scale, int bits);

/* elasticbit_runtime.cu:83-101 (make_row_scales); b=16 writes nothing */
void ebo_row_scales(const float* w, int rows, int cols, int bits, float* scales);

/* elasticbit_runtime.cu:150-186 (pack_exact_codes).  Returns 0, or -1 when a
 * code lies outside [-qmax, qmax]. payload must hold ebo_packed_bytes(). */
int ebo_pack_codes(const int16_t* codes, size_t count, int bits, uint8_t* payload);

/* elasticbit_runtime.cu:103-148 (pack_exact_weights).  b=16 stores fp16(w). */
void ebo_pack_weights(const float* w, int rows, int cols, int bits,
                      const float* scales, uint8_t* payload);

/* elasticbit_runtime.cu:188-206 (extract_code_host) */
uint32_t ebo_extract(const uint8_t* payload, size_t payload_bytes, size_t index, int bits);

/* Signed codes q = u - qmax for every element (inverse of ebo_pack_codes). */
void ebo_unpack_codes(const uint8_t* payload, size_t payload_bytes, size_t count,
                      int bits, int16_t* codes);

/* elasticbit_runtime.cu:208-238 (dequantize_payload_host): fp16_rn(q*s) as
 * float; b=16 widens the stored fp16.  out16 (optional) receives the bits. */
void ebo_dequantize(const uint8_t* payload, size_t payload_bytes, const float* scales,
                    int rows, int cols, int bits, float* out, uint16_t* out16);

/* Output semantics, fp64 accumulation (no output rounding):
 *   intdot (hardwareNative, elasticbit_runtime.cu:538-558,594-608):
 *       y[m][r] = s_r * sum_c q_rc * x_mc
 *   w16 (W16A16 / fullPrecision / prefill, :635-647, core.py:465-471):
 *       y[m][r] = sum_c fp16_rn(q_rc * s_r) * x_mc
 * x is fp16 bits [M][cols]; y is [M][rows].  b=16 uses the stored fp16. */
void ebo_linear_intdot(const uint8_t* payload, size_t payload_bytes, const float* scales,
                       int rows, int cols, int bits, const uint16_t* x16, int M, double* y);
void ebo_linear_w16(const uint8_t* payload, size_t payload_bytes, const float* scales,
                    int rows, int cols, int bits, const uint16_t* x16, int M, double* y);

/* CPU baseline GEMV (the reference has no CPU forward): decode the canonical
 * stream as dequantize_payload_host does, accumulate in fp32 per row in column
 * order, round to fp16.  OpenMP over rows; returns the thread count used. */
int ebo_gemv_f32_baseline(const uint8_t* payload, size_t payload_bytes, const float* scales,
                          int rows, int cols, int bits, const uint16_t* x16,
                          int row_begin, int row_end, uint16_t* y16, int threads);

/* Host analyzer, elasticbit_runtime.cu:280-436: 14 candidates b=3..16. */
typedef struct {
    int bits;
    double hardware_native_error;
    double full_precision_error;
    double error;
    uint64_t storage_bytes;
} ebo_analysis;

int ebo_analyze(const float* w, int rows, int cols, const float* calib, int samples,
                ebo_analysis* out14);
/* elasticbit_runtime.cu:408-427 (select_analysis): index into out14 */
int ebo_select(const ebo_analysis* a, int n, double threshold);

/* FNV-1a 64 (elasticbit_runtime.cu:682-690) */
uint64_t ebo_fnv1a64(const void* data, size_t size);

/* MLB4 (elasticbit_runtime.cu:692-712, 1024-1049): serialise into buf (needs
 * 80 + 4*scale_count + payload_bytes bytes).  Returns the byte count. */
size_t ebo_mlb4_write(uint8_t* buf, int rows, int cols, int bits,
                      const float* scales, const uint8_t* payload, size_t payload_bytes,
                      double threshold, double selected_error);

/* Legacy op bolt/ops_cuda.cu:2708-2750: y[m][o] = sum_k x[m][k] *
 * ((u - 2^(b-1)) * scale[(o*K+k)/group]) + bias[o], fp64 accumulation. */
void ebo_packed_linear(const double* x, int M, const uint8_t* packed, const double* scales,
                       const double* bias, int bits, int group_size, int out_features,
                       int in_features, double* y);

#ifdef __cplusplus
}
#endif

#endif
