/*
 * ElasticBit for MI355X (gfx950) -- C ABI of libelasticbit_hip.so.
 *
 * This ABI replaces the pybind11 module mlbricks.elasticbit._C and the torch
 * op mlbricks_native::elastic_linear_packed of MLBricks.  Each declaration
 * cites the reference interface it stands in for (paths relative to the
 * MLBricks repository root; "runtime.cu" is
 * mlbricks/elasticbit/csrc/elasticbit_runtime.cu).
 *
 * Conventions
 *  - Every int-returning call returns EB_OK (0) or an error status; the
 *    message is available from eb_last_error() on the calling thread.
 *    EB_INVALID_ARGUMENT maps to the reference's std::invalid_argument
 *    (Python ValueError); the others map to std::runtime_error (RuntimeError).
 *  - Device pointers are plain HIP device addresses; streams are hipStream_t
 *    passed as void* (NULL = the legacy default stream).  No call synchronises
 *    the stream it is given, and no call allocates on the forward path.
 *  - fp16 data is IEEE binary16 bit patterns (uint16_t / void*).
 *  - An eb_matrix owns its host canonical storage and its device execution
 *    buffers; callers own x / y / out buffers.
 */
#ifndef MLBRICKS_AMD_ELASTICBIT_H
#define MLBRICKS_AMD_ELASTICBIT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EB_ABI_VERSION 1

enum {
    EB_OK = 0,
    EB_INVALID_ARGUMENT = 1, /* std::invalid_argument in the reference */
    EB_RUNTIME_ERROR = 2,    /* std::runtime_error (file I/O, checksums, no device) */
    EB_DEVICE_ERROR = 3      /* a HIP call failed (CUDA_CHECK, runtime.cu:26-35) */
};

enum {
    EB_POLICY_HARDWARE_NATIVE = 1, /* runtime.cu:253-256 DecodePolicy::HardwareNative */
    EB_POLICY_FULL_PRECISION = 2   /* DecodePolicy::FullPrecision */
};

enum { EB_DTYPE_F32 = 0, EB_DTYPE_F16 = 1, EB_DTYPE_BF16 = 2 };

typedef struct eb_matrix eb_matrix;

/* Read-only properties, runtime.cu:1051-1066 (rows, cols, storageBits, ...). */
typedef struct {
    int rows;
    int cols;
    int storage_bits;
    int execution_width;
    int decode_policy;          /* EB_POLICY_* */
    int device_index;           /* -1 when the matrix has no device copy */
    uint64_t storage_bytes;     /* canonical payload + fp32 scales */
    uint64_t execution_bytes;   /* device execution buffers */
    uint64_t original_bytes;    /* 2 * rows * cols */
    double threshold;
    double selected_error;
    double memory_reduction;
    char execution_planner[32];
} eb_props;

/* One analyzer candidate, runtime.cu:272-278 (BitAnalysis) / :438-483. */
typedef struct {
    int bits;
    double hardware_native_error;
    double full_precision_error;
    double error;
    uint64_t storage_bytes;
    double memory_reduction;
    int passes;
} eb_bit_analysis;

/* Backend metadata, runtime.cu:1386-1409 (backend_info_py). */
typedef struct {
    int available;              /* a HIP device is present */
    int device_index;
    int compute_units;
    int weight_widths[16];
    int n_weight_widths;
    int validated;
    char device[128];
    char architecture[64];
    char activate_dtype[16];
    char prefill[16];
    char decode_planner[32];
    char decode_engine[32];
    char decode_status[32];
    char decode_validation[64];
} eb_backend;

/* Thread-local message of the last failing call on this thread. */
const char* eb_last_error(void);
int eb_abi_version(void);

/* ---- analyzer and backend ------------------------------------------------ */

/* _C.analyze, runtime.cu:438-483 (analyze_py; algorithm :280-436).
 * out14 receives b = 3..16; *selected_index the chosen entry. */
int eb_analyze(const float* weights, int rows, int cols, const float* calibration,
               int samples, double threshold, eb_bit_analysis* out14, int* selected_index);

/* _C.backendInfo, runtime.cu:1386-1409. */
int eb_backend_info(eb_backend* out);

/* ---- factories (RuntimeMatrix static methods, runtime.cu:720-871) --------- */

/* RuntimeMatrix.compress, runtime.cu:720-746: analyze, then pack. */
int eb_compress(const float* weights, int rows, int cols, const float* calibration,
                int samples, double threshold, int policy, eb_matrix** out);

/* RuntimeMatrix._compressSelected, runtime.cu:748-776. */
int eb_compress_selected(const float* weights, int rows, int cols, int selected_bits,
                         double threshold, double selected_error, int policy, eb_matrix** out);

/* RuntimeMatrix._compressSelectedCodes, runtime.cu:778-808. */
int eb_compress_selected_codes(const int16_t* codes, const float* scales, int rows, int cols,
                               int selected_bits, double threshold, double selected_error,
                               int policy, eb_matrix** out);

/* eb_compress_selected_codes with the codes in device memory (int16
 * [rows][cols] on the current HIP device; scales on the host), as the GPU
 * width search leaves them.  The canonical bitstream (pack_exact_codes,
 * runtime.cu:150-186) is packed on the device and repacked there; only the
 * packed stream, b bits per weight, is copied back for the matrix's host
 * copy.  Same validation and errors as the host version.  Synchronous. */
int eb_compress_selected_codes_device(const int16_t* codes_dev, const float* scales, int rows, int cols,
                                      int selected_bits, double threshold, double selected_error,
                                      int policy, eb_matrix** out);

/* RuntimeMatrix.load, runtime.cu:810-871 (MLB4 reader). */
int eb_load(const char* path, int policy, eb_matrix** out);

/* RuntimeMatrix.save, runtime.cu:1024-1049 (MLB4 writer). */
int eb_save(const eb_matrix* m, const char* path);

/* ~RuntimeMatrix, runtime.cu:716,1370-1383.  NULL is ignored. */
void eb_destroy(eb_matrix* m);

/* ---- properties and policy ------------------------------------------------ */

/* RuntimeMatrix read-only properties, runtime.cu:1051-1066. */
int eb_get_props(const eb_matrix* m, eb_props* out);

/* RuntimeMatrix.setDecodePolicy, runtime.cu:975-980. */
int eb_set_decode_policy(eb_matrix* m, int policy);

/* Canonical storage (the MLB4 body): scales (rows floats, none for b=16) and
 * payload (storage_bytes - 4*rows bytes).  Either pointer may be NULL. */
int eb_get_canonical(const eb_matrix* m, float* scales_out, uint8_t* payload_out);

/* ---- host-side compute ----------------------------------------------------- */

/* RuntimeMatrix.dequantize, runtime.cu:967-973: fp16_rn(q*s) as float [rows*cols]. */
int eb_dequantize_host(const eb_matrix* m, float* out);

/* RuntimeMatrix.forward (numpy), runtime.cu:873-900: one fp32 row [cols] ->
 * fp32 [rows], synchronous, on the legacy default stream. */
int eb_forward_host(eb_matrix* m, const float* x, float* y);

/* RuntimeMatrix.benchmark, runtime.cu:933-965: ms per launch (M = 1). */
int eb_benchmark(eb_matrix* m, const float* x, int iterations, double* ms_per_iteration);

/* ---- device compute (stream-ordered, no allocation) ------------------------ */

/* RuntimeMatrix.forwardTorch, runtime.cu:902-931 (decode, M = 1) and the
 * prefill route materialize + F.linear, core.py:462-471 (M > 1):
 *   y[M][rows] = x[M][cols] . W^T (+ bias), fp16 in, fp16 out, fp32 accumulate.
 * hardwareNative: b <= 12 computes fp16_rn(s_r * sum q*x); b >= 13 and
 * fullPrecision compute fp16_rn(sum fp16_rn(q*s_r) * x).  bias (may be NULL)
 * is added as torch does, y = fp16_rn(y + bias).  Any M >= 1. */
int eb_forward(const eb_matrix* m, const void* x_f16, int64_t M, void* y_f16,
               const void* bias_f16, void* stream);

/* Several matrices that read the same activations (no single-call
 * counterpart in the reference: Stage-2F concatenates the materialized fp16
 * weights of Q/K/V and Gate/Up and runs one F.linear, stage2f.py:382-420):
 *   ys[j][M][rows_j] = x[M][cols] . W_j^T (+ biases[j]),  j < count,
 * each as eb_forward computes it.  Every matrix has the same cols and lives
 * on one device; biases may be NULL, as may any biases[j].  Consecutive
 * matrices of one width and policy (up to four) share one launch for
 * M <= 16, and up to M = 64 where the decode kernel is the faster route for
 * each of them, so the decode of a QKV or Gate/Up group pays one launch. */
int eb_forward_multi(const eb_matrix* const* ms, int count, const void* x_f16, int64_t M,
                     void* const* ys_f16, const void* const* biases_f16, void* stream);

/* The GPU width search of ElasticBit.compress (_selectBitsTorch,
 * core.py:112-195) fused into one pass over the weights.  For fp16 weights
 * w [rows][cols] and up to EB_ANALYZE_MAX_SAMPLES fp16 calibration rows
 * x [samples][cols] (device pointers), with max_abs[r] = max_c |w[r][c]|
 * (fp32, device), it writes partials [ceil(rows / EB_ANALYZE_TILE_ROWS)]
 * [EB_ANALYZE_SUMS] (fp32, device): per tile of weight rows, sum |ref|^2,
 * then sum |full_b - ref|^2 for b = 3..15, then sum |hw_b - ref|^2 for
 * b = 3..12, where ref = fp16(x . w^T), full_b = fp16(x . fp16(q_b s_b)^T) and
 * hw_b = fp16((x . q_b^T) s_b).  The tiles' sums give the reference's relL2
 * errors (core.py:103-108); more calibration rows are more calls.  The
 * reference measures hw_b only for b <= 8 because it runs W16A16 above; this
 * runtime's hardwareNative runs the integer-code product up to b = 12, so
 * its error is measured there too.  Stream-ordered, allocates nothing. */
enum { EB_ANALYZE_TILE_ROWS = 16, EB_ANALYZE_MAX_SAMPLES = 32, EB_ANALYZE_SUMS = 24 };
int eb_analyze_widths_device(const void* w_f16, int64_t rows, int64_t cols, const void* x_f16, int64_t samples,
                             const float* max_abs, float* partials, void* stream);

/* No counterpart in the reference.  eb_analyze_widths_device for callers
 * that cannot allocate (code under HIP graph capture, allocation-free
 * compression or serving loops): the per-tile partial sums stay in a static
 * device array of the library (1.5 MiB per device, held until the process
 * ends), and totals [EB_ANALYZE_SUMS] (double, device, caller-owned) receives
 * their sums over the tiles, added on the device in a fixed order.  At most
 * EB_ANALYZE_STATIC_MAX_ROWS rows (EB_INVALID_ARGUMENT beyond).  Calls no
 * allocator.  Every call on a device shares that device's array: calls that
 * overlap on one device (concurrent streams) race.  Stream-ordered. */
enum { EB_ANALYZE_STATIC_MAX_ROWS = 262144 };
int eb_analyze_widths_device_totals(const void* w_f16, int64_t rows, int64_t cols, const void* x_f16,
                                    int64_t samples, const float* max_abs, double* totals, void* stream);

/* RuntimeMatrix._materializeTorch, runtime.cu:982-1022: out [rows][cols] fp16
 * = fp16_rn(q*s) (b = 16: the stored fp16). */
int eb_materialize_fp16(const eb_matrix* m, void* out_f16, void* stream);

/* Parity probe (no reference counterpart as a call; the reference unpacks
 * with extract_code_host, runtime.cu:188-206): out [rows][cols] int16 codes
 * q = u - qmax.  Fails for b = 16. */
int eb_unpack_codes(const eb_matrix* m, int16_t* out, void* stream);

/* mlbricks_native::elastic_linear_packed, bolt/ops.cpp:1012-1043 and
 * bolt/ops_cuda.cu:2708-2795: y[M][N] = x . W^T + bias with
 * W[o][k] = (u - 2^(b-1)) * scales[(o*K + k) / group_size], 2 <= b <= 8.
 * x / bias / y share x_dtype; scales have scale_dtype (EB_DTYPE_*). */
int eb_packed_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed,
                     const void* scales, int scale_dtype, const void* bias, int bits,
                     int64_t group_size, int64_t out_features, int64_t in_features,
                     void* y, void* stream);

/* Tuning control (no counterpart in the reference, which hands M > 1 to the
 * vendor GEMM): the output tile shape of the prefill route (M > 16, b <= 15,
 * hardwareNative or fullPrecision).  EB_PREFILL_TILES_AUTO (the default)
 * picks the shape with the fewer estimated rounds over the GPU's compute
 * units; NARROW forces 128 x 256 tiles; WIDE forces 256 x 256 tiles with
 * four waves where M and rows are both at least 256, WIDE8 the same tiles
 * with eight waves (for both, when the tiles end in a partial round of the
 * compute units, part of the output runs as 192 x 256 tiles in a second
 * launch where that is estimated faster); WIDE_PLAIN and WIDE8_PLAIN run
 * 256 x 256 tiles only, WIDE_SHORT and WIDE8_SHORT 192 x 256 tiles only.
 * Results agree within the output tolerance between shapes and are
 * bit-identical among the modes of one wave count; the sum order differs
 * otherwise.  Process-wide, read at each launch. */
enum { EB_PREFILL_TILES_AUTO = 0, EB_PREFILL_TILES_NARROW = 1, EB_PREFILL_TILES_WIDE = 2,
       EB_PREFILL_TILES_WIDE8 = 3, EB_PREFILL_TILES_WIDE8_PLAIN = 4, EB_PREFILL_TILES_WIDE8_SHORT = 5,
       EB_PREFILL_TILES_WIDE_PLAIN = 6, EB_PREFILL_TILES_WIDE_SHORT = 7 };
int eb_set_prefill_tiles(int mode);

/* Inspection (no counterpart in the reference): the launches of the
 * 256 x 256 prefill kernels (four or eight waves) for an M x rows output on a
 * device with `cus` compute units, under the current tile mode
 * (EB_PREFILL_TILES_AUTO, WIDE and WIDE8 plan alike).  rects receives three rectangles of five int32 each:
 * first activation row, activation blocks, block height (256 or 192),
 * first 256-row weight block, weight blocks.  The first two rectangles are
 * the 256 x 256 launch, the third the 192 x 256 launch; unused ones are
 * zero.  *cost (may be NULL) receives the plan's estimated time in full
 * rounds of 256 x 256 tiles. */
int eb_prefill_plan(int64_t M, int rows, int cus, int32_t* rects, double* cost);

/* ---- host codec (the packer inside the RuntimeMatrix constructors) --------- */

/* pack_exact_codes, runtime.cu:150-186.  payload_bytes must equal
 * ceil(count*bits/8). */
int eb_host_pack_codes(const int16_t* codes, uint64_t count, int bits, uint8_t* payload,
                       uint64_t payload_bytes);

/* extract_code_host over every element, runtime.cu:188-206: codes = u - qmax. */
int eb_host_unpack_codes(const uint8_t* payload, uint64_t payload_bytes, uint64_t count,
                         int bits, int16_t* codes);

#ifdef __cplusplus
}
#endif

#endif
