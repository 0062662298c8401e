// ElasticBit host runtime for MI355X: canonical codec, host analyzer, MLB4
// files, the matrix handle with its device execution buffers, and the C ABI
// declared in include/elasticbit.h.
//
// Compiled with -ffp-contract=off: the analyzer's float sums must round exactly
// as written (elasticbit_runtime.cu:280-392 is plain sequential fp32).
// Reference citations are to mlbricks/elasticbit/csrc/elasticbit_runtime.cu
// ("runtime.cu") unless another file is named.
#include "elasticbit.h"
#include "eb_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------

thread_local std::string g_last_error;

struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define EB_HIP(call)                                                                          \
    do {                                                                                      \
        hipError_t eb_err__ = (call);                                                         \
        if (eb_err__ != hipSuccess) {                                                         \
            throw DeviceError(std::string("HIP error: ") + hipGetErrorString(eb_err__) +      \
                              " at " + __FILE__ + ":" + std::to_string(__LINE__));            \
        }                                                                                     \
    } while (0)

int set_error(int code, const char* what) {
    g_last_error = what;
    return code;
}

template <typename F>
int guarded(F&& body) {
    try {
        body();
        return EB_OK;
    } catch (const std::invalid_argument& e) {
        return set_error(EB_INVALID_ARGUMENT, e.what());
    } catch (const DeviceError& e) {
        return set_error(EB_DEVICE_ERROR, e.what());
    } catch (const std::bad_alloc&) {
        return set_error(EB_RUNTIME_ERROR, "ElasticBit: out of host memory");
    } catch (const std::exception& e) {
        return set_error(EB_RUNTIME_ERROR, e.what());
    } catch (...) {
        return set_error(EB_RUNTIME_ERROR, "ElasticBit: unknown error");
    }
}

void require(bool ok, const char* message) {
    if (!ok) throw std::invalid_argument(message);
}

// ---------------------------------------------------------------------------
// constants and scalar rules (runtime.cu:54-81)
// ---------------------------------------------------------------------------

constexpr int kMinBits = 3;
constexpr int kMaxBits = 15;
constexpr int kFallbackBits = 16;

void validate_storage_bits(int bits) {                 // runtime.cu:58-62
    if (bits < kMinBits || bits > kFallbackBits) {
        throw std::invalid_argument("ElasticBit storage bits must be between 3 and 16");
    }
}

inline int32_t qmax_for_bits(int bits) { return (1 << (bits - 1)) - 1; }   // :64-67

inline size_t packed_bytes(size_t count, int bits) {                         // :69-71
    return (count * static_cast<size_t>(bits) + 7u) / 8u;
}

// IEEE binary16 conversions via the compiler's _Float16 (round to nearest even).
inline uint16_t f32_to_f16_bits(float v) {
    const _Float16 h = static_cast<_Float16>(v);
    uint16_t bits;
    std::memcpy(&bits, &h, sizeof(bits));
    return bits;
}

inline float f16_bits_to_f32(uint16_t bits) {
    _Float16 h;
    std::memcpy(&h, &bits, sizeof(bits));
    return static_cast<float>(h);
}

inline float round_to_fp16(float v) { return static_cast<float>(static_cast<_Float16>(v)); }  // :73-75

inline int32_t quantize_scalar(float value, float scale, int bits) {       // :77-81
    const int32_t qmax = qmax_for_bits(bits);
    const float ratio = value / scale;
    const int32_t q = static_cast<int32_t>(std::nearbyint(ratio));
    return std::max(-qmax, std::min(qmax, q));
}

void check_threshold(double threshold) {
    if (!std::isfinite(threshold) || threshold < 0.0) {
        throw std::invalid_argument("threshold must be a finite non-negative value");
    }
}

int parse_policy(int policy) {
    if (policy != EB_POLICY_HARDWARE_NATIVE && policy != EB_POLICY_FULL_PRECISION) {
        throw std::invalid_argument("decodePolicy must be 'hardwareNative' or 'fullPrecision'");
    }
    return policy;
}

// Worker count for the host O(N*K) loops.
unsigned host_threads(size_t work) {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t by_work = work / (1u << 16) + 1u;
    return static_cast<unsigned>(std::min<size_t>({static_cast<size_t>(hw), by_work, size_t(32)}));
}

template <typename F>
void parallel_for(size_t n, F&& fn) {
    const unsigned t = host_threads(n);
    if (t <= 1 || n < 2) {
        fn(size_t(0), n);
        return;
    }
    std::vector<std::thread> pool;
    const size_t chunk = (n + t - 1) / t;
    for (unsigned i = 0; i < t; ++i) {
        const size_t b = i * chunk;
        const size_t e = std::min(n, b + chunk);
        if (b >= e) break;
        pool.emplace_back([&fn, b, e] { fn(b, e); });
    }
    for (auto& th : pool) th.join();
}

// ---------------------------------------------------------------------------
// canonical storage (runtime.cu:83-238)
// ---------------------------------------------------------------------------

std::vector<float> make_row_scales(const float* w, int rows, int cols, int bits) {  // :83-101
    if (bits == kFallbackBits) return {};
    const float qmax = static_cast<float>(qmax_for_bits(bits));
    std::vector<float> scales(rows, 1.0f);
    for (int r = 0; r < rows; ++r) {
        const float* p = w + static_cast<size_t>(r) * cols;
        float max_abs = 0.0f;
        for (int c = 0; c < cols; ++c) max_abs = std::max(max_abs, std::fabs(p[c]));
        scales[r] = max_abs > 0.0f ? max_abs / qmax : 1.0f;
    }
    return scales;
}

// Writes the b-bit offset codes u of elements [begin, end) of a group of
// eight-code chunks: 8 codes are exactly b bytes, so chunks never share a byte
// and threads may pack disjoint chunk ranges.
template <typename CodeAt>
void pack_chunks(size_t count, int bits, uint8_t* payload, size_t payload_bytes, CodeAt&& code_at) {
    const size_t chunks = (count + 7) / 8;
    parallel_for(chunks, [&](size_t cb, size_t ce) {
        for (size_t chunk = cb; chunk < ce; ++chunk) {
            uint64_t acc = 0;      // up to 8 * 15 = 120 bits: flushed by bytes
            int acc_bits = 0;
            size_t out = chunk * static_cast<size_t>(bits);
            const size_t first = chunk * 8;
            const size_t last = std::min(count, first + 8);
            for (size_t i = first; i < last; ++i) {
                acc |= static_cast<uint64_t>(code_at(i)) << acc_bits;
                acc_bits += bits;
                while (acc_bits >= 8) {
                    payload[out++] = static_cast<uint8_t>(acc & 0xFFu);
                    acc >>= 8;
                    acc_bits -= 8;
                }
            }
            if (acc_bits > 0 && out < payload_bytes) payload[out] = static_cast<uint8_t>(acc & 0xFFu);
        }
    });
}

std::vector<uint8_t> pack_exact_codes(const int16_t* codes, size_t count, int bits) {  // :150-186
    validate_storage_bits(bits);
    if (bits == kFallbackBits) {
        throw std::invalid_argument("prequantized codes are only valid for 3..15-bit storage");
    }
    const int32_t qmax = qmax_for_bits(bits);
    for (size_t i = 0; i < count; ++i) {
        if (codes[i] < -qmax || codes[i] > qmax) {
            throw std::invalid_argument("prequantized ElasticBit code exceeds selected bit range");
        }
    }
    std::vector<uint8_t> payload(packed_bytes(count, bits), 0u);
    pack_chunks(count, bits, payload.data(), payload.size(),
                [&](size_t i) { return static_cast<uint32_t>(codes[i] + qmax); });
    return payload;
}

std::vector<uint8_t> pack_exact_weights(const float* w, int rows, int cols, int bits,
                                        const std::vector<float>& scales) {   // :103-148
    validate_storage_bits(bits);
    const size_t count = static_cast<size_t>(rows) * cols;
    if (bits == kFallbackBits) {
        std::vector<uint8_t> payload(count * 2u);
        for (size_t i = 0; i < count; ++i) {
            const uint16_t h = f32_to_f16_bits(w[i]);
            std::memcpy(&payload[2 * i], &h, 2);
        }
        return payload;
    }
    const int32_t qmax = qmax_for_bits(bits);
    std::vector<uint8_t> payload(packed_bytes(count, bits), 0u);
    pack_chunks(count, bits, payload.data(), payload.size(), [&](size_t i) {
        const size_t r = i / static_cast<size_t>(cols);
        return static_cast<uint32_t>(quantize_scalar(w[i], scales[r], bits) + qmax);
    });
    return payload;
}

inline uint32_t extract_code_host(const uint8_t* payload, size_t nbytes, size_t index, int bits) {  // :188-206
    const size_t bit = index * static_cast<size_t>(bits);
    const size_t byte = bit >> 3;
    uint32_t word = 0;
    for (int k = 0; k < 3; ++k) {
        if (byte + k < nbytes) word |= static_cast<uint32_t>(payload[byte + k]) << (8 * k);
    }
    return (word >> (bit & 7u)) & ((1u << bits) - 1u);
}

std::vector<float> dequantize_payload_host(const std::vector<uint8_t>& payload,
                                           const std::vector<float>& scales, int rows, int cols,
                                           int bits) {   // :208-238
    const size_t count = static_cast<size_t>(rows) * cols;
    std::vector<float> out(count);
    if (bits == kFallbackBits) {
        for (size_t i = 0; i < count; ++i) {
            uint16_t h;
            std::memcpy(&h, &payload[2 * i], 2);
            out[i] = f16_bits_to_f32(h);
        }
        return out;
    }
    const int32_t qmax = qmax_for_bits(bits);
    parallel_for(static_cast<size_t>(rows), [&](size_t rb, size_t re) {
        for (size_t r = rb; r < re; ++r) {
            const float s = scales[r];
            for (int c = 0; c < cols; ++c) {
                const size_t i = r * cols + c;
                const int32_t q = static_cast<int32_t>(extract_code_host(payload.data(), payload.size(), i, bits)) - qmax;
                out[i] = round_to_fp16(static_cast<float>(q) * s);
            }
        }
    });
    return out;
}

// ---------------------------------------------------------------------------
// host analyzer (runtime.cu:280-436)
// ---------------------------------------------------------------------------

struct Analysis {
    int bits = 16;
    double hw = 0.0;
    double full = 0.0;
    double error = 0.0;
    size_t storage_bytes = 0;
};

// One (sample, row) pair's float sums for one width, exactly as :332-369.
struct RowSums {
    float hw;
    float full;
};

std::vector<Analysis> analyze_all_bits(const float* w, int rows, int cols, const float* calib, int samples) {
    if (rows <= 0 || cols <= 0 || samples <= 0) {
        throw std::invalid_argument("weights and calibration must be non-empty");
    }
    const size_t count = static_cast<size_t>(rows) * cols;
    std::vector<float> wh(count);
    for (size_t i = 0; i < count; ++i) wh[i] = round_to_fp16(w[i]);
    std::vector<float> xh(static_cast<size_t>(samples) * cols);
    for (size_t i = 0; i < xh.size(); ++i) xh[i] = round_to_fp16(calib[i]);

    // fp16_reference_outputs, :280-310
    std::vector<float> refs(static_cast<size_t>(samples) * rows);
    parallel_for(static_cast<size_t>(rows), [&](size_t rb, size_t re) {
        for (int s = 0; s < samples; ++s) {
            const float* in = &xh[static_cast<size_t>(s) * cols];
            for (size_t r = rb; r < re; ++r) {
                const float* rp = &wh[r * cols];
                float sum = 0.0f;
                for (int c = 0; c < cols; ++c) {
                    const float p = rp[c] * in[c];
                    sum = sum + p;
                }
                refs[static_cast<size_t>(s) * rows + r] = sum;
            }
        }
    });

    std::vector<Analysis> out;
    std::vector<RowSums> sums(static_cast<size_t>(samples) * rows);
    std::vector<int32_t> q(count);
    for (int bits = kMinBits; bits <= kFallbackBits; ++bits) {
        const std::vector<float> scales = make_row_scales(w, rows, cols, bits);
        parallel_for(static_cast<size_t>(rows), [&](size_t rb, size_t re) {
            if (bits != kFallbackBits) {
                for (size_t r = rb; r < re; ++r)
                    for (int c = 0; c < cols; ++c) q[r * cols + c] = quantize_scalar(w[r * cols + c], scales[r], bits);
            }
            for (int s = 0; s < samples; ++s) {
                const float* in = &xh[static_cast<size_t>(s) * cols];
                for (size_t r = rb; r < re; ++r) {
                    float hw = 0.0f;
                    float full = 0.0f;
                    if (bits == kFallbackBits) {
                        for (int c = 0; c < cols; ++c) {
                            const float p = wh[r * cols + c] * in[c];
                            hw = hw + p;
                        }
                        full = hw;
                    } else if (bits <= 8) {
                        const float scale = scales[r];
                        float idot = 0.0f;
                        for (int c = 0; c < cols; ++c) {
                            const int32_t qq = q[r * cols + c];
                            const float p = static_cast<float>(qq) * in[c];
                            idot = idot + p;
                            const float deq = round_to_fp16(static_cast<float>(qq) * scale);
                            const float p2 = deq * in[c];
                            full = full + p2;
                        }
                        hw = idot * scale;
                    } else {
                        const float scale = scales[r];
                        for (int c = 0; c < cols; ++c) {
                            const float deq = round_to_fp16(static_cast<float>(q[r * cols + c]) * scale);
                            const float p = deq * in[c];
                            hw = hw + p;
                        }
                        full = hw;
                    }
                    sums[static_cast<size_t>(s) * rows + r] = RowSums{hw, full};
                }
            }
        });
        // long-double accumulation in the reference's sample-major order, :371-385
        long double hw_num = 0.0L, full_num = 0.0L, denom = 0.0L;
        for (size_t i = 0; i < sums.size(); ++i) {
            const double ref = refs[i];
            const double hd = static_cast<double>(sums[i].hw) - ref;
            const double fd = static_cast<double>(sums[i].full) - ref;
            hw_num += static_cast<long double>(hd) * hd;
            full_num += static_cast<long double>(fd) * fd;
            denom += static_cast<long double>(ref) * ref;
        }
        const long double safe = std::max(denom, 1.0e-30L);
        Analysis a;
        a.bits = bits;
        a.hw = std::sqrt(static_cast<double>(hw_num / safe));
        a.full = std::sqrt(static_cast<double>(full_num / safe));
        a.error = std::max(a.hw, a.full);
        a.storage_bytes = bits == kFallbackBits ? count * 2u
                                                : packed_bytes(count, bits) + static_cast<size_t>(rows) * 4u;
        out.push_back(a);
    }
    return out;
}

size_t select_analysis(const std::vector<Analysis>& a, double threshold) {   // :408-427
    check_threshold(threshold);
    for (size_t i = 0; i < a.size(); ++i) {
        if (a[i].bits <= kMaxBits && a[i].error <= threshold) return i;
    }
    if (a.back().bits != kFallbackBits) throw std::runtime_error("ElasticBit analyzer internal fallback error");
    return a.size() - 1;
}

// ---------------------------------------------------------------------------
// FNV-1a and the MLB4 header (runtime.cu:682-712)
// ---------------------------------------------------------------------------

uint64_t fnv1a64(const void* data, size_t size) {
    // published FNV-1a 64-bit parameters
    const uint8_t* p = static_cast<const uint8_t*>(data);
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < size; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

#pragma pack(push, 1)
struct MLB4Header {
    char magic[4];
    uint16_t version;
    uint16_t header_bytes;
    uint32_t rows;
    uint32_t cols;
    uint8_t storage_bits;
    uint8_t reserved[3];
    uint32_t scale_count;
    uint64_t scale_bytes;
    uint64_t payload_bytes;
    uint64_t original_fp16_bytes;
    uint64_t scale_checksum;
    uint64_t payload_checksum;
    double threshold;
    double selected_error;
};
#pragma pack(pop)
static_assert(sizeof(MLB4Header) == 80, "MLB4 header is 80 bytes");

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

bool device_present() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return n > 0;
}

// Makes `device` current for the lifetime of the guard.
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        EB_HIP(hipGetDevice(&previous_));
        if (previous_ != device) EB_HIP(hipSetDevice(device));
        target_ = device;
    }
    ~DeviceGuard() {
        if (previous_ != target_) (void)hipSetDevice(previous_);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int previous_ = 0;
    int target_ = 0;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

// ---------------------------------------------------------------------------
// the matrix handle
// ---------------------------------------------------------------------------

struct eb_matrix {
    int rows = 0;
    int cols = 0;
    int bits = kFallbackBits;
    double threshold = 0.0;
    double selected_error = 0.0;
    int policy = EB_POLICY_HARDWARE_NATIVE;

    std::vector<float> scales;      // canonical storage (MLB4 body)
    std::vector<uint8_t> payload;

    int device = -1;                // -1: host-only (no HIP device present)
    void* d_exec = nullptr;         // planes + scales (or raw fp16), one allocation
    size_t exec_bytes = 0;
    ebk::DevMatrix dev;
    uint16_t* d_host_in = nullptr;  // numpy-path staging, allocated on first use
    uint16_t* d_host_out = nullptr;

    ~eb_matrix() { release(); }

    void release() noexcept {
        if (device < 0) return;
        int prev = 0;
        const bool have_prev = hipGetDevice(&prev) == hipSuccess;
        if (have_prev && prev != device) (void)hipSetDevice(device);
        if (d_exec) (void)hipFree(d_exec);
        if (d_host_in) (void)hipFree(d_host_in);
        if (d_host_out) (void)hipFree(d_host_out);
        if (have_prev && prev != device) (void)hipSetDevice(prev);
        d_exec = nullptr;
        d_host_in = d_host_out = nullptr;
    }

    // Upload the canonical stream and re-lay it out as bit planes on the
    // current device (the reference widens at the same point,
    // configure_execution_weights, runtime.cu:1315-1334).
    // Execution layout on the current device, repacked from the canonical
    // stream: `d_canon` when the caller already holds a device copy, else
    // an upload of `payload`.
    void build_device(const uint8_t* d_canon = nullptr) {
        if (!device_present()) return;
        EB_HIP(hipGetDevice(&device));
        const int gpr = (cols + ebk::kGroup - 1) / ebk::kGroup;
        const int spr = (gpr + ebk::kTileGroups - 1) / ebk::kTileGroups;
        const int rtiles = (rows + ebk::kTileRows - 1) / ebk::kTileRows;
        const size_t groups = static_cast<size_t>(rtiles) * spr * ebk::kTileSlots;
        size_t offs[6] = {0, 0, 0, 0, 0, 0};
        const int widths[5] = {8, 4, 2, 1, 16};
        size_t total = 0;
        for (int i = 0; i < 5; ++i) {
            offs[i] = total;
            total = align_up(total + ebk::plane_bytes(bits, widths[i], groups), 256);
        }
        offs[5] = total;
        if (bits != kFallbackBits) total = align_up(total + scales.size() * sizeof(float), 256);
        EB_HIP(hipMalloc(&d_exec, total));
        exec_bytes = total;
        uint8_t* base = static_cast<uint8_t*>(d_exec);

        ebk::DevMatrixOut out;
        out.rows = rows;
        out.cols = cols;
        out.gpr = gpr;
        out.spr = spr;
        out.rtiles = rtiles;
        out.bits = bits;
        auto at = [&](int i, int width) -> uint8_t* {
            return ebk::plane_bytes(bits, width, groups) ? base + offs[i] : nullptr;
        };
        out.p8 = at(0, 8);
        out.p4 = at(1, 4);
        out.p2 = at(2, 2);
        out.p1 = at(3, 1);
        out.w16 = reinterpret_cast<uint16_t*>(at(4, 16));

        dev = ebk::DevMatrix{};
        dev.p8 = out.p8;
        dev.p4 = out.p4;
        dev.p2 = out.p2;
        dev.p1 = out.p1;
        dev.w16 = out.w16;
        dev.rows = rows;
        dev.cols = cols;
        dev.gpr = gpr;
        dev.spr = spr;
        dev.rtiles = rtiles;
        dev.bits = bits;
        if (bits != kFallbackBits) {
            float* d_scales = reinterpret_cast<float*>(base + offs[5]);
            EB_HIP(hipMemcpy(d_scales, scales.data(), scales.size() * sizeof(float), hipMemcpyHostToDevice));
            dev.scales = d_scales;
        }

        if (d_canon) {
            EB_HIP(ebk::launch_repack(d_canon, payload.size(), out, nullptr));
            EB_HIP(hipStreamSynchronize(nullptr));
            return;
        }
        void* d_copy = nullptr;
        EB_HIP(hipMalloc(&d_copy, std::max<size_t>(payload.size(), 1)));
        hipError_t err = hipMemcpy(d_copy, payload.data(), payload.size(), hipMemcpyHostToDevice);
        if (err == hipSuccess) {
            err = ebk::launch_repack(static_cast<const uint8_t*>(d_copy), payload.size(), out, nullptr);
        }
        if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
        (void)hipFree(d_copy);
        EB_HIP(err);
    }

    void require_device() const {
        if (device < 0) {
            throw std::runtime_error(
                "ElasticBit requires its CUDA runtime: no HIP (gfx950) device is available to this matrix");
        }
    }

    // hardwareNative b <= 12 multiplies the integer codes (exact in fp16)
    // and scales once; b >= 13 and fullPrecision use the decoded fp16 weights.
    bool exact_w16() const { return policy == EB_POLICY_FULL_PRECISION || bits > 12; }

    int execution_width() const {
        if (bits == kFallbackBits || policy == EB_POLICY_FULL_PRECISION) return 16;
        return bits;
    }

    const char* execution_planner() const {
        return policy == EB_POLICY_FULL_PRECISION ? "fullPrecision" : "gfx950BitPlane";
    }

    size_t storage_bytes() const { return payload.size() + scales.size() * sizeof(float); }
    size_t original_bytes() const { return static_cast<size_t>(rows) * cols * 2u; }
};

namespace {

std::unique_ptr<eb_matrix> make_matrix(int rows, int cols, int bits, double threshold, double error,
                                       int policy, std::vector<float>&& scales,
                                       std::vector<uint8_t>&& payload) {
    auto m = std::make_unique<eb_matrix>();
    m->rows = rows;
    m->cols = cols;
    m->bits = bits;
    m->threshold = threshold;
    m->selected_error = error;
    m->policy = policy;
    m->scales = std::move(scales);
    m->payload = std::move(payload);
    m->build_device();
    return m;
}

void check_dims(int rows, int cols) {
    require(rows > 0 && cols > 0, "ElasticBit matrix dimensions must be positive");
}

std::unique_ptr<eb_matrix> from_weights(const float* w, int rows, int cols, int bits, double threshold,
                                        double error, int policy) {
    check_dims(rows, cols);
    validate_storage_bits(bits);
    std::vector<float> scales = make_row_scales(w, rows, cols, bits);
    std::vector<uint8_t> payload = pack_exact_weights(w, rows, cols, bits, scales);
    return make_matrix(rows, cols, bits, threshold, error, policy, std::move(scales), std::move(payload));
}

void fill_analysis(const Analysis& a, size_t original, eb_bit_analysis* out, double threshold) {
    out->bits = a.bits;
    out->hardware_native_error = a.hw;
    out->full_precision_error = a.full;
    out->error = a.error;
    out->storage_bytes = a.storage_bytes;
    out->memory_reduction = 1.0 - static_cast<double>(a.storage_bytes) / static_cast<double>(original);
    out->passes = a.error <= threshold ? 1 : 0;
}

template <size_t N>
void copy_str(char (&dst)[N], const std::string& src) {
    std::snprintf(dst, N, "%s", src.c_str());
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

const char* eb_last_error(void) { return g_last_error.c_str(); }

int eb_abi_version(void) { return EB_ABI_VERSION; }

int eb_analyze(const float* weights, int rows, int cols, const float* calibration, int samples,
               double threshold, eb_bit_analysis* out14, int* selected_index) {
    return guarded([&] {
        require(weights && calibration && out14, "analyze: null pointer");
        const auto analyses = analyze_all_bits(weights, rows, cols, calibration, samples);
        const size_t sel = select_analysis(analyses, threshold);
        const size_t original = static_cast<size_t>(rows) * cols * 2u;
        for (size_t i = 0; i < analyses.size(); ++i) fill_analysis(analyses[i], original, &out14[i], threshold);
        if (selected_index) *selected_index = static_cast<int>(sel);
    });
}

int eb_backend_info(eb_backend* out) {
    return guarded([&] {
        require(out != nullptr, "backendInfo: null pointer");
        std::memset(out, 0, sizeof(*out));
        copy_str(out->activate_dtype, "float16");
        copy_str(out->prefill, "native");
        copy_str(out->decode_planner, "gfx950BitPlane");
        copy_str(out->decode_engine, "BitPlaneMFMA");
        copy_str(out->decode_status, "experimental");
        copy_str(out->decode_validation, "unvalidated");
        out->n_weight_widths = 14;
        for (int b = kMinBits; b <= kFallbackBits; ++b) out->weight_widths[b - kMinBits] = b;
        out->device_index = -1;
        if (!device_present()) return;
        int device = 0;
        EB_HIP(hipGetDevice(&device));
        hipDeviceProp_t prop;
        EB_HIP(hipGetDeviceProperties(&prop, device));
        out->available = 1;
        out->device_index = device;
        out->compute_units = prop.multiProcessorCount;
        copy_str(out->device, prop.name);
        std::string arch = prop.gcnArchName;
        const size_t colon = arch.find(':');
        if (colon != std::string::npos) arch = arch.substr(0, colon);
        copy_str(out->architecture, arch);
    });
}

int eb_compress(const float* weights, int rows, int cols, const float* calibration, int samples,
                double threshold, int policy, eb_matrix** out) {
    return guarded([&] {
        require(weights && calibration && out, "compress: null pointer");
        parse_policy(policy);
        const auto analyses = analyze_all_bits(weights, rows, cols, calibration, samples);
        const Analysis& sel = analyses[select_analysis(analyses, threshold)];
        *out = from_weights(weights, rows, cols, sel.bits, threshold, sel.error, policy).release();
    });
}

int eb_compress_selected(const float* weights, int rows, int cols, int selected_bits, double threshold,
                         double selected_error, int policy, eb_matrix** out) {
    return guarded([&] {                                 // runtime.cu:748-776
        require(weights && out, "compressSelected: null pointer");
        validate_storage_bits(selected_bits);
        check_threshold(threshold);
        if (!std::isfinite(selected_error) || selected_error < 0.0) {
            throw std::invalid_argument("selectedError must be a finite non-negative value");
        }
        if (selected_bits <= kMaxBits && selected_error > threshold) {
            throw std::invalid_argument("selected compressed width does not satisfy threshold");
        }
        if (selected_bits == kFallbackBits) selected_error = 0.0;
        parse_policy(policy);
        *out = from_weights(weights, rows, cols, selected_bits, threshold, selected_error, policy).release();
    });
}

int eb_compress_selected_codes(const int16_t* codes, const float* scales, int rows, int cols,
                               int selected_bits, double threshold, double selected_error, int policy,
                               eb_matrix** out) {
    return guarded([&] {                                 // runtime.cu:778-808, 1109-1141
        require(codes && scales && out, "compressSelectedCodes: null pointer");
        validate_storage_bits(selected_bits);
        if (selected_bits == kFallbackBits) {
            throw std::invalid_argument("prequantized codes require 3..15-bit storage");
        }
        check_threshold(threshold);
        if (!std::isfinite(selected_error) || selected_error < 0.0 || selected_error > threshold) {
            throw std::invalid_argument("selected compressed width does not satisfy threshold");
        }
        parse_policy(policy);
        check_dims(rows, cols);
        std::vector<float> s(scales, scales + rows);
        for (float v : s) {
            if (!std::isfinite(v) || v <= 0.0f) {
                throw std::invalid_argument("ElasticBit scales must be finite and positive");
            }
        }
        std::vector<uint8_t> payload = pack_exact_codes(codes, static_cast<size_t>(rows) * cols, selected_bits);
        *out = make_matrix(rows, cols, selected_bits, threshold, selected_error, policy, std::move(s),
                           std::move(payload)).release();
    });
}

int eb_compress_selected_codes_device(const int16_t* codes_dev, const float* scales, int rows, int cols,
                                      int selected_bits, double threshold, double selected_error, int policy,
                                      eb_matrix** out) {
    return guarded([&] {                                 // runtime.cu:778-808, 150-186
        require(codes_dev && scales && out, "compressSelectedCodes: null pointer");
        validate_storage_bits(selected_bits);
        if (selected_bits == kFallbackBits) {
            throw std::invalid_argument("prequantized codes require 3..15-bit storage");
        }
        check_threshold(threshold);
        if (!std::isfinite(selected_error) || selected_error < 0.0 || selected_error > threshold) {
            throw std::invalid_argument("selected compressed width does not satisfy threshold");
        }
        parse_policy(policy);
        check_dims(rows, cols);
        require(device_present(), "ElasticBit requires its CUDA runtime: no HIP (gfx950) device is available");
        std::vector<float> s(scales, scales + rows);
        for (float v : s) {
            if (!std::isfinite(v) || v <= 0.0f) {
                throw std::invalid_argument("ElasticBit scales must be finite and positive");
            }
        }
        const size_t count = static_cast<size_t>(rows) * cols;
        const size_t nbytes = packed_bytes(count, selected_bits);
        // one allocation: the stream, then the range flag (256-byte aligned)
        const size_t flag_off = align_up(std::max<size_t>(nbytes, 1), 256);
        void* d_buf = nullptr;
        EB_HIP(hipMalloc(&d_buf, flag_off + sizeof(int)));
        auto* d_canon = static_cast<uint8_t*>(d_buf);
        auto* d_bad = reinterpret_cast<int*>(d_canon + flag_off);
        std::unique_ptr<eb_matrix> m;
        try {
            EB_HIP(hipMemset(d_bad, 0, sizeof(int)));
            EB_HIP(ebk::launch_pack_codes(codes_dev, count, selected_bits, d_canon, nbytes, d_bad, nullptr));
            int bad = 0;
            EB_HIP(hipMemcpy(&bad, d_bad, sizeof(int), hipMemcpyDeviceToHost));
            if (bad) throw std::invalid_argument("prequantized ElasticBit code exceeds selected bit range");
            std::vector<uint8_t> payload(nbytes);
            EB_HIP(hipMemcpy(payload.data(), d_canon, nbytes, hipMemcpyDeviceToHost));
            m = std::make_unique<eb_matrix>();
            m->rows = rows;
            m->cols = cols;
            m->bits = selected_bits;
            m->threshold = threshold;
            m->selected_error = selected_error;
            m->policy = policy;
            m->scales = std::move(s);
            m->payload = std::move(payload);
            m->build_device(d_canon);
        } catch (...) {
            (void)hipFree(d_buf);
            throw;
        }
        (void)hipFree(d_buf);
        *out = m.release();
    });
}

int eb_load(const char* path, int policy, eb_matrix** out) {
    return guarded([&] {                                 // runtime.cu:810-871
        require(path && out, "load: null pointer");
        parse_policy(policy);
        std::ifstream stream(path, std::ios::binary | std::ios::ate);
        if (!stream) throw std::runtime_error(std::string("failed to open ElasticBit file: ") + path);
        const std::streamsize file_size = stream.tellg();
        stream.seekg(0, std::ios::beg);
        MLB4Header h{};
        stream.read(reinterpret_cast<char*>(&h), sizeof(h));
        if (!stream || std::memcmp(h.magic, "MLB4", 4) != 0) throw std::runtime_error("invalid ElasticBit MLB4 file");
        if (h.version != 4 || h.header_bytes != sizeof(MLB4Header)) {
            throw std::runtime_error("unsupported ElasticBit MLB4 version");
        }
        validate_storage_bits(h.storage_bits);
        if (h.rows == 0 || h.cols == 0 || h.rows > 0x7fffffffu || h.cols > 0x7fffffffu) {
            throw std::runtime_error("invalid ElasticBit matrix dimensions");
        }
        const size_t count = static_cast<size_t>(h.rows) * h.cols;
        const size_t expected_payload = h.storage_bits == kFallbackBits ? count * 2u : packed_bytes(count, h.storage_bits);
        const size_t expected_scales = h.storage_bits == kFallbackBits ? 0u : h.rows;
        const size_t expected_scale_bytes = expected_scales * sizeof(float);
        const size_t expected_file = sizeof(MLB4Header) + expected_scale_bytes + expected_payload;
        if (h.scale_count != expected_scales || h.scale_bytes != expected_scale_bytes ||
            h.payload_bytes != expected_payload || h.original_fp16_bytes != count * 2u ||
            file_size != static_cast<std::streamsize>(expected_file)) {
            throw std::runtime_error("invalid ElasticBit MLB4 metadata");
        }
        std::vector<float> scales(expected_scales);
        if (!scales.empty()) stream.read(reinterpret_cast<char*>(scales.data()), expected_scale_bytes);
        std::vector<uint8_t> payload(expected_payload);
        stream.read(reinterpret_cast<char*>(payload.data()), expected_payload);
        if (!stream) throw std::runtime_error("truncated ElasticBit MLB4 file");
        const uint64_t sc = scales.empty() ? fnv1a64(nullptr, 0) : fnv1a64(scales.data(), expected_scale_bytes);
        const uint64_t pc = fnv1a64(payload.data(), payload.size());
        if (sc != h.scale_checksum || pc != h.payload_checksum) {
            throw std::runtime_error("ElasticBit MLB4 checksum mismatch");
        }
        *out = make_matrix(static_cast<int>(h.rows), static_cast<int>(h.cols), h.storage_bits, h.threshold,
                           h.selected_error, policy, std::move(scales), std::move(payload)).release();
    });
}

int eb_save(const eb_matrix* m, const char* path) {
    return guarded([&] {                                 // runtime.cu:1024-1049
        require(m && path, "save: null pointer");
        MLB4Header h{};
        std::memcpy(h.magic, "MLB4", 4);
        h.version = 4;
        h.header_bytes = sizeof(MLB4Header);
        h.rows = static_cast<uint32_t>(m->rows);
        h.cols = static_cast<uint32_t>(m->cols);
        h.storage_bits = static_cast<uint8_t>(m->bits);
        h.scale_count = static_cast<uint32_t>(m->scales.size());
        h.scale_bytes = m->scales.size() * sizeof(float);
        h.payload_bytes = m->payload.size();
        h.original_fp16_bytes = m->original_bytes();
        h.scale_checksum = m->scales.empty() ? fnv1a64(nullptr, 0) : fnv1a64(m->scales.data(), h.scale_bytes);
        h.payload_checksum = fnv1a64(m->payload.data(), m->payload.size());
        h.threshold = m->threshold;
        h.selected_error = m->selected_error;
        std::ofstream stream(path, std::ios::binary);
        if (!stream) throw std::runtime_error(std::string("failed to open ElasticBit output: ") + path);
        stream.write(reinterpret_cast<const char*>(&h), sizeof(h));
        if (!m->scales.empty()) stream.write(reinterpret_cast<const char*>(m->scales.data()), h.scale_bytes);
        stream.write(reinterpret_cast<const char*>(m->payload.data()), h.payload_bytes);
        if (!stream) throw std::runtime_error("failed while writing ElasticBit output");
    });
}

void eb_destroy(eb_matrix* m) { delete m; }

int eb_get_props(const eb_matrix* m, eb_props* out) {
    return guarded([&] {
        require(m && out, "props: null pointer");
        std::memset(out, 0, sizeof(*out));
        out->rows = m->rows;
        out->cols = m->cols;
        out->storage_bits = m->bits;
        out->execution_width = m->execution_width();
        out->decode_policy = m->policy;
        out->device_index = m->device;
        out->storage_bytes = m->storage_bytes();
        out->execution_bytes = m->exec_bytes;
        out->original_bytes = m->original_bytes();
        out->threshold = m->threshold;
        out->selected_error = m->selected_error;
        out->memory_reduction = 1.0 - static_cast<double>(m->storage_bytes()) / static_cast<double>(m->original_bytes());
        copy_str(out->execution_planner, m->execution_planner());
    });
}

int eb_set_decode_policy(eb_matrix* m, int policy) {
    return guarded([&] {                                 // runtime.cu:975-980
        require(m != nullptr, "setDecodePolicy: null matrix");
        m->policy = parse_policy(policy);
    });
}

int eb_get_canonical(const eb_matrix* m, float* scales_out, uint8_t* payload_out) {
    return guarded([&] {
        require(m != nullptr, "canonical: null matrix");
        if (scales_out && !m->scales.empty()) std::memcpy(scales_out, m->scales.data(), m->scales.size() * sizeof(float));
        if (payload_out) std::memcpy(payload_out, m->payload.data(), m->payload.size());
    });
}

int eb_dequantize_host(const eb_matrix* m, float* out) {
    return guarded([&] {                                 // runtime.cu:967-973
        require(m && out, "dequantize: null pointer");
        const auto v = dequantize_payload_host(m->payload, m->scales, m->rows, m->cols, m->bits);
        std::memcpy(out, v.data(), v.size() * sizeof(float));
    });
}

static void ensure_host_io(eb_matrix* m) {
    if (!m->d_host_in) EB_HIP(hipMalloc(reinterpret_cast<void**>(&m->d_host_in), static_cast<size_t>(m->cols) * 2u));
    if (!m->d_host_out) EB_HIP(hipMalloc(reinterpret_cast<void**>(&m->d_host_out), static_cast<size_t>(m->rows) * 2u));
}

static void launch_forward(const eb_matrix* m, const uint16_t* x, int64_t M, uint16_t* y, const uint16_t* bias,
                           hipStream_t stream) {
    EB_HIP(ebk::launch_linear(m->dev, m->exact_w16(), x, M, y, bias, stream));
}

int eb_forward_host(eb_matrix* m, const float* x, float* y) {
    return guarded([&] {                                 // runtime.cu:873-900
        require(m && x && y, "forward: null pointer");
        m->require_device();
        DeviceGuard guard(m->device);
        ensure_host_io(m);
        std::vector<uint16_t> xin(m->cols);
        for (int c = 0; c < m->cols; ++c) xin[c] = f32_to_f16_bits(x[c]);
        EB_HIP(hipMemcpy(m->d_host_in, xin.data(), xin.size() * 2u, hipMemcpyHostToDevice));
        launch_forward(m, m->d_host_in, 1, m->d_host_out, nullptr, nullptr);
        std::vector<uint16_t> yout(m->rows);
        EB_HIP(hipMemcpy(yout.data(), m->d_host_out, yout.size() * 2u, hipMemcpyDeviceToHost));
        for (int r = 0; r < m->rows; ++r) y[r] = f16_bits_to_f32(yout[r]);
    });
}

int eb_benchmark(eb_matrix* m, const float* x, int iterations, double* ms_per_iteration) {
    return guarded([&] {                                 // runtime.cu:933-965
        require(m && x && ms_per_iteration, "benchmark: null pointer");
        require(iterations > 0, "iterations must be positive");
        m->require_device();
        DeviceGuard guard(m->device);
        ensure_host_io(m);
        std::vector<uint16_t> xin(m->cols);
        for (int c = 0; c < m->cols; ++c) xin[c] = f32_to_f16_bits(x[c]);
        EB_HIP(hipMemcpy(m->d_host_in, xin.data(), xin.size() * 2u, hipMemcpyHostToDevice));
        for (int i = 0; i < 20; ++i) launch_forward(m, m->d_host_in, 1, m->d_host_out, nullptr, nullptr);
        EB_HIP(hipDeviceSynchronize());
        hipEvent_t start, stop;
        EB_HIP(hipEventCreate(&start));
        EB_HIP(hipEventCreate(&stop));
        EB_HIP(hipEventRecord(start, nullptr));
        for (int i = 0; i < iterations; ++i) launch_forward(m, m->d_host_in, 1, m->d_host_out, nullptr, nullptr);
        EB_HIP(hipEventRecord(stop, nullptr));
        EB_HIP(hipEventSynchronize(stop));
        float ms = 0.0f;
        EB_HIP(hipEventElapsedTime(&ms, start, stop));
        (void)hipEventDestroy(start);
        (void)hipEventDestroy(stop);
        *ms_per_iteration = static_cast<double>(ms) / iterations;
    });
}

int eb_forward(const eb_matrix* m, const void* x_f16, int64_t M, void* y_f16, const void* bias_f16, void* stream) {
    return guarded([&] {                                 // runtime.cu:902-931; core.py:446-471
        require(m && x_f16 && y_f16, "forward: null pointer");
        require(M >= 1 && M <= 0x7fffffffLL, "forward: M must be in [1, 2^31)");
        m->require_device();
        DeviceGuard guard(m->device);
        launch_forward(m, static_cast<const uint16_t*>(x_f16), M, static_cast<uint16_t*>(y_f16),
                       static_cast<const uint16_t*>(bias_f16), static_cast<hipStream_t>(stream));
    });
}

int eb_forward_multi(const eb_matrix* const* ms, int count, const void* x_f16, int64_t M, void* const* ys_f16,
                     const void* const* biases_f16, void* stream) {
    return guarded([&] {
        require(ms && ys_f16 && x_f16, "forward_multi: null pointer");
        require(count >= 1, "forward_multi: count must be positive");
        require(M >= 1 && M <= 0x7fffffffLL, "forward: M must be in [1, 2^31)");
        for (int j = 0; j < count; ++j) {
            require(ms[j] && ys_f16[j], "forward_multi: null pointer");
            ms[j]->require_device();
            require(ms[j]->cols == ms[0]->cols, "forward_multi: matrices must share in_features");
            require(ms[j]->device == ms[0]->device, "forward_multi: matrices must be on one device");
        }
        DeviceGuard guard(ms[0]->device);
        // consecutive matrices of one width and arithmetic share a launch
        ebk::DevMatrix dev[ebk::kMultiMax];
        uint16_t* ys[ebk::kMultiMax];
        const uint16_t* bs[ebk::kMultiMax];
        for (int j0 = 0; j0 < count;) {
            const bool w16 = ms[j0]->exact_w16();
            int n = 0;
            while (j0 + n < count && n < ebk::kMultiMax && ms[j0 + n]->bits == ms[j0]->bits &&
                   ms[j0 + n]->exact_w16() == w16) {
                dev[n] = ms[j0 + n]->dev;
                ys[n] = static_cast<uint16_t*>(ys_f16[j0 + n]);
                bs[n] = biases_f16 ? static_cast<const uint16_t*>(biases_f16[j0 + n]) : nullptr;
                ++n;
            }
            EB_HIP(ebk::launch_linear_multi(dev, n, w16, static_cast<const uint16_t*>(x_f16), M, ys, bs,
                                            static_cast<hipStream_t>(stream)));
            j0 += n;
        }
    });
}

int eb_analyze_widths_device(const void* w_f16, int64_t rows, int64_t cols, const void* x_f16, int64_t samples,
                             const float* max_abs, float* partials, void* stream) {
    return guarded([&] {                                 // core.py:112-195
        static_assert(EB_ANALYZE_TILE_ROWS == ebk::kAnalyzeTileRows && EB_ANALYZE_SUMS == ebk::kAnalyzeSums &&
                          EB_ANALYZE_MAX_SAMPLES == ebk::kAnalyzeMaxSamples,
                      "analyzer constants");
        require(w_f16 && x_f16 && max_abs && partials, "analyze_widths: null pointer");
        require(rows >= 1 && cols >= 1 && rows <= 0x7fffffffLL && cols <= 0x7fffffffLL,
                "analyze_widths: rows and cols must be in [1, 2^31)");
        require(samples >= 1 && samples <= EB_ANALYZE_MAX_SAMPLES,
                "analyze_widths: samples must be in [1, 32]");
        EB_HIP(ebk::launch_analyze_widths(static_cast<const uint16_t*>(w_f16), static_cast<int>(rows),
                                          static_cast<int>(cols), static_cast<const uint16_t*>(x_f16),
                                          static_cast<int>(samples), max_abs, partials,
                                          static_cast<hipStream_t>(stream)));
    });
}

int eb_analyze_widths_device_totals(const void* w_f16, int64_t rows, int64_t cols, const void* x_f16,
                                    int64_t samples, const float* max_abs, double* totals, void* stream) {
    return guarded([&] {
        static_assert(EB_ANALYZE_STATIC_MAX_ROWS == ebk::kAnalyzeScratchTiles * ebk::kAnalyzeTileRows,
                      "static scratch size");
        require(w_f16 && x_f16 && max_abs && totals, "analyze_widths_totals: null pointer");
        require(rows >= 1 && cols >= 1 && cols <= 0x7fffffffLL,
                "analyze_widths_totals: rows and cols must be positive");
        require(rows <= EB_ANALYZE_STATIC_MAX_ROWS,
                "analyze_widths_totals: rows exceed the static scratch (262144 rows)");
        require(samples >= 1 && samples <= EB_ANALYZE_MAX_SAMPLES,
                "analyze_widths_totals: samples must be in [1, 32]");
        EB_HIP(ebk::launch_analyze_widths_totals(static_cast<const uint16_t*>(w_f16), static_cast<int>(rows),
                                                 static_cast<int>(cols), static_cast<const uint16_t*>(x_f16),
                                                 static_cast<int>(samples), max_abs, totals,
                                                 static_cast<hipStream_t>(stream)));
    });
}

int eb_materialize_fp16(const eb_matrix* m, void* out_f16, void* stream) {
    return guarded([&] {                                 // runtime.cu:982-1022
        require(m && out_f16, "materialize: null pointer");
        m->require_device();
        DeviceGuard guard(m->device);
        EB_HIP(ebk::launch_materialize(m->dev, static_cast<uint16_t*>(out_f16), static_cast<hipStream_t>(stream)));
    });
}

int eb_unpack_codes(const eb_matrix* m, int16_t* out, void* stream) {
    return guarded([&] {
        require(m && out, "unpack: null pointer");
        require(m->bits != kFallbackBits, "fp16 storage has no integer codes");
        m->require_device();
        DeviceGuard guard(m->device);
        EB_HIP(ebk::launch_unpack(m->dev, out, static_cast<hipStream_t>(stream)));
    });
}

int eb_packed_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed, const void* scales,
                     int scale_dtype, const void* bias, int bits, int64_t group_size, int64_t out_features,
                     int64_t in_features, void* y, void* stream) {
    return guarded([&] {                                 // bolt/ops.cpp:1012-1043
        require(x && packed && scales && y, "elastic_linear_packed: null pointer");
        require(bits >= 2 && bits <= 8, "bits must be in [2,8]");
        require(group_size > 0 && out_features > 0 && in_features > 0, "invalid ElasticBit dimensions");
        require(M >= 0, "elastic_linear_packed: negative row count");
        require(x_dtype >= EB_DTYPE_F32 && x_dtype <= EB_DTYPE_BF16, "x/scales must be floating point");
        require(scale_dtype >= EB_DTYPE_F32 && scale_dtype <= EB_DTYPE_BF16, "x/scales must be floating point");
        require(out_features <= 0x7fffffffLL && (M + 3) / 4 <= 0x7fffffffLL, "elastic_linear_packed: shape too large");
        if (M == 0) return;
        EB_HIP(ebk::launch_packed_linear(x, x_dtype, M, packed, scales, scale_dtype, bias, bits, group_size,
                                         out_features, in_features, y, static_cast<hipStream_t>(stream)));
    });
}

int eb_set_prefill_tiles(int mode) {
    return guarded([&] {
        require(mode == EB_PREFILL_TILES_AUTO || mode == EB_PREFILL_TILES_NARROW || mode == EB_PREFILL_TILES_WIDE ||
                    mode == EB_PREFILL_TILES_WIDE8 || mode == EB_PREFILL_TILES_WIDE8_PLAIN ||
                    mode == EB_PREFILL_TILES_WIDE8_SHORT || mode == EB_PREFILL_TILES_WIDE_PLAIN ||
                    mode == EB_PREFILL_TILES_WIDE_SHORT,
                "prefill tile mode must be auto (0), narrow (1), wide (2), wide with eight waves (3), "
                "the same without round balancing (4), 192-row tiles with eight waves (5), four-wave wide "
                "tiles without round balancing (6) or 192-row tiles with four waves (7)");
        ebk::set_prefill_tiles(mode);
    });
}

int eb_prefill_plan(int64_t M, int rows, int cus, int32_t* rects, double* cost) {
    return guarded([&] {
        require(M >= 1 && M <= 0x7fffffffLL && rows >= 1 && cus >= 1, "prefill plan: M, rows and cus must be positive");
        require(rects != nullptr, "prefill plan: rects is null");
        const double c = ebk::prefill_pp_plan_rects(M, rows, cus, ebk::prefill_tiles_mode(), rects);
        if (cost) *cost = c;
    });
}

int eb_host_pack_codes(const int16_t* codes, uint64_t count, int bits, uint8_t* payload, uint64_t payload_bytes) {
    return guarded([&] {
        require(codes && payload, "pack: null pointer");
        const auto p = pack_exact_codes(codes, count, bits);
        require(p.size() == payload_bytes, "pack: payload_bytes must equal ceil(count*bits/8)");
        std::memcpy(payload, p.data(), p.size());
    });
}

int eb_host_unpack_codes(const uint8_t* payload, uint64_t payload_bytes, uint64_t count, int bits, int16_t* codes) {
    return guarded([&] {
        require(payload && codes, "unpack: null pointer");
        validate_storage_bits(bits);
        require(bits != kFallbackBits, "fp16 storage has no integer codes");
        require(payload_bytes >= packed_bytes(count, bits), "unpack: payload too small");
        const int32_t qmax = qmax_for_bits(bits);
        parallel_for(count, [&](size_t b, size_t e) {
            for (size_t i = b; i < e; ++i) {
                codes[i] = static_cast<int16_t>(static_cast<int32_t>(extract_code_host(payload, payload_bytes, i, bits)) - qmax);
            }
        });
    });
}

}  // extern "C"
