// mlq CPU oracle -- TEST INFRASTRUCTURE ONLY.
//
// A from-scratch C++ restatement of mini-llama.cpp's CPU quantized-linear path.
// It is the checker for the HIP kernels and the "port" CPU baseline; nothing in
// the product library links or calls it.  Only tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg may load it.
//
// Build: oracle/Makefile (g++ -O2 -ffp-contract=off, no -march), matching the
// reference Release flags (CMakeLists.txt:292) so the rounding sequence of the
// scalar linear is reproduced bit for bit: one multiply and one add per element,
// each rounded to fp32, in ascending k order.
//
// Pinning (what checks each function; all live in tests/):
//   fp16 encode  -- golden bytes from the compiled reference (tests/golden),
//                   exhaustive comparison with a numpy closed form over every
//                   fp16 bucket boundary, overflow/NaN -> Inf special cases.
//   fp16 decode  -- all 65536 inputs against numpy.float16 (IEEE binary16).
//   quantizers   -- golden block bytes from the compiled reference, KATs from
//                   tests/test_quant.cpp, round-trip bounds, zero/tail cases.
//   linear       -- golden y bits from the compiled reference, fp64 brute force
//                   on small shapes, Q4_1 known answer 64.0, thread-count
//                   invariance.
//
// Reference citations are to /root/reference (yus3nable/mini-llama-cpp-release).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr int kQK = 32;  // elements per block for every format (quantized_tensor.h:24,37,51)

// Block layouts: quantized_tensor.h:26-29 (Q8_0), :39-42 (Q4_0), :53-57 (Q4_1).
// The byte layout is the ggml one and is the storage contract of the whole path.
#pragma pack(push, 1)
struct Q8Block { uint16_t d; int8_t q[32]; };
struct Q40Block { uint16_t d; uint8_t q[16]; };
struct Q41Block { uint16_t d; uint16_t m; uint8_t q[16]; };
#pragma pack(pop)
static_assert(sizeof(Q8Block) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(Q40Block) == 18, "Q4_0 block is 18 bytes");
static_assert(sizeof(Q41Block) == 20, "Q4_1 block is 20 bytes");

enum QType { kF32 = 0, kQ8_0 = 1, kQ4_0 = 2, kQ4_1 = 3 };  // QuantType order, quantized_tensor.h:13-18

// --- binary16 codec -------------------------------------------------------

// f32 -> binary16 bits, following src/quant.cpp:19-55.  Rounding looks only at
// the first discarded bit (bit 12 of the f32 fraction) and rounds the magnitude
// up when it is set: ties go away from zero, unlike IEEE round-to-even.
// Exponent overflow, +-Inf and NaN all become +-Inf; values below half the
// smallest subnormal flush to a signed zero.
uint16_t half_from_float(float value) {
    uint32_t u;
    std::memcpy(&u, &value, sizeof u);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = static_cast<int>((u >> 23) & 0xffu) - 112;  // 127 -> 15 rebias
    const uint32_t frac = u & 0x7fffffu;

    if (e >= 31) {
        return static_cast<uint16_t>(sign | 0x7c00u);
    }
    if (e <= 0) {
        if (e < -10) {
            return static_cast<uint16_t>(sign);
        }
        uint32_t sig = (frac | 0x800000u) >> (1 - e);
        if (sig & 0x1000u) sig += 0x2000u;  // carry may promote to the smallest normal
        return static_cast<uint16_t>(sign | (sig >> 13));
    }
    uint32_t sig = frac;
    int exp_h = e;
    if (sig & 0x1000u) {
        sig += 0x2000u;
        if (sig & 0x800000u) {  // fraction overflowed into the exponent
            sig = 0;
            if (++exp_h >= 31) {
                return static_cast<uint16_t>(sign | 0x7c00u);
            }
        }
    }
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(exp_h) << 10) | (sig >> 13));
}

// binary16 bits -> f32, the exact IEEE value (src/quant.cpp:57-86 computes the
// same thing by renormalising subnormals bit by bit).
float float_from_half(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t frac = h & 0x3ffu;
    uint32_t bits;
    if (e == 31) {
        bits = 0x7f800000u | (frac << 13);  // Inf / NaN, payload kept
    } else if (e == 0) {
        // zero or subnormal: frac * 2^-24, exact in f32
        const float mag = static_cast<float>(frac) * 5.9604644775390625e-08f;
        std::memcpy(&bits, &mag, sizeof bits);
    } else {
        bits = ((e + 112u) << 23) | (frac << 13);
    }
    bits |= sign;
    float out;
    std::memcpy(&out, &bits, sizeof out);
    return out;
}

// std::round on float: half away from zero (roundf), then the int cast the
// reference applies.  Inputs here are bounded by the clamps that follow.
inline int round_to_int(float v) { return static_cast<int>(std::round(v)); }

// --- quantizers -------------------------------------------------------------
// Each walks `rows` rows of `row_len` floats and emits ceil(row_len/32) blocks
// per row; the last block of a row may be partial ("tail").

// src/quant.cpp:112-170.  d = fp16(max|v| / 127); q = clamp(round(v / d), +-127)
// using the *stored* d; tail slots hold q = 0; an all-zero block has d = 0.
void quantize_q8_0_rows(const float* src, int rows, int row_len, Q8Block* out) {
    const int nb = (row_len + kQK - 1) / kQK;
    for (int r = 0; r < rows; ++r) {
        const float* row = src + static_cast<size_t>(r) * row_len;
        for (int b = 0; b < nb; ++b) {
            const int k0 = b * kQK;
            const int len = std::min(kQK, row_len - k0);
            Q8Block blk;
            std::memset(&blk, 0, sizeof blk);
            float amax = 0.0f;
            for (int i = 0; i < len; ++i) {
                const float a = std::fabs(row[k0 + i]);
                if (a > amax) amax = a;
            }
            if (amax > 0.0f) {
                blk.d = half_from_float(amax / 127.0f);
                const float dq = float_from_half(blk.d);
                const float inv = (dq == 0.0f) ? 0.0f : 1.0f / dq;
                for (int i = 0; i < len; ++i) {
                    const int q = round_to_int(row[k0 + i] * inv);
                    blk.q[i] = static_cast<int8_t>(std::max(-127, std::min(127, q)));
                }
            }
            out[static_cast<size_t>(r) * nb + b] = blk;
        }
    }
}

// src/quant.cpp:207-270.  d = fp16(max|v| / 7) (symmetric, not ggml's signed
// max / -8); q = clamp(round(v / d + 8), 0, 15); byte j packs element j in the
// low nibble and element j+16 in the high nibble; missing tail elements act as
// v = 0 (nibble 8); an all-zero block is d = 0 with zero bytes.
void quantize_q4_0_rows(const float* src, int rows, int row_len, Q40Block* out) {
    const int nb = (row_len + kQK - 1) / kQK;
    for (int r = 0; r < rows; ++r) {
        const float* row = src + static_cast<size_t>(r) * row_len;
        for (int b = 0; b < nb; ++b) {
            const int k0 = b * kQK;
            const int len = std::min(kQK, row_len - k0);
            Q40Block blk;
            std::memset(&blk, 0, sizeof blk);
            float amax = 0.0f;
            for (int i = 0; i < len; ++i) {
                const float a = std::fabs(row[k0 + i]);
                if (a > amax) amax = a;
            }
            if (amax > 0.0f) {
                blk.d = half_from_float(amax / 7.0f);
                const float dq = float_from_half(blk.d);
                const float inv = (dq == 0.0f) ? 0.0f : 1.0f / dq;
                for (int j = 0; j < 16; ++j) {
                    const float lo = (j < len) ? row[k0 + j] * inv : 0.0f;
                    const float hi = (j + 16 < len) ? row[k0 + j + 16] * inv : 0.0f;
                    const int qlo = std::max(0, std::min(15, round_to_int(lo + 8.0f)));
                    const int qhi = std::max(0, std::min(15, round_to_int(hi + 8.0f)));
                    blk.q[j] = static_cast<uint8_t>(qlo | (qhi << 4));
                }
            }
            out[static_cast<size_t>(r) * nb + b] = blk;
        }
    }
}

// tests/test_cuda_quant.cpp:129-180 (the product has no Q4_1 quantizer; this
// test-local routine is the one the reference's Q4_1 parity tests use).
// d = fp16((max - min) / 15), m = fp16(min), q = clamp(round((v - m) / d), 0, 15)
// with the stored d and m; tail nibbles are 0; a constant block has d = 0 and
// m = fp16(min).
void quantize_q4_1_rows(const float* src, int rows, int row_len, Q41Block* out) {
    const int nb = (row_len + kQK - 1) / kQK;
    for (int r = 0; r < rows; ++r) {
        const float* row = src + static_cast<size_t>(r) * row_len;
        for (int b = 0; b < nb; ++b) {
            const int k0 = b * kQK;
            const int len = std::min(kQK, row_len - k0);
            float lo = INFINITY;
            float hi = -INFINITY;
            for (int i = 0; i < len; ++i) {
                lo = std::min(lo, row[k0 + i]);
                hi = std::max(hi, row[k0 + i]);
            }
            Q41Block blk;
            std::memset(&blk, 0, sizeof blk);
            const float range = hi - lo;
            if (range > 0.0f) {
                blk.d = half_from_float(range / 15.0f);
                blk.m = half_from_float(lo);
                const float dq = float_from_half(blk.d);
                const float mq = float_from_half(blk.m);
                const float inv = (dq == 0.0f) ? 0.0f : 1.0f / dq;
                for (int j = 0; j < 16; ++j) {
                    int q0 = 0, q1 = 0;
                    if (j < len) q0 = round_to_int((row[k0 + j] - mq) * inv);
                    if (j + 16 < len) q1 = round_to_int((row[k0 + j + 16] - mq) * inv);
                    q0 = std::max(0, std::min(15, q0));
                    q1 = std::max(0, std::min(15, q1));
                    blk.q[j] = static_cast<uint8_t>(q0 | (q1 << 4));
                }
            } else {
                blk.m = half_from_float(lo == INFINITY ? 0.0f : lo);
            }
            out[static_cast<size_t>(r) * nb + b] = blk;
        }
    }
}

// --- per-element dequant (src/quant.cpp:435-461) ----------------------------
// The scale is decoded per element, exactly as the reference does; d*q is
// exact in f32, the Q4_1 "+ m" rounds once.
inline float elem_q8_0(const Q8Block& b, int i) {
    return float_from_half(b.d) * static_cast<float>(b.q[i]);
}
inline int nibble(const uint8_t* q, int i) {
    return i < 16 ? (q[i] & 0x0f) : (q[i - 16] >> 4);
}
inline float elem_q4_0(const Q40Block& b, int i) {
    return float_from_half(b.d) * static_cast<float>(nibble(b.q, i) - 8);
}
inline float elem_q4_1(const Q41Block& b, int i) {
    const float prod = float_from_half(b.d) * static_cast<float>(nibble(b.q, i));
    return prod + float_from_half(b.m);
}

// --- parallel_for (src/thread_pool.cpp:23-73) --------------------------------
// n items in n_threads contiguous chunks (the first n % n_threads chunks get one
// extra item); runs inline when n < 16 * n_threads; threads are created and
// joined per call; the first exception thrown by a worker is rethrown.
int resolve_threads(int requested) {
    if (requested > 0) return requested;
    const unsigned hw = std::thread::hardware_concurrency();
    return hw > 0 ? static_cast<int>(hw) : 4;
}

void parallel_for(int n, int requested_threads, const std::function<void(int, int)>& body) {
    if (n <= 0) return;
    int nt = resolve_threads(requested_threads);
    if (n < nt * 16) {
        body(0, n);
        return;
    }
    nt = std::min(nt, n);
    const int base = n / nt;
    const int extra = n % nt;
    std::vector<std::thread> pool;
    pool.reserve(nt);
    std::exception_ptr first;
    std::mutex first_lock;
    int begin = 0;
    for (int t = 0; t < nt; ++t) {
        const int end = begin + base + (t < extra ? 1 : 0);
        if (end > begin) {
            pool.emplace_back([begin, end, &body, &first, &first_lock] {
                try {
                    body(begin, end);
                } catch (...) {
                    std::lock_guard<std::mutex> g(first_lock);
                    if (!first) first = std::current_exception();
                }
            });
        }
        begin = end;
    }
    for (auto& th : pool) th.join();
    if (first) std::rethrow_exception(first);
}

// --- scalar quantized linear (src/quant.cpp:367-433) --------------------------
// y[r, j] = sum_b sum_k elem(W[j, b], k) * x[r, 32 b + k], one f32 multiply and
// one f32 add per element in ascending k, work item = (r, j) flattened row-major.
template <typename Block, float (*Elem)(const Block&, int)>
void linear_rows(const float* x, int rows, int K, const Block* w, int M, float* y, int threads) {
    const int nb = (K + kQK - 1) / kQK;
    parallel_for(rows * M, threads, [&](int begin, int end) {
        for (int item = begin; item < end; ++item) {
            const int r = item / M;
            const int j = item % M;
            const float* xr = x + static_cast<size_t>(r) * K;
            const Block* wr = w + static_cast<size_t>(j) * nb;
            float acc = 0.0f;
            for (int b = 0; b < nb; ++b) {
                const int k0 = b * kQK;
                const int k1 = std::min(k0 + kQK, K);
                for (int k = k0; k < k1; ++k) {
                    const float prod = Elem(wr[b], k - k0) * xr[k];
                    acc = acc + prod;
                }
            }
            y[static_cast<size_t>(r) * M + j] = acc;
        }
    });
}

void set_error(char* err, size_t len, const std::string& msg) {
    if (err != nullptr && len > 0) {
        std::snprintf(err, len, "%s", msg.c_str());
    }
}

}  // namespace

extern "C" {

size_t mlq_oracle_block_bytes(int qtype) {
    switch (qtype) {
        case kQ8_0: return sizeof(Q8Block);
        case kQ4_0: return sizeof(Q40Block);
        case kQ4_1: return sizeof(Q41Block);
        default: return 0;
    }
}

uint16_t mlq_oracle_fp16_from_f32(float v) { return half_from_float(v); }
float mlq_oracle_f32_from_fp16(uint16_t h) { return float_from_half(h); }

void mlq_oracle_fp16_from_f32_n(const float* v, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = half_from_float(v[i]);
}
void mlq_oracle_f32_from_fp16_n(const uint16_t* h, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = float_from_half(h[i]);
}

// Quantize `rows` x `row_len` floats; returns the number of blocks written
// (rows * ceil(row_len / 32)) or -1 for a bad type / size.  Rows are split over
// `threads` workers; each row is independent so the bytes do not depend on it.
long long mlq_oracle_quantize(int qtype, const float* src, int rows, int row_len, void* out, int threads) {
    if (rows <= 0 || row_len <= 0) return -1;
    const int nb = (row_len + kQK - 1) / kQK;
    auto run = [&](int r0, int r1) {
        const float* s = src + static_cast<size_t>(r0) * row_len;
        const size_t off = static_cast<size_t>(r0) * nb;
        switch (qtype) {
            case kQ8_0: quantize_q8_0_rows(s, r1 - r0, row_len, static_cast<Q8Block*>(out) + off); break;
            case kQ4_0: quantize_q4_0_rows(s, r1 - r0, row_len, static_cast<Q40Block*>(out) + off); break;
            case kQ4_1: quantize_q4_1_rows(s, r1 - r0, row_len, static_cast<Q41Block*>(out) + off); break;
            default: break;
        }
    };
    if (qtype != kQ8_0 && qtype != kQ4_0 && qtype != kQ4_1) return -1;
    parallel_for(rows, threads <= 0 ? 1 : threads, run);
    return static_cast<long long>(rows) * nb;
}

// Dequantize to f32 (src/quant.cpp:172-202, 272-312, 317-358).
int mlq_oracle_dequantize(int qtype, const void* blocks, int rows, int row_len, float* dst) {
    if (rows <= 0 || row_len <= 0) return -1;
    const int nb = (row_len + kQK - 1) / kQK;
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < row_len; ++k) {
            const size_t bi = static_cast<size_t>(r) * nb + k / kQK;
            float v;
            switch (qtype) {
                case kQ8_0: v = elem_q8_0(static_cast<const Q8Block*>(blocks)[bi], k % kQK); break;
                case kQ4_0: v = elem_q4_0(static_cast<const Q40Block*>(blocks)[bi], k % kQK); break;
                case kQ4_1: v = elem_q4_1(static_cast<const Q41Block*>(blocks)[bi], k % kQK); break;
                default: return -1;
            }
            dst[static_cast<size_t>(r) * row_len + k] = v;
        }
    }
    return 0;
}

// The reference CPU quant linear: x [rows, K] f32, W = M*ceil(K/32) blocks,
// y [rows, M] f32.  Validation mirrors src/quant.cpp:374-408.  Returns 0, or -1
// with a message in err.
int mlq_oracle_linear(int qtype, const float* x, int rows, int K, const void* blocks,
                      size_t n_blocks, int M, float* y, int threads, char* err, size_t err_len) {
    try {
        if (rows <= 0 || K <= 0 || M <= 0) {
            throw std::runtime_error("linear_quantized: empty tensors are not supported");
        }
        const int nb = (K + kQK - 1) / kQK;
        const size_t expected = static_cast<size_t>(M) * nb;
        if (n_blocks != expected) {
            throw std::runtime_error("linear_quantized: block count mismatch: expected " +
                                     std::to_string(expected) + ", got " + std::to_string(n_blocks));
        }
        switch (qtype) {
            case kQ8_0:
                linear_rows<Q8Block, elem_q8_0>(x, rows, K, static_cast<const Q8Block*>(blocks), M, y, threads);
                break;
            case kQ4_0:
                linear_rows<Q40Block, elem_q4_0>(x, rows, K, static_cast<const Q40Block*>(blocks), M, y, threads);
                break;
            case kQ4_1:
                linear_rows<Q41Block, elem_q4_1>(x, rows, K, static_cast<const Q41Block*>(blocks), M, y, threads);
                break;
            default:
                throw std::runtime_error("linear: unknown quant type");
        }
        return 0;
    } catch (const std::exception& e) {
        set_error(err, err_len, e.what());
        return -1;
    }
}

// First index of the maximum; ties keep the lowest index (src/ops.cpp:179-192).
int mlq_oracle_argmax(const float* v, size_t n) {
    if (n == 0) return -1;
    size_t best = 0;
    for (size_t i = 1; i < n; ++i) {
        if (v[i] > v[best]) best = i;
    }
    return static_cast<int>(best);
}

int mlq_oracle_hardware_threads(void) { return resolve_threads(0); }

}  // extern "C"
