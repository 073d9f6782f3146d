// The C ABI (include/llm_engine_amd.h): argument checks, kernel choice and
// the library-owned scratch. Replaces the host half of
// /root/reference/src/cuda_matmul.cu (matmul_impl :399-448, Scratch
// :268-297, DeviceTensor/DeviceQTensor memory :452-525, entry points
// :527-574).
//
// Every argument is checked on the host before any HIP call, so each error
// path can be exercised without a GPU. Errors come back as status codes with
// a message for em_last_error(); the messages name both shapes as
// "(A is MxK, B is KxN)", as the reference's exceptions do.
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "internal.hpp"
#include "llm_engine_amd.h"

namespace em {

std::string shapes(std::size_t m, std::size_t n, std::size_t k) {
    return "(A is " + std::to_string(m) + "x" + std::to_string(k) + ", B is " + std::to_string(k) +
           "x" + std::to_string(n) + ")";
}

namespace {

thread_local std::string g_error;

std::mutex g_scratch_mu;
float* g_scratch[kSlots] = {};
std::size_t g_scratch_cap[kSlots] = {};
std::atomic<std::size_t> g_generation{0};


// a * b >= 2^31, without overflow: the kernels index with int
// (cuda_matmul.cu:414-417).
bool too_many(std::size_t a, std::size_t b) {
    constexpr std::size_t kLimit = (std::size_t{1} << 31) - 1;
    return a != 0 && b > kLimit / a;
}


// Strip copies of registered int8 weights (em_q8_register): the row-major
// buffer's address -> its shape and a copy in the strip layout.
struct StripCopy {
    std::size_t k, n;
    int8_t* packed;
};
std::mutex g_strip_mu;
std::unordered_map<const void*, StripCopy>& strip_copies() {
    static std::unordered_map<const void*, StripCopy> m;
    return m;
}

// The strip copy of B if one is registered for this shape, else null. The
// caller holds g_strip_mu.
const int8_t* strip_copy_locked(const void* B, std::size_t k, std::size_t n) {
    const auto it = strip_copies().find(B);
    if (it == strip_copies().end() || it->second.k != k || it->second.n != n) return nullptr;
    return it->second.packed;
}

const int8_t* strip_copy_of(const void* B, std::size_t k, std::size_t n) {
    std::lock_guard<std::mutex> lock(g_strip_mu);
    return strip_copy_locked(B, k, n);
}

// launch(P) with B's strip copy P, if one is registered for this shape; the
// registry stays locked until launch returns, so no em_q8_unregister or
// em_free on another thread can free P between the lookup and the launch
// (they wait for the device before freeing, so the queued kernel finishes
// first). False, nothing launched, without a copy.
template <class Launch>
bool with_strip_copy(const void* B, std::size_t k, std::size_t n, Launch launch) {
    std::lock_guard<std::mutex> lock(g_strip_mu);
    const int8_t* P = strip_copy_locked(B, k, n);
    if (!P) return false;
    launch(P);
    return true;
}

// Frees every strip copy registered for a buffer that starts inside
// [base, base + bytes). The caller holds g_strip_mu.
void drop_copies_locked(const char* base, std::size_t bytes) {
    auto& map = strip_copies();
    bool synced = false;
    for (auto it = map.begin(); it != map.end();) {
        const char* key = static_cast<const char*>(it->first);
        if (key >= base && key < base + bytes) {
            if (!synced) {
                (void)hipDeviceSynchronize();  // a queued product may still read the copy
                synced = true;
            }
            (void)hipFree(it->second.packed);
            it = map.erase(it);
        } else {
            ++it;
        }
    }
}

// One-row products over registered weights run the strip-layout GEMV: one
// launch and no split-K partials. Up to 8192 rows of B it beat the
// row-major split-K call at every width measured (4096^2: 4.6 against 6.5
// us; 4096 x 11008: 9.1 against 11.8; 4096 x 32000: 21.8 against 25.4),
// and without a norm up to 12288 rows when B has at least 4096 columns
// (one pass of gemv_row_kernel at 512 threads, one workgroup per strip:
// 11008 x 4096 10.6 against 11.9, 12288 x 4096 10.9 against 12.2; with 64
// strips, 11008 x 1024, 7.5 against 7.0). Deeper, the strip kernel loops
// over batches and lost (11008 rows before the one-pass kernel: 13.7
// against 11.6); from two rows the GEMV's multiply-adds per byte grow with
// m and the row-major kernels win.
bool strip_row_takes(std::size_t k, std::size_t n, bool norm) {
    return k <= 8192 || (!norm && k <= 12288 && n >= 4096);
}

// Decode batches (2 .. 16 rows) over registered weights: decode_mfma.hip.
// EM_DECODE_MFMA=0 keeps them on the row-major kernels.
bool decode_mfma_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("EM_DECODE_MFMA");
        return !(v && v[0] == '0');
    }();
    return on;
}

}  // namespace

const int8_t* registered_strip(const void* B, std::size_t k, std::size_t n) {
    return strip_copy_of(B, k, n);
}

// The matmul entry points. `workspace` (em_matmul_q8_noalloc, with the
// skinny kernel): called once the shape is valid and a GPU is present, it
// returns the caller's buffer for split-K partials and its size in floats;
// the product then allocates nothing, and a shape whose partials do not fit
// is rejected before any launch.
template <class BT>
int matmul_entry(std::size_t m, std::size_t n, std::size_t k, const float* A, const BT* B,
                 const float* scale, float* C, int kernel, int accumulate,
                 const float* rms_weight, void* stream, Workspace workspace) {
    if (kernel < EM_KERNEL_AUTOMATIC || kernel > EM_KERNEL_SKINNY)
        return fail(EM_EINVAL, "matmul_cuda: unknown kernel " + std::to_string(kernel));
    // automatic: skinny up to 8 rows, as the reference (cuda_matmul.cu:406-410).
    // Above that, the B-streaming fp32 MFMA kernel (tiled_split), except
    // where tiled_preferred picks the LDS-tiled GEMM (large m, small B, or
    // wide B from 256 rows): the reference switches to tiled past 64 rows.
    // int8 B goes to the exact-split bf16 MFMA
    // kernel instead (split_bf16.hip: at 4096^2, 1.1x faster than
    // tiled_split at m = 9-16 and 1.3-2.6x from m = 32 to 512), and so do
    // int8 products of fewer rows where it beats the GEMV
    // (split_bf16_preferred). fp32 B of 2^25 values or more takes tiled_split
    // from 4 rows (4096 x 11008: 35.9 against 38.4 us at m = 4, 36.5
    // against 41.8 at m = 8; at 4096^2 the GEMV stays ahead, 18.1 against
    // 19.2 at m = 8). tiled takes what B's width or alignment rules out.
    const bool automatic = kernel == EM_KERNEL_AUTOMATIC;
    if (automatic) kernel = m <= 8 ? EM_KERNEL_SKINNY : EM_KERNEL_TILED_SPLIT;
    if (kernel == EM_KERNEL_SKINNY && m > 8)
        return fail(EM_EINVAL,
                    "matmul_cuda: skinny kernel takes at most 8 rows " + shapes(m, n, k));
    if (too_many(m, k) || too_many(k, n) || too_many(m, n))
        return fail(EM_EINVAL, "matmul_cuda: more than 2^31 elements " + shapes(m, n, k));
    if (m == 0 || n == 0) return EM_OK;
    if (!C) return fail(EM_EINVAL, "matmul_cuda: C is null " + shapes(m, n, k));
    if (k && (!A || !B))
        return fail(EM_EINVAL, "matmul_cuda: A or B is null " + shapes(m, n, k));
    if (std::is_same<BT, int8_t>::value && k && !scale)
        return fail(EM_EINVAL, "matmul_cuda: int8 B needs its column scales " + shapes(m, n, k));
    if (!device_present()) return fail(EM_ENODEV, "matmul_cuda: no usable GPU");
    float* ws = nullptr;
    std::size_t ws_floats = 0;
    if (workspace) {
        ws = workspace(&ws_floats);
        if (!ws) return EM_EDEVICE;  // workspace() set the message
    }

    hipStream_t s = static_cast<hipStream_t>(stream);
    try {
        if (k == 0) {
            if (!accumulate) run_fill_zero(C, m * n, s);
            hip_check(hipGetLastError(), "launch");
            return EM_OK;
        }
        MatmulArgs a{};
        a.m = static_cast<int>(m);
        a.n = static_cast<int>(n);
        a.k = static_cast<int>(k);
        a.A = A;
        a.B = B;
        a.scale = scale;
        a.C = C;
        a.accumulate = accumulate != 0;
        a.rms_weight = rms_weight;
        a.stream = s;
        if (std::is_same<BT, int8_t>::value && kernel == EM_KERNEL_SKINNY && m == 1 &&
            strip_row_takes(k, n, rms_weight != nullptr)) {
            if (with_strip_copy(B, k, n, [&](const int8_t* P) { run_gemv_packed(a, P); })) {
                hip_check(hipGetLastError(), "launch");
                return EM_OK;
            }
        }
        if (std::is_same<BT, int8_t>::value && automatic && m >= 2 && decode_mfma_enabled() &&
            decode_mfma_supported(a)) {
            if (with_strip_copy(B, k, n, [&](const int8_t* P) { run_decode_mfma(a, P); })) {
                hip_check(hipGetLastError(), "launch");
                return EM_OK;
            }
        }
        if (std::is_same<BT, int8_t>::value && automatic && strip_split_supported(a) &&
            strip_split_preferred(a.m, a.n, a.k)) {
            if (with_strip_copy(B, k, n, [&](const int8_t* P) { run_strip_split(a, P); })) {
                hip_check(hipGetLastError(), "launch");
                return EM_OK;
            }
        }
        if (std::is_same<BT, int8_t>::value && automatic && split_bf16_preferred(a.m, a.n, a.k) &&
            split_bf16_supports(a)) {
            run_split_bf16(a);  // fuses the norm
            hip_check(hipGetLastError(), "launch");
            return EM_OK;
        }
        if (!std::is_same<BT, int8_t>::value && automatic && m >= 4 &&
            static_cast<long long>(n) * static_cast<long long>(k) >= (1LL << 25) &&
            tiled_split_supports<BT>(a))
            kernel = EM_KERNEL_TILED_SPLIT;
        if (!std::is_same<BT, int8_t>::value && automatic && tiled_preferred(a))
            kernel = EM_KERNEL_TILED;
        if (rms_weight && kernel != EM_KERNEL_SKINNY) {
            float* normed = scratch(kNorm, m * k);
            run_rmsnorm_rows(a.m, a.k, A, rms_weight, normed, s);
            a.A = normed;
            a.rms_weight = nullptr;
        }
        switch (kernel) {
            case EM_KERNEL_NAIVE: run_naive<BT>(a); break;
            case EM_KERNEL_TILED: run_tiled<BT>(a); break;
            case EM_KERNEL_TILED_SPLIT:
                if (tiled_split_supports<BT>(a)) {
                    run_tiled_split<BT>(a);
                } else {
                    run_tiled<BT>(a);
                }
                break;
            default:
                if (ws) {
                    const std::size_t need = skinny_partial_floats<BT>(a);
                    if (need > ws_floats)
                        return fail(EM_EINVAL, "matmul_q8_noalloc: split-K partials need " +
                                                   std::to_string(need * sizeof(float)) +
                                                   " bytes, more than the static scratch's " +
                                                   std::to_string(ws_floats * sizeof(float)) +
                                                   " " + shapes(m, n, k));
                    a.partials = ws;
                }
                run_skinny<BT>(a);
                break;
        }
        hip_check(hipGetLastError(), "launch");
    } catch (const DeviceError& e) {
        return fail(EM_EDEVICE, e.what());
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, std::string("hip: ") + e.what());
    }
    return EM_OK;
}

template int matmul_entry<float>(std::size_t, std::size_t, std::size_t, const float*,
                                 const float*, const float*, float*, int, int, const float*,
                                 void*, Workspace);
template int matmul_entry<int8_t>(std::size_t, std::size_t, std::size_t, const float*,
                                  const int8_t*, const float*, float*, int, int, const float*,
                                  void*, Workspace);

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

bool device_present() {
    int count = 0;
    return hipGetDeviceCount(&count) == hipSuccess && count > 0;
}

float* scratch(ScratchSlot slot, std::size_t floats) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (floats > g_scratch_cap[slot]) {
        // Queued kernels may still read the old buffer.
        hip_check(hipDeviceSynchronize(), "synchronize before scratch growth");
        if (g_scratch[slot]) hip_check(hipFree(g_scratch[slot]), "free scratch");
        g_scratch[slot] = nullptr;
        g_scratch_cap[slot] = 0;
        void* p = nullptr;
        hip_check(hipMalloc(&p, floats * sizeof(float)), "alloc scratch");
        g_scratch[slot] = static_cast<float*>(p);
        g_scratch_cap[slot] = floats;
        g_generation.fetch_add(1);
    }
    return g_scratch[slot];
}

std::size_t scratch_generation() { return g_generation.load(); }

unsigned* tile_counters(std::size_t count) {
    static unsigned* words = nullptr;
    static std::size_t cap = 0;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (count > cap) {
        hip_check(hipDeviceSynchronize(), "synchronize before counter growth");
        if (words) hip_check(hipFree(words), "free tile counters");
        words = nullptr;
        cap = 0;
        void* p = nullptr;
        hip_check(hipMalloc(&p, count * sizeof(unsigned)), "alloc tile counters");
        hip_check(hipMemset(p, 0, count * sizeof(unsigned)), "clear tile counters");
        hip_check(hipDeviceSynchronize(), "clear tile counters");
        words = static_cast<unsigned*>(p);
        cap = count;
        g_generation.fetch_add(1);
    }
    return words;
}


int cu_count() {
    static const int cus = [] {
        int device = 0, n = 0;
        if (hipGetDevice(&device) != hipSuccess) return 256;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
            return 256;
        return n > 0 ? n : 256;
    }();
    return cus;
}

}  // namespace em

using em::fail;
using em::too_many;

extern "C" {

const char* em_last_error(void) { return em::g_error.c_str(); }

int em_available(void) { return em::device_present() ? 1 : 0; }

int em_synchronize(void) {
    if (!em::device_present()) return fail(EM_ENODEV, "synchronize: no usable GPU");
    const hipError_t err = hipDeviceSynchronize();
    if (err != hipSuccess)
        return fail(EM_EDEVICE, std::string("hip: synchronize: ") + hipGetErrorString(err));
    return EM_OK;
}

size_t em_scratch_generation(void) { return em::scratch_generation(); }

int em_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(EM_EINVAL, "em_malloc: null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return EM_OK;
    if (!em::device_present()) return fail(EM_ENODEV, "alloc: no usable GPU");
    const hipError_t err = hipMalloc(ptr, bytes);
    if (err != hipSuccess) {
        *ptr = nullptr;
        return fail(EM_EDEVICE, std::string("hip: alloc: ") + hipGetErrorString(err));
    }
    return EM_OK;
}

int em_free(void* ptr) {
    if (!ptr) return EM_OK;
    {
        // Strip copies registered for B inside this allocation go with it:
        // a later allocation at the same address must not find them.
        std::lock_guard<std::mutex> lock(em::g_strip_mu);
        if (!em::strip_copies().empty()) {
            void* base = nullptr;
            size_t bytes = 0;
            if (hipMemGetAddressRange(&base, &bytes, ptr) != hipSuccess || !base) {
                base = ptr;
                bytes = 1;
            }
            em::drop_copies_locked(static_cast<const char*>(base), bytes);
        }
    }
    const hipError_t err = hipFree(ptr);
    if (err != hipSuccess)
        return fail(EM_EDEVICE, std::string("hip: free: ") + hipGetErrorString(err));
    return EM_OK;
}

// Synchronous copies, ordered after the calling thread's default-stream work
// (the stream the C++ layer queues products on), as cudaMemcpy is in the
// reference's upload() / download().
static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* what) {
    if (bytes == 0) return EM_OK;
    if (!dst || !src) return fail(EM_EINVAL, std::string(what) + ": null pointer");
    if (!em::device_present()) return fail(EM_ENODEV, std::string(what) + ": no usable GPU");
    hipError_t err = hipMemcpyAsync(dst, src, bytes, kind, hipStreamPerThread);
    if (err == hipSuccess) err = hipStreamSynchronize(hipStreamPerThread);
    if (err != hipSuccess)
        return fail(EM_EDEVICE, std::string("hip: ") + what + ": " + hipGetErrorString(err));
    return EM_OK;
}

int em_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    return copy(dst, src, bytes, hipMemcpyHostToDevice, "upload");
}

int em_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, "download");
}

int em_matmul_f32(size_t m, size_t n, size_t k, const float* A, const float* B, float* C,
                  int kernel, int accumulate, const float* rms_weight, void* stream) {
    return em::matmul_entry<float>(m, n, k, A, B, nullptr, C, kernel, accumulate, rms_weight,
                                   stream);
}

int em_matmul_q8(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
                 const float* scale, float* C, int kernel, int accumulate,
                 const float* rms_weight, void* stream) {
    return em::matmul_entry<int8_t>(m, n, k, A, B, scale, C, kernel, accumulate, rms_weight,
                                    stream);
}

int em_quantize_q8(size_t rows, size_t cols, const float* B, int8_t* q, float* scale,
                   void* stream) {
    if (em::too_many(rows, cols))
        return fail(EM_EINVAL, "quantize_q8: more than 2^31 elements (B is " +
                                   std::to_string(rows) + "x" + std::to_string(cols) + ")");
    if (cols == 0) return EM_OK;
    if (!scale || (rows && (!B || !q))) return fail(EM_EINVAL, "quantize_q8: null pointer");
    if (!em::device_present()) return fail(EM_ENODEV, "quantize_q8: no usable GPU");
    try {
        em::run_quantize_q8(static_cast<int>(rows), static_cast<int>(cols), B, q, scale,
                            static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_dequantize_q8(size_t rows, size_t cols, const int8_t* q, const float* scale, float* out,
                     void* stream) {
    if (em::too_many(rows, cols)) return fail(EM_EINVAL, "dequantize: more than 2^31 elements");
    if (rows == 0 || cols == 0) return EM_OK;
    if (!q || !scale || !out) return fail(EM_EINVAL, "dequantize: null pointer");
    if (!em::device_present()) return fail(EM_ENODEV, "dequantize: no usable GPU");
    try {
        em::run_dequantize_q8(static_cast<int>(rows), static_cast<int>(cols), q, scale, out,
                              static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}


int em_pack_q8(size_t k, size_t n, const int8_t* B, int8_t* packed, void* stream) {
    if (too_many(k, n)) return fail(EM_EINVAL, "pack_q8: more than 2^31 elements");
    if (n % 16 || k % 4)
        return fail(EM_EINVAL, "pack_q8: n must be a multiple of 16 and k of 4 (B is " +
                                   std::to_string(k) + "x" + std::to_string(n) + ")");
    if (k == 0 || n == 0) return EM_OK;
    if (!B || !packed) return fail(EM_EINVAL, "pack_q8: null pointer");
    if (reinterpret_cast<uintptr_t>(B) % 16 || reinterpret_cast<uintptr_t>(packed) % 16)
        return fail(EM_EINVAL, "pack_q8: B and packed must be 16-byte aligned");
    if (!em::device_present()) return fail(EM_ENODEV, "pack_q8: no usable GPU");
    try {
        em::run_pack_strips(static_cast<int>(k), static_cast<int>(n), B, packed,
                            static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_q8_register(const int8_t* B, size_t k, size_t n, void* stream) {
    if (too_many(k, n)) return fail(EM_EINVAL, "q8_register: more than 2^31 elements");
    if (k == 0 || n == 0) return EM_OK;
    if (!B) return fail(EM_EINVAL, "q8_register: null pointer");
    static const bool enabled = [] {
        const char* v = std::getenv("EM_STRIP_COPY");
        return !(v && v[0] == '0');
    }();
    // Shapes the strip layout cannot hold are left row-major.
    if (!enabled || n % 16 || k % 4 || reinterpret_cast<uintptr_t>(B) % 16) return EM_OK;
    if (!em::device_present()) return fail(EM_ENODEV, "q8_register: no usable GPU");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    try {
        std::lock_guard<std::mutex> lock(em::g_strip_mu);
        auto& map = em::strip_copies();
        auto it = map.find(B);
        if (it != map.end() && (it->second.k != k || it->second.n != n)) {
            em::hip_check(hipFree(it->second.packed), "free strip copy");
            map.erase(it);
            it = map.end();
        }
        if (it == map.end()) {
            void* p = nullptr;
            em::hip_check(hipMalloc(&p, k * n), "alloc strip copy");
            it = map.emplace(B, em::StripCopy{k, n, static_cast<int8_t*>(p)}).first;
        }
        // Packed (again) from B's current bytes; load-time work, so the
        // stream is drained before the copy is used on any other stream.
        em::run_pack_strips(static_cast<int>(k), static_cast<int>(n), B, it->second.packed, s);
        em::hip_check(hipGetLastError(), "launch");
        em::hip_check(hipStreamSynchronize(s), "pack strip copy");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_q8_unregister(const int8_t* B) {
    std::lock_guard<std::mutex> lock(em::g_strip_mu);
    auto& map = em::strip_copies();
    const auto it = map.find(B);
    if (it == map.end()) return EM_OK;
    hipError_t err = hipDeviceSynchronize();  // a queued product may still read the copy
    const hipError_t err2 = hipFree(it->second.packed);
    if (err == hipSuccess) err = err2;
    map.erase(it);
    if (err != hipSuccess)
        return fail(EM_EDEVICE, std::string("hip: free strip copy: ") + hipGetErrorString(err));
    return EM_OK;
}

int em_q8_registered(const int8_t* B, size_t k, size_t n) {
    return em::strip_copy_of(B, k, n) ? 1 : 0;
}

int em_unpack_q8(size_t k, size_t n, const int8_t* packed, int8_t* B, void* stream) {
    if (too_many(k, n)) return fail(EM_EINVAL, "unpack_q8: more than 2^31 elements");
    if (n % 16 || k % 4)
        return fail(EM_EINVAL, "unpack_q8: n must be a multiple of 16 and k of 4");
    if (k == 0 || n == 0) return EM_OK;
    if (!B || !packed) return fail(EM_EINVAL, "unpack_q8: null pointer");
    if (reinterpret_cast<uintptr_t>(B) % 16 || reinterpret_cast<uintptr_t>(packed) % 16)
        return fail(EM_EINVAL, "unpack_q8: B and packed must be 16-byte aligned");
    if (!em::device_present()) return fail(EM_ENODEV, "unpack_q8: no usable GPU");
    try {
        em::run_unpack_strips(static_cast<int>(k), static_cast<int>(n), packed, B,
                              static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_matmul_q8_packed(size_t m, size_t n, size_t k, const float* A, const int8_t* packed,
                        const float* scale, float* C, int accumulate, const float* rms_weight,
                        void* stream) {
    if (m > 16)
        return fail(EM_EINVAL, "matmul_q8_packed: the strip layout takes at most 16 rows " +
                                   em::shapes(m, n, k));
    if (too_many(m, k) || too_many(k, n) || too_many(m, n))
        return fail(EM_EINVAL, "matmul_q8_packed: more than 2^31 elements " + em::shapes(m, n, k));
    if (n % 16 || k % 4)
        return fail(EM_EINVAL, "matmul_q8_packed: n must be a multiple of 16 and k of 4 " +
                                   em::shapes(m, n, k));
    if (m == 0 || n == 0) return EM_OK;
    if (!C) return fail(EM_EINVAL, "matmul_q8_packed: C is null " + em::shapes(m, n, k));
    if (k && (!A || !packed || !scale))
        return fail(EM_EINVAL, "matmul_q8_packed: A, B or scale is null " + em::shapes(m, n, k));
    if (k && reinterpret_cast<uintptr_t>(packed) % 16)
        return fail(EM_EINVAL, "matmul_q8_packed: packed B must be 16-byte aligned");
    auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (m > 8 && k && (!a16(A) || !a16(C) || !a16(scale) || (rms_weight && !a16(rms_weight))))
        return fail(EM_EINVAL, "matmul_q8_packed: 9 to 16 rows need A, C, the scales and the "
                               "norm weight 16-byte aligned " + em::shapes(m, n, k));
    if (m > 8 && n > (size_t{1} << 18))
        return fail(EM_EINVAL, "matmul_q8_packed: 9 to 16 rows take at most 2^18 columns " +
                                   em::shapes(m, n, k));
    if (!em::device_present()) return fail(EM_ENODEV, "matmul_q8_packed: no usable GPU");
    hipStream_t s = static_cast<hipStream_t>(stream);
    try {
        if (k == 0) {
            if (!accumulate) em::run_fill_zero(C, m * n, s);
        } else {
            em::MatmulArgs a{};
            a.m = static_cast<int>(m);
            a.n = static_cast<int>(n);
            a.k = static_cast<int>(k);
            a.A = A;
            a.B = packed;
            a.scale = scale;
            a.C = C;
            a.accumulate = accumulate != 0;
            a.rms_weight = rms_weight;
            a.stream = s;
            if (m > 8) {
                em::run_strip_split(a, packed);  // strip_split_supported holds: checked above
            } else if (m >= 2 && em::decode_mfma_enabled() && em::decode_mfma_supported(a)) {
                em::run_decode_mfma(a, packed);
            } else {
                em::run_gemv_packed(a, packed);
            }
        }
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
    if (bytes == 0) return EM_OK;
    if (!buf || !sink) return fail(EM_EINVAL, "stream_read: null pointer");
    if (bytes % 16 || reinterpret_cast<uintptr_t>(buf) % 16)
        return fail(EM_EINVAL, "stream_read: buffer and size must be multiples of 16 bytes");
    if (!em::device_present()) return fail(EM_ENODEV, "stream_read: no usable GPU");
    try {
        em::run_stream_read(buf, bytes, sink, static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

int em_probe_empty(unsigned blocks, void* stream) {
    if (blocks == 0 || blocks > 65535) return fail(EM_EINVAL, "probe_empty: 1..65535 workgroups");
    if (!em::device_present()) return fail(EM_ENODEV, "probe_empty: no usable GPU");
    em::run_probe_empty(static_cast<int>(blocks), static_cast<hipStream_t>(stream));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(EM_EDEVICE, std::string("hip: launch: ") + hipGetErrorString(err));
    return EM_OK;
}

int em_probe_read(const void* buf, size_t bytes, uint32_t* sink, unsigned blocks, unsigned depth,
                  int contiguous, void* stream) {
    if (bytes == 0) return EM_OK;
    if (!buf || !sink) return fail(EM_EINVAL, "probe_read: null pointer");
    if (bytes % 16 || reinterpret_cast<uintptr_t>(buf) % 16)
        return fail(EM_EINVAL, "probe_read: buffer and size must be multiples of 16 bytes");
    if (blocks == 0 || blocks > 65535) return fail(EM_EINVAL, "probe_read: 1..65535 workgroups");
    if (depth != 4 && depth != 8 && depth != 16)
        return fail(EM_EINVAL, "probe_read: depth must be 4, 8 or 16");
    if (!em::device_present()) return fail(EM_ENODEV, "probe_read: no usable GPU");
    em::run_probe_read(buf, bytes, static_cast<int>(blocks), static_cast<int>(depth),
                       contiguous != 0, sink, static_cast<hipStream_t>(stream));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(EM_EDEVICE, std::string("hip: launch: ") + hipGetErrorString(err));
    return EM_OK;
}

int em_probe_read_columns(const void* buf, unsigned rows, unsigned row_bytes, unsigned seg_bytes,
                          unsigned slices, unsigned depth, int xcd, uint32_t* sink, void* stream) {
    if (rows == 0) return EM_OK;
    if (!buf || !sink) return fail(EM_EINVAL, "probe_read_columns: null pointer");
    if (seg_bytes < 64 || seg_bytes > 1024 || (seg_bytes & (seg_bytes - 1)))
        return fail(EM_EINVAL, "probe_read_columns: segment must be 64, 128, 256, 512 or 1024 bytes");
    if (row_bytes == 0 || row_bytes % seg_bytes || reinterpret_cast<uintptr_t>(buf) % 16)
        return fail(EM_EINVAL, "probe_read_columns: rows must be whole segments, buffer 16-byte aligned");
    if (static_cast<unsigned long long>(rows) * row_bytes >= (1ULL << 31))
        return fail(EM_EINVAL, "probe_read_columns: at most 2^31 bytes");
    if (slices == 0 || slices > rows) return fail(EM_EINVAL, "probe_read_columns: 1..rows slices");
    if (static_cast<unsigned long long>(row_bytes / seg_bytes) * slices > 65535)
        return fail(EM_EINVAL, "probe_read_columns: at most 65535 workgroups");
    if (depth != 8 && depth != 16) return fail(EM_EINVAL, "probe_read_columns: depth must be 8 or 16");
    if (!em::device_present()) return fail(EM_ENODEV, "probe_read_columns: no usable GPU");
    em::run_probe_read_columns(buf, static_cast<int>(rows), static_cast<int>(row_bytes),
                               static_cast<int>(seg_bytes), static_cast<int>(slices),
                               static_cast<int>(depth), xcd != 0, sink,
                               static_cast<hipStream_t>(stream));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(EM_EDEVICE, std::string("hip: launch: ") + hipGetErrorString(err));
    return EM_OK;
}

static em::AttnShape to_shape(const em_attention_shape& s) {
    return {s.n_heads, s.n_kv_heads, s.head_size, s.seq_len, s.q_stride, s.kv_stride, s.out_stride};
}

int em_attention_check(const em_attention_shape* s, int kernel) {
    if (!s) return fail(EM_EINVAL, "attention: null shape");
    const std::string why = em::attention_reject(to_shape(*s), kernel);
    return why.empty() ? EM_OK : fail(EM_EINVAL, why);
}

size_t em_attention_scratch_floats(const em_attention_shape* s, size_t rows, int kernel) {
    if (!s || !em::attention_reject(to_shape(*s), kernel).empty()) return 0;
    return em::attention_scratch_floats(to_shape(*s), rows, kernel);
}

int em_attention(const em_attention_shape* s, size_t rows, const int* pos_dev, const float* q,
                 const float* key_cache, const float* value_cache, float* out, float* scratch,
                 int kernel, void* stream) {
    if (const int rc = em_attention_check(s, kernel)) return rc;
    if (rows == 0) return EM_OK;
    const em::AttnShape sh = to_shape(*s);
    if (rows > static_cast<size_t>(sh.seq_len))
        return fail(EM_EINVAL, "attention: more rows than seq_len");
    if (too_many(rows, sh.q_stride) || too_many(rows, sh.out_stride))
        return fail(EM_EINVAL, "attention: more than 2^31 elements");
    if (!pos_dev || !q || !key_cache || !value_cache || !out)
        return fail(EM_EINVAL, "attention: null pointer");
    if (em::attention_uses_split(sh, rows, kernel)) {
        const bool partials = em::attention_needs_scratch(sh, rows, kernel);
        if (partials && !scratch) return fail(EM_EINVAL, "attention: split needs scratch");
        auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
        if (!a16(q) || !a16(key_cache) || !a16(value_cache) || !a16(out) ||
            (partials && !a16(scratch)))
            return fail(EM_EINVAL, "attention: split needs 16-byte aligned q, caches, out, scratch");
    }
    if (!em::device_present()) return fail(EM_ENODEV, "attention: no usable GPU");
    try {
        em::run_attention(sh, static_cast<int>(rows), pos_dev, q, key_cache, value_cache, out,
                          scratch, kernel, static_cast<hipStream_t>(stream));
        em::hip_check(hipGetLastError(), "launch");
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
    return EM_OK;
}

}  // extern "C"
