// em_matmul_q8_noalloc: em_matmul_q8 with the skinny kernel, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc). The GEMV's split-K
// partials, which em_matmul_q8 keeps in grow-only library scratch, go to a
// file-scope device array of kScratchBytes (32 MiB) instead; the call allocates
// nothing (no hipMalloc, hipFree or allocating library routine) and runs
// the same kernels as em_matmul_q8 with EM_KERNEL_SKINNY, so its results are
// the same bits. No counterpart in the reference.
//
// The array is one per GPU (each device that loads the library holds its
// own copy until the process ends). In host code its name is only a
// stand-in: the device address comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that address is handed to
// kernels. Every call on a GPU shares that GPU's array, so calls that
// overlap on one GPU (on different streams, or from several host threads)
// race on it; calls on one stream are ordered. Nothing in it needs to start
// at zero: every partial is written before it is read.
#include <mutex>
#include <string>

#include "internal.hpp"
#include "llm_engine_amd.h"

namespace {

// 32 MiB: the partials of every Llama-7B-shaped decode product up to 8
// rows (the widest, 8 rows of the 4096 x 32000 classifier: 32 slices x 8 x
// 32000 floats = 31.25 MiB; 8 rows of 4096 x 11008: 10.75 MiB; one row of
// 4096 x 32000: 2 MiB).
constexpr std::size_t kScratchBytes = std::size_t{32} << 20;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace em {
namespace {

std::mutex g_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, its address taken on first use.
float* device_scratch(std::size_t* floats) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        fail(EM_EDEVICE, "matmul_q8_noalloc: no current device for the static scratch");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        // ::scratch: inside namespace em the bare name is the library's
        // grow-only scratch() function.
        const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
        if (rc != hipSuccess || !ptr) {
            fail(EM_EDEVICE, std::string("matmul_q8_noalloc: hipGetSymbolAddress: ") +
                                 hipGetErrorString(rc));
            return nullptr;
        }
        g_scratch_ptr[device] = static_cast<float*>(ptr);
    }
    *floats = kScratchBytes / sizeof(float);
    return g_scratch_ptr[device];
}

}  // namespace
}  // namespace em

extern "C" int em_matmul_q8_noalloc(size_t m, size_t n, size_t k, const float* A,
                                    const int8_t* B, const float* scale, float* C,
                                    int accumulate, const float* rms_weight, void* stream) {
    return em::matmul_entry<int8_t>(m, n, k, A, B, scale, C, EM_KERNEL_SKINNY, accumulate,
                                    rms_weight, stream, em::device_scratch);
}
