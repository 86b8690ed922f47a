// jh_op_gemm_splitk_noalloc: jh_op_gemm_splitk with its FP32 partial sums in
// a fixed, file-scope device array instead of a caller workspace, for callers
// that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The kernels are jh_op_gemm_splitk's; only
// where their partial sums live differs.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/julia1_hip_ops.h"
#include "abi_util.hpp"
#include "kernels.hpp"

namespace {

// Split-K partial sums: splits x rows x N floats.  Every call on a device
// shares that device's copy, which keeps the last call's contents; the
// partial pass writes every element it reduces, so nothing is cleared.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device address of `scratch` per device ordinal.  The array's name is a host
// stand-in; only the address hipGetSymbolAddress returns, with that device
// current, may be handed to kernels.
constexpr int kMaxDevices = 64;
float* scratch_ptr[kMaxDevices];
std::once_flag scratch_once[kMaxDevices];

float* device_scratch() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw jh_error(JH_ERR_DEVICE, "device ordinal out of range");
    hipError_t err = hipSuccess;
    std::call_once(scratch_once[dev], [&] {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err == hipSuccess) scratch_ptr[dev] = (float*)p;
    });
    if (err != hipSuccess) throw jh_error(JH_ERR_DEVICE, std::string("hipGetSymbolAddress: ") + hipGetErrorString(err));
    if (!scratch_ptr[dev]) throw jh_error(JH_ERR_DEVICE, "split-K scratch has no address on this device");
    return scratch_ptr[dev];
}

inline int as_int(size_t v, const char* what) {
    if (v > (size_t)0x7fffffff) throw jh_error(JH_ERR_INVALID, std::string(what) + " too large");
    return (int)v;
}

}  // namespace

extern "C" {

int jh_op_gemm_splitk_noalloc(int epilogue, const void* x, size_t ldx, const int32_t* gather, size_t rows,
                              const void* w, size_t n, size_t k, void* out, size_t ldo, size_t col,
                              const float* bias, const int32_t* pos, const float* cos_t, const float* sin_t,
                              size_t rope_cols, int splits, void* stream) {
    return jh_guarded([&] {
        GemmArgs a{(const bf16_t*)x, (long)ldx, gather, as_int(rows, "rows"), (const bf16_t*)w, as_int(n, "n"),
                   as_int(k, "k"), out, (long)ldo, as_int(col, "col"), bias, pos, cos_t, sin_t,
                   as_int(rope_cols, "rope_cols")};
        if (splits < 0) throw jh_error(JH_ERR_INVALID, "gemm: negative split count");
        if (splits > 1 && (size_t)splits * rows * n * sizeof(float) > kScratchBytes)
            throw jh_error(JH_ERR_INVALID, "gemm: split-K partials (splits x rows x N floats) exceed the " +
                                               std::to_string(kScratchBytes >> 20) + " MiB scratch");
        a.partial = device_scratch();
        a.partial_bytes = kScratchBytes;
        a.splits = splits;
        launch_gemm(epilogue, a, (hipStream_t)stream);
    });
}

}  // extern "C"
