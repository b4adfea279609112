// Error state of the C ABI and the workspace fill.
#include <string>

#include "common.hpp"

namespace oom {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int launched(const char* what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return OOM_OK;
    return fail(OOM_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}

// Grid-stride zero fill of n 16-byte words, then the byte tail.
__global__ void __launch_bounds__(256) fill_zero(uint4* p, size_t words, uint8_t* tail, int tail_bytes) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < words; i += (size_t)gridDim.x * blockDim.x) p[i] = make_uint4(0, 0, 0, 0);
    if (blockIdx.x == 0 && (int)threadIdx.x < tail_bytes) tail[threadIdx.x] = 0;
}

}  // namespace oom

extern "C" const char* oom_last_error(void) { return oom::g_last_error.c_str(); }

extern "C" int oom_workspace_init(void* ws, size_t bytes, void* stream) {
    if (bytes == 0) return OOM_OK;
    OOM_REQUIRE(ws != nullptr, "oom_workspace_init: null workspace");
    OOM_REQUIRE(oom::aligned(ws, 16), "oom_workspace_init: workspace must be 16-byte aligned");
    size_t words = bytes / 16;
    int tail = (int)(bytes % 16);
    int blocks = (int)std::min<size_t>(1024, std::max<size_t>(1, (words + 255) / 256));
    hipLaunchKernelGGL(oom::fill_zero, dim3(blocks), dim3(256), 0, oom::as_stream(stream),
                       reinterpret_cast<uint4*>(ws), words, reinterpret_cast<uint8_t*>(ws) + words * 16, tail);
    return oom::launched("oom_workspace_init");
}
