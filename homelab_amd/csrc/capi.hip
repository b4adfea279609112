// Error state of the C ABI, the device status word of the kernels' bounded waits, and
// the workspace fill.
#include <atomic>
#include <mutex>
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

// The device's status word: a kernel whose bounded wait gives up stores 1 here (its
// outputs are invalid); oom_status exchanges it for 0 and reads the old value back through
// the line's second word. One 256-byte line per device
// (each device holds its own copy of a __device__ variable, at its own address).
static __device__ __align__(256) uint32_t status_line[64];

// Word 0 of the status line exchanged for 0 (one atomic step), the old value stored to
// word 1 for the host to copy.
__global__ void __launch_bounds__(64) status_take(uint32_t* line) {
    if (threadIdx.x == 0) {
        const uint32_t v = __hip_atomic_exchange(line, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(line + 1, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

constexpr int MAX_DEVICES = 64;
static std::mutex g_dev_mu;
static uint32_t* g_status_ptr[MAX_DEVICES] = {};
static std::atomic<uint32_t> g_wait_limit{DEFAULT_WAIT_LIMIT};
static std::mutex g_status_mu;

// The address of the current device's status word, looked up once per device with that
// device current (nullptr if the runtime refuses).
uint32_t* status_word() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    uint32_t* p = __atomic_load_n(&g_status_ptr[dev], __ATOMIC_ACQUIRE);
    if (p) return p;
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if (!g_status_ptr[dev]) {
        void* q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(status_line)) != hipSuccess || !q) {
            (void)hipGetLastError();
            return nullptr;
        }
        __atomic_store_n(&g_status_ptr[dev], reinterpret_cast<uint32_t*>(q), __ATOMIC_RELEASE);
    }
    return g_status_ptr[dev];
}

uint32_t wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }

}  // namespace oom

extern "C" int oom_set_wait_limit(uint32_t spins) {
    oom::g_wait_limit.store(spins ? spins : oom::DEFAULT_WAIT_LIMIT, std::memory_order_relaxed);
    return OOM_OK;
}

extern "C" int oom_status(void* stream) {
    using namespace oom;
    uint32_t* p = status_word();
    if (!p) return fail(OOM_ERR_LAUNCH, "oom_status: the device status word has no address");
    hipStream_t st = as_stream(stream);
    std::lock_guard<std::mutex> lock(g_status_mu);  // one reader of word 1 at a time
    // read and clear in one atomic exchange, so a give-up set by a kernel of another
    // stream between a read and a separate clear cannot be lost; the value read goes to
    // the line's second word, which the host then copies
    hipLaunchKernelGGL(status_take, dim3(1), dim3(64), 0, st, p);
    if (int rc = launched("oom_status")) return rc;
    uint32_t v = 0;
    if (hipMemcpyAsync(&v, p + 1, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(OOM_ERR_LAUNCH, std::string("oom_status: ") + hipGetErrorString(hipGetLastError()));
    if (v == 0) return OOM_OK;
    return fail(OOM_ERR_KERNEL,
                "a bounded wait inside a kernel gave up (grid not resident at once, or a wait limit set by "
                "oom_set_wait_limit): the outputs of that call are invalid");
}

extern "C" const char* oom_last_error(void) { return oom::g_last_error.c_str(); }

#ifdef OOM_STAMPS
// The profiling build's stamp buffer (see stream.hpp); not part of the default library's ABI.
namespace oom {
static uint64_t* g_stamps = nullptr;
uint64_t* stamps_buffer() { return g_stamps; }
}  // namespace oom
extern "C" void oom_debug_set_stamps(void* buf) { oom::g_stamps = reinterpret_cast<uint64_t*>(buf); }
#endif

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
