// oom_moe_decode_fp8_noalloc: the decode MoE step of oom_moe_decode_fp8 for callers that
// cannot allocate (code under graph capture, tight serving loops): its workspace is a
// file-scope device array of NOALLOC_BYTES, not caller memory.
//
// Each device holds its own copy of `scratch` at its own address. The host-side name of
// the array is not a device address, so the address is looked up once per device with
// hipGetSymbolAddress (that device current) and only that address is handed to kernels.
// The array is zero when the code object loads. The header's barrier counters only grow
// and agree again whenever a call ends (a call whose wait gave up too), its tickets are
// reset by their users, and the rest of the workspace is written before it is read, so
// no call clears anything.
// All calls on one device share the array: calls that overlap in time on one device
// (two streams, two threads) race, so a caller orders them on one stream.
#include <mutex>

#include "common.hpp"

extern "C" int oom_moe_decode_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                                  int E, int k, const OomFp8Record* geo, int32_t* ids, float* weights, void* out,
                                  int out_dtype, void* ws, size_t ws_bytes, void* stream);
extern "C" size_t oom_moe_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo);

namespace oom {

constexpr size_t NOALLOC_BYTES = size_t(4) << 20;  // covers T <= 16, k <= 8, hidden <= 4096, inter <= 2048
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// The current device's address of `scratch` (looked up on the first call on the device).
static int scratch_ptr(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        (void)hipGetLastError();
        return fail(OOM_ERR_LAUNCH, "oom_moe_decode_fp8_noalloc: no current device");
    }
    void* p = __atomic_load_n(&g_scratch_ptr[dev], __ATOMIC_ACQUIRE);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev];
        if (!p) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                (void)hipGetLastError();
                return fail(OOM_ERR_LAUNCH, std::string("oom_moe_decode_fp8_noalloc: hipGetSymbolAddress: ") +
                                                hipGetErrorString(e));
            }
            __atomic_store_n(&g_scratch_ptr[dev], p, __ATOMIC_RELEASE);
        }
    }
    *out = p;
    return OOM_OK;
}

}  // namespace oom

extern "C" size_t oom_moe_decode_fp8_noalloc_max_bytes(void) { return oom::NOALLOC_BYTES; }

extern "C" int oom_moe_decode_fp8_noalloc(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs,
                                          int T, int E, int k, const OomFp8Record* geo, int32_t* ids, float* weights,
                                          void* out, int out_dtype, void* stream) {
    using namespace oom;
    OOM_REQUIRE(geo != nullptr && T >= 1 && E >= 1 && k >= 1, "oom_moe_decode_fp8_noalloc: shape");
    const size_t need = oom_moe_decode_fp8_workspace_size(T, E, k, geo);
    if (need == 0 || need > NOALLOC_BYTES)
        return fail(OOM_ERR_WORKSPACE, "oom_moe_decode_fp8_noalloc: the step needs " + std::to_string(need) +
                                           " bytes of scratch, more than its " + std::to_string(NOALLOC_BYTES) +
                                           " (use oom_moe_decode_fp8 with a workspace)");
    void* ws = nullptr;
    if (int rc = scratch_ptr(&ws)) return rc;
    return oom_moe_decode_fp8(logits, x, x_dtype, all_recs, T, E, k, geo, ids, weights, out, out_dtype, ws,
                              NOALLOC_BYTES, stream);
}
