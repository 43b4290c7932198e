// Allocation-free decode attention step.
//
// loom_gqa_decode_step_noalloc runs loom_gqa_decode_step (RoPE + cache append
// + chunked attention + merge) with its per-chunk partial records in a
// file-scope device array instead of a caller-allocated workspace, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops).  Each device holds its own copy of the array; its address is
// looked up once per device with hipGetSymbolAddress and that address, never
// the array's host-side name, is what the kernels receive.  Calls that
// overlap on one device share the array and race.
#include <mutex>

#include "loom_common.h"

namespace loom {

// One launch's records: B * KVH * nchunks * (2G + 2G*HD) fp32 (about 1.2 MB at
// B = 32, 2 kv heads of 96, group 4).  The kernels write every record they
// read, so the array needs no clearing between calls.
static __device__ __align__(256) unsigned char scratch[LOOM_GQA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device (nullptr + error on failure).
static float* scratch_ptr(int* rc) {
    static std::mutex mu;
    static void* ptrs[kMaxDevices] = {nullptr};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("gqa_decode_step_noalloc: no usable current device (%s)",
                  e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
        *rc = LOOM_ERR_INVALID;
        return nullptr;
    }
    std::lock_guard<std::mutex> g(mu);
    if (ptrs[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("gqa_decode_step_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                      hipGetErrorString(e));
            *rc = LOOM_ERR_LAUNCH;
            return nullptr;
        }
        ptrs[dev] = p;
    }
    *rc = LOOM_OK;
    return (float*)ptrs[dev];
}

}  // namespace loom

using namespace loom;

extern "C" int loom_gqa_decode_step_noalloc(int dtype, const void* qkv, void* k_cache,
                                            void* v_cache, int64_t cache_stride_b,
                                            int64_t cache_stride_t, int64_t cache_stride_h,
                                            const float* cos_table, const float* sin_table,
                                            void* q_out, void* c_out, void* kctx_out,
                                            int64_t out_stride_b, int64_t B, int64_t len,
                                            const int64_t* pos_dev, int64_t QH, int64_t KVH,
                                            int64_t HD, void* stream) {
    clear_error();
    LOOM_CHECK(B >= 0 && len >= 1 && KVH >= 1 && QH >= KVH && QH % KVH == 0,
               "gqa_decode_step_noalloc: bad shape B=%lld len=%lld QH=%lld KVH=%lld",
               (long long)B, (long long)len, (long long)QH, (long long)KVH);
    const int64_t need = loom_gqa_workspace_bytes(B, len, QH, KVH, HD);
    LOOM_CHECK(need <= (int64_t)LOOM_GQA_NOALLOC_SCRATCH_BYTES,
               "gqa_decode_step_noalloc: B=%lld, len=%lld, QH=%lld, KVH=%lld, HD=%lld needs %lld "
               "bytes of partial records, above the %lld-byte static scratch; use "
               "loom_gqa_decode_step with a workspace",
               (long long)B, (long long)len, (long long)QH, (long long)KVH, (long long)HD,
               (long long)need, (long long)LOOM_GQA_NOALLOC_SCRATCH_BYTES);
    int rc = LOOM_OK;
    float* ws = scratch_ptr(&rc);
    if (ws == nullptr) return rc;
    return loom_gqa_decode_step(dtype, qkv, k_cache, v_cache, cache_stride_b, cache_stride_t,
                                cache_stride_h, cos_table, sin_table, q_out, c_out, kctx_out,
                                out_stride_b, ws, (int64_t)LOOM_GQA_NOALLOC_SCRATCH_BYTES, B, len,
                                pos_dev, QH, KVH, HD, stream);
}
