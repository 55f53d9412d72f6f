// SPDX-License-Identifier: MIT
// mi355x_mul_mat_noalloc: mi355x_mul_mat with its workspace (the fp16 activation pack and the
// row scales) in a file-scope device array instead of caller memory, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops). The array is per device: each
// GPU the library runs on holds its own copy, at its own address, until the process ends. Host
// code never passes the array's name to a kernel (on the host it names a stand-in, not device
// memory); the device address is resolved once per device with hipGetSymbolAddress, with that
// device current, and only that address is used.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "../../include/mi355x_kernels.h"

namespace {

constexpr size_t kScratchBytes = MI355X_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_lock;
void * g_scratch_dev[kMaxDevices] = {};

// The device address of `scratch` on the current device, resolved on the first call there.
int scratch_on_current_device(void ** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return MI355X_E_DEVICE;
    }
    std::lock_guard<std::mutex> g(g_lock);
    if (!g_scratch_dev[dev]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "[mi355x] mi355x_mul_mat_noalloc: hipGetSymbolAddress failed on device %d: %s\n", dev,
                    hipGetErrorString(e));
            (void)hipGetLastError();
            return MI355X_E_DEVICE;
        }
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return MI355X_OK;
}

}  // namespace

extern "C" {

MI355X_API int mi355x_mul_mat_noalloc(int wtype, const void * w_dev, int64_t N, int64_t K,
                                      const float * x_dev, int64_t ldx, int64_t M,
                                      float * dst_dev, int64_t ldd, void * stream) {
    if (M == 0) return MI355X_OK;
    const size_t need = mi355x_mul_mat_workspace(M, K);
    if (need == 0) return MI355X_E_ARG;
    if (need > kScratchBytes) {
        fprintf(stderr,
                "[mi355x] mi355x_mul_mat_noalloc: M %lld x K %lld needs %zu bytes of workspace, past the %zu-byte "
                "static scratch; call mi355x_mul_mat with a workspace instead\n",
                (long long)M, (long long)K, need, kScratchBytes);
        return MI355X_E_NOMEM;
    }
    void * ws = nullptr;
    const int st = scratch_on_current_device(&ws);
    if (st != MI355X_OK) return st;
    return mi355x_mul_mat(wtype, w_dev, N, K, x_dev, ldx, M, dst_dev, ldd, ws, kScratchBytes, stream);
}

}  // extern "C"
