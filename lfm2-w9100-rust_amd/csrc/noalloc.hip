// noalloc.hip -- the library's one entry point that allocates nothing:
// lfm_argmax_noalloc, the greedy argmax of lfm_argmax over a file-scope device
// scratch array instead of per-call device allocations.  For callers that
// cannot call hipMalloc (tight serving loops, harnesses that forbid it).
//
// The scratch array lives in this file's code object; each device the library
// runs on holds its own copy until the process ends.  Its device address is
// taken once per device with hipGetSymbolAddress when the library sets the
// device up (lfm_noalloc_setup, called by the code-object loader on the
// device's first launching call), and only that address is used from host
// code: the array's name in host code is a host-side stand-in, not a device
// address.
//
// Layout of the scratch (NOALLOC_SCRATCH_BYTES = 8448 bytes):
//   [0, 64)             DevState of the two-stage argmax (halt must read 0:
//                       cleared by k_noalloc_clear before every call)
//   [256, 256 + 8192)   (value, index) partials of up to NOALLOC_ARGMAX_WGS
//                       workgroups, all written by k_argmax before
//                       k_argmax_final reads them
// Every call on a device shares that device's array and leaves the last
// call's contents in it: calls that overlap on one device race.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "../../include/lfm_hip.h"
#include "host_err.h"
#include "kargs.h"
#include "launch_host.h"

#define NOALLOC_STATE_BYTES 256
#define NOALLOC_SCRATCH_BYTES (NOALLOC_STATE_BYTES + NOALLOC_ARGMAX_WGS * 2 * 4)
#define NOALLOC_MAX_DEVICES 64
static_assert(sizeof(DevState) <= NOALLOC_STATE_BYTES, "state block");

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex g_mu;
static void *g_ptr[NOALLOC_MAX_DEVICES]; // device address of `scratch`, per device

// Zeroes the argmax state block (a fill kernel rather than a memset, so that a
// caller capturing the calls into a graph records no memset node).
static __global__ void k_noalloc_clear(uint32_t *words, uint32_t n)
{
    if (threadIdx.x < n)
        words[threadIdx.x] = 0u;
}

int lfm_noalloc_setup(int dev)
{
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return fail(LFM_EDEVICE, "device %d: no scratch slot (at most %d devices)", dev,
                    NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[dev])
        return LFM_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return fail(LFM_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
    g_ptr[dev] = p;
    return LFM_OK;
}

extern "C" int lfm_argmax_noalloc(const float *v, uint32_t n, uint32_t *index, float *value)
{
    if (!v || n == 0 || !index)
        return fail(LFM_EINVAL, "lfm_argmax_noalloc: empty input");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return fail(LFM_EDEVICE, "lfm_argmax_noalloc: no current device");
    void *base;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        base = g_ptr[dev];
    }
    if (!base)
        return fail(LFM_ESTATE, "lfm_argmax_noalloc: the library is not set up on device %d "
                    "(its first launching call, e.g. lfm_engine_create or lfm_argmax, does that)", dev);
    const uint32_t grid = lfm_argmax_grid(n);
    const size_t need = NOALLOC_STATE_BYTES + (size_t)grid * 2 * 4;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(LFM_ERANGE, "lfm_argmax_noalloc: %zu scratch bytes needed, %d available", need,
                    NOALLOC_SCRATCH_BYTES);
    DevState *st = (DevState *)base;
    float *partial = (float *)((uint8_t *)base + NOALLOC_STATE_BYTES);
    (void)hipGetLastError(); // a launch error below is this call's, not an earlier call's
    hipLaunchKernelGGL(k_noalloc_clear, dim3(1), dim3(64), 0, 0, (uint32_t *)st,
                       (uint32_t)(sizeof(DevState) / 4));
    if (hipGetLastError() != hipSuccess)
        return fail(LFM_EDEVICE, "lfm_argmax_noalloc: clear launch failed");
    int rc = lfm_argmax_enqueue(v, n, st, partial, nullptr);
    if (rc != LFM_OK)
        return rc;
    DevState h;
    if (hipMemcpy(&h, st, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(LFM_EDEVICE, "lfm_argmax_noalloc: result copy failed");
    *index = h.last_token;
    if (value)
        *value = h.last_value;
    return LFM_OK;
}
