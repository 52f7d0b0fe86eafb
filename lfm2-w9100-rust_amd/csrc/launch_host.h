// launch_host.h -- host-side launch helpers shared by the library's sources
// (engine.cpp, noalloc.hip); not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "kargs.h"

// Workgroups of the first argmax stage: one per 256 values, at most
// NOALLOC_ARGMAX_WGS (the stage is grid-stride beyond that).
#define NOALLOC_ARGMAX_WGS 1024
__attribute__((visibility("hidden"))) uint32_t lfm_argmax_grid(uint32_t n);

// Enqueues the two-stage argmax of v[0..n) (k_argmax, k_argmax_final) on stream
// s with caller-provided buffers: st (a DevState whose halt field reads 0) and
// partial (2 * lfm_argmax_grid(n) floats).  The result lands in st->last_token
// and st->last_value.  Uses the code objects already loaded on the current
// device, or loads them (the device's first launching call).
__attribute__((visibility("hidden"))) int lfm_argmax_enqueue(const float *v, uint32_t n,
                                                             DevState *st, float *partial,
                                                             hipStream_t s);

// Per-device set-up of the no-allocation entry point (noalloc.hip): takes the
// device address of its scratch array.  Called with the device current, once,
// when the device's code objects are loaded.
__attribute__((visibility("hidden"))) int lfm_noalloc_setup(int dev);
