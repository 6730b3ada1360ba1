// g4_internal.h -- host-side plumbing shared by the entry points: the
// library stream, status codes and the last-error message.
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>

#include "../../include/g4hip.h"

hipStream_t g4_stream();
int g4_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int g4_hip_status(hipError_t e);   // 0 or G4_ERR_HIP (message recorded)
int g4_check_launch(const char* kernel);
int g4_num_cus();
// device address of the allocation-free attention's scratch on `device`
// (current), resolved once per device; called by g4_init
int g4_attn_scratch_setup(int device);
// last pass of an argmax over np per-workgroup keys (argmax_key order):
// the index to *out / *dtok (each optional), *dpos advanced if given
int g4_argmax_final(const void* part, int np, int* out, int* dtok, int* dpos);

#define G4_CHECK_ARG(cond, ...)                          \
    do {                                                 \
        if (!(cond)) return g4_fail(G4_ERR_ARG, __VA_ARGS__); \
    } while (0)
#define G4_CHECK(cond, code, ...)                        \
    do {                                                 \
        if (!(cond)) return g4_fail(code, __VA_ARGS__);  \
    } while (0)
#define G4_HIP(expr)                                     \
    do {                                                 \
        int rc_ = g4_hip_status(expr);                   \
        if (rc_) return rc_;                             \
    } while (0)
