// rkv_host.h -- host helpers shared by the C-ABI translation units
// (rkv_runtime.cpp, rkv_serve.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/rkv.h"

namespace rkv {
namespace host {

// Records "op: message" as the calling thread's rkv_last_error() and
// returns `code` (HarError{operation, message}, har-vulkan/src/lib.rs:19-56).
rkv_status fail(rkv_status code, const char *op, const char *fmt, ...)
    __attribute__((format(printf, 3, 4)));
// A HIP runtime error as RKV_ERR_DEVICE.
rkv_status hip_fail(const char *op, hipError_t e);
// Makes ctx's device current for the calling thread.
rkv_status use_device(rkv_ctx *ctx, const char *op);

}  // namespace host
}  // namespace rkv
