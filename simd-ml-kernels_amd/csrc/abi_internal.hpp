// abi_internal.hpp -- status and device helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "smk_hip.h"

namespace smk::abi {

const char* last_error();
int ok();                                     // clears the thread's error, returns SMK_OK
int fail(int code, const std::string& msg);   // records msg, returns code
int hip_fail(hipError_t e, const char* what); // maps a HIP error to SMK_ERR_DEVICE / _OUT_OF_MEMORY
int use_device();                             // selects the library's device on this thread
}  // namespace smk::abi

#include "launch.hpp"

namespace smk::abi {
smk::GemvTuning tuning_snapshot();            // the diagnostics settings (smk_set_*) now in force
int check_gemv_args(int M, int N, int K, const void* x, const void* W, const void* y);
int gemv_launch_fail(hipError_t e, const smk::GemvTuning& t, int M, int N, int K);

}  // namespace smk::abi

#define SMK_HIP(call, what)                                           \
    do {                                                              \
        const hipError_t e_ = (call);                                 \
        if (e_ != hipSuccess) return ::smk::abi::hip_fail(e_, what);  \
    } while (0)
