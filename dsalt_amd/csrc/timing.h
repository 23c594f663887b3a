// Opt-in per-kernel timing: when enabled (dsalt_timing_enable), every kernel
// the library enqueues is bracketed by two HIP events recorded on its stream;
// dsalt_timing_report() waits for them and returns per-kernel launch counts
// and total milliseconds.  Disabled, the launch macro costs one flag load.
#pragma once

#include <hip/hip_runtime.h>

namespace dsalt {

bool timing_enabled();
void timing_begin(const char* name, hipStream_t stream);
void timing_end(hipStream_t stream);

}  // namespace dsalt

#define DSALT_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                 \
    do {                                                                            \
        const bool dsalt_timed_ = ::dsalt::timing_enabled();                        \
        if (dsalt_timed_) ::dsalt::timing_begin(name, stream);                      \
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);        \
        if (dsalt_timed_) ::dsalt::timing_end(stream);                              \
    } while (0)
