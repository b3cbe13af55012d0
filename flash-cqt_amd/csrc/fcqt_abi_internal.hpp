// Host-side helpers shared by the C-ABI launchers (argument checks and
// launch-status capture). Not part of the public header.
#pragma once

#include <cstdint>
#include <cstdio>
#include <hip/hip_runtime.h>

#include "../../include/flashcqt.h"

namespace fcqt {

// grid.x = workgroups per slice * batch must stay below 2^31; the band
// kernel has the most workgroups per slice (< 256), so this is generous.
constexpr int64_t kMaxBatch = 1 << 22;

// fcqt_analysis runs batches of kAnalysisChunkMinBatch slices and more in
// chunks of kAnalysisChunk (the measurements are at the loop in abi.hip)
constexpr int64_t kAnalysisChunk = FCQT_ANALYSIS_CHUNK;
constexpr int64_t kAnalysisChunkMinBatch = FCQT_ANALYSIS_CHUNK_MIN_BATCH;
static_assert(kAnalysisChunk == 128 && kAnalysisChunkMinBatch == 256, "chunk constants of the header");

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Checks shared by the band launchers (FCQT_OK, FCQT_EARG or FCQT_EALIGN):
// record and task tables, the descriptor's coefficient span against ncoef,
// layout, alignment; defined in bands.hip.
int check_band_args(const fcqt_tables* tab, const int32_t* rec, const float* cre, const float* cim, int layout,
                    int64_t batch);

// Text of the last failed launch on this host thread.
inline char* last_error_buf() {
    static thread_local char buf[256] = {0};
    return buf;
}

// Status of the launch just issued: FCQT_OK, or FCQT_ELAUNCH with the HIP
// error text recorded for fcqt_last_hip_error().
inline int launch_status() {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return FCQT_OK;
    std::snprintf(last_error_buf(), 256, "%s (%d)", hipGetErrorString(e), (int)e);
    return FCQT_ELAUNCH;
}

}  // namespace fcqt
