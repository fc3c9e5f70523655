#pragma once

// ROCm profiler range annotations (roctx), the counterpart of the reference's NVTX ranges
// (include/zcgvs/core/nvtx.hpp:12-37). Compiled out unless ZCGVS_WITH_ROCTX is defined
// (build.py --roctx), so the default build carries no profiler dependency; with it, the ranges
// appear in rocprofv3 --marker-trace output.

#ifdef ZCGVS_WITH_ROCTX
#include <rocprofiler-sdk-roctx/roctx.h>
#endif

namespace zcgvs {

class TraceRange {
public:
    explicit TraceRange(const char* name) {
#ifdef ZCGVS_WITH_ROCTX
        roctxRangePushA(name);
#else
        (void)name;
#endif
    }

    ~TraceRange() {
#ifdef ZCGVS_WITH_ROCTX
        roctxRangePop();
#endif
    }

    TraceRange(const TraceRange&) = delete;
    TraceRange& operator=(const TraceRange&) = delete;
};

}  // namespace zcgvs

#define ZCGVS_TRACE_CONCAT_INNER(a, b) a##b
#define ZCGVS_TRACE_CONCAT(a, b) ZCGVS_TRACE_CONCAT_INNER(a, b)
#define ZCGVS_TRACE_RANGE(name) ::zcgvs::TraceRange ZCGVS_TRACE_CONCAT(zcgvs_trace_range_, __LINE__)(name)
