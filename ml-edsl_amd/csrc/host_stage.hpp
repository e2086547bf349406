// Host <-> device copies for the synchronous host-buffer entry points,
// staged through a pinned ring (host_stage.cpp). Internal; not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace edsl {
namespace rt {

// Throws the runtime's Failure for a HIP error (defined in runtime.cpp).
void check_hip(hipError_t e, const char* what);

// rows x cols elements of `es` bytes: host rows with pitch hld elements,
// device rows with pitch dld (>= cols). Both enqueue on `stream`; stage_h2d
// returns once the host buffer may be reused (the last DMAs may still be in
// flight), stage_d2h once the host buffer holds the data.
void stage_h2d(void* dev, int64_t dld, const void* host, int64_t hld, int64_t rows, int64_t cols, size_t es,
               hipStream_t stream);
void stage_d2h(void* host, int64_t hld, const void* dev, int64_t dld, int64_t rows, int64_t cols, size_t es,
               hipStream_t stream);

}  // namespace rt
}  // namespace edsl
