#pragma once
// Library-owned device scratch for kernels that combine partial results
// across workgroups (the deterministic reduce). The reference needs none
// because it combines with float atomics after an in-stream memset
// (src/reduce.cu:46, :64); this library instead keeps one small buffer per
// (device, stream) pair:
//   * calls on one stream are ordered by the stream, so they may share it;
//   * calls on different streams get different buffers, so launchers stay
//     reentrant across streams and host threads like the reference's.
// The buffer is allocated (hipMalloc, then a zero fill of its counter enqueued
// on that same stream) the first time a stream is used on a device, and kept
// until process exit. Later calls on that stream allocate nothing, so only
// the first call on a stream must happen outside HIP graph capture.

#include <hip/hip_runtime.h>

#include <cstddef>

namespace opl {

struct ReduceScratch {
  double* partials;    // one fp64 partial sum per workgroup
  unsigned* counter;   // arrival counter; zero between launches
};

// Upper bound on the reduce grid; sizes the partials array.
constexpr int kReduceMaxBlocks = 2048;

// Returns the scratch for `stream` on the current device, allocating it on
// first use. Thread-safe.
hipError_t reduce_scratch_for_stream(hipStream_t stream, ReduceScratch* out);

}  // namespace opl
