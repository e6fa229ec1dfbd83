#pragma once
// Library-owned device scratch for the deterministic reduce, which writes one
// fp64 partial per workgroup in its first launch and combines them in a
// second. The reference needs none because it combines with float atomics
// after an in-stream memset (src/reduce.cu:46, :64); this library instead
// keeps one small buffer per (device, stream) pair:
//   * launches on one stream are ordered by the stream, so they may share it;
//   * launches on different streams get different buffers, so the launcher
//     stays reentrant across streams and host threads like the reference's.
// The buffer is allocated with hipMalloc the first time a stream is used on
// a device and kept until process exit; later calls on that stream allocate
// nothing, so only the first call on a stream must happen outside HIP graph
// capture.

#include <hip/hip_runtime.h>

namespace opl {

// Upper bound on the reduce grid; sizes the partials array (8 KiB).
constexpr int kReduceMaxBlocks = 1024;

// Returns the partials buffer (kReduceMaxBlocks doubles) for `stream` on the
// current device, allocating it on first use. Thread-safe.
hipError_t reduce_partials_for_stream(hipStream_t stream, double** out);

}  // namespace opl
