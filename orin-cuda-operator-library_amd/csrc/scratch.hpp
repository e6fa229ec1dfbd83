#pragma once
// Library-owned device scratch, kept per (device, stream).
//
// 1. Reduce partials: the deterministic reduce writes one fp64 partial per
// workgroup in its first launch and combines them in a second. The reference needs none because it combines with float atomics
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

#include <cstddef>

namespace opl {

// Upper bound on the reduce grid; sizes the partials array (8 KiB).
constexpr int kReduceMaxBlocks = 1024;

// Returns the partials buffer (kReduceMaxBlocks doubles) for `stream` on the
// current device, allocating it on first use. Thread-safe.
hipError_t reduce_partials_for_stream(hipStream_t stream, double** out);

// 2. Operand / partials workspace: GEMMs whose operands do not meet the
// fast kernels' shape / alignment rules are first copied into zero-padded,
// aligned buffers here; decode GEMMs keep their split-K partial sums here,
// and register-staged attention on small grids its per-split partial
// outputs. Grow-only: a request larger than the current
// buffer allocates a new one of max(bytes, 2 x current) and retires the old
// one without freeing it (kernels earlier in the stream may still read it,
// and freeing would synchronize), so total memory stays under twice the
// largest request. The same stream-ordering and first-use rules as for the
// partials apply. Thread-safe.
hipError_t workspace_for_stream(hipStream_t stream, std::size_t bytes,
                                void** out);

}  // namespace opl
