#pragma once
// Device scratch for the launch sequences that need memory beyond the
// caller's buffers, and the lease that hands it out. The library never
// allocates device memory: scratch is either the caller's workspace or a
// fixed static array per GPU.
//
// Users (each sizes its plan to the scratch it is offered; less scratch
// means fewer splits or a slower kernel, never an error):
//   * reduce: one fp64 partial per workgroup (at most 2 KiB);
//   * softmax and RMSNorm rows split over workgroups (rows longer than
//     32768 columns, or few rows longer than 4096): one partial per row
//     and segment (8 or 4 bytes);
//   * decode GEMMs (M <= 16): split-K partial sums;
//   * large fp16 GEMMs whose rows are not 4-byte aligned: operand copies
//     with chunk-padded rows;
//   * GEMMs whose last round of 256 x 256 tiles fills at most half the CUs,
//     or whose grid of 128 x 128 tiles is smaller than the CU count:
//     split-K partial tiles;
//   * register-staged attention on small grids: per-split partials.
// The reference launchers need none of this (src/reduce.cu:54-69 combines
// with float atomics after an in-stream memset) and are reentrant because
// they share nothing.
//
// Where scratch comes from:
//   * a caller workspace (the *_ws entry points of the C ABI): the caller
//     owns it and orders its uses on its streams; the lease only hands it
//     out. The torch binding passes a tensor from torch's stream-ordered,
//     capture-aware caching allocator here;
//   * otherwise the device arena: a static __device__ array of kArenaBytes,
//     one per GPU, held from the library's load to process exit. Every
//     stream of a GPU shares it, so a lease on the arena
//       - holds that GPU's host mutex while the sequence is enqueued,
//       - makes the stream wait (hipStreamWaitEvent) for the end of the
//         previous arena sequence when that one ran on another stream,
//       - records the end of its own sequence in the GPU's event (with no
//         system-scope fence: only this GPU's kernels wait on it).
//     Arena sequences therefore run one after another on the device,
//     whatever streams and host threads issue them, and nothing blocks the
//     host. Library-held device memory is kArenaBytes per GPU (plus the
//     no-allocation reduce's 2 KiB), whatever the number of calls, streams
//     or captured graphs.
//   * under stream capture the arena's event chain is left out of the
//     graph: a replay uses the arena without waiting for other arena users.
//     Replays must therefore not overlap another arena sequence on the same
//     GPU (replay in stream order with the other calls that use it), or the
//     capturing caller passes a workspace (the torch binding always does).

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <tuple>

namespace opl {

// Bytes of each GPU's arena (under 0.1% of an MI355X's 288 GB). It holds
// the padded copies of fp16 GEMM operands up to 8191^3 (both copied, 256
// MiB), and every plan at the reference's benchmark sizes in full, split
// last rounds included.
constexpr std::size_t kArenaBytes = std::size_t(256) << 20;

// Plans are computed for a scratch capacity: kUnlimited for workspace-size
// queries and the *_ws entry points, kArenaBytes for the others.
constexpr std::size_t kUnlimited = ~std::size_t(0);

class ScratchLease {
 public:
  // workspace != nullptr: the caller's [workspace, workspace + bytes).
  // Otherwise the current device's arena (locked for the lease's lifetime).
  // Check status() before data().
  ScratchLease(hipStream_t stream, void* workspace, std::size_t bytes);
  ~ScratchLease();
  ScratchLease(const ScratchLease&) = delete;
  ScratchLease& operator=(const ScratchLease&) = delete;

  hipError_t status() const { return status_; }
  // 256-byte aligned.
  void* data() const { return data_; }
  std::size_t capacity() const { return capacity_; }

  // Enqueues `kernel` as the sequence's last launch. On the eager arena the
  // chain's event rides on it as hipExtLaunchKernel's stop event, so it
  // completes with the kernel: a separate hipEventRecord at release adds a
  // marker of its own, measured at ~0.7 us per call on a 13 us reduce (the
  // stop event: ~0.2 us). Elsewhere (a caller workspace, capture) it is a
  // plain launch. Sequences whose last launch is a long kernel leave the
  // record to the destructor instead.
  template <typename... Params, typename... Args>
  hipError_t launch_last(void (*kernel)(Params...), dim3 grid, dim3 block, Args... args);

  struct Device;  // one GPU's arena state (scratch.hip)

 private:
  hipStream_t stream_;
  hipError_t status_ = hipSuccess;
  void* data_ = nullptr;
  std::size_t capacity_ = 0;
  bool capturing_ = false;
  bool recorded_ = false;  // the chain's event rides on the last launch
  Device* device_ = nullptr;

  hipEvent_t chain_event() const;  // nullptr unless on the eager arena
};

template <typename... Params, typename... Args>
hipError_t ScratchLease::launch_last(void (*kernel)(Params...), dim3 grid, dim3 block,
                                     Args... args) {
  static_assert(sizeof...(Params) == sizeof...(Args), "one argument per parameter");
  const hipEvent_t event = chain_event();
  if (event == nullptr) {
    kernel<<<grid, block, 0, stream_>>>(args...);
    return hipGetLastError();
  }
  std::tuple<Params...> values(static_cast<Params>(args)...);
  void* pointers[sizeof...(Params) > 0 ? sizeof...(Params) : 1];
  std::apply([&](auto&... v) {
    std::size_t i = 0;
    ((pointers[i++] = static_cast<void*>(&v)), ...);
  }, values);
  const hipError_t status = hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid,
                                               block, pointers, 0, stream_, nullptr, event, 0);
  if (status == hipSuccess) recorded_ = true;
  return status;
}

// Where a call's scratch comes from. Workspace mode (the *_ws entry points
// and the workspace-size queries): plans assume unlimited capacity and the
// entry point checks the caller's workspace against the plan. Otherwise the
// arena, and plans fit kArenaBytes.
struct ScratchSource {
  bool workspace_mode = false;
  void* data = nullptr;
  std::size_t bytes = 0;
  std::size_t capacity() const { return workspace_mode ? kUnlimited : kArenaBytes; }
};

// Checks a *_ws call's workspace against the bytes its plan needs: enough
// bytes, and a 256-byte aligned pointer (every torch allocation is) when
// any are needed.
inline bool workspace_ok(const void* workspace, std::size_t bytes, std::size_t needed) {
  if (needed == 0) return true;
  return workspace != nullptr && bytes >= needed &&
         (reinterpret_cast<std::size_t>(workspace) & 255u) == 0;
}

}  // namespace opl
