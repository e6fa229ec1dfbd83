#pragma once
// Library-owned device scratch and the lease that serialises its users.
//
// Some launch sequences need device memory beyond the caller's buffers:
//   * reduce: one fp64 partial per workgroup, summed by a second launch;
//   * decode GEMMs (M <= 16): split-K partial sums, summed by a second
//     launch;
//   * GEMMs whose operands miss the fast kernels' shape / alignment rules:
//     zero-padded aligned operand copies;
//   * fp16 GEMMs whose last round of 256x256 tiles fills at most half the
//     CUs: split-K partial tiles of that round, summed by a second launch;
//   * register-staged attention on small grids: per-split partial outputs,
//     merged by a second launch.
// The reference launchers need none of this (src/reduce.cu:54-69 combines
// with float atomics after an in-stream memset) and are reentrant because
// they share nothing; this library keeps the reentrancy as follows.
//
// Scratch is kept per (device, stream key). The stream key is the stream
// handle, except that hipStreamPerThread names a different stream in every
// host thread, so its key also holds the thread. A ScratchLease locks the
// key's scratch from construction to destruction; a launcher constructs one
// before its first enqueue that touches the scratch and keeps it until its
// last such enqueue has returned. Two host threads that launch on one stream
// (the null stream included) therefore enqueue their sequences one after the
// other, never interleaved, and stream order then keeps the device work of
// one sequence from overlapping the next.
//
// Eager buffers grow on demand: a request larger than the key's buffer
// allocates a new one of max(request, 2 x current) and retires the old one
// without freeing it (kernels earlier in the stream may still read it, and
// freeing would synchronize), so memory per key stays under twice its
// largest request. Buffers live until process exit.
//
// Under stream capture the lease never touches the stream's eager buffer:
// each request gets a buffer of its own, allocated with the thread's capture
// mode switched to relaxed for the allocation (hipMalloc does not enqueue on
// the capturing stream). The graph's kernels
// then own that memory: eager calls on the capture stream, or on the stream
// the graph is replayed on, can run concurrently with a replay without
// sharing scratch. Two replays of one graph that overlap in time share it,
// as with any graph that holds intermediate buffers. Capture-private
// buffers are kept until process exit (a graph's lifetime is not visible
// to the library).

#include <hip/hip_runtime.h>

#include <cstddef>

namespace opl {

struct Scratch {
  void* data = nullptr;  // >= the requested bytes, 256-byte aligned
};

class ScratchLease {
 public:
  // Locks the scratch of `stream` on the current device (eager streams) or
  // notes that `stream` is capturing. Check status() before get().
  explicit ScratchLease(hipStream_t stream);
  ~ScratchLease();
  ScratchLease(const ScratchLease&) = delete;
  ScratchLease& operator=(const ScratchLease&) = delete;

  hipError_t status() const { return status_; }

  // Scratch of at least `bytes`.
  hipError_t get(std::size_t bytes, Scratch* out);

  struct Entry;  // one key's buffer and lock (scratch.hip)

 private:
  hipStream_t stream_;
  hipError_t status_ = hipSuccess;
  bool capturing_ = false;
  Entry* entry_ = nullptr;
};

}  // namespace opl
