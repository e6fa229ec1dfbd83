// Library scratch: the per-GPU arena and the lease (the design is described
// in scratch.hpp).

#include "scratch.hpp"

#include <map>
#include <memory>
#include <mutex>

namespace opl {

namespace {

// One arena per GPU: each device holds its own copy of this array, at its
// own address, from the code object's load to process exit. Host code
// never passes the name itself to a kernel (in host code it is a host-side
// stand-in): the lease looks up each device's address once.
static __device__ __align__(256) unsigned char arena[kArenaBytes];

}  // namespace

struct ScratchLease::Device {
  std::mutex mutex;              // held by an arena lease for its sequence
  unsigned char* base = nullptr;  // this device's `arena`
  hipEvent_t done = nullptr;     // end of the latest eager arena sequence
  hipStream_t last = nullptr;    // the stream it was enqueued on
  bool recorded = false;
};

namespace {

struct Registry {
  std::mutex mutex;  // guards `devices` only
  std::map<int, std::unique_ptr<ScratchLease::Device>> devices;
};

Registry& registry() {
  // Leaked on purpose: the arena lives until process exit and the registry
  // must outlive any static destructor that might still launch.
  static Registry* instance = new Registry();
  return *instance;
}

// The current device's arena state, set up on its first use: the arena's
// address (hipGetSymbolAddress, with that device current) and the event of
// the sequence chain. Set-up runs with this thread's capture mode relaxed,
// so that a first use under stream capture may make these calls.
hipError_t current_device(ScratchLease::Device** out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  Registry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  auto& slot = reg.devices[device];
  if (!slot) {
    std::unique_ptr<ScratchLease::Device> fresh(new ScratchLease::Device());
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    status = hipThreadExchangeStreamCaptureMode(&mode);
    if (status != hipSuccess) {
      reg.devices.erase(device);
      return status;
    }
    void* base = nullptr;
    status = hipGetSymbolAddress(&base, HIP_SYMBOL(arena));
    // Arena users all run on this GPU, so the event needs no system-scope
    // fence: each kernel's own end-of-kernel (device-scope) release already
    // makes its writes visible to later kernels on the GPU, whatever their
    // stream. With the default system-scope fence every record flushed the
    // caches for the host: ~1.2 us per call as a stop event, ~2.8 us as a
    // separate record, against ~0.2 / ~0.7 us without it (13 us reduce).
    if (status == hipSuccess)
      status = hipEventCreateWithFlags(&fresh->done,
                                       hipEventDisableTiming | hipEventDisableSystemFence);
    hipStreamCaptureMode restore = mode;
    const hipError_t restored = hipThreadExchangeStreamCaptureMode(&restore);
    if (status == hipSuccess) status = restored;
    if (status != hipSuccess) {
      if (fresh->done != nullptr) (void)hipEventDestroy(fresh->done);
      reg.devices.erase(device);
      return status;
    }
    fresh->base = static_cast<unsigned char*>(base);
    slot = std::move(fresh);
  }
  *out = slot.get();  // entries are never erased once set up
  return hipSuccess;
}

}  // namespace

ScratchLease::ScratchLease(hipStream_t stream, void* workspace, std::size_t bytes)
    : stream_(stream) {
  if (workspace != nullptr) {
    data_ = workspace;
    capacity_ = bytes;
    return;
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  status_ = hipStreamIsCapturing(stream, &capture);
  if (status_ != hipSuccess) return;
  if (capture == hipStreamCaptureStatusInvalidated) {
    status_ = hipErrorStreamCaptureInvalidated;
    return;
  }
  capturing_ = capture == hipStreamCaptureStatusActive;
  Device* device = nullptr;
  status_ = current_device(&device);
  if (status_ != hipSuccess) return;
  device->mutex.lock();
  device_ = device;
  // hipStreamPerThread names a different stream in every host thread, so
  // the same handle does not mean the same stream there.
  const bool other_stream = stream != device->last || stream == hipStreamPerThread;
  if (!capturing_ && device->recorded && other_stream) {
    status_ = hipStreamWaitEvent(stream, device->done, 0);
    if (status_ != hipSuccess) {
      // Nothing is enqueued: release without recording, so the chain still
      // ends at the previous sequence.
      device_ = nullptr;
      device->mutex.unlock();
      return;
    }
  }
  data_ = device->base;
  capacity_ = kArenaBytes;
}

hipEvent_t ScratchLease::chain_event() const {
  return device_ != nullptr && !capturing_ ? device_->done : nullptr;
}

ScratchLease::~ScratchLease() {
  if (device_ == nullptr) return;
  // Unless the last launch carried it, the event is recorded here, even
  // after a failed launch: the stream already waits for the previous
  // sequence, so the record still marks a point after every earlier arena
  // sequence, which is all a later waiter needs.
  if (!capturing_ && (recorded_ || hipEventRecord(device_->done, stream_) == hipSuccess)) {
    device_->last = stream_;
    device_->recorded = true;
  }
  device_->mutex.unlock();
}

}  // namespace opl
