// Library scratch: registry and lease (the design is described in
// scratch.hpp).

#include "scratch.hpp"

#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <tuple>
#include <vector>

namespace opl {

namespace {

using Key = std::tuple<int, hipStream_t, std::thread::id>;

}  // namespace

struct ScratchLease::Entry {
  std::mutex mutex;           // held by the lease for the whole sequence
  void* base = nullptr;
  std::size_t data_bytes = 0;
};

namespace {

struct Registry {
  std::mutex mutex;  // guards the map and the retired list only
  std::map<Key, std::unique_ptr<ScratchLease::Entry>> entries;
  std::vector<void*> retired;  // outgrown and capture-private buffers
};

Registry& registry() {
  // Leaked on purpose: device memory lives until process exit and the
  // registry must outlive any static destructor that might still launch.
  static Registry* instance = new Registry();
  return *instance;
}

}  // namespace

ScratchLease::ScratchLease(hipStream_t stream) : stream_(stream) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  status_ = hipStreamIsCapturing(stream, &capture);
  if (status_ != hipSuccess) return;
  if (capture == hipStreamCaptureStatusInvalidated) {
    status_ = hipErrorStreamCaptureInvalidated;
    return;
  }
  if (capture == hipStreamCaptureStatusActive) {
    capturing_ = true;
    return;
  }
  int device = 0;
  status_ = hipGetDevice(&device);
  if (status_ != hipSuccess) return;
  const std::thread::id owner =
      stream == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
  Registry& reg = registry();
  {
    std::lock_guard<std::mutex> lock(reg.mutex);
    auto& slot = reg.entries[Key(device, stream, owner)];
    if (!slot) slot.reset(new Entry());
    entry_ = slot.get();  // entries are never erased
  }
  entry_->mutex.lock();
}

ScratchLease::~ScratchLease() {
  if (entry_ != nullptr) entry_->mutex.unlock();
}

hipError_t ScratchLease::get(std::size_t bytes, Scratch* out) {
  if (status_ != hipSuccess) return status_;
  if (capturing_) {
    // Relaxed mode for this thread only, for the allocation only.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    hipError_t status = hipThreadExchangeStreamCaptureMode(&mode);
    if (status != hipSuccess) return status;
    void* base = nullptr;
    status = hipMalloc(&base, bytes);
    hipStreamCaptureMode restore = mode;
    const hipError_t restored = hipThreadExchangeStreamCaptureMode(&restore);
    if (status != hipSuccess) return status;
    if (restored != hipSuccess) return restored;
    {
      Registry& reg = registry();
      std::lock_guard<std::mutex> lock(reg.mutex);
      reg.retired.push_back(base);
    }
    out->data = base;
    return hipSuccess;
  }
  if (entry_->base == nullptr || entry_->data_bytes < bytes) {
    const std::size_t grow =
        entry_->data_bytes * 2 > bytes ? entry_->data_bytes * 2 : bytes;
    void* fresh = nullptr;
    const hipError_t status = hipMalloc(&fresh, grow);
    if (status != hipSuccess) return status;
    if (entry_->base != nullptr) {
      Registry& reg = registry();
      std::lock_guard<std::mutex> lock(reg.mutex);
      reg.retired.push_back(entry_->base);
    }
    entry_->base = fresh;
    entry_->data_bytes = grow;
  }
  out->data = entry_->base;
  return hipSuccess;
}

}  // namespace opl
