#include "scratch.hpp"

#include <map>
#include <mutex>
#include <utility>

namespace opl {

namespace {

struct ScratchRegistry {
  std::mutex mutex;
  std::map<std::pair<int, hipStream_t>, ReduceScratch> by_stream;
};

ScratchRegistry& registry() {
  // Leaked on purpose: device memory lives until process exit and the
  // registry must outlive any static destructor that might still launch.
  static ScratchRegistry* instance = new ScratchRegistry();
  return *instance;
}

}  // namespace

hipError_t reduce_scratch_for_stream(hipStream_t stream, ReduceScratch* out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  ScratchRegistry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  const auto key = std::make_pair(device, stream);
  auto found = reg.by_stream.find(key);
  if (found != reg.by_stream.end()) {
    *out = found->second;
    return hipSuccess;
  }
  // Layout: [counter (256 B slot)] [partials: kReduceMaxBlocks doubles].
  constexpr std::size_t kCounterSlot = 256;
  const std::size_t bytes =
      kCounterSlot + sizeof(double) * static_cast<std::size_t>(kReduceMaxBlocks);
  void* base = nullptr;
  status = hipMalloc(&base, bytes);
  if (status != hipSuccess) return status;
  // Zero the counter on the consumer's stream, so it is ordered before the
  // first reduce that uses it without any device-wide synchronization.
  status = hipMemsetAsync(base, 0, kCounterSlot, stream);
  if (status != hipSuccess) {
    (void)hipFree(base);
    return status;
  }
  ReduceScratch scratch;
  scratch.counter = static_cast<unsigned*>(base);
  scratch.partials = reinterpret_cast<double*>(static_cast<char*>(base) +
                                               kCounterSlot);
  reg.by_stream.emplace(key, scratch);
  *out = scratch;
  return hipSuccess;
}

}  // namespace opl
