#include "scratch.hpp"

#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace opl {

namespace {

struct Workspace {
  void* ptr = nullptr;
  std::size_t bytes = 0;
};

struct ScratchRegistry {
  std::mutex mutex;
  std::map<std::pair<int, hipStream_t>, double*> by_stream;
  std::map<std::pair<int, hipStream_t>, Workspace> workspaces;
  std::vector<void*> retired;  // outgrown workspaces, never freed
};

ScratchRegistry& registry() {
  // Leaked on purpose: device memory lives until process exit and the
  // registry must outlive any static destructor that might still launch.
  static ScratchRegistry* instance = new ScratchRegistry();
  return *instance;
}

}  // namespace

hipError_t reduce_partials_for_stream(hipStream_t stream, double** out) {
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
  void* base = nullptr;
  status = hipMalloc(&base, sizeof(double) * kReduceMaxBlocks);
  if (status != hipSuccess) return status;
  reg.by_stream.emplace(key, static_cast<double*>(base));
  *out = static_cast<double*>(base);
  return hipSuccess;
}

hipError_t workspace_for_stream(hipStream_t stream, std::size_t bytes,
                                void** out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  ScratchRegistry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  Workspace& ws = reg.workspaces[std::make_pair(device, stream)];
  if (ws.bytes < bytes) {
    const std::size_t grow = ws.bytes * 2 > bytes ? ws.bytes * 2 : bytes;
    void* fresh = nullptr;
    status = hipMalloc(&fresh, grow);
    if (status != hipSuccess) return status;
    if (ws.ptr != nullptr) reg.retired.push_back(ws.ptr);
    ws.ptr = fresh;
    ws.bytes = grow;
  }
  *out = ws.ptr;
  return hipSuccess;
}

}  // namespace opl
