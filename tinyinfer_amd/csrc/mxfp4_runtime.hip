// Library-wide host state: device properties, tuning options and the split-K
// workspaces.  Everything here may be reached from several host threads at
// once (the C ABI is callable from any thread), so every piece of shared state
// is either initialised once under std::call_once or guarded by a mutex, and
// option values are atomics.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "mxfp4_launch.hpp"

namespace tinyinfer {

// ------------------------------------------------------------ device info

namespace {

constexpr int kMaxDevices = 64;
std::once_flag g_dev_once[kMaxDevices];
DeviceInfo g_dev_info[kMaxDevices];

}  // namespace

DeviceInfo device_info() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DeviceInfo{};
  std::call_once(g_dev_once[dev], [dev] {
    hipDeviceProp_t prop;
    DeviceInfo d;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      d.cus = prop.multiProcessorCount;
      d.lds_per_block = (int64_t)prop.sharedMemPerBlock;
      d.gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    } else {
      (void)hipGetLastError();
    }
    g_dev_info[dev] = d;
  });
  return g_dev_info[dev];
}

// ------------------------------------------------------------ options

namespace {

// name, default, then the accepted values: a range [lo, hi], or for `pow2`
// only 1, 2 and 4 (and 0 = choose automatically)
struct OptSpec {
  const char* name;
  int dflt;
  int lo;
  int hi;
  bool pow2;
};

constexpr OptSpec kSpecs[kOptCount] = {
    {"TINYINFER_ROWSTREAM", 1, 0, 1, false},
    {"TINYINFER_ROWPAIR", 1, 0, 1, false},
    {"TINYINFER_TILE", 1, 0, 1, false},
    {"TINYINFER_TILE_GU", 1, 0, 1, false},
    {"TINYINFER_ROW_SPLIT_GATEUP", 0, 0, 4, true},
    {"TINYINFER_ROW_SPLIT_DOWN", 0, 0, 4, true},
    {"TINYINFER_GEMM_RING", 1, 0, 1, false},
    {"TINYINFER_RING_KSPLIT", 0, 0, 32, false},
    {"TINYINFER_RING_WR_GU", 4, 2, 4, true},
    {"TINYINFER_RING_NW_GU", 8, 4, 8, false},
    {"TINYINFER_RING_WR_DN", 4, 2, 4, true},
    {"TINYINFER_RING_NW_DN", 8, 4, 8, false},
    {"TINYINFER_SKINNY_NW", 0, 0, 8, false},
    {"TINYINFER_STREAM_SPU_GU", 0, 0, 3, false},
    {"TINYINFER_STREAM_SPU_DN", 0, 0, 4, false},
    {"TINYINFER_STREAM_XREG", 1, 0, 1, false},
    {"TINYINFER_WORKSPACE_MB", 512, 0, 1 << 20, false},
    {"TINYINFER_DECODE_SPIN", 1 << 20, 0, 1 << 30, false},
    {"TINYINFER_RING_TAIL", 1, 0, 1, false},
};

bool valid_value(const OptSpec& s, int v) {
  if (v < s.lo || v > s.hi) return false;
  if (s.pow2 && v != 0 && v != 1 && v != 2 && v != 4) return false;
  // waves per workgroup: 4 or 8 (0 = automatic for the skinny kernels)
  if (std::strstr(s.name, "_NW") && v != 0 && v != 4 && v != 8) return false;
  return true;
}

std::once_flag g_opt_once;
std::atomic<int> g_opt[kOptCount];

void load_options() {
  std::call_once(g_opt_once, [] {
    for (int i = 0; i < kOptCount; ++i) {
      int v = kSpecs[i].dflt;
      if (const char* e = std::getenv(kSpecs[i].name)) {
        char* end = nullptr;
        const long p = std::strtol(e, &end, 10);
        if (end != e && *end == '\0' && p >= -(1L << 30) && p <= (1L << 30) && valid_value(kSpecs[i], (int)p))
          v = (int)p;
      }
      g_opt[i].store(v, std::memory_order_relaxed);
    }
  });
}

int find_option(const char* name) {
  if (!name) return -1;
  for (int i = 0; i < kOptCount; ++i)
    if (std::strcmp(kSpecs[i].name, name) == 0) return i;
  return -1;
}

}  // namespace

int option(Opt o) {
  load_options();
  return g_opt[o].load(std::memory_order_relaxed);
}

bool set_option(const char* name, int value) {
  load_options();
  const int i = find_option(name);
  if (i < 0 || !valid_value(kSpecs[i], value)) return false;
  g_opt[i].store(value, std::memory_order_relaxed);
  return true;
}

bool get_option(const char* name, int* value) {
  load_options();
  const int i = find_option(name);
  if (i < 0 || !value) return false;
  *value = g_opt[i].load(std::memory_order_relaxed);
  return true;
}

// ------------------------------------------------------------ workspaces

// One fp32 buffer per (device, stream), grown on demand up to the limit
// TINYINFER_WORKSPACE_MB (per buffer).  A buffer that is replaced by a larger
// one is retired, not freed: kernels still queued, and graphs captured with
// it, hold its address.  Growth is refused during graph capture (allocation
// is not a capturable operation).  release_workspaces() frees them all.
namespace {

struct WsState {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> bufs;
  std::vector<std::pair<int, void*>> retired;
  size_t held = 0;
};

WsState& ws_state() {
  static WsState* s = new WsState;   // never destroyed: may be used during static destruction
  return *s;
}

}  // namespace

size_t workspace_limit() { return (size_t)option(kOptWorkspaceMB) << 20; }

float* gemm_split_workspace(size_t bytes, hipStream_t st) {
  if (bytes > workspace_limit()) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  WsState& s = ws_state();
  std::lock_guard<std::mutex> lock(s.mu);
  auto& b = s.bufs[{dev, st}];
  if (b.second >= bytes) return static_cast<float*>(b.first);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  size_t want = (bytes + (64u << 20) - 1) & ~size_t((64u << 20) - 1);
  if (want > workspace_limit()) want = bytes;
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (b.first) s.retired.push_back({dev, b.first});
  s.held += want;
  b = {p, want};
  return static_cast<float*>(p);
}

size_t workspace_bytes_held() {
  WsState& s = ws_state();
  std::lock_guard<std::mutex> lock(s.mu);
  return s.held;
}

hipError_t release_workspaces() {
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return hipErrorNoDevice;
  WsState& s = ws_state();
  std::lock_guard<std::mutex> lock(s.mu);
  // every device that holds a buffer finishes its queued work first
  std::vector<int> devs;
  for (auto& kv : s.bufs) devs.push_back(kv.first.first);
  for (auto& r : s.retired) devs.push_back(r.first);
  hipError_t err = hipSuccess;
  for (int d : devs) {
    if (hipSetDevice(d) != hipSuccess || hipDeviceSynchronize() != hipSuccess) err = hipErrorUnknown;
  }
  for (auto& kv : s.bufs) {
    if (hipSetDevice(kv.first.first) == hipSuccess && kv.second.first) (void)hipFree(kv.second.first);
  }
  for (auto& r : s.retired) {
    if (hipSetDevice(r.first) == hipSuccess) (void)hipFree(r.second);
  }
  s.bufs.clear();
  s.retired.clear();
  s.held = 0;
  (void)hipSetDevice(cur);
  (void)hipGetLastError();
  return err;
}

}  // namespace tinyinfer
