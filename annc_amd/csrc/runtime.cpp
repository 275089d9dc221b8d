// runtime.cpp -- errors, per-stream state and host-operand staging.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <algorithm>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace annc {
namespace {

thread_local std::string g_last_error;

struct StreamState {
  int* status = nullptr;
};

std::mutex g_mu;
// Keyed by (device, stream): the NULL stream exists once per device.
std::map<std::pair<int, hipStream_t>, StreamState> g_streams;

// Workspace per (device, stream) and calling thread: threads that enqueue on
// one stream interleave their launches, so each call's partials need a
// buffer no other thread writes.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
thread_local std::map<std::pair<int, hipStream_t>, Workspace> t_workspaces;
// Outgrown workspaces, kept until the process ends: a HIP graph captured with
// one replays with its address (guarded by g_mu).
std::vector<void*> g_retired;
// The synchronous XLA/TF entries run on a library stream of the calling
// thread: concurrent callers never share a stream, so their kernels cannot
// interleave.
thread_local std::map<int, hipStream_t> t_lib_streams;

int current_device() {
  int dev = 0;
  (void)hipGetDevice(&dev);
  return dev;
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
  if (code == ANNC_OK) {
    g_last_error.clear();
    return code;
  }
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int* stream_status(hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  StreamState& st = g_streams[{current_device(), stream}];
  if (!st.status) {
    if (hipMalloc(&st.status, sizeof(int)) != hipSuccess) {
      st.status = nullptr;
      return nullptr;
    }
    if (hipMemset(st.status, 0, sizeof(int)) != hipSuccess) return nullptr;
  }
  return st.status;
}

void* stream_workspace(hipStream_t stream, size_t bytes) {
  Workspace& w = t_workspaces[{current_device(), stream}];
  if (bytes <= w.bytes) return w.ptr;
  // No allocation while the stream is being captured into a graph (hipMalloc
  // would break the capture): callers then take a path that needs no
  // workspace
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (stream && hipStreamIsCapturing(stream, &cap) == hipSuccess &&
      cap != hipStreamCaptureStatusNone)
    return nullptr;
  // At least twice the outgrown size, so the retired buffers together stay
  // below the live one.
  const size_t want = std::max({size_t(1) << 20, bytes + bytes / 4, 2 * w.bytes});
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (w.ptr) {
    std::lock_guard<std::mutex> lock(g_mu);
    g_retired.push_back(w.ptr);
  }
  w.ptr = p;
  w.bytes = want;
  return p;
}

hipStream_t lib_stream() {
  const int dev = current_device();
  auto it = t_lib_streams.find(dev);
  if (it != t_lib_streams.end()) return it->second;
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) s = nullptr;
  t_lib_streams[dev] = s;
  return s;
}

bool is_device_ptr(const void* p) {
  if (!p) return false;
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // unregistered host memory: not an error here
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

int read_i64(const void* src, int64_t count, int64_t* dst) {
  if (count <= 0) return ANNC_OK;
  if (!src) return set_error(ANNC_INVALID_ARGUMENT, "null shape operand");
  if (is_device_ptr(src)) {
    ANNC_HIP_TRY(hipMemcpy(dst, src, sizeof(int64_t) * count, hipMemcpyDeviceToHost));
  } else {
    std::memcpy(dst, src, sizeof(int64_t) * count);
  }
  return ANNC_OK;
}

namespace {
// Pinned bounce buffers of the calling thread, one per device (kept until
// the process ends: releasing them at thread exit could run after the HIP
// runtime has shut down).
thread_local std::map<int, char*> t_pinned;
}  // namespace

int read_back(hipStream_t stream, std::initializer_list<ReadBack> items) {
  size_t total = 0;
  for (const ReadBack& it : items) total += (it.bytes + 15) & ~size_t(15);
  if (total > kReadBackBytes)
    return set_error(ANNC_INTERNAL, "read-back of %zu bytes above the %zu-byte buffer", total,
                     kReadBackBytes);
  char*& pin = t_pinned[current_device()];
  if (!pin) {
    ANNC_HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&pin), kReadBackBytes,
                               hipHostMallocDefault));
  }
  size_t off = 0;
  for (const ReadBack& it : items) {
    ANNC_HIP_TRY(hipMemcpyAsync(pin + off, it.src, it.bytes, hipMemcpyDeviceToHost, stream));
    off += (it.bytes + 15) & ~size_t(15);
  }
  ANNC_HIP_TRY(hipStreamSynchronize(stream));
  off = 0;
  for (const ReadBack& it : items) {
    std::memcpy(it.dst, pin + off, it.bytes);
    off += (it.bytes + 15) & ~size_t(15);
  }
  return ANNC_OK;
}

namespace {
// Grow-only device staging memory of the calling thread (one per device).
// A Staging object carves its buffers from it and releases them when it is
// destroyed, after its stream has drained, so the next synchronous call of
// the thread reuses the memory with no hipMalloc/hipFree (hipFree would
// synchronise the whole device).
struct Arena {
  char* base = nullptr;
  size_t size = 0, used = 0, want = 0;
  int depth = 0;  // live Staging objects of the thread on this device
};
thread_local std::map<int, Arena> t_arenas;
constexpr size_t kStagingAlign = 256;
}  // namespace

Staging::Staging(hipStream_t stream) : stream_(stream) { ++t_arenas[current_device()].depth; }

Staging::~Staging() {
  // Work of a call that returned without finish() may still use the memory:
  // drain the stream before handing it back.
  if (!finished_) (void)hipStreamSynchronize(stream_);
  for (void* p : owned_) (void)hipFree(p);
  Arena& ar = t_arenas[current_device()];
  if (--ar.depth > 0) return;  // an enclosing Staging still holds its buffers
  ar.used = 0;
  if (ar.want > ar.size) {  // grow for the next call: nothing is in flight now
    (void)hipStreamSynchronize(stream_);
    if (ar.base) (void)hipFree(ar.base);
    ar.base = nullptr;
    ar.size = 0;
    const size_t grow = ar.want + ar.want / 4;
    if (hipMalloc(reinterpret_cast<void**>(&ar.base), grow) == hipSuccess)
      ar.size = grow;
    else
      ar.base = nullptr;
    ar.want = 0;
  }
}

void* Staging::alloc(size_t bytes) {
  if (bytes == 0) bytes = 4;
  const size_t rounded = (bytes + kStagingAlign - 1) / kStagingAlign * kStagingAlign;
  Arena& ar = t_arenas[current_device()];
  if (ar.base && ar.used + rounded <= ar.size) {
    void* p = ar.base + ar.used;
    ar.used += rounded;
    return p;
  }
  ar.want = std::max(ar.want, ar.used + rounded);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    status_ = set_error(ANNC_RESOURCE_EXHAUSTED, "hipMalloc(%zu) failed: %s", bytes,
                        hipGetErrorString(e));
    return nullptr;
  }
  owned_.push_back(p);
  return p;
}

const void* Staging::in(const void* p, size_t bytes) {
  if (!p || status_ != ANNC_OK) return p;
  if (is_device_ptr(p)) return p;
  void* d = alloc(bytes);
  if (!d) return nullptr;
  hipError_t e = hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, stream_);
  if (e != hipSuccess) {
    status_ = set_error(ANNC_INTERNAL, "host-to-device copy failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  return d;
}

void* Staging::out(void* p, size_t bytes) {
  if (!p || status_ != ANNC_OK) return p;
  if (is_device_ptr(p)) return p;
  void* d = alloc(bytes);
  if (!d) return nullptr;
  pending_.push_back({p, d, bytes});
  return d;
}

void* Staging::scratch(size_t bytes) {
  if (status_ != ANNC_OK) return nullptr;
  return alloc(bytes);
}

int Staging::finish() {
  if (status_ != ANNC_OK) return status_;
  for (const Pending& q : pending_) {
    hipError_t e = hipMemcpyAsync(q.host, q.dev, q.bytes, hipMemcpyDeviceToHost, stream_);
    if (e != hipSuccess)
      return status_ = set_error(ANNC_INTERNAL, "device-to-host copy failed: %s",
                                 hipGetErrorString(e));
  }
  hipError_t e = hipStreamSynchronize(stream_);
  if (e != hipSuccess)
    return status_ = set_error(ANNC_INTERNAL, "stream synchronize failed: %s",
                               hipGetErrorString(e));
  pending_.clear();
  finished_ = true;
  return ANNC_OK;
}

}  // namespace annc

extern "C" {

const char* annc_hip_last_error(void) { return annc::g_last_error.c_str(); }

const char* annc_hip_version(void) { return "annc-hip 0.1.0 (gfx950)"; }

int annc_hip_stream_status(void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* st = annc::stream_status(s);
  if (!st) return annc::set_error(ANNC_INTERNAL, "status word allocation failed");
  int host = 0;
  const int rc = annc::read_back(s, {{&host, st, sizeof(int)}});
  if (rc != ANNC_OK) return rc;
  if (host != 0) {
    ANNC_HIP_TRY(hipMemset(st, 0, sizeof(int)));
    return annc::set_error(ANNC_INVALID_ARGUMENT,
                           "row id out of range of the embedding table in a kernel on this stream");
  }
  annc::clear_error();
  return ANNC_OK;
}

}  // extern "C"
