// common.h -- shared runtime helpers of libannc_hip (errors, streams,
// per-stream device scratch, staging of host operands for the synchronous
// XLA / TF entry points).
#pragma once

#include <hip/hip_runtime.h>

#include <initializer_list>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "annc_hip.h"

namespace annc {

// Records `code` and a printf-style message as this thread's last error and
// returns `code`.  ANNC_OK clears the message.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Device status word for `stream` (zeroed on first use).  Kernels OR bit 0
// into it when they meet an out-of-range row id.
int* stream_status(hipStream_t stream);

// Grow-only device scratch owned by the library, one per (device, stream,
// calling thread).  An outgrown buffer is kept until the process ends (graphs
// captured with it replay with its address).  nullptr while the stream is
// being captured and the buffer is too small, or when hipMalloc fails.
void* stream_workspace(hipStream_t stream, size_t bytes);

// The library's own stream of the calling thread on the current device
// (default priority), used by the synchronous entry points.
hipStream_t lib_stream();

// True for memory the GPU can address directly (device or managed).
bool is_device_ptr(const void* p);

// Copies `count` int64 values from host or device memory into `dst`.
int read_i64(const void* src, int64_t count, int64_t* dst);

// Small device-to-host reads after the work queued on `stream`: every
// (host dst, device src, bytes) goes through a pinned buffer of the calling
// thread (hipHostMalloc'd once per device, at most kReadBackBytes in all),
// then one synchronisation; a pageable destination would make the runtime
// stage each copy.
struct ReadBack {
  void* dst;
  const void* src;
  size_t bytes;
};
constexpr size_t kReadBackBytes = 64 << 10;
int read_back(hipStream_t stream, std::initializer_list<ReadBack> items);

// Staging for synchronous entry points whose operands may live in host
// memory: inputs are copied to device scratch, outputs are produced in
// device scratch and copied back by finish().  Device operands pass through.
// The scratch comes from a grow-only arena of the calling thread and is
// released when the Staging object is destroyed (after its stream drained).
class Staging {
 public:
  explicit Staging(hipStream_t stream);
  ~Staging();
  Staging(const Staging&) = delete;
  Staging& operator=(const Staging&) = delete;

  // Device view of an input of `bytes` bytes at `p` (NULL stays NULL).
  const void* in(const void* p, size_t bytes);
  // Device buffer for an output that finish() delivers to `p`.
  void* out(void* p, size_t bytes);
  // Device scratch of `bytes` bytes, released with the Staging object.
  void* scratch(size_t bytes);
  // Copies host outputs back and synchronises.  Returns ANNC_OK or an error.
  int finish();
  int status() const { return status_; }
  hipStream_t stream() const { return stream_; }

 private:
  struct Pending {
    void* host;
    void* dev;
    size_t bytes;
  };
  void* alloc(size_t bytes);
  hipStream_t stream_;
  int status_ = ANNC_OK;
  bool finished_ = false;
  std::vector<void*> owned_;
  std::vector<Pending> pending_;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace annc

#define ANNC_HIP_TRY(expr)                                                          \
  do {                                                                              \
    hipError_t annc_e_ = (expr);                                                    \
    if (annc_e_ != hipSuccess)                                                      \
      return ::annc::set_error(ANNC_INTERNAL, "%s failed: %s", #expr,               \
                               hipGetErrorString(annc_e_));                         \
  } while (0)

#define ANNC_REQUIRE(cond, ...)                                                     \
  do {                                                                              \
    if (!(cond)) return ::annc::set_error(ANNC_INVALID_ARGUMENT, __VA_ARGS__);      \
  } while (0)
