// Shared host-side plumbing of the EXL3 library: error convention, HIP checks, buffer and pack handles.
//
// Error convention (include/engine.h:4-5 of the reference): int functions return 0 / -1, pointer functions NULL, and
// the message is kept per thread for ne_last_error().
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/ijah_exl3.h"

namespace ijah {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

std::string strfmt(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void set_last_error(const std::string &msg);

#define IJ_CHECK(cond, ...)                                                  \
  do {                                                                       \
    if (!(cond)) throw ::ijah::Error(::ijah::strfmt(__VA_ARGS__));           \
  } while (0)
#define IJ_HIP(call)                                                                                        \
  do {                                                                                                      \
    hipError_t e_ = (call);                                                                                 \
    if (e_ != hipSuccess) throw ::ijah::Error(::ijah::strfmt("%s: %s", #call, hipGetErrorString(e_)));      \
  } while (0)

// Runs f, converting exceptions into -1 + last error (reference core/engine.hpp:36-44).
template <typename F>
int c_call(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return -1;
  }
}

// The library's stream: every entry point enqueues here; synchronous entry points wait on it.
hipStream_t stream();
void ensure_device();
bool device_available();  // a HIP device is visible (no throw)

}  // namespace ijah

// Device memory handle. The reference's buffers are unified memory; here the bytes live in HBM and `host` is a lazily
// allocated mirror that ne_buf_contents() refreshes (device -> host) and ne_buf_flush() writes back.
struct ne_buf {
  void *dev = nullptr;
  uint64_t size = 0;
  void *host = nullptr;
  bool owned = true;     // ne_free releases the memory
  bool readonly = false; // pack-owned tensor copies refuse ne_upload (reference core/capi.mm:65)
  bool external = false; // dev memory not owned by this handle (a view)
  ~ne_buf();
};
