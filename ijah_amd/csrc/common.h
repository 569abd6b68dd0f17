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

// the caller's pending mirror writes of b pushed to the device (not while the library stream is captured), then
// b's device address
void mirror_push(const struct ::ne_buf *b);
void *ne_dev(const struct ::ne_buf *b);

}  // namespace ijah

// Device memory handle. The reference's buffers are unified memory; here the bytes live in HBM and `host` is a lazily
// allocated mirror that ne_buf_contents() refreshes (device -> host). `snap` holds what the mirror last received from
// the device: before any library call uses the buffer, the bytes the caller changed in the mirror since then (and
// only those) go to the device (ne_dev), so the reference's write-through-numpy-then-run pattern works, and an
// untouched mirror never overwrites newer device data.
struct ne_buf {
  void *dev = nullptr;
  uint64_t size = 0;
  void *host = nullptr;
  void *snap = nullptr;
  bool owned = true;     // ne_free releases the memory
  bool readonly = false; // pack-owned tensor copies refuse ne_upload (reference core/capi.mm:65)
  bool external = false; // dev memory not owned by this handle (a view)
  ~ne_buf();
};
