// device.h — device handle, scoped device selection, scratch buffers and the
// exception-to-status guard used by every extern "C" entry point.
#pragma once

#include <hip/hip_runtime.h>

#include <exception>
#include <new>
#include <string>

#include "common.h"

struct pgd_dev {
  int ordinal;
  hipStream_t stream = nullptr;
  explicit pgd_dev(int ord) : ordinal(ord) {
    int prev = 0;
    PGD_HIP(hipGetDevice(&prev));
    PGD_HIP(hipSetDevice(ord));
    // default priority, non-blocking w.r.t. the legacy null stream
    PGD_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    (void)hipSetDevice(prev);
  }
  ~pgd_dev() {
    if (stream) {
      int prev = 0;
      (void)hipGetDevice(&prev);
      (void)hipSetDevice(ordinal);
      (void)hipStreamSynchronize(stream);
      (void)hipStreamDestroy(stream);
      (void)hipSetDevice(prev);
    }
  }
};

namespace pgd {

// Makes dev current for the scope; restores the previous device after.
struct DeviceScope {
  int prev = -1;
  explicit DeviceScope(const pgd_dev* dev) {
    PGD_CHECK(dev, kErrArg, "null device");
    PGD_HIP(hipGetDevice(&prev));
    if (prev != dev->ordinal) PGD_HIP(hipSetDevice(dev->ordinal));
    else prev = -1;
  }
  ~DeviceScope() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

// Owning device buffer (freed after the stream it was used on drains).
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  explicit DevBuf(size_t n) : bytes(n) {
    hipError_t e = hipMalloc(&p, n ? n : 1);
    if (e != hipSuccess) throw Error{kErrAlloc, std::string("hipMalloc: ") + hipGetErrorString(e)};
  }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) {
    o.p = nullptr;
    o.bytes = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      reset();
      p = o.p;
      bytes = o.bytes;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  ~DevBuf() { reset(); }
  template <class T>
  T* as() const {
    return reinterpret_cast<T*>(p);
  }
};

template <class F>
int guard(F&& f) {
  try {
    f();
    return kOk;
  } catch (const Error& e) {
    set_error(e.msg);
    return e.code;
  } catch (const std::bad_alloc&) {
    set_error("host allocation failed");
    return kErrAlloc;
  } catch (const std::exception& e) {
    set_error(e.what());
    return kErrState;
  } catch (...) {
    set_error("unknown error");
    return kErrState;
  }
}

}  // namespace pgd
