// Library-wide C-ABI pieces: error reporting and build identification.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace kf {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return KF_OK;
  set_error("%s: launch failed: %s (%s)", what, hipGetErrorName(err), hipGetErrorString(err));
  if (err == hipErrorOutOfMemory) return KF_ERR_OUT_OF_MEMORY;
  if (err == hipErrorLaunchOutOfResources || err == hipErrorInvalidConfiguration)
    return KF_ERR_OUT_OF_RESOURCES;
  return KF_ERR_LAUNCH;
}

}  // namespace kf

extern "C" int kf_abi_version(void) { return 5; }

extern "C" const char* kf_build_target(void) { return "gfx950"; }

// The build passes the digest of the sources it compiled (kernelforge/build.py).
#ifndef KF_SOURCE_DIGEST
#define KF_SOURCE_DIGEST "unknown"
#endif
extern "C" const char* kf_source_digest(void) { return KF_SOURCE_DIGEST; }

extern "C" const char* kf_last_error(void) { return kf::g_last_error; }

extern "C" int kf_stream_capture_id(void* stream, unsigned long long* id) {
  if (id == nullptr) {
    kf::set_error("stream_capture_id: null output");
    return KF_ERR_INVALID_ARGUMENT;
  }
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long seq = 0;
  const hipError_t err = hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &seq);
  if (err != hipSuccess) {
    kf::set_error("stream_capture_id: %s", hipGetErrorName(err));
    return KF_ERR_LAUNCH;
  }
  *id = status == hipStreamCaptureStatusActive ? seq : 0;
  return KF_OK;
}
