// C-ABI plumbing: error strings, version, and the cold-tier host API
// (pinned host pool, asynchronous host-to-device prefetch, streams, events).
#include "rfsn_common.h"

#include <mutex>

namespace rfsn {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
  set_error(msg);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RFSN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return RFSN_OK;
}

static int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(RFSN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return RFSN_OK;
}

}  // namespace rfsn

using namespace rfsn;

extern "C" int rfsn_abi_version(void) { return RFSN_ABI_VERSION; }

extern "C" const char* rfsn_last_error(void) { return g_last_error.c_str(); }

extern "C" int rfsn_host_alloc(size_t bytes, void** ptr_out) {
  RFSN_REQUIRE(ptr_out != nullptr, "host_alloc: null output pointer");
  *ptr_out = nullptr;
  if (bytes == 0) return RFSN_OK;
  return hip_status(hipHostMalloc(ptr_out, bytes, hipHostMallocDefault), "hipHostMalloc");
}

extern "C" int rfsn_host_free(void* ptr) {
  if (ptr == nullptr) return RFSN_OK;
  return hip_status(hipHostFree(ptr), "hipHostFree");
}

extern "C" int rfsn_prefetch_h2d(const rfsn_copy* copies, int32_t count, void* stream) {
  RFSN_REQUIRE(count >= 0 && (count == 0 || copies != nullptr), "prefetch_h2d: bad copy list");
  for (int32_t i = 0; i < count; ++i) {
    if (copies[i].bytes == 0) continue;
    RFSN_REQUIRE(copies[i].dst_dev && copies[i].src_host, "prefetch_h2d: null pointer in copy list");
    int st = hip_status(hipMemcpyAsync(copies[i].dst_dev, copies[i].src_host, copies[i].bytes,
                                       hipMemcpyHostToDevice, (hipStream_t)stream),
                        "hipMemcpyAsync");
    if (st) return st;
  }
  return RFSN_OK;
}

extern "C" int rfsn_stream_create(void** out) {
  RFSN_REQUIRE(out != nullptr, "stream_create: null output");
  hipStream_t s = nullptr;
  int st = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  *out = (void*)s;
  return st;
}

extern "C" int rfsn_stream_destroy(void* s) {
  if (s == nullptr) return RFSN_OK;
  return hip_status(hipStreamDestroy((hipStream_t)s), "hipStreamDestroy");
}

extern "C" int rfsn_event_create(void** out) {
  RFSN_REQUIRE(out != nullptr, "event_create: null output");
  hipEvent_t e = nullptr;
  int st = hip_status(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags");
  *out = (void*)e;
  return st;
}

extern "C" int rfsn_event_destroy(void* e) {
  if (e == nullptr) return RFSN_OK;
  return hip_status(hipEventDestroy((hipEvent_t)e), "hipEventDestroy");
}

extern "C" int rfsn_event_record(void* e, void* s) {
  RFSN_REQUIRE(e != nullptr, "event_record: null event");
  return hip_status(hipEventRecord((hipEvent_t)e, (hipStream_t)s), "hipEventRecord");
}

extern "C" int rfsn_stream_wait_event(void* s, void* e) {
  RFSN_REQUIRE(e != nullptr, "stream_wait_event: null event");
  return hip_status(hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0), "hipStreamWaitEvent");
}

extern "C" int rfsn_event_synchronize(void* e) {
  RFSN_REQUIRE(e != nullptr, "event_synchronize: null event");
  return hip_status(hipEventSynchronize((hipEvent_t)e), "hipEventSynchronize");
}

extern "C" int rfsn_stream_query(void* s) {
  const hipError_t r = hipStreamQuery((hipStream_t)s);
  if (r == hipSuccess) return 1;
  if (r == hipErrorNotReady) return 0;
  return hip_status(r, "hipStreamQuery");
}

extern "C" int rfsn_event_query(void* e) {
  RFSN_REQUIRE(e != nullptr, "event_query: null event");
  const hipError_t r = hipEventQuery((hipEvent_t)e);
  if (r == hipSuccess) return 1;
  if (r == hipErrorNotReady) return 0;
  return hip_status(r, "hipEventQuery");
}
