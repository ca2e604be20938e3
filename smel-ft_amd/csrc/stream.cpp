// Layer weight stager: chunked host -> device copies on copy streams with event ordering (no host synchronisation).
// Replaces the upload of smel/stream.py:53-79 (per-tensor non_blocking copies, a worker thread blocked on the copy
// event, record_stream for the compute stream).
#include "../../include/smel_stream.h"
#include "abi_util.h"

extern "C" int smel_event_create(hipEvent_t* out) {
  SMEL_REQUIRE(out, SMEL_EINVAL, "event_create: null output");
  const hipError_t e = hipEventCreateWithFlags(out, hipEventDisableTiming);
  SMEL_REQUIRE(e == hipSuccess, (int)e, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int smel_event_destroy(hipEvent_t ev) {
  if (!ev) return 0;
  const hipError_t e = hipEventDestroy(ev);
  SMEL_REQUIRE(e == hipSuccess, (int)e, "hipEventDestroy: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int smel_event_record(hipEvent_t ev, hipStream_t stream) {
  SMEL_REQUIRE(ev, SMEL_EINVAL, "event_record: null event");
  const hipError_t e = hipEventRecord(ev, stream);
  SMEL_REQUIRE(e == hipSuccess, (int)e, "hipEventRecord: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int smel_stream_wait(hipStream_t stream, hipEvent_t ev) {
  SMEL_REQUIRE(ev, SMEL_EINVAL, "stream_wait: null event");
  const hipError_t e = hipStreamWaitEvent(stream, ev, 0);
  SMEL_REQUIRE(e == hipSuccess, (int)e, "hipStreamWaitEvent: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int smel_h2d_regions(const smel_h2d_region* regions, int32_t n, int64_t chunk_bytes,
                                const hipStream_t* streams, const hipEvent_t* done, int32_t n_streams,
                                hipEvent_t after) {
  SMEL_REQUIRE(n >= 0 && (n == 0 || regions), SMEL_EINVAL, "h2d_regions: bad region list");
  SMEL_REQUIRE(chunk_bytes > 0, SMEL_EINVAL, "h2d_regions: chunk_bytes %lld", (long long)chunk_bytes);
  SMEL_REQUIRE(n_streams >= 1 && n_streams <= 8 && streams && done, SMEL_EINVAL,
               "h2d_regions: %d copy streams (1..8, with a done event each)", n_streams);
  for (int32_t i = 0; i < n_streams; ++i) SMEL_REQUIRE(done[i], SMEL_EINVAL, "h2d_regions: null done event %d", i);
  for (int32_t i = 0; i < n; ++i)
    SMEL_REQUIRE(regions[i].bytes >= 0 && (regions[i].bytes == 0 || (regions[i].dst && regions[i].src)),
                 SMEL_EINVAL, "h2d_regions: region %d has a null pointer or a negative size", i);
  hipError_t e;
  if (after) {
    for (int32_t i = 0; i < n_streams; ++i) {
      e = hipStreamWaitEvent(streams[i], after, 0);
      SMEL_REQUIRE(e == hipSuccess, (int)e, "hipStreamWaitEvent: %s", hipGetErrorString(e));
    }
  }
  int32_t s = 0;
  for (int32_t i = 0; i < n; ++i) {
    const char* src = static_cast<const char*>(regions[i].src);
    char* dst = static_cast<char*>(regions[i].dst);
    for (int64_t off = 0; off < regions[i].bytes; off += chunk_bytes) {
      const int64_t nb = regions[i].bytes - off < chunk_bytes ? regions[i].bytes - off : chunk_bytes;
      e = hipMemcpyAsync(dst + off, src + off, (size_t)nb, hipMemcpyHostToDevice, streams[s]);
      SMEL_REQUIRE(e == hipSuccess, (int)e, "hipMemcpyAsync (region %d, offset %lld): %s", i, (long long)off,
                   hipGetErrorString(e));
      s = (s + 1) % n_streams;
    }
  }
  for (int32_t i = 0; i < n_streams; ++i) {
    e = hipEventRecord(done[i], streams[i]);
    SMEL_REQUIRE(e == hipSuccess, (int)e, "hipEventRecord: %s", hipGetErrorString(e));
  }
  return 0;
}
