/* C-ABI of the layer weight stager (libsmel_moe.so): host -> device copies of a layer's tensors from pinned host
 * memory on copy streams, ordered against the compute stream with events (no host synchronisation).
 *
 * Same conventions as smel_moe.h (0 on success, SMEL_E* or hipError_t codes, message in smel_last_error()).
 * The reference uploads a layer in a worker thread, one `tensor.to(device, non_blocking=True)` per tensor on a side
 * stream, then blocks that thread on the copy's event (smel/stream.py:53-69) and makes the compute stream safe with
 * `record_stream` (:71-79). Here the copies are chunked over one or more copy streams (each a separate DMA queue),
 * every copy stream first waits for the event that says the destination slot is free, and records its own done
 * event, which the compute stream waits on before the layer's first kernel.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smel_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  void* dst;        /* device memory */
  const void* src;  /* pinned host memory (e.g. torch.empty(..., pin_memory=True)) */
  int64_t bytes;
} smel_h2d_region;

/* Events without timing (hipEventDisableTiming), for ordering only. */
int smel_event_create(hipEvent_t* out);
int smel_event_destroy(hipEvent_t ev);
/* hipEventRecord(ev, stream) / hipStreamWaitEvent(stream, ev): the ordering steps around a stage. */
int smel_event_record(hipEvent_t ev, hipStream_t stream);
int smel_stream_wait(hipStream_t stream, hipEvent_t ev);

/* Copy n regions host -> device. The regions are cut into chunks of at most chunk_bytes (> 0), dealt to the
 * n_streams copy streams in turn; each stream first waits `after` (may be null: the destination is free already),
 * then copies its chunks in order and records done[i]. Replaces the per-tensor upload of `_StreamingSource._upload`
 * smel/stream.py:53-69 (without its worker-thread `ev.synchronize()`: the caller waits on done[] on the compute
 * stream instead). n_streams in [1, 8]. */
int smel_h2d_regions(const smel_h2d_region* regions, int32_t n, int64_t chunk_bytes, const hipStream_t* streams,
                     const hipEvent_t* done, int32_t n_streams, hipEvent_t after);

#ifdef __cplusplus
}
#endif
