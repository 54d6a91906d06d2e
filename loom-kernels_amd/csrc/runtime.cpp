// Command runtime and graph capture/replay on HIP streams.
//
// Restates the ownership contract of crates/loom-infer-cuda/src/command/ and
// crates/loom-infer-cuda/src/graph/mod.rs for a C ABI: a queue is one caller
// stream plus one preallocated completion event; bindings are a typed arena of
// device ranges; a scope records one completion event after any number of
// commands; a failed submission poisons the scope and the queue; settling
// in-flight work synchronizes the stream, then the device, and aborts when
// neither proves quiescence.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "loom_internal.hpp"

using loom::fail;

namespace loom {

hipError_t synchronize_stream_or_abort(hipStream_t stream) {
  hipError_t s = hipStreamSynchronize(stream);
  if (s == hipSuccess) return hipSuccess;
  hipError_t d = hipDeviceSynchronize();
  if (d == hipSuccess) return s;
  fprintf(stderr,
          "loom-infer-hip cannot confirm HIP quiescence after stream and device "
          "synchronization failed; aborting to preserve resource safety: stream=%s; "
          "device=%s\n",
          hipGetErrorString(s), hipGetErrorString(d));
  abort();
}

loom_status_t query_device(int device, DeviceInfo *out, loom_error_t *err) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "device", 0, 0, 0, 0, 0.0, e);
  out->device = device;
  out->cus = prop.multiProcessorCount;
  const char *arch = prop.gcnArchName;
  out->gfx950 = arch[0] == 'g' && arch[1] == 'f' && arch[2] == 'x' && arch[3] == '9' &&
                arch[4] == '5' && arch[5] == '0';
  return LOOM_OK;
}

static bool lease_is_readable(const Lease &l) { return !l.vacant; }

loom_status_t resolve_command(loom_command_scope *scope, const loom_handle_t *handles,
                              const OperandSpec *specs, int count, const Lease **out,
                              loom_error_t *err) {
  if (!scope || scope->finished) return fail(err, LOOM_NULL_ARGUMENT, "scope");
  // prepare_command / require_command_capacity (submission.rs:154-184)
  if (scope->submission_error) return fail(err, LOOM_CMD_SCOPE_POISONED);
  if (scope->submitted + 1 > scope->queue->max_commands)
    return fail(err, LOOM_CMD_COMMAND_CAPACITY_EXCEEDED, nullptr, scope->queue->max_commands);
  loom_bindings *b = scope->bindings;
  // validate_binding_request (resolve.rs:856-877)
  for (int i = 0; i < count; ++i)
    if (handles[i].set_id != b->set_id) return fail(err, LOOM_CMD_BINDING_SET_MISMATCH);
  for (int i = 0; i < count; ++i) {
    for (int j = 0; j < i; ++j)
      if (handles[j].slot == handles[i].slot) return fail(err, LOOM_CMD_DUPLICATE_BINDING_SLOT);
    if (handles[i].slot >= b->leases.size())
      return fail(err, LOOM_CMD_BINDING_SLOT_OUT_OF_RANGE, nullptr, handles[i].slot,
                  b->leases.size());
  }
  // ResolveElement::read / write (binding.rs:257-304), in operand order.
  for (int i = 0; i < count; ++i) {
    const Lease &l = b->leases[handles[i].slot];
    int64_t slot = (int64_t)handles[i].slot;
    if (l.vacant) return fail(err, LOOM_CMD_BINDING_SLOT_VACANT, nullptr, slot);
    if (l.dtype != specs[i].dtype) return fail(err, LOOM_CMD_BINDING_TYPE_MISMATCH, nullptr, slot);
    if (specs[i].write && !l.writable)
      return fail(err, LOOM_CMD_BINDING_IS_READ_ONLY, nullptr, slot);
    (void)lease_is_readable;
    out[i] = &l;
  }
  return LOOM_OK;
}

loom_status_t record_launch(loom_command_scope *scope, hipError_t launch_status,
                            loom_error_t *err) {
  // record_cuda_submission / record_failed_cuda_submission (submission.rs:211-238)
  if (scope->submitted >= scope->queue->max_commands ||
      scope->queue->retained != scope->submitted) {
    fprintf(stderr,
            "loom-infer-hip detected an internal command-accounting violation after GPU "
            "submission; aborting to preserve resource safety\n");
    abort();
  }
  scope->queue->retained += 1;
  scope->submitted += 1;
  if (launch_status != hipSuccess) {
    scope->queue->poisoned = true;
    scope->submission_error = launch_status;
    return fail(err, LOOM_CMD_DRIVER, "launch", 0, 0, 0, 0, 0.0, launch_status);
  }
  return LOOM_OK;
}

namespace {
__global__ void zero_words_kernel(uint32_t *p, uint64_t n) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}
}  // namespace

loom_status_t queue_workspace(loom_command_queue *q, uint64_t bytes, bool zeroed,
                              uint8_t **out, loom_error_t *err) {
  uint8_t *&buf = zeroed ? q->zeroed : q->scratch;
  uint64_t &have = zeroed ? q->zeroed_bytes : q->scratch_bytes;
  if (bytes <= have && buf) {
    *out = buf;
    return LOOM_OK;
  }
  // The zero-initialised append workspace is sized for every append plan when
  // the queue is created; it never grows.
  if (zeroed)
    return fail(err, LOOM_ENQ_WORKSPACE_NOT_RESERVED, "append validation workspace",
                (int64_t)have, (int64_t)bytes);
  // The split-KV scratch grows to the next 1 MiB multiple, but never while the
  // stream is being captured: an allocation is not a stream operation and
  // would not replay.  Such callers reserve it before capture.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(q->stream, &cap);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "queue workspace", 0, 0, 0, 0, 0.0, e);
  if (cap != hipStreamCaptureStatusNone)
    return fail(err, LOOM_ENQ_WORKSPACE_NOT_RESERVED, "split-KV workspace", (int64_t)have,
                (int64_t)bytes);
  const uint64_t want = std::max<uint64_t>(((bytes + (1u << 20) - 1) >> 20) << 20, 1u << 20);
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(q->device);
  void *p = nullptr;
  e = hipMalloc(&p, want);
  hipSetDevice(prev);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "queue workspace", 0, 0, 0, 0, 0.0, e);
  if (buf) q->retired.push_back(buf);
  buf = (uint8_t *)p;
  have = want;
  *out = buf;
  return LOOM_OK;
}

uint32_t read_device_status(const loom_command_queue *q) {
  uint32_t bits = 0;
  if (!q || !q->status_host) return 0;
  for (int i = 0; i < kStatusWords; ++i) {
    const uint32_t w = __atomic_load_n(&q->status_host[i], __ATOMIC_ACQUIRE);
    if (w) bits |= 1u << i;
  }
  return bits;
}

}  // namespace loom

struct loom_command_completion {
  loom_command_queue *queue = nullptr;
  loom_bindings *bindings = nullptr;
  uint64_t submitted = 0;
  int32_t submission_error = 0;
  int32_t record_error = 0;
  int32_t poll_error = 0;
  bool complete = false;
};

namespace {

// completion.rs:93-125 settle(): returns the reported failure (hip status)
// or 0; `sync_error` receives the fallback synchronization status.
int32_t settle(loom_command_completion *c, int32_t *sync_error) {
  *sync_error = 0;
  if (c->submitted == 0) return c->submission_error;
  hipStream_t st = c->queue->stream;
  int32_t reported = c->submission_error ? c->submission_error
                     : c->record_error   ? c->record_error
                                         : c->poll_error;
  if (reported) {
    *sync_error = loom::synchronize_stream_or_abort(st);
    return reported;
  }
  hipError_t e = hipEventSynchronize(c->queue->completion_event);
  if (e == hipSuccess) return 0;
  *sync_error = loom::synchronize_stream_or_abort(st);
  return e;
}


// The queue's device status words (pinned, mapped host memory, zeroed) and its
// append validation workspace (device memory, zero-filled by a kernel on the
// queue's stream, so every later command on the queue sees it zero).
loom_status_t init_queue_memory(loom_command_queue *q, loom_error_t *err) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(q->stream, &cap);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "stream", 0, 0, 0, 0, 0.0, e);
  const uint64_t ws_bytes = loom::append_workspace_bytes();
  if (cap != hipStreamCaptureStatusNone)
    return fail(err, LOOM_ENQ_WORKSPACE_NOT_RESERVED, "append validation workspace", 0,
                (int64_t)ws_bytes);
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(q->device);
  void *h = nullptr, *d = nullptr, *w = nullptr;
  e = hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocPortable);
  if (e == hipSuccess) {
    memset(h, 0, 64);
    e = hipHostGetDevicePointer(&d, h, 0);
  }
  if (e == hipSuccess) e = hipMalloc(&w, ws_bytes);
  if (e == hipSuccess) {
    const uint64_t words = ws_bytes / 4;
    hipLaunchKernelGGL(loom::zero_words_kernel,
                       dim3((unsigned)std::min<uint64_t>((words + 255) / 256, 1024)), dim3(256), 0,
                       q->stream, (uint32_t *)w, words);
    e = hipGetLastError();
  }
  hipSetDevice(prev);
  q->status_host = (uint32_t *)h;
  q->status_dev = (uint32_t *)d;
  q->zeroed = (uint8_t *)w;
  q->zeroed_bytes = w ? ws_bytes : 0;
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "queue memory", 0, 0, 0, 0, 0.0, e);
  return LOOM_OK;
}

}  // namespace

extern "C" {

// ---- queue ------------------------------------------------------------------
loom_status_t loom_command_queue_new(void *hip_stream, uint64_t max_commands,
                                     loom_command_queue_t **out, loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (max_commands == 0) return fail(err, LOOM_CMD_ZERO_COMMAND_CAPACITY);
  hipStream_t stream = (hipStream_t)hip_stream;
  int device = 0;
  hipError_t e = hipStreamGetDevice(stream, &device);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "stream", 0, 0, 0, 0, 0.0, e);
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(device);
  hipEvent_t ev = nullptr;
  e = hipEventCreateWithFlags(&ev, loom::kCompletionEventFlags);
  hipSetDevice(prev);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "event", 0, 0, 0, 0, 0.0, e);
  auto *q = new loom_command_queue;
  q->id = loom::fresh_id();
  q->stream = stream;
  q->device = device;
  q->completion_event = ev;
  q->max_commands = max_commands;
  loom_status_t rc = init_queue_memory(q, err);
  if (rc) {
    loom_command_queue_free(q);
    return rc;
  }
  *out = q;
  return loom::ok(err);
}

void loom_command_queue_free(loom_command_queue_t *q) {
  if (!q) return;
  // submission.rs:102-118 Drop
  if (q->retained) {
    hipError_t e = loom::synchronize_stream_or_abort(q->stream);
    q->retained = 0;
    if (e != hipSuccess)
      fprintf(stderr,
              "loom-infer-hip command queue synchronized after a stream error during drop: %s\n",
              hipGetErrorString(e));
  }
  if (q->scratch || q->zeroed || !q->retired.empty()) {
    // Commands that used the workspaces may still run (their completion was
    // dropped unsettled only after it synchronized, but a caller may free the
    // queue with work outstanding on a stream it shares with others).
    loom::synchronize_stream_or_abort(q->stream);
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(q->device);
    if (q->scratch) hipFree(q->scratch);
    if (q->zeroed) hipFree(q->zeroed);
    for (void *p : q->retired) hipFree(p);
    hipSetDevice(prev);
  }
  if (q->status_host) hipHostFree(q->status_host);
  hipEventDestroy(q->completion_event);
  if (q->owns_stream) hipStreamDestroy(q->stream);
  delete q;
}

loom_status_t loom_command_queue_reserve_workspace(loom_command_queue_t *q,
                                                   uint64_t scratch_bytes, uint64_t zeroed_bytes,
                                                   loom_error_t *err) {
  if (!q) return fail(err, LOOM_NULL_ARGUMENT, "queue");
  if (q->active) return fail(err, LOOM_CMD_SCOPE_ACTIVE);
  uint8_t *p = nullptr;
  loom_status_t rc = LOOM_OK;
  if (scratch_bytes) rc = loom::queue_workspace(q, scratch_bytes, false, &p, err);
  if (!rc && zeroed_bytes) rc = loom::queue_workspace(q, zeroed_bytes, true, &p, err);
  return rc ? rc : loom::ok(err);
}

uint64_t loom_command_queue_workspace_bytes(const loom_command_queue_t *q) {
  return q ? q->scratch_bytes + q->zeroed_bytes : 0;
}

uint64_t loom_command_queue_max_commands(const loom_command_queue_t *q) {
  return q ? q->max_commands : 0;
}
int loom_command_queue_is_poisoned(const loom_command_queue_t *q) { return q ? q->poisoned : 0; }

loom_status_t loom_command_queue_bindings(loom_command_queue_t *q, uint64_t capacity,
                                          loom_bindings_t **out, loom_error_t *err) {
  if (!q || !out) return fail(err, LOOM_NULL_ARGUMENT, "queue");
  if (capacity == 0) return fail(err, LOOM_CMD_ZERO_BINDING_CAPACITY);
  auto *b = new loom_bindings;
  b->queue_id = q->id;
  b->set_id = loom::fresh_id();
  b->stream = q->stream;
  b->device = q->device;
  b->capacity = capacity;
  b->leases.reserve(capacity);
  *out = b;
  return loom::ok(err);
}

// ---- bindings ---------------------------------------------------------------
void loom_bindings_free(loom_bindings_t *b) { delete b; }
uint64_t loom_bindings_len(const loom_bindings_t *b) { return b ? b->leases.size() : 0; }
uint64_t loom_bindings_capacity(const loom_bindings_t *b) { return b ? b->capacity : 0; }

static uint64_t dtype_size(loom_dtype_t d) {
  switch (d) {
    case LOOM_DTYPE_F32:
    case LOOM_DTYPE_I32: return 4;
    case LOOM_DTYPE_F16:
    case LOOM_DTYPE_BF16: return 2;
    default: return 1;
  }
}

static loom_status_t bind(loom_bindings_t *b, const void *ptr, uint64_t numel,
                          loom_dtype_t dtype, bool writable, loom_handle_t *out,
                          loom_error_t *err) {
  if (!b || !out) return fail(err, LOOM_NULL_ARGUMENT, "bindings");
  if (b->moved) return fail(err, LOOM_CMD_BINDINGS_IN_USE);
  if ((int)dtype < 0 || (int)dtype > LOOM_DTYPE_U8)
    return fail(err, LOOM_UNSUPPORTED_DTYPE, nullptr, dtype);
  // check_buffer (binding.rs:109-125): the allocation belongs to the stream's device.
  if (ptr) {
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, ptr);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(err, LOOM_CMD_BUFFER_CONTEXT_MISMATCH, nullptr, -1, b->device);
    }
    if (attr.type != hipMemoryTypeDevice || attr.device != b->device)
      return fail(err, LOOM_CMD_BUFFER_CONTEXT_MISMATCH, nullptr,
                  attr.type == hipMemoryTypeDevice ? attr.device : -1, b->device);
  } else if (numel != 0) {
    return fail(err, LOOM_NULL_ARGUMENT, "device_ptr");
  }
  // reserve_slot (binding.rs:127-135)
  if (b->leases.size() == b->capacity)
    return fail(err, LOOM_CMD_BINDING_CAPACITY_EXCEEDED, nullptr, b->capacity);
  // Rust's move semantics make aliased writable leases impossible; here the
  // byte ranges are checked instead.
  const uintptr_t lo = (uintptr_t)ptr, hi = lo + numel * dtype_size(dtype);
  for (size_t i = 0; i < b->leases.size(); ++i) {
    const loom::Lease &l = b->leases[i];
    if (l.vacant || !(writable || l.writable)) continue;
    uintptr_t llo = l.ptr, lhi = l.ptr + l.numel * dtype_size(l.dtype);
    if (lo < lhi && llo < hi) return fail(err, LOOM_CMD_ALIASED_BINDING, nullptr, (int64_t)i);
  }
  loom::Lease l;
  l.ptr = lo;
  l.numel = numel;
  l.dtype = dtype;
  l.writable = writable;
  b->leases.push_back(l);
  out->set_id = b->set_id;
  out->slot = b->leases.size() - 1;
  return loom::ok(err);
}

loom_status_t loom_bindings_bind_read(loom_bindings_t *b, const void *ptr, uint64_t numel,
                                      loom_dtype_t dtype, loom_handle_t *out,
                                      loom_error_t *err) {
  return bind(b, ptr, numel, dtype, false, out, err);
}

loom_status_t loom_bindings_bind_read_write(loom_bindings_t *b, void *ptr, uint64_t numel,
                                            loom_dtype_t dtype, loom_handle_t *out,
                                            loom_error_t *err) {
  return bind(b, ptr, numel, dtype, true, out, err);
}

loom_status_t loom_bindings_take_read_write(loom_bindings_t *b, loom_handle_t h, void **ptr,
                                            uint64_t *numel, loom_error_t *err) {
  if (!b) return fail(err, LOOM_NULL_ARGUMENT, "bindings");
  if (b->moved) return fail(err, LOOM_CMD_BINDINGS_IN_USE);
  // binding.rs:93-107 and the macro's __take_read_write (:230-252)
  if (h.set_id != b->set_id) return fail(err, LOOM_CMD_BINDING_SET_MISMATCH);
  if (h.slot >= b->leases.size())
    return fail(err, LOOM_CMD_BINDING_SLOT_OUT_OF_RANGE, nullptr, h.slot, b->leases.size());
  loom::Lease &l = b->leases[h.slot];
  if (l.vacant) return fail(err, LOOM_CMD_BINDING_SLOT_VACANT, nullptr, h.slot);
  if (!l.writable) return fail(err, LOOM_CMD_BINDING_IS_READ_ONLY, nullptr, h.slot);
  if (ptr) *ptr = (void *)l.ptr;
  if (numel) *numel = l.numel;
  l.vacant = true;
  return loom::ok(err);
}

// ---- scope ------------------------------------------------------------------
loom_status_t loom_command_queue_begin(loom_command_queue_t *q, loom_bindings_t *b,
                                       loom_command_scope_t **out, loom_error_t *err) {
  if (!q || !b || !out) return fail(err, LOOM_NULL_ARGUMENT, "queue");
  // submission.rs:73-99
  if (q->active) return fail(err, LOOM_CMD_SCOPE_ACTIVE);
  if (q->poisoned) return fail(err, LOOM_CMD_QUEUE_POISONED);
  if (b->moved) return fail(err, LOOM_CMD_BINDINGS_IN_USE);
  if (b->queue_id != q->id || b->stream != q->stream || b->device != q->device)
    return fail(err, LOOM_CMD_BINDINGS_QUEUE_MISMATCH);
  if (q->retained) {
    q->poisoned = true;
    return fail(err, LOOM_CMD_QUEUE_POISONED);
  }
  auto *s = new loom_command_scope;
  s->queue = q;
  s->bindings = b;
  s->scope_id = loom::fresh_id();
  b->moved = true;
  q->active = true;
  *out = s;
  return loom::ok(err);
}

uint64_t loom_command_scope_submitted(const loom_command_scope_t *s) {
  return s ? s->submitted : 0;
}

loom_status_t loom_command_scope_finish(loom_command_scope_t *s, loom_command_completion_t **out,
                                        loom_error_t *err) {
  if (!s || !out || s->capturing) return fail(err, LOOM_NULL_ARGUMENT, "scope");
  // submission.rs:131-151
  loom_command_queue *q = s->queue;
  int32_t record_error = 0;
  if (s->submitted > 0 && !s->submission_error) {
    hipError_t e = hipEventRecord(q->completion_event, q->stream);
    if (e != hipSuccess) record_error = e;
  }
  auto *c = new loom_command_completion;
  c->queue = q;
  c->bindings = s->bindings;
  c->submitted = s->submitted;
  c->submission_error = s->submission_error;
  c->record_error = record_error;
  s->finished = true;
  delete s;
  *out = c;
  return loom::ok(err);
}

void loom_command_scope_free(loom_command_scope_t *s) {
  if (!s) return;
  // submission.rs:286-316 Drop of an unfinished scope
  loom_command_queue *q = s->queue;
  if (s->submitted > 0) {
    hipError_t e = loom::synchronize_stream_or_abort(q->stream);
    if (s->submission_error || e != hipSuccess) q->poisoned = true;
  } else if (s->submission_error) {
    q->poisoned = true;
  }
  q->retained = 0;
  q->active = false;
  if (s->bindings) delete s->bindings;  // the bindings moved into the scope drop with it
  delete s;
}

// ---- completion -------------------------------------------------------------
uint64_t loom_command_completion_submitted(const loom_command_completion_t *c) {
  return c ? c->submitted : 0;
}

loom_status_t loom_command_completion_is_complete(loom_command_completion_t *c, int *complete,
                                                  loom_error_t *err) {
  if (!c || !complete) return fail(err, LOOM_NULL_ARGUMENT, "completion");
  // completion.rs:37-60
  int32_t e = c->submission_error ? c->submission_error
              : c->record_error   ? c->record_error
                                  : c->poll_error;
  if (e) return fail(err, LOOM_CMD_DRIVER, "completion", 0, 0, 0, 0, 0.0, e);
  if (c->submitted == 0) {
    *complete = 1;
    return loom::ok(err);
  }
  hipError_t q = hipEventQuery(c->queue->completion_event);
  if (q == hipSuccess) {
    *complete = 1;
  } else if (q == hipErrorNotReady) {
    *complete = 0;
  } else {
    c->poll_error = q;
    return fail(err, LOOM_CMD_DRIVER, "completion", 0, 0, 0, 0, 0.0, q);
  }
  return loom::ok(err);
}

loom_status_t loom_command_completion_wait(loom_command_completion_t *c, loom_bindings_t **out,
                                           loom_error_t *err) {
  if (!c) return fail(err, LOOM_NULL_ARGUMENT, "completion");
  // completion.rs:62-83
  int32_t sync_error = 0;
  int32_t failure = settle(c, &sync_error);
  loom_command_queue *q = c->queue;
  q->retained = 0;
  q->active = false;
  loom_bindings *b = c->bindings;
  const bool ran = c->submitted > 0;
  delete c;
  // A settled command whose kernels reported a device status did not complete
  // as specified: the completion fails and poisons the queue.
  const uint32_t status = !failure && ran ? loom::read_device_status(q) : 0;
  if (!failure && !status) {
    b->moved = false;
    if (out) *out = b;
    return loom::ok(err);
  }
  q->poisoned = true;
  delete b;
  if (out) *out = nullptr;
  if (status) return fail(err, LOOM_CMD_DEVICE_STATUS, "completion", status);
  return fail(err, LOOM_CMD_DRIVER, "completion", 0, 0, 0, 0, 0.0, failure);
}

void loom_command_completion_free(loom_command_completion_t *c) {
  if (!c) return;
  // completion.rs:128-144 Drop
  int32_t sync_error = 0;
  int32_t failure = settle(c, &sync_error);
  c->queue->retained = 0;
  c->queue->active = false;
  if (failure || (c->submitted > 0 && loom::read_device_status(c->queue)))
    c->queue->poisoned = true;
  delete c->bindings;
  delete c;
}

}  // extern "C"

// ---- graphs -------------------------------------------------------------------
struct loom_graph_queue {
  loom_command_queue *queue = nullptr;  // owns its private stream
  bool consumed = false;
};

struct loom_captured_graph {
  hipGraph_t graph = nullptr;
  loom_command_queue *queue = nullptr;  // private stream + event, moved from the graph queue
  loom_bindings *bindings = nullptr;
  uint64_t commands = 0;
};

// One captured kernel node, replayed with hipLaunchKernel: the function, its
// launch shape and the node's own copy of the kernel arguments (owned by the
// hipGraph, which the executable keeps).
struct ReplayLaunch {
  const void *func = nullptr;
  dim3 grid, block;
  void **params = nullptr;
  unsigned shared = 0;
};

struct loom_graph_exec {
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  // The captured graph as a chain of kernel nodes (empty if it is not one)
  // and how launch() replays it (LOOM_GRAPH_REPLAY_*).
  std::vector<ReplayLaunch> chain;
  int32_t replay_mode = LOOM_GRAPH_REPLAY_HIP_GRAPH_LAUNCH;
  loom_command_queue *queue = nullptr;
  hipEvent_t completion_event = nullptr;
  loom_bindings *bindings = nullptr;
  uint64_t commands = 0;
  uint64_t launches = 0;
  bool in_flight = false;
  int32_t record_error = 0;
  int32_t poll_error = 0;
  uint32_t device_status = 0;  // status words read at the last settlement
  bool poisoned = false;
};

struct loom_graph_completion {
  loom_graph_exec *exec = nullptr;
  uint64_t launch_index = 0;
  bool settled = false;
};

namespace {

// settle_exec's failure value when the replay completed but its kernels
// reported a device status (not a hipError_t).
constexpr int32_t kDeviceStatusFailure = -1;

// graph/mod.rs:418-446 settle_in_flight.
int32_t settle_exec(loom_graph_exec *x, int32_t *sync_error) {
  *sync_error = 0;
  if (!x->in_flight) return 0;
  int32_t failure = 0;
  if (x->record_error) {
    failure = x->record_error;
    *sync_error = loom::synchronize_stream_or_abort(x->queue->stream);
  } else if (x->poll_error) {
    failure = x->poll_error;
    *sync_error = loom::synchronize_stream_or_abort(x->queue->stream);
  } else {
    hipError_t e = hipEventSynchronize(x->completion_event);
    if (e != hipSuccess) {
      failure = e;
      *sync_error = loom::synchronize_stream_or_abort(x->queue->stream);
    } else {
      x->device_status = loom::read_device_status(x->queue);
      if (x->device_status) failure = kDeviceStatusFailure;
    }
  }
  x->in_flight = false;
  x->record_error = 0;
  x->poll_error = 0;
  return failure;
}

loom_status_t settlement_error(loom_error_t *err, const char *op, int32_t failure,
                               int32_t sync_error, uint32_t device_status = 0) {
  if (failure == kDeviceStatusFailure)
    return fail(err, LOOM_CMD_DEVICE_STATUS, op, device_status);
  if (sync_error)
    return fail(err, LOOM_GRAPH_SETTLEMENT, op, sync_error, 0, 0, 0, 0.0, failure);
  return fail(err, LOOM_GRAPH_DRIVER, op, 0, 0, 0, 0, 0.0, failure);
}

__global__ void grid_probe_kernel(int *p, int v) {
  if (p) p[blockIdx.x] = v;
}

// How this HIP runtime reports a captured kernel node: its grid in workgroups
// (1) or in work-items (2), with kernelParams an array of pointers to the
// argument values; 0 when the node does not read back as expected (the
// executable then replays with hipGraphLaunch only).  Probed once per process
// by capturing (never running) a launch of known shape and arguments.
int probe_node_grid_semantics() {
  int probed = 0;
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return probed;
  int *const marker = reinterpret_cast<int *>(uintptr_t{0x7a5e1000});  // never dereferenced
  hipGraph_t g = nullptr;
  if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    hipLaunchKernelGGL(grid_probe_kernel, dim3(3), dim3(64), 0, s, marker, 7);
    (void)hipStreamEndCapture(s, &g);
  }
  if (g) {
    hipGraphNode_t node = nullptr;
    size_t n = 1;
    hipKernelNodeParams p{};
    if (hipGraphGetNodes(g, &node, &n) == hipSuccess && n == 1 &&
        hipGraphKernelNodeGetParams(node, &p) == hipSuccess && p.blockDim.x == 64 &&
        p.blockDim.y == 1 && p.blockDim.z == 1 && p.kernelParams && !p.extra &&
        p.kernelParams[0] && p.kernelParams[1] &&
        *static_cast<int **>(p.kernelParams[0]) == marker &&
        *static_cast<int *>(p.kernelParams[1]) == 7) {
      if (p.gridDim.x == 3 && p.gridDim.y == 1 && p.gridDim.z == 1) probed = 1;
      else if (p.gridDim.x == 3 * 64 && p.gridDim.y == 1 && p.gridDim.z == 1) probed = 2;
    }
    hipGraphDestroy(g);
  }
  (void)hipGetLastError();
  hipStreamDestroy(s);
  return probed;
}
// Probed once per process (a function-local static: initialised once even
// when several threads instantiate graphs at the same time).
int node_grid_semantics() {
  static const int probed = probe_node_grid_semantics();
  return probed;
}

// The graph's nodes as a chain of kernel nodes in dependency order (each node
// depends on exactly the one before it), or false.
bool kernel_chain(hipGraph_t g, std::vector<ReplayLaunch> *out) {
  const int sem = node_grid_semantics();
  if (!sem) return false;
  size_t n = 0;
  if (hipGraphGetNodes(g, nullptr, &n) != hipSuccess || n == 0) return false;
  std::vector<hipGraphNode_t> nodes(n), order;
  if (hipGraphGetNodes(g, nodes.data(), &n) != hipSuccess) return false;
  std::vector<hipGraphNode_t> dep(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    hipGraphNodeType t;
    if (hipGraphNodeGetType(nodes[i], &t) != hipSuccess || t != hipGraphNodeTypeKernel) return false;
    size_t nd = 0;
    if (hipGraphNodeGetDependencies(nodes[i], nullptr, &nd) != hipSuccess || nd > 1) return false;
    if (nd == 1 && hipGraphNodeGetDependencies(nodes[i], &dep[i], &nd) != hipSuccess) return false;
  }
  hipGraphNode_t prev = nullptr;
  for (size_t k = 0; k < n; ++k) {  // follow the chain from its root
    size_t found = n;
    for (size_t i = 0; i < n; ++i)
      if (dep[i] == prev && std::find(order.begin(), order.end(), nodes[i]) == order.end()) {
        if (found != n) return false;  // two nodes after one: not a chain
        found = i;
      }
    if (found == n) return false;
    order.push_back(nodes[found]);
    prev = nodes[found];
  }
  std::vector<ReplayLaunch> chain;
  for (hipGraphNode_t node : order) {
    hipKernelNodeParams p{};
    if (hipGraphKernelNodeGetParams(node, &p) != hipSuccess || !p.func || !p.kernelParams || p.extra)
      return false;
    ReplayLaunch l;
    l.func = p.func;
    l.block = p.blockDim;
    l.grid = p.gridDim;
    if (sem == 2) {
      if (!p.blockDim.x || !p.blockDim.y || !p.blockDim.z || p.gridDim.x % p.blockDim.x ||
          p.gridDim.y % p.blockDim.y || p.gridDim.z % p.blockDim.z)
        return false;
      l.grid = dim3(p.gridDim.x / p.blockDim.x, p.gridDim.y / p.blockDim.y, p.gridDim.z / p.blockDim.z);
    }
    l.params = p.kernelParams;
    l.shared = p.sharedMemBytes;
    chain.push_back(l);
  }
  *out = std::move(chain);
  return true;
}

void destroy_exec(loom_graph_exec *x) {
  if (x->exec) hipGraphExecDestroy(x->exec);
  if (x->graph) hipGraphDestroy(x->graph);
  if (x->completion_event) hipEventDestroy(x->completion_event);
  if (x->queue) {
    x->queue->retained = 0;
    loom_command_queue_free(x->queue);
  }
  x->exec = nullptr;
  x->graph = nullptr;
  x->completion_event = nullptr;
  x->queue = nullptr;
}

}  // namespace

extern "C" {

loom_status_t loom_graph_queue_new(int device, uint64_t max_commands, loom_graph_queue_t **out,
                                   loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  int prev = 0;
  hipGetDevice(&prev);
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "device", 0, 0, 0, 0, 0.0, e);
  hipStream_t stream = nullptr;
  // Default stream priority; non-blocking so the legacy default stream never
  // joins a capture.
  e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
  hipSetDevice(prev);
  if (e != hipSuccess) return fail(err, LOOM_CMD_DRIVER, "stream", 0, 0, 0, 0, 0.0, e);
  loom_command_queue *q = nullptr;
  loom_status_t rc = loom_command_queue_new(stream, max_commands, &q, err);
  if (rc) {
    hipStreamDestroy(stream);
    return rc;
  }
  q->owns_stream = true;
  auto *g = new loom_graph_queue;
  g->queue = q;
  *out = g;
  return loom::ok(err);
}

void loom_graph_queue_free(loom_graph_queue_t *g) {
  if (!g) return;
  if (g->queue) loom_command_queue_free(g->queue);
  delete g;
}

loom_status_t loom_graph_queue_bindings(loom_graph_queue_t *g, uint64_t capacity,
                                        loom_bindings_t **out, loom_error_t *err) {
  if (!g || g->consumed) return fail(err, LOOM_NULL_ARGUMENT, "graph_queue");
  return loom_command_queue_bindings(g->queue, capacity, out, err);
}

loom_status_t loom_graph_queue_reserve_workspace(loom_graph_queue_t *g, uint64_t scratch_bytes,
                                                 uint64_t zeroed_bytes, loom_error_t *err) {
  if (!g || g->consumed) return fail(err, LOOM_NULL_ARGUMENT, "graph_queue");
  return loom_command_queue_reserve_workspace(g->queue, scratch_bytes, zeroed_bytes, err);
}

uint64_t loom_graph_queue_workspace_bytes(const loom_graph_queue_t *g) {
  return g && g->queue ? loom_command_queue_workspace_bytes(g->queue) : 0;
}

loom_status_t loom_graph_queue_begin_capture(loom_graph_queue_t *g, loom_bindings_t *b,
                                             loom_command_scope_t **out, loom_error_t *err) {
  if (!g || g->consumed || !b || !out) return fail(err, LOOM_NULL_ARGUMENT, "graph_queue");
  // graph/mod.rs:54-70: input readiness by one device synchronization.
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(g->queue->device);
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    fprintf(stderr,
            "loom-infer-hip cannot establish HIP graph input readiness: %s; aborting before "
            "releasing caller-supplied allocations\n",
            hipGetErrorString(e));
    abort();
  }
  hipSetDevice(prev);
  loom_command_scope_t *s = nullptr;
  loom_status_t rc = loom_command_queue_begin(g->queue, b, &s, err);
  if (rc) return rc;
  e = hipStreamBeginCapture(g->queue->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    s->bindings->moved = false;
    s->bindings = nullptr;
    g->queue->active = false;
    delete s;
    return fail(err, LOOM_GRAPH_DRIVER, "capture begin", 0, 0, 0, 0, 0.0, e);
  }
  s->capturing = true;
  g->consumed = true;
  *out = s;
  return loom::ok(err);
}

loom_status_t loom_graph_queue_end_capture(loom_graph_queue_t *g, loom_command_scope_t *s,
                                           loom_captured_graph_t **out, loom_error_t *err) {
  if (!g || !s || !out || !s->capturing || s->queue != g->queue)
    return fail(err, LOOM_NULL_ARGUMENT, "scope");
  // graph/mod.rs:82-131 capture_checked after the closure returns.
  loom_command_queue *q = g->queue;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(q->stream, &graph);
  loom_bindings *bindings = s->bindings;
  const uint64_t submitted = s->submitted;
  const int32_t sub_err = s->submission_error;
  delete s;
  q->retained = 0;
  q->active = false;
  g->queue = nullptr;
  auto fail_all = [&](loom_status_t rc) {
    if (graph) hipGraphDestroy(graph);
    delete bindings;
    loom_command_queue_free(q);
    return rc;
  };
  if (e != hipSuccess) return fail_all(fail(err, LOOM_GRAPH_DRIVER, "capture end", 0, 0, 0, 0, 0.0, e));
  if (!graph) return fail_all(fail(err, LOOM_GRAPH_CAPTURE_INVALIDATED));
  if (sub_err) return fail_all(fail(err, LOOM_CMD_DRIVER, "launch", 0, 0, 0, 0, 0.0, sub_err));
  if (submitted == 0) return fail_all(fail(err, LOOM_GRAPH_EMPTY_CAPTURE));
  auto *c = new loom_captured_graph;
  c->graph = graph;
  c->queue = q;
  c->bindings = bindings;
  c->commands = submitted;
  *out = c;
  return loom::ok(err);
}

uint64_t loom_captured_graph_commands(const loom_captured_graph_t *c) {
  return c ? c->commands : 0;
}

void loom_captured_graph_free(loom_captured_graph_t *c) {
  if (!c) return;
  if (c->graph) hipGraphDestroy(c->graph);
  delete c->bindings;
  loom_command_queue_free(c->queue);
  delete c;
}

loom_status_t loom_captured_graph_instantiate(loom_captured_graph_t *c, loom_graph_exec_t **out,
                                              loom_error_t *err) {
  if (!c || !out) return fail(err, LOOM_NULL_ARGUMENT, "graph");
  // graph/mod.rs:183-206
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(c->queue->device);
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, loom::kCompletionEventFlags);
  hipGraphExec_t exec = nullptr;
  if (e == hipSuccess) e = hipGraphInstantiate(&exec, c->graph, nullptr, nullptr, 0);
  hipSetDevice(prev);
  if (e != hipSuccess) {
    if (ev) hipEventDestroy(ev);
    loom_captured_graph_free(c);
    return fail(err, LOOM_GRAPH_DRIVER, "instantiate", 0, 0, 0, 0, 0.0, e);
  }
  if (!exec) {
    hipEventDestroy(ev);
    loom_captured_graph_free(c);
    return fail(err, LOOM_GRAPH_NULL_EXECUTABLE_HANDLE);
  }
  auto *x = new loom_graph_exec;
  x->exec = exec;
  x->graph = c->graph;
  if (kernel_chain(c->graph, &x->chain)) x->replay_mode = LOOM_GRAPH_REPLAY_KERNEL_NODES;
  x->queue = c->queue;
  x->completion_event = ev;
  x->bindings = c->bindings;
  x->commands = c->commands;
  delete c;
  *out = x;
  return loom::ok(err);
}

uint64_t loom_graph_exec_commands(const loom_graph_exec_t *x) { return x ? x->commands : 0; }

int32_t loom_graph_exec_replay_mode(const loom_graph_exec_t *x) { return x ? x->replay_mode : 0; }

loom_status_t loom_graph_exec_set_replay_mode(loom_graph_exec_t *x, int32_t mode,
                                              loom_error_t *err) {
  if (!x) return fail(err, LOOM_NULL_ARGUMENT, "exec");
  if (x->in_flight) return fail(err, LOOM_GRAPH_REPLAY_IN_FLIGHT);
  if (mode == LOOM_GRAPH_REPLAY_HIP_GRAPH_LAUNCH ||
      (mode == LOOM_GRAPH_REPLAY_KERNEL_NODES && !x->chain.empty())) {
    x->replay_mode = mode;
    return loom::ok(err);
  }
  return fail(err, LOOM_PLAN_INVALID_OPTION, "replay_mode", mode);
}
uint64_t loom_graph_exec_launches(const loom_graph_exec_t *x) { return x ? x->launches : 0; }

loom_status_t loom_graph_exec_launch(loom_graph_exec_t *x, loom_graph_completion_t **out,
                                     loom_error_t *err) {
  if (!x || !out) return fail(err, LOOM_NULL_ARGUMENT, "exec");
  // graph/mod.rs:249-293
  if (x->poisoned) return fail(err, LOOM_GRAPH_EXECUTION_POISONED);
  if (x->in_flight) return fail(err, LOOM_GRAPH_REPLAY_IN_FLIGHT);
  if (x->launches == UINT64_MAX) return fail(err, LOOM_GRAPH_LAUNCH_COUNT_EXHAUSTED);
  x->in_flight = true;
  x->record_error = 0;
  x->poll_error = 0;
  hipError_t e = hipSuccess;
  if (x->replay_mode == LOOM_GRAPH_REPLAY_KERNEL_NODES) {
    // The captured kernel nodes with their captured arguments, in order, on
    // the replay stream: the same work as hipGraphLaunch of this chain, at
    // the cost of one kernel launch per node.
    for (const ReplayLaunch &l : x->chain) {
      e = hipLaunchKernel(l.func, l.grid, l.block, l.params, l.shared, x->queue->stream);
      if (e != hipSuccess) break;
    }
  } else {
    e = hipGraphLaunch(x->exec, x->queue->stream);
  }
  if (e != hipSuccess) {
    hipError_t sync = loom::synchronize_stream_or_abort(x->queue->stream);
    x->in_flight = false;
    x->poisoned = true;
    return settlement_error(err, "launch", e, sync);
  }
  x->launches += 1;
  hipError_t r = hipEventRecord(x->completion_event, x->queue->stream);
  if (r != hipSuccess) x->record_error = r;
  auto *c = new loom_graph_completion;
  c->exec = x;
  c->launch_index = x->launches;
  *out = c;
  return loom::ok(err);
}

loom_status_t loom_graph_exec_measure_launch_ms(loom_graph_exec_t *x, void *start, void *end,
                                                float *ms, loom_error_t *err) {
  if (!x || !start || !end || !ms) return fail(err, LOOM_NULL_ARGUMENT, "exec");
  // graph/mod.rs:301-323
  hipError_t e = hipEventRecord((hipEvent_t)start, x->queue->stream);
  if (e == hipErrorInvalidHandle || e == hipErrorInvalidResourceHandle)
    return fail(err, LOOM_GRAPH_TIMING_EVENT_CONTEXT_MISMATCH);
  if (e != hipSuccess) return fail(err, LOOM_GRAPH_DRIVER, "timing start event record", 0, 0, 0, 0, 0.0, e);
  loom_graph_completion_t *c = nullptr;
  loom_status_t rc = loom_graph_exec_launch(x, &c, err);
  if (rc) return rc;
  e = hipEventRecord((hipEvent_t)end, x->queue->stream);
  if (e != hipSuccess) {
    loom_graph_completion_free(c);
    return fail(err, LOOM_GRAPH_DRIVER, "timing end event record", 0, 0, 0, 0, 0.0, e);
  }
  rc = loom_graph_completion_wait(c, err);
  if (rc) return rc;
  // The end event follows the completion event on the stream.
  e = hipEventSynchronize((hipEvent_t)end);
  if (e != hipSuccess) return fail(err, LOOM_GRAPH_DRIVER, "timing end event wait", 0, 0, 0, 0, 0.0, e);
  e = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end);
  if (e != hipSuccess) return fail(err, LOOM_GRAPH_DRIVER, "timing event elapsed query", 0, 0, 0, 0, 0.0, e);
  return loom::ok(err);
}

loom_status_t loom_graph_exec_into_bindings(loom_graph_exec_t *x, loom_bindings_t **out,
                                            loom_error_t *err) {
  if (!x || !out) return fail(err, LOOM_NULL_ARGUMENT, "exec");
  // graph/mod.rs:326-339
  int32_t sync = 0;
  int32_t failure = settle_exec(x, &sync);
  if (failure) {
    x->poisoned = true;
    return settlement_error(err, "completion", failure, sync, x->device_status);
  }
  loom_bindings *b = x->bindings;
  x->bindings = nullptr;
  destroy_exec(x);
  delete x;
  b->moved = false;
  *out = b;
  return loom::ok(err);
}

void loom_graph_exec_free(loom_graph_exec_t *x) {
  if (!x) return;
  int32_t sync = 0;
  if (settle_exec(x, &sync)) x->poisoned = true;
  destroy_exec(x);
  delete x->bindings;
  delete x;
}

uint64_t loom_graph_completion_launch_index(const loom_graph_completion_t *c) {
  return c ? c->launch_index : 0;
}

loom_status_t loom_graph_completion_is_complete(loom_graph_completion_t *c, int *complete,
                                                loom_error_t *err) {
  if (!c || !complete) return fail(err, LOOM_NULL_ARGUMENT, "completion");
  loom_graph_exec *x = c->exec;
  if (x->record_error)
    return fail(err, LOOM_GRAPH_DRIVER, "completion event record", 0, 0, 0, 0, 0.0, x->record_error);
  if (x->poll_error)
    return fail(err, LOOM_GRAPH_DRIVER, "completion event query", 0, 0, 0, 0, 0.0, x->poll_error);
  hipError_t q = hipEventQuery(x->completion_event);
  if (q == hipSuccess) {
    *complete = 1;
  } else if (q == hipErrorNotReady) {
    *complete = 0;
  } else {
    x->poll_error = q;
    return fail(err, LOOM_GRAPH_DRIVER, "completion event query", 0, 0, 0, 0, 0.0, q);
  }
  return loom::ok(err);
}

loom_status_t loom_graph_completion_wait(loom_graph_completion_t *c, loom_error_t *err) {
  if (!c) return fail(err, LOOM_NULL_ARGUMENT, "completion");
  loom_graph_exec *x = c->exec;
  delete c;
  int32_t sync = 0;
  int32_t failure = settle_exec(x, &sync);
  if (!failure) return loom::ok(err);
  x->poisoned = true;
  return settlement_error(err, "completion", failure, sync, x->device_status);
}

void loom_graph_completion_free(loom_graph_completion_t *c) {
  if (!c) return;
  int32_t sync = 0;
  if (settle_exec(c->exec, &sync)) c->exec->poisoned = true;
  delete c;
}

}  // extern "C"
