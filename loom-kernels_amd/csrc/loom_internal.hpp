// Internal types shared by the host layer of libloom_infer_hip.so.
// Not part of the ABI: include/loom_infer_hip.h is.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "loom_infer_hip.h"

namespace loom {

constexpr uint64_t kHeadDim = LOOM_HEAD_DIM;
constexpr uint64_t kPageSize = LOOM_PAGE_SIZE;
constexpr uint64_t kStateWidth = LOOM_PARTIAL_STATE_WIDTH;

// ---- errors ---------------------------------------------------------------
// Fills `err` (if any) with the variant payload and its Display text and
// returns `code`.
loom_status_t fail(loom_error_t *err, loom_status_t code, const char *operand = nullptr,
                   int64_t f0 = 0, int64_t f1 = 0, int64_t f2 = 0, int64_t f3 = 0,
                   double value = 0.0, int32_t hip_status = 0);
inline loom_status_t ok(loom_error_t *err) {
  if (err) {
    err->code = LOOM_OK;
    err->message[0] = 0;
  }
  return LOOM_OK;
}

uint64_t fresh_id();

// ---- command runtime --------------------------------------------------------
struct Lease {
  uintptr_t ptr = 0;
  uint64_t numel = 0;
  loom_dtype_t dtype = LOOM_DTYPE_U8;
  bool writable = false;
  bool vacant = false;
};

}  // namespace loom

struct loom_bindings {
  uint64_t queue_id = 0;
  uint64_t set_id = 0;
  hipStream_t stream = nullptr;
  int device = 0;
  std::vector<loom::Lease> leases;
  uint64_t capacity = 0;
  bool moved = false;  // held by a live scope, completion or graph
};

struct loom_command_queue {
  uint64_t id = 0;
  hipStream_t stream = nullptr;
  int device = 0;
  hipEvent_t completion_event = nullptr;
  uint64_t max_commands = 0;
  uint64_t retained = 0;  // commands submitted and not yet settled
  bool poisoned = false;
  bool owns_stream = false;
  bool active = false;  // a scope or completion borrows the queue (Rust's &mut)
  // Device workspaces owned by the queue for the enqueue forms that take the
  // reference's argument structs (no workspace operand).  `scratch` holds
  // split-KV states (no initialisation needed; grown on demand outside
  // stream capture, or reserved ahead).  `zeroed` holds the append
  // validation state: allocated and zero-filled when the queue is created
  // (its size is the same for every append plan), it carries the append
  // kernels' epoch from one command to the next; all zeros is a valid
  // starting state.  Commands on one queue are ordered on its one stream, so
  // they reuse the buffers without races.  A buffer that grows is retired,
  // not freed, until the queue is dropped: commands already submitted may
  // use it.
  uint8_t *scratch = nullptr;
  uint64_t scratch_bytes = 0;
  uint8_t *zeroed = nullptr;
  uint64_t zeroed_bytes = 0;
  std::vector<void *> retired;
  // Device-written status words in pinned, mapped host memory (kStatusWords).
  // A kernel that could not finish a command as specified (see DeviceStatus)
  // stores 1 into one of them; settling the completion (or the graph replay)
  // reads them and reports LOOM_CMD_DEVICE_STATUS, poisoning the queue.
  uint32_t *status_host = nullptr;
  uint32_t *status_dev = nullptr;
};

struct loom_command_scope {
  loom_command_queue *queue = nullptr;
  loom_bindings *bindings = nullptr;
  uint64_t scope_id = 0;
  uint64_t submitted = 0;
  int32_t submission_error = 0;  // hipError_t of a failed launch, 0 if none
  bool finished = false;
  bool capturing = false;
};

namespace loom {

// Resolution of one command's operands (command/resolve.rs:843-885 plus the
// element-type and access checks of binding.rs:257-304).
struct OperandSpec {
  const char *name;
  loom_dtype_t dtype;
  bool write;
};

// Checks scope health and capacity (submission.rs:154-184) and resolves the
// handles; on success `out[i]` points at the leases in the scope's bindings.
loom_status_t resolve_command(loom_command_scope *scope, const loom_handle_t *handles,
                              const OperandSpec *specs, int count, const Lease **out,
                              loom_error_t *err);
// Records one kernel submission (or a failed one, which poisons the scope and
// the queue: submission.rs:211-279).
loom_status_t record_launch(loom_command_scope *scope, hipError_t launch_status,
                            loom_error_t *err);

// submission.rs / completion.rs:165-182: synchronize the stream, then the
// device; abort when neither proves quiescence.
hipError_t synchronize_stream_or_abort(hipStream_t stream);

// The queue's workspace of at least `bytes` (allocated or grown on first
// need; see loom_command_queue).  `zeroed` selects the zero-initialised
// buffer.
loom_status_t queue_workspace(loom_command_queue *queue, uint64_t bytes, bool zeroed,
                              uint8_t **out, loom_error_t *err);

// Device status words of a command queue (loom_command_queue::status_*).
enum DeviceStatus : int {
  // An append token workgroup gave up waiting for the validation verdicts and
  // wrote nothing: a valid command may be applied only in part.
  kStatusAppendVerdictWait = 0,
  // The append's epoch handover gave up waiting for every workgroup to start:
  // the validation workspace is marked broken (it must be zeroed again).
  kStatusAppendHandover = 1,
  // An append command found its validation workspace marked broken and wrote
  // nothing.
  kStatusAppendRefused = 2,
  kStatusWords = 4
};
// Bytes of the append validation workspace (one size for every plan).
uint64_t append_workspace_bytes();
// Reads and reports the queue's device status words (0 when all are clear);
// the returned value has bit i set for word i.
uint32_t read_device_status(const loom_command_queue *queue);

// Flags of the completion events of command queues and graph executables.
// They only order host waits (nothing waits on them from another stream),
// and after a wait the host reads nothing but the device status words, which
// kernels write with system-scope stores (through to host memory).  Outputs
// are device memory, read through stream-ordered copies that carry their own
// fences.  So the events skip the system-scope release an event record does
// by default (an L2 writeback): −1.5 µs on a one-kernel graph replay, from
// the launch call to its completion event.
constexpr unsigned kCompletionEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;

// Device facts used by providers.
struct DeviceInfo {
  int device = 0;
  int cus = 0;
  bool gfx950 = false;
};
loom_status_t query_device(int device, DeviceInfo *out, loom_error_t *err);

}  // namespace loom
