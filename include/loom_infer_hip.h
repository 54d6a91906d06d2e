/*
 * loom_infer_hip.h — C ABI of libloom_infer_hip.so, the MI355X (gfx950)
 * implementation of Loom Infer's paged-KV decode path:
 *
 *   fused NeoX RoPE + paged K/V append  ->  paged decode attention
 *   (balanced split over KV pages, then a log2-LSE merge kernel)  ->  hipGraph
 *   fixed-address capture and replay.
 *
 * The ABI mirrors the reference's Rust contract sequence
 *   Spec::new -> Provider::plan_* -> queue.bindings(n) / bind_read /
 *   bind_read_write -> queue.begin -> plan.enqueue_into(scope, args) ->
 *   scope.finish() -> completion.wait() -> take_read_write
 * (crates/loom-infer-cuda/src/attention/decode.rs:1067, :1199, :1452-1487;
 *  crates/loom-infer-cuda/src/rope/mod.rs:628-682, :758, :846, :963-1047;
 *  crates/loom-infer-cuda/src/command/{binding,submission,completion}.rs;
 *  crates/loom-infer-cuda/src/graph/mod.rs).
 *
 * Conventions
 *   - Every function returns a loom_status_t by value and never throws or
 *     aborts across the ABI, except where the reference aborts: a failed
 *     stream AND device synchronization while settling in-flight work
 *     (command/completion.rs:165-182, graph/mod.rs:679-685).
 *   - `err` may be NULL; when given it receives the variant payload and a
 *     human-readable message equal to the reference's Display text.
 *   - Buffers are raw device pointers with an element count and dtype.
 *     Binding a buffer read-write transfers it to the binding set until the
 *     command completion that used it is settled and the caller takes it back.
 *   - No function here allocates device memory except *_new/_load, graph
 *     instantiation, loom_command_queue_reserve_workspace and a
 *     loom_paged_decode_enqueue_bf16 whose split-KV states need more than
 *     the queue's workspace holds, outside stream capture (under capture it
 *     fails with LOOM_ENQ_WORKSPACE_NOT_RESERVED instead); every other
 *     enqueue never allocates.
 */
#ifndef LOOM_INFER_HIP_H
#define LOOM_INFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LOOM_INFER_HIP_ABI_VERSION 1u
#define LOOM_HEAD_DIM 128u                       /* single_decode/mod.rs:8 */
#define LOOM_PAGE_SIZE 16u                       /* paged_decode/mod.rs:9 */
#define LOOM_PARTIAL_STATE_WIDTH 130u            /* single_decode/mod.rs:13 */
#define LOOM_APPEND_MAX_TOKENS 64u               /* paged_append/mod.rs:12 */
/* Bulk explicit-token append (no reference counterpart: the reference caps the
 * explicit contract at 64 tokens; this contract keeps its semantics and lifts
 * the cap for batched multi-token appends). */
#define LOOM_APPEND_MAX_TOKENS_EXTENDED 8192u

/* ------------------------------------------------------------------------ */
/* Status codes.                                                              */
typedef int32_t loom_status_t;
enum {
  LOOM_OK = 0,
  /* ContractError, crates/loom-infer/src/error.rs:6-109 (same order). */
  LOOM_ZERO_DIMENSION = 1,
  LOOM_ELEMENT_COUNT_OVERFLOW = 2,
  LOOM_INVALID_EPSILON = 3,
  LOOM_UNSUPPORTED_HEAD_DIMENSION = 4,
  LOOM_UNSUPPORTED_PAGE_SIZE = 5,
  LOOM_INVALID_HEAD_MAPPING = 6,
  LOOM_INVALID_PARTITION_COUNT = 7,
  LOOM_INVALID_INDPTR_START = 8,
  LOOM_NON_MONOTONIC_INDPTR = 9,
  LOOM_EMPTY_RAGGED_REQUEST = 10,
  LOOM_RAGGED_QUERY_LONGER_THAN_KV = 11,
  LOOM_INVALID_PAGE_INDPTR_START = 12,
  LOOM_NON_MONOTONIC_PAGE_INDPTR = 13,
  LOOM_EMPTY_PAGED_REQUEST = 14,
  LOOM_PAGE_INDEX_OUT_OF_RANGE = 15,
  LOOM_INVALID_LAST_PAGE_LENGTH = 16,
  LOOM_INVALID_ROTARY_DIMENSION = 17,
  LOOM_INVALID_ROPE_SCALE = 18,
  LOOM_INVALID_ROPE_THETA = 19,
  LOOM_NEGATIVE_POSITION_ID = 20,
  LOOM_UNSUPPORTED_APPEND_TOKEN_COUNT = 21,
  LOOM_APPEND_BATCH_INDEX_OUT_OF_RANGE = 22,
  LOOM_APPEND_POSITION_OUT_OF_RANGE = 23,
  LOOM_DUPLICATE_PAGE_APPEND_SLOT = 24,
  LOOM_DUPLICATE_PAGE_APPEND_TOKEN_SLOT = 25,
  LOOM_UNSUPPORTED_DTYPE = 26,
  LOOM_LENGTH_MISMATCH = 27,

  /* CommandError, crates/loom-infer-cuda/src/command/mod.rs:67-107. */
  LOOM_CMD_ZERO_COMMAND_CAPACITY = 40,
  LOOM_CMD_ZERO_BINDING_CAPACITY = 41,
  LOOM_CMD_IDENTIFIER_SPACE_EXHAUSTED = 42,
  LOOM_CMD_BINDINGS_QUEUE_MISMATCH = 43,
  LOOM_CMD_QUEUE_POISONED = 44,
  LOOM_CMD_SCOPE_POISONED = 45,
  LOOM_CMD_BINDING_CAPACITY_EXCEEDED = 46,
  LOOM_CMD_BUFFER_CONTEXT_MISMATCH = 47,
  LOOM_CMD_BINDING_SET_MISMATCH = 48,
  LOOM_CMD_BINDING_SLOT_OUT_OF_RANGE = 49,
  LOOM_CMD_BINDING_IS_READ_ONLY = 50,
  LOOM_CMD_BINDING_SLOT_VACANT = 51,
  LOOM_CMD_BINDING_TYPE_MISMATCH = 52,
  LOOM_CMD_DUPLICATE_BINDING_SLOT = 53,
  LOOM_CMD_COMMAND_CAPACITY_EXCEEDED = 54,
  LOOM_CMD_EXTERNAL = 55,
  LOOM_CMD_DRIVER = 56,
  /* C-ABI ownership checks that Rust's type system performs statically. */
  LOOM_CMD_ALIASED_BINDING = 57,      /* a read-write range overlaps another lease */
  LOOM_CMD_BINDINGS_IN_USE = 58,      /* bindings were moved into a live scope */
  LOOM_NULL_ARGUMENT = 59,
  LOOM_CMD_SCOPE_ACTIVE = 60,         /* the queue already has a live scope or unsettled completion */
  /* No reference counterpart: a kernel of a settled command (or graph replay)
   * reported through the queue's device status words that it could not finish
   * the command as specified (fields[0]: bit 0 = an append token workgroup
   * gave up waiting for the validation verdicts, so a valid command may be
   * applied only in part; bit 1 = the append's epoch handover gave up, the
   * validation workspace is marked broken; bit 2 = an append found its
   * workspace marked broken and wrote nothing).  The queue (or graph
   * execution) is poisoned.  An append command is idempotent: re-running it
   * on a healthy queue writes the same bytes. */
  LOOM_CMD_DEVICE_STATUS = 61,

  /* Plan errors (decode.rs:1498-1513, rope/mod.rs:1049-1061). */
  LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE = 70,
  LOOM_PLAN_STATE_COUNT_OVERFLOW = 71,
  LOOM_PLAN_UNSUPPORTED_HEAD_DIMENSION = 72,
  LOOM_PLAN_UNSUPPORTED_ROTARY_DIMENSION = 73,
  LOOM_PLAN_UNSUPPORTED_DEVICE = 74,   /* the provider only loads on gfx950 */
  LOOM_PLAN_INVALID_OPTION = 75,

  /* Enqueue errors (decode.rs:1515-1551, rope/mod.rs:1062-1077). */
  LOOM_ENQ_LENGTH_MISMATCH = 90,
  LOOM_ENQ_PAGE_INDICES_TOO_SHORT = 91,
  LOOM_ENQ_MISALIGNED_BUFFER = 92,
  LOOM_ENQ_PAGE_INDICES_TOO_LONG = 93, /* more pages than the plan's workspace covers */
  LOOM_ENQ_STATIC_SCRATCH_TOO_SMALL = 94, /* plan workspace beyond the static scratch */
  LOOM_ENQ_STATIC_SCRATCH_BUSY = 96, /* an allocation-free command of another stream
                                        still holds this device's static scratch */
  LOOM_ENQ_WORKSPACE_NOT_RESERVED = 95, /* the queue's workspace would have to grow while
                                           its stream is being captured */

  /* GraphError, crates/loom-infer-cuda/src/graph/mod.rs:688-721. */
  LOOM_GRAPH_DEFAULT_STREAM_UNSUPPORTED = 110,
  LOOM_GRAPH_EMPTY_CAPTURE = 111,
  LOOM_GRAPH_CAPTURE_INVALIDATED = 112,
  LOOM_GRAPH_NULL_EXECUTABLE_HANDLE = 113,
  LOOM_GRAPH_EXECUTION_POISONED = 114,
  LOOM_GRAPH_REPLAY_IN_FLIGHT = 115,
  LOOM_GRAPH_LAUNCH_COUNT_EXHAUSTED = 116,
  LOOM_GRAPH_TIMING_EVENT_CONTEXT_MISMATCH = 117,
  LOOM_GRAPH_DRIVER = 118,
  LOOM_GRAPH_SETTLEMENT = 119
};

/* Variant payload: `fields` hold the variant's integer fields in declaration
 * order (floats are stored as their f64 value in `value`), `operand` names the
 * buffer for LengthMismatch-like variants, `hip_status` the HIP error for
 * driver variants. */
typedef struct loom_error {
  int32_t code;
  int32_t hip_status;
  const char *operand;
  int64_t fields[4];
  double value;
  char message[256];
} loom_error_t;

/* Returns the Display text for a status code without payload. */
const char *loom_status_name(loom_status_t status);
uint32_t loom_abi_version(void);

typedef enum loom_dtype {
  LOOM_DTYPE_F32 = 0, /* dtype.rs:2-20 */
  LOOM_DTYPE_F16 = 1,
  LOOM_DTYPE_BF16 = 2,
  LOOM_DTYPE_I32 = 3, /* binding.rs:230-234 element types */
  LOOM_DTYPE_U8 = 4
} loom_dtype_t;

/* ------------------------------------------------------------------------ */
/* K/V page layout (no reference counterpart: the reference supports NHD only
 * and lists HND as unsupported, docs/results/h20-bf16-rope-paged-kv-append-
 * tokens-correctness-20260806.json contract.unsupported).  NHD pages are
 * [16, Hkv, 128] (token-major); HND pages are [Hkv, 16, 128] (head-major: one
 * kv-head's 16 rows are 4 KiB contiguous).  Every paged operation (decode,
 * append, paged prefill) reads and writes the layout its spec names. */
typedef enum loom_kv_layout {
  LOOM_KV_LAYOUT_NHD = 0,
  LOOM_KV_LAYOUT_HND = 1
} loom_kv_layout_t;

/* K/V page element type (no reference counterpart: the reference lists FP8 KV
 * storage as unsupported, same record).  FP8 pages hold OCP E4M3 bytes with
 * per-tensor scales passed at enqueue as a device f32 [2] operand
 * (k_scale, v_scale): K = fp8 * k_scale, V = fp8 * v_scale.  Append encodes
 * K (after RoPE, from FP32) and V as fp8(x / scale): saturating to +-448,
 * round to nearest even.  Decode reads them; the query, output and LSE stay
 * BF16 / FP32. */
typedef enum loom_kv_dtype {
  LOOM_KV_DTYPE_BF16 = 0,
  LOOM_KV_DTYPE_FP8_E4M3 = 1
} loom_kv_dtype_t;

/* ------------------------------------------------------------------------ */
/* Paged batch-decode contract, crates/loom-infer/src/attention/paged_decode/mod.rs */
typedef struct loom_paged_decode_spec {
  uint64_t batch_size;
  uint64_t max_num_pages;
  uint64_t num_query_heads;
  uint64_t num_kv_heads;
  float softmax_scale;
  uint32_t kv_layout; /* loom_kv_layout_t; LOOM_KV_LAYOUT_NHD from spec_new */
  uint32_t kv_dtype;  /* loom_kv_dtype_t; LOOM_KV_DTYPE_BF16 from spec_new */
  uint32_t page_size; /* token rows per page: 16 from spec_new; 32 or 64 through
                         loom_paged_decode_spec_with_page_size */
} loom_paged_decode_spec_t;

/* Bf16PagedBatchDecodeSpec::new, paged_decode/mod.rs:28-82. */
loom_status_t loom_paged_decode_spec_new(uint64_t batch_size, uint64_t max_num_pages,
                                         uint64_t num_query_heads, uint64_t num_kv_heads,
                                         uint64_t head_dim, uint64_t page_size,
                                         loom_paged_decode_spec_t *out, loom_error_t *err);
/* The same spec with another K/V page layout (no reference counterpart; the
 * paged append specs embed this spec and take their layout from it).
 * LOOM_PLAN_INVALID_OPTION for an unknown layout. */
loom_status_t loom_paged_decode_spec_with_kv_layout(const loom_paged_decode_spec_t *spec,
                                                    uint32_t kv_layout,
                                                    loom_paged_decode_spec_t *out,
                                                    loom_error_t *err);
/* The same spec with another K/V page element type (no reference
 * counterpart; append specs take it from their embedded decode spec). */
loom_status_t loom_paged_decode_spec_with_kv_dtype(const loom_paged_decode_spec_t *spec,
                                                   uint32_t kv_dtype,
                                                   loom_paged_decode_spec_t *out,
                                                   loom_error_t *err);
/* The same spec with another page size (no reference counterpart: the
 * reference's spec_new accepts 16 only, and so does this library's).  32 and 64
 * rows per page are accepted for paged decode and paged append (each page is
 * streamed as page_size / 16 blocks of 16 rows); LOOM_UNSUPPORTED_PAGE_SIZE
 * otherwise, LOOM_ELEMENT_COUNT_OVERFLOW when pool * page_size does not fit
 * 31 bits.  The page-table contract scales with it: last_page_len lies in
 * 1..page_size and token t of a request sits in page t / page_size, row
 * t % page_size. */
loom_status_t loom_paged_decode_spec_with_page_size(const loom_paged_decode_spec_t *spec,
                                                    uint32_t page_size,
                                                    loom_paged_decode_spec_t *out,
                                                    loom_error_t *err);
/* validate_page_table, paged_decode/mod.rs:152-213 (host metadata). */
loom_status_t loom_paged_decode_validate_page_table(const loom_paged_decode_spec_t *spec,
                                                    const int32_t *page_indptr, uint64_t n_indptr,
                                                    const int32_t *page_indices,
                                                    uint64_t n_indices,
                                                    const int32_t *last_page_len,
                                                    uint64_t n_last, loom_error_t *err);
/* request_kv_len / physical_page_for_token, paged_decode/mod.rs:252-278, on a
 * validated table.  Return LOOM_OK and fill the outputs (the reference's
 * Some), or LOOM_PAGE_INDEX_OUT_OF_RANGE for the reference's None. */
loom_status_t loom_paged_decode_request_kv_len(const loom_paged_decode_spec_t *spec,
                                               const int32_t *page_indptr,
                                               const int32_t *last_page_len, uint64_t request,
                                               uint64_t *kv_len);
loom_status_t loom_paged_decode_physical_page_for_token(
    const loom_paged_decode_spec_t *spec, const int32_t *page_indptr,
    const int32_t *page_indices, const int32_t *last_page_len, uint64_t request,
    uint64_t logical_token, uint64_t *physical_page, uint64_t *page_offset);

/* Fused RoPE + one-token append, paged_append/mod.rs:16-131. */
typedef struct loom_rope_append_spec {
  loom_paged_decode_spec_t paged;
} loom_rope_append_spec_t;
loom_status_t loom_rope_append_spec_new(uint64_t batch_size, uint64_t max_num_pages,
                                        uint64_t num_query_heads, uint64_t num_kv_heads,
                                        uint64_t head_dim, uint64_t page_size,
                                        loom_rope_append_spec_t *out, loom_error_t *err);
/* paged_append/mod.rs:95-131: page table + duplicate final slot rejection
 * (reported for the first (first_request, second_request) pair in the
 * reference's nested-loop order; computed in O(B) with a hash map). */
loom_status_t loom_rope_append_validate_page_table(const loom_rope_append_spec_t *spec,
                                                   const int32_t *page_indptr,
                                                   uint64_t n_indptr,
                                                   const int32_t *page_indices,
                                                   uint64_t n_indices,
                                                   const int32_t *last_page_len,
                                                   uint64_t n_last, loom_error_t *err);

/* Explicit-token append, paged_append/mod.rs:136-317. */
typedef struct loom_rope_append_tokens_spec {
  loom_paged_decode_spec_t paged;
  uint64_t tokens;
  uint64_t max_tokens; /* 64 (reference contract) or the extended bound */
} loom_rope_append_tokens_spec_t;
/* Bf16RopePagedKvAppendTokensSpec::new, paged_append/mod.rs:144-177 (T <= 64). */
loom_status_t loom_rope_append_tokens_spec_new(uint64_t tokens, uint64_t batch_size,
                                               uint64_t max_num_pages,
                                               uint64_t num_query_heads,
                                               uint64_t num_kv_heads, uint64_t head_dim,
                                               uint64_t page_size,
                                               loom_rope_append_tokens_spec_t *out,
                                               loom_error_t *err);
/* Same contract with T <= LOOM_APPEND_MAX_TOKENS_EXTENDED (no reference
 * counterpart; for callers that append whole prefill chunks in one command). */
loom_status_t loom_rope_append_tokens_spec_new_extended(
    uint64_t tokens, uint64_t batch_size, uint64_t max_num_pages, uint64_t num_query_heads,
    uint64_t num_kv_heads, uint64_t head_dim, uint64_t page_size,
    loom_rope_append_tokens_spec_t *out, loom_error_t *err);
/* validate_metadata, paged_append/mod.rs:244-317.  `slots` (optional, 2*T)
 * receives (physical_page, offset) per token. Duplicates are found in O(T)
 * and reported as the first (first_token, second_token) pair in token order. */
loom_status_t loom_rope_append_tokens_validate_metadata(
    const loom_rope_append_tokens_spec_t *spec, const int32_t *batch_indices, uint64_t n_batch,
    const int32_t *positions, uint64_t n_positions, const int32_t *page_indptr,
    uint64_t n_indptr, const int32_t *page_indices, uint64_t n_indices,
    const int32_t *last_page_len, uint64_t n_last, uint64_t *slots, loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Command runtime, crates/loom-infer-cuda/src/command/.                       */
typedef struct loom_command_queue loom_command_queue_t;
typedef struct loom_bindings loom_bindings_t;
typedef struct loom_command_scope loom_command_scope_t;
typedef struct loom_command_completion loom_command_completion_t;

/* Opaque binding handle (binding.rs:310-336 Read/ReadWrite/Write). */
typedef struct loom_handle {
  uint64_t set_id;
  uint64_t slot;
} loom_handle_t;

/* CommandQueue::new(stream, max_commands), submission.rs:31-46.  `stream` is
 * a hipStream_t owned by the caller (it must outlive the queue).  Beyond the
 * reference, the queue allocates its append validation workspace here (device
 * memory, zero-filled by a kernel on `stream`; fails with
 * LOOM_ENQ_WORKSPACE_NOT_RESERVED if `stream` is being captured) and four
 * device status words in pinned host memory, which kernels write when they
 * cannot finish a command as specified (see LOOM_CMD_DEVICE_STATUS). */
loom_status_t loom_command_queue_new(void *hip_stream, uint64_t max_commands,
                                     loom_command_queue_t **out, loom_error_t *err);
/* Drop: synchronizes the stream if commands are still retained. */
void loom_command_queue_free(loom_command_queue_t *queue);
/* No reference counterpart: the reference's plans need no workspace.  The
 * paged-decode enqueue that takes the reference's argument struct keeps its
 * split-KV states in a device buffer owned by the queue; this allocates it
 * ahead of the first command (`scratch_bytes` = a decode plan's
 * workspace_bytes) so that those enqueues allocate nothing, which is required
 * when they are captured.  `zeroed_bytes` (an append plan's workspace_bytes)
 * is already held from queue creation; asking for more than that fails with
 * LOOM_ENQ_WORKSPACE_NOT_RESERVED.  Buffers only grow; they are freed with the
 * queue (or with the graph that captured its commands). */
loom_status_t loom_command_queue_reserve_workspace(loom_command_queue_t *queue,
                                                   uint64_t scratch_bytes, uint64_t zeroed_bytes,
                                                   loom_error_t *err);
uint64_t loom_command_queue_workspace_bytes(const loom_command_queue_t *queue);
uint64_t loom_command_queue_max_commands(const loom_command_queue_t *queue);
int loom_command_queue_is_poisoned(const loom_command_queue_t *queue);

/* CommandQueue::bindings(capacity), submission.rs:58-70. */
loom_status_t loom_command_queue_bindings(loom_command_queue_t *queue, uint64_t capacity,
                                          loom_bindings_t **out, loom_error_t *err);
void loom_bindings_free(loom_bindings_t *bindings);
uint64_t loom_bindings_len(const loom_bindings_t *bindings);
uint64_t loom_bindings_capacity(const loom_bindings_t *bindings);
/* bind_read / bind_read_write, binding.rs:38-91.  The device pointer must
 * belong to the queue stream's device (BufferContextMismatch otherwise). */
loom_status_t loom_bindings_bind_read(loom_bindings_t *bindings, const void *device_ptr,
                                      uint64_t numel, loom_dtype_t dtype, loom_handle_t *out,
                                      loom_error_t *err);
loom_status_t loom_bindings_bind_read_write(loom_bindings_t *bindings, void *device_ptr,
                                            uint64_t numel, loom_dtype_t dtype,
                                            loom_handle_t *out, loom_error_t *err);
/* take_read_write, binding.rs:93-107: returns the owned buffer and vacates
 * the slot. */
loom_status_t loom_bindings_take_read_write(loom_bindings_t *bindings, loom_handle_t handle,
                                            void **device_ptr, uint64_t *numel,
                                            loom_error_t *err);

/* CommandQueue::begin, submission.rs:73-99.  On success the bindings move
 * into the scope; the caller gets them back from completion_wait. */
loom_status_t loom_command_queue_begin(loom_command_queue_t *queue, loom_bindings_t *bindings,
                                       loom_command_scope_t **out, loom_error_t *err);
/* CommandScope::finish, submission.rs:131-151: records the one completion
 * event.  Consumes the scope. */
loom_status_t loom_command_scope_finish(loom_command_scope_t *scope,
                                        loom_command_completion_t **out, loom_error_t *err);
/* Drop of an unfinished scope (synchronizes if anything was submitted). */
void loom_command_scope_free(loom_command_scope_t *scope);
uint64_t loom_command_scope_submitted(const loom_command_scope_t *scope);

uint64_t loom_command_completion_submitted(const loom_command_completion_t *completion);
/* is_complete / wait, completion.rs:37-83.  wait consumes the completion and
 * returns the bindings (NULL and freed on failure, as the reference drops them). */
loom_status_t loom_command_completion_is_complete(loom_command_completion_t *completion,
                                                  int *complete, loom_error_t *err);
loom_status_t loom_command_completion_wait(loom_command_completion_t *completion,
                                           loom_bindings_t **bindings, loom_error_t *err);
/* Drop: waits, poisons the queue on failure, frees the bindings. */
void loom_command_completion_free(loom_command_completion_t *completion);

/* ------------------------------------------------------------------------ */
/* Paged decode provider and plan, crates/loom-infer-cuda/src/attention/decode.rs */
typedef struct loom_decode_provider loom_decode_provider_t;
typedef struct loom_paged_decode_plan loom_paged_decode_plan_t;

/* DecodeProvider::load, decode.rs:1009-1014: binds the gfx950 kernels of this
 * library on `device` (LOOM_PLAN_UNSUPPORTED_DEVICE on other targets). */
loom_status_t loom_decode_provider_load(int device, loom_decode_provider_t **out,
                                        loom_error_t *err);
void loom_decode_provider_free(loom_decode_provider_t *provider);

typedef enum loom_paged_decode_algorithm {
  /* The valid requests' pages form one list cut into `teams` equal ranges;
   * a team is one wave per (kv-head, tile of up to 8 query heads), so the
   * whole GQA group shares each K/V byte.  Requests that cross a range
   * boundary merge through log2-LSE states in a second kernel. */
  LOOM_PAGED_DECODE_BALANCED_SPLIT_KV = 1,
  /* Small page capacity (max_total_pages <= 128, teams option 0): one
   * workgroup of 4-16 waves per (request, kv-head, tile), one launch.  When
   * few such workgroups would stream long requests (max_total_pages / B >=
   * 16 and at most 2 * CUs workgroups after splitting), each request's pages
   * split over 2-8 workgroups of 4 waves (plan info `teams`), whose states a
   * second kernel merges. */
  LOOM_PAGED_DECODE_DIRECT = 2
} loom_paged_decode_algorithm_t;

/* Plan flag (no reference counterpart; the reference rejects rebinding and
 * graph updates, graph/mod.rs:3-6): the page_indices operand is a capacity.
 * The device guard accepts page_indptr[B] <= len(page_indices) instead of
 * requiring equality, and entries past page_indptr[B] are ignored, so one
 * captured graph can be replayed as an engine rewrites the page table in
 * place between steps (growing sequences, new pages). */
#define LOOM_PLAN_PAGE_INDICES_CAPACITY 1u

/* Planner inputs.  Zero means "choose for this device". */
typedef struct loom_paged_decode_plan_options {
  uint64_t max_total_pages; /* upper bound of page_indices length; 0 -> max_num_pages */
  uint32_t teams;           /* page ranges; 0 -> chosen for the device (or the direct
                               algorithm when max_total_pages <= 128) */
  uint32_t flags;           /* 0 or LOOM_PLAN_PAGE_INDICES_CAPACITY */
} loom_paged_decode_plan_options_t;

typedef struct loom_paged_decode_plan_info {
  loom_paged_decode_spec_t spec;
  int32_t algorithm;
  uint32_t teams;            /* balanced: page ranges; direct: workgroups per
                                (request, kv-head, tile) when split, else 0 */
  uint32_t group_tile;       /* query heads per wave column block */
  uint32_t group_tiles;      /* ceil(group / group_tile) */
  uint64_t max_total_pages;
  uint64_t state_slots;      /* balanced: teams + batch; split direct: teams * batch */
  uint64_t workspace_bytes;  /* header_bytes + state_slots * Hq * 132 FP32 */
  uint64_t header_bytes;     /* (batch + 2) int64 page prefixes, 256-byte rounded */
  uint32_t block_threads;
  uint32_t grid_blocks;
  uint32_t device_cus;
  uint32_t flags;
} loom_paged_decode_plan_info_t;

/* DecodeProvider::plan_bf16_paged_batch, decode.rs:1067-1103.  The plan
 * depends only on the spec and options, never on page-table contents. */
loom_status_t loom_decode_provider_plan_bf16_paged_batch(
    const loom_decode_provider_t *provider, const loom_paged_decode_spec_t *spec,
    const loom_paged_decode_plan_options_t *options, loom_paged_decode_plan_t **out,
    loom_error_t *err);
void loom_paged_decode_plan_free(loom_paged_decode_plan_t *plan);
void loom_paged_decode_plan_get_info(const loom_paged_decode_plan_t *plan,
                                     loom_paged_decode_plan_info_t *info);

/* Bf16PagedBatchDecodeArgs, decode.rs:1452-1487, plus the caller-owned
 * split-KV state workspace (u8, exactly plan.workspace_bytes; no
 * initialization needed, contents are scratch between commands). */
typedef struct loom_paged_decode_args {
  loom_handle_t query;         /* Read<bf16>  [B, Hq, 128] */
  loom_handle_t key_pages;     /* Read<bf16>  [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t value_pages;   /* Read<bf16>  [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t page_indptr;   /* Read<i32>   [B+1] */
  loom_handle_t page_indices;  /* Read<i32>   [>= B] */
  loom_handle_t last_page_len; /* Read<i32>   [B] */
  loom_handle_t output;        /* Write<bf16> [B, Hq, 128] */
  loom_handle_t lse;           /* Write<f32>  [B, Hq], log2 domain */
  loom_handle_t workspace;     /* Write<u8>   [workspace_bytes] */
  loom_handle_t kv_scales;     /* Read<f32> [2] for FP8 pages (K/V pages are then
                                  Read<u8>); {0, 0} for BF16 pages */
} loom_paged_decode_args_t;

/* Bf16PagedBatchDecodePlan::enqueue_into, decode.rs:1199-1296: one command of
 * two stream-ordered kernels (balanced split-KV partials, then the merge of
 * requests that cross a team's page range). */
loom_status_t loom_paged_decode_enqueue(const loom_paged_decode_plan_t *plan,
                                        loom_command_scope_t *scope,
                                        const loom_paged_decode_args_t *args,
                                        loom_error_t *err);

/* Bf16PagedBatchDecodeArgs exactly as the reference declares it
 * (decode.rs:1452-1487): eight operands, no workspace. */
typedef struct loom_bf16_paged_batch_decode_args {
  loom_handle_t query;         /* Read<bf16>  [B, Hq, 128] */
  loom_handle_t key_pages;     /* Read<bf16>  [pool, P, Hkv, 128] */
  loom_handle_t value_pages;   /* Read<bf16>  [pool, P, Hkv, 128] */
  loom_handle_t page_indptr;   /* Read<i32>   [B+1] */
  loom_handle_t page_indices;  /* Read<i32>   [>= B] */
  loom_handle_t last_page_len; /* Read<i32>   [B] */
  loom_handle_t output;        /* Write<bf16> [B, Hq, 128] */
  loom_handle_t lse;           /* Write<f32>  [B, Hq], log2 domain */
} loom_bf16_paged_batch_decode_args_t;

/* Bf16PagedBatchDecodePlan::enqueue_into(scope, Bf16PagedBatchDecodeArgs),
 * decode.rs:1199-1296, with the reference's argument struct.  The split-KV
 * states live in a workspace owned by the scope's command queue: it is
 * allocated (hipMalloc) the first time a command needs more than the queue
 * holds, then reused by every later command on that queue (stream-ordered, so
 * without races), and freed with the queue.  While the queue's stream is
 * being captured it never grows: a command that would need more fails with
 * LOOM_ENQ_WORKSPACE_NOT_RESERVED.  Callers that must not allocate here
 * reserve it first (loom_command_queue_reserve_workspace with
 * plan.workspace_bytes) or pass their own (loom_paged_decode_enqueue).  BF16
 * pages only (the reference's args carry no FP8 scales). */
loom_status_t loom_paged_decode_enqueue_bf16(const loom_paged_decode_plan_t *plan,
                                             loom_command_scope_t *scope,
                                             const loom_bf16_paged_batch_decode_args_t *args,
                                             loom_error_t *err);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory at all (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): the same command as loom_paged_decode_enqueue_bf16,
 * with the split-KV workspace in a static device array of this library
 * (LOOM_PAGED_DECODE_STATIC_SCRATCH_BYTES per device, held until the process
 * ends; its address is looked up when a decode provider is loaded on the
 * device).  Allocates nothing.  Plans whose workspace_bytes exceed the array
 * are rejected with LOOM_ENQ_STATIC_SCRATCH_TOO_SMALL (BASELINE-sized plans
 * need at most ~11 MiB).  Every call on a device shares its one array: calls
 * ordered on one stream never conflict.  An eager call on another stream than
 * the device's previous allocation-free command, while that command has not
 * finished, is rejected with LOOM_ENQ_STATIC_SCRATCH_BUSY (nothing is
 * enqueued; the caller orders the streams or waits, then retries).  Calls
 * under stream capture are not checked (the captured work runs later): the
 * caller keeps replays of such graphs ordered with every other
 * allocation-free command on the device, or they race. */
#define LOOM_PAGED_DECODE_STATIC_SCRATCH_BYTES (32u << 20)
loom_status_t loom_paged_decode_enqueue_bf16_no_alloc(
    const loom_paged_decode_plan_t *plan, loom_command_scope_t *scope,
    const loom_bf16_paged_batch_decode_args_t *args, loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Contiguous single decode, crates/loom-infer/src/attention/single_decode/    */
/* mod.rs:15-194 and decode.rs:1016-1064, :1108-1181, :1301-1450: Q/O        */
/* [Hq, 128], K/V [kv_len, Hkv, 128] (NHD, contiguous), LSE [Hq] log2.        */
typedef struct loom_single_decode_spec {
  uint64_t kv_len;
  uint64_t num_query_heads;
  uint64_t num_kv_heads;
  float softmax_scale;
} loom_single_decode_spec_t;

typedef struct loom_single_decode_split_k_spec {
  loom_single_decode_spec_t decode;
  uint64_t partitions;
} loom_single_decode_split_k_spec_t;

/* Bf16SingleDecodeSpec::new, single_decode/mod.rs:31-70. */
loom_status_t loom_single_decode_spec_new(uint64_t kv_len, uint64_t num_query_heads,
                                          uint64_t num_kv_heads, uint64_t head_dim,
                                          loom_single_decode_spec_t *out, loom_error_t *err);
/* Bf16SingleDecodeSplitKSpec::new, single_decode/mod.rs:131-145. */
loom_status_t loom_single_decode_split_k_spec_new(const loom_single_decode_spec_t *decode,
                                                  uint64_t partitions,
                                                  loom_single_decode_split_k_spec_t *out,
                                                  loom_error_t *err);
/* partition_token_range, single_decode/mod.rs:167-181: balanced contiguous
 * partitions (the first kv_len % P get one token more).  LOOM_OK, or
 * LOOM_INVALID_PARTITION_COUNT for the reference's None. */
loom_status_t loom_single_decode_split_k_partition_token_range(
    const loom_single_decode_split_k_spec_t *spec, uint64_t partition, uint64_t *start,
    uint64_t *end);

typedef struct loom_single_decode_plan loom_single_decode_plan_t;
typedef struct loom_single_decode_split_k_plan loom_single_decode_split_k_plan_t;

/* DecodeProvider::plan_bf16, decode.rs:1016-1032: one workgroup per
 * (kv-head, tile of up to 8 query heads) streams the whole KV range. */
loom_status_t loom_decode_provider_plan_bf16(const loom_decode_provider_t *provider,
                                             const loom_single_decode_spec_t *spec,
                                             loom_single_decode_plan_t **out, loom_error_t *err);
void loom_single_decode_plan_free(loom_single_decode_plan_t *plan);

/* Bf16SingleDecodeArgs, decode.rs:1394-1420. */
typedef struct loom_single_decode_args {
  loom_handle_t query;  /* Read<bf16>  [Hq, 128] */
  loom_handle_t key;    /* Read<bf16>  [kv_len, Hkv, 128] */
  loom_handle_t value;  /* Read<bf16>  [kv_len, Hkv, 128] */
  loom_handle_t output; /* Write<bf16> [Hq, 128] */
  loom_handle_t lse;    /* Write<f32>  [Hq] */
} loom_single_decode_args_t;

/* Bf16SingleDecodePlan::enqueue_into, decode.rs:1120-1180: one command. */
loom_status_t loom_single_decode_enqueue(const loom_single_decode_plan_t *plan,
                                         loom_command_scope_t *scope,
                                         const loom_single_decode_args_t *args,
                                         loom_error_t *err);

/* DecodeProvider::plan_bf16_split_k, decode.rs:1034-1064: one wave per
 * (partition, kv-head, tile) writes the partition's log2-domain states. */
loom_status_t loom_decode_provider_plan_bf16_split_k(
    const loom_decode_provider_t *provider, const loom_single_decode_split_k_spec_t *spec,
    loom_single_decode_split_k_plan_t **out, loom_error_t *err);
void loom_single_decode_split_k_plan_free(loom_single_decode_split_k_plan_t *plan);
/* workspace_required_bytes, decode.rs:1316-1320: Hq * partitions * 130 * 4. */
uint64_t loom_single_decode_split_k_workspace_bytes(const loom_single_decode_split_k_plan_t *plan);

/* Bf16SingleDecodeSplitKArgs, decode.rs:1422-1450: the workspace holds the
 * partial states [Hq, partitions, 130] = (max_log2, normalizer, acc[128]). */
typedef struct loom_single_decode_split_k_args {
  loom_handle_t query;
  loom_handle_t key;
  loom_handle_t value;
  loom_handle_t workspace; /* ReadWrite<f32> [Hq * partitions * 130] */
  loom_handle_t output;
  loom_handle_t lse;
} loom_single_decode_split_k_args_t;

/* Bf16SingleDecodeSplitKPlan::enqueue_into, decode.rs:1322-1392: two
 * commands (partials, then the merge) in one scope. */
loom_status_t loom_single_decode_split_k_enqueue(const loom_single_decode_split_k_plan_t *plan,
                                                 loom_command_scope_t *scope,
                                                 const loom_single_decode_split_k_args_t *args,
                                                 loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Paged causal prefill, crates/loom-infer/src/attention/paged_prefill/mod.rs  */
/* Q/O [nnz_qo, Hq, 128] ragged by qo_indptr; K/V pages [pool, P, Hkv, 128]      */
/* (NHD) by page_indptr / page_indices / last_page_len; LSE [nnz_qo, Hq]       */
/* log2.  Bottom-right causal mask: row i of a request with qo_len rows sees   */
/* KV tokens 0 .. kv_len - qo_len + i.                                         */
typedef struct loom_paged_prefill_spec {
  uint64_t batch_size;
  uint64_t nnz_qo;
  uint64_t max_num_pages;
  uint64_t num_query_heads;
  uint64_t num_kv_heads;
  float softmax_scale;
  uint32_t kv_layout; /* loom_kv_layout_t; LOOM_KV_LAYOUT_NHD from spec_new */
  uint32_t page_size; /* 16 from spec_new; 32 or 64 through
                         loom_paged_prefill_spec_with_page_size */
  uint32_t kv_dtype;  /* loom_kv_dtype_t; LOOM_KV_DTYPE_BF16 from spec_new */
} loom_paged_prefill_spec_t;

/* Bf16PagedPrefillSpec::new, paged_prefill/mod.rs:30-91. */
loom_status_t loom_paged_prefill_spec_new(uint64_t batch_size, uint64_t nnz_qo,
                                          uint64_t max_num_pages, uint64_t num_query_heads,
                                          uint64_t num_kv_heads, uint64_t head_dim,
                                          uint64_t page_size, loom_paged_prefill_spec_t *out,
                                          loom_error_t *err);
/* The same spec with another K/V page layout (no reference counterpart). */
loom_status_t loom_paged_prefill_spec_with_kv_layout(const loom_paged_prefill_spec_t *spec,
                                                     uint32_t kv_layout,
                                                     loom_paged_prefill_spec_t *out,
                                                     loom_error_t *err);
/* The same spec with FP8 E4M3 K/V pages (no reference counterpart; the pages
 * and the kv_scales operand as for paged decode). */
loom_status_t loom_paged_prefill_spec_with_kv_dtype(const loom_paged_prefill_spec_t *spec,
                                                    uint32_t kv_dtype,
                                                    loom_paged_prefill_spec_t *out,
                                                    loom_error_t *err);
/* The same spec with 32- or 64-row pages (no reference counterpart; the same
 * contract as loom_paged_decode_spec_with_page_size). */
loom_status_t loom_paged_prefill_spec_with_page_size(const loom_paged_prefill_spec_t *spec,
                                                     uint32_t page_size,
                                                     loom_paged_prefill_spec_t *out,
                                                     loom_error_t *err);
/* validate_metadata, paged_prefill/mod.rs:161-264 (host metadata). */
loom_status_t loom_paged_prefill_validate_metadata(const loom_paged_prefill_spec_t *spec,
                                                   const int32_t *qo_indptr, uint64_t n_qo,
                                                   const int32_t *page_indptr, uint64_t n_indptr,
                                                   const int32_t *page_indices,
                                                   uint64_t n_indices,
                                                   const int32_t *last_page_len,
                                                   uint64_t n_last, loom_error_t *err);
/* causal_kv_end, paged_prefill/mod.rs:374-383, on validated metadata:
 * LOOM_OK, or LOOM_EMPTY_RAGGED_REQUEST for the reference's None (request or
 * query index out of range). */
loom_status_t loom_paged_prefill_causal_kv_end(const loom_paged_prefill_spec_t *spec,
                                               const int32_t *qo_indptr,
                                               const int32_t *page_indptr,
                                               const int32_t *last_page_len, uint64_t request,
                                               uint64_t query_index, uint64_t *end);

typedef struct loom_prefill_provider loom_prefill_provider_t;
typedef struct loom_paged_prefill_plan loom_paged_prefill_plan_t;

/* PrefillProvider::load (crates/loom-infer-cuda/src/attention/prefill.rs:2278-2288). */
loom_status_t loom_prefill_provider_load(int device, loom_prefill_provider_t **out,
                                         loom_error_t *err);
void loom_prefill_provider_free(loom_prefill_provider_t *provider);

typedef enum loom_paged_prefill_algorithm {
  /* One workgroup of `waves` waves per (request, kv-head, tile of 16
   * flattened (query row, group head) pairs).  The waves split the tile's
   * causal page range; per page, S = K·Qᵀ and O += P·V both run on MFMA, and
   * the wave states merge in LDS.  No workspace. */
  LOOM_PAGED_PREFILL_ROW_TILE = 1,
  /* For long prompts: one workgroup of four waves per (request, kv-head, tile
   * of 64 flattened pairs), one 16-column tile per wave.  Every wave walks the
   * whole causal page range; each K/V block is loaded once per workgroup,
   * staged through LDS and read by all four waves, so a workgroup reads a
   * quarter of the L2 bytes per column that ROW_TILE reads.  No cross-wave
   * merge.  No workspace. */
  LOOM_PAGED_PREFILL_WIDE_TILE = 2,
  /* Long prompts on BF16 or FP8 pages (paged prefill only): WIDE_TILE's
   * columns and page walk with 32-token blocks loaded straight into LDS, the
   * query fragments in registers and the softmax weights P rounded once to
   * BF16 for the P·V product (the normalizer is summed in FP32; within the
   * attention tolerance of the f32 reference).  One or two 16-column query
   * tiles per wave (64 or 128 columns per workgroup); plans whose grid fits
   * one round of two workgroups per CU (and, with one tile per wave, requests
   * averaging 1024 rows or more) run two groups of four waves that split the
   * K/V blocks and merge in LDS (block_threads 512).  No workspace. */
  LOOM_PAGED_PREFILL_LONG_TILE = 3
} loom_paged_prefill_algorithm_t;

/* Prefill plan flags (no reference counterpart): force ROW_TILE, WIDE_TILE
 * or LONG_TILE; with none, the plan picks one from the spec. */
#define LOOM_PLAN_PREFILL_TILE_16 2u
#define LOOM_PLAN_PREFILL_TILE_64 4u
#define LOOM_PLAN_PREFILL_TILE_LONG 8u

typedef struct loom_paged_prefill_plan_options {
  uint32_t waves; /* waves per workgroup: 0 (the default, four), 4, 8 or 16 */
  uint32_t flags; /* LOOM_PLAN_PAGE_INDICES_CAPACITY (paged only) and at most one of
                     LOOM_PLAN_PREFILL_TILE_16 / _64 / _LONG (the last two: four waves;
                     _LONG: paged prefill only) */
} loom_paged_prefill_plan_options_t;

typedef struct loom_paged_prefill_plan_info {
  loom_paged_prefill_spec_t spec;
  int32_t algorithm;
  uint32_t waves;
  uint64_t row_tiles;  /* upper bound of tiles over any valid qo_indptr:
                          min(C, floor((C + (t - 1) * batch) / t)), C = nnz_qo * group,
                          t = 16 (ROW_TILE), 64 (WIDE_TILE) or 64 / 128 (LONG_TILE)
                          columns per tile */
  uint32_t block_threads; /* waves * 64; 512 for LONG_TILE plans with two wave groups */
  uint64_t grid_blocks; /* row_tiles * Hkv */
  uint32_t flags;
} loom_paged_prefill_plan_info_t;

/* PrefillProvider::plan_bf16_paged, prefill.rs:2289-2330.  The plan depends
 * only on the spec (and options), never on metadata contents. */
loom_status_t loom_prefill_provider_plan_bf16_paged(const loom_prefill_provider_t *provider,
                                                    const loom_paged_prefill_spec_t *spec,
                                                    loom_paged_prefill_plan_t **out,
                                                    loom_error_t *err);
/* The same plan with planner options (no reference counterpart). */
loom_status_t loom_prefill_provider_plan_bf16_paged_options(
    const loom_prefill_provider_t *provider, const loom_paged_prefill_spec_t *spec,
    const loom_paged_prefill_plan_options_t *options, loom_paged_prefill_plan_t **out,
    loom_error_t *err);
void loom_paged_prefill_plan_free(loom_paged_prefill_plan_t *plan);
void loom_paged_prefill_plan_get_info(const loom_paged_prefill_plan_t *plan,
                                      loom_paged_prefill_plan_info_t *info);

/* Bf16PagedPrefillArgs, prefill.rs:2852-2890. */
typedef struct loom_paged_prefill_args {
  loom_handle_t query;         /* Read<bf16>  [nnz_qo, Hq, 128] */
  loom_handle_t key_pages;     /* Read<bf16>  [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t value_pages;   /* Read<bf16>  [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t qo_indptr;     /* Read<i32>   [B+1] */
  loom_handle_t page_indptr;   /* Read<i32>   [B+1] */
  loom_handle_t page_indices;  /* Read<i32>   [>= B] */
  loom_handle_t last_page_len; /* Read<i32>   [B] */
  loom_handle_t output;        /* Write<bf16> [nnz_qo, Hq, 128] */
  loom_handle_t lse;           /* Write<f32>  [nnz_qo, Hq], log2 domain */
  loom_handle_t kv_scales;     /* Read<f32> [2] for FP8 pages (K/V pages are then
                                  Read<u8>); {0, 0} for BF16 pages */
} loom_paged_prefill_args_t;

/* Bf16PagedPrefillPlan::enqueue_into, prefill.rs:2447-2560: one command, one
 * kernel.  Device guards as prefill.rs:293-342: invalid global metadata leaves
 * every output untouched; a request with an invalid page range, last-page
 * length, page index or qo_len > kv_len keeps its sentinels, and so does every
 * request after the first malformed qo_indptr range.  Q, K, V and O must be
 * 4-byte aligned, as in the reference (prefill.rs:2496-2503, 3015-3029). */
loom_status_t loom_paged_prefill_enqueue(const loom_paged_prefill_plan_t *plan,
                                         loom_command_scope_t *scope,
                                         const loom_paged_prefill_args_t *args,
                                         loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Ragged causal prefill, crates/loom-infer/src/attention/ragged_prefill/     */
/* mod.rs: Q/O [nnz_qo, Hq, 128], K/V [nnz_kv, Hkv, 128] contiguous NHD rows,  */
/* both ragged by i32 indptr arrays; same bottom-right causal mask.          */
typedef struct loom_ragged_prefill_spec {
  uint64_t batch_size;
  uint64_t nnz_qo;
  uint64_t nnz_kv;
  uint64_t num_query_heads;
  uint64_t num_kv_heads;
  float softmax_scale;
} loom_ragged_prefill_spec_t;

/* Bf16RaggedPrefillSpec::new, ragged_prefill/mod.rs:27-79. */
loom_status_t loom_ragged_prefill_spec_new(uint64_t batch_size, uint64_t nnz_qo,
                                           uint64_t nnz_kv, uint64_t num_query_heads,
                                           uint64_t num_kv_heads, uint64_t head_dim,
                                           loom_ragged_prefill_spec_t *out, loom_error_t *err);
/* validate_metadata, ragged_prefill/mod.rs:140-193. */
loom_status_t loom_ragged_prefill_validate_metadata(const loom_ragged_prefill_spec_t *spec,
                                                    const int32_t *qo_indptr, uint64_t n_qo,
                                                    const int32_t *kv_indptr, uint64_t n_kv,
                                                    loom_error_t *err);
/* causal_kv_end, ragged_prefill/mod.rs:233-242 (an absolute KV row) on
 * validated metadata: LOOM_OK, or LOOM_EMPTY_RAGGED_REQUEST for None. */
loom_status_t loom_ragged_prefill_causal_kv_end(const loom_ragged_prefill_spec_t *spec,
                                                const int32_t *qo_indptr,
                                                const int32_t *kv_indptr, uint64_t request,
                                                uint64_t query_index, uint64_t *end);

typedef struct loom_ragged_prefill_plan loom_ragged_prefill_plan_t;

typedef struct loom_ragged_prefill_plan_info {
  loom_ragged_prefill_spec_t spec;
  int32_t algorithm;          /* LOOM_PAGED_PREFILL_ROW_TILE or _WIDE_TILE: the same
                                 kernel designs */
  uint32_t waves;
  uint64_t row_tiles;
  uint32_t block_threads;
  uint64_t grid_blocks;
  uint64_t workspace_numel;   /* 0: this plan needs no workspace */
} loom_ragged_prefill_plan_info_t;

/* PrefillProvider::plan_bf16_ragged, prefill.rs:2331-2410.  `options` may be
 * NULL; its `flags` must be 0 (no page table). */
loom_status_t loom_prefill_provider_plan_bf16_ragged(const loom_prefill_provider_t *provider,
                                                     const loom_ragged_prefill_spec_t *spec,
                                                     const loom_paged_prefill_plan_options_t *options,
                                                     loom_ragged_prefill_plan_t **out,
                                                     loom_error_t *err);
void loom_ragged_prefill_plan_free(loom_ragged_prefill_plan_t *plan);
void loom_ragged_prefill_plan_get_info(const loom_ragged_prefill_plan_t *plan,
                                       loom_ragged_prefill_plan_info_t *info);
/* workspace_required_numel, prefill.rs:2640-2646: 0 for this plan. */
uint64_t loom_ragged_prefill_workspace_numel(const loom_ragged_prefill_plan_t *plan);

/* Bf16RaggedPrefillArgs, prefill.rs:2893-2931.  `workspace` is the optional
 * with_workspace operand ({0, 0} when absent); this plan needs none and
 * ignores it. */
typedef struct loom_ragged_prefill_args {
  loom_handle_t query;     /* Read<bf16>  [nnz_qo, Hq, 128] */
  loom_handle_t key;       /* Read<bf16>  [nnz_kv, Hkv, 128] */
  loom_handle_t value;     /* Read<bf16>  [nnz_kv, Hkv, 128] */
  loom_handle_t qo_indptr; /* Read<i32>   [B+1] */
  loom_handle_t kv_indptr; /* Read<i32>   [B+1] */
  loom_handle_t output;    /* Write<bf16> [nnz_qo, Hq, 128] */
  loom_handle_t lse;       /* Write<f32>  [nnz_qo, Hq], log2 domain */
  loom_handle_t workspace; /* optional ReadWrite<f32> */
} loom_ragged_prefill_args_t;

/* Bf16RaggedPrefillPlan::enqueue_into, prefill.rs:2648-2760: one command, one
 * kernel.  Device guards as prefill.rs:102-138: invalid global indptr words
 * write nothing; a row belongs to the first request whose qo range ends after
 * it, and keeps its sentinels when that request fails its guards. */
loom_status_t loom_ragged_prefill_enqueue(const loom_ragged_prefill_plan_t *plan,
                                          loom_command_scope_t *scope,
                                          const loom_ragged_prefill_args_t *args,
                                          loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Fused RoPE + paged append provider, crates/loom-infer-cuda/src/rope/mod.rs */
typedef struct loom_rope_provider loom_rope_provider_t;
typedef struct loom_rope_append_plan loom_rope_append_plan_t;

loom_status_t loom_rope_provider_load(int device, loom_rope_provider_t **out,
                                      loom_error_t *err);
void loom_rope_provider_free(loom_rope_provider_t *provider);

typedef struct loom_rope_append_plan_info {
  uint64_t tokens;          /* B for the one-token form */
  uint64_t batch_size;
  uint64_t num_query_heads;
  uint64_t num_kv_heads;
  int32_t explicit_tokens;  /* 0: one token per request at kv_len-1 */
  uint64_t workspace_bytes; /* the validation workspace, one fixed layout for every
                               plan: a header (epoch, broken flag), one start tag per
                               workgroup of the largest grid, 64 copies of the chunk
                               verdicts, two duplicate-slot hash tables and the
                               two-launch verdicts.  It carries the epoch from one
                               command to the next (all zeros is a valid start) */
  uint32_t validate_blocks;
} loom_rope_append_plan_info_t;

/* RopeProvider::plan_bf16_paged_append, rope/mod.rs:628-654. */
loom_status_t loom_rope_provider_plan_bf16_paged_append(const loom_rope_provider_t *provider,
                                                        const loom_rope_append_spec_t *spec,
                                                        loom_rope_append_plan_t **out,
                                                        loom_error_t *err);
/* RopeProvider::plan_bf16_paged_append_tokens, rope/mod.rs:656-682. */
loom_status_t loom_rope_provider_plan_bf16_paged_append_tokens(
    const loom_rope_provider_t *provider, const loom_rope_append_tokens_spec_t *spec,
    loom_rope_append_plan_t **out, loom_error_t *err);
/* Append plan flags (no reference counterpart).
 * LOOM_PLAN_APPEND_TWO_LAUNCH: commands that take the chunk-validated path
 *   (T > 64 or more than 4096 page indices) run as two kernels, validation
 *   then apply, ordered on the stream, instead of one kernel whose token
 *   workgroups wait (bounded) for the validation workgroups' verdicts.  For
 *   callers that cannot rule out other streams or processes holding CUs
 *   while the append runs; slower at small T (one more launch).
 * LOOM_PLAN_APPEND_TEST_NO_WAIT: for tests of the failure path only: every
 *   bounded wait of the one-launch form gives up at once, so the command
 *   writes nothing and its completion fails with LOOM_CMD_DEVICE_STATUS
 *   (and the validation workspace is marked broken: zero it again before
 *   reusing it). */
#define LOOM_PLAN_APPEND_TWO_LAUNCH 8u
#define LOOM_PLAN_APPEND_TEST_NO_WAIT 16u
/* The same two plans with plan flags (LOOM_PLAN_PAGE_INDICES_CAPACITY and the
 * append flags above; no reference counterpart). */
loom_status_t loom_rope_provider_plan_bf16_paged_append_flags(
    const loom_rope_provider_t *provider, const loom_rope_append_spec_t *spec, uint32_t flags,
    loom_rope_append_plan_t **out, loom_error_t *err);
loom_status_t loom_rope_provider_plan_bf16_paged_append_tokens_flags(
    const loom_rope_provider_t *provider, const loom_rope_append_tokens_spec_t *spec,
    uint32_t flags, loom_rope_append_plan_t **out, loom_error_t *err);
void loom_rope_append_plan_free(loom_rope_append_plan_t *plan);
void loom_rope_append_plan_get_info(const loom_rope_append_plan_t *plan,
                                    loom_rope_append_plan_info_t *info);

/* Bf16RopePagedKvAppendArgs / ...TokensArgs, rope/mod.rs:963-1047, plus the
 * caller-owned validation workspace (u8, plan.workspace_bytes, zero before its
 * first command and not written by the caller afterwards; it carries the
 * commands' epoch from one command to the next, and all zeros is a valid
 * starting state; one workspace may serve several append plans in stream
 * order; after a command fails with LOOM_CMD_DEVICE_STATUS bit 1 it is marked
 * broken and must be zeroed again).  batch_indices/positions are unused
 * (pass {0,0}) for the one-token form. */
typedef struct loom_rope_append_args {
  loom_handle_t query;         /* Read<bf16> [T, Hq, 128] */
  loom_handle_t key;           /* Read<bf16> [T, Hkv, 128] */
  loom_handle_t value;         /* Read<bf16> [T, Hkv, 128] */
  loom_handle_t batch_indices; /* Read<i32>  [T] (explicit form) */
  loom_handle_t positions;     /* Read<i32>  [T] (explicit form) */
  loom_handle_t page_indptr;   /* Read<i32>  [B+1] */
  loom_handle_t page_indices;  /* Read<i32>  [>= B] */
  loom_handle_t last_page_len; /* Read<i32>  [B] */
  loom_handle_t query_output;  /* Write<bf16> [T, Hq, 128] */
  loom_handle_t key_pages;     /* Write<bf16> [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t value_pages;   /* Write<bf16> [pool, P, Hkv, 128]; P = page_size */
  loom_handle_t workspace;     /* Write<u8> */
  loom_handle_t kv_scales;     /* Read<f32> [2] for FP8 pages (K/V pages are then
                                  Write<u8>); {0, 0} for BF16 pages */
} loom_rope_append_args_t;

/* enqueue_into, rope/mod.rs:758-830 / :846-934: one kernel per command.  Its
 * first workgroups validate the metadata in chunks (whole page table, batch
 * indices, positions, duplicate physical slots) while one workgroup per token
 * loads and rotates; the token workgroups write only after every chunk has
 * passed.  Commands with T <= 64 and at most 4096 page indices run as one
 * kernel that validates in every workgroup.  Invalid device metadata leaves
 * every output untouched (the reference's sentinel guard).  The token
 * workgroups' wait for the verdicts is bounded (about 0.3 s); a wait that
 * gives up is reported when the completion settles (LOOM_CMD_DEVICE_STATUS,
 * the queue is poisoned): a workgroup that gave up wrote nothing, so an
 * invalid command still writes nothing, while a valid one may be applied in
 * part and should be re-run (appends are idempotent).  Plans with
 * LOOM_PLAN_APPEND_TWO_LAUNCH never wait. */
loom_status_t loom_rope_append_enqueue(const loom_rope_append_plan_t *plan,
                                       loom_command_scope_t *scope,
                                       const loom_rope_append_args_t *args,
                                       loom_error_t *err);

/* Bf16RopePagedKvAppendArgs and Bf16RopePagedKvAppendTokensArgs exactly as
 * the reference declares them (rope/mod.rs:963-1047): no workspace, BF16
 * pages. */
typedef struct loom_bf16_rope_paged_kv_append_args {
  loom_handle_t query;         /* Read<bf16>  [B, Hq, 128] */
  loom_handle_t key;           /* Read<bf16>  [B, Hkv, 128] */
  loom_handle_t value;         /* Read<bf16>  [B, Hkv, 128] */
  loom_handle_t page_indptr;   /* Read<i32>   [B+1] */
  loom_handle_t page_indices;  /* Read<i32>   [>= B] */
  loom_handle_t last_page_len; /* Read<i32>   [B] */
  loom_handle_t query_output;  /* Write<bf16> [B, Hq, 128] */
  loom_handle_t key_pages;     /* Write<bf16> [pool, P, Hkv, 128] */
  loom_handle_t value_pages;   /* Write<bf16> [pool, P, Hkv, 128] */
} loom_bf16_rope_paged_kv_append_args_t;

typedef struct loom_bf16_rope_paged_kv_append_tokens_args {
  loom_handle_t query;         /* Read<bf16>  [T, Hq, 128] */
  loom_handle_t key;           /* Read<bf16>  [T, Hkv, 128] */
  loom_handle_t value;         /* Read<bf16>  [T, Hkv, 128] */
  loom_handle_t batch_indices; /* Read<i32>   [T] */
  loom_handle_t positions;     /* Read<i32>   [T] */
  loom_handle_t page_indptr;   /* Read<i32>   [B+1] */
  loom_handle_t page_indices;  /* Read<i32>   [>= B] */
  loom_handle_t last_page_len; /* Read<i32>   [B] */
  loom_handle_t query_output;  /* Write<bf16> [T, Hq, 128] */
  loom_handle_t key_pages;     /* Write<bf16> [pool, P, Hkv, 128] */
  loom_handle_t value_pages;   /* Write<bf16> [pool, P, Hkv, 128] */
} loom_bf16_rope_paged_kv_append_tokens_args_t;

/* Bf16RopePagedKvAppendPlan::enqueue_into (rope/mod.rs:758-830) and
 * Bf16RopePagedKvAppendTokensPlan::enqueue_into (:846-934) with the
 * reference's argument structs.  The validation words live in a
 * zero-initialised workspace owned by the scope's command queue, allocated
 * when the queue is created (one size serves every append plan), so these
 * enqueues never allocate.
 * A one-token plan takes the first form, an explicit-token plan the second
 * (LOOM_NULL_ARGUMENT "args" otherwise). */
loom_status_t loom_rope_append_enqueue_bf16(const loom_rope_append_plan_t *plan,
                                            loom_command_scope_t *scope,
                                            const loom_bf16_rope_paged_kv_append_args_t *args,
                                            loom_error_t *err);
loom_status_t loom_rope_append_tokens_enqueue_bf16(
    const loom_rope_append_plan_t *plan, loom_command_scope_t *scope,
    const loom_bf16_rope_paged_kv_append_tokens_args_t *args, loom_error_t *err);

/* ------------------------------------------------------------------------ */
/* Graph capture and replay, crates/loom-infer-cuda/src/graph/mod.rs           */
typedef struct loom_graph_queue loom_graph_queue_t;
typedef struct loom_captured_graph loom_captured_graph_t;
typedef struct loom_graph_exec loom_graph_exec_t;
typedef struct loom_graph_completion loom_graph_completion_t;

/* GraphQueue::new, graph/mod.rs:34-40: a private non-blocking stream. */
loom_status_t loom_graph_queue_new(int device, uint64_t max_commands,
                                   loom_graph_queue_t **out, loom_error_t *err);
void loom_graph_queue_free(loom_graph_queue_t *queue);
loom_status_t loom_graph_queue_bindings(loom_graph_queue_t *queue, uint64_t capacity,
                                        loom_bindings_t **out, loom_error_t *err);
/* No reference counterpart: loom_command_queue_reserve_workspace and
 * loom_command_queue_workspace_bytes for the graph queue's private command
 * queue.  A reference-shaped paged-decode command captured on a graph queue
 * needs its split-KV workspace reserved here first (the capture does not
 * allocate: LOOM_ENQ_WORKSPACE_NOT_RESERVED). */
loom_status_t loom_graph_queue_reserve_workspace(loom_graph_queue_t *queue, uint64_t scratch_bytes,
                                                 uint64_t zeroed_bytes, loom_error_t *err);
uint64_t loom_graph_queue_workspace_bytes(const loom_graph_queue_t *queue);
/* GraphQueue::capture split in two C calls (graph/mod.rs:54-131): begin
 * synchronizes the device, begins thread-local capture on the private stream
 * and returns an ordinary scope to enqueue into; end_capture finishes the
 * capture and consumes the queue and the scope. */
loom_status_t loom_graph_queue_begin_capture(loom_graph_queue_t *queue,
                                             loom_bindings_t *bindings,
                                             loom_command_scope_t **scope, loom_error_t *err);
loom_status_t loom_graph_queue_end_capture(loom_graph_queue_t *queue,
                                           loom_command_scope_t *scope,
                                           loom_captured_graph_t **out, loom_error_t *err);
uint64_t loom_captured_graph_commands(const loom_captured_graph_t *graph);
void loom_captured_graph_free(loom_captured_graph_t *graph);
/* CapturedGraph::instantiate, graph/mod.rs:183-206. Consumes the graph. */
loom_status_t loom_captured_graph_instantiate(loom_captured_graph_t *graph,
                                              loom_graph_exec_t **out, loom_error_t *err);
uint64_t loom_graph_exec_commands(const loom_graph_exec_t *exec);
/* No reference counterpart: how loom_graph_exec_launch replays the captured
 * graph.  LOOM_GRAPH_REPLAY_KERNEL_NODES (the default whenever the capture is
 * a chain of kernel nodes, which every capture of this library's commands
 * is): each captured kernel node is launched with hipLaunchKernel, with the
 * node's captured function, launch shape and argument copy, in dependency
 * order, on the replay stream — the same work at the same fixed addresses.
 * On MI355X with ROCm 7 a hipGraphLaunch of a one-node graph costs 15-23 us
 * of host time before the kernel can start, against about 2.3 us for one
 * hipLaunchKernel.  LOOM_GRAPH_REPLAY_HIP_GRAPH_LAUNCH submits the
 * instantiated hipGraphExec with hipGraphLaunch (the only mode for other
 * graphs).  set_replay_mode fails with LOOM_PLAN_INVALID_OPTION for a mode
 * the graph cannot use and LOOM_GRAPH_REPLAY_IN_FLIGHT while a replay is in
 * flight. */
#define LOOM_GRAPH_REPLAY_HIP_GRAPH_LAUNCH 1
#define LOOM_GRAPH_REPLAY_KERNEL_NODES 2
int32_t loom_graph_exec_replay_mode(const loom_graph_exec_t *exec);
loom_status_t loom_graph_exec_set_replay_mode(loom_graph_exec_t *exec, int32_t mode,
                                              loom_error_t *err);
uint64_t loom_graph_exec_launches(const loom_graph_exec_t *exec);
/* GraphExec::launch, graph/mod.rs:249-293. */
loom_status_t loom_graph_exec_launch(loom_graph_exec_t *exec, loom_graph_completion_t **out,
                                     loom_error_t *err);
/* GraphExec::measure_launch_ms, graph/mod.rs:301-323 (events created on the
 * exec's device by the caller, passed as hipEvent_t). */
loom_status_t loom_graph_exec_measure_launch_ms(loom_graph_exec_t *exec, void *start_event,
                                                void *end_event, float *ms, loom_error_t *err);
/* GraphExec::into_bindings, graph/mod.rs:326-339. Consumes the exec. */
loom_status_t loom_graph_exec_into_bindings(loom_graph_exec_t *exec, loom_bindings_t **out,
                                            loom_error_t *err);
void loom_graph_exec_free(loom_graph_exec_t *exec);
uint64_t loom_graph_completion_launch_index(const loom_graph_completion_t *completion);
loom_status_t loom_graph_completion_is_complete(loom_graph_completion_t *completion,
                                                int *complete, loom_error_t *err);
/* wait consumes the completion. */
loom_status_t loom_graph_completion_wait(loom_graph_completion_t *completion,
                                         loom_error_t *err);
/* Drop: settles the replay. */
void loom_graph_completion_free(loom_graph_completion_t *completion);

#ifdef __cplusplus
}
#endif
#endif /* LOOM_INFER_HIP_H */
