// Contract layer: specifications, host-side metadata validation and the error
// taxonomy of crates/loom-infer/src/error.rs (+ the command, plan, enqueue and
// graph errors of crates/loom-infer-cuda).
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "loom_internal.hpp"

namespace loom {

namespace {

const char *dtype_name(int64_t d) {
  switch (d) {
    case LOOM_DTYPE_F32: return "F32";
    case LOOM_DTYPE_F16: return "F16";
    case LOOM_DTYPE_BF16: return "Bf16";
    case LOOM_DTYPE_I32: return "I32";
    default: return "U8";
  }
}

// Display text, error.rs:111-272 and the thiserror strings of the CUDA crate.
void format_message(loom_error_t *e) {
  char *m = e->message;
  const size_t n = sizeof(e->message);
  const int64_t *f = e->fields;
  const char *op = e->operand ? e->operand : "?";
  switch (e->code) {
    case LOOM_OK: snprintf(m, n, "ok"); break;
    case LOOM_ZERO_DIMENSION: snprintf(m, n, "tensor dimensions must be nonzero"); break;
    case LOOM_ELEMENT_COUNT_OVERFLOW: snprintf(m, n, "tensor element count overflowed"); break;
    case LOOM_INVALID_EPSILON:
      snprintf(m, n, "RMSNorm epsilon must be finite and positive, got %g", e->value);
      break;
    case LOOM_UNSUPPORTED_HEAD_DIMENSION:
      snprintf(m, n, "unsupported attention head dimension: expected %lld, got %lld",
               (long long)f[0], (long long)f[1]);
      break;
    case LOOM_UNSUPPORTED_PAGE_SIZE:
      snprintf(m, n, "unsupported KV page size: expected %lld, got %lld", (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_INVALID_HEAD_MAPPING:
      snprintf(m, n, "query heads must be divisible by KV heads: query=%lld, KV=%lld",
               (long long)f[0], (long long)f[1]);
      break;
    case LOOM_INVALID_PARTITION_COUNT:
      snprintf(m, n, "attention partition count must be in 1..=%lld, got %lld",
               (long long)f[1], (long long)f[0]);
      break;
    case LOOM_INVALID_INDPTR_START:
      snprintf(m, n, "%s must start at zero, got %lld", op, (long long)f[0]);
      break;
    case LOOM_NON_MONOTONIC_INDPTR:
      snprintf(m, n, "%s must be nondecreasing at request %lld, got %lld then %lld", op,
               (long long)f[0], (long long)f[1], (long long)f[2]);
      break;
    case LOOM_EMPTY_RAGGED_REQUEST:
      snprintf(m, n, "%s request %lld has zero length", op, (long long)f[0]);
      break;
    case LOOM_RAGGED_QUERY_LONGER_THAN_KV:
      snprintf(m, n,
               "ragged prefill request %lld has query length %lld greater than KV length %lld",
               (long long)f[0], (long long)f[1], (long long)f[2]);
      break;
    case LOOM_INVALID_PAGE_INDPTR_START:
      snprintf(m, n, "page indptr must start at zero, got %lld", (long long)f[0]);
      break;
    case LOOM_NON_MONOTONIC_PAGE_INDPTR:
      snprintf(m, n, "page indptr must be nondecreasing at request %lld, got %lld then %lld",
               (long long)f[0], (long long)f[1], (long long)f[2]);
      break;
    case LOOM_EMPTY_PAGED_REQUEST:
      snprintf(m, n, "paged decode request %lld has no KV pages", (long long)f[0]);
      break;
    case LOOM_PAGE_INDEX_OUT_OF_RANGE:
      snprintf(m, n, "page index at position %lld must be in 0..%lld, got %lld",
               (long long)f[0], (long long)f[2], (long long)f[1]);
      break;
    case LOOM_INVALID_LAST_PAGE_LENGTH:
      snprintf(m, n, "last page length for request %lld must be in 1..=%lld, got %lld",
               (long long)f[0], (long long)f[2], (long long)f[1]);
      break;
    case LOOM_INVALID_ROTARY_DIMENSION:
      snprintf(m, n,
               "RoPE rotary dimension must be positive, even, and no greater than head "
               "dimension %lld, got %lld",
               (long long)f[1], (long long)f[0]);
      break;
    case LOOM_INVALID_ROPE_SCALE:
      snprintf(m, n, "RoPE scale must be finite and positive, got %g", e->value);
      break;
    case LOOM_INVALID_ROPE_THETA:
      snprintf(m, n, "RoPE theta must be finite and greater than one, got %g", e->value);
      break;
    case LOOM_NEGATIVE_POSITION_ID:
      snprintf(m, n, "RoPE position ID at token %lld must be nonnegative, got %lld",
               (long long)f[0], (long long)f[1]);
      break;
    case LOOM_UNSUPPORTED_APPEND_TOKEN_COUNT:
      snprintf(m, n, "explicit paged KV append supports at most %lld tokens, got %lld",
               (long long)f[0], (long long)f[1]);
      break;
    case LOOM_APPEND_BATCH_INDEX_OUT_OF_RANGE:
      snprintf(m, n, "paged KV append batch index at token %lld must be in 0..%lld, got %lld",
               (long long)f[0], (long long)f[2], (long long)f[1]);
      break;
    case LOOM_APPEND_POSITION_OUT_OF_RANGE:
      snprintf(m, n,
               "paged KV append position at token %lld for request %lld must be in 0..%lld, "
               "got %lld",
               (long long)f[0], (long long)f[1], (long long)f[3], (long long)f[2]);
      break;
    case LOOM_DUPLICATE_PAGE_APPEND_SLOT:
      snprintf(m, n,
               "paged KV append requests %lld and %lld target the same physical slot (%lld, "
               "%lld)",
               (long long)f[0], (long long)f[1], (long long)f[2], (long long)f[3]);
      break;
    case LOOM_DUPLICATE_PAGE_APPEND_TOKEN_SLOT:
      snprintf(m, n,
               "paged KV append tokens %lld and %lld target the same physical slot (%lld, "
               "%lld)",
               (long long)f[0], (long long)f[1], (long long)f[2], (long long)f[3]);
      break;
    case LOOM_UNSUPPORTED_DTYPE:
      snprintf(m, n, "unsupported dtype %s", dtype_name(f[0]));
      break;
    case LOOM_LENGTH_MISMATCH:
    case LOOM_ENQ_LENGTH_MISMATCH:
      snprintf(m, n, "%s length mismatch: expected %lld, got %lld", op, (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_CMD_ZERO_COMMAND_CAPACITY:
      snprintf(m, n, "command queues require capacity for at least one command");
      break;
    case LOOM_CMD_ZERO_BINDING_CAPACITY:
      snprintf(m, n, "checked bindings require capacity for at least one resource");
      break;
    case LOOM_CMD_IDENTIFIER_SPACE_EXHAUSTED:
      snprintf(m, n, "command queue identifier space is exhausted");
      break;
    case LOOM_CMD_BINDINGS_QUEUE_MISMATCH:
      snprintf(m, n, "the checked bindings were created by a different command queue");
      break;
    case LOOM_CMD_QUEUE_POISONED:
      snprintf(m, n, "the command queue is poisoned by an earlier completion failure");
      break;
    case LOOM_CMD_SCOPE_POISONED:
      snprintf(m, n, "the command scope is poisoned by an earlier submission failure");
      break;
    case LOOM_CMD_BINDING_CAPACITY_EXCEEDED:
      snprintf(m, n, "checked binding capacity %lld is exhausted", (long long)f[0]);
      break;
    case LOOM_CMD_BUFFER_CONTEXT_MISMATCH:
      snprintf(m, n,
               "buffer belongs to HIP device %lld, but the queue stream belongs to device %lld",
               (long long)f[0], (long long)f[1]);
      break;
    case LOOM_CMD_BINDING_SET_MISMATCH:
      snprintf(m, n, "the resource handle belongs to a different checked binding set");
      break;
    case LOOM_CMD_BINDING_SLOT_OUT_OF_RANGE:
      snprintf(m, n, "binding slot %lld is out of range for %lld bindings", (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_CMD_BINDING_IS_READ_ONLY:
      snprintf(m, n, "binding slot %lld is read-only", (long long)f[0]);
      break;
    case LOOM_CMD_BINDING_SLOT_VACANT:
      snprintf(m, n, "binding slot %lld has already been removed", (long long)f[0]);
      break;
    case LOOM_CMD_BINDING_TYPE_MISMATCH:
      snprintf(m, n, "binding slot %lld has a different element type than its resource handle",
               (long long)f[0]);
      break;
    case LOOM_CMD_DUPLICATE_BINDING_SLOT:
      snprintf(m, n, "one command cannot use the same binding slot for multiple operands");
      break;
    case LOOM_CMD_COMMAND_CAPACITY_EXCEEDED:
      snprintf(m, n, "command scope capacity %lld is exhausted", (long long)f[0]);
      break;
    case LOOM_CMD_EXTERNAL:
      snprintf(m, n, "%s command submission failed with status %lld", op, (long long)f[0]);
      break;
    case LOOM_CMD_DRIVER:
      snprintf(m, n, "HIP driver error %d (%s)", e->hip_status,
               hipGetErrorString((hipError_t)e->hip_status));
      break;
    case LOOM_CMD_ALIASED_BINDING:
      snprintf(m, n, "a read-write binding overlaps binding slot %lld of the same set",
               (long long)f[0]);
      break;
    case LOOM_CMD_BINDINGS_IN_USE:
      snprintf(m, n, "the checked bindings are owned by a live command scope or graph");
      break;
    case LOOM_CMD_SCOPE_ACTIVE:
      snprintf(m, n, "the command queue already has a live scope or an unsettled completion");
      break;
    case LOOM_CMD_DEVICE_STATUS:
      snprintf(m, n,
               "a kernel reported device status %#llx: the command did not complete as "
               "specified (1: append verdict wait gave up, 2: append epoch handover gave up, "
               "4: append workspace marked broken)",
               (unsigned long long)f[0]);
      break;
    case LOOM_NULL_ARGUMENT:
      snprintf(m, n, "required argument %s is null", op);
      break;
    case LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE:
      snprintf(m, n, "%s state count %lld exceeds the HIP grid range", op, (long long)f[0]);
      break;
    case LOOM_PLAN_STATE_COUNT_OVERFLOW:
      snprintf(m, n, "%s state count overflowed", op);
      break;
    case LOOM_PLAN_UNSUPPORTED_HEAD_DIMENSION:
      snprintf(m, n, "%s requires head dimension %lld, got %lld", op, (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_PLAN_UNSUPPORTED_ROTARY_DIMENSION:
      snprintf(m, n, "standard RoPE requires rotary dimension %lld, got %lld", (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_PLAN_UNSUPPORTED_DEVICE:
      snprintf(m, n, "HIP device %lld is not gfx950; the provider has no kernels for it",
               (long long)f[0]);
      break;
    case LOOM_PLAN_INVALID_OPTION:
      snprintf(m, n, "invalid planner option %s=%lld", op, (long long)f[0]);
      break;
    case LOOM_ENQ_PAGE_INDICES_TOO_SHORT:
      snprintf(m, n, "page_indices requires at least %lld entries, got %lld", (long long)f[0],
               (long long)f[1]);
      break;
    case LOOM_ENQ_MISALIGNED_BUFFER:
      snprintf(m, n, "%s requires %s to be %lld-byte aligned, got %#llx", "paged batch decode",
               op, (long long)f[1], (unsigned long long)f[0]);
      break;
    case LOOM_ENQ_PAGE_INDICES_TOO_LONG:
      snprintf(m, n, "page_indices has %lld entries but the plan's workspace covers %lld",
               (long long)f[1], (long long)f[0]);
      break;
    case LOOM_ENQ_STATIC_SCRATCH_TOO_SMALL:
      snprintf(m, n,
               "the plan's %s needs %lld bytes but the static scratch of the allocation-free "
               "enqueue holds %lld",
               op, (long long)f[1], (long long)f[0]);
      break;
    case LOOM_ENQ_STATIC_SCRATCH_BUSY:
      snprintf(m, n,
               "the static scratch of device %lld is held by an allocation-free command of "
               "another stream that has not finished (order the streams, or wait, and retry)",
               (long long)f[0]);
      break;
    case LOOM_ENQ_WORKSPACE_NOT_RESERVED:
      snprintf(m, n,
               "the command queue's %s holds %lld bytes, the command needs %lld, and the queue's "
               "stream is being captured (reserve the workspace before capture)",
               op, (long long)f[0], (long long)f[1]);
      break;
    case LOOM_GRAPH_DEFAULT_STREAM_UNSUPPORTED:
      snprintf(m, n, "HIP graph capture requires a non-default stream");
      break;
    case LOOM_GRAPH_EMPTY_CAPTURE: snprintf(m, n, "HIP graph capture recorded no commands"); break;
    case LOOM_GRAPH_CAPTURE_INVALIDATED:
      snprintf(m, n, "HIP graph capture was invalidated and returned no graph");
      break;
    case LOOM_GRAPH_NULL_EXECUTABLE_HANDLE:
      snprintf(m, n, "HIP graph instantiation returned a null executable handle");
      break;
    case LOOM_GRAPH_EXECUTION_POISONED:
      snprintf(m, n, "HIP graph execution is poisoned by an earlier replay failure");
      break;
    case LOOM_GRAPH_REPLAY_IN_FLIGHT: snprintf(m, n, "a HIP graph replay is already in flight"); break;
    case LOOM_GRAPH_LAUNCH_COUNT_EXHAUSTED: snprintf(m, n, "HIP graph launch count is exhausted"); break;
    case LOOM_GRAPH_TIMING_EVENT_CONTEXT_MISMATCH:
      snprintf(m, n, "HIP graph timing events belong to a different device");
      break;
    case LOOM_GRAPH_DRIVER:
      snprintf(m, n, "HIP graph %s failed: %s", op, hipGetErrorString((hipError_t)e->hip_status));
      break;
    case LOOM_GRAPH_SETTLEMENT:
      snprintf(m, n, "HIP graph %s failed: %s; fallback stream synchronization also reported: %s",
               op, hipGetErrorString((hipError_t)e->hip_status),
               hipGetErrorString((hipError_t)f[0]));
      break;
    default: snprintf(m, n, "loom status %d", e->code); break;
  }
}

}  // namespace

loom_status_t fail(loom_error_t *err, loom_status_t code, const char *operand, int64_t f0,
                   int64_t f1, int64_t f2, int64_t f3, double value, int32_t hip_status) {
  if (err) {
    err->code = code;
    err->hip_status = hip_status;
    err->operand = operand;
    err->fields[0] = f0;
    err->fields[1] = f1;
    err->fields[2] = f2;
    err->fields[3] = f3;
    err->value = value;
    format_message(err);
  }
  return code;
}

uint64_t fresh_id() {
  // submission.rs:328-332: a process-wide, never-reused identifier.
  static std::atomic<uint64_t> next{1};
  return next.fetch_add(1, std::memory_order_relaxed);
}

}  // namespace loom

using loom::fail;

namespace {

loom_status_t require_len(loom_error_t *err, const char *buffer, uint64_t actual,
                          uint64_t expected) {
  if (actual == expected) return LOOM_OK;
  return fail(err, LOOM_LENGTH_MISMATCH, buffer, (int64_t)expected, (int64_t)actual);
}

bool mul_ovf(uint64_t a, uint64_t b, uint64_t *o) { return __builtin_mul_overflow(a, b, o); }

// Token rows per page of a paged spec (16 unless set by spec_with_page_size).
uint64_t page_rows(const loom_paged_decode_spec_t *s) {
  return s->page_size ? s->page_size : loom::kPageSize;
}
uint64_t prefill_page_rows(const loom_paged_prefill_spec_t *s) {
  return s->page_size ? s->page_size : loom::kPageSize;
}

// Request geometry on a validated table (paged_decode/mod.rs:242-278).
int64_t kv_len_of(const int32_t *indptr, const int32_t *last, uint64_t r, uint64_t page) {
  return ((int64_t)indptr[r + 1] - indptr[r] - 1) * (int64_t)page + last[r];
}

}  // namespace

extern "C" {

uint32_t loom_abi_version(void) { return LOOM_INFER_HIP_ABI_VERSION; }

const char *loom_status_name(loom_status_t status) {
  static thread_local loom_error_t e;
  fail(&e, status);
  return e.message;
}

// paged_decode/mod.rs:28-82.
loom_status_t loom_paged_decode_spec_new(uint64_t batch, uint64_t pool, uint64_t hq,
                                         uint64_t hkv, uint64_t head_dim, uint64_t page_size,
                                         loom_paged_decode_spec_t *out, loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (batch == 0 || pool == 0 || hq == 0 || hkv == 0 || head_dim == 0 || page_size == 0)
    return fail(err, LOOM_ZERO_DIMENSION);
  if (head_dim != loom::kHeadDim)
    return fail(err, LOOM_UNSUPPORTED_HEAD_DIMENSION, nullptr, loom::kHeadDim, head_dim);
  if (page_size != loom::kPageSize)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_size);
  if (hq % hkv != 0) return fail(err, LOOM_INVALID_HEAD_MAPPING, nullptr, hq, hkv);
  uint64_t t;
  if (batch == UINT64_MAX || mul_ovf(batch, hq, &t) || mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  if (mul_ovf(pool, page_size, &t) || mul_ovf(t, hkv, &t) || mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->batch_size = batch;
  out->max_num_pages = pool;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / std::sqrt((float)head_dim);
  out->kv_layout = LOOM_KV_LAYOUT_NHD;
  out->kv_dtype = LOOM_KV_DTYPE_BF16;
  out->page_size = (uint32_t)loom::kPageSize;
  return loom::ok(err);
}

loom_status_t loom_paged_decode_spec_with_page_size(const loom_paged_decode_spec_t *spec,
                                                    uint32_t page_size,
                                                    loom_paged_decode_spec_t *out,
                                                    loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (page_size != 16 && page_size != 32 && page_size != 64)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_size);
  uint64_t t;
  if (mul_ovf(spec->max_num_pages, page_size, &t) || t > (uint64_t)INT32_MAX ||
      mul_ovf(t, spec->num_kv_heads, &t) || mul_ovf(t, loom::kHeadDim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  *out = *spec;
  out->page_size = page_size;
  return loom::ok(err);
}

loom_status_t loom_paged_decode_spec_with_kv_dtype(const loom_paged_decode_spec_t *spec,
                                                   uint32_t kv_dtype,
                                                   loom_paged_decode_spec_t *out,
                                                   loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (kv_dtype != LOOM_KV_DTYPE_BF16 && kv_dtype != LOOM_KV_DTYPE_FP8_E4M3)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_dtype", kv_dtype);
  *out = *spec;
  out->kv_dtype = kv_dtype;
  return loom::ok(err);
}

loom_status_t loom_paged_decode_spec_with_kv_layout(const loom_paged_decode_spec_t *spec,
                                                    uint32_t kv_layout,
                                                    loom_paged_decode_spec_t *out,
                                                    loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (kv_layout != LOOM_KV_LAYOUT_NHD && kv_layout != LOOM_KV_LAYOUT_HND)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_layout", kv_layout);
  *out = *spec;
  out->kv_layout = kv_layout;
  return loom::ok(err);
}

// single_decode/mod.rs:31-70.
loom_status_t loom_single_decode_spec_new(uint64_t kv_len, uint64_t hq, uint64_t hkv,
                                          uint64_t head_dim, loom_single_decode_spec_t *out,
                                          loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (kv_len == 0 || hq == 0 || hkv == 0 || head_dim == 0) return fail(err, LOOM_ZERO_DIMENSION);
  if (head_dim != loom::kHeadDim)
    return fail(err, LOOM_UNSUPPORTED_HEAD_DIMENSION, nullptr, loom::kHeadDim, head_dim);
  if (hq % hkv != 0) return fail(err, LOOM_INVALID_HEAD_MAPPING, nullptr, hq, hkv);
  uint64_t t;
  if (mul_ovf(hq, head_dim, &t)) return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  if (mul_ovf(hkv, head_dim, &t) || mul_ovf(kv_len, t, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->kv_len = kv_len;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / std::sqrt((float)head_dim);
  return loom::ok(err);
}

// single_decode/mod.rs:131-145.
loom_status_t loom_single_decode_split_k_spec_new(const loom_single_decode_spec_t *decode,
                                                  uint64_t partitions,
                                                  loom_single_decode_split_k_spec_t *out,
                                                  loom_error_t *err) {
  if (!decode || !out) return fail(err, LOOM_NULL_ARGUMENT, "decode");
  if (partitions == 0 || partitions > decode->kv_len)
    return fail(err, LOOM_INVALID_PARTITION_COUNT, nullptr, partitions, decode->kv_len);
  uint64_t t;
  if (mul_ovf(decode->num_query_heads, partitions, &t) ||
      mul_ovf(t, loom::kStateWidth, &t) || mul_ovf(t, 4, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->decode = *decode;
  out->partitions = partitions;
  return loom::ok(err);
}

// single_decode/mod.rs:167-181.
loom_status_t loom_single_decode_split_k_partition_token_range(
    const loom_single_decode_split_k_spec_t *spec, uint64_t partition, uint64_t *start,
    uint64_t *end) {
  if (!spec || !start || !end) return LOOM_NULL_ARGUMENT;
  const uint64_t P = spec->partitions, L = spec->decode.kv_len;
  if (partition >= P) return LOOM_INVALID_PARTITION_COUNT;
  const uint64_t base = L / P, rem = L % P;
  const uint64_t s0 = partition * base + (partition < rem ? partition : rem);
  *start = s0;
  *end = s0 + base + (partition < rem ? 1 : 0);
  return LOOM_OK;
}

// paged_decode/mod.rs:152-213.
loom_status_t loom_paged_decode_validate_page_table(const loom_paged_decode_spec_t *s,
                                                    const int32_t *indptr, uint64_t n_indptr,
                                                    const int32_t *indices, uint64_t n_indices,
                                                    const int32_t *last, uint64_t n_last,
                                                    loom_error_t *err) {
  if (!s) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  loom_status_t rc;
  if ((rc = require_len(err, "page_indptr", n_indptr, s->batch_size + 1))) return rc;
  if ((rc = require_len(err, "last_page_len", n_last, s->batch_size))) return rc;
  if (indptr[0] != 0) return fail(err, LOOM_INVALID_PAGE_INDPTR_START, nullptr, indptr[0]);
  for (uint64_t r = 0; r < s->batch_size; ++r) {
    int32_t a = indptr[r], b = indptr[r + 1];
    if (b < a) return fail(err, LOOM_NON_MONOTONIC_PAGE_INDPTR, nullptr, r, a, b);
    if (b == a) return fail(err, LOOM_EMPTY_PAGED_REQUEST, nullptr, r);
    if (last[r] < 1 || last[r] > (int32_t)page_rows(s))
      return fail(err, LOOM_INVALID_LAST_PAGE_LENGTH, nullptr, r, last[r], page_rows(s));
  }
  if (indptr[s->batch_size] < 0) return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  if ((rc = require_len(err, "page_indices", n_indices, (uint64_t)indptr[s->batch_size])))
    return rc;
  for (uint64_t p = 0; p < n_indices; ++p)
    if (indices[p] < 0 || (uint64_t)indices[p] >= s->max_num_pages)
      return fail(err, LOOM_PAGE_INDEX_OUT_OF_RANGE, nullptr, p, indices[p], s->max_num_pages);
  return loom::ok(err);
}

loom_status_t loom_paged_decode_request_kv_len(const loom_paged_decode_spec_t *s,
                                               const int32_t *indptr, const int32_t *last,
                                               uint64_t request, uint64_t *kv_len) {
  if (!s || request >= s->batch_size) return LOOM_PAGE_INDEX_OUT_OF_RANGE;
  *kv_len = (uint64_t)kv_len_of(indptr, last, request, page_rows(s));
  return LOOM_OK;
}

loom_status_t loom_paged_decode_physical_page_for_token(const loom_paged_decode_spec_t *s,
                                                        const int32_t *indptr,
                                                        const int32_t *indices,
                                                        const int32_t *last, uint64_t request,
                                                        uint64_t token, uint64_t *page,
                                                        uint64_t *offset) {
  if (!s || request >= s->batch_size) return LOOM_PAGE_INDEX_OUT_OF_RANGE;
  if ((int64_t)token >= kv_len_of(indptr, last, request, page_rows(s)))
    return LOOM_PAGE_INDEX_OUT_OF_RANGE;
  *page = (uint64_t)indices[(uint64_t)indptr[request] + token / page_rows(s)];
  *offset = token % page_rows(s);
  return LOOM_OK;
}

// paged_append/mod.rs:22-40.
loom_status_t loom_rope_append_spec_new(uint64_t batch, uint64_t pool, uint64_t hq,
                                        uint64_t hkv, uint64_t head_dim, uint64_t page_size,
                                        loom_rope_append_spec_t *out, loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  return loom_paged_decode_spec_new(batch, pool, hq, hkv, head_dim, page_size, &out->paged,
                                    err);
}

// paged_append/mod.rs:95-131.  The reference scans all pairs in (first,
// second) order; the first reported pair is the smallest `first` request that
// has a later duplicate, with its smallest such `second`.  One pass with a map
// from slot to the first two requests that use it gives the same pair.
loom_status_t loom_rope_append_validate_page_table(const loom_rope_append_spec_t *spec,
                                                   const int32_t *indptr, uint64_t n_indptr,
                                                   const int32_t *indices, uint64_t n_indices,
                                                   const int32_t *last, uint64_t n_last,
                                                   loom_error_t *err) {
  if (!spec) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  const loom_paged_decode_spec_t *s = &spec->paged;
  loom_status_t rc = loom_paged_decode_validate_page_table(s, indptr, n_indptr, indices,
                                                           n_indices, last, n_last, err);
  if (rc) return rc;
  std::unordered_map<uint64_t, std::pair<int64_t, int64_t>> seen;
  seen.reserve(s->batch_size * 2);
  for (uint64_t r = 0; r < s->batch_size; ++r) {
    int64_t pos = kv_len_of(indptr, last, r, page_rows(s)) - 1;
    uint64_t page = (uint64_t)indices[(uint64_t)indptr[r] + (uint64_t)pos / page_rows(s)];
    uint64_t key = page * page_rows(s) + (uint64_t)pos % page_rows(s);
    auto it = seen.find(key);
    if (it == seen.end())
      seen.emplace(key, std::make_pair((int64_t)r, (int64_t)-1));
    else if (it->second.second < 0)
      it->second.second = (int64_t)r;
  }
  int64_t best_first = -1, best_second = -1;
  uint64_t best_key = 0;
  for (auto &kv : seen) {
    if (kv.second.second < 0) continue;
    if (best_first < 0 || kv.second.first < best_first) {
      best_first = kv.second.first;
      best_second = kv.second.second;
      best_key = kv.first;
    }
  }
  if (best_first >= 0)
    return fail(err, LOOM_DUPLICATE_PAGE_APPEND_SLOT, nullptr, best_first, best_second,
                (int64_t)(best_key / page_rows(s)), (int64_t)(best_key % page_rows(s)));
  return loom::ok(err);
}

static loom_status_t tokens_spec_new(uint64_t tokens, uint64_t max_tokens, uint64_t batch,
                                     uint64_t pool, uint64_t hq, uint64_t hkv, uint64_t head_dim,
                                     uint64_t page_size, loom_rope_append_tokens_spec_t *out,
                                     loom_error_t *err) {
  // paged_append/mod.rs:144-177.
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (tokens == 0) return fail(err, LOOM_ZERO_DIMENSION);
  if (tokens > max_tokens)
    return fail(err, LOOM_UNSUPPORTED_APPEND_TOKEN_COUNT, nullptr, max_tokens, tokens);
  loom_status_t rc =
      loom_paged_decode_spec_new(batch, pool, hq, hkv, head_dim, page_size, &out->paged, err);
  if (rc) return rc;
  uint64_t t;
  if (mul_ovf(tokens, hq, &t) || mul_ovf(t, head_dim, &t) || mul_ovf(tokens, hkv, &t) ||
      mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->tokens = tokens;
  out->max_tokens = max_tokens;
  return loom::ok(err);
}

loom_status_t loom_rope_append_tokens_spec_new(uint64_t tokens, uint64_t batch, uint64_t pool,
                                               uint64_t hq, uint64_t hkv, uint64_t head_dim,
                                               uint64_t page_size,
                                               loom_rope_append_tokens_spec_t *out,
                                               loom_error_t *err) {
  return tokens_spec_new(tokens, LOOM_APPEND_MAX_TOKENS, batch, pool, hq, hkv, head_dim,
                         page_size, out, err);
}

loom_status_t loom_rope_append_tokens_spec_new_extended(uint64_t tokens, uint64_t batch,
                                                        uint64_t pool, uint64_t hq,
                                                        uint64_t hkv, uint64_t head_dim,
                                                        uint64_t page_size,
                                                        loom_rope_append_tokens_spec_t *out,
                                                        loom_error_t *err) {
  return tokens_spec_new(tokens, LOOM_APPEND_MAX_TOKENS_EXTENDED, batch, pool, hq, hkv,
                         head_dim, page_size, out, err);
}

// paged_append/mod.rs:244-317.  The duplicate scan uses a hash map; the first
// reported pair is (earliest token with that slot, the current token), the
// same pair the reference's linear search returns.
loom_status_t loom_rope_append_tokens_validate_metadata(
    const loom_rope_append_tokens_spec_t *spec, const int32_t *batch_indices, uint64_t n_batch,
    const int32_t *positions, uint64_t n_positions, const int32_t *indptr, uint64_t n_indptr,
    const int32_t *indices, uint64_t n_indices, const int32_t *last, uint64_t n_last,
    uint64_t *slots, loom_error_t *err) {
  if (!spec) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  const loom_paged_decode_spec_t *s = &spec->paged;
  loom_status_t rc;
  if ((rc = require_len(err, "batch_indices", n_batch, spec->tokens))) return rc;
  if ((rc = require_len(err, "positions", n_positions, spec->tokens))) return rc;
  if ((rc = loom_paged_decode_validate_page_table(s, indptr, n_indptr, indices, n_indices, last,
                                                  n_last, err)))
    return rc;
  std::unordered_map<uint64_t, uint64_t> seen;
  seen.reserve(spec->tokens * 2);
  for (uint64_t t = 0; t < spec->tokens; ++t) {
    int32_t bi = batch_indices[t];
    if (bi < 0 || (uint64_t)bi >= s->batch_size)
      return fail(err, LOOM_APPEND_BATCH_INDEX_OUT_OF_RANGE, nullptr, t, bi, s->batch_size);
    int64_t kv_len = kv_len_of(indptr, last, (uint64_t)bi, page_rows(s));
    int32_t p = positions[t];
    if (p < 0 || p >= kv_len)
      return fail(err, LOOM_APPEND_POSITION_OUT_OF_RANGE, nullptr, t, bi, p, kv_len);
    uint64_t page = (uint64_t)indices[(uint64_t)indptr[bi] + (uint64_t)p / page_rows(s)];
    uint64_t off = (uint64_t)p % page_rows(s);
    uint64_t key = page * page_rows(s) + off;
    auto it = seen.find(key);
    if (it != seen.end())
      return fail(err, LOOM_DUPLICATE_PAGE_APPEND_TOKEN_SLOT, nullptr, (int64_t)it->second, t,
                  page, off);
    seen.emplace(key, t);
    if (slots) {
      slots[2 * t] = page;
      slots[2 * t + 1] = off;
    }
  }
  return loom::ok(err);
}

// ---- paged causal prefill (paged_prefill/mod.rs) ------------------------------
// Bf16PagedPrefillSpec::new, paged_prefill/mod.rs:30-91.
loom_status_t loom_paged_prefill_spec_new(uint64_t batch, uint64_t nnz_qo, uint64_t pool,
                                          uint64_t hq, uint64_t hkv, uint64_t head_dim,
                                          uint64_t page_size, loom_paged_prefill_spec_t *out,
                                          loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (batch == 0 || nnz_qo == 0 || pool == 0 || hq == 0 || hkv == 0 || head_dim == 0 ||
      page_size == 0)
    return fail(err, LOOM_ZERO_DIMENSION);
  if (head_dim != loom::kHeadDim)
    return fail(err, LOOM_UNSUPPORTED_HEAD_DIMENSION, nullptr, loom::kHeadDim, head_dim);
  if (page_size != loom::kPageSize)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_size);
  if (hq % hkv != 0) return fail(err, LOOM_INVALID_HEAD_MAPPING, nullptr, hq, hkv);
  if (nnz_qo > (uint64_t)INT32_MAX) return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  uint64_t t;
  if (batch == UINT64_MAX || mul_ovf(nnz_qo, hq, &t) || mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  if (mul_ovf(pool, page_size, &t) || mul_ovf(t, hkv, &t) || mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->batch_size = batch;
  out->nnz_qo = nnz_qo;
  out->max_num_pages = pool;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / std::sqrt((float)head_dim);
  out->kv_layout = LOOM_KV_LAYOUT_NHD;
  out->page_size = (uint32_t)loom::kPageSize;
  out->kv_dtype = LOOM_KV_DTYPE_BF16;
  return loom::ok(err);
}

loom_status_t loom_paged_prefill_spec_with_kv_dtype(const loom_paged_prefill_spec_t *spec,
                                                    uint32_t kv_dtype,
                                                    loom_paged_prefill_spec_t *out,
                                                    loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (kv_dtype != LOOM_KV_DTYPE_BF16 && kv_dtype != LOOM_KV_DTYPE_FP8_E4M3)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_dtype", kv_dtype);
  *out = *spec;
  out->kv_dtype = kv_dtype;
  return loom::ok(err);
}

loom_status_t loom_paged_prefill_spec_with_page_size(const loom_paged_prefill_spec_t *spec,
                                                     uint32_t page_size,
                                                     loom_paged_prefill_spec_t *out,
                                                     loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (page_size != 16 && page_size != 32 && page_size != 64)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_size);
  uint64_t t;
  if (mul_ovf(spec->max_num_pages, page_size, &t) || t > (uint64_t)INT32_MAX ||
      mul_ovf(t, spec->num_kv_heads, &t) || mul_ovf(t, loom::kHeadDim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  *out = *spec;
  out->page_size = page_size;
  return loom::ok(err);
}

loom_status_t loom_paged_prefill_spec_with_kv_layout(const loom_paged_prefill_spec_t *spec,
                                                     uint32_t kv_layout,
                                                     loom_paged_prefill_spec_t *out,
                                                     loom_error_t *err) {
  if (!spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  if (kv_layout != LOOM_KV_LAYOUT_NHD && kv_layout != LOOM_KV_LAYOUT_HND)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_layout", kv_layout);
  *out = *spec;
  out->kv_layout = kv_layout;
  return loom::ok(err);
}

// validate_metadata + validate_query_indptr, paged_prefill/mod.rs:161-264.
loom_status_t loom_paged_prefill_validate_metadata(const loom_paged_prefill_spec_t *s,
                                                   const int32_t *qo, uint64_t n_qo,
                                                   const int32_t *indptr, uint64_t n_indptr,
                                                   const int32_t *indices, uint64_t n_indices,
                                                   const int32_t *last, uint64_t n_last,
                                                   loom_error_t *err) {
  if (!s) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  const uint64_t B = s->batch_size;
  loom_status_t rc;
  if ((rc = require_len(err, "qo_indptr", n_qo, B + 1))) return rc;
  if ((rc = require_len(err, "page_indptr", n_indptr, B + 1))) return rc;
  if ((rc = require_len(err, "last_page_len", n_last, B))) return rc;
  if (qo[0] != 0) return fail(err, LOOM_INVALID_INDPTR_START, "qo_indptr", qo[0]);
  for (uint64_t r = 0; r < B; ++r) {
    if (qo[r + 1] < qo[r])
      return fail(err, LOOM_NON_MONOTONIC_INDPTR, "qo_indptr", r, qo[r], qo[r + 1]);
    if (qo[r + 1] == qo[r]) return fail(err, LOOM_EMPTY_RAGGED_REQUEST, "qo_indptr", r);
  }
  if ((rc = require_len(err, "qo_indptr", (uint64_t)qo[B], s->nnz_qo))) return rc;
  if (indptr[0] != 0) return fail(err, LOOM_INVALID_PAGE_INDPTR_START, nullptr, indptr[0]);
  for (uint64_t r = 0; r < B; ++r) {
    const int32_t a = indptr[r], b = indptr[r + 1];
    if (b < a) return fail(err, LOOM_NON_MONOTONIC_PAGE_INDPTR, nullptr, r, a, b);
    if (b == a) return fail(err, LOOM_EMPTY_PAGED_REQUEST, nullptr, r);
    if (last[r] < 1 || last[r] > (int32_t)prefill_page_rows(s))
      return fail(err, LOOM_INVALID_LAST_PAGE_LENGTH, nullptr, r, last[r], prefill_page_rows(s));
    const int64_t qo_len = (int64_t)qo[r + 1] - qo[r];
    const int64_t kv_len = kv_len_of(indptr, last, r, prefill_page_rows(s));
    if (qo_len > kv_len)
      return fail(err, LOOM_RAGGED_QUERY_LONGER_THAN_KV, nullptr, r, qo_len, kv_len);
  }
  if ((rc = require_len(err, "page_indices", n_indices, (uint64_t)indptr[B]))) return rc;
  for (uint64_t p = 0; p < n_indices; ++p)
    if (indices[p] < 0 || (uint64_t)indices[p] >= s->max_num_pages)
      return fail(err, LOOM_PAGE_INDEX_OUT_OF_RANGE, nullptr, p, indices[p], s->max_num_pages);
  return loom::ok(err);
}

// causal_kv_end, paged_prefill/mod.rs:374-383.
loom_status_t loom_paged_prefill_causal_kv_end(const loom_paged_prefill_spec_t *s,
                                               const int32_t *qo, const int32_t *indptr,
                                               const int32_t *last, uint64_t request,
                                               uint64_t query_index, uint64_t *end) {
  if (!s || !end || request >= s->batch_size) return LOOM_EMPTY_RAGGED_REQUEST;
  const int64_t qo_len = (int64_t)qo[request + 1] - qo[request];
  if ((int64_t)query_index >= qo_len) return LOOM_EMPTY_RAGGED_REQUEST;
  *end = (uint64_t)(kv_len_of(indptr, last, request, prefill_page_rows(s)) - qo_len +
                    (int64_t)query_index + 1);
  return LOOM_OK;
}

// ---- ragged causal prefill (ragged_prefill/mod.rs) -----------------------------
// Bf16RaggedPrefillSpec::new, ragged_prefill/mod.rs:27-79.
loom_status_t loom_ragged_prefill_spec_new(uint64_t batch, uint64_t nnz_qo, uint64_t nnz_kv,
                                           uint64_t hq, uint64_t hkv, uint64_t head_dim,
                                           loom_ragged_prefill_spec_t *out, loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  if (batch == 0 || nnz_qo == 0 || nnz_kv == 0 || hq == 0 || hkv == 0 || head_dim == 0)
    return fail(err, LOOM_ZERO_DIMENSION);
  if (head_dim != loom::kHeadDim)
    return fail(err, LOOM_UNSUPPORTED_HEAD_DIMENSION, nullptr, loom::kHeadDim, head_dim);
  if (hq % hkv != 0) return fail(err, LOOM_INVALID_HEAD_MAPPING, nullptr, hq, hkv);
  if (nnz_qo > (uint64_t)INT32_MAX || nnz_kv > (uint64_t)INT32_MAX)
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  uint64_t t;
  if (batch == UINT64_MAX || mul_ovf(nnz_qo, hq, &t) || mul_ovf(t, head_dim, &t) ||
      mul_ovf(nnz_kv, hkv, &t) || mul_ovf(t, head_dim, &t))
    return fail(err, LOOM_ELEMENT_COUNT_OVERFLOW);
  out->batch_size = batch;
  out->nnz_qo = nnz_qo;
  out->nnz_kv = nnz_kv;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / std::sqrt((float)head_dim);
  return loom::ok(err);
}

namespace {
// ragged_prefill/mod.rs:169-193 validate_indptr.
loom_status_t ragged_indptr(loom_error_t *err, const char *buffer, const int32_t *p,
                            uint64_t B, uint64_t total) {
  if (p[0] != 0) return fail(err, LOOM_INVALID_INDPTR_START, buffer, p[0]);
  for (uint64_t r = 0; r < B; ++r) {
    if (p[r + 1] < p[r]) return fail(err, LOOM_NON_MONOTONIC_INDPTR, buffer, r, p[r], p[r + 1]);
    if (p[r + 1] == p[r]) return fail(err, LOOM_EMPTY_RAGGED_REQUEST, buffer, r);
  }
  return require_len(err, buffer, (uint64_t)p[B], total);
}
}  // namespace

// validate_metadata, ragged_prefill/mod.rs:140-167.
loom_status_t loom_ragged_prefill_validate_metadata(const loom_ragged_prefill_spec_t *s,
                                                    const int32_t *qo, uint64_t n_qo,
                                                    const int32_t *kv, uint64_t n_kv,
                                                    loom_error_t *err) {
  if (!s) return fail(err, LOOM_NULL_ARGUMENT, "spec");
  const uint64_t B = s->batch_size;
  loom_status_t rc;
  if ((rc = require_len(err, "qo_indptr", n_qo, B + 1))) return rc;
  if ((rc = require_len(err, "kv_indptr", n_kv, B + 1))) return rc;
  if ((rc = ragged_indptr(err, "qo_indptr", qo, B, s->nnz_qo))) return rc;
  if ((rc = ragged_indptr(err, "kv_indptr", kv, B, s->nnz_kv))) return rc;
  for (uint64_t r = 0; r < B; ++r) {
    const int64_t ql = (int64_t)qo[r + 1] - qo[r], kl = (int64_t)kv[r + 1] - kv[r];
    if (ql > kl) return fail(err, LOOM_RAGGED_QUERY_LONGER_THAN_KV, nullptr, r, ql, kl);
  }
  return loom::ok(err);
}

// causal_kv_end, ragged_prefill/mod.rs:233-242.
loom_status_t loom_ragged_prefill_causal_kv_end(const loom_ragged_prefill_spec_t *s,
                                                const int32_t *qo, const int32_t *kv,
                                                uint64_t request, uint64_t query_index,
                                                uint64_t *end) {
  if (!s || !end || request >= s->batch_size) return LOOM_EMPTY_RAGGED_REQUEST;
  const int64_t ql = (int64_t)qo[request + 1] - qo[request];
  const int64_t kl = (int64_t)kv[request + 1] - kv[request];
  if ((int64_t)query_index >= ql) return LOOM_EMPTY_RAGGED_REQUEST;
  *end = (uint64_t)((int64_t)kv[request] + kl - ql + (int64_t)query_index + 1);
  return LOOM_OK;
}

}  // extern "C"
