/*
 * CPU restatement of the loom-infer reference (TEST INFRASTRUCTURE ONLY).
 * See loom_oracle.h for scope, pins and the arithmetic-order rules.
 * Build: oracle/build_oracle.sh (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include "loom_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 128u
#define PAGE_SIZE 16u
#define APPEND_MAX_TOKENS 64u
#define STATE_WIDTH (HEAD_DIM + 2u)
/* core::f32::consts::LOG2_E */
static const float LOG2E_F32 = 1.44269504088896340735992468100189214f;

static int fail(lo_error *err, int code, const char *buffer, int64_t a, int64_t b,
                int64_t c, int64_t d) {
  if (err) {
    err->code = code;
    err->buffer = buffer;
    err->f[0] = a;
    err->f[1] = b;
    err->f[2] = c;
    err->f[3] = d;
  }
  return code;
}

/* error.rs:276-290 require_len: LengthMismatch {buffer, expected, actual}. */
static int require_len(lo_error *err, const char *buffer, size_t actual, size_t expected) {
  if (actual == expected) return LO_OK;
  return fail(err, LO_LENGTH_MISMATCH, buffer, (int64_t)expected, (int64_t)actual, 0, 0);
}

/* ------------------------------------------------------------------------ */
/* half 2.7.1 bf16::from_f32 / to_f32 (Cargo.lock:232-235): round to nearest
 * even on the upper 16 bits; NaN keeps its high bits with the quiet bit set. */
uint16_t lo_bf16_from_f32(float value) {
  uint32_t x;
  memcpy(&x, &value, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  const uint32_t round_bit = 0x8000u;
  if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0)
    return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

float lo_bf16_to_f32(uint16_t bits) {
  uint32_t x = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void lo_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = lo_bf16_from_f32(src[i]);
}

void lo_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = lo_bf16_to_f32(src[i]);
}

/* crates/loom-infer-validation/src/support/fixture.rs:5-16: xorshift64
 * (13, 7, 17) from 0x9e3779b97f4a7c15 ^ salt; value ((s % 2001) - 1000)/2048. */
void lo_deterministic_bf16(size_t len, uint64_t salt, uint16_t *out) {
  uint64_t state = 0x9e3779b97f4a7c15ull ^ salt;
  for (size_t i = 0; i < len; ++i) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    int32_t sgn = (int32_t)(state % 2001u) - 1000;
    out[i] = lo_bf16_from_f32((float)sgn / 2048.0f);
  }
}

/* support/comparison.rs:6-20 digest_bf16 and the compare_bits fold. */
uint64_t lo_digest_bf16(const uint16_t *values, size_t n) {
  uint64_t d = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) d = (d ^ (uint64_t)values[i]) * 0x100000001b3ull;
  return d;
}

uint64_t lo_digest_f32(const float *values, size_t n) {
  uint64_t d = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) {
    uint32_t bits;
    memcpy(&bits, &values[i], 4);
    d = (d ^ (uint64_t)bits) * 0x100000001b3ull;
  }
  return d;
}

/* ------------------------------------------------------------------------ */
static int mul_overflows(size_t a, size_t b, size_t *out) {
  return __builtin_mul_overflow(a, b, out);
}

/* paged_decode/mod.rs:28-82 Bf16PagedBatchDecodeSpec::new. */
int lo_paged_spec_new(size_t batch, size_t pool, size_t hq, size_t hkv,
                      size_t head_dim, size_t page_size, lo_paged_spec *out,
                      lo_error *err) {
  if (batch == 0 || pool == 0 || hq == 0 || hkv == 0 || head_dim == 0 || page_size == 0)
    return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (head_dim != HEAD_DIM)
    return fail(err, LO_UNSUPPORTED_HEAD_DIMENSION, NULL, HEAD_DIM, (int64_t)head_dim, 0, 0);
  if (page_size != PAGE_SIZE)
    return fail(err, LO_UNSUPPORTED_PAGE_SIZE, NULL, PAGE_SIZE, (int64_t)page_size, 0, 0);
  if (hq % hkv != 0)
    return fail(err, LO_INVALID_HEAD_MAPPING, NULL, (int64_t)hq, (int64_t)hkv, 0, 0);
  size_t t;
  if (batch == SIZE_MAX || mul_overflows(batch, hq, &t) || mul_overflows(t, head_dim, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  if (mul_overflows(pool, page_size, &t) || mul_overflows(t, hkv, &t) ||
      mul_overflows(t, head_dim, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  out->batch_size = batch;
  out->max_num_pages = pool;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / sqrtf((float)head_dim);
  return LO_OK;
}

/* paged_decode/mod.rs:152-213 validate_page_table. */
int lo_paged_validate(const lo_paged_spec *s, const int32_t *indptr, size_t n_indptr,
                      const int32_t *indices, size_t n_indices, const int32_t *last,
                      size_t n_last, lo_error *err) {
  int rc;
  if ((rc = require_len(err, "page_indptr", n_indptr, s->batch_size + 1))) return rc;
  if ((rc = require_len(err, "last_page_len", n_last, s->batch_size))) return rc;
  if (indptr[0] != 0) return fail(err, LO_INVALID_PAGE_INDPTR_START, NULL, indptr[0], 0, 0, 0);
  for (size_t r = 0; r < s->batch_size; ++r) {
    int32_t start = indptr[r], end = indptr[r + 1];
    if (end < start)
      return fail(err, LO_NON_MONOTONIC_PAGE_INDPTR, NULL, (int64_t)r, start, end, 0);
    if (end == start) return fail(err, LO_EMPTY_PAGED_REQUEST, NULL, (int64_t)r, 0, 0, 0);
    int32_t len = last[r];
    if (len < 1 || len > (int32_t)PAGE_SIZE)
      return fail(err, LO_INVALID_LAST_PAGE_LENGTH, NULL, (int64_t)r, len, PAGE_SIZE, 0);
  }
  int32_t total = indptr[s->batch_size];
  if (total < 0) return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  if ((rc = require_len(err, "page_indices", n_indices, (size_t)total))) return rc;
  for (size_t p = 0; p < n_indices; ++p) {
    int32_t idx = indices[p];
    if (idx < 0 || (size_t)idx >= s->max_num_pages)
      return fail(err, LO_PAGE_INDEX_OUT_OF_RANGE, NULL, (int64_t)p, idx,
                  (int64_t)s->max_num_pages, 0);
  }
  return LO_OK;
}

/* paged_decode/mod.rs:252-257 request_kv_len. */
int64_t lo_paged_request_kv_len(const int32_t *indptr, const int32_t *last, size_t batch,
                                size_t request) {
  if (request >= batch) return -1;
  int64_t pages = (int64_t)indptr[request + 1] - (int64_t)indptr[request];
  return (pages - 1) * (int64_t)PAGE_SIZE + (int64_t)last[request];
}

/* paged_decode/mod.rs:260-278 physical_page_for_token. */
int lo_paged_physical_page_for_token(const int32_t *indptr, const int32_t *indices,
                                     const int32_t *last, size_t batch, size_t request,
                                     size_t token, int64_t *page, int64_t *offset) {
  int64_t kv_len = lo_paged_request_kv_len(indptr, last, batch, request);
  if (kv_len < 0 || (int64_t)token >= kv_len) return -1;
  size_t slot = token / PAGE_SIZE;
  *page = indices[(size_t)indptr[request] + slot];
  *offset = (int64_t)(token % PAGE_SIZE);
  return 0;
}

static inline float dot_bf16(const uint16_t *q, const uint16_t *k) {
  float sum = 0.0f;
  for (unsigned c = 0; c < HEAD_DIM; ++c)
    sum = fmaf(lo_bf16_to_f32(q[c]), lo_bf16_to_f32(k[c]), sum);
  return sum;
}

/* paged_decode/mod.rs:305-363: the per-(request, query head) loop. */
void lo_paged_decode_requests(const lo_paged_spec *s, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v,
                              const int32_t *indptr, const int32_t *indices,
                              const int32_t *last, size_t r0, size_t r1, uint16_t *out,
                              float *lse) {
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  float state[HEAD_DIM];
  for (size_t r = r0; r < r1; ++r) {
    int64_t kv_len = lo_paged_request_kv_len(indptr, last, s->batch_size, r);
    size_t page_start = (size_t)indptr[r];
    for (size_t h = 0; h < hq; ++h) {
      const uint16_t *qrow = q + (r * hq + h) * HEAD_DIM;
      size_t kvh = h / group;
      float max_score = 0.0f, normalizer = 0.0f;
      memset(state, 0, sizeof(state));
      for (int64_t t = 0; t < kv_len; ++t) {
        size_t page = (size_t)indices[page_start + (size_t)t / PAGE_SIZE];
        size_t off = (size_t)t % PAGE_SIZE;
        size_t kv_off = ((page * PAGE_SIZE + off) * hkv + kvh) * HEAD_DIM;
        float score = dot_bf16(qrow, k + kv_off) * s->softmax_scale;
        if (t == 0) {
          max_score = score;
          normalizer = 1.0f;
          for (unsigned c = 0; c < HEAD_DIM; ++c) state[c] = lo_bf16_to_f32(v[kv_off + c]);
          continue;
        }
        float next_max = fmaxf(max_score, score);
        float prev_w = expf(max_score - next_max);
        float cur_w = expf(score - next_max);
        normalizer = normalizer * prev_w + cur_w;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          state[c] = state[c] * prev_w + lo_bf16_to_f32(v[kv_off + c]) * cur_w;
        max_score = next_max;
      }
      uint16_t *orow = out + (r * hq + h) * HEAD_DIM;
      for (unsigned c = 0; c < HEAD_DIM; ++c) orow[c] = lo_bf16_from_f32(state[c] / normalizer);
      lse[r * hq + h] = (max_score + logf(normalizer)) * LOG2E_F32;
    }
  }
}

/* paged_decode/mod.rs:287-366 paged_batch_decode_bf16_reference. */
int lo_paged_decode_reference(const lo_paged_spec *s, const uint16_t *q, size_t nq,
                              const uint16_t *k, size_t nk, const uint16_t *v, size_t nv,
                              const int32_t *indptr, size_t n_indptr,
                              const int32_t *indices, size_t n_indices,
                              const int32_t *last, size_t n_last, uint16_t *out,
                              size_t nout, float *lse, size_t nlse, lo_error *err) {
  const size_t qn = s->batch_size * s->num_query_heads * HEAD_DIM;
  const size_t kvn = s->max_num_pages * PAGE_SIZE * s->num_kv_heads * HEAD_DIM;
  int rc;
  if ((rc = require_len(err, "Q", nq, qn))) return rc;
  if ((rc = require_len(err, "K_pages", nk, kvn))) return rc;
  if ((rc = require_len(err, "V_pages", nv, kvn))) return rc;
  if ((rc = require_len(err, "O", nout, qn))) return rc;
  if ((rc = require_len(err, "LSE", nlse, s->batch_size * s->num_query_heads))) return rc;
  if ((rc = lo_paged_validate(s, indptr, n_indptr, indices, n_indices, last, n_last, err)))
    return rc;
  lo_paged_decode_requests(s, q, k, v, indptr, indices, last, 0, s->batch_size, out, lse);
  return LO_OK;
}

/* ------------------------------------------------------------------------ */
/* single_decode/mod.rs:30-68 Bf16SingleDecodeSpec::new. */
int lo_single_spec_new(size_t kv_len, size_t hq, size_t hkv, size_t head_dim,
                       lo_single_spec *out, lo_error *err) {
  if (kv_len == 0 || hq == 0 || hkv == 0 || head_dim == 0)
    return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (head_dim != HEAD_DIM)
    return fail(err, LO_UNSUPPORTED_HEAD_DIMENSION, NULL, HEAD_DIM, (int64_t)head_dim, 0, 0);
  if (hq % hkv != 0)
    return fail(err, LO_INVALID_HEAD_MAPPING, NULL, (int64_t)hq, (int64_t)hkv, 0, 0);
  size_t t;
  if (mul_overflows(hq, head_dim, &t) || mul_overflows(hkv, head_dim, &t) ||
      mul_overflows(kv_len, t, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  out->kv_len = kv_len;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / sqrtf((float)head_dim);
  return LO_OK;
}

/* single_decode/mod.rs:200-261 single_decode_bf16_reference. */
int lo_single_decode_reference(const lo_single_spec *s, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, uint16_t *out,
                               float *lse) {
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  float state[HEAD_DIM];
  for (size_t h = 0; h < hq; ++h) {
    const uint16_t *qrow = q + h * HEAD_DIM;
    size_t kvh = h / group;
    float max_score = 0.0f, normalizer = 0.0f;
    memset(state, 0, sizeof(state));
    for (size_t t = 0; t < s->kv_len; ++t) {
      size_t kv_off = (t * hkv + kvh) * HEAD_DIM;
      float score = dot_bf16(qrow, k + kv_off) * s->softmax_scale;
      if (t == 0) {
        max_score = score;
        normalizer = 1.0f;
        for (unsigned c = 0; c < HEAD_DIM; ++c) state[c] = lo_bf16_to_f32(v[kv_off + c]);
        continue;
      }
      float next_max = fmaxf(max_score, score);
      float prev_w = expf(max_score - next_max);
      float cur_w = expf(score - next_max);
      normalizer = normalizer * prev_w + cur_w;
      for (unsigned c = 0; c < HEAD_DIM; ++c)
        state[c] = state[c] * prev_w + lo_bf16_to_f32(v[kv_off + c]) * cur_w;
      max_score = next_max;
    }
    for (unsigned c = 0; c < HEAD_DIM; ++c)
      out[h * HEAD_DIM + c] = lo_bf16_from_f32(state[c] / normalizer);
    lse[h] = (max_score + logf(normalizer)) * LOG2E_F32;
  }
  return LO_OK;
}

/* single_decode/mod.rs:171-185 partition_token_range. */
int lo_split_k_partition(size_t kv_len, size_t partitions, size_t partition, size_t *start,
                         size_t *end) {
  if (partition >= partitions) return -1;
  size_t base = kv_len / partitions, rem = kv_len % partitions;
  size_t extra_before = partition < rem ? partition : rem;
  *start = partition * base + extra_before;
  *end = *start + base + (partition < rem ? 1 : 0);
  return 0;
}

static int split_k_check(const lo_single_spec *s, size_t partitions, lo_error *err) {
  /* single_decode/mod.rs:131-145 Bf16SingleDecodeSplitKSpec::new. */
  if (partitions == 0 || partitions > s->kv_len)
    return fail(err, LO_INVALID_PARTITION_COUNT, NULL, (int64_t)partitions,
                (int64_t)s->kv_len, 0, 0);
  return LO_OK;
}

/* single_decode/mod.rs:264-329 split-K partial states [Hq, P, 130]. */
int lo_split_k_partials_reference(const lo_single_spec *s, size_t partitions,
                                  const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                  float *workspace, lo_error *err) {
  int rc;
  if ((rc = split_k_check(s, partitions, err))) return rc;
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  for (size_t h = 0; h < hq; ++h) {
    const uint16_t *qrow = q + h * HEAD_DIM;
    size_t kvh = h / group;
    for (size_t p = 0; p < partitions; ++p) {
      size_t t0, t1;
      lo_split_k_partition(s->kv_len, partitions, p, &t0, &t1);
      float *st = workspace + (h * partitions + p) * STATE_WIDTH;
      float *acc = st + 2;
      memset(acc, 0, HEAD_DIM * sizeof(float));
      float m = 0.0f, l = 0.0f;
      for (size_t t = t0; t < t1; ++t) {
        size_t kv_off = (t * hkv + kvh) * HEAD_DIM;
        float score_log2 = dot_bf16(qrow, k + kv_off) * s->softmax_scale * LOG2E_F32;
        if (t == t0) {
          m = score_log2;
          l = 1.0f;
          for (unsigned c = 0; c < HEAD_DIM; ++c) acc[c] = lo_bf16_to_f32(v[kv_off + c]);
          continue;
        }
        float next_max = fmaxf(m, score_log2);
        float prev_w = exp2f(m - next_max);
        float cur_w = exp2f(score_log2 - next_max);
        l = l * prev_w + cur_w;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          acc[c] = acc[c] * prev_w + lo_bf16_to_f32(v[kv_off + c]) * cur_w;
        m = next_max;
      }
      st[0] = m;
      st[1] = l;
    }
  }
  return LO_OK;
}

/* single_decode/mod.rs:332-381 split-K merge. */
int lo_split_k_merge_reference(const lo_single_spec *s, size_t partitions,
                               const float *workspace, uint16_t *out, float *lse,
                               lo_error *err) {
  int rc;
  if ((rc = split_k_check(s, partitions, err))) return rc;
  float merged[HEAD_DIM];
  for (size_t h = 0; h < s->num_query_heads; ++h) {
    float mm = 0.0f, ml = 0.0f;
    for (size_t p = 0; p < partitions; ++p) {
      const float *st = workspace + (h * partitions + p) * STATE_WIDTH;
      float pm = st[0], pl = st[1];
      if (p == 0) {
        mm = pm;
        ml = pl;
        memcpy(merged, st + 2, sizeof(merged));
        continue;
      }
      float next_max = fmaxf(mm, pm);
      float mw = exp2f(mm - next_max);
      float pw = exp2f(pm - next_max);
      ml = ml * mw + pl * pw;
      for (unsigned c = 0; c < HEAD_DIM; ++c) merged[c] = merged[c] * mw + st[2 + c] * pw;
      mm = next_max;
    }
    for (unsigned c = 0; c < HEAD_DIM; ++c)
      out[h * HEAD_DIM + c] = lo_bf16_from_f32(merged[c] / ml);
    lse[h] = mm + log2f(ml);
  }
  return LO_OK;
}

/* ------------------------------------------------------------------------ */
/* rope/mod.rs:136-161 rotate_tensor (NeoX split-half). */
/* One head row rotated in FP32 (the values rotate_tensor rounds to BF16). */
static void rotate_row_f32(const uint16_t *in, int32_t pos, size_t head_dim, size_t rotary_dim,
                           float scale, float theta, float *out) {
  size_t half = rotary_dim / 2;
  for (size_t p = 0; p < half; ++p) {
    float exponent = 2.0f * (float)p / (float)rotary_dim;
    float inv_freq = powf(theta, -exponent) / scale;
    float angle = (float)pos * inv_freq;
    float sn = sinf(angle), cs = cosf(angle);
    float first = lo_bf16_to_f32(in[p]);
    float second = lo_bf16_to_f32(in[half + p]);
    out[p] = first * cs - second * sn;
    out[half + p] = second * cs + first * sn;
  }
  for (size_t c = rotary_dim; c < head_dim; ++c) out[c] = lo_bf16_to_f32(in[c]);
}

/* rope/mod.rs:136-161 rotate_tensor (NeoX split-half). */
static void rotate_tensor(const uint16_t *in, const int32_t *pos, size_t tokens,
                          uint16_t *out, size_t heads, size_t head_dim, size_t rotary_dim,
                          float scale, float theta) {
  float row[HEAD_DIM];
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t h = 0; h < heads; ++h) {
      size_t base = (t * heads + h) * head_dim;
      rotate_row_f32(in + base, pos[t], head_dim, rotary_dim, scale, theta, row);
      for (size_t c = 0; c < rotary_dim; ++c) out[base + c] = lo_bf16_from_f32(row[c]);
      for (size_t c = rotary_dim; c < head_dim; ++c) out[base + c] = in[base + c];
    }
  }
}

/* rope/mod.rs:21-63 spec checks + rope/mod.rs:111-134 reference. */
int lo_rope_pos_ids_reference(size_t tokens, size_t qh, size_t kh, size_t head_dim,
                              size_t rotary_dim, float scale, float theta,
                              const uint16_t *q, const uint16_t *k, const int32_t *pos,
                              uint16_t *q_out, uint16_t *k_out, lo_error *err) {
  if (tokens == 0 || qh == 0 || kh == 0 || head_dim == 0)
    return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (rotary_dim == 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim)
    return fail(err, LO_INVALID_ROTARY_DIMENSION, NULL, (int64_t)rotary_dim,
                (int64_t)head_dim, 0, 0);
  if (!isfinite(scale) || scale <= 0.0f)
    return fail(err, LO_INVALID_ROPE_SCALE, NULL, 0, 0, 0, 0);
  if (!isfinite(theta) || theta <= 1.0f)
    return fail(err, LO_INVALID_ROPE_THETA, NULL, 0, 0, 0, 0);
  for (size_t t = 0; t < tokens; ++t)
    if (pos[t] < 0) return fail(err, LO_NEGATIVE_POSITION_ID, NULL, (int64_t)t, pos[t], 0, 0);
  rotate_tensor(q, pos, tokens, q_out, qh, head_dim, rotary_dim, scale, theta);
  rotate_tensor(k, pos, tokens, k_out, kh, head_dim, rotary_dim, scale, theta);
  return LO_OK;
}

/* ------------------------------------------------------------------------ */
/* paged_append/mod.rs:95-131: the extended page table plus the pairwise
 * duplicate final-slot scan in (first, second) order. */
int lo_append_validate(const lo_paged_spec *s, const int32_t *indptr, size_t n_indptr,
                       const int32_t *indices, size_t n_indices, const int32_t *last,
                       size_t n_last, lo_error *err) {
  int rc = lo_paged_validate(s, indptr, n_indptr, indices, n_indices, last, n_last, err);
  if (rc) return rc;
  const size_t b = s->batch_size;
  for (size_t i = 0; i < b; ++i) {
    int64_t pi, oi;
    lo_paged_physical_page_for_token(indptr, indices, last, b, i,
                                     (size_t)lo_paged_request_kv_len(indptr, last, b, i) - 1,
                                     &pi, &oi);
    for (size_t j = i + 1; j < b; ++j) {
      int64_t pj, oj;
      lo_paged_physical_page_for_token(indptr, indices, last, b, j,
                                       (size_t)lo_paged_request_kv_len(indptr, last, b, j) - 1,
                                       &pj, &oj);
      if (pi == pj && oi == oj)
        return fail(err, LO_DUPLICATE_PAGE_APPEND_SLOT, NULL, (int64_t)i, (int64_t)j, pi, oi);
    }
  }
  return LO_OK;
}

static void copy_slot(const lo_paged_spec *s, int64_t page, int64_t off, size_t src_row,
                      const uint16_t *rot_k, const uint16_t *v, uint16_t *k_pages,
                      uint16_t *v_pages) {
  const size_t hkv = s->num_kv_heads;
  for (size_t h = 0; h < hkv; ++h) {
    size_t src = (src_row * hkv + h) * HEAD_DIM;
    size_t dst = (((size_t)page * PAGE_SIZE + (size_t)off) * hkv + h) * HEAD_DIM;
    memcpy(k_pages + dst, rot_k + src, HEAD_DIM * 2);
    memcpy(v_pages + dst, v + src, HEAD_DIM * 2);
  }
}

/* paged_append/mod.rs:360-425 rope_paged_kv_append_bf16_reference.  Buffer
 * lengths are implied by the spec here (checked by the callers). */
int lo_append_reference(const lo_paged_spec *s, const uint16_t *q, const uint16_t *k,
                        const uint16_t *v, const int32_t *indptr, size_t n_indptr,
                        const int32_t *indices, size_t n_indices, const int32_t *last,
                        size_t n_last, uint16_t *q_out, uint16_t *k_pages,
                        uint16_t *v_pages, lo_error *err) {
  int rc = lo_append_validate(s, indptr, n_indptr, indices, n_indices, last, n_last, err);
  if (rc) return rc;
  const size_t b = s->batch_size;
  int32_t *pos = malloc(b * sizeof(int32_t));
  uint16_t *rot_k = malloc(b * s->num_kv_heads * HEAD_DIM * 2);
  for (size_t r = 0; r < b; ++r) pos[r] = (int32_t)(lo_paged_request_kv_len(indptr, last, b, r) - 1);
  rc = lo_rope_pos_ids_reference(b, s->num_query_heads, s->num_kv_heads, HEAD_DIM, HEAD_DIM,
                                 1.0f, 10000.0f, q, k, pos, q_out, rot_k, err);
  if (rc == LO_OK) {
    for (size_t r = 0; r < b; ++r) {
      int64_t page, off;
      lo_paged_physical_page_for_token(indptr, indices, last, b, r, (size_t)pos[r], &page, &off);
      copy_slot(s, page, off, r, rot_k, v, k_pages, v_pages);
    }
  }
  free(pos);
  free(rot_k);
  return rc;
}

/* paged_append/mod.rs:144-177 (token bound) + :244-317 validate_metadata. */
int lo_append_tokens_validate(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                              const int32_t *batch_indices, const int32_t *positions,
                              const int32_t *indptr, size_t n_indptr,
                              const int32_t *indices, size_t n_indices,
                              const int32_t *last, size_t n_last, int64_t *slots,
                              lo_error *err) {
  if (tokens == 0) return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (tokens > max_tokens)
    return fail(err, LO_UNSUPPORTED_APPEND_TOKEN_COUNT, NULL, (int64_t)max_tokens,
                (int64_t)tokens, 0, 0);
  int rc = lo_paged_validate(s, indptr, n_indptr, indices, n_indices, last, n_last, err);
  if (rc) return rc;
  const size_t b = s->batch_size;
  for (size_t t = 0; t < tokens; ++t) {
    int32_t bi = batch_indices[t];
    if (bi < 0 || (size_t)bi >= b)
      return fail(err, LO_APPEND_BATCH_INDEX_OUT_OF_RANGE, NULL, (int64_t)t, bi, (int64_t)b, 0);
    int64_t kv_len = lo_paged_request_kv_len(indptr, last, b, (size_t)bi);
    int32_t p = positions[t];
    int64_t page, off;
    if (p < 0 || lo_paged_physical_page_for_token(indptr, indices, last, b, (size_t)bi,
                                                  (size_t)p, &page, &off) != 0)
      return fail(err, LO_APPEND_POSITION_OUT_OF_RANGE, NULL, (int64_t)t, bi, p, kv_len);
    for (size_t f = 0; f < t; ++f)
      if (slots[2 * f] == page && slots[2 * f + 1] == off)
        return fail(err, LO_DUPLICATE_PAGE_APPEND_TOKEN_SLOT, NULL, (int64_t)f, (int64_t)t,
                    page, off);
    slots[2 * t] = page;
    slots[2 * t + 1] = off;
  }
  return LO_OK;
}

/* paged_append/mod.rs:429-489 rope_paged_kv_append_tokens_bf16_reference. */
int lo_append_tokens_reference(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                               const uint16_t *q, const uint16_t *k, const uint16_t *v,
                               const int32_t *batch_indices, const int32_t *positions,
                               const int32_t *indptr, size_t n_indptr,
                               const int32_t *indices, size_t n_indices,
                               const int32_t *last, size_t n_last, uint16_t *q_out,
                               uint16_t *k_pages, uint16_t *v_pages, lo_error *err) {
  int64_t *slots = malloc(2 * (tokens ? tokens : 1) * sizeof(int64_t));
  int rc = lo_append_tokens_validate(s, tokens, max_tokens, batch_indices, positions, indptr,
                                     n_indptr, indices, n_indices, last, n_last, slots, err);
  if (rc == LO_OK) {
    uint16_t *rot_k = malloc(tokens * s->num_kv_heads * HEAD_DIM * 2);
    rc = lo_rope_pos_ids_reference(tokens, s->num_query_heads, s->num_kv_heads, HEAD_DIM,
                                   HEAD_DIM, 1.0f, 10000.0f, q, k, positions, q_out, rot_k,
                                   err);
    if (rc == LO_OK)
      for (size_t t = 0; t < tokens; ++t)
        copy_slot(s, slots[2 * t], slots[2 * t + 1], t, rot_k, v, k_pages, v_pages);
    free(rot_k);
  }
  free(slots);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* paged_prefill/mod.rs:30-91 Bf16PagedPrefillSpec::new. */
int lo_prefill_spec_new(size_t batch, size_t nnz_qo, size_t pool, size_t hq, size_t hkv,
                        size_t head_dim, size_t page_size, lo_prefill_spec *out,
                        lo_error *err) {
  if (batch == 0 || nnz_qo == 0 || pool == 0 || hq == 0 || hkv == 0 || head_dim == 0 ||
      page_size == 0)
    return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (head_dim != HEAD_DIM)
    return fail(err, LO_UNSUPPORTED_HEAD_DIMENSION, NULL, HEAD_DIM, (int64_t)head_dim, 0, 0);
  if (page_size != PAGE_SIZE)
    return fail(err, LO_UNSUPPORTED_PAGE_SIZE, NULL, PAGE_SIZE, (int64_t)page_size, 0, 0);
  if (hq % hkv != 0)
    return fail(err, LO_INVALID_HEAD_MAPPING, NULL, (int64_t)hq, (int64_t)hkv, 0, 0);
  if (nnz_qo > (size_t)INT32_MAX) return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  size_t t;
  if (batch == SIZE_MAX || mul_overflows(nnz_qo, hq, &t) || mul_overflows(t, head_dim, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  if (mul_overflows(pool, page_size, &t) || mul_overflows(t, hkv, &t) ||
      mul_overflows(t, head_dim, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  out->batch_size = batch;
  out->nnz_qo = nnz_qo;
  out->max_num_pages = pool;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / sqrtf((float)head_dim);
  return LO_OK;
}

/* paged_prefill/mod.rs:161-274 validate_metadata and validate_query_indptr. */
int lo_prefill_validate(const lo_prefill_spec *s, const int32_t *qo, size_t n_qo,
                        const int32_t *indptr, size_t n_indptr, const int32_t *indices,
                        size_t n_indices, const int32_t *last, size_t n_last, lo_error *err) {
  int rc;
  const size_t B = s->batch_size;
  if ((rc = require_len(err, "qo_indptr", n_qo, B + 1))) return rc;
  if ((rc = require_len(err, "page_indptr", n_indptr, B + 1))) return rc;
  if ((rc = require_len(err, "last_page_len", n_last, B))) return rc;
  if (qo[0] != 0) return fail(err, LO_INVALID_INDPTR_START, "qo_indptr", qo[0], 0, 0, 0);
  for (size_t r = 0; r < B; ++r) {
    if (qo[r + 1] < qo[r])
      return fail(err, LO_NON_MONOTONIC_INDPTR, "qo_indptr", (int64_t)r, qo[r], qo[r + 1], 0);
    if (qo[r + 1] == qo[r]) return fail(err, LO_EMPTY_RAGGED_REQUEST, "qo_indptr", (int64_t)r,
                                        0, 0, 0);
  }
  if ((rc = require_len(err, "qo_indptr", (size_t)qo[B], s->nnz_qo))) return rc;
  if (indptr[0] != 0) return fail(err, LO_INVALID_PAGE_INDPTR_START, NULL, indptr[0], 0, 0, 0);
  for (size_t r = 0; r < B; ++r) {
    int32_t start = indptr[r], end = indptr[r + 1];
    if (end < start)
      return fail(err, LO_NON_MONOTONIC_PAGE_INDPTR, NULL, (int64_t)r, start, end, 0);
    if (end == start) return fail(err, LO_EMPTY_PAGED_REQUEST, NULL, (int64_t)r, 0, 0, 0);
    int32_t tail = last[r];
    if (tail < 1 || tail > (int32_t)PAGE_SIZE)
      return fail(err, LO_INVALID_LAST_PAGE_LENGTH, NULL, (int64_t)r, tail, PAGE_SIZE, 0);
    int64_t qo_len = (int64_t)qo[r + 1] - qo[r];
    int64_t kv_len = ((int64_t)end - start - 1) * (int64_t)PAGE_SIZE + tail;
    if (qo_len > kv_len)
      return fail(err, LO_RAGGED_QUERY_LONGER_THAN_KV, NULL, (int64_t)r, qo_len, kv_len, 0);
  }
  if ((rc = require_len(err, "page_indices", n_indices, (size_t)indptr[B]))) return rc;
  for (size_t p = 0; p < n_indices; ++p) {
    int32_t idx = indices[p];
    if (idx < 0 || (size_t)idx >= s->max_num_pages)
      return fail(err, LO_PAGE_INDEX_OUT_OF_RANGE, NULL, (int64_t)p, idx,
                  (int64_t)s->max_num_pages, 0);
  }
  return LO_OK;
}

/* paged_prefill/mod.rs:374-383: kv_len - qo_len + query_index + 1. */
int64_t lo_prefill_causal_kv_end(const lo_prefill_spec *s, const int32_t *qo,
                                 const int32_t *indptr, const int32_t *last, size_t request,
                                 size_t query_index) {
  if (request >= s->batch_size) return -1;
  int64_t qo_len = (int64_t)qo[request + 1] - qo[request];
  if ((int64_t)query_index >= qo_len) return -1;
  int64_t kv_len = lo_paged_request_kv_len(indptr, last, s->batch_size, request);
  return kv_len - qo_len + (int64_t)query_index + 1;
}

/* paged_prefill/mod.rs:405-446: per (query row, query head), the online
 * softmax over the causal KV prefix, in the natural-log domain; LSE is
 * converted to log2 at the end. */
void lo_prefill_requests(const lo_prefill_spec *s, const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, const int32_t *qo, const int32_t *indptr,
                         const int32_t *indices, const int32_t *last, size_t r0, size_t r1,
                         uint16_t *out, float *lse) {
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  float state[HEAD_DIM];
  for (size_t r = r0; r < r1; ++r) {
    const size_t page_start = (size_t)indptr[r];
    for (size_t row = (size_t)qo[r]; row < (size_t)qo[r + 1]; ++row) {
      const int64_t end =
          lo_prefill_causal_kv_end(s, qo, indptr, last, r, row - (size_t)qo[r]);
      for (size_t h = 0; h < hq; ++h) {
        const uint16_t *qrow = q + (row * hq + h) * HEAD_DIM;
        const size_t kvh = h / group;
        float max_score = 0.0f, normalizer = 0.0f;
        memset(state, 0, sizeof(state));
        for (int64_t t = 0; t < end; ++t) {
          size_t page = (size_t)indices[page_start + (size_t)t / PAGE_SIZE];
          size_t kv_off = ((page * PAGE_SIZE + (size_t)t % PAGE_SIZE) * hkv + kvh) * HEAD_DIM;
          float score = dot_bf16(qrow, k + kv_off) * s->softmax_scale;
          if (t == 0) {
            max_score = score;
            normalizer = 1.0f;
            for (unsigned c = 0; c < HEAD_DIM; ++c) state[c] = lo_bf16_to_f32(v[kv_off + c]);
            continue;
          }
          float next_max = fmaxf(max_score, score);
          float prev_w = expf(max_score - next_max);
          float cur_w = expf(score - next_max);
          normalizer = normalizer * prev_w + cur_w;
          for (unsigned c = 0; c < HEAD_DIM; ++c)
            state[c] = state[c] * prev_w + lo_bf16_to_f32(v[kv_off + c]) * cur_w;
          max_score = next_max;
        }
        uint16_t *orow = out + (row * hq + h) * HEAD_DIM;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          orow[c] = lo_bf16_from_f32(state[c] / normalizer);
        lse[row * hq + h] = (max_score + logf(normalizer)) * LOG2E_F32;
      }
    }
  }
}

/* paged_prefill/mod.rs:386-446 paged_prefill_bf16_reference. */
int lo_prefill_reference(const lo_prefill_spec *s, const uint16_t *q, size_t nq,
                         const uint16_t *k, size_t nk, const uint16_t *v, size_t nv,
                         const int32_t *qo, size_t n_qo, const int32_t *indptr,
                         size_t n_indptr, const int32_t *indices, size_t n_indices,
                         const int32_t *last, size_t n_last, uint16_t *out, size_t nout,
                         float *lse, size_t nlse, lo_error *err) {
  const size_t qn = s->nnz_qo * s->num_query_heads * HEAD_DIM;
  const size_t kvn = s->max_num_pages * PAGE_SIZE * s->num_kv_heads * HEAD_DIM;
  int rc;
  if ((rc = require_len(err, "Q", nq, qn))) return rc;
  if ((rc = require_len(err, "K_pages", nk, kvn))) return rc;
  if ((rc = require_len(err, "V_pages", nv, kvn))) return rc;
  if ((rc = require_len(err, "O", nout, qn))) return rc;
  if ((rc = require_len(err, "LSE", nlse, s->nnz_qo * s->num_query_heads))) return rc;
  if ((rc = lo_prefill_validate(s, qo, n_qo, indptr, n_indptr, indices, n_indices, last, n_last,
                                err)))
    return rc;
  lo_prefill_requests(s, q, k, v, qo, indptr, indices, last, 0, s->batch_size, out, lse);
  return LO_OK;
}

/* ------------------------------------------------------------------------ */
/* ragged_prefill/mod.rs:27-79 Bf16RaggedPrefillSpec::new. */
int lo_ragged_spec_new(size_t batch, size_t nnz_qo, size_t nnz_kv, size_t hq, size_t hkv,
                       size_t head_dim, lo_ragged_spec *out, lo_error *err) {
  if (batch == 0 || nnz_qo == 0 || nnz_kv == 0 || hq == 0 || hkv == 0 || head_dim == 0)
    return fail(err, LO_ZERO_DIMENSION, NULL, 0, 0, 0, 0);
  if (head_dim != HEAD_DIM)
    return fail(err, LO_UNSUPPORTED_HEAD_DIMENSION, NULL, HEAD_DIM, (int64_t)head_dim, 0, 0);
  if (hq % hkv != 0)
    return fail(err, LO_INVALID_HEAD_MAPPING, NULL, (int64_t)hq, (int64_t)hkv, 0, 0);
  if (nnz_qo > (size_t)INT32_MAX || nnz_kv > (size_t)INT32_MAX)
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  size_t t;
  if (batch == SIZE_MAX || mul_overflows(nnz_qo, hq, &t) || mul_overflows(t, head_dim, &t) ||
      mul_overflows(nnz_kv, hkv, &t) || mul_overflows(t, head_dim, &t))
    return fail(err, LO_ELEMENT_COUNT_OVERFLOW, NULL, 0, 0, 0, 0);
  out->batch_size = batch;
  out->nnz_qo = nnz_qo;
  out->nnz_kv = nnz_kv;
  out->num_query_heads = hq;
  out->num_kv_heads = hkv;
  out->softmax_scale = 1.0f / sqrtf((float)head_dim);
  return LO_OK;
}

/* ragged_prefill/mod.rs:169-193 validate_indptr. */
static int ragged_indptr(lo_error *err, const char *buffer, const int32_t *p, size_t B,
                         size_t total) {
  if (p[0] != 0) return fail(err, LO_INVALID_INDPTR_START, buffer, p[0], 0, 0, 0);
  for (size_t r = 0; r < B; ++r) {
    if (p[r + 1] < p[r]) return fail(err, LO_NON_MONOTONIC_INDPTR, buffer, (int64_t)r, p[r],
                                     p[r + 1], 0);
    if (p[r + 1] == p[r]) return fail(err, LO_EMPTY_RAGGED_REQUEST, buffer, (int64_t)r, 0, 0, 0);
  }
  return require_len(err, buffer, (size_t)p[B], total);
}

/* ragged_prefill/mod.rs:140-167 validate_metadata. */
int lo_ragged_validate(const lo_ragged_spec *s, const int32_t *qo, size_t n_qo,
                       const int32_t *kv, size_t n_kv, lo_error *err) {
  int rc;
  const size_t B = s->batch_size;
  if ((rc = require_len(err, "qo_indptr", n_qo, B + 1))) return rc;
  if ((rc = require_len(err, "kv_indptr", n_kv, B + 1))) return rc;
  if ((rc = ragged_indptr(err, "qo_indptr", qo, B, s->nnz_qo))) return rc;
  if ((rc = ragged_indptr(err, "kv_indptr", kv, B, s->nnz_kv))) return rc;
  for (size_t r = 0; r < B; ++r) {
    int64_t qo_len = (int64_t)qo[r + 1] - qo[r], kv_len = (int64_t)kv[r + 1] - kv[r];
    if (qo_len > kv_len)
      return fail(err, LO_RAGGED_QUERY_LONGER_THAN_KV, NULL, (int64_t)r, qo_len, kv_len, 0);
  }
  return LO_OK;
}

/* ragged_prefill/mod.rs:233-242: kv_start + kv_len - qo_len + query_index + 1. */
int64_t lo_ragged_causal_kv_end(const lo_ragged_spec *s, const int32_t *qo, const int32_t *kv,
                                size_t request, size_t query_index) {
  if (request >= s->batch_size) return -1;
  int64_t qo_len = (int64_t)qo[request + 1] - qo[request];
  int64_t kv_len = (int64_t)kv[request + 1] - kv[request];
  if ((int64_t)query_index >= qo_len) return -1;
  return (int64_t)kv[request] + kv_len - qo_len + (int64_t)query_index + 1;
}

/* ragged_prefill/mod.rs:262-329: the per-(query row, query head) loop. */
void lo_ragged_requests(const lo_ragged_spec *s, const uint16_t *q, const uint16_t *k,
                        const uint16_t *v, const int32_t *qo, const int32_t *kv, size_t r0,
                        size_t r1, uint16_t *out, float *lse) {
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  float state[HEAD_DIM];
  for (size_t r = r0; r < r1; ++r) {
    const int64_t kv_start = kv[r];
    for (size_t row = (size_t)qo[r]; row < (size_t)qo[r + 1]; ++row) {
      const int64_t end = lo_ragged_causal_kv_end(s, qo, kv, r, row - (size_t)qo[r]);
      for (size_t h = 0; h < hq; ++h) {
        const uint16_t *qrow = q + (row * hq + h) * HEAD_DIM;
        const size_t kvh = h / group;
        float max_score = 0.0f, normalizer = 0.0f;
        memset(state, 0, sizeof(state));
        for (int64_t t = kv_start; t < end; ++t) {
          size_t kv_off = ((size_t)t * hkv + kvh) * HEAD_DIM;
          float score = dot_bf16(qrow, k + kv_off) * s->softmax_scale;
          if (t == kv_start) {
            max_score = score;
            normalizer = 1.0f;
            for (unsigned c = 0; c < HEAD_DIM; ++c) state[c] = lo_bf16_to_f32(v[kv_off + c]);
            continue;
          }
          float next_max = fmaxf(max_score, score);
          float prev_w = expf(max_score - next_max);
          float cur_w = expf(score - next_max);
          normalizer = normalizer * prev_w + cur_w;
          for (unsigned c = 0; c < HEAD_DIM; ++c)
            state[c] = state[c] * prev_w + lo_bf16_to_f32(v[kv_off + c]) * cur_w;
          max_score = next_max;
        }
        uint16_t *orow = out + (row * hq + h) * HEAD_DIM;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          orow[c] = lo_bf16_from_f32(state[c] / normalizer);
        lse[row * hq + h] = (max_score + logf(normalizer)) * LOG2E_F32;
      }
    }
  }
}

/* ragged_prefill/mod.rs:246-329 ragged_prefill_bf16_reference. */
int lo_ragged_reference(const lo_ragged_spec *s, const uint16_t *q, size_t nq,
                        const uint16_t *k, size_t nk, const uint16_t *v, size_t nv,
                        const int32_t *qo, size_t n_qo, const int32_t *kv, size_t n_kv,
                        uint16_t *out, size_t nout, float *lse, size_t nlse, lo_error *err) {
  const size_t qn = s->nnz_qo * s->num_query_heads * HEAD_DIM;
  const size_t kvn = s->nnz_kv * s->num_kv_heads * HEAD_DIM;
  int rc;
  if ((rc = require_len(err, "Q", nq, qn))) return rc;
  if ((rc = require_len(err, "K", nk, kvn))) return rc;
  if ((rc = require_len(err, "V", nv, kvn))) return rc;
  if ((rc = require_len(err, "O", nout, qn))) return rc;
  if ((rc = require_len(err, "LSE", nlse, s->nnz_qo * s->num_query_heads))) return rc;
  if ((rc = lo_ragged_validate(s, qo, n_qo, kv, n_kv, err))) return rc;
  lo_ragged_requests(s, q, k, v, qo, kv, 0, s->batch_size, out, lse);
  return LO_OK;
}

/* ------------------------------------------------------------------------ */
/* FP8 E4M3 KV storage (no reference counterpart: the reference lists FP8 KV
 * as unsupported).  OCP E4M3 ("fn": bias 7, no infinities, 0x7F/0xFF NaN,
 * largest finite 448).  Encoding saturates finite values to +-448 and rounds
 * to nearest even; subnormals are m * 2^-9. */
uint8_t lo_fp8_e4m3_from_f32(float x) {
  if (isnan(x)) return 0x7F;
  const uint8_t s = signbit(x) ? 0x80 : 0x00;
  const float a = fabsf(x);
  if (a >= 448.0f) return s | 0x7E;
  if (a < 0.015625f) { /* below 2^-6: subnormal grid m * 2^-9 (m = 8 is 2^-6) */
    const float m = nearbyintf(a * 512.0f);
    return s | (uint8_t)m;
  }
  int e;
  const float fr = frexpf(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  int exp = e - 1;                 /* a = (2 fr) * 2^exp, 2 fr in [1, 2) */
  int m = (int)nearbyintf((2.0f * fr - 1.0f) * 8.0f);
  if (m == 8) {
    m = 0;
    ++exp;
  }
  int code = ((exp + 7) << 3) | m;
  if (code > 0x7E) code = 0x7E;
  return s | (uint8_t)code;
}

float lo_fp8_e4m3_to_f32(uint8_t b) {
  const int e = (b >> 3) & 0xF, m = b & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (b & 0x80) ? -v : v;
}

void lo_fp8_e4m3_from_f32_array(const float *src, uint8_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = lo_fp8_e4m3_from_f32(src[i]);
}

void lo_fp8_e4m3_to_f32_array(const uint8_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = lo_fp8_e4m3_to_f32(src[i]);
}

/* The paged decode loop of lo_paged_decode_requests over FP8 pages: K and V
 * elements are fp8 * k_scale and fp8 * v_scale in FP32. */
void lo_paged_decode_fp8_requests(const lo_paged_spec *s, const uint16_t *q, const uint8_t *k,
                                  const uint8_t *v, const int32_t *indptr,
                                  const int32_t *indices, const int32_t *last, size_t r0,
                                  size_t r1, float k_scale, float v_scale, uint16_t *out,
                                  float *lse) {
  const size_t hq = s->num_query_heads, hkv = s->num_kv_heads, group = hq / hkv;
  float state[HEAD_DIM];
  for (size_t r = r0; r < r1; ++r) {
    int64_t kv_len = lo_paged_request_kv_len(indptr, last, s->batch_size, r);
    size_t page_start = (size_t)indptr[r];
    for (size_t h = 0; h < hq; ++h) {
      const uint16_t *qrow = q + (r * hq + h) * HEAD_DIM;
      size_t kvh = h / group;
      float max_score = 0.0f, normalizer = 0.0f;
      memset(state, 0, sizeof(state));
      for (int64_t t = 0; t < kv_len; ++t) {
        size_t page = (size_t)indices[page_start + (size_t)t / PAGE_SIZE];
        size_t off = (size_t)t % PAGE_SIZE;
        size_t kv_off = ((page * PAGE_SIZE + off) * hkv + kvh) * HEAD_DIM;
        float dot = 0.0f;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          dot = fmaf(lo_bf16_to_f32(qrow[c]), lo_fp8_e4m3_to_f32(k[kv_off + c]) * k_scale, dot);
        float score = dot * s->softmax_scale;
        if (t == 0) {
          max_score = score;
          normalizer = 1.0f;
          for (unsigned c = 0; c < HEAD_DIM; ++c)
            state[c] = lo_fp8_e4m3_to_f32(v[kv_off + c]) * v_scale;
          continue;
        }
        float next_max = fmaxf(max_score, score);
        float prev_w = expf(max_score - next_max);
        float cur_w = expf(score - next_max);
        normalizer = normalizer * prev_w + cur_w;
        for (unsigned c = 0; c < HEAD_DIM; ++c)
          state[c] = state[c] * prev_w + lo_fp8_e4m3_to_f32(v[kv_off + c]) * v_scale * cur_w;
        max_score = next_max;
      }
      uint16_t *orow = out + (r * hq + h) * HEAD_DIM;
      for (unsigned c = 0; c < HEAD_DIM; ++c) orow[c] = lo_bf16_from_f32(state[c] / normalizer);
      lse[r * hq + h] = (max_score + logf(normalizer)) * LOG2E_F32;
    }
  }
}

/* The explicit-token append of lo_append_tokens_reference writing FP8 pages:
 * the FP32 rotated K row divided by k_scale and the V row divided by v_scale,
 * each encoded with lo_fp8_e4m3_from_f32.  The query output stays BF16. */
int lo_append_tokens_fp8_reference(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                                   const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                   const int32_t *batch_indices, const int32_t *positions,
                                   const int32_t *indptr, size_t n_indptr,
                                   const int32_t *indices, size_t n_indices,
                                   const int32_t *last, size_t n_last, float k_scale,
                                   float v_scale, uint16_t *q_out, uint8_t *k_pages,
                                   uint8_t *v_pages, lo_error *err) {
  int64_t *slots = malloc(2 * (tokens ? tokens : 1) * sizeof(int64_t));
  int rc = lo_append_tokens_validate(s, tokens, max_tokens, batch_indices, positions, indptr,
                                     n_indptr, indices, n_indices, last, n_last, slots, err);
  if (rc == LO_OK) {
    uint16_t *rot_k = malloc(tokens * s->num_kv_heads * HEAD_DIM * 2);
    rc = lo_rope_pos_ids_reference(tokens, s->num_query_heads, s->num_kv_heads, HEAD_DIM,
                                   HEAD_DIM, 1.0f, 10000.0f, q, k, positions, q_out, rot_k,
                                   err);
    free(rot_k);
    if (rc == LO_OK) {
      const size_t hkv = s->num_kv_heads;
      float row[HEAD_DIM];
      for (size_t t = 0; t < tokens; ++t)
        for (size_t h = 0; h < hkv; ++h) {
          const size_t src = (t * hkv + h) * HEAD_DIM;
          const size_t dst = (((size_t)slots[2 * t] * PAGE_SIZE + (size_t)slots[2 * t + 1]) * hkv +
                              h) * HEAD_DIM;
          rotate_row_f32(k + src, positions[t], HEAD_DIM, HEAD_DIM, 1.0f, 10000.0f, row);
          for (unsigned c = 0; c < HEAD_DIM; ++c) {
            k_pages[dst + c] = lo_fp8_e4m3_from_f32(row[c] / k_scale);
            v_pages[dst + c] = lo_fp8_e4m3_from_f32(lo_bf16_to_f32(v[src + c]) / v_scale);
          }
        }
    }
  }
  free(slots);
  return rc;
}
