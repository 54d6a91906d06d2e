/*
 * CPU restatement of the loom-infer reference algorithms for the paged-KV
 * decode path.  TEST INFRASTRUCTURE ONLY: this library is the parity checker
 * used by tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py.  The product library (libloom_infer_hip.so) never links, loads or
 * calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Arithmetic follows the Rust reference
 * operation by operation: `mul_add` is fmaf, `exp`/`ln`/`exp2`/`log2`/`powf`/
 * `sin`/`cos` are the C library functions the Rust std lowers to, and the file
 * is compiled with -ffp-contract=off so `a*b + c*d` rounds every product, as
 * Rust does.
 *
 * Parity pins (checked in tests/test_oracle_golden.py):
 *   - bf16 conversion, xorshift fixture and FNV digest: the reference's
 *     comparison known-answer test and the fixture digests in its evidence
 *     records;
 *   - paged decode, single decode (direct and split-K), one-token append and
 *     explicit-token append: output digests recorded in the reference's H20
 *     correctness records where the GPU matched the CPU oracle bit for bit;
 *   - paged prefill: the known-answer outputs of the reference's unit tests
 *     (bottom-right mask over physical pages, GQA head mapping with reused
 *     pages), bit equality with the pinned paged decode when every request
 *     has one query row, the fixture digests of its evidence records, and the
 *     f64 brute force (its recorded output digests come from GPU runs with
 *     bit mismatches, so they are not oracle pins);
 *   - FP8 E4M3 KV storage (no reference counterpart): the codec against
 *     torch.float8_e4m3fn (every code decoded, saturating encode of a dense
 *     sweep), the FP8 decode loop against the BF16 one on exactly
 *     representable values;
 *   - ragged prefill: output digests of the reference's ragged correctness
 *     records with 0 GPU mismatches (mha_equal_lengths, mqa_append_mixed,
 *     gqa4_mixed), its unit tests' known answers and error matrices;
 *   - validation: the known-answer mapping tables and error matrices of the
 *     reference's unit tests;
 *   - closed forms (Q=0 => mean(V), LSE=log2(L); RoPE pos 0 = identity) and
 *     an f64 brute-force softmax for tolerances.
 * Functions with no such pin: none (the LSE bits are only pinned within the
 * reference's own 1e-2 tolerance, see the golden tests).
 */
#ifndef LOOM_ORACLE_H
#define LOOM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ContractError variants, crates/loom-infer/src/error.rs:6-109, in order. */
enum lo_err {
  LO_OK = 0,
  LO_ZERO_DIMENSION = 1,
  LO_ELEMENT_COUNT_OVERFLOW = 2,
  LO_INVALID_EPSILON = 3,
  LO_UNSUPPORTED_HEAD_DIMENSION = 4,
  LO_UNSUPPORTED_PAGE_SIZE = 5,
  LO_INVALID_HEAD_MAPPING = 6,
  LO_INVALID_PARTITION_COUNT = 7,
  LO_INVALID_INDPTR_START = 8,
  LO_NON_MONOTONIC_INDPTR = 9,
  LO_EMPTY_RAGGED_REQUEST = 10,
  LO_RAGGED_QUERY_LONGER_THAN_KV = 11,
  LO_INVALID_PAGE_INDPTR_START = 12,
  LO_NON_MONOTONIC_PAGE_INDPTR = 13,
  LO_EMPTY_PAGED_REQUEST = 14,
  LO_PAGE_INDEX_OUT_OF_RANGE = 15,
  LO_INVALID_LAST_PAGE_LENGTH = 16,
  LO_INVALID_ROTARY_DIMENSION = 17,
  LO_INVALID_ROPE_SCALE = 18,
  LO_INVALID_ROPE_THETA = 19,
  LO_NEGATIVE_POSITION_ID = 20,
  LO_UNSUPPORTED_APPEND_TOKEN_COUNT = 21,
  LO_APPEND_BATCH_INDEX_OUT_OF_RANGE = 22,
  LO_APPEND_POSITION_OUT_OF_RANGE = 23,
  LO_DUPLICATE_PAGE_APPEND_SLOT = 24,
  LO_DUPLICATE_PAGE_APPEND_TOKEN_SLOT = 25,
  LO_UNSUPPORTED_DTYPE = 26,
  LO_LENGTH_MISMATCH = 27
};

/* Error payload: fields of the variant in declaration order. */
typedef struct lo_error {
  int32_t code;
  const char *buffer;
  int64_t f[4];
} lo_error;

typedef struct lo_paged_spec {
  size_t batch_size, max_num_pages, num_query_heads, num_kv_heads;
  float softmax_scale;
} lo_paged_spec;

typedef struct lo_single_spec {
  size_t kv_len, num_query_heads, num_kv_heads;
  float softmax_scale;
} lo_single_spec;

/* ---- storage helpers (half 2.7.1 bf16; validation support files) ---- */
uint16_t lo_bf16_from_f32(float value);
float lo_bf16_to_f32(uint16_t bits);
void lo_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n);
void lo_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n);
void lo_deterministic_bf16(size_t len, uint64_t salt, uint16_t *out);
uint64_t lo_digest_bf16(const uint16_t *values, size_t n);
uint64_t lo_digest_f32(const float *values, size_t n);

/* ---- paged decode contract (paged_decode/mod.rs) ---- */
int lo_paged_spec_new(size_t batch, size_t pool, size_t hq, size_t hkv,
                      size_t head_dim, size_t page_size, lo_paged_spec *out,
                      lo_error *err);
int lo_paged_validate(const lo_paged_spec *s, const int32_t *indptr,
                      size_t n_indptr, const int32_t *indices, size_t n_indices,
                      const int32_t *last, size_t n_last, lo_error *err);
/* Returns 0 and fills (page, offset) or -1 when out of range. */
int lo_paged_physical_page_for_token(const int32_t *indptr, const int32_t *indices,
                                     const int32_t *last, size_t batch, size_t request,
                                     size_t token, int64_t *page, int64_t *offset);
int64_t lo_paged_request_kv_len(const int32_t *indptr, const int32_t *last,
                                size_t batch, size_t request);
int lo_paged_decode_reference(const lo_paged_spec *s, const uint16_t *q, size_t nq,
                              const uint16_t *k, size_t nk, const uint16_t *v,
                              size_t nv, const int32_t *indptr, size_t n_indptr,
                              const int32_t *indices, size_t n_indices,
                              const int32_t *last, size_t n_last, uint16_t *out,
                              size_t nout, float *lse, size_t nlse, lo_error *err);
/* Same arithmetic restricted to requests [r0, r1): the bounded CPU-baseline
 * sample.  Metadata must already be valid. */
void lo_paged_decode_requests(const lo_paged_spec *s, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v,
                              const int32_t *indptr, const int32_t *indices,
                              const int32_t *last, size_t r0, size_t r1,
                              uint16_t *out, float *lse);

/* ---- single decode + split-K (single_decode/mod.rs) ---- */
int lo_single_spec_new(size_t kv_len, size_t hq, size_t hkv, size_t head_dim,
                       lo_single_spec *out, lo_error *err);
int lo_single_decode_reference(const lo_single_spec *s, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, uint16_t *out,
                               float *lse);
int lo_split_k_partition(size_t kv_len, size_t partitions, size_t partition,
                         size_t *start, size_t *end);
int lo_split_k_partials_reference(const lo_single_spec *s, size_t partitions,
                                  const uint16_t *q, const uint16_t *k,
                                  const uint16_t *v, float *workspace, lo_error *err);
int lo_split_k_merge_reference(const lo_single_spec *s, size_t partitions,
                               const float *workspace, uint16_t *out, float *lse,
                               lo_error *err);

/* ---- paged causal prefill (paged_prefill/mod.rs) ---- */
typedef struct lo_prefill_spec {
  size_t batch_size, nnz_qo, max_num_pages, num_query_heads, num_kv_heads;
  float softmax_scale;
} lo_prefill_spec;
int lo_prefill_spec_new(size_t batch, size_t nnz_qo, size_t pool, size_t hq, size_t hkv,
                        size_t head_dim, size_t page_size, lo_prefill_spec *out,
                        lo_error *err);
int lo_prefill_validate(const lo_prefill_spec *s, const int32_t *qo_indptr, size_t n_qo,
                        const int32_t *page_indptr, size_t n_indptr, const int32_t *indices,
                        size_t n_indices, const int32_t *last, size_t n_last, lo_error *err);
/* causal_kv_end (paged_prefill/mod.rs:374-383): -1 for the reference's None. */
int64_t lo_prefill_causal_kv_end(const lo_prefill_spec *s, const int32_t *qo_indptr,
                                 const int32_t *page_indptr, const int32_t *last,
                                 size_t request, size_t query_index);
int lo_prefill_reference(const lo_prefill_spec *s, const uint16_t *q, size_t nq,
                         const uint16_t *k, size_t nk, const uint16_t *v, size_t nv,
                         const int32_t *qo_indptr, size_t n_qo, const int32_t *page_indptr,
                         size_t n_indptr, const int32_t *indices, size_t n_indices,
                         const int32_t *last, size_t n_last, uint16_t *out, size_t nout,
                         float *lse, size_t nlse, lo_error *err);
/* The same loop restricted to requests [r0, r1) (bounded CPU-baseline sample;
 * metadata must already be valid). */
void lo_prefill_requests(const lo_prefill_spec *s, const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, const int32_t *qo_indptr,
                         const int32_t *page_indptr, const int32_t *indices,
                         const int32_t *last, size_t r0, size_t r1, uint16_t *out,
                         float *lse);

/* ---- ragged causal prefill (ragged_prefill/mod.rs) ---- */
typedef struct lo_ragged_spec {
  size_t batch_size, nnz_qo, nnz_kv, num_query_heads, num_kv_heads;
  float softmax_scale;
} lo_ragged_spec;
int lo_ragged_spec_new(size_t batch, size_t nnz_qo, size_t nnz_kv, size_t hq, size_t hkv,
                       size_t head_dim, lo_ragged_spec *out, lo_error *err);
int lo_ragged_validate(const lo_ragged_spec *s, const int32_t *qo_indptr, size_t n_qo,
                       const int32_t *kv_indptr, size_t n_kv, lo_error *err);
/* causal_kv_end (ragged_prefill/mod.rs:233-242): an absolute KV row; -1 for None. */
int64_t lo_ragged_causal_kv_end(const lo_ragged_spec *s, const int32_t *qo_indptr,
                                const int32_t *kv_indptr, size_t request, size_t query_index);
int lo_ragged_reference(const lo_ragged_spec *s, const uint16_t *q, size_t nq,
                        const uint16_t *k, size_t nk, const uint16_t *v, size_t nv,
                        const int32_t *qo_indptr, size_t n_qo, const int32_t *kv_indptr,
                        size_t n_kv, uint16_t *out, size_t nout, float *lse, size_t nlse,
                        lo_error *err);
/* Requests [r0, r1) only (bounded CPU-baseline sample; metadata valid). */
void lo_ragged_requests(const lo_ragged_spec *s, const uint16_t *q, const uint16_t *k,
                        const uint16_t *v, const int32_t *qo_indptr, const int32_t *kv_indptr,
                        size_t r0, size_t r1, uint16_t *out, float *lse);

/* ---- RoPE (rope/mod.rs) ---- */
int lo_rope_pos_ids_reference(size_t tokens, size_t qh, size_t kh, size_t head_dim,
                              size_t rotary_dim, float scale, float theta,
                              const uint16_t *q, const uint16_t *k,
                              const int32_t *pos, uint16_t *q_out, uint16_t *k_out,
                              lo_error *err);

/* ---- fused RoPE + paged append (paged_append/mod.rs) ---- */
int lo_append_validate(const lo_paged_spec *s, const int32_t *indptr, size_t n_indptr,
                       const int32_t *indices, size_t n_indices, const int32_t *last,
                       size_t n_last, lo_error *err);
int lo_append_reference(const lo_paged_spec *s, const uint16_t *q, const uint16_t *k,
                        const uint16_t *v, const int32_t *indptr, size_t n_indptr,
                        const int32_t *indices, size_t n_indices, const int32_t *last,
                        size_t n_last, uint16_t *q_out, uint16_t *k_pages,
                        uint16_t *v_pages, lo_error *err);
/* max_tokens: 64 restates the reference contract; a larger bound is the
 * extended bulk contract (same semantics, O(T^2) duplicate scan kept). */
int lo_append_tokens_validate(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                              const int32_t *batch_indices, const int32_t *positions,
                              const int32_t *indptr, size_t n_indptr,
                              const int32_t *indices, size_t n_indices,
                              const int32_t *last, size_t n_last, int64_t *slots,
                              lo_error *err);
int lo_append_tokens_reference(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                               const uint16_t *q, const uint16_t *k, const uint16_t *v,
                               const int32_t *batch_indices, const int32_t *positions,
                               const int32_t *indptr, size_t n_indptr,
                               const int32_t *indices, size_t n_indices,
                               const int32_t *last, size_t n_last, uint16_t *q_out,
                               uint16_t *k_pages, uint16_t *v_pages, lo_error *err);

/* ---- FP8 E4M3 KV storage (no reference counterpart) ---- */
uint8_t lo_fp8_e4m3_from_f32(float x);
float lo_fp8_e4m3_to_f32(uint8_t b);
void lo_fp8_e4m3_from_f32_array(const float *src, uint8_t *dst, size_t n);
void lo_fp8_e4m3_to_f32_array(const uint8_t *src, float *dst, size_t n);
void lo_paged_decode_fp8_requests(const lo_paged_spec *s, const uint16_t *q, const uint8_t *k,
                                  const uint8_t *v, const int32_t *indptr,
                                  const int32_t *indices, const int32_t *last, size_t r0,
                                  size_t r1, float k_scale, float v_scale, uint16_t *out,
                                  float *lse);
int lo_append_tokens_fp8_reference(const lo_paged_spec *s, size_t tokens, size_t max_tokens,
                                   const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                   const int32_t *batch_indices, const int32_t *positions,
                                   const int32_t *indptr, size_t n_indptr,
                                   const int32_t *indices, size_t n_indices,
                                   const int32_t *last, size_t n_last, float k_scale,
                                   float v_scale, uint16_t *q_out, uint8_t *k_pages,
                                   uint8_t *v_pages, lo_error *err);

#ifdef __cplusplus
}
#endif
#endif
