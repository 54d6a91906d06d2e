// Fused NeoX RoPE + paged K/V append for gfx950, BF16 or FP8 pages, D128, 16-64 rows per page.
//
// Semantics: crates/loom-infer/src/attention/paged_append/mod.rs:360-489 (the
// CPU reference, one-token and explicit-token forms) via
// crates/loom-infer/src/rope/mod.rs:136-161 (NeoX split-half rotation), with
// the all-or-nothing device guard of crates/loom-infer-cuda/src/rope/mod.rs
// (invalid metadata anywhere leaves every output untouched).
//
// MI355X design:
//   * one launch per command, validation once per command, not once per
//     workgroup: the grid's first workgroups each check one chunk of the
//     page-index array, the request table and the tokens' (request,
//     position, slot), one token per thread, find duplicate physical slots by
//     inserting every key into a workspace hash set with agent-scope
//     compare-and-swap (O(T) in all), and publish an epoch-tagged verdict;
//   * one workgroup per token overlaps that validation with its own work: it
//     loads its Q/K/V rows, walks the page table for its slot, computes the
//     token's 64 (sin, cos) pairs into LDS, then waits for the verdicts and,
//     if all pass, 16 lanes per 256-byte head row rotate Q/K and scatter K/V
//     rows into the page slot with 16-byte loads and stores;
//   * small commands (T <= 64, <= 4096 page indices) run as one launch in
//     which every workgroup validates the whole command itself (the
//     reference's approach), so there is no second kernel;
//   * inverse frequencies come from the host's powf (the reference's exact
//     values); angle = pos * inv_freq in FP32; products are rounded separately
//     (no FMA contraction) as in the Rust reference.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attn_device.hpp"
#include "loom_internal.hpp"

using loom::fail;

namespace {

constexpr int kValidateThreads = 256;
// Tokens per token-validation workgroup (one per thread; 64 and 128 measured
// no faster).
constexpr int kTokensPerChunk = 256;
constexpr int kApplyThreads = 256;
// Page indices per validation workgroup: at least 2048 (8 per thread), and
// enough that at most kMaxIndexBlocks workgroups check them.
constexpr int kIndicesPerValidateBlock = 2048;
constexpr int kMaxIndexBlocks = 64;
// Batches whose request table the validation workgroups keep in LDS.
constexpr int kValidateLdsBatch = 2048;
constexpr int kMaxTokens = LOOM_APPEND_MAX_TOKENS_EXTENDED;
// Commands this small run as one fused launch (every workgroup validates).
constexpr int kFusedMaxTokens = 64;
constexpr int64_t kFusedMaxIndices = 4096;
// Hash set for duplicate slots: a power of two >= 2T.
__host__ __device__ constexpr int hash_slots(int tokens) {
  int n = 64;
  while (n < 2 * tokens) n <<= 1;
  return n;
}
// Validation workgroups of a command: at most kMaxIndexBlocks for the page
// indices, then one per 256 tokens or 256 requests, whichever is more.
__host__ __device__ constexpr int64_t max_validate_blocks(int64_t tokens, int64_t batch) {
  const int64_t t = (tokens + kTokensPerChunk - 1) / kTokensPerChunk, b = (batch + 255) / 256;
  return kMaxIndexBlocks + (t > b ? t : b);
}
// Largest batch of the append contracts (the request table is indexed in 32
// bits; validation chunks cover 256 requests each).
constexpr int64_t kMaxBatch = 65536;
constexpr int kMaxValidateBlocks = (int)max_validate_blocks(kMaxTokens, kMaxBatch);
constexpr int kMaxGrid = kMaxTokens + kMaxValidateBlocks;
constexpr int kTableSlots = hash_slots(kMaxTokens);
// Workspace of the chunk-validated paths, in u32 words, one layout for every
// plan (a command queue's workspace serves all of its plans).  It must be zero
// before its first command; after that it needs no clearing: one-launch
// commands are told apart by the epoch's tags, and each command empties the
// hash table the next command will use.  The workspace therefore carries
// state (the epoch) from one command to the next; all zeros is a valid
// starting state.
//   [0, 2)   epoch (u64).  Every one-launch workgroup reads it at start and
//            tags its start word with epoch + 1; workgroup 0 advances it once
//            every start word carries that tag, i.e. once every workgroup of
//            the command has read it.
//   [2]      broken: 1 once an epoch handover gave up waiting (workgroup 0
//            then leaves the epoch as it is, so a workgroup that starts late
//            still belongs to its own command).  Every later command on this
//            workspace writes nothing and reports it, until the workspace is
//            zeroed again.
//   [3, 64)  reserved
//   started  [kMaxGrid] (u64): each workgroup's start tag, epoch + 1 (the
//            validation workgroups first, then one per token)
//   signals  [kSignalCopies][kMaxValidateBlocks] (u64): chunk b's verdict
//            (epoch + 1) * 2 + valid, written to every copy; the workgroups
//            of copy r = blockIdx % kSignalCopies poll copy r, so no word is
//            polled by more than ~T / kSignalCopies workgroups (same-address
//            accesses of many workgroups serialize)
//   tables   [2][kTableSlots]: duplicate-slot hash sets, key + 1, 0 = empty;
//            the one-launch command with epoch e inserts into table e & 1 and
//            empties table (e + 1) & 1 for the next command; a two-launch
//            command (which leaves the epoch alone) inserts into table e & 1
//            and its apply kernel empties it again
//   verdicts [kMaxValidateBlocks]: the two-launch form's chunk verdicts
//            (1 = valid), written by its validation kernel and read by its
//            apply kernel in stream order
constexpr int kWsHeaderWords = 64;
constexpr int kWsEpoch = 0, kWsBroken = 2;
constexpr int kSignalCopies = 64;
constexpr int64_t kWsStarted = kWsHeaderWords;
constexpr int64_t kWsSignals = kWsStarted + 2 * (int64_t)kMaxGrid;
constexpr int64_t kWsTables = kWsSignals + 2 * (int64_t)kSignalCopies * kMaxValidateBlocks;
constexpr int64_t kWsVerdicts = kWsTables + 2 * (int64_t)kTableSlots;
constexpr int64_t kWsWords = kWsVerdicts + kMaxValidateBlocks;
// Polls before a workgroup gives up waiting (about 0.3 s).  Reaching it means
// the validation workgroups were not scheduled in that time (for example, the
// CUs of one XCD held by long kernels of other streams or processes); the
// command then fails loudly through the queue's device status words.
constexpr int kPollLimit = 1 << 18;
struct WsLayout {
  uint64_t *started;  // workgroup g's start tag
  uint64_t *signals;  // copy r, chunk b at signals[r * kMaxValidateBlocks + b]
  uint32_t *tables;   // table p at tables + p * kTableSlots
};
__host__ __device__ constexpr int64_t ws_words(int64_t, int64_t) { return kWsWords; }
__device__ inline WsLayout ws_layout(uint32_t *ws) {
  WsLayout w;
  w.started = reinterpret_cast<uint64_t *>(ws + kWsStarted);
  w.signals = reinterpret_cast<uint64_t *>(ws + kWsSignals);
  w.tables = ws + kWsTables;
  return w;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct AppendArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  const int32_t *batch_indices;  // null: one token per request at kv_len-1
  const int32_t *positions;
  const int32_t *indptr;
  const int32_t *indices;
  const int32_t *last;
  uint16_t *q_out;
  uint16_t *k_pages;
  uint16_t *v_pages;
  uint32_t *ws;  // see WsLayout
  // The command queue's device status words (pinned host memory;
  // loom::DeviceStatus): a workgroup that cannot finish the command as
  // specified stores 1 into one of them.
  uint32_t *status;
  // Polls of a bounded wait before giving up (kPollLimit; 0 makes every wait
  // give up at once, a plan option for testing the failure path).
  int32_t poll_limit;
  int32_t index_chunk;      // page indices per index-validation workgroup
  int32_t index_blocks;     // index-validation workgroups (the first ones)
  int32_t validate_blocks;  // validation workgroups of this command
  int32_t tokens;
  int32_t batch;
  int32_t hq;
  int32_t hkv;
  int64_t pool;
  int64_t n_indices;
  // page_indices is a capacity (LOOM_PLAN_PAGE_INDICES_CAPACITY): only the
  // first indptr[B] entries are part of the page table.
  int32_t indices_capacity;
  // Page slot geometry: slot (page, off) of kv-head h starts at element
  // page * page_rows * Hkv * 128 + h * head_elems + off * row_elems (NHD: 128,
  // Hkv * 128; HND pages: page_rows * 128, 128).
  int32_t head_elems;
  int32_t row_elems;
  int32_t page_rows;  // 16, 32 or 64
  // FP8 E4M3 pages: device [k_scale, v_scale]; the pages hold fp8(x / scale)
  // bytes.  Null for BF16 pages.
  const float *kv_scales;
  float inv_freq[64];
};

// Request and token geometry shared by both kernels.  Returns false for any
// invalid mapping; on success fills the physical slot.
// Entries of page_indices that belong to the page table: all of them, or the
// first indptr[B] for capacity plans (ipB = indptr[B]).
__device__ __forceinline__ int64_t table_pages(const AppendArgs &a, int32_t ipB) {
  return a.indices_capacity ? min<int64_t>(max(ipB, 0), a.n_indices) : a.n_indices;
}
// rope/mod.rs:143-150 and paged_decode/mod.rs:164-170: indptr[0] = 0 and
// indptr[B] = len(page_indices) (<= for capacity plans).
__device__ __forceinline__ bool table_bounds_bad(const AppendArgs &a, int32_t ip0, int32_t ipB) {
  return ip0 != 0 || ipB < 0 ||
         (a.indices_capacity ? (int64_t)ipB > a.n_indices : (int64_t)ipB != a.n_indices);
}

// `ip` / `ln`: the request table (page_indptr, last_page_len), in global
// memory or an LDS copy.
// `r` / `p_given`: the token's request and (explicit form) position.
// The slot from the request's table words (st, en) = page_indptr[r, r + 1]
// and tl = last_page_len[r].
__device__ __forceinline__ bool slot_from(const AppendArgs &a, int r, int p_given, int64_t pages,
                                          int32_t st, int32_t en, int32_t tl, int *req, int *pos,
                                          int64_t *page, int *off) {
  if (st < 0 || en <= st || (int64_t)en > pages || tl < 1 || tl > a.page_rows) return false;
  const int kv_len = (en - st - 1) * a.page_rows + tl;
  const int p = a.batch_indices ? p_given : kv_len - 1;
  if (p < 0 || p >= kv_len) return false;
  const int32_t pg = a.indices[st + p / a.page_rows];
  if (pg < 0 || (int64_t)pg >= a.pool) return false;
  *req = r;
  *pos = p;
  *page = pg;
  *off = p % a.page_rows;
  return true;
}
__device__ __forceinline__ bool slot_of(const AppendArgs &a, int r, int p_given, int64_t pages,
                                        int *req, int *pos, int64_t *page, int *off,
                                        const int32_t *ip, const int32_t *ln) {
  if (r < 0 || r >= a.batch) return false;
  return slot_from(a, r, p_given, pages, ip[r], ip[r + 1], ln[r], req, pos, page, off);
}
__device__ __forceinline__ bool token_slot(const AppendArgs &a, int t, int64_t pages, int *req,
                                           int *pos, int64_t *page, int *off,
                                           const int32_t *ip, const int32_t *ln) {
  // both words in one round trip
  const int r = a.batch_indices ? a.batch_indices[t] : t;
  const int p_given = a.batch_indices ? a.positions[t] : 0;
  return slot_of(a, r, p_given, pages, req, pos, page, off, ip, ln);
}
// Token t's slot for an apply workgroup (every thread the same).  A request
// table of fewer than 64 requests comes whole, in the token words' round
// trip (each wave its own copy, in registers), so the walk is two round
// trips instead of three.
__device__ __forceinline__ bool token_slot_apply(const AppendArgs &a, int t, int tid, int64_t pages,
                                                 int *req, int *pos, int64_t *page, int *off) {
  if (a.batch >= 64) return token_slot(a, t, pages, req, pos, page, off, a.indptr, a.last);
  const int lane = tid & 63;
  const int32_t ipv = lane <= a.batch ? a.indptr[lane] : 0;
  const int32_t lnv = lane < a.batch ? a.last[lane] : 0;
  const int rg = a.batch_indices ? a.batch_indices[t] : t;
  const int pgv = a.batch_indices ? a.positions[t] : 0;
  const bool in = rg >= 0 && rg < a.batch;
  const int rs = in ? rg : 0;
  const int32_t st = __shfl(ipv, rs, 64), en = __shfl(ipv, rs + 1, 64), tl = __shfl(lnv, rs, 64);
  return in && slot_from(a, rg, pgv, pages, st, en, tl, req, pos, page, off);
}

// Stores 1 into the queue's device status word `word` (system scope: the
// words live in host memory and are read when the command is settled).
__device__ __forceinline__ void report_status(const AppendArgs &a, int word) {
  __hip_atomic_store(&a.status[word], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The workspace's epoch and broken word, read together at the start of a
// command.
struct WsEpoch {
  uint64_t epoch;
  uint32_t broken;
};
__device__ __forceinline__ WsEpoch read_epoch(const AppendArgs &a) {
  WsEpoch e;
  e.epoch = __hip_atomic_load(reinterpret_cast<uint64_t *>(a.ws + kWsEpoch), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
  e.broken = __hip_atomic_load(a.ws + kWsBroken, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return e;
}

// The words of read_epoch as of this point of the program: an empty asm that
// takes them in vector registers keeps everything computed from them (their
// moves to scalar registers, the tag, the table choice) after it, so the
// load's round trip overlaps whatever was issued before this point.
__device__ __forceinline__ WsEpoch settle(WsEpoch e) {
  asm volatile("" : "+v"(e.epoch), "+v"(e.broken));
  return e;
}

// A workgroup of the one-launch append refuses on a broken workspace (nothing
// inserted, nothing written) and otherwise tags its start word: it has read
// the epoch.  Returns whether it refused.
__device__ __forceinline__ bool refused_or_started(const AppendArgs &a, uint64_t *started,
                                                   const WsEpoch &ep, int tid) {
  if (tid == 0) {
    if (ep.broken)
      report_status(a, loom::kStatusAppendRefused);
    else
      __hip_atomic_store(&started[blockIdx.x], ep.epoch + 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  return ep.broken != 0u;
}

// Validation of chunk b, all-or-nothing.  Chunks [0, index_blocks) check the
// page indices [b*chunk, (b+1)*chunk) (rope/mod.rs:143-150), chunk 0 also
// the table bounds; chunk index_blocks + j checks requests [j*256, (j+1)*256)
// (paged_decode/mod.rs:164-205) and tokens [j*256, (j+1)*256)
// (paged_append/mod.rs:262-309), one token per thread, and inserts every
// valid slot key into the hash set, table ep.epoch & 1 of `tables`
// (agent-scope compare-and-swap, so two tokens with one slot meet whichever
// XCDs they run on; the second finds the first).  The two kinds run in different workgroups so that neither
// waits for the other's loads.  Returns nonzero if the chunk is invalid; on
// a broken workspace it inserts nothing and fails every token.
// `s_ip` / `s_last` hold kValidateLdsBatch + 1 / kValidateLdsBatch words of
// LDS; `s_or` one word per wave for the verdict.
__device__ __forceinline__ int validate_chunk(const AppendArgs &a, int b, int tid, int32_t *s_ip,
                                              int32_t *s_last, uint32_t *tables, WsEpoch ep,
                                              uint32_t (&s_or)[kValidateThreads / 64]) {
  int bad = 0;
  const int32_t ipB = a.indptr[a.batch];
  const int64_t pages = table_pages(a, ipB);
  if (b < a.index_blocks) {
    // page indices: all loads issued before any is tested
    const int32_t ip0 = a.indptr[0];
    const int64_t lo = (int64_t)b * a.index_chunk;
    const int64_t hi = min<int64_t>(lo + a.index_chunk, a.n_indices);
    int32_t pgs[kIndicesPerValidateBlock / kValidateThreads];
    for (int64_t base = lo; base < hi; base += kIndicesPerValidateBlock) {
#pragma unroll
      for (int j = 0; j < kIndicesPerValidateBlock / kValidateThreads; ++j) {
        const int64_t i = base + j * kValidateThreads + tid;
        pgs[j] = i < hi ? a.indices[i] : 0;
      }
#pragma unroll
      for (int j = 0; j < kIndicesPerValidateBlock / kValidateThreads; ++j)
        bad |= (base + j * kValidateThreads + tid < min<int64_t>(hi, pages) &&
                (pgs[j] < 0 || (int64_t)pgs[j] >= a.pool)) ? 1 : 0;
    }
    if (b == 0 && tid == 0) bad |= table_bounds_bad(a, ip0, ipB) ? 1 : 0;
    return loom_dev::block_or(bad != 0, s_or) ? 1 : 0;
  }
  const int j = b - a.index_blocks;
  // This chunk's tokens' requests and positions, its requests and the request
  // table into LDS (batches up to kValidateLdsBatch) in one round trip, so a
  // token's slot is one more.
  const int t = j * kTokensPerChunk + tid;
  const bool has_token = tid < kTokensPerChunk && t < a.tokens;
  int r_given = 0, p_given = 0;
  if (has_token) {
    r_given = a.batch_indices ? a.batch_indices[t] : t;
    p_given = a.batch_indices ? a.positions[t] : 0;
  }
  const bool lds_table = a.batch <= kValidateLdsBatch;
  if (lds_table) {
    for (int r = tid; r <= a.batch; r += kValidateThreads) {
      s_ip[r] = a.indptr[r];
      if (r < a.batch) s_last[r] = a.last[r];
    }
  }
  const int32_t *ip = lds_table ? s_ip : a.indptr;
  const int32_t *ln = lds_table ? s_last : a.last;
  const int r = j * kValidateThreads + tid;
  if (r < a.batch) {
    const int32_t st = a.indptr[r], en = a.indptr[r + 1], tl = a.last[r];
    bad |= (en <= st || tl < 1 || tl > a.page_rows) ? 1 : 0;
  }
  __syncthreads();  // the LDS request table
  ep = settle(ep);
  uint32_t *const table = ep.broken ? nullptr : tables + (ep.epoch & 1u) * kTableSlots;
  if (has_token) {
    int rr = 0, p = 0, off = 0;
    int64_t pg = 0;
    if (table && slot_of(a, r_given, p_given, pages, &rr, &p, &pg, &off, ip, ln)) {
      const uint32_t key = (uint32_t)(pg * a.page_rows + off);
      // Open addressing over the whole table (load T / kTableSlots <= 1/2):
      // every probe sequence ends at an empty entry or at the same key (a
      // duplicate slot).  The validation workgroup's verdict waits for its
      // slowest thread, and every further probe is another agent-scope round
      // trip, so the table is used at its lowest load.
      const uint32_t mask = (uint32_t)kTableSlots - 1u;
      uint32_t h = (key * 0x9E3779B1u) >> 16 & mask;
      while (true) {
        uint32_t expected = 0u;
        if (__hip_atomic_compare_exchange_strong(&table[h], &expected, key + 1u,
                                                 __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
          break;
        if (expected == key + 1u) {
          bad = 1;  // another token already holds this slot
          break;
        }
        h = (h + 1u) & mask;
      }
    } else {
      bad = 1;
    }
  }
  return loom_dev::block_or(bad != 0, s_or) ? 1 : 0;
}

// The row slices of thread `tid` for token t (Q rows, then K rows with their
// V row; rows tid / 16 + 16 i), loaded before the command's validity is known
// so the loads overlap the metadata round trips and one another.
constexpr int kPreloadRows = 3;  // row iterations preloaded: Hq + Hkv <= 48
struct RowSlice {
  u32x4 x, v;
};
struct RowSlices {
  RowSlice r[kPreloadRows];
};

__device__ __forceinline__ RowSlice load_slice(const AppendArgs &a, int t, int row, int c) {
  RowSlice f = {{0, 0, 0, 0}, {0, 0, 0, 0}};
  if (row < a.hq + a.hkv) {
    const bool is_kv = row >= a.hq;
    const uint16_t *src = is_kv ? a.k + ((int64_t)t * a.hkv + row - a.hq) * 128
                                : a.q + ((int64_t)t * a.hq + row) * 128;
    f.x = *reinterpret_cast<const u32x4 *>(src + c * 8);
    if (is_kv)
      f.v = *reinterpret_cast<const u32x4 *>(a.v + ((int64_t)t * a.hkv + row - a.hq) * 128 + c * 8);
  }
  return f;
}

__device__ __forceinline__ RowSlices load_first_slices(const AppendArgs &a, int t, int tid) {
  RowSlices f;
#pragma unroll
  for (int i = 0; i < kPreloadRows; ++i)
    f.r[i] = load_slice(a, t, (tid >> 4) + i * (kApplyThreads / 16), tid & 15);
  return f;
}

// (sin, cos) of the token's 64 angles into LDS, by threads 0..63.
__device__ __forceinline__ void token_sincos(const AppendArgs &a, int pos, int tid, float *s_sin,
                                             float *s_cos) {
  if (tid < 64) {
    const float angle = (float)pos * a.inv_freq[tid];
    // sin/cos of the FP32 angle evaluated in FP64 and rounded once: the
    // correctly rounded FP32 value.  The host C library's sinf / cosf (which
    // the reference calls) are within one FP32 ulp of it and differ for about
    // 2.6% of the (sin, cos) pairs at these angles; where the rotation cancels
    // (x1*cos - x2*sin much smaller than its terms) that one-ulp difference
    // can move a small BF16 output by more than one BF16 ulp.
    const double ad = (double)angle;
    s_sin[tid] = (float)sin(ad);
    s_cos[tid] = (float)cos(ad);
  }
}

// Rotates one Q/K row slice of token t (NeoX split-half) and, for K rows,
// scatters K and V into slot (page, off): 16 lanes per 256-byte head row,
// 16-byte loads and stores.
template <bool FP8>
__device__ __forceinline__ void apply_row(const AppendArgs &a, int t, int64_t page, int off,
                                          int row, int c, const float *s_sin, const float *s_cos,
                                          const RowSlice &sl) {
  {
    const bool is_kv = row >= a.hq;
    const int kh = row - a.hq;
    const int64_t kv_dst =
        page * a.page_rows * a.hkv * 128 + (int64_t)kh * a.head_elems + (int64_t)off * a.row_elems;
    uint16_t *dst = is_kv ? a.k_pages + kv_dst : a.q_out + ((int64_t)t * a.hq + row) * 128;
    // the other half of the NeoX pair: lane c ^ 8 of the same 16-lane row
    const u32x4 x = sl.x;
    u32x4 xp;
#pragma unroll
    for (int e = 0; e < 4; ++e) xp[e] = (uint32_t)__shfl_xor((int)x[e], 8, 16);

    const bool fp8 = FP8 && is_kv;
    float y[8];
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int elem = c * 8 + e * 2 + h;
          const int pair = elem & 63;
          const float self = __uint_as_float(h ? (x[e] & 0xffff0000u) : (x[e] << 16));
          const float other = __uint_as_float(h ? (xp[e] & 0xffff0000u) : (xp[e] << 16));
          const float cs = s_cos[pair], sn = s_sin[pair];
          // first half: first*cos - second*sin; second half: second*cos + first*sin
          y[2 * e + h] = (c < 8) ? (self * cs - other * sn) : (self * cs + other * sn);
        }
      }
    }
    const u32x4 vv = sl.v;
    if (fp8) {
      // FP8 pages: the FP32 rotated K and the V row, divided by their scales
      // (correctly rounded) and encoded; 8 bytes per lane.
      const float ks = a.kv_scales[0], vs = a.kv_scales[1];
      loom_dev::u32x2 k8 = {0, 0}, v8 = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float vf = __uint_as_float((i & 1) ? (vv[i >> 1] & 0xffff0000u) : (vv[i >> 1] << 16));
        k8[i >> 2] |= loom_dev::fp8_e4m3_from_f32(y[i] / ks) << (8 * (i & 3));
        v8[i >> 2] |= loom_dev::fp8_e4m3_from_f32(vf / vs) << (8 * (i & 3));
      }
      uint8_t *kp = reinterpret_cast<uint8_t *>(a.k_pages) + kv_dst + c * 8;
      uint8_t *vp = reinterpret_cast<uint8_t *>(a.v_pages) + kv_dst + c * 8;
      __builtin_nontemporal_store(k8, reinterpret_cast<loom_dev::u32x2 *>(kp));
      __builtin_nontemporal_store(v8, reinterpret_cast<loom_dev::u32x2 *>(vp));
      return;
    }
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = loom_dev::bf16x2_pack(y[2 * e], y[2 * e + 1]);
    // Streaming stores: nothing in this command reads them back, and dirty
    // L2 lines would only be written back at the end of the kernel.
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(dst + c * 8));
    if (is_kv) __builtin_nontemporal_store(vv, reinterpret_cast<u32x4 *>(a.v_pages + kv_dst + c * 8));
  }
}

// Rotates the Q/K rows of token t and scatters its K/V rows into slot
// (page, off).
template <bool FP8>
__device__ __forceinline__ void apply_token(const AppendArgs &a, int t, int64_t page, int off,
                                            int tid, const float *s_sin, const float *s_cos,
                                            const RowSlices &pre) {
  const int c = tid & 15;
  const int rows = a.hq + a.hkv;
  int row = tid >> 4;
#pragma unroll
  for (int it = 0; it < kPreloadRows + 1; ++it) {
    // rows beyond the preloaded iterations (Hq + Hkv > 48) load in a loop
    if (it == kPreloadRows) {
      for (; row < rows; row += kApplyThreads / 16) {
        const RowSlice one = load_slice(a, t, row, c);
        apply_row<FP8>(a, t, page, off, row, c, s_sin, s_cos, one);
      }
      break;
    }
    if (row >= rows) break;
    apply_row<FP8>(a, t, page, off, row, c, s_sin, s_cos, pre.r[it]);
    row += kApplyThreads / 16;
  }
}

// One launch per command.  Workgroups 0..V-1 each validate one chunk of the
// command (validate_chunk) and publish the chunk's verdict, tagged with the
// command's epoch, to every signal copy, then empty their share of the hash
// table the next command will use; every token workgroup meanwhile loads its
// token's Q/K/V row slices, walks the page table for its own slot and
// computes the token's (sin, cos) pairs, then polls one signal copy until all
// V verdicts carry this command's tag and applies the token only if every
// chunk is valid.  The decision rests on the polled words alone, so no
// acquire or release fence is needed.  Last, workgroup 0 waits until every
// workgroup has tagged its start word and advances the epoch for the next
// command (stream order, graph replays).
//
// Progress: the validation workgroups wait for nothing before publishing, and
// workgroup 0 waits for start tags only after publishing, so every other
// workgroup can finish and free its place.  Whether the validation
// workgroups get a CU before the token workgroups' waits run out depends on
// the dispatcher: the hardware dispatches a launch's workgroups in index
// order on each XCD (the V <= 320 validation workgroups come first), but HIP
// does not promise it, and other streams or processes may hold the CUs of an
// XCD for longer than a wait lasts.  Every wait is therefore bounded
// (poll_limit), and a give-up is never silent:
//   * a token workgroup that gives up writes nothing and reports
//     kStatusAppendVerdictWait.  The verdicts it did not see cannot make an
//     invalid command write anything (every writer saw all verdicts valid),
//     so the only possible harm is a valid command applied in part, and the
//     command's completion fails (LOOM_CMD_DEVICE_STATUS);
//   * if workgroup 0's handover gives up, it leaves the epoch as it is (a
//     workgroup that starts late still reads this command's epoch and
//     belongs to this command), marks the workspace broken and reports
//     kStatusAppendHandover; every later command on the workspace then writes
//     nothing and reports kStatusAppendRefused until it is zeroed.
// Same-address atomics of many workgroups serialize (about 0.1 us each here),
// so there is no shared counter: every polled word has a few readers and one
// writer.
template <bool FP8>
__global__ __launch_bounds__(kApplyThreads) __attribute__((amdgpu_waves_per_eu(6)))
void append_validated_kernel(AppendArgs a) {
  __shared__ int32_t s_ip[kValidateLdsBatch + 1], s_last[kValidateLdsBatch];
  __shared__ uint32_t s_or[kValidateThreads / 64];
  __shared__ float s_cos[64], s_sin[64];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  const WsLayout w = ws_layout(a.ws);
  // The epoch and broken words are first needed at the slot-key inserts (a
  // validation workgroup) or the verdict polls (a token workgroup): their
  // round trip overlaps the metadata and row loads issued before those.
  const WsEpoch ep0 = read_epoch(a);

  if ((int)blockIdx.x < a.validate_blocks) {
    // validation workgroup b
    const int b = blockIdx.x;
    const int bad = validate_chunk(a, b, tid, s_ip, s_last, w.tables, ep0, s_or);
    const WsEpoch ep = settle(ep0);
    const uint64_t epoch = ep.epoch;
    const uint64_t tag = epoch + 1u;
    if (refused_or_started(a, w.started, ep, tid)) return;
    if (tid < kSignalCopies)
      __hip_atomic_store(&w.signals[tid * kMaxValidateBlocks + b], tag * 2u + (bad ? 0u : 1u),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // empty this chunk's share of the next command's table (the previous
    // command's, complete in stream order)
    uint32_t *next = w.tables + ((epoch + 1u) & 1u) * kTableSlots;
    for (int i = b * kValidateThreads + tid; i < kTableSlots; i += a.validate_blocks * kValidateThreads)
      next[i] = 0u;
    if (b != 0) return;
    // Workgroup 0 advances the epoch once every workgroup has read it.
    const int grid = (int)gridDim.x;
    int polls = 0;
    bool all_started = false;
    while (polls < a.poll_limit) {
      int mine = 1;
      for (int base = 0; base < grid; base += 4 * kValidateThreads) {
        uint64_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int g = base + k * kValidateThreads + tid;
          v[k] = g < grid ? __hip_atomic_load(&w.started[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : tag;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) mine &= v[k] == tag;
      }
      if (__syncthreads_and(mine)) {
        all_started = true;
        break;
      }
      ++polls;
      __builtin_amdgcn_s_sleep(2);
    }
    if (tid == 0) {
      if (all_started) {
        __hip_atomic_store(reinterpret_cast<uint64_t *>(a.ws + kWsEpoch), tag, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      } else {
        __hip_atomic_store(a.ws + kWsBroken, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        report_status(a, loom::kStatusAppendHandover);
      }
    }
    return;
  }

  // token workgroup t
  const int t = blockIdx.x - a.validate_blocks;
  // The token's own slot and position (the validation chunks check the same
  // walk; nothing is written unless they all pass).
  int r = 0, pos = 0, off = 0;
  int64_t page = 0;
  const int64_t pages = table_pages(a, a.indptr[a.batch]);
  if (!token_slot_apply(a, t, tid, pages, &r, &pos, &page, &off)) pos = 0, page = 0;
  // The walk has waited for loads issued after the epoch's: the start tag
  // costs no extra round trip here, and goes out before the row loads.
  const WsEpoch ep = settle(ep0);
  const uint64_t tag = ep.epoch + 1u;
  if (refused_or_started(a, w.started, ep, tid)) return;
  // Row loads after the walk: the validation's dependent loads run while the
  // memory system is not yet flooded with the command's row traffic, and the
  // rows still arrive before the verdicts.
  const RowSlices first = load_first_slices(a, t, tid);
  token_sincos(a, pos, tid, s_sin, s_cos);
  if (tid < 64) {  // wave 0 polls copy t % kSignalCopies
    const uint64_t *copy = w.signals + (t % kSignalCopies) * kMaxValidateBlocks;
    int polls = 0, ready = 0, valid = 0;
    while (polls < a.poll_limit) {
      int mine_ready = 1, mine_valid = 1;
      for (int b = tid; b < a.validate_blocks; b += 64) {
        const uint64_t v = __hip_atomic_load(&copy[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mine_ready &= (v >> 1) == tag;
        mine_valid &= (int)(v & 1u);
      }
      ready = __all(mine_ready);
      valid = __all(mine_valid);
      if (ready) break;
      ++polls;
      __builtin_amdgcn_s_sleep(2);
    }
    if (tid == 0) {
      s_bad = !(ready && valid);
      if (!ready) report_status(a, loom::kStatusAppendVerdictWait);
    }
  }
  __syncthreads();
  if (!s_bad) apply_token<FP8>(a, t, page, off, tid, s_sin, s_cos, first);
}

// Two-launch form (plan flag LOOM_PLAN_APPEND_TWO_LAUNCH), for callers that
// cannot rule out other work holding CUs while the append runs: the
// validation kernel publishes one verdict per chunk, and the apply kernel,
// ordered after it on the stream, reads them.  Nothing waits on another
// workgroup.  The epoch is read, not advanced: this form inserts slot keys
// into table e & 1 and its apply kernel empties that table again, so the
// one-launch form's invariants hold for whatever command comes next.
__global__ __launch_bounds__(kValidateThreads) void append_validate_kernel(AppendArgs a) {
  __shared__ int32_t s_ip[kValidateLdsBatch + 1], s_last[kValidateLdsBatch];
  __shared__ uint32_t s_or[kValidateThreads / 64];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const WsEpoch ep = read_epoch(a);
  int bad = 1;
  if (ep.broken) {
    if (b == 0 && tid == 0) report_status(a, loom::kStatusAppendRefused);
  } else {
    bad = validate_chunk(a, b, tid, s_ip, s_last, ws_layout(a.ws).tables, ep, s_or);
  }
  if (tid == 0)
    __hip_atomic_store(a.ws + kWsVerdicts + b, bad ? 0u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool FP8>
__global__ __launch_bounds__(kApplyThreads) __attribute__((amdgpu_waves_per_eu(6)))
void append_apply_kernel(AppendArgs a) {
  __shared__ float s_cos[64], s_sin[64];
  __shared__ uint32_t s_ok[kApplyThreads / 64];
  const int tid = threadIdx.x;
  const int t = blockIdx.x;
  const WsEpoch ep = read_epoch(a);
  // every chunk's verdict (written by the validation kernel before this one)
  int ok = 1;
  for (int b = tid; b < a.validate_blocks; b += kApplyThreads)
    ok &= (int)__hip_atomic_load(a.ws + kWsVerdicts + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int r = 0, pos = 0, off = 0;
  int64_t page = 0;
  const int64_t pages = table_pages(a, a.indptr[a.batch]);
  if (!token_slot_apply(a, t, tid, pages, &r, &pos, &page, &off)) pos = 0, page = 0;
  const RowSlices first = load_first_slices(a, t, tid);
  token_sincos(a, pos, tid, s_sin, s_cos);
  // empty this workgroup's share of the table the validation kernel filled
  if (!ep.broken) {
    uint32_t *table = ws_layout(a.ws).tables + (ep.epoch & 1u) * kTableSlots;
    for (int i = t * kApplyThreads + tid; i < kTableSlots; i += a.tokens * kApplyThreads) table[i] = 0u;
  }
  if (loom_dev::block_or(!ok, s_ok)) return;
  apply_token<FP8>(a, t, page, off, tid, s_sin, s_cos, first);
}

// Small commands (T <= 64 tokens, <= 4096 page indices): one launch.  Every
// workgroup (one per token) validates the whole command itself, as the
// reference's kernels do, and applies its own token only if all of it is
// valid, so the all-or-nothing guard needs no second kernel.
template <bool FP8>
__global__ __launch_bounds__(kApplyThreads) void append_fused_small_kernel(AppendArgs a) {
  __shared__ float s_cos[64], s_sin[64];
  __shared__ __align__(16) uint32_t s_keys[kFusedMaxTokens];
  __shared__ uint32_t s_bad[kApplyThreads / 64], s_dup[kApplyThreads / 64];
  const int tid = threadIdx.x;
  const int t = blockIdx.x;
  const RowSlices first = load_first_slices(a, t, tid);
  // Wave 1 takes this workgroup's token position straight from the metadata
  // and computes its (sin, cos) pairs while wave 0 walks the validation's
  // dependent loads.  Nothing is written unless the validation passes, and
  // then this position is the validated one (explicit tokens: positions[t];
  // one-token form: kv_len - 1 of request t).
  if (tid >= 64 && tid < 128) {
    int pos_t;
    if (a.batch_indices) {
      pos_t = a.positions[t];
    } else {
      const int32_t st = a.indptr[t], en = a.indptr[t + 1], tl = a.last[t];
      pos_t = (en - st - 1) * a.page_rows + tl - 1;
    }
    token_sincos(a, pos_t, tid - 64, s_sin, s_cos);
  }

  int bad = 0;
  const int32_t ip0 = a.indptr[0], ipB = a.indptr[a.batch];
  const int64_t pages = table_pages(a, ipB);
  // page indices (rope/mod.rs:143-150)
#pragma unroll 4
  for (int64_t i = tid; i < pages; i += kApplyThreads) {
    const int32_t pg = a.indices[i];
    bad |= (pg < 0 || (int64_t)pg >= a.pool) ? 1 : 0;
  }
  // request table (paged_decode/mod.rs:164-205)
  if (tid == 0) bad |= table_bounds_bad(a, ip0, ipB) ? 1 : 0;
  for (int r = tid; r < a.batch; r += kApplyThreads) {
    const int32_t st = a.indptr[r], en = a.indptr[r + 1], tl = a.last[r];
    bad |= (en <= st || tl < 1 || tl > a.page_rows) ? 1 : 0;
  }
  // tokens (paged_append/mod.rs:262-309)
  if (tid < a.tokens) {
    int r, p, off;
    int64_t pg;
    uint32_t key = 0xffffffffu;
    if (token_slot(a, tid, pages, &r, &p, &pg, &off, a.indptr, a.last))
      key = (uint32_t)(pg * a.page_rows + off);
    else
      bad = 1;
    s_keys[tid] = key;
  }
  if (loom_dev::block_or(bad != 0, s_bad)) return;
  // duplicate physical slots: token i against every earlier token, four
  // keys per LDS read
  int dup = 0;
  if (tid < a.tokens) {
    const uint32_t k = s_keys[tid];
    for (int j = 0; j < tid; j += 4) {
      const u32x4 kk = *reinterpret_cast<const u32x4 *>(&s_keys[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dup |= (j + e < tid && kk[e] == k) ? 1 : 0;
    }
  }
  if (loom_dev::block_or(dup != 0, s_dup)) return;
  const uint32_t key = s_keys[t];
  // key = page * page_rows + row
  apply_token<FP8>(a, t, key / (uint32_t)a.page_rows, (int)(key % (uint32_t)a.page_rows), tid, s_sin,
              s_cos, first);
}

}  // namespace

namespace loom {
uint64_t append_workspace_bytes() { return (uint64_t)kWsWords * 4; }
}  // namespace loom

struct loom_rope_provider {
  loom::DeviceInfo dev;
};

struct loom_rope_append_plan {
  loom_rope_append_plan_info_t info{};
  uint64_t max_num_pages = 0;
  uint32_t flags = 0;
  uint32_t kv_layout = LOOM_KV_LAYOUT_NHD;
  uint32_t kv_dtype = LOOM_KV_DTYPE_BF16;
  uint32_t page_rows = 16;
  float inv_freq[64];
};

extern "C" {

loom_status_t loom_rope_provider_load(int device, loom_rope_provider_t **out, loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  loom::DeviceInfo dev;
  loom_status_t rc = loom::query_device(device, &dev, err);
  if (rc) return rc;
  if (!dev.gfx950) return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, nullptr, device);
  auto *p = new loom_rope_provider;
  p->dev = dev;
  *out = p;
  return loom::ok(err);
}

void loom_rope_provider_free(loom_rope_provider_t *p) { delete p; }

static loom_status_t make_plan(const loom_paged_decode_spec_t &s, uint64_t tokens,
                               bool explicit_tokens, uint32_t flags,
                               loom_rope_append_plan_t **out, loom_error_t *err) {
  if (flags & ~(LOOM_PLAN_PAGE_INDICES_CAPACITY | LOOM_PLAN_APPEND_TWO_LAUNCH |
                LOOM_PLAN_APPEND_TEST_NO_WAIT))
    return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", flags);
  if (s.kv_layout != LOOM_KV_LAYOUT_NHD && s.kv_layout != LOOM_KV_LAYOUT_HND)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_layout", s.kv_layout);
  if (s.kv_dtype != LOOM_KV_DTYPE_BF16 && s.kv_dtype != LOOM_KV_DTYPE_FP8_E4M3)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_dtype", s.kv_dtype);
  // rope/mod.rs:628-682: states = tokens * (Hq + Hkv) must fit the grid.
  uint64_t rows = s.num_query_heads + s.num_kv_heads, states;
  if (rows < s.num_query_heads || __builtin_mul_overflow(tokens, rows, &states))
    return fail(err, LOOM_PLAN_STATE_COUNT_OVERFLOW, "RoPE");
  if (states > (uint64_t)INT32_MAX || tokens > (uint64_t)kMaxTokens)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "RoPE", states);
  // The validation chunks and the workspace layout cover batches up to
  // kMaxBatch requests.
  if (s.batch_size > (uint64_t)kMaxBatch)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "RoPE batch", s.batch_size);
  // Slot keys are page*page_rows+offset in 32 bits.
  const uint64_t page_rows = s.page_size ? s.page_size : loom::kPageSize;
  if (page_rows != 16 && page_rows != 32 && page_rows != 64)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_rows);
  if (s.max_num_pages >= (1ull << 32) / page_rows)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "RoPE page pool", s.max_num_pages);
  auto *p = new loom_rope_append_plan;
  p->info.tokens = tokens;
  p->info.batch_size = s.batch_size;
  p->info.num_query_heads = s.num_query_heads;
  p->info.num_kv_heads = s.num_kv_heads;
  p->info.explicit_tokens = explicit_tokens ? 1 : 0;
  p->info.workspace_bytes = ws_words((int64_t)tokens, (int64_t)s.batch_size) * 4;
  p->info.validate_blocks = 0;  // depends on the bound page_indices length
  p->max_num_pages = s.max_num_pages;
  p->flags = flags;
  p->kv_layout = s.kv_layout;
  p->kv_dtype = s.kv_dtype;
  p->page_rows = (uint32_t)page_rows;
  // rope/mod.rs:148-149 with rope_scale = 1, rope_theta = 1e4, rotary_dim = 128
  // (paged_append/mod.rs:395-403): the reference's exact FP32 inverse frequencies.
  for (int i = 0; i < 64; ++i) {
    const float exponent = 2.0f * (float)i / 128.0f;
    p->inv_freq[i] = std::pow(10000.0f, -exponent) / 1.0f;
  }
  *out = p;
  return loom::ok(err);
}

loom_status_t loom_rope_provider_plan_bf16_paged_append(const loom_rope_provider_t *provider,
                                                        const loom_rope_append_spec_t *spec,
                                                        loom_rope_append_plan_t **out,
                                                        loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  return make_plan(spec->paged, spec->paged.batch_size, false, 0, out, err);
}

loom_status_t loom_rope_provider_plan_bf16_paged_append_flags(
    const loom_rope_provider_t *provider, const loom_rope_append_spec_t *spec, uint32_t flags,
    loom_rope_append_plan_t **out, loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  return make_plan(spec->paged, spec->paged.batch_size, false, flags, out, err);
}

loom_status_t loom_rope_provider_plan_bf16_paged_append_tokens(
    const loom_rope_provider_t *provider, const loom_rope_append_tokens_spec_t *spec,
    loom_rope_append_plan_t **out, loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  return make_plan(spec->paged, spec->tokens, true, 0, out, err);
}

loom_status_t loom_rope_provider_plan_bf16_paged_append_tokens_flags(
    const loom_rope_provider_t *provider, const loom_rope_append_tokens_spec_t *spec,
    uint32_t flags, loom_rope_append_plan_t **out, loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  return make_plan(spec->paged, spec->tokens, true, flags, out, err);
}

void loom_rope_append_plan_free(loom_rope_append_plan_t *p) { delete p; }

void loom_rope_append_plan_get_info(const loom_rope_append_plan_t *p,
                                    loom_rope_append_plan_info_t *info) {
  if (p && info) *info = p->info;
}

}  // extern "C"

namespace {

// enqueue_into, rope/mod.rs:758-830 / :846-934.  `hs_all` holds the thirteen
// handles of loom_rope_append_args_t; with `queue_ws` the validation words
// live in the command queue's zero-initialised workspace and the workspace
// handle is not an operand.
loom_status_t rope_append_enqueue_impl(const loom_rope_append_plan_t *plan,
                                       loom_command_scope_t *scope, const loom_handle_t *hs_all,
                                       bool queue_ws, loom_error_t *err) {
  const loom_rope_append_plan_info_t &pi = plan->info;
  const bool ex = pi.explicit_tokens != 0;
  // Operand order of Bf16RopePagedKvAppend{,Tokens}Args (rope/mod.rs:963-1047).
  const bool fp8 = plan->kv_dtype == LOOM_KV_DTYPE_FP8_E4M3;
  if (fp8 && queue_ws)  // the reference-shaped args carry no scales
    return fail(err, LOOM_ENQ_LENGTH_MISMATCH, "kv_scales", 2, 0);
  const loom_dtype_t kv_t = fp8 ? LOOM_DTYPE_U8 : LOOM_DTYPE_BF16;
  loom::OperandSpec ops[13] = {
      {"query", LOOM_DTYPE_BF16, false},        {"key", LOOM_DTYPE_BF16, false},
      {"value", LOOM_DTYPE_BF16, false},        {"batch_indices", LOOM_DTYPE_I32, false},
      {"positions", LOOM_DTYPE_I32, false},     {"page_indptr", LOOM_DTYPE_I32, false},
      {"page_indices", LOOM_DTYPE_I32, false},  {"last_page_len", LOOM_DTYPE_I32, false},
      {"query_output", LOOM_DTYPE_BF16, true},  {"key_pages", kv_t, true},
      {"value_pages", kv_t, true},              {"workspace", LOOM_DTYPE_U8, true},
      {"kv_scales", LOOM_DTYPE_F32, false}};
  // The one-token form has no batch_indices/positions operands; only FP8
  // plans take kv_scales.
  loom::OperandSpec sel_ops[13];
  loom_handle_t sel[13];
  int map[13];
  int n = 0;
  for (int i = 0; i < 13; ++i) {
    if (!ex && (i == 3 || i == 4)) continue;
    if (queue_ws && i == 11) continue;
    if (!fp8 && i == 12) continue;
    sel_ops[n] = ops[i];
    sel[n] = hs_all[i];
    map[i] = n++;
  }
  const loom::Lease *l[13];
  loom_status_t rc = loom::resolve_command(scope, sel, sel_ops, n, l, err);
  if (rc) return rc;
  if (fp8 && l[map[12]]->numel != 2)
    return fail(err, LOOM_ENQ_LENGTH_MISMATCH, "kv_scales", 2, l[map[12]]->numel);
  auto L = [&](int i) { return l[map[i]]; };
  const uint64_t T = pi.tokens, B = pi.batch_size, hq = pi.num_query_heads,
                 hkv = pi.num_kv_heads;
  const uint64_t kvn = plan->max_num_pages * plan->page_rows * hkv * loom::kHeadDim;
  struct Want {
    int i;
    uint64_t n;
  };
  const Want wants[] = {{0, T * hq * 128}, {1, T * hkv * 128}, {2, T * hkv * 128},
                        {3, T},           {4, T},             {5, B + 1},
                        {7, B},           {8, T * hq * 128},  {9, kvn},
                        {10, kvn},        {11, pi.workspace_bytes}};
  for (const Want &w : wants) {
    if (!ex && (w.i == 3 || w.i == 4)) continue;
    if (queue_ws && w.i == 11) continue;
    if (w.i == 7) {  // page_indices precedes last_page_len in the reference order
      if (L(6)->numel < B)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_SHORT, nullptr, B, L(6)->numel);
    }
    if (L(w.i)->numel != w.n)
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[w.i].name, w.n, L(w.i)->numel);
  }
  // The reference's append checks no alignment (rope/mod.rs:1062-1077): the
  // kernels' 16-byte row accesses need none on gfx950 (global and buffer
  // accesses run in unaligned mode).  The caller-owned validation workspace
  // takes 32-bit atomics and must be 16-byte aligned.
  uint32_t *ws = nullptr;
  if (queue_ws) {
    uint8_t *p = nullptr;
    rc = loom::queue_workspace(scope->queue, pi.workspace_bytes, true, &p, err);
    if (rc) return rc;
    ws = (uint32_t *)p;
  } else {
    if (L(11)->ptr % 16 != 0)
      return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, "workspace", (int64_t)L(11)->ptr, 16);
    ws = (uint32_t *)L(11)->ptr;
  }

  AppendArgs a{};
  a.q = (const uint16_t *)L(0)->ptr;
  a.k = (const uint16_t *)L(1)->ptr;
  a.v = (const uint16_t *)L(2)->ptr;
  a.batch_indices = ex ? (const int32_t *)L(3)->ptr : nullptr;
  a.positions = ex ? (const int32_t *)L(4)->ptr : nullptr;
  a.indptr = (const int32_t *)L(5)->ptr;
  a.indices = (const int32_t *)L(6)->ptr;
  a.last = (const int32_t *)L(7)->ptr;
  a.q_out = (uint16_t *)L(8)->ptr;
  a.k_pages = (uint16_t *)L(9)->ptr;
  a.v_pages = (uint16_t *)L(10)->ptr;
  a.ws = ws;
  a.tokens = (int32_t)T;
  a.batch = (int32_t)B;
  a.hq = (int32_t)hq;
  a.hkv = (int32_t)hkv;
  a.pool = (int64_t)plan->max_num_pages;
  a.n_indices = (int64_t)L(6)->numel;
  a.indices_capacity = (plan->flags & LOOM_PLAN_PAGE_INDICES_CAPACITY) ? 1 : 0;
  a.kv_scales = fp8 ? (const float *)l[map[12]]->ptr : nullptr;
  a.page_rows = (int32_t)plan->page_rows;
  a.head_elems = plan->kv_layout == LOOM_KV_LAYOUT_HND ? a.page_rows * 128 : 128;
  a.row_elems = plan->kv_layout == LOOM_KV_LAYOUT_HND ? 128 : (int32_t)hkv * 128;
  for (int i = 0; i < 64; ++i) a.inv_freq[i] = plan->inv_freq[i];

  // page-index chunks: 2048 per workgroup, or more so that at most
  // kMaxIndexBlocks workgroups check them (a multiple of 2048)
  const uint64_t n_idx = L(6)->numel;
  const uint64_t per_block = (n_idx + kMaxIndexBlocks - 1) / kMaxIndexBlocks;
  const uint64_t chunk = std::max<uint64_t>(
      kIndicesPerValidateBlock,
      (per_block + kIndicesPerValidateBlock - 1) / kIndicesPerValidateBlock * kIndicesPerValidateBlock);
  const uint64_t iblocks = std::max<uint64_t>(1, (n_idx + chunk - 1) / chunk);
  const uint64_t vblocks = iblocks + std::max<uint64_t>({1, (T + kTokensPerChunk - 1) / kTokensPerChunk,
                                                         (B + kValidateThreads - 1) / kValidateThreads});
  a.index_chunk = (int32_t)chunk;
  a.index_blocks = (int32_t)iblocks;
  a.validate_blocks = (int32_t)vblocks;
  a.status = scope->queue->status_dev;
  a.poll_limit = (plan->flags & LOOM_PLAN_APPEND_TEST_NO_WAIT) ? 0 : kPollLimit;
  hipStream_t stream = scope->queue->stream;
  if (T <= (uint64_t)kFusedMaxTokens && (int64_t)L(6)->numel <= kFusedMaxIndices) {
    hipLaunchKernelGGL(fp8 ? append_fused_small_kernel<true> : append_fused_small_kernel<false>,
                       dim3((unsigned)T), dim3(kApplyThreads), 0,
                       stream, a);
    return loom::record_launch(scope, hipGetLastError(), err);
  }
  // One launch: the validation workgroups first, then one per token (the
  // plan's bounds keep both within the workspace layout).
  const uint64_t grid = vblocks + T;
  if (vblocks > (uint64_t)kMaxValidateBlocks || grid > (uint64_t)kMaxGrid)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "RoPE validation grid", grid);
  if (plan->flags & LOOM_PLAN_APPEND_TWO_LAUNCH) {
    hipLaunchKernelGGL(append_validate_kernel, dim3((unsigned)vblocks), dim3(kValidateThreads), 0,
                       stream, a);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) {
      hipLaunchKernelGGL(fp8 ? append_apply_kernel<true> : append_apply_kernel<false>,
                         dim3((unsigned)T), dim3(kApplyThreads), 0, stream, a);
      e = hipGetLastError();
    }
    return loom::record_launch(scope, e, err);
  }
  hipLaunchKernelGGL(fp8 ? append_validated_kernel<true> : append_validated_kernel<false>,
                     dim3((unsigned)grid), dim3(kApplyThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  return loom::record_launch(scope, e, err);
}

}  // namespace

extern "C" {

loom_status_t loom_rope_append_enqueue(const loom_rope_append_plan_t *plan,
                                       loom_command_scope_t *scope,
                                       const loom_rope_append_args_t *args, loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_handle_t hs[13] = {args->query,        args->key,           args->value,
                                args->batch_indices, args->positions,    args->page_indptr,
                                args->page_indices, args->last_page_len, args->query_output,
                                args->key_pages,    args->value_pages,   args->workspace,
                                args->kv_scales};
  return rope_append_enqueue_impl(plan, scope, hs, false, err);
}

loom_status_t loom_rope_append_enqueue_bf16(const loom_rope_append_plan_t *plan,
                                            loom_command_scope_t *scope,
                                            const loom_bf16_rope_paged_kv_append_args_t *args,
                                            loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  if (plan->info.explicit_tokens)  // the tokens plan takes the tokens args
    return fail(err, LOOM_NULL_ARGUMENT, "args");
  const loom_handle_t none{0, 0};
  const loom_handle_t hs[13] = {args->query,        args->key,           args->value,
                                none,               none,                args->page_indptr,
                                args->page_indices, args->last_page_len, args->query_output,
                                args->key_pages,    args->value_pages,   none,
                                none};
  return rope_append_enqueue_impl(plan, scope, hs, true, err);
}

loom_status_t loom_rope_append_tokens_enqueue_bf16(
    const loom_rope_append_plan_t *plan, loom_command_scope_t *scope,
    const loom_bf16_rope_paged_kv_append_tokens_args_t *args, loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  if (!plan->info.explicit_tokens)  // the one-token plan takes the one-token args
    return fail(err, LOOM_NULL_ARGUMENT, "args");
  const loom_handle_t none{0, 0};
  const loom_handle_t hs[13] = {args->query,        args->key,           args->value,
                                args->batch_indices, args->positions,    args->page_indptr,
                                args->page_indices, args->last_page_len, args->query_output,
                                args->key_pages,    args->value_pages,   none,
                                none};
  return rope_append_enqueue_impl(plan, scope, hs, true, err);
}

}  // extern "C"
