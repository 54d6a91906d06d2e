// Paged decode attention for gfx950 (MI355X), D128, BF16 or FP8 pages of 16-64 rows, NHD or HND.
//
// Semantics: crates/loom-infer/src/attention/paged_decode/mod.rs:287-366 (the
// CPU reference), with the device metadata guards of
// crates/loom-infer-cuda/src/attention/decode.rs:224-248 and :430-478 (an
// invalid request keeps its output sentinels; valid requests complete).
//
// Work decomposition (MI355X-first, not the reference's warp-per-head):
//   * the pages of all valid requests form one virtual list; it is cut into
//     `teams` equal ranges, and each team is hkv x group-tiles waves, one per
//     (kv-head, tile of up to 8 query heads), all walking the same pages.  The
//     whole GQA group of a kv-head shares every K/V byte, so K/V is read from
//     HBM once per kv-head; every wave gets the same number of pages whatever
//     the lengths, and the grid is one wave per SIMD slot of the chip, so
//     there is no tail of partially filled launch rounds;
//   * the grid depends only on the plan (graph-replay safe); each workgroup
//     rebuilds the virtual list with one prefix scan of the page table;
//   * workgroup b runs on XCD b % 8, and the waves of a team are placed on one
//     XCD, so the kv-heads of a page are fetched together through one L2;
//   * per page, S = K·Qᵀ runs on MFMA (v_mfma_f32_16x16x32_bf16: 16 tokens x
//     16 query columns x 32 dims, 4 issues for D=128) with K staged through a
//     padded LDS tile; online softmax in the log2 domain (v_exp_f32); P·V on
//     the VALU in FP32;
//   * K/V rows are fetched with raw buffer loads whose range covers only the
//     valid rows of the page, so the look-ahead past a segment and the tail of
//     a request's last page move no bytes;
//   * a request inside one team's range is finished in place.  Otherwise each
//     team leaves one FP32 state per (request, query head) in the workspace,
//     (max_log2, normalizer, acc[128]) as in crates/loom-infer/src/attention/
//     single_decode/mod.rs:10-13, and a second, stream-ordered merge kernel
//     combines them.  The kernel boundary makes the states visible across the
//     8 XCD L2s; an in-kernel last-arriver merge would need an agent-scope
//     release per wave, i.e. an L2 write-back, which costs more than the launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "attn_device.hpp"
#include "loom_internal.hpp"

using loom::fail;
using namespace loom_dev;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kLdsPrefix = 512;      // requests whose prefix and metadata stay in LDS
constexpr int kMaxScanBlocks = 256;  // scan blocks of kThreads requests: batch <= 65536
// FP32 split state: (max_log2, normalizer, 2 pad, acc[128]), 16-byte aligned.
constexpr int kStateStride = 132;
// Plans whose page capacity is at most this use the direct kernel (one launch,
// no split): such calls are launch- and latency-bound.
#ifndef LOOM_DECODE_DIRECT_MAX_PAGES
#define LOOM_DECODE_DIRECT_MAX_PAGES 128
#endif
constexpr int kKRowBytes = 256 + 16;
constexpr int kKTileBytes = 16 * kKRowBytes;
#ifndef LOOM_DECODE_DEPTH
#define LOOM_DECODE_DEPTH 2
#endif
// Waves per SIMD the register allocation must allow (HIP's second launch
// bound) for the direct and single-decode kernels.  The page step's registers
// do not depend on the tile width (both products accumulate in MFMA tiles of
// 16 query columns).
#ifndef LOOM_DECODE_WAVES
#define LOOM_DECODE_WAVES 3
#endif
constexpr int waves_per_eu_for(int) { return LOOM_DECODE_WAVES; }
template <int GT>
constexpr int waves_per_eu() {
  return waves_per_eu_for(GT);
}
// Pages in flight per wave (register buffers of 32 VGPRs each).
constexpr int kDepth = LOOM_DECODE_DEPTH;
// The balanced split kernel streams fewer, deeper page streams: a register
// budget of two waves per SIMD and three pages in flight per wave, with the
// grid sized to about 13 waves per 4 CUs (planner).  Measured on MI355X over
// configs 3-5 (80..384 teams of 8 waves, depths 2-6, 1-3 waves per SIMD):
// 96-104 teams of 8 waves with three pages in flight beat the full-occupancy
// grid (384 teams, two pages) by 7-10%, and grids whose workgroups do not
// spread evenly over an XCD's 32 CUs (160, 192, 320 teams) lose 5-20%.
#ifndef LOOM_DECODE_SPLIT_DEPTH
#define LOOM_DECODE_SPLIT_DEPTH 3
#endif
#ifndef LOOM_DECODE_SPLIT_WAVES
#define LOOM_DECODE_SPLIT_WAVES 2
#endif
#ifndef LOOM_DECODE_SPLIT_WAVES_PER_4CU
#define LOOM_DECODE_SPLIT_WAVES_PER_4CU 13
#endif
// FP8 pages carry half the bytes per page step, so the page step's
// instructions, not HBM, bound a wave: the grid fills the register budget
// (2 waves per SIMD).  Measured on config 3: 256 teams 99 us, 104 teams 150 us.
#ifndef LOOM_DECODE_SPLIT_WAVES_PER_4CU_FP8
#define LOOM_DECODE_SPLIT_WAVES_PER_4CU_FP8 32
#endif
#ifndef LOOM_DECODE_SPLIT_DEPTH_FP8
#define LOOM_DECODE_SPLIT_DEPTH_FP8 3
#endif
// Pages in flight per wave of the split kernel (FP8 pages take half the
// registers per page).
template <bool FP8>
constexpr int split_depth() {
  return FP8 ? LOOM_DECODE_SPLIT_DEPTH_FP8 : LOOM_DECODE_SPLIT_DEPTH;
}
// Normalizer written into a state whose pages failed the guard.
constexpr float kPoisonNormalizer = -1.0f;


struct DecodeArgs {
  // Distinct buffers (the binding rules forbid a writable operand aliasing any
  // other), so uniform loads of the metadata can go through the scalar cache.
  const uint16_t *__restrict__ q;
  const uint16_t *__restrict__ k;
  const uint16_t *__restrict__ v;
  const int32_t *__restrict__ indptr;
  const int32_t *__restrict__ indices;
  const int32_t *__restrict__ last;
  uint16_t *__restrict__ out;
  float *__restrict__ lse;
  // Workspace: header[0] = pages in the virtual list (-1: batch rejected),
  // header[1 + r] = virtual page prefix of request r (r = 0..B); then the
  // split states [teams + B][Hq][kStateStride].
  int64_t *__restrict__ header;
  float *__restrict__ states;
  int32_t batch;
  int32_t hq;
  int32_t hkv;
  int32_t group;
  int32_t members;  // hkv * group tiles: waves per team
  int32_t teams;
  int64_t pool;
  int64_t n_indices;
  float scale_log2;
  // page_indices is a capacity: the global guard accepts indptr[B] <= its
  // length instead of requiring equality (fixed-address graphs replayed over
  // changing page tables).
  int32_t indices_capacity;
  // K/V row geometry: row t of kv-head h starts at element
  // t * Hkv * 128 + h * head_elems + (t % 16) * (row_elems - Hkv * 128), i.e.
  // NHD: head_elems 128, row_elems Hkv * 128; HND pages: head_elems 16 * 128,
  // row_elems 128 (t is a multiple of 16 for pages).  Contiguous K/V is NHD.
  int32_t head_elems;
  int32_t row_elems;
  // Token rows per page (16, 32 or 64) and log2 of the 16-row blocks per page:
  // the kernels stream 16-row blocks, block j of page p starting at token row
  // p * page_rows + 16 * j.
  int32_t page_rows;
  int32_t blocks_lg;
  int64_t page_elems;   // page_rows * Hkv * 128: elements per page (all kv-heads)
  int32_t block_elems;  // 16 * row_elems: element step between a page's blocks
  // FP8 E4M3 pages: device [k_scale, v_scale] (K = fp8 * k_scale, V = fp8 *
  // v_scale); null for BF16 pages.
  const float *__restrict__ kv_scales;
  // Direct kernel: workgroups per (request, kv-head, tile).  1: the workgroup
  // writes O and LSE; more: each writes the state of its share of the
  // request's blocks to states[((split * B + r) * Hq + qh) * kStateStride]
  // and paged_decode_direct_merge_kernel combines them.
  int32_t splits;
};

// decode.rs:233-246: indptr[B] is the page_indices length (or, for plans made
// with LOOM_PLAN_PAGE_INDICES_CAPACITY, at most that length).
__device__ __forceinline__ bool batch_pages_ok(const DecodeArgs &a, int32_t ipB) {
  return ipB >= 0 && (a.indices_capacity ? (int64_t)ipB <= a.n_indices
                                         : (int64_t)ipB == a.n_indices);
}





template <int GT>
struct Smem {
  int64_t incl[kLdsPrefix];           // inclusive page prefix, requests < kLdsPrefix
  int32_t req_st[kLdsPrefix];         // indptr[r] and last_page_len[r], same requests
  int32_t req_tl[kLdsPrefix];
  int64_t blk_excl[kMaxScanBlocks];   // exclusive page prefix of each scan block
  int64_t wave_tot[kWaves];
  // Per-wave K tile: 16 token rows of 256 bytes padded to kKRowBytes so the
  // MFMA fragment reads (16 rows, same column) hit 16 distinct bank groups.
  uint8_t ktile[kWaves][kKTileBytes];
  u32x4 qfrag[kWaves][4][64];  // per wave: MFMA B fragments of its query tile
};

// One page of K and V for one wave, both as whole 256-byte rows: lane
// (col = lane%16, quad = lane/16) holds columns [8*col, 8*col+8) of rows
// 4*quad + j, j = 0..3, so every load instruction covers four full rows.
struct PageRegs {
  u32x4 k[4];
  u32x4 v[4];
};

// 16 consecutive token rows starting at token row `token0` of the K/V
// buffers (a page of a paged cache, NHD or HND, or any 16 tokens of a
// contiguous NHD one).  `token0` and `valid_rows` are wave-uniform (the
// resource lives in SGPRs).
__device__ __forceinline__ void load_rows(PageRegs &r, const DecodeArgs &a, int64_t elem0,
                                          int valid_rows, int lane, int kvh) {
  const int col = lane & 15, quad = lane >> 4;
  const int64_t first = elem0 + (int64_t)kvh * a.head_elems;
  const __amdgpu_buffer_rsrc_t rk = page_rows_rsrc(a.k + first, valid_rows, a.row_elems);
  const __amdgpu_buffer_rsrc_t rv = page_rows_rsrc(a.v + first, valid_rows, a.row_elems);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = (quad * 4 + j) * a.row_elems * 2 + col * 16;
    r.k[j] = load16_rows<LOOM_DECODE_NT_K>(rk, off);
    r.v[j] = load16_rows<LOOM_DECODE_NT_V>(rv, off);
  }
}

// Element offset (kv-head 0) of block `sub` of page `page`.
__device__ __forceinline__ int64_t block_elem(const DecodeArgs &a, int page, int sub) {
  return (int64_t)page * a.page_elems + (int64_t)(sub * a.block_elems);
}
// Element offset (kv-head 0) of token row `token` of contiguous NHD K/V.
__device__ __forceinline__ int64_t token_elem(const DecodeArgs &a, int64_t token) {
  return token * a.hkv * 128;
}

__device__ __forceinline__ void load_page(PageRegs &r, const DecodeArgs &a, int page, int sub,
                                          int valid_rows, int lane, int kvh) {
  load_rows(r, a, block_elem(a, page, sub), valid_rows, lane, kvh);
}

// The same 16 rows stored as FP8 E4M3 (one byte per element, so a row of one
// kv-head is 128 bytes): lane (col, quad) holds 8 bytes of each of rows
// 4*quad + j.  Half the registers of a BF16 page in flight; widened to the
// BF16 PageRegs layout (exactly) when the page is consumed.
struct PageRegs8 {
  u32x2 k[4];
  u32x2 v[4];
};

template <bool FP8>
using PageBuf = typename std::conditional<FP8, PageRegs8, PageRegs>::type;

__device__ __forceinline__ void load_rows(PageRegs8 &r, const DecodeArgs &a, int64_t elem0,
                                          int valid_rows, int lane, int kvh) {
  const int col = lane & 15, quad = lane >> 4;
  const int64_t first = elem0 + (int64_t)kvh * a.head_elems;
  const uint8_t *k8 = reinterpret_cast<const uint8_t *>(a.k) + first;
  const uint8_t *v8 = reinterpret_cast<const uint8_t *>(a.v) + first;
  const int bytes = valid_rows > 0 ? (valid_rows - 1) * a.row_elems + 128 : 0;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(k8), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(v8), 0, bytes, 0x00020000);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = (quad * 4 + j) * a.row_elems + col * 8;
    r.k[j] = load8_rows<LOOM_DECODE_NT_K>(rk, off);
    r.v[j] = load8_rows<LOOM_DECODE_NT_V>(rv, off);
  }
}

__device__ __forceinline__ void load_page(PageRegs8 &r, const DecodeArgs &a, int page, int sub,
                                          int valid_rows, int lane, int kvh) {
  load_rows(r, a, block_elem(a, page, sub), valid_rows, lane, kvh);
}

// K and V row words (BF16 pairs) of a page in either form; FP8 E4M3 bytes
// widen to BF16 exactly.
__device__ __forceinline__ u32x4 k_words(const PageRegs &r, int j) { return r.k[j]; }
__device__ __forceinline__ u32x4 k_words(const PageRegs8 &r, int j) {
  return fp8x8_to_bf16x8(r.k[j]);
}
__device__ __forceinline__ u32x4 v_words(const PageRegs &r, int j) { return r.v[j]; }
__device__ __forceinline__ u32x4 v_words(const PageRegs8 &r, int j) {
  return fp8x8_to_bf16x8(r.v[j]);
}

// 16-row blocks request r contributes to the virtual block list (0 if the
// request fails the per-request guard of decode.rs:430-478, last_page_len in
// 1..page_rows): page_rows / 16 per page, ceil(last / 16) on its last page.
// With 16-row pages a block is a page.
__device__ __forceinline__ int request_pages(const DecodeArgs &a, int32_t st, int32_t en,
                                             int32_t tl, int32_t ipB) {
  const bool valid = st >= 0 && en > st && en <= ipB && tl >= 1 && tl <= a.page_rows;
  return valid ? ((en - st - 1) << a.blocks_lg) + ((tl + 15) >> 4) : 0;
}
// Valid rows of a request's last block.
__device__ __forceinline__ int last_block_rows(int32_t tl) { return ((tl - 1) & 15) + 1; }

// Teams split the virtual page list into equal ranges: team t owns
// [team_start(t), team_start(t+1)).
// floor(n / d) for 0 <= n < 2^53, d > 0, without the long 64-bit integer
// division sequence: a double-precision estimate, corrected to the exact value.
__device__ __forceinline__ int64_t floor_div(int64_t n, int64_t d) {
  int64_t q = (int64_t)((double)n / (double)d);
  while (q * d > n) --q;
  while ((q + 1) * d <= n) ++q;
  return q;
}

__device__ __forceinline__ int64_t team_start(int64_t total, int64_t t, int teams) {
  return floor_div(total * t, teams);
}
// The team whose range holds virtual page v (0 <= v < total): the largest t
// with team_start(t) <= v.
__device__ __forceinline__ int64_t team_of(int64_t total, int64_t v, int teams) {
  return floor_div((v + 1) * teams + total - 1, total) - 1;
}

// Per-wave decode of one (request, kv-head, tile of GT query heads): the
// online-softmax state over the pages the wave streams, and the page step.
// Both products run on MFMA; the accumulator acc[e][i] holds O[query column
// col][dim 32 quad + 8 i + e] (unnormalized), so every lane owns 32 output
// dims of one query column and its softmax state is the column's.
template <int GT>
struct WaveDecoder {
  const DecodeArgs &a;
  uint8_t *kt;          // this wave's K tile (16 rows of kKRowBytes)
  u32x4 (*qfrag)[64];   // [4][64] MFMA B fragments of the query tile
  int lane, col, quad, kvh;
  float m_run, l_run;
  f32x4 acc[8];

  __device__ void reset() {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Q fragment: column `col` is query head qh0 + col (zero beyond gcount);
  // MFMA c contracts dims 32c + 8*quad + [0, 8), the slices the K fragments
  // read.  `prefetched` lets the caller issue other loads before the LDS write.
  __device__ void load_q(int r, int qh0, int gcount, u32x4 (&qr)[4]) const {
    const uint16_t *qp = a.q + ((int64_t)r * a.hq + qh0 + col) * 128 + quad * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] = col < gcount ? load16(qp + c * 32) : u32x4{0, 0, 0, 0};
  }
  __device__ void store_q(const u32x4 (&qr)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) qfrag[c][lane] = qr[c];
    wave_lds_fence();
  }

  // One page: S = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ on MFMA, online softmax in between.
  // `rows` is the number of valid token rows (16, the request's tail on its
  // last page, 0 for a page index that failed the guard).
  template <class Page>
  __device__ void process(const Page &pr, int rows) {
    u32x4 kf[4];
    // K rows -> LDS tile -> MFMA A fragments (lane: token row `col`, dims
    // 32c + 8*quad + [0, 8)).
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(kt + (quad * 4 + j) * kKRowBytes + col * 16) = k_words(pr, j);
    wave_lds_fence();
#pragma unroll
    for (int c = 0; c < 4; ++c)
      kf[c] = *reinterpret_cast<const u32x4 *>(kt + col * kKRowBytes + (c * 4 + quad) * 16);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[c]), as_bf16x8(qfrag[c][lane]), s,
                                                  0, 0, 0);
    // s[i] = S[token 4 quad + i][query column col]
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = (quad * 4 + i < rows) ? s[i] * a.scale_log2 : -INFINITY;
    const float mx = quad_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
    const float m_new = fmaxf(m_run, mx);
    const float al = fast_exp2(m_run - m_new);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_new);
    l_run = l_run * al + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    // Rescale only when some column's max moved (after a stream's first pages
    // it rarely does); the branch is wave-uniform.
    if (__builtin_amdgcn_ballot_w64(al != 1.0f))
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= al;
    // Pᵀ as the B fragment of v_mfma_f32_16x16x32_bf16 (lane: query column
    // col, k = 8 quad + [0, 8)): k = 8 quad + i is token 4 quad + i with its
    // BF16 high part, k = 8 quad + 4 + i the same token's BF16 residual, so
    // each weight keeps 16 significant bits.
    uint32_t pb[4], rb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pb[i] = __float_as_uint(p[i]);
      rb[i] = __float_as_uint(p[i] - __uint_as_float(pb[i] & 0xffff0000u));
    }
    const bf16x8 pt = as_bf16x8(pack_hi16(pb[0], pb[1]), pack_hi16(pb[2], pb[3]),
                                pack_hi16(rb[0], rb[1]), pack_hi16(rb[2], rb[3]));
    // Vᵀ block e as the A fragment: row col is dim 8 col + e, k = 8 quad +
    // [0, 4) and 8 quad + 4 + [0, 4) both token 4 quad + [0, 4), straight from
    // the V rows this lane loaded.  Rows past the valid ones were loaded as
    // zeros and have zero weight.
    u32x4 vw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) vw[j] = v_words(pr, j);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = e >> 1;
      const uint32_t x01 = (e & 1) ? pack_hi16(vw[0][w], vw[1][w]) : pack_lo16(vw[0][w], vw[1][w]);
      const uint32_t x23 = (e & 1) ? pack_hi16(vw[2][w], vw[3][w]) : pack_lo16(vw[2][w], vw[3][w]);
      acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(x01, x23, x01, x23), pt, acc[e],
                                                       0, 0, 0);
    }
  }

  // Streams 16-row blocks 0..n-1 (n >= 1) through a kDepth-deep pipeline:
  // each step issues the loads of the block kDepth-1 steps ahead before
  // consuming the current one.  Loads past the end have no valid rows and
  // touch no memory; the unrolled buffer rotation lets the compiler wait for
  // exactly the oldest block's loads.  tok_of(i) (element offset of block i's
  // first row for kv-head 0)
  // and rows_of(i) must be wave-uniform.
  template <bool FP8 = false, class TokOf, class RowsOf>
  __device__ void stream(int n, TokOf tok_of, RowsOf rows_of) {
    PageBuf<FP8> buf[kDepth];
#pragma unroll
    for (int j = 0; j < kDepth - 1; ++j) load_rows(buf[j], a, tok_of(j), rows_of(j), lane, kvh);
    int i = 0;
    while (true) {
#pragma unroll
      for (int s = 0; s < kDepth; ++s) {
        load_rows(buf[(s + kDepth - 1) % kDepth], a, tok_of(i + kDepth - 1),
                  rows_of(i + kDepth - 1), lane, kvh);
        process(buf[s], rows_of(i));
        if (++i >= n) return;
      }
    }
  }

  // The column's normalizer (sum over the four row quads); acc and m_run
  // need no reduction.
  __device__ float reduce() const { return quad_sum(l_run); }
};

// Normalized output of one query column: the 32 dims acc[e][i] (dim
// 32 quad + 8 i + e) divided by the normalizer, times V's scale on FP8 pages,
// as BF16 at o[0..32).
template <bool FP8>
__device__ __forceinline__ void store_out_row(uint16_t *o, const f32x4 (&acc)[8], float l,
                                              float v_scale) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x0 = acc[2 * e][i] / l, x1 = acc[2 * e + 1][i] / l;
      if constexpr (FP8) {
        x0 *= v_scale;
        x1 *= v_scale;
      }
      w[e] = bf16x2_pack(x0, x1);
    }
    *reinterpret_cast<u32x4 *>(o + i * 8) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// Copies a wave's column state to LDS row `dst` (dims 32 quad + [0, 32)).
__device__ __forceinline__ void stash_acc(float *dst, const f32x4 (&acc)[8], int quad) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float *o = dst + quad * 32 + i * 8;
    *reinterpret_cast<f32x4 *>(o) = f32x4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
    *reinterpret_cast<f32x4 *>(o + 4) = f32x4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
  }
}

// Teams in use for `total` virtual pages: at most the planned count, and at
// least kMinTeamPages pages each (short batches are latency-bound: fewer, longer
// page streams and shorter merges beat one page per wave).
#ifndef LOOM_DECODE_MIN_TEAM_PAGES
#define LOOM_DECODE_MIN_TEAM_PAGES 4
#endif
__device__ __forceinline__ int active_teams(int64_t total, int teams) {
  const int64_t by_pages = total / LOOM_DECODE_MIN_TEAM_PAGES;
  return (int)max<int64_t>(1, min<int64_t>(teams, by_pages));
}

template <int GT, bool FP8 = false>
__global__ __launch_bounds__(kThreads, LOOM_DECODE_SPLIT_WAVES) void paged_decode_split_kv_kernel(
    DecodeArgs a) {
  __shared__ Smem<GT> sm;
  constexpr int kSD = split_depth<FP8>();
  // FP8 pages: K's scale folds into the score scale, V's into the output.
  float v_scale = 1.0f;
  if constexpr (FP8) {
    a.scale_log2 *= a.kv_scales[0];
    v_scale = a.kv_scales[1];
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps team state in SGPRs
  const int col = lane & 15, quad = lane >> 4;

  // ---- virtual page list: prefix scan of the valid requests' page counts ---
  // The guard words and the first block's metadata are loaded together (one
  // round trip); the global guard is applied after the scan.
  const int32_t ip0 = a.indptr[0];
  const int32_t ipB = a.indptr[a.batch];
  int64_t carry = 0;
  for (int base = 0, blk = 0; base < a.batch; base += kThreads, ++blk) {
    const int r = base + tid;
    int cnt = 0;
    if (r < a.batch) {
      const int32_t st = a.indptr[r], en = a.indptr[r + 1], tl = a.last[r];
      cnt = request_pages(a, st, en, tl, ipB);
      if (r < kLdsPrefix) {
        sm.req_st[r] = st;
        sm.req_tl[r] = last_block_rows(tl);
      }
    }
    const int64_t x = wave_incl_scan64(cnt, lane);
    if (lane == 63) sm.wave_tot[wave] = x;
    __syncthreads();
    int64_t before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      const int64_t t = sm.wave_tot[i];
      before += (i < wave) ? t : 0;
      tot += t;
    }
    const int64_t incl = carry + before + x;
    if (r < a.batch) {
      if (r < kLdsPrefix) sm.incl[r] = incl;
      if (blockIdx.x == 0) a.header[1 + r] = incl - cnt;
    }
    if (tid == 0) sm.blk_excl[blk] = carry;
    carry += tot;
    __syncthreads();
  }
  const int64_t total = carry;
  // Global guard (decode.rs:233-246): the whole batch is rejected, in every
  // workgroup, and the merge kernel is told through the header.
  const bool batch_ok = ip0 == 0 && batch_pages_ok(a, ipB);
  if (blockIdx.x == 0 && tid == 0) {
    a.header[0] = batch_ok ? total : -1;
    a.header[1 + a.batch] = total;
  }
  if (!batch_ok) return;

  // ---- this wave's team and member ----------------------------------------
  // Workgroup b runs on XCD b % 8.  The members of a team (the kv-heads and
  // group tiles of one page range) are consecutive waves of one XCD, so they
  // share its L2 and walk the same pages at the same time; team t lives on
  // XCD t % 8, so any number of active teams spreads over all eight.
  const int xcd_wave = (int)(blockIdx.x >> 3) * kWaves + wave;
  const int teams = active_teams(total, a.teams);
  const int team = (xcd_wave / a.members) * 8 + (int)(blockIdx.x & 7);
  const int member = xcd_wave % a.members;
  if (team >= teams) return;  // no workgroup barrier follows
  const int kvh = member % a.hkv;
  const int gt = member / a.hkv;
  const int64_t v_begin = team_start(total, team, teams);
  const int64_t v_end = team_start(total, team + 1, teams);
  if (v_begin >= v_end) return;

  // ---- the request holding v_begin ----------------------------------------
  int r;
  int64_t pre;
  {
    int found = -1;
    int64_t inc = 0;
    if (a.batch <= kLdsPrefix) {
      for (int base = 0; base < a.batch && found < 0; base += 64) {
        const int rr = base + lane;
        const int64_t x = rr < a.batch ? sm.incl[rr] : INT64_MAX;
        const uint64_t m = __ballot(x > v_begin);
        if (m) {
          found = base + __builtin_ctzll(m);
          inc = sm.incl[found];
        }
      }
    } else {
      // the scan block holding v_begin, then its requests again from memory
      int blk = 0;
      const int nblk = (a.batch + kThreads - 1) / kThreads;
      for (int b0 = 0; b0 < nblk; b0 += 64) {
        const int bb = b0 + lane;
        const uint64_t m = __ballot(bb < nblk && sm.blk_excl[bb] <= v_begin);
        if (m) blk = b0 + 63 - __builtin_clzll(m);
      }
      int64_t c = sm.blk_excl[blk];
      for (int base = blk * kThreads; found < 0 && base < a.batch; base += 64) {
        const int rr = base + lane;
        int cnt = 0;
        if (rr < a.batch) cnt = request_pages(a, a.indptr[rr], a.indptr[rr + 1], a.last[rr], ipB);
        const int64_t x = c + wave_incl_scan64(cnt, lane);
        const uint64_t m = __ballot(rr < a.batch && x > v_begin);
        if (m) {
          const int l0 = __builtin_ctzll(m);
          found = base + l0;
          inc = __shfl(x, l0, 64);
        }
        c = __shfl(x, 63, 64);
      }
    }
    if (found < 0) return;  // unreachable: v_begin < total
    r = uni(found);
    int cnt0;
    if (r < kLdsPrefix) {
      cnt0 = (int)(inc - (r > 0 ? sm.incl[r - 1] : 0));
    } else {
      cnt0 = request_pages(a, a.indptr[r], a.indptr[r + 1], a.last[r], ipB);
    }
    pre = uni64(inc - uni(cnt0));
  }

  const int g_base = gt * GT;
  const int gcount = min(GT, a.group - g_base);
  uint8_t *kt = sm.ktile[wave];

  // Metadata of request rr: page count in the virtual list (0 if it fails the
  // per-request guard), first page position and tail length; LDS copies for
  // the first kLdsPrefix requests.
  auto request_meta = [&](int rr, int32_t &st_out, int32_t &tl_out) -> int {
    int c;
    if (rr < kLdsPrefix) {
      st_out = sm.req_st[rr];
      tl_out = sm.req_tl[rr];
      c = (int)(sm.incl[rr] - (rr > 0 ? sm.incl[rr - 1] : 0));
    } else {
      st_out = a.indptr[rr];
      tl_out = a.last[rr];
      c = request_pages(a, st_out, a.indptr[rr + 1], tl_out, ipB);
      tl_out = last_block_rows(tl_out);
    }
    st_out = uni(st_out);
    tl_out = uni(tl_out);
    return uni(c);
  };
  WaveDecoder<GT> w{a, kt, sm.qfrag[wave], lane, col, quad, kvh};
  const int64_t qh_base = (int64_t)kvh * a.group + g_base;

  // ---- one continuous page stream over [v_begin, v_end) --------------------
  // Two cursors walk the virtual list: the load cursor kSD-1 pages ahead of
  // the process cursor.  Page indices come in blocks of 64 (one per lane, read
  // back with v_readlane), the next block fetched while the current one is
  // used, so the K/V pipeline does not drain at request or block boundaries;
  // at a request boundary the process side finishes the piece and fetches the
  // next request's Q while the next pages' loads are in flight.
  struct Cursor {
    int r;
    int64_t pre;
    int cnt;
    int32_t st, tl;
  };
  auto advance = [&](Cursor &c, int64_t vv) {
    while (vv >= c.pre + c.cnt) {
      c.pre += c.cnt;
      do {
        if (++c.r >= a.batch) {  // unreachable: vv < total
          c.cnt = INT32_MAX;
          return;
        }
        c.cnt = request_meta(c.r, c.st, c.tl);
      } while (c.cnt == 0);
    }
  };
  // Page indices of virtual pages [v0, v0 + 64) (lane i: page v0 + i; 0 past
  // the range).  Each lane walks forward from cursor c (at or before v0) to
  // the request holding its page: requests with no pages are skipped.
  auto block_indices = [&](const Cursor &c, int64_t v0) -> int {
    const int64_t vv = v0 + lane;
    if (vv >= v_end) return 0;
    int rr = c.r, cn = c.cnt;
    int64_t pr = c.pre;
    int32_t sto = c.st;
    while (vv >= pr + cn) {
      pr += cn;
      do {
        ++rr;
        if (rr < kLdsPrefix) {
          sto = sm.req_st[rr];
          cn = (int)(sm.incl[rr] - sm.incl[rr - 1]);
        } else {
          sto = a.indptr[rr];
          cn = request_pages(a, sto, a.indptr[rr + 1], a.last[rr], ipB);
        }
      } while (cn == 0);
    }
    return a.indices[sto + ((int)(vv - pr) >> a.blocks_lg)];
  };
  const int n = (int)(v_end - v_begin);
  int ib = 0, ib_next = 0;  // index blocks: current and next
  // Page index, block within the page and valid rows of virtual block vl (0
  // rows: past the range, or an index failing the guard of decode.rs:284-289).
  auto describe = [&](Cursor &c, int64_t vl, int &page, int &blk, int &rows) {
    page = 0;
    blk = 0;
    rows = 0;
    if (vl >= v_end) return;
    advance(c, vl);
    const int k = (int)(vl - v_begin);
    if ((k & 63) == 0 && k > 0) {
      ib = ib_next;
      if (k + 64 < n) ib_next = block_indices(c, vl + 64);
    }
    const int32_t idx = __builtin_amdgcn_readlane(ib, k & 63);
    if (idx >= 0 && (int64_t)idx < a.pool) {
      page = idx;
      blk = (int)(vl - c.pre) & ((1 << a.blocks_lg) - 1);
      rows = (int)(vl - c.pre) == c.cnt - 1 ? c.tl : 16;
    }
  };

  Cursor lc;
  lc.r = r;
  lc.pre = pre;
  lc.cnt = request_meta(r, lc.st, lc.tl);
  Cursor pc = lc;
  bool bad = false;
  ib = block_indices(lc, v_begin);
  if (n > 64) ib_next = block_indices(lc, v_begin + 64);

  auto begin_piece = [&]() {
    u32x4 qr[4];
    w.load_q(pc.r, kvh * a.group + g_base, gcount, qr);
    w.store_q(qr);
    w.reset();
    bad = false;
  };
  auto finish_piece = [&]() {
    const int rr = pc.r;
    const bool whole = v_begin <= pc.pre && pc.pre + pc.cnt <= v_end;
    const float l_tot = w.reduce();
    const float m_run = w.m_run;
    const auto &acc = w.acc;
    // Lane (col, quad) holds dims 32 quad + [0, 32) of query head qh_base + col.
    const bool mine = col < gcount;
    if (whole) {
      // The request lies inside this wave's range: final output in place.  An
      // invalid page index leaves the request's sentinels untouched.
      if (!bad && mine) {
        uint16_t *o = a.out + ((int64_t)rr * a.hq + qh_base + col) * 128 + quad * 32;
        store_out_row<FP8>(o, acc, l_tot, v_scale);
        if (quad == 0) a.lse[(int64_t)rr * a.hq + qh_base + col] = m_run + __log2f(l_tot);
      }
    } else {
      // Split request: one state per (team, request), slot team + r (unique:
      // along the virtual list either the team or the request advances).
      float *st = a.states + (((int64_t)(team + rr) * a.hq + qh_base + col) * kStateStride);
      if (mine) {
        if (bad) {
          if (quad == 0) {
            st[0] = 0.0f;
            st[1] = kPoisonNormalizer;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float *o = st + 4 + quad * 32 + i * 8;
            *reinterpret_cast<f32x4 *>(o) = f32x4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
            *reinterpret_cast<f32x4 *>(o + 4) = f32x4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
          }
          if (quad == 0) {
            st[0] = m_run;
            st[1] = l_tot;
          }
        }
      }
    }
  };

  // Pipeline: page v+kSD-1 is issued before page v is consumed; the
  // unrolled buffer rotation lets the compiler wait for exactly the oldest
  // page's loads.
  PageBuf<FP8> buf[kSD];
  int brows[kSD];
#pragma unroll
  for (int j = 0; j < kSD - 1; ++j) {
    int pg, blk;
    describe(lc, v_begin + j, pg, blk, brows[j]);
    load_page(buf[j], a, pg, blk, brows[j], lane, kvh);
  }
  // Issue priority by progress (see the page loop): every wave starts high.
  __builtin_amdgcn_s_setprio(3);
  begin_piece();
  int64_t v = v_begin;
  int i = 0;
  while (true) {
#pragma unroll
    for (int s = 0; s < kSD; ++s) {
      {
        const int nb = (s + kSD - 1) % kSD;
        int pg, blk;
        describe(lc, v + kSD - 1, pg, blk, brows[nb]);
        load_page(buf[nb], a, pg, blk, brows[nb], lane, kvh);
      }
      if (v >= pc.pre + pc.cnt) {
        finish_piece();
        advance(pc, v);
        begin_piece();
      }
      bad |= brows[s] == 0;
      w.process(buf[s], brows[s]);
      ++v;
      if (++i >= n) goto stream_done;
      // Waves ahead of schedule yield issue priority to the ones behind: all
      // waves have the same number of pages, but the SIMD arbiter favours the
      // oldest waves, so without this the first workgroups on a CU finish far
      // earlier and the last ones stream alone at the end (measured: wave end
      // times spread over 88..196 us on config 3; 131..178 us with this).
      if ((i & 7) == 0) {
        const int q = (4 * i) / n;
        if (q == 1) __builtin_amdgcn_s_setprio(2);
        else if (q == 2) __builtin_amdgcn_s_setprio(1);
        else if (q >= 3) __builtin_amdgcn_s_setprio(0);
      }
    }
  }
stream_done:
  finish_piece();
}

// Direct decode for small page tables: one workgroup per (request, kv-head,
// tile), its W waves taking pages w, w+W, ... of the request and merging in
// LDS, so the request finishes in one launch (no scan, no split states, no
// merge kernel).  Used when the plan's page capacity is small, where the call
// is launch- and latency-bound.  With a.splits > 1 each request's blocks are
// cut into a.splits equal ranges, one workgroup each, which write states for
// paged_decode_direct_merge_kernel instead of O and LSE.
template <int GT, int W = kWaves>
struct DirectSmem {
  uint8_t ktile[W][kKTileBytes];
  u32x4 qfrag[W][4][64];
  float wm[W][GT];
  float wl[W][GT];
  float wacc[W][GT][128];
  uint32_t bad[W];  // per-wave invalid-page-index flags
};

// W waves per workgroup (4 for the tiniest tables; 8 when a request may hold
// more pages, so each wave streams fewer of them).
// Waves per SIMD the direct kernel's LDS allows (160 KiB per CU), at most the
// register target.
template <int GT, int W>
constexpr int direct_waves_per_eu() {
  const int per_cu = (int)((160 * 1024) / sizeof(DirectSmem<GT, W>)) * W / 4;
  return per_cu < 1 ? 1 : per_cu < waves_per_eu<GT>() ? per_cu : waves_per_eu<GT>();
}

template <int GT, int W, bool FP8 = false>
__global__ __launch_bounds__(W * 64, (direct_waves_per_eu<GT, W>())) void paged_decode_direct_kernel(
    DecodeArgs a) {
  __shared__ DirectSmem<GT, W> sm;
  float v_scale = 1.0f;
  if constexpr (FP8) {
    a.scale_log2 *= a.kv_scales[0];
    v_scale = a.kv_scales[1];
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, quad = lane >> 4;
  const int split = (int)(blockIdx.x % a.splits);
  const int head = (int)(blockIdx.x / a.splits);
  const int kvh = head % a.hkv;
  const int rest = head / a.hkv;
  const int gt = rest % a.members;  // members = group tiles for this kernel
  const int r = rest / a.members;

  const int g_base = gt * GT;
  const int gcount = min(GT, a.group - g_base);
  const int64_t qh_base = (int64_t)kvh * a.group + g_base;
  // Split workgroups always write their state (a poisoned normalizer for
  // a request that fails a guard), so the merge never reads a stale one.
  auto state_of = [&](int g) {
    return a.states + (((int64_t)split * a.batch + r) * a.hq + qh_base + g) * kStateStride;
  };
  auto poison = [&]() {
    if (a.splits > 1 && tid < gcount) state_of(tid)[1] = kPoisonNormalizer;
  };
  WaveDecoder<GT> w{a, sm.ktile[wave], sm.qfrag[wave], lane, col, quad, kvh};
  // One round trip for the guard words (decode.rs:233-246 global, :430-478
  // per request), the query tile and, when the page-index array has at most
  // 128 entries (as direct plans' tables do), the whole array (two words per
  // lane): the request's page indices are then read from registers.
  u32x4 qr[4];
  w.load_q(r, kvh * a.group + g_base, gcount, qr);
  const bool small_table = a.n_indices <= 128;
  int tbl0 = 0, tbl1 = 0;
  if (small_table) {
    if (lane < a.n_indices) tbl0 = a.indices[lane];
    if (lane + 64 < a.n_indices) tbl1 = a.indices[lane + 64];
  }
  const int32_t ip0 = a.indptr[0], ipB = a.indptr[a.batch];
  const int32_t st = uni(a.indptr[r]), en = uni(a.indptr[r + 1]), tl = uni(a.last[r]);
  if (ip0 != 0 || !batch_pages_ok(a, ipB)) return poison();
  const int cnt = request_pages(a, st, en, tl, ipB);
  if (cnt == 0) return poison();

  // this split's blocks [lo, hi) of the request; this wave's: request-local
  // positions lo + wave + W*i (block b is block b % (page_rows / 16) of the
  // request's page b / (page_rows / 16))
  const int lo = (int)((int64_t)cnt * split / a.splits);
  const int hi = (int)((int64_t)cnt * (split + 1) / a.splits);
  const int mine = hi - lo > wave ? (hi - lo - wave + W - 1) / W : 0;
  const int tl_rows = last_block_rows(tl);
  const int bmask = (1 << a.blocks_lg) - 1;
  bool bad = false;
  {
    int idx = 0;
    if (small_table) {
      const int j = st + ((lo + wave + W * lane) >> a.blocks_lg);  // < 128 for this wave's blocks
      const int lo = __shfl(tbl0, j & 63, 64), hi = __shfl(tbl1, j & 63, 64);
      if (lane < min(mine, 64)) idx = j < 64 ? lo : hi;
    } else if (lane < min(mine, 64)) {
      idx = a.indices[st + ((lo + wave + W * lane) >> a.blocks_lg)];
    }
    w.store_q(qr);
    w.reset();
    for (int s0 = 0; s0 < mine; s0 += 64) {
      if (s0 > 0)
        idx = lane < min(mine - s0, 64)
                  ? a.indices[st + ((lo + wave + W * (s0 + lane)) >> a.blocks_lg)]
                  : 0;
      const int n = min(mine - s0, 64);
      const int ok = (idx >= 0 && (int64_t)idx < a.pool) ? 1 : 0;
      bad |= __ballot(lane < n && !ok) != 0;
      auto tok_of = [&](int i) {
        const int j = min(i, n - 1);
        return block_elem(a, __builtin_amdgcn_readlane(idx, j), (lo + wave + W * (s0 + j)) & bmask);
      };
      auto rows_of = [&](int i) {
        if (i >= n || !__builtin_amdgcn_readlane(ok, i)) return 0;
        return lo + wave + W * (s0 + i) == cnt - 1 ? tl_rows : 16;
      };
      w.template stream<FP8>(n, tok_of, rows_of);
    }
  }
  const float l_tot = w.reduce();
  if (col < GT) {
    if (quad == 0) {
      sm.wm[wave][col] = w.m_run;
      sm.wl[wave][col] = l_tot;
    }
    stash_acc(sm.wacc[wave][col], w.acc, quad);
  }
  // An invalid page index anywhere in the request keeps its sentinels.
  if (block_or(bad, sm.bad)) return poison();

  // Workgroup merge of the W wave states (a wave without pages has max -inf
  // and weight 0).
  for (int idx = tid; idx < GT * 128; idx += W * 64) {
    const int g = idx >> 7, d = idx & 127;
    if (g >= gcount) continue;
    float M = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < W; ++wv) M = fmaxf(M, sm.wm[wv][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int wv = 0; wv < W; ++wv) {
      const float f = fast_exp2(sm.wm[wv][g] - M);
      L = fmaf(sm.wl[wv][g], f, L);
      O = fmaf(sm.wacc[wv][g][d], f, O);
    }
    if (a.splits > 1) {  // this split's state: max, normalizer, unnormalized O
      // (a split without blocks has max -inf: weight and O zero)
      const bool empty = M == -INFINITY;
      float *ss = state_of(g);
      ss[4 + d] = empty ? 0.f : O;
      if (d == 0) {
        ss[0] = M;
        ss[1] = empty ? 0.f : L;
      }
      continue;
    }
    float o = O / L;
    if constexpr (FP8) o *= v_scale;
    a.out[((int64_t)r * a.hq + qh_base + g) * 128 + d] = f32_to_bf16(o);
    if (d == 0) a.lse[(int64_t)r * a.hq + qh_base + g] = M + __log2f(L);
  }
}

// Combines the a.splits states of one (request, query head) written by the
// direct kernel into O and log2-LSE (128 lanes, one per output column, in
// split order); a poisoned state leaves the request's sentinels.
constexpr int kMaxDirectSplits = 8;
constexpr uint64_t kMaxDirectSplitsPlanned = kMaxDirectSplits;
__global__ __launch_bounds__(128) void paged_decode_direct_merge_kernel(DecodeArgs a) {
  const int tid = threadIdx.x;
  const int r = blockIdx.x / a.hq;
  const int qh = blockIdx.x % a.hq;
  float ms[kMaxDirectSplits], ls[kMaxDirectSplits], xs[kMaxDirectSplits];
#pragma unroll
  for (int u = 0; u < kMaxDirectSplits; ++u) {
    ms[u] = -INFINITY;
    ls[u] = 0.f;
    xs[u] = 0.f;
    if (u < a.splits) {
      const float *ss = a.states + (((int64_t)u * a.batch + r) * a.hq + qh) * kStateStride;
      ms[u] = ss[0];
      ls[u] = ss[1];
      xs[u] = ss[4 + tid];
    }
  }
  float M = -INFINITY;
  bool poisoned = false;
#pragma unroll
  for (int u = 0; u < kMaxDirectSplits; ++u) {
    M = fmaxf(M, ms[u]);
    poisoned |= ls[u] < 0.0f;
  }
  if (poisoned) return;
  float l = 0.f, o = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxDirectSplits; ++u) {
    const float f = fast_exp2(ms[u] - M);
    l = fmaf(ls[u], f, l);
    o = fmaf(xs[u], f, o);
  }
  float ov = o / l;
  if (a.kv_scales) ov *= a.kv_scales[1];  // FP8 pages: V's scale
  a.out[((int64_t)r * a.hq + qh) * 128 + tid] = f32_to_bf16(ov);
  if (tid == 0) a.lse[(int64_t)r * a.hq + qh] = M + __log2f(l);
}

// Merges the states of one (request, query head) whose pages span several
// teams into O and log2-LSE: one wave, 2 output columns per lane, one pass
// with a running max over blocks of 16 teams (one load round trip per
// block). The header written by the partial kernel gives the request's
// virtual page range; a poisoned state (invalid page index) leaves the
// request's sentinels.
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int kBlock = 16;
  const int lane = threadIdx.x;
  const int r = blockIdx.x / a.hq;
  const int qh = blockIdx.x % a.hq;
  const int64_t total = a.header[0];
  const int64_t pre = a.header[1 + r], pend = a.header[2 + r];
  if (total <= 0 || pend <= pre) return;
  const int teams = active_teams(total, a.teams);
  const int64_t t0 = team_of(total, pre, teams), t1 = team_of(total, pend - 1, teams);
  if (t0 == t1) return;
  const bool all_nonempty = total >= teams;
  float M = -INFINITY, l = 0.f;
  f32x2 o = {0.f, 0.f};
  bool poisoned = false;
  for (int64_t t = t0; t <= t1; t += kBlock) {
    float ms[kBlock], ls[kBlock];
    f32x2 xs[kBlock];
#pragma unroll
    for (int u = 0; u < kBlock; ++u) {
      ms[u] = -INFINITY;
      ls[u] = 0.f;
      xs[u] = f32x2{0.f, 0.f};
      const int64_t tu = t + u;
      if (tu <= t1 && (all_nonempty || team_start(total, tu, teams) <
                                           team_start(total, tu + 1, teams))) {
        const float *ss = a.states + ((tu + r) * a.hq + qh) * (int64_t)kStateStride;
        ms[u] = ss[0];
        ls[u] = ss[1];
        xs[u] = *reinterpret_cast<const f32x2 *>(ss + 4 + 2 * lane);
      }
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < kBlock; ++u) {
      mb = fmaxf(mb, ms[u]);
      poisoned |= ls[u] < 0.0f;
    }
    // A block of empty teams (possible when there are fewer pages than
    // teams) leaves the state as it is.
    if (mb == -INFINITY) continue;
    const float sc = fast_exp2(M - mb);
    l *= sc;
    o[0] *= sc;
    o[1] *= sc;
#pragma unroll
    for (int u = 0; u < kBlock; ++u) {
      const float f = fast_exp2(ms[u] - mb);
      l = fmaf(ls[u], f, l);
      o[0] = fmaf(xs[u][0], f, o[0]);
      o[1] = fmaf(xs[u][1], f, o[1]);
    }
    M = mb;
  }
  if (poisoned) return;
  float v0 = o[0] / l, v1 = o[1] / l;
  if (a.kv_scales) {  // FP8 pages: V's scale
    v0 *= a.kv_scales[1];
    v1 *= a.kv_scales[1];
  }
  *reinterpret_cast<uint32_t *>(a.out + ((int64_t)r * a.hq + qh) * 128 + 2 * lane) =
      bf16x2_pack(v0, v1);
  if (lane == 0) a.lse[(int64_t)r * a.hq + qh] = M + __log2f(l);
}

// ---- contiguous single decode -------------------------------------------------
// K/V [kv_len, Hkv, 128] contiguous (single_decode/mod.rs:15-20): any 16
// consecutive tokens form a block with the paged layout's row stride, so the
// page step, the loads and the range-limited buffer resources are shared.

// Bf16SingleDecodePlan: one workgroup per (kv-head, tile); wave w takes the
// 16-token blocks w, w+4, ... and the 4 wave states merge in LDS.
template <int GT>
__global__ __launch_bounds__(kThreads, waves_per_eu<GT>()) void single_decode_kernel(
    DecodeArgs a, int64_t kv_len) {
  __shared__ DirectSmem<GT> sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, quad = lane >> 4;
  const int kvh = (int)(blockIdx.x % a.hkv);
  const int gt = (int)(blockIdx.x / a.hkv);
  const int g_base = gt * GT;
  const int gcount = min(GT, a.group - g_base);
  WaveDecoder<GT> w{a, sm.ktile[wave], sm.qfrag[wave], lane, col, quad, kvh};
  const int64_t nblk = (kv_len + 15) / 16;
  const int mine = nblk > wave ? (int)((nblk - wave + kWaves - 1) / kWaves) : 0;
  {
    u32x4 qr[4];
    w.load_q(0, kvh * a.group + g_base, gcount, qr);
    w.store_q(qr);
  }
  w.reset();
  if (mine > 0) {
    auto tok_of = [&](int i) {
      return token_elem(a, (int64_t)(wave + kWaves * min(i, mine - 1)) * 16);
    };
    auto rows_of = [&](int i) {
      if (i >= mine) return 0;
      return (int)min<int64_t>(16, kv_len - (int64_t)(wave + kWaves * i) * 16);
    };
    w.stream(mine, tok_of, rows_of);
  }
  const float l_tot = w.reduce();
  if (col < GT) {
    if (quad == 0) {
      sm.wm[wave][col] = w.m_run;
      sm.wl[wave][col] = l_tot;
    }
    stash_acc(sm.wacc[wave][col], w.acc, quad);
  }
  __syncthreads();
  const int64_t qh_base = (int64_t)kvh * a.group + g_base;
  for (int idx = tid; idx < GT * 128; idx += kThreads) {
    const int g = idx >> 7, d = idx & 127;
    if (g >= gcount) continue;
    float M = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) M = fmaxf(M, sm.wm[wv][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const float f = fast_exp2(sm.wm[wv][g] - M);
      L = fmaf(sm.wl[wv][g], f, L);
      O = fmaf(sm.wacc[wv][g][d], f, O);
    }
    a.out[(qh_base + g) * 128 + d] = f32_to_bf16(O / L);
    if (d == 0) a.lse[qh_base + g] = M + __log2f(L);
  }
}

// Bf16SingleDecodeSplitKPlan partials: one wave per (partition, kv-head,
// tile) over the partition's balanced token range (single_decode/mod.rs:
// 167-181), writing (max_log2, normalizer, acc[128]) per query head into the
// workspace [Hq, partitions, 130] (single_decode/mod.rs:10-13, :183-193).
template <int GT>
__global__ __launch_bounds__(kThreads, waves_per_eu<GT>()) void single_decode_split_k_kernel(
    DecodeArgs a, int64_t kv_len, int partitions, float *__restrict__ ws) {
  __shared__ DirectSmem<GT> sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, quad = lane >> 4;
  const int64_t wid = (int64_t)blockIdx.x * kWaves + wave;
  if (wid >= (int64_t)partitions * a.members) return;  // no workgroup barrier follows
  const int part = (int)(wid / a.members), member = (int)(wid % a.members);
  const int kvh = member % a.hkv, gt = member / a.hkv;
  const int g_base = gt * GT;
  const int gcount = min(GT, a.group - g_base);
  const int64_t base = kv_len / partitions, rem = kv_len % partitions;
  const int64_t start = part * base + min<int64_t>(part, rem);
  const int64_t end = start + base + (part < rem ? 1 : 0);
  WaveDecoder<GT> w{a, sm.ktile[wave], sm.qfrag[wave], lane, col, quad, kvh};
  {
    u32x4 qr[4];
    w.load_q(0, kvh * a.group + g_base, gcount, qr);
    w.store_q(qr);
  }
  w.reset();
  const int nb = (int)((end - start + 15) / 16);
  auto tok_of = [&](int i) { return token_elem(a, start + (int64_t)min(i, nb - 1) * 16); };
  auto rows_of = [&](int i) {
    return i >= nb ? 0 : (int)min<int64_t>(16, end - start - (int64_t)i * 16);
  };
  w.stream(nb, tok_of, rows_of);
  const float l_tot = w.reduce();
  const int64_t qh_base = (int64_t)kvh * a.group + g_base;
  if (col < gcount) {
    // [Hq, P, 130] rows are 8-byte aligned: dims as float2 pairs
    float *st = ws + ((qh_base + col) * partitions + part) * (int64_t)loom::kStateWidth;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        *reinterpret_cast<float2 *>(st + 2 + quad * 32 + i * 8 + e) =
            float2{w.acc[e][i], w.acc[e + 1][i]};
    if (quad == 0) {
      st[0] = w.m_run;
      st[1] = l_tot;
    }
  }
}

// Split-K merge (single_decode/mod.rs:332-381): one workgroup of 128 lanes
// (one per output column) per query head.
// One workgroup of four waves per query head: wave w takes partitions w, w +
// 4, ..., each lane two of the 128 dims; the first kMergeBatch partitions of
// every wave are loaded before the heads' maximum is reduced, so up to 64
// partitions take one memory round trip.  The waves' sums are combined in
// LDS in wave order (deterministic).  Empty partitions (max -inf, normalizer
// 0) weigh nothing.
constexpr int kMergeWaves = 4, kMergeBatch = 16;
__global__ __launch_bounds__(kMergeWaves * 64) void single_decode_split_k_merge_kernel(
    DecodeArgs a, int partitions, const float *__restrict__ ws) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qh = blockIdx.x;
  const float *row = ws + (int64_t)qh * partitions * loom::kStateWidth;
  float ms[kMergeBatch], ls[kMergeBatch];
  f32x2 xs[kMergeBatch];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int p = base + u * kMergeWaves;
      if (p < partitions) {
        const float *ss = row + (int64_t)p * loom::kStateWidth;
        ms[u] = ss[0];
        ls[u] = ss[1];
        xs[u] = *reinterpret_cast<const f32x2 *>(ss + 2 + 2 * lane);
      } else {
        ms[u] = -INFINITY;
        ls[u] = 0.f;
        xs[u] = f32x2{0.f, 0.f};
      }
    }
  };
  load_batch(wave);
  float mloc = -INFINITY;
  for (int p = tid; p < partitions; p += kMergeWaves * 64)
    mloc = fmaxf(mloc, row[(int64_t)p * loom::kStateWidth]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  __shared__ float s_m[kMergeWaves], s_l[kMergeWaves];
  __shared__ f32x2 s_o[kMergeWaves][64];
  if (lane == 0) s_m[wave] = mloc;
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < kMergeWaves; ++w) M = fmaxf(M, s_m[w]);
  float l = 0.f;
  f32x2 o = {0.f, 0.f};
  for (int base = wave;; base += kMergeWaves * kMergeBatch) {
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float f = ms[u] == -INFINITY ? 0.f : fast_exp2(ms[u] - M);
      l = fmaf(ls[u], f, l);
      o[0] = fmaf(xs[u][0], f, o[0]);
      o[1] = fmaf(xs[u][1], f, o[1]);
    }
    if (base + kMergeWaves * kMergeBatch >= partitions) break;
    load_batch(base + kMergeWaves * kMergeBatch);
  }
  if (lane == 0) s_l[wave] = l;
  s_o[wave][lane] = o;
  __syncthreads();
  if (wave == 0) {
    float lt = s_l[0];
    f32x2 ot = s_o[0][lane];
#pragma unroll
    for (int w = 1; w < kMergeWaves; ++w) {
      lt += s_l[w];
      ot[0] += s_o[w][lane][0];
      ot[1] += s_o[w][lane][1];
    }
    *reinterpret_cast<uint32_t *>(a.out + (int64_t)qh * 128 + 2 * lane) =
        bf16x2_pack(ot[0] / lt, ot[1] / lt);
    if (lane == 0) a.lse[qh] = M + __log2f(lt);
  }
}

}  // namespace

// ---- provider / plan / enqueue -----------------------------------------------
struct loom_decode_provider {
  loom::DeviceInfo dev;
};

struct loom_paged_decode_plan {
  loom_paged_decode_plan_info_t info{};
  int device = 0;
};

struct loom_single_decode_plan {
  loom_single_decode_spec_t spec;
  uint32_t group_tile = 1, group_tiles = 1;
};

struct loom_single_decode_split_k_plan {
  loom_single_decode_split_k_spec_t spec;
  uint32_t group_tile = 1, group_tiles = 1;
};

namespace {
uint32_t group_tile_for(uint64_t group) {
  return group <= 1 ? 1u : group <= 2 ? 2u : group <= 4 ? 4u : 8u;
}

// Single-decode argument block shared by both plans (batch of one request).
DecodeArgs single_args(const loom_single_decode_spec_t &s, uint32_t gtiles, uintptr_t q,
                       uintptr_t k, uintptr_t v, uintptr_t o, uintptr_t lse) {
  DecodeArgs a{};
  a.q = (const uint16_t *)q;
  a.k = (const uint16_t *)k;
  a.v = (const uint16_t *)v;
  a.out = (uint16_t *)o;
  a.lse = (float *)lse;
  a.batch = 1;
  a.hq = (int32_t)s.num_query_heads;
  a.hkv = (int32_t)s.num_kv_heads;
  a.group = (int32_t)(s.num_query_heads / s.num_kv_heads);
  a.members = (int32_t)(s.num_kv_heads * gtiles);
  a.scale_log2 = s.softmax_scale * 1.44269504088896340736f;
  a.head_elems = 128;  // contiguous K/V: NHD rows
  a.row_elems = a.hkv * 128;
  a.page_rows = 16;
  a.blocks_lg = 0;
  a.page_elems = (int64_t)16 * a.hkv * 128;
  a.block_elems = 16 * a.row_elems;
  a.splits = 1;
  return a;
}
}  // namespace

namespace {
template <bool FP8>
void launch_direct(const loom_paged_decode_plan_info_t &pi, dim3 g3, dim3 bd, hipStream_t stream,
                   const DecodeArgs &a) {
  if (pi.block_threads == 4 * 64) {
    switch (pi.group_tile) {
      case 1: hipLaunchKernelGGL((paged_decode_direct_kernel<1, 4, FP8>), g3, bd, 0, stream, a); break;
      case 2: hipLaunchKernelGGL((paged_decode_direct_kernel<2, 4, FP8>), g3, bd, 0, stream, a); break;
      case 4: hipLaunchKernelGGL((paged_decode_direct_kernel<4, 4, FP8>), g3, bd, 0, stream, a); break;
      default: hipLaunchKernelGGL((paged_decode_direct_kernel<8, 4, FP8>), g3, bd, 0, stream, a); break;
    }
  } else if (pi.block_threads == 16 * 64) {
    if (pi.group_tile == 1)
      hipLaunchKernelGGL((paged_decode_direct_kernel<1, 16, FP8>), g3, bd, 0, stream, a);
    else
      hipLaunchKernelGGL((paged_decode_direct_kernel<2, 16, FP8>), g3, bd, 0, stream, a);
  } else {
    switch (pi.group_tile) {
      case 1: hipLaunchKernelGGL((paged_decode_direct_kernel<1, 8, FP8>), g3, bd, 0, stream, a); break;
      case 2: hipLaunchKernelGGL((paged_decode_direct_kernel<2, 8, FP8>), g3, bd, 0, stream, a); break;
      case 4: hipLaunchKernelGGL((paged_decode_direct_kernel<4, 8, FP8>), g3, bd, 0, stream, a); break;
      default: hipLaunchKernelGGL((paged_decode_direct_kernel<8, 8, FP8>), g3, bd, 0, stream, a); break;
    }
  }
}

template <bool FP8>
void launch_split(const loom_paged_decode_plan_info_t &pi, dim3 g3, dim3 b3, hipStream_t stream,
                  const DecodeArgs &a) {
  switch (pi.group_tile) {
    case 1: hipLaunchKernelGGL((paged_decode_split_kv_kernel<1, FP8>), g3, b3, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((paged_decode_split_kv_kernel<2, FP8>), g3, b3, 0, stream, a); break;
    case 4: hipLaunchKernelGGL((paged_decode_split_kv_kernel<4, FP8>), g3, b3, 0, stream, a); break;
    default: hipLaunchKernelGGL((paged_decode_split_kv_kernel<8, FP8>), g3, b3, 0, stream, a); break;
  }
}
}  // namespace

namespace {
loom_status_t bind_static_scratch(int device, loom_error_t *err);
}  // namespace

extern "C" {

loom_status_t loom_decode_provider_load(int device, loom_decode_provider_t **out,
                                        loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  loom::DeviceInfo dev;
  loom_status_t rc = loom::query_device(device, &dev, err);
  if (rc) return rc;
  if (!dev.gfx950) return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, nullptr, device);
  // set-up of the allocation-free enqueue: this device's scratch address
  rc = bind_static_scratch(device, err);
  if (rc) return rc;
  auto *p = new loom_decode_provider;
  p->dev = dev;
  *out = p;
  return loom::ok(err);
}

void loom_decode_provider_free(loom_decode_provider_t *p) { delete p; }

loom_status_t loom_decode_provider_plan_bf16_paged_batch(
    const loom_decode_provider_t *provider, const loom_paged_decode_spec_t *spec,
    const loom_paged_decode_plan_options_t *options, loom_paged_decode_plan_t **out,
    loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  loom_paged_decode_plan_options_t opt{};
  if (options) opt = *options;
  const uint64_t B = spec->batch_size, hq = spec->num_query_heads, hkv = spec->num_kv_heads;
  const uint64_t group = hq / hkv;
  // Query heads per workgroup column block: the group rounded up to a power
  // of two, at most 8.
  const uint32_t gtile = group <= 1 ? 1u : group <= 2 ? 2u : group <= 4 ? 4u : 8u;
  const uint64_t gtiles = (group + gtile - 1) / gtile;
  if (opt.flags & ~LOOM_PLAN_PAGE_INDICES_CAPACITY)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", opt.flags);
  if (spec->kv_layout != LOOM_KV_LAYOUT_NHD && spec->kv_layout != LOOM_KV_LAYOUT_HND)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_layout", spec->kv_layout);
  if (spec->kv_dtype != LOOM_KV_DTYPE_BF16 && spec->kv_dtype != LOOM_KV_DTYPE_FP8_E4M3)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_dtype", spec->kv_dtype);
  const uint32_t page_rows = spec->page_size ? spec->page_size : (uint32_t)loom::kPageSize;
  if (page_rows != 16 && page_rows != 32 && page_rows != 64)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, page_rows);
  const uint64_t max_pages = opt.max_total_pages ? opt.max_total_pages : spec->max_num_pages;
  if (max_pages < B) return fail(err, LOOM_PLAN_INVALID_OPTION, "max_total_pages", max_pages);
  if (max_pages > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "max_total_pages", max_pages);

  if (B > (uint64_t)kMaxScanBlocks * kThreads)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "batch_size", B);

  if (opt.teams == 0 && max_pages <= LOOM_DECODE_DIRECT_MAX_PAGES) {
    // More waves per request when a request may hold more pages; 16-wave
    // workgroups only where the page step fits 128 VGPRs (tiles of <= 2 heads).
    uint32_t waves = max_pages <= 32 ? 4 : gtile <= 2 ? 16 : 8;
    const uint64_t heads = B * gtiles * hkv;
    // Few (request, kv-head, tile) workgroups with long requests leave most
    // CUs idle and stream each request through one CU: split each request's
    // blocks over 2-8 workgroups of 4 waves (at least 8 pages each on
    // average, at most two workgroups per CU), combined by a merge kernel.
    // Config 1 (32 workgroups, 64 pages each): 10.3 -> 8.1 us per call.
    uint64_t splits = 1;
    for (uint64_t s = kMaxDirectSplitsPlanned; s >= 2; s /= 2)
      if (max_pages / B >= s * 8 && heads * s <= 2 * (uint64_t)provider->dev.cus) {
        splits = s;
        waves = 4;
        break;
      }
    const uint64_t grid = heads * splits;
    if (grid > (uint64_t)INT32_MAX || B * hq > (uint64_t)INT32_MAX)
      return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "paged batch-decode", grid);
    auto *p = new loom_paged_decode_plan;
    p->device = provider->dev.device;
    loom_paged_decode_plan_info_t &i = p->info;
    i.spec = *spec;
    i.algorithm = LOOM_PAGED_DECODE_DIRECT;
    i.group_tile = gtile;
    i.group_tiles = (uint32_t)gtiles;
    i.max_total_pages = max_pages;
    i.teams = (uint32_t)(splits > 1 ? splits : 0);
    i.state_slots = splits > 1 ? splits * B : 0;
    // (unused without splits; kept for a uniform operand list)
    i.workspace_bytes = splits > 1 ? splits * B * hq * kStateStride * 4 : 256;
    i.header_bytes = 0;
    i.block_threads = waves * 64;
    i.grid_blocks = (uint32_t)grid;
    i.device_cus = (uint32_t)provider->dev.cus;
    i.flags = opt.flags;
    *out = p;
    return loom::ok(err);
  }

  // Teams: about 13 waves per 4 CUs (a fraction of the register budget's
  // slots, so the whole grid is resident at once, each CU holds at most one
  // workgroup of each XCD's share and every wave streams the same number of
  // pages; see LOOM_DECODE_SPLIT_WAVES_PER_4CU).
  const uint64_t members = hkv * gtiles;
  const uint64_t slots =
      (uint64_t)provider->dev.cus *
      (spec->kv_dtype == LOOM_KV_DTYPE_FP8_E4M3 ? LOOM_DECODE_SPLIT_WAVES_PER_4CU_FP8
                                                : LOOM_DECODE_SPLIT_WAVES_PER_4CU) / 4;
  uint64_t teams = opt.teams ? opt.teams : std::max<uint64_t>(1, slots / members);
  // Each XCD (every 8th workgroup) holds ceil(teams / 8) whole teams.
  const uint64_t xcd_waves = (teams + 7) / 8 * members;
  const uint64_t grid = (xcd_waves + kWaves - 1) / kWaves * 8;
  if (grid > (uint64_t)INT32_MAX || teams > (uint64_t)INT32_MAX || B * hq > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "paged batch-decode", grid);
  const uint64_t header_bytes = ((B + 2) * 8 + 255) / 256 * 256;
  const uint64_t state_slots = teams + B;
  const uint64_t state_bytes = state_slots * hq * kStateStride * 4;

  auto *p = new loom_paged_decode_plan;
  p->device = provider->dev.device;
  loom_paged_decode_plan_info_t &i = p->info;
  i.spec = *spec;
  i.algorithm = LOOM_PAGED_DECODE_BALANCED_SPLIT_KV;
  i.teams = (uint32_t)teams;
  i.group_tile = gtile;
  i.group_tiles = (uint32_t)gtiles;
  i.max_total_pages = max_pages;
  i.state_slots = state_slots;
  i.workspace_bytes = header_bytes + state_bytes;
  i.header_bytes = header_bytes;
  i.block_threads = kThreads;
  i.grid_blocks = (uint32_t)grid;
  i.device_cus = (uint32_t)provider->dev.cus;
  i.flags = opt.flags;
  *out = p;
  return loom::ok(err);
}

void loom_paged_decode_plan_free(loom_paged_decode_plan_t *p) { delete p; }

void loom_paged_decode_plan_get_info(const loom_paged_decode_plan_t *p,
                                     loom_paged_decode_plan_info_t *info) {
  if (p && info) *info = p->info;
}

}  // extern "C"

namespace {

// Where a paged-decode command finds its split-KV workspace.
enum class DecodeWorkspace {
  kOperand,  // the `workspace` handle of loom_paged_decode_args_t
  kQueue,    // the command queue's own workspace (reference-shaped args)
  kStatic,   // this library's per-device static scratch (no allocation)
};

// The per-device address of `scratch` below, looked up once per device when
// a decode provider is loaded there (hipGetSymbolAddress with the device
// current).  Host code uses these addresses, never the array's name.
constexpr int kMaxDevices = 64;
uint8_t *g_scratch_ptr[kMaxDevices] = {};
// Completion of the device's last eager allocation-free command (an event
// created with the scratch address, recorded after each such command) and
// the stream it ran on: a later call on another stream checks the event.
hipEvent_t g_scratch_done[kMaxDevices] = {};
hipStream_t g_scratch_stream[kMaxDevices] = {};
bool g_scratch_used[kMaxDevices] = {};
std::mutex g_scratch_mu;

}  // namespace

// Static scratch of loom_paged_decode_enqueue_bf16_no_alloc: the split-KV
// header and states of one command.  Every command on a device shares that
// device's copy and keeps the last command's contents (the partial kernel
// rewrites the header and every state it reads, so nothing needs clearing);
// commands that overlap in time on one device race (an eager call on another
// stream while the previous command runs is rejected; captured calls are not
// checked).
static __device__ __align__(256) uint8_t scratch[LOOM_PAGED_DECODE_STATIC_SCRATCH_BYTES];

namespace {

loom_status_t bind_static_scratch(int device, loom_error_t *err) {
  if (device < 0 || device >= kMaxDevices)
    return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, "device", device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return LOOM_OK;
  int prev = 0;
  hipGetDevice(&prev);
  hipError_t e = hipSetDevice(device);
  void *ptr = nullptr;
  hipEvent_t done = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e == hipSuccess) e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
  hipSetDevice(prev);
  if (e != hipSuccess || !ptr)
    return fail(err, LOOM_CMD_DRIVER, "static scratch", 0, 0, 0, 0, 0.0, e);
  g_scratch_ptr[device] = (uint8_t *)ptr;
  g_scratch_done[device] = done;
  return LOOM_OK;
}

// Bf16PagedBatchDecodePlan::enqueue_into, decode.rs:1199-1296.  `hs` holds
// the ten handles of loom_paged_decode_args_t; with the queue's workspace the
// workspace handle is not an operand.
loom_status_t paged_decode_enqueue_impl(const loom_paged_decode_plan_t *plan,
                                        loom_command_scope_t *scope, const loom_handle_t *hs_all,
                                        DecodeWorkspace where, loom_error_t *err) {
  const loom_paged_decode_plan_info_t &pi = plan->info;
  const loom_paged_decode_spec_t &s = pi.spec;
  // FP8 pages are u8 operands plus the [k_scale, v_scale] operand.
  const bool fp8 = s.kv_dtype == LOOM_KV_DTYPE_FP8_E4M3;
  const loom_dtype_t kv_t = fp8 ? LOOM_DTYPE_U8 : LOOM_DTYPE_BF16;
  const loom::OperandSpec ops_all[10] = {
      {"Q", LOOM_DTYPE_BF16, false},           {"K_pages", kv_t, false},
      {"V_pages", kv_t, false},                {"page_indptr", LOOM_DTYPE_I32, false},
      {"page_indices", LOOM_DTYPE_I32, false}, {"last_page_len", LOOM_DTYPE_I32, false},
      {"O", LOOM_DTYPE_BF16, true},            {"LSE", LOOM_DTYPE_F32, true},
      {"workspace", LOOM_DTYPE_U8, true},      {"kv_scales", LOOM_DTYPE_F32, false}};
  const bool ws_operand = where == DecodeWorkspace::kOperand;
  if (fp8 && !ws_operand)  // the reference-shaped args carry no scales
    return fail(err, LOOM_ENQ_LENGTH_MISMATCH, "kv_scales", 2, 0);
  loom::OperandSpec ops[10];
  loom_handle_t hs[10];
  int map[10];
  int nops = 0;
  for (int i = 0; i < 10; ++i) {
    map[i] = -1;
    if (i == 8 && !ws_operand) continue;
    if (i == 9 && !fp8) continue;
    ops[nops] = ops_all[i];
    hs[nops] = hs_all[i];
    map[i] = nops++;
  }
  const loom::Lease *lr[10];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, nops, lr, err);
  if (rc) return rc;
  auto l = [&](int i) { return lr[map[i]]; };
  if (fp8 && l(9)->numel != 2)
    return fail(err, LOOM_ENQ_LENGTH_MISMATCH, "kv_scales", 2, l(9)->numel);
  // decode.rs:1216-1242: exact lengths before submission.
  const uint64_t qn = s.batch_size * s.num_query_heads * loom::kHeadDim;
  const uint64_t page_rows = s.page_size ? s.page_size : loom::kPageSize;
  const uint64_t kvn = s.max_num_pages * page_rows * s.num_kv_heads * loom::kHeadDim;
  const uint64_t want[9] = {qn, kvn, kvn, s.batch_size + 1, 0, s.batch_size, qn,
                            s.batch_size * s.num_query_heads, pi.workspace_bytes};
  for (int i = 0; i < 9; ++i) {
    if (i == 8 && !ws_operand) continue;
    if (i == 4) {
      if (l(4)->numel < s.batch_size)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_SHORT, nullptr, s.batch_size, l(4)->numel);
      if (l(4)->numel > pi.max_total_pages)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_LONG, nullptr, pi.max_total_pages,
                    l(4)->numel);
      continue;
    }
    if (l(i)->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops_all[i].name, want[i], l(i)->numel);
  }
  // decode.rs:1243-1251 / :1585-1600: Q, K/V pages and O on 4-byte
  // boundaries (the kernels' 16-byte accesses do not need more: global and
  // buffer accesses of gfx950 run in unaligned mode).  The caller-owned
  // workspace takes 16-byte vector stores of the split states.
  for (int i : {0, 1, 2, 6, 7})
    if (l(i)->ptr % 4 != 0)
      return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, ops_all[i].name, (int64_t)l(i)->ptr, 4);
  if (ws_operand && l(8)->ptr % 16 != 0)
    return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, "workspace", (int64_t)l(8)->ptr, 16);
  if (fp8 && l(9)->ptr % 4 != 0)
    return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, "kv_scales", (int64_t)l(9)->ptr, 4);

  uint8_t *ws = nullptr;
  if (where == DecodeWorkspace::kOperand) {
    ws = (uint8_t *)l(8)->ptr;
  } else if (where == DecodeWorkspace::kQueue) {
    rc = loom::queue_workspace(scope->queue, pi.workspace_bytes, false, &ws, err);
    if (rc) return rc;
  } else {
    if (pi.workspace_bytes > LOOM_PAGED_DECODE_STATIC_SCRATCH_BYTES)
      return fail(err, LOOM_ENQ_STATIC_SCRATCH_TOO_SMALL, "workspace",
                  LOOM_PAGED_DECODE_STATIC_SCRATCH_BYTES, pi.workspace_bytes);
    const int dev = scope->queue->device;
    ws = (dev >= 0 && dev < kMaxDevices) ? g_scratch_ptr[dev] : nullptr;
    if (!ws)  // no decode provider was loaded on this device
      return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, "static scratch", dev);
  }
  DecodeArgs a{};
  a.kv_scales = fp8 ? (const float *)l(9)->ptr : nullptr;
  a.q = (const uint16_t *)l(0)->ptr;
  a.k = (const uint16_t *)l(1)->ptr;
  a.v = (const uint16_t *)l(2)->ptr;
  a.indptr = (const int32_t *)l(3)->ptr;
  a.indices = (const int32_t *)l(4)->ptr;
  a.last = (const int32_t *)l(5)->ptr;
  a.out = (uint16_t *)l(6)->ptr;
  a.lse = (float *)l(7)->ptr;
  a.header = (int64_t *)ws;
  a.states = (float *)(ws + pi.header_bytes);
  a.batch = (int32_t)s.batch_size;
  a.hq = (int32_t)s.num_query_heads;
  a.hkv = (int32_t)s.num_kv_heads;
  a.group = (int32_t)(s.num_query_heads / s.num_kv_heads);
  const bool direct = pi.algorithm == LOOM_PAGED_DECODE_DIRECT;
  // the direct kernel indexes (request, tile, kv-head) and takes the tile count here
  a.members = (int32_t)(direct ? pi.group_tiles : s.num_kv_heads * pi.group_tiles);
  a.teams = (int32_t)pi.teams;
  a.splits = direct && pi.teams > 1 ? (int32_t)pi.teams : 1;
  a.pool = (int64_t)s.max_num_pages;
  a.n_indices = (int64_t)l(4)->numel;
  a.indices_capacity = (pi.flags & LOOM_PLAN_PAGE_INDICES_CAPACITY) ? 1 : 0;
  a.scale_log2 = s.softmax_scale * 1.44269504088896340736f;
  const bool hnd = s.kv_layout == LOOM_KV_LAYOUT_HND;
  a.head_elems = hnd ? (int32_t)page_rows * 128 : 128;
  a.row_elems = hnd ? 128 : a.hkv * 128;
  a.page_rows = (int32_t)page_rows;
  a.blocks_lg = page_rows == 64 ? 2 : page_rows == 32 ? 1 : 0;
  a.page_elems = (int64_t)page_rows * a.hkv * 128;
  a.block_elems = 16 * a.row_elems;

  const uint64_t grid = pi.grid_blocks;
  hipStream_t stream = scope->queue->stream;
  const dim3 g3((unsigned)grid), b3(kThreads);
  if (direct) {
    const dim3 bd(pi.block_threads);
    if (fp8)
      launch_direct<true>(pi, g3, bd, stream, a);
    else
      launch_direct<false>(pi, g3, bd, stream, a);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && a.splits > 1) {
      hipLaunchKernelGGL(paged_decode_direct_merge_kernel,
                         dim3((unsigned)(s.batch_size * s.num_query_heads)), dim3(128), 0, stream, a);
      e = hipGetLastError();
    }
    return loom::record_launch(scope, e, err);
  }
  if (fp8)
    launch_split<true>(pi, g3, b3, stream, a);
  else
    launch_split<false>(pi, g3, b3, stream, a);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    // One command: the partial kernel, then the merge of split requests.
    hipLaunchKernelGGL(paged_decode_merge_kernel, dim3((unsigned)(s.batch_size * s.num_query_heads)),
                       dim3(64), 0, stream, a);
    e = hipGetLastError();
  }
  return loom::record_launch(scope, e, err);
}

}  // namespace

extern "C" {

loom_status_t loom_paged_decode_enqueue(const loom_paged_decode_plan_t *plan,
                                        loom_command_scope_t *scope,
                                        const loom_paged_decode_args_t *args,
                                        loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_handle_t hs[10] = {args->query,       args->key_pages,    args->value_pages,
                                args->page_indptr, args->page_indices, args->last_page_len,
                                args->output,      args->lse,          args->workspace,
                                args->kv_scales};
  return paged_decode_enqueue_impl(plan, scope, hs, DecodeWorkspace::kOperand, err);
}

static void ref_handles(const loom_bf16_paged_batch_decode_args_t *a, loom_handle_t *hs) {
  const loom_handle_t none{0, 0};
  const loom_handle_t v[10] = {a->query,       a->key_pages,    a->value_pages,
                               a->page_indptr, a->page_indices, a->last_page_len,
                               a->output,      a->lse,          none,
                               none};
  for (int i = 0; i < 10; ++i) hs[i] = v[i];
}

loom_status_t loom_paged_decode_enqueue_bf16(const loom_paged_decode_plan_t *plan,
                                             loom_command_scope_t *scope,
                                             const loom_bf16_paged_batch_decode_args_t *args,
                                             loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  loom_handle_t hs[10];
  ref_handles(args, hs);
  return paged_decode_enqueue_impl(plan, scope, hs, DecodeWorkspace::kQueue, err);
}

loom_status_t loom_paged_decode_enqueue_bf16_no_alloc(
    const loom_paged_decode_plan_t *plan, loom_command_scope_t *scope,
    const loom_bf16_paged_batch_decode_args_t *args, loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  if (!scope->queue) return fail(err, LOOM_NULL_ARGUMENT, "scope");
  loom_handle_t hs[10];
  ref_handles(args, hs);
  const int dev = scope->queue->device;
  hipStream_t stream = scope->queue->stream;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, "static scratch", dev);
  // Held from the check through the launch and the record, so calls from
  // several host threads are checked in the order they launch.
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool eager = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
  if (eager && g_scratch_used[dev] && g_scratch_stream[dev] != stream &&
      hipEventQuery(g_scratch_done[dev]) == hipErrorNotReady)
    return fail(err, LOOM_ENQ_STATIC_SCRATCH_BUSY, "static scratch", dev);
  const loom_status_t rc = paged_decode_enqueue_impl(plan, scope, hs, DecodeWorkspace::kStatic, err);
  if (rc == LOOM_OK && eager && g_scratch_done[dev] &&
      hipEventRecord(g_scratch_done[dev], stream) == hipSuccess) {
    g_scratch_stream[dev] = stream;
    g_scratch_used[dev] = true;
  }
  return rc;
}




// ---- contiguous single decode: plans and enqueue -------------------------------
loom_status_t loom_decode_provider_plan_bf16(const loom_decode_provider_t *provider,
                                             const loom_single_decode_spec_t *spec,
                                             loom_single_decode_plan_t **out, loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  // decode.rs:1020-1023: the launch range of the query heads
  if (spec->num_query_heads > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "single-decode query heads",
                spec->num_query_heads);
  auto *p = new loom_single_decode_plan;
  p->spec = *spec;
  const uint64_t group = spec->num_query_heads / spec->num_kv_heads;
  p->group_tile = group_tile_for(group);
  p->group_tiles = (uint32_t)((group + p->group_tile - 1) / p->group_tile);
  *out = p;
  return loom::ok(err);
}

void loom_single_decode_plan_free(loom_single_decode_plan_t *p) { delete p; }

loom_status_t loom_decode_provider_plan_bf16_split_k(
    const loom_decode_provider_t *provider, const loom_single_decode_split_k_spec_t *spec,
    loom_single_decode_split_k_plan_t **out, loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  const loom_single_decode_spec_t &d = spec->decode;
  if (d.num_query_heads > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "single-decode query heads",
                d.num_query_heads);
  const uint64_t group = d.num_query_heads / d.num_kv_heads;
  const uint32_t gtile = group_tile_for(group);
  const uint64_t gtiles = (group + gtile - 1) / gtile;
  // decode.rs:1041-1046: the partial states (here: waves) must fit the grid
  const uint64_t waves = spec->partitions * d.num_kv_heads * gtiles;
  if (spec->partitions > (uint64_t)INT32_MAX || waves / kWaves + 1 > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "single-decode partial states",
                spec->partitions * d.num_query_heads);
  auto *p = new loom_single_decode_split_k_plan;
  p->spec = *spec;
  p->group_tile = gtile;
  p->group_tiles = (uint32_t)gtiles;
  *out = p;
  return loom::ok(err);
}

void loom_single_decode_split_k_plan_free(loom_single_decode_split_k_plan_t *p) { delete p; }

uint64_t loom_single_decode_split_k_workspace_bytes(const loom_single_decode_split_k_plan_t *p) {
  return p ? p->spec.decode.num_query_heads * p->spec.partitions * loom::kStateWidth * 4 : 0;
}

namespace {
// decode.rs:1683-1696 checks 4-byte alignment for its packed pairs, and so
// do these: their 16-byte accesses need no more on gfx950 (global and buffer
// accesses run in unaligned mode).
loom_status_t require_aligned(const char *name, uintptr_t ptr, uintptr_t alignment,
                              loom_error_t *err) {
  if (ptr % alignment != 0)
    return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, name, (int64_t)ptr, (int64_t)alignment);
  return LOOM_OK;
}
}  // namespace

loom_status_t loom_single_decode_enqueue(const loom_single_decode_plan_t *plan,
                                         loom_command_scope_t *scope,
                                         const loom_single_decode_args_t *args,
                                         loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_single_decode_spec_t &s = plan->spec;
  static const loom::OperandSpec ops[5] = {{"Q", LOOM_DTYPE_BF16, false},
                                           {"K", LOOM_DTYPE_BF16, false},
                                           {"V", LOOM_DTYPE_BF16, false},
                                           {"O", LOOM_DTYPE_BF16, true},
                                           {"LSE", LOOM_DTYPE_F32, true}};
  const loom_handle_t hs[5] = {args->query, args->key, args->value, args->output, args->lse};
  const loom::Lease *l[5];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, 5, l, err);
  if (rc) return rc;
  const uint64_t qn = s.num_query_heads * loom::kHeadDim;
  const uint64_t kvn = s.kv_len * s.num_kv_heads * loom::kHeadDim;
  const uint64_t want[5] = {qn, kvn, kvn, qn, s.num_query_heads};
  for (int i = 0; i < 5; ++i)
    if (l[i]->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[i].name, want[i], l[i]->numel);
  for (int i : {0, 1, 2})
    if ((rc = require_aligned(ops[i].name, l[i]->ptr, 4, err))) return rc;
  if ((rc = require_aligned("O", l[3]->ptr, 4, err))) return rc;
  DecodeArgs a = single_args(s, plan->group_tiles, l[0]->ptr, l[1]->ptr, l[2]->ptr, l[3]->ptr,
                             l[4]->ptr);
  const dim3 g3((unsigned)(s.num_kv_heads * plan->group_tiles)), b3(kThreads);
  hipStream_t stream = scope->queue->stream;
  const int64_t L = (int64_t)s.kv_len;
  switch (plan->group_tile) {
    case 1: hipLaunchKernelGGL(single_decode_kernel<1>, g3, b3, 0, stream, a, L); break;
    case 2: hipLaunchKernelGGL(single_decode_kernel<2>, g3, b3, 0, stream, a, L); break;
    case 4: hipLaunchKernelGGL(single_decode_kernel<4>, g3, b3, 0, stream, a, L); break;
    default: hipLaunchKernelGGL(single_decode_kernel<8>, g3, b3, 0, stream, a, L); break;
  }
  return loom::record_launch(scope, hipGetLastError(), err);
}

loom_status_t loom_single_decode_split_k_enqueue(const loom_single_decode_split_k_plan_t *plan,
                                                 loom_command_scope_t *scope,
                                                 const loom_single_decode_split_k_args_t *args,
                                                 loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_single_decode_spec_t &s = plan->spec.decode;
  // decode.rs:1327: both commands must fit before either is submitted
  if (scope->submitted + 2 > scope->queue->max_commands)
    return fail(err, LOOM_CMD_COMMAND_CAPACITY_EXCEEDED, nullptr, scope->queue->max_commands);
  static const loom::OperandSpec ops[6] = {
      {"Q", LOOM_DTYPE_BF16, false},        {"K", LOOM_DTYPE_BF16, false},
      {"V", LOOM_DTYPE_BF16, false},        {"workspace", LOOM_DTYPE_F32, true},
      {"O", LOOM_DTYPE_BF16, true},         {"LSE", LOOM_DTYPE_F32, true}};
  const loom_handle_t hs[6] = {args->query, args->key,    args->value,
                               args->workspace, args->output, args->lse};
  const loom::Lease *l[6];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, 6, l, err);
  if (rc) return rc;
  const uint64_t qn = s.num_query_heads * loom::kHeadDim;
  const uint64_t kvn = s.kv_len * s.num_kv_heads * loom::kHeadDim;
  const uint64_t wsn = s.num_query_heads * plan->spec.partitions * loom::kStateWidth;
  const uint64_t want[6] = {qn, kvn, kvn, wsn, qn, s.num_query_heads};
  for (int i = 0; i < 6; ++i)
    if (l[i]->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[i].name, want[i], l[i]->numel);
  for (int i : {0, 1, 2})
    if ((rc = require_aligned(ops[i].name, l[i]->ptr, 4, err))) return rc;
  if ((rc = require_aligned("workspace", l[3]->ptr, 8, err))) return rc;
  if ((rc = require_aligned("O", l[4]->ptr, 4, err))) return rc;
  DecodeArgs a = single_args(s, plan->group_tiles, l[0]->ptr, l[1]->ptr, l[2]->ptr, l[4]->ptr,
                             l[5]->ptr);
  float *ws = (float *)l[3]->ptr;
  const int P = (int)plan->spec.partitions;
  const uint64_t waves = (uint64_t)P * a.members;
  const dim3 g3((unsigned)((waves + kWaves - 1) / kWaves)), b3(kThreads);
  hipStream_t stream = scope->queue->stream;
  const int64_t L = (int64_t)s.kv_len;
  switch (plan->group_tile) {
    case 1: hipLaunchKernelGGL(single_decode_split_k_kernel<1>, g3, b3, 0, stream, a, L, P, ws); break;
    case 2: hipLaunchKernelGGL(single_decode_split_k_kernel<2>, g3, b3, 0, stream, a, L, P, ws); break;
    case 4: hipLaunchKernelGGL(single_decode_split_k_kernel<4>, g3, b3, 0, stream, a, L, P, ws); break;
    default: hipLaunchKernelGGL(single_decode_split_k_kernel<8>, g3, b3, 0, stream, a, L, P, ws); break;
  }
  rc = loom::record_launch(scope, hipGetLastError(), err);
  if (rc) return rc;
  hipLaunchKernelGGL(single_decode_split_k_merge_kernel, dim3((unsigned)s.num_query_heads),
                     dim3(kMergeWaves * 64), 0, stream, a, P, (const float *)ws);
  return loom::record_launch(scope, hipGetLastError(), err);
}

}  // extern "C"
