// Paged causal prefill attention for gfx950 (MI355X), BF16 D128, NHD or HND pages of 16-64 rows
// caches, ragged query rows.
//
// Semantics: crates/loom-infer/src/attention/paged_prefill/mod.rs:386-446 (the
// CPU reference: bottom-right causal mask, row i of a request with qo_len rows
// sees KV tokens 0 .. kv_len - qo_len + i) with the device metadata guards of
// crates/loom-infer-cuda/src/attention/prefill.rs:293-342 (invalid global
// metadata writes nothing; an invalid request keeps its sentinels).
//
// Work decomposition (MI355X-first, not the reference's warp per (row, head)):
//   * the query rows of one request and the query heads of one kv-head's GQA
//     group are flattened, (row, group head) -> row * group + head, and cut
//     into tiles of 16; a workgroup owns one (tile, kv-head), so the 16
//     columns share every K/V byte it reads;
//   * the tile's causal page range (up to its last column's end) is split
//     over W waves (page w, w + W, ...); each wave streams its pages through
//     a two-deep register pipeline of raw buffer loads whose range covers only
//     the page's valid rows;
//   * per page, S = K·Qᵀ is four v_mfma_f32_16x16x32_bf16 (16 tokens x 16
//     columns x 128 dims) with K loaded straight into the A-fragment layout,
//     the online softmax runs in the log2 domain with a per-column causal
//     mask, and O += P·V is eight column blocks of v_mfma_f32_16x16x32_bf16:
//     the S accumulator already has the B-fragment layout of Pᵀ, and the V
//     rows as loaded give each lane the four tokens of one head dimension.
//     P enters as a BF16 high part and a BF16 residual in the two halves of
//     the k = 32 operand (one MFMA per block), so the weights carry 16
//     significant bits (relative error below 2^-15 against FP32 weights);
//   * the W wave states merge in LDS (max, rescale, deterministic tree sum)
//     and wave 0 writes O and the log2 LSE.
// Wide tiles (long prompts; LOOM_PAGED_PREFILL_WIDE_TILE): a workgroup of
// four waves owns 64 columns, one 16-column tile per wave; every wave walks
// the whole causal block range, each block loaded once per workgroup (a
// quarter per wave) into an LDS ring and read back by all four, so the L2
// bytes per column fall fourfold; each wave finishes its own tile (no merge).
// No workspace and one launch; the grid depends only on the plan.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "attn_device.hpp"
#include "loom_internal.hpp"

using loom::fail;
using namespace loom_dev;

namespace {


struct PrefillArgs {
  const uint16_t *__restrict__ q;
  const uint16_t *__restrict__ k;
  const uint16_t *__restrict__ v;
  const int32_t *__restrict__ qo;
  const int32_t *__restrict__ indptr;
  const int32_t *__restrict__ indices;
  const int32_t *__restrict__ last;
  uint16_t *__restrict__ out;
  float *__restrict__ lse;
  int32_t batch;
  int32_t nnz;
  int32_t hq;
  int32_t hkv;
  int32_t group;
  int64_t pool;
  int64_t n_indices;
  float scale_log2;
  int32_t indices_capacity;
  // Ragged (contiguous) K/V: `indptr` is kv_indptr over [nnz_kv, Hkv, 128]
  // rows; `indices` and `last` are unused.
  int32_t nnz_kv;
  // K/V row geometry (NHD: head_elems 128, row_elems Hkv * 128; HND pages:
  // head_elems 16 * 128, row_elems 128): token row t of kv-head h, t a
  // multiple of 16 for pages, starts at t * Hkv * 128 + h * head_elems.
  int32_t head_elems;
  int32_t row_elems;
  // Paged K/V: token rows per page (16, 32 or 64) and log2 of the 16-row
  // blocks per page; the kernel streams 16-row blocks, block j of page p
  // starting at token row p * page_rows + 16 * j.
  int32_t page_rows;
  int32_t blocks_lg;
  // Tiles per dispatch layer (one workgroup on each CU that the kv-heads of
  // one workgroup's XCD share: CUs / Hkv) for the serpentine tile order; 0:
  // plain heaviest-first order.
  int32_t tile_layer;
  // Nonzero (paged long tiles, at most 64 requests): tiles of all requests in
  // order of their distance from their request's end (rank k: the k-th
  // heaviest tile of every request), instead of request by request.
  int32_t tile_interleave;
  // FP8 E4M3 pages: device [k_scale, v_scale] (K = fp8 * k_scale, V = fp8 *
  // v_scale); null for BF16 pages.
  const float *kv_scales;
};

// Tile count given to a request whose qo range is malformed: larger than any
// tile index, so neither it nor any later request owns a tile (the reference's
// request search returns at the first malformed range, prefill.rs:303-313).
constexpr int64_t kNoTiles = (int64_t)1 << 50;

// Pages in flight per wave (32 VGPRs each): 16-wave workgroups have 128
// registers per lane and no room for a prefetch; 4 and 8 waves use two (deeper
// pipelines measured slower on the small shapes).
#ifndef LOOM_PREFILL_DEPTH
#define LOOM_PREFILL_DEPTH 2
#endif
constexpr int prefill_depth(int w) { return w >= 16 ? 1 : LOOM_PREFILL_DEPTH; }

template <int W, bool SH, int LT = 0>
struct PrefillSmem {
  int64_t wave_tot[W];
  int32_t wave_max[W];
  int32_t req;
  int32_t tile0;
  // the located request's qo_indptr pair, page (or kv) indptr pair, tail, and
  // the first flattened column it owns
  int32_t meta[6];
  // MFMA B fragments of 16 query columns (per wave: SH; long tiles keep them
  // in registers)
  u32x4 qfrag[LT ? 0 : SH ? W : 1][4][64];
  float m[W][16];      // per-wave running max (log2 domain) per column
  float l[W][16];      // per-wave normalizer per column
  uint32_t bad[W];     // per-wave invalid-page-index flags
  f32x4 red[(SH || LT) ? 0 : (W / 2 > 0 ? W / 2 : 1)][4][64];  // tree-sum staging (row tiles only)
};

// One page of K (A-fragment layout) and V (row layout) for one wave.
// K: lane (col, quad) holds dims [32c + 8 quad, +8) of token row col.
// V: lane (col, quad) holds dims [8 col, +8) of token rows 4 quad + j.
struct PrefillPage {
  u32x4 k[4];
  u32x4 v[4];
};

// elem0: element offset of the block's first row for kv-head 0.
__device__ __forceinline__ void load_prefill_page(PrefillPage &p, const PrefillArgs &a,
                                                  int64_t elem0, int rows, int lane, int kvh) {
  const int col = lane & 15, quad = lane >> 4;
  const int64_t first = elem0 + (int64_t)kvh * a.head_elems;
  const __amdgpu_buffer_rsrc_t rk = page_rows_rsrc(a.k + first, rows, a.row_elems);
  const __amdgpu_buffer_rsrc_t rv = page_rows_rsrc(a.v + first, rows, a.row_elems);
  const int row_bytes = a.row_elems * 2;
#pragma unroll
  for (int c = 0; c < 4; ++c) p.k[c] = load16_rows<false>(rk, col * row_bytes + (32 * c + 8 * quad) * 2);
#pragma unroll
  for (int j = 0; j < 4; ++j) p.v[j] = load16_rows<false>(rv, (quad * 4 + j) * row_bytes + col * 16);
}

// The same block on FP8 E4M3 pages (one byte per element): 8 bytes per lane
// per fragment, widened to the BF16 layout above (exactly) when consumed.
struct PrefillPage8 {
  u32x2 k[4];
  u32x2 v[4];
};

__device__ __forceinline__ void load_prefill_page(PrefillPage8 &p, const PrefillArgs &a,
                                                  int64_t elem0, int rows, int lane, int kvh) {
  const int col = lane & 15, quad = lane >> 4;
  const int64_t first = elem0 + (int64_t)kvh * a.head_elems;
  const uint8_t *k8 = reinterpret_cast<const uint8_t *>(a.k) + first;
  const uint8_t *v8 = reinterpret_cast<const uint8_t *>(a.v) + first;
  const int bytes = rows > 0 ? (rows - 1) * a.row_elems + 128 : 0;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(k8), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(v8), 0, bytes, 0x00020000);
#pragma unroll
  for (int c = 0; c < 4; ++c) p.k[c] = load8_rows<false>(rk, col * a.row_elems + 32 * c + 8 * quad);
#pragma unroll
  for (int j = 0; j < 4; ++j) p.v[j] = load8_rows<false>(rv, (quad * 4 + j) * a.row_elems + col * 8);
}

__device__ __forceinline__ const PrefillPage &expand(const PrefillPage &p) { return p; }
__device__ __forceinline__ PrefillPage expand(const PrefillPage8 &p) {
  PrefillPage o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o.k[j] = fp8x8_to_bf16x8(p.k[j]);
    o.v[j] = fp8x8_to_bf16x8(p.v[j]);
  }
  return o;
}

template <bool FP8>
using PrefillBuf = typename std::conditional<FP8, PrefillPage8, PrefillPage>::type;

struct PrefillWave {
  const PrefillArgs &a;
  const u32x4 (*qfrag)[64];
  int lane, col, quad, kvh;
  int64_t end_col;  // causal end (exclusive) of this lane's column, 0 if unused
  float m_run, l_run;
  f32x4 acc[8];     // acc[e][r] = O[column col][dim 32 quad + 8 r + e]

  __device__ void reset() {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // `lt0`: logical token index of the page's first row in the request.
  __device__ void process(const PrefillPage &pg, int64_t lt0) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pg.k[c]), as_bf16x8(qfrag[c][lane]),
                                                  s, 0, 0, 0);
    // s[i] = S[token 4 quad + i][column col]; tokens at or past the column's
    // causal end (which also covers the rows past kv_len) are masked.
    const int vis = (int)max<int64_t>(-1, min<int64_t>(16, end_col - lt0));
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = (quad * 4 + i < vis) ? s[i] * a.scale_log2 : -INFINITY;
    const float mx = quad_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // column with nothing visible yet
    const float al = fast_exp2(m_run - m_use);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_use);
    l_run = l_run * al + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    // Rescale only when some column's max moved (after the first pages of a
    // stream it rarely does); the branch is wave-uniform.
    if (__builtin_amdgcn_ballot_w64(al != 1.0f))
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= al;
    // Pᵀ as the B fragment of v_mfma_f32_16x16x32_bf16 (lane: column col,
    // k = 8 quad + [0, 8)): k = 8 quad + i is token 4 quad + i with its BF16
    // high part, k = 8 quad + 4 + i the same token's BF16 residual.
    uint32_t pb[4], rb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pb[i] = __float_as_uint(p[i]);
      rb[i] = __float_as_uint(p[i] - __uint_as_float(pb[i] & 0xffff0000u));
    }
    const bf16x8 pt = as_bf16x8(pack_hi16(pb[0], pb[1]), pack_hi16(pb[2], pb[3]),
                                pack_hi16(rb[0], rb[1]), pack_hi16(rb[2], rb[3]));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // Vᵀ block e as the A fragment: row col is dim 8 col + e, k = 8 quad +
      // [0, 4) and 8 quad + 4 + [0, 4) both tokens 4 quad + [0, 4), straight
      // from the V rows this lane loaded
      const int w = e >> 1;
      const uint32_t x01 = (e & 1) ? pack_hi16(pg.v[0][w], pg.v[1][w]) : pack_lo16(pg.v[0][w], pg.v[1][w]);
      const uint32_t x23 = (e & 1) ? pack_hi16(pg.v[2][w], pg.v[3][w]) : pack_lo16(pg.v[2][w], pg.v[3][w]);
      acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(x01, x23, x01, x23), pt, acc[e],
                                                       0, 0, 0);
    }
  }

  // Pages 0..n-1 of this wave's share through a D-deep pipeline: the loads of
  // page i + D - 1 are issued before page i is consumed (loads past the end
  // have no valid rows and move no bytes).  page_tok(i): element offset of
  // block i's first row (kv-head 0); rows_of(i): valid rows (0 past the end);
  // lt_of(i): logical token of its first row.  All wave-uniform.
  template <int D, bool FP8, class PageTok, class RowsOf>
  __device__ void prime(PrefillBuf<FP8> (&buf)[D], PageTok page_tok, RowsOf rows_of) {
#pragma unroll
    for (int j = 0; j < D - 1; ++j) load_prefill_page(buf[j], a, page_tok(j), rows_of(j), lane, kvh);
  }

  // `primed`: the loads of pages 0..D-2 are already in flight in `buf`.
  template <int D, bool FP8, class PageTok, class RowsOf, class LtOf>
  __device__ void stream(PrefillBuf<FP8> (&buf)[D], bool primed, int n, PageTok page_tok,
                         RowsOf rows_of, LtOf lt_of) {
    if (!primed) prime<D, FP8>(buf, page_tok, rows_of);
    int i = 0;
    while (true) {
#pragma unroll
      for (int s = 0; s < D; ++s) {
        load_prefill_page(buf[(s + D - 1) % D], a, page_tok(i + D - 1), rows_of(i + D - 1), lane,
                          kvh);
        process(expand(buf[s]), lt_of(i));
        if (++i >= n) return;
      }
    }
  }

  // Wide tiles (four waves, BF16): blocks 0..n-1 are loaded once per
  // workgroup, each wave fetching one quarter (wave w: K for w < 2, V
  // otherwise, rows 8 (w & 1) .. +8, two 16-byte loads per lane) two blocks
  // ahead, stored into a two-slot LDS ring of 272-byte rows (fragment reads
  // conflict free) and read back by every wave in the register layout of
  // load_prefill_page.  One barrier per block: a slot is rewritten two blocks
  // later, after every wave has passed the barrier that follows its reads.
  // `own_end`: causal end of this wave's last column; blocks at or past it
  // are staged but not computed.
#ifndef LOOM_PREFILL_WIDE_AHEAD
#define LOOM_PREFILL_WIDE_AHEAD 2
#endif
  static constexpr int kWideAhead = LOOM_PREFILL_WIDE_AHEAD;  // blocks in flight per wave
  // FP8 pages: each 16-byte chunk is loaded as its 8 E4M3 bytes and widened
  // to BF16 (exactly) before it is stored, so the ring holds the BF16 layout.
  template <bool FP8, class PageTok, class RowsOf, class LtOf>
  __device__ void stream_shared(int n, PageTok page_tok, RowsOf rows_of, LtOf lt_of,
                                u32x4 (*ring)[2][16][17], int wave, int64_t own_end) {
    const int mat = wave >> 1, row0 = 8 * (wave & 1);
    const uint16_t *src = mat ? a.v : a.k;
    auto fetch = [&](int i, u32x4 (&d)[2]) {
      const int64_t first = page_tok(i) + (int64_t)kvh * a.head_elems;
      const int rows = rows_of(i);
      if constexpr (FP8) {
        const uint8_t *s8 = reinterpret_cast<const uint8_t *>(src) + first;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(s8), 0, rows > 0 ? (rows - 1) * a.row_elems + 128 : 0,
            0x00020000);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int ch = lane + 64 * j;
          d[j] = fp8x8_to_bf16x8(
              load8_rows<false>(r, (row0 + (ch >> 4)) * a.row_elems + (ch & 15) * 8));
        }
      } else {
        const __amdgpu_buffer_rsrc_t r = page_rows_rsrc(src + first, rows, a.row_elems);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int ch = lane + 64 * j;
          d[j] = load16_rows<false>(r, (row0 + (ch >> 4)) * a.row_elems * 2 + (ch & 15) * 16);
        }
      }
    };
    auto step = [&](int i, u32x4 (&d)[2]) {
      u32x4 (*slot)[16][17] = ring[i & 1];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ch = lane + 64 * j;
        slot[mat][row0 + (ch >> 4)][ch & 15] = d[j];
      }
      fetch(i + kWideAhead, d);  // past the end: no valid rows, no traffic
      __syncthreads();
      const int64_t lt0 = lt_of(i);
      if (lt0 < own_end) {
        PrefillPage pg;
#pragma unroll
        for (int c = 0; c < 4; ++c) pg.k[c] = slot[0][col][4 * c + quad];
#pragma unroll
        for (int j = 0; j < 4; ++j) pg.v[j] = slot[1][4 * quad + j][col];
        process(pg, lt0);
      }
    };
    u32x4 d[kWideAhead][2];
#pragma unroll
    for (int j = 0; j < kWideAhead; ++j) fetch(j, d[j]);
    for (int i = 0;;) {
#pragma unroll
      for (int j = 0; j < kWideAhead; ++j) {
        step(i, d[j]);
        if (++i >= n) return;
      }
    }
  }

};

// ---- long tiles (LOOM_PAGED_PREFILL_LONG_TILE, BF16 pages) --------------------
// A workgroup of four waves owns 16 * CT * 4 flattened columns; each wave owns
// CT tiles of 16 and walks the whole causal range in 32-token blocks (two
// 16-row blocks).  Each block is loaded straight into a two-slot LDS ring
// (buffer loads to LDS: no VGPRs, LDS stores or transposes), in 1 KB regions
// of 16 rows x 32 dims:
//   K region (h, c): unit (row r, 16-byte chunk j) at 16 j + r, so a lane's A
//   fragment of S = K·Qᵀ (row col, dims 32c + 8 quad ..) is one conflict-free
//   16-byte read;
//   V region (h, c): unit (r, j) at 32 (j >> 1) + 2 r + (j & 1), read with
//   the transposing ds_read_b64_tr_b16 into the A fragment of Oᵀ += Vᵀ·Pᵀ
//   (one dimension, eight tokens: two reads).
// Every fragment read is one lane address plus a compile-time offset.  The
// query fragments stay in registers and every K and V fragment read from LDS
// feeds all CT tiles.  P enters the MFMA as BF16 (one rounding per weight;
// the normalizer is summed in FP32), so each 32-token block is 8 S and 8 P·V
// MFMAs of 16x16x32 per tile, against 12 per 16 tokens with the wide tiles'
// high/residual split of P.  acc[t][e][i] = O[column col of tile t][dim
// 16 e + 4 quad + i].
// Lazy rescale threshold of the long tiles (log2 units).
constexpr float kLazyRescaleLog2 = 8.0f;

template <int CT, bool FP8, int G = 1>
struct LongWave {
  const PrefillArgs &a;
  int lane, col, quad, kvh;
  int64_t end_col[CT];  // causal end (exclusive) of the lane's column of each tile
  int64_t full_end;     // smallest causal end of the wave's valid columns
  float m_run[CT];      // reference max (log2 domain, scaled) of each column: at most
                        // kLazyRescaleLog2 below the running max
  f32x4 lsum[CT];       // running normalizer of each column (every element)
  f32x4 acc[CT][8];
  u32x4 qf[CT][4];      // B fragments of the query tiles
  int rpos = 0;         // ring slot of the next block staged

  // K regions (4h + c), then V regions; on FP8 E4M3 pages regions of 16 rows
  // x 64 dims (one byte each), K (2h + c) then V
  static constexpr int kSlotBytes = FP8 ? 8192 : 16384;
  static constexpr int kVBase = kSlotBytes / 2;

  __device__ void reset() {
#pragma unroll
    for (int t = 0; t < CT; ++t) {
      m_run[t] = -INFINITY;
      lsum[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[t][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // S = K·Qᵀ of the block in `slot` for every tile: s0 tokens 0-15, s1 16-31.
  struct Scores {
    f32x4 s0[CT], s1[CT];
  };
  __device__ void scores(const uint8_t *slot, Scores &sc) const {
    // BF16: K region (h, c) holds dims 32c .. 32c + 31 of 16-row block h.
    // FP8: K region (h, cc) dims 64cc .. 64cc + 63, unit (row r, 16-byte chunk
    // j) at 16 j + r; the lane's 8 dims 32c + 8 quad .. are half quad & 1 of
    // unit 2 (c & 1) + (quad >> 1) of region (h, c >> 1), widened to BF16
    // (exactly) after the read.
    const uint8_t *kt = FP8 ? slot + 256 * (quad >> 1) + 16 * col + 8 * (quad & 1)
                            : slot + (16 * quad + col) * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 k0, k1;
      if constexpr (FP8) {
        const int o = (c >> 1) * 1024 + 512 * (c & 1);
        k0 = fp8x8_to_bf16x8(*reinterpret_cast<const u32x2 *>(kt + o));
        k1 = fp8x8_to_bf16x8(*reinterpret_cast<const u32x2 *>(kt + 2048 + o));
      } else {
        k0 = *reinterpret_cast<const u32x4 *>(kt + c * 1024);
        k1 = *reinterpret_cast<const u32x4 *>(kt + (4 + c) * 1024);
      }
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        sc.s0[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k0), as_bf16x8(qf[t][c]),
                                                           c ? sc.s0[t] : z, 0, 0, 0);
        sc.s1[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k1), as_bf16x8(qf[t][c]),
                                                           c ? sc.s1[t] : z, 0, 0, 0);
      }
    }
  }

  // The online softmax and O += P·V of the block in `slot` from its scores.
  // `full`: every token of the block lies inside the causal range of every
  // valid column of the wave (no masking needed).
  __device__ void apply(const uint8_t *slot, const Scores &sc, int64_t lt0, bool full) {
    const f32x4 *s0 = sc.s0, *s1 = sc.s1;
    bf16x8 pt[CT];
#pragma unroll
    for (int t = 0; t < CT; ++t) {
      // sr[i] = S[token 4 quad + i][column], sr[4 + i] = S[16 + 4 quad + i][column]
      // (unscaled); tokens at or past the column's causal end are masked
      float sr[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sr[i] = s0[t][i];
        sr[4 + i] = s1[t][i];
      }
      if (!full) {
        const int vis = (int)max<int64_t>(-1, min<int64_t>(32, end_col[t] - lt0));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sr[i] = (quad * 4 + i < vis) ? sr[i] : -INFINITY;
          sr[4 + i] = (16 + quad * 4 + i < vis) ? sr[4 + i] : -INFINITY;
        }
      }
      // the scale is positive, so the max is taken before scaling
      // (IEEE maximum: no NaN quieting of the MFMA results, three inputs per
      // instruction)
      const float ml = fmax_nan(fmax_nan(fmax_nan(sr[0], sr[1]), sr[2]),
                                fmax_nan(fmax_nan(fmax_nan(sr[3], sr[4]), sr[5]),
                                         fmax_nan(sr[6], sr[7])));
      // Lazy rescale: the column's reference max moves only when a score
      // exceeds it by more than 2^8 (weights stay <= 256, exact in range for
      // BF16 and FP32), so after the first blocks O and the normalizer are
      // almost never rescaled.  LSE = reference max + log2(normalizer).
      // The column max (across the four row quads) is needed only when some
      // lane's own max passes the threshold: rounding is monotonic, so no
      // lane passing means no column passes.
      if (__builtin_amdgcn_ballot_w64(ml * a.scale_log2 > m_run[t] + kLazyRescaleLog2)) {
        const float mx = quad_max_nan(ml) * a.scale_log2;
        const bool grow = mx > m_run[t] + kLazyRescaleLog2;
        const float m_ref = grow ? mx : m_run[t];
        // (a column with nothing visible before has O = 0: nothing to rescale)
        if (__builtin_amdgcn_ballot_w64(grow && m_run[t] != -INFINITY)) {
          // 1 where the max stays; 0 where nothing was visible
          const float al = fast_exp2(m_run[t] - (m_ref == -INFINITY ? 0.0f : m_ref));
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[t][e] *= al;
          lsum[t] *= al;
        }
        m_run[t] = m_ref;
      }
      const float m_use = m_run[t] == -INFINITY ? 0.0f : m_run[t];  // nothing visible yet
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = fast_exp2(fmaf(sr[i], a.scale_log2, -m_use));
      // Pᵀ as the B fragment (lane: column, k = 8 quad + [0, 8)): k = 8 quad +
      // i is token 4 quad + i, k = 8 quad + 4 + i token 16 + 4 quad + i
      pt[t] = as_bf16x8(bf16x2_pack(p[0], p[1]), bf16x2_pack(p[2], p[3]), bf16x2_pack(p[4], p[5]),
                        bf16x2_pack(p[6], p[7]));
      // the normalizer on the matrix core: a ones matrix times Pᵀ sums each
      // column's BF16 weights (the ones the P·V product uses) into every row
      lsum[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u), pt[t], lsum[t], 0, 0, 0);
    }
    // V region (h, e / 2) of 16-row block h: lane 4k + m of a quad addresses
    // dims 16 e + 4m .. + 3 of token row 4 quad + k, and the transposing read
    // gives lane col the four tokens 4 quad .. 4 quad + 3 (16 + 4 quad .. for
    // block 1) of dim 16 e + col, as the Pᵀ fragment orders them
    //
    // FP8: V region (h, cc) holds dims 64cc .. 64cc + 63 of block h, unit (row
    // r, chunk j) at 16 j + ((r + 8h) & 15); lane c of a quad addresses dims
    // 16 e + 8 (c & 1) .. + 7 of token row 4 quad + ((c >> 1) & 3) of block
    // c >> 3, and the transposing byte read (ds_read_b64_tr_b8: lane i
    // receives byte i % 8 of the 8 bytes lane 2k + i / 8 addresses, k =
    // 0..7) gives lane col the eight tokens of dim 16 e + col in Pᵀ order.
    const int hv = col >> 3, rv = (4 * quad + ((col >> 1) & 3) + 8 * hv) & 15;
    const uint8_t *vl =
        FP8 ? slot + kVBase + 2048 * hv + 16 * rv + 8 * (col & 1)
            : slot + kVBase + (8 * quad + 2 * (col >> 2) + ((col & 3) >> 1)) * 16 + (col & 1) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bf16x8 va;
      if constexpr (FP8) {
        const u32x2 b = lds_read_tr8(vl + (e >> 2) * 1024 + 256 * (e & 3));
        const u32x4 w = fp8x8_to_bf16x8(b);
        va = as_bf16x8(w[0], w[1], w[2], w[3]);
      } else {
        const u32x2 lo = lds_read_tr16(vl + (e >> 1) * 1024 + 512 * (e & 1));
        const u32x2 hi = lds_read_tr16(vl + (4 + (e >> 1)) * 1024 + 512 * (e & 1));
        va = as_bf16x8(lo[0], lo[1], hi[0], hi[1]);
      }
#pragma unroll
      for (int t = 0; t < CT; ++t)
        acc[t][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pt[t], acc[t][e], 0, 0, 0);
    }
  }

  // 16-row blocks 0..n16-1 of the current page-index window as 32-token
  // blocks (the second half of the last one is empty when n16 is odd: no
  // rows).  Each block is 16 buffer loads of 1 KB straight into LDS (64 lanes
  // x 16 bytes, written in lane order); wave w loads K and V regions (h =
  // w / 2, c = 2 (w & 1), c + 1) of 16-row block h.  Rows past a page's
  // valid rows read as zeros (buffer bounds).  Two ring slots, used in turn
  // across windows (`rpos`): after barrier i, block i + 1 goes into the slot
  // block i - 1 used (every wave has finished it), one block step ahead of
  // its use; before barrier i, each wave waits for its own loads of block i.
  // A new window's first block goes into the slot after the previous
  // window's last block.  (Loading two blocks ahead through a third slot
  // measured the same at 4-8K rows and 25% slower on a 1024-row prompt.)
  // G wave groups (the wave's group `grp`, its wave within the group `wave`)
  // split the blocks: group g takes blocks g, g + G, ..., through a ring of
  // its own, in lockstep with the others (one workgroup barrier per step).
  template <class PageOff, class RowsOf, class LtOf>
  __device__ void stream(int n16, PageOff page_off, RowsOf rows_of, LtOf lt_of, uint8_t *ring,
                         int wave, int grp, int64_t own_end) {
    const int row_bytes = a.row_elems * (FP8 ? 1 : 2);
    const int nb = (n16 + 1) >> 1;
    const int h = wave >> 1, c0 = FP8 ? (wave & 1) : 2 * (wave & 1);
    // BF16 K: LDS unit l = (row l & 15, chunk l >> 4); V: (row (l >> 1) & 15,
    // chunk 2 (l >> 5) + (l & 1)); region c0 + 1 is 64 bytes further per row.
    // FP8 (one region of K and one of V per wave): K unit l = (row l & 15,
    // chunk l >> 4); V unit l = (row ((l & 15) + 8h) & 15, chunk l >> 4).
    const int koff = FP8 ? (lane & 15) * row_bytes + 64 * c0 + (lane >> 4) * 16
                         : (lane & 15) * row_bytes + (4 * c0 + (lane >> 4)) * 16;
    const int voff = FP8 ? (((lane & 15) + 8 * h) & 15) * row_bytes + 64 * c0 + (lane >> 4) * 16
                         : ((lane >> 1) & 15) * row_bytes + (4 * c0 + 2 * (lane >> 5) + (lane & 1)) * 16;
    const uint8_t *kb = reinterpret_cast<const uint8_t *>(a.k) + (int64_t)kvh * a.head_elems * (FP8 ? 1 : 2);
    const uint8_t *vb = reinterpret_cast<const uint8_t *>(a.v) + (int64_t)kvh * a.head_elems * (FP8 ? 1 : 2);
    auto slot_at = [&](int r) { return ring + (grp * 2 + r) * kSlotBytes; };
    auto next_slot = [](int r) { return r ^ 1; };
    // LDS byte address of this group's ring (one generic-to-LDS conversion)
    const uint32_t ring_lds =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring +
        (uint32_t)(grp * 2 * kSlotBytes);
    auto issue = [&](int i, int slot) {
      const int b16 = 2 * i + h;
      const int rows = rows_of(b16);
      const uint64_t off = page_off(b16);  // bytes
      const int bytes = rows > 0 ? ((rows - 1) * a.row_elems + 128) * (FP8 ? 1 : 2) : 0;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t *>(kb + off), 0, bytes, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t *>(vb + off), 0, bytes, 0x00020000);
      const uint32_t sl = ring_lds + (uint32_t)(slot * kSlotBytes);
      if constexpr (FP8) {
        lds_load16_at(rk, sl + (2 * h + c0) * 1024, koff);
        lds_load16_at(rv, sl + kVBase + (2 * h + c0) * 1024, voff);
      } else {
        const uint32_t kr = sl + (4 * h + c0) * 1024;
        lds_load16_at(rk, kr, koff);
        lds_load16_at(rk, kr + 1024, koff + 64);
        lds_load16_at(rv, kr + 8192, voff);
        lds_load16_at(rv, kr + 9216, voff + 64);
      }
    };
    int cur = rpos;
    if (grp < nb) issue(grp, cur);
    const int steps = (nb + G - 1) / G;
    for (int j = 0; j < steps; ++j) {
      const int i = G * j + grp;
      wait_vmcnt<0>();  // this wave's loads of block i
      __syncthreads();
      if (i + G < nb) issue(i + G, next_slot(cur));
      const int64_t lt0 = lt_of(2 * i);
      if (i < nb && lt0 < own_end) {
        Scores sc;
        scores(slot_at(cur), sc);
        apply(slot_at(cur), sc, lt0, lt0 + 32 <= full_end);
      }
      cur = next_slot(cur);
    }
    rpos = cur;
  }
};

// Query tiles per wave of the long-tile algorithm: two (128 columns per
// workgroup) when that still gives at least kLongTwoMinGrid workgroups (two
// per CU), else one (64 columns).  Measured on GQA4 32/8 prompts, two tiles
// per wave at three waves per SIMD against one tile at four: 980 against 747
// TFLOP/s at 8192 rows, 804-841 against 627 at 4096, 778 against 623 on 4 x
// 2048 rows, 185-191 against 185 on 8 x 256; on 1 x 1024 rows (256 against
// 512 workgroups) the two measured the same.
constexpr int kLongTwoMinGrid = 512;

// SH: the wide-tile algorithm (W = 4, BF16): 16 * W columns per workgroup,
// one 16-column tile per wave, every wave over the whole page range.
// LT: the long-tile algorithm (SH's columns and block walk; 32-token blocks,
// query fragments in registers, BF16 P, Vᵀ staged transposed).
template <int W, bool RAGGED, bool FP8, bool SH, int LT = 0>
__device__ __forceinline__ void prefill_body(const PrefillArgs &args) {
  static_assert(!SH || W == 4 || (LT >= 1 && W == 8),
                "wide tiles: four waves; long tiles: four, or two groups of four with one tile");
  static_assert(!LT || SH, "long tiles: the wide tiles' columns");
  // Long tiles: four waves own the query tiles; G groups of them split the
  // K/V blocks and merge at the end.
  constexpr int G = LT ? W / 4 : 1;
  constexpr int TC = LT ? 16 * 4 * LT : SH ? 16 * W : 16;  // flattened columns per workgroup
  // FP8 pages: K's scale folds into the score scale, V's into the output.
  PrefillArgs a = args;
  float v_scale = 1.0f;
  if constexpr (FP8) {
    a.scale_log2 *= a.kv_scales[0];
    v_scale = a.kv_scales[1];
  }
  __shared__ PrefillSmem<W, SH, LT> sm;
  // long tiles: two K/V block slots per wave group (two groups: at least the
  // merge staging of four waves' column states, 34 floats per lane and tile)
  constexpr int kRingBytes = LT ? 2 * G * (FP8 ? 8192 : 16384) : 16;
  constexpr int kMergeBytes = G == 2 ? LT * 34 * 4 * 64 * 4 : 0;
  __shared__ __align__(16) uint8_t lring[kRingBytes > kMergeBytes ? kRingBytes : kMergeBytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, quad = lane >> 4;
  const int kvh = (int)(blockIdx.x % a.hkv);
  // Tiles in reverse order: a request's later rows see longer causal ranges,
  // so the heaviest tiles are dispatched first and the launch does not end
  // with a few long tiles running alone (the grid's excess workgroups, which
  // find no tile, come first and exit at once).  Workgroup b runs on XCD
  // b % 8; with the kv-head fastest, each XCD keeps to a fixed set of
  // kv-heads, whose K/V its L2 shares across tiles.
  const int64_t n_tiles = (int64_t)(gridDim.x / a.hkv), m = blockIdx.x / a.hkv;
  int64_t rank = m;
  if (a.tile_layer > 0) {
    // Serpentine: every other layer of tile_layer workgroups (one per CU of
    // the XCDs this kv-head runs on) takes its tiles in reverse, so a CU's
    // successive workgroups pair heavy tiles with light ones instead of
    // stacking the heaviest of every layer.
    const int64_t L = a.tile_layer, layer = m / L, c = m - layer * L;
    const int64_t width = min(L, n_tiles - layer * L);
    rank = layer * L + ((layer & 1) ? width - 1 - c : c);
  }
  const int64_t tile = n_tiles - 1 - rank;
  const bool interleave = !RAGGED && LT && a.tile_interleave != 0;

  // Metadata in as few dependent round trips as possible: the global guard
  // words and every request's qo range, page (kv) range and tail are loaded
  // together; the guards are applied after the scan that locates this tile.
  const int32_t qo0 = a.qo[0], qoB = a.qo[a.batch];
  const int32_t ip0 = a.indptr[0], ipB = a.indptr[a.batch];
  // A page-index array of at most 128 entries (the reference's shapes) is
  // loaded whole in the same round trip, two words per lane: the request's
  // page indices and their check then come from registers, so the query tile
  // and the first K/V blocks share the second round trip.
  const bool small_table = !RAGGED && !SH && a.n_indices <= 128;
  int tbl0 = 0, tbl1 = 0;
  if (small_table) {
    if (lane < a.n_indices) tbl0 = a.indices[lane];
    if (lane + 64 < a.n_indices) tbl1 = a.indices[lane + 64];
  }

  // Locate the request owning this tile: prefix of the requests' tile counts.
  // Paged (prefill.rs:303-313): rows belong to the requests before the first
  // malformed qo range.  Ragged (prefill.rs:111-137): row q belongs to the
  // first request r with q < qo_indptr[r+1], i.e. r owns the rows from
  // max(qo_indptr[r], max(qo_indptr[1..r])) to qo_indptr[r+1], and a request
  // failing its guards keeps its rows' sentinels.
  if (tid == 0) sm.req = -1;
  int64_t carry = 0;
  int32_t carry_max = 0;
  for (int base = 0; base < a.batch; base += W * 64) {
    const int r = base + tid;
    int64_t cnt = 0;
    int32_t s0 = 0, s1 = 0, p0 = 0, p1 = 0, t1 = 0, fbeg = 0;
    if (r < a.batch) {
      s0 = a.qo[r];
      s1 = a.qo[r + 1];
      p0 = a.indptr[r];
      p1 = a.indptr[r + 1];
      if constexpr (!RAGGED) t1 = a.last[r];
    }
    if constexpr (RAGGED) {
      // exclusive running max of the qo ends before r
      int32_t x = r < a.batch ? s1 : INT32_MIN;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x = max(x, y);
      }
      if (lane == 63) sm.wave_max[wave] = x;
      __syncthreads();
      int32_t before = carry_max, blk = carry_max;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        before = i < wave ? max(before, sm.wave_max[i]) : before;
        blk = max(blk, sm.wave_max[i]);
      }
      const int32_t up = __shfl_up(x, 1, 64);
      const int32_t excl = lane > 0 ? max(before, up) : before;
      carry_max = blk;
      if (r < a.batch) {
        const bool ok = s0 >= 0 && s1 > s0 && s1 <= a.nnz && p0 >= 0 && p1 > p0 &&
                        p1 <= a.nnz_kv && s1 - s0 <= p1 - p0;
        const int32_t lo = max(s0, excl);
        if (ok && s1 > lo) {
          cnt = ((int64_t)(s1 - lo) * a.group + TC - 1) / TC;
          fbeg = (lo - s0) * a.group;
        }
      }
    } else {
      if (r < a.batch)
        cnt = (s0 >= 0 && s1 > s0 && s1 <= a.nnz) ? ((int64_t)(s1 - s0) * a.group + TC - 1) / TC
                                                  : kNoTiles;
    }
    if (interleave && wave == 0) {
      // (at most 64 requests: wave 0 holds every count, one pass.)  Rank
      // rank - excess is the j-th of the tiles k from their request's end,
      // where k is the largest with F(k) = sum of min(k, count) <= it and j
      // counts requests with more than k tiles in request order; requests
      // from the first malformed qo range on own no tile.
      const bool in = r < a.batch;
      const uint64_t badm = __ballot(in && cnt == kNoTiles);
      const int first_bad = badm ? __builtin_ctzll(badm) : 64;
      const int c = (in && lane < first_bad) ? (int)cnt : 0;
      const int total = wave_sum_i32(c);
      const int64_t rr = rank - (n_tiles - total);
      if (rr >= 0) {
        int lo = 0, hi = wave_max_i32(c);
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (wave_sum_i32(min(mid, c)) <= rr) lo = mid;
          else hi = mid;
        }
        const int j = (int)(rr - wave_sum_i32(min(lo, c)));
        const uint64_t more = __ballot(c > lo);
        const int below = (int)__builtin_amdgcn_mbcnt_hi(
            (uint32_t)(more >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)more, 0u));
        if (c > lo && below == j) {
          sm.req = r;
          sm.tile0 = c - 1 - lo;
          sm.meta[0] = s0;
          sm.meta[1] = s1;
          sm.meta[2] = p0;
          sm.meta[3] = p1;
          sm.meta[4] = t1;
          sm.meta[5] = fbeg;
        }
      }
    }
    const int64_t x = wave_incl_scan64(cnt, lane);
    if (lane == 63) sm.wave_tot[wave] = x;
    __syncthreads();
    int64_t before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const int64_t t = sm.wave_tot[i];
      before += (i < wave) ? t : 0;
      tot += t;
    }
    const int64_t incl = carry + before + x;
    if (!interleave && r < a.batch && tile < incl && tile >= incl - cnt && cnt != kNoTiles) {
      sm.req = r;
      sm.tile0 = (int32_t)(tile - (incl - cnt));
      sm.meta[0] = s0;
      sm.meta[1] = s1;
      sm.meta[2] = p0;
      sm.meta[3] = p1;
      sm.meta[4] = t1;
      sm.meta[5] = fbeg;
    }
    carry += tot;
    __syncthreads();
    if (carry > tile || interleave) break;
  }
  // Global guards (prefill.rs:293-300 paged, :102-108 ragged).
  if constexpr (RAGGED) {
    if (qo0 != 0 || qoB != a.nnz || ip0 != 0 || ipB != a.nnz_kv) return;
  } else {
    const bool pages_ok = ipB >= 0 && (a.indices_capacity ? (int64_t)ipB <= a.n_indices
                                                          : (int64_t)ipB == a.n_indices);
    if (qo0 != 0 || qoB != a.nnz || ip0 != 0 || !pages_ok) return;
  }
  const int r = uni(sm.req);
  if (r < 0) return;
  const int tile0 = uni(sm.tile0);
  const int fbeg = uni(sm.meta[5]);

  // Per-request guards (paged: prefill.rs:316-342; ragged: applied in the
  // scan above, a failing request owns no tile).
  const int32_t qs = uni(sm.meta[0]), qe = uni(sm.meta[1]);
  const int32_t ps = uni(sm.meta[2]), pe = uni(sm.meta[3]);
  int req_pages;
  int32_t tl;
  int64_t kv_len;
  if constexpr (RAGGED) {
    kv_len = pe - ps;
    req_pages = (int)((kv_len + 15) / 16);
    tl = (int32_t)(kv_len - (int64_t)(req_pages - 1) * 16);
  } else {
    tl = uni(sm.meta[4]);
    if (ps < 0 || pe <= ps || pe > ipB || tl < 1 || tl > a.page_rows) return;
    kv_len = (int64_t)(pe - ps - 1) * a.page_rows + tl;
    // 16-row blocks of the request and the valid rows of its last one
    req_pages = (int)((kv_len + 15) / 16);
    tl = (int32_t)(kv_len - (int64_t)(req_pages - 1) * 16);
  }
  const int qo_len = qe - qs;
  if ((int64_t)qo_len > kv_len) return;

  // This lane's column and the tile's page range.
  // (fcols <= nnz_qo * Hq fits int32: the plan checks it)
  const int fcols = qo_len * a.group;
  // first column of this wave's tile(s)
  const int wq = LT ? (wave & 3) : wave;  // long tiles: the wave's tiles within its group
  const int grp = LT ? (wave >> 2) : 0;
  const int own0 = fbeg + tile0 * TC + (LT ? 16 * LT * wq : SH ? 16 * wave : 0);
  const int f = own0 + col;
  const bool colv = f < fcols;
  const int qi = colv ? (int)((uint32_t)f / (uint32_t)a.group) : 0;
  const int gh = colv ? f - qi * a.group : 0;
  const int f_last = min(fbeg + tile0 * TC + TC - 1, fcols - 1);
  const int64_t tile_end = kv_len - qo_len + (int)((uint32_t)f_last / (uint32_t)a.group) + 1;
  // (the page counts are wave-uniform; pinning them to SGPRs keeps the buffer
  // resources below scalar, with no waterfall loops around the loads)
  const int npages = uni((int)((tile_end + 15) / 16));
  // (SH: every wave walks every block; otherwise wave w takes blocks w, w + W, ...)
  const int mine = SH ? npages : uni(npages > wave ? (npages - wave + W - 1) / W : 0);
  auto blk = [&](int i) { return SH ? i : wave + W * i; };

  // Every page index of the request is checked (the reference rejects the
  // whole request; the verdict is read after the stream) and each wave takes
  // its first block of page indices: from the registers of a small table, else
  // in one round trip with the query tile (wave 0).
  bool bad = false;
  int idx = 0;
  if constexpr (!RAGGED) {
    if (small_table) {
      // entries ps..pe-1 of the table (pe <= n_indices <= 128)
      const int j0 = lane, j1 = lane + 64;
      bad = (j0 >= ps && j0 < pe && (tbl0 < 0 || (int64_t)tbl0 >= a.pool)) ||
            (j1 >= ps && j1 < pe && (tbl1 < 0 || (int64_t)tbl1 >= a.pool));
      const int j = ps + (blk(lane) >> a.blocks_lg);  // < pe for this wave's blocks
      const int x0 = __shfl(tbl0, j & 63, 64), x1 = __shfl(tbl1, j & 63, 64);
      if (lane < min(mine, 64)) idx = j < 64 ? x0 : x1;
    } else {
      for (int i = tid; i < pe - ps; i += W * 64) {
        const int32_t x = a.indices[ps + i];
        bad |= x < 0 || (int64_t)x >= a.pool;
      }
      idx = lane < min(mine, 64) ? a.indices[ps + (blk(lane) >> a.blocks_lg)] : 0;
    }
  }

  PrefillWave w{a, sm.qfrag[(SH && !LT) ? wave : 0], lane, col, quad, kvh};
  w.end_col = colv ? kv_len - qo_len + qi + 1 : 0;
  w.reset();
  // Long tiles: this lane's column of each of the wave's tiles.
  constexpr int LTT = LT ? LT : 1;
  LongWave<LTT, FP8, G> lw{a, lane, col, quad, kvh};
  bool colv_t[LTT];
  int qi_t[LTT], gh_t[LTT];
  if constexpr (LT) {
#pragma unroll
    for (int t = 0; t < LTT; ++t) {
      const int ft = own0 + 16 * t + col;
      colv_t[t] = ft < fcols;
      qi_t[t] = colv_t[t] ? (int)((uint32_t)ft / (uint32_t)a.group) : 0;
      gh_t[t] = colv_t[t] ? ft - qi_t[t] * a.group : 0;
      lw.end_col[t] = colv_t[t] ? kv_len - qo_len + qi_t[t] + 1 : 0;
    }
    // the smallest causal end of the wave's valid columns: blocks before it
    // need no mask (the columns past fcols are discarded, so they do not count)
    int64_t fe = INT64_MAX;
#pragma unroll
    for (int t = 0; t < LTT; ++t) fe = colv_t[t] ? min(fe, lw.end_col[t]) : fe;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const int64_t y = ((int64_t)__shfl_xor((int)(fe >> 32), o, 64) << 32) |
                        (uint32_t)__shfl_xor((int)(uint32_t)fe, o, 64);
      fe = min(fe, y);
    }
    lw.full_end = uni64(fe);
    lw.reset();
  }
  // The current block of up to 64 page indices (one per lane) of this wave.
  int s0 = 0;
  int n = uni(min(mine, 64));
  int ok = (RAGGED || (idx >= 0 && (int64_t)idx < a.pool)) ? 1 : 0;
  auto page_tok = [&](int i) {
    if constexpr (RAGGED) return ((int64_t)ps + (int64_t)blk(s0 + i) * 16) * a.hkv * 128;
    const int j = uni(min(i, n - 1));
    const int b = blk(s0 + j);
    return (int64_t)__builtin_amdgcn_readlane(idx, j) * a.page_rows * a.hkv * 128 +
           (int64_t)((b & ((1 << a.blocks_lg) - 1)) * 16) * a.row_elems;
  };
  auto rows_of = [&](int i) {
    if (i >= n || !__builtin_amdgcn_readlane(ok, i)) return 0;
    return uni(blk(s0 + i) == req_pages - 1 ? (int)tl : 16);
  };
  auto lt_of = [&](int i) { return (int64_t)blk(s0 + i) * 16; };
  // Long tiles: byte offset of 16-row block i of the window in K or V (kv-head
  // 0), with 32-bit factors: a page's bytes (page_rows x Hkv x 128 elements)
  // are far below 2^32, and an index failing the guard has no valid rows, so
  // its loads read nothing whatever the offset.
  const uint32_t page_bytes = (uint32_t)(a.page_rows * a.hkv * 128 * (FP8 ? 1 : 2));
  const uint32_t block_bytes = (uint32_t)(16 * a.row_elems * (FP8 ? 1 : 2));
  auto page_off = [&](int i) -> uint64_t {
    const int j = uni(min(i, n - 1));
    const uint32_t pg = (uint32_t)__builtin_amdgcn_readlane(idx, j);
    const uint32_t sub = (uint32_t)(blk(s0 + j) & ((1 << a.blocks_lg) - 1));
    return (uint64_t)pg * page_bytes + sub * block_bytes;
  };
  // The query tile's loads and the first blocks' loads go out together,
  // before the barrier that publishes the tile.  They follow the first index
  // block, so no wait for it holds back the page loads.  Lanes past the tile's
  // last column load row 0 of Q (it exists, since a tile was found) and store
  // zeros: with no branch around the loads, no wait at a join stalls them.
  // (the empty asm pins the index check here, ahead of the query loads: sunk
  // below them, its wait for a loaded index block would also wait for Q)
  asm volatile("" ::"v"(ok) : "memory");
  u32x4 qr[4];
  if constexpr (LT) {
#pragma unroll
    for (int t = 0; t < LTT; ++t) {
      const uint16_t *qp = colv_t[t] ? a.q + ((int64_t)(qs + qi_t[t]) * a.hq +
                                              (int64_t)kvh * a.group + gh_t[t]) * 128 + quad * 8
                                     : a.q + quad * 8;
#pragma unroll
      for (int c = 0; c < 4; ++c) lw.qf[t][c] = load16(qp + c * 32);
    }
  } else if (SH || wave == 0) {
    const uint16_t *qp =
        colv ? a.q + ((int64_t)(qs + qi) * a.hq + (int64_t)kvh * a.group + gh) * 128 + quad * 8
             : a.q + quad * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] = load16(qp + c * 32);
  }
  constexpr int D = SH ? 1 : prefill_depth(W);
  PrefillBuf<FP8> buf[D];
  if constexpr (!SH) {
    if (mine > 0) w.template prime<D, FP8>(buf, page_tok, rows_of);
  }
  if (!LT && (SH || wave == 0)) {
#pragma unroll
    for (int c = 0; c < 4; ++c) sm.qfrag[SH ? wave : 0][c][lane] = colv ? qr[c] : u32x4{0, 0, 0, 0};
  }
  if constexpr (LT) {
#pragma unroll
    for (int t = 0; t < LTT; ++t)
#pragma unroll
      for (int c = 0; c < 4; ++c) lw.qf[t][c] = colv_t[t] ? lw.qf[t][c] : u32x4{0, 0, 0, 0};
  }
  __syncthreads();

  for (; s0 < mine; s0 += 64) {
    if (s0 > 0) {
      n = uni(min(mine - s0, 64));
      if constexpr (!RAGGED) idx = lane < n ? a.indices[ps + (blk(s0 + lane) >> a.blocks_lg)] : 0;
      ok = (RAGGED || (idx >= 0 && (int64_t)idx < a.pool)) ? 1 : 0;
    }
    if constexpr (SH) {
      // causal end of this wave's last column (0: the wave's tile is empty)
      const int last_own = own0 + (LT ? 16 * LTT : 16) - 1;
      const int64_t own_end =
          own0 < fcols
              ? kv_len - qo_len + (int)((uint32_t)min(last_own, fcols - 1) / (uint32_t)a.group) + 1
              : 0;
      if constexpr (LT) {
        lw.stream(n, page_off, rows_of, lt_of, lring, wq, grp, uni64(own_end));
      } else {
        __shared__ u32x4 ring[2][2][16][17];
        w.template stream_shared<FP8>(n, page_tok, rows_of, lt_of, ring, wave, uni64(own_end));
      }
    } else {
      w.template stream<D, FP8>(buf, s0 == 0, n, page_tok, rows_of, lt_of);
    }
  }

  if constexpr (LT) {
    // Each wave finishes its own tiles; an invalid page index anywhere in the
    // request keeps its sentinels.
    float Lt[LTT];
#pragma unroll
    for (int t = 0; t < LTT; ++t) Lt[t] = lw.lsum[t][0];
    if (block_or(bad, sm.bad)) return;
    if constexpr (G == 2) {
      // Group 1 hands its column states to group 0 through the ring's LDS
      // (every wave is past its last ring read: block_or's barrier), and
      // group 0 merges them with its own, as the split-K merge does.
      static_assert(LTT * 34 * 4 * 64 * 4 <= sizeof(lring), "merge staging fits the ring");
      float *xs = reinterpret_cast<float *>(lring) + wq * (LTT * 34 * 64) + lane;
      if (grp == 1) {
#pragma unroll
        for (int t = 0; t < LTT; ++t) {
          float *x = xs + t * 34 * 64;
          x[0] = lw.m_run[t];
          x[64] = Lt[t];
#pragma unroll
          for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[(2 + 4 * e + i) * 64] = lw.acc[t][e][i];
        }
      }
      __syncthreads();
      if (grp == 1) return;
#pragma unroll
      for (int t = 0; t < LTT; ++t) {
        const float *x = xs + t * 34 * 64;
        const float m1 = x[0], l1 = x[64], m0 = lw.m_run[t];
        const float M = fmaxf(m0, m1);
        const float f0 = m0 == -INFINITY ? 0.0f : fast_exp2(m0 - M);
        const float f1 = m1 == -INFINITY ? 0.0f : fast_exp2(m1 - M);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            lw.acc[t][e][i] = lw.acc[t][e][i] * f0 + x[(2 + 4 * e + i) * 64] * f1;
        Lt[t] = Lt[t] * f0 + l1 * f1;
        lw.m_run[t] = M;
      }
    }
#pragma unroll
    for (int t = 0; t < LTT; ++t) {
      if (!colv_t[t]) continue;
      const float inv = 1.0f / Lt[t];
      const int64_t row_head = (int64_t)(qs + qi_t[t]) * a.hq + (int64_t)kvh * a.group + gh_t[t];
      // acc[t][e][i] = O[column][16 e + 4 quad + i]: 8 bytes per dim block
      uint16_t *orow = a.out + row_head * 128 + quad * 4;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<u32x2 *>(orow + 16 * e) =
            u32x2{bf16x2_pack(lw.acc[t][e][0] * inv * v_scale, lw.acc[t][e][1] * inv * v_scale),
                  bf16x2_pack(lw.acc[t][e][2] * inv * v_scale, lw.acc[t][e][3] * inv * v_scale)};
      if (quad == 0) a.lse[row_head] = lw.m_run[t] + __log2f(Lt[t]);
    }
    return;
  } else if constexpr (SH) {
    // No cross-wave merge: each wave finishes its own tile.
    const float L = quad_sum(w.l_run);
    if (block_or(bad, sm.bad) || !colv) return;
    const float inv = 1.0f / L;
    const int64_t row_head = (int64_t)(qs + qi) * a.hq + (int64_t)kvh * a.group + gh;
    uint16_t *orow = a.out + row_head * 128 + quad * 32;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      u32x4 o;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2)
        o[e2] = bf16x2_pack(w.acc[2 * e2][r4] * inv * v_scale, w.acc[2 * e2 + 1][r4] * inv * v_scale);
      *reinterpret_cast<u32x4 *>(orow + r4 * 8) = o;
    }
    if (quad == 0) a.lse[row_head] = w.m_run + __log2f(L);
    return;
  }

  // Wave states -> LDS; an invalid page index anywhere in the request keeps
  // its sentinels.  Every value below belongs to the lane's own column.
  const float l_tot = quad_sum(w.l_run);
  if (quad == 0) {
    sm.m[wave][col] = w.m_run;
    sm.l[wave][col] = l_tot;
  }
  if (block_or(bad, sm.bad)) return;
  float M = -INFINITY;
#pragma unroll
  for (int wv = 0; wv < W; ++wv) M = fmaxf(M, sm.m[wv][col]);
  {
    const float fac = M == -INFINITY ? 0.0f : fast_exp2(w.m_run - M);
#pragma unroll
    for (int e = 0; e < 8; ++e) w.acc[e] *= fac;
  }
  // Deterministic tree sum of the accumulators of the waves that streamed
  // pages (wave w streamed iff w < npages), half of them per pass.
  const int active = min(npages, W);
#pragma unroll
  for (int s = W / 2; s >= 1; s >>= 1) {
    if (s >= active) continue;  // waves s.. hold nothing: skip the round (uniform)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (wave >= s && wave < 2 * s)
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.red[wave - s][e][lane] = w.acc[4 * h + e];
      __syncthreads();
      if (wave < s)
#pragma unroll
        for (int e = 0; e < 4; ++e) w.acc[4 * h + e] += sm.red[wave][e][lane];
      if (s > 1 || h == 0) __syncthreads();
    }
  }
  if (wave != 0 || !colv) return;
  float L = 0.0f;
#pragma unroll
  for (int wv = 0; wv < W; ++wv) L = fmaf(sm.l[wv][col], fast_exp2(sm.m[wv][col] - M), L);
  const float inv = 1.0f / L;
  const int64_t row_head = (int64_t)(qs + qi) * a.hq + (int64_t)kvh * a.group + gh;
  uint16_t *orow = a.out + row_head * 128 + quad * 32;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    u32x4 o;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2)
      o[e2] = bf16x2_pack(w.acc[2 * e2][r4] * inv * v_scale, w.acc[2 * e2 + 1][r4] * inv * v_scale);
    *reinterpret_cast<u32x4 *>(orow + r4 * 8) = o;
  }
  if (quad == 0) a.lse[row_head] = M + __log2f(L);
}

// At least three waves per SIMD: the per-block chain (MFMA, softmax, MFMA)
// leaves a wave waiting most of the time, and a third wave per SIMD fills
// those gaps (the four-wave BF16 kernel would otherwise settle at two).
constexpr int kPrefillWavesPerEu = 3;

// Long tiles: three waves per SIMD (three workgroups of 33.4 KB LDS per CU).
// With two query tiles per wave that is 168 registers: a few values live
// across the whole walk go to scratch, outside the block loop.  Measured
// against two waves per SIMD (176 registers, no scratch): 975 against 869
// TFLOP/s at 8192 rows, 822 against 695 at 4096.
template <int W, bool FP8, bool SH = false, int LT = 0>
__global__ __launch_bounds__(W * 64, LT ? (W == 8 ? (LT == 1 ? 4 : 2) : 3) : kPrefillWavesPerEu) void paged_prefill_kernel(PrefillArgs a) {
  prefill_body<W, false, FP8, SH, LT>(a);
}

// Ragged prefill: contiguous K/V rows [nnz_kv, Hkv, 128]; any 16 consecutive
// rows of a request form a block with the paged layout's row stride, so the
// same page step and range-limited loads serve it.
template <int W, bool SH = false>
__global__ __launch_bounds__(W * 64, kPrefillWavesPerEu) void ragged_prefill_kernel(PrefillArgs a) {
  prefill_body<W, true, false, SH>(a);
}

}  // namespace

// ---- provider / plan / enqueue -----------------------------------------------
struct loom_prefill_provider {
  loom::DeviceInfo dev;
};

struct loom_paged_prefill_plan {
  loom_paged_prefill_plan_info_t info{};
  uint32_t tile_cols = 16;  // flattened columns per workgroup
  uint32_t long_groups = 1;  // long tiles: wave groups splitting the K/V blocks
  uint32_t tile_layer = 0;   // serpentine tile order layer (PrefillArgs::tile_layer)
  bool tile_interleave = false;  // PrefillArgs::tile_interleave
};

struct loom_ragged_prefill_plan {
  loom_ragged_prefill_plan_info_t info{};
};

namespace {
// Waves per workgroup.  The reference picks its kernel from the average page
// capacity per request (prefill.rs:2417-2426); here four waves measured
// fastest on every shape of the reference's records, short and long (the
// per-page dependency chain, not load latency, bounds a wave, and deeper
// prefetch or more waves per tile did not shorten it), so the default is
// four whatever the spec; 8 and 16 stay available as plan options.
uint32_t waves_for() { return 4u; }

// Grid of a prefill plan: the most 16-column tiles any valid qo_indptr can
// produce (every request wastes less than one tile), times the kv-heads.
// prefill.rs:2293-2298 / :2335-2340: the (row, head) states must fit the
// launch range; the kernel indexes columns with int32.
loom_status_t prefill_grid(uint64_t batch, uint64_t nnz_qo, uint64_t hq, uint64_t hkv,
                           uint64_t tile_cols, uint64_t *tiles, uint64_t *grid,
                           loom_error_t *err) {
  const uint64_t states = nnz_qo * hq;
  if (states > (uint64_t)INT32_MAX || batch > (uint64_t)INT32_MAX - 1)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "prefill", states);
  const uint64_t cols = nnz_qo * (hq / hkv);
  *tiles = std::min(cols, (cols + (tile_cols - 1) * batch) / tile_cols);
  *grid = *tiles * hkv;
  if (*grid > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "prefill", states);
  return LOOM_OK;
}

// Columns per workgroup of a prefill plan: 64 (wide tiles) or 16.  Forced by
// the plan flags; otherwise wide when the average request has
// at least LOOM_PREFILL_WIDE_MIN_COLS flattened columns and the wide grid
// still holds LOOM_PREFILL_WIDE_MIN_GRID workgroups.  Measured on GQA4
// 32/8 prompts (qo = kv): wide 1.5-1.7x faster from 4 x 2048 and 8 x 256
// rows up, even at 1 x 1024 rows (512 workgroups), slower at 1 x 512 (256).
#ifndef LOOM_PREFILL_WIDE_MIN_COLS
#define LOOM_PREFILL_WIDE_MIN_COLS 256
#endif
#ifndef LOOM_PREFILL_WIDE_MIN_GRID
#define LOOM_PREFILL_WIDE_MIN_GRID 512
#endif
#ifndef LOOM_PREFILL_LONG_DEFAULT
#define LOOM_PREFILL_LONG_DEFAULT 1
#endif
// The long tiles from a 64-column grid of this many workgroups: measured on
// GQA4 32/8 prompts, 16.6 against 21.9 us (row tiles) at 1 x 512 rows (256
// workgroups), 11.0 against 9.8 us at 1 x 256 (128).
#ifndef LOOM_PREFILL_LONG_MIN_GRID
#define LOOM_PREFILL_LONG_MIN_GRID 256
#endif
#ifndef LOOM_PREFILL_LONG_GROUPS
#define LOOM_PREFILL_LONG_GROUPS 2
#endif
loom_status_t prefill_tile_cols(uint32_t flags, uint32_t waves, uint64_t batch,
                                uint64_t nnz_qo, uint64_t hq, uint64_t hkv, bool long_ok,
                                bool long_default, uint32_t *tile_cols, bool *long_tile,
                                loom_error_t *err) {
  const uint32_t t = flags & (LOOM_PLAN_PREFILL_TILE_16 | LOOM_PLAN_PREFILL_TILE_64 |
                              LOOM_PLAN_PREFILL_TILE_LONG);
  *long_tile = false;
  if (t & (t - 1)) return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", flags);
  if ((t == LOOM_PLAN_PREFILL_TILE_64 || t == LOOM_PLAN_PREFILL_TILE_LONG) && waves != 4)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "waves", waves);
  if (t == LOOM_PLAN_PREFILL_TILE_LONG && !long_ok)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", flags);
  if (t) {
    *tile_cols = t == LOOM_PLAN_PREFILL_TILE_16 ? 16 : 64;
    *long_tile = t == LOOM_PLAN_PREFILL_TILE_LONG;
    if (*long_tile && (nnz_qo * (hq / hkv) / 128) * hkv >= kLongTwoMinGrid) *tile_cols = 128;
    return LOOM_OK;
  }
  const uint64_t cols = nnz_qo * (hq / hkv);
  const uint64_t grid64 = (cols / 64) * hkv;
  const bool long_requests = waves == 4 && batch > 0 && cols >= LOOM_PREFILL_WIDE_MIN_COLS * batch;
  // Long prompts on BF16 pages take the long tiles, from a smaller grid than
  // the wide tiles need (see the algorithm's measurements in the plan's
  // documentation).
  *long_tile = long_requests && long_ok && long_default && LOOM_PREFILL_LONG_DEFAULT &&
               grid64 >= LOOM_PREFILL_LONG_MIN_GRID;
  if (*long_tile) {
    *tile_cols = (cols / 128) * hkv >= kLongTwoMinGrid ? 128 : 64;
    return LOOM_OK;
  }
  *tile_cols = long_requests && grid64 >= LOOM_PREFILL_WIDE_MIN_GRID ? 64 : 16;
  return LOOM_OK;
}

loom_status_t require_aligned(const char *name, uintptr_t ptr, uintptr_t alignment,
                              loom_error_t *err) {
  if (ptr % alignment != 0)
    return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, name, (int64_t)ptr, (int64_t)alignment);
  return LOOM_OK;
}
}  // namespace

extern "C" {

loom_status_t loom_prefill_provider_load(int device, loom_prefill_provider_t **out,
                                         loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  loom::DeviceInfo dev;
  loom_status_t rc = loom::query_device(device, &dev, err);
  if (rc) return rc;
  if (!dev.gfx950) return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, nullptr, device);
  auto *p = new loom_prefill_provider;
  p->dev = dev;
  *out = p;
  return loom::ok(err);
}

void loom_prefill_provider_free(loom_prefill_provider_t *p) { delete p; }

loom_status_t loom_prefill_provider_plan_bf16_paged_options(
    const loom_prefill_provider_t *provider, const loom_paged_prefill_spec_t *spec,
    const loom_paged_prefill_plan_options_t *options, loom_paged_prefill_plan_t **out,
    loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  const loom_paged_prefill_plan_options_t opt =
      options ? *options : loom_paged_prefill_plan_options_t{0, 0};
  if (opt.flags & ~(LOOM_PLAN_PAGE_INDICES_CAPACITY | LOOM_PLAN_PREFILL_TILE_16 |
                    LOOM_PLAN_PREFILL_TILE_64 | LOOM_PLAN_PREFILL_TILE_LONG))
    return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", opt.flags);
  if (spec->kv_layout != LOOM_KV_LAYOUT_NHD && spec->kv_layout != LOOM_KV_LAYOUT_HND)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_layout", spec->kv_layout);
  if (spec->page_size != 0 && spec->page_size != 16 && spec->page_size != 32 &&
      spec->page_size != 64)
    return fail(err, LOOM_UNSUPPORTED_PAGE_SIZE, nullptr, loom::kPageSize, spec->page_size);
  if (spec->kv_dtype != LOOM_KV_DTYPE_BF16 && spec->kv_dtype != LOOM_KV_DTYPE_FP8_E4M3)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "kv_dtype", spec->kv_dtype);
  if (opt.waves != 0 && opt.waves != 4 && opt.waves != 8 && opt.waves != 16)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "waves", opt.waves);
  const uint32_t waves = opt.waves ? opt.waves : waves_for();
  uint32_t tile_cols = 16;
  bool long_tile = false;
  loom_status_t rc = prefill_tile_cols(opt.flags, waves, spec->batch_size, spec->nnz_qo,
                                       spec->num_query_heads, spec->num_kv_heads, true, true,
                                       &tile_cols, &long_tile, err);
  if (rc) return rc;
  uint64_t tiles = 0, grid = 0;
  rc = prefill_grid(spec->batch_size, spec->nnz_qo, spec->num_query_heads, spec->num_kv_heads,
                    tile_cols, &tiles, &grid, err);
  if (rc) return rc;
  auto *p = new loom_paged_prefill_plan;
  p->info.spec = *spec;
  p->info.algorithm = long_tile        ? LOOM_PAGED_PREFILL_LONG_TILE
                      : tile_cols == 64 ? LOOM_PAGED_PREFILL_WIDE_TILE
                                        : LOOM_PAGED_PREFILL_ROW_TILE;
  p->tile_cols = tile_cols;
  // Long tiles of one query tile per wave (grids too small for two): two
  // groups of four waves split each tile's K/V blocks, halving the longest
  // tiles' serial block walk, when the grid fits one round of two such
  // workgroups per CU or the requests are long enough (1024 rows on average)
  // that the heaviest tiles dominate.  Measured (GQA4 32/8, BF16 / FP8 pages,
  // two groups against one): 1 x 512 rows -6% / -15%, 1 x 1024 -2% / -16%,
  // 1 x 1536 -10% / +2%, and 2 x 512 rows (520 workgroups, a second round)
  // +6% / -4%.  Long tiles of two query tiles per wave (one such 8-wave
  // workgroup per CU) split into two groups only on grids of at most two
  // workgroups per CU: 1 x 2048 rows -11% / -13%, but
  // 1 x 3072 +16%, 1 x 4096 +27%, 1 x 8192 +25% and 4 x 2048 +36% (the
  // 8-wave, 2-tile workgroup holds two waves per SIMD and 70 KB of LDS).
  const bool two_per_cu = grid <= 2 * (uint64_t)provider->dev.cus;
  const bool grouped = long_tile &&
                       ((tile_cols == 64 && (two_per_cu || spec->nnz_qo >= 1024 * spec->batch_size)) ||
                        (tile_cols == 128 && two_per_cu));
  p->long_groups = grouped ? LOOM_PREFILL_LONG_GROUPS : 1;
  // Serpentine tile order when the whole grid is resident at once (long
  // tiles: three 4-wave workgroups per CU; two 8-wave ones of one tile per
  // wave; one of two tiles per wave).  A second round is dispatched as CUs
  // free up, where heaviest-first order balances better.  Measured (GQA4
  // 32/8, BF16, same box): 1 x 1024 rows 28.6 -> 25.3 us, 2 x 512 18.5 ->
  // 17.2, 1 x 3072 100.5 -> 98.0, 8 x 256 20.1 -> 19.8; on grids of more
  // than one round 1 x 2048 (two tiles, two groups) 58 -> 70, 1 x 4096 141 ->
  // 147, 4 x 2048 153 -> 163.
  const uint64_t cus = provider->dev.cus, hkv_n = spec->num_kv_heads;
  const uint64_t resident = p->long_groups == 2 ? (tile_cols == 128 ? 1 : 2) : 3;
  // Requests' tiles interleaved by their distance from the request's end, so
  // that every request's heaviest tiles are dispatched first (the kernel
  // takes up to 64 requests, whose tile counts one wave holds).  Measured (GQA4
  // 32/8, BF16 / FP8 pages, same box): 3 x 512 rows -8% / -19%, 4 x 512 -3% /
  // -4%, 8 x 256 -3% / -6%, 8 x 1024 -8% / -16%, 4 x 2048 -4% / -7%, 16 x 512
  // 0 / -6%, 2 x 4096 (more than two rounds) 0 / -12%; two requests on a grid
  // of one or two rounds lost (2 x 512 +9% / +4%, 2 x 1024 +2% / +2%), and
  // so did many short requests (32 x 256 +2%, 64 x 128 +5%).
  const uint64_t b = spec->batch_size;
  p->tile_interleave = long_tile && b <= 16 &&
                       (b >= 3 || (b == 2 && grid > 2 * cus * resident));
  p->tile_layer = long_tile && hkv_n > 0 && cus >= hkv_n && grid <= cus * resident
                      ? (uint32_t)(cus / hkv_n) : 0;

  p->info.waves = waves;
  p->info.row_tiles = tiles;
  p->info.block_threads = p->info.waves * 64 * p->long_groups;
  p->info.grid_blocks = grid;
  p->info.flags = opt.flags;
  *out = p;
  return loom::ok(err);
}

loom_status_t loom_prefill_provider_plan_bf16_paged(const loom_prefill_provider_t *provider,
                                                    const loom_paged_prefill_spec_t *spec,
                                                    loom_paged_prefill_plan_t **out,
                                                    loom_error_t *err) {
  return loom_prefill_provider_plan_bf16_paged_options(provider, spec, nullptr, out, err);
}

void loom_paged_prefill_plan_free(loom_paged_prefill_plan_t *p) { delete p; }

void loom_paged_prefill_plan_get_info(const loom_paged_prefill_plan_t *p,
                                      loom_paged_prefill_plan_info_t *info) {
  if (p && info) *info = p->info;
}

// Bf16PagedPrefillPlan::enqueue_into, prefill.rs:2456-2560.
loom_status_t loom_paged_prefill_enqueue(const loom_paged_prefill_plan_t *plan,
                                         loom_command_scope_t *scope,
                                         const loom_paged_prefill_args_t *args,
                                         loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_paged_prefill_spec_t &s = plan->info.spec;
  // FP8 pages are u8 operands plus the [k_scale, v_scale] operand.
  const bool fp8 = s.kv_dtype == LOOM_KV_DTYPE_FP8_E4M3;
  const loom_dtype_t kv_t = fp8 ? LOOM_DTYPE_U8 : LOOM_DTYPE_BF16;
  const loom::OperandSpec ops[10] = {
      {"Q", LOOM_DTYPE_BF16, false},           {"K_pages", kv_t, false},
      {"V_pages", kv_t, false},                {"qo_indptr", LOOM_DTYPE_I32, false},
      {"page_indptr", LOOM_DTYPE_I32, false},  {"page_indices", LOOM_DTYPE_I32, false},
      {"last_page_len", LOOM_DTYPE_I32, false}, {"O", LOOM_DTYPE_BF16, true},
      {"LSE", LOOM_DTYPE_F32, true},           {"kv_scales", LOOM_DTYPE_F32, false}};
  const loom_handle_t hs[10] = {args->query,       args->key_pages,   args->value_pages,
                                args->qo_indptr,   args->page_indptr, args->page_indices,
                                args->last_page_len, args->output,    args->lse,
                                args->kv_scales};
  const loom::Lease *l[10];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, fp8 ? 10 : 9, l, err);
  if (rc) return rc;
  if (fp8 && l[9]->numel != 2)
    return fail(err, LOOM_ENQ_LENGTH_MISMATCH, "kv_scales", 2, l[9]->numel);
  if (fp8 && l[9]->ptr % 4 != 0)
    return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, "kv_scales", (int64_t)l[9]->ptr, 4);
  // prefill.rs:2474-2495: exact spans, page_indices at least B entries.
  const uint64_t qn = s.nnz_qo * s.num_query_heads * loom::kHeadDim;
  const uint64_t page_rows = s.page_size ? s.page_size : loom::kPageSize;
  const uint64_t kvn = s.max_num_pages * page_rows * s.num_kv_heads * loom::kHeadDim;
  const uint64_t want[9] = {qn, kvn, kvn, s.batch_size + 1, s.batch_size + 1, 0,
                            s.batch_size, qn, s.nnz_qo * s.num_query_heads};
  for (int i = 0; i < 9; ++i) {
    if (i == 5) {
      if (l[5]->numel < s.batch_size)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_SHORT, "page_indices", s.batch_size,
                    l[5]->numel);
      continue;
    }
    if (l[i]->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[i].name, want[i], l[i]->numel);
  }
  for (int i : {0, 1, 2, 7})
    if ((rc = require_aligned(ops[i].name, l[i]->ptr, 4, err))) return rc;
  PrefillArgs a{};
  a.kv_scales = fp8 ? (const float *)l[9]->ptr : nullptr;
  a.q = (const uint16_t *)l[0]->ptr;
  a.k = (const uint16_t *)l[1]->ptr;
  a.v = (const uint16_t *)l[2]->ptr;
  a.qo = (const int32_t *)l[3]->ptr;
  a.indptr = (const int32_t *)l[4]->ptr;
  a.indices = (const int32_t *)l[5]->ptr;
  a.last = (const int32_t *)l[6]->ptr;
  a.out = (uint16_t *)l[7]->ptr;
  a.lse = (float *)l[8]->ptr;
  a.batch = (int32_t)s.batch_size;
  a.nnz = (int32_t)s.nnz_qo;
  a.hq = (int32_t)s.num_query_heads;
  a.hkv = (int32_t)s.num_kv_heads;
  a.group = (int32_t)(s.num_query_heads / s.num_kv_heads);
  a.pool = (int64_t)s.max_num_pages;
  a.n_indices = (int64_t)l[5]->numel;
  a.scale_log2 = s.softmax_scale * 1.44269504088896340736f;
  a.indices_capacity = (plan->info.flags & LOOM_PLAN_PAGE_INDICES_CAPACITY) ? 1 : 0;
  const bool hnd = s.kv_layout == LOOM_KV_LAYOUT_HND;
  a.head_elems = hnd ? (int32_t)page_rows * 128 : 128;
  a.row_elems = hnd ? 128 : a.hkv * 128;
  a.page_rows = (int32_t)page_rows;
  a.blocks_lg = page_rows == 64 ? 2 : page_rows == 32 ? 1 : 0;
  a.tile_layer = (int32_t)plan->tile_layer;
  a.tile_interleave = plan->tile_interleave ? 1 : 0;
  hipStream_t stream = scope->queue->stream;
  const dim3 grid((unsigned)plan->info.grid_blocks), block(plan->info.block_threads);
  if (fp8) {
    switch (plan->info.waves) {
      case 4:
        if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->tile_cols == 128 && plan->long_groups == 2)
          hipLaunchKernelGGL((paged_prefill_kernel<8, true, true, 2>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->tile_cols == 128)
          hipLaunchKernelGGL((paged_prefill_kernel<4, true, true, 2>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->long_groups == 2)
          hipLaunchKernelGGL((paged_prefill_kernel<8, true, true, 1>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE)
          hipLaunchKernelGGL((paged_prefill_kernel<4, true, true, 1>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_WIDE_TILE)
          hipLaunchKernelGGL((paged_prefill_kernel<4, true, true>), grid, block, 0, stream, a);
        else
          hipLaunchKernelGGL((paged_prefill_kernel<4, true>), grid, block, 0, stream, a);
        break;
      case 8: hipLaunchKernelGGL((paged_prefill_kernel<8, true>), grid, block, 0, stream, a); break;
      default:
        hipLaunchKernelGGL((paged_prefill_kernel<16, true>), grid, block, 0, stream, a);
        break;
    }
  } else {
    switch (plan->info.waves) {
      case 4:
        if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->tile_cols == 128 && plan->long_groups == 2)
          hipLaunchKernelGGL((paged_prefill_kernel<8, false, true, 2>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->tile_cols == 128)
          hipLaunchKernelGGL((paged_prefill_kernel<4, false, true, 2>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE && plan->long_groups == 2)
          hipLaunchKernelGGL((paged_prefill_kernel<8, false, true, 1>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_LONG_TILE)
          hipLaunchKernelGGL((paged_prefill_kernel<4, false, true, 1>), grid, block, 0, stream, a);
        else if (plan->info.algorithm == LOOM_PAGED_PREFILL_WIDE_TILE)
          hipLaunchKernelGGL((paged_prefill_kernel<4, false, true>), grid, block, 0, stream, a);
        else
          hipLaunchKernelGGL((paged_prefill_kernel<4, false>), grid, block, 0, stream, a);
        break;
      case 8: hipLaunchKernelGGL((paged_prefill_kernel<8, false>), grid, block, 0, stream, a); break;
      default:
        hipLaunchKernelGGL((paged_prefill_kernel<16, false>), grid, block, 0, stream, a);
        break;
    }
  }
  return loom::record_launch(scope, hipGetLastError(), err);
}

// ---- ragged prefill: plan and enqueue ------------------------------------------
loom_status_t loom_prefill_provider_plan_bf16_ragged(
    const loom_prefill_provider_t *provider, const loom_ragged_prefill_spec_t *spec,
    const loom_paged_prefill_plan_options_t *options, loom_ragged_prefill_plan_t **out,
    loom_error_t *err) {
  if (!provider || !spec || !out) return fail(err, LOOM_NULL_ARGUMENT, "provider");
  const loom_paged_prefill_plan_options_t opt =
      options ? *options : loom_paged_prefill_plan_options_t{0, 0};
  if (opt.flags & ~(LOOM_PLAN_PREFILL_TILE_16 | LOOM_PLAN_PREFILL_TILE_64))
    return fail(err, LOOM_PLAN_INVALID_OPTION, "flags", opt.flags);
  if (opt.waves != 0 && opt.waves != 4 && opt.waves != 8 && opt.waves != 16)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "waves", opt.waves);
  const uint32_t waves = opt.waves ? opt.waves : waves_for();
  uint32_t tile_cols = 16;
  bool long_tile = false;
  loom_status_t rc = prefill_tile_cols(opt.flags, waves, spec->batch_size, spec->nnz_qo,
                                       spec->num_query_heads, spec->num_kv_heads, false, false,
                                       &tile_cols, &long_tile, err);
  if (rc) return rc;
  uint64_t tiles = 0, grid = 0;
  rc = prefill_grid(spec->batch_size, spec->nnz_qo, spec->num_query_heads, spec->num_kv_heads,
                    tile_cols, &tiles, &grid, err);
  if (rc) return rc;
  auto *p = new loom_ragged_prefill_plan;
  p->info.spec = *spec;
  p->info.algorithm = tile_cols == 64 ? LOOM_PAGED_PREFILL_WIDE_TILE : LOOM_PAGED_PREFILL_ROW_TILE;
  p->info.waves = waves;
  p->info.row_tiles = tiles;
  p->info.block_threads = p->info.waves * 64;
  p->info.grid_blocks = grid;
  p->info.workspace_numel = 0;
  *out = p;
  return loom::ok(err);
}

void loom_ragged_prefill_plan_free(loom_ragged_prefill_plan_t *p) { delete p; }

void loom_ragged_prefill_plan_get_info(const loom_ragged_prefill_plan_t *p,
                                       loom_ragged_prefill_plan_info_t *info) {
  if (p && info) *info = p->info;
}

uint64_t loom_ragged_prefill_workspace_numel(const loom_ragged_prefill_plan_t *p) {
  return p ? p->info.workspace_numel : 0;
}

// Bf16RaggedPrefillPlan::enqueue_into, prefill.rs:2648-2760 (the one-kernel
// algorithms: the optional workspace operand is not used).
loom_status_t loom_ragged_prefill_enqueue(const loom_ragged_prefill_plan_t *plan,
                                          loom_command_scope_t *scope,
                                          const loom_ragged_prefill_args_t *args,
                                          loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_ragged_prefill_spec_t &s = plan->info.spec;
  static const loom::OperandSpec ops[7] = {
      {"Q", LOOM_DTYPE_BF16, false},         {"K", LOOM_DTYPE_BF16, false},
      {"V", LOOM_DTYPE_BF16, false},         {"qo_indptr", LOOM_DTYPE_I32, false},
      {"kv_indptr", LOOM_DTYPE_I32, false},  {"O", LOOM_DTYPE_BF16, true},
      {"LSE", LOOM_DTYPE_F32, true}};
  const loom_handle_t hs[7] = {args->query,     args->key,    args->value, args->qo_indptr,
                               args->kv_indptr, args->output, args->lse};
  const loom::Lease *l[7];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, 7, l, err);
  if (rc) return rc;
  // prefill.rs:2700-2712: exact spans.
  const uint64_t qn = s.nnz_qo * s.num_query_heads * loom::kHeadDim;
  const uint64_t kvn = s.nnz_kv * s.num_kv_heads * loom::kHeadDim;
  const uint64_t want[7] = {qn, kvn, kvn, s.batch_size + 1, s.batch_size + 1, qn,
                            s.nnz_qo * s.num_query_heads};
  for (int i = 0; i < 7; ++i)
    if (l[i]->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[i].name, want[i], l[i]->numel);
  for (int i : {0, 1, 2, 5})
    if ((rc = require_aligned(ops[i].name, l[i]->ptr, 4, err))) return rc;
  PrefillArgs a{};
  a.q = (const uint16_t *)l[0]->ptr;
  a.k = (const uint16_t *)l[1]->ptr;
  a.v = (const uint16_t *)l[2]->ptr;
  a.qo = (const int32_t *)l[3]->ptr;
  a.indptr = (const int32_t *)l[4]->ptr;
  a.out = (uint16_t *)l[5]->ptr;
  a.lse = (float *)l[6]->ptr;
  a.batch = (int32_t)s.batch_size;
  a.nnz = (int32_t)s.nnz_qo;
  a.nnz_kv = (int32_t)s.nnz_kv;
  a.hq = (int32_t)s.num_query_heads;
  a.hkv = (int32_t)s.num_kv_heads;
  a.group = (int32_t)(s.num_query_heads / s.num_kv_heads);
  a.scale_log2 = s.softmax_scale * 1.44269504088896340736f;
  a.head_elems = 128;  // contiguous K/V: NHD rows
  a.row_elems = a.hkv * 128;
  a.page_rows = 16;
  a.blocks_lg = 0;
  hipStream_t stream = scope->queue->stream;
  const dim3 grid((unsigned)plan->info.grid_blocks), block(plan->info.block_threads);
  switch (plan->info.waves) {
    case 4:
      if (plan->info.algorithm == LOOM_PAGED_PREFILL_WIDE_TILE)
        hipLaunchKernelGGL((ragged_prefill_kernel<4, true>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL(ragged_prefill_kernel<4>, grid, block, 0, stream, a);
      break;
    case 8: hipLaunchKernelGGL(ragged_prefill_kernel<8>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(ragged_prefill_kernel<16>, grid, block, 0, stream, a); break;
  }
  return loom::record_launch(scope, hipGetLastError(), err);
}

}  // extern "C"
