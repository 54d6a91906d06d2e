// Paged decode attention for gfx950 (MI355X), BF16 NHD D128 page-16 caches.
//
// Semantics: crates/loom-infer/src/attention/paged_decode/mod.rs:287-366 (the
// CPU reference), with the device metadata guards of
// crates/loom-infer-cuda/src/attention/decode.rs:224-248 and :430-478 (an
// invalid request keeps its output sentinels; valid requests complete).
//
// Work decomposition (MI355X-first, not the reference's warp-per-head):
//   * one workgroup (4 wave64) per (KV chunk, kv-head, group tile); a chunk is
//     `chunk_pages` consecutive pages of one request.  The whole GQA group of
//     the kv-head (up to 8 query heads per tile) shares every K/V byte, so K/V
//     is read from HBM once per kv-head instead of once per query head;
//   * chunk slots are flattened over ragged requests with a workgroup-local
//     prefix scan of the page table, so the grid depends only on buffer
//     capacities (graph-replay safe) and every workgroup carries real work;
//   * per page, S = K·Qᵀ runs on MFMA (v_mfma_f32_16x16x32_bf16: 16 tokens x
//     16 query columns x 32 dims, 4 issues for D=128); K rows feed the A
//     operand straight from 16-byte global loads;
//   * online softmax in the log2 domain (v_exp_f32), P·V on the VALU in FP32
//     with 16-byte V row loads (16 lanes cover one 256-byte row);
//   * waves merge through LDS; a request that fits one chunk is finished in
//     place.  Longer requests leave one FP32 state per (chunk, query head) in
//     the workspace [chunk][Hq][130] = (max_log2, normalizer, acc[128]) (the
//     split-K state layout of crates/loom-infer/src/attention/single_decode/
//     mod.rs:10-13) and a second, stream-ordered merge kernel combines them.
//     The kernel boundary makes the states visible across the 8 XCD L2s; an
//     in-kernel last-arriver merge would need an agent-scope release per
//     workgroup, i.e. an L2 write-back, which costs more than the launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "loom_internal.hpp"

using loom::fail;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxChunkPages = 256;  // one page index per thread in the guard
constexpr int kKRowBytes = 256 + 16;
#ifndef LOOM_DECODE_DEPTH
#define LOOM_DECODE_DEPTH 2
#endif
// Waves per SIMD the register allocation must allow (HIP's second launch
// bound); more resident waves hide HBM latency better than deeper per-wave
// prefetch on this kernel.
#ifndef LOOM_DECODE_WAVES_TILE4
#define LOOM_DECODE_WAVES_TILE4 2
#endif
template <int GT>
constexpr int waves_per_eu() {
  return GT <= 2 ? 3 : GT == 4 ? LOOM_DECODE_WAVES_TILE4 : 2;
}
// Pages in flight per wave (register buffers of 32 VGPRs each).
constexpr int kDepth = LOOM_DECODE_DEPTH;
// Normalizer written into the states of a chunk whose pages failed the guard.
constexpr float kPoisonNormalizer = -1.0f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct DecodeArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  const int32_t *indptr;
  const int32_t *indices;
  const int32_t *last;
  uint16_t *out;
  float *lse;
  float *states;  // [max_chunks][hq][130]
  int32_t batch;
  int32_t hq;
  int32_t hkv;
  int32_t group;
  int32_t group_tiles;
  int32_t chunk_pages;
  int64_t pool;
  int64_t n_indices;
  int64_t grid_slots;  // chunk slots covered by the grid
  float scale_log2;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// half::bf16::from_f32 (round to nearest even, quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}

// K/V pages are read exactly once per kv-head: nontemporal loads keep them
// from displacing reusable lines in L2/MALL (measured on MI355X: a plain
// streaming read tops out near 6.2 TB/s, a nontemporal one near 6.9 TB/s).
#ifndef LOOM_DECODE_NT_K
#define LOOM_DECODE_NT_K 1
#endif
#ifndef LOOM_DECODE_NT_V
#define LOOM_DECODE_NT_V 1
#endif
template <bool NT>
__device__ __forceinline__ u32x4 load16_stream(const uint16_t *p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return *reinterpret_cast<const u32x4 *>(p);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int GT>
struct Smem {
  int pages[kMaxChunkPages];
  float p[kWaves][GT][16];
  float alpha[kWaves][GT];
  float wm[kWaves][GT];
  float wl[kWaves][GT];
  float wacc[kWaves][GT][128];
  // Per-wave K tile: 16 token rows of 256 bytes padded to kKRowBytes so the
  // MFMA fragment reads (16 rows, same column) hit 16 distinct bank groups.
  uint8_t ktile[kWaves][16 * kKRowBytes];
  u32x4 qfrag[4][64];  // MFMA B fragments of the query tile, per lane
  int wave_tot[kWaves];
  int req, split, nsplit;
  int req_start, req_end, tail;
  long long prefix;
};

// One page of K and V for one wave, both as whole 256-byte rows: lane
// (col = lane%16, quad = lane/16) holds columns [8*col, 8*col+8) of rows
// 4*quad + j, j = 0..3, so every load instruction covers four full rows.
struct PageRegs {
  u32x4 k[4];
  u32x4 v[4];
};

__device__ __forceinline__ void load_page(PageRegs &r, const DecodeArgs &a, int page, int lane,
                                          int kvh) {
  const int col = lane & 15, quad = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t row = ((int64_t)page * 16 + quad * 4 + j) * a.hkv + kvh;
    r.k[j] = load16_stream<LOOM_DECODE_NT_K>(a.k + row * 128 + col * 8);
    r.v[j] = load16_stream<LOOM_DECODE_NT_V>(a.v + row * 128 + col * 8);
  }
}

template <int GT>
__global__ __launch_bounds__(kThreads, waves_per_eu<GT>()) void paged_decode_split_kv_kernel(
    DecodeArgs a) {
  __shared__ Smem<GT> sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;

  int w = blockIdx.x;
  const int kvh = w % a.hkv;
  w /= a.hkv;
  const int gt = w % a.group_tiles;
  const long long slot = w / a.group_tiles;

  // ---- flattened chunk schedule: prefix scan of chunks per request ---------
  // The global guard words and each thread's (start, end, tail) are loaded in
  // one round trip; the request found by the scan is handed over through LDS.
  const int32_t ip0 = a.indptr[0];
  const int32_t ipB = a.indptr[a.batch];
  if (tid == 0) sm.req = -1;
  long long carry = 0;
  for (int base = 0; base < a.batch; base += kThreads) {
    const int r = base + tid;
    int c = 0, st = 0, en = 0, tl = 0;
    if (r < a.batch) {
      st = a.indptr[r];
      en = a.indptr[r + 1];
      tl = a.last[r];
      const bool valid = st >= 0 && en > st && en <= ipB && tl >= 1 && tl <= 16;
      c = valid ? (en - st + a.chunk_pages - 1) / a.chunk_pages : 0;
    }
    int x = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) sm.wave_tot[wave] = x;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      const int t = sm.wave_tot[i];
      before += (i < wave) ? t : 0;
      tot += t;
    }
    const long long incl = carry + before + x, excl = incl - c;
    if (c > 0 && slot >= excl && slot < incl) {
      sm.req = r;
      sm.split = (int)(slot - excl);
      sm.nsplit = c;
      sm.prefix = excl;
      sm.req_start = st;
      sm.req_end = en;
      sm.tail = tl;
    }
    carry += tot;
    __syncthreads();
  }
  // Global guard (decode.rs:233-246), and more chunks than the grid covers
  // (only possible with overlapping request ranges): the whole batch is
  // rejected, consistently in every workgroup.
  if (ip0 != 0 || ipB < 0 || (int64_t)ipB != a.n_indices || carry > a.grid_slots) return;
  const int r = sm.req;
  if (r < 0) return;
  const int split = sm.split, nsplit = sm.nsplit;
  const long long prefix = sm.prefix;
  const int req_end = sm.req_end;
  const int tail = sm.tail;
  const int p0 = sm.req_start + split * a.chunk_pages;
  const int npages = min(a.chunk_pages, req_end - p0);
  const int g_base = gt * GT;
  const int gcount = min(GT, a.group - g_base);

  // ---- page indices of this chunk, then the Q fragment (both in flight) ----
  int pg = 0;
  if (tid < npages) pg = a.indices[p0 + tid];
  // Q fragment: column `col` is query head g of this tile; MFMA c contracts
  // dims 32c + 8*quad + [0, 8), the slices the K fragments read from LDS.
  // The fragments are identical in every wave; wave 0 parks them in LDS so they
  // do not occupy 16 VGPRs through the page loop.
  const bool col_valid = col < gcount;
  if (wave == 0) {
    const int qh = kvh * a.group + g_base + col;
    const uint16_t *qp = a.q + ((int64_t)r * a.hq + qh) * 128 + quad * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      sm.qfrag[c][lane] = col_valid ? load16(qp + c * 32) : u32x4{0, 0, 0, 0};
  }
  // ---- page validation for this chunk (decode.rs:284-289 guard) -----------
  int bad = 0;
  if (tid < npages) {
    sm.pages[tid] = pg;
    bad = (pg < 0 || (int64_t)pg >= a.pool) ? 1 : 0;
  }
  bad = __syncthreads_or(bad);
  if (bad) {
    // The request keeps its output sentinels: a single-chunk request simply
    // writes nothing; a multi-chunk one marks this chunk's states so the
    // merge kernel skips the whole request.
    if (nsplit > 1 && tid < gcount) {
      const int64_t qh = (int64_t)kvh * a.group + g_base + tid;
      float *st = a.states + ((prefix + split) * a.hq + qh) * (int64_t)loom::kStateWidth;
      st[0] = 0.0f;
      st[1] = kPoisonNormalizer;
    }
    return;
  }

  float m_run = -INFINITY, l_run = 0.0f;
  float acc[GT][8];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;

  auto process = [&](const PageRegs &pr, int page_idx) {
    const bool last_page = (p0 + page_idx == req_end - 1);
    const int valid_tokens = last_page ? tail : 16;
    // K rows -> LDS tile -> MFMA A fragments (lane: token row `col`, dims
    // 32c + 8*quad + [0, 8)).
    uint8_t *kt = sm.ktile[wave];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(kt + (quad * 4 + j) * kKRowBytes + col * 16) = pr.k[j];
    wave_lds_fence();
    u32x4 kf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      kf[c] = *reinterpret_cast<const u32x4 *>(kt + col * kKRowBytes + (c * 4 + quad) * 16);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[c]), as_bf16x8(sm.qfrag[c][lane]),
                                                  s, 0, 0, 0);
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sv[i] = (quad * 4 + i < valid_tokens) ? s[i] * a.scale_log2 : -INFINITY;
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_new);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    if (col < GT) {
      *reinterpret_cast<f32x4 *>(&sm.p[wave][col][quad * 4]) = f32x4{p[0], p[1], p[2], p[3]};
      if (quad == 0) sm.alpha[wave][col] = alpha;
    }
    wave_lds_fence();
    // P·V on lane (col = 8-column slice, quad = rows 4*quad..4*quad+3).  Columns
    // of the tile beyond the group carry finite junk and are never stored.
    f32x4 pp[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float al = sm.alpha[wave][g];
      pp[g] = *reinterpret_cast<const f32x4 *>(&sm.p[wave][g][quad * 4]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= al;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = quad * 4 + j < valid_tokens;
      float vf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wv = ok ? pr.v[j][e] : 0u;
        vf[2 * e] = bf16_lo(wv);
        vf[2 * e + 1] = bf16_hi(wv);
      }
#pragma unroll
      for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pp[g][j], vf[e], acc[g][e]);
    }
    wave_lds_fence();
  };

  // ---- main loop: pages wave, wave+4, ... of this chunk, kDepth-deep --------
  // Every step issues the loads of the page kDepth-1 steps ahead before it
  // consumes the current one.  Loads are unconditional (the index is clamped to
  // the wave's last page) and the buffer rotation is unrolled, so the compiler
  // waits for exactly the oldest page's loads instead of draining the queue.
  const int my_pages = npages > wave ? (npages - wave + kWaves - 1) / kWaves : 0;
  if (my_pages > 0) {
    auto page_of = [&](int it) { return sm.pages[wave + kWaves * min(it, my_pages - 1)]; };
    PageRegs buf[kDepth];
#pragma unroll
    for (int j = 0; j < kDepth - 1; ++j) load_page(buf[j], a, page_of(j), lane, kvh);
    int it = 0;
    while (true) {
#pragma unroll
      for (int s = 0; s < kDepth; ++s) {
        load_page(buf[(s + kDepth - 1) % kDepth], a, page_of(it + kDepth - 1), lane, kvh);
        process(buf[s], wave + kWaves * it);
        if (++it >= my_pages) goto pages_done;
      }
    }
  }
pages_done:

  // ---- wave reduction over the 4 row quads ---------------------------------
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[g][e];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      acc[g][e] = x;
    }
  if (quad == 0) {
    if (col < GT) {
      sm.wm[wave][col] = m_run;
      sm.wl[wave][col] = l_tot;
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.wacc[wave][g][col * 8 + e] = acc[g][e];
  }
  __syncthreads();

  // ---- workgroup merge of the 4 wave states --------------------------------
  const int64_t qh_base = (int64_t)kvh * a.group + g_base;
  float *chunk_states = a.states + ((prefix + split) * a.hq) * (int64_t)loom::kStateWidth;
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
    const int64_t qh = qh_base + g;
    if (nsplit == 1) {
      a.out[((int64_t)r * a.hq + qh) * 128 + d] = f32_to_bf16(O / L);
      if (d == 0) a.lse[(int64_t)r * a.hq + qh] = M + __log2f(L);
    } else {
      float *st = chunk_states + qh * (int64_t)loom::kStateWidth;
      if (d == 0) {
        st[0] = M;
        st[1] = L;
      }
      st[2 + d] = O;
    }
  }
}

// Merges the chunk states of one (request, query head) into O and log2-LSE:
// one workgroup of 128 lanes (one per output column) per state row, for the
// requests that span more than one chunk.  Same request validity and chunk
// schedule as the partial kernel; a poisoned chunk (invalid page) leaves the
// request's sentinels untouched.
__global__ __launch_bounds__(128) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ long long s_wave_sum[2][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = blockIdx.x / a.hq;
  const int qh = blockIdx.x % a.hq;
  const int32_t ip0 = a.indptr[0];
  const int32_t ipB = a.indptr[a.batch];
  if (ip0 != 0 || ipB < 0 || (int64_t)ipB != a.n_indices) return;
  // chunks before r and in total (the partial kernel's prefix scan)
  long long before = 0, total = 0;
  for (int rr = tid; rr < a.batch; rr += 128) {
    const int32_t st = a.indptr[rr], en = a.indptr[rr + 1], tl = a.last[rr];
    const bool valid = st >= 0 && en > st && en <= ipB && tl >= 1 && tl <= 16;
    const long long c = valid ? (en - st + a.chunk_pages - 1) / a.chunk_pages : 0;
    total += c;
    before += rr < r ? c : 0;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    before += __shfl_xor(before, o, 64);
    total += __shfl_xor(total, o, 64);
  }
  if (lane == 0) {
    s_wave_sum[wave][0] = before;
    s_wave_sum[wave][1] = total;
  }
  __syncthreads();
  before = s_wave_sum[0][0] + s_wave_sum[1][0];
  total = s_wave_sum[0][1] + s_wave_sum[1][1];
  if (total > a.grid_slots) return;
  const int32_t st = a.indptr[r], en = a.indptr[r + 1], tl = a.last[r];
  if (!(st >= 0 && en > st && en <= ipB && tl >= 1 && tl <= 16)) return;
  const int nsplit = (en - st + a.chunk_pages - 1) / a.chunk_pages;
  if (nsplit <= 1) return;

  const int64_t stride = (int64_t)a.hq * loom::kStateWidth;
  const float *row = a.states + (before * a.hq + qh) * (int64_t)loom::kStateWidth;
  // Pass 1: the global max and the poison marks, with the splits spread over
  // the 128 lanes (one load round trip for up to 128 splits).
  float mloc = -INFINITY;
  int poisoned = 0;
  for (int sidx = tid; sidx < nsplit; sidx += 128) {
    const float *ss = row + sidx * stride;
    mloc = fmaxf(mloc, ss[0]);
    poisoned |= ss[1] < 0.0f;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
    poisoned |= __shfl_xor(poisoned, o, 64);
  }
  __shared__ float s_m[2];
  __shared__ int s_p[2];
  if (lane == 0) {
    s_m[wave] = mloc;
    s_p[wave] = poisoned;
  }
  __syncthreads();
  if (s_p[0] | s_p[1]) return;
  const float M = fmaxf(s_m[0], s_m[1]);
  // Pass 2: weighted sums; the unroll keeps eight splits' loads in flight.
  float l = 0.f, o = 0.f;
  int sidx = 0;
  for (; sidx + 8 <= nsplit; sidx += 8) {
    float ms[8], ls[8], xs[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float *ss = row + (sidx + u) * stride;
      ms[u] = ss[0];
      ls[u] = ss[1];
      xs[u] = ss[2 + tid];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float f = fast_exp2(ms[u] - M);
      l = fmaf(ls[u], f, l);
      o = fmaf(xs[u], f, o);
    }
  }
  for (; sidx < nsplit; ++sidx) {
    const float *ss = row + sidx * stride;
    const float f = fast_exp2(ss[0] - M);
    l = fmaf(ss[1], f, l);
    o = fmaf(ss[2 + tid], f, o);
  }
  a.out[((int64_t)r * a.hq + qh) * 128 + tid] = f32_to_bf16(o / l);
  if (tid == 0) a.lse[(int64_t)r * a.hq + qh] = M + __log2f(l);
}

}  // namespace

// ---- provider / plan / enqueue -----------------------------------------------
struct loom_decode_provider {
  loom::DeviceInfo dev;
};

struct loom_paged_decode_plan {
  loom_paged_decode_plan_info_t info;
  int device = 0;
};

extern "C" {

loom_status_t loom_decode_provider_load(int device, loom_decode_provider_t **out,
                                        loom_error_t *err) {
  if (!out) return fail(err, LOOM_NULL_ARGUMENT, "out");
  loom::DeviceInfo dev;
  loom_status_t rc = loom::query_device(device, &dev, err);
  if (rc) return rc;
  if (!dev.gfx950) return fail(err, LOOM_PLAN_UNSUPPORTED_DEVICE, nullptr, device);
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
  // of two, at most 8 (P·V accumulators are GT x 8 floats per lane).
  const uint32_t gtile = group <= 1 ? 1u : group <= 2 ? 2u : group <= 4 ? 4u : 8u;
  const uint64_t gtiles = (group + gtile - 1) / gtile;
  const uint64_t max_pages = opt.max_total_pages ? opt.max_total_pages : spec->max_num_pages;
  if (max_pages < B) return fail(err, LOOM_PLAN_INVALID_OPTION, "max_total_pages", max_pages);
  if (max_pages > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "max_total_pages", max_pages);

  // Chunk size: enough (request, kv-head, tile, chunk) workgroups to cover
  // every CU several times at the expected length, and as long a chunk as
  // that allows (fewer states to merge).
  uint32_t chunk = opt.chunk_pages;
  if (chunk == 0) {
    const uint64_t expected = opt.expected_kv_len ? opt.expected_kv_len : 4096;
    const uint64_t pages = (expected + loom::kPageSize - 1) / loom::kPageSize;
    const uint64_t units = B * hkv * gtiles;
    const uint64_t target_wgs = 8ull * (uint64_t)provider->dev.cus;
    const uint64_t splits = std::max<uint64_t>(1, (target_wgs + units - 1) / units);
    uint64_t c = (pages + splits - 1) / splits;
    c = (c + 3) / 4 * 4;
    chunk = (uint32_t)std::min<uint64_t>(kMaxChunkPages, std::max<uint64_t>(4, c));
  }
  if (chunk < 4 || chunk > (uint32_t)kMaxChunkPages || chunk % 4 != 0)
    return fail(err, LOOM_PLAN_INVALID_OPTION, "chunk_pages", chunk);

  const uint64_t max_chunks = (max_pages + chunk - 1) / chunk + B;
  const uint64_t grid = max_chunks * hkv * gtiles;
  if (grid > (uint64_t)INT32_MAX || B * hq > (uint64_t)INT32_MAX)
    return fail(err, LOOM_PLAN_STATE_COUNT_OUT_OF_RANGE, "paged batch-decode", grid);
  const uint64_t state_bytes = max_chunks * hq * loom::kStateWidth * 4;

  auto *p = new loom_paged_decode_plan;
  p->device = provider->dev.device;
  loom_paged_decode_plan_info_t &i = p->info;
  i.spec = *spec;
  i.algorithm = LOOM_PAGED_DECODE_SPLIT_KV_GROUP;
  i.chunk_pages = chunk;
  i.group_tile = gtile;
  i.group_tiles = (uint32_t)gtiles;
  i.max_total_pages = max_pages;
  i.max_chunks = max_chunks;
  i.workspace_bytes = state_bytes;
  i.block_threads = kThreads;
  i.device_cus = (uint32_t)provider->dev.cus;
  *out = p;
  return loom::ok(err);
}

void loom_paged_decode_plan_free(loom_paged_decode_plan_t *p) { delete p; }

void loom_paged_decode_plan_get_info(const loom_paged_decode_plan_t *p,
                                     loom_paged_decode_plan_info_t *info) {
  if (p && info) *info = p->info;
}

loom_status_t loom_paged_decode_enqueue(const loom_paged_decode_plan_t *plan,
                                        loom_command_scope_t *scope,
                                        const loom_paged_decode_args_t *args,
                                        loom_error_t *err) {
  if (!plan || !scope || !args) return fail(err, LOOM_NULL_ARGUMENT, "plan");
  const loom_paged_decode_plan_info_t &pi = plan->info;
  const loom_paged_decode_spec_t &s = pi.spec;
  static const loom::OperandSpec ops[9] = {
      {"Q", LOOM_DTYPE_BF16, false},           {"K_pages", LOOM_DTYPE_BF16, false},
      {"V_pages", LOOM_DTYPE_BF16, false},     {"page_indptr", LOOM_DTYPE_I32, false},
      {"page_indices", LOOM_DTYPE_I32, false}, {"last_page_len", LOOM_DTYPE_I32, false},
      {"O", LOOM_DTYPE_BF16, true},            {"LSE", LOOM_DTYPE_F32, true},
      {"workspace", LOOM_DTYPE_U8, true}};
  const loom_handle_t hs[9] = {args->query,       args->key_pages,     args->value_pages,
                               args->page_indptr, args->page_indices,  args->last_page_len,
                               args->output,      args->lse,           args->workspace};
  const loom::Lease *l[9];
  loom_status_t rc = loom::resolve_command(scope, hs, ops, 9, l, err);
  if (rc) return rc;
  // decode.rs:1216-1242: exact lengths before submission.
  const uint64_t qn = s.batch_size * s.num_query_heads * loom::kHeadDim;
  const uint64_t kvn = s.max_num_pages * loom::kPageSize * s.num_kv_heads * loom::kHeadDim;
  const uint64_t want[9] = {qn, kvn, kvn, s.batch_size + 1, 0, s.batch_size, qn,
                            s.batch_size * s.num_query_heads, pi.workspace_bytes};
  for (int i = 0; i < 9; ++i) {
    if (i == 4) {
      if (l[4]->numel < s.batch_size)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_SHORT, nullptr, s.batch_size, l[4]->numel);
      if (l[4]->numel > pi.max_total_pages)
        return fail(err, LOOM_ENQ_PAGE_INDICES_TOO_LONG, nullptr, pi.max_total_pages,
                    l[4]->numel);
      continue;
    }
    if (l[i]->numel != want[i])
      return fail(err, LOOM_ENQ_LENGTH_MISMATCH, ops[i].name, want[i], l[i]->numel);
  }
  // 16-byte vector loads and stores (decode.rs:1243-1251 checks 4 bytes for its
  // packed pairs; this kernel moves 16 bytes per lane).
  const int align_ops[5] = {0, 1, 2, 6, 8};
  for (int i : align_ops)
    if (l[i]->ptr % 16 != 0)
      return fail(err, LOOM_ENQ_MISALIGNED_BUFFER, ops[i].name, (int64_t)l[i]->ptr, 16);

  DecodeArgs a;
  a.q = (const uint16_t *)l[0]->ptr;
  a.k = (const uint16_t *)l[1]->ptr;
  a.v = (const uint16_t *)l[2]->ptr;
  a.indptr = (const int32_t *)l[3]->ptr;
  a.indices = (const int32_t *)l[4]->ptr;
  a.last = (const int32_t *)l[5]->ptr;
  a.out = (uint16_t *)l[6]->ptr;
  a.lse = (float *)l[7]->ptr;
  a.states = (float *)l[8]->ptr;
  a.batch = (int32_t)s.batch_size;
  a.hq = (int32_t)s.num_query_heads;
  a.hkv = (int32_t)s.num_kv_heads;
  a.group = (int32_t)(s.num_query_heads / s.num_kv_heads);
  a.group_tiles = (int32_t)pi.group_tiles;
  a.chunk_pages = (int32_t)pi.chunk_pages;
  a.pool = (int64_t)s.max_num_pages;
  a.n_indices = (int64_t)l[4]->numel;
  a.grid_slots = (int64_t)((l[4]->numel + pi.chunk_pages - 1) / pi.chunk_pages + s.batch_size);
  a.scale_log2 = s.softmax_scale * 1.44269504088896340736f;

  const uint64_t grid = (uint64_t)a.grid_slots * s.num_kv_heads * pi.group_tiles;
  hipStream_t stream = scope->queue->stream;
  const dim3 g3((unsigned)grid), b3(kThreads);
  switch (pi.group_tile) {
    case 1: hipLaunchKernelGGL(paged_decode_split_kv_kernel<1>, g3, b3, 0, stream, a); break;
    case 2: hipLaunchKernelGGL(paged_decode_split_kv_kernel<2>, g3, b3, 0, stream, a); break;
    case 4: hipLaunchKernelGGL(paged_decode_split_kv_kernel<4>, g3, b3, 0, stream, a); break;
    default: hipLaunchKernelGGL(paged_decode_split_kv_kernel<8>, g3, b3, 0, stream, a); break;
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    // One command: the split kernel, then the merge of multi-chunk requests.
    hipLaunchKernelGGL(paged_decode_merge_kernel, dim3((unsigned)(s.batch_size * s.num_query_heads)),
                       dim3(128), 0, stream, a);
    e = hipGetLastError();
  }
  return loom::record_launch(scope, e, err);
}

}  // extern "C"
