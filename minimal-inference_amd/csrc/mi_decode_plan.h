// The decode work plan: items (contiguous page ranges of one request) and
// the single-workgroup code that cuts a batch into them.  Shared by the
// decode library (decode_plan_kernel, mi_decode.hip) and the page-table step
// that plans the decode it has just laid out in the same launch
// (mi_page_table.hip).
//
// Reference: the decode wrapper's plan() (scheduler.py:402-413, 905-916,
// 927-938).  plan() cuts every request's page list into `nsplit` contiguous
// page ranges ("items") so that items x kv_heads ("units") fill one resident
// round of kUnitsPerCU waves per CU, and copies the first kInlinePages page
// ids of each item into the item, so a wave of the run starts its page loads
// right after reading the item.
#pragma once

#include "mi_common.h"

namespace mi {
namespace dplan {

constexpr int kPageSize = 16;
// Units (waves) per CU in the plan's resident round: 6 measured faster than 8
// (fewer splits, so less partial traffic and shorter merges) and than 4, 5, 7.
#ifndef MI_DECODE_UNITS_PER_CU
#define MI_DECODE_UNITS_PER_CU 6
#endif
constexpr int kUnitsPerCU = MI_DECODE_UNITS_PER_CU;
#ifndef MI_DECODE_MIN_CHUNK
#define MI_DECODE_MIN_CHUNK 4  // pages per item at least (2, 4, 8: 4 measured best on short contexts)
#endif
#ifndef MI_DECODE_MERGE_BUDGET
#define MI_DECODE_MERGE_BUDGET 40  // average splits x group per (request, KV head) the plan aims under
#endif
constexpr int kInlinePages = 24;
// Ints between two per-(request, KV head) merge counters: one 128-byte line
// each, so the units' counting atomics on different counters do not queue on
// one line.
constexpr int kCounterStride = 32;
constexpr int kPlanThreads = 1024;  // both planning kernels run one workgroup of this size

// One item = a contiguous page range of one request.  Read by a wave with one
// 4-byte load per lane (lane l gets word l), so the page ids come first.
struct alignas(128) DecodeItem {
  int pages[kInlinePages];  // kv_indices[page_begin ..] copied by plan(), -1 past the end
  int b;                    // request
  int page_begin;           // absolute position in kv_indices
  int page_end;
  int last_valid;  // valid tokens in the item's final page (0 when empty)
  int split;
  int nsplit;
  int item_base;  // item index of split 0 of this request
  int kv_len;     // the request's tokens (its decode position + 1)
};
static_assert(sizeof(DecodeItem) == 128, "item is read as 32 lanes x 4 bytes");
constexpr int kItemB = kInlinePages, kItemBegin = kInlinePages + 1, kItemEnd = kInlinePages + 2,
              kItemLast = kInlinePages + 3, kItemNsplit = kInlinePages + 5, kItemBase = kInlinePages + 6,
              kItemKvLen = kInlinePages + 7;

// error: 1 = a request's items did not fit the workspace (its rows are not
// computed); 2 = the page-table step that should have laid out the batch
// failed (no items).
struct DecodeHeader {
  int num_units;
  int num_items;
  int chunk_pages;
  int error;
};

struct DecodeLayout {
  size_t items, counters, pml, po, total;
  int max_items;
};

inline DecodeLayout decode_layout(int batch, int hq, int hkv, int head_dim, int max_units) {
  const int group = hq / hkv;
  DecodeLayout L;
  L.max_items = max_units / hkv;
  size_t off = 256;  // header
  L.items = off;
  off = align_up(off + size_t(L.max_items) * sizeof(DecodeItem), 256);
  L.counters = off;
  off = align_up(off + size_t(batch) * hkv * kCounterStride * sizeof(int), 256);
  L.pml = off;
  off = align_up(off + size_t(max_units) * group * 2 * sizeof(float), 256);
  L.po = off;
  off = align_up(off + size_t(max_units) * group * head_dim * sizeof(uint16_t), 256);
  L.total = off;
  return L;
}

// Units the workspace holds when the caller does not fix max_units: all of
// it, capped at 65536 (enough for 8-page items over ~32M tokens x heads).
inline int units_that_fit(size_t bytes, int batch, int hq, int hkv, int head_dim) {
  const int group = hq / hkv;
  const size_t fixed = 256 + 2 * 256 + size_t(batch) * hkv * kCounterStride * sizeof(int);
  if (bytes <= fixed) return 0;
  const size_t per_unit = sizeof(DecodeItem) / size_t(hkv) + 1 + size_t(group) * (2 * sizeof(float) + head_dim * sizeof(uint16_t));
  size_t n = (bytes - fixed) / per_unit;
  n = n > 65536 ? 65536 : n;
  while (n > 0 && decode_layout(batch, hq, hkv, head_dim, int(n)).total > bytes) n -= hkv;
  return int(n);
}

inline int default_max_units(int batch, int hkv) { return 4 * num_cus() * kUnitsPerCU + batch * hkv; }

struct PlanParams {
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_page_len;
  int batch, hkv, target_units, max_items;
  DecodeHeader* header;
  DecodeItem* items;
  int* counters;
};

// Checks the decode shape and the workspace and fills everything of
// PlanParams but the three CSR pointers (mi_decode.hip; `who` prefixes the
// error message).  Returns MI_OK or an MI_ERR_* code with the message set.
int plan_setup(const char* who, void* workspace, size_t workspace_bytes, int batch, int hq, int hkv, int head_dim,
               int page_size, int max_units, PlanParams* pp);

// ------------------------------------------------------------------ device

// Inclusive scan over the block: shuffles inside each wave, then the wave
// totals through LDS (two barriers).  *total receives the block-wide sum.
__device__ inline int block_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = int(blockDim.x >> 6);
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(v, o);
    if (lane >= o) v += y;
  }
  __syncthreads();  // the previous call's readers are done with wsum
  if (lane == 63) wsum[w] = v;
  __syncthreads();
  int pre = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    const int s = wsum[i];
    pre += (i < w) ? s : 0;
    tot += s;
  }
  *total = tot;
  return v + pre;
}

__device__ __forceinline__ int request_pages(const PlanParams& p, int b) {
  return max(0, p.indptr[b + 1] - p.indptr[b]);
}
// Items of a request of np pages at q16 / 16 pages per item (q16 in 1/16
// pages: a fractional item length lets the item count land close to the
// limit, and items then hold floor or ceil of np / nsplit pages).
__device__ __forceinline__ int items_of(int np, int q16) { return max(1, (np * 16 + q16 - 1) / q16); }

// Candidate k (0-based) of a search round over [lo, hi): nw + 1 equal steps
// (32-bit: hi - lo <= 16 x the longest request's pages, under 2^26 here).
__device__ __forceinline__ int candidate(int lo, int hi, int k, int nw) {
  return lo + (k + 1) * (hi - lo) / (nw + 1);
}

// floor(a * b / c) for 0 <= a <= max(1, b), 0 <= b: 32-bit while a * b fits.
__device__ __forceinline__ int mul_div(int a, int b, int c) {
  return (b <= 46340) ? a * b / c : int((long long)a * b / c);
}

// Wave-wide int sum / max, every lane gets the result: DPP inside each row of
// 16 lanes, then the gfx950 permlane16 / permlane32 swaps (no LDS traffic).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int wave_sum_i(int x) {
  x += dpp_i<kDppQuadSwap1>(x);
  x += dpp_i<kDppQuadSwap2>(x);
  x += dpp_i<kDppRowHalfMirror>(x);
  x += dpp_i<kDppRowMirror>(x);
  auto r = __builtin_amdgcn_permlane16_swap(unsigned(x), unsigned(x), false, false);
  x = int(r[0]) + int(r[1]);
  r = __builtin_amdgcn_permlane32_swap(unsigned(x), unsigned(x), false, false);
  return int(r[0]) + int(r[1]);
}
__device__ __forceinline__ int wave_max_i(int x) {
  x = max(x, dpp_i<kDppQuadSwap1>(x));
  x = max(x, dpp_i<kDppQuadSwap2>(x));
  x = max(x, dpp_i<kDppRowHalfMirror>(x));
  x = max(x, dpp_i<kDppRowMirror>(x));
  auto r = __builtin_amdgcn_permlane16_swap(unsigned(x), unsigned(x), false, false);
  x = max(int(r[0]), int(r[1]));
  r = __builtin_amdgcn_permlane32_swap(unsigned(x), unsigned(x), false, false);
  return max(int(r[0]), int(r[1]));
}

// The search's item limit and its starting range [lo, hi] for q16 (see
// plan_q16).
__device__ __forceinline__ void search_range(const PlanParams& p, int max_np, long long total_np, int* limit,
                                             int* lo, int* hi) {
  const int round_items = max(1, p.target_units / p.hkv);
  int lim = ((p.batch + round_items - 1) / round_items) * round_items;
  lim = min(max(lim, 1), p.max_items);
  // q16 = 16 * max_np gives one item per request, which fits (max_items >=
  // batch); every q16 below 16 total / limit has more than `limit` items.
  const int h = 16 * max(max_np, 1);
  // Items of fewer than MI_DECODE_MIN_CHUNK pages only add merge work: the
  // splits of short contexts do not need that much parallelism.
  const int l = min(h, max(16 * MI_DECODE_MIN_CHUNK, int((16 * total_np + lim - 1) / lim)));
  // Each request's items exceed 16 np / q16 by less than one, so the items
  // of all of them stay under 16 total / q16 + batch: any q16 of at least
  // 16 total / (limit - batch) fits, which bounds the search far tighter.
  int u = h;
  if (lim > p.batch) u = min(u, max(l, int((16 * total_np + (lim - p.batch) - 1) / (lim - p.batch))));
  *lo = l;
  *hi = u;
  *limit = lim;
}

// Pages per item, in 1/16 pages ("q16"): the smallest value whose items fit
// the limit (the item count is non-increasing in q16).  The limit is one
// resident round of units (target_units / kv_heads items), so no wave runs a
// second unit -- or whole rounds when the batch alone needs more -- and never
// more items than the workspace holds.  Page counts come from s_np when
// `cached` (batch <= kPlanThreads), else from the CSR in global memory.
__device__ inline int plan_q16(const PlanParams& p, const int* s_np, bool cached, int max_np, long long total_np) {
  __shared__ int ok[2][kPlanThreads / 64], cand[2][kPlanThreads / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = int(blockDim.x >> 6);
  int limit, lo, hi;
  search_range(p, max_np, total_np, &limit, &lo, &hi);
  // Parallel search: each round every wave counts the items of one of nw
  // candidates spread over [lo, hi) (one barrier per round, results double
  // buffered); the range shrinks (nw + 1)-fold per round.  The answer stays
  // in [lo, hi]: a candidate that fits bounds it above, one that does not
  // bounds it below; the largest candidate is below hi and the smallest at or
  // above lo, so every round moves lo up or hi down.
  for (int round = 0; lo < hi; ++round) {
    const int c = candidate(lo, hi, w, nw);
    int cnt = 0;
    for (int b = lane; b < p.batch; b += 64) cnt += items_of(cached ? s_np[b] : request_pages(p, b), c);
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
    if (lane == 0) {
      ok[round & 1][w] = cnt <= limit;
      cand[round & 1][w] = c;
    }
    __syncthreads();
    int nlo = lo, nhi = hi;
    for (int i = 0; i < nw; ++i) {
      const int ci = cand[round & 1][i];
      if (ok[round & 1][i]) nhi = min(nhi, ci); else nlo = max(nlo, ci + 1);
    }
    lo = nlo;
    hi = nhi;
  }
  return lo;
}

// Item `idx` of a chunk of requests starting at request `base`: scan[0..n)
// is the chunk's inclusive scan of items per request (request r of the chunk
// owns items scan[r-1] .. scan[r]-1), `running` the items before the chunk.
__device__ inline void write_item(const PlanParams& p, int idx, const int* scan, int n, int running, int base,
                                  const int* s_np, const int* s_pb0, const int* s_lpl) {
  int lo_r = 0, hi_r = n - 1;  // request r: the first with scan[r] > idx
  while (lo_r < hi_r) {
    const int mid = (lo_r + hi_r) >> 1;
    if (scan[mid] > idx) hi_r = mid; else lo_r = mid + 1;
  }
  const int r = lo_r;
  const int nsr = scan[r] - (r > 0 ? scan[r - 1] : 0);
  const int first = running + scan[r] - nsr;
  if (first + nsr > p.max_items) return;  // the request does not fit: none of its items
  const int sp = idx - (scan[r] - nsr);
  const int npr = s_np[r];
  DecodeItem it;
  it.b = base + r;
  it.page_begin = s_pb0[r] + mul_div(sp, npr, nsr);
  it.page_end = s_pb0[r] + mul_div(sp + 1, npr, nsr);
  it.last_valid = (npr == 0) ? 0 : (sp == nsr - 1 ? s_lpl[r] : kPageSize);
  it.split = sp;
  it.nsplit = nsr;
  it.item_base = first;
  it.kv_len = (npr == 0) ? 0 : (npr - 1) * kPageSize + s_lpl[r];
  // all kInlinePages loads issued together from in-range positions (clamped
  // to the item's last page), the ones past the end dropped after
  if (it.page_end > it.page_begin) {
    const int last = it.page_end - 1;
    int v[kInlinePages];
#pragma unroll
    for (int j = 0; j < kInlinePages; ++j) v[j] = p.indices[min(it.page_begin + j, last)];
#pragma unroll
    for (int j = 0; j < kInlinePages; ++j) it.pages[j] = (it.page_begin + j <= last) ? v[j] : -1;
  } else {
#pragma unroll
    for (int j = 0; j < kInlinePages; ++j) it.pages[j] = -1;
  }
  p.items[first + sp] = it;
}

__device__ inline void write_header(const PlanParams& p, int running, int q16) {
  const int items = min(running, p.max_items);
  p.header->num_items = items;
  p.header->num_units = items * p.hkv;
  p.header->chunk_pages = (q16 + 15) / 16;  // the longest item
  p.header->error = (running > p.max_items) ? 1 : 0;
}

// Writes the items at q16, the zeroed merge counters and the header.  When
// `cached`, s_np / s_pb0 / s_lpl hold every request's page count, first page
// and clamped last-page length; otherwise they are scratch of kPlanThreads
// entries filled here one chunk of requests at a time from the CSR.
__device__ inline void plan_items(const PlanParams& p, int q16, bool cached, int* s_np, int* s_pb0, int* s_lpl) {
  __shared__ int wsum[kPlanThreads / 64];
  __shared__ int scan[kPlanThreads];
  const int t = threadIdx.x;
  // The scan gives each request's first item, then every thread writes whole
  // items (one item per thread per round, its inline page ids loaded
  // together), finding the item's request by binary search over the scan.
  int running = 0;
  for (int base = 0; base < p.batch; base += blockDim.x) {
    const int b = base + t;
    int ns = 0;
    if (b < p.batch) {
      if (!cached) {
        const int pb0 = p.indptr[b], pb1 = p.indptr[b + 1], lpl = p.last_page_len[b];
        s_np[t] = max(0, pb1 - pb0);
        s_pb0[t] = pb0;
        s_lpl[t] = min(max(lpl, 1), kPageSize);
      }
      ns = items_of(s_np[t], q16);
    }
    int chunk_total = 0;
    scan[t] = block_scan(ns, wsum, &chunk_total);
    __syncthreads();  // publishes scan and s_np / s_pb0 / s_lpl
    for (int idx = t; idx < chunk_total; idx += blockDim.x)
      write_item(p, idx, scan, int(blockDim.x), running, base, s_np, s_pb0, s_lpl);
    running += chunk_total;
    __syncthreads();  // the next round rewrites scan and s_*
  }
  for (int i = t; i < p.batch * p.hkv; i += blockDim.x) p.counters[i * kCounterStride] = 0;
  if (t == 0) write_header(p, running, q16);
}

// Batches of at most 64 requests (the engine's decode batches): wave 0 holds
// one request per lane and does the reductions, a binary search for q16
// (wave-wide sums, no barriers) and the scan of items per request; then one
// barrier and every thread writes items.  Same result as plan_q16 +
// plan_items.
__device__ inline void plan_small(const PlanParams& p, const int* s_np, const int* s_pb0, const int* s_lpl) {
  __shared__ int scan[64];
  __shared__ int s_q16;
  const int t = threadIdx.x, lane = t & 63;
  if (t < 64) {
    const int np = lane < p.batch ? s_np[lane] : 0;
    int limit, lo, hi;
    search_range(p, wave_max_i(np), wave_sum_i(np), &limit, &lo, &hi);
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (wave_sum_i(lane < p.batch ? items_of(np, mid) : 0) <= limit) hi = mid; else lo = mid + 1;
    }
    int v = lane < p.batch ? items_of(np, lo) : 0;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(v, o);
      if (lane >= o) v += y;
    }
    scan[lane] = v;
    if (lane == 0) s_q16 = lo;
  }
  __syncthreads();
  const int total = scan[63];
  for (int idx = t; idx < total; idx += blockDim.x) write_item(p, idx, scan, 64, 0, 0, s_np, s_pb0, s_lpl);
  for (int i = t; i < p.batch * p.hkv; i += blockDim.x) p.counters[i * kCounterStride] = 0;
  if (t == 0) write_header(p, total, s_q16);
}

// The plan of a batch whose per-request page count, first page and clamped
// last-page length are in s_np / s_pb0 / s_lpl (batch <= kPlanThreads):
// block-wide max and total, then plan_q16 and plan_items.
__device__ inline void plan_from_lds(const PlanParams& p, int* s_np, int* s_pb0, int* s_lpl) {
  if (p.batch <= 64) {
    __syncthreads();  // s_np / s_pb0 / s_lpl of every request are written
    plan_small(p, s_np, s_pb0, s_lpl);
    return;
  }
  __shared__ int red[2][kPlanThreads / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, nw = int(blockDim.x >> 6);
  int mx = 0, tot = 0;
  if (t < p.batch) mx = tot = s_np[t];
  for (int o = 32; o > 0; o >>= 1) {
    mx = max(mx, __shfl_xor(mx, o));
    tot += __shfl_xor(tot, o);
  }
  if (lane == 0) {
    red[0][w] = mx;
    red[1][w] = tot;
  }
  __syncthreads();
  int max_np = 0;
  long long total_np = 0;
  for (int i = 0; i < nw; ++i) {
    max_np = max(max_np, red[0][i]);
    total_np += red[1][i];
  }
  const int q16 = plan_q16(p, s_np, true, max_np, total_np);
  plan_items(p, q16, true, s_np, s_pb0, s_lpl);
}

}  // namespace dplan
}  // namespace mi
