// Device page table: FIFO free-page ring, per-slot page lists, CSR build.
//
// Reference semantics being moved onto the GPU:
//   PagedKVCache free list   scheduler.py:205-221 (deque; popleft / append)
//   allocation call order    scheduler.py:596-600 (admit -> prefill ->
//                            decode -> retire), admission 624-637, decode
//                            growth 843-847, release at retire 984-1003
//   build_csr_metadata       scheduler.py:267-302
//   decode metadata/padding  scheduler.py:862-901
//
// The ring and the page lists never leave the device.  The host keeps only
// counts (free pages, pages per slot), which follow deterministically from
// the request lengths, so admission decisions need no device read.  One step
// is one single-workgroup launch; pops and pushes are parallel but use
// exclusive-scan offsets so the page order is exactly the sequential deque
// order.  Released pages are zeroed across all layers by mi_pages_zero.
#include "mi_common.h"
#include "mi_decode_plan.h"

namespace {

constexpr int kHeaderWords = 16;  // head, free, error, capacity, ...
// The error word's bits: 1 release, 2 admission, 4 growth, 8 indices
// capacity, 16 malformed ops (the step); the fused decode plan's error
// (1 items did not fit, 2 no complete CSR to plan) shifted by this.
constexpr int kPlanErrorShift = 8;
constexpr int kThreads = 1024;

struct Layout {
  size_t ring, slot_np, slot_pages, total;  // word offsets / bytes
};

Layout layout(int num_pages, int max_slots, int mpps) {
  Layout L;
  const size_t cap = size_t(num_pages > 0 ? num_pages - 1 : 0);
  L.ring = kHeaderWords;
  L.slot_np = L.ring + mi::align_up(cap, 4);
  L.slot_pages = L.slot_np + mi::align_up(size_t(max_slots), 4);
  L.total = (L.slot_pages + size_t(max_slots) * mpps) * sizeof(int32_t);
  return L;
}

__global__ void init_kernel(int32_t* st, int cap, int max_slots, size_t ring, size_t slot_np) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int stride = gridDim.x * blockDim.x;
  for (int i = t; i < cap; i += stride) st[ring + i] = i;
  for (int i = t; i < max_slots; i += stride) st[slot_np + i] = 0;
  if (t == 0) {
    st[0] = 0;    // head
    st[1] = cap;  // free
    st[2] = 0;    // error
    st[3] = cap;
  }
}

struct StepParams {
  int32_t* st;
  int cap, max_slots, mpps, page_size;
  size_t ring, slot_np, slot_pages;
  const int32_t* ops;
  int ops_len;
  int32_t *indptr, *indices, *last_page_len, *batch_indices, *positions, *released;
  int64_t capacity;
};

// Inclusive scans of two values over the block and the OR of a flag:
// shuffles inside each wave, then the wave totals through LDS (two
// barriers).  wsum holds 3 x (kThreads / 64) ints.
__device__ void scan2_incl(int& a, int& b, int flag, int* wsum, int* tot_a, int* tot_b, int* any_flag) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  constexpr int nw = kThreads / 64;
  for (int o = 1; o < 64; o <<= 1) {
    const int ya = __shfl_up(a, o), yb = __shfl_up(b, o);
    if (lane >= o) {
      a += ya;
      b += yb;
    }
  }
  const bool wave_flag = __ballot(flag) != 0;
  __syncthreads();  // the previous scan's readers are done with wsum
  if (lane == 63) {
    wsum[w] = a;
    wsum[nw + w] = b;
    wsum[2 * nw + w] = wave_flag;
  }
  __syncthreads();
  int pa = 0, pb = 0, ta = 0, tb = 0, f = 0;
  for (int i = 0; i < nw; ++i) {
    const int sa = wsum[i], sb = wsum[nw + i];
    if (i < w) {
      pa += sa;
      pb += sb;
    }
    ta += sa;
    tb += sb;
    f |= wsum[2 * nw + i];
  }
  a += pa;
  b += pb;
  *tot_a = ta;
  *tot_b = tb;
  *any_flag = f;
}

// One page-table step (release, admit, decode growth, CSR of the padded
// decode rows) by one workgroup of kThreads.  When row_np is given, thread t
// also leaves row t's page count, first page and last-page length there
// (LDS) for a plan in the same launch, and when row_idx is given and the CSR
// holds at most row_idx_cap page ids, a copy of them there too.  Returns 0
// when the CSR is complete,
// 1 when the ops are malformed (nothing done), 2 when the CSR was cut at the
// indices capacity; the value is the same in every thread.
__device__ int step_body(const StepParams& p, int* row_np, int* row_pb0, int* row_lpl, int* row_idx,
                         int row_idx_cap) {
  __shared__ int buf[3 * (kThreads / 64)];
  __shared__ int s_indptr[kThreads + 1];
  __shared__ int s_slot[kThreads];  // decode row -> slot
  __shared__ int head, freec, err, rel_off, total;
  const int t = threadIdx.x;
  int32_t* ring = p.st + p.ring;
  int32_t* slot_np = p.st + p.slot_np;
  int32_t* slot_pages = p.st + p.slot_pages;

  if (t == 0) {
    head = p.st[0];
    freec = p.st[1];
    err = p.st[2];
    rel_off = 0;
  }
  const int n_rel = p.ops_len >= 4 ? p.ops[0] : 0;
  const int n_adm = p.ops_len >= 4 ? p.ops[1] : 0;
  const int n_dec = p.ops_len >= 4 ? p.ops[2] : 0;
  const int padded = p.ops_len >= 4 ? p.ops[3] : 0;
  const int32_t* rel_slots = p.ops + 4;
  const int32_t* adm_slots = rel_slots + n_rel;
  const int32_t* adm_np = adm_slots + n_adm;
  const int32_t* dec_slots = adm_np + n_adm;
  const int32_t* dec_pos = dec_slots + n_dec;
  const bool ops_ok = p.ops_len >= 4 && n_rel >= 0 && n_adm >= 0 && n_dec >= 0 && padded >= n_dec &&
                      padded <= kThreads && 4 + n_rel + 2 * n_adm + 2 * n_dec <= p.ops_len;
  __syncthreads();
  if (!ops_ok) {
    if (t == 0) p.st[2] = err | 16;
    return 1;
  }

  // 1. release, in order: pages go to the ring tail
  for (int k = 0; k < n_rel; ++k) {
    const int s = rel_slots[k];
    const bool ok = s >= 0 && s < p.max_slots;
    const int np = ok ? slot_np[s] : 0;
    const int tail = (head + freec) % max(p.cap, 1);
    for (int j = t; j < np; j += kThreads) {
      const int pg = slot_pages[size_t(s) * p.mpps + j];
      ring[(tail + j) % p.cap] = pg;
      if (p.released) p.released[rel_off + j] = pg;
    }
    __syncthreads();
    if (t == 0) {
      if (!ok) err |= 1;
      if (freec + np > p.cap) err |= 1;
      freec += np;
      rel_off += np;
      if (ok) slot_np[s] = 0;
    }
    __syncthreads();
  }

  // 2. admit, in order: pop from the ring head
  for (int k = 0; k < n_adm; ++k) {
    const int s = adm_slots[k];
    const int n = adm_np[k];
    const int cur = (s >= 0 && s < p.max_slots) ? slot_np[s] : 0;
    const bool ok = s >= 0 && s < p.max_slots && n >= 0 && n <= freec && cur + n <= p.mpps;
    if (ok)
      for (int j = t; j < n; j += kThreads) slot_pages[size_t(s) * p.mpps + cur + j] = ring[(head + j) % p.cap];
    __syncthreads();
    if (t == 0) {
      if (ok) {
        head = (head + n) % max(p.cap, 1);
        freec -= n;
        slot_np[s] = cur + n;
      } else {
        err |= 2;
      }
    }
    __syncthreads();
  }

  // 3 + 4. Decode growth, rows in order, to ceil((pos + 1) / page_size)
  // pages, and the CSR of the padded rows (rows >= n_dec own only the
  // scratch page).  One scan carries each row's growth and its page count
  // after growth; when the growth cannot be served the decode rows get no
  // pages and the CSR holds the padding rows alone (a closed form).
  const int h0 = head, f0 = freec;
  int s_row = -1, np_row = 0, need = 0, pos_row = 0;
  if (t < n_dec) {
    s_row = dec_slots[t];
    pos_row = dec_pos[t];
    s_slot[t] = s_row;
    if (s_row >= 0 && s_row < p.max_slots && pos_row >= 0) {
      np_row = slot_np[s_row];
      need = max(0, (pos_row + 1 + p.page_size - 1) / p.page_size - np_row);
      if (np_row + need > p.mpps) need = -1;
    } else {
      need = -1;
    }
  }
  const int bad = need < 0 ? 1 : 0;
  if (need < 0) need = 0;
  int need_incl = need;
  int rows_incl = (t < padded) ? ((t < n_dec) ? np_row + need : 1) : 0;
  int need_total, rows_total, any_bad;
  scan2_incl(need_incl, rows_incl, bad, buf, &need_total, &rows_total, &any_bad);
  const bool grow_ok = !any_bad && need_total <= f0;
  if (grow_ok && t < n_dec) {
    const int first = need_incl - need;
    for (int j = 0; j < need; ++j)
      slot_pages[size_t(s_row) * p.mpps + np_row + j] = ring[(h0 + first + j) % p.cap];
    np_row += need;
    slot_np[s_row] = np_row;
  }
  const int new_head = grow_ok ? (h0 + need_total) % max(p.cap, 1) : h0;
  const int new_free = grow_ok ? f0 - need_total : f0;
  const int rows_np = (t < padded) ? ((t < n_dec) ? (grow_ok ? np_row : 0) : 1) : 0;
  const int ip = grow_ok ? rows_incl : (t < padded ? max(0, t - n_dec + 1) : 0);
  const int tot_pages = grow_ok ? rows_total : padded - n_dec;
  if (t < padded) s_indptr[t + 1] = ip;
  if (t == 0) s_indptr[0] = 0;
  __syncthreads();  // s_indptr and the grown page lists are visible to every thread
  // padded + 1 entries: with padded == kThreads the last one has no thread of its own
  for (int i = t; i <= padded; i += kThreads) p.indptr[i] = s_indptr[i];
  if (t < padded) {
    int last = 1;
    if (t < n_dec) {
      const int seq = pos_row + 1;
      last = seq % p.page_size;
      if (last == 0 && seq > 0) last = p.page_size;
      p.positions[t] = pos_row;
    } else {
      p.positions[t] = 0;
    }
    p.last_page_len[t] = last;
    p.batch_indices[t] = t;
    if (row_np) {
      row_np[t] = rows_np;
      row_pb0[t] = ip - rows_np;
      row_lpl[t] = min(max(last, 1), mi::dplan::kPageSize);
    }
  }
  const int lim = int(min<int64_t>(tot_pages, p.capacity));
  const bool copy_idx = row_idx != nullptr && lim <= row_idx_cap;
  for (int idx = t; idx < lim; idx += kThreads) {
    int lo = 0, hi = padded;  // find row r with s_indptr[r] <= idx < s_indptr[r+1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_indptr[mid] <= idx) lo = mid; else hi = mid;
    }
    const int r = lo;
    const int j = idx - s_indptr[r];
    int pg = p.cap;  // scratch page id == num_pages - 1 == cap
    if (r < n_dec) pg = slot_pages[size_t(s_slot[r]) * p.mpps + j];
    p.indices[idx] = pg;
    if (copy_idx) row_idx[idx] = pg;
  }
  __syncthreads();
  if (t == 0) {
    p.st[0] = new_head;
    p.st[1] = new_free;
    p.st[2] = err | ((!grow_ok && n_dec > 0) ? 4 : 0) | (tot_pages > p.capacity ? 8 : 0);
  }
  return tot_pages > p.capacity ? 2 : 0;
}

__global__ __launch_bounds__(kThreads) void step_kernel(StepParams p) {
  step_body(p, nullptr, nullptr, nullptr, nullptr, 0);
}

// Page ids the fused kernel keeps on chip for the plan's items (32 KB).
constexpr int kLdsPageIds = 8192;

// The step, then the decode plan of its padded rows in the same workgroup:
// the plan takes each row's page count, first page and last-page length from
// LDS and the page ids from the indices the step has just written (visible to
// the workgroup after the step's barriers).  If the step did not lay out a
// complete CSR of exactly pp.batch rows, the plan is empty with error 2.
__global__ __launch_bounds__(kThreads) void step_plan_kernel(StepParams p, mi::dplan::PlanParams pp) {
  __shared__ int s_np[kThreads], s_pb0[kThreads], s_lpl[kThreads];
  __shared__ int s_idx[kLdsPageIds];
  const int status = step_body(p, s_np, s_pb0, s_lpl, s_idx, kLdsPageIds);
  const int padded = p.ops_len >= 4 ? p.ops[3] : -1;
  if (status != 0 || padded != pp.batch) {
    if (threadIdx.x == 0) {
      pp.header->num_units = 0;
      pp.header->num_items = 0;
      pp.header->chunk_pages = 0;
      pp.header->error = 2;
      p.st[2] |= 2 << kPlanErrorShift;  // sticky, beside the step's own bits
    }
    return;
  }
  // the items read their page ids from the on-chip copy when the CSR fit it
  if (pp.batch > 0 && s_pb0[pp.batch - 1] + s_np[pp.batch - 1] <= kLdsPageIds) pp.indices = s_idx;
  mi::dplan::plan_from_lds(pp, s_np, s_pb0, s_lpl);
  // thread 0 wrote the plan's header: its error, if any, joins the sticky
  // word, so every step's plan of a decode window is checked at its read-back
  if (threadIdx.x == 0) {
    const int perr = pp.header->error;
    if (perr) p.st[2] |= perr << kPlanErrorShift;
  }
}

__global__ void zero_kernel(uint4* pools, int64_t layer_stride16, int layers, int64_t page16,
                            const int32_t* ids, int n_pages, int64_t num_pages) {
  const int64_t per_layer = int64_t(n_pages) * page16;
  const int64_t total = per_layer * layers;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t l = i / per_layer;
    const int64_t r = i - l * per_layer;
    const int64_t k = r / page16;
    const int64_t c = r - k * page16;
    const int64_t pg = ids[k];
    if (pg < 0 || pg >= num_pages) continue;
    pools[l * layer_stride16 + pg * page16 + c] = make_uint4(0, 0, 0, 0);
  }
}

}  // namespace

extern "C" size_t mi_page_table_state_size(int32_t num_pages, int32_t max_slots, int32_t max_pages_per_slot) {
  if (num_pages < 2 || max_slots <= 0 || max_pages_per_slot <= 0) return 0;
  return layout(num_pages, max_slots, max_pages_per_slot).total;
}

extern "C" size_t mi_page_table_error_offset(int32_t, int32_t, int32_t) { return 2 * sizeof(int32_t); }

extern "C" int mi_page_table_init(void* state, int32_t num_pages, int32_t max_slots,
                                  int32_t max_pages_per_slot, mi_stream_t stream) {
  mi::clear_error();
  if (!state || num_pages < 2 || max_slots <= 0 || max_pages_per_slot <= 0)
    return mi::fail(MI_ERR_INVALID, "page table init: bad arguments");
  const Layout L = layout(num_pages, max_slots, max_pages_per_slot);
  hipLaunchKernelGGL(init_kernel, dim3(64), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<int32_t*>(state), num_pages - 1, max_slots, L.ring, L.slot_np);
  return mi::check_launch("page_table init_kernel");
}

namespace {

int make_step_params(const char* who, void* state, int32_t num_pages, int32_t max_slots, int32_t max_pages_per_slot,
                     const int32_t* ops, int32_t ops_len, int32_t page_size, int32_t* indptr, int32_t* indices,
                     int64_t indices_capacity, int32_t* last_page_len, int32_t* batch_indices, int32_t* positions,
                     int32_t* released_pages, StepParams* sp) {
  if (!state || !ops || ops_len < 4 || num_pages < 2 || max_slots <= 0 || max_pages_per_slot <= 0 ||
      page_size <= 0)
    return mi::fail(MI_ERR_INVALID, "%s: bad arguments", who);
  if (!indptr || !indices || !last_page_len || !batch_indices || !positions)
    return mi::fail(MI_ERR_INVALID, "%s: null output", who);
  const Layout L = layout(num_pages, max_slots, max_pages_per_slot);
  sp->st = static_cast<int32_t*>(state);
  sp->cap = num_pages - 1;
  sp->max_slots = max_slots;
  sp->mpps = max_pages_per_slot;
  sp->page_size = page_size;
  sp->ring = L.ring;
  sp->slot_np = L.slot_np;
  sp->slot_pages = L.slot_pages;
  sp->ops = ops;
  sp->ops_len = ops_len;
  sp->indptr = indptr;
  sp->indices = indices;
  sp->last_page_len = last_page_len;
  sp->batch_indices = batch_indices;
  sp->positions = positions;
  sp->released = released_pages;
  sp->capacity = indices_capacity;
  return MI_OK;
}

}  // namespace

extern "C" int mi_page_table_step(void* state, int32_t num_pages, int32_t max_slots,
                                  int32_t max_pages_per_slot, const int32_t* ops, int32_t ops_len,
                                  int32_t page_size, int32_t* indptr, int32_t* indices,
                                  int64_t indices_capacity, int32_t* last_page_len,
                                  int32_t* batch_indices, int32_t* positions, int32_t* released_pages,
                                  mi_stream_t stream) {
  mi::clear_error();
  StepParams sp;
  const int rc = make_step_params("page table step", state, num_pages, max_slots, max_pages_per_slot, ops, ops_len,
                                  page_size, indptr, indices, indices_capacity, last_page_len, batch_indices,
                                  positions, released_pages, &sp);
  if (rc) return rc;
  hipLaunchKernelGGL(step_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), sp);
  return mi::check_launch("page_table step_kernel");
}

extern "C" int mi_page_table_step_decode_plan(void* state, int32_t num_pages, int32_t max_slots,
                                              int32_t max_pages_per_slot, const int32_t* ops, int32_t ops_len,
                                              int32_t page_size, int32_t* indptr, int32_t* indices,
                                              int64_t indices_capacity, int32_t* last_page_len,
                                              int32_t* batch_indices, int32_t* positions, int32_t* released_pages,
                                              int32_t batch_size, void* decode_workspace,
                                              size_t decode_workspace_bytes, int32_t num_qo_heads,
                                              int32_t num_kv_heads, int32_t head_dim, mi_stream_t stream) {
  mi::clear_error();
  StepParams sp;
  int rc = make_step_params("page table step + decode plan", state, num_pages, max_slots, max_pages_per_slot, ops,
                            ops_len, page_size, indptr, indices, indices_capacity, last_page_len, batch_indices,
                            positions, released_pages, &sp);
  if (rc) return rc;
  if (batch_size < 0 || batch_size > kThreads)
    return mi::fail(MI_ERR_INVALID, "page table step + decode plan: batch %d (1..%d padded rows)", batch_size,
                    kThreads);
  mi::dplan::PlanParams pp;
  rc = mi::dplan::plan_setup("page table step + decode plan", decode_workspace, decode_workspace_bytes, batch_size,
                             num_qo_heads, num_kv_heads, head_dim, page_size, 0, &pp);
  if (rc) return rc;
  pp.indptr = indptr;
  pp.indices = indices;
  pp.last_page_len = last_page_len;
  hipLaunchKernelGGL(step_plan_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), sp, pp);
  return mi::check_launch("page_table step_plan_kernel");
}

extern "C" int mi_pages_zero(void* pools, int64_t layer_stride_bytes, int32_t num_layers, int64_t num_pages,
                             int64_t page_bytes, const int32_t* page_ids, int32_t n_pages, mi_stream_t stream) {
  mi::clear_error();
  if (n_pages == 0 || num_layers == 0) return MI_OK;
  if (!pools || !page_ids || n_pages < 0 || num_layers < 0 || page_bytes <= 0 || page_bytes % 16 ||
      layer_stride_bytes % 16 || (reinterpret_cast<uintptr_t>(pools) & 15))
    return mi::fail(MI_ERR_INVALID, "pages zero: bad arguments (16-byte granularity required)");
  const int64_t work = int64_t(n_pages) * num_layers * (page_bytes / 16);
  int64_t blocks = (work + 255) / 256;
  const int64_t cap = int64_t(mi::num_cus()) * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(zero_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint4*>(pools), layer_stride_bytes / 16, num_layers, page_bytes / 16, page_ids,
                     n_pages, num_pages);
  return mi::check_launch("pages zero_kernel");
}
