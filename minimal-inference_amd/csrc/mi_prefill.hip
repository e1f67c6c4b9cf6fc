// Ragged (varlen) causal prefill attention over the paged pool, bf16 MFMA.
//
// Reference: the prefill wrapper's plan() (scheduler.py:704-716: qo_indptr,
// paged_kv_indptr / indices / last_page_len, causal=True) and run()
// (model.py:235, mode == "prefill").  Query row i of request b sees KV tokens
// j <= i + (kv_len - qo_len); the reference always has kv_len == qo_len.
//
// plan() (one workgroup) lists 64-row query tiles of every request, the
// heaviest (last) tile of a request first.  run() launches (tiles, q_heads)
// workgroups of four waves; wave w owns query rows 16w..16w+15 of the tile.
// Per 32-token KV tile:
//   S^T = K Q^T  -- 16x16x32 MFMAs; K rows come straight from the pool with
//                   16-byte loads, Q^T is held in registers;
//   online softmax per query row in the exp2 domain;
//   O += P V     -- the S^T accumulator layout is reused as the P operand
//                   (each lane already holds 8 keys of one query row); V is
//                   staged transposed in LDS by the workgroup so every lane
//                   reads its 8 keys of one head_dim column as two 8-byte
//                   LDS reads.
// Waves whose rows are causally finished skip the MFMAs of a tile but keep
// the workgroup barriers.
#include <math.h>

#include "mi_common.h"

namespace {

constexpr int kPageSize = 16;
constexpr int kTileRows = 64;
constexpr int kKvTile = 32;

struct alignas(32) PrefillTile {
  int b;
  int q_begin;  // absolute first query row of the tile
  int q_rows;   // rows in this tile (<= 64)
  int qo_len;
  int kv_len;
  int row0;           // first row of the tile within its request
  int kv_page_begin;  // absolute position of the request's first page in kv_indices
  int pad;
};

struct PrefillHeader {
  int num_tiles;
  int error;
};

size_t tile_capacity(int batch, int64_t total_q) { return size_t(total_q / kTileRows + batch + 1); }

size_t prefill_ws_bytes(int batch, int64_t total_q) {
  return 256 + mi::align_up(tile_capacity(batch, total_q) * sizeof(PrefillTile), 256);
}

struct PlanParams {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int batch;
  int capacity;
  PrefillHeader* header;
  PrefillTile* tiles;
};

__global__ __launch_bounds__(1024) void prefill_plan_kernel(PlanParams p) {
  __shared__ int buf[1024];
  __shared__ int total_sh;
  const int t = threadIdx.x;
  int running = 0;
  for (int base = 0; base < p.batch; base += blockDim.x) {
    const int b = base + t;
    int nt = 0, qo = 0, kv = 0, np = 0;
    if (b < p.batch) {
      qo = max(0, p.qo_indptr[b + 1] - p.qo_indptr[b]);
      np = max(0, p.kv_indptr[b + 1] - p.kv_indptr[b]);
      kv = np > 0 ? (np - 1) * kPageSize + min(max(p.last_page_len[b], 1), kPageSize) : 0;
      nt = (qo + kTileRows - 1) / kTileRows;
    }
    buf[t] = nt;
    __syncthreads();
    for (int o = 1; o < int(blockDim.x); o <<= 1) {
      const int add = (t >= o) ? buf[t - o] : 0;
      __syncthreads();
      buf[t] += add;
      __syncthreads();
    }
    const int first = running + buf[t] - nt;
    if (t == 0) total_sh = buf[blockDim.x - 1];
    __syncthreads();
    for (int k = 0; k < nt; ++k) {
      const int idx = first + k;
      if (idx >= p.capacity) break;
      PrefillTile tile;
      tile.b = b;
      tile.row0 = (nt - 1 - k) * kTileRows;
      tile.q_begin = p.qo_indptr[b] + tile.row0;
      tile.q_rows = min(kTileRows, qo - tile.row0);
      tile.qo_len = qo;
      tile.kv_len = kv;
      tile.kv_page_begin = p.kv_indptr[b];
      tile.pad = 0;
      p.tiles[idx] = tile;
    }
    running += total_sh;
    __syncthreads();
  }
  if (t == 0) {
    p.header->num_tiles = min(running, p.capacity);
    p.header->error = running > p.capacity ? 1 : 0;
  }
}

struct RunParams {
  const PrefillHeader* header;
  const PrefillTile* tiles;
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* pool;
  int64_t num_pages;
  const int32_t* indices;
  uint16_t* out;
  int64_t o_st, o_sh;
  int64_t total_q;
  int hkv, group, causal;
  float scale_log2;
};

template <int D>
__global__ __launch_bounds__(256) void prefill_run_kernel(RunParams p) {
  constexpr int KSTEPS = D / 32;
  constexpr int NT = D / 16;
  constexpr int VT_STRIDE = kKvTile + 8;  // bf16 per transposed row (80 bytes)
  __shared__ __attribute__((aligned(16))) uint16_t vt[D * VT_STRIDE];

  const int hq = blockIdx.y;
  const int hkv = hq / p.group;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, kb = lane >> 4;
  const int64_t tok_stride = int64_t(p.hkv) * D;
  const int64_t kv_stride = kPageSize * tok_stride;
  const int64_t page_stride = 2 * kv_stride;
  const int num_tiles = p.header->num_tiles;

  for (int ti = blockIdx.x; ti < num_tiles; ti += gridDim.x) {
    const PrefillTile t = p.tiles[ti];
    const int off = t.kv_len - t.qo_len;
    const int local = 16 * w + n;  // this lane's query row within the tile
    const bool qvalid = local < t.q_rows && (t.q_begin + local) < p.total_q;
    mi::bf16x8_t qb[KSTEPS];
    {
      const uint16_t* qrow = p.q + int64_t(t.q_begin + (qvalid ? local : 0)) * p.q_st + int64_t(hq) * p.q_sh + kb * 8;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (qvalid) v = mi::load16(qrow + s * 32);
        qb[s] = mi::as_bf16x8(v);
      }
    }
    int wave_hi = 0;
    if (16 * w < t.q_rows) {
      const int last_row = t.row0 + min(16 * w + 15, t.q_rows - 1);
      wave_hi = p.causal ? min(t.kv_len, last_row + off + 1) : t.kv_len;
    }
    int block_hi = p.causal ? min(t.kv_len, t.row0 + t.q_rows + off) : t.kv_len;
    block_hi = max(block_hi, 0);
    const int ntile = (block_hi + kKvTile - 1) / kKvTile;

    mi::f32x4_t o[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = mi::f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;
    const int qr = t.row0 + local;  // request-relative query index

    for (int kt = 0; kt < ntile; ++kt) {
      const int kv0 = kt * kKvTile;
      __syncthreads();
      for (int c = threadIdx.x; c < kKvTile * (D / 8); c += blockDim.x) {
        const int kv = c / (D / 8), dc = c - kv * (D / 8);
        const int j = kv0 + kv;
        uint4 v = make_uint4(0, 0, 0, 0);
        const int64_t page = j < t.kv_len ? p.indices[t.kv_page_begin + j / kPageSize] : -1;
        if (page >= 0 && page < p.num_pages) {
          v = mi::load16(p.pool + page * page_stride + kv_stride + (j % kPageSize) * tok_stride +
                         int64_t(hkv) * D + dc * 8);
        }
        uint16_t* col = vt + (dc * 8) * VT_STRIDE + kv;
        col[0 * VT_STRIDE] = uint16_t(v.x);
        col[1 * VT_STRIDE] = uint16_t(v.x >> 16);
        col[2 * VT_STRIDE] = uint16_t(v.y);
        col[3 * VT_STRIDE] = uint16_t(v.y >> 16);
        col[4 * VT_STRIDE] = uint16_t(v.z);
        col[5 * VT_STRIDE] = uint16_t(v.z >> 16);
        col[6 * VT_STRIDE] = uint16_t(v.w);
        col[7 * VT_STRIDE] = uint16_t(v.w >> 16);
      }
      __syncthreads();
      if (kv0 >= wave_hi) continue;

      // ---- S^T = K Q^T for keys kv0 + g*16 + (0..15)
      float sv[2][4];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int jk = kv0 + g * 16 + n;
        uint4 ka[KSTEPS];
        const int64_t kpage = jk < t.kv_len ? p.indices[t.kv_page_begin + jk / kPageSize] : -1;
        if (kpage >= 0 && kpage < p.num_pages) {
          const int64_t page = kpage;
          const uint16_t* krow = p.pool + page * page_stride + (jk % kPageSize) * tok_stride + int64_t(hkv) * D + kb * 8;
#pragma unroll
          for (int s = 0; s < KSTEPS; ++s) ka[s] = mi::load16(krow + s * 32);
        } else {
#pragma unroll
          for (int s = 0; s < KSTEPS; ++s) ka[s] = make_uint4(0, 0, 0, 0);
        }
        mi::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) c = mi::mfma_16x16x32_bf16(mi::as_bf16x8(ka[s]), qb[s], c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = kv0 + g * 16 + 4 * kb + i;
          const bool ok = qvalid && j < t.kv_len && (!p.causal || j <= qr + off);
          sv[g][i] = ok ? c[i] * p.scale_log2 : -INFINITY;
        }
      }
      // ---- online softmax for query row n (lanes n, n+16, n+32, n+48)
      float mx = sv[0][0];
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[g][i]);
      mx = fmaxf(mx, mi::lane_shuffle(mx, lane ^ 16));
      mx = fmaxf(mx, mi::lane_shuffle(mx, lane ^ 32));
      const float m_new = fmaxf(m_run, mx);
      const bool dead = (m_new == -INFINITY);
      const float alpha = dead ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      float pv[2][4];
      float psum = 0.f;
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[g][i] = dead ? 0.f : __builtin_amdgcn_exp2f(sv[g][i] - m_new);
          psum += pv[g][i];
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
      float ao[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ao[i] = mi::lane_shuffle(alpha, 4 * kb + i);
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[j][i] *= ao[i];

      // ---- O += P V
      uint4 pa_u;
      pa_u.x = mi::pack_bf16x2(pv[0][0], pv[0][1]);
      pa_u.y = mi::pack_bf16x2(pv[0][2], pv[0][3]);
      pa_u.z = mi::pack_bf16x2(pv[1][0], pv[1][1]);
      pa_u.w = mi::pack_bf16x2(pv[1][2], pv[1][3]);
      const mi::bf16x8_t pa = mi::as_bf16x8(pa_u);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const uint16_t* row = vt + (j * 16 + n) * VT_STRIDE;
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * kb);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * kb);
        const uint4 vb = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[j] = mi::mfma_16x16x32_bf16(pa, mi::as_bf16x8(vb), o[j]);
      }
    }

    // ---- normalise and store: lane holds rows 4*kb + i, column j*16 + n
    float l_tot = l_run + mi::lane_shuffle(l_run, lane ^ 16);
    l_tot += mi::lane_shuffle(l_tot, lane ^ 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = mi::lane_shuffle(l_tot, 4 * kb + i);
      const float inv = li > 0.f ? 1.f / li : 0.f;
      const int r = 16 * w + 4 * kb + i;
      if (r < t.q_rows && t.q_begin + r < p.total_q) {
        uint16_t* orow = p.out + int64_t(t.q_begin + r) * p.o_st + int64_t(hq) * p.o_sh;
#pragma unroll
        for (int j = 0; j < NT; ++j) orow[j * 16 + n] = mi::f32_to_bf16(o[j][i] * inv);
      }
    }
  }
}

}  // namespace

extern "C" size_t mi_prefill_workspace_size(int32_t batch_size, int64_t total_q) {
  if (batch_size < 0 || total_q < 0) return 0;
  return prefill_ws_bytes(batch_size, total_q);
}

extern "C" int mi_prefill_plan(void* workspace, size_t workspace_bytes, const int32_t* qo_indptr,
                               const int32_t* kv_indptr, const int32_t* kv_last_page_len,
                               int32_t batch_size, int64_t total_q, int32_t page_size,
                               mi_stream_t stream) {
  mi::clear_error();
  if (batch_size < 0 || total_q < 0) return mi::fail(MI_ERR_INVALID, "prefill plan: negative sizes");
  if (page_size != kPageSize) return mi::fail(MI_ERR_UNSUPPORTED, "prefill plan: page_size %d (built for 16)", page_size);
  const size_t need = prefill_ws_bytes(batch_size, total_q);
  if (!workspace || workspace_bytes < need)
    return mi::fail(MI_ERR_WORKSPACE, "prefill plan: workspace %zu bytes, need %zu", workspace_bytes, need);
  if (batch_size > 0 && (!qo_indptr || !kv_indptr || !kv_last_page_len))
    return mi::fail(MI_ERR_INVALID, "prefill plan: null indptr argument");
  char* ws = static_cast<char*>(workspace);
  PlanParams pp;
  pp.qo_indptr = qo_indptr;
  pp.kv_indptr = kv_indptr;
  pp.last_page_len = kv_last_page_len;
  pp.batch = batch_size;
  pp.capacity = int(tile_capacity(batch_size, total_q));
  pp.header = reinterpret_cast<PrefillHeader*>(ws);
  pp.tiles = reinterpret_cast<PrefillTile*>(ws + 256);
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), pp);
  return mi::check_launch("prefill_plan_kernel");
}

extern "C" int mi_prefill_run(void* workspace, size_t workspace_bytes, const void* q,
                              int64_t q_stride_token, int64_t q_stride_head, const void* paged_kv_cache,
                              int64_t num_pages, const int32_t* kv_indices, void* out,
                              int64_t out_stride_token, int64_t out_stride_head, int32_t batch_size,
                              int64_t total_q, int32_t num_qo_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t page_size, int32_t causal, float sm_scale,
                              mi_stream_t stream) {
  mi::clear_error();
  if (batch_size < 0 || total_q < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || num_qo_heads % num_kv_heads)
    return mi::fail(MI_ERR_INVALID, "prefill run: bad sizes");
  if (page_size != kPageSize) return mi::fail(MI_ERR_UNSUPPORTED, "prefill run: page_size %d (built for 16)", page_size);
  if (head_dim != 64 && head_dim != 128)
    return mi::fail(MI_ERR_UNSUPPORTED, "prefill run: head_dim %d (built for 64, 128)", head_dim);
  if (num_qo_heads > 65535) return mi::fail(MI_ERR_INVALID, "prefill run: too many heads");
  const size_t need = prefill_ws_bytes(batch_size, total_q);
  if (!workspace || workspace_bytes < need)
    return mi::fail(MI_ERR_WORKSPACE, "prefill run: workspace %zu bytes, need %zu", workspace_bytes, need);
  if (total_q == 0 || batch_size == 0) return MI_OK;
  if (!q || !paged_kv_cache || !kv_indices || !out) return mi::fail(MI_ERR_INVALID, "prefill run: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(paged_kv_cache) & 15) ||
      q_stride_token % 8 || q_stride_head % 8)
    return mi::fail(MI_ERR_INVALID, "prefill run: q rows and pool must be 16-byte aligned");
  char* ws = static_cast<char*>(workspace);
  RunParams rp;
  rp.header = reinterpret_cast<const PrefillHeader*>(ws);
  rp.tiles = reinterpret_cast<const PrefillTile*>(ws + 256);
  rp.q = static_cast<const uint16_t*>(q);
  rp.q_st = q_stride_token;
  rp.q_sh = q_stride_head;
  rp.pool = static_cast<const uint16_t*>(paged_kv_cache);
  rp.num_pages = num_pages;
  rp.indices = kv_indices;
  rp.out = static_cast<uint16_t*>(out);
  rp.o_st = out_stride_token;
  rp.o_sh = out_stride_head;
  rp.total_q = total_q;
  rp.hkv = num_kv_heads;
  rp.group = num_qo_heads / num_kv_heads;
  rp.causal = causal ? 1 : 0;
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf(float(head_dim));
  rp.scale_log2 = scale * mi::kLog2e;
  int64_t gx = int64_t(tile_capacity(batch_size, total_q));
  if (gx > 65535) gx = 65535;
  const dim3 grid{static_cast<uint32_t>(gx), static_cast<uint32_t>(num_qo_heads), 1u};
  if (head_dim == 64)
    hipLaunchKernelGGL(prefill_run_kernel<64>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), rp);
  else
    hipLaunchKernelGGL(prefill_run_kernel<128>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), rp);
  return mi::check_launch("prefill_run_kernel");
}
