// Ragged (varlen) causal prefill attention over the paged pool, bf16 MFMA.
//
// Reference: the prefill wrapper's plan() (scheduler.py:704-716: qo_indptr,
// paged_kv_indptr / indices / last_page_len, causal=True) and run()
// (model.py:235, mode == "prefill").  Query row i of request b sees KV tokens
// j <= i + (kv_len - qo_len); the reference always has kv_len == qo_len.
//
// Work decomposition.  A workgroup (4 waves) owns `bm` query positions of one
// request and ALL `group` Q heads of one KV head: bm x group (position, head)
// rows in position-major order, cut into row blocks of 16 rows dealt to the
// waves round robin (three per wave for head_dim 128, two for 64, one for 256,
// computed together so every K / V operand read from LDS feeds all of them).
// bm = rows / group (192 rows for head_dim 128: 24 positions for group 8, 48
// for group 4), so every K/V byte the workgroup stages serves all the heads
// of its group.  (8-wave workgroups over twice the positions halve the
// staging per wave but measured 10 % slower: two independent 4-wave
// workgroups per CU keep computing across each other's barriers.)  plan()
// lists the tiles request
// by request (longest prompt first), each request's tiles heaviest first; the
// grid maps tile-major, so the XCD that a KV head's workgroups land on runs
// one request's tiles back to back and finds its K / V in L2.
//
// Per 64-key tile: the workgroup stages K and V in LDS (double buffered: the
// next tile's global loads are in flight while this one is consumed; one
// barrier per tile); each wave, per row block:
//   S^T = K Q^T  -- 16x16x32 MFMAs, K rows read from LDS as the A operand,
//                   Q^T held in registers as B; lane (g, n) gets
//                   S^T[key 4g+i][row n] for each 16-key block;
//   online softmax per row in the exp2 domain with a lazy running max
//   (rescale only when the max grows by more than 2^8); row maxima across
//   lane groups with the gfx950 lane-swap instructions;
//   O += P V     -- 16x16x32 MFMAs over 32 keys: the S^T accumulators of two
//                   key blocks are exactly the P operand (lane (g, n) holds
//                   keys {4g+i} of both), and V comes from the gfx950 LDS
//                   transpose read in the same key order.
#include <math.h>

#include <type_traits>

#include "mi_common.h"

namespace {

// s_waitcnt immediate (gfx9 encoding): vmcnt = 0, expcnt = 7, lgkmcnt = 15.
constexpr int kWaitVmcnt0 = 0x0F70;
// Buffer resource word 3 for gfx9 raw buffers (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;

constexpr int kPageSize = 16;
constexpr int kMinRows = 8;    // fewest query positions per workgroup (head_dim 256, group 8)
constexpr int kKvTile = 64;    // keys per staged tile (4 pages)
constexpr float kLazyRescale = 8.0f;
#ifndef PREFILL_WAVES
#define PREFILL_WAVES 2
#endif
// 32-byte row pad: the transpose reads of V (four rows x 32 bytes per
// 16 lanes) and the 16-byte K reads both land on distinct banks (a 16-byte
// pad measured 13.9M bank-conflict cycles per launch on the Mistral-7B
// batch, 32 bytes none).
#ifndef PREFILL_RS_PAD
#define PREFILL_RS_PAD 32
#endif
// K / V tiles staged straight to LDS by the gfx950 buffer loads with the
// `lds` modifier (no staging registers, no LDS store instructions).  A wave's
// load instruction fills 1 KB of LDS, lane l at byte 16 l, so the rows are
// unpadded and a 16-byte chunk's place in its row is permuted instead
// (chunk_slot) to keep the reads off shared banks.
#ifndef PREFILL_DMA
#define PREFILL_DMA 1
#endif
// Output staging: pad bytes after every 8 columns (32 bytes each) of a
// column-major 16-row block, so the 8-byte writes of a half wave and the
// transpose reads of two lane groups fall on distinct banks.
constexpr int kOutPad = 144;

struct alignas(32) PrefillTile {
  int b;
  int q_begin;  // absolute first query row of the tile
  int q_rows;   // positions in this tile (<= bm)
  int qo_len;
  int kv_len;
  int row0;           // first position of the tile within its request
  int kv_page_begin;  // absolute position of the request's first page in kv_indices
  int pad;
};

struct PrefillHeader {
  int num_tiles;
  int error;
  int bm;
  int pad;
};

// Waves per workgroup.
constexpr int waves_for(int /*head_dim*/) { return 4; }

// Row blocks of 16 (position, head) rows per wave: three for head_dim 128
// (each K / V operand read from LDS then feeds three blocks), two for 64, one
// for 256.
int row_blocks(int /*group*/, int head_dim) { return head_dim > 128 ? 1 : head_dim == 128 ? 3 : 2; }

// Query positions per workgroup: the workgroup's 16 * waves * row blocks rows
// hold bm positions x group heads, bm = rows / group.
int rows_per_tile(int group, int head_dim) {
  const int bm = 16 * waves_for(head_dim) * row_blocks(group, head_dim) / group;
  return bm < kMinRows ? kMinRows : bm;
}

size_t tile_capacity(int batch, int64_t total_q) { return size_t(total_q / kMinRows + batch + 1); }

size_t prefill_ws_bytes(int batch, int64_t total_q) {
  return 256 + mi::align_up(tile_capacity(batch, total_q) * sizeof(PrefillTile), 256);
}

struct PlanParams {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int batch;
  int capacity;
  int bm;
  PrefillHeader* header;
  PrefillTile* tiles;
};

// Inclusive scan over the block; *total gets the block-wide sum.  Ends with a
// barrier so `buf` may be reused at once.
__device__ int block_scan(int v, int* buf, int* total) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int o = 1; o < int(blockDim.x); o <<= 1) {
    const int add = (t >= o) ? buf[t - o] : 0;
    __syncthreads();
    buf[t] += add;
    __syncthreads();
  }
  const int r = buf[t];
  *total = buf[blockDim.x - 1];
  __syncthreads();
  return r;
}

// Tile order: requests by decreasing prompt length (ties by index), each
// request's tiles from the end of its prompt (most keys) to the start.  The
// run kernel maps consecutive tiles of one (request, KV head) to consecutive
// workgroups of one XCD, so they share the request's K / V in that XCD's L2.
__global__ __launch_bounds__(1024) void prefill_plan_kernel(PlanParams p) {
  __shared__ int buf[1024];
  const int t = threadIdx.x;
  int total = 0;
  for (int base = 0; base < p.batch; base += blockDim.x) {
    const int b = base + t;
    int nt = 0, start = 0;
    if (b < p.batch) {
      const int qo = max(0, p.qo_indptr[b + 1] - p.qo_indptr[b]);
      nt = (qo + p.bm - 1) / p.bm;
      // tiles of the requests ordered before b
      for (int c = 0; c < p.batch; ++c) {
        const int qc = max(0, p.qo_indptr[c + 1] - p.qo_indptr[c]);
        if (qc > qo || (qc == qo && c < b)) start += (qc + p.bm - 1) / p.bm;
      }
      if (start + nt <= p.capacity) {
        const int np = max(0, p.kv_indptr[b + 1] - p.kv_indptr[b]);
        const int kv = np > 0 ? (np - 1) * kPageSize + min(max(p.last_page_len[b], 1), kPageSize) : 0;
        for (int k = 0; k < nt; ++k) {
          PrefillTile tile;
          tile.b = b;
          tile.row0 = (nt - 1 - k) * p.bm;
          tile.q_begin = p.qo_indptr[b] + tile.row0;
          tile.q_rows = min(p.bm, qo - tile.row0);
          tile.qo_len = qo;
          tile.kv_len = kv;
          tile.kv_page_begin = p.kv_indptr[b];
          tile.pad = 0;
          p.tiles[start + k] = tile;
        }
      }
    }
    int chunk_total = 0;
    block_scan(nt, buf, &chunk_total);
    total += chunk_total;
  }
  if (t == 0) {
    p.header->num_tiles = min(total, p.capacity);
    p.header->error = total > p.capacity ? 1 : 0;
    p.header->bm = p.bm;
  }
}

struct RunParams {
  const PrefillHeader* header;
  const PrefillTile* tiles;
  const uint16_t* q;
  int64_t q_st, q_sh;
  int64_t q_ext;  // elements one position's heads span: (heads - 1) * q_sh + head_dim
  const uint16_t* pool;
  int64_t num_pages;
  const int32_t* indices;
  uint16_t* out;
  int64_t o_st, o_sh, o_ext;
  int64_t total_q;
  int hkv, group, causal, bm;
  float scale_log2;
};

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(8))) short s16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(8))) float f32x8_v;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_v;
typedef __attribute__((address_space(3))) char lds_t;

typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;

__device__ __forceinline__ void lds_store16(lds_t* p, u32x4_t v) { *(__attribute__((address_space(3))) u32x4_t*)p = v; }
__device__ __forceinline__ void lds_store8(lds_t* p, u32x2_t v) { *(__attribute__((address_space(3))) u32x2_t*)p = v; }
__device__ __forceinline__ u32x4_t lds_load16(const lds_t* p) {
  return *(const __attribute__((address_space(3))) u32x4_t*)p;
}
// gfx950 LDS transpose read: the 16 lanes of a group address 4 rows x 16
// bf16 (lane j: row j/4, elements 4*(j%4)..+3) and lane j receives column j.
__device__ __forceinline__ s16x4_t lds_read_tr16(const lds_t* p) {
  typedef __attribute__((address_space(3))) bf16x4_t lds_v4;
  return __builtin_bit_cast(s16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4*)p));
}
// 16 bytes per lane from a buffer straight to LDS: lane l's bytes land at
// dst + 16 l (dst wave-uniform).  The builtin exists for the device pass only
// (the host pass would drop the kernel stubs that reference it).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, lds_t* dst, int voffset, int soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16, voffset, soffset, 0, 0);
#endif
}
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int wave_max_i(int x) {
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Slot (16-byte unit of the row) where chunk c of tile row r is staged when
// the rows are unpadded: c XOR a per-row value.  Measured with
// SQ_LDS_BANK_CONFLICT on the Mistral-7B / Qwen2.5-72B head batches (per
// launch): no permutation 70.8M / 210.8M conflict cycles; XOR (r & 15) 6.8M /
// 16.8M; XOR 2 (r & 7) 1.8M / 1.9M (what the 32-byte row pad gave), so the 8
// rows of a K read group and the 4 rows x 32 bytes of a V transpose-read
// group land on distinct banks.  128-byte rows (head_dim 64) put two rows in
// a bank period and take XOR 2 ((r >> 1) & 3).
template <int D>
__device__ __forceinline__ int chunk_slot(int r, int c) {
  if constexpr (D == 64) return c ^ (((r >> 1) & 3) << 1);
  else return c ^ ((r & 7) << 1);
}

template <int D, int MAXRB_>
struct PrefillTraits {
  static constexpr int WAVES = waves_for(D);
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int KSTEPS = D / 32;            // 16x16x32 MFMAs per 16-key block of S^T
  static constexpr int NT = D / 16;                // 16-wide head_dim tiles of O
  static constexpr int CPR = D / 8;                // 16-byte chunks per token row
  static constexpr int LOADS = kKvTile * CPR / THREADS;  // 16-byte loads per thread per tile, K and V each
  static_assert(LOADS >= 1 && kKvTile * CPR % THREADS == 0, "tile staging split");
  static constexpr int RS = PREFILL_DMA ? D * 2 : D * 2 + PREFILL_RS_PAD;  // LDS row stride
  static constexpr int TILE = kKvTile * RS;        // bytes of one staged K or V tile
  static constexpr int MAXRB = MAXRB_;             // row blocks per wave
  static constexpr int OUT_BLK = 8 * 32 + kOutPad;  // output staging: bytes per 8 columns
  static constexpr int OB = D / 8 * OUT_BLK;         // output staging: bytes per row block
  // LDS: the double-buffered K / V tiles, reused for the output staging
  static constexpr int SMEM = 2 * 2 * TILE > WAVES * MAXRB * OB ? 2 * 2 * TILE : WAVES * MAXRB * OB;
};

template <int D, int MAXRB>
__global__ __launch_bounds__(64 * waves_for(D)) __attribute__((amdgpu_waves_per_eu(D <= 128 ? PREFILL_WAVES : 1))) void prefill_run_kernel(RunParams p) {
  using T = PrefillTraits<D, MAXRB>;
  __shared__ __attribute__((aligned(16))) char smem[T::SMEM];  // [buffer][K, V], then the output rows
  lds_t* lds = (lds_t*)smem;

  const int tile_idx = int(blockIdx.x) / p.hkv;
  const int hkv = int(blockIdx.x) - tile_idx * p.hkv;
  if (tile_idx >= p.header->num_tiles) return;  // whole workgroup
  const PrefillTile t = p.tiles[tile_idx];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, n = lane & 15;
  const int off = t.kv_len - t.qo_len;
  // the workgroup's rows in position-major order: row R is position R / group
  // of the tile, head R % group of this KV head's group; row block rb holds
  // rows 16 rb .. 16 rb + 15
  const int nrows = p.bm * p.group;
  const int nrb = (nrows + 15) / 16;


  // ---- this wave's row blocks: rb = w, w + 4
  mi::bf16x8_t qb[T::MAXRB][T::KSTEPS];
  mi::f32x4_t o[T::MAXRB][T::NT];
  float m_run[T::MAXRB], l_run[T::MAXRB];
  int qpos[T::MAXRB];     // request-relative position of this lane's row n (-1: none)
  int lim[T::MAXRB];      // last key this lane's row may see (-1: none)
  int rb_hi[T::MAXRB];    // keys this row block needs (causal)
  int head[T::MAXRB];     // this lane's row's Q head
  int lpos[T::MAXRB];     // this lane's row's position within the tile (-1: none)
  int nblk = 0;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.q + int64_t(t.q_begin) * p.q_st), (short)0,
      int((int64_t(max(t.q_rows, 1) - 1) * p.q_st + p.q_ext) * 2), kBufferWord3);
#pragma unroll
  for (int r = 0; r < T::MAXRB; ++r) {
    const int rb = w + T::WAVES * r;
    const bool has = rb < nrb;
    nblk += has ? 1 : 0;
    const int row = rb * 16 + n;
    const int local = row / p.group;
    head[r] = hkv * p.group + (row - local * p.group);
    const bool valid = has && row < nrows && local < t.q_rows;
    lpos[r] = valid ? local : -1;
    qpos[r] = valid ? t.row0 + local : -1;
    lim[r] = !valid ? -1 : (p.causal ? min(t.kv_len - 1, qpos[r] + off) : t.kv_len - 1);
    const int last = t.row0 + min((rb * 16 + 15) / p.group, t.q_rows - 1);  // the block's last position
    rb_hi[r] = !has ? 0 : (p.causal ? min(t.kv_len, last + off + 1) : t.kv_len);
    // Q rows through a descriptor over the tile's rows: a row past the tile
    // reads out of range (zeros), so the loads are unconditional
    const int qoff = valid ? int((int64_t(local) * p.q_st + int64_t(head[r]) * p.q_sh + g * 8) * 2) : 0x7ffffff0;
#pragma unroll
    for (int s = 0; s < T::KSTEPS; ++s)
      qb[r][s] = __builtin_bit_cast(mi::bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, s * 64, 0));
#pragma unroll
    for (int j = 0; j < T::NT; ++j) o[r][j] = mi::f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
  }
  // smallest valid row position of the wave (for the unmasked-tile test)
  int qmin = 0x7fffffff;
#pragma unroll
  for (int r = 0; r < T::MAXRB; ++r)
    if (qpos[r] >= 0) qmin = min(qmin, qpos[r]);
  qmin = -wave_max_i(-qmin);
  int block_hi = p.causal ? min(t.kv_len, t.row0 + t.q_rows + off) : t.kv_len;
  block_hi = max(block_hi, 0);
  const int ntile = (block_hi + kKvTile - 1) / kKvTile;

  // ---- staging.  Load i of a thread covers token ltok + TPL i of the tile
  // and 16-byte chunk ldc of that token's row: a wave's 64 lanes cover whole
  // rows of one page (1 KB <= 16 rows), so the page id is wave-uniform -- a
  // scalar load, fetched one tile ahead -- and each page gets a buffer
  // descriptor (size 0 past the request's pages; on the request's last page
  // the size stops after its valid V rows, so the V rows past kv_len read as
  // zeros: P is 0 there, but 0 * NaN would poison the MFMA).  No address
  // arithmetic or branches per load.
  const int tok_bytes = p.hkv * D * 2;
  const int kv_bytes = kPageSize * tok_bytes;
  const int page_bytes = 2 * kv_bytes;
  const int npages_req = (t.kv_len + kPageSize - 1) / kPageSize;
  const int last_rows = t.kv_len - (npages_req - 1) * kPageSize;
  int voff[T::LOADS], pit[T::LOADS];
#if PREFILL_DMA
  // Load i of wave w fills 1 KB block b = WAVES i + w of the tile: RPB rows,
  // lane l taking row b RPB + l / CPR and slot l % CPR of it, i.e. the chunk
  // chunk_slot(row, slot) (the permutation is its own inverse); a block lies
  // inside one page, so the page index is wave-uniform.
  constexpr int RPB = 1024 / (D * 2);
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
#pragma unroll
  for (int i = 0; i < T::LOADS; ++i) {
    const int bk = T::WAVES * i + wv;
    const int tr = bk * RPB + lane / T::CPR;
    pit[i] = __builtin_amdgcn_readfirstlane(bk * RPB / kPageSize);
    voff[i] = (tr % kPageSize) * tok_bytes + hkv * D * 2 + chunk_slot<D>(tr, lane % T::CPR) * 16;
  }
#else
  constexpr int TPL = T::THREADS / T::CPR;
  const int ltok = int(threadIdx.x) / T::CPR, ldc = int(threadIdx.x) - ltok * T::CPR;
#pragma unroll
  for (int i = 0; i < T::LOADS; ++i) {
    const int tt = ltok + TPL * i;
    pit[i] = __builtin_amdgcn_readfirstlane(tt / kPageSize);
    voff[i] = (tt % kPageSize) * tok_bytes + hkv * D * 2 + ldc * 16;
  }
  u32x4_t kreg[T::LOADS], vreg[T::LOADS];
#endif
  int pid[T::LOADS];
  // page ids through the constant address space: a uniform index then
  // compiles to a scalar load (kv_indices is not written during the launch)
  typedef __attribute__((address_space(4))) const int32_t const_i32;
  const const_i32* kv_ids = (const const_i32*)(p.indices);
  auto fetch_ids = [&](int kt) {
#pragma unroll
    for (int i = 0; i < T::LOADS; ++i) {
      const int pg_idx = kt * (kKvTile / kPageSize) + pit[i];
      // the index is clamped into the request's pages (it has >= 1 page
      // whenever there is a tile), then the id is dropped past the end
      const int v = kv_ids[t.kv_page_begin + min(pg_idx, npages_req - 1)];
      pid[i] = (kt < ntile && pg_idx < npages_req) ? v : -1;
    }
  };
  auto load_tile = [&](int kt, int buf) {
#pragma unroll
    for (int i = 0; i < T::LOADS; ++i) {
      const int pg = pid[i];
      const bool ok = pg >= 0 && pg < p.num_pages;
      const int pg_idx = kt * (kKvTile / kPageSize) + pit[i];
      const int size = !ok ? 0 : (pg_idx == npages_req - 1 ? kv_bytes + last_rows * tok_bytes : page_bytes);
      const char* base = reinterpret_cast<const char*>(p.pool) + (ok ? int64_t(pg) * page_bytes : 0);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, size, kBufferWord3);
#if PREFILL_DMA
      lds_t* kdst = lds + buf * 2 * T::TILE + 1024 * (T::WAVES * i + wv);
      lds_dma16(rs, kdst, voff[i], 0);
      lds_dma16(rs, kdst + T::TILE, voff[i], kv_bytes);
#else
      (void)buf;
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[i], 0, 0);
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[i], kv_bytes, 0);
#endif
    }
  };
  auto store_tile = [&](int buf) {
#if !PREFILL_DMA
    lds_t* kl = lds + buf * 2 * T::TILE + ltok * T::RS + ldc * 16;
    lds_t* vl = kl + T::TILE;
#pragma unroll
    for (int i = 0; i < T::LOADS; ++i) {
      lds_store16(kl + TPL * i * T::RS, kreg[i]);
      lds_store16(vl + TPL * i * T::RS, vreg[i]);
    }
#else
    (void)buf;
#endif
  };

  if (ntile > 0) {
    fetch_ids(0);
    load_tile(0, 0);
    fetch_ids(1);
    store_tile(0);
  }
  // Everything loaded so far (Q, tile 0, the next page ids) is waited for
  // here, so the loop head carries no pending load from before the loop;
  // without it the compiler put a full vmcnt(0) before the first score MFMA
  // of every tile, which also waited for the next tile's prefetch.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();

  // LDS read offsets inside a staged tile: K row kb 16 + n (chunk 4 s + g) for
  // the score operand, V rows 4 g + n / 4 (bytes 32 j + 8 (n & 3)) for the
  // transpose reads; tile rows are r and r + 16 k, whose permutation depends
  // on r % 16 only.
  int koff[T::KSTEPS], voff_lds[T::NT];
#pragma unroll
  for (int s2 = 0; s2 < T::KSTEPS; ++s2)
    koff[s2] = PREFILL_DMA ? n * T::RS + chunk_slot<D>(n, 4 * s2 + g) * 16 : n * T::RS + (4 * s2 + g) * 16;
#pragma unroll
  for (int j = 0; j < T::NT; ++j) {
    const int vr = 4 * g + (n >> 2);
    voff_lds[j] = PREFILL_DMA ? vr * T::RS + chunk_slot<D>(vr, 2 * j + ((n & 3) >> 1)) * 16 + (n & 1) * 8
                              : vr * T::RS + (n & 3) * 8 + 32 * j;
  }

  for (int kt = 0; kt < ntile; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntile) {
      load_tile(kt + 1, buf ^ 1);
      fetch_ids(kt + 2);
    }
    const int kv0 = kt * kKvTile;
    const lds_t* kl = lds + buf * 2 * T::TILE;
    const lds_t* vl = kl + T::TILE;
    // All of the wave's row blocks are computed together so each K / V
    // operand read from LDS feeds MAXRB MFMAs.  A block with nothing left to
    // do (causally finished, or absent: qpos = -1) masks every key and adds
    // exactly zero, so no per-block branches are needed.
    bool any = false;
#pragma unroll
    for (int r = 0; r < T::MAXRB; ++r) any = any || (r < nblk && kv0 < rb_hi[r]);
    if (any) {
      // No key of the tile needs a mask: all are < kv_len and (causal) visible
      // to the wave's first valid row.  (Rows past the tile's end hold zero
      // queries and are never written, so they need no mask either.)
      const bool full = kv0 + kKvTile <= t.kv_len && (!p.causal || kv0 + kKvTile - 1 <= qmin + off);
      // ---- one tile: S^T for the four 16-key blocks (raw scores; the softmax
      // scale is applied inside the exponent; two copies of the score loop,
      // so full tiles carry no mask code), the row maxima, one lazy-rescale
      // branch for the wave, then exp / pack / P V half by half, so the P V
      // MFMAs of keys 0-31 can overlap the exponentials of keys 32-63.
      float sv[T::MAXRB][4][4];
      auto scores = [&](auto masked) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          mi::bf16x8_t ka[T::KSTEPS];
#pragma unroll
          for (int s = 0; s < T::KSTEPS; ++s)
            ka[s] = __builtin_bit_cast(mi::bf16x8_t, lds_load16(kl + kb * 16 * T::RS + koff[s]));
#pragma unroll
          for (int r = 0; r < T::MAXRB; ++r) {
            mi::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < T::KSTEPS; ++s) c = mi::mfma_16x16x32_bf16(ka[s], qb[r][s], c);
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[r][kb][i] = c[i];
            if constexpr (decltype(masked)::value) {
              // key kv0 + kb*16 + 4g + i is visible iff kb*16 + i <= lim - kv0 - 4g
              const int rel = lim[r] - kv0 - 4 * g;
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (kb * 16 + i > rel) sv[r][kb][i] = -INFINITY;
            }
          }
        }
      };
      // The score MFMAs and the row maxima run at raised wave priority: the
      // other workgroup's wave on the SIMD is then usually in its softmax /
      // P V part, and the arbiter issues this wave's MFMAs first while that
      // VALU work fills the gaps (Qwen2.5-72B / Qwen2.5-7B head batches
      // -1.9..-2.2 / -1.1..-1.5 % over three boxes, Mistral-7B heads
      // -1.2..+0.9 %; around the P V MFMAs as well: no better; the reverse
      // -- priority over the softmax instead -- gains the same: what helps is
      // that the two workgroups' waves on a SIMD stop moving in step)
      __builtin_amdgcn_s_setprio(1);
      if (full) scores(std::false_type{});
      else scores(std::true_type{});
      {
        float mloc[T::MAXRB];
        bool need[T::MAXRB];
        bool any_need = false;
#pragma unroll
        for (int r = 0; r < T::MAXRB; ++r) {
          float m = sv[r][0][0];
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) m = fmaxf(m, sv[r][kb][i]);
          mloc[r] = max_xor32(max_xor16(m)) * p.scale_log2;  // scale > 0 keeps the arg max
          need[r] = mloc[r] > m_run[r] + kLazyRescale;
          any_need = any_need || need[r];
        }
        __builtin_amdgcn_s_setprio(0);
        if (__builtin_amdgcn_ballot_w64(any_need)) {
#pragma unroll
          for (int r = 0; r < T::MAXRB; ++r) {
            // a row that has seen no key yet (m_run = -inf) still has O = 0
            // and l = 0: only its max moves, nothing is rescaled
            const bool scale = need[r] && m_run[r] != -INFINITY;
            const float f = scale ? __builtin_amdgcn_exp2f(m_run[r] - mloc[r]) : 1.f;
            m_run[r] = need[r] ? mloc[r] : m_run[r];
            l_run[r] *= f;
            if (__builtin_amdgcn_ballot_w64(scale)) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float fo = mi::lane_shuffle(f, 4 * g + i);
#pragma unroll
                for (int j = 0; j < T::NT; ++j) o[r][j][i] *= fo;
              }
            }
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // exp2(-inf - m) = 0 for masked keys; m is taken as 0 while the row
          // has seen no key (m_run still -inf), avoiding -inf - -inf
          mi::bf16x8_t pa[T::MAXRB];
#pragma unroll
          for (int r = 0; r < T::MAXRB; ++r) {
            const float m_use = (m_run[r] == -INFINITY) ? 0.f : m_run[r];
            float pv[2][4];
            float ps = 0.f;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                pv[kk][i] = __builtin_amdgcn_exp2f(fmaf(sv[r][2 * h + kk][i], p.scale_log2, -m_use));
                ps += pv[kk][i];
              }
            l_run[r] += ps;
            pa[r] = __builtin_bit_cast(
                mi::bf16x8_t, __builtin_convertvector((f32x8_v){pv[0][0], pv[0][1], pv[0][2], pv[0][3], pv[1][0],
                                                                pv[1][1], pv[1][2], pv[1][3]},
                                                      bf16x8_v));
          }
          // ---- O += P V over key blocks (2h, 2h + 1)
          const lds_t* v0 = vl + 2 * h * 16 * T::RS;
#if PREFILL_DMA
          // The transpose reads go through inline asm here: with the builtin the
          // compiler waited for every load to LDS in flight (the next tile's)
          // before the first of them.  One statement per group of 4 columns:
          // 8 reads (the second page's rows 16 * RS further) and the wait for
          // them, so its outputs hold the data when it ends.
          static_assert(T::NT % 4 == 0, "column groups of 4");
          const uint32_t vb0 = uint32_t(reinterpret_cast<uintptr_t>(v0));
#pragma unroll
          for (int q = 0; q < T::NT / 4; ++q) {
            const int j0 = 4 * q;
            u32x2_t ra[4], rb[4];
            asm volatile(
                "ds_read_b64_tr_b16 %0, %8\n\t"
                "ds_read_b64_tr_b16 %1, %8 offset:%12\n\t"
                "ds_read_b64_tr_b16 %2, %9\n\t"
                "ds_read_b64_tr_b16 %3, %9 offset:%12\n\t"
                "ds_read_b64_tr_b16 %4, %10\n\t"
                "ds_read_b64_tr_b16 %5, %10 offset:%12\n\t"
                "ds_read_b64_tr_b16 %6, %11\n\t"
                "ds_read_b64_tr_b16 %7, %11 offset:%12\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(ra[0]), "=&v"(rb[0]), "=&v"(ra[1]), "=&v"(rb[1]), "=&v"(ra[2]), "=&v"(rb[2]), "=&v"(ra[3]),
                  "=&v"(rb[3])
                : "v"(vb0 + voff_lds[j0]), "v"(vb0 + voff_lds[j0 + 1]), "v"(vb0 + voff_lds[j0 + 2]),
                  "v"(vb0 + voff_lds[j0 + 3]), "i"(16 * T::RS)
                : "memory");
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const mi::bf16x8_t vb =
                  __builtin_bit_cast(mi::bf16x8_t, u32x4_t{ra[jj].x, ra[jj].y, rb[jj].x, rb[jj].y});
#pragma unroll
              for (int r = 0; r < T::MAXRB; ++r) o[r][j0 + jj] = mi::mfma_16x16x32_bf16(pa[r], vb, o[r][j0 + jj]);
            }
          }
#else
          const lds_t* v1 = v0 + 16 * T::RS;
#pragma unroll
          for (int j = 0; j < T::NT; ++j) {
            const s16x4_t a = lds_read_tr16(v0 + voff_lds[j]), b = lds_read_tr16(v1 + voff_lds[j]);
            const mi::bf16x8_t vb =
                __builtin_bit_cast(mi::bf16x8_t, (s16x8_t){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]});
#pragma unroll
            for (int r = 0; r < T::MAXRB; ++r) o[r][j] = mi::mfma_16x16x32_bf16(pa[r], vb, o[r][j]);
          }
#endif
        }
      }
    }
    if (kt + 1 < ntile) store_tile(buf ^ 1);
#if PREFILL_DMA
    // the next tile's rows are in LDS (the loads went straight there)
    if (kt + 1 < ntile) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
#endif
    __syncthreads();
  }

  // ---- normalise and store.  Lane (g, n) holds O rows 4g + i, columns 16j + n.
  // The normalised rows go through LDS (the K / V buffers are free after the
  // loop's last barrier) as a column-major block per row block: element
  // (row, col) at byte col * 32 + (col / 8) * kOutPad + row * 2, so a lane's
  // four rows of one column are one 8-byte write, and the LDS transpose read
  // of a 4-column x 16-row block hands lane n four consecutive columns of row
  // n: two reads give 16 contiguous bytes of an output row, one 16-byte store
  // through a descriptor over the tile's output rows (rows past the tile get
  // an out-of-range offset, so the stores are unconditional).
  constexpr int kOutBlk = T::OUT_BLK;
  constexpr int OB = T::OB;
  lds_t* const ob = lds + w * T::MAXRB * OB;
  const int wcol = n * 32 + (n >> 3) * kOutPad + 8 * g;
#pragma unroll
  for (int r = 0; r < T::MAXRB; ++r) {
    if (r >= nblk) continue;
    const float lt = sum_xor32(sum_xor16(l_run[r]));
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = mi::lane_shuffle(lt, 4 * g + i);
      inv[i] = li > 0.f ? mi::fast_rcp(li) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < T::NT; ++j)  // column 16j + n: 8-column block 2j + n / 8
      lds_store8(ob + r * OB + j * 2 * kOutBlk + wcol,
                 u32x2_t{mi::cvt_pk_bf16(o[r][j][0] * inv[0], o[r][j][1] * inv[1]),
                         mi::cvt_pk_bf16(o[r][j][2] * inv[2], o[r][j][3] * inv[3])});
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.out + int64_t(t.q_begin) * p.o_st), (short)0,
      int((int64_t(max(t.q_rows, 1) - 1) * p.o_st + p.o_ext) * 2), kBufferWord3);
  // lane (g, n) reads columns 32q + 8g + [0, 8) of row n
  const int rcol = g * kOutBlk + (n >> 2) * 32 + (n & 3) * 8;
#pragma unroll
  for (int r = 0; r < T::MAXRB; ++r) {
    if (r >= nblk) continue;
    const int local = lpos[r];
    const bool valid = local >= 0 && t.q_begin + local < p.total_q;
    const int off = valid ? int((int64_t(local) * p.o_st + int64_t(head[r]) * p.o_sh) * 2) + 16 * g : 0x7ffffff0;
#pragma unroll
    for (int q = 0; q < D / 32; ++q) {
      const lds_t* src = ob + r * OB + q * 4 * kOutBlk + rcol;
      const s16x4_t a = lds_read_tr16(src), c = lds_read_tr16(src + 128);
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4_t, (s16x8_t){a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]}), ro, off, 64 * q, 0);
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
                               int32_t batch_size, int64_t total_q, int32_t num_qo_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                               mi_stream_t stream) {
  mi::clear_error();
  if (batch_size < 0 || total_q < 0) return mi::fail(MI_ERR_INVALID, "prefill plan: negative sizes");
  if (num_qo_heads <= 0 || num_kv_heads <= 0 || num_qo_heads % num_kv_heads)
    return mi::fail(MI_ERR_INVALID, "prefill plan: bad head counts (%d, %d)", num_qo_heads, num_kv_heads);
  if (num_qo_heads / num_kv_heads > 8)
    return mi::fail(MI_ERR_UNSUPPORTED, "prefill plan: group %d (built for 1..8)", num_qo_heads / num_kv_heads);
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
  pp.bm = rows_per_tile(num_qo_heads / num_kv_heads, head_dim);
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
  if (num_qo_heads / num_kv_heads > 8)
    return mi::fail(MI_ERR_UNSUPPORTED, "prefill run: group %d (built for 1..8)", num_qo_heads / num_kv_heads);
  if (page_size != kPageSize) return mi::fail(MI_ERR_UNSUPPORTED, "prefill run: page_size %d (built for 16)", page_size);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return mi::fail(MI_ERR_UNSUPPORTED, "prefill run: head_dim %d (built for 64, 128, 256)", head_dim);
  const size_t need = prefill_ws_bytes(batch_size, total_q);
  if (!workspace || workspace_bytes < need)
    return mi::fail(MI_ERR_WORKSPACE, "prefill run: workspace %zu bytes, need %zu", workspace_bytes, need);
  if (total_q == 0 || batch_size == 0) return MI_OK;
  if (!q || !paged_kv_cache || !kv_indices || !out) return mi::fail(MI_ERR_INVALID, "prefill run: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(paged_kv_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 15) || q_stride_token % 8 || q_stride_head % 8 ||
      out_stride_token % 8 || out_stride_head % 8)
    return mi::fail(MI_ERR_INVALID, "prefill run: q rows, out rows and pool must be 16-byte aligned");
  if (q_stride_token < 0 || q_stride_head < 0 || out_stride_token < 0 || out_stride_head < 0)
    return mi::fail(MI_ERR_INVALID, "prefill run: negative stride");
  const int64_t grid = int64_t(tile_capacity(batch_size, total_q)) * num_kv_heads;
  if (grid > 0x7fffffff) return mi::fail(MI_ERR_INVALID, "prefill run: too many tiles");
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
  rp.bm = rows_per_tile(rp.group, head_dim);
  // a tile addresses its q / out rows through one buffer descriptor each, by
  // 32-bit byte offsets from its first position: any strides (heads inside a
  // position's row, or head-major) whose tile extent fits
  rp.q_ext = int64_t(num_qo_heads - 1) * q_stride_head + head_dim;
  rp.o_ext = int64_t(num_qo_heads - 1) * out_stride_head + head_dim;
  const int64_t q_span = (int64_t(rp.bm) - 1) * q_stride_token + rp.q_ext;
  const int64_t o_span = (int64_t(rp.bm) - 1) * out_stride_token + rp.o_ext;
  if (q_span > 0x3fffffff || o_span > 0x3fffffff)
    return mi::fail(MI_ERR_INVALID, "prefill run: q / out strides span %lld / %lld elements per tile (at most 2^30)",
                    (long long)q_span, (long long)o_span);
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf(float(head_dim));
  rp.scale_log2 = scale * mi::kLog2e;
  const dim3 g{static_cast<uint32_t>(grid), 1u, 1u};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((prefill_run_kernel<64, 2>), g, dim3(64 * waves_for(64)), 0, s, rp); break;
    case 128: hipLaunchKernelGGL((prefill_run_kernel<128, 3>), g, dim3(64 * waves_for(128)), 0, s, rp); break;
    default: hipLaunchKernelGGL((prefill_run_kernel<256, 1>), g, dim3(64 * waves_for(256)), 0, s, rp); break;
  }
  return mi::check_launch("prefill_run_kernel");
}
