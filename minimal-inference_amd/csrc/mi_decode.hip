// Split-K paged decode attention for gfx950.
//
// Reference: the decode wrapper's plan() (scheduler.py:402-413, 905-916,
// 927-938) and run() (model.py:235); the math is softmax(q K^T * scale) V over
// the request's kv_len tokens with KV head h / group for Q head h
// (model.py:286-295 restates it with repeat_interleave + SDPA).
//
// Work decomposition.  plan() (mi_decode_plan.h) cuts every request's page
// list into contiguous page ranges ("items"); items x kv_heads are the
// "units" of the run.  One 64-lane wave runs one unit and
// serves all `group` Q heads of its KV head, so each KV byte is read from HBM
// once per step; a workgroup of W waves (two for head_dim <= 128 and even
// kv_heads) runs W neighbouring KV heads of one item and loads their pages
// together, W * head_dim * 2 contiguous bytes per token row.
//
// Per 16-token page, one wave:
//   * loads its share of the workgroup's K and V rows through a per-page
//     buffer descriptor (size 0 for an invalid or absent page: the loads
//     return zeros and touch no memory), NB pages in flight, and stages them
//     in the LDS slot of the head they belong to (a barrier per page pair);
//   * S^T = K Q^T with 16x16x32 bf16 MFMAs (Q columns are the group's heads,
//     zero-padded to 16);
//   * online softmax in the exp2 domain with a lazy running max (rescale only
//     when the max grows by more than 2^8, so rescales are rare);
//   * O += P V with 16x16x32 bf16 MFMAs over two pages: the S^T accumulators
//     already are the P operand, V comes from the gfx950 LDS transpose read.
//
// Split merge without cache flushes.  Units of a request with several splits
// write (O, m, l) partials -- O rows as bf16 (the merged output is bf16
// anyway; bf16 rows halve the partial traffic), m and l as fp32 -- with
// device-coherent (sc1) 16-byte stores, wait for them, and bump a
// per-(request, KV head) counter; the unit that sees the count reach
// nsplit-1 reads the partials back (16 bytes per lane, eight splits per
// round trip -- sixteen at head_dim 64, whose next eight splits' rows load
// with the first eight), merges them, and resets the counter.  No agent-scope fence
// (and so no whole-L2 writeback / invalidate) is executed, and run() is one
// launch with no memset.
#include <math.h>

#include <mutex>

#include "mi_common.h"
#include "mi_decode_plan.h"

namespace {

using namespace mi::dplan;

constexpr float kLazyRescale = 8.0f;  // log2 units
// Pages in flight per wave: two for head_dim 128 (one page pair; four
// measured slower on every decode shape here since the workgroups load
// together), four for 64.
#ifndef MI_DECODE_NB128
#define MI_DECODE_NB128 2
#endif
#ifndef MI_DECODE_NB64
#define MI_DECODE_NB64 4
#endif
#ifndef MI_DECODE_WAVES
#define MI_DECODE_WAVES 2
#endif
#ifndef MI_DECODE_RS_PAD
#define MI_DECODE_RS_PAD 16
#endif
// s_waitcnt immediate (gfx9 encoding): vmcnt = 0, expcnt = 7, lgkmcnt = 15.
constexpr int kWaitVmcnt0 = 0x0F70;
// Buffer resource word 3 for gfx9 raw buffers (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer intrinsics: nt (non-temporal / streaming).
constexpr int kCacheNT = 2;

// ------------------------------------------------------------------ plan
// One workgroup: each request's page count, first page and last-page length
// are read once (into LDS when the batch fits one block), then the shared
// search and item writer (mi_decode_plan.h).
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanParams p) {
  __shared__ int s_np[kPlanThreads], s_pb0[kPlanThreads], s_lpl[kPlanThreads];
  __shared__ int red[2][kPlanThreads / 64];
  const int t = threadIdx.x;
  if (p.batch <= int(blockDim.x)) {
    if (t < p.batch) {
      const int pb0 = p.indptr[t], pb1 = p.indptr[t + 1], lpl = p.last_page_len[t];  // one round trip
      s_np[t] = max(0, pb1 - pb0);
      s_pb0[t] = pb0;
      s_lpl[t] = min(max(lpl, 1), kPageSize);
    }
    plan_from_lds(p, s_np, s_pb0, s_lpl);
    return;
  }
  const int lane = t & 63, w = t >> 6, nw = int(blockDim.x >> 6);
  int mx = 0, tot = 0;
  for (int b = t; b < p.batch; b += blockDim.x) {
    const int np = request_pages(p, b);
    mx = max(mx, np);
    tot += np;
  }
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
  const int q16 = plan_q16(p, s_np, false, max_np, total_np);
  plan_items(p, q16, false, s_np, s_pb0, s_lpl);
}

// ------------------------------------------------------------------ run
template <int D, int G>
struct DecodeTraits {
  static constexpr int KSTEPS = D / 32;  // 16x16x32 MFMAs for S^T = K Q^T
  static constexpr int NT = D / 16;      // 16-wide head_dim tiles for O += P V
  static constexpr int CPR = D / 8;      // 16-byte chunks per token row of one head
  static constexpr int LPI = CPR / 4;    // 16-byte loads per lane per page, for K and for V
  static constexpr int RS = D * 2 + MI_DECODE_RS_PAD;  // LDS row stride in bytes (the pad spreads the banks)
  static constexpr int SLOT = 4 * kPageSize * RS;  // two pages of K and V in LDS
  static constexpr int RX = 4 * D * 2;  // RoPE + append form: cos, sin, new K, new V rows of a wave
  // Pages in flight per wave (~128-160 registers of staging).
  static constexpr int NB = (D == 64) ? MI_DECODE_NB64 : (D == 128) ? MI_DECODE_NB128 : 2;
  static_assert(G >= 1 && G <= 16, "group size");
  static_assert((NB - 1) * 2 * LPI <= 63, "vmcnt range");
  static_assert(NB % 2 == 0, "pages are consumed in pairs");
};

struct RunParams {
  const DecodeHeader* header;
  const DecodeItem* items;
  int* counters;
  float* pml;    // per (unit, head): m, l
  uint16_t* po;  // per (unit, head): bf16 partial O row
  int pml_bytes, po_bytes;
  const uint16_t* q;  // q rows; with RoPE the fused qkv rows (q heads first)
  int64_t q_sb, q_sh;
  char* pool;  // written only by the RoPE + append form
  int64_t num_pages;
  const int32_t* indices;
  uint16_t* out;
  int64_t o_sb, o_sh;
  int hkv;
  int max_items;
  float scale_log2;
  // RoPE + append form: the cos / sin tables and the byte offset of K head 0
  // in a qkv row (V head 0 follows the K heads)
  const uint16_t* cos;
  const uint16_t* sin;
  int table_rows;
  int k_col_bytes;
};

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

template <int D, int G>
struct PageRegs {
  u32x4_t k[DecodeTraits<D, G>::LPI];
  u32x4_t v[DecodeTraits<D, G>::LPI];
};

template <typename F>
__device__ __forceinline__ F coherent_load(const F* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename F>
__device__ __forceinline__ void coherent_store(F* p, F v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((address_space(3))) char lds_t;

__device__ __forceinline__ void lds_store16(lds_t* p, u32x4_t v) {
  *(__attribute__((address_space(3))) u32x4_t*)p = v;
}
__device__ __forceinline__ u32x4_t lds_load16(const lds_t* p) {
  return *(const __attribute__((address_space(3))) u32x4_t*)p;
}
// gfx950 LDS transpose read: the 16 lanes of a group address 4 rows x 16
// bf16 (lane j: row j/4, elements 4*(j%4)..+3) and lane j receives column j.
__device__ __forceinline__ s16x4_t lds_read_tr16(const lds_t* p) {
  typedef __attribute__((address_space(3))) bf16x4_t lds_v4;
  return __builtin_bit_cast(s16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4*)p));
}

typedef __attribute__((ext_vector_type(4))) float f32x4_v;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_v;
typedef __attribute__((ext_vector_type(8))) float f32x8_v;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_v;
typedef __attribute__((ext_vector_type(8))) short s16x8_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_v;

// Max / sum of x and its value in lane ^ 16 (resp. lane ^ 32), with the
// gfx950 lane-swap instructions: swapping x with itself leaves x in one
// result and the partner's x in the other, for every lane.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Wave-wide max / sum, every lane gets the result (no LDS traffic).
__device__ __forceinline__ float wave_max_fast(float x) { return max_xor32(max_xor16(mi::group16_max(x))); }
__device__ __forceinline__ float wave_sum_fast(float x) { return sum_xor32(sum_xor16(mi::group16_sum(x))); }

// Word (lane & 31) of the item of unit u.  The index is clamped to the item
// array, so the read is in bounds even before the unit count is known.
__device__ __forceinline__ int load_item_word(const RunParams& p, int u) {
  const int idx = min(u / p.hkv, p.max_items - 1);
  return reinterpret_cast<const int*>(p.items + idx)[threadIdx.x & 31];
}

// Max / sum over each aligned group of LR lanes (8, 16 or 32); every lane
// gets the result.
template <int LR>
__device__ __forceinline__ float group_max(float x) {
  static_assert(LR == 8 || LR == 16 || LR == 32, "group width");
  x = fmaxf(x, mi::dpp<mi::kDppQuadSwap1>(x));
  x = fmaxf(x, mi::dpp<mi::kDppQuadSwap2>(x));
  x = fmaxf(x, mi::dpp<mi::kDppRowHalfMirror>(x));
  if constexpr (LR >= 16) x = fmaxf(x, mi::dpp<mi::kDppRowMirror>(x));
  if constexpr (LR >= 32) x = max_xor16(x);
  return x;
}
template <int LR>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(LR == 8 || LR == 16 || LR == 32, "group width");
  x += mi::dpp<mi::kDppQuadSwap1>(x);
  x += mi::dpp<mi::kDppQuadSwap2>(x);
  x += mi::dpp<mi::kDppRowHalfMirror>(x);
  if constexpr (LR >= 16) x += mi::dpp<mi::kDppRowMirror>(x);
  if constexpr (LR >= 32) x = sum_xor16(x);
  return x;
}

// Split-K tail of a unit: publish the partial (O rows, m, l), count, and
// the last unit of the (request, KV head) merges all splits.  Partials are
// written and read device-coherent (sc1: through to the memory side, so
// splits on other XCDs see them; keeping them in one XCD's L2 when all
// splits of a request share an XCD measured no faster).
//
// Partial O rows are bf16 in "lane order": position j * NT + t of a head's
// row holds dim 16 t + j, which is what lane (g, j) of the MFMA accumulators
// holds for head 4 g + i, so a lane publishes a head with one contiguous
// store of NT values.  The merge reads rows back 16 bytes per lane: one load
// covers R = 1024 / (2 D) rows, lane l taking row l / LR (a head) and 16-byte
// chunk l % LR; the splits' m and l are laid out the same way (lane l: head
// l / LR of a row group, split l % LR of a split group), so the weight of
// split s for a lane's head is a shuffle inside its LR-lane group.
template <int D, int G>
__device__ __forceinline__ void publish_merge(const RunParams& p, int u, int b, int hkv, int nsplit, int item_base,
                                              const mi::f32x4_t (&acc)[DecodeTraits<D, G>::NT], float m_run,
                                              float lt) {
  using T = DecodeTraits<D, G>;
  constexpr int NT = T::NT;
  constexpr int CP = 16;  // cache policy: sc1 (device scope)
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, j = lane & 15;
  const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(p.po, (short)0, p.po_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(p.pml, (short)0, p.pml_bytes, kBufferWord3);
  {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < G) {
        uint32_t w[NT / 2];
#pragma unroll
        for (int t = 0; t < NT / 2; ++t) w[t] = mi::cvt_pk_bf16(acc[2 * t][i], acc[2 * t + 1][i]);
        const int off = (u * G + h) * D * 2 + j * NT * 2;
        if constexpr (NT == 4) {
          __builtin_amdgcn_raw_buffer_store_b64((__attribute__((ext_vector_type(2))) unsigned int){w[0], w[1]}, rpo, off, 0, CP);
        } else {
#pragma unroll
          for (int q = 0; q < NT / 8; ++q)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]}, rpo,
                                                   off + 16 * q, 0, CP);
        }
      }
    }
    if (lane < G)  // lane h holds m_run / lt of head h
      __builtin_amdgcn_raw_buffer_store_b64(
          (__attribute__((ext_vector_type(2))) unsigned int){__float_as_uint(m_run), __float_as_uint(lt)}, rml,
          (u * G + lane) * 8, 0, CP);
  }
  // Wait until this wave's stores are acknowledged (vmcnt 0; expcnt /
  // lgkmcnt left free), so they are visible before the counter moves.  The
  // fence keeps the compiler from reordering around it.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  int prev = 0;
  int* counter = p.counters + (b * p.hkv + hkv) * kCounterStride;
  if (lane == 0) prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = mi::read_lane_i(prev, 0);
  if (prev != nsplit - 1) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  constexpr int R = 1024 / (2 * D);   // rows per 16-byte load: 4 (D 128), 8 (D 64), 2 (D 256)
  constexpr int LR = 64 / R;          // lanes per row
  constexpr int A = (G + R - 1) / R;  // row groups covering the G heads
  constexpr int C = 64 / LR;          // split groups per round of 64 splits
  constexpr int KB = 8;  // splits whose rows are loaded together (16 measured slower)
  static_assert(LR % KB == 0, "batches inside a split group");
  const int hg = lane / LR, sg = lane % LR;
  float M[A], Lt[A], sum[A][8];
#pragma unroll
  for (int a = 0; a < A; ++a) {
    M[a] = -INFINITY;
    Lt[a] = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sum[a][k] = 0.f;
  }
  auto unit_of = [&](int s) { return (item_base + s) * p.hkv + hkv; };
  auto load_batch = [&](u32x4_t (&v)[KB][A], int s0, int nr) {
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const int us = unit_of(min(s0 + q, nr - 1));
#pragma unroll
      for (int a = 0; a < A; ++a) {
        const int h = min(a * R + hg, G - 1);
        v[q][a] = __builtin_amdgcn_raw_buffer_load_b128(rpo, (us * G + h) * D * 2 + sg * 16, 0, CP);
      }
    }
  };
  for (int r0 = 0; r0 < nsplit; r0 += 64) {
    const int nr = min(64, nsplit - r0);
    // (m, l) of split c LR + sg, head a R + hg; the first rows load with them
    typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
    u32x2_t ml[A][C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int us = unit_of(r0 + min(c * LR + sg, nr - 1));
#pragma unroll
      for (int a = 0; a < A; ++a)
        ml[a][c] = __builtin_amdgcn_raw_buffer_load_b64(rml, (us * G + min(a * R + hg, G - 1)) * 8, 0, CP);
    }
    // With one batch per split group (LR == KB: head_dim 64), the next
    // group's rows are loaded with this group's, so a merge of up to 2 KB
    // splits takes one round trip and longer ones overlap each batch's loads
    // with the previous batch's arithmetic.
    constexpr bool PF = (LR == KB);
    u32x4_t v[KB][A], v2[PF ? KB : 1][A];
    load_batch(v, r0, r0 + nr);
    if constexpr (PF) load_batch(v2, r0 + LR, r0 + nr);  // clamped: in bounds when the group is absent
    float wgt[A][C];
#pragma unroll
    for (int a = 0; a < A; ++a) {
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (c * LR + sg < nr) mx = fmaxf(mx, __uint_as_float(ml[a][c].x));
      const float Mn = fmaxf(M[a], group_max<LR>(mx));
      const float f = (M[a] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M[a] - Mn);
      Lt[a] *= f;
#pragma unroll
      for (int k = 0; k < 8; ++k) sum[a][k] *= f;
      float ls = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const float ms = __uint_as_float(ml[a][c].x);
        wgt[a][c] = (c * LR + sg < nr && ms != -INFINITY) ? __builtin_amdgcn_exp2f(ms - Mn) : 0.f;
        ls += wgt[a][c] * __uint_as_float(ml[a][c].y);
      }
      Lt[a] += group_sum<LR>(ls);
      M[a] = Mn;
    }
    if constexpr (PF) {
      // the weights of split group c (a select chain: no indexed array)
      struct W { float w[A]; };
      auto group_w = [&](int c) {
        W x;
#pragma unroll
        for (int a = 0; a < A; ++a) {
          x.w[a] = wgt[a][0];
#pragma unroll
          for (int cc = 1; cc < C; ++cc) x.w[a] = (c == cc) ? wgt[a][cc] : x.w[a];
        }
        return x;
      };
      // rows of the KB splits from c LR + q0 on, held in vv, weighted by wc
      auto accum = [&](const u32x4_t (&vv)[KB][A], const W wc_, int c, int q0) {
        const float* wc = wc_.w;
        const int s0 = c * LR + q0;
#pragma unroll
        for (int q = 0; q < KB; ++q) {
          if (s0 + q >= nr) break;
#pragma unroll
          for (int a = 0; a < A; ++a) {
            const float w = mi::lane_shuffle(wc[a], hg * LR + q0 + q);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              sum[a][2 * k] += w * mi::bf16_lo(vv[q][a][k]);
              sum[a][2 * k + 1] += w * mi::bf16_hi(vv[q][a][k]);
            }
          }
        }
      };
      // unrolled: a runtime group index made the compiler turn the weight
      // select into an indexed stack array
#pragma unroll
      for (int c = 0; c < C; c += 2) {
        if (c * LR >= nr) break;
        accum(v, group_w(c), c, 0);
        if ((c + 2) * LR < nr) load_batch(v, r0 + (c + 2) * LR, r0 + nr);
        if ((c + 1) * LR >= nr) break;
        accum(v2, group_w(c + 1), c + 1, 0);
        if ((c + 3) * LR < nr) load_batch(v2, r0 + (c + 3) * LR, r0 + nr);
      }
    } else {
#pragma nounroll
      for (int c = 0; c < C; ++c) {
        if (c * LR >= nr) break;
        float wc[A];
#pragma unroll
        for (int a = 0; a < A; ++a) {
          wc[a] = wgt[a][0];
#pragma unroll
          for (int cc = 1; cc < C; ++cc) wc[a] = (c == cc) ? wgt[a][cc] : wc[a];
        }
#pragma unroll
        for (int q0 = 0; q0 < LR; q0 += KB) {
          const int s0 = c * LR + q0;
          if (s0 >= nr) break;
          if (s0 > 0) load_batch(v, r0 + s0, r0 + nr);
#pragma unroll
          for (int q = 0; q < KB; ++q) {
            if (s0 + q >= nr) break;
#pragma unroll
            for (int a = 0; a < A; ++a) {
              const float w = mi::lane_shuffle(wc[a], hg * LR + q0 + q);
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                sum[a][2 * k] += w * mi::bf16_lo(v[q][a][k]);
                sum[a][2 * k + 1] += w * mi::bf16_hi(v[q][a][k]);
              }
            }
          }
        }
      }
    }
  }
  // lane (hg, sg) holds row positions 8 sg .. 8 sg + 7 of head a R + hg
#pragma unroll
  for (int a = 0; a < A; ++a) {
    const int h = a * R + hg;
    if (h < G) {
      const float inv = Lt[a] > 0.f ? mi::fast_rcp(Lt[a]) : 0.f;
      uint16_t* orow = p.out + int64_t(b) * p.o_sb + int64_t(hkv * G + h) * p.o_sh;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int pos = sg * 8 + k;
        orow[16 * (pos % NT) + pos / NT] = mi::cvt_bf16(sum[a][k] * inv);
      }
    }
  }
  if (lane == 0) coherent_store(counter, 0);
}

// One unit: (item, KV head).  Lane l of the wave is (g, j) = (l >> 4, l & 15).
//
//   page loads : raw buffer loads through a per-page descriptor (base = the
//                page, size = the page, or size 0 for a missing / invalid
//                page, whose loads then return zeros without touching
//                memory); 128 contiguous bytes per token row per instruction
//                (8 lanes per row, 8 rows per instruction); NB pages in
//                flight in registers, issued NB pages ahead of use;
//   LDS slot   : the page's K and V rows of this head, row-major with padding;
//   S^T = K Q^T: 16x16x32 MFMAs; lane (g, j) reads K row j, d-chunk g + 4s
//                from LDS (its A operand) and holds Q row j (head j) as B;
//                it receives S^T[token 4g+i][head j];
//   softmax    : per head j, lazy running max in the exp2 domain;
//   O += P V   : 16x16x16 MFMAs; P[head j][token 4g+i] is exactly the S^T
//                accumulator each lane already holds, and V comes from the
//                LDS transpose read (lane (g, j) gets V[4g..4g+3][16t + j]);
//                O[head 4g+i][16t + j] accumulates in registers.
//
// With ROPE (mi_decode_rope_append_run) the q rows are the fused qkv rows:
// every unit rotates its q heads with the request's cos / sin row, and the
// unit holding the request's last page (the last split) also rotates its KV
// head's new K row, takes the V row, stages both in LDS in place of the
// pool's stale slot and writes them to the slot -- the decode step's RoPE
// (model.py:169-170) and append (model.py:203-216) done by the attention
// launch (model.py:235) with the same bf16 arithmetic as rope_append_kernel.
template <int D, int G, int W, int S, int NB, bool ROPE>
__device__ __forceinline__ void decode_unit(const RunParams& p, int u, int iv, lds_t* wg_lds, lds_t* rx) {
  using T = DecodeTraits<D, G>;
  using Regs = PageRegs<D, G>;
  static_assert((NB - 1) * 2 * T::LPI <= 63 && NB % 2 == 0, "vmcnt range; pages are consumed in pairs");
  const int lane = threadIdx.x & 63;
  const int hkv = u - (u / p.hkv) * p.hkv;
  const int b = mi::read_lane_i(iv, kItemB);
  const int page_begin = mi::read_lane_i(iv, kItemBegin);
  const int npg = mi::read_lane_i(iv, kItemEnd) - page_begin;
  const int last_valid = mi::read_lane_i(iv, kItemLast);
  const int nsplit = mi::read_lane_i(iv, kItemNsplit);
  const int item_base = mi::read_lane_i(iv, kItemBase);
  if (nsplit == 0) return;  // a padding item (the same for every wave of the workgroup)
  const int g = lane >> 4, j = lane & 15;

  // Q^T as the B operand: column j = head j of the group (zero when j >= G:
  // those lanes read out of the descriptor's range, which returns zeros, so
  // the loads are unconditional and nothing waits on them early).
  mi::bf16x8_t qb[T::KSTEPS];
  {
    const uint16_t* q0 = p.q + int64_t(b) * p.q_sb + int64_t(hkv * G) * p.q_sh;
    const int q_bytes = int((G - 1) * p.q_sh * 2) + D * 2;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)q0, (short)0, q_bytes, kBufferWord3);
    const int qoff = (j < G) ? int(j * p.q_sh * 2) + g * 16 : 0x7ffffff0;
#pragma unroll
    for (int s = 0; s < T::KSTEPS; ++s)
      qb[s] = __builtin_bit_cast(mi::bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, s * 64, 0));
  }
  // RoPE + append: the loads go out with Q's, before the page loads, and are
  // used after the first pages are issued.  Lane l < D/8 loads chunk l of
  // the cos row, the next D/8 lanes the sin row, for the wave's LDS copy
  // (`rx`: cos, sin, new K, new V rows), from which the rotations read; the
  // q chunks of lane (g, j) are g + 4 s, whose RoPE partners (d + D/2) are
  // chunks s + KSTEPS / 2 of the same lane.  The new K row rotates in units
  // of 8 pairs (d, d + D/2): lane l < D/16 takes d = 8 l + [0, 8); lanes 32 ..
  // 32 + D/8 - 1 carry the V chunks.  Only the last split of a request
  // appends (its rows load through a size-0 descriptor otherwise); lanes
  // without a part read out of range.
  constexpr int RK = D / 16, VC = D / 8;
  const int split = u / p.hkv - item_base;
  const bool appender = ROPE && split == nsplit - 1 && npg > 0;
  u32x4_t c_v, s_v, k_lo, k_hi, v_new;
  int new_page = -1;
  if constexpr (ROPE) {
    // the decode position kv_len - 1 is the RoPE row: no load on the way
    const int rp = min(max(mi::read_lane_i(iv, kItemKvLen) - 1, 0), p.table_rows - 1);
    // one descriptor per table (a per-lane table pointer would make the
    // descriptor divergent); lanes outside a table's range read zeros
    const bool is_cos = lane < VC, is_sin = lane >= VC && lane < 2 * VC;
    const __amdgpu_buffer_rsrc_t rcos =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.cos + int64_t(rp) * D), (short)0, D * 2, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rsin =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.sin + int64_t(rp) * D), (short)0, D * 2, kBufferWord3);
    c_v = __builtin_amdgcn_raw_buffer_load_b128(rcos, is_cos ? 16 * lane : 0x7ffffff0, 0, 0);
    s_v = __builtin_amdgcn_raw_buffer_load_b128(rsin, is_sin ? 16 * (lane - VC) : 0x7ffffff0, 0, 0);
    // this head's K row and V row in the qkv row (V heads follow the K heads)
    const char* krow = reinterpret_cast<const char*>(p.q + int64_t(b) * p.q_sb) + p.k_col_bytes + hkv * D * 2;
    const __amdgpu_buffer_rsrc_t rkv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)krow, (short)0, appender ? (p.hkv + 1) * D * 2 : 0, kBufferWord3);
    const int ko = lane < RK ? 16 * lane : 0x7ffffff0;
    k_lo = __builtin_amdgcn_raw_buffer_load_b128(rkv, ko, 0, 0);
    k_hi = __builtin_amdgcn_raw_buffer_load_b128(rkv, ko, D, 0);
    const int vo = (lane >= 32 && lane < 32 + VC) ? p.hkv * D * 2 + 16 * (lane - 32) : 0x7ffffff0;
    v_new = __builtin_amdgcn_raw_buffer_load_b128(rkv, vo, 0, 0);
  }

  // The W waves of a workgroup run heads h0 .. h0 + W - 1 of one item and
  // load its pages together: wave w loads token rows [w RPW, (w + 1) RPW) of
  // all W heads -- W * D * 2 contiguous bytes per row, which streams
  // measurably faster than one head's D * 2 -- and every lane stages its 16
  // bytes into the LDS slot of the head they belong to.  Byte offsets inside
  // a page: lane part (voffset), instruction part (soffset).
  constexpr int SW = W * D * 2, LPR = SW / 16, RPI = 64 / LPR, RPW = kPageSize / W;
  static_assert(SW <= 1024 && RPW == RPI * T::LPI, "load layout");
  const int tok_bytes = p.hkv * D * 2;
  const int kv_bytes = kPageSize * tok_bytes;
  const int page_bytes = 2 * kv_bytes;
  // wave wv of the workgroup: head w of its W heads, lane group sg of S
  const int wv = (W * S == 1) ? 0 : __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int w = wv % W, sg = wv / W;
  const int row0 = w * RPW;
  const int lrow = lane / LPR, lbyte = (lane % LPR) * 16;
  const int lhead = lbyte / (D * 2), lchunk = (lbyte % (D * 2)) / 16;
  const int voff = lrow * tok_bytes + (hkv - w) * D * 2 + lbyte;
  lds_t* const lds = wg_lds + (sg * W + w) * T::SLOT;  // this wave's head
  lds_t* const stage_lds = wg_lds + (sg * W + lhead) * T::SLOT;  // the head of this lane's loaded bytes

  int pidv = iv;  // page ids of the current group, lane k = page k of the group

  auto page_id = [&](int k) { return __builtin_amdgcn_readlane(pidv, k & 63); };
  auto page_ok = [&](int k, int pg, int gsize) { return k < gsize && pg >= 0 && pg < p.num_pages; };
  // With S > 1 lane groups, a unit's pages are dealt to them pair by pair:
  // page k of lane group sg's sequence is page act(k) of the id group, and
  // all groups walk sequences of the same length vsize(gsize) (a missing
  // pair loads through a size-0 descriptor and is masked), so every wave of
  // the workgroup reaches the same barriers.
  auto act = [&](int k) { return S == 1 ? k : 2 * S * (k >> 1) + 2 * sg + (k & 1); };
  auto vsize = [&](int gs) { return S == 1 ? gs : 2 * (((gs + 1) / 2 + S - 1) / S); };
  auto issue = [&](Regs& r, int k, int gsize) {
    const int a = act(k);
    const int pg = page_id(a);
    const bool ok = page_ok(a, pg, gsize);
    const char* base = ok ? p.pool + int64_t(pg) * page_bytes : p.pool;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, ok ? page_bytes : 0, kBufferWord3);
    // K / V are read once per launch: non-temporal loads (nt) keep them from
    // evicting what is reused from L2 -- the work items, Q and the split
    // partials (Mistral-7B B=32: 20.6 -> 19.4 us; Qwen2.5-7B B=48: 29.1 ->
    // 26.9 us; Qwen2.5-72B B=48: 60.7 -> 57.5 us)
#pragma unroll
    for (int i = 0; i < T::LPI; ++i) {
      const int so = (row0 + i * RPI) * tok_bytes;
      r.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, so, kCacheNT);
      r.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, so + kv_bytes, kCacheNT);
    }
  };

  mi::f32x4_t acc[T::NT];
#pragma unroll
  for (int t = 0; t < T::NT; ++t) acc[t] = mi::f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // head j
  float l_run = 0.f;        // head j, this lane's tokens

  // LDS slots: page a of a pair at [0, 2 pages), page b after it
  auto k_slot = [&](int which) { return lds + which * 2 * kPageSize * T::RS; };
  auto v_slot = [&](int which) { return lds + which * 2 * kPageSize * T::RS + kPageSize * T::RS; };

  // Two pages (32 tokens) per step: one softmax update, and O += P V as
  // 16x16x32 MFMAs whose A operand is the pair of S^T accumulators (lane
  // (g, j) holds tokens 4g+i of both pages) and whose B operand is the two
  // pages' transpose reads in the same token order.
  auto stage = [&](const Regs& r, int valid, int which) {
    // this wave's rows of the page to LDS (V rows past `valid` as zeros on a
    // partial page: P is 0 there, but 0 * NaN would poison the MFMA)
    lds_t* kl = stage_lds + which * 2 * kPageSize * T::RS + lrow * T::RS + lchunk * 16;
    lds_t* vl = kl + kPageSize * T::RS;
#pragma unroll
    for (int i = 0; i < T::LPI; ++i) lds_store16(kl + (row0 + i * RPI) * T::RS, r.k[i]);
    if (valid == kPageSize) {
#pragma unroll
      for (int i = 0; i < T::LPI; ++i) lds_store16(vl + (row0 + i * RPI) * T::RS, r.v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < T::LPI; ++i) {
        const int row = row0 + i * RPI + lrow;
        lds_store16(vl + (row0 + i * RPI) * T::RS, (row < valid) ? r.v[i] : u32x4_t{0, 0, 0, 0});
      }
    }
  };
  // RoPE + append form, at the first page pair: the cos / sin rows go to
  // `rx`, the q heads rotate in place, and this head's new K row (rotated)
  // and V row go to `rx`; the new row later overwrites the pool's stale row
  // in the staging slot of its page, and is written to the pool at the end
  auto rotate = [&]() {
    if constexpr (ROPE) {
      // cos row, then sin row.  The load registers are loop-invariant: the
      // opaque step keeps the compiler from merging them (a select) before
      // the first page loads, which would wait for these loads there.
      __asm__ volatile("" : "+v"(c_v), "+v"(s_v));
      if (lane < 2 * VC) lds_store16(rx + 16 * lane, lane < VC ? c_v : s_v);
      const lds_t* cr = rx;
      const lds_t* sr = rx + D * 2;
#pragma unroll
      for (int s = 0; s < T::KSTEPS / 2; ++s) {
        const int c1 = (g + 4 * s) * 16, c2 = (g + 4 * (s + T::KSTEPS / 2)) * 16;
        uint4 o1, o2;
        mi::rope8(__builtin_bit_cast(uint4, qb[s]), __builtin_bit_cast(uint4, qb[s + T::KSTEPS / 2]),
                  __builtin_bit_cast(uint4, lds_load16(cr + c1)), __builtin_bit_cast(uint4, lds_load16(sr + c1)),
                  __builtin_bit_cast(uint4, lds_load16(cr + c2)), __builtin_bit_cast(uint4, lds_load16(sr + c2)),
                  o1, o2);
        qb[s] = __builtin_bit_cast(mi::bf16x8_t, o1);
        qb[s + T::KSTEPS / 2] = __builtin_bit_cast(mi::bf16x8_t, o2);
      }
      if (appender) {
        // k_lo / k_hi likewise: without the opaque step the compiler hoisted
        // their bf16 unpacking above the first page loads, and every wave
        // then waited for its Q, cos / sin and new-row loads before issuing a
        // page (Mistral-7B B=32 fused launch +0.8 us)
        __asm__ volatile("" : "+v"(k_lo), "+v"(k_hi));
        if (lane < RK) {
          uint4 o1, o2;
          mi::rope8(__builtin_bit_cast(uint4, k_lo), __builtin_bit_cast(uint4, k_hi),
                    __builtin_bit_cast(uint4, lds_load16(cr + 16 * lane)),
                    __builtin_bit_cast(uint4, lds_load16(sr + 16 * lane)),
                    __builtin_bit_cast(uint4, lds_load16(cr + D + 16 * lane)),
                    __builtin_bit_cast(uint4, lds_load16(sr + D + 16 * lane)), o1, o2);
          lds_store16(rx + 4 * D + 16 * lane, __builtin_bit_cast(u32x4_t, o1));
          lds_store16(rx + 5 * D + 16 * lane, __builtin_bit_cast(u32x4_t, o2));
        }
        if (lane >= 32 && lane < 32 + VC) lds_store16(rx + 6 * D + 16 * (lane - 32), v_new);
      }
    }
  };
  // the new K / V row into row `row` of staging slot `which` of this head
  auto inject = [&](int which, int row) {
    if constexpr (ROPE) {
      lds_t* kl = lds + which * 2 * kPageSize * T::RS + row * T::RS;
      if (lane < VC) lds_store16(kl + 16 * lane, lds_load16(rx + 4 * D + 16 * lane));
      if (lane >= 32 && lane < 32 + VC)
        lds_store16(kl + kPageSize * T::RS + 16 * (lane - 32), lds_load16(rx + 6 * D + 16 * (lane - 32)));
    }
  };
  // the workgroup's waves exchange staged rows: LDS writes done, then a
  // barrier (no wait on the page loads in flight)
  auto wg_sync = [&]() {
    if constexpr (W > 1) __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  auto scores = [&](int which, int valid, float (&sv)[4]) {
    const lds_t* kl = k_slot(which);
    mi::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < T::KSTEPS; ++s)
      c = mi::mfma_16x16x32_bf16(__builtin_bit_cast(mi::bf16x8_t, lds_load16(kl + j * T::RS + (g + 4 * s) * 16)),
                                 qb[s], c);
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = (4 * g + i < valid) ? c[i] * p.scale_log2 : -INFINITY;
  };
  // `next` reloads the two staging register sets with the next pages as
  // soon as their rows are in LDS, so the loads of the next pair are in
  // flight while this pair is consumed (Qwen2.5-7B B=48: 25.4 -> 24.8 us,
  // Qwen2.5-72B: 69.7 -> 68.9 us; Mistral-7B B=32 unchanged).
  // `inj` (RoPE + append form): the slot (0 / 1) whose page holds the new
  // token, or -1.  The injection follows the barrier, so it overwrites
  // whatever any wave staged into that row; a wave reads only its own
  // head's slot, so no second barrier is needed.
  bool rot_pending = ROPE;
  auto consume2 = [&](Regs& ra, int va, Regs& rb, int vb, int inj, auto&& next) {
    stage(ra, va, 0);
    stage(rb, vb, 1);
    // the RoPE rotations at the first pair, once its staging registers are
    // free (before that, the pages in flight leave no room: 217 -> 256 VGPRs
    // and spills with group 5..8)
    if (ROPE && rot_pending) {
      rotate();
      rot_pending = false;
    }
    next(ra, rb);
    wg_sync();
    if (ROPE && inj >= 0) inject(inj, last_valid - 1);
    float sa[4], sb[4];
    scores(0, va, sa);
    scores(1, vb, sb);
    // ---- online softmax for head j, lazy rescale
    float mloc = fmaxf(fmaxf(fmaxf(sa[0], sa[1]), fmaxf(sa[2], sa[3])), fmaxf(fmaxf(sb[0], sb[1]), fmaxf(sb[2], sb[3])));
    mloc = max_xor16(mloc);
    mloc = max_xor32(mloc);
    const bool need = mloc > m_run + kLazyRescale;
    if (__builtin_amdgcn_ballot_w64(need)) {
      // a head that has seen no token yet (m_run = -inf) still has O = 0 and
      // l = 0: only its max moves, nothing is rescaled
      const bool scale = need && m_run != -INFINITY;
      const float f = scale ? __builtin_amdgcn_exp2f(m_run - mloc) : 1.f;
      m_run = need ? mloc : m_run;
      l_run *= f;
      if (__builtin_amdgcn_ballot_w64(scale)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float fo = mi::lane_shuffle(f, 4 * g + i);
#pragma unroll
          for (int t = 0; t < T::NT; ++t) acc[t][i] *= fo;
        }
      }
    }
    // exp2(-inf - m) = 0 for masked tokens; m is taken as 0 while no token
    // of the head has been seen (m_run still -inf), avoiding -inf - -inf
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    float pv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(sa[i] - m_use);
      pv[4 + i] = __builtin_amdgcn_exp2f(sb[i] - m_use);
    }
    l_run += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
    const mi::bf16x8_t pa = __builtin_bit_cast(
        mi::bf16x8_t,
        __builtin_convertvector((f32x8_v){pv[0], pv[1], pv[2], pv[3], pv[4], pv[5], pv[6], pv[7]}, bf16x8_v));
    // ---- O += P V
    const lds_t* va_row = v_slot(0) + (4 * g + (j >> 2)) * T::RS + (j & 3) * 8;
    const lds_t* vb_row = v_slot(1) + (4 * g + (j >> 2)) * T::RS + (j & 3) * 8;
#pragma unroll
    for (int t = 0; t < T::NT; ++t) {
      const s16x4_t x = lds_read_tr16(va_row + 32 * t), y = lds_read_tr16(vb_row + 32 * t);
      const mi::bf16x8_t vbop = __builtin_bit_cast(mi::bf16x8_t, (s16x8_t){x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]});
      acc[t] = mi::mfma_16x16x32_bf16(pa, vbop, acc[t]);
    }
    wg_sync();  // every wave is done reading the slots before they are restaged
  };

  // ---- stream the pages: groups of page ids (the item's inline copy first,
  // then 64 at a time from kv_indices), NB pages in flight.  Every load is
  // unconditional -- past the group's end it goes through a size-0
  // descriptor -- and the only branches around code are VMEM-free (the tail
  // consumes), so the compiler's wait before consuming a page is exactly
  // "NB-1 pages still outstanding".
  Regs buf[NB];
  int g_start = 0, gsize = min(npg, kInlinePages);
  while (true) {
#pragma unroll
    for (int s = 0; s < NB; ++s) issue(buf[s], s, gsize);
    auto page_valid = [&](int k) {
      const int a = act(k);
      const int valid = (g_start + a == npg - 1) ? last_valid : kPageSize;
      return page_ok(a, page_id(a), gsize) ? valid : 0;
    };
    // the slot of the pair (k, k + 1) that holds the new token, for its appender
    auto inj_slot = [&](int k) {
      return !appender ? -1 : g_start + act(k) == npg - 1 ? 0 : g_start + act(k + 1) == npg - 1 ? 1 : -1;
    };
    const int vs = vsize(gsize);
    const int full = vs / NB;
    for (int it = 0; it < full; ++it) {
#pragma unroll
      for (int s = 0; s < NB; s += 2) {
        const int k = it * NB + s;
        consume2(buf[s], page_valid(k), buf[s + 1], page_valid(k + 1), inj_slot(k), [&](Regs& x, Regs& y) {
                   issue(x, k + NB, gsize);
                   issue(y, k + 1 + NB, gsize);
                 });
      }
    }
    // the last rem (< NB) pages; a pair's second page past the group's end
    // was loaded through a size-0 descriptor (zeros) and is fully masked
    const int rem = vs - full * NB;
#pragma unroll
    for (int s = 0; s < NB - 1; s += 2)
      if (s < rem) consume2(buf[s], page_valid(full * NB + s), buf[s + 1],
                            s + 1 < rem ? page_valid(full * NB + s + 1) : 0, inj_slot(full * NB + s),
                            [](Regs&, Regs&) {});
    if (ROPE && g_start + gsize >= npg) new_page = page_id(npg - 1 - g_start);  // the last group
    g_start += gsize;
    if (g_start >= npg) break;
    gsize = min(64, npg - g_start);
    pidv = (lane < gsize) ? p.indices[page_begin + g_start + lane] : -1;
    // Wait here, while only size-0 loads are outstanding, so the loop head
    // carries no pending load (the first group's Q loads stay in flight).
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }

  // ---- the append: the new K / V row from `rx` to its slot, one 16-byte
  // chunk per lane (a page id outside the pool writes nothing)
  if constexpr (ROPE) {
    if (appender && sg == 0) {
      const bool ok = new_page >= 0 && new_page < p.num_pages;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(ok ? p.pool + int64_t(new_page) * page_bytes : p.pool), (short)0, ok ? page_bytes : 0,
          kBufferWord3);
      const int row_off = (last_valid - 1) * tok_bytes + hkv * D * 2;
      const bool kl = lane < VC, vl = lane >= 32 && lane < 32 + VC;
      const int c = kl ? lane : lane - 32;
      const u32x4_t x = lds_load16(rx + (kl ? 4 * D : 6 * D) + 16 * (c & (VC - 1)));
      __builtin_amdgcn_raw_buffer_store_b128(x, rs, kl ? row_off + 16 * c : vl ? kv_bytes + row_off + 16 * c : 0x7ffffff0,
                                             0, 0);
    }
  }

  // ---- lane groups 1 .. S-1 hand their state (O accumulators, m, l) to
  // lane group 0 through their own LDS slots, free after the last step's
  // barrier; the second barrier keeps the slots from being restaged before
  // group 0 has read them
  if constexpr (S > 1) {
    static_assert(T::NT * 1024 + 512 <= T::SLOT, "hand-off fits the slot");
    if (sg > 0) {
      lds_t* const xs = wg_lds + (sg * W + w) * T::SLOT;
#pragma unroll
      for (int t = 0; t < T::NT; ++t) lds_store16(xs + (t * 64 + lane) * 16, __builtin_bit_cast(u32x4_t, acc[t]));
      *(__attribute__((address_space(3))) f32x2_v*)(xs + T::NT * 1024 + lane * 8) = f32x2_v{m_run, l_run};
    }
    __syncthreads();  // every wave of the workgroup, whatever W
    if (sg == 0) {
#pragma unroll
      for (int o = 1; o < S; ++o) {
        const lds_t* const xs = wg_lds + (o * W + w) * T::SLOT;
        mi::f32x4_t acc1[T::NT];
#pragma unroll
        for (int t = 0; t < T::NT; ++t) acc1[t] = __builtin_bit_cast(mi::f32x4_t, lds_load16(xs + (t * 64 + lane) * 16));
        const f32x2_v ml1 = *(const __attribute__((address_space(3))) f32x2_v*)(xs + T::NT * 1024 + lane * 8);
        // m of head j (the same in every lane of head j); a group that saw
        // no token has m = -inf, O = 0, l = 0 and weight 0
        const float mm = fmaxf(m_run, ml1.x);
        const float f0 = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - mm);
        const float f1 = (ml1.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ml1.x - mm);
        l_run = l_run * f0 + ml1.y * f1;
        m_run = mm;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a0 = mi::lane_shuffle(f0, 4 * g + i), a1 = mi::lane_shuffle(f1, 4 * g + i);
#pragma unroll
          for (int t = 0; t < T::NT; ++t) acc[t][i] = acc[t][i] * a0 + acc1[t][i] * a1;
        }
      }
    }
    __syncthreads();
    if (sg > 0) return;
  }

  // ---- per-head denominators; O rows are heads 4g + i
  float lt = sum_xor16(l_run);
  lt = sum_xor32(lt);
  float lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lo[i] = mi::lane_shuffle(lt, 4 * g + i);

  if (nsplit == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < G) {
        const float inv = lo[i] > 0.f ? mi::fast_rcp(lo[i]) : 0.f;
        uint16_t* orow = p.out + int64_t(b) * p.o_sb + int64_t(hkv * G + h) * p.o_sh + j;
#pragma unroll
        for (int t = 0; t < T::NT; ++t) orow[16 * t] = mi::cvt_bf16(acc[t][i] * inv);
      }
    }
    return;
  }

  publish_merge<D, G>(p, u, b, hkv, nsplit, item_base, acc, m_run, lt);
}

// A workgroup of W waves runs units blockIdx * W + w, w < W: W consecutive
// KV heads of one item (W divides kv_heads, and the unit count is a multiple
// of kv_heads, so the waves of a workgroup run the same number of units).
// head_dim <= 128: registers capped at 256 per wave, so at least two waves
// share a SIMD (the plan's 6 units per CU fit).  head_dim 256 needs the full
// register file.
template <int D, int G, int W, int S, bool ROPE>
__global__ __launch_bounds__(64 * W * S) __attribute__((amdgpu_waves_per_eu(D <= 128 ? MI_DECODE_WAVES : 1))) void decode_run_kernel(
    RunParams p) {
  using T = DecodeTraits<D, G>;
  __shared__ __attribute__((aligned(16))) char slot[W * S * T::SLOT + (ROPE ? W * S * T::RX : 0)];
  lds_t* lds = (lds_t*)slot;
  lds_t* rx = lds + W * S * T::SLOT + (ROPE ? int(threadIdx.x >> 6) * T::RX : 0);  // this wave's RoPE rows
  // Every argument is read from the argument segment at once, up front:
  // left to the compiler, some of these reads came after the plan's header
  // and item loads, each one more round trip before the first page load.
  __asm__ volatile("" ::"s"(p.header), "s"(p.items), "s"(p.q), "s"(p.pool), "s"(p.cos), "s"(p.sin), "s"(p.q_sb),
                   "s"(p.q_sh), "s"(p.num_pages), "s"(p.hkv), "s"(p.max_items), "s"(p.table_rows),
                   "s"(p.k_col_bytes), "s"(p.counters), "s"(p.pml), "s"(p.po), "s"(p.out), "s"(p.o_sb), "s"(p.o_sh),
                   "s"(p.indices), "s"(p.scale_log2), "s"(p.pml_bytes), "s"(p.po_bytes));
  // the unit is wave-uniform (readfirstlane): its head, request and row
  // pointers then live in scalar registers, and the buffer descriptors built
  // from them need no per-lane (waterfall) loops
  int u = int(blockIdx.x) * W + (W == 1 ? 0 : __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6) % W));
  // The first item is read before the unit count is known (in bounds either
  // way), so the reads are in flight together.  The first check reads the
  // item as well (a split count is never negative): with the count alone the
  // compiler sank the item load below it, one more round trip before the
  // first page load (fused launch ~1 % slower on every decode shape).
  int iv = load_item_word(p, u);
  const int num_units = p.header->num_units;
  if (!((u < num_units) & (mi::read_lane_i(iv, kItemNsplit) >= 0))) return;
  while (true) {
    decode_unit<D, G, W, S, T::NB, ROPE>(p, u, iv, lds, rx);
    u += int(gridDim.x) * W;
    if (u >= num_units) break;
    iv = load_item_word(p, u);
  }
}

typedef void (*RunKernel)(RunParams);

template <int D, int W, int S, bool ROPE>
RunKernel pick_group(int g) {
  switch (g) {
    case 1: return decode_run_kernel<D, 1, W, S, ROPE>;
    case 2: return decode_run_kernel<D, 2, W, S, ROPE>;
    case 3: return decode_run_kernel<D, 3, W, S, ROPE>;
    case 4: return decode_run_kernel<D, 4, W, S, ROPE>;
    case 5: return decode_run_kernel<D, 5, W, S, ROPE>;
    case 6: return decode_run_kernel<D, 6, W, S, ROPE>;
    case 7: return decode_run_kernel<D, 7, W, S, ROPE>;
    case 8: return decode_run_kernel<D, 8, W, S, ROPE>;
    default: return nullptr;
  }
}

// KV heads per workgroup: two when kv_heads is even and a row slice of one
// head is short (head_dim <= 128), else one.
int waves_per_group(int head_dim, int hkv) { return (head_dim <= 128 && hkv % 2 == 0) ? 2 : 1; }

template <bool ROPE>
RunKernel pick_kernel(int head_dim, int group, int waves, int lanes) {
  switch (head_dim) {
    case 64:
      if (lanes == 2) return waves == 2 ? pick_group<64, 2, 2, ROPE>(group) : pick_group<64, 1, 2, ROPE>(group);
      return waves == 2 ? pick_group<64, 2, 1, ROPE>(group) : pick_group<64, 1, 1, ROPE>(group);
    case 128: return waves == 2 ? pick_group<128, 2, 1, ROPE>(group) : pick_group<128, 1, 1, ROPE>(group);
    case 256: return waves == 1 ? pick_group<256, 1, 1, ROPE>(group) : nullptr;
    default: return nullptr;
  }
}

// Units the plan aims at: one resident round of kUnitsPerCU per CU, but at
// most ~MI_DECODE_MERGE_BUDGET / group splits per (request, KV head) on
// average -- the merge's cost grows with splits x group (Qwen2.5-7B, group
// 7: 4 units per CU instead of 6 took ~1 us off) -- and at least two per CU.
int plan_target_units(int batch, int hq, int hkv) {
  const int group = hq / hkv;
  const long long cap = (long long)(MI_DECODE_MERGE_BUDGET / group) * batch * hkv;
  const int round = mi::num_cus() * kUnitsPerCU;
  return int(cap < round ? (cap > mi::num_cus() * 2 ? cap : mi::num_cus() * 2) : round);
}

// Lane groups per unit: two when the plan aims at no more than three units
// per CU at head_dim 64 -- too few waves to overlap each wave's per-step
// chain (Qwen2.5-0.5B heads, B=32: one two-wave workgroup per CU, each page
// pair 0.92 us of which 0.06 us waiting for its loads) -- so each unit's
// pages are split over two waves per head and merged in LDS.  Else one.
int lane_groups(int head_dim, int batch, int hq, int hkv) {
  return (head_dim == 64 && plan_target_units(batch, hq, hkv) <= mi::num_cus() * 3) ? 2 : 1;
}

// Workgroups of the run launch: one resident round of units (capped by the
// workspace), W units each (kUnitsPerCU per CU, or 3 with two lane groups).
int run_grid(int max_units, int waves, int lanes) {
  return max(1, min(max_units, mi::num_cus() * (lanes == 2 ? 3 : kUnitsPerCU)) / waves);
}

int check_shape(const char* who, int batch, int hq, int hkv, int head_dim, int page_size) {
  if (batch < 0 || hq <= 0 || hkv <= 0)
    return mi::fail(MI_ERR_INVALID, "%s: bad batch/head counts (%d, %d, %d)", who, batch, hq, hkv);
  if (hq % hkv != 0)
    return mi::fail(MI_ERR_INVALID, "%s: num_qo_heads %d not a multiple of num_kv_heads %d", who, hq, hkv);
  if (page_size != kPageSize)
    return mi::fail(MI_ERR_UNSUPPORTED, "%s: page_size %d (built for 16)", who, page_size);
  if (!pick_kernel<false>(head_dim, hq / hkv, waves_per_group(head_dim, hkv), 1))
    return mi::fail(MI_ERR_UNSUPPORTED, "%s: head_dim %d / group %d not built (head_dim 64/128/256, group 1..8)",
                    who, head_dim, hq / hkv);
  return MI_OK;
}

}  // namespace

extern "C" size_t mi_decode_workspace_size(int32_t batch_size, int32_t num_qo_heads,
                                           int32_t num_kv_heads, int32_t head_dim, int32_t max_units) {
  if (batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  if (max_units <= 0) max_units = default_max_units(batch_size, num_kv_heads);
  return decode_layout(batch_size, num_qo_heads, num_kv_heads, head_dim, max_units).total;
}

int mi::dplan::plan_setup(const char* who, void* workspace, size_t workspace_bytes, int batch, int hq, int hkv,
                          int head_dim, int page_size, int max_units, PlanParams* pp) {
  int rc = check_shape(who, batch, hq, hkv, head_dim, page_size);
  if (rc) return rc;
  if (max_units <= 0) max_units = units_that_fit(workspace_bytes, batch, hq, hkv, head_dim);
  const DecodeLayout L = decode_layout(batch, hq, hkv, head_dim, max_units);
  if (!workspace || workspace_bytes < L.total)
    return mi::fail(MI_ERR_WORKSPACE, "%s: workspace %zu bytes, need %zu", who, workspace_bytes, L.total);
  if (L.max_items < batch)
    return mi::fail(MI_ERR_WORKSPACE, "%s: room for %d units, need at least batch*kv_heads = %d", who, max_units,
                    batch * hkv);
  char* ws = static_cast<char*>(workspace);
  pp->batch = batch;
  pp->hkv = hkv;
  pp->target_units = plan_target_units(batch, hq, hkv);
  pp->max_items = L.max_items;
  pp->header = reinterpret_cast<DecodeHeader*>(ws);
  pp->items = reinterpret_cast<DecodeItem*>(ws + L.items);
  pp->counters = reinterpret_cast<int*>(ws + L.counters);
  return MI_OK;
}

extern "C" int mi_decode_plan(void* workspace, size_t workspace_bytes, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              int32_t batch_size, int32_t num_qo_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t page_size, int32_t max_units, mi_stream_t stream) {
  mi::clear_error();
  PlanParams pp;
  const int rc = mi::dplan::plan_setup("decode plan", workspace, workspace_bytes, batch_size, num_qo_heads,
                                       num_kv_heads, head_dim, page_size, max_units, &pp);
  if (rc) return rc;
  if (batch_size > 0 && (!kv_indptr || !kv_indices || !kv_last_page_len))
    return mi::fail(MI_ERR_INVALID, "decode plan: null indptr / indices / last_page_len");
  pp.indptr = kv_indptr;
  pp.indices = kv_indices;
  pp.last_page_len = kv_last_page_len;
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, static_cast<hipStream_t>(stream), pp);
  return mi::check_launch("decode_plan_kernel");
}

namespace {

// The run launch shared by the plain and the RoPE + append forms: checks the
// workspace and arguments, fills what the kernel reads of a plan, launches.
// `rp` arrives with the q / pool / out / RoPE fields set.
int launch_run(const char* who, bool rope, RunParams rp, void* workspace, size_t workspace_bytes, int32_t batch_size,
               int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float sm_scale,
               int32_t max_units, mi_stream_t stream) {
  int rc = check_shape(who, batch_size, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  if (batch_size == 0) return MI_OK;
  if (max_units <= 0) max_units = units_that_fit(workspace_bytes, batch_size, num_qo_heads, num_kv_heads, head_dim);
  const DecodeLayout L = decode_layout(batch_size, num_qo_heads, num_kv_heads, head_dim, max_units);
  if (!workspace || workspace_bytes < L.total)
    return mi::fail(MI_ERR_WORKSPACE, "%s: workspace %zu bytes, need %zu", who, workspace_bytes, L.total);
  // the plan's own bound (every wave reads a work item before it knows the
  // unit count, clamped to the item array, which must not be empty)
  if (L.max_items < batch_size)
    return mi::fail(MI_ERR_WORKSPACE, "%s: room for %d units, need at least batch*kv_heads = %d", who, max_units,
                    batch_size * num_kv_heads);
  if (!rp.q || !rp.pool || !rp.indices || !rp.out) return mi::fail(MI_ERR_INVALID, "%s: null pointer argument", who);
  if ((reinterpret_cast<uintptr_t>(rp.q) & 15) || (reinterpret_cast<uintptr_t>(rp.pool) & 15) || rp.q_sb % 8 ||
      rp.q_sh % 8)
    return mi::fail(MI_ERR_INVALID, "%s: q rows and pool must be 16-byte aligned", who);
  char* ws = static_cast<char*>(workspace);
  rp.header = reinterpret_cast<const DecodeHeader*>(ws);
  rp.items = reinterpret_cast<const DecodeItem*>(ws + L.items);
  rp.counters = reinterpret_cast<int*>(ws + L.counters);
  rp.pml = reinterpret_cast<float*>(ws + L.pml);
  rp.po = reinterpret_cast<uint16_t*>(ws + L.po);
  rp.pml_bytes = int(L.po - L.pml);
  rp.po_bytes = int(L.total - L.po);
  rp.hkv = num_kv_heads;
  rp.max_items = L.max_items;
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf(float(head_dim));
  rp.scale_log2 = scale * mi::kLog2e;
  const int waves = waves_per_group(head_dim, num_kv_heads);
  const int lanes = lane_groups(head_dim, batch_size, num_qo_heads, num_kv_heads);
  RunKernel k = rope ? pick_kernel<true>(head_dim, num_qo_heads / num_kv_heads, waves, lanes)
                     : pick_kernel<false>(head_dim, num_qo_heads / num_kv_heads, waves, lanes);
  hipLaunchKernelGGL(k, dim3(run_grid(max_units, waves, lanes)), dim3(64 * waves * lanes), 0,
                     static_cast<hipStream_t>(stream), rp);
  return mi::check_launch("decode_run_kernel");
}

}  // namespace

extern "C" int mi_decode_run(void* workspace, size_t workspace_bytes, const void* q,
                             int64_t q_stride_batch, int64_t q_stride_head, const void* paged_kv_cache,
                             int64_t num_pages, const int32_t* kv_indices, void* out,
                             int64_t out_stride_batch, int64_t out_stride_head, int32_t batch_size,
                             int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, float sm_scale, int32_t max_units, mi_stream_t stream) {
  mi::clear_error();
  RunParams rp = {};
  rp.q = static_cast<const uint16_t*>(q);
  rp.q_sb = q_stride_batch;
  rp.q_sh = q_stride_head;
  rp.pool = static_cast<char*>(const_cast<void*>(paged_kv_cache));  // read only in this form
  rp.num_pages = num_pages;
  rp.indices = kv_indices;
  rp.out = static_cast<uint16_t*>(out);
  rp.o_sb = out_stride_batch;
  rp.o_sh = out_stride_head;
  return launch_run("decode run", false, rp, workspace, workspace_bytes, batch_size, num_qo_heads, num_kv_heads,
                    head_dim, page_size, sm_scale, max_units, stream);
}

extern "C" int mi_decode_rope_append_run(void* workspace, size_t workspace_bytes, const void* qkv,
                                         int64_t qkv_stride_token, const void* cos_table, const void* sin_table,
                                         int64_t table_rows,
                                         void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indices,
                                         void* out, int64_t out_stride_batch, int64_t out_stride_head,
                                         int32_t batch_size, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t page_size, float sm_scale, int32_t max_units,
                                         mi_stream_t stream) {
  mi::clear_error();
  if (batch_size > 0 && (!cos_table || !sin_table))
    return mi::fail(MI_ERR_INVALID, "decode rope append run: null RoPE table");
  if (table_rows <= 0 || table_rows > (int64_t(1) << 30))
    return mi::fail(MI_ERR_INVALID, "decode rope append run: table_rows %lld", (long long)table_rows);
  if ((reinterpret_cast<uintptr_t>(cos_table) & 15) || (reinterpret_cast<uintptr_t>(sin_table) & 15))
    return mi::fail(MI_ERR_INVALID, "decode rope append run: cos / sin tables must be 16-byte aligned");
  if (num_kv_heads > 0 && qkv_stride_token < int64_t(num_qo_heads + 2 * num_kv_heads) * head_dim)
    return mi::fail(MI_ERR_INVALID, "decode rope append run: qkv row stride %lld shorter than (Hq + 2 Hkv) * D",
                    (long long)qkv_stride_token);
  RunParams rp = {};
  rp.q = static_cast<const uint16_t*>(qkv);
  rp.q_sb = qkv_stride_token;
  rp.q_sh = head_dim;
  rp.pool = static_cast<char*>(paged_kv_cache);
  rp.num_pages = num_pages;
  rp.indices = kv_indices;
  rp.out = static_cast<uint16_t*>(out);
  rp.o_sb = out_stride_batch;
  rp.o_sh = out_stride_head;
  rp.cos = static_cast<const uint16_t*>(cos_table);
  rp.sin = static_cast<const uint16_t*>(sin_table);
  rp.table_rows = int(table_rows);
  rp.k_col_bytes = num_qo_heads * head_dim * 2;
  return launch_run("decode rope append run", true, rp, workspace, workspace_bytes, batch_size, num_qo_heads,
                    num_kv_heads, head_dim, page_size, sm_scale, max_units, stream);
}

// ------------------------------------------------------------------ no caller workspace
// Decode attention for callers that cannot allocate (code under graph capture
// that may not call hipMalloc, allocation-free serving loops): plan and run
// in one call, the work list in a static device array instead of a
// caller-supplied workspace.  Every call on a device shares that device's
// array, so calls that overlap on one device (other streams, other threads)
// race; the plan rewrites everything the run reads, and its per-(request,
// KV head) counters start at zero on every call.
namespace {

constexpr size_t kStaticScratchBytes = size_t(16) << 20;
__device__ __attribute__((aligned(256))) char scratch[kStaticScratchBytes];

// Device address of `scratch`, looked up once per device with that device
// current (the host-side name is only a stand-in for the symbol).
void* scratch_address(int device) {
  static std::mutex mu;
  static void* addr[64] = {nullptr};
  if (device < 0 || device >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[device]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    addr[device] = ptr;
  }
  return addr[device];
}

}  // namespace

extern "C" size_t mi_decode_static_capacity(void) { return kStaticScratchBytes; }

extern "C" int mi_decode_static(const void* q, int64_t q_stride_batch, int64_t q_stride_head,
                                const void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indptr,
                                const int32_t* kv_indices, const int32_t* kv_last_page_len, void* out,
                                int64_t out_stride_batch, int64_t out_stride_head, int32_t batch_size,
                                int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                float sm_scale, mi_stream_t stream) {
  mi::clear_error();
  int rc = check_shape("decode static", batch_size, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  if (batch_size == 0) return MI_OK;
  // one resident round of units plus one item per request: the work list
  // the plan needs for this batch, which must fit the static array
  const int max_units = mi::num_cus() * kUnitsPerCU + batch_size * num_kv_heads;
  const size_t need = decode_layout(batch_size, num_qo_heads, num_kv_heads, head_dim, max_units).total;
  if (need > kStaticScratchBytes)
    return mi::fail(MI_ERR_WORKSPACE,
                    "decode static: batch %d x %d KV heads (group %d, head_dim %d) needs a %zu-byte work list, "
                    "over the %zu-byte static scratch; use mi_decode_plan / mi_decode_run with a workspace",
                    batch_size, num_kv_heads, num_qo_heads / num_kv_heads, head_dim, need, kStaticScratchBytes);
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return mi::fail(MI_ERR_LAUNCH, "decode static: no current device");
  void* ws = scratch_address(device);
  if (!ws) return mi::fail(MI_ERR_LAUNCH, "decode static: hipGetSymbolAddress of the scratch array failed");
  rc = mi_decode_plan(ws, kStaticScratchBytes, kv_indptr, kv_indices, kv_last_page_len, batch_size, num_qo_heads,
                      num_kv_heads, head_dim, page_size, max_units, stream);
  if (rc) return rc;
  return mi_decode_run(ws, kStaticScratchBytes, q, q_stride_batch, q_stride_head, paged_kv_cache, num_pages,
                       kv_indices, out, out_stride_batch, out_stride_head, batch_size, num_qo_heads, num_kv_heads,
                       head_dim, page_size, sm_scale, max_units, stream);
}
