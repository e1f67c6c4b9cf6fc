// Fused batched sampler: greedy argmax, temperature, top-p, multinomial.
//
// Reference: sample_batch (scheduler.py:319-343) and sample (310-316).
//   * temperatures are held in the logits dtype, i.e. rounded to bf16 (327);
//   * rows with temperature <= 0 take argmax(logits), first index on ties
//     (328, 339-341); NaN ranks above every number, as in torch.argmax;
//   * other rows draw from softmax(bf16(logit / clamp(t, 1e-6))) in fp32
//     (331-336).  top-p (an extension) keeps the smallest set of most likely
//     tokens whose mass reaches top_p, ties at the boundary included.
//
// Each row is split into chunks of 4,096 tokens, one 256-thread workgroup
// per (chunk, row), in two launches.  Sampled rows draw by the exponential
// race (Gumbel-max): argmax_i (s_i * log2 e - log2(-log2 u_i)) selects i with
// probability proportional to exp(s_i).
//   pass 1, rows without top-p: each wave's winner over its 1,024 tokens (the
//     greedy argmax, or the race); pass 2's chunk-0 workgroup of the row
//     takes the best of the row's wave winners.
//   pass 1, top-p rows: the chunk's max key and a 1,024-bin histogram of
//     probability mass over key >> 6 (relative to the chunk max) with its 32
//     super-bin sums.  The histogram adds 2^40 fixed-point masses with 64-bit
//     integer LDS atomics: exact, so no sum depends on the order of the
//     additions, and several times faster than float LDS atomics on gfx950.
//   pass 2, top-p rows: every workgroup of the row combines the chunks'
//     super-bin sums (scaled to the row max), finds the super-bin where the
//     mass accumulated from the top reaches top_p of the total, then the
//     boundary bin inside it from that super-bin's 32 bins of every chunk --
//     the same arithmetic in the same order in every workgroup, so all of
//     them agree.  Then the race over the tokens above the boundary bin and,
//     for the boundary bin's 64 keys, their mass and race winner per key.
//     The row's last workgroup (an agent-scope counter; partials written and
//     read device-coherent, so no workgroup ever waits for another) resolves
//     the boundary key exactly (ties at it kept) and picks the winner over
//     the kept tokens.
// u_i comes from Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011) with counter (token / 4, row,
// offset) and key = seed.  Pass 1 reads the offset and keeps a copy in the
// workspace; pass 2 reads the copy, so one workgroup of it can advance the
// offset with no count of the grid's workgroups.
#include <math.h>

#include "mi_common.h"

namespace {

constexpr uint32_t kNaNKey = 0x10000u;

// Order-preserving 16-bit key of a bf16 value; -0 and +0 share a key and NaN
// (either sign) ranks above +inf.
__device__ __forceinline__ uint32_t bf16_key(uint16_t b) {
  if ((b & 0x7fffu) > 0x7f80u) return kNaNKey;
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~uint32_t(b) & 0xffffu) : (uint32_t(b) | 0x8000u);
}

__device__ __forceinline__ float key_to_f32(uint32_t k) {
  const uint32_t b = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
  return __uint_as_float(b << 16);
}

// Philox4x32-10 (Salmon et al. 2011): multipliers 0xD2511F53 / 0xCD9E8D57,
// Weyl key increments 0x9E3779B9 / 0xBB67AE85.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
    const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
    c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
    k.x += 0x9E3779B9u;
    k.y += 0xBB67AE85u;
  }
  return c;
}

// Uniform in (0, 1) from 24 random bits.
__device__ __forceinline__ float u01(uint32_t x) { return (float(x >> 8) + 0.5f) * (1.0f / 16777216.0f); }

constexpr int kT = 256;              // threads per workgroup
constexpr int kGroupsPerThread = 4;  // 4-token groups per thread
constexpr int kChunk = kT * kGroupsPerThread * 4;  // 4,096 tokens per workgroup
// ints between two rows' counters in the workspace (one 128-byte line each)
constexpr int kCntStride = 32;
constexpr int kBins = 1024;          // histogram bins: key >> 6
constexpr int kSub = 64;             // keys per bin
constexpr int kSup = 32;             // super-bins of kBins / kSup bins
constexpr int kBinsPerSup = kBins / kSup;
constexpr int kGrp = kT / kSup;      // thread groups of the per-row combines
constexpr int kNW = kT / 64;
constexpr int kMaxChunks = 256;      // vocabularies up to 1,048,576 tokens
// 16-bit keys: the bf16 order key, with NaN (either sign) as 0xFFFF -- above
// +inf, whose key is 0xFF80 -- and 0 marking a slot past the vocabulary (no
// bf16 value maps to 0: -inf is 0x007F).
constexpr uint32_t kNaN16 = 0xFFFFu;
// Masses in [0, 1] as 2^40 fixed point: a chunk's 4,096 tokens sum to at
// most 2^52, a row's 2^20 tokens to at most 2^60.
constexpr float kFix = 1099511627776.0f;
constexpr float kUnfix = 1.0f / 1099511627776.0f;

__device__ __forceinline__ unsigned long long to_fix(float m) { return static_cast<unsigned long long>(m * kFix); }
__device__ __forceinline__ float from_fix(unsigned long long q) { return static_cast<float>(q) * kUnfix; }

struct SampleParams {
  const uint16_t* logits;
  int64_t stride;
  int batch, vocab, chunks;
  const float* temperature;
  const float* top_p;
  uint2 seed;
  uint64_t* offset;
  int64_t* out;
  // workspace: counters (zero between calls) and per-chunk partials
  int* cnt;
  uint64_t* off_copy;            // the draw offset as pass 1 read it
  unsigned long long* part;      // [row][chunk][kNW] wave winners, rows without top-p
  uint32_t* cmax;                // [row][chunk] max key, top-p rows
  float* sup;                    // [row][chunk][kSup] super-bin mass, relative to the chunk max
  float* bins;                   // [row][chunk][kBins] bin mass, relative to the chunk max
  unsigned long long* best;      // [row][chunk] race winner above the boundary bin
  unsigned long long* sub_mass;  // [row][chunk][kSub] boundary-bin key mass (fixed point, relative to the row max)
  unsigned long long* sub_best;  // [row][chunk][kSub] boundary-bin key race winner
};

// ---------------------------------------------------------------- lanes
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long x) {
  return (static_cast<unsigned long long>(dpp_u<CTRL>(uint32_t(x >> 32))) << 32) | dpp_u<CTRL>(uint32_t(x));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp_u<mi::kDppQuadSwap1>(x));
  x = max(x, dpp_u<mi::kDppQuadSwap2>(x));
  x = max(x, dpp_u<mi::kDppRowHalfMirror>(x));
  x = max(x, dpp_u<mi::kDppRowMirror>(x));
  // the swaps exchange values between lane halves; both results are taken
  // (one of them is the lane's own value)
  {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = max(x, max(uint32_t(r[0]), uint32_t(r[1])));
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    x = max(x, max(uint32_t(r[0]), uint32_t(r[1])));
  }
  return x;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
  x = max(x, dpp_u64<mi::kDppQuadSwap1>(x));
  x = max(x, dpp_u64<mi::kDppQuadSwap2>(x));
  x = max(x, dpp_u64<mi::kDppRowHalfMirror>(x));
  x = max(x, dpp_u64<mi::kDppRowMirror>(x));
  {
    const uint32_t hi = uint32_t(x >> 32), lo = uint32_t(x);
    const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    x = max(x, (static_cast<unsigned long long>(uint32_t(rh[0])) << 32) | uint32_t(rl[0]));
    x = max(x, (static_cast<unsigned long long>(uint32_t(rh[1])) << 32) | uint32_t(rl[1]));
  }
  {
    const uint32_t hi = uint32_t(x >> 32), lo = uint32_t(x);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    x = max(x, (static_cast<unsigned long long>(uint32_t(rh[0])) << 32) | uint32_t(rl[0]));
    x = max(x, (static_cast<unsigned long long>(uint32_t(rh[1])) << 32) | uint32_t(rl[1]));
  }
  return x;
}

// Workgroup max; `s` holds one value per wave and is not reused by the caller
// before its next barrier.
template <typename U>
__device__ __forceinline__ U block_max(U x, U* s) {
  if constexpr (sizeof(U) == 8) x = wave_max_u64(x);
  else x = wave_max_u32(x);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
  __syncthreads();
  U r = s[0];
#pragma unroll
  for (int k = 1; k < kNW; ++k) r = max(r, s[k]);
  return r;
}

// (value, index) packed so that a larger u64 is a larger value, then a lower
// index: the value's order-preserving bits above the complemented index.  0
// stands for "no token".
__device__ __forceinline__ uint32_t f32_order(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ unsigned long long pack_arg(uint32_t ordered, int idx) {
  return (static_cast<unsigned long long>(ordered) << 32) | uint32_t(~uint32_t(idx));
}
// The id a row's winner stands for: 0 when no token won.
__device__ __forceinline__ int64_t winner_id(unsigned long long pk, int vocab) {
  const int idx = int(~uint32_t(pk));
  return (pk >> 32) != 0 && idx >= 0 && idx < vocab ? idx : 0;
}

template <typename F>
__device__ __forceinline__ F coherent_load(const F* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename F>
__device__ __forceinline__ void coherent_store(F* p, F v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte device-coherent (sc1) buffer store for the histograms: the
// partials travel between workgroups on different XCDs.
constexpr int kCacheSc1 = 16;
constexpr int kBufferWord3 = 0x00020000;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes), kBufferWord3);
}

// After this workgroup's coherent stores: wait for them, count the chunk in
// `counter`; true in every thread of the row's last workgroup.
__device__ __forceinline__ bool last_of_row(int* counter, int chunks, int* s_flag) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores are acknowledged
  __syncthreads();
  if (threadIdx.x == 0)
    *s_flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == chunks - 1;
  __syncthreads();
  const bool last = *s_flag;
  if (last) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (threadIdx.x == 0) coherent_store(counter, 0);  // ready for the next call
  }
  return last;
}

struct RowParams {
  bool greedy;
  float tc;  // clamped bf16 temperature
  float tp;
};

__device__ __forceinline__ RowParams row_params(const SampleParams& p, int row) {
  RowParams r;
  const float tq = mi::bf16_to_f32(mi::f32_to_bf16(p.temperature[row]));
  r.greedy = !(tq > 0.f);  // <= 0 (and NaN) is greedy
  const float tmin = mi::bf16_to_f32(mi::f32_to_bf16(1e-6f));
  r.tc = fmaxf(tq, tmin);
  r.tp = (!r.greedy && p.top_p) ? p.top_p[row] : 1.0f;
  return r;
}

// The keys of this thread's 4 groups of 4 tokens of chunk c: the raw logits'
// (greedy rows) or those of bf16(x / t) (sampled rows); 0 past the
// vocabulary.  Group n of the thread is global group c * kT * 4 + n * kT +
// tid (tokens 4g .. 4g + 3, the draw's Philox counter).  All loads are
// issued before any is used.
__device__ __forceinline__ void chunk_keys(const SampleParams& p, int row, int c, const RowParams& rp,
                                           uint32_t (&k)[kGroupsPerThread][4], int (&g)[kGroupsPerThread]) {
  const uint16_t* x = p.logits + int64_t(row) * p.stride;
  const int V = p.vocab;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 7) == 0;
  uint16_t raw[kGroupsPerThread][4];
#pragma unroll
  for (int n = 0; n < kGroupsPerThread; ++n) {
    g[n] = (c * kGroupsPerThread + n) * kT + int(threadIdx.x);
    const int t0 = 4 * g[n];
#pragma unroll
    for (int e = 0; e < 4; ++e) raw[n][e] = 0;
    if (vec && t0 + 3 < V) {
      const uint2 w = *reinterpret_cast<const uint2*>(x + t0);
      raw[n][0] = uint16_t(w.x);
      raw[n][1] = uint16_t(w.x >> 16);
      raw[n][2] = uint16_t(w.y);
      raw[n][3] = uint16_t(w.y >> 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (t0 + e < V) raw[n][e] = x[t0 + e];
    }
  }
#pragma unroll
  for (int n = 0; n < kGroupsPerThread; ++n) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // bf16(x / t): the fp32 quotient rounded to nearest even by v_cvt_pk_bf16_f32
      const uint16_t sv = rp.greedy ? raw[n][e] : mi::cvt_bf16(mi::bf16_to_f32(raw[n][e]) / rp.tc);
      const uint32_t kk = bf16_key(sv);
      k[n][e] = (4 * g[n] + e < V) ? (kk == kNaNKey ? kNaN16 : kk) : 0u;
    }
  }
}

// A chunk (or row) whose max key is that of a real, finite-or-+inf value has
// mass to histogram: not NaN (the row then keeps every token), not -inf
// (every token of it has mass 0) and not an empty slot.
__device__ __forceinline__ bool has_mass(uint32_t max_key) {
  return max_key != 0u && max_key != kNaN16 && key_to_f32(max_key) != -INFINITY;
}

// The race value of a token with key kk (> 0) and random bits r; false for a
// token of mass 0 (-inf), which never wins.  NaN ranks above every number.
__device__ __forceinline__ bool race_value(uint32_t kk, uint32_t r, float& v, float& s) {
  if (kk == kNaN16) {
    v = INFINITY;
    s = 0.f;
    return true;
  }
  s = key_to_f32(kk);
  if (s == -INFINITY) return false;
  v = s * mi::kLog2e - __log2f(-__log2f(u01(r)));
  return true;
}

// Lanes 0..n-1 of one wave hold the masses H of n items in key order (the
// highest last).  In every lane: the item where the mass accumulated from the
// top reaches `target` -- a < target <= a + H, with a = `above0` + the mass of
// the items above it; the highest such item if rounding makes several --, or
// -1; `lowest` = the lowest item with H > 0 (or -1), `a_sel` = a of the
// item found.
__device__ __forceinline__ void boundary_search(float H, float above0, float target, int& sel, int& lowest,
                                                float& a_sel) {
  const int lane = threadIdx.x & 63;
  float incl = H;  // mass of the items >= this one
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_down(incl, o);
    if (lane + o < 64) incl += y;
  }
  float excl = __shfl_down(incl, 1);  // mass of the items above this one
  if (lane == 63) excl = 0.f;
  const float a = above0 + excl;
  const uint64_t hit = __ballot(H > 0.f && a < target && a + H >= target);
  const uint64_t nonempty = __ballot(H > 0.f);
  sel = hit ? 63 - __builtin_clzll(hit) : -1;
  lowest = nonempty ? __builtin_ctzll(nonempty) : -1;
  a_sel = sel >= 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), sel)) : 0.f;
}

__global__ __launch_bounds__(kT) void sample_pass1(SampleParams p) {
  __shared__ __align__(16) unsigned long long hist[kBins];
  __shared__ uint32_t s_max[kNW];
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const RowParams rp = row_params(p, row);
  const bool top_p = !rp.greedy && rp.tp < 1.0f;
  const int pc = row * p.chunks + c;
  static_assert(kBins == 4 * kT, "each thread owns 4 bins");
  if (pc == 0 && tid == 0) coherent_store(p.off_copy, *p.offset);
  if (top_p) {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    reinterpret_cast<uint4*>(hist)[2 * tid] = z;
    reinterpret_cast<uint4*>(hist)[2 * tid + 1] = z;
  }
  uint32_t k[kGroupsPerThread][4];
  int g[kGroupsPerThread];
  chunk_keys(p, row, c, rp, k, g);

  if (!top_p) {
    // the wave's winner: greedy argmax, or the race over every token
    unsigned long long win = 0;
    if (rp.greedy) {
#pragma unroll
      for (int n = 0; n < kGroupsPerThread; ++n)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (k[n][e]) win = max(win, pack_arg(k[n][e], 4 * g[n] + e));
    } else {
      const uint64_t off = *p.offset;
#pragma unroll
      for (int n = 0; n < kGroupsPerThread; ++n) {
        if (!(k[n][0] | k[n][1] | k[n][2] | k[n][3])) continue;  // past the vocabulary: no Philox block
        const uint4 r = philox4x32_10(make_uint4(uint32_t(g[n]), uint32_t(row), uint32_t(off), uint32_t(off >> 32)),
                                      p.seed);
        const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v, s;
          if (k[n][e] && race_value(k[n][e], rr[e], v, s)) win = max(win, pack_arg(f32_order(v), 4 * g[n] + e));
        }
      }
    }
    win = wave_max_u64(win);
    if (lane == 0) coherent_store(&p.part[size_t(pc) * kNW + w], win);
    return;
  }

  // top-p rows: the chunk max, then the histogram relative to it
  uint32_t m = 0;
#pragma unroll
  for (int n = 0; n < kGroupsPerThread; ++n)
#pragma unroll
    for (int e = 0; e < 4; ++e) m = max(m, k[n][e]);
  const uint32_t cm = block_max(m, s_max);  // its barrier also orders the zeroing
  if (has_mass(cm)) {
    // (no NaN key here: it would be the max)
    const float smax_c = key_to_f32(cm) * mi::kLog2e;
#pragma unroll
    for (int n = 0; n < kGroupsPerThread; ++n)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t kk = k[n][e];
        if (kk == 0u) continue;
        const unsigned long long q = to_fix(__builtin_amdgcn_exp2f(key_to_f32(kk) * mi::kLog2e - smax_c));
        if (q) atomicAdd(&hist[kk >> 6], q);
      }
  }
  __syncthreads();
  const uint4 h01 = reinterpret_cast<const uint4*>(hist)[2 * tid];
  const uint4 h23 = reinterpret_cast<const uint4*>(hist)[2 * tid + 1];
  const unsigned long long q0 = (static_cast<unsigned long long>(h01.y) << 32) | h01.x;
  const unsigned long long q1 = (static_cast<unsigned long long>(h01.w) << 32) | h01.z;
  const unsigned long long q2 = (static_cast<unsigned long long>(h23.y) << 32) | h23.x;
  const unsigned long long q3 = (static_cast<unsigned long long>(h23.w) << 32) | h23.z;
  const __amdgpu_buffer_rsrc_t rb = rsrc_of(p.bins + size_t(pc) * kBins, kBins * sizeof(float));
  const u32x4_t v = {__float_as_uint(from_fix(q0)), __float_as_uint(from_fix(q1)), __float_as_uint(from_fix(q2)),
                     __float_as_uint(from_fix(q3))};
  __builtin_amdgcn_raw_buffer_store_b128(v, rb, 16 * tid, 0, kCacheSc1);
  // super-bin j = bins 32j .. 32j + 31 = threads 8j .. 8j + 7: exact sum over 8 lanes
  static_assert(kBinsPerSup == 32, "a super-bin is 8 threads' bins");
  unsigned long long s = q0 + q1 + q2 + q3;
  s += dpp_u64<mi::kDppQuadSwap1>(s);
  s += dpp_u64<mi::kDppQuadSwap2>(s);
  s += dpp_u64<mi::kDppRowHalfMirror>(s);
  if ((tid & 7) == 0) coherent_store(&p.sup[size_t(pc) * kSup + (tid >> 3)], from_fix(s));
  if (tid == 0) coherent_store(&p.cmax[pc], cm);
}

struct RowInfo {
  float smax;    // row max scaled logit x log2 e
  int bstar;     // boundary bin, -1: every token is kept
  float above;   // mass of the bins above it (relative to the row max)
  float target;  // top_p x total mass (+inf: every key of the boundary bin is kept)
};

// The top-p boundary of a row from pass 1's chunk partials, in every
// workgroup of the row.  `mc` = this thread's chunk max (chunk tid), `sv` =
// the super-bin sums of chunks grp + kGrp * u (super-bin tid % kSup).
__device__ __forceinline__ RowInfo row_boundary(const SampleParams& p, int row, float tp, uint32_t mc,
                                                const float (&sv0)[8], float* s_scale, float (*s_part)[kSup],
                                                uint32_t* s_u32, float* s_f, int* s_i) {
  const int tid = threadIdx.x, j = tid & (kSup - 1), grp = tid / kSup;
  const int C = p.chunks, base = row * C;
  RowInfo ri;
  ri.bstar = -1;
  ri.above = 0.f;
  ri.target = 0.f;
  const uint32_t M = block_max(mc, s_u32);
  ri.smax = has_mass(M) ? key_to_f32(M) * mi::kLog2e : 0.f;
  if (!has_mass(M)) return ri;  // NaN or no mass: every token is kept
  if (tid < C) s_scale[tid] = has_mass(mc) ? __builtin_amdgcn_exp2f(key_to_f32(mc) * mi::kLog2e - ri.smax) : 0.f;
  __syncthreads();
  // super-bin totals, scaled to the row max, in chunk order
  float part = 0.f;
  for (int c0 = 0; c0 < C; c0 += kGrp * 8) {
    float sv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cc = c0 + grp + kGrp * u;
      sv[u] = c0 == 0 ? sv0[u] : (cc < C ? coherent_load(&p.sup[size_t(base + cc) * kSup + j]) : 0.f);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cc = c0 + grp + kGrp * u;
      if (cc < C) {
        const float sc = s_scale[cc];
        if (sc != 0.f) part += sc * sv[u];
      }
    }
  }
  s_part[grp][j] = part;
  __syncthreads();
  if (tid < 64) {
    float S = 0.f;
    if (tid < kSup)
#pragma unroll
      for (int q = 0; q < kGrp; ++q) S += s_part[q][tid];
    float Z = S;
    Z += __shfl_xor(Z, 1);
    Z += __shfl_xor(Z, 2);
    Z += __shfl_xor(Z, 4);
    Z += __shfl_xor(Z, 8);
    Z += __shfl_xor(Z, 16);
    Z += __shfl_xor(Z, 32);
    const float target = tp * Z;
    int sel, lowest;
    float a_sel;
    boundary_search(S, 0.f, target, sel, lowest, a_sel);
    if (tid == 0) {
      // rounding left no super-bin: keep every token down to the lowest
      // non-empty one
      s_i[0] = sel >= 0 ? sel : max(lowest, 0);  // (the row max's super-bin is never empty)
      s_f[0] = a_sel;
      s_f[1] = sel >= 0 ? target : INFINITY;
    }
  }
  __syncthreads();
  const int sstar = s_i[0];
  const float aboveS = s_f[0], target = s_f[1];
  // the bins of the boundary super-bin, scaled to the row max, in chunk order
  part = 0.f;
  for (int c0 = 0; c0 < C; c0 += kGrp * 8) {
    float bv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cc = c0 + grp + kGrp * u;
      bv[u] = cc < C ? coherent_load(&p.bins[size_t(base + cc) * kBins + sstar * kBinsPerSup + j]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cc = c0 + grp + kGrp * u;
      if (cc < C) {
        const float sc = s_scale[cc];
        if (sc != 0.f) part += sc * bv[u];
      }
    }
  }
  s_part[grp][j] = part;
  __syncthreads();
  if (tid < 64) {
    float B = 0.f;
    if (tid < kSup)
#pragma unroll
      for (int q = 0; q < kGrp; ++q) B += s_part[q][tid];
    int sel, lowest;
    float a_sel;
    boundary_search(B, aboveS, target, sel, lowest, a_sel);
    if (tid == 0) {
      // none found (rounding, or every token kept down to this super-bin):
      // the lowest non-empty bin, all of its keys kept
      s_i[1] = sstar * kBinsPerSup + (sel >= 0 ? sel : (lowest >= 0 ? lowest : 0));
      s_f[2] = sel >= 0 ? a_sel : 0.f;
      s_f[3] = sel >= 0 ? target : INFINITY;
    }
  }
  __syncthreads();
  ri.bstar = s_i[1];
  ri.above = s_f[2];
  ri.target = s_f[3];
  return ri;
}

__global__ __launch_bounds__(kT) void sample_pass2(SampleParams p) {
  __shared__ float s_scale[kMaxChunks];
  __shared__ float s_part[kGrp][kSup];
  __shared__ unsigned long long sub_mass[kSub];
  __shared__ unsigned long long sub_best[kSub];
  __shared__ unsigned long long s_m64[kNW][kSub];
  __shared__ unsigned long long s_b64[kNW][kSub];
  __shared__ unsigned long long s_win[kNW];
  __shared__ unsigned long long s_win2[kNW];
  __shared__ uint32_t s_u32[kNW];
  __shared__ float s_f[4];
  __shared__ int s_i[2];
  __shared__ int s_flag;
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const RowParams rp = row_params(p, row);
  const bool top_p = !rp.greedy && rp.tp < 1.0f;
  const int C = p.chunks, base = row * C;
  if (!top_p) {
    // rows drawn in pass 1: the best of the row's wave winners
    if (c == 0) {
      unsigned long long best = 0;
      for (int i = tid; i < C * kNW; i += kT) best = max(best, coherent_load(&p.part[size_t(base) * kNW + i]));
      best = block_max(best, s_win);
      if (tid == 0) p.out[row] = winner_id(best, p.vocab);
    }
  } else {
    if (tid < kSub) {
      sub_mass[tid] = 0ull;
      sub_best[tid] = 0ull;
    }
    // pass 1's partials of the row (chunk maxima, the first 64 chunks'
    // super-bin sums), then this chunk's logits, all in flight together
    const uint32_t mc = tid < C ? coherent_load(&p.cmax[base + tid]) : 0u;
    float sv0[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cc = tid / kSup + kGrp * u;
      sv0[u] = cc < C ? coherent_load(&p.sup[size_t(base + cc) * kSup + (tid & (kSup - 1))]) : 0.f;
    }
    const uint64_t off = coherent_load(p.off_copy);
    uint32_t k[kGroupsPerThread][4];
    int g[kGroupsPerThread];
    chunk_keys(p, row, c, rp, k, g);
    const RowInfo ri = row_boundary(p, row, rp.tp, mc, sv0, s_scale, s_part, s_u32, s_f, s_i);

    const uint32_t kmin = ri.bstar < 0 ? 1u : uint32_t(ri.bstar) << 6;  // lowest key that may be kept
    unsigned long long win = 0;
#pragma unroll
    for (int n = 0; n < kGroupsPerThread; ++n) {
      bool any = false;
#pragma unroll
      for (int e = 0; e < 4; ++e) any = any || k[n][e] >= kmin;
      if (!any) continue;  // a group with no candidate skips its Philox block
      const uint4 r = philox4x32_10(make_uint4(uint32_t(g[n]), uint32_t(row), uint32_t(off), uint32_t(off >> 32)),
                                    p.seed);
      const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t kk = k[n][e];
        float v, s;
        if (kk < kmin || !race_value(kk, rr[e], v, s)) continue;
        const unsigned long long pk = pack_arg(f32_order(v), 4 * g[n] + e);
        if (ri.bstar >= 0 && int(kk >> 6) == ri.bstar) {
          // (no NaN key here: the row max would be NaN)
          const unsigned long long q = to_fix(__builtin_amdgcn_exp2f(s * mi::kLog2e - ri.smax));
          if (q) atomicAdd(&sub_mass[kk & 63], q);
          atomicMax(&sub_best[kk & 63], pk);
        } else {
          win = max(win, pk);
        }
      }
    }
    win = block_max(win, s_win);  // its barrier also completes sub_*
    const int pc = base + c;
    if (tid == 0) coherent_store(&p.best[pc], win);
    if (ri.bstar >= 0 && tid < kSub) {
      coherent_store(&p.sub_mass[size_t(pc) * kSub + tid], sub_mass[tid]);
      coherent_store(&p.sub_best[size_t(pc) * kSub + tid], sub_best[tid]);
    }
    if (last_of_row(&p.cnt[row * kCntStride], C, &s_flag)) {
      unsigned long long bb = 0;
      for (int cc = tid; cc < C; cc += kT) bb = max(bb, coherent_load(&p.best[base + cc]));
      if (ri.bstar >= 0) {
        // key `lane` of the boundary bin over chunks w, w + kNW, ... (8 in flight)
        unsigned long long m = 0, b = 0;
        for (int c0 = w; c0 < C; c0 += kNW * 8) {
          unsigned long long mv[8], bv[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int cc = min(c0 + kNW * u, C - 1);
            mv[u] = coherent_load(&p.sub_mass[size_t(base + cc) * kSub + lane]);
            bv[u] = coherent_load(&p.sub_best[size_t(base + cc) * kSub + lane]);
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (c0 + kNW * u >= C) break;
            m += mv[u];
            b = max(b, bv[u]);
          }
        }
        s_m64[w][lane] = m;
        s_b64[w][lane] = b;
      }
      bb = wave_max_u64(bb);
      if (lane == 0) s_win2[w] = bb;
      __syncthreads();
      if (tid < 64) {
        unsigned long long best = max(max(s_win2[0], s_win2[1]), max(s_win2[2], s_win2[3]));
        if (ri.bstar >= 0) {
          unsigned long long m = 0, b = 0;
#pragma unroll
          for (int q = 0; q < kNW; ++q) {
            m += s_m64[q][lane];
            b = max(b, s_b64[q][lane]);
          }
          // the boundary key; if rounding left none, the lowest non-empty key
          int sel, lowest;
          float a_sel;
          boundary_search(from_fix(m), ri.above, ri.target, sel, lowest, a_sel);
          const int sstar = sel >= 0 ? sel : (lowest >= 0 ? lowest : 64);
          if (lane < sstar) b = 0;  // below the boundary: not kept
          best = max(best, wave_max_u64(b));
        }
        if (tid == 0) p.out[row] = winner_id(best, p.vocab);
      }
    }
  }
  // the next call's offset: every reader of the offset ran in pass 1
  if (c == 0 && row == 0 && tid == 0) coherent_store(p.offset, coherent_load(p.off_copy) + 1);
}

constexpr int kMaxRows = 65535;

struct SampleLayout {
  size_t cnt, off_copy, part, cmax, sup, bins, best, sub_mass, sub_best, total;
};

SampleLayout sample_layout(int batch, int vocab) {
  SampleLayout L;
  const int chunks = (vocab + kChunk - 1) / kChunk;
  const size_t rc = size_t(batch) * chunks;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = mi::align_up(off + bytes, 256);
    return at;
  };
  // counters at fixed offsets, sized for the largest batch a call takes, so
  // calls of different batch sizes on one workspace never lay partials over
  // them (every call leaves them at zero); one 128-byte line per row, so the
  // rows' workgroups do not queue their counting atomics on a shared line
  // (B=32 x 32,768: 19.1 -> 18.2 us; 48 x 152,064 top-p: 40.5 -> 35.7 us)
  L.cnt = take(size_t(kMaxRows) * kCntStride * sizeof(int));
  L.off_copy = take(sizeof(uint64_t));
  L.part = take(rc * kNW * sizeof(unsigned long long));
  L.cmax = take(rc * sizeof(uint32_t));
  L.sup = take(rc * kSup * sizeof(float));
  L.bins = take(rc * kBins * sizeof(float));
  L.best = take(rc * sizeof(unsigned long long));
  L.sub_mass = take(rc * kSub * sizeof(unsigned long long));
  L.sub_best = take(rc * kSub * sizeof(unsigned long long));
  L.total = off;
  return L;
}

int chunks_of(int vocab) { return (vocab + kChunk - 1) / kChunk; }

}  // namespace

extern "C" size_t mi_sample_workspace_size(int32_t batch_size, int32_t vocab_size) {
  if (batch_size <= 0 || batch_size > kMaxRows || vocab_size <= 0) return 0;
  return sample_layout(batch_size, vocab_size).total;
}

extern "C" int mi_sample(const void* logits, int64_t logits_row_stride, int32_t batch_size,
                         int32_t vocab_size, const float* temperature, const float* top_p,
                         uint64_t seed, uint64_t* rng_offset, int64_t* out_tokens, void* workspace,
                         size_t workspace_bytes, mi_stream_t stream) {
  mi::clear_error();
  if (batch_size < 0 || vocab_size <= 0 || logits_row_stride < vocab_size)
    return mi::fail(MI_ERR_INVALID, "sample: bad sizes (batch %d, vocab %d, stride %lld)", batch_size,
                    vocab_size, (long long)logits_row_stride);
  if (batch_size == 0) return MI_OK;
  if (batch_size > kMaxRows) return mi::fail(MI_ERR_INVALID, "sample: batch %d over %d rows", batch_size, kMaxRows);
  if (!logits || !temperature || !rng_offset || !out_tokens)
    return mi::fail(MI_ERR_INVALID, "sample: null pointer argument");
  const int chunks = chunks_of(vocab_size);
  if (chunks > kMaxChunks)
    return mi::fail(MI_ERR_UNSUPPORTED, "sample: vocab %d over %d tokens", vocab_size, kMaxChunks * kChunk);
  const SampleLayout L = sample_layout(batch_size, vocab_size);
  if (!workspace || workspace_bytes < L.total)
    return mi::fail(MI_ERR_WORKSPACE, "sample: workspace %zu bytes, need %zu", workspace_bytes, L.total);
  char* ws = static_cast<char*>(workspace);
  SampleParams sp;
  sp.logits = static_cast<const uint16_t*>(logits);
  sp.stride = logits_row_stride;
  sp.batch = batch_size;
  sp.vocab = vocab_size;
  sp.chunks = chunks;
  sp.temperature = temperature;
  sp.top_p = top_p;
  sp.seed = make_uint2(uint32_t(seed), uint32_t(seed >> 32));
  sp.offset = rng_offset;
  sp.out = out_tokens;
  sp.cnt = reinterpret_cast<int*>(ws + L.cnt);
  sp.off_copy = reinterpret_cast<uint64_t*>(ws + L.off_copy);
  sp.part = reinterpret_cast<unsigned long long*>(ws + L.part);
  sp.cmax = reinterpret_cast<uint32_t*>(ws + L.cmax);
  sp.sup = reinterpret_cast<float*>(ws + L.sup);
  sp.bins = reinterpret_cast<float*>(ws + L.bins);
  sp.best = reinterpret_cast<unsigned long long*>(ws + L.best);
  sp.sub_mass = reinterpret_cast<unsigned long long*>(ws + L.sub_mass);
  sp.sub_best = reinterpret_cast<unsigned long long*>(ws + L.sub_best);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(chunks), unsigned(batch_size), 1u};
  hipLaunchKernelGGL(sample_pass1, grid, dim3(kT), 0, s, sp);
  int rc = mi::check_launch("sample_pass1");
  if (rc) return rc;
  hipLaunchKernelGGL(sample_pass2, grid, dim3(kT), 0, s, sp);
  return mi::check_launch("sample_pass2");
}
