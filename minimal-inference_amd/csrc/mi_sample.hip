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
// per (chunk, row), in two launches; the last workgroup of a row to finish a
// launch (an agent-scope counter; partials written and read device-coherent,
// so no workgroup ever waits for another) combines the row's chunks:
//   pass 1: the scaled logits' 16-bit order keys; per chunk the greedy
//     argmax, the max key and, for top-p rows, a 1,024-bin histogram of
//     probability mass over key >> 6 (relative to the chunk's max).  The last
//     workgroup writes a greedy row's id, or finds the row's top-p boundary
//     bin: the bin where the mass accumulated from the top reaches top_p of
//     the total.
//   pass 2 (sampled rows): the exponential race (Gumbel-max):
//     argmax_i (s_i * log2 e - log2(-log2 u_i)), which selects i with
//     probability proportional to exp(s_i), over the tokens above the
//     boundary bin, and for the boundary bin's 64 keys their mass and race
//     winner per key.  The last workgroup resolves the boundary key exactly
//     (ties at it kept) and picks the winner over the kept tokens.
// u_i comes from Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011) with counter (token / 4, row,
// offset) and key = seed; the last workgroup of pass 2 advances the offset.
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
constexpr int kBins = 1024;          // pass-1 bins: key >> 6
constexpr int kSub = 64;             // keys per bin
constexpr int kNW = kT / 64;
constexpr int kMaxChunks = 256;      // vocabularies up to 1,048,576 tokens
// 16-bit keys: the bf16 order key, with NaN (either sign) as 0xFFFF -- above
// +inf, whose key is 0xFF80 -- and 0 marking a slot past the vocabulary (no
// bf16 value maps to 0: -inf is 0x007F).
constexpr uint32_t kNaN16 = 0xFFFFu;

struct RowInfo {
  float smax;    // max scaled logit x log2 e
  int bstar;     // boundary bin, -1: every token is kept
  float above;   // mass of the bins above it (relative to the max)
  float target;  // top_p x total mass
};

struct SampleParams {
  const uint16_t* logits;
  int64_t stride;
  int batch, vocab, chunks;
  const float* temperature;
  const float* top_p;
  uint2 seed;
  uint64_t* offset;
  int64_t* out;
  // workspace (zero counters between calls)
  int* cnt1;
  int* cnt2;
  int* done;
  RowInfo* info;
  uint32_t* p1_max;
  unsigned long long* p1_arg;
  float* p1_bins;
  unsigned long long* p2_best;
  float* p2_sub_mass;
  unsigned long long* p2_sub_best;
};

// (key, index) argmax: larger key wins, lower index breaks ties.
__device__ __forceinline__ void better(uint32_t& bk, int& bi, uint32_t k, int i) {
  if (k > bk || (k == bk && i < bi)) {
    bk = k;
    bi = i;
  }
}
__device__ __forceinline__ void betterf(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// (value, index) argmax across lanes without LDS: each step fetches a
// partner's pair with a DPP or lane-swap move and keeps the better one.
template <typename F>
__device__ __forceinline__ void arg_take(F& bv, int& bi, uint32_t ov_bits, int oi) {
  const F ov = __builtin_bit_cast(F, ov_bits);
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}
template <int CTRL, typename F>
__device__ __forceinline__ void arg_dpp(F& bv, int& bi) {
  const uint32_t ov = uint32_t(__builtin_amdgcn_update_dpp(0, int(__builtin_bit_cast(uint32_t, bv)), CTRL, 0xf, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xf, 0xf, false);
  arg_take(bv, bi, ov, oi);
}
// Every lane of each aligned group of 16 ends with the group's best pair.
template <typename F>
__device__ __forceinline__ void group16_argmax(F& bv, int& bi) {
  arg_dpp<mi::kDppQuadSwap1>(bv, bi);
  arg_dpp<mi::kDppQuadSwap2>(bv, bi);
  arg_dpp<mi::kDppRowHalfMirror>(bv, bi);
  arg_dpp<mi::kDppRowMirror>(bv, bi);
}
// The swaps exchange values between lane halves; both results are taken
// (one of them is the lane's own pair, which changes nothing).
template <typename F>
__device__ __forceinline__ void wave_argmax(F& bv, int& bi) {
  group16_argmax(bv, bi);
  {
    const uint32_t v = __builtin_bit_cast(uint32_t, bv);
    const auto rv = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(uint32_t(bi), uint32_t(bi), false, false);
    arg_take(bv, bi, rv[0], int(ri[0]));
    arg_take(bv, bi, rv[1], int(ri[1]));
  }
  {
    const uint32_t v = __builtin_bit_cast(uint32_t, bv);
    const auto rv = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(uint32_t(bi), uint32_t(bi), false, false);
    arg_take(bv, bi, rv[0], int(ri[0]));
    arg_take(bv, bi, rv[1], int(ri[1]));
  }
}

// Workgroup argmax (larger value, then lower index) over kNW waves; every
// thread gets the result.  `lowest` ranks below every candidate.  sv / si
// hold one pair per wave; the call starts and ends with them free.
template <typename F, int NW = kNW>
__device__ __forceinline__ void block_argmax(F& bv, int& bi, F* sv, int* si, F lowest) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  wave_argmax(bv, bi);
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  F v = lowest;
  int i = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    const F ov = sv[k];
    const int oi = si[k];
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  bv = v;
  bi = i;
  __syncthreads();
}

template <int NW = kNW>
__device__ __forceinline__ float block_sum(float x, float* sf) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  x = mi::wave_sum(x);
  if (lane == 0) sf[w] = x;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NW; ++k) s += sf[k];
  __syncthreads();
  return s;
}

// (value, index) packed so that a larger u64 is a larger value, then a lower
// index: the value's order-preserving bits above the complemented index.
__device__ __forceinline__ uint32_t f32_order(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ unsigned long long pack_arg(uint32_t ordered, int idx) {
  return (static_cast<unsigned long long>(ordered) << 32) | uint32_t(~uint32_t(idx));
}
__device__ __forceinline__ int arg_index(unsigned long long pk) { return int(~uint32_t(pk)); }

template <typename F>
__device__ __forceinline__ F coherent_load(const F* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename F>
__device__ __forceinline__ void coherent_store(F* p, F v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte device-coherent (sc1) buffer accesses for the histograms: the
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

__global__ __launch_bounds__(kT) void sample_pass1(SampleParams p) {
  __shared__ float bins[kNW][kBins];  // one copy per wave: fewer colliding LDS atomics
  __shared__ float s_scale[kMaxChunks];
  __shared__ uint32_t sv[kNW];
  __shared__ int si[kNW];
  __shared__ float sf[kNW];
  __shared__ int s_flag;
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const RowParams rp = row_params(p, row);
  const bool hist = !rp.greedy && rp.tp < 1.0f;
  if (hist)
    for (int i = tid; i < kNW * kBins; i += kT) (&bins[0][0])[i] = 0.f;
  uint32_t k[kGroupsPerThread][4];
  int g[kGroupsPerThread];
  chunk_keys(p, row, c, rp, k, g);
  uint32_t bk = 0;
  int bi = 0x7fffffff;
#pragma unroll
  for (int n = 0; n < kGroupsPerThread; ++n)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (k[n][e]) better(bk, bi, k[n][e], 4 * g[n] + e);
  block_argmax<uint32_t>(bk, bi, sv, si, 0u);  // ends with a barrier: bins are zeroed
  const int pc = row * p.chunks + c;
  if (rp.greedy) {
    if (tid == 0) coherent_store(&p.p1_arg[pc], pack_arg(bk, bi));
  } else {
    if (tid == 0) coherent_store(&p.p1_max[pc], bk);
    if (hist && has_mass(bk)) {
      const float smax_c = key_to_f32(bk) * mi::kLog2e;
#pragma unroll
      for (int n = 0; n < kGroupsPerThread; ++n)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kk = k[n][e];
          if (kk == 0u || kk == kNaN16) continue;
          atomicAdd(&bins[tid >> 6][kk >> 6], __builtin_amdgcn_exp2f(key_to_f32(kk) * mi::kLog2e - smax_c));
        }
    }
    if (hist) {
      __syncthreads();
      static_assert(kBins == 4 * kT, "one 16-byte store of 4 bins per thread");
      const __amdgpu_buffer_rsrc_t rb = rsrc_of(p.p1_bins + size_t(pc) * kBins, kBins * sizeof(float));
      float b4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        b4[q] = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < kNW; ++c2) b4[q] += bins[c2][4 * tid + q];
      }
      const u32x4_t v = {__float_as_uint(b4[0]), __float_as_uint(b4[1]), __float_as_uint(b4[2]), __float_as_uint(b4[3])};
      __builtin_amdgcn_raw_buffer_store_b128(v, rb, 16 * tid, 0, kCacheSc1);
    }
  }
  if (!last_of_row(&p.cnt1[row], p.chunks, &s_flag)) return;

  // ---- the row's last workgroup
  const int base = row * p.chunks;
  if (rp.greedy) {
    unsigned long long best = 0;
    for (int cc = tid; cc < p.chunks; cc += kT) best = max(best, coherent_load(&p.p1_arg[base + cc]));
    uint32_t hi = uint32_t(best >> 32);
    int lo = arg_index(best);
    block_argmax<uint32_t>(hi, lo, sv, si, 0u);
    if (tid == 0) p.out[row] = (hi != 0u && lo < p.vocab) ? lo : 0;
    return;
  }
  uint32_t M = 0;
  for (int cc = tid; cc < p.chunks; cc += kT) M = max(M, coherent_load(&p.p1_max[base + cc]));
  {
    int unused = 0;
    block_argmax<uint32_t>(M, unused, sv, si, 0u);
  }
  RowInfo ri;
  ri.smax = has_mass(M) ? key_to_f32(M) * mi::kLog2e : 0.f;
  ri.bstar = -1;
  ri.above = 0.f;
  ri.target = 0.f;
  if (hist && has_mass(M)) {
    // thread t owns bins 4t .. 4t + 3: H = sum over chunks of the chunk's
    // bins x 2^(chunk max - row max)
    // each chunk's scale (0: it carries no mass and wrote no bins), then
    // its bins, eight chunks' loads in flight at a time
    for (int cc = tid; cc < p.chunks; cc += kT) {
      const uint32_t mc = coherent_load(&p.p1_max[base + cc]);
      s_scale[cc] = has_mass(mc) ? __builtin_amdgcn_exp2f(key_to_f32(mc) * mi::kLog2e - ri.smax) : 0.f;
    }
    __syncthreads();
    float H[4] = {0.f, 0.f, 0.f, 0.f};
    const __amdgpu_buffer_rsrc_t rb = rsrc_of(p.p1_bins + size_t(base) * kBins, size_t(p.chunks) * kBins * 4);
    for (int c0 = 0; c0 < p.chunks; c0 += 8) {
      u32x4_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = __builtin_amdgcn_raw_buffer_load_b128(rb, ((c0 + u) * kBins + 4 * tid) * 4, 0, kCacheSc1);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (c0 + u >= p.chunks) break;
        const float sc = s_scale[c0 + u];
        if (sc == 0.f) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) H[q] += __uint_as_float(v[u][q]) * sc;
      }
    }
    const float mine = H[0] + H[1] + H[2] + H[3];
    const float Z = block_sum(mine, sf);
    const float target = rp.tp * Z;
    // mass strictly above bin 4t + 3: the bins of threads t' > t (a suffix
    // scan over the workgroup: inclusive prefix from the top)
    float incl = mine;  // becomes sum over threads >= t
    const int lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_down(incl, o);
      if (lane + o < 64) incl += y;
    }
    if (lane == 0) sf[w] = incl;  // wave totals
    __syncthreads();
    float later = 0.f;
#pragma unroll
    for (int q = 0; q < kNW; ++q) later += (q > w) ? sf[q] : 0.f;
    __syncthreads();
    float a = incl + later - mine;  // mass of bins above 4t + 3
    // the boundary: the bin b with H[b] > 0 and above(b) < target <= above(b) + H[b]
    int pick = -1, lowest = -1;
    float pick_above = 0.f;
#pragma unroll
    for (int q = 3; q >= 0; --q) {
      if (H[q] > 0.f) {
        if (pick < 0 && a < target && a + H[q] >= target) {
          pick = 4 * tid + q;
          pick_above = a;
        }
        lowest = 4 * tid + q;
      }
      a += H[q];
    }
    // one thread holds the boundary (argmax of "found", lowest bin first);
    // if rounding left none, the lowest non-empty bin (every token kept down
    // to it)
    uint32_t has = pick >= 0 ? 1u : 0u;
    int bsel = pick >= 0 ? pick : 0x7fffffff;
    block_argmax<uint32_t>(has, bsel, sv, si, 0u);
    uint32_t nonempty = lowest >= 0 ? 1u : 0u;
    int lo_bin = lowest >= 0 ? lowest : 0x7fffffff;
    block_argmax<uint32_t>(nonempty, lo_bin, sv, si, 0u);
    if (has) {
      ri.bstar = bsel;
      // the thread that found it publishes its `above`
      if (pick >= 0) sf[0] = pick_above;
      __syncthreads();
      ri.above = sf[0];
    } else {
      ri.bstar = lo_bin;
      ri.above = 0.f;  // unused: the boundary key search falls back to the lowest non-empty key
    }
    ri.target = has ? target : INFINITY;
  }
  if (tid == 0) p.info[row] = ri;
}

__global__ __launch_bounds__(kT) void sample_pass2(SampleParams p) {
  __shared__ float sub_mass[kNW][kSub];  // one copy per wave
  __shared__ unsigned long long sub_best[kNW][kSub];
  __shared__ float svf[kNW];
  __shared__ int si[kNW];
  __shared__ int s_flag;
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const RowParams rp = row_params(p, row);
  if (!rp.greedy) {
    const RowInfo ri = p.info[row];
    const uint64_t off = *p.offset;
    if (ri.bstar >= 0) {
      (&sub_mass[0][0])[tid] = 0.f;  // kT == kNW * kSub
      (&sub_best[0][0])[tid] = 0ull;
    }
    __syncthreads();
    uint32_t k[kGroupsPerThread][4];
    int g[kGroupsPerThread];
    chunk_keys(p, row, c, rp, k, g);
    const uint32_t kmin = ri.bstar < 0 ? 1u : uint32_t(ri.bstar) << 6;  // lowest key that may be kept
    float bv = -INFINITY;
    int bi = 0x7fffffff;
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
        if (kk < kmin) continue;
        const int i = 4 * g[n] + e;
        float v;
        float sc = 0.f;
        if (kk == kNaN16) {
          v = INFINITY;
        } else {
          sc = key_to_f32(kk);
          if (sc == -INFINITY) continue;
          v = sc * mi::kLog2e - __log2f(-__log2f(u01(rr[e])));
        }
        if (ri.bstar >= 0 && int(kk >> 6) == ri.bstar) {
          atomicAdd(&sub_mass[tid >> 6][kk & 63], __builtin_amdgcn_exp2f(sc * mi::kLog2e - ri.smax));
          atomicMax(&sub_best[tid >> 6][kk & 63], pack_arg(f32_order(v), i));
        } else {
          betterf(bv, bi, v, i);
        }
      }
    }
    block_argmax<float>(bv, bi, svf, si, -INFINITY);  // ends with a barrier: sub_* are complete
    const int pc = row * p.chunks + c;
    if (tid == 0) coherent_store(&p.p2_best[pc], bi == 0x7fffffff ? 0ull : pack_arg(f32_order(bv), bi));
    if (ri.bstar >= 0 && tid < kSub) {
      float m = 0.f;
      unsigned long long b = 0;
#pragma unroll
      for (int c2 = 0; c2 < kNW; ++c2) {
        m += sub_mass[c2][tid];
        b = max(b, sub_best[c2][tid]);
      }
      coherent_store(&p.p2_sub_mass[size_t(pc) * kSub + tid], m);
      coherent_store(&p.p2_sub_best[size_t(pc) * kSub + tid], b);
    }
    if (last_of_row(&p.cnt2[row], p.chunks, &s_flag)) {
      const int base = row * p.chunks;
      unsigned long long best = 0;
      for (int cc = tid; cc < p.chunks; cc += kT) best = max(best, coherent_load(&p.p2_best[base + cc]));
      if (ri.bstar >= 0) {
        // wave 0: lane s holds key (bstar << 6) | s of the boundary bin
        if (tid < 64) {
          float m = 0.f;
          unsigned long long b = 0;
          for (int c0 = 0; c0 < p.chunks; c0 += 8) {
            float mv[8];
            unsigned long long bv8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const int cc = min(c0 + u, p.chunks - 1);
              mv[u] = coherent_load(&p.p2_sub_mass[size_t(base + cc) * kSub + tid]);
              bv8[u] = coherent_load(&p.p2_sub_best[size_t(base + cc) * kSub + tid]);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              if (c0 + u >= p.chunks) break;
              m += mv[u];
              b = max(b, bv8[u]);
            }
          }
          // mass of the bin's keys above lane s: suffix sum over lanes > s
          float incl = m;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_down(incl, o);
            if (tid + o < 64) incl += y;
          }
          const float above = ri.above + incl - m;
          const uint64_t hit = __ballot(m > 0.f && above < ri.target && above + m >= ri.target);
          const uint64_t nonempty = __ballot(m > 0.f);
          // the boundary key; if rounding left none, the lowest non-empty key
          const int sstar = hit ? 63 - __builtin_clzll(hit) : (nonempty ? __builtin_ctzll(nonempty) : 64);
          if (tid < sstar) b = 0;  // below the boundary: not kept
          // max over the wave
          for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long ob =
                (static_cast<unsigned long long>(uint32_t(__shfl_xor(int(b >> 32), o))) << 32) |
                uint32_t(__shfl_xor(int(uint32_t(b)), o));
            b = max(b, ob);
          }
          if (tid == 0) sub_best[0][0] = b;
        }
        __syncthreads();
        best = max(best, sub_best[0][0]);
      }
      // the row's best over its chunks (thread 0 holds chunk 0's; reduce)
      {
        uint32_t hi = uint32_t(best >> 32);
        int lo = best ? arg_index(best) : 0x7fffffff;
        block_argmax<uint32_t>(hi, lo, reinterpret_cast<uint32_t*>(svf), si, 0u);
        if (tid == 0) p.out[row] = (hi != 0u && lo < p.vocab) ? lo : 0;
      }
    }
  }
  // every workgroup of the grid counts itself; the last one advances the
  // draw offset (every workgroup has read it by then)
  if (tid == 0) {
    const int total = p.chunks * p.batch;
    if (__hip_atomic_fetch_add(p.done, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == total - 1) {
      coherent_store(p.offset, coherent_load(p.offset) + 1);
      coherent_store(p.done, 0);
    }
  }
}

constexpr int kMaxRows = 65535;

struct SampleLayout {
  size_t cnt1, cnt2, done, info, p1_max, p1_arg, p1_bins, p2_best, p2_sub_mass, p2_sub_best, total;
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
  // them (every call leaves them at zero)
  L.cnt1 = take(size_t(kMaxRows) * sizeof(int));
  L.cnt2 = take(size_t(kMaxRows) * sizeof(int));
  L.done = take(sizeof(int));
  L.info = take(size_t(batch) * sizeof(RowInfo));
  L.p1_max = take(rc * sizeof(uint32_t));
  L.p1_arg = take(rc * sizeof(unsigned long long));
  L.p1_bins = take(rc * kBins * sizeof(float));
  L.p2_best = take(rc * sizeof(unsigned long long));
  L.p2_sub_mass = take(rc * kSub * sizeof(float));
  L.p2_sub_best = take(rc * kSub * sizeof(unsigned long long));
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
  sp.cnt1 = reinterpret_cast<int*>(ws + L.cnt1);
  sp.cnt2 = reinterpret_cast<int*>(ws + L.cnt2);
  sp.done = reinterpret_cast<int*>(ws + L.done);
  sp.info = reinterpret_cast<RowInfo*>(ws + L.info);
  sp.p1_max = reinterpret_cast<uint32_t*>(ws + L.p1_max);
  sp.p1_arg = reinterpret_cast<unsigned long long*>(ws + L.p1_arg);
  sp.p1_bins = reinterpret_cast<float*>(ws + L.p1_bins);
  sp.p2_best = reinterpret_cast<unsigned long long*>(ws + L.p2_best);
  sp.p2_sub_mass = reinterpret_cast<float*>(ws + L.p2_sub_mass);
  sp.p2_sub_best = reinterpret_cast<unsigned long long*>(ws + L.p2_sub_best);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(chunks), unsigned(batch_size), 1u};
  hipLaunchKernelGGL(sample_pass1, grid, dim3(kT), 0, s, sp);
  int rc = mi::check_launch("sample_pass1");
  if (rc) return rc;
  hipLaunchKernelGGL(sample_pass2, grid, dim3(kT), 0, s, sp);
  return mi::check_launch("sample_pass2");
}
