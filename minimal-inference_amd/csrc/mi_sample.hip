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
// One 1024-thread workgroup per row.  Rows of up to 40,960 tokens are read
// once: the 16-bit keys of the scaled logits go to LDS, and every later pass
// (top-p radix passes, draw) works on those; larger vocabularies re-read and
// re-scale the row per pass.  The draw is an exponential race
// (Gumbel-max): argmax_i (s_i * log2 e - log2(-log2 u_i)), which selects i with
// probability proportional to exp(s_i); u_i comes from Philox4x32-10 (Salmon,
// Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011)
// with counter (token / 4, row, offset) and key = seed.  The top-p boundary
// is found exactly on the 16-bit bf16 key of s_i with four 4-bit radix passes
// of probability mass (per-thread LDS bins, no atomics), so no sort is needed.
#include <math.h>

#include "mi_common.h"

namespace {

constexpr int kThreads = 1024;
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

struct SampleParams {
  const uint16_t* logits;
  int64_t stride;
  int batch, vocab;
  const float* temperature;
  const float* top_p;
  uint2 seed;
  const uint64_t* offset;
  int64_t* out;
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

// Workgroup argmax (larger value, then lower index); every thread gets the
// result.  `lowest` ranks below every candidate.  sv / si hold one pair per
// wave; the call starts and ends with them free.
template <typename F>
__device__ __forceinline__ void block_argmax(F& bv, int& bi, F* sv, int* si, F lowest) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  wave_argmax(bv, bi);
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  F v = lane < kThreads / 64 ? sv[lane] : lowest;
  int i = lane < kThreads / 64 ? si[lane] : 0x7fffffff;
  group16_argmax(v, i);  // the kThreads / 64 = 16 pairs sit in lanes 0..15
  bv = __builtin_bit_cast(F, uint32_t(__builtin_amdgcn_readfirstlane(int(__builtin_bit_cast(uint32_t, v)))));
  bi = __builtin_amdgcn_readfirstlane(i);
  __syncthreads();
}

__global__ __launch_bounds__(kThreads) void sample_kernel(SampleParams p) {
  __shared__ float bins[16 * kThreads];  // per-thread private radix bins
  __shared__ float bin_tot[16];
  __shared__ uint32_t sh_u[16];
  __shared__ float sh_f[16];
  __shared__ int sh_i[16];
  __shared__ uint32_t sh_prefix;
  __shared__ float sh_above, sh_target;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* x = p.logits + int64_t(row) * p.stride;
  const int V = p.vocab;

  const uint16_t tb = mi::f32_to_bf16(p.temperature[row]);
  const float tq = mi::bf16_to_f32(tb);
  const bool greedy = !(tq > 0.f);  // <= 0 (and NaN) is greedy

  if (greedy) {
    uint32_t bk = 0;
    int bi = 0x7fffffff;
    for (int i = tid; i < V; i += kThreads) better(bk, bi, bf16_key(x[i]), i);
    block_argmax<uint32_t>(bk, bi, sh_u, sh_i, 0u);
    if (tid == 0) p.out[row] = bi < V ? bi : 0;
    return;
  }

  // clamp(min=1e-6) in bf16, then s_i = bf16(logit_i / t)
  const float tmin = mi::bf16_to_f32(mi::f32_to_bf16(1e-6f));
  const float tc = fmaxf(tq, tmin);
  auto scaled = [&](int i) -> uint16_t { return mi::cvt_bf16(mi::bf16_to_f32(x[i]) / tc); };

  // ---- max key
  uint32_t mk = 0;
  {
    int unused = 0;
    for (int i = tid; i < V; i += kThreads) better(mk, unused, bf16_key(scaled(i)), 0);
    block_argmax<uint32_t>(mk, unused, sh_u, sh_i, 0u);
  }
  const float smax = key_to_f32(mk) * mi::kLog2e;

  uint32_t kstar = 0;
  const float tp = p.top_p ? p.top_p[row] : 1.0f;
  if (tp < 1.0f && mk != kNaNKey) {
    uint32_t prefix = 0;
    if (tid == 0) sh_above = 0.f;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 12 - 4 * pass;
#pragma unroll
      for (int d = 0; d < 16; ++d) bins[d * kThreads + tid] = 0.f;
      for (int i = tid; i < V; i += kThreads) {
        const uint32_t k = bf16_key(scaled(i));
        if (k == kNaNKey) continue;
        if (pass > 0 && (k >> (shift + 4)) != prefix) continue;
        const float mass = __builtin_amdgcn_exp2f(key_to_f32(k) * mi::kLog2e - smax);
        bins[((k >> shift) & 15) * kThreads + tid] += mass;
      }
      __syncthreads();
      {
        const int w = tid >> 6, lane = tid & 63;  // wave w sums digit w
        float s = 0.f;
        for (int j = lane; j < kThreads; j += 64) s += bins[w * kThreads + j];
        s = mi::wave_sum(s);
        if (lane == 0) bin_tot[w] = s;
      }
      __syncthreads();
      if (tid == 0) {
        if (pass == 0) {
          float z = 0.f;
          for (int d = 0; d < 16; ++d) z += bin_tot[d];
          sh_target = tp * z;
        }
        float above = sh_above;
        int pick = -1, lowest = -1;
        for (int d = 15; d >= 0; --d) {
          if (bin_tot[d] <= 0.f) continue;
          lowest = d;
          if (above + bin_tot[d] >= sh_target) {
            pick = d;
            break;
          }
          above += bin_tot[d];
        }
        if (pick < 0) {  // rounding left the target unreached: take the last digit
          pick = lowest < 0 ? 0 : lowest;
          above = sh_above;
          for (int d = 15; d > pick; --d) above += bin_tot[d];
        }
        sh_above = above;
        sh_prefix = (prefix << 4) | uint32_t(pick);
      }
      __syncthreads();
      prefix = sh_prefix;
      __syncthreads();
    }
    kstar = prefix;
  }

  // ---- exponential race over the kept tokens
  const uint64_t off = *p.offset;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int g = tid; g * 4 < V; g += kThreads) {
    const uint4 r = philox4x32_10(make_uint4(uint32_t(g), uint32_t(row), uint32_t(off), uint32_t(off >> 32)), p.seed);
    const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * g + e;
      if (i >= V) break;
      const uint32_t k = bf16_key(scaled(i));
      if (k < kstar) continue;
      float v;
      if (k == kNaNKey) {
        v = INFINITY;
      } else {
        const float s = key_to_f32(k);
        if (s == -INFINITY) continue;
        v = s * mi::kLog2e - __log2f(-__log2f(u01(rr[e])));
      }
      betterf(bv, bi, v, i);
    }
  }
  block_argmax<float>(bv, bi, sh_f, sh_i, -INFINITY);
  if (tid == 0) p.out[row] = bi < V ? bi : 0;
}

// ---------------------------------------------------------------- cached rows
// 16-bit keys for the register cache: the bf16 order key, with NaN (either
// sign) as 0xFFFF -- above +inf, whose key is 0xFF80 -- and 0 marking a slot
// past the vocabulary (no bf16 value maps to 0: -inf is 0x007F).
constexpr uint32_t kNaN16 = 0xFFFFu;
__device__ __forceinline__ uint32_t key16(uint16_t b) {
  const uint32_t k = bf16_key(b);
  return k == kNaNKey ? kNaN16 : k;
}

// Keys of rows up to kCachedVocab tokens live in LDS (80 KB) next to the
// radix bins (64 KB); one workgroup per CU either way.
constexpr int kCachedVocab = 40960;

__global__ __launch_bounds__(kThreads) void sample_cached_kernel(SampleParams p) {
  __shared__ float bins[16 * kThreads];  // per-thread private radix bins
  __shared__ uint2 keys[kCachedVocab / 4];  // 4 packed 16-bit keys per group
  __shared__ float bin_tot[16];
  __shared__ uint32_t sh_u[16];
  __shared__ float sh_f[16];
  __shared__ int sh_i[16];
  __shared__ uint32_t sh_prefix;
  __shared__ float sh_above, sh_target;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* x = p.logits + int64_t(row) * p.stride;
  const int V = p.vocab;
  const int NG = (V + 3) / 4;  // 4-token groups; group g = tokens 4g .. 4g+3 (the draw's Philox counter)
  const uint16_t tb = mi::f32_to_bf16(p.temperature[row]);
  const float tq = mi::bf16_to_f32(tb);
  const bool greedy = !(tq > 0.f);  // <= 0 (and NaN) is greedy
  const float tmin = mi::bf16_to_f32(mi::f32_to_bf16(1e-6f));
  const float tc = fmaxf(tq, tmin);
  auto key_of = [](uint2 w, int e) -> uint32_t { return ((e < 2 ? w.x : w.y) >> (16 * (e & 1))) & 0xffffu; };

  // ---- read the row once: keys of the raw logits (greedy rows) or of
  // bf16(x / t) (sampled rows); 0 past the vocabulary.  All of a thread's
  // loads are issued before any is used (one memory round trip).
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 7) == 0;
  uint32_t bk = 0, mk = 0;
  int bi = 0x7fffffff;
  constexpr int kMaxG = kCachedVocab / 4 / kThreads;  // groups per thread
  uint16_t raw[kMaxG][4];
#pragma unroll
  for (int n = 0; n < kMaxG; ++n) {
    const int t0 = 4 * (tid + n * kThreads);
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
  for (int n = 0; n < kMaxG; ++n) {
    const int gi = tid + n * kThreads;
    if (gi >= NG) break;
    const int t0 = 4 * gi;
    const uint16_t* v = raw[n];
    uint32_t k[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // bf16(x / t): the fp32 quotient rounded to nearest even by v_cvt_pk_bf16_f32
      const uint16_t sv = greedy ? v[e] : mi::cvt_bf16(mi::bf16_to_f32(v[e]) / tc);
      k[e] = (t0 + e < V) ? key16(sv) : 0u;
      if (t0 + e < V) better(bk, bi, k[e], t0 + e);
      mk = max(mk, k[e]);
    }
    keys[gi] = make_uint2(k[0] | (k[1] << 16), k[2] | (k[3] << 16));
  }

  if (greedy) {
    block_argmax<uint32_t>(bk, bi, sh_u, sh_i, 0u);
    if (tid == 0) p.out[row] = bi < V ? bi : 0;
    return;
  }
  {
    int unused = 0;
    block_argmax<uint32_t>(mk, unused, sh_u, sh_i, 0u);  // ends with barriers: keys[] is complete
  }
  const float smax = key_to_f32(mk) * mi::kLog2e;

  // ---- top-p boundary key: four 4-bit radix passes over the cached keys
  uint32_t kstar = 0;
  const float tp = p.top_p ? p.top_p[row] : 1.0f;
  if (tp < 1.0f && mk != kNaN16) {
    uint32_t prefix = 0;
    if (tid == 0) sh_above = 0.f;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 12 - 4 * pass;
#pragma unroll
      for (int d = 0; d < 16; ++d) bins[d * kThreads + tid] = 0.f;
      for (int gi = tid; gi < NG; gi += kThreads) {
        const uint2 w = keys[gi];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t k = key_of(w, e);
          if (k == 0u || (pass > 0 && (k >> (shift + 4)) != prefix)) continue;
          const float mass = __builtin_amdgcn_exp2f(key_to_f32(k) * mi::kLog2e - smax);
          bins[((k >> shift) & 15) * kThreads + tid] += mass;  // private bin
        }
      }
      __syncthreads();
      {
        const int w = tid >> 6, lane = tid & 63;  // wave w sums digit w
        float s = 0.f;
        for (int j = lane; j < kThreads; j += 64) s += bins[w * kThreads + j];
        s = mi::wave_sum(s);
        if (lane == 0) bin_tot[w] = s;
      }
      __syncthreads();
      if (tid < 64) {
        // Wave 0, lane d < 16 holds digit d's mass.  The digit is the highest
        // non-empty d whose mass together with everything above it (the
        // masses above the current prefix, plus digits > d) reaches the
        // target; if rounding leaves the target unreached, the lowest
        // non-empty digit.
        const int lane = tid;
        const float bt = lane < 16 ? bin_tot[lane] : 0.f;
        float target;
        if (pass == 0) {
          target = tp * mi::wave_sum(bt);
          if (lane == 0) sh_target = target;
        } else {
          target = sh_target;
        }
        float c = bt;  // suffix sum over digits >= lane
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float up = __shfl_down(c, o);
          if (lane + o < 16) c += up;
        }
        const float above0 = sh_above;
        const uint64_t hit = __ballot(lane < 16 && bt > 0.f && above0 + c >= target);
        const uint64_t nonempty = __ballot(lane < 16 && bt > 0.f);
        const int pick = hit ? 63 - __builtin_clzll(hit) : (nonempty ? __builtin_ctzll(nonempty) : 0);
        const float c_above = __shfl(c, pick + 1);  // digits > pick (lane 16 holds 0)
        if (lane == 0) {
          sh_above = above0 + (pick + 1 < 16 ? c_above : 0.f);
          sh_prefix = (prefix << 4) | uint32_t(pick);
        }
      }
      __syncthreads();
      prefix = sh_prefix;
      __syncthreads();
    }
    kstar = prefix;
  }

  // ---- exponential race over the kept tokens; a group with no kept token
  // skips its Philox block
  const uint64_t off = *p.offset;
  float bv = -INFINITY;
  bi = 0x7fffffff;
  for (int gi = tid; gi < NG; gi += kThreads) {
    const uint2 w = keys[gi];
    bool any = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) any = any || (4 * gi + e < V && key_of(w, e) >= kstar);
    if (!any) continue;
    const uint4 r = philox4x32_10(make_uint4(uint32_t(gi), uint32_t(row), uint32_t(off), uint32_t(off >> 32)), p.seed);
    const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * gi + e;
      const uint32_t k = key_of(w, e);
      if (i >= V || k < kstar) continue;
      float v;
      if (k == kNaN16) {
        v = INFINITY;
      } else {
        const float sc = key_to_f32(k);
        if (sc == -INFINITY) continue;
        v = sc * mi::kLog2e - __log2f(-__log2f(u01(rr[e])));
      }
      betterf(bv, bi, v, i);
    }
  }
  block_argmax<float>(bv, bi, sh_f, sh_i, -INFINITY);
  if (tid == 0) p.out[row] = bi < V ? bi : 0;
}

__global__ void advance_offset_kernel(uint64_t* off) {
  if (threadIdx.x == 0 && blockIdx.x == 0) off[0] += 1;
}

}  // namespace

extern "C" int mi_sample(const void* logits, int64_t logits_row_stride, int32_t batch_size,
                         int32_t vocab_size, const float* temperature, const float* top_p,
                         uint64_t seed, uint64_t* rng_offset, int64_t* out_tokens, mi_stream_t stream) {
  mi::clear_error();
  if (batch_size < 0 || vocab_size <= 0 || logits_row_stride < vocab_size)
    return mi::fail(MI_ERR_INVALID, "sample: bad sizes (batch %d, vocab %d, stride %lld)", batch_size,
                    vocab_size, (long long)logits_row_stride);
  if (batch_size == 0) return MI_OK;
  if (!logits || !temperature || !rng_offset || !out_tokens)
    return mi::fail(MI_ERR_INVALID, "sample: null pointer argument");
  SampleParams sp;
  sp.logits = static_cast<const uint16_t*>(logits);
  sp.stride = logits_row_stride;
  sp.batch = batch_size;
  sp.vocab = vocab_size;
  sp.temperature = temperature;
  sp.top_p = top_p;
  sp.seed = make_uint2(uint32_t(seed), uint32_t(seed >> 32));
  sp.offset = rng_offset;
  sp.out = out_tokens;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vocab_size <= kCachedVocab)
    hipLaunchKernelGGL(sample_cached_kernel, dim3(batch_size), dim3(kThreads), 0, s, sp);
  else
    hipLaunchKernelGGL(sample_kernel, dim3(batch_size), dim3(kThreads), 0, s, sp);
  int rc = mi::check_launch("sample_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(advance_offset_kernel, dim3(1), dim3(64), 0, s, rng_offset);
  return mi::check_launch("advance_offset_kernel");
}
