// Fused residual add + RMSNorm, and the SiLU-gated product, for the dense
// layers around the attention path.
//
// Reference: DecoderLayer.forward (model.py:324-344) adds each sub-layer's
// output to the residual stream and the next pre-norm RMSNorm
// (model.py:115-122, F.rms_norm with the norm weight) reads it; the MLP
// (model.py:301-311) is down(silu(gate(x)) * up(x)).  Here one kernel does
// the add and the following norm (two torch kernels), and one kernel the
// SiLU and the product (two torch kernels over strided halves of the fused
// gate/up projection).
//
//   add_rms  : x' = bf16(x + d) (the bf16 add: fp32 sum, rounded), written
//              back when asked; h = bf16(x' * rsqrt(mean(x'^2) + eps) * w),
//              all in fp32, one rounding;
//   silu_mul : out = bf16(bf16(g / (1 + exp(-g))) * u) -- silu in fp32 and
//              rounded to bf16 as torch's bf16 silu is, then the bf16 product.
#include <math.h>

#include <algorithm>

#include "mi_common.h"

namespace {

constexpr int kNormMaxThreads = 1024;
constexpr int kMaxChunks = 2;  // 16-byte chunks per thread: hidden <= 1024 * 2 * 8 = 16384

struct AddRmsParams {
  const uint16_t* x;
  int64_t x_stride;
  const uint16_t* delta;  // null: no add
  int64_t d_stride;
  const uint16_t* weight;
  uint16_t* x_out;  // null: the sum is not stored
  int64_t xo_stride;
  uint16_t* h_out;  // null: no norm
  int64_t h_stride;
  int hidden;
  float eps;
};

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// One workgroup per row, one or two 16-byte chunks per thread (up to 1,024
// threads): every load of the row -- x, delta and the norm weight -- is
// issued before anything is computed or stored (x may be written in place),
// so a row costs one memory round trip; the row stays in registers between
// the sum and the normalisation.
__global__ __launch_bounds__(kNormMaxThreads) void add_rms_kernel(AddRmsParams p) {
  __shared__ float red[kNormMaxThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int nch = p.hidden / 8;
  const uint16_t* x = p.x + row * p.x_stride;
  uint4 xv[kMaxChunks], dv[kMaxChunks], wv[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = tid + c * nt;
    xv[c] = dv[c] = wv[c] = make_uint4(0u, 0u, 0u, 0u);
    if (ch < nch) {
      // x and delta are read once (non-temporal: prefill rows 101 -> 91 us)
      xv[c] = mi::load16_nt(x + ch * 8);
      if (p.delta) dv[c] = mi::load16_nt(p.delta + row * p.d_stride + ch * 8);
      if (p.h_out) wv[c] = ld16(p.weight + ch * 8);
    }
  }
  float v[kMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = tid + c * nt;
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    const uint32_t dw[4] = {dv[c].x, dv[c].y, dv[c].z, dv[c].w};
    uint32_t ow[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // the bf16 add: fp32 sum rounded to bf16 (zeros past the row add nothing)
      ow[k] = p.delta ? mi::cvt_pk_bf16(mi::bf16_lo(xw[k]) + mi::bf16_lo(dw[k]), mi::bf16_hi(xw[k]) + mi::bf16_hi(dw[k]))
                      : xw[k];
      const float a = mi::bf16_lo(ow[k]), b = mi::bf16_hi(ow[k]);
      v[c][2 * k] = a;
      v[c][2 * k + 1] = b;
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
    if (p.x_out && ch < nch) st16(p.x_out + row * p.xo_stride + ch * 8, make_uint4(ow[0], ow[1], ow[2], ow[3]));
  }
  if (!p.h_out) return;
  ss = mi::wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < nt / 64; ++w) tot += red[w];
  const float rstd = rsqrtf(tot / float(p.hidden) + p.eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = tid + c * nt;
    if (ch >= nch) break;
    const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
    uint32_t hw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      hw[k] = mi::cvt_pk_bf16(v[c][2 * k] * rstd * mi::bf16_lo(ww[k]), v[c][2 * k + 1] * rstd * mi::bf16_hi(ww[k]));
    st16(p.h_out + row * p.h_stride + ch * 8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
  }
}

struct SiluMulParams {
  const uint16_t* gu;
  int64_t gu_stride;
  uint16_t* out;
  int64_t o_stride;
  int inter;
  int64_t rows;
};

__device__ __forceinline__ float silu_bf16(float g) {
  return mi::bf16_to_f32(mi::f32_to_bf16(g / (1.0f + expf(-g))));
}

// One thread per 8 outputs (16 bytes of g, of u and of out).
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluMulParams p) {
  const int per_row = p.inter / 8;
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= p.rows * per_row) return;
  const int64_t row = t / per_row;
  const int ch = int(t - row * per_row);
  const uint16_t* g = p.gu + row * p.gu_stride + ch * 8;
  const uint4 gv = mi::load16_nt(g), uv = mi::load16_nt(g + p.inter);
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t ow[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    ow[k] = mi::pack_bf16x2(silu_bf16(mi::bf16_lo(gw[k])) * mi::bf16_lo(uw[k]),
                            silu_bf16(mi::bf16_hi(gw[k])) * mi::bf16_hi(uw[k]));
  st16(p.out + row * p.o_stride + ch * 8, make_uint4(ow[0], ow[1], ow[2], ow[3]));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" int mi_add_rms_norm(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                               const void* weight, void* x_out, int64_t x_out_stride, void* h_out,
                               int64_t h_stride, int64_t rows, int32_t hidden, float eps, mi_stream_t stream) {
  mi::clear_error();
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > kNormMaxThreads * kMaxChunks * 8)
    return mi::fail(MI_ERR_INVALID, "add_rms_norm: hidden %d (multiple of 8, <= %d)", hidden,
                    kNormMaxThreads * kMaxChunks * 8);
  if (rows == 0) return MI_OK;
  if (!x || (h_out && !weight) || (!h_out && !x_out))
    return mi::fail(MI_ERR_INVALID, "add_rms_norm: null pointer argument");
  if (!aligned16(x) || (delta && !aligned16(delta)) || (weight && !aligned16(weight)) ||
      (x_out && !aligned16(x_out)) || (h_out && !aligned16(h_out)) || x_stride % 8 || delta_stride % 8 ||
      x_out_stride % 8 || h_stride % 8)
    return mi::fail(MI_ERR_INVALID, "add_rms_norm: rows must be 16-byte aligned");
  if (rows > 0x7fffffff) return mi::fail(MI_ERR_INVALID, "add_rms_norm: too many rows");
  AddRmsParams p;
  p.x = static_cast<const uint16_t*>(x);
  p.x_stride = x_stride;
  p.delta = static_cast<const uint16_t*>(delta);
  p.d_stride = delta_stride;
  p.weight = static_cast<const uint16_t*>(weight);
  p.x_out = static_cast<uint16_t*>(x_out);
  p.xo_stride = x_out_stride;
  p.h_out = static_cast<uint16_t*>(h_out);
  p.h_stride = h_stride;
  p.hidden = hidden;
  p.eps = eps;
  // a thread per 16-byte chunk up to 1,024 threads, two chunks each beyond
  const int nch = hidden / 8;
  const int threads = std::min(kNormMaxThreads, (nch + 63) / 64 * 64);
  hipLaunchKernelGGL(add_rms_kernel, dim3(uint32_t(rows)), dim3(threads), 0, static_cast<hipStream_t>(stream), p);
  return mi::check_launch("add_rms_kernel");
}

extern "C" int mi_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride, int64_t rows,
                           int32_t intermediate, mi_stream_t stream) {
  mi::clear_error();
  if (rows < 0 || intermediate <= 0 || intermediate % 8)
    return mi::fail(MI_ERR_INVALID, "silu_mul: intermediate %d (multiple of 8)", intermediate);
  if (rows == 0) return MI_OK;
  if (!gate_up || !out) return mi::fail(MI_ERR_INVALID, "silu_mul: null pointer argument");
  if (!aligned16(gate_up) || !aligned16(out) || gate_up_stride % 8 || out_stride % 8 ||
      gate_up_stride < 2 * int64_t(intermediate))
    return mi::fail(MI_ERR_INVALID, "silu_mul: rows must be 16-byte aligned, stride >= 2 * intermediate");
  SiluMulParams p;
  p.gu = static_cast<const uint16_t*>(gate_up);
  p.gu_stride = gate_up_stride;
  p.out = static_cast<uint16_t*>(out);
  p.o_stride = out_stride;
  p.inter = intermediate;
  p.rows = rows;
  const int64_t n = rows * (intermediate / 8);
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return mi::fail(MI_ERR_INVALID, "silu_mul: too many rows");
  hipLaunchKernelGGL(silu_mul_kernel, dim3(uint32_t(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return mi::check_launch("silu_mul_kernel");
}
