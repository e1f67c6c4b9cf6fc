// Paged KV append: scatter new K/V rows into their page slots.
//
// Reference call: model.py:207-216 (flashinfer.page.append_paged_kv_cache),
// NHD pool layout scheduler.py:195-202.  Slot placement is integer-exact:
// page = kv_indices[kv_indptr[b] + pos / page_size], slot = pos % page_size.
//
// One workgroup per token (grid-stride over tokens): the token's slot is a
// chain of wave-uniform scalar loads (batch index and position, the
// request's page-list start, the page id) done once per token, and each
// thread moves 16-byte chunks (8 bf16) of K and the same chunks of V, so a
// wave writes 1 KiB of contiguous head rows per instruction.  The plain
// append issues its first chunk's loads before the slot chain (18,240
// prompt rows: 24.2 -> 23.9 us).
#include <algorithm>

#include "mi_common.h"

#ifndef MI_APPEND_THREADS
#define MI_APPEND_THREADS 256
#endif

namespace {

struct AppendParams {
  const uint16_t* key;
  const uint16_t* value;
  int64_t ks_tok, ks_head, vs_tok, vs_head;
  const int32_t* batch_indices;
  const int32_t* positions;
  int64_t num_tokens;
  uint16_t* pool;
  int64_t num_pages;
  const int32_t* indices;
  const int32_t* indptr;
  int32_t batch_size, num_kv_heads, head_dim, page_size;
};

typedef __attribute__((address_space(4))) const int32_t const_i32;

// Base of token i's slot row in the pool (null: the token is not placed --
// bad batch index or position, slot outside request b's page list, or a page
// id outside the pool).  The index arrays are read through the constant
// address space: with a wave-uniform token index the loads are scalar.
__device__ __forceinline__ uint16_t* token_slot(const int32_t* batch_indices, const int32_t* positions,
                                                const int32_t* indptr, const int32_t* indices, int64_t i,
                                                int batch_size, int64_t num_pages, int page_size, uint16_t* pool,
                                                int64_t page_stride, int64_t tok_stride) {
  const const_i32* bi = (const const_i32*)batch_indices;
  const const_i32* ps = (const const_i32*)positions;
  const const_i32* ip = (const const_i32*)indptr;
  const const_i32* ix = (const const_i32*)indices;
  // three round trips: batch index and position together, then the
  // request's page-list bounds together, then the page id
  const int b = bi[i];
  const int pos = ps[i];
  const bool placed = (b >= 0) & (b < batch_size) & (pos >= 0);
  const int bc = placed ? b : 0;
  const int lo = ip[bc], hi = ip[bc + 1];
  const int64_t it = int64_t(lo) + (placed ? pos : 0) / page_size;
  if (!placed || it >= hi) return nullptr;
  const int64_t page = ix[it];
  if (page < 0 || page >= num_pages) return nullptr;
  return pool + page * page_stride + int64_t(pos % page_size) * tok_stride;
}

typedef __attribute__((ext_vector_type(4))) unsigned int ap_u32x4;
// Buffer resource word 3 for gfx9 raw buffers (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;

__global__ __launch_bounds__(256) void append_kernel(AppendParams p) {
  const int chunks = p.head_dim >> 3;
  const int per_token = p.num_kv_heads * chunks;
  const int64_t tok_stride = int64_t(p.num_kv_heads) * p.head_dim;
  const int64_t kv_stride = int64_t(p.page_size) * tok_stride;
  const int64_t page_stride = 2 * kv_stride;
  const int u0 = threadIdx.x;
  const int h0 = u0 / chunks, c0 = (u0 - h0 * chunks) * 8;
  for (int64_t i = blockIdx.x; i < p.num_tokens; i += gridDim.x) {
    // the first chunk's rows do not depend on the slot: their loads go out
    // before the slot's chain of scalar loads
    uint4 k0 = make_uint4(0, 0, 0, 0), v0 = make_uint4(0, 0, 0, 0);
    if (u0 < per_token) {
      k0 = mi::load16(p.key + i * p.ks_tok + h0 * p.ks_head + c0);
      v0 = mi::load16(p.value + i * p.vs_tok + h0 * p.vs_head + c0);
    }
    uint16_t* slot = token_slot(p.batch_indices, p.positions, p.indptr, p.indices, i, p.batch_size, p.num_pages,
                                p.page_size, p.pool, page_stride, tok_stride);
    // stores through a descriptor of the slot's row (size 0 when the token is
    // not placed: the stores write nothing), so the loads above are used on
    // every path and stay ahead of the chain
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        slot ? (void*)slot : (void*)p.pool, (short)0, slot ? int(kv_stride * 2 + tok_stride * 2) : 0, kBufferWord3);
    if (u0 < per_token) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(ap_u32x4, k0), rs, (h0 * p.head_dim + c0) * 2, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(ap_u32x4, v0), rs,
                                             int(kv_stride * 2) + (h0 * p.head_dim + c0) * 2, 0, 0);
    }
    for (int u = u0 + int(blockDim.x); u < per_token; u += blockDim.x) {
      const int h = u / chunks;
      const int c = (u - h * chunks) * 8;
      const uint4 kv = mi::load16(p.key + i * p.ks_tok + h * p.ks_head + c);
      const uint4 vv = mi::load16(p.value + i * p.vs_tok + h * p.vs_head + c);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(ap_u32x4, kv), rs, (h * p.head_dim + c) * 2, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(ap_u32x4, vv), rs,
                                             int(kv_stride * 2) + (h * p.head_dim + c) * 2, 0, 0);
    }
  }
}

// ------------------------------------------------------------ RoPE + append
// Rotate-half RoPE on the fused qkv rows, then the K/V append, in one pass.
//
// Replaces, per layer, the reference's apply_rotary_emb on q and k
// (model.py:92-107, called at model.py:169-170) followed by the append
// (model.py:203-216).  The arithmetic is mi::rope8: the reference's bf16
// composition x * cos + rotate_half(x) * sin with cos / sin already in bf16
// (server.py:251), bit-identical to the unfused ops.
//
// Work units per token: (H_q + H_kv) heads x D/16 rotate units (8 pairs
// (j, j + D/2) each: one 16-byte load from each half) and H_kv x D/8 copy
// units for V.  Q is written to q_out (may alias qkv's q columns: every unit
// reads both of its halves before writing them); rotated K and V go to the
// token's page slot with the same placement rule as append_kernel.
struct RopeAppendParams {
  const uint16_t* qkv;
  int64_t qkv_stride;  // elements between tokens; q heads, k heads, v heads contiguous
  const int32_t* rope_pos;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t table_rows;
  uint16_t* q_out;
  int64_t qo_stride_tok, qo_stride_head;
  const int32_t* batch_indices;
  const int32_t* positions;
  int64_t num_tokens;
  uint16_t* pool;
  int64_t num_pages;
  const int32_t* indices;
  const int32_t* indptr;
  int32_t batch_size, num_qo_heads, num_kv_heads, head_dim, page_size;
};

// One workgroup per token (grid-stride over tokens): the RoPE row and the
// slot are looked up once per token with scalar loads; the threads rotate
// the q heads first, then the k heads and copy the V chunks into the slot.
// The qkv rows are read once and loaded non-temporal (80 -> 71 us on 18,240
// rows of 32 / 8 heads; the same loads made the plain append slower, 26 ->
// 29 us, so append_kernel keeps ordinary loads).
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendParams p) {
  const int d = p.head_dim, half = d >> 1;
  const int upr = d >> 4;  // rotate units per head
  const int rot_units = (p.num_qo_heads + p.num_kv_heads) * upr;
  const int per_token = rot_units + p.num_kv_heads * (d >> 3);
  const int64_t tok_stride = int64_t(p.num_kv_heads) * d;
  const int64_t kv_stride = int64_t(p.page_size) * tok_stride;
  const int64_t page_stride = 2 * kv_stride;
  const const_i32* rope_pos = (const const_i32*)p.rope_pos;
  for (int64_t i = blockIdx.x; i < p.num_tokens; i += gridDim.x) {
    int rp = rope_pos[i];
    rp = rp < 0 ? 0 : (rp >= p.table_rows ? int(p.table_rows - 1) : rp);
    const uint16_t* cs = p.cos + int64_t(rp) * d;
    const uint16_t* sn = p.sin + int64_t(rp) * d;
    const uint16_t* row = p.qkv + i * p.qkv_stride;
    const int q_units = p.num_qo_heads * upr;
    for (int u = threadIdx.x; u < q_units; u += blockDim.x) {
      const int h = u / upr;
      const int c = (u - h * upr) * 8;
      const uint16_t* src = row + int64_t(h) * d;
      uint4 o1, o2;
      mi::rope8(mi::load16_nt(src + c), mi::load16_nt(src + half + c), mi::load16(cs + c), mi::load16(sn + c),
            mi::load16(cs + half + c), mi::load16(sn + half + c), o1, o2);
      uint16_t* dst = p.q_out + i * p.qo_stride_tok + int64_t(h) * p.qo_stride_head;
      mi::store16(dst + c, o1);
      mi::store16(dst + half + c, o2);
    }
    // the K heads and V chunks go to the slot (null: not placed); the slot
    // lookup after the q heads measured faster than before them (85 -> 80 us
    // on 18,240 rows of 32 / 8 heads)
    uint16_t* slot = token_slot(p.batch_indices, p.positions, p.indptr, p.indices, i, p.batch_size, p.num_pages,
                                p.page_size, p.pool, page_stride, tok_stride);
    if (!slot) continue;
    for (int u = q_units + threadIdx.x; u < per_token; u += blockDim.x) {
      if (u < rot_units) {
        const int h = u / upr;
        const int c = (u - h * upr) * 8;
        const uint16_t* src = row + int64_t(h) * d;
        uint4 o1, o2;
        mi::rope8(mi::load16_nt(src + c), mi::load16_nt(src + half + c), mi::load16(cs + c), mi::load16(sn + c),
              mi::load16(cs + half + c), mi::load16(sn + half + c), o1, o2);
        uint16_t* dst = slot + int64_t(h - p.num_qo_heads) * d;
        mi::store16(dst + c, o1);
        mi::store16(dst + half + c, o2);
      } else {
        const int v = u - rot_units;
        const int kh = v / (d >> 3);
        const int c = (v - kh * (d >> 3)) * 8;
        mi::store16(slot + kv_stride + int64_t(kh) * d + c,
                    mi::load16_nt(row + int64_t(p.num_qo_heads + p.num_kv_heads + kh) * d + c));
      }
    }
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

extern "C" int mi_paged_kv_append(const void* append_key, int64_t key_stride_token,
                                  int64_t key_stride_head, const void* append_value,
                                  int64_t value_stride_token, int64_t value_stride_head,
                                  const int32_t* batch_indices, const int32_t* positions,
                                  int64_t num_tokens, void* paged_kv_cache, int64_t num_pages,
                                  const int32_t* kv_indices, const int32_t* kv_indptr,
                                  const int32_t* kv_last_page_len, int32_t batch_size,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                  mi_stream_t stream) {
  (void)kv_last_page_len;  // slot placement depends on positions only
  mi::clear_error();
  if (num_tokens < 0 || batch_size < 0 || num_kv_heads <= 0 || num_pages <= 0)
    return mi::fail(MI_ERR_INVALID, "append: bad sizes (tokens=%lld batch=%d kv_heads=%d pages=%lld)",
                    (long long)num_tokens, batch_size, num_kv_heads, (long long)num_pages);
  if (head_dim <= 0 || head_dim % 8 != 0)
    return mi::fail(MI_ERR_UNSUPPORTED, "append: head_dim %d must be a positive multiple of 8", head_dim);
  if (page_size <= 0) return mi::fail(MI_ERR_INVALID, "append: page_size %d", page_size);
  if (num_tokens == 0) return MI_OK;
  if (!append_key || !append_value || !batch_indices || !positions || !paged_kv_cache ||
      !kv_indices || !kv_indptr)
    return mi::fail(MI_ERR_INVALID, "append: null pointer argument");
  if (!aligned16(append_key) || !aligned16(append_value) || !aligned16(paged_kv_cache) ||
      key_stride_token % 8 || key_stride_head % 8 || value_stride_token % 8 || value_stride_head % 8)
    return mi::fail(MI_ERR_INVALID, "append: key/value rows and pool must be 16-byte aligned");

  AppendParams p{static_cast<const uint16_t*>(append_key),
                 static_cast<const uint16_t*>(append_value),
                 key_stride_token,
                 key_stride_head,
                 value_stride_token,
                 value_stride_head,
                 batch_indices,
                 positions,
                 num_tokens,
                 static_cast<uint16_t*>(paged_kv_cache),
                 num_pages,
                 kv_indices,
                 kv_indptr,
                 batch_size,
                 num_kv_heads,
                 head_dim,
                 page_size};
  // one workgroup per token, up to 256 threads over its chunks
  const int64_t per_token = int64_t(num_kv_heads) * (head_dim / 8);
  const int threads = int(std::min<int64_t>(MI_APPEND_THREADS, (per_token + 63) / 64 * 64));
  const int64_t blocks = std::min<int64_t>(num_tokens, int64_t(1) << 20);
  hipLaunchKernelGGL(append_kernel, dim3(unsigned(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), p);
  return mi::check_launch("append_kernel");
}

extern "C" int mi_rope_append(const void* qkv, int64_t qkv_stride_token, const int32_t* rope_positions,
                              const void* cos_table, const void* sin_table, int64_t table_rows, void* q_out,
                              int64_t q_out_stride_token, int64_t q_out_stride_head,
                              const int32_t* batch_indices, const int32_t* positions, int64_t num_tokens,
                              void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indices,
                              const int32_t* kv_indptr, const int32_t* kv_last_page_len, int32_t batch_size,
                              int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                              mi_stream_t stream) {
  (void)kv_last_page_len;  // slot placement depends on positions only
  mi::clear_error();
  if (num_tokens < 0 || batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || num_pages <= 0 ||
      table_rows <= 0)
    return mi::fail(MI_ERR_INVALID, "rope_append: bad sizes (tokens=%lld batch=%d heads=%d/%d pages=%lld rows=%lld)",
                    (long long)num_tokens, batch_size, num_qo_heads, num_kv_heads, (long long)num_pages,
                    (long long)table_rows);
  if (head_dim <= 0 || head_dim % 16 != 0)
    return mi::fail(MI_ERR_UNSUPPORTED, "rope_append: head_dim %d must be a positive multiple of 16", head_dim);
  if (page_size <= 0) return mi::fail(MI_ERR_INVALID, "rope_append: page_size %d", page_size);
  if (num_tokens == 0) return MI_OK;
  if (!qkv || !rope_positions || !cos_table || !sin_table || !q_out || !batch_indices || !positions ||
      !paged_kv_cache || !kv_indices || !kv_indptr)
    return mi::fail(MI_ERR_INVALID, "rope_append: null pointer argument");
  if (!aligned16(qkv) || !aligned16(cos_table) || !aligned16(sin_table) || !aligned16(q_out) ||
      !aligned16(paged_kv_cache) || qkv_stride_token % 8 || q_out_stride_token % 8 || q_out_stride_head % 8)
    return mi::fail(MI_ERR_INVALID, "rope_append: qkv / q_out rows, tables and pool must be 16-byte aligned");
  if (qkv_stride_token < int64_t(num_qo_heads + 2 * num_kv_heads) * head_dim)
    return mi::fail(MI_ERR_INVALID, "rope_append: qkv row stride %lld shorter than (Hq + 2 Hkv) * D",
                    (long long)qkv_stride_token);
  RopeAppendParams p{static_cast<const uint16_t*>(qkv),
                     qkv_stride_token,
                     rope_positions,
                     static_cast<const uint16_t*>(cos_table),
                     static_cast<const uint16_t*>(sin_table),
                     table_rows,
                     static_cast<uint16_t*>(q_out),
                     q_out_stride_token,
                     q_out_stride_head,
                     batch_indices,
                     positions,
                     num_tokens,
                     static_cast<uint16_t*>(paged_kv_cache),
                     num_pages,
                     kv_indices,
                     kv_indptr,
                     batch_size,
                     num_qo_heads,
                     num_kv_heads,
                     head_dim,
                     page_size};
  const int64_t per_token = int64_t(num_qo_heads + num_kv_heads) * (head_dim / 16) + int64_t(num_kv_heads) * (head_dim / 8);
  // one workgroup per token, up to 256 threads over its units
  const int threads = int(std::min<int64_t>(MI_APPEND_THREADS, (per_token + 63) / 64 * 64));
  const int64_t blocks = std::min<int64_t>(num_tokens, int64_t(1) << 20);
  hipLaunchKernelGGL(rope_append_kernel, dim3(unsigned(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), p);
  return mi::check_launch("rope_append_kernel");
}
