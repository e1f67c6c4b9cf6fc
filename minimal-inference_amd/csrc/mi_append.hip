// Paged KV append: scatter new K/V rows into their page slots.
//
// Reference call: model.py:207-216 (flashinfer.page.append_paged_kv_cache),
// NHD pool layout scheduler.py:195-202.  Slot placement is integer-exact:
// page = kv_indices[kv_indptr[b] + pos / page_size], slot = pos % page_size.
//
// Each thread moves one 16-byte chunk (8 bf16) of K and the same chunk of V,
// so a wave writes 1 KiB of contiguous head rows per instruction and the
// kernel streams at HBM rate for prefill-sized appends.
#include "mi_common.h"

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

__global__ __launch_bounds__(256) void append_kernel(AppendParams p) {
  const int chunks = p.head_dim >> 3;
  const int64_t per_token = int64_t(p.num_kv_heads) * chunks;
  const int64_t total = p.num_tokens * per_token;
  const int64_t tok_stride = int64_t(p.num_kv_heads) * p.head_dim;
  const int64_t kv_stride = int64_t(p.page_size) * tok_stride;
  const int64_t page_stride = 2 * kv_stride;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i = idx / per_token;
    const int r = int(idx - i * per_token);
    const int h = r / chunks;
    const int c = r - h * chunks;
    const int b = p.batch_indices[i];
    const int pos = p.positions[i];
    if (b < 0 || b >= p.batch_size || pos < 0) continue;
    const int64_t it = int64_t(p.indptr[b]) + pos / p.page_size;
    if (it >= p.indptr[b + 1]) continue;
    const int64_t page = p.indices[it];
    if (page < 0 || page >= p.num_pages) continue;
    const int slot = pos % p.page_size;
    uint16_t* dst = p.pool + page * page_stride + slot * tok_stride + int64_t(h) * p.head_dim + c * 8;
    const uint4 kv = mi::load16(p.key + i * p.ks_tok + h * p.ks_head + c * 8);
    const uint4 vv = mi::load16(p.value + i * p.vs_tok + h * p.vs_head + c * 8);
    mi::store16(dst, kv);
    mi::store16(dst + kv_stride, vv);
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
  const int64_t work = num_tokens * num_kv_heads * (head_dim / 8);
  const int threads = 256;
  int64_t blocks = (work + threads - 1) / threads;
  const int64_t cap = int64_t(mi::num_cus()) * 16;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(append_kernel, dim3(unsigned(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), p);
  return mi::check_launch("append_kernel");
}
