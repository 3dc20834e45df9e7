// Decode-time append into one pool page, fused: the new K/V rows are
// written to the page's pool block and (through the pinned host alias) to
// its host block, the page's running per-element key minimum / maximum fold
// in the new keys, and its fp32 mean key is recomputed over every valid row.
// One thread owns one element of a row (kv_heads * head_dim elements), so
// every access of a wave is contiguous.
//
// The mean is summed in double in row order and rounded to fp32 once (the
// oracle sums in the same order). Min/max propagate NaN like torch.minimum
// / torch.maximum.
#include "nhs_common.h"

namespace nhs {

constexpr int kAppendThreads = 256;
constexpr int kAppendBatch = 64;  // earlier rows loaded together for the page mean (one round for P <= 64)

struct AppendArgs {
  const void* k;
  const void* v;
  int64_t token_stride;  // elements between consecutive tokens of k and v
  int dtype;
  int row_elems;
  int64_t plane_elems;   // page_size * row_elems
  char* pool_block;      // the page's pool block [2, P, row_elems]
  char* host_block;      // its host block, or null
  int within, count;
  float* summary;
  void* minimum;
  void* maximum;
};

__device__ __forceinline__ float nan_min(float a, float b) { return (a != a || b != b) ? a + b : (b < a ? b : a); }
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || b != b) ? a + b : (b > a ? b : a); }

// Element e of every appended row of one page (T: the KV storage type, so
// every load below is a plain load of a known width).
template <typename T>
__device__ __forceinline__ void append_element(const AppendArgs& a, int e) {
  constexpr int esize = T::bytes;
  float lo = load_elem(a.minimum, T::dtype, e);
  float hi = load_elem(a.maximum, T::dtype, e);
  double sum = 0.0;
  // the earlier keys of the page, loaded kAppendBatch at a time before they
  // are summed (in row order)
  // Loads are unconditional (rows past `within` re-read the last earlier
  // row, which is in bounds) so that no branch separates them; only the
  // sum is masked.
  for (int r0 = 0; r0 < a.within; r0 += kAppendBatch) {
    float keys[kAppendBatch];
#pragma unroll
    for (int j = 0; j < kAppendBatch; ++j) {
      const int r = min(r0 + j, a.within - 1);
      keys[j] = load_elem(a.pool_block, T::dtype, (int64_t)r * a.row_elems + e);
    }
#pragma unroll
    for (int j = 0; j < kAppendBatch; ++j)
      if (r0 + j < a.within) sum += (double)keys[j];
  }
  for (int t = 0; t < a.count; ++t) {
    const int64_t src = (int64_t)t * a.token_stride + e;
    const int64_t row = (int64_t)(a.within + t) * a.row_elems + e;
    // copy the raw element bits: no conversion touches the stored values
    if (esize == 4) {
      const uint32_t kb = static_cast<const uint32_t*>(a.k)[src], vb = static_cast<const uint32_t*>(a.v)[src];
      reinterpret_cast<uint32_t*>(a.pool_block)[row] = kb;
      reinterpret_cast<uint32_t*>(a.pool_block)[a.plane_elems + row] = vb;
      if (a.host_block) {
        reinterpret_cast<uint32_t*>(a.host_block)[row] = kb;
        reinterpret_cast<uint32_t*>(a.host_block)[a.plane_elems + row] = vb;
      }
    } else {
      const uint16_t kb = static_cast<const uint16_t*>(a.k)[src], vb = static_cast<const uint16_t*>(a.v)[src];
      reinterpret_cast<uint16_t*>(a.pool_block)[row] = kb;
      reinterpret_cast<uint16_t*>(a.pool_block)[a.plane_elems + row] = vb;
      if (a.host_block) {
        reinterpret_cast<uint16_t*>(a.host_block)[row] = kb;
        reinterpret_cast<uint16_t*>(a.host_block)[a.plane_elems + row] = vb;
      }
    }
    const float key = load_elem(a.k, T::dtype, src);
    lo = nan_min(lo, key);
    hi = nan_max(hi, key);
    sum += (double)key;
  }
  store_elem(a.minimum, T::dtype, e, lo);
  store_elem(a.maximum, T::dtype, e, hi);
  a.summary[e] = (float)(sum / (double)(a.within + a.count));
}

template <typename T>
__global__ __launch_bounds__(kAppendThreads) void append_page_kernel(AppendArgs a) {
  const int e = blockIdx.x * kAppendThreads + threadIdx.x;
  if (e < a.row_elems) append_element<T>(a, e);
}

struct AppendItemsArgs {
  const char* k;
  const char* v;
  int64_t token_stride;  // elements between the items' rows
  int dtype, row_elems, page_size;
  char* pool;
  int64_t pool_block_bytes;  // the pool's block stride (host blocks are contiguous)
  char* host;
  const nhs_layer_item* items;
  const int64_t* lengths;
};

// Item blockIdx.y appends its one token; its page and row follow from its
// length and its page tables.
template <typename T>
__global__ __launch_bounds__(kAppendThreads) void append_items_kernel(AppendItemsArgs g) {
  const int e = blockIdx.x * kAppendThreads + threadIdx.x;
  if (e >= g.row_elems) return;
  const int b = blockIdx.y;
  const nhs_layer_item& item = g.items[b];
  const int64_t length = g.lengths[b];
  const int64_t page = length / g.page_size;
  constexpr int esize = T::bytes;
  const int64_t plane = (int64_t)g.page_size * g.row_elems;
  const int64_t block_bytes = 2 * plane * esize;
  const int64_t page_offset = page * g.row_elems;
  AppendArgs a;
  a.k = g.k + (int64_t)b * g.token_stride * esize;
  a.v = g.v + (int64_t)b * g.token_stride * esize;
  a.token_stride = g.token_stride;
  a.dtype = g.dtype;
  a.row_elems = g.row_elems;
  a.plane_elems = plane;
  a.pool_block = g.pool + (int64_t)item.resident[page] * g.pool_block_bytes;
  a.host_block = g.host ? g.host + (int64_t)item.source[page] * block_bytes : nullptr;
  a.within = (int)(length - page * g.page_size);
  a.count = 1;
  a.summary = item.summaries + page_offset;
  a.minimum = static_cast<char*>(item.minimum) + page_offset * esize;
  a.maximum = static_cast<char*>(item.maximum) + page_offset * esize;
  append_element<T>(a, e);
}

}  // namespace nhs

extern "C" int nhs_append_page(const void* k, const void* v, int64_t token_stride, int32_t kv_dtype,
                               int32_t row_elems, int32_t page_size, void* pool, int64_t pool_block_stride,
                               int64_t block, int32_t within,
                               int32_t count, void* host_alias, int64_t host_page, float* summary, void* minimum,
                               void* maximum, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  if (!k || !v || !pool || !summary || !minimum || !maximum) return fail(NHS_ERR_INVALID, "nhs_append_page: null pointer");
  if (!valid_dtype(kv_dtype)) return fail(NHS_ERR_INVALID, "nhs_append_page: bad dtype");
  if (row_elems < 1 || page_size < 1 || block < 0 || within < 0 || count < 1 || within + count > page_size ||
      token_stride < row_elems || (host_alias && host_page < 0))
    return fail(NHS_ERR_INVALID, "nhs_append_page: invalid page, rows or strides");
  AppendArgs a;
  a.k = k;
  a.v = v;
  a.token_stride = token_stride;
  a.dtype = kv_dtype;
  a.row_elems = row_elems;
  a.plane_elems = (int64_t)page_size * row_elems;
  const int64_t block_bytes = 2 * a.plane_elems * elem_size(kv_dtype);
  if (pool_block_stride == 0) pool_block_stride = block_bytes;
  if (pool_block_stride < block_bytes || pool_block_stride % elem_size(kv_dtype))
    return fail(NHS_ERR_INVALID, "nhs_append_page: pool_block_stride below a block or not a whole element");
  a.pool_block = static_cast<char*>(pool) + block * pool_block_stride;
  a.host_block = host_alias ? static_cast<char*>(host_alias) + host_page * block_bytes : nullptr;
  a.within = within;
  a.count = count;
  a.summary = summary;
  a.minimum = minimum;
  a.maximum = maximum;
  const dim3 grid((unsigned)((row_elems + kAppendThreads - 1) / kAppendThreads)), threads(kAppendThreads);
  if (kv_dtype == NHS_BF16)
    launch(append_page_kernel<BF16>, grid, threads, 0, (hipStream_t)stream, ev.start, ev.stop, a);
  else if (kv_dtype == NHS_F16)
    launch(append_page_kernel<F16>, grid, threads, 0, (hipStream_t)stream, ev.start, ev.stop, a);
  else
    launch(append_page_kernel<F32>, grid, threads, 0, (hipStream_t)stream, ev.start, ev.stop, a);
  return launch_status("nhs_append_page");
}

extern "C" int nhs_append_items(int32_t batch, const void* k, const void* v, int64_t token_stride, int32_t kv_dtype,
                                int32_t row_elems, int32_t page_size, void* pool, int64_t pool_block_stride,
                                void* host_alias,
                                const nhs_layer_item* items, const int64_t* lengths, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  if (!k || !v || !pool || !items || !lengths) return fail(NHS_ERR_INVALID, "nhs_append_items: null pointer");
  if (!valid_dtype(kv_dtype)) return fail(NHS_ERR_INVALID, "nhs_append_items: bad dtype");
  if (batch < 0 || batch > 65535 || row_elems < 1 || page_size < 1 || token_stride < row_elems)
    return fail(NHS_ERR_INVALID, "nhs_append_items: invalid batch, rows or strides");
  if (batch == 0) return NHS_OK;
  AppendItemsArgs g;
  g.k = static_cast<const char*>(k);
  g.v = static_cast<const char*>(v);
  g.token_stride = token_stride;
  g.dtype = kv_dtype;
  g.row_elems = row_elems;
  g.page_size = page_size;
  g.pool = static_cast<char*>(pool);
  const int64_t block_bytes = 2 * (int64_t)page_size * row_elems * elem_size(kv_dtype);
  if (pool_block_stride == 0) pool_block_stride = block_bytes;
  if (pool_block_stride < block_bytes || pool_block_stride % elem_size(kv_dtype))
    return fail(NHS_ERR_INVALID, "nhs_append_items: pool_block_stride below a block or not a whole element");
  g.pool_block_bytes = pool_block_stride;
  g.host = static_cast<char*>(host_alias);
  g.items = items;
  g.lengths = lengths;
  const dim3 grid((unsigned)((row_elems + kAppendThreads - 1) / kAppendThreads), (unsigned)batch), block(kAppendThreads);
  if (kv_dtype == NHS_BF16)
    launch(append_items_kernel<BF16>, grid, block, 0, (hipStream_t)stream, ev.start, ev.stop, g);
  else if (kv_dtype == NHS_F16)
    launch(append_items_kernel<F16>, grid, block, 0, (hipStream_t)stream, ev.start, ev.stop, g);
  else
    launch(append_items_kernel<F32>, grid, block, 0, (hipStream_t)stream, ev.start, ev.stop, g);
  return launch_status("nhs_append_items");
}
