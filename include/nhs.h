/*
 * nhs.h - C ABI of the MI355X (gfx950) sparse-decode library, libnhs_hip.so.
 *
 * Every entry point takes plain device pointers, element counts and strides
 * (in elements, not bytes, unless the name says bytes), enqueues its kernels
 * on the given hipStream_t (passed as void*; NULL means the null stream) and
 * returns an int status without synchronising. No entry point allocates
 * device or host memory: the caller owns every buffer, including workspaces,
 * whose size is returned by the matching *_workspace_bytes function. All
 * kernels are capturable in a HIP graph (no host readback, no memset nodes).
 *
 * Status: NHS_OK (0) on success, a negative NHS_ERR_* for an argument the
 * library rejects before launching anything, or a positive hipError_t from
 * the launch. nhs_last_error() returns a message for the last failure on the
 * calling thread.
 *
 * Memory layouts (shared with the Python side):
 *   pool  [blocks, 2, page_size, kv_heads, head_dim]   K plane 0, V plane 1
 *   host  [host_pages, 2, page_size, kv_heads, head_dim] (pinned, same layout)
 *   A physical row r lives in block r / page_size at offset r % page_size;
 *   its K bytes and its V bytes are each kv_heads*head_dim contiguous elements.
 *   Host blocks are contiguous. Pool blocks are pool_block_stride bytes apart
 *   (0: contiguous, 2*page_size*kv_heads*head_dim elements); a larger stride
 *   leaves a gap after each block. The cache pads each block by three head
 *   slots (3*head_dim elements), so that consecutive blocks shift a KV head's
 *   bytes by three head slots in the address: HBM then serves every KV head
 *   at the same rate (with contiguous blocks some heads' slots are slower).
 */
#ifndef NHS_H
#define NHS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  NHS_OK = 0,
  NHS_ERR_INVALID = -1,     /* argument out of range or inconsistent */
  NHS_ERR_UNSUPPORTED = -2, /* no kernel for this shape / dtype */
  NHS_ERR_WORKSPACE = -3    /* caller workspace smaller than required */
};

/* Element types for pools, host KV, queries, bounds and outputs. */
enum { NHS_F32 = 0, NHS_F16 = 1, NHS_BF16 = 2 };

/* Library limits (checked; exceeding one returns NHS_ERR_UNSUPPORTED). */
#define NHS_MAX_POSITIONS 32768  /* resolver: selected positions per item (hybrid.py:36 caps U at 32768) */
#define NHS_MAX_HOT_ROWS 32768   /* resolver: hot rows per item (hybrid.py:36) */
#define NHS_MAX_SELECT_PAGES 16384 /* selectors: pages per request held in registers (more: a looping kernel) */

/*
 * Device tables of one (request, layer), for the batched decode entry points
 * (nhs_*_items): an array of these lives in device memory, one entry per
 * batch item, and stays valid while the request is admitted (the tables are
 * allocated at admission and only their contents change). Layouts are those
 * of the strided entry points; alignment (16 bytes for the bounds and
 * summaries) is the caller's duty and is not checked, since the library
 * cannot read device memory before launching.
 */
typedef struct nhs_layer_item {
  const int32_t* source;   /* page -> host page, -1 unset      [n_pages] */
  const int32_t* resident; /* page -> pool block, -1 none      [n_pages] */
  const int32_t* hot;      /* hot block table    [ceil(hot_rows/page_size)] */
  int32_t* tags;           /* hot row tags (host rows, -1 empty) [hot_rows] */
  int64_t* lru;            /* hot slot LRU order                 [hot_rows] */
  void* minimum;           /* Quest key bounds, KV dtype [n_pages, kv_heads, head_dim] */
  void* maximum;
  float* summaries;        /* fp32 mean keys             [n_pages, kv_heads, head_dim] */
  int64_t n_pages;
} nhs_layer_item;

/* 2: the pool block stride arguments of the gather, attention and appends */
int nhs_abi_version(void);
const char* nhs_last_error(void);

/*
 * Per-kernel timing hook: the next nhs_* entry point called on this thread
 * stamps `start_event` with the begin of its first kernel and `stop_event`
 * with the end of its last kernel (either may be NULL), taken from the
 * dispatches themselves through hipExtLaunchKernel, then forgets both.
 * The events must be created timing hipEvent_t of the launch's device.
 * No counterpart in the reference, which times its Triton launches with
 * torch.cuda.Event pairs; marker packets around a kernel add several us of
 * queue latency that a dispatch's own timestamps do not have.
 */
int nhs_set_launch_events(void* start_event, void* stop_event);

/*
 * Device alias of pinned host memory allocated by hipHostMalloc (torch's
 * pin_memory=True). The library never registers or unregisters memory.
 * Replaces MappedHost, nano_hisparse/row_kernels.py:10-32 (a libcuda
 * cuPointerGetAttribute call through ctypes).
 */
int nhs_host_device_ptr(const void* pinned_host, void** device_alias);

/*
 * Host-row gather: for each plan entry i in [0, n_entries) with
 * miss_host_rows[i] >= 0 and miss_device_rows[i] >= 0, copy the K plane row
 * and the V plane row (plane_bytes = kv_heads*head_dim*element_size each)
 * from host row miss_host_rows[i] to pool row miss_device_rows[i]. Plans of
 * several requests may be concatenated. Rows are copied with coalesced
 * 16-byte loads from the host alias over PCIe. plane_bytes must be a
 * multiple of 4.
 * Replaces _gather / gather_rows, nano_hisparse/row_kernels.py:35-70
 * (CPU twin nano_hisparse/hybrid.py:452-459).
 */
int nhs_gather_rows(const void* host_alias, void* pool,
                    const int64_t* miss_host_rows, const int64_t* miss_device_rows,
                    int64_t n_entries, int32_t page_size, int64_t plane_bytes,
                    int64_t pool_block_stride, void* stream);

/*
 * Caps the workgroups of every later nhs_gather_rows launch (process-wide;
 * 0, the default, launches one workgroup per 16 plan entries). Each
 * workgroup then loops over groups of entries. A few dozen workgroups reach
 * the host link's rate; a cap leaves the other compute units to kernels that
 * run beside the gather. No counterpart in the reference.
 */
int nhs_set_gather_workgroups(int32_t workgroups);

/*
 * Physical-row GQA decode attention, split-K over rows with an online
 * softmax. For request b and query head h (kv head
 * h / (q_heads / kv_heads)):
 *   out[b,h] = softmax_r(q[b,h] . K[row] * head_dim^-0.5) . V[row]
 * over the rows rows[b, h, c] >= 0 (c < n_rows); rows < 0 are masked and a
 * head with no valid row yields zeros. rows_head_stride == 0 means every
 * query head of a request shares one row list (the default shared
 * selection); otherwise each head has its own list. Accumulation is fp32;
 * out has the query's dtype. head_dim*kv element size must be a multiple of
 * 16 bytes and at most 2048 bytes; pool rows must be below 2^31. The splits
 * are merged in the same launch by the last workgroup of each head group,
 * found with arrival counters at the front of the workspace: its first
 * 260 KiB (the counters and a zero block read in place of masked rows) must
 * be zero before the first call on a workspace, every call leaves them zero,
 * and calls that share a workspace must not overlap.
 * batch * q_heads <= 65536.
 * Replaces _attend / attend_rows, nano_hisparse/row_kernels.py:73-135 (torch
 * twin nano_hisparse/attention.py:26-35).
 */
int64_t nhs_attend_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim,
                                   int32_t n_rows);
int nhs_attend_rows(const void* query, int32_t q_dtype, int64_t q_batch_stride,
                    int64_t q_head_stride, const void* pool, int32_t kv_dtype,
                    int64_t pool_block_stride, const int64_t* rows, int64_t rows_batch_stride,
                    int64_t rows_head_stride, int64_t rows_col_stride, int32_t batch, int32_t n_rows, int32_t q_heads,
                    int32_t kv_heads, int32_t head_dim, int32_t page_size, void* out,
                    int64_t out_batch_stride, int64_t out_head_stride, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * nhs_attend_rows without a workspace argument, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Its
 * workspace is a file-scope device array of NHS_ATTEND_NOALLOC_BYTES that
 * each GPU holds until the process ends; a shape whose
 * nhs_attend_workspace_bytes exceeds it returns NHS_ERR_WORKSPACE. The
 * call allocates nothing; a device's first call sets the array up on the
 * caller's stream. Every call on one GPU shares the array, so calls that
 * overlap on one GPU race. Results equal nhs_attend_rows's bit for bit.
 */
#define NHS_ATTEND_NOALLOC_BYTES (32ll << 20)
int nhs_attend_rows_noalloc(const void* query, int32_t q_dtype, int64_t q_batch_stride,
                            int64_t q_head_stride, const void* pool, int32_t kv_dtype,
                            int64_t pool_block_stride, const int64_t* rows, int64_t rows_batch_stride,
                            int64_t rows_head_stride, int64_t rows_col_stride, int32_t batch,
                            int32_t n_rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                            int32_t page_size, void* out, int64_t out_batch_stride,
                            int64_t out_head_stride, void* stream);

/*
 * Row resolver for `batch` independent (request, layer) items, one
 * workgroup each, with no host round trip. Item b reads positions[b, :n]
 * (int32 or int64 per positions_i64), its page tables source/resident
 * [n_pages] and hot block table hot[ceil(hot_rows/page_size)], and updates
 * its row tags[hot_rows] (int32, -1 empty) and LRU permutation
 * lru[hot_rows] (int64) in place. It writes physical[b, :n] (input order,
 * -1 for padding, duplicates and rows without host backing),
 * miss_host[b, :n] / miss_device[b, :n] (compact prefix in ascending
 * logical order, then -1) and counts[b, 0:3] = unique resident hits, hot
 * hits, misses; counts_total[0:3] (may be NULL) is incremented by them.
 * lengths[b] (int64, may be NULL to use `length` for every item) is the
 * causal length. n <= hot_rows (the reference's max_union_rows <=
 * hot_rows), n <= NHS_MAX_POSITIONS, hot_rows <= NHS_MAX_HOT_ROWS;
 * with batch > 1, plan_stride >= n. Above 4096 positions the item's
 * physical / miss_host / miss_device rows also serve as scratch during the
 * call (sorted keys, per-entry state) before they receive the results.
 * Bit-exact with resolve_rows, nano_hisparse/row_index.py:62-140.
 */
int nhs_resolve_rows(int32_t batch, int32_t n, const void* positions, int32_t positions_i64,
                     int64_t positions_stride, const int32_t* source, const int32_t* resident,
                     int64_t page_table_stride, int32_t n_pages, const int32_t* hot,
                     int64_t hot_stride, int32_t* tags, int64_t tags_stride, int64_t* lru,
                     int64_t lru_stride, int32_t hot_rows, const int64_t* lengths,
                     int64_t length, int32_t page_size, int64_t* physical, int64_t* miss_host,
                     int64_t* miss_device, int64_t plan_stride, int64_t* counts,
                     int64_t* counts_total, void* stream);

/*
 * Quest page selection for `batch` requests. Request b scores each of its
 * count = ceil(lengths[b]/page_size) pages (count is clamped to max_pages):
 *   score[p] = (sum_h sum_d max(q[h,d]*min[p,h/g,d], q[h,d]*max[p,h/g,d])) / q_heads
 * in fp32 with a fixed summation order: per KV head j and dimension d, with
 * a / b the smaller / larger of the two bounds (swapped when max < min),
 * the GQA group's terms are a*Qneg + b*Qpos (Qpos / Qneg: the sums, in head
 * order from 0.0, of the group's positive / non-positive q[h,d]); a bound
 * row is cut into chunks of 32 bytes when it is a multiple of 32 bytes of at
 * most 64 chunks, else of 16 bytes when a multiple of 16 bytes of at most
 * 64 chunks, else of one element up to 64 elements, else of
 * ceil(head_dim/64) elements (the last chunk shorter); each chunk is summed
 * from 0.0 in element order with t = fma(nneg ? a : 0, Qneg, t),
 * t = fma(npos ? b : 0, Qpos, t) (npos, nneg: whether any head contributed
 * to Qpos, Qneg); chunk sums (padded with +0.0 to a power of two) are added
 * as a pairwise tree; KV-head sums are added sequentially j = 0..kv_heads-1.
 * As torch.maximum does, a chunk sums to NaN when it holds a NaN bound, or
 * a bound of +-inf (+-0) at a d where a head's query is +-0 (+-inf); NaN
 * scores are stored as 0x7fc00000. Any group size and head_dim;
 * kv_heads * head_dim <= 16384 when a page needs the general kernel.
 * Page count-1, and page 0 when keep_sink and top_pages > 1 and
 * count > 1, are forced (+inf in the reference). Ranking, as torch.topk's:
 * NaN pages first, then forced pages, then scores descending; ties at the
 * k-th rank go to the lowest pages. The top_pages chosen pages are written
 * ascending to pages[b, :top_pages]
 * (-1 padded when count < top_pages) and expanded to causal token positions
 * positions[b, :top_pages*page_size] (ascending, -1 padded). scores[b, :]
 * (max_pages floats) keeps the scores, also when top_pages >= max_pages
 * (every page is then kept). With pages and positions both NULL only the
 * scores are computed, for nhs_select_resolve_rows / _items.
 * minimum/maximum are [max_pages, kv_heads, head_dim] per request.
 * Replaces quest_selection, nano_hisparse/selection.py:69-91.
 */
int nhs_quest_select(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                     int64_t q_head_stride, const void* minimum, const void* maximum,
                     int32_t bounds_dtype, int64_t bounds_batch_stride, int32_t q_heads,
                     int32_t kv_heads, int32_t head_dim, const int64_t* lengths, int64_t length,
                     int32_t page_size, int32_t max_pages, int32_t top_pages, int32_t keep_sink,
                     float* scores, int32_t* pages, int32_t* positions, void* stream);

/*
 * Page-mean selection ("mean" selector) for `batch` requests: the query is
 * averaged over each GQA group, dotted with the fp32 per-page mean keys
 * summaries[p, kv_heads, head_dim], pages {0, count-1} ({count-1} when
 * top_pages == 1) are always kept and the best top_pages - |kept| other
 * pages (score descending, page ascending; NaN ranks first, below the kept
 * pages) are added. Output layout, and the scores-only form (pages and
 * positions NULL), as in nhs_quest_select. Replaces select_pages,
 * nano_hisparse/selection.py:119-145.
 */
int nhs_mean_select(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                    int64_t q_head_stride, const float* summaries, int64_t summaries_batch_stride,
                    int32_t q_heads, int32_t kv_heads, int32_t head_dim, const int64_t* lengths,
                    int64_t length, int32_t page_size, int32_t max_pages, int32_t top_pages,
                    float* scores, int32_t* pages, int32_t* positions, void* stream);

/*
 * Decode-time append into one page (replaces HostStore.append's block
 * write, _update_bounds and _mirror, nano_hisparse/storage.py:258-331):
 * rows [within, within + count) of pool block `block` (layout
 * [2, page_size, row_elems], row_elems = kv_heads * head_dim) receive
 * k[t * token_stride ...] and v[t * token_stride ...] for t < count. The
 * page's minimum/maximum [row_elems] (KV dtype) fold in the new keys
 * exactly (NaN propagates), and summary [row_elems] (fp32) becomes the mean
 * of keys [0, within + count), summed in double in row order and rounded
 * once. With a non-null host_alias (from nhs_host_device_ptr) the new rows
 * are also written to host block `host_page`, so the host mirror is
 * complete when the kernel is.
 */
int nhs_append_page(const void* k, const void* v, int64_t token_stride, int32_t kv_dtype, int32_t row_elems,
                    int32_t page_size, void* pool, int64_t pool_block_stride, int64_t block,
                    int32_t within, int32_t count,
                    void* host_alias, int64_t host_page, float* summary, void* minimum, void* maximum,
                    void* stream);

/*
 * Batched decode-time append: item b appends one token, k/v rows at
 * k + b * token_stride (row_elems elements each), at position lengths[b]
 * (its layer length before the append) of items[b]: page
 * p = lengths[b] / page_size, row lengths[b] % page_size of pool block
 * items[b].resident[p] and, with a host_alias, of host page
 * items[b].source[p]. Bounds and the page mean are updated as in
 * nhs_append_page (same arithmetic, bit-identical results). The caller binds
 * the page (resident[p], source[p]) before the call and increments its
 * lengths after it. No counterpart in the reference, which appends request
 * by request (storage.py:258-331); this is the batched engine step's form.
 */
int nhs_append_items(int32_t batch, const void* k, const void* v, int64_t token_stride, int32_t kv_dtype,
                     int32_t row_elems, int32_t page_size, void* pool, int64_t pool_block_stride,
                     void* host_alias,
                     const nhs_layer_item* items, const int64_t* lengths, void* stream);

/*
 * nhs_quest_select over per-item bounds: item b reads items[b].minimum /
 * .maximum ([n_pages, kv_heads, head_dim], n_pages >= its page count) and
 * lengths[b]. Results are bit-identical to nhs_quest_select on the same
 * bounds. Batched form of quest_selection, nano_hisparse/selection.py:69-91.
 */
int nhs_quest_select_items(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                           int64_t q_head_stride, const nhs_layer_item* items, int32_t bounds_dtype,
                           int32_t q_heads, int32_t kv_heads, int32_t head_dim, const int64_t* lengths,
                           int32_t page_size, int32_t max_pages, int32_t top_pages, int32_t keep_sink,
                           float* scores, int32_t* pages, int32_t* positions, void* stream);

/*
 * nhs_resolve_rows over per-item tables: item b reads items[b].source /
 * .resident (n_pages entries), .hot and updates .tags / .lru in place.
 * Outputs and limits as nhs_resolve_rows; lengths is required. Batched form
 * of resolve_rows, nano_hisparse/row_index.py:62-140.
 */
int nhs_resolve_items(int32_t batch, int32_t n, const void* positions, int32_t positions_i64,
                      int64_t positions_stride, const nhs_layer_item* items, int32_t hot_rows,
                      const int64_t* lengths, int32_t page_size, int64_t* physical, int64_t* miss_host,
                      int64_t* miss_device, int64_t plan_stride, int64_t* counts, int64_t* counts_total,
                      void* stream);

/*
 * Page selection and row resolution in one launch, one workgroup per item:
 * the selection step of nhs_quest_select (mode 0, keep_sink as there) or
 * nhs_mean_select (mode 1) on scores[b, :max_pages] as their scores-only
 * form leaves them, writing pages[b, :top_pages] and
 * positions[b, :n] (n = top_pages * page_size) exactly as the selector
 * does, then nhs_resolve_rows on those n positions (int32, in order). Every
 * output is bit-identical to the selector launch followed by the resolver
 * launch. Requires max(max_pages, top_pages) <= 1024, or max_pages <= 4096
 * with top_pages <= 256, and n <= 4096, else returns NHS_ERR_UNSUPPORTED
 * (the two launches handle any size). Tables,
 * outputs and plan_stride as nhs_resolve_rows; the selection stays in LDS,
 * so no launch boundary and no global round trip separate the two steps.
 * Replaces the sequence quest_selection / select_pages then resolve_rows
 * (nano_hisparse/selection.py:69-91, 119-145; row_index.py:62-140).
 */
int nhs_select_resolve_rows(int32_t batch, const float* scores, int32_t max_pages, int32_t mode,
                            int32_t top_pages, int32_t keep_sink, const int32_t* source,
                            const int32_t* resident, int64_t page_table_stride, int32_t n_pages,
                            const int32_t* hot, int64_t hot_stride, int32_t* tags, int64_t tags_stride,
                            int64_t* lru, int64_t lru_stride, int32_t hot_rows, const int64_t* lengths,
                            int64_t length, int32_t page_size, int32_t* pages, int32_t* positions,
                            int64_t* physical, int64_t* miss_host, int64_t* miss_device,
                            int64_t plan_stride, int64_t* counts, int64_t* counts_total, void* stream);

/*
 * nhs_select_resolve_rows over per-item tables, as nhs_resolve_items reads
 * them (lengths required).
 */
int nhs_select_resolve_items(int32_t batch, const float* scores, int32_t max_pages, int32_t mode,
                             int32_t top_pages, int32_t keep_sink, const nhs_layer_item* items,
                             int32_t hot_rows, const int64_t* lengths, int32_t page_size, int32_t* pages,
                             int32_t* positions, int64_t* physical, int64_t* miss_host,
                             int64_t* miss_device, int64_t plan_stride, int64_t* counts,
                             int64_t* counts_total, void* stream);

/*
 * Elementwise stages of the batched decode layer (model.py:43-71, 140-158 of
 * the reference run them as separate torch operations). Each computes in
 * fp32 and rounds to the dtype wherever the torch expression rounds, so only
 * the reduction order of the RMSNorm mean differs from torch.
 *
 * nhs_add_rmsnorm: per row of `width` elements, h = x + delta (rounded;
 * delta may be NULL) is written back to x when write_back, and
 * out = round(round(h * rsqrt(mean(h^2) + eps)) * weight)
 * (RMSNorm.forward, model.py:49-51, after the residual add of _finish,
 * model.py:156-158).
 */
int nhs_add_rmsnorm(int32_t rows, int32_t width, int32_t dtype, void* x, const void* delta, int32_t write_back,
                    const void* weight, float eps, void* out, void* stream);

/*
 * nhs_rope: rotary embedding in place on `rows` rows of t (row_stride
 * elements apart), each holding `heads` heads of head_dim; cos/sin are
 * [rows, head_dim/2] in the dtype. For d < head_dim/2 with lo = t[d],
 * hi = t[d + head_dim/2]: t[d] = round(round(lo*c) + round(-hi*s)),
 * t[d + head_dim/2] = round(round(hi*c) + round(lo*s))
 * (the rope closure, model.py:147-151).
 */
int nhs_rope(int32_t rows, int32_t heads, int32_t head_dim, int32_t dtype, void* t, int64_t row_stride,
             const void* cos, const void* sin, void* stream);

/*
 * nhs_silu_mul: out[r, i] = round(round(silu(g)) * u) with g = gate_up[r, i],
 * u = gate_up[r, inter + i] (MLP.forward, model.py:70-71, on a fused
 * gate/up projection).
 */
int nhs_silu_mul(int32_t rows, int32_t inter, int32_t dtype, const void* gate_up, void* out, void* stream);

/*
 * Linear layer for up to 16 token rows (decode): y[m, n] = sum_k x[m, k] *
 * w[n, k] (+ bias[n]), bf16 or fp16 (dtype), fp32 accumulation, one
 * rounding. w is [n, k] row-major (torch Linear weight layout); n a multiple
 * of 16, k of 2048; strides in elements (x and w rows 16-byte aligned); bias
 * may be NULL. Replaces the decode projections of the reference's layers
 * (model.py:43-71, nn.Linear q/k/v/o and gate/up/down, and the lm_head at
 * model.py:221), which at decode batch sizes stream the weights.
 */
int nhs_linear_small_m(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, const void* bias,
                       int32_t dtype, int32_t m, int32_t n, int32_t k, void* y, int64_t y_row_stride, void* stream);

/*
 * nhs_linear_small_m followed by nhs_silu_mul in one launch, bit-identical
 * to the two: w is the fused [gate; up] weight [2 * inter, k] (no bias) and
 * y[m, inter] = round(round(silu(g)) * u) for g, u the rounded gate and up
 * outputs (MLP.forward, model.py:70-71). inter a multiple of 8.
 */
int nhs_linear_silu_mul(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int32_t dtype,
                        int32_t m, int32_t inter, int32_t k, void* y, int64_t y_row_stride, void* stream);

/*
 * nhs_linear_small_m followed by nhs_rope on the first rope_heads heads of
 * each output row, in one launch, bit-identical to the two: y[m, n] holds
 * n / head_dim heads of head_dim (a fused q/k/v projection: the q and k
 * heads rotate, the v heads do not); cos/sin are [m, head_dim / 2]
 * (Model._project's q/k/v projections and rope closure, model.py:134-153).
 * head_dim a multiple of 16, n of head_dim.
 */
int nhs_linear_rope(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, const void* bias,
                    int32_t dtype, int32_t m, int32_t n, int32_t k, int32_t head_dim, int32_t rope_heads,
                    const void* cos, const void* sin, void* y, int64_t y_row_stride, void* stream);

/*
 * Causal GQA self-attention over one prompt (prefill), flash-attention style
 * on MFMA: out[s, h] = softmax_{t <= s}(q[s, h] . k[t, h / g] * D^-1/2) .
 * v[t, h / g] for s < seq, g = q_heads / kv_heads, fp32 accumulation. bf16 or
 * fp16, head_dim 64 or 128, strides in elements (multiples of 8, dims
 * contiguous), 16-byte aligned tensors. Replaces the dense causal
 * F.scaled_dot_product_attention of Model.prefill (model.py:170-180 of the
 * reference), whose flash and memory-efficient backends this PyTorch build
 * does not provide on gfx950 (its math fallback materialises seq x seq
 * scores per head).
 */
int nhs_prefill_attention(const void* q, int64_t q_seq_stride, int64_t q_head_stride, const void* k,
                          int64_t k_seq_stride, int64_t k_head_stride, const void* v, int64_t v_seq_stride,
                          int64_t v_head_stride, int32_t dtype, int32_t seq, int32_t q_heads, int32_t kv_heads,
                          int32_t head_dim, void* out, int64_t out_seq_stride, int64_t out_head_stride,
                          void* stream);

/*
 * Legacy per-head selections: out[h, c] = columns[h, c] in [0, n) ?
 * shared_rows[columns[h, c]] : -1 for h < heads, c < width.
 * Replaces the head_columns branch of resolve_rows,
 * nano_hisparse/row_index.py:130-134.
 */
int nhs_expand_columns(const int64_t* shared_rows, int64_t n, const int64_t* columns,
                       int64_t heads, int64_t width, int64_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NHS_H */
