// Host-row gather: copies missed KV rows from pinned host memory (read by the
// compute units through the host alias, over PCIe) into hot-buffer rows of
// the device pool. A row is two planes (K and V) of plane_bytes each; in both
// the host and the pool layout a block is [2, page_size, kv_heads, head_dim],
// so plane `pl` of row r starts at (r/P)*block + (pl*P + r%P) * plane_bytes,
// with block = 2*P*plane_bytes on the host and the pool's block stride
// (which may exceed it) on the device.
//
// A workgroup takes groups of kRowsPerBlock consecutive plan entries, group
// blockIdx.x, blockIdx.x + gridDim.x, ... A thread owns vector column c of
// every plane and issues the loads of all its rows before the stores, so
// each lane keeps kRowsPerBlock 16-byte PCIe reads in flight. Plan entries
// past a request's misses are -1; a group whose entries are all -1 costs
// one read of them. The grid is capped (nhs_set_gather_workgroups): a few
// dozen workgroups already saturate the host link, and waves that wait on
// PCIe reads would otherwise hold compute units that concurrent kernels need.
// 16-byte rows are stored non-temporally: the gathered bytes go to HBM while
// the kernel waits on PCIe anyway, instead of as dirty cache lines that the
// next kernel's memory traffic would have to write back (the gather itself
// also runs ~2% faster that way).
#include <atomic>

#include "nhs_common.h"

namespace nhs {

constexpr int kGatherThreads = 256;
constexpr int kRowsPerBlock = 16;  // 16 reads in flight per lane reach the copy engine's PCIe rate
std::atomic<int> g_gather_workgroups{0};  // 0: one workgroup per group of entries

typedef unsigned int gather_u32x4 __attribute__((ext_vector_type(4)));

template <typename V>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_kernel(const char* __restrict__ host,
                                                                     char* __restrict__ pool,
                                                                     const int64_t* __restrict__ miss_host,
                                                                     const int64_t* __restrict__ miss_dev,
                                                                     int64_t n_entries, int page_size,
                                                                     int64_t plane_bytes, int64_t pool_block_bytes) {
  __shared__ int64_t src_base[kRowsPerBlock];
  __shared__ int64_t dst_base[kRowsPerBlock];
  __shared__ int live;
  const int64_t block_bytes = 2 * (int64_t)page_size * plane_bytes;
  const int64_t groups = (n_entries + kRowsPerBlock - 1) / kRowsPerBlock;
  for (int64_t group = blockIdx.x; group < groups; group += gridDim.x) {
  const int64_t first = group * kRowsPerBlock;
  __syncthreads();  // the previous group's bases have been read
  if (threadIdx.x == 0) live = 0;
  __syncthreads();
  if (threadIdx.x < kRowsPerBlock) {
    int64_t i = first + threadIdx.x;
    int64_t s = -1, d = -1;
    if (i < n_entries) {
      s = miss_host[i];
      d = miss_dev[i];
    }
    if (s >= 0 && d >= 0) {
      src_base[threadIdx.x] = (s / page_size) * block_bytes + (s % page_size) * plane_bytes;
      dst_base[threadIdx.x] = (d / page_size) * pool_block_bytes + (d % page_size) * plane_bytes;
      atomicAdd(&live, 1);
    } else {
      src_base[threadIdx.x] = -1;
      dst_base[threadIdx.x] = -1;
    }
  }
  __syncthreads();
  if (live == 0) continue;  // uniform: `live` is shared

  int64_t sb[kRowsPerBlock], db[kRowsPerBlock];
#pragma unroll
  for (int r = 0; r < kRowsPerBlock; ++r) {
    sb[r] = src_base[r];
    db[r] = dst_base[r];
  }
  const int vecs_per_plane = (int)(plane_bytes / (int64_t)sizeof(V));
  const int64_t plane_stride = (int64_t)page_size * plane_bytes;
  for (int c = threadIdx.x; c < 2 * vecs_per_plane; c += kGatherThreads) {
    const int plane = c >= vecs_per_plane;
    const int64_t off = plane * plane_stride + (int64_t)(c - plane * vecs_per_plane) * (int64_t)sizeof(V);
    V buf[kRowsPerBlock];
#pragma unroll
    for (int r = 0; r < kRowsPerBlock; ++r)
      if (sb[r] >= 0) buf[r] = *reinterpret_cast<const V*>(host + sb[r] + off);
#pragma unroll
    for (int r = 0; r < kRowsPerBlock; ++r)
      if (db[r] >= 0) {
        if constexpr (sizeof(V) == 16)
          __builtin_nontemporal_store(__builtin_bit_cast(gather_u32x4, buf[r]),
                                      reinterpret_cast<gather_u32x4*>(pool + db[r] + off));
        else
          *reinterpret_cast<V*>(pool + db[r] + off) = buf[r];
      }
  }
  }
}

}  // namespace nhs

extern "C" int nhs_gather_rows(const void* host_alias, void* pool, const int64_t* miss_host_rows,
                               const int64_t* miss_device_rows, int64_t n_entries, int32_t page_size,
                               int64_t plane_bytes, int64_t pool_block_stride, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  if (!host_alias || !pool || !miss_host_rows || !miss_device_rows)
    return fail(NHS_ERR_INVALID, "nhs_gather_rows: null pointer");
  if (n_entries < 0 || page_size < 1 || plane_bytes < 4 || plane_bytes % 4)
    return fail(NHS_ERR_INVALID, "nhs_gather_rows: need n_entries >= 0, page_size >= 1, plane_bytes a multiple of 4");
  const int64_t block_bytes = 2 * (int64_t)page_size * plane_bytes;
  if (pool_block_stride == 0) pool_block_stride = block_bytes;
  if (pool_block_stride < block_bytes)
    return fail(NHS_ERR_INVALID, "nhs_gather_rows: pool_block_stride below 2 * page_size * plane_bytes");
  if (n_entries == 0) return NHS_OK;
  if (plane_bytes / 4 > 0x3fffffff) return fail(NHS_ERR_UNSUPPORTED, "nhs_gather_rows: rows too wide");
  const uintptr_t align = (uintptr_t)host_alias | (uintptr_t)pool | (uintptr_t)pool_block_stride;
  int64_t blocks = (n_entries + kRowsPerBlock - 1) / kRowsPerBlock;
  const int cap = g_gather_workgroups.load(std::memory_order_relaxed);
  if (cap > 0 && blocks > cap) blocks = cap;
  if (blocks > 0x7fffffff) blocks = 0x7fffffff;
  hipStream_t s = (hipStream_t)stream;
  if (plane_bytes % 16 == 0 && align % 16 == 0) {
    launch(gather_rows_kernel<uint4>, dim3((unsigned)blocks), dim3(kGatherThreads), 0, s, ev.start, ev.stop,
           (const char*)host_alias, (char*)pool, miss_host_rows, miss_device_rows, n_entries, page_size, plane_bytes,
           pool_block_stride);
  } else if (plane_bytes % 8 == 0 && align % 8 == 0) {
    launch(gather_rows_kernel<uint2>, dim3((unsigned)blocks), dim3(kGatherThreads), 0, s, ev.start, ev.stop,
           (const char*)host_alias, (char*)pool, miss_host_rows, miss_device_rows, n_entries, page_size, plane_bytes,
           pool_block_stride);
  } else {
    if (align % 4) return fail(NHS_ERR_INVALID, "nhs_gather_rows: host and pool must be 4-byte aligned");
    launch(gather_rows_kernel<uint32_t>, dim3((unsigned)blocks), dim3(kGatherThreads), 0, s, ev.start, ev.stop,
           (const char*)host_alias, (char*)pool, miss_host_rows, miss_device_rows, n_entries, page_size, plane_bytes,
           pool_block_stride);
  }
  return launch_status("nhs_gather_rows");
}

extern "C" int nhs_set_gather_workgroups(int32_t workgroups) {
  if (workgroups < 0) return nhs::fail(NHS_ERR_INVALID, "nhs_set_gather_workgroups: negative");
  nhs::g_gather_workgroups.store(workgroups, std::memory_order_relaxed);
  return NHS_OK;
}
