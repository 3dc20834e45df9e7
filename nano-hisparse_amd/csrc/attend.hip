// Physical-row GQA decode attention over selected pool rows, one launch.
//
// A workgroup of 4 waves owns one request, up to G query heads that share a
// row list (the GQA group of one KV head, or one head for per-head lists)
// and one contiguous split of the row list. A row's K (and V) for a KV head
// is head_dim contiguous elements = `row_chunks` 16-byte chunks; lane `sub`
// of a row's `lpr` lanes holds chunks sub, sub + lanes_used, ... (C of them),
// so each load instruction of a row's lanes covers contiguous bytes. The
// chunks stay packed in registers: with a 16-bit query of the KV dtype the
// scores use v_dot2 on packed pairs, otherwise fp32 FMAs. Each loaded K/V
// chunk serves all G query heads, so the pool is read once per KV head.
// Scores are reduced across a row's lanes with DPP; an online softmax in
// base 2 (scale * log2 e applied after the dot) accumulates (m, l, acc) per
// row slot; slots are merged by shuffles, waves through LDS, and the
// workgroup writes (m, l, acc) of its split to the workspace.
//
// The last workgroup of a head group to finish (an arrival counter in the
// workspace, reset to zero by that workgroup) merges the splits, divides by
// the softmax denominator (0 when no row was valid) and stores the output in
// the query's dtype. The workspace's counter region (its first 256 KiB) must
// be zero before the first call; every call leaves it at zero.
#include <math.h>

#include <stdlib.h>

#include <mutex>
#include <vector>

#include "nhs_common.h"

namespace nhs {

constexpr int kAttendThreads = 256;
constexpr int kAttendWaves = kAttendThreads / kWave;
constexpr int kMaxSplits = 64;
constexpr int kMinRowsPerSplit = 32;
constexpr int kStage = 1024;  // row indices staged in LDS per pass
// Arrival counters occupy a fixed region at the front of the workspace, so a
// call never finds another call's partials where it expects a counter.
constexpr int kCounterSlots = 65536;
constexpr int64_t kCounterBytes = kCounterSlots * (int64_t)sizeof(int);

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct AttendArgs {
  const void* q;
  int q_dtype;
  int64_t q_bs, q_hs;
  const void* pool;
  const int64_t* rows;
  int64_t r_bs, r_hs, r_cs;
  int n_rows, rows_per_split, n_splits;
  int q_heads, kv_heads, group, head_dim, page_size;
  int lpr_log2, lanes_used, chunks_per_kv;
  FastDiv page_div;
  float qscale;
  float* ws;          // partials [B, q_heads, n_splits, 2 + head_dim]
  int* counters;      // [B, gridDim.y]
  void* out;
  int out_dtype;
  int64_t out_bs, out_hs;
};

template <typename T>
__device__ __forceinline__ float packed_dot(uint32_t k, uint32_t q, float acc) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k), __builtin_bit_cast(bf16x2_t, q), acc,
                                           false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, k), __builtin_bit_cast(f16x2_t, q), acc, false);
}

// element e (0..E-1) of a 16-byte chunk, as fp32
template <typename T>
__device__ __forceinline__ float chunk_elem(const uint4& v, int e) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (T::dtype == NHS_F32) {
    return __uint_as_float(w[e]);
  } else {
    uint32_t word = w[e >> 1];
    if constexpr (T::dtype == NHS_BF16)
      return (e & 1) ? __uint_as_float(word & 0xffff0000u) : __uint_as_float(word << 16);
    else
      return f16_bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
  }
}

// Agent-coherent accesses (sc1): visible across the XCDs' separate L2s.
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int G, int C, bool PK>
__global__ __launch_bounds__(kAttendThreads) void attend_kernel(AttendArgs a) {
  constexpr int E = 16 / T::bytes;
  constexpr int U = C == 1 ? 4 : 2;  // rows per lane slot per iteration
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lpr = 1 << a.lpr_log2;
  const int slots = kWave >> a.lpr_log2;
  const int slot = lane >> a.lpr_log2;
  const int sub = lane & (lpr - 1);
  const bool data_lane = sub < a.lanes_used;

  const int split = blockIdx.x;
  const int kv = blockIdx.y / a.chunks_per_kv;
  const int chunk = blockIdx.y - kv * a.chunks_per_kv;
  const int b = blockIdx.z;
  const int h0 = kv * a.group + chunk * G;
  const int nh = min(G, a.group - chunk * G);
  const int64_t* rows = a.rows + (int64_t)b * a.r_bs + (int64_t)h0 * a.r_hs;

  // query chunks of this lane (same dim mapping as the K/V chunks)
  uint32_t qp[PK ? G : 1][C][4];
  float qf[PK ? 1 : G][C][E];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int d0 = (c * a.lanes_used + sub) * E;
      const bool live = g < nh && data_lane;
      const int64_t qo = (int64_t)b * a.q_bs + (int64_t)(h0 + (live ? g : 0)) * a.q_hs + d0;
      if constexpr (PK) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          qp[g][c][w] = live ? *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.q) + qo + 2 * w) : 0u;
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) qf[g][c][e] = live ? load_elem(a.q, a.q_dtype, qo + e) : 0.f;
      }
    }

  float m[G], l[G], acc[G][C][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][c][e] = 0.f;
  }

  const int row_begin = split * a.rows_per_split;
  const int row_end = min(a.n_rows, row_begin + a.rows_per_split);
  const int64_t row_bytes = (int64_t)a.kv_heads * a.head_dim * T::bytes;  // one plane row, all KV heads
  const int64_t plane_bytes = (int64_t)a.page_size * row_bytes;
  const char* pool = static_cast<const char*>(a.pool) + (int64_t)kv * a.head_dim * T::bytes;
  const int per_iter = kAttendWaves * slots * U;

  // The split's rows are staged in LDS as K-plane row indices of the pool
  // (block * 2P + offset; 0xffffffff for masked rows), kStage at a time, so
  // the loop below issues its K/V loads back to back without waiting on
  // index loads. Pool rows are < 2^31, checked on the host.
  __shared__ uint32_t krow[kStage];
  for (int s0 = row_begin; s0 < row_end; s0 += kStage) {
    const int s1 = min(row_end, s0 + kStage);
    __syncthreads();
    for (int i = s0 + (int)threadIdx.x; i < s1; i += kAttendThreads) {
      const int64_t r = rows[(int64_t)i * a.r_cs];
      uint32_t kr_idx = 0xffffffffu;
      if (r >= 0) {
        const uint32_t blk = a.page_div.div((uint32_t)r);
        kr_idx = blk * (uint32_t)a.page_size + (uint32_t)r;  // blk*2P + (r - blk*P)
      }
      krow[i - s0] = kr_idx;
    }
    __syncthreads();
    for (int base = s0; base < s1; base += per_iter) {
      uint4 kr[U][C], vr[U][C];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c_idx = base + (u * kAttendWaves + wave) * slots + slot;
        const uint32_t ki = c_idx < s1 ? krow[c_idx - s0] : 0xffffffffu;
        ok[u] = ki != 0xffffffffu;
        if (ok[u] && data_lane) {
          const char* kp = pool + (int64_t)ki * row_bytes;
#pragma unroll
          for (int c = 0; c < C; ++c) {
            const int64_t cb = (int64_t)(c * a.lanes_used + sub) * 16;
            kr[u][c] = *reinterpret_cast<const uint4*>(kp + cb);
            vr[u][c] = *reinterpret_cast<const uint4*>(kp + plane_bytes + cb);
          }
        } else {
#pragma unroll
          for (int c = 0; c < C; ++c) kr[u][c] = vr[u][c] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
      float p[G][U], alpha[G];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float dot = 0.f;
#pragma unroll
          for (int c = 0; c < C; ++c) {
            if constexpr (PK) {
              dot = packed_dot<T>(kr[u][c].x, qp[g][c][0], dot);
              dot = packed_dot<T>(kr[u][c].y, qp[g][c][1], dot);
              dot = packed_dot<T>(kr[u][c].z, qp[g][c][2], dot);
              dot = packed_dot<T>(kr[u][c].w, qp[g][c][3], dot);
            } else {
#pragma unroll
              for (int e = 0; e < E; ++e) dot += qf[g][c][e] * chunk_elem<T>(kr[u][c], e);
            }
          }
          p[g][u] = dot;
        }
      // sum each score over the lanes of its row, one DPP stage at a time
      if (lpr >= 2) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += dpp_f32<0xB1>(p[g][u]);
      }
      if (lpr >= 4) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += dpp_f32<0x4E>(p[g][u]);
      }
      if (lpr >= 8) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += dpp_f32<0x141>(p[g][u]);
      }
      if (lpr >= 16) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += dpp_f32<0x140>(p[g][u]);
      }
      if (lpr >= 32) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += __shfl_xor(p[g][u], 16);
      }
      if (lpr >= 64) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) p[g][u] += __shfl_xor(p[g][u], 32);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = m[g];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          p[g][u] = ok[u] ? p[g][u] * a.qscale : -INFINITY;
          mx = fmaxf(mx, p[g][u]);
        }
        const float ref = mx == -INFINITY ? 0.f : mx;  // keeps exp2 arguments finite
        alpha[g] = exp2f(m[g] - ref);
        float psum = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          p[g][u] = exp2f(p[g][u] - ref);
          psum += p[g][u];
        }
        l[g] = l[g] * alpha[g] + psum;
        m[g] = mx;
      }
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          float v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) v[u] = chunk_elem<T>(vr[u][c], e);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float x = acc[g][c][e] * alpha[g];
#pragma unroll
            for (int u = 0; u < U; ++u) x += p[g][u] * v[u];
            acc[g][c][e] = x;
          }
        }
    }
  }

  // merge the row slots of this wave (lanes that differ in the slot bits)
  for (int st = lpr; st < kWave; st <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m_o = __shfl_xor(m[g], st);
      const float l_o = __shfl_xor(l[g], st);
      const float mx = fmaxf(m[g], m_o);
      const float ref = mx == -INFINITY ? 0.f : mx;
      const float fa = exp2f(m[g] - ref), fb = exp2f(m_o - ref);
      l[g] = l[g] * fa + l_o * fb;
      m[g] = mx;
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float o = __shfl_xor(acc[g][c][e], st);
          acc[g][c][e] = acc[g][c][e] * fa + o * fb;
        }
    }
  }

  // merge the waves through LDS: [wave][g][2 + head_dim]
  extern __shared__ float lds[];
  __shared__ int last_arrival;
  const int stride = 2 + a.head_dim;
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float* w = lds + (wave * G + g) * stride;
      if (sub == 0) {
        w[0] = m[g];
        w[1] = l[g];
      }
      if (data_lane)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) w[2 + (c * a.lanes_used + sub) * E + e] = acc[g][c][e];
    }
  }
  __syncthreads();
  float* part = a.ws + (((int64_t)b * a.q_heads + h0) * a.n_splits + split) * stride;
  for (int idx = threadIdx.x; idx < nh * stride; idx += kAttendThreads) {
    const int g = idx / stride;
    const int j = idx - g * stride;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttendWaves; ++w) M = fmaxf(M, lds[(w * G + g) * stride]);
    float o;
    if (j == 0) {
      o = M;
    } else {
      o = 0.f;
      if (M != -INFINITY)
#pragma unroll
        for (int w = 0; w < kAttendWaves; ++w) {
          const float* src = lds + (w * G + g) * stride;
          o += src[j] * exp2f(src[0] - M);
        }
    }
    st_coherent(part + (int64_t)g * a.n_splits * stride + j, o);
  }

  // the last workgroup of this head group merges the splits
  __shared__ float split_m[8 * kMaxSplits];
  __shared__ float split_w[8 * kMaxSplits];
  // The partials were written with agent-coherent stores; waiting for them to
  // complete before the arrival orders them without an L2 writeback (an
  // agent-scope fence would write back and invalidate this XCD's whole L2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* counter = a.counters + (int64_t)b * gridDim.y + blockIdx.y;
  if (threadIdx.x == 0)
    last_arrival = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.n_splits - 1;
  __syncthreads();
  if (!last_arrival) return;
  const float* base_part = a.ws + ((int64_t)b * a.q_heads + h0) * a.n_splits * stride;
  const int ns = a.n_splits;
  for (int idx = threadIdx.x; idx < nh * ns; idx += kAttendThreads) {
    const int g = idx / ns, s = idx - g * ns;
    const float* hp = base_part + ((int64_t)g * ns + s) * stride;
    split_m[idx] = ld_coherent(hp);
    split_w[idx] = ld_coherent(hp + 1);
  }
  __syncthreads();
  if (threadIdx.x < nh) {
    const int g = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, split_m[g * ns + s]);
    float L = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < ns; ++s) L += split_w[g * ns + s] * exp2f(split_m[g * ns + s] - M);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (int s = 0; s < ns; ++s)  // weight of split s in the output
      split_w[g * ns + s] = inv > 0.f ? exp2f(split_m[g * ns + s] - M) * inv : 0.f;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < nh * a.head_dim; idx += kAttendThreads) {
    const int g = idx / a.head_dim;
    const int d = idx - g * a.head_dim;
    const float* hp = base_part + (int64_t)g * ns * stride + 2 + d;
    const float* wg = split_w + g * ns;
    float v = 0.f;
#pragma unroll 8
    for (int s = 0; s < ns; ++s) v += ld_coherent(hp + (int64_t)s * stride) * wg[s];
    store_elem(a.out, a.out_dtype, (int64_t)b * a.out_bs + (int64_t)(h0 + g) * a.out_hs + d, v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*AttendKernel)(AttendArgs);

template <typename T, int G, int C, bool PK>
static AttendKernel pick3() {
  return attend_kernel<T, G, C, PK>;
}

template <typename T, bool PK>
static AttendKernel pick2(int G, int C) {
  switch (G * 4 + C) {
    case 1 * 4 + 1: return pick3<T, 1, 1, PK>();
    case 1 * 4 + 2: return pick3<T, 1, 2, PK>();
    case 2 * 4 + 1: return pick3<T, 2, 1, PK>();
    case 2 * 4 + 2: return pick3<T, 2, 2, PK>();
    case 4 * 4 + 1: return pick3<T, 4, 1, PK>();
    case 4 * 4 + 2: return pick3<T, 4, 2, PK>();
    case 8 * 4 + 1: return pick3<T, 8, 1, PK>();
    case 8 * 4 + 2: return pick3<T, 8, 2, PK>();
  }
  return nullptr;
}

static AttendKernel pick_kernel(int kv_dtype, bool packed, int G, int C) {
  switch (kv_dtype) {
    case NHS_F32: return pick2<F32, false>(G, C);
    case NHS_F16: return packed ? pick2<F16, true>(G, C) : pick2<F16, false>(G, C);
    default: return packed ? pick2<BF16, true>(G, C) : pick2<BF16, false>(G, C);
  }
}

static int max_splits_for(int n_rows) {
  int s = n_rows / kMinRowsPerSplit;
  return s < 1 ? 1 : s > kMaxSplits ? kMaxSplits : s;
}

// Workgroups of `kernel` resident on the whole current device at once,
// cached per (device, kernel, LDS size).
static int device_capacity(AttendKernel kernel, size_t lds) {
  struct Entry {
    int dev;
    AttendKernel kernel;
    size_t lds;
    int capacity;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.dev == dev && e.kernel == kernel && e.lds == lds) return e.capacity;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), kAttendThreads,
                                                   lds) != hipSuccess)
    return 0;
  std::lock_guard<std::mutex> lock(mu);
  cache.push_back({dev, kernel, lds, per_cu * cus});
  return per_cu * cus;
}

}  // namespace nhs

extern "C" int64_t nhs_attend_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t n_rows) {
  if (batch < 1 || q_heads < 1 || head_dim < 1 || n_rows < 1) return 0;
  int64_t partials = (int64_t)batch * q_heads * nhs::max_splits_for(n_rows) * (head_dim + 2) * (int64_t)sizeof(float);
  return nhs::kCounterBytes + partials;
}

extern "C" int nhs_attend_rows(const void* query, int32_t q_dtype, int64_t q_batch_stride, int64_t q_head_stride,
                               const void* pool, int32_t kv_dtype, const int64_t* rows, int64_t rows_batch_stride,
                               int64_t rows_head_stride, int64_t rows_col_stride, int32_t batch, int32_t n_rows,
                               int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size, void* out,
                               int64_t out_batch_stride, int64_t out_head_stride, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  using namespace nhs;
  if (!query || !pool || !rows || !out || !workspace) return fail(NHS_ERR_INVALID, "nhs_attend_rows: null pointer");
  if (!valid_dtype(q_dtype) || !valid_dtype(kv_dtype)) return fail(NHS_ERR_INVALID, "nhs_attend_rows: bad dtype");
  if (batch < 1 || n_rows < 1 || q_heads < 1 || kv_heads < 1 || head_dim < 1 || page_size < 1 ||
      q_heads % kv_heads)
    return fail(NHS_ERR_INVALID, "nhs_attend_rows: invalid shape");
  if (batch > 65535 || (int64_t)batch * q_heads > kCounterSlots)
    return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: batch * q_heads must be <= %d", kCounterSlots);
  const int64_t need = nhs_attend_workspace_bytes(batch, q_heads, head_dim, n_rows);
  if (workspace_bytes < need)
    return fail(NHS_ERR_WORKSPACE, "nhs_attend_rows: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
  const int esize = elem_size(kv_dtype);
  const int row_chunks = head_dim * esize / 16;
  if ((head_dim * esize) % 16 || row_chunks > 128)
    return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: head_dim*element size must be a multiple of 16 bytes, <= 2048");
  if ((uintptr_t)pool % 16) return fail(NHS_ERR_INVALID, "nhs_attend_rows: pool must be 16-byte aligned");
  const bool packed = q_dtype == kv_dtype && kv_dtype != NHS_F32 && q_head_stride % 2 == 0 &&
                      q_batch_stride % 2 == 0 && (uintptr_t)query % 4 == 0;

  AttendArgs a;
  a.q = query;
  a.q_dtype = q_dtype;
  a.q_bs = q_batch_stride;
  a.q_hs = q_head_stride;
  a.pool = pool;
  a.rows = rows;
  a.r_bs = rows_batch_stride;
  a.r_hs = rows_head_stride;
  a.r_cs = rows_col_stride;
  a.n_rows = n_rows;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.page_size = page_size;
  a.page_div = FastDiv((uint32_t)page_size);
  int C = row_chunks > 64 ? 2 : 1;
  if (const char* env = getenv("NHS_ATTEND_C")) C = atoi(env) == 2 && row_chunks % 2 == 0 ? 2 : 1;  // TEMP tuning
  if (row_chunks / C > 64) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: rows too wide");
  a.lanes_used = row_chunks / C;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.qscale = (float)(1.4426950408889634 / sqrt((double)head_dim));
  a.group = q_heads / kv_heads;
  int G;
  if (rows_head_stride != 0) {
    G = 1;  // one head per workgroup; its own row list
    a.chunks_per_kv = a.group;
  } else {
    const int group = a.group;
    G = group >= 8 ? 8 : group >= 4 ? (group == 4 ? 4 : 8) : group == 3 ? 4 : group;
    a.chunks_per_kv = (group + G - 1) / G;
  }
  AttendKernel kernel = pick_kernel(kv_dtype, packed, G, C);
  if (!kernel) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: no kernel for G=%d C=%d", G, C);
  const size_t lds = (size_t)kAttendWaves * G * (2 + head_dim) * sizeof(float);
  const int groups = kv_heads * a.chunks_per_kv;
  const int items = batch * groups;
  const int capacity = device_capacity(kernel, lds);
  int splits = capacity > 0 ? capacity / items : 1;
  if (splits < 1) splits = 1;
  if (splits > max_splits_for(n_rows)) splits = max_splits_for(n_rows);
  a.n_splits = splits;
  a.rows_per_split = (n_rows + splits - 1) / splits;
  a.counters = static_cast<int*>(workspace);
  a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  a.out = out;
  a.out_dtype = q_dtype;
  a.out_bs = out_batch_stride;
  a.out_hs = out_head_stride;
  dim3 grid((unsigned)splits, (unsigned)groups, (unsigned)batch);
  hipLaunchKernelGGL(kernel, grid, dim3(kAttendThreads), lds, (hipStream_t)stream, a);
  return launch_status("nhs_attend_rows");
}
