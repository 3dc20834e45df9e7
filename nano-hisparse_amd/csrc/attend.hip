// Physical-row GQA decode attention over selected pool rows, one launch.
//
// A workgroup of 8 waves owns one request, up to G query heads that share a
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
// row slot; slots are merged by shuffles and waves through LDS.
//
// The grid is one balanced round of about one workgroup per CU. A (request,
// KV head) that gets two CUs is split by query heads (two workgroups of G
// heads read the same rows on one XCD, the second read mostly from L2) and
// its workgroups store the normalised output directly; beyond that the row
// list is split, each split writes (m, l, acc) to the workspace, and the
// last workgroup of a head group to finish (an arrival counter in the
// workspace, reset to zero by that workgroup) merges the splits, divides by
// the softmax denominator (0 when no row was valid) and stores the output in
// the query's dtype. The workspace's first 260 KiB (arrival counters and a
// zero block) must be zero before the first call; every call leaves them so.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "nhs_common.h"

namespace nhs {

constexpr int kAttendThreads = 512;
constexpr int kAttendWaves = kAttendThreads / kWave;
constexpr int kMaxSplits = 32;
constexpr int kMinRowsPerSplit = 32;
constexpr int kStage = 4096;  // row indices staged in LDS per pass (16 KiB)
constexpr int kStagePerThread = kStage / kAttendThreads;
constexpr int kIssueGroups = 2;  // row groups whose loads a wave issues together
constexpr int kMaxHeadChunks = 2;  // query-head chunks that re-read one KV head's rows
// Arrival counters occupy a fixed region at the front of the workspace, so a
// call never finds another call's partials where it expects a counter.
constexpr int kCounterSlots = 65536;
constexpr int64_t kCounterBytes = kCounterSlots * (int64_t)sizeof(int);
// A zero block follows the counters; the kernel never writes it and reads it
// in place of masked rows (it must cover the widest row, 2 KiB).
constexpr int64_t kZeroBytes = 4096;
constexpr int64_t kHeaderBytes = kCounterBytes + kZeroBytes;

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
  int kv_items;  // batch * kv_heads
  FastDiv page_div;
  FastDiv plane2_div;  // by 2 * page_size: a K-plane row index -> its block
  int64_t block_pad;   // pool block stride minus 2 * page_size rows
  float qscale;
  const char* zeros;  // kZeroBytes of zeros
  float* ws;          // partials [B, q_heads, n_splits, 2 + head_dim]
  int* counters;      // [B, kv_heads * chunks_per_kv]
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

__device__ __forceinline__ uint32_t word_of(const uint4& v, int w) {
  return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// two fp32 weights packed as a pair of the KV dtype (bf16: round to nearest
// even; f16: round toward zero), and back
template <typename T>
__device__ __forceinline__ uint32_t pack_pair(float a, float b) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
template <typename T>
__device__ __forceinline__ float pair_lo(uint32_t v) {
  return T::dtype == NHS_BF16 ? __uint_as_float(v << 16) : f16_bits_to_f32(v & 0xffffu);
}
template <typename T>
__device__ __forceinline__ float pair_hi(uint32_t v) {
  return T::dtype == NHS_BF16 ? __uint_as_float(v & 0xffff0000u) : f16_bits_to_f32(v >> 16);
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

  // 1-D grid, id = kv_item + kv_items * (chunk * n_splits + split): the
  // workgroups of one (request, KV head) are kv_items apart, so they land on
  // the same XCD (workgroups go to the 8 XCDs round robin) whenever kv_items
  // is a multiple of 8, and the head chunks that read the same rows share
  // that XCD's L2.
  const int kv_item = (int)(blockIdx.x % (unsigned)a.kv_items);
  const int rest = (int)(blockIdx.x / (unsigned)a.kv_items);
  const int split = rest % a.n_splits;
  const int chunk = rest / a.n_splits;
  const int b = kv_item / a.kv_heads;
  const int kv = kv_item - b * a.kv_heads;
  const int head_group = kv * a.chunks_per_kv + chunk;
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
  const int per_iter = kAttendWaves * slots * U;  // rows of one group (all waves)

  // The split's rows are staged in LDS as K-plane row indices of the pool
  // (block * 2P + offset; 0xffffffff for masked rows), kStage at a time, so
  // the loop below issues its K/V loads back to back without waiting on
  // index loads. Pool rows are < 2^31, checked on the host.
  __shared__ __attribute__((aligned(16))) uint32_t krow[kStage];
  __shared__ int progress[kAttendWaves];  // passes each wave has issued
  for (int s0 = row_begin; s0 < row_end; s0 += kStage) {
    const int s1 = min(row_end, s0 + kStage);
    // every index load of the stage is issued before the first is used
    int64_t rv[kStagePerThread];
#pragma unroll
    for (int j = 0; j < kStagePerThread; ++j) {
      const int i = s0 + j * kAttendThreads + (int)threadIdx.x;
      rv[j] = i < s1 ? rows[(int64_t)i * a.r_cs] : -1;
    }
#pragma unroll
    for (int j = 0; j < kStagePerThread; ++j) {
      const int i = s0 + j * kAttendThreads + (int)threadIdx.x;
      uint32_t kr_idx = 0xffffffffu;
      if (rv[j] >= 0) {
        const uint32_t blk = a.page_div.div((uint32_t)rv[j]);
        kr_idx = blk * (uint32_t)a.page_size + (uint32_t)rv[j];  // blk*2P + (r - blk*P)
      }
      if (i < s1) krow[i - s0] = kr_idx;
    }
    if (threadIdx.x < kAttendWaves) progress[threadIdx.x] = 0;
    __syncthreads();
    // Each pass issues the loads of kIssueGroups row groups back to back and
    // then consumes the groups in order, so a wave keeps up to
    // kIssueGroups * U rows per lane in flight. No loaded register is carried
    // across passes: a carried prefetch makes the compiler copy registers at
    // the loop edge, and the copy waits for every outstanding load.
    // Loads are unconditional: masked rows, padding lanes and rows past the
    // end read the workspace's zero block instead, so no branch separates a
    // load from its use.
    // A lane's U rows are consecutive entries of the staged list, read from
    // LDS with one vector read.
    auto issue = [&](int base, uint4 (&kd)[U][C], uint4 (&vd)[U][C], bool (&okd)[U]) {
      const int first = base + (wave * slots + slot) * U;
      // the read address is clamped into the array (U-aligned); entries at or
      // past s1 are masked by position, so the read needs no branch
      const int at = min(first - s0, kStage - U);
      uint32_t w[U];
      if constexpr (U == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(&krow[at]);
        w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(&krow[at]);
        w[0] = v.x, w[1] = v.y;
      }
      uint32_t ki[U];
#pragma unroll
      for (int u = 0; u < U; ++u) ki[u] = first + u < s1 ? w[u] : 0xffffffffu;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        okd[u] = ki[u] != 0xffffffffu;
        const bool live = okd[u] && data_lane;
        // row ki of the K planes: block ki / 2P, whose stride may exceed its rows by block_pad
        const int64_t at = (int64_t)ki[u] * row_bytes + (int64_t)a.plane2_div.div(ki[u]) * a.block_pad;
        const char* kp = live ? pool + at : a.zeros;
        const int64_t vo = live ? plane_bytes : 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int64_t cb = (int64_t)(c * a.lanes_used + sub) * 16;
          kd[u][c] = *reinterpret_cast<const uint4*>(kp + cb);
          vd[u][c] = *reinterpret_cast<const uint4*>(kp + vo + cb);
        }
      }
    };
    auto consume = [&](const uint4 (&kr)[U][C], const uint4 (&vr)[U][C], const bool (&ok)[U]) {
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
        // arguments are <= 0: v_exp_f32 without range reduction (a weight below
        // 2^-126 flushes to 0)
        alpha[g] = __builtin_amdgcn_exp2f(m[g] - ref);
#pragma unroll
        for (int u = 0; u < U; ++u) p[g][u] = __builtin_amdgcn_exp2f(p[g][u] - ref);
        m[g] = mx;
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][c][e] *= alpha[g];
      if constexpr (PK) {
        // P.V in fp32, as the reference's numerator (row_kernels.py:109-110):
        // each V element is widened once and serves the G heads' weights.
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float psum = 0.f;
#pragma unroll
          for (int u = 0; u < U; ++u) psum += p[g][u];
          l[g] = l[g] * alpha[g] + psum;
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int u = 0; u < U; ++u) {
              const uint32_t x = word_of(vr[u][c], w);
              const float lo = pair_lo<T>(x), hi = pair_hi<T>(x);
#pragma unroll
              for (int g = 0; g < G; ++g) {
                acc[g][c][2 * w] = __builtin_fmaf(p[g][u], lo, acc[g][c][2 * w]);
                acc[g][c][2 * w + 1] = __builtin_fmaf(p[g][u], hi, acc[g][c][2 * w + 1]);
              }
            }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float psum = 0.f;
#pragma unroll
          for (int u = 0; u < U; ++u) psum += p[g][u];
          l[g] = l[g] * alpha[g] + psum;
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
              float x = acc[g][c][e];
#pragma unroll
              for (int u = 0; u < U; ++u) x += p[g][u] * v[u];
              acc[g][c][e] = x;
            }
          }
      }
    };
    // The waves of a workgroup share every pass (a static split of the rows,
    // so the summation order and the result do not depend on timing). Waves
    // that win issue arbitration would run microseconds ahead of the others
    // and leave the CU with too few loads in flight at the end, so each wave
    // publishes its pass count in LDS and sets its issue priority by its lag
    // behind the slowest wave (3 when level, 1 one pass ahead, 0 beyond).
    int pass = 0;
    for (int base = s0; base < s1; base += kIssueGroups * per_iter, ++pass) {
      uint4 kk[kIssueGroups][U][C], vv[kIssueGroups][U][C];
      bool okk[kIssueGroups][U];
#pragma unroll
      for (int gi = 0; gi < kIssueGroups; ++gi) issue(base + gi * per_iter, kk[gi], vv[gi], okk[gi]);
      if (lane == 0) progress[wave] = pass;
      int slowest = pass;
#pragma unroll
      for (int w = 0; w < kAttendWaves; ++w) slowest = min(slowest, progress[w]);
      if (pass > slowest + 1)
        __builtin_amdgcn_s_setprio(0);
      else if (pass > slowest)
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
      for (int gi = 0; gi < kIssueGroups; ++gi)
        if (base + gi * per_iter < s1) consume(kk[gi], vv[gi], okk[gi]);
    }
    __builtin_amdgcn_s_setprio(0);
    if (s1 < row_end) __syncthreads();  // the next stage rewrites krow
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
  if (a.n_splits == 1) {  // the workgroup saw every row: normalise and store
    for (int idx = threadIdx.x; idx < nh * a.head_dim; idx += kAttendThreads) {
      const int g = idx / a.head_dim;
      const int d = idx - g * a.head_dim;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kAttendWaves; ++w) M = fmaxf(M, lds[(w * G + g) * stride]);
      float L = 0.f, v = 0.f;
      if (M != -INFINITY)
#pragma unroll
        for (int w = 0; w < kAttendWaves; ++w) {
          const float* src = lds + (w * G + g) * stride;
          const float f = exp2f(src[0] - M);
          L += src[1] * f;
          v += src[2 + d] * f;
        }
      v = L > 0.f ? v / L : 0.f;
      store_elem(a.out, a.out_dtype, (int64_t)b * a.out_bs + (int64_t)(h0 + g) * a.out_hs + d, v);
    }
    return;
  }
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
  // The partials were written with agent-coherent stores; waiting for them to
  // complete before the arrival orders them without an L2 writeback (an
  // agent-scope fence would write back and invalidate this XCD's whole L2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* counter = a.counters + (int64_t)b * a.kv_heads * a.chunks_per_kv + head_group;
  if (threadIdx.x == 0)
    last_arrival = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.n_splits - 1;
  __syncthreads();
  if (!last_arrival) return;
  const float* base_part = a.ws + ((int64_t)b * a.q_heads + h0) * a.n_splits * stride;
  const int ns = a.n_splits;
  // Each thread loads, in one batch, the split statistics of its head and
  // its element of every split, then merges them.
  for (int idx = threadIdx.x; idx < nh * a.head_dim; idx += kAttendThreads) {
    const int g = idx / a.head_dim;
    const int d = idx - g * a.head_dim;
    const float* hp = base_part + (int64_t)g * ns * stride;
    float ms[kMaxSplits], ls[kMaxSplits], vs[kMaxSplits];
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) {
      ms[s] = ld_coherent(hp + (int64_t)s * stride);
      ls[s] = ld_coherent(hp + (int64_t)s * stride + 1);
      vs[s] = ld_coherent(hp + (int64_t)s * stride + 2 + d);
    }
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ms[s]);
    float L = 0.f, v = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < ns; ++s) {
        const float w = exp2f(ms[s] - M);
        L += ls[s] * w;
        v += vs[s] * w;
      }
    v = L > 0.f ? v / L : 0.f;
    store_elem(a.out, a.out_dtype, (int64_t)b * a.out_bs + (int64_t)(h0 + g) * a.out_hs + d, v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- attend_mfma_kernel: Q K^T on MFMA, P V on the VALU ---------------------
//
// Serves 16-bit KV with a query of the same dtype, head_dim 128, one row list
// shared by the query heads of a request and at most 8 query heads per KV
// head (the GQA shapes of Llama-3-8B and Qwen2-7B). A workgroup of 8 waves
// (two per SIMD) owns one (request, KV head, row split): every row is read
// once per KV head, and the row-level work (addresses, score reduction,
// softmax) is done once per row instead of once per 16-lane row slot. Wave w
// takes tiles w, w + 8, ... of 16 rows, stages their K / V byte offsets in
// its own part of LDS, and works in rounds: the loads of kMDepth tiles, then
// their computation (no loaded register is carried across rounds). The two
// waves of a SIMD are kept level by issue priorities. Per tile, in one wave:
//  - lane l loads chunk l % 16 (16 bytes) of K and of V of rows 4i + l / 16,
//    i = 0..3: each load instruction covers 4 whole 256-byte head rows;
//  - the K chunks go through the wave's LDS tile (chunk c of row r at slot
//    c ^ r: both the writes and the reads below are free of bank conflicts)
//    into the MFMA operand layout of v_mfma_f32_16x16x32 (measured on gfx950:
//    lane l supplies A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16],
//    j = 0..7, and holds D[4 (l / 16) + i][l % 16], i = 0..3): A = the query
//    (head l % 16, zero beyond the group), B = K^T (row l % 16), four k-steps
//    of 32 dims, so lane l ends with the scores of heads 4 (l / 16) + i against
//    row l % 16;
//  - a DPP max over the 16 lanes that share a head gives the tile's max, and
//    the online softmax in base 2 (scale * log2 e applied to the scores)
//    updates the head's running max, its per-lane partial denominators, and
//    P = exp2(score - max);
//  - P goes through LDS to the layout of the V chunks: lane l accumulates
//    P[h][row] * V[row][8 (l % 16) + e] in fp32 for every head h of the group
//    over its rows 4i + l / 16 (the weights stay fp32, as the reference's
//    numerator, row_kernels.py:109-110). When a head's running max moves, its
//    accumulators are scaled by exp2(m_old - m_new), read to a scalar from a
//    lane that holds the head (a factor of exactly 1 is skipped: the bits
//    are the same).
// At the end the four row classes of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48,
// whose accumulators share each head's running max) are summed, the waves
// merge through LDS, and a row split is merged across workgroups by the last
// one to arrive, as in attend_kernel.
constexpr int kMThreads = 512;
constexpr int kMWaves = kMThreads / kWave;
constexpr int kMD = 128;       // head_dim
constexpr int kMTile = 16;     // rows per tile: the MFMA's N
constexpr int kMStage = 1024;  // rows staged in LDS per pass
constexpr int kMMaxGroup = 8;
constexpr int kMDepth = 2;  // tiles whose loads a wave issues together
constexpr int kMWs = kMD + 4;     // floats per partial row in the workspace: m, l, 2 unused, acc
constexpr int kMMaxSplits = 16;
static_assert(kMStage / (kMTile * kMWaves) <= 8, "a wave stages at most two groups of four tiles per pass");

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct AttendMArgs {
  const void* q;
  int64_t q_bs, q_hs;
  const char* pool;
  const int64_t* rows;
  int64_t r_bs, r_cs;
  int n_rows, rows_per_split, n_splits;
  int q_heads, kv_heads, group, page_size;
  int kv_items;
  FastDiv page_div;
  int64_t block_stride;  // pool block stride, bytes
  int64_t row_bytes;     // one plane row, all KV heads, bytes
  float qscale;
  const char* zeros;  // kZeroBytes of zeros
  float* ws;          // partials [B, q_heads, n_splits, head_dim + 4]
  int* counters;      // [B, kv_heads]
  void* out;
  int64_t out_bs, out_hs;
};

template <typename T>
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// max over the 16 lanes of a DPP row, in every lane of the row
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));   // lane ^ 1
  x = fmaxf(x, dpp_f32<0x4E>(x));   // lane ^ 2
  x = fmaxf(x, dpp_f32<0x141>(x));  // quads swap within 8
  x = fmaxf(x, dpp_f32<0x140>(x));  // halves swap within 16
  return x;
}

__device__ __forceinline__ float readlane_f32(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Keeps the compiler from moving memory accesses across this point: the
// LDS tiles are written by some lanes of a wave and read by others, which
// the hardware orders (a wave's LDS instructions execute in order) but the
// compiler cannot see.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// Four 16-byte agent-coherent (sc1) loads, waited for before the asm ends
// (so the compiler never sees registers with loads in flight).
__device__ __forceinline__ void ld4x16_coherent(const u32x4_t* p0, const u32x4_t* p1, const u32x4_t* p2,
                                                const u32x4_t* p3, u32x4_t (&o)[4]) {
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %5, off sc1\n\t"
      "global_load_dwordx4 %2, %6, off sc1\n\t"
      "global_load_dwordx4 %3, %7, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])
      : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
      : "memory");
}

// one tile's loaded chunks: K and V of rows 4i + lane / 16
struct MTile {
  u32x4_t k[4], v[4];
};

template <typename T, int G, int DEPTH>
__global__ __launch_bounds__(kMThreads) void attend_mfma_kernel(AttendMArgs a) {
  constexpr int GQ = (G + 3) / 4;  // 4-head groups of MFMA output lanes
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lrow = lane & 15;  // MFMA row / chunk of a loaded row
  const int lgrp = lane >> 4;  // MFMA k-group / loaded row within 4
  // grid: id = kv_item + kv_items * split, so the splits of a (request, KV
  // head) are kv_items apart (on one XCD when kv_items is a multiple of 8)
  const int kv_item = (int)(blockIdx.x % (unsigned)a.kv_items);
  const int split = (int)(blockIdx.x / (unsigned)a.kv_items);
  const int b = kv_item / a.kv_heads;
  const int kh = kv_item - b * a.kv_heads;
  const int h0 = kh * a.group;
  const int64_t* rows = a.rows + (int64_t)b * a.r_bs;

  // the query as the MFMA A operand: head lrow, dims 8 lgrp + 32 ks .. +8
  u32x4_t qa[kMD / 32];
#pragma unroll
  for (int ks = 0; ks < kMD / 32; ++ks) {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (lrow < G) {
      const uint16_t* qp = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_bs + (int64_t)(h0 + lrow) * a.q_hs +
                           8 * lgrp + 32 * ks;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = (uint32_t)qp[2 * e] | ((uint32_t)qp[2 * e + 1] << 16);
    }
    qa[ks] = (u32x4_t){w[0], w[1], w[2], w[3]};
  }

  float m[4], lsum[4];  // heads 4 lgrp + i: running max, this lane's partial denominator
  float acc[G][8];      // heads 0..G-1, dims 8 lrow + e, over this lane's rows
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lsum[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  // K, V byte offsets from the head's pool base and 1 for a valid row, of a
  // pass's rows, padded with masked rows to whole rounds of DEPTH tiles per
  // wave
  constexpr int kRound = DEPTH * kMTile * kMWaves;
  __shared__ __attribute__((aligned(16))) int64_t soff[kMStage + kRound][2];
  __shared__ uint8_t sok[kMStage + kRound];
  __shared__ u32x4_t ktile[kMWaves][kMTile][16];                      // K chunks, swizzled
  __shared__ __attribute__((aligned(16))) float ptile[kMWaves][kMTile][16];  // P[row][head]
  __shared__ int progress[kMWaves];                                           // tiles each wave has started

  const char* pool_kh = a.pool + (int64_t)kh * kMD * T::bytes;
  const int64_t zoff = a.zeros - pool_kh;  // masked rows read the zero block
  const char* pool_lane = pool_kh + lrow * 16;
  const int64_t plane = (int64_t)a.page_size * a.row_bytes;
  const int row_begin = split * a.rows_per_split;
  const int row_end = min(a.n_rows, row_begin + a.rows_per_split);

  // Each wave clears its own slot; another wave's slot may hold an older
  // value until that wave starts its first tile, which only shifts issue
  // priorities for a moment, so no barrier holds back the first loads.
  if (lane == 0) progress[wave] = 0;
  int started = 0;  // tiles this wave has started, over all passes
  for (int s0 = row_begin; s0 < row_end; s0 += kMStage) {
    const int len = min(kMStage, row_end - s0);
    const int padded = (len + kRound - 1) / kRound * kRound;
    const int ntw = padded / (kMTile * kMWaves);  // tiles of each wave, a multiple of DEPTH, at most 8
    // Each wave stages the rows of its own tiles t = wave + kMWaves * j
    // (lane: tile j0 + l / 16, row l % 16), so no workgroup barrier waits
    // for the slowest wave's index loads; only this wave reads them. Both
    // index loads of a lane are issued before either is used.
    int64_t r2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 4 * h + lgrp;
      const int i = (wave + kMWaves * j) * kMTile + lrow;
      r2[h] = j < ntw && i < len ? rows[(int64_t)(s0 + i) * a.r_cs] : -1;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 4 * h + lgrp;
      const int i = (wave + kMWaves * j) * kMTile + lrow;
      const int64_t r = r2[h];
      if (j < ntw) {
        int64_t ko = zoff, vo = zoff;
        if (r >= 0) {
          const uint32_t blk = a.page_div.div((uint32_t)r);
          ko = (int64_t)blk * a.block_stride + (int64_t)((uint32_t)r - blk * (uint32_t)a.page_size) * a.row_bytes;
          vo = ko + plane;
        }
        soff[i][0] = ko;
        soff[i][1] = vo;
        sok[i] = r >= 0;
      }
    }
    lds_order();

    auto load = [&](int j, MTile& d) __attribute__((always_inline)) {
      const int t = wave + kMWaves * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = t * kMTile + 4 * i + lgrp;
        const int64_t ko = soff[r][0], vo = soff[r][1];
        d.k[i] = *reinterpret_cast<const u32x4_t*>(pool_lane + ko);
        d.v[i] = *reinterpret_cast<const u32x4_t*>(pool_lane + vo);
      }
    };
    auto compute = [&](int j, const MTile& d) __attribute__((always_inline)) {
      const int t = wave + kMWaves * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + lgrp;
        ktile[wave][r][lrow ^ r] = d.k[i];
      }
      const bool ok = sok[t * kMTile + lrow];
      lds_order();
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kMD / 32; ++ks) s = mfma_16x16x32<T>(qa[ks], ktile[wave][lrow][(4 * ks + lgrp) ^ lrow], s);
      float p[4], alpha[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sc = ok ? s[i] * a.qscale : -INFINITY;
        const float mx = fmaxf(m[i], row_max16(sc));
        const float ref = mx == -INFINITY ? 0.f : mx;  // keeps exp2 arguments finite
        // arguments are <= 0: v_exp_f32 without range reduction (a weight
        // below 2^-126 flushes to 0)
        alpha[i] = __builtin_amdgcn_exp2f(m[i] - ref);
        p[i] = __builtin_amdgcn_exp2f(sc - ref);
        lsum[i] = lsum[i] * alpha[i] + p[i];
        m[i] = mx;
      }
      *reinterpret_cast<float4*>(&ptile[wave][lrow][4 * lgrp]) = make_float4(p[0], p[1], p[2], p[3]);
      float al[G];
      bool moved = false;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        al[h] = readlane_f32(alpha[h & 3], 16 * (h >> 2));
        moved |= al[h] != 1.f;
      }
      if (moved) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] *= al[h];
      }
      lds_order();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + lgrp;
        float ph[GQ * 4];
#pragma unroll
        for (int gq = 0; gq < GQ; ++gq) {
          const float4 v = *reinterpret_cast<const float4*>(&ptile[wave][r][4 * gq]);
          ph[4 * gq] = v.x, ph[4 * gq + 1] = v.y, ph[4 * gq + 2] = v.z, ph[4 * gq + 3] = v.w;
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t x = d.v[i][w];
          const float lo = pair_lo<T>(x), hi = pair_hi<T>(x);
#pragma unroll
          for (int h = 0; h < G; ++h) {
            acc[h][2 * w] = __builtin_fmaf(ph[h], lo, acc[h][2 * w]);
            acc[h][2 * w + 1] = __builtin_fmaf(ph[h], hi, acc[h][2 * w + 1]);
          }
        }
      }
      lds_order();
    };

    // Each round issues the loads of DEPTH tiles, then computes them in
    // order; no loaded register is carried into the next round (a carried
    // register makes the compiler wait for every load in flight at the loop
    // edge).
    // The two waves of a SIMD share its issue slots; the one that wins
    // arbitration would run far ahead and leave the CU with too few loads
    // in flight at the end. Each wave publishes the tiles it has started and
    // sets its issue priority by its lead over the slowest wave of the
    // workgroup (3 when level, 1 one round ahead, 0 beyond). The tile
    // assignment stays static, so the result does not depend on timing.
    for (int j = 0; j < ntw; j += DEPTH) {
      MTile t[DEPTH];
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) load(j + d, t[d]);
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        if (lane == 0) progress[wave] = started;
        int slowest = started;
#pragma unroll
        for (int w = 0; w < kMWaves; ++w) slowest = min(slowest, progress[w]);
        if (started > slowest + DEPTH)
          __builtin_amdgcn_s_setprio(0);
        else if (started > slowest)
          __builtin_amdgcn_s_setprio(1);
        else
          __builtin_amdgcn_s_setprio(3);
        compute(j + d, t[d]);
        ++started;
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }

  // denominators over the 16 lanes of each head; accumulators over the four
  // row classes of the wave
#pragma unroll
  for (int i = 0; i < 4; ++i) lsum[i] = group_sum(lsum[i], 16);
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[h][e] += __shfl_xor(acc[h][e], 16);
      acc[h][e] += __shfl_xor(acc[h][e], 32);
    }

  // merge the waves through LDS: [wave][g][2 + head_dim]
  extern __shared__ float lds[];
  __shared__ int last_arrival;
  constexpr int stride = 2 + kMD;
  if (lgrp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float* w = lds + (wave * G + h) * stride + 2 + 8 * lrow;
      *reinterpret_cast<float4*>(w) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      *reinterpret_cast<float4*>(w + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  if (lrow == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * lgrp + i;
      if (h < G) {
        lds[(wave * G + h) * stride] = m[i];
        lds[(wave * G + h) * stride + 1] = lsum[i];
      }
    }
  }
  __syncthreads();
  if (a.n_splits == 1) {  // the workgroup saw every row: normalise and store
    for (int idx = threadIdx.x; idx < G * kMD; idx += kMThreads) {
      const int g = idx / kMD;
      const int d = idx - g * kMD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kMWaves; ++w) M = fmaxf(M, lds[(w * G + g) * stride]);
      float L = 0.f, v = 0.f;
      if (M != -INFINITY)
#pragma unroll
        for (int w = 0; w < kMWaves; ++w) {
          const float* src = lds + (w * G + g) * stride;
          const float f = exp2f(src[0] - M);
          L += src[1] * f;
          v += src[2 + d] * f;
        }
      v = L > 0.f ? v / L : 0.f;
      store_elem(a.out, T::dtype, (int64_t)b * a.out_bs + (int64_t)(h0 + g) * a.out_hs + d, v);
    }
    return;
  }
  // this split's partial: a row of kMWs floats per head, [m, l, 0, 0, acc]
  // (16-byte aligned). The rows of a (request, KV head) form one block
  // starting at row (b * q_heads + h0) * n_splits, ordered [head][split].
  float* part = a.ws + (((int64_t)b * a.q_heads + h0) * a.n_splits + split) * kMWs;
  for (int idx = threadIdx.x; idx < G * kMWs; idx += kMThreads) {
    const int g = idx / kMWs;
    const int j = idx - g * kMWs;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) M = fmaxf(M, lds[(w * G + g) * stride]);
    float o = 0.f;
    if (j == 0) {
      o = M;
    } else if (j == 1 || j >= 4) {
      const int c = j == 1 ? 1 : j - 2;  // column of the waves' rows
      if (M != -INFINITY)
#pragma unroll
        for (int w = 0; w < kMWaves; ++w) {
          const float* src = lds + (w * G + g) * stride;
          o += src[c] * exp2f(src[0] - M);
        }
    }
    st_coherent(part + (int64_t)g * a.n_splits * kMWs + j, o);
  }
  // the last workgroup of this (request, KV head) merges the splits; the
  // partials' agent-coherent stores complete before the arrival
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* counter = a.counters + (int64_t)b * a.kv_heads + kh;
  if (threadIdx.x == 0)
    last_arrival = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.n_splits - 1;
  __syncthreads();
  if (!last_arrival) return;
  // every partial row of this (request, KV head) into LDS (the waves' rows
  // are no longer read), four 16-byte coherent loads per thread at a time
  const int ns = a.n_splits;
  const u32x4_t* block = reinterpret_cast<const u32x4_t*>(a.ws + ((int64_t)b * a.q_heads + h0) * ns * kMWs);
  const int nvec = G * ns * (kMWs / 4);
  for (int v0 = 0; v0 < nvec; v0 += 4 * kMThreads) {
    u32x4_t o[4];
    const u32x4_t* p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) p[k] = block + min(v0 + k * kMThreads + (int)threadIdx.x, nvec - 1);
    ld4x16_coherent(p[0], p[1], p[2], p[3], o);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = v0 + k * kMThreads + (int)threadIdx.x;
      if (i < nvec) reinterpret_cast<u32x4_t*>(lds)[i] = o[k];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kMD; idx += kMThreads) {
    const int g = idx / kMD;
    const int d = idx - g * kMD;
    const float* hp = lds + g * ns * kMWs;
    float M = -INFINITY;
    for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, hp[sp * kMWs]);
    float L = 0.f, v = 0.f;
    if (M != -INFINITY)
      for (int sp = 0; sp < ns; ++sp) {
        const float w = exp2f(hp[sp * kMWs] - M);
        L += hp[sp * kMWs + 1] * w;
        v += hp[sp * kMWs + 4 + d] * w;
      }
    v = L > 0.f ? v / L : 0.f;
    store_elem(a.out, T::dtype, (int64_t)b * a.out_bs + (int64_t)(h0 + g) * a.out_hs + d, v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*AttendMKernel)(AttendMArgs);

static AttendMKernel pick_mfma(int kv_dtype, int G) {
#define NHS_M_CASE(GG) \
  case GG: return kv_dtype == NHS_BF16 ? attend_mfma_kernel<BF16, GG, kMDepth> : attend_mfma_kernel<F16, GG, kMDepth>;
  switch (G) {
    NHS_M_CASE(1) NHS_M_CASE(2) NHS_M_CASE(3) NHS_M_CASE(4) NHS_M_CASE(5) NHS_M_CASE(6) NHS_M_CASE(7) NHS_M_CASE(8)
  }
#undef NHS_M_CASE
  return nullptr;
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
    case 7 * 4 + 1: return pick3<T, 7, 1, PK>();
    case 7 * 4 + 2: return pick3<T, 7, 2, PK>();
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

// Shapes served by attend_mfma_kernel: 16-bit KV with a query of the same
// dtype, head_dim 128, one row list per request, at most 8 query heads per
// KV head. Every other shape runs attend_kernel.
static bool mfma_shape(int kv_dtype, int q_dtype, int64_t rows_head_stride, int head_dim, int group) {
  return (kv_dtype == NHS_BF16 || kv_dtype == NHS_F16) && q_dtype == kv_dtype && rows_head_stride == 0 &&
         head_dim == kMD && group >= 1 && group <= kMMaxGroup;
}

static int max_splits_for(int n_rows) {
  int s = n_rows / kMinRowsPerSplit;
  return s < 1 ? 1 : s > kMaxSplits ? kMaxSplits : s;
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static std::mutex mu;
  static std::vector<std::pair<int, int>> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : cache)
    if (e.first == dev) return e.second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  cache.emplace_back(dev, cus);
  return cus;
}

}  // namespace nhs

extern "C" int64_t nhs_attend_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t n_rows) {
  if (batch < 1 || q_heads < 1 || head_dim < 1 || n_rows < 1) return 0;
  int64_t partials = (int64_t)batch * q_heads * nhs::max_splits_for(n_rows) * (head_dim + 4) * (int64_t)sizeof(float);
  return nhs::kHeaderBytes + partials;
}

extern "C" int nhs_attend_rows(const void* query, int32_t q_dtype, int64_t q_batch_stride, int64_t q_head_stride,
                               const void* pool, int32_t kv_dtype, int64_t pool_block_stride, const int64_t* rows,
                               int64_t rows_batch_stride,
                               int64_t rows_head_stride, int64_t rows_col_stride, int32_t batch, int32_t n_rows,
                               int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size, void* out,
                               int64_t out_batch_stride, int64_t out_head_stride, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
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
  const int64_t block_bytes = 2 * (int64_t)page_size * kv_heads * head_dim * esize;
  if (pool_block_stride == 0) pool_block_stride = block_bytes;
  if (pool_block_stride < block_bytes || pool_block_stride % 16)
    return fail(NHS_ERR_INVALID, "nhs_attend_rows: pool_block_stride must be a multiple of 16 bytes, at least a block");
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
  a.plane2_div = FastDiv(2u * (uint32_t)page_size);
  a.block_pad = pool_block_stride - block_bytes;
  const int C = row_chunks > 64 ? 2 : 1;
  if (row_chunks / C > 64) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: rows too wide");
  a.lanes_used = row_chunks / C;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.qscale = (float)(1.4426950408889634 / sqrt((double)head_dim));
  a.group = q_heads / kv_heads;
  // Grid: one balanced round, about one 8-wave workgroup per CU. A (request,
  // KV head) whose share is several CUs is first divided by query heads
  // (chunks of G heads that each read every row: the repeated reads hit the
  // XCD's L2, and no split merge is needed), then by row splits (merged by
  // the last workgroup to finish).
  const int cus = device_cus();
  const int kv_items = batch * kv_heads;
  if (mfma_shape(kv_dtype, q_dtype, rows_head_stride, head_dim, a.group)) {
    // attend_mfma_kernel: one workgroup per (request, KV head, row split),
    // about one per CU; splits of whole 128-row blocks (every wave gets
    // whole tiles), at most kMMaxSplits
    AttendMArgs m;
    m.q = query;
    m.q_bs = q_batch_stride;
    m.q_hs = q_head_stride;
    m.pool = static_cast<const char*>(pool);
    m.rows = rows;
    m.r_bs = rows_batch_stride;
    m.r_cs = rows_col_stride;
    m.n_rows = n_rows;
    m.q_heads = q_heads;
    m.kv_heads = kv_heads;
    m.group = a.group;
    m.page_size = page_size;
    m.kv_items = kv_items;
    m.page_div = a.page_div;
    m.block_stride = pool_block_stride;
    m.row_bytes = (int64_t)kv_heads * head_dim * esize;
    m.qscale = a.qscale;
    const int target = cus > 0 ? cus : 256;
    int splits = (target + kv_items / 2) / kv_items;
    if (splits < 1) splits = 1;
    if (splits > max_splits_for(n_rows)) splits = max_splits_for(n_rows);
    if (splits > kMMaxSplits) splits = kMMaxSplits;
    const int block = kMTile * kMWaves;
    int per = (n_rows + splits - 1) / splits;
    per = (per + block - 1) / block * block;
    splits = (n_rows + per - 1) / per;
    if ((int64_t)kv_items * splits > 0x7fffffff) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: grid too large");
    m.n_splits = splits;
    m.rows_per_split = per;
    m.counters = static_cast<int*>(workspace);
    m.zeros = static_cast<const char*>(workspace) + kCounterBytes;
    m.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kHeaderBytes);
    m.out = out;
    m.out_bs = out_batch_stride;
    m.out_hs = out_head_stride;
    AttendMKernel kernel = pick_mfma(kv_dtype, a.group);
    const size_t lds = (size_t)std::max(kMWaves * a.group * (2 + kMD), a.group * splits * kMWs) * sizeof(float);
    launch(kernel, dim3((unsigned)(kv_items * splits)), dim3(kMThreads), lds, (hipStream_t)stream, ev.start, ev.stop,
           m);
    return launch_status("nhs_attend_rows");
  }
  const int share = cus > 0 ? (cus + kv_items / 2) / kv_items : 1;  // workgroups per (request, KV head)
  int G;
  if (rows_head_stride != 0) {
    G = 1;  // one head per workgroup; its own row list
    a.chunks_per_kv = a.group;
  } else {
    int chunks = 1;
    while (chunks * 2 <= share && chunks * 2 <= a.group && chunks * 2 <= kMaxHeadChunks) chunks *= 2;
    const int per_chunk = (a.group + chunks - 1) / chunks;
    // 7 has its own instance (Qwen2 groups of 7 heads): rounded up to 8, one
    // head of every group would be computed and masked
    G = per_chunk <= 1 ? 1 : per_chunk <= 2 ? 2 : per_chunk <= 4 ? 4 : per_chunk == 7 ? 7 : 8;
    a.chunks_per_kv = (a.group + G - 1) / G;
  }
  AttendKernel kernel = pick_kernel(kv_dtype, packed, G, C);
  if (!kernel) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: no kernel for G=%d C=%d", G, C);
  const size_t lds = (size_t)kAttendWaves * G * (2 + head_dim) * sizeof(float);
  const int units = kv_items * a.chunks_per_kv;
  int splits = cus > 0 ? (cus + units / 2) / units : 1;
  if (splits < 1) splits = 1;
  if (splits > max_splits_for(n_rows)) splits = max_splits_for(n_rows);
  if ((int64_t)units * splits > 0x7fffffff) return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: grid too large");
  a.kv_items = kv_items;
  a.n_splits = splits;
  a.rows_per_split = (n_rows + splits - 1) / splits;
  a.counters = static_cast<int*>(workspace);
  a.zeros = static_cast<const char*>(workspace) + kCounterBytes;
  a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kHeaderBytes);
  a.out = out;
  a.out_dtype = q_dtype;
  a.out_bs = out_batch_stride;
  a.out_hs = out_head_stride;
  launch(kernel, dim3((unsigned)(units * splits)), dim3(kAttendThreads), lds, (hipStream_t)stream, ev.start, ev.stop,
         a);
  return launch_status("nhs_attend_rows");
}

// ---- allocation-free entry point -------------------------------------------
//
// nhs_attend_rows_noalloc runs nhs_attend_rows on a workspace held in this
// file-scope device array, for callers that cannot allocate. Each GPU the
// library runs on holds its own copy until the process ends. On a device's
// first call (with that device current) the array's device address is
// looked up with hipGetSymbolAddress and kept per device, and its header
// (arrival counters and zero block) is cleared by a fill kernel on the
// caller's stream; every call leaves the header zero again. Host code uses
// only the looked-up address, never the array's name. All calls on one GPU
// share the array, so calls that overlap on one GPU race.
namespace nhs {

constexpr int64_t kNoAllocScratchBytes = NHS_ATTEND_NOALLOC_BYTES;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

__global__ void clear_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// The current device's address of `scratch`, set up on its first call.
static int scratch_on_device(hipStream_t stream, void** out) {
  static std::mutex mu;
  static std::vector<std::pair<int, void*>> addresses;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "nhs_attend_rows_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& a : addresses)
    if (a.first == dev) {
      *out = a.second;
      return NHS_OK;
    }
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(e != hipSuccess ? (int)e : NHS_ERR_INVALID, "nhs_attend_rows_noalloc: hipGetSymbolAddress: %s",
                hipGetErrorString(e));
  hipLaunchKernelGGL(clear_words_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint32_t*>(p),
                     kHeaderBytes / (int64_t)sizeof(uint32_t));
  const int st = launch_status("nhs_attend_rows_noalloc");
  if (st != NHS_OK) return st;
  addresses.emplace_back(dev, p);
  *out = p;
  return NHS_OK;
}

}  // namespace nhs

extern "C" int nhs_attend_rows_noalloc(const void* query, int32_t q_dtype, int64_t q_batch_stride,
                                       int64_t q_head_stride, const void* pool, int32_t kv_dtype,
                                       int64_t pool_block_stride, const int64_t* rows,
                                       int64_t rows_batch_stride, int64_t rows_head_stride, int64_t rows_col_stride,
                                       int32_t batch, int32_t n_rows, int32_t q_heads, int32_t kv_heads,
                                       int32_t head_dim, int32_t page_size, void* out, int64_t out_batch_stride,
                                       int64_t out_head_stride, void* stream) {
  using namespace nhs;
  const int64_t need = nhs_attend_workspace_bytes(batch, q_heads, head_dim, n_rows);
  if (need > kNoAllocScratchBytes)
    return fail(NHS_ERR_WORKSPACE,
                "nhs_attend_rows_noalloc: this shape needs %lld bytes of scratch, above the %lld-byte maximum",
                (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int st = scratch_on_device((hipStream_t)stream, &ws);
  if (st != NHS_OK) return st;
  return nhs_attend_rows(query, q_dtype, q_batch_stride, q_head_stride, pool, kv_dtype, pool_block_stride, rows,
                         rows_batch_stride,
                         rows_head_stride, rows_col_stride, batch, n_rows, q_heads, kv_heads, head_dim, page_size, out,
                         out_batch_stride, out_head_stride, ws, kNoAllocScratchBytes, stream);
}
