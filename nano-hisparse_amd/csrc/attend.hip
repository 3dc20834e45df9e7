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
  int64_t partials = (int64_t)batch * q_heads * nhs::max_splits_for(n_rows) * (head_dim + 2) * (int64_t)sizeof(float);
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
