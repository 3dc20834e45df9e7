// Physical-row GQA decode attention over selected pool rows.
//
// Pass 1 (attend_split_kernel): a workgroup of 4 waves owns one request, up
// to G query heads that share a row list (the GQA group of one KV head, or a
// single head for per-head row lists) and one contiguous split of the row
// list. Each row's K (and V) for the KV head is head_dim contiguous elements;
// `lpr` lanes (a power of two) read it as 16-byte chunks of E elements, so a
// wave covers 64/lpr rows per load instruction. The loaded K/V chunks stay in
// registers and are applied to all G query heads: the pool is read once per
// KV head, not once per query head. Scores are reduced across the lpr lanes
// of a row with DPP, then an online softmax (base 2, the scale*log2(e) folded
// into q) accumulates (m, l, acc) per row slot. Slots are merged within the
// wave by shuffles and across waves through LDS; the workgroup writes
// (m, l, acc[head_dim]) for its split to the fp32 workspace.
//
// Pass 2 (attend_combine_kernel): merges the splits of each (request, head),
// divides by the softmax denominator (0 when no row was valid) and stores
// the query's dtype.
#include <math.h>

#include "nhs_common.h"

namespace nhs {

constexpr int kAttendThreads = 256;
constexpr int kAttendWaves = kAttendThreads / kWave;
constexpr int kUnroll = 4;  // rows per lane slot per iteration (loads in flight)

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
  float* ws;
};

__device__ __forceinline__ void merge_state(float& m, float& l, float m_o, float l_o, float& a, float& b) {
  float mx = fmaxf(m, m_o);
  if (mx == -INFINITY) {
    a = 0.f;
    b = 0.f;
    return;
  }
  a = exp2f(m - mx);
  b = exp2f(m_o - mx);
  l = l * a + l_o * b;
  m = mx;
}

template <typename T, int E, int G>
__global__ __launch_bounds__(kAttendThreads) void attend_split_kernel(AttendArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lpr = 1 << a.lpr_log2;
  const int slots = kWave >> a.lpr_log2;  // rows per wave per load
  const int slot = lane >> a.lpr_log2;
  const int sub = lane & (lpr - 1);
  const bool data_lane = sub < a.lanes_used;

  const int split = blockIdx.x;
  const int kv = blockIdx.y / a.chunks_per_kv;
  const int chunk = blockIdx.y - kv * a.chunks_per_kv;
  const int b = blockIdx.z;
  const int h0 = kv * a.group + chunk * G;  // first query head of this workgroup
  const int nh = min(G, a.group - chunk * G);

  // Per-head row lists (legacy selections) give each query head its own list;
  // such launches use G == 1 so the workgroup's heads share one list.
  const int64_t* rows = a.rows + (int64_t)b * a.r_bs + (int64_t)h0 * a.r_hs;

  float qv[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      int d = sub * E + e;
      qv[g][e] = (g < nh && data_lane && d < a.head_dim)
                     ? load_elem(a.q, a.q_dtype, (int64_t)b * a.q_bs + (int64_t)(h0 + g) * a.q_hs + d) * a.qscale
                     : 0.f;
    }

  float m[G], l[G], acc[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
  }

  const int row_begin = split * a.rows_per_split;
  const int row_end = min(a.n_rows, row_begin + a.rows_per_split);
  const int64_t row_elems = (int64_t)a.kv_heads * a.head_dim;           // one plane row
  const int64_t plane_elems = (int64_t)a.page_size * row_elems;         // V offset from K
  const int64_t block_elems = 2 * plane_elems;
  const int per_iter = kAttendWaves * slots * kUnroll;

  for (int base = row_begin; base < row_end; base += per_iter) {
    float kf[kUnroll][E], vf[kUnroll][E];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int c = base + (u * kAttendWaves + wave) * slots + slot;
      int64_t r = c < row_end ? rows[(int64_t)c * a.r_cs] : -1;
      ok[u] = r >= 0;
      if (r >= 0 && data_lane) {
        // Pool rows are < 2^31 (checked on the host from the pool size).
        uint32_t ru = (uint32_t)r;
        uint32_t blk32 = a.page_div.div(ru);
        int64_t blk = blk32;
        int64_t off = ru - blk32 * (uint32_t)a.page_size;
        int64_t kidx = blk * block_elems + off * row_elems + (int64_t)kv * a.head_dim + sub * E;
        load_vec<T, E>(a.pool, kidx, kf[u]);
        load_vec<T, E>(a.pool, kidx + plane_elems, vf[u]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) kf[u][e] = vf[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[kUnroll];
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) dot += qv[g][e] * kf[u][e];
        dot = group_sum(dot, lpr);
        s[u] = ok[u] ? dot : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      if (mx == -INFINITY) continue;  // nothing valid yet for this head
      float alpha = exp2f(m[g] - mx);
      float psum = 0.f;
      float p[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        p[u] = exp2f(s[u] - mx);
        psum += p[u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float v = acc[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v += p[u] * vf[u][e];
        acc[g][e] = v;
      }
      m[g] = mx;
    }
  }

  // Merge the row slots of this wave (lanes that differ in the slot bits).
  for (int st = lpr; st < kWave; st <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float m_o = __shfl_xor(m[g], st);
      float l_o = __shfl_xor(l[g], st);
      float fa, fb;
      merge_state(m[g], l[g], m_o, l_o, fa, fb);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float acc_o = __shfl_xor(acc[g][e], st);
        acc[g][e] = acc[g][e] * fa + acc_o * fb;
      }
    }
  }

  // Merge the 4 waves through LDS: [wave][g][2 + head_dim].
  extern __shared__ float lds[];
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
        for (int e = 0; e < E; ++e)
          if (sub * E + e < a.head_dim) w[2 + sub * E + e] = acc[g][e];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < nh * (a.head_dim + 2); idx += kAttendThreads) {
    int g = idx / (a.head_dim + 2);
    int j = idx - g * (a.head_dim + 2);
    float M = -INFINITY;
    for (int w = 0; w < kAttendWaves; ++w) M = fmaxf(M, lds[(w * G + g) * stride]);
    float out;
    if (j == 0) {
      out = M;
    } else {
      out = 0.f;
      if (M != -INFINITY)
        for (int w = 0; w < kAttendWaves; ++w) {
          const float* src = lds + (w * G + g) * stride;
          out += src[j] * exp2f(src[0] - M);
        }
    }
    int64_t o = (((int64_t)b * a.q_heads + h0 + g) * a.n_splits + split) * stride + j;
    a.ws[o] = out;
  }
}

__global__ __launch_bounds__(128) void attend_combine_kernel(const float* __restrict__ ws, int n_splits, int head_dim,
                                                             int q_heads, void* out, int out_dtype, int64_t out_bs,
                                                             int64_t out_hs) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int stride = 2 + head_dim;
  const float* base = ws + ((int64_t)b * q_heads + h) * n_splits * stride;
  float M = -INFINITY;
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, base[(int64_t)s * stride]);
  float L = 0.f;
  if (M != -INFINITY)
    for (int s = 0; s < n_splits; ++s) L += base[(int64_t)s * stride + 1] * exp2f(base[(int64_t)s * stride] - M);
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float v = 0.f;
    if (L > 0.f) {
      for (int s = 0; s < n_splits; ++s)
        v += base[(int64_t)s * stride + 2 + d] * exp2f(base[(int64_t)s * stride] - M);
      v /= L;
    }
    store_elem(out, out_dtype, (int64_t)b * out_bs + (int64_t)h * out_hs + d, v);
  }
}

// Number of row splits per (request, head); the workspace holds
// batch*q_heads*splits*(head_dim+2) floats.
static int attend_splits(int batch, int q_heads, int n_rows) {
  const int target_heads = 4096;  // aim for >= ~4 workgroups per CU on 256 CUs
  int max_splits = (n_rows + 63) / 64;
  int want = (target_heads + batch * q_heads - 1) / (batch * q_heads);
  int s = want < max_splits ? want : max_splits;
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

template <typename T, int E, int G>
static void launch_split(const AttendArgs& a, dim3 grid, hipStream_t s) {
  size_t lds = (size_t)kAttendWaves * G * (2 + a.head_dim) * sizeof(float);
  hipLaunchKernelGGL((attend_split_kernel<T, E, G>), grid, dim3(kAttendThreads), lds, s, a);
}

template <typename T, int E>
static int dispatch_g(const AttendArgs& a, int G, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_split<T, E, 1>(a, grid, s); break;
    case 2: launch_split<T, E, 2>(a, grid, s); break;
    case 4: launch_split<T, E, 4>(a, grid, s); break;
    case 8: launch_split<T, E, 8>(a, grid, s); break;
    default: return fail(NHS_ERR_UNSUPPORTED, "attend: no kernel for %d heads per workgroup", G);
  }
  return NHS_OK;
}

}  // namespace nhs

extern "C" int64_t nhs_attend_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t n_rows) {
  if (batch < 1 || q_heads < 1 || head_dim < 1 || n_rows < 1) return 0;
  return (int64_t)batch * q_heads * nhs::attend_splits(batch, q_heads, n_rows) * (head_dim + 2) * (int64_t)sizeof(float);
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
  int64_t need = nhs_attend_workspace_bytes(batch, q_heads, head_dim, n_rows);
  if (workspace_bytes < need)
    return fail(NHS_ERR_WORKSPACE, "nhs_attend_rows: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
  const int esize = elem_size(kv_dtype);
  const int row_bytes = head_dim * esize;
  if (row_bytes % 16 || row_bytes > 1024)
    return fail(NHS_ERR_UNSUPPORTED, "nhs_attend_rows: head_dim*element size must be a multiple of 16 bytes, <= 1024");
  if ((uintptr_t)pool % 16) return fail(NHS_ERR_INVALID, "nhs_attend_rows: pool must be 16-byte aligned");

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
  a.n_splits = attend_splits(batch, q_heads, n_rows);
  a.rows_per_split = (n_rows + a.n_splits - 1) / a.n_splits;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.page_size = page_size;
  a.page_div = FastDiv((uint32_t)page_size);
  a.lanes_used = row_bytes / 16;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.qscale = (float)(1.4426950408889634 / sqrt((double)head_dim));
  a.ws = static_cast<float*>(workspace);

  const int group = q_heads / kv_heads;
  int G;
  if (rows_head_stride != 0) {
    // Each query head has its own row list: one head per workgroup, and a
    // "group" of one so that head h maps to KV head h / (q_heads/kv_heads).
    G = 1;
  } else {
    G = group >= 8 ? 8 : group >= 4 ? (group == 4 ? 4 : 8) : group == 3 ? 4 : group;
  }
  dim3 grid;
  if (rows_head_stride != 0) {
    // One workgroup per query head; express it as kv_heads "kv" units of
    // `group` chunks of one head each.
    a.group = group;
    a.chunks_per_kv = group;
  } else {
    a.group = group;
    a.chunks_per_kv = (group + G - 1) / G;
  }
  grid = dim3((unsigned)a.n_splits, (unsigned)(kv_heads * a.chunks_per_kv), (unsigned)batch);
  hipStream_t s = (hipStream_t)stream;
  int st;
  switch (kv_dtype) {
    case NHS_F32: st = dispatch_g<F32, 4>(a, G, grid, s); break;
    case NHS_F16: st = dispatch_g<F16, 8>(a, G, grid, s); break;
    default: st = dispatch_g<BF16, 8>(a, G, grid, s); break;
  }
  if (st != NHS_OK) return st;
  st = launch_status("nhs_attend_rows (split)");
  if (st != NHS_OK) return st;
  hipLaunchKernelGGL(attend_combine_kernel, dim3((unsigned)q_heads, (unsigned)batch), dim3(128), 0, s, a.ws,
                     a.n_splits, head_dim, q_heads, out, q_dtype, out_batch_stride, out_head_stride);
  return launch_status("nhs_attend_rows (combine)");
}
