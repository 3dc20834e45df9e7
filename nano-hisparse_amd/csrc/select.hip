// Page selectors: Quest min/max-bound scoring (selection.py:69-91) and the
// page-mean selector (selection.py:119-145), each followed by one shared
// top-k per request, page -> token expansion and -1 padding.
//
// Scoring (one wave per page, 4 waves per workgroup): a page's bounds for one
// KV head are head_dim contiguous elements, read as E-element chunks by
// `lpr` lanes (a power of two; lanes past head_dim/E contribute +0.0). Every
// lane sums its chunk sequentially, the lanes of a head are summed by the
// pairwise DPP tree of group_sum(), and lane 0 of the wave sums the heads
// sequentially. This order is fixed and restated by the CPU oracle, so the
// scores and the chosen pages are bit-identical to it. FMA contraction is
// disabled in this file so that products are rounded before they are added.
//
// Selection (one workgroup per request): keys are the scores mapped to
// order-preserving uint32 (required pages get the maximum key). Up to 1024
// pages, one wave finds the key of the k-th best page bit by bit with ballots;
// beyond, a 4-pass 8-bit radix select does. Ties at that key go to the lowest
// page indices, and the chosen pages are emitted in ascending order and
// expanded to token positions.
#include <math.h>

#include "nhs_common.h"

#pragma clang fp contract(off)

namespace nhs {

constexpr int kScoreThreads = 256;
constexpr int kScoreWaves = kScoreThreads / kWave;
constexpr int kPagesPerBlock = 8;
constexpr int kQuestThreads = 512;
constexpr int kSelectThreads = 1024;
constexpr int kMaxSelectPerThread = NHS_MAX_SELECT_PAGES / kSelectThreads;  // 16
constexpr int kSelectWaveThreads = 256;  // one-wave selection; 4 waves expand the positions

enum { kModeQuest = 0, kModeMean = 1 };

struct ScoreArgs {
  const void* q;
  int q_dtype;
  int q_vec;  // query rows may be read with 16-byte loads
  int64_t q_bs, q_hs;
  const void* lo;   // quest: minimum; mean: summaries (fp32)
  const void* hi;   // quest: maximum
  int64_t b_bs;     // elements between requests' bound tensors
  int q_heads, kv_heads, head_dim, group;
  int lanes_used, lpr_log2;
  int pages_per_step, pages_per_block;
  const int64_t* lengths;
  int64_t length;
  int page_size, max_pages;
  float* scores;
  const nhs_layer_item* items;  // per-item bounds (then lo, hi and b_bs are unused)
};

// Request b's bound rows: from its item entry, or strided from lo / hi.
template <typename T>
__device__ __forceinline__ void bounds_of(const ScoreArgs& a, int b, const char*& lo, const char*& hi) {
  if (a.items) {
    lo = static_cast<const char*>(a.items[b].minimum);
    hi = static_cast<const char*>(a.items[b].maximum);
  } else {
    lo = static_cast<const char*>(a.lo) + (int64_t)b * a.b_bs * T::bytes;
    hi = static_cast<const char*>(a.hi) + (int64_t)b * a.b_bs * T::bytes;
  }
}

__device__ __forceinline__ float torch_maximum(float a, float b) {
  // torch.maximum propagates NaN from either operand.
  if (a != a || b != b) return a + b;
  return a > b ? a : b;
}

__device__ __forceinline__ int page_count(const int64_t* lengths, int64_t length, int b, int page_size, int max_pages) {
  int64_t len = lengths ? lengths[b] : length;
  if (len <= 0) return 0;
  int64_t c = (len + page_size - 1) / page_size;
  return (int)(c < max_pages ? c : max_pages);
}

// Quest bounds score: (sum_h sum_d max(q*min, q*max)) / q_heads.
//
// The heads of one KV head's GQA group contribute q*kmax where q > 0 and
// q*kmin elsewhere (kmax >= kmin), so per (KV head, d) the group's terms are
//   kmin[d] * Qneg[d] + kmax[d] * Qpos[d]
// with Qpos / Qneg the group's positive / non-positive query sums (added in
// head order from 0.0, once per request). A lane keeps them for its chunk
// and scores a page with two fmas per element, t = fma(kmin', Qneg, t) then
// t = fma(kmax', Qpos, t), where kmin' (kmax') is 0 when no head of the
// group is non-positive (positive) at d, so a bound nobody selects is never
// multiplied. Chunk sums are added as a pairwise tree over a KV head's
// lanes, the KV-head sums sequentially; the CPU oracle sums in this order.
//
// element e of E packed elements of T (raw 32-bit words), widened exactly to fp32
template <typename T, int E>
__device__ __forceinline__ float packed_elem(const uint32_t (&w)[E * T::bytes / 4], int e) {
  if constexpr (T::bytes == 4) {
    return __uint_as_float(w[e]);
  } else {
    const uint32_t word = w[e >> 1];
    if constexpr (T::dtype == NHS_BF16)
      return __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
    else
      return f16_bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
  }
}

// The per-lane grouped sums (and the masks of which side has contributors).
// Branch-free: a query value adds +0.0 to the other side's sum, which leaves
// it unchanged (the positive sum starts at +0.0 and only grows, the
// non-positive one starts at +0.0 and never becomes -0.0); the side flags
// are bit e of two per-lane masks.
template <int E, int G>
struct GroupedQuery {
  static_assert(E <= 32, "side masks hold one bit per element");
  float pos[E], neg[E];
  uint32_t has_pos = 0, has_neg = 0;  // bit e: a head of the group is > 0 (<= 0) at element e
  // qv: the lane's slices of the group's query heads; live: this lane holds
  // data (padding lanes add exactly +0)
  __device__ __forceinline__ void init(const float (&qv)[G][E], int group, bool live) {
#pragma clang fp contract(off)
    uint32_t hp_bits = 0, hn_bits = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float p = 0.f, n = 0.f;
      uint32_t hp = 0, hn = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float q = qv[g][e];
        const bool in_group = g < group;
        const bool up = q > 0.f;
        p = p + (in_group && up ? q : 0.f);
        n = n + (in_group && !up ? q : 0.f);
        hp |= (uint32_t)(in_group && up);
        hn |= (uint32_t)(in_group && !up);
      }
      pos[e] = p, neg[e] = n;
      hp_bits |= hp << e;
      hn_bits |= hn << e;
    }
    has_pos = live ? hp_bits : 0u;
    has_neg = live ? hn_bits : 0u;
  }
  // init() from the heads' slices kept packed in T (widened element by element)
  // (all G heads are in the group)
  template <typename T>
  __device__ __forceinline__ void init_packed(const uint32_t (&qw)[G][E * T::bytes / 4], bool live) {
#pragma clang fp contract(off)
    uint32_t hp_bits = 0, hn_bits = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float p = 0.f, n = 0.f;
      uint32_t hp = 0, hn = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float q = packed_elem<T, E>(qw[g], e);
        const bool up = q > 0.f;
        p = p + (up ? q : 0.f);
        n = n + (up ? 0.f : q);
        hp |= (uint32_t)up;
        hn |= (uint32_t)!up;
      }
      pos[e] = p, neg[e] = n;
      hp_bits |= hp << e;
      hn_bits |= hn << e;
    }
    has_pos = live ? hp_bits : 0u;
    has_neg = live ? hn_bits : 0u;
  }
  // chunk() of bounds kept packed in T
  template <typename T>
  __device__ __forceinline__ float chunk_packed(const uint32_t (&mn)[E * T::bytes / 4],
                                                const uint32_t (&mx)[E * T::bytes / 4]) const {
    float x = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      x = __builtin_fmaf((has_neg >> e) & 1u ? packed_elem<T, E>(mn, e) : 0.f, neg[e], x);
      x = __builtin_fmaf((has_pos >> e) & 1u ? packed_elem<T, E>(mx, e) : 0.f, pos[e], x);
    }
    return x;
  }
  // this lane's chunk sum for one page's bounds
  __device__ __forceinline__ float chunk(const float (&mn)[E], const float (&mx)[E]) const {
    float x = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      x = __builtin_fmaf((has_neg >> e) & 1u ? mn[e] : 0.f, neg[e], x);
      x = __builtin_fmaf((has_pos >> e) & 1u ? mx[e] : 0.f, pos[e], x);
    }
    return x;
  }
};
//
// General kernel, for pages wider than one wave: lanes are laid out as (page
// of the step, kv head, chunk), so a lane keeps one kv head's query slices
// in registers for the whole kernel; the next step's bounds are requested
// before the current step is summed.
template <typename T, int E, int G>
__global__ __launch_bounds__(kQuestThreads) void quest_score_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float smem[];
  const int pages_per_step = a.pages_per_step;
  float* qs = smem;                              // [q_heads * head_dim]
  float* hs = smem + a.q_heads * a.head_dim;     // [pages_per_step][kv_heads]
  const int b = blockIdx.y;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int p_begin = blockIdx.x * a.pages_per_block;
  if (p_begin >= count) return;
  const int p_end = min(count, p_begin + a.pages_per_block);
  for (int i = threadIdx.x; i < a.q_heads * a.head_dim; i += blockDim.x) {
    const int h = i / a.head_dim, d = i - h * a.head_dim;
    qs[i] = load_elem(a.q, a.q_dtype, (int64_t)b * a.q_bs + (int64_t)h * a.q_hs + d);
  }
  __syncthreads();
  const int lpr = 1 << a.lpr_log2;
  const int lanes_per_page = a.kv_heads << a.lpr_log2;
  const int page_local = threadIdx.x / lanes_per_page;
  const int within = threadIdx.x - page_local * lanes_per_page;
  const int kh = within >> a.lpr_log2;
  const int sub = within & (lpr - 1);
  const bool active = page_local < pages_per_step;
  const bool data = active && sub < a.lanes_used;
  float qv[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < E; ++e) qv[g][e] = data && g < a.group ? qs[(kh * a.group + g) * a.head_dim + sub * E + e] : 0.f;
  GroupedQuery<E, G> gq;
  gq.init(qv, a.group, data);
  const char *lo, *hi;
  bounds_of<T>(a, b, lo, hi);
  const int64_t page_elems = (int64_t)a.kv_heads * a.head_dim;
  const int64_t lane_off = data ? (int64_t)kh * a.head_dim + sub * E : 0;
  auto load = [&](int p, float (&mn)[E], float (&mx)[E]) {
    const int pc = (active && p < p_end) ? p : p_begin;  // idle lanes reread a live page
    load_vec<T, E>(lo, (int64_t)pc * page_elems + lane_off, mn);
    load_vec<T, E>(hi, (int64_t)pc * page_elems + lane_off, mx);
  };
  float mn[E], mx[E], mn2[E], mx2[E];
  load(p_begin + page_local, mn, mx);
  for (int base = p_begin; base < p_end; base += pages_per_step) {
    const int p = base + page_local;
    load(p + pages_per_step, mn2, mx2);
    const float t = group_sum(gq.chunk(mn, mx), lpr);
    if (active && sub == 0 && p < p_end) hs[page_local * a.kv_heads + kh] = t;
    __syncthreads();
    if ((int)threadIdx.x < pages_per_step && base + (int)threadIdx.x < p_end) {
      const float* row = hs + threadIdx.x * a.kv_heads;
      float total = row[0];
      for (int h = 1; h < a.kv_heads; ++h) total = total + row[h];
      a.scores[(int64_t)b * a.max_pages + base + threadIdx.x] = total / (float)a.q_heads;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      mn[e] = mn2[e];
      mx[e] = mx2[e];
    }
  }
}

// Page kernel, for pages that fit one wave (kv_heads * lanes per head <=
// 64, 32-byte chunks): lane = (page of the wave, kv head, chunk). A wave
// loads its query slices straight into registers, issues the bounds of all
// its page_slots(G) page slots, forms the grouped sums, then scores every
// slot (per-lane chunk sum, DPP tree over a KV head's lanes) and forms the
// slots' sequential KV-head sums together from lane reads, with no barrier.
// It is instantiated for each group size G (1..8), so no head is masked.
constexpr int kPageThreads = 256;
constexpr int kPageWaves = kPageThreads / kWave;
// Page slots per wave: 2 up to 4 query heads per KV head, else 4. With the
// smaller group the second slot pair is better spent on more waves (Quest +
// select 17.0-17.6 against 18.0 us at Llama-3-8B heads); with 7 heads the
// query registers dominate, waves per SIMD stay at 3 and 2 slots lost (58
// against 49 us at Qwen2-7B heads).
__host__ __device__ constexpr int page_slots(int group) { return group <= 4 ? 2 : 4; }

template <typename T, int E, int G>
__global__ __launch_bounds__(kPageThreads) void quest_page_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int ppw = a.pages_per_step;  // pages per wave slot
  constexpr int S = page_slots(G);
  const int wave_first = (blockIdx.x * kPageWaves + wave) * S * ppw;
  if (wave_first >= count) return;
  const int lanes_per_page = a.kv_heads << a.lpr_log2;
  const int page_local = lane / lanes_per_page;
  const int within = lane - page_local * lanes_per_page;
  const int kh = within >> a.lpr_log2;
  const int sub = within & ((1 << a.lpr_log2) - 1);
  const bool data = page_local < ppw && sub < a.lanes_used;

  // Query slices and bounds stay packed in their dtype until folded or
  // scored (widening them at load time doubled the registers and halved
  // the waves a SIMD holds). The bounds of every slot are requested before
  // the query slices are used, so the two memory latencies overlap.
  constexpr int W = E * T::bytes / 4;  // 32-bit words of a lane's 32-byte chunk
  int64_t qi[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qi[g] = (int64_t)b * a.q_bs + (data ? (int64_t)(kh * G + g) * a.q_hs + sub * E : 0);
  const char *lo, *hi;
  bounds_of<T>(a, b, lo, hi);
  const int64_t page_elems = (int64_t)a.kv_heads * a.head_dim;
  const int64_t lane_off = data ? (int64_t)kh * a.head_dim + sub * E : 0;
  uint32_t mn[S][W], mx[S][W];
  auto load_bounds = [&]() {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int p = wave_first + s * ppw + page_local;
      const int pc = p < count ? p : wave_first;  // lanes past the end reread a live page
      const uint4* lp = reinterpret_cast<const uint4*>(lo + ((int64_t)pc * page_elems + lane_off) * T::bytes);
      const uint4* hp = reinterpret_cast<const uint4*>(hi + ((int64_t)pc * page_elems + lane_off) * T::bytes);
#pragma unroll
      for (int v = 0; v < W / 4; ++v) {
        const uint4 x = lp[v], y = hp[v];
        mn[s][4 * v] = x.x, mn[s][4 * v + 1] = x.y, mn[s][4 * v + 2] = x.z, mn[s][4 * v + 3] = x.w;
        mx[s][4 * v] = y.x, mx[s][4 * v + 1] = y.y, mx[s][4 * v + 2] = y.z, mx[s][4 * v + 3] = y.w;
      }
    }
  };
  GroupedQuery<E, G> gq;  // G is the group size here: nothing to mask
  if (a.q_vec && a.q_dtype == T::dtype) {
    uint32_t qw[G][W];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4* qp = reinterpret_cast<const uint4*>(static_cast<const char*>(a.q) + qi[g] * T::bytes);
#pragma unroll
      for (int v = 0; v < W / 4; ++v) {
        const uint4 x = qp[v];
        qw[g][4 * v] = x.x, qw[g][4 * v + 1] = x.y, qw[g][4 * v + 2] = x.z, qw[g][4 * v + 3] = x.w;
      }
    }
    load_bounds();
    gq.template init_packed<T>(qw, data);
  } else {
    float qv[G][E];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < E; ++e) qv[g][e] = load_elem(a.q, a.q_dtype, qi[g] + (data ? e : 0));
    load_bounds();
    gq.init(qv, G, data);
  }
  const int lpr = 1 << a.lpr_log2;
  const int page_lane0 = page_local * lanes_per_page;
  // every slot is scored first (slots past count hold a live page's bounds
  // and are not stored), then the KV-head sums of all slots are formed
  // together: each group of 8 heads issues its lane reads for every slot
  // before the adds, which stay sequential in head order
  float t[S], total[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    t[s] = group_sum(gq.template chunk_packed<T>(mn[s], mx[s]), lpr);
    total[s] = 0.f;
  }
  for (int h0 = 0; h0 < a.kv_heads; h0 += 8) {
    float v[S][8];
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const int src = page_lane0 + ((h0 + h < a.kv_heads ? h0 + h : h0) << a.lpr_log2);
#pragma unroll
      for (int s = 0; s < S; ++s) v[s][h] = __shfl(t[s], src);
    }
#pragma unroll
    for (int h = 0; h < 8; ++h)
      if (h0 + h < a.kv_heads)
#pragma unroll
        for (int s = 0; s < S; ++s) total[s] = h0 + h == 0 ? v[s][h] : total[s] + v[s][h];
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int p0 = wave_first + s * ppw;
    if (within == 0 && page_local < ppw && p0 + page_local < count)
      a.scores[(int64_t)b * a.max_pages + p0 + page_local] = total[s] / (float)a.q_heads;
  }
}

// Page-mean score: sum_kh sum_d gq[kh,d] * summary[p,kh,d], with
// gq = (sum_g q[kh*G+g]) / G.
template <int E>
__global__ __launch_bounds__(kScoreThreads) void mean_score_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float smem[];
  float* gq = smem;                                   // [kv_heads * head_dim]
  float* hs = smem + a.kv_heads * a.head_dim;         // [waves][kv_heads]
  const int b = blockIdx.y;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int p_begin = blockIdx.x * kPagesPerBlock;
  if (p_begin >= count) return;
  const int group = a.q_heads / a.kv_heads;
  for (int i = threadIdx.x; i < a.kv_heads * a.head_dim; i += kScoreThreads) {
    int kh = i / a.head_dim, d = i - kh * a.head_dim;
    float s = load_elem(a.q, a.q_dtype, (int64_t)b * a.q_bs + (int64_t)(kh * group) * a.q_hs + d);
    for (int g = 1; g < group; ++g)
      s = s + load_elem(a.q, a.q_dtype, (int64_t)b * a.q_bs + (int64_t)(kh * group + g) * a.q_hs + d);
    gq[i] = s / (float)group;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = 1 << a.lpr_log2;
  const int heads_per_pass = kWave >> a.lpr_log2;
  const int sub = lane & (lpr - 1);
  const int64_t page_elems = (int64_t)a.kv_heads * a.head_dim;
  for (int it = 0; it < kPagesPerBlock / kScoreWaves; ++it) {
    const int p = p_begin + it * kScoreWaves + wave;
    const bool live = p < count;
    for (int kh0 = 0; kh0 < a.kv_heads; kh0 += heads_per_pass) {
      const int kh = kh0 + (lane >> a.lpr_log2);
      const bool data = live && kh < a.kv_heads && sub < a.lanes_used;
      float t = 0.f;
      if (data) {
        float sv[E];
        int64_t idx = (int64_t)b * a.b_bs + (int64_t)p * page_elems + (int64_t)kh * a.head_dim + sub * E;
        load_vec<F32, E>(a.lo, idx, sv);
        const float* g = gq + kh * a.head_dim + sub * E;
        t = g[0] * sv[0];
#pragma unroll
        for (int e = 1; e < E; ++e) t = t + g[e] * sv[e];
      }
      t = group_sum(t, lpr);
      if (live && kh < a.kv_heads && sub == 0) hs[wave * a.kv_heads + kh] = t;
    }
    __syncthreads();
    if (live && lane == 0) {
      float total = hs[wave * a.kv_heads];
      for (int kh = 1; kh < a.kv_heads; ++kh) total = total + hs[wave * a.kv_heads + kh];
      a.scores[(int64_t)b * a.max_pages + p] = total;
    }
    __syncthreads();
  }
}

__device__ __forceinline__ uint32_t order_key(float s) {
  if (s != s) return 0xfffffffeu;  // NaN ranks just below required pages
  uint32_t u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0u;  // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelectArgs {
  const float* scores;
  const int64_t* lengths;
  int64_t length;
  int page_size, max_pages, top_pages, keep_sink, mode;
  FastDiv page_div;
  int32_t* pages;
  int32_t* positions;
};

// THREADS = 1024 covers NHS_MAX_SELECT_PAGES; a 256-thread workgroup (4
// waves: cheaper barriers and histogram passes) covers up to 4096 pages.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void select_topk_kernel(SelectArgs a) {
  __shared__ int32_t chosen[NHS_MAX_SELECT_PAGES];
  __shared__ int32_t hist[256];
  __shared__ int32_t scan[THREADS / 64 + 1];
  __shared__ int32_t pick[2];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int64_t len = a.lengths ? a.lengths[b] : a.length;
  const int k = a.top_pages < count ? a.top_pages : count;
  const int per = (count + THREADS - 1) / THREADS;  // <= 16
  const int p0 = tid * per;

  bool sel[kMaxSelectPerThread];
#pragma unroll
  for (int q = 0; q < kMaxSelectPerThread; ++q) sel[q] = q < per && p0 + q < count;

  if (a.top_pages < count) {
    const float* sc = a.scores + (int64_t)b * a.max_pages;
    const bool second = a.mode == kModeQuest ? (a.keep_sink && a.top_pages > 1 && count > 1) : a.top_pages > 1;
    uint32_t key[kMaxSelectPerThread];
#pragma unroll
    for (int q = 0; q < kMaxSelectPerThread; ++q) {
      int p = p0 + q;
      key[q] = 0u;
      if (q < per && p < count)
        key[q] = (p == count - 1 || (second && p == 0)) ? 0xffffffffu : order_key(sc[p]);
    }
    uint32_t prefix = 0u, pmask = 0u;
    int need = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kMaxSelectPerThread; ++q)
        if (q < per && p0 + q < count && (key[q] & pmask) == prefix) atomicAdd(&hist[(key[q] >> shift) & 255u], 1);
      __syncthreads();
      if (tid < 64) {
        // lane l holds bins 255-4l .. 252-4l (descending digit order)
        int c[4], csum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c[i] = hist[255 - 4 * tid - i];
          csum += c[i];
        }
        int incl = csum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          int o = __shfl_up(incl, d);
          if (tid >= d) incl += o;
        }
        int before = incl - csum;
        if (before < need && incl >= need) {
          int cum = before;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (cum + c[i] >= need) {
              pick[0] = 255 - 4 * tid - i;
              pick[1] = need - cum;
              break;
            }
            cum += c[i];
          }
        }
      }
      __syncthreads();
      prefix |= (uint32_t)pick[0] << shift;
      pmask |= 255u << shift;
      need = pick[1];
      __syncthreads();
    }
    // prefix is the key of the k-th best page; `need` pages with that key
    // are taken, lowest page index first.
    int local_ties = 0;
#pragma unroll
    for (int q = 0; q < kMaxSelectPerThread; ++q) local_ties += sel[q] && key[q] == prefix;
    int total_ties;
    int tie_rank = block_exclusive_scan<int>(local_ties, scan, &total_ties);
#pragma unroll
    for (int q = 0; q < kMaxSelectPerThread; ++q) {
      if (!sel[q]) continue;
      if (key[q] == prefix) {
        sel[q] = tie_rank < need;
        ++tie_rank;
      } else {
        sel[q] = key[q] > prefix;
      }
    }
  }

  int local = 0;
#pragma unroll
  for (int q = 0; q < kMaxSelectPerThread; ++q) local += sel[q];
  int n_sel;
  int out = block_exclusive_scan<int>(local, scan, &n_sel);
#pragma unroll
  for (int q = 0; q < kMaxSelectPerThread; ++q)
    if (sel[q]) chosen[out++] = p0 + q;
  for (int i = n_sel + tid; i < a.top_pages; i += THREADS) chosen[i] = -1;
  __syncthreads();
  int32_t* pages = a.pages + (int64_t)b * a.top_pages;
  for (int i = tid; i < a.top_pages; i += THREADS) pages[i] = chosen[i];
  const int P = a.page_size;
  const int64_t n_pos = (int64_t)a.top_pages * P;
  int32_t* pos = a.positions + (int64_t)b * n_pos;
  for (int64_t i = tid; i < n_pos; i += THREADS) {
    uint32_t j = a.page_div.div((uint32_t)i);
    int32_t p = chosen[j];
    int64_t t = (int64_t)p * P + (int64_t)((uint32_t)i - j * (uint32_t)P);
    pos[i] = (p >= 0 && t < len) ? (int32_t)t : -1;
  }
}

// Up to kWave * KPL pages: the selection runs in one wave, with no LDS and no
// barrier until the output. Page q * kWave + lane sits in slot q of that lane.
// The key of the k-th best page, the largest x with at least top_pages keys
// >= x, is found bit by bit, most significant first: at each bit the wave
// counts the keys >= the prefix found so far with that bit set (a compare, a
// ballot and a popcount per slot) and keeps the bit when the count reaches
// top_pages. Every key above it is taken, ties at it go to the lowest pages,
// and the chosen pages come out in ascending order (ranks from mbcnt). The
// other waves join for the page -> token expansion.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <int KPL>
__global__ __launch_bounds__(kSelectWaveThreads) void select_wave_kernel(SelectArgs a) {
  __shared__ int32_t chosen[kWave * KPL];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int64_t len = a.lengths ? a.lengths[b] : a.length;
  if (tid < kWave) {
    const int lane = tid;
    // the score loads are issued before the page count arrives (pages past
    // max_pages read page 0; values past count are never used, and none are
    // when every page is kept)
    const float* sc = a.scores + (int64_t)b * a.max_pages;
    float sv[KPL];
#pragma unroll
    for (int q = 0; q < KPL; ++q) sv[q] = sc[q * kWave + lane < a.max_pages ? q * kWave + lane : 0];
    bool sel[KPL];
#pragma unroll
    for (int q = 0; q < KPL; ++q) sel[q] = q * kWave + lane < count;
    if (a.top_pages < count) {
      const bool second = a.mode == kModeQuest ? (a.keep_sink && a.top_pages > 1 && count > 1) : a.top_pages > 1;
      // pages past count keep key 0, below every score's key (>= 0x007fffff),
      // so no prefix tested below (it always has a bit set) matches them
      uint32_t key[KPL];
#pragma unroll
      for (int q = 0; q < KPL; ++q) {
        const int p = q * kWave + lane;
        key[q] = p >= count ? 0u : (p == count - 1 || (second && p == 0)) ? 0xffffffffu : order_key(sv[q]);
      }
      // prefix = the largest key x with at least top_pages keys >= x, i.e.
      // the key of the k-th best page
      uint32_t prefix = 0u;
#pragma unroll
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        int c = 0;
#pragma unroll
        for (int q = 0; q < KPL; ++q) c += __popcll(__ballot(key[q] >= cand));
        if (c >= a.top_pages) prefix = cand;
      }
      int above = 0;
#pragma unroll
      for (int q = 0; q < KPL; ++q) above += __popcll(__ballot(key[q] > prefix));
      // every page above that key is taken, then the first `need` pages with
      // that key in page order (slot, then lane)
      const int need = a.top_pages - above;
      int before = 0;
#pragma unroll
      for (int q = 0; q < KPL; ++q) {
        const bool tie = key[q] == prefix;
        const uint64_t m = __ballot(tie);
        sel[q] = key[q] > prefix || (tie && before + lanes_below(m) < need);
        before += __popcll(m);
      }
    }
    int n_sel = 0;
#pragma unroll
    for (int q = 0; q < KPL; ++q) {
      const uint64_t m = __ballot(sel[q]);
      if (sel[q]) chosen[n_sel + lanes_below(m)] = q * kWave + lane;
      n_sel += __popcll(m);
    }
    for (int i = n_sel + lane; i < a.top_pages; i += kWave) chosen[i] = -1;
  }
  __syncthreads();
  int32_t* pages = a.pages + (int64_t)b * a.top_pages;
  for (int i = tid; i < a.top_pages; i += kSelectWaveThreads) pages[i] = chosen[i];
  const int P = a.page_size;
  const int64_t n_pos = (int64_t)a.top_pages * P;
  int32_t* pos = a.positions + (int64_t)b * n_pos;
  if (P % 4 == 0 && (uintptr_t)a.positions % 16 == 0) {
    // four positions of one page per 16-byte store (n_pos is a multiple of 4)
    for (int64_t i = 4 * (int64_t)tid; i < n_pos; i += 4 * kSelectWaveThreads) {
      const uint32_t j = a.page_div.div((uint32_t)i);
      const int32_t p = chosen[j];
      const int64_t t = (int64_t)p * P + (int64_t)((uint32_t)i - j * (uint32_t)P);
      int4 v;
      v.x = (p >= 0 && t < len) ? (int32_t)t : -1;
      v.y = (p >= 0 && t + 1 < len) ? (int32_t)(t + 1) : -1;
      v.z = (p >= 0 && t + 2 < len) ? (int32_t)(t + 2) : -1;
      v.w = (p >= 0 && t + 3 < len) ? (int32_t)(t + 3) : -1;
      *reinterpret_cast<int4*>(pos + i) = v;
    }
  } else {
    for (int64_t i = tid; i < n_pos; i += kSelectWaveThreads) {
      const uint32_t j = a.page_div.div((uint32_t)i);
      const int32_t p = chosen[j];
      const int64_t t = (int64_t)p * P + (int64_t)((uint32_t)i - j * (uint32_t)P);
      pos[i] = (p >= 0 && t < len) ? (int32_t)t : -1;
    }
  }
}

static int check_select_common(const char* who, int32_t batch, const void* query, int q_dtype, int32_t q_heads,
                               int32_t kv_heads, int32_t head_dim, const int64_t* lengths, int64_t length,
                               int32_t page_size, int32_t max_pages, int32_t top_pages, float* scores,
                               int32_t* pages, int32_t* positions) {
  if (!query || !scores || !pages || !positions) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (!valid_dtype(q_dtype)) return fail(NHS_ERR_INVALID, "%s: bad query dtype", who);
  if (batch < 0 || q_heads < 1 || kv_heads < 1 || head_dim < 1 || page_size < 1 || max_pages < 1 ||
      top_pages < 1 || q_heads % kv_heads)
    return fail(NHS_ERR_INVALID, "%s: invalid shape or page budget", who);
  if (max_pages > NHS_MAX_SELECT_PAGES || top_pages > NHS_MAX_SELECT_PAGES)
    return fail(NHS_ERR_UNSUPPORTED, "%s: at most %d pages", who, NHS_MAX_SELECT_PAGES);
  if ((int64_t)top_pages * page_size >= (1ll << 31))
    return fail(NHS_ERR_UNSUPPORTED, "%s: top_pages * page_size must be < 2^31", who);
  if (!lengths && (length < 0 || length >= (1ll << 31)))
    return fail(NHS_ERR_INVALID, "%s: length must be in [0, 2^31)", who);
  return NHS_OK;
}

// Chunking of a bound row (head_dim elements of `esize` bytes) into lanes:
// 16-byte chunks when the row is a multiple of 16 bytes, else one element
// per lane (head_dim <= 64). Returns elements per lane, or 0 if unsupported.
static int chunk_elems(int head_dim, int esize) {
  if ((head_dim * esize) % 16 == 0 && head_dim * esize / 16 <= 64) return 16 / esize;
  if (head_dim <= 64) return 1;
  return 0;
}

// Quest cuts a bound row into 32-byte chunks when it is a multiple of 32
// bytes of at most 64 chunks, else as chunk_elems() does.
static int quest_chunk_elems(int head_dim, int esize) {
  if ((head_dim * esize) % 32 == 0 && head_dim * esize / 32 <= 64) return 32 / esize;
  return chunk_elems(head_dim, esize);
}

static int launch_select(const SelectArgs& s, int batch, hipStream_t stream, const char* who, hipEvent_t start,
                         hipEvent_t stop) {
  const int wave_pages = s.max_pages > s.top_pages ? s.max_pages : s.top_pages;
  if (wave_pages <= kWave * 8)
    launch(select_wave_kernel<8>, dim3((unsigned)batch), dim3(kSelectWaveThreads), 0, stream, start, stop, s);
  else if (wave_pages <= kWave * 16)
    launch(select_wave_kernel<16>, dim3((unsigned)batch), dim3(kSelectWaveThreads), 0, stream, start, stop, s);
  else if (s.max_pages <= 256 * kMaxSelectPerThread)
    launch(select_topk_kernel<256>, dim3((unsigned)batch), dim3(256), 0, stream, start, stop, s);
  else
    launch(select_topk_kernel<kSelectThreads>, dim3((unsigned)batch), dim3(kSelectThreads), 0, stream, start, stop, s);
  return launch_status(who);
}

}  // namespace nhs

namespace nhs {

// nhs_quest_select and nhs_quest_select_items: strided bounds (minimum,
// maximum, bounds_batch_stride) or per-item bounds (items).
static int quest_select(const char* who, int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                        int64_t q_head_stride, const void* minimum, const void* maximum, int64_t bounds_batch_stride,
                        const nhs_layer_item* items, int32_t bounds_dtype, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, const int64_t* lengths, int64_t length, int32_t page_size,
                        int32_t max_pages, int32_t top_pages, int32_t keep_sink, float* scores, int32_t* pages,
                        int32_t* positions, void* stream) {
  LaunchEvents ev = take_launch_events();
  int st = check_select_common(who, batch, query, q_dtype, q_heads, kv_heads, head_dim, lengths, length, page_size,
                               max_pages, top_pages, scores, pages, positions);
  if (st != NHS_OK) return st;
  if (items ? !lengths : (!minimum || !maximum)) return fail(NHS_ERR_INVALID, "%s: null bounds", who);
  if (!valid_dtype(bounds_dtype)) return fail(NHS_ERR_INVALID, "%s: bad bounds dtype", who);
  if ((int64_t)q_heads * head_dim + 8 * q_heads > 16384)
    return fail(NHS_ERR_UNSUPPORTED, "%s: q_heads * head_dim too large", who);
  const int esize = elem_size(bounds_dtype);
  const int E = quest_chunk_elems(head_dim, esize);
  if (E == 0) return fail(NHS_ERR_UNSUPPORTED, "%s: head_dim %d unsupported", who, head_dim);
  if (!items && E > 1 && (((uintptr_t)minimum | (uintptr_t)maximum) % 16 || (bounds_batch_stride * esize) % 16))
    return fail(NHS_ERR_INVALID, "%s: bounds must be 16-byte aligned", who);
  if (batch == 0) return NHS_OK;
  hipStream_t s = (hipStream_t)stream;
  ScoreArgs a{};
  a.q = query;
  a.q_dtype = q_dtype;
  {
    const int qes = elem_size(q_dtype);
    a.q_vec = (E * qes) % 16 == 0 && (uintptr_t)query % 16 == 0 && (q_head_stride * qes) % 16 == 0 &&
              (q_batch_stride * qes) % 16 == 0;
  }
  a.q_bs = q_batch_stride;
  a.q_hs = q_head_stride;
  a.lo = minimum;
  a.hi = maximum;
  a.b_bs = bounds_batch_stride;
  a.items = items;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.lanes_used = head_dim / E;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.lengths = lengths;
  a.length = length;
  a.page_size = page_size;
  a.max_pages = max_pages;
  a.scores = scores;
  a.group = q_heads / kv_heads;
  const int lanes_per_page = kv_heads << a.lpr_log2;
  if (a.group > 8 || lanes_per_page > kQuestThreads)
    return fail(NHS_ERR_UNSUPPORTED, "%s: needs q_heads/kv_heads <= 8 and kv_heads * lanes per head <= %d", who,
                kQuestThreads);
  const int G = a.group == 1 ? 1 : a.group == 2 ? 2 : a.group <= 4 ? 4 : 8;
  void (*kernel)(ScoreArgs) = nullptr;
  dim3 grid, block;
  size_t lds = 0;
  const int ppw = lanes_per_page <= kWave ? kWave / lanes_per_page : 0;
  if (E * esize == 32 && ppw > 0) {
    // a page fits one wave: the page kernel
    a.pages_per_step = ppw;
    a.pages_per_block = kPageWaves * page_slots(a.group) * ppw;
    grid = dim3((unsigned)((max_pages + a.pages_per_block - 1) / a.pages_per_block), (unsigned)batch);
    block = dim3(kPageThreads);
    switch (bounds_dtype * 16 + a.group) {  // instantiated for every group size: no masked heads
#define NHS_PAGE_CASE(DT, TY, EE, GG) \
  case DT * 16 + GG: kernel = quest_page_kernel<TY, EE, GG>; break;
#define NHS_PAGE_GS(DT, TY, EE)                                                                         \
  NHS_PAGE_CASE(DT, TY, EE, 1) NHS_PAGE_CASE(DT, TY, EE, 2) NHS_PAGE_CASE(DT, TY, EE, 3) NHS_PAGE_CASE(DT, TY, EE, 4) \
  NHS_PAGE_CASE(DT, TY, EE, 5) NHS_PAGE_CASE(DT, TY, EE, 6) NHS_PAGE_CASE(DT, TY, EE, 7) NHS_PAGE_CASE(DT, TY, EE, 8)
      NHS_PAGE_GS(NHS_F32, F32, 8)
      NHS_PAGE_GS(NHS_F16, F16, 16)
      NHS_PAGE_GS(NHS_BF16, BF16, 16)
#undef NHS_PAGE_GS
#undef NHS_PAGE_CASE
    }
  } else {
    const int threads = lanes_per_page >= 256 ? ((lanes_per_page + 63) / 64) * 64 : 256;
    a.pages_per_step = threads / lanes_per_page;
    a.pages_per_block = a.pages_per_step * ((kPagesPerBlock + a.pages_per_step - 1) / a.pages_per_step);
    grid = dim3((unsigned)((max_pages + a.pages_per_block - 1) / a.pages_per_block), (unsigned)batch);
    block = dim3(threads);
    lds = ((size_t)q_heads * head_dim + (size_t)a.pages_per_step * kv_heads) * sizeof(float);
    switch (bounds_dtype * 1024 + E * 16 + G) {
#define NHS_QUEST_CASE(DT, TY, EE, GG) \
  case DT * 1024 + EE * 16 + GG: kernel = quest_score_kernel<TY, EE, GG>; break;
#define NHS_QUEST_GS(DT, TY, EE) \
  NHS_QUEST_CASE(DT, TY, EE, 1) NHS_QUEST_CASE(DT, TY, EE, 2) NHS_QUEST_CASE(DT, TY, EE, 4) NHS_QUEST_CASE(DT, TY, EE, 8)
      NHS_QUEST_GS(NHS_F32, F32, 8)
      NHS_QUEST_GS(NHS_F32, F32, 4)
      NHS_QUEST_GS(NHS_F32, F32, 1)
      NHS_QUEST_GS(NHS_F16, F16, 16)
      NHS_QUEST_GS(NHS_F16, F16, 8)
      NHS_QUEST_GS(NHS_F16, F16, 1)
      NHS_QUEST_GS(NHS_BF16, BF16, 16)
      NHS_QUEST_GS(NHS_BF16, BF16, 8)
      NHS_QUEST_GS(NHS_BF16, BF16, 1)
#undef NHS_QUEST_GS
#undef NHS_QUEST_CASE
    }
  }
  if (top_pages < max_pages) {  // scores are not needed when every page is kept
    if (!kernel) return fail(NHS_ERR_UNSUPPORTED, "%s: no scoring kernel", who);
    launch(kernel, grid, block, lds, s, ev.start, nullptr, a);
    ev.start = nullptr;  // the start event belongs to the first kernel
    st = launch_status(who);
    if (st != NHS_OK) return st;
  }
  SelectArgs sa;
  sa.scores = scores;
  sa.lengths = lengths;
  sa.length = length;
  sa.page_size = page_size;
  sa.max_pages = max_pages;
  sa.top_pages = top_pages;
  sa.keep_sink = keep_sink;
  sa.mode = kModeQuest;
  sa.page_div = FastDiv((uint32_t)page_size);
  sa.pages = pages;
  sa.positions = positions;
  return launch_select(sa, batch, s, who, ev.start, ev.stop);
}

}  // namespace nhs

extern "C" int nhs_quest_select(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                                int64_t q_head_stride, const void* minimum, const void* maximum,
                                int32_t bounds_dtype, int64_t bounds_batch_stride, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, const int64_t* lengths, int64_t length, int32_t page_size,
                                int32_t max_pages, int32_t top_pages, int32_t keep_sink, float* scores,
                                int32_t* pages, int32_t* positions, void* stream) {
  return nhs::quest_select("nhs_quest_select", batch, query, q_dtype, q_batch_stride, q_head_stride, minimum, maximum,
                           bounds_batch_stride, nullptr, bounds_dtype, q_heads, kv_heads, head_dim, lengths, length,
                           page_size, max_pages, top_pages, keep_sink, scores, pages, positions, stream);
}

extern "C" int nhs_quest_select_items(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                                      int64_t q_head_stride, const nhs_layer_item* items, int32_t bounds_dtype,
                                      int32_t q_heads, int32_t kv_heads, int32_t head_dim, const int64_t* lengths,
                                      int32_t page_size, int32_t max_pages, int32_t top_pages, int32_t keep_sink,
                                      float* scores, int32_t* pages, int32_t* positions, void* stream) {
  if (!items) return nhs::fail(NHS_ERR_INVALID, "nhs_quest_select_items: null items");
  return nhs::quest_select("nhs_quest_select_items", batch, query, q_dtype, q_batch_stride, q_head_stride, nullptr,
                           nullptr, 0, items, bounds_dtype, q_heads, kv_heads, head_dim, lengths, 0, page_size,
                           max_pages, top_pages, keep_sink, scores, pages, positions, stream);
}

extern "C" int nhs_mean_select(int32_t batch, const void* query, int32_t q_dtype, int64_t q_batch_stride,
                               int64_t q_head_stride, const float* summaries, int64_t summaries_batch_stride,
                               int32_t q_heads, int32_t kv_heads, int32_t head_dim, const int64_t* lengths,
                               int64_t length, int32_t page_size, int32_t max_pages, int32_t top_pages, float* scores,
                               int32_t* pages, int32_t* positions, void* stream) {
  using namespace nhs;
  LaunchEvents ev = take_launch_events();
  const char* who = "nhs_mean_select";
  int st = check_select_common(who, batch, query, q_dtype, q_heads, kv_heads, head_dim, lengths, length, page_size,
                               max_pages, top_pages, scores, pages, positions);
  if (st != NHS_OK) return st;
  if (!summaries) return fail(NHS_ERR_INVALID, "%s: null summaries", who);
  if ((int64_t)kv_heads * head_dim + 4 * kv_heads > 16384)
    return fail(NHS_ERR_UNSUPPORTED, "%s: kv_heads * head_dim too large", who);
  const int E = chunk_elems(head_dim, 4);
  if (E == 0) return fail(NHS_ERR_UNSUPPORTED, "%s: head_dim %d unsupported", who, head_dim);
  if (E > 1 && (uintptr_t)summaries % 16) return fail(NHS_ERR_INVALID, "%s: summaries must be 16-byte aligned", who);
  if (batch == 0) return NHS_OK;
  hipStream_t s = (hipStream_t)stream;
  ScoreArgs a{};
  a.q = query;
  a.q_dtype = q_dtype;
  a.q_bs = q_batch_stride;
  a.q_hs = q_head_stride;
  a.lo = summaries;
  a.hi = nullptr;
  a.b_bs = summaries_batch_stride;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.lanes_used = head_dim / E;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.lengths = lengths;
  a.length = length;
  a.page_size = page_size;
  a.max_pages = max_pages;
  a.scores = scores;
  dim3 grid((unsigned)((max_pages + kPagesPerBlock - 1) / kPagesPerBlock), (unsigned)batch);
  size_t lds = ((size_t)kv_heads * head_dim + (size_t)kScoreWaves * kv_heads) * sizeof(float);
  if (top_pages < max_pages) {
    if (E == 4)
      launch(mean_score_kernel<4>, grid, dim3(kScoreThreads), lds, s, ev.start, nullptr, a);
    else
      launch(mean_score_kernel<1>, grid, dim3(kScoreThreads), lds, s, ev.start, nullptr, a);
    ev.start = nullptr;
    st = launch_status(who);
    if (st != NHS_OK) return st;
  }
  SelectArgs sa;
  sa.scores = scores;
  sa.lengths = lengths;
  sa.length = length;
  sa.page_size = page_size;
  sa.max_pages = max_pages;
  sa.top_pages = top_pages;
  sa.keep_sink = 1;
  sa.mode = kModeMean;
  sa.page_div = FastDiv((uint32_t)page_size);
  sa.pages = pages;
  sa.positions = positions;
  return launch_select(sa, batch, s, who, ev.start, ev.stop);
}
