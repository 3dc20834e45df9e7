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

#include "select_common.h"

#pragma clang fp contract(off)

namespace nhs {

constexpr int kScoreThreads = 256;
constexpr int kScoreWaves = kScoreThreads / kWave;
constexpr int kPagesPerBlock = 8;
constexpr int kQuestThreads = 512;
constexpr int kSelectThreads = 1024;
constexpr int kMaxSelectPerThread = NHS_MAX_SELECT_PAGES / kSelectThreads;  // 16
constexpr int kSelectWaveThreads = 256;  // one-wave selection; 4 waves expand the positions
// The general Quest kernel's folded query (2 floats and a byte per (KV
// head, d)) and KV-head sums fit the 160 KiB of LDS a workgroup may use.
constexpr size_t kMaxQuestLds = 160 * 1024;
constexpr int kMaxQuestFold = 16384;  // kv_heads * head_dim, for the message

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
  int elems;           // elements per lane chunk (the last chunk of a row may be shorter)
  int heads_per_pass;  // general Quest kernel: KV heads scored together
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

// Quest bounds score: (sum_h sum_d torch.maximum(q*lo, q*hi)) / q_heads.
//
// With a = the smaller and b = the larger bound of an element (a = hi and
// b = lo when hi < lo), the heads of one KV head's GQA group contribute q*b
// where q > 0 and q*a elsewhere, so per (KV head, d) the group's terms are
//   a[d] * Qneg[d] + b[d] * Qpos[d]
// with Qpos / Qneg the group's positive / non-positive query sums (added in
// head order from 0.0, once per request). A lane keeps them for its chunk
// and scores a page with two fmas per element, t = fma(a', Qneg, t) then
// t = fma(b', Qpos, t), where a' (b') is 0 when no head of the group is
// non-positive (positive) at d. Chunk sums are added as a pairwise tree
// over a KV head's lanes, the KV-head sums sequentially; the CPU oracle sums
// in this order.
//
// Special values follow torch.maximum, which is NaN when either product is:
// a chunk sums to NaN when it holds a NaN bound, a bound of +-inf at a d
// where a head's query is +-0, or a bound of +-0 at a d where a head's query
// is +-inf (0 * inf). NaN scores are stored as the quiet NaN 0x7fc00000.
//
// Side bits of a (KV head, d): a head of the group is > 0, is not > 0, is
// +-0, is +-inf.
enum : uint32_t { kSidePos = 1u, kSideNeg = 2u, kSideZero = 4u, kSideInf = 8u };

__device__ __forceinline__ void fold_query(float q, float& p, float& n, uint32_t& side) {
  // branch-free: a query value adds +0.0 to the other side's sum, which
  // leaves it unchanged (the positive sum starts at +0.0 and only grows, the
  // non-positive one starts at +0.0 and never becomes -0.0)
  const bool up = q > 0.f;
  p = p + (up ? q : 0.f);
  n = n + (up ? 0.f : q);
  side |= (up ? kSidePos : kSideNeg) | (q == 0.f ? kSideZero : 0u) | (__builtin_isinf(q) ? kSideInf : 0u);
}

__device__ __forceinline__ float quest_fma2(float x, float lo, float hi, float pos, float neg, bool use_pos,
                                            bool use_neg) {
  const bool sw = hi < lo;
  const float a = sw ? hi : lo, b = sw ? lo : hi;
  x = __builtin_fmaf(use_neg ? a : 0.f, neg, x);
  return __builtin_fmaf(use_pos ? b : 0.f, pos, x);
}

// 0 * inf inside one of the products of an element whose group holds a zero
// or an infinite query
__device__ __forceinline__ bool zero_inf_product(float lo, float hi, bool zero_q, bool inf_q) {
  return (zero_q && (__builtin_isinf(lo) || __builtin_isinf(hi))) || (inf_q && (lo == 0.f || hi == 0.f));
}

__device__ __forceinline__ float canonical_score(float s) { return s != s ? __uint_as_float(0x7fc00000u) : s; }

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

// Nonzero when a packed word of T holds a NaN. For 16-bit types both halves
// at once: |x| + (0x8000 - the smallest NaN magnitude) reaches bit 15 exactly
// for a NaN, and no half carries into the other.
template <typename T>
__device__ __forceinline__ uint32_t nan_bits(uint32_t w) {
  if constexpr (T::bytes == 4) {
    return (w & 0x7fffffffu) > 0x7f800000u ? 1u : 0u;
  } else {
    constexpr uint32_t add = T::dtype == NHS_BF16 ? 0x007f007fu : 0x03ff03ffu;
    return ((w & 0x7fff7fffu) + add) & 0x80008000u;
  }
}

// For a lane whose query chunk has zero / infinite elements (masks zero_m,
// inf_m): whether one 32-bit word of a page's lower and upper bounds
// (elements e0 .. e0 + 4 / T::bytes - 1, packed in T) meets them in 0 * inf,
// as zero_inf_product() per element, on the packed bits: a +-inf or +-0
// bound element against a zero_m or inf_m bit.
template <typename T>
__device__ __forceinline__ uint32_t zero_inf_word(uint32_t zero_m, uint32_t inf_m, uint32_t lo_w, uint32_t hi_w,
                                                  int e0) {
  constexpr int per = 4 / T::bytes;  // elements per word
  constexpr uint32_t kMag = T::bytes == 4 ? 0x7fffffffu : 0x7fffu;
  constexpr uint32_t kInf = T::bytes == 4 ? 0x7f800000u : T::dtype == NHS_BF16 ? 0x7f80u : 0x7c00u;
  uint32_t bad = 0u;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    const uint32_t l = (lo_w >> (16 * i)) & kMag, h = (hi_w >> (16 * i)) & kMag;
    const uint32_t zq = (zero_m >> (e0 + i)) & 1u, iq = (inf_m >> (e0 + i)) & 1u;
    bad |= ((zq && (l == kInf || h == kInf)) || (iq && (l == 0u || h == 0u))) ? 1u : 0u;
  }
  return bad;
}

// The per-lane grouped sums of E elements. pos[e] adds the group's query
// values > 0 and neg[e] the others (NaN included), in head order from +0.0;
// a side with no contributor stays +0.0 and neither sum is ever -0.0. The
// fold uses the NaN-propagating maximum / minimum: maximum(q, 0) is q > 0 ?
// q : +0 and minimum(q, 0) is q > 0 ? +0 : q, except that a NaN q makes
// both sums NaN (the chunk is NaN either way).
//
// Which heads contribute is recovered from the sums where it matters: a head
// of the group is > 0 at e iff pos[e] > 0, and one is < 0 or NaN iff
// !(neg[e] >= 0). A side holding only +-0 queries sums to +0 and reads as
// no contributor; it can only change the chunk against an infinite bound,
// where the 0 * inf test makes the chunk NaN anyway.
template <int E, int G>
struct GroupedQuery {
  float pos[E], neg[E];
  static __device__ __forceinline__ void add(float q, float& p, float& n) {
    p = p + __builtin_elementwise_maximum(q, 0.f);
    n = n + __builtin_elementwise_minimum(q, 0.f);
  }
  __device__ __forceinline__ void clear_if_idle(bool live) {
    // padding lanes add exactly +0 against finite bounds
    if (!live) {
#pragma unroll
      for (int e = 0; e < E; ++e) pos[e] = neg[e] = 0.f;
    }
  }
  // Folds EF elements of the lane's query slices into pos / neg[0 .. EF)
  // (heads >= group are ignored).
  template <int EF>
  __device__ __forceinline__ void fold(const float (&qv)[G][EF], int group) {
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < EF; ++e) {
      float p = 0.f, n = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (g < group) add(qv[g][e], p, n);
      pos[e] = p, neg[e] = n;
    }
  }
  // fold() from the heads' slices kept packed in T (widened element by
  // element; all G heads are in the group)
  template <typename T, int EF>
  __device__ __forceinline__ void fold_packed(const uint32_t (&qw)[G][EF * T::bytes / 4]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < EF; ++e) {
      float p = 0.f, n = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) add(packed_elem<T, EF>(qw[g], e), p, n);
      pos[e] = p, neg[e] = n;
    }
  }
  // For a wave whose lanes l and l + 32 hold the same query chunk: lane l
  // folded its first E / 2 elements and lane l + 32 the other E / 2 into
  // pos / neg[0 .. E / 2). v_permlane32_swap of a register with itself
  // gives every lane the lower half-wave's value and the upper one's.
  __device__ __forceinline__ void join_halves() {
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(pos[e]), __float_as_uint(pos[e]), false, false);
      const auto n = __builtin_amdgcn_permlane32_swap(__float_as_uint(neg[e]), __float_as_uint(neg[e]), false, false);
      pos[e] = __uint_as_float(p[0]), pos[E / 2 + e] = __uint_as_float(p[1]);
      neg[e] = __uint_as_float(n[0]), neg[E / 2 + e] = __uint_as_float(n[1]);
    }
  }
  // The chunk sum for one page's bounds kept packed in T, every bound
  // multiplied: t = fma(lo, neg, t), t = fma(hi, pos, t). Against finite,
  // ordered bounds (lo <= hi) and finite sums it equals chunk_exact() bit
  // for bit: an unused bound meets a +0 sum and adds +-0, which leaves t
  // unchanged since t is never -0. Any infinite or NaN bound or sum makes it
  // non-finite (inf * a nonzero sum is inf, inf * +0 is NaN). inverted is
  // set when some hi < lo.
  template <typename T>
  __device__ __forceinline__ float chunk_fast(const uint32_t (&mn)[E * T::bytes / 4],
                                              const uint32_t (&mx)[E * T::bytes / 4], bool& inverted) const {
    float x = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float lo = packed_elem<T, E>(mn, e), hi = packed_elem<T, E>(mx, e);
      inverted |= hi < lo;
      x = __builtin_fmaf(lo, neg[e], x);
      x = __builtin_fmaf(hi, pos[e], x);
    }
    return x;
  }
  // The chunk sum with the reference's semantics before its NaN and 0 * inf
  // tests: bounds ordered (a = hi, b = lo when hi < lo), t = fma(a', neg, t)
  // then t = fma(b', pos, t), where a' (b') is 0 when no head of the group
  // is < 0 or NaN (> 0) at e.
  template <typename T>
  __device__ __forceinline__ float chunk_exact(const uint32_t (&mn)[E * T::bytes / 4],
                                               const uint32_t (&mx)[E * T::bytes / 4]) const {
    float x = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e)
      x = quest_fma2(x, packed_elem<T, E>(mn, e), packed_elem<T, E>(mx, e), pos[e], neg[e], pos[e] > 0.f,
                     !(neg[e] >= 0.f));
    return x;
  }
  // Nonzero when the chunk of one page's bounds holds a NaN (integer tests
  // on the packed bits).
  template <typename T>
  __device__ __forceinline__ uint32_t nan_bound(const uint32_t (&mn)[E * T::bytes / 4],
                                                const uint32_t (&mx)[E * T::bytes / 4]) const {
    constexpr int W = E * T::bytes / 4;
    uint32_t bad = 0u;
#pragma unroll
    for (int w = 0; w < W; ++w) bad |= nan_bits<T>(mn[w]) | nan_bits<T>(mx[w]);
    return bad;
  }
};
//
// General kernel, for any group size, head_dim and KV head count: the
// workgroup folds the query once into LDS (Qpos, Qneg and the side bits of
// every (KV head, d), the heads of a group added in order), then lanes laid
// out as (page of the step, KV head, chunk) score pages. A chunk is E
// elements (E = 0: a.elems elements read one by one, the last chunk of a
// row shorter). When a page needs more lanes than the workgroup has, its KV
// heads are taken in passes. Each lane's chunk sum, the DPP tree over a KV
// head's lanes and the sequential KV-head sum follow the page kernel's order.
template <typename T, int E>
__global__ __launch_bounds__(kQuestThreads) void quest_score_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float smem[];
  const int kvd = a.kv_heads * a.head_dim;
  float* fpos = smem;                                           // [kv_heads * head_dim]
  float* fneg = smem + kvd;                                     // [kv_heads * head_dim]
  float* hs = smem + 2 * kvd;                                   // [pages_per_step][kv_heads]
  uint8_t* fside = reinterpret_cast<uint8_t*>(hs + a.pages_per_step * a.kv_heads);  // [kv_heads * head_dim]
  const int b = blockIdx.y;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int p_begin = blockIdx.x * a.pages_per_block;
  if (p_begin >= count) return;
  const int p_end = min(count, p_begin + a.pages_per_block);
  for (int i = threadIdx.x; i < kvd; i += blockDim.x) {
    const int kh = i / a.head_dim, d = i - kh * a.head_dim;
    float p = 0.f, n = 0.f;
    uint32_t side = 0u;
    for (int g = 0; g < a.group; ++g)
      fold_query(load_elem(a.q, a.q_dtype, (int64_t)b * a.q_bs + (int64_t)(kh * a.group + g) * a.q_hs + d), p, n,
                 side);
    fpos[i] = p, fneg[i] = n, fside[i] = (uint8_t)side;
  }
  __syncthreads();
  const int ne = E > 0 ? E : a.elems;
  const int lpr = 1 << a.lpr_log2;
  const int heads_per_pass = a.heads_per_pass;
  const int lanes_per_page = heads_per_pass << a.lpr_log2;
  const int page_local = threadIdx.x / lanes_per_page;
  const int within = threadIdx.x - page_local * lanes_per_page;
  const int kh_local = within >> a.lpr_log2;
  const int sub = within & (lpr - 1);
  const bool active = page_local < a.pages_per_step;
  const char *lo, *hi;
  bounds_of<T>(a, b, lo, hi);
  const int64_t page_elems = (int64_t)kvd;
  for (int base = p_begin; base < p_end; base += a.pages_per_step) {
    const int p = base + page_local;
    for (int kh0 = 0; kh0 < a.kv_heads; kh0 += heads_per_pass) {
      const int kh = kh0 + kh_local;
      const bool data = active && p < p_end && kh < a.kv_heads && sub < a.lanes_used;
      float x = 0.f;
      if (data) {
        const int d0 = sub * ne;
        const int d1 = min(d0 + ne, a.head_dim);
        const int64_t off = (int64_t)p * page_elems + (int64_t)kh * a.head_dim;
        bool bad = false;
        if constexpr (E > 0) {
          float mn[E], mx[E];
          load_vec<T, E>(lo, off + d0, mn);
          load_vec<T, E>(hi, off + d0, mx);
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const int i = kh * a.head_dim + d0 + e;
            const uint32_t side = fside[i];
            x = quest_fma2(x, mn[e], mx[e], fpos[i], fneg[i], side & kSidePos, side & kSideNeg);
            bad |= mn[e] != mn[e] || mx[e] != mx[e] || zero_inf_product(mn[e], mx[e], side & kSideZero, side & kSideInf);
          }
        } else {
          for (int d = d0; d < d1; ++d) {
            const int i = kh * a.head_dim + d;
            const uint32_t side = fside[i];
            const float l = load_elem(lo, T::dtype, off + d), h = load_elem(hi, T::dtype, off + d);
            x = quest_fma2(x, l, h, fpos[i], fneg[i], side & kSidePos, side & kSideNeg);
            bad |= l != l || h != h || zero_inf_product(l, h, side & kSideZero, side & kSideInf);
          }
        }
        if (bad) x = __uint_as_float(0x7fc00000u);
      }
      const float t = group_sum(x, lpr);
      if (data && sub == 0) hs[page_local * a.kv_heads + kh] = t;
    }
    __syncthreads();
    if ((int)threadIdx.x < a.pages_per_step && base + (int)threadIdx.x < p_end) {
      const float* row = hs + threadIdx.x * a.kv_heads;
      float total = row[0];
      for (int h = 1; h < a.kv_heads; ++h) total = total + row[h];
      a.scores[(int64_t)b * a.max_pages + base + threadIdx.x] = canonical_score(total / (float)a.q_heads);
    }
    __syncthreads();
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

template <typename T, int E, int G, bool SPLIT>
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
  // SPLIT (a page takes 32 lanes, so lanes l and l + 32 hold the same query
  // chunk): a lane folds half of its chunk, lanes 32..63 the second half,
  // and the halves are joined across the wave.
  constexpr int EF = SPLIT ? E / 2 : E;  // elements folded per lane
  constexpr int WF = EF * T::bytes / 4;
  const int fold_off = SPLIT ? (lane >> 5) * EF : 0;
  int64_t qi[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qi[g] = (int64_t)b * a.q_bs + (data ? (int64_t)(kh * G + g) * a.q_hs + sub * E + fold_off : 0);
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
    uint32_t qw[G][WF];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4* qp = reinterpret_cast<const uint4*>(static_cast<const char*>(a.q) + qi[g] * T::bytes);
#pragma unroll
      for (int v = 0; v < WF / 4; ++v) {
        const uint4 x = qp[v];
        qw[g][4 * v] = x.x, qw[g][4 * v + 1] = x.y, qw[g][4 * v + 2] = x.z, qw[g][4 * v + 3] = x.w;
      }
    }
    load_bounds();
    gq.template fold_packed<T, EF>(qw);
  } else {
    float qv[G][EF];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EF; ++e) qv[g][e] = load_elem(a.q, a.q_dtype, qi[g] + (data ? e : 0));
    load_bounds();
    gq.template fold<EF>(qv, G);
  }
  if constexpr (SPLIT) gq.join_halves();
  gq.clear_if_idle(data);
  const int lpr = 1 << a.lpr_log2;
  const int page_lane0 = page_local * lanes_per_page;
  // every slot is scored first (slots past count hold a live page's bounds
  // and are not stored), then the KV-head sums of all slots are formed
  // together: each group of 8 heads issues its lane reads for every slot
  // before the adds, which stay sequential in head order.
  float t[S], total[S];
  uint32_t slow = 0u;  // bit s: slot s needs the exact chunk sum
#pragma unroll
  for (int s = 0; s < S; ++s) {
    bool inverted = false;
    t[s] = gq.template chunk_fast<T>(mn[s], mx[s], inverted);
    slow |= (!__builtin_isfinite(t[s]) || inverted ? 1u : 0u) << s;
  }
  // A lane whose fast chunk sum is not finite, or whose bounds are inverted,
  // recomputes it exactly; only infinite or NaN bounds or query values,
  // inverted bounds or an overflow lead here. The chunk is NaN when a bound
  // is NaN, or when a bound meets a zero or infinite query element in
  // 0 * inf. The bounds and the query's zero / infinite elements are re-read
  // from memory, so this path holds no registers through the fast one.
  if (slow) {
    uint32_t zero_m = 0u, inf_m = 0u;  // bit e: a head of the group is +-0 (+-inf) at element e
    if (data) {
#pragma unroll 1
      for (int g = 0; g < G; ++g) {
        const int64_t q0 = (int64_t)b * a.q_bs + (int64_t)(kh * G + g) * a.q_hs + sub * E;
#pragma unroll 4
        for (int e = 0; e < E; ++e) {
          const float q = load_elem(a.q, a.q_dtype, q0 + e);
          zero_m |= (q == 0.f ? 1u : 0u) << e;
          inf_m |= (__builtin_isinf(q) ? 1u : 0u) << e;
        }
      }
    }
#pragma unroll 1
    for (int s = 0; s < S; ++s) {
      if (!((slow >> s) & 1u)) continue;
      const int p = wave_first + s * ppw + page_local;
      const int64_t at = ((int64_t)(p < count ? p : wave_first) * page_elems + lane_off) * T::bytes;
      const uint4* lp = reinterpret_cast<const uint4*>(lo + at);
      const uint4* hp = reinterpret_cast<const uint4*>(hi + at);
      uint32_t lw[W], hw[W];
#pragma unroll
      for (int v = 0; v < W / 4; ++v) {
        const uint4 x = lp[v], y = hp[v];
        lw[4 * v] = x.x, lw[4 * v + 1] = x.y, lw[4 * v + 2] = x.z, lw[4 * v + 3] = x.w;
        hw[4 * v] = y.x, hw[4 * v + 1] = y.y, hw[4 * v + 2] = y.z, hw[4 * v + 3] = y.w;
      }
      float x = gq.template chunk_exact<T>(lw, hw);
      uint32_t bad = gq.template nan_bound<T>(lw, hw);
#pragma unroll
      for (int w = 0; w < W; ++w) bad |= zero_inf_word<T>(zero_m, inf_m, lw[w], hw[w], w * (4 / T::bytes));
      if (bad) x = __uint_as_float(0x7fc00000u);
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2)
        if (s2 == s) t[s2] = x;
    }
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    t[s] = group_sum(t[s], lpr);
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
      a.scores[(int64_t)b * a.max_pages + p0 + page_local] = canonical_score(total[s] / (float)a.q_heads);
  }
}

// Page-mean score: sum_kh sum_d gq[kh,d] * summary[p,kh,d], with
// gq = (sum_g q[kh*G+g]) / G. E = 0: a.elems elements per lane, read one by
// one (the last chunk of a row shorter).
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
        const int ne = E > 0 ? E : a.elems;
        const int64_t idx = (int64_t)b * a.b_bs + (int64_t)p * page_elems + (int64_t)kh * a.head_dim + sub * ne;
        const float* g = gq + kh * a.head_dim + sub * ne;
        if constexpr (E > 0) {
          float sv[E];
          load_vec<F32, E>(a.lo, idx, sv);
          t = g[0] * sv[0];
#pragma unroll
          for (int e = 1; e < E; ++e) t = t + g[e] * sv[e];
        } else {
          const float* sv = static_cast<const float*>(a.lo) + idx;
          const int n = min(ne, a.head_dim - sub * ne);
          t = g[0] * sv[0];
          for (int e = 1; e < n; ++e) t = t + g[e] * sv[e];
        }
      }
      t = group_sum(t, lpr);
      if (live && kh < a.kv_heads && sub == 0) hs[wave * a.kv_heads + kh] = t;
    }
    __syncthreads();
    if (live && lane == 0) {
      float total = hs[wave * a.kv_heads];
      for (int kh = 1; kh < a.kv_heads; ++kh) total = total + hs[wave * a.kv_heads + kh];
      a.scores[(int64_t)b * a.max_pages + p] = canonical_score(total);
    }
    __syncthreads();
  }
}

struct SelectArgs {
  const float* scores;
  const int64_t* lengths;
  int64_t length;
  int page_size, max_pages, top_pages, keep_sink, mode;
  uint32_t forced_key;  // key of the forced (required) pages
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
        key[q] = (p == count - 1 || (second && p == 0)) ? a.forced_key : order_key(sc[p]);
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

// Writes request b's chosen pages (top_pages entries, -1 padded, in LDS) to
// pages and expands them to token positions (-1 past the request's length),
// with the kSelectWaveThreads threads of the workgroup.
__device__ __forceinline__ void write_selection(const SelectArgs& a, int b, const int32_t* chosen, int64_t len) {
  const int tid = threadIdx.x;
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

// Up to kWave * KPL pages, for more than kWavesMaxTop chosen: wave 0 selects
// (wave_select), then the four waves expand the chosen pages to token
// positions.
template <int KPL>
__global__ __launch_bounds__(kSelectWaveThreads) void select_wave_kernel(SelectArgs a) {
  __shared__ int32_t chosen[kWave * KPL];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int64_t len = a.lengths ? a.lengths[b] : a.length;
  if (tid < kWave)
    wave_select<KPL>(a.scores + (int64_t)b * a.max_pages, a.max_pages, count, a.top_pages, a.mode, a.keep_sink,
                     a.forced_key, chosen);
  __syncthreads();
  write_selection(a, b, chosen, len);
}

// Up to 4 * kWave * KPL pages and kWavesMaxTop chosen (the selectors' kernel
// whenever at most kWavesMaxTop pages are chosen, up to 4096 pages): the
// four waves rank (four_wave_rank), then expand the chosen pages to token
// positions.
template <int KPL, int KPL2>
__global__ __launch_bounds__(kSelectWaveThreads) void select_waves_kernel(SelectArgs a) {
  static_assert(kSelectWaveThreads == 4 * kWave, "four_wave_rank ranks with four waves");
  __shared__ uint32_t cand_key[4 * kWavesMaxTop];
  __shared__ int32_t cand_page[4 * kWavesMaxTop];
  __shared__ int n_cand[4];
  __shared__ int32_t chosen[kWavesMaxTop];
  const int b = blockIdx.x;
  // the score loads are issued before the page count arrives
  float sv[KPL];
  wave_scores_at<KPL>(a.scores + (int64_t)b * a.max_pages, a.max_pages, (int)(threadIdx.x / kWave) * kWave * KPL, sv);
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int64_t len = a.lengths ? a.lengths[b] : a.length;
  four_wave_rank<KPL, KPL2>(sv, count, a.top_pages, a.mode, a.keep_sink, a.forced_key, cand_key, cand_page, n_cand,
                            chosen);
  __syncthreads();
  write_selection(a, b, chosen, len);
}

// Any page count (beyond the register kernels' 16384): every pass recomputes
// the keys from the scores (which stay in L2), a 4-pass 8-bit radix select
// over an LDS histogram finds the k-th key, and the chosen pages are
// compacted in page order, 1024 pages per block scan, straight into
// `pages`. The page -> token expansion then reads them back (written by this
// workgroup before the barrier).
constexpr int kSelectLargeThreads = 1024;

__global__ __launch_bounds__(kSelectLargeThreads) void select_large_kernel(SelectArgs a) {
  __shared__ int32_t hist[256];
  __shared__ int32_t scan[kSelectLargeThreads / 64 + 1];
  __shared__ int32_t pick[2];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int count = page_count(a.lengths, a.length, b, a.page_size, a.max_pages);
  const int64_t len = a.lengths ? a.lengths[b] : a.length;
  int32_t* pages = a.pages + (int64_t)b * a.top_pages;
  int n_sel = 0;
  if (a.top_pages < count) {
    const float* sc = a.scores + (int64_t)b * a.max_pages;
    const bool second = a.mode == kModeQuest ? (a.keep_sink && a.top_pages > 1 && count > 1) : a.top_pages > 1;
    auto key_of = [&](int p) -> uint32_t {
      return (p == count - 1 || (second && p == 0)) ? a.forced_key : order_key(sc[p]);
    };
    uint32_t prefix = 0u, pmask = 0u;
    int need = a.top_pages;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      for (int p = tid; p < count; p += kSelectLargeThreads) {
        const uint32_t k = key_of(p);
        if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1);
      }
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
          const int o = __shfl_up(incl, d);
          if (tid >= d) incl += o;
        }
        const int before = incl - csum;
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
    // every key above `prefix` is taken, then the first `need` pages with it
    int tie_base = 0;
    for (int c0 = 0; c0 < count; c0 += kSelectLargeThreads) {
      const int p = c0 + tid;
      const uint32_t k = p < count ? key_of(p) : 0u;
      const bool tie = p < count && k == prefix;
      int n_tie;
      const int tie_rank = tie_base + block_exclusive_scan<int32_t>(tie ? 1 : 0, scan, &n_tie);
      const bool sel = p < count && (k > prefix || (tie && tie_rank < need));
      int n_here;
      const int out = n_sel + block_exclusive_scan<int32_t>(sel ? 1 : 0, scan, &n_here);
      if (sel) pages[out] = p;
      tie_base += n_tie;
      n_sel += n_here;
    }
  } else {
    n_sel = count;
    for (int i = tid; i < count; i += kSelectLargeThreads) pages[i] = i;
  }
  for (int i = n_sel + tid; i < a.top_pages; i += kSelectLargeThreads) pages[i] = -1;
  __syncthreads();
  const int P = a.page_size;
  const int64_t n_pos = (int64_t)a.top_pages * P;
  int32_t* pos = a.positions + (int64_t)b * n_pos;
  for (int64_t i = tid; i < n_pos; i += kSelectLargeThreads) {
    const uint32_t j = a.page_div.div((uint32_t)i);
    const int32_t p = pages[j];
    const int64_t t = (int64_t)p * P + (int64_t)((uint32_t)i - j * (uint32_t)P);
    pos[i] = (p >= 0 && t < len) ? (int32_t)t : -1;
  }
}

static int check_select_common(const char* who, int32_t batch, const void* query, int q_dtype, int32_t q_heads,
                               int32_t kv_heads, int32_t head_dim, const int64_t* lengths, int64_t length,
                               int32_t page_size, int32_t max_pages, int32_t top_pages, float* scores,
                               int32_t* pages, int32_t* positions) {
  if (!query || !scores) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (!pages != !positions) return fail(NHS_ERR_INVALID, "%s: pages and positions are both given or both null", who);
  if (!valid_dtype(q_dtype)) return fail(NHS_ERR_INVALID, "%s: bad query dtype", who);
  if (batch < 0 || q_heads < 1 || kv_heads < 1 || head_dim < 1 || page_size < 1 || max_pages < 1 ||
      top_pages < 1 || q_heads % kv_heads)
    return fail(NHS_ERR_INVALID, "%s: invalid shape or page budget", who);
  if ((int64_t)top_pages * page_size >= (1ll << 31) || (int64_t)max_pages * page_size >= (1ll << 32))
    return fail(NHS_ERR_UNSUPPORTED, "%s: top_pages * page_size must be < 2^31", who);
  if (!lengths && (length < 0 || length >= (1ll << 31)))
    return fail(NHS_ERR_INVALID, "%s: length must be in [0, 2^31)", who);
  return NHS_OK;
}

// Chunking of a bound row (head_dim elements of `esize` bytes) into lanes:
// 16-byte chunks when the row is a multiple of 16 bytes of at most 64
// chunks, else one element per lane up to 64 elements, else
// ceil(head_dim / 64) elements (the last lane's chunk shorter). Returns the
// elements per lane.
static int chunk_elems(int head_dim, int esize) {
  if ((head_dim * esize) % 16 == 0 && head_dim * esize / 16 <= 64) return 16 / esize;
  if (head_dim <= 64) return 1;
  return (head_dim + 63) / 64;
}

// A chunk of E elements is loaded as one vector when it is 16 or 32 bytes
// and divides the row; otherwise element by element (kernel instance E = 0).
static bool vector_chunk(int head_dim, int E, int esize) {
  return head_dim % E == 0 && (E * esize == 16 || E * esize == 32);
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
  if (wave_pages > NHS_MAX_SELECT_PAGES) {
    launch(select_large_kernel, dim3((unsigned)batch), dim3(kSelectLargeThreads), 0, stream, start, stop, s);
  } else if (wave_pages <= 4 * kWave * 16 && s.top_pages <= kWavesMaxTop) {
    // four ranking waves (KPL pages per lane each) and their <= 4 * top_pages
    // candidates, KPL2 per lane
    const int c = 4 * s.top_pages;
    const int kpl = wave_pages <= 4 * kWave * 2 ? 2 : wave_pages <= 4 * kWave * 4 ? 4 : wave_pages <= 4 * kWave * 8 ? 8 : 16;
    const int kpl2 = c <= 2 * kWave ? 2 : c <= 4 * kWave ? 4 : 16;
    void (*k)(SelectArgs) = nullptr;
    switch (kpl * 32 + kpl2) {
#define NHS_WAVES_CASE(A, B) \
  case A * 32 + B: k = select_waves_kernel<A, B>; break;
      NHS_WAVES_CASE(2, 2) NHS_WAVES_CASE(2, 4) NHS_WAVES_CASE(2, 16)
      NHS_WAVES_CASE(4, 2) NHS_WAVES_CASE(4, 4) NHS_WAVES_CASE(4, 16)
      NHS_WAVES_CASE(8, 2) NHS_WAVES_CASE(8, 4) NHS_WAVES_CASE(8, 16)
      NHS_WAVES_CASE(16, 2) NHS_WAVES_CASE(16, 4) NHS_WAVES_CASE(16, 16)
#undef NHS_WAVES_CASE
    }
    launch(k, dim3((unsigned)batch), dim3(kSelectWaveThreads), 0, stream, start, stop, s);
  } else if (wave_pages <= kWave * 8) {
    launch(select_wave_kernel<8>, dim3((unsigned)batch), dim3(kSelectWaveThreads), 0, stream, start, stop, s);
  } else if (wave_pages <= kWave * 16) {
    launch(select_wave_kernel<16>, dim3((unsigned)batch), dim3(kSelectWaveThreads), 0, stream, start, stop, s);
  } else if (s.max_pages <= 256 * kMaxSelectPerThread) {
    launch(select_topk_kernel<256>, dim3((unsigned)batch), dim3(256), 0, stream, start, stop, s);
  } else {
    launch(select_topk_kernel<kSelectThreads>, dim3((unsigned)batch), dim3(kSelectThreads), 0, stream, start, stop, s);
  }
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
  const int esize = elem_size(bounds_dtype);
  const int E = quest_chunk_elems(head_dim, esize);
  const bool vec = vector_chunk(head_dim, E, esize);
  if (!items && vec && (((uintptr_t)minimum | (uintptr_t)maximum) % 16 || (bounds_batch_stride * esize) % 16))
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
  a.elems = E;
  a.lanes_used = (head_dim + E - 1) / E;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.lengths = lengths;
  a.length = length;
  a.page_size = page_size;
  a.max_pages = max_pages;
  a.scores = scores;
  a.group = q_heads / kv_heads;
  const int lpr = 1 << a.lpr_log2;
  const int lanes_per_page = kv_heads * lpr;
  void (*kernel)(ScoreArgs) = nullptr;
  dim3 grid, block;
  size_t lds = 0;
  const int ppw = lanes_per_page <= kWave ? kWave / lanes_per_page : 0;
  if (vec && E * esize == 32 && ppw > 0 && a.group <= 8) {
    // a page fits one wave: the page kernel
    a.pages_per_step = ppw;
    a.pages_per_block = kPageWaves * page_slots(a.group) * ppw;
    grid = dim3((unsigned)((max_pages + a.pages_per_block - 1) / a.pages_per_block), (unsigned)batch);
    block = dim3(kPageThreads);
    // SPLIT when a page takes exactly half a wave: the two half-waves fold
    // the same query chunks, so each folds half of them
    const int split = lanes_per_page == kWave / 2 ? 1 : 0;
    switch ((bounds_dtype * 16 + a.group) * 2 + split) {  // instantiated for every group size: no masked heads
#define NHS_PAGE_CASE(DT, TY, EE, GG)                                                  \
  case (DT * 16 + GG) * 2: kernel = quest_page_kernel<TY, EE, GG, false>; break;      \
  case (DT * 16 + GG) * 2 + 1: kernel = quest_page_kernel<TY, EE, GG, true>; break;
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
    // the general kernel: the folded query in LDS; a page's KV heads in
    // passes when they need more lanes than the workgroup has
    const int threads = kQuestThreads;
    a.heads_per_pass = lanes_per_page <= threads ? kv_heads : threads / lpr;
    a.pages_per_step = threads / (a.heads_per_pass * lpr);
    a.pages_per_block = a.pages_per_step * ((kPagesPerBlock + a.pages_per_step - 1) / a.pages_per_step);
    grid = dim3((unsigned)((max_pages + a.pages_per_block - 1) / a.pages_per_block), (unsigned)batch);
    block = dim3(threads);
    const size_t kvd = (size_t)kv_heads * head_dim;
    lds = kvd * (2 * sizeof(float) + 1) + (size_t)a.pages_per_step * kv_heads * sizeof(float);
    if (lds > kMaxQuestLds)
      return fail(NHS_ERR_UNSUPPORTED, "%s: kv_heads * head_dim = %zu exceeds %d", who, kvd, kMaxQuestFold);
    const int EV = vec ? E : 0;
    switch (bounds_dtype * 64 + EV) {
#define NHS_QUEST_CASE(DT, TY, EE) \
  case DT * 64 + EE: kernel = quest_score_kernel<TY, EE>; break;
      NHS_QUEST_CASE(NHS_F32, F32, 8)
      NHS_QUEST_CASE(NHS_F32, F32, 4)
      NHS_QUEST_CASE(NHS_F32, F32, 0)
      NHS_QUEST_CASE(NHS_F16, F16, 16)
      NHS_QUEST_CASE(NHS_F16, F16, 8)
      NHS_QUEST_CASE(NHS_F16, F16, 0)
      NHS_QUEST_CASE(NHS_BF16, BF16, 16)
      NHS_QUEST_CASE(NHS_BF16, BF16, 8)
      NHS_QUEST_CASE(NHS_BF16, BF16, 0)
#undef NHS_QUEST_CASE
    }
  }
  // The scores are computed also when every page is kept (top_pages >=
  // max_pages): scores[b, :] then still holds them, and the caller's start
  // event always stamps this first kernel.
  if (!kernel) return fail(NHS_ERR_UNSUPPORTED, "%s: no scoring kernel", who);
  launch(kernel, grid, block, lds, s, ev.start, pages ? nullptr : ev.stop, a);
  ev.start = nullptr;  // the start event belongs to the first kernel
  st = launch_status(who);
  if (st != NHS_OK) return st;
  if (!pages) return NHS_OK;  // scores only
  SelectArgs sa;
  sa.scores = scores;
  sa.lengths = lengths;
  sa.length = length;
  sa.page_size = page_size;
  sa.max_pages = max_pages;
  sa.top_pages = top_pages;
  sa.keep_sink = keep_sink;
  sa.mode = kModeQuest;
  sa.forced_key = kForcedQuest;
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
  if (((size_t)kv_heads * head_dim + (size_t)kScoreWaves * kv_heads) * sizeof(float) > kMaxQuestLds)
    return fail(NHS_ERR_UNSUPPORTED, "%s: kv_heads * head_dim too large", who);
  const int E = chunk_elems(head_dim, 4);
  const bool vec = vector_chunk(head_dim, E, 4);
  if (vec && ((uintptr_t)summaries % 16 || (summaries_batch_stride * 4) % 16))
    return fail(NHS_ERR_INVALID, "%s: summaries must be 16-byte aligned", who);
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
  a.elems = E;
  a.lanes_used = (head_dim + E - 1) / E;
  a.lpr_log2 = ilog2(a.lanes_used);
  a.lengths = lengths;
  a.length = length;
  a.page_size = page_size;
  a.max_pages = max_pages;
  a.scores = scores;
  dim3 grid((unsigned)((max_pages + kPagesPerBlock - 1) / kPagesPerBlock), (unsigned)batch);
  size_t lds = ((size_t)kv_heads * head_dim + (size_t)kScoreWaves * kv_heads) * sizeof(float);
  {  // computed also when every page is kept, as the Quest scores are
    hipEvent_t stop = pages ? nullptr : ev.stop;
    if (vec)
      launch(mean_score_kernel<4>, grid, dim3(kScoreThreads), lds, s, ev.start, stop, a);
    else if (E == 1)
      launch(mean_score_kernel<1>, grid, dim3(kScoreThreads), lds, s, ev.start, stop, a);
    else
      launch(mean_score_kernel<0>, grid, dim3(kScoreThreads), lds, s, ev.start, stop, a);
    ev.start = nullptr;
    st = launch_status(who);
    if (st != NHS_OK) return st;
  }
  if (!pages) return NHS_OK;  // scores only
  SelectArgs sa;
  sa.scores = scores;
  sa.lengths = lengths;
  sa.length = length;
  sa.page_size = page_size;
  sa.max_pages = max_pages;
  sa.top_pages = top_pages;
  sa.keep_sink = 1;
  sa.mode = kModeMean;
  sa.forced_key = kRequiredMean;
  sa.page_div = FastDiv((uint32_t)page_size);
  sa.pages = pages;
  sa.positions = positions;
  return launch_select(sa, batch, s, who, ev.start, ev.stop);
}
