// Page ranking shared by the selectors (select.hip) and the fused select +
// resolve kernel (resolve.hip): order-preserving keys of the page scores and
// the one-wave top-k of up to kWave * KPL pages.
#pragma once

#include "nhs_common.h"

namespace nhs {

enum { kModeQuest = 0, kModeMean = 1 };

// Keys in descending rank order. Numbers map to 0x007fffff .. 0xff800000
// (+inf); NaN ranks above every number, as in torch.topk. Quest's forced
// pages are +inf in the reference (selection.py:86-89), so NaN pages outrank
// them: they take kForcedQuest, just below NaN. The mean selector adds its
// required pages outside the top-k (selection.py:138-145): kRequiredMean,
// above NaN.
constexpr uint32_t kKeyNaN = 0xfffffffeu;
constexpr uint32_t kForcedQuest = 0xfffffffdu;
constexpr uint32_t kRequiredMean = 0xffffffffu;

__device__ __forceinline__ uint32_t order_key(float s) {
  if (s != s) return kKeyNaN;
  uint32_t u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0u;  // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Pages of request b: ceil(length / page_size), at most max_pages.
__device__ __forceinline__ int page_count(const int64_t* lengths, int64_t length, int b, int page_size, int max_pages) {
  int64_t len = lengths ? lengths[b] : length;
  if (len <= 0) return 0;
  int64_t c = (len + page_size - 1) / page_size;
  return (int)(c < max_pages ? c : max_pages);
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Top-k of up to kWave * KPL pages in one wave, with no LDS and no barrier:
// page q * kWave + lane sits in slot q of that lane. The key of the k-th best
// page, the largest x with at least top_pages keys >= x, is found bit by bit,
// most significant first: at each bit the wave counts the keys >= the prefix
// found so far with that bit set (a compare, a ballot and a popcount per
// slot) and keeps the bit when the count reaches top_pages; it stops early
// once exactly top_pages keys are >= the prefix. Every key above the prefix
// is taken, ties at it go to the lowest pages, and the chosen pages come out
// in ascending order (ranks from mbcnt), then -1 up to top_pages.
// Called by the 64 lanes of one wave: wave_scores loads the request's scores
// sc (pages < max(max_pages, 1); pages past max_pages read page 0, values
// past count are never used, and none are when every page is kept), and
// wave_rank selects from them into chosen (kWave * KPL entries). A caller
// issues the score loads early, so that waiting for them does not also wait
// for loads issued after them.
// The scores of pages base + q * kWave + lane (slot q); pages past
// max_pages read page 0.
template <int KPL>
__device__ __forceinline__ void wave_scores_at(const float* sc, int max_pages, int base, float (&sv)[KPL]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int q = 0; q < KPL; ++q) {
    const int p = base + q * kWave + lane;
    sv[q] = sc[p < max_pages ? p : 0];
  }
}

template <int KPL>
__device__ __forceinline__ void wave_scores(const float* sc, int max_pages, float (&sv)[KPL]) {
  wave_scores_at<KPL>(sc, max_pages, 0, sv);
}

// Marks sel[q] for the top_pages best keys of a wave (slot q of lane l is
// item q * kWave + l): the largest prefix x with at least top_pages keys >= x
// is found bit by bit; every key above it is taken, then the ties at it in
// item order. Items without a key hold 0, below every real key (>= 0x007fffff),
// and top_pages must be below the number of real keys, so the prefix always
// has a bit set and no 0 key matches or ties with it.
template <int KPL>
__device__ __forceinline__ void wave_topk(const uint32_t (&key)[KPL], int top_pages, bool (&sel)[KPL]) {
  // prefix = the largest key x with at least top_pages keys >= x, i.e. the
  // key of the k-th best item (or, after an early stop, a smaller x with
  // exactly top_pages keys >= x)
  uint32_t prefix = 0u;
#pragma unroll
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = prefix | (1u << bit);
    // all KPL ballots are formed before any is counted, so the compares
    // write separate mask registers and issue back to back
    uint64_t m[KPL];
#pragma unroll
    for (int q = 0; q < KPL; ++q) m[q] = __ballot(key[q] >= cand);
    int c = 0;
#pragma unroll
    for (int q = 0; q < KPL; ++q) c += __popcll(m[q]);
    if (c >= top_pages) prefix = cand;
    // Exactly top_pages keys >= cand: they are the selection whatever the
    // k-th key's lower bits, and the tie step below takes every key equal
    // to the prefix, so the search can stop (c is the same in every lane).
    if (c == top_pages) break;
  }
  int above = 0;
#pragma unroll
  for (int q = 0; q < KPL; ++q) above += __popcll(__ballot(key[q] > prefix));
  // every item above that key is taken, then the first `need` items with
  // that key in item order (slot, then lane)
  const int need = top_pages - above;
  int before = 0;
#pragma unroll
  for (int q = 0; q < KPL; ++q) {
    const bool tie = key[q] == prefix;
    const uint64_t m = __ballot(tie);
    sel[q] = key[q] > prefix || (tie && before + lanes_below(m) < need);
    before += __popcll(m);
  }
}

// The key of page p of a request of count pages whose score is sv: 0 at or
// past count, forced_key for the forced pages (the last page; the first too
// when Quest keeps the sink, or always for the mean selector when
// top_pages > 1), else order_key(sv).
__device__ __forceinline__ uint32_t page_key(float sv, int p, int count, int mode, int keep_sink, int top_pages,
                                             uint32_t forced_key) {
  const bool second = mode == kModeQuest ? (keep_sink && top_pages > 1 && count > 1) : top_pages > 1;
  return p >= count ? 0u : (p == count - 1 || (second && p == 0)) ? forced_key : order_key(sv);
}

template <int KPL>
__device__ __forceinline__ void wave_rank(const float (&sv)[KPL], int count, int top_pages, int mode, int keep_sink,
                                          uint32_t forced_key, int32_t* chosen) {
  const int lane = threadIdx.x & (kWave - 1);
  bool sel[KPL];
#pragma unroll
  for (int q = 0; q < KPL; ++q) sel[q] = q * kWave + lane < count;
  if (top_pages < count) {
    uint32_t key[KPL];
#pragma unroll
    for (int q = 0; q < KPL; ++q)
      key[q] = page_key(sv[q], q * kWave + lane, count, mode, keep_sink, top_pages, forced_key);
    wave_topk<KPL>(key, top_pages, sel);
  }
  int n_sel = 0;
#pragma unroll
  for (int q = 0; q < KPL; ++q) {
    const uint64_t m = __ballot(sel[q]);
    if (sel[q]) chosen[n_sel + lanes_below(m)] = q * kWave + lane;
    n_sel += __popcll(m);
  }
  for (int i = n_sel + lane; i < top_pages; i += kWave) chosen[i] = -1;
}

// Top-k of up to 4 * kWave * KPL pages, at most kWavesMaxTop chosen, by four
// waves: each ranks its own kWave * KPL pages (wave_topk) and keeps its best
// min(top_pages, its pages) as candidates in LDS, in page order; after a
// barrier wave 0 ranks the candidates, KPL2 per lane (KPL2 * kWave >=
// 4 * top_pages). A page outside its wave's best top_pages has top_pages
// pages before it in (key descending, page ascending) order, so the
// candidates hold the whole selection; and since they stay in page order,
// ties still go to the lowest pages.
// Called by every thread of a workgroup of at least four waves (it holds
// one barrier). Wave w < 4 passes the scores of pages w * kWave * KPL +
// q * kWave + lane in sv (wave_scores_at); other waves' sv are unused.
// cand_key and cand_page hold 4 * kWavesMaxTop entries each and n_cand 4, in
// LDS. Wave 0 writes chosen (top_pages entries, ascending, -1 padded),
// complete after the caller's next barrier.
constexpr int kWavesMaxTop = 256;
template <int KPL, int KPL2>
__device__ __forceinline__ void four_wave_rank(const float (&sv)[KPL], int count, int top_pages, int mode,
                                               int keep_sink, uint32_t forced_key, uint32_t* cand_key,
                                               int32_t* cand_page, int* n_cand, int32_t* chosen) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int top = top_pages;
  if (top < count && wave < 4) {
    const int base = wave * kWave * KPL;
    const int mine = min(max(count - base, 0), kWave * KPL);  // this wave's pages
    uint32_t key[KPL];
    bool sel[KPL];
#pragma unroll
    for (int q = 0; q < KPL; ++q) {
      const int p = base + q * kWave + lane;
      key[q] = page_key(sv[q], p, count, mode, keep_sink, top, forced_key);
      sel[q] = p < count;
    }
    if (top < mine) wave_topk<KPL>(key, top, sel);
    int n = 0;
#pragma unroll
    for (int q = 0; q < KPL; ++q) {
      const uint64_t m = __ballot(sel[q]);
      if (sel[q]) {
        const int i = wave * kWavesMaxTop + n + lanes_below(m);
        cand_key[i] = key[q];
        cand_page[i] = base + q * kWave + lane;
      }
      n += __popcll(m);
    }
    if (lane == 0) n_cand[wave] = n;
  }
  __syncthreads();
  if (wave != 0) return;
  if (top >= count) {  // every page is kept
    for (int i = lane; i < top; i += kWave) chosen[i] = i < count ? i : -1;
    return;
  }
  // candidate j in page order: wave w's i-th, j = (the waves before) + i
  const int n0 = n_cand[0], n1 = n0 + n_cand[1], n2 = n1 + n_cand[2], n3 = n2 + n_cand[3];
  uint32_t key2[KPL2];
  int32_t page2[KPL2];
  bool sel2[KPL2];
#pragma unroll
  for (int q = 0; q < KPL2; ++q) {
    const int j = q * kWave + lane;
    const int w = j < n0 ? 0 : j < n1 ? 1 : j < n2 ? 2 : 3;
    const int i = w * kWavesMaxTop + j - (w == 0 ? 0 : w == 1 ? n0 : w == 2 ? n1 : n2);
    sel2[q] = j < n3;
    key2[q] = sel2[q] ? cand_key[i] : 0u;
    page2[q] = sel2[q] ? cand_page[i] : -1;
  }
  if (top < n3) wave_topk<KPL2>(key2, top, sel2);
  int n_sel = 0;
#pragma unroll
  for (int q = 0; q < KPL2; ++q) {
    const uint64_t m = __ballot(sel2[q]);
    if (sel2[q]) chosen[n_sel + lanes_below(m)] = page2[q];
    n_sel += __popcll(m);
  }
  for (int i = n_sel + lane; i < top; i += kWave) chosen[i] = -1;
}

template <int KPL>
__device__ __forceinline__ void wave_select(const float* sc, int max_pages, int count, int top_pages, int mode,
                                            int keep_sink, uint32_t forced_key, int32_t* chosen) {
  float sv[KPL];
  wave_scores<KPL>(sc, max_pages, sv);
  wave_rank<KPL>(sv, count, top_pages, mode, keep_sink, forced_key, chosen);
}

}  // namespace nhs
