// Row resolver: logical token positions -> physical pool rows, with resident
// lookup, hot-row lookup and LRU miss assignment, for `batch` independent
// (request, layer) items in one launch (one 1024-thread workgroup per item).
//
// The semantics are those of resolve_rows (nano_hisparse/row_index.py:62-140),
// restated as LDS passes instead of sorts over the hot rows:
//  0. (resolve_rows_kernel<KPL > 0>, nhs_select_resolve_*) waves 0-3 (wave 0
//     alone when more than 256 pages are chosen) select the top_pages best
//     pages of the item's scores as the selectors do (four_wave_rank /
//     wave_rank, select_common.h) while the other waves stage the tables;
//     the chosen pages expanded to tokens are the positions.
//  1. keys (norm << 32 | input index), norm = raw if 0 <= raw < length else
//     length, bitonic-sorted in LDS unless already in order: sorted order =
//     ascending logical, and the first entry of each run of equal positions
//     is its first occurrence in the input.
//  2. per sorted entry: page/offset, source and resident tables (staged in
//     LDS at entry when they fit), host row, valid / resident_hit /
//     needs_hot.
//  3. an LDS hash of the host rows that need the hot buffer.
//  4. one coalesced pass over tags: a tag found in the hash is a hot hit for
//     that host row and marks its slot protected.
//  5. victims = lru stably partitioned (unprotected first): the lru values
//     are staged in LDS and ranked in 1024-slot chunks with wave ballots
//     and a DPP scan of the per-wave counts.
//     The same pass writes the new lru: it is the lru stably partitioned by
//     category (untouched, inserted, hit, inserted hit). Misses take the
//     first n_miss victims, so with U / Pr the unprotected / protected slots
//     in lru order, m = min(n_miss, |U|) and e = n_miss - m, the new lru is
//     U[m:] ++ U[:m] ++ Pr[e:] ++ Pr[:e], a rotation of each part. n_miss is
//     summed with the protected count before the pass.
//  6. miss ranks by a block scan; assigned slot = victims[rank].
//  7. physical rows (scattered back to input order), compact miss plan, tag
//     writes for misses.
#include "select_common.h"

namespace nhs {

constexpr int kResolveThreads = 1024;
constexpr int kMaxK = 4096;                       // sorted entries per item held in LDS (resolve_rows_kernel)
constexpr int kMaxH = NHS_MAX_HOT_ROWS;           // hot rows per item
constexpr int kKPerThread = kMaxK / kResolveThreads;  // 4
constexpr int kHashCap = 2 * kMaxK;                // load factor <= 1/2
constexpr int kRegH = 8;        // hot rows per thread whose tag and lru are loaded at entry (H <= 8192)
constexpr int kHotCache = 1024; // hot blocks staged in LDS at entry
constexpr int kWaves = kResolveThreads / 64;
constexpr int kRankGroup = 4;   // 1024-slot chunks ranked per barrier
constexpr int kTableCache = 2048;  // page table entries staged in LDS at entry
constexpr int kFusedWavePages = kWave * 16;      // pages the fused select ranks in one wave
constexpr int kFusedMaxPages = 4 * kFusedWavePages;  // ... in four waves (at most kWavesMaxTop chosen)

struct ResolveArgs {
  int n;  // positions per item
  const void* positions;
  int positions_i64;
  int64_t positions_stride;
  const int32_t* source;
  const int32_t* resident;
  int64_t page_stride;
  int n_pages;
  const int32_t* hot;
  int64_t hot_stride;
  int32_t* tags;
  int64_t tags_stride;
  int64_t* lru;
  int64_t lru_stride;
  int hot_rows;
  const int64_t* lengths;
  int64_t length;
  int page_size;
  FastDiv page_div;
  int64_t* physical;
  int64_t* miss_host;
  int64_t* miss_device;
  int64_t plan_stride;
  int64_t* counts;
  int64_t* counts_total;
  const nhs_layer_item* items;  // per-item tables (then the strided table fields are unused)
  // fused selection (resolve_rows_kernel<KPL > 0>): the positions are the
  // top_pages best pages of `scores` expanded to tokens, n = top_pages * P
  const float* scores;  // [batch, max_pages]
  int max_pages, top_pages, keep_sink, mode;
  uint32_t forced_key;
  int32_t* pages_out;      // [batch, top_pages]
  int32_t* positions_out;  // [batch, n]
};

struct ResolveShared {
  union {
    struct {
      uint64_t keys[kMaxK];           // phase 1-2
      int32_t src[kTableCache];       // the item's page tables, when they fit
      int32_t res[kTableCache];
      int32_t chosen[kFusedWavePages]; // fused selection: chosen pages, ascending, -1 padded
    } e;
    struct {
      int32_t hkey[kHashCap];  // phase 3-4: wanted host rows
      int32_t hslot[kHashCap]; // hot slot holding that host row, or -1
    } hash;
    uint16_t lru16[kMaxH];     // phase 5: the item's lru, staged
  } u;
  uint32_t prot[kMaxH / 32];  // protected slot bits
  int32_t victims[kMaxK];     // victims[0 .. min(n, H)-1]
  int32_t red[2][kWaves * 8];                    // one scratch row per block reduction
  int32_t wcount[2][kRankGroup][kWaves];         // per-wave unprotected counts, double-buffered
  int32_t hot[kHotCache];                      // the item's hot block table, when it fits
};

// Block reductions with one barrier each. Every call site passes its own
// scratch row, so no barrier is needed before the scratch is reused.

// Sum of x over each 16-lane row of the wave, in every lane of the row.
__device__ __forceinline__ int row_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);  // row_half_mirror
  x += __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);  // row_mirror
  return x;
}

// Sums of N ints over the block; every thread receives the sums. Wave sums
// are row sums read from lanes 0, 16, 32, 48; after the barrier lane w
// (< kWaves) of every wave reads wave w's sums and a row sum adds them.
template <int N>
__device__ __forceinline__ void block_sums(int (&v)[N], int32_t* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int r = row_sum(v[i]);
    const int t = __builtin_amdgcn_readlane(r, 0) + __builtin_amdgcn_readlane(r, 16) +
                  __builtin_amdgcn_readlane(r, 32) + __builtin_amdgcn_readlane(r, 48);
    if (lane == 0) scratch[wave * N + i] = t;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __builtin_amdgcn_readlane(row_sum(lane < kWaves ? scratch[lane * N + i] : 0), 0);
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
__device__ __forceinline__ int block_scan(int v, int32_t* scratch, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  int before = 0, t = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int x = scratch[w];
    t += x;
    before += w < wave ? x : 0;
  }
  *total = t;
  return before + incl - v;
}

// Victims and the new lru (phase 5): the lru (staged in lru16) stably
// partitioned into unprotected slots U and protected slots Pr, each in lru
// order; victims[rank] = the rank-th slot of U ++ Pr for rank < vlimit. The
// new lru is U[m:] ++ U[:m] ++ Pr[e:] ++ Pr[:e] with m = min(inserted, |U|)
// and e = inserted - m, inserted = min(n_miss, H) (more misses than hot rows
// reuse the last victim, so at most H slots are inserted).
// The lru is walked in 1024-slot chunks, kRankGroup chunks per barrier. A
// slot's rank among the unprotected slots of its chunk is its lane's rank in
// the wave's ballot plus the unprotected counts of the lower waves: lane w
// (< kWaves) of every wave reads wave w's count (ucount, double-buffered, so
// a buffer is rewritten only after every thread has passed the next group's
// barrier) and a DPP scan over those 16 lanes gives the prefixes. Valid
// slots are a prefix of the threads, so a protected slot's rank is its
// thread index minus the unprotected slots below it. Ends without a
// barrier: callers synchronise before reading victims.
static_assert(kWaves == 16, "one row of 16 lanes holds the wave counts");
template <typename V>
__device__ __forceinline__ void partition_lru(const uint16_t* lru16, const uint32_t* prot, int H, int n_prot,
                                              int n_miss, int vlimit, V* victims, NHS_GLOBAL int64_t* lru_out,
                                              int32_t (*ucount)[kRankGroup][kWaves]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n_unprot = H - n_prot;
  const int inserted = n_miss < H ? n_miss : H;
  const int m_u = inserted < n_unprot ? inserted : n_unprot;
  const int e_p = inserted - m_u;
  auto prot_bit = [&](int v) { return (int)((prot[v >> 5] >> (v & 31)) & 1u); };
  const int n_chunks = (H + kResolveThreads - 1) / kResolveThreads;
  int base_u = 0, base_p = 0, parity = 0;
  for (int g0 = 0; g0 < n_chunks; g0 += kRankGroup, parity ^= 1) {
    const int chunks = min(kRankGroup, n_chunks - g0);
    int vv[kRankGroup], below[kRankGroup];
    bool valid[kRankGroup], unprot[kRankGroup];
#pragma unroll
    for (int c = 0; c < kRankGroup; ++c) {
      valid[c] = unprot[c] = false;
      vv[c] = below[c] = 0;
      if (c < chunks) {
        const int r = (g0 + c) * kResolveThreads + tid;
        valid[c] = r < H;
        vv[c] = valid[c] ? lru16[r] : 0;
        unprot[c] = valid[c] && !prot_bit(vv[c]);
        const uint64_t m = __ballot(unprot[c]);
        below[c] = lanes_below(m);
        if (lane == 0) ucount[parity][c][wave] = __popcll(m);
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kRankGroup; ++c) {
      if (c < chunks) {
        // inclusive scan of the wave counts over lanes 0..15 (row_shr 1, 2, 4, 8)
        int x = lane < kWaves ? ucount[parity][c][lane] : 0;
        x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);
        x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);
        x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);
        x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);
        const int total_u = __builtin_amdgcn_readlane(x, kWaves - 1);
        const int waves_below = wave > 0 ? __builtin_amdgcn_readlane(x, wave - 1) : 0;
        const int n_valid = min(kResolveThreads, H - (g0 + c) * kResolveThreads);
        if (valid[c]) {
          const int within_u = waves_below + below[c];
          int rank, pos;
          if (unprot[c]) {
            const int u = base_u + within_u;
            rank = u;
            pos = u >= m_u ? u - m_u : n_unprot - m_u + u;
          } else {
            const int pr = base_p + tid - within_u;
            rank = n_unprot + pr;
            pos = n_unprot + (pr >= e_p ? pr - e_p : n_prot - e_p + pr);
          }
          if (rank < vlimit) victims[rank] = (V)vv[c];
          // pos < H for a permutation; the check keeps a corrupt lru (clamped
          // duplicates, so the protected count and the ranks disagree) in bounds
          if (pos >= 0 && pos < H) lru_out[pos] = vv[c];
        }
        base_u += total_u;
        base_p += n_valid - total_u;
      }
    }
  }
}

// Writes an item's [resident hits, hot hits, misses] and adds them to the
// running totals.
__device__ __forceinline__ void write_counts(const ResolveArgs& a, int b, int rhit, int hhit, int miss) {
  int64_t* c = a.counts + (int64_t)b * 3;
  c[0] = rhit;
  c[1] = hhit;
  c[2] = miss;
  if (a.counts_total) {
    atomicAdd((unsigned long long*)&a.counts_total[0], (unsigned long long)rhit);
    atomicAdd((unsigned long long*)&a.counts_total[1], (unsigned long long)hhit);
    atomicAdd((unsigned long long*)&a.counts_total[2], (unsigned long long)miss);
  }
}

__device__ __forceinline__ uint32_t hash_row(int32_t key) { return (uint32_t)key * 2654435761u; }

// Linear probing, four slots per LDS round trip: the probe loop runs until
// every lane of the wave is done, so each round reads the next four slots at
// once (at load factor <= 1/2, and 1/8 at the usual 1024 wanted rows, a
// lane rarely needs a second round).
__device__ __forceinline__ int hash_find(const int32_t* hkey, int32_t key) {
  constexpr uint32_t m = kHashCap - 1;
  uint32_t h = hash_row(key) & m;
  while (true) {
    const int32_t k0 = hkey[h], k1 = hkey[(h + 1) & m], k2 = hkey[(h + 2) & m], k3 = hkey[(h + 3) & m];
    if (k0 == key) return (int)h;
    if (k0 == -1) return -1;
    if (k1 == key) return (int)((h + 1) & m);
    if (k1 == -1) return -1;
    if (k2 == key) return (int)((h + 2) & m);
    if (k2 == -1) return -1;
    if (k3 == key) return (int)((h + 3) & m);
    if (k3 == -1) return -1;
    h = (h + 4) & m;
  }
}

// KPL = 0: the positions are read from a.positions. KPL = 8 or 16: the
// workgroup first selects the top_pages best of the request's page scores
// as the selectors do (KPL2 = 0: wave 0, wave_rank over up to kWave * KPL
// pages; KPL2 > 0: waves 0-3, four_wave_rank over up to 4 * kWave * KPL
// pages with KPL2 candidates per lane) and the positions are the chosen
// pages expanded to tokens, written to pages_out and positions_out as the
// selectors write them; they come out sorted.
template <int KPL, int KPL2 = 0>
__global__ __launch_bounds__(kResolveThreads) void resolve_rows_kernel(ResolveArgs a) {
  constexpr int kSelectors = KPL == 0 ? 0 : KPL2 > 0 ? 4 : 1;  // waves that rank the scores
  __shared__ ResolveShared sh;
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int n = a.n;
  const int H = a.hot_rows;
  const int P = a.page_size;
  const int64_t length = a.lengths ? a.lengths[b] : a.length;
  int kp = 1;
  while (kp < n) kp <<= 1;
  // fused selection: the ranking waves' score loads go first
  float sv[KPL > 0 ? KPL : 1];
  if constexpr (KPL > 0)
    if (tid < kSelectors * kWave)
      wave_scores_at<KPL>(a.scores + (int64_t)b * a.max_pages, a.max_pages, (int)(tid / kWave) * kWave * KPL, sv);

  // This item's tables: from its entry in the item table, or strided.
  const nhs_layer_item* item = a.items ? a.items + b : nullptr;
  NHS_GLOBAL const int32_t* source = to_global(item ? item->source : a.source + (int64_t)b * a.page_stride);
  NHS_GLOBAL const int32_t* resident = to_global(item ? item->resident : a.resident + (int64_t)b * a.page_stride);
  const int n_pages = item ? (int)item->n_pages : a.n_pages;
  NHS_GLOBAL int32_t* const tags = to_global(item ? item->tags : a.tags + (int64_t)b * a.tags_stride);
  NHS_GLOBAL int64_t* const lru_out = to_global(item ? item->lru : a.lru + (int64_t)b * a.lru_stride);

  // Loads that depend on nothing are issued first: the tags and lru of the
  // first kRegH * kResolveThreads hot rows (registers) and the hot block
  // table (LDS), so their latency overlaps the position lookups below.
  NHS_GLOBAL const int32_t* tags_in = tags;
  NHS_GLOBAL const int64_t* lru_in = lru_out;
  int32_t tag_r[kRegH];
  int64_t lru_r[kRegH];
#pragma unroll
  for (int i = 0; i < kRegH; ++i) {
    const int r = i * kResolveThreads + tid;
    tag_r[i] = r < H ? tags_in[r] : -1;
    lru_r[i] = r < H ? lru_in[r] : 0;
  }
  const int hot_blocks = (H + P - 1) / P;
  const bool hot_cached = hot_blocks <= kHotCache;
  NHS_GLOBAL const int32_t* hot = to_global(item ? item->hot : a.hot + (int64_t)b * a.hot_stride);
  // Tables staged in LDS: the hot block table and, when they fit, the page
  // tables, so the lookups below wait for no second global load. With the
  // fused selection, the ranking waves stage nothing: their LDS writes would
  // wait for these loads before they could rank the scores.
  const int stager = (int)tid - kSelectors * kWave;
  const int stagers = kResolveThreads - kSelectors * kWave;
  if (hot_cached)
    for (int i = stager; i >= 0 && i < hot_blocks; i += stagers) sh.hot[i] = hot[i];
  const bool staged = n_pages >= 1 && n_pages <= kTableCache;
  if (staged)
    for (int i = stager; i >= 0 && i < n_pages; i += stagers) {
      sh.u.e.src[i] = source[i];
      sh.u.e.res[i] = resident[i];
    }

  // ---- 0. fused selection --------------------------------------------------
  if constexpr (KPL > 0) {
    const int count = page_count(a.lengths, a.length, b, P, a.max_pages);
    if constexpr (KPL2 == 0) {
      if (tid < kWave) wave_rank<KPL>(sv, count, a.top_pages, a.mode, a.keep_sink, a.forced_key, sh.u.e.chosen);
    } else {
      // the candidates live in the key array, unused until phase 1
      static_assert(sizeof(sh.u.e.keys) >= 8 * 4 * kWavesMaxTop, "candidates fit the key array");
      uint32_t* cand = reinterpret_cast<uint32_t*>(sh.u.e.keys);
      four_wave_rank<KPL, KPL2>(sv, count, a.top_pages, a.mode, a.keep_sink, a.forced_key, cand,
                                reinterpret_cast<int32_t*>(cand + 4 * kWavesMaxTop), sh.red[0], sh.u.e.chosen);
    }
    __syncthreads();
    for (int i = tid; i < a.top_pages; i += kResolveThreads) a.pages_out[(int64_t)b * a.top_pages + i] = sh.u.e.chosen[i];
  }

  // ---- 1. keys; sorted unless a pair is inverted ---------------------------
  // A thread owns the contiguous run j0 .. j0 + per - 1 of sorted entries.
  // Selector output is already in order (ascending positions, -1 padding at
  // the end maps to `length`), so the page table lookups for the entries in
  // input order are issued right away (after the barrier, from LDS, when the
  // tables are staged) and kept when no pair is inverted. The fused
  // selection's positions are in order by construction: pages ascending,
  // and only the last page (count - 1, the highest chosen) or the padding
  // pages hold positions at or past the length.
  const int per = (n + kResolveThreads - 1) / kResolveThreads;  // <= kKPerThread
  const int j0 = tid * per;
  uint64_t key[kKPerThread];
  int64_t src[kKPerThread], res[kKPerThread];
  auto lookup = [&](int q) {
    if (n_pages < 1) return;  // no pages: every entry stays unset (-1)
    const int64_t lg = (int64_t)(key[q] >> 32);
    // Positions are < 2^31 (int32 host tags); page = min(lg / P, n_pages - 1).
    const uint32_t pg = a.page_div.div((uint32_t)lg);
    const int page = pg < (uint32_t)(n_pages - 1) ? (int)pg : n_pages - 1;
    src[q] = staged ? sh.u.e.src[page] : source[page];
    res[q] = staged ? sh.u.e.res[page] : resident[page];
  };
#pragma unroll
  for (int q = 0; q < kKPerThread; ++q) {
    const int j = j0 + q;
    key[q] = ~0ull;
    src[q] = res[q] = -1;
    if (q < per && j < n) {
      int64_t raw;
      if constexpr (KPL > 0) {
        const uint32_t jp = a.page_div.div((uint32_t)j);
        const int32_t p = sh.u.e.chosen[jp];
        const int64_t t = (int64_t)p * P + (int64_t)((uint32_t)j - jp * (uint32_t)P);
        raw = (p >= 0 && t < length) ? t : -1;
        a.positions_out[(int64_t)b * n + j] = (int32_t)raw;
      } else {
        raw = a.positions_i64 ? static_cast<const int64_t*>(a.positions)[(int64_t)b * a.positions_stride + j]
                              : (int64_t) static_cast<const int32_t*>(a.positions)[(int64_t)b * a.positions_stride + j];
      }
      const int64_t norm = (raw >= 0 && raw < length) ? raw : length;
      key[q] = ((uint64_t)norm << 32) | (uint32_t)j;
      sh.u.e.keys[j] = key[q];
      if (!staged) lookup(q);
    }
  }
  for (int i = n + tid; i < kp; i += kResolveThreads) sh.u.e.keys[i] = ~0ull;  // sort padding
  __syncthreads();
  bool sorted = true;
  if constexpr (KPL == 0) {
    int inverted = 0;
    for (int i = tid; i + 1 < n; i += kResolveThreads) inverted |= sh.u.e.keys[i] > sh.u.e.keys[i + 1];
    sorted = !__syncthreads_or(inverted);
  }
  if (sorted && staged) {
#pragma unroll
    for (int q = 0; q < kKPerThread; ++q)
      if (q < per && j0 + q < n) lookup(q);
  }
  if (!sorted) {
    for (int k = 2; k <= kp; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < kp; i += kResolveThreads) {
          int ixj = i ^ j;
          if (ixj > i) {
            uint64_t x = sh.u.e.keys[i], y = sh.u.e.keys[ixj];
            bool up = (i & k) == 0;
            if ((x > y) == up) {
              sh.u.e.keys[i] = y;
              sh.u.e.keys[ixj] = x;
            }
          }
        }
        __syncthreads();
      }
    }
#pragma unroll
    for (int q = 0; q < kKPerThread; ++q) {
      const int j = j0 + q;
      if (q < per && j < n) {
        key[q] = sh.u.e.keys[j];
        lookup(q);
      }
    }
  }

  // ---- 2. per sorted entry -------------------------------------------------
  int64_t host[kKPerThread];
  int32_t in_idx[kKPerThread], res_blk[kKPerThread], off[kKPerThread];
  bool run_start[kKPerThread], rhit[kKPerThread], nhot[kKPerThread];
#pragma unroll
  for (int q = 0; q < kKPerThread; ++q) {
    int j = j0 + q;
    rhit[q] = nhot[q] = run_start[q] = false;
    host[q] = -1;
    in_idx[q] = 0;
    res_blk[q] = -1;
    off[q] = 0;
    if (q < per && j < n) {
      int64_t lg = (int64_t)(key[q] >> 32);
      in_idx[q] = (int32_t)(key[q] & 0xffffffffu);
      run_start[q] = j == 0 || (int64_t)(sh.u.e.keys[j - 1] >> 32) != lg;
      bool unique = lg < length && run_start[q];
      uint32_t pg = a.page_div.div((uint32_t)lg);
      int32_t o = (int32_t)((uint32_t)lg - pg * (uint32_t)P);
      off[q] = o;
      host[q] = src[q] * P + o;
      bool valid = unique && src[q] >= 0;
      rhit[q] = valid && res[q] >= 0;
      nhot[q] = valid && !rhit[q];
      res_blk[q] = (int32_t)res[q];
    }
  }
  __syncthreads();  // keys are dead from here on; the union becomes the hash

  // ---- 3. hash of host rows that need the hot buffer -----------------------
  for (int i = tid; i < kHashCap; i += kResolveThreads) {
    sh.u.hash.hkey[i] = -1;
    sh.u.hash.hslot[i] = -1;
  }
  for (int i = tid; i < kMaxH / 32; i += kResolveThreads) sh.prot[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kKPerThread; ++q) {
    if (!nhot[q]) continue;
    int32_t key = (int32_t)host[q];
    uint32_t h = hash_row(key) & (kHashCap - 1);
    while (true) {
      int32_t prev = atomicCAS(&sh.u.hash.hkey[h], -1, key);
      if (prev == -1 || prev == key) break;
      h = (h + 1) & (kHashCap - 1);
    }
  }
  __syncthreads();

  // ---- 4. scan tags: hot hits and protected slots ---------------------------
  auto scan_tag = [&](int s, int32_t t) {
    if (t >= 0) {
      int h = hash_find(sh.u.hash.hkey, t);
      if (h >= 0) {
        sh.u.hash.hslot[h] = s;
        atomicOr(&sh.prot[s >> 5], 1u << (s & 31));
      }
    }
  };
#pragma unroll
  for (int i = 0; i < kRegH; ++i)
    if (i * kResolveThreads + tid < H) scan_tag(i * kResolveThreads + tid, tag_r[i]);
  for (int s = kRegH * kResolveThreads + tid; s < H; s += kResolveThreads) scan_tag(s, tags[s]);
  __syncthreads();

  bool hhit[kKPerThread], miss[kKPerThread];
  int32_t slot[kKPerThread];
  int local_miss = 0, local_rhit = 0, local_hhit = 0;
#pragma unroll
  for (int q = 0; q < kKPerThread; ++q) {
    hhit[q] = miss[q] = false;
    slot[q] = 0;
    local_rhit += rhit[q];
    if (nhot[q]) {
      int h = hash_find(sh.u.hash.hkey, (int32_t)host[q]);
      int32_t es = sh.u.hash.hslot[h];
      hhit[q] = es >= 0;
      miss[q] = !hhit[q];
      slot[q] = es;
      local_miss += miss[q];
      local_hhit += hhit[q];
    }
  }

  // ---- 5. victims: lru stably partitioned, unprotected slots first ---------
  __syncthreads();  // the hash is dead; the union now stages the lru
  // the lru is a permutation of [0, H); values are clamped so bad input stays in bounds
#pragma unroll
  for (int i = 0; i < kRegH; ++i) {
    const int r = i * kResolveThreads + tid;
    if (r < H) sh.u.lru16[r] = (uint16_t)(lru_r[i] < 0 ? 0 : lru_r[i] >= H ? H - 1 : lru_r[i]);
  }
  for (int r = kRegH * kResolveThreads + tid; r < H; r += kResolveThreads) {
    const int64_t v = lru_in[r];
    sh.u.lru16[r] = (uint16_t)(v < 0 ? 0 : v >= H ? H - 1 : v);
  }
  // protected slots, misses, resident hits, hot hits
  int tot4[4] = {0, local_miss, local_rhit, local_hhit};
  for (int i = tid; i < (H + 31) / 32; i += kResolveThreads) tot4[0] += __popc(sh.prot[i]);
  block_sums<4>(tot4, sh.red[0]);  // barrier: lru16 staged
  const int n_prot = tot4[0];
  const int vlimit = n < H ? n : H;
  if (tid == 0) write_counts(a, b, tot4[2], tot4[3], tot4[1]);
  partition_lru(sh.u.lru16, sh.prot, H, n_prot, tot4[1], vlimit, sh.victims, lru_out, sh.wcount);
  __syncthreads();  // victims complete

  // ---- 6. miss ranks ----------------------------------------------------------
  int n_miss;
  const int miss_before = block_scan(local_miss, sh.red[1], &n_miss);

  // ---- 7. physical rows, plan, tag writes, counts ----------------------------
  int64_t* phys_out = a.physical + (int64_t)b * a.plan_stride;
  int64_t* mh = a.miss_host + (int64_t)b * a.plan_stride;
  int64_t* md = a.miss_device + (int64_t)b * a.plan_stride;
  {
    int64_t rank = miss_before;
#pragma unroll
    for (int q = 0; q < kKPerThread; ++q) {
      int j = j0 + q;
      if (!(q < per && j < n)) continue;
      int64_t phys = -1;
      if (rhit[q]) {
        phys = (int64_t)res_blk[q] * P + off[q];
      } else if (nhot[q]) {
        int32_t s;
        if (hhit[q]) {
          s = slot[q];
        } else {
          int64_t vr = rank < H - 1 ? rank : H - 1;
          s = sh.victims[vr];
        }
        uint32_t sb = a.page_div.div((uint32_t)s);
        int64_t hp = (int64_t)(hot_cached ? sh.hot[sb] : hot[sb]) * P + (int64_t)((uint32_t)s - sb * (uint32_t)P);
        phys = hp;
        if (miss[q]) {
          mh[rank] = host[q];
          md[rank] = hp;
          tags[s] = (int32_t)host[q];
          ++rank;
        }
      }
      phys_out[in_idx[q]] = run_start[q] ? phys : -1;
    }
  }
  for (int i = tid; i < n; i += kResolveThreads)
    if (i >= n_miss) {
      mh[i] = -1;
      md[i] = -1;
    }
}

// ---- more than 4096 positions: resolve_large_kernel -------------------------
//
// One 1024-thread workgroup per item, for n up to NHS_MAX_POSITIONS. The
// sorted entries fit neither registers nor LDS, so the item's own plan
// outputs (3 x n int64, written last) hold the intermediate state:
//  - unsorted input: keys (norm << 32 | input index) radix-sorted by norm
//    (stable, 4 bits per pass over the bits of `length`) between physical
//    and miss_host, ending in miss_host; sorted input (selector output)
//    derives key j from positions[j] and materialises nothing;
//  - one int32 of state per sorted entry in the upper half of miss_device.
// Phases 2-4 run in rounds of kMaxK sorted entries (an LDS hash of the
// round's wanted host rows, then one pass over the tags); phase 5 is the
// small kernel's; phases 6-7 walk the sorted entries in chunks of 1024 with
// one block scan each. A chunk's plan writes land at miss ranks <= the
// sorted index being written, i.e. on keys and states already read.
constexpr int kLargeMaxK = NHS_MAX_POSITIONS;
constexpr int kRadixBits = 4;
constexpr int kRadixBins = 1 << kRadixBits;

struct LargeShared {
  union {
    uint16_t cnt[kRadixBins * kResolveThreads];  // radix counts, then offsets: [digit][thread]
    struct {
      int32_t hkey[kHashCap];   // a round's wanted host rows
      int32_t hslot[kHashCap];  // hot slot holding that host row, or -1
    } hash;
    uint16_t lru16[kMaxH];      // phase 5: the item's lru, staged
  } u;
  uint16_t victims[kMaxH];
  uint32_t prot[kMaxH / 32];
  int32_t red[4][kWaves * 8];
  int32_t wcount[2][kRankGroup][kWaves];
  int32_t hot[kHotCache];
};

// state of a sorted entry: the hot slot of a hit in bits 0-15, then flags
enum : uint32_t { kStRun = 1u << 16, kStRes = 1u << 17, kStHot = 1u << 18, kStHit = 1u << 19 };

__global__ __launch_bounds__(kResolveThreads) void resolve_large_kernel(ResolveArgs a) {
  __shared__ LargeShared sh;
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int n = a.n;
  const int H = a.hot_rows;
  const int P = a.page_size;
  const int64_t length = a.lengths ? a.lengths[b] : a.length;

  const nhs_layer_item* item = a.items ? a.items + b : nullptr;
  NHS_GLOBAL const int32_t* source = to_global(item ? item->source : a.source + (int64_t)b * a.page_stride);
  NHS_GLOBAL const int32_t* resident = to_global(item ? item->resident : a.resident + (int64_t)b * a.page_stride);
  const int n_pages = item ? (int)item->n_pages : a.n_pages;
  NHS_GLOBAL int32_t* const tags = to_global(item ? item->tags : a.tags + (int64_t)b * a.tags_stride);
  NHS_GLOBAL int64_t* const lru_out = to_global(item ? item->lru : a.lru + (int64_t)b * a.lru_stride);
  NHS_GLOBAL const int32_t* hot = to_global(item ? item->hot : a.hot + (int64_t)b * a.hot_stride);
  const int hot_blocks = (H + P - 1) / P;
  const bool hot_cached = hot_blocks <= kHotCache;
  if (hot_cached)
    for (int i = tid; i < hot_blocks; i += kResolveThreads) sh.hot[i] = hot[i];

  int64_t* const phys_out = a.physical + (int64_t)b * a.plan_stride;
  int64_t* const mh = a.miss_host + (int64_t)b * a.plan_stride;
  int64_t* const md = a.miss_device + (int64_t)b * a.plan_stride;
  uint64_t* const keys = reinterpret_cast<uint64_t*>(mh);         // sorted keys (unsorted input)
  uint64_t* const keys2 = reinterpret_cast<uint64_t*>(phys_out);  // the radix sort's other buffer
  uint32_t* const state = reinterpret_cast<uint32_t*>(md) + n;    // [n]: upper half of miss_device

  auto norm_at = [&](int j) -> int64_t {
    const int64_t raw = a.positions_i64
                            ? static_cast<const int64_t*>(a.positions)[(int64_t)b * a.positions_stride + j]
                            : (int64_t) static_cast<const int32_t*>(a.positions)[(int64_t)b * a.positions_stride + j];
    return (raw >= 0 && raw < length) ? raw : length;
  };

  // ---- 1. sorted keys --------------------------------------------------------
  int inverted = 0;
  for (int i = tid; i + 1 < n; i += kResolveThreads) inverted |= norm_at(i) > norm_at(i + 1);
  const bool sorted = !__syncthreads_or(inverted);
  if (!sorted) {
    // norm <= length < 2^31; an inversion needs length >= 1, so passes >= 1
    int bits = 0;
    while (bits < 31 && (length >> bits) != 0) ++bits;
    const int passes = (bits + kRadixBits - 1) / kRadixBits;
    const int per = (n + kResolveThreads - 1) / kResolveThreads;
    const int j0 = tid * per, j1 = min(n, j0 + per);  // a thread's run, in order: the sort is stable
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = 32 + pass * kRadixBits;
      const bool to_keys = ((passes - 1 - pass) & 1) == 0;  // the last pass writes `keys`
      uint64_t* dst = to_keys ? keys : keys2;
      const uint64_t* prev = to_keys ? keys2 : keys;
      auto src_key = [&](int j) -> uint64_t {
        return pass == 0 ? (((uint64_t)norm_at(j) << 32) | (uint32_t)j) : prev[j];
      };
#pragma unroll
      for (int d = 0; d < kRadixBins; ++d) sh.u.cnt[d * kResolveThreads + tid] = 0;
      for (int j = j0; j < j1; ++j) ++sh.u.cnt[((src_key(j) >> shift) & (kRadixBins - 1)) * kResolveThreads + tid];
      __syncthreads();
      // exclusive scan of the counts in (digit, thread) order: thread t owns
      // entries [16t, 16t + 16) of the flattened table
      uint16_t* c = sh.u.cnt + tid * kRadixBins;
      int v[kRadixBins], s = 0;
#pragma unroll
      for (int i = 0; i < kRadixBins; ++i) {
        v[i] = c[i];
        s += v[i];
      }
      int total;
      int run = block_scan(s, sh.red[pass & 1], &total);
#pragma unroll
      for (int i = 0; i < kRadixBins; ++i) {
        c[i] = (uint16_t)run;
        run += v[i];
      }
      __syncthreads();
      for (int j = j0; j < j1; ++j) {
        const uint64_t k = src_key(j);
        dst[sh.u.cnt[((k >> shift) & (kRadixBins - 1)) * kResolveThreads + tid]++] = k;
      }
      __syncthreads();
    }
  }
  auto key_at = [&](int j) -> uint64_t { return sorted ? (((uint64_t)norm_at(j) << 32) | (uint32_t)j) : keys[j]; };

  // ---- 2-4. per sorted entry, hash join with the tags in rounds -------------
  for (int i = tid; i < kMaxH / 32; i += kResolveThreads) sh.prot[i] = 0u;
  int local_rhit = 0, local_hhit = 0, local_miss = 0;
  constexpr int kPer = kMaxK / kResolveThreads;
  for (int r0 = 0; r0 < n; r0 += kMaxK) {
    for (int i = tid; i < kHashCap; i += kResolveThreads) {
      sh.u.hash.hkey[i] = -1;
      sh.u.hash.hslot[i] = -1;
    }
    __syncthreads();
    uint32_t st[kPer];
    int32_t hrow[kPer];
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int j = r0 + q * kResolveThreads + tid;
      st[q] = 0u;
      hrow[q] = -1;
      if (j < n) {
        const uint64_t key = key_at(j);
        const int64_t lg = (int64_t)(key >> 32);
        const bool run = j == 0 || (int64_t)(key_at(j - 1) >> 32) != lg;
        const uint32_t pg = a.page_div.div((uint32_t)lg);
        const int32_t off = (int32_t)((uint32_t)lg - pg * (uint32_t)P);
        const int64_t page = pg < (uint32_t)(n_pages - 1) ? (int64_t)pg : (int64_t)(n_pages - 1);
        // an item with no pages reads no table: every entry stays unset (-1)
        const int64_t src = n_pages >= 1 ? source[page] : -1, res = n_pages >= 1 ? resident[page] : -1;
        const bool valid = lg < length && run && src >= 0;
        const bool rhit = valid && res >= 0;
        const bool nhot = valid && !rhit;
        st[q] = (run ? kStRun : 0u) | (rhit ? kStRes : 0u) | (nhot ? kStHot : 0u);
        local_rhit += rhit;
        if (nhot) {
          hrow[q] = (int32_t)(src * P + off);
          uint32_t h = hash_row(hrow[q]) & (kHashCap - 1);
          while (true) {
            const int32_t prev = atomicCAS(&sh.u.hash.hkey[h], -1, hrow[q]);
            if (prev == -1 || prev == hrow[q]) break;
            h = (h + 1) & (kHashCap - 1);
          }
        }
      }
    }
    __syncthreads();
    for (int s = tid; s < H; s += kResolveThreads) {
      const int32_t t = tags[s];
      if (t >= 0) {
        const int h = hash_find(sh.u.hash.hkey, t);
        if (h >= 0) {
          sh.u.hash.hslot[h] = s;
          atomicOr(&sh.prot[s >> 5], 1u << (s & 31));
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int j = r0 + q * kResolveThreads + tid;
      if (j >= n) continue;
      if (st[q] & kStHot) {
        const int32_t es = sh.u.hash.hslot[hash_find(sh.u.hash.hkey, hrow[q])];
        if (es >= 0) {
          st[q] |= kStHit | (uint32_t)es;
          ++local_hhit;
        } else {
          ++local_miss;
        }
      }
      state[j] = st[q];
    }
    __syncthreads();  // the hash is cleared for the next round
  }

  // ---- 5. victims and the new lru ---------------------------------------------
  for (int r = tid; r < H; r += kResolveThreads) {
    const int64_t v = lru_out[r];
    sh.u.lru16[r] = (uint16_t)(v < 0 ? 0 : v >= H ? H - 1 : v);
  }
  int tot4[4] = {0, local_miss, local_rhit, local_hhit};
  for (int i = tid; i < (H + 31) / 32; i += kResolveThreads) tot4[0] += __popc(sh.prot[i]);
  block_sums<4>(tot4, sh.red[2]);  // barrier: lru16 staged
  const int vlimit = n < H ? n : H;
  if (tid == 0) write_counts(a, b, tot4[2], tot4[3], tot4[1]);
  partition_lru(sh.u.lru16, sh.prot, H, tot4[0], tot4[1], vlimit, sh.victims, lru_out, sh.wcount);
  __syncthreads();  // victims complete

  // ---- 6-7. miss ranks, physical rows, plan, tag writes ----------------------
  int rank_base = 0;
  for (int c0 = 0, parity = 0; c0 < n; c0 += kResolveThreads, parity ^= 1) {
    const int j = c0 + tid;
    uint64_t key = 0;
    uint32_t st = 0u;
    if (j < n) {
      key = key_at(j);
      st = state[j];
    }
    const bool miss = (st & kStHot) && !(st & kStHit);
    int n_here;
    const int rank = rank_base + block_scan(miss ? 1 : 0, sh.red[parity], &n_here);  // barrier: reads done
    if (j < n) {
      int64_t phys = -1;
      if (st & (kStRes | kStHot)) {
        const int64_t lg = (int64_t)(key >> 32);
        const uint32_t pg = a.page_div.div((uint32_t)lg);
        const int32_t off = (int32_t)((uint32_t)lg - pg * (uint32_t)P);
        const int64_t page = pg < (uint32_t)(n_pages - 1) ? (int64_t)pg : (int64_t)(n_pages - 1);
        if (st & kStRes) {
          phys = (int64_t)resident[page] * P + off;
        } else {
          const int32_t s = (st & kStHit) ? (int32_t)(st & 0xffffu) : (int32_t)sh.victims[rank < H - 1 ? rank : H - 1];
          const uint32_t sb = a.page_div.div((uint32_t)s);
          const int64_t hp =
              (int64_t)(hot_cached ? sh.hot[sb] : hot[sb]) * P + (int64_t)((uint32_t)s - sb * (uint32_t)P);
          phys = hp;
          if (miss) {
            const int64_t host = (int64_t)source[page] * P + off;
            mh[rank] = host;
            md[rank] = hp;
            tags[s] = (int32_t)host;
          }
        }
      }
      phys_out[(uint32_t)key] = (st & kStRun) ? phys : -1;
    }
    rank_base += n_here;
  }
  __syncthreads();
  for (int i = rank_base + tid; i < n; i += kResolveThreads) {
    mh[i] = -1;
    md[i] = -1;
  }
}

}  // namespace nhs

namespace nhs {

static int check_resolve(const char* who, int32_t batch, int32_t n, const void* positions, int32_t hot_rows,
                         const int64_t* lengths, int64_t length, int32_t page_size, const int64_t* physical,
                         const int64_t* miss_host, const int64_t* miss_device, int64_t plan_stride,
                         const int64_t* counts) {
  if (!positions || !physical || !miss_host || !miss_device || !counts)
    return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (batch < 0 || n < 1 || hot_rows < 1 || page_size < 1)
    return fail(NHS_ERR_INVALID, "%s: need n, n_pages, hot_rows, page_size >= 1", who);
  if (n > kLargeMaxK || hot_rows > kMaxH)
    return fail(NHS_ERR_UNSUPPORTED, "%s: n <= %d and hot_rows <= %d required", who, kLargeMaxK, kMaxH);
  // a selection names at most max_union_rows <= hot_rows rows (HotConfig,
  // hybrid.py:36-37), so its misses always fit the hot buffer
  if (n > hot_rows) return fail(NHS_ERR_INVALID, "%s: n (%d) must be <= hot_rows (%d)", who, n, hot_rows);
  if (!lengths && (length < 0 || length >= (1ll << 31)))
    return fail(NHS_ERR_INVALID, "%s: length must be in [0, 2^31)", who);
  if (batch > 1 && plan_stride < n)
    return fail(NHS_ERR_INVALID, "%s: plan_stride must be >= n (items' plans may not overlap)", who);
  return NHS_OK;
}

static void fill_common(ResolveArgs& a, int32_t n, const void* positions, int32_t positions_i64,
                        int64_t positions_stride, int32_t hot_rows, const int64_t* lengths, int64_t length,
                        int32_t page_size, int64_t* physical, int64_t* miss_host, int64_t* miss_device,
                        int64_t plan_stride, int64_t* counts, int64_t* counts_total) {
  a = ResolveArgs{};
  a.n = n;
  a.positions = positions;
  a.positions_i64 = positions_i64;
  a.positions_stride = positions_stride;
  a.hot_rows = hot_rows;
  a.lengths = lengths;
  a.length = length;
  a.page_size = page_size;
  a.page_div = FastDiv((uint32_t)page_size);
  a.physical = physical;
  a.miss_host = miss_host;
  a.miss_device = miss_device;
  a.plan_stride = plan_stride;
  a.counts = counts;
  a.counts_total = counts_total;
}

}  // namespace nhs

extern "C" int nhs_resolve_rows(int32_t batch, int32_t n, const void* positions, int32_t positions_i64,
                                int64_t positions_stride, const int32_t* source, const int32_t* resident,
                                int64_t page_table_stride, int32_t n_pages, const int32_t* hot, int64_t hot_stride,
                                int32_t* tags, int64_t tags_stride, int64_t* lru, int64_t lru_stride,
                                int32_t hot_rows, const int64_t* lengths, int64_t length, int32_t page_size,
                                int64_t* physical, int64_t* miss_host, int64_t* miss_device, int64_t plan_stride,
                                int64_t* counts, int64_t* counts_total, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_resolve_rows";
  int st = check_resolve(who, batch, n, positions, hot_rows, lengths, length, page_size, physical, miss_host,
                         miss_device, plan_stride, counts);
  if (st != NHS_OK) return st;
  if (!source || !resident || !hot || !tags || !lru) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (n_pages < 1) return fail(NHS_ERR_INVALID, "%s: need n, n_pages, hot_rows, page_size >= 1", who);
  if (batch == 0) return NHS_OK;
  ResolveArgs a;
  fill_common(a, n, positions, positions_i64, positions_stride, hot_rows, lengths, length, page_size, physical,
              miss_host, miss_device, plan_stride, counts, counts_total);
  a.source = source;
  a.resident = resident;
  a.page_stride = page_table_stride;
  a.n_pages = n_pages;
  a.hot = hot;
  a.hot_stride = hot_stride;
  a.tags = tags;
  a.tags_stride = tags_stride;
  a.lru = lru;
  a.lru_stride = lru_stride;
  launch(n <= kMaxK ? resolve_rows_kernel<0> : resolve_large_kernel, dim3((unsigned)batch), dim3(kResolveThreads), 0,
         (hipStream_t)stream, ev.start, ev.stop, a);
  return launch_status(who);
}

extern "C" int nhs_resolve_items(int32_t batch, int32_t n, const void* positions, int32_t positions_i64,
                                 int64_t positions_stride, const nhs_layer_item* items, int32_t hot_rows,
                                 const int64_t* lengths, int32_t page_size, int64_t* physical, int64_t* miss_host,
                                 int64_t* miss_device, int64_t plan_stride, int64_t* counts, int64_t* counts_total,
                                 void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_resolve_items";
  int st = check_resolve(who, batch, n, positions, hot_rows, lengths, 0, page_size, physical, miss_host,
                         miss_device, plan_stride, counts);
  if (st != NHS_OK) return st;
  if (!items || !lengths) return fail(NHS_ERR_INVALID, "%s: null items or lengths", who);
  if (batch == 0) return NHS_OK;
  ResolveArgs a;
  fill_common(a, n, positions, positions_i64, positions_stride, hot_rows, lengths, 0, page_size, physical, miss_host,
              miss_device, plan_stride, counts, counts_total);
  a.items = items;
  launch(n <= kMaxK ? resolve_rows_kernel<0> : resolve_large_kernel, dim3((unsigned)batch), dim3(kResolveThreads), 0,
         (hipStream_t)stream, ev.start, ev.stop, a);
  return launch_status(who);
}

// ---- fused selection + resolution ------------------------------------------

namespace nhs {

// The fused launch: resolve_rows_kernel<KPL, KPL2> over `batch` items whose
// positions are their selections: four ranking waves (KPL pages per lane
// each, KPL2 candidates per lane) when at most kWavesMaxTop pages are
// chosen, else one (up to 1024 pages). Rejects shapes beyond the fused
// selection (1024 pages, or 4096 with at most kWavesMaxTop chosen) or the
// LDS-held entries with NHS_ERR_UNSUPPORTED, so that a caller can fall back
// to a selector launch and a resolver launch.
static int launch_select_resolve(const char* who, ResolveArgs& a, int32_t batch, const float* scores,
                                 int32_t max_pages, int32_t mode, int32_t top_pages, int32_t keep_sink,
                                 int32_t* pages, int32_t* positions, hipStream_t stream, const LaunchEvents& ev) {
  if (!scores || !pages || !positions) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (mode != kModeQuest && mode != kModeMean) return fail(NHS_ERR_INVALID, "%s: mode is 0 (Quest) or 1 (mean)", who);
  if (max_pages < 1 || top_pages < 1) return fail(NHS_ERR_INVALID, "%s: need max_pages, top_pages >= 1", who);
  const int wave_pages = max_pages > top_pages ? max_pages : top_pages;
  if ((wave_pages > kFusedWavePages && (wave_pages > kFusedMaxPages || top_pages > kWavesMaxTop)) ||
      (int64_t)top_pages * a.page_size > kMaxK)
    return fail(NHS_ERR_UNSUPPORTED,
                "%s: max(max_pages, top_pages) <= %d, or max_pages <= %d with top_pages <= %d, and top_pages * "
                "page_size <= %d required",
                who, kFusedWavePages, kFusedMaxPages, kWavesMaxTop, kMaxK);
  a.scores = scores;
  a.max_pages = max_pages;
  a.top_pages = top_pages;
  a.keep_sink = keep_sink;
  a.mode = mode;
  a.forced_key = mode == kModeQuest ? kForcedQuest : kRequiredMean;
  a.pages_out = pages;
  a.positions_out = positions;
  if (batch == 0) return NHS_OK;
  void (*kernel)(ResolveArgs);
  // four ranking waves whenever at most kWavesMaxTop are chosen; candidates
  // per lane for their <= 4 * top_pages candidates
  const int c = 4 * top_pages;
  if (top_pages > kWavesMaxTop)
    kernel = wave_pages <= kWave * 8 ? resolve_rows_kernel<8> : resolve_rows_kernel<16>;
  else if (wave_pages <= 4 * kWave * 2)
    kernel = c <= 2 * kWave ? resolve_rows_kernel<2, 2> : c <= 4 * kWave ? resolve_rows_kernel<2, 4> : resolve_rows_kernel<2, 16>;
  else if (wave_pages <= 4 * kWave * 4)
    kernel = c <= 2 * kWave ? resolve_rows_kernel<4, 2> : c <= 4 * kWave ? resolve_rows_kernel<4, 4> : resolve_rows_kernel<4, 16>;
  else if (wave_pages <= 4 * kWave * 8)
    kernel = c <= 2 * kWave ? resolve_rows_kernel<8, 2> : c <= 4 * kWave ? resolve_rows_kernel<8, 4> : resolve_rows_kernel<8, 16>;
  else
    kernel = c <= 2 * kWave ? resolve_rows_kernel<16, 2> : c <= 4 * kWave ? resolve_rows_kernel<16, 4> : resolve_rows_kernel<16, 16>;
  launch(kernel, dim3((unsigned)batch), dim3(kResolveThreads), 0, stream, ev.start, ev.stop, a);
  return launch_status(who);
}

}  // namespace nhs

extern "C" int nhs_select_resolve_rows(int32_t batch, const float* scores, int32_t max_pages, int32_t mode,
                                       int32_t top_pages, int32_t keep_sink, const int32_t* source,
                                       const int32_t* resident, int64_t page_table_stride, int32_t n_pages,
                                       const int32_t* hot, int64_t hot_stride, int32_t* tags, int64_t tags_stride,
                                       int64_t* lru, int64_t lru_stride, int32_t hot_rows, const int64_t* lengths,
                                       int64_t length, int32_t page_size, int32_t* pages, int32_t* positions,
                                       int64_t* physical, int64_t* miss_host, int64_t* miss_device,
                                       int64_t plan_stride, int64_t* counts, int64_t* counts_total, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_select_resolve_rows";
  if (top_pages < 1 || page_size < 1) return fail(NHS_ERR_INVALID, "%s: need top_pages, page_size >= 1", who);
  if ((int64_t)top_pages * page_size > kLargeMaxK)
    return fail(NHS_ERR_UNSUPPORTED, "%s: top_pages * page_size must be <= %d", who, kLargeMaxK);
  const int32_t n = top_pages * page_size;
  int st = check_resolve(who, batch, n, scores, hot_rows, lengths, length, page_size, physical, miss_host,
                         miss_device, plan_stride, counts);
  if (st != NHS_OK) return st;
  if (!source || !resident || !hot || !tags || !lru) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (n_pages < 1) return fail(NHS_ERR_INVALID, "%s: need n, n_pages, hot_rows, page_size >= 1", who);
  ResolveArgs a;
  fill_common(a, n, nullptr, 0, 0, hot_rows, lengths, length, page_size, physical, miss_host, miss_device,
              plan_stride, counts, counts_total);
  a.source = source;
  a.resident = resident;
  a.page_stride = page_table_stride;
  a.n_pages = n_pages;
  a.hot = hot;
  a.hot_stride = hot_stride;
  a.tags = tags;
  a.tags_stride = tags_stride;
  a.lru = lru;
  a.lru_stride = lru_stride;
  return launch_select_resolve(who, a, batch, scores, max_pages, mode, top_pages, keep_sink, pages, positions,
                               (hipStream_t)stream, ev);
}

extern "C" int nhs_select_resolve_items(int32_t batch, const float* scores, int32_t max_pages, int32_t mode,
                                        int32_t top_pages, int32_t keep_sink, const nhs_layer_item* items,
                                        int32_t hot_rows, const int64_t* lengths, int32_t page_size, int32_t* pages,
                                        int32_t* positions, int64_t* physical, int64_t* miss_host,
                                        int64_t* miss_device, int64_t plan_stride, int64_t* counts,
                                        int64_t* counts_total, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_select_resolve_items";
  if (top_pages < 1 || page_size < 1) return fail(NHS_ERR_INVALID, "%s: need top_pages, page_size >= 1", who);
  if ((int64_t)top_pages * page_size > kLargeMaxK)
    return fail(NHS_ERR_UNSUPPORTED, "%s: top_pages * page_size must be <= %d", who, kLargeMaxK);
  const int32_t n = top_pages * page_size;
  int st = check_resolve(who, batch, n, scores, hot_rows, lengths, 0, page_size, physical, miss_host, miss_device,
                         plan_stride, counts);
  if (st != NHS_OK) return st;
  if (!items || !lengths) return fail(NHS_ERR_INVALID, "%s: null items or lengths", who);
  ResolveArgs a;
  fill_common(a, n, nullptr, 0, 0, hot_rows, lengths, 0, page_size, physical, miss_host, miss_device, plan_stride,
              counts, counts_total);
  a.items = items;
  return launch_select_resolve(who, a, batch, scores, max_pages, mode, top_pages, keep_sink, pages, positions,
                               (hipStream_t)stream, ev);
}
