/*
 * CPU oracle for the sparse decode step. TEST INFRASTRUCTURE ONLY: it is the
 * checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * compare the HIP library against; the product never links or calls it.
 *
 * Each function restates one reference function of nano-hisparse
 * (paths relative to the reference repository):
 *   oracle_gather_rows   nano_hisparse/hybrid.py:452-459 (CPU gather loop)
 *   oracle_attend_rows   nano_hisparse/attention.py:26-35 (masked softmax);
 *                        computed in double precision
 *   oracle_attend_rows_f32  the same, in the reference path's float32
 *                        arithmetic (the CPU baseline's attention)
 *   oracle_quest_select  nano_hisparse/selection.py:69-91 + :44-62
 *   oracle_mean_select   nano_hisparse/selection.py:119-145
 *   oracle_resolve_rows  nano_hisparse/row_index.py:62-140
 *   oracle_append_bounds nano_hisparse/storage.py:302-309
 *
 * The selectors sum fp32 terms in one fixed order, which the HIP kernels
 * follow exactly (the reference sums in torch's CPU reduction order, which
 * no other implementation reproduces): a bound row of head_dim elements is
 * cut into E-element chunks (Quest: E = 32 bytes / element size when the
 * row is a multiple of 32 bytes of at most 64 chunks; otherwise, and for
 * the mean selector, 16 bytes / element size when the row is a multiple of
 * 16 bytes of at most 64 chunks, else 1 up to 64 elements, else
 * ceil(head_dim / 64) with a shorter last chunk);
 * each chunk is summed sequentially from 0.0; the chunk sums, padded with
 * +0.0 to a power of two, are added as a pairwise tree in chunk order; the
 * per-KV-head sums are added sequentially.
 *
 * Quest (selection.py:84-85) sums torch.maximum(q*lo, q*hi) over the query
 * heads and dimensions. For one KV head and dimension d, with a = the
 * smaller and b = the larger of the two bounds (a = hi, b = lo when
 * hi < lo, else a = lo, b = hi), a head of its GQA group contributes q*b if
 * q > 0 and q*a otherwise, so the group's terms are
 *   a[d] * Qneg[d] + b[d] * Qpos[d],
 * with Qpos / Qneg the sums of the group's positive / non-positive query
 * values at d (added sequentially in head order from 0.0). Each chunk step
 * is t = fma(nneg ? a : 0, Qneg, t) then t = fma(npos ? b : 0, Qpos, t),
 * where npos / nneg say whether any head contributed to Qpos / Qneg.
 *
 * Special values follow torch.maximum, which returns NaN when either
 * product is NaN: a page's score is NaN when one of its bounds is NaN, when
 * a head's query is +-0 at a d where a bound is +-inf, or when a head's
 * query is +-inf at a d where a bound is +-0 (each is 0 * inf in one of the
 * two products). The chunk holding such an element sums to NaN. +-inf
 * terms of both signs add to NaN, as in the reference's sum. Every NaN score
 * is stored as the quiet NaN 0x7fc00000.
 *
 * The score is the sum over KV heads divided by q_heads. The mean selector
 * rounds each product before adding it. Build with -ffp-contract=off so no
 * other product is fused.
 *
 * Ranking (torch.topk, selection.py:90): NaN ranks above every number,
 * including the +inf given to Quest's forced pages (selection.py:86-89), so
 * NaN pages take slots first; then forced pages; then scores in descending
 * order. Ties at the k-th key go to the lowest page. The mean selector
 * (selection.py:138-145) always keeps its required pages, so they rank
 * above NaN there.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { F32 = 0, F16 = 1, BF16 = 2 };

/* IEEE binary16 -> binary32, from the format definition (exact). */
static float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while (!(man & 0x400));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static float load_elem(const void* p, int dtype, int64_t i) {
  if (dtype == F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  if (dtype == BF16) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
  }
  return half_to_float(h);
}

static int elem_size(int dtype) { return dtype == F32 ? 4 : 2; }

/* ---- gather --------------------------------------------------------------- */

void oracle_gather_rows(const void* host, void* pool, const int64_t* miss_host, const int64_t* miss_dev, int64_t n,
                        int page_size, int64_t plane_bytes) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t s = miss_host[i], d = miss_dev[i];
    if (s < 0 || d < 0) continue;
    for (int plane = 0; plane < 2; ++plane) {
      int64_t so = ((s / page_size) * 2 * page_size + plane * page_size + s % page_size) * plane_bytes;
      int64_t dof = ((d / page_size) * 2 * page_size + plane * page_size + d % page_size) * plane_bytes;
      memcpy((char*)pool + dof, (const char*)host + so, (size_t)plane_bytes);
    }
  }
}

/* ---- attention -------------------------------------------------------------- */

void oracle_attend_rows(const void* q, int q_dtype, int64_t q_bs, int64_t q_hs, const void* pool, int kv_dtype,
                        const int64_t* rows, int64_t r_bs, int64_t r_hs, int64_t r_cs, int batch, int n_rows,
                        int q_heads, int kv_heads, int head_dim, int page_size, float* out) {
  const int group = q_heads / kv_heads;
  const double scale = 1.0 / sqrt((double)head_dim);
  double* s = (double*)malloc(sizeof(double) * (size_t)n_rows);
  double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < q_heads; ++h) {
      const int kh = h / group;
      double mx = -INFINITY;
      for (int c = 0; c < n_rows; ++c) {
        int64_t r = rows[(int64_t)b * r_bs + (int64_t)h * r_hs + (int64_t)c * r_cs];
        s[c] = -INFINITY;
        if (r < 0) continue;
        int64_t k0 = ((r / page_size) * 2 * page_size + r % page_size) * (int64_t)kv_heads * head_dim +
                     (int64_t)kh * head_dim;
        double dot = 0.0;
        for (int d = 0; d < head_dim; ++d)
          dot += (double)load_elem(q, q_dtype, (int64_t)b * q_bs + (int64_t)h * q_hs + d) *
                 (double)load_elem(pool, kv_dtype, k0 + d);
        s[c] = dot * scale;
        if (s[c] > mx) mx = s[c];
      }
      for (int d = 0; d < head_dim; ++d) acc[d] = 0.0;
      double den = 0.0;
      if (mx != -INFINITY)
        for (int c = 0; c < n_rows; ++c) {
          if (s[c] == -INFINITY) continue;
          int64_t r = rows[(int64_t)b * r_bs + (int64_t)h * r_hs + (int64_t)c * r_cs];
          int64_t v0 = ((r / page_size) * 2 * page_size + page_size + r % page_size) * (int64_t)kv_heads * head_dim +
                       (int64_t)kh * head_dim;
          double p = exp(s[c] - mx);
          den += p;
          for (int d = 0; d < head_dim; ++d) acc[d] += p * (double)load_elem(pool, kv_dtype, v0 + d);
        }
      float* o = out + ((int64_t)b * q_heads + h) * head_dim;
      for (int d = 0; d < head_dim; ++d) o[d] = den > 0.0 ? (float)(acc[d] / den) : 0.0f;
    }
  free(s);
  free(acc);
}

/* The reference's CPU attention (attention.py:26-35) in its own float32
   arithmetic: K and V widened to float32; a row's score is the float32 sum
   over d of q[d] * k[d] (products rounded, summed in d order) times the
   float32 value of head_dim^-0.5; masked rows get -inf; softmax as
   exp(s - max) / sum in float32; NaN weights (every row masked) become 0
   (nan_to_num); the output is the float32 sum of weight * v in row order. */
void oracle_attend_rows_f32(const void* q, int q_dtype, int64_t q_bs, int64_t q_hs, const void* pool, int kv_dtype,
                            const int64_t* rows, int64_t r_bs, int64_t r_hs, int64_t r_cs, int batch, int n_rows,
                            int q_heads, int kv_heads, int head_dim, int page_size, float* out) {
  const int group = q_heads / kv_heads;
  const float scale = (float)(1.0 / sqrt((double)head_dim));
  float* s = (float*)malloc(sizeof(float) * (size_t)n_rows);
  float* qv = (float*)malloc(sizeof(float) * (size_t)head_dim);
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < q_heads; ++h) {
      const int kh = h / group;
      for (int d = 0; d < head_dim; ++d) qv[d] = load_elem(q, q_dtype, (int64_t)b * q_bs + (int64_t)h * q_hs + d);
      float mx = -INFINITY;
      for (int c = 0; c < n_rows; ++c) {
        int64_t r = rows[(int64_t)b * r_bs + (int64_t)h * r_hs + (int64_t)c * r_cs];
        s[c] = -INFINITY;
        if (r < 0) continue;
        int64_t k0 = ((r / page_size) * 2 * page_size + r % page_size) * (int64_t)kv_heads * head_dim +
                     (int64_t)kh * head_dim;
        float dot = 0.0f;
        for (int d = 0; d < head_dim; ++d) {
          const float prod = load_elem(pool, kv_dtype, k0 + d) * qv[d];
          dot += prod;
        }
        s[c] = dot * scale;
        if (s[c] > mx) mx = s[c];
      }
      float* o = out + ((int64_t)b * q_heads + h) * head_dim;
      for (int d = 0; d < head_dim; ++d) o[d] = 0.0f;
      if (mx == -INFINITY) continue;  /* softmax of all -inf is NaN, then 0 */
      float den = 0.0f;
      for (int c = 0; c < n_rows; ++c) {
        s[c] = s[c] == -INFINITY ? 0.0f : expf(s[c] - mx);
        den += s[c];
      }
      for (int c = 0; c < n_rows; ++c) {
        int64_t r = rows[(int64_t)b * r_bs + (int64_t)h * r_hs + (int64_t)c * r_cs];
        if (r < 0) continue;
        const float w = s[c] / den;
        int64_t v0 = ((r / page_size) * 2 * page_size + page_size + r % page_size) * (int64_t)kv_heads * head_dim +
                     (int64_t)kh * head_dim;
        for (int d = 0; d < head_dim; ++d) {
          const float prod = w * load_elem(pool, kv_dtype, v0 + d);
          o[d] += prod;
        }
      }
    }
  free(s);
  free(qv);
}

/* ---- selectors ---------------------------------------------------------------- */

/* Elements per lane chunk: 16 bytes when the row is a multiple of 16 bytes
   of at most 64 chunks; else one element per lane up to 64 elements; else
   ceil(head_dim / 64) elements (the last lane's chunk is shorter). */
static int chunk_elems(int head_dim, int esize) {
  if ((head_dim * esize) % 16 == 0 && head_dim * esize / 16 <= 64) return 16 / esize;
  if (head_dim <= 64) return 1;
  return (head_dim + 63) / 64;
}

/* Quest cuts a bound row into 32-byte chunks when it is a multiple of 32
   bytes of at most 64 chunks, else as chunk_elems() does. */
static int quest_chunk_elems(int head_dim, int esize) {
  if ((head_dim * esize) % 32 == 0 && head_dim * esize / 32 <= 64) return 32 / esize;
  return chunk_elems(head_dim, esize);
}

/* The quiet NaN every NaN score is stored as. */
static float canonical_nan(void) {
  const uint32_t bits = 0x7fc00000u;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

/* Pairwise tree over t[0..L) (L a power of two), in place. */
static float tree_sum(float* t, int L) {
  for (int s = 1; s < L; s <<= 1)
    for (int i = 0; i + s < L; i += 2 * s) t[i] = t[i] + t[i + s];
  return t[0];
}

static int page_count(int64_t len, int page_size, int max_pages) {
  if (len <= 0) return 0;
  int64_t c = (len + page_size - 1) / page_size;
  return (int)(c < max_pages ? c : max_pages);
}

/* Quest score of every page p < count of one request (order in the header). */
static void quest_scores_one(const void* q, int q_dtype, int64_t q_hs, const void* lo, const void* hi, int bdt,
                             int q_heads, int kv_heads, int head_dim, int count, float* scores) {
  const int group = q_heads / kv_heads;
  const int E = quest_chunk_elems(head_dim, elem_size(bdt));
  const int used = (head_dim + E - 1) / E, L = pow2_at_least(used);
  const size_t n = (size_t)kv_heads * head_dim;
  float* qpos = (float*)malloc(sizeof(float) * n);
  float* qneg = (float*)malloc(sizeof(float) * n);
  /* bit 0: a head is > 0; bit 1: a head is not > 0; bit 2: a head is +-0;
     bit 3: a head is +-inf */
  unsigned char* side = (unsigned char*)malloc(n);
  float* t = (float*)malloc(sizeof(float) * (size_t)L);
  float* hs = (float*)malloc(sizeof(float) * (size_t)kv_heads);
  for (int kh = 0; kh < kv_heads; ++kh)
    for (int d = 0; d < head_dim; ++d) {
      float pos = 0.0f, neg = 0.0f;
      unsigned char f = 0;
      for (int g = 0; g < group; ++g) {
        float qd = load_elem(q, q_dtype, (int64_t)(kh * group + g) * q_hs + d);
        if (qd > 0.0f) {
          pos = pos + qd;
          f |= 1;
        } else {
          neg = neg + qd;
          f |= 2;
        }
        if (qd == 0.0f) f |= 4;
        if (isinf(qd)) f |= 8;
      }
      qpos[kh * head_dim + d] = pos, qneg[kh * head_dim + d] = neg;
      side[kh * head_dim + d] = f;
    }
  for (int p = 0; p < count; ++p) {
    for (int kh = 0; kh < kv_heads; ++kh) {
      const int64_t base = ((int64_t)p * kv_heads + kh) * head_dim;
      for (int l = 0; l < L; ++l) {
        t[l] = 0.0f;
        int bad = 0;
        for (int d = l * E; l < used && d < head_dim && d < (l + 1) * E; ++d) {
          const int i = kh * head_dim + d;
          const float x = load_elem(lo, bdt, base + d), y = load_elem(hi, bdt, base + d);
          const float a = y < x ? y : x, b = y < x ? x : y;
          const unsigned char f = side[i];
          t[l] = fmaf((f & 2) ? a : 0.0f, qneg[i], t[l]);
          t[l] = fmaf((f & 1) ? b : 0.0f, qpos[i], t[l]);
          bad |= isnan(x) || isnan(y);
          bad |= (f & 4) && (isinf(x) || isinf(y));
          bad |= (f & 8) && (x == 0.0f || y == 0.0f);
        }
        if (bad) t[l] = NAN;
      }
      hs[kh] = tree_sum(t, L);
    }
    float total = hs[0];
    for (int kh = 1; kh < kv_heads; ++kh) total = total + hs[kh];
    total = total / (float)q_heads;
    scores[p] = total != total ? canonical_nan() : total;
  }
  free(qpos);
  free(qneg);
  free(side);
  free(t);
  free(hs);
}

static void mean_scores_one(const void* q, int q_dtype, int64_t q_hs, const float* summ, int q_heads, int kv_heads,
                            int head_dim, int count, float* scores) {
  const int group = q_heads / kv_heads;
  const int E = chunk_elems(head_dim, 4);
  const int used = (head_dim + E - 1) / E, L = pow2_at_least(used);
  float* gq = (float*)malloc(sizeof(float) * (size_t)kv_heads * head_dim);
  float* t = (float*)malloc(sizeof(float) * (size_t)L);
  for (int kh = 0; kh < kv_heads; ++kh)
    for (int d = 0; d < head_dim; ++d) {
      float s = load_elem(q, q_dtype, (int64_t)(kh * group) * q_hs + d);
      for (int g = 1; g < group; ++g) s = s + load_elem(q, q_dtype, (int64_t)(kh * group + g) * q_hs + d);
      gq[kh * head_dim + d] = s / (float)group;
    }
  for (int p = 0; p < count; ++p) {
    float total = 0.0f;
    for (int kh = 0; kh < kv_heads; ++kh) {
      const float* sv = summ + ((int64_t)p * kv_heads + kh) * head_dim;
      const float* g = gq + kh * head_dim;
      for (int l = 0; l < L; ++l) {
        t[l] = 0.0f;
        for (int d = l * E; l < used && d < head_dim && d < (l + 1) * E; ++d) {
          float x = g[d] * sv[d];
          t[l] = d == l * E ? x : t[l] + x;
        }
      }
      float hsum = tree_sum(t, L);
      total = kh == 0 ? hsum : total + hsum;
    }
    scores[p] = total != total ? canonical_nan() : total;
  }
  free(gq);
  free(t);
}

/* Keys in descending rank order: NaN 0xfffffffe above every number (+inf is
   0xff800000); Quest's forced pages 0xfffffffd, just below NaN; the mean
   selector's required pages 0xffffffff, above NaN. */
enum { KEY_NAN = 0xfffffffeu, KEY_QUEST_FORCED = 0xfffffffdu, KEY_MEAN_REQUIRED = 0xffffffffu };

static uint32_t order_key(float s) {
  if (s != s) return KEY_NAN;
  uint32_t u;
  memcpy(&u, &s, 4);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
  uint32_t key;
  int page;
} KeyPage;

static int cmp_keypage_desc(const void* a, const void* b) {
  const KeyPage* x = (const KeyPage*)a;
  const KeyPage* y = (const KeyPage*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->page - y->page;
}

static int cmp_int(const void* a, const void* b) {
  int x = *(const int*)a, y = *(const int*)b;
  return (x > y) - (x < y);
}

/* Top-k of one request by (score desc, page asc); required pages first. */
static void select_one(const float* scores, int count, int64_t len, int page_size, int top_pages, int second,
                       uint32_t forced_key, int32_t* pages, int32_t* positions) {
  int* chosen = (int*)malloc(sizeof(int) * (size_t)(top_pages > 0 ? top_pages : 1));
  int n_sel = 0;
  if (top_pages >= count) {
    for (int p = 0; p < count; ++p) chosen[n_sel++] = p;
  } else {
    KeyPage* kp = (KeyPage*)malloc(sizeof(KeyPage) * (size_t)count);
    for (int p = 0; p < count; ++p) {
      kp[p].page = p;
      kp[p].key = (p == count - 1 || (second && p == 0)) ? forced_key : order_key(scores[p]);
    }
    qsort(kp, (size_t)count, sizeof(KeyPage), cmp_keypage_desc);
    for (int i = 0; i < top_pages; ++i) chosen[n_sel++] = kp[i].page;
    free(kp);
    qsort(chosen, (size_t)n_sel, sizeof(int), cmp_int);
  }
  for (int i = 0; i < top_pages; ++i) pages[i] = i < n_sel ? chosen[i] : -1;
  for (int64_t i = 0; i < (int64_t)top_pages * page_size; ++i) {
    int32_t p = pages[i / page_size];
    int64_t t = (int64_t)p * page_size + i % page_size;
    positions[i] = (p >= 0 && t < len) ? (int32_t)t : -1;
  }
  free(chosen);
}

void oracle_quest_select(int batch, const void* q, int q_dtype, int64_t q_bs, int64_t q_hs, const void* minimum,
                         const void* maximum, int bounds_dtype, int64_t b_bs, int q_heads, int kv_heads, int head_dim,
                         const int64_t* lengths, int page_size, int max_pages, int top_pages, int keep_sink,
                         float* scores, int32_t* pages, int32_t* positions) {
  const int esize = elem_size(bounds_dtype);
  for (int b = 0; b < batch; ++b) {
    const int count = page_count(lengths[b], page_size, max_pages);
    float* sc = scores + (int64_t)b * max_pages;
    if (top_pages < count)
      quest_scores_one((const char*)q + ((int64_t)b * q_bs) * elem_size(q_dtype), q_dtype, q_hs,
                       (const char*)minimum + (int64_t)b * b_bs * esize, (const char*)maximum + (int64_t)b * b_bs * esize,
                       bounds_dtype, q_heads, kv_heads, head_dim, count, sc);
    const int second = keep_sink && top_pages > 1 && count > 1;
    select_one(sc, count, lengths[b], page_size, top_pages, second, KEY_QUEST_FORCED, pages + (int64_t)b * top_pages,
               positions + (int64_t)b * top_pages * page_size);
  }
}

void oracle_mean_select(int batch, const void* q, int q_dtype, int64_t q_bs, int64_t q_hs, const float* summaries,
                        int64_t s_bs, int q_heads, int kv_heads, int head_dim, const int64_t* lengths, int page_size,
                        int max_pages, int top_pages, float* scores, int32_t* pages, int32_t* positions) {
  for (int b = 0; b < batch; ++b) {
    const int count = page_count(lengths[b], page_size, max_pages);
    float* sc = scores + (int64_t)b * max_pages;
    if (top_pages < count)
      mean_scores_one((const char*)q + ((int64_t)b * q_bs) * elem_size(q_dtype), q_dtype, q_hs, summaries + b * s_bs,
                      q_heads, kv_heads, head_dim, count, sc);
    select_one(sc, count, lengths[b], page_size, top_pages, top_pages > 1, KEY_MEAN_REQUIRED,
               pages + (int64_t)b * top_pages,
               positions + (int64_t)b * top_pages * page_size);
  }
}

/* ---- resolver ------------------------------------------------------------------ */

typedef struct {
  int64_t v;
  int64_t i;
} Pair;

static int cmp_pair(const void* a, const void* b) {
  const Pair* x = (const Pair*)a;
  const Pair* y = (const Pair*)b;
  if (x->v != y->v) return x->v < y->v ? -1 : 1;
  return (x->i > y->i) - (x->i < y->i);
}

static int cmp_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return (x > y) - (x < y);
}

/* first index i in sorted a[0..n) with a[i] >= x */
static int64_t lower_bound(const int64_t* a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) / 2;
    if (a[mid] < x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

/* Stable partition of perm[0..H) by key[perm[r]] (ascending key). */
static void stable_by_key(const int64_t* perm, const int* key, int nkeys, int64_t H, int64_t* out) {
  int64_t pos = 0;
  for (int k = 0; k < nkeys; ++k)
    for (int64_t r = 0; r < H; ++r)
      if (key[perm[r]] == k) out[pos++] = perm[r];
}

/*
 * One resolver item, following row_index.py:62-140 step by step. Tables are
 * int64 here; tags and lru are updated in place.
 */
void oracle_resolve_rows(const int64_t* raw, int64_t n, const int64_t* source, const int64_t* resident, int64_t n_pages,
                         const int64_t* hot, int64_t* tags, int64_t* lru, int64_t H, int64_t length, int64_t page_size,
                         int64_t* physical, int64_t* miss_host, int64_t* miss_device, int64_t* counts) {
  int64_t* norm = malloc(sizeof(int64_t) * n);
  int64_t* logical = malloc(sizeof(int64_t) * n);
  char* valid_raw = malloc(n);
  int64_t* host = malloc(sizeof(int64_t) * n);
  int64_t* offset = malloc(sizeof(int64_t) * n);
  int64_t* res = malloc(sizeof(int64_t) * n);
  char* valid = malloc(n);
  char* rhit = malloc(n);
  char* nhot = malloc(n);
  char* hhit = malloc(n);
  char* miss = malloc(n);
  int64_t* existing = malloc(sizeof(int64_t) * n);
  int64_t* assigned = malloc(sizeof(int64_t) * n);
  int64_t* hot_phys = malloc(sizeof(int64_t) * n);
  int64_t* phys = malloc(sizeof(int64_t) * n);
  int64_t* miss_rank = malloc(sizeof(int64_t) * n);
  int64_t* wanted_sorted = malloc(sizeof(int64_t) * n);
  Pair* tag_pairs = malloc(sizeof(Pair) * H);
  int64_t* sorted_tags = malloc(sizeof(int64_t) * H);
  int* prot = calloc(H, sizeof(int));
  int* category = calloc(H, sizeof(int));
  int64_t* victims = malloc(sizeof(int64_t) * H);
  int64_t* updates = malloc(sizeof(int64_t) * H);
  int64_t* new_lru = malloc(sizeof(int64_t) * H);
  int64_t* first_input = malloc(sizeof(int64_t) * n);

  for (int64_t i = 0; i < n; ++i) {  /* :69-72 */
    valid_raw[i] = raw[i] >= 0 && raw[i] < length;
    norm[i] = valid_raw[i] ? raw[i] : length;
    logical[i] = norm[i];
  }
  qsort(logical, (size_t)n, sizeof(int64_t), cmp_i64);
  for (int64_t j = 0; j < n; ++j) {  /* :73-82 */
    int unique = logical[j] < length && (j == 0 || logical[j] != logical[j - 1]);
    int64_t page = logical[j] / page_size;
    if (page > n_pages - 1) page = n_pages - 1;
    offset[j] = logical[j] % page_size;
    int64_t src = source[page];
    res[j] = resident[page];
    host[j] = src * page_size + offset[j];
    valid[j] = unique && src >= 0;
    rhit[j] = valid[j] && res[j] >= 0;
    nhot[j] = valid[j] && !rhit[j];
    wanted_sorted[j] = nhot[j] ? host[j] : -1;
  }
  for (int64_t s = 0; s < H; ++s) {  /* :87-90: tags.sort() */
    tag_pairs[s].v = tags[s];
    tag_pairs[s].i = s;
  }
  qsort(tag_pairs, (size_t)H, sizeof(Pair), cmp_pair);
  for (int64_t s = 0; s < H; ++s) sorted_tags[s] = tag_pairs[s].v;
  for (int64_t j = 0; j < n; ++j) {
    int64_t lk = lower_bound(sorted_tags, H, host[j]);
    if (lk > H - 1) lk = H - 1;
    hhit[j] = nhot[j] && sorted_tags[lk] == host[j];
    existing[j] = tag_pairs[lk].i;
  }
  qsort(wanted_sorted, (size_t)n, sizeof(int64_t), cmp_i64);  /* :91-93 */
  for (int64_t s = 0; s < H; ++s) {
    int64_t lk = lower_bound(wanted_sorted, n, tags[s]);
    if (lk > n - 1) lk = n - 1;
    prot[s] = tags[s] >= 0 && wanted_sorted[lk] == tags[s];
  }
  stable_by_key(lru, prot, 2, H, victims);  /* :97-98 */
  int64_t cum = 0;
  for (int64_t j = 0; j < n; ++j) {  /* :99-106 */
    miss[j] = nhot[j] && !hhit[j];
    cum += miss[j];
    miss_rank[j] = cum - 1;
    int64_t vr = miss_rank[j] < 0 ? 0 : (miss_rank[j] > H - 1 ? H - 1 : miss_rank[j]);
    assigned[j] = victims[vr];
    int64_t slot = hhit[j] ? existing[j] : assigned[j];
    hot_phys[j] = hot[slot / page_size] * page_size + slot % page_size;
    phys[j] = rhit[j] ? res[j] * page_size + offset[j] : hot_phys[j];
    if (!valid[j]) phys[j] = -1;
  }
  for (int64_t s = 0; s < H; ++s) updates[s] = -1;  /* :109-116 */
  for (int64_t j = 0; j < n; ++j)
    if (miss[j]) updates[assigned[j]] = host[j];
  for (int64_t s = 0; s < H; ++s) {
    int inserted = updates[s] >= 0;
    if (inserted) tags[s] = updates[s];
    category[s] = inserted + 2 * prot[s];
  }
  stable_by_key(lru, category, 4, H, new_lru);
  memcpy(lru, new_lru, sizeof(int64_t) * H);
  for (int64_t i = 0; i < n; ++i) miss_host[i] = miss_device[i] = -1;  /* :118-123 */
  for (int64_t j = 0; j < n; ++j)
    if (miss[j]) {
      miss_host[miss_rank[j]] = host[j];
      miss_device[miss_rank[j]] = hot_phys[j];
    }
  for (int64_t k = 0; k < n; ++k) first_input[k] = n;  /* :124-129 */
  for (int64_t i = 0; i < n; ++i) {
    int64_t f = lower_bound(logical, n, norm[i]);
    if (f > n - 1) f = n - 1;
    if (i < first_input[f]) first_input[f] = i;
  }
  for (int64_t i = 0; i < n; ++i) {
    int64_t f = lower_bound(logical, n, norm[i]);
    if (f > n - 1) f = n - 1;
    int keep = valid_raw[i] && first_input[f] == i;
    physical[i] = keep ? phys[f] : -1;
  }
  counts[0] = counts[1] = counts[2] = 0;  /* :135-140 */
  for (int64_t j = 0; j < n; ++j) {
    counts[0] += rhit[j];
    counts[1] += hhit[j];
    counts[2] += miss[j];
  }
  free(norm); free(logical); free(valid_raw); free(host); free(offset); free(res); free(valid); free(rhit);
  free(nhot); free(hhit); free(miss); free(existing); free(assigned); free(hot_phys); free(phys); free(miss_rank);
  free(wanted_sorted); free(tag_pairs); free(sorted_tags); free(prot); free(category); free(victims); free(updates);
  free(new_lru); free(first_input);
}

/* ---- bounds producer ----------------------------------------------------------------- */

/*
 * storage.py:302-309 for one page of one layer: summary = mean of the
 * page's first `valid` keys (fp32), min/max updated with the new keys
 * [within, within + count). Keys are [P, kv_heads, head_dim] (KV dtype);
 * minimum/maximum are fp32 copies of the KV-dtype values (exact).
 */
void oracle_append_bounds(const void* page_keys, int kv_dtype, int within, int count, int row_elems, float* summary,
                          float* minimum, float* maximum) {
  const int valid = within + count;
  for (int e = 0; e < row_elems; ++e) {
    double s = 0.0;
    for (int t = 0; t < valid; ++t) s += load_elem(page_keys, kv_dtype, (int64_t)t * row_elems + e);
    summary[e] = (float)(s / valid);
    for (int t = within; t < valid; ++t) {
      float k = load_elem(page_keys, kv_dtype, (int64_t)t * row_elems + e);
      /* torch.minimum / torch.maximum: NaN from either side propagates */
      if (k != k || minimum[e] != minimum[e]) minimum[e] = k + minimum[e];
      else if (k < minimum[e]) minimum[e] = k;
      if (k != k || maximum[e] != maximum[e]) maximum[e] = k + maximum[e];
      else if (k > maximum[e]) maximum[e] = k;
    }
  }
}
