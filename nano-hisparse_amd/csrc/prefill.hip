// Causal GQA self-attention for prefill (flash-attention forward, MFMA).
//
// out[s, h] = softmax_{t <= s}(q[s, h] . k[t, h/g] * D^-1/2) . v[t, h/g] for
// one prompt of `seq` tokens, bf16 or fp16 in, fp32 accumulation. A
// workgroup of 8 waves owns 128 queries of one query head (16 per wave) and
// walks the key tiles of 64 up to the diagonal with an online softmax.
//
// MFMA v_mfma_f32_16x16x32 (bf16 / f16): lane l supplies row l%16 of A and
// column l%16 of B at k = (l/16)*8 .. +7, and receives D rows (l/16)*4 + i,
// column l%16. The scores are computed transposed, S^T = K Q^T (A = 16 key
// rows of the LDS K tile, B = the wave's 16 query rows kept in registers),
// so a lane holds keys (l/16)*4 + i of every 16-key block for its query
// column l%16: a query's softmax statistics live in the 4 lanes l%16 = n and
// are reduced with two lane swaps. The output is accumulated transposed too,
// O^T = V^T P^T: its B operand (P^T, keys x queries) is the score layout
// itself once the k index of a 32-key step is taken as (block 2j, keys
// (l/16)*4 + i) then (block 2j+1, keys (l/16)*4 + i) -- the A operand (V^T
// rows from the transposed LDS V tile) uses the same key order -- and the
// rescaling by a query's max stays in its lane. The weights are rounded to
// the input dtype for the P.V product and the denominator sums the same
// rounded weights, so each output is an exact convex combination of V rows.
#include <math.h>

#include "nhs_common.h"

namespace nhs {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfBM = 16 * kPfWaves;  // queries per workgroup
constexpr int kPfBN = 64;             // keys per tile

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_f16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ pf_f32x4 mfma16x16x32(uint4 a, uint4 b, pf_f32x4 c) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8, a), __builtin_bit_cast(pf_bf16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pf_f16x8, a), __builtin_bit_cast(pf_f16x8, b), c,
                                                 0, 0, 0);
}

typedef float pf_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 pf_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 pf_f16x2 __attribute__((ext_vector_type(2)));

// two fp32 weights as a packed pair of the input dtype (round to nearest
// even, by the hardware conversions)
template <typename T>
__device__ __forceinline__ uint32_t pf_pack(float lo, float hi) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((pf_f32x2){lo, hi}, pf_bf16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((pf_f32x2){lo, hi}, pf_f16x2));
}
template <typename T>
__device__ __forceinline__ float pf_unpack(uint32_t v, int half) {
  const uint32_t b = half ? v >> 16 : v & 0xffffu;
  return T::dtype == NHS_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// 16-bit element (word w, half) of a 16-byte chunk
__device__ __forceinline__ uint32_t pf_get16(const uint4& v, int w, int half) {
  const uint32_t x = w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
  return half ? x >> 16 : x & 0xffffu;
}

struct PrefillArgs {
  const char* q;
  const char* k;
  const char* v;
  int64_t q_s, q_h, k_s, k_h, v_s, v_h;  // element strides
  int seq, q_heads, group;
  float scale_log2;  // D^-1/2 * log2(e)
  char* out;
  int64_t o_s, o_h;
};

template <typename T, int D>
__global__ __launch_bounds__(kPfThreads) void prefill_attention_kernel(PrefillArgs a) {
  constexpr int KS = D / 32;   // 32-wide k steps of Q.K
  constexpr int DB = D / 16;   // 16-wide dim blocks of the output
  constexpr int KROW = D * 2 + 16;       // bytes per K row in LDS (padded)
  constexpr int VROW = kPfBN * 2 + 16;   // bytes per V^T row in LDS (padded)
  // two buffers per tile: tile t+1 is stored while tile t is read, one barrier per tile
  __shared__ __attribute__((aligned(16))) char ks_buf[2][kPfBN * KROW];
  __shared__ __attribute__((aligned(16))) char vt_buf[2][D * VROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, n = lane & 15;
  const int n_qblocks = (a.seq + kPfBM - 1) / kPfBM;
  const int qb = n_qblocks - 1 - (int)blockIdx.x;  // the longest rows first
  const int h = blockIdx.y;
  const int kvh = h / a.group;
  const int q0 = qb * kPfBM;
  const int query = q0 + wave * 16 + n;  // this lane's query (column of S^T)
  const bool q_live = query < a.seq;

  // the wave's query rows as B operands: dims ks*32 + g4*8 .. +7
  uint4 qf[KS];
  {
    const int qr = q_live ? query : a.seq - 1;
    const char* qp = a.q + ((int64_t)qr * a.q_s + (int64_t)h * a.q_h) * T::bytes;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const uint4*>(qp + (s * 32 + g4 * 8) * T::bytes);
  }

  float m = -INFINITY, l = 0.f;
  pf_f32x4 o[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) o[b] = (pf_f32x4){0.f, 0.f, 0.f, 0.f};

  // tile staging: thread t loads K row t/KT's dims [(t%KT)*D/KT, +D/KT) and
  // the VR V rows VR*(t/16) .. +VR-1 at dims 8*(t%16) .. +7 (D = 64 uses the
  // first half of the threads for V)
  constexpr int KT = kPfThreads / kPfBN;        // threads per K row
  constexpr int KCH = D * 2 / KT / 16;          // 16-byte chunks of K per thread
  constexpr int VR = kPfBN * 16 / kPfThreads;   // V rows per thread (16 groups of 8 dims)
  static_assert(KCH >= 1 && (VR == 2 || VR == 4), "tile staging layout");
  const int krow = tid / KT, kcol = (tid % KT) * (D / KT);
  const int vkg = tid >> 4, vdg = tid & 15;
  const bool v_thread = vdg * 8 < D;
  const int last_key = min(a.seq, q0 + kPfBM) - 1;
  const int n_tiles = last_key / kPfBN + 1;
  uint4 kreg[KCH], vreg[VR];
  auto load_tile = [&](int t0) {
    const int kr = min(t0 + krow, a.seq - 1);  // rows past the end re-read the last key (masked below)
    const char* kp = a.k + ((int64_t)kr * a.k_s + (int64_t)kvh * a.k_h + kcol) * T::bytes;
#pragma unroll
    for (int c = 0; c < KCH; ++c) kreg[c] = *reinterpret_cast<const uint4*>(kp + c * 16);
    if (v_thread)
#pragma unroll
      for (int r = 0; r < VR; ++r) {
        const int vr = min(t0 + vkg * VR + r, a.seq - 1);
        vreg[r] = *reinterpret_cast<const uint4*>(a.v + ((int64_t)vr * a.v_s + (int64_t)kvh * a.v_h + vdg * 8) * T::bytes);
      }
  };
  auto store_tile = [&](int buf) {
    char* ks_lds = ks_buf[buf];
    char* vt_lds = vt_buf[buf];
#pragma unroll
    for (int c = 0; c < KCH; ++c)
      *reinterpret_cast<uint4*>(ks_lds + krow * KROW + kcol * T::bytes + c * 16) = kreg[c];
    if (v_thread)
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // V^T[dim 8*vdg + j][keys VR*vkg .. +VR-1]
        const int half = j & 1, w = j >> 1;
        const uint32_t e0 = pf_get16(vreg[0], w, half), e1 = pf_get16(vreg[1], w, half);
        char* dst = vt_lds + (vdg * 8 + j) * VROW + vkg * VR * 2;
        if constexpr (VR == 4) {
          const uint32_t e2 = pf_get16(vreg[2], w, half), e3 = pf_get16(vreg[3], w, half);
          *reinterpret_cast<uint2*>(dst) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
        } else {
          *reinterpret_cast<uint32_t*>(dst) = e0 | (e1 << 16);
        }
      }
  };

  load_tile(0);
  store_tile(0);
  if (n_tiles > 1) load_tile(kPfBN);
  for (int t = 0; t < n_tiles; ++t) {
    const int t0 = t * kPfBN;
    // tile t's buffer is complete and every wave is done with tile t-1's
    // buffer, which now takes tile t+1 (loaded during tile t-1's math)
    __syncthreads();
    if (t + 1 < n_tiles) {
      store_tile((t + 1) & 1);
      if (t + 2 < n_tiles) load_tile(t0 + 2 * kPfBN);  // in flight during this tile's math
    }
    const char* ks_lds = ks_buf[t & 1];
    const char* vt_lds = vt_buf[t & 1];

    // S^T for 4 key blocks of 16: s[kb] holds keys t0 + kb*16 + g4*4 + i
    pf_f32x4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s[kb] = (pf_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const uint4 kf = *reinterpret_cast<const uint4*>(ks_lds + (kb * 16 + n) * KROW + (st * 32 + g4 * 8) * T::bytes);
        s[kb] = mfma16x16x32<T>(kf, qf[st], s[kb]);
      }
    }
    // scale, mask (causal and past the end; a tile wholly below the wave's
    // diagonal and inside the prompt needs none), running max
    float mx = m;
    if (t0 + kPfBN - 1 <= q0 + wave * 16 && t0 + kPfBN <= a.seq) {  // uniform over the wave
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[kb][i] = s[kb][i] * a.scale_log2;
          mx = fmaxf(mx, s[kb][i]);
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = t0 + kb * 16 + g4 * 4 + i;
          const float x = (key <= query && key < a.seq) ? s[kb][i] * a.scale_log2 : -INFINITY;
          s[kb][i] = x;
          mx = fmaxf(mx, x);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float ref = mx == -INFINITY ? 0.f : mx;
    const float alpha = __builtin_amdgcn_exp2f(m - ref);
    m = mx;
    // weights rounded to the input dtype, packed as P^T B operands: step j
    // (keys of blocks 2j and 2j+1) is {s[2j][0..3], s[2j+1][0..3]}
    uint4 pb[2];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t w[4];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const pf_f32x4& sv = s[2 * j + half];
        const uint32_t a01 = pf_pack<T>(__builtin_amdgcn_exp2f(sv[0] - ref), __builtin_amdgcn_exp2f(sv[1] - ref));
        const uint32_t a23 = pf_pack<T>(__builtin_amdgcn_exp2f(sv[2] - ref), __builtin_amdgcn_exp2f(sv[3] - ref));
        w[half * 2] = a01, w[half * 2 + 1] = a23;
        psum += pf_unpack<T>(a01, 0) + pf_unpack<T>(a01, 1) + pf_unpack<T>(a23, 0) + pf_unpack<T>(a23, 1);
      }
      pb[j] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    psum += __shfl_xor(psum, 16);
    psum += __shfl_xor(psum, 32);
    l = l * alpha + psum;
    // O^T += V^T P^T: dim block b, keys in the same order as pb
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      o[b] *= alpha;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const char* vrow = vt_lds + (b * 16 + n) * VROW;
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + ((2 * j) * 16 + g4 * 4) * 2);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + ((2 * j + 1) * 16 + g4 * 4) * 2);
        o[b] = mfma16x16x32<T>(make_uint4(lo.x, lo.y, hi.x, hi.y), pb[j], o[b]);
      }
    }
  }
  if (!q_live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  char* op = a.out + ((int64_t)query * a.o_s + (int64_t)h * a.o_h) * T::bytes;
#pragma unroll
  for (int b = 0; b < DB; ++b) {  // this lane: dims b*16 + g4*4 .. +3 of its query
    const uint32_t w0 = pf_pack<T>(o[b][0] * inv, o[b][1] * inv), w1 = pf_pack<T>(o[b][2] * inv, o[b][3] * inv);
    *reinterpret_cast<uint2*>(op + (b * 16 + g4 * 4) * T::bytes) = make_uint2(w0, w1);
  }
}

}  // namespace nhs

extern "C" int nhs_prefill_attention(const void* q, int64_t q_seq_stride, int64_t q_head_stride, const void* k,
                                     int64_t k_seq_stride, int64_t k_head_stride, const void* v,
                                     int64_t v_seq_stride, int64_t v_head_stride, int32_t dtype, int32_t seq,
                                     int32_t q_heads, int32_t kv_heads, int32_t head_dim, void* out,
                                     int64_t out_seq_stride, int64_t out_head_stride, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_prefill_attention";
  if (!q || !k || !v || !out) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (dtype != NHS_BF16 && dtype != NHS_F16) return fail(NHS_ERR_UNSUPPORTED, "%s: bf16 or fp16 only", who);
  if (head_dim != 64 && head_dim != 128) return fail(NHS_ERR_UNSUPPORTED, "%s: head_dim 64 or 128", who);
  if (seq < 1 || q_heads < 1 || kv_heads < 1 || q_heads % kv_heads)
    return fail(NHS_ERR_INVALID, "%s: invalid shape", who);
  const int64_t strides[] = {q_seq_stride, q_head_stride, k_seq_stride, k_head_stride, v_seq_stride,
                             v_head_stride, out_seq_stride, out_head_stride};
  for (int64_t st : strides)
    if (st % 8) return fail(NHS_ERR_INVALID, "%s: strides must be multiples of 8 elements", who);
  if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16) != 0)
    return fail(NHS_ERR_INVALID, "%s: tensors must be 16-byte aligned", who);
  PrefillArgs a;
  a.q = static_cast<const char*>(q);
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.q_s = q_seq_stride, a.q_h = q_head_stride;
  a.k_s = k_seq_stride, a.k_h = k_head_stride;
  a.v_s = v_seq_stride, a.v_h = v_head_stride;
  a.seq = seq;
  a.q_heads = q_heads;
  a.group = q_heads / kv_heads;
  a.scale_log2 = (float)(1.4426950408889634 / sqrt((double)head_dim));
  a.out = static_cast<char*>(out);
  a.o_s = out_seq_stride, a.o_h = out_head_stride;
  const dim3 grid((unsigned)((seq + kPfBM - 1) / kPfBM), (unsigned)q_heads), block(kPfThreads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NHS_BF16) {
    if (head_dim == 128)
      launch(prefill_attention_kernel<BF16, 128>, grid, block, 0, s, ev.start, ev.stop, a);
    else
      launch(prefill_attention_kernel<BF16, 64>, grid, block, 0, s, ev.start, ev.stop, a);
  } else {
    if (head_dim == 128)
      launch(prefill_attention_kernel<F16, 128>, grid, block, 0, s, ev.start, ev.stop, a);
    else
      launch(prefill_attention_kernel<F16, 64>, grid, block, 0, s, ev.start, ev.stop, a);
  }
  return launch_status(who);
}
